"""Host packers of libfrx_ternary.so (no GPU) — bit-exact with the oracle."""
import os

import numpy as np
import pytest

import ferrisres_amd as frx
import oracle
from ferrisres_amd import synth


@pytest.mark.parametrize("n", [0, 1, 3, 4, 17, 1000, 4097])
def test_pack_unpack_u8(n):
    rng = np.random.default_rng(n)
    v = rng.integers(-1, 2, size=n).astype(np.int8)
    p = frx.pack_ternary_u8(v)
    np.testing.assert_array_equal(p, oracle.pack_ternary(v))
    np.testing.assert_array_equal(frx.unpack_ternary_u8(p, n), v)


def test_pack_u8_out_of_range():
    v = np.array([3, -2, 1, 0, -1], np.int8)
    np.testing.assert_array_equal(frx.pack_ternary_u8(v), oracle.pack_ternary(v))


@pytest.mark.parametrize("n", [1, 16, 17, 333, 8192])
def test_repack_u32(n):
    rng = np.random.default_rng(n + 1)
    v = rng.integers(-1, 2, size=n).astype(np.int8)
    p = oracle.pack_ternary(v)
    np.testing.assert_array_equal(frx.repack_u8_to_u32(p, n), oracle.pack_ternary_u32(p, n))


def test_gpu_packed_matches_reference_bridge():
    rng = np.random.default_rng(3)
    t = rng.integers(-1, 2, size=(40, 128)).astype(np.int8)
    w, s = frx.gpu_packed(t, 0.125)
    bridge = oracle.pack_ternary_u32(oracle.pack_ternary(t), t.size).reshape(40, 8)
    np.testing.assert_array_equal(w, bridge)
    assert (s == np.float32(0.125)).all()


def test_pack_sparse24_gpu_matches_oracle():
    t = synth.sparse24_uniform("pk", "w", 33, 100)
    meta, sc = frx.pack_sparse24_gpu(t, with_scales=True)
    m2, s2 = oracle.pack_sparse24_gpu(t)
    np.testing.assert_array_equal(meta, m2)
    np.testing.assert_array_equal(sc, s2)


def test_pack_sparse24_gpu_rejects_bad_groups():
    with pytest.raises(frx.FrxError) as e:
        frx.pack_sparse24_gpu(np.array([[1, 0, 0, 0]], np.int8))
    assert e.value.kind == "Shape"


@pytest.mark.parametrize("seed", [0, 1])
def test_sparse24_cpu_to_gpu_transcoder(seed):
    rng = np.random.default_rng(seed)
    rows, cols = 19, 72
    # arbitrary ternary -> CPU 2:4 (lossy for groups with < 2 nonzeros)
    t = rng.integers(-1, 2, size=(rows, cols)).astype(np.int8)
    p, s = oracle.sparse24_cpu_from_ternary(t, rows, cols)
    meta = frx.sparse24_cpu_to_gpu(p, s, rows, cols)
    np.testing.assert_array_equal(oracle.sparse24_gpu_decode(meta, rows, cols).ravel(),
                                  oracle.sparse24_cpu_to_ternary(p, s, rows, cols))
    # on true 2:4 input the transcoded metadata equals the GPU packer's
    t24 = synth.sparse24_uniform("tc", str(seed), rows, cols)
    p, s = oracle.sparse24_cpu_from_ternary(t24, rows, cols)
    m2, _ = oracle.pack_sparse24_gpu(t24)
    np.testing.assert_array_equal(frx.sparse24_cpu_to_gpu(p, s, rows, cols), m2)


def test_sparse24_transcoder_patterns_6_7_follow_to_ternary():
    """Raw CPU-layout bytes (every pattern nibble 0..7, any sign bits): the
    transcoded GPU metadata decodes to the matrix to_ternary reads from the
    CPU layout (patterns 6 and 7 fall back to pattern 0 there,
    sparse_ternary.rs:172-176)."""
    rng = np.random.default_rng(67)
    rows, cols = 13, 96
    ng = rows * cols // 4
    p = rng.integers(0, 256, size=(ng + 1) // 2, dtype=np.uint8)
    s = rng.integers(0, 256, size=(ng + 3) // 4, dtype=np.uint8)
    assert ((p & 7) >= 6).any() and ((p >> 4) >= 6).any()
    meta = frx.sparse24_cpu_to_gpu(p, s, rows, cols)
    np.testing.assert_array_equal(oracle.sparse24_gpu_decode(meta, rows, cols).ravel(),
                                  oracle.sparse24_cpu_to_ternary(p, s, rows, cols))


def test_sparse_indices_host_equals_oracle():
    """frx_ternary_sparse_indices (ternary_sparse_indices, ternary.rs:681-707)
    equals the oracle's CSR lists, the reference KAT included."""
    import json
    kats = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))
    kat = kats["sparse_indices_counts"]
    po, pi, no, ni = frx.ternary_sparse_indices(np.array(kat["ternary"], np.int8).reshape(kat["rows"], kat["cols"]))
    for r in range(kat["rows"]):
        assert list(pi[po[r]:po[r + 1]]) == kat["pos"][r]
        assert list(ni[no[r]:no[r + 1]]) == kat["neg"][r]
    t = np.random.default_rng(3).integers(-1, 2, size=(57, 130)).astype(np.int8)
    a = frx.ternary_sparse_indices(t)
    b = oracle.ternary_sparse_indices(t, 57, 130)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x[:len(y)], y)
