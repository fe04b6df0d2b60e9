"""The CPU oracle against the reference's own known-answer tests (data in
tests/golden/reference_kats.json, transcribed from the reference's tests)."""
import json
import os

import numpy as np
import pytest

import oracle

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


@pytest.mark.parametrize("kat", KATS["dense_u32_matmul"], ids=lambda k: k["source"].split()[-1])
def test_dense_u32_matmul_kats(kat):
    v = np.array(kat["values"], np.int8).reshape(kat["rows"], kat["cols"])
    packed = oracle.pack_rows_u32(v)
    out = oracle.ternary_matmul_u32(packed, kat["scales"], kat["input"], kat["seq"], kat["cols"], kat["rows"])
    np.testing.assert_allclose(out.ravel(), kat["expected"], atol=kat["tol"], rtol=0)


def test_pack_rows_u32_codes_kat():
    kat = KATS["pack_rows_u32_codes"][0]
    v = np.array(kat["values"], np.int8).reshape(1, kat["cols"])
    packed = oracle.pack_rows_u32(v).ravel()
    assert packed.size == kat["words"]
    for i, code in enumerate(kat["codes"]):
        assert (int(packed[i // 16]) >> (2 * (i % 16))) & 3 == code, i


@pytest.mark.parametrize("kat", KATS["pack_u8_roundtrip"], ids=lambda k: str(k["values"]))
def test_pack_u8_roundtrip_kats(kat):
    v = np.array(kat["values"], np.int8)
    p = oracle.pack_ternary(v)
    assert p.size == kat["packed_len"]
    np.testing.assert_array_equal(oracle.unpack_ternary(p, v.size), v)


def test_pack_u8_cycle_kat():
    kat = KATS["pack_u8_cycle"]
    v = (np.arange(kat["n"]) % 3 - 1).astype(np.int8)
    p = oracle.pack_ternary(v)
    assert p.size == kat["packed_len"]
    np.testing.assert_array_equal(oracle.unpack_ternary(p, v.size), v)


@pytest.mark.parametrize("kat", KATS["i8_matmul"], ids=lambda k: k["source"].split()[-1])
def test_i8_matmul_kats(kat):
    out = oracle.ternary_matmul_i8(kat["ternary"], kat["scale"], kat["input"], kat["out_rows"], kat["in_cols"], kat["seq"])
    np.testing.assert_allclose(out, kat["expected"], atol=kat["tol"], rtol=0)


def test_packed_matmul_kat():
    kat = KATS["packed_matmul"][0]
    p = oracle.pack_ternary(np.array(kat["ternary"], np.int8))
    out = oracle.ternary_matmul_packed(p, kat["scale"], kat["input"], kat["out_rows"], kat["in_cols"], kat["seq"])
    np.testing.assert_allclose(out, kat["expected"], atol=kat["tol"], rtol=0)
    ref = oracle.ternary_matmul_i8(kat["ternary"], kat["scale"], kat["input"], kat["out_rows"], kat["in_cols"], kat["seq"])
    np.testing.assert_allclose(out, ref, atol=1e-5, rtol=0)


@pytest.mark.parametrize("kat", KATS["sparse24_gpu"], ids=lambda k: k["source"].split()[-1])
def test_sparse24_gpu_kats(kat):
    w = np.array(kat["weights"], np.int8).reshape(kat["rows"], kat["cols"])
    meta, scales = oracle.pack_sparse24_gpu(w)
    out = oracle.sparse24_gpu_matmul(meta, scales, kat["input"], kat["seq"], kat["cols"], kat["rows"])
    np.testing.assert_allclose(out.ravel(), kat["expected"], atol=kat["tol"], rtol=0)


def test_sparse24_gpu_packer_rejects_non_24():
    with pytest.raises(ValueError):
        oracle.pack_sparse24_gpu(np.array([[1, 1, 1, 0]], np.int8))


def test_sparse24_cpu_signs_kat():
    kat = KATS["sparse24_cpu_signs"]
    p, s = oracle.sparse24_cpu_from_ternary(kat["ternary"], kat["rows"], kat["cols"])
    d = oracle.sparse24_cpu_to_ternary(p, s, kat["rows"], kat["cols"])
    for pos, val in kat["expected_positions"].items():
        assert d[int(pos)] == val


def test_sparse24_cpu_known_output_kat():
    kat = KATS["sparse24_cpu_known_output"]
    p, s = oracle.sparse24_cpu_from_ternary(kat["ternary"], kat["rows"], kat["cols"])
    out = oracle.sparse24_cpu_matmul(p, s, kat["scale"], kat["rows"], kat["cols"], kat["input"], 1)
    np.testing.assert_allclose(out, kat["expected"], atol=kat["tol"], rtol=0)
    dec = oracle.sparse24_cpu_matmul_decode(p, s, kat["scale"], kat["rows"], kat["cols"], kat["input"])
    np.testing.assert_array_equal(dec, out)


def test_sparse24_cpu_basic_kat():
    kat = KATS["sparse24_cpu_basic"]
    p, s = oracle.sparse24_cpu_from_ternary(kat["ternary"], kat["rows"], kat["cols"])
    d = oracle.sparse24_cpu_to_ternary(p, s, kat["rows"], kat["cols"]).reshape(-1, 4)
    assert ((d != 0).sum(axis=1) <= kat["max_nonzeros_per_group"]).all()


@pytest.mark.parametrize("kat", KATS["routing"], ids=lambda k: k["source"].split()[-1])
def test_routing_kats(kat):
    # Router = identity matrix, so the logits are exactly the inputs.
    logits = np.array(kat["logits"], np.float32)[None, :]
    e = logits.shape[1]
    idx, w, _ = oracle.moe_route(logits, np.eye(e, dtype=np.float32), kat["top_k"])
    assert list(idx[0]) == kat["expected_idx"]
    sel = logits[0, kat["expected_idx"]].astype(np.float64)
    expect = np.exp(sel) / np.exp(sel).sum()
    np.testing.assert_allclose(w[0], expect, atol=kat["weight_tol"], rtol=0)
    if "sum_tol" in kat:
        assert abs(float(w[0].sum()) - 1.0) < kat["sum_tol"]


def test_ternary_stats_kat():
    kat = KATS["ternary_stats"]
    counts, ratios, comp = oracle.ternary_stats(np.array(kat["values"], np.int8))
    assert list(counts) == [kat["num_neg1"], kat["num_zero"], kat["num_pos1"]]
    assert abs(float(ratios[1]) - kat["ratio_zero"]) < kat["ratio_tol"]
    assert abs(comp - kat["compression_ratio_vs_f32"]) < 0.01


def test_sparse_indices_kat():
    kat = KATS["sparse_indices_counts"]
    po, pi, no, ni = oracle.ternary_sparse_indices(np.array(kat["ternary"], np.int8), kat["rows"], kat["cols"])
    for r in range(kat["rows"]):
        assert list(pi[po[r]:po[r + 1]]) == kat["pos"][r]
        assert list(ni[no[r]:no[r + 1]]) == kat["neg"][r]


def test_sparse_decode_vs_general_kat():
    kat = KATS["sparse_decode_vs_general"]
    rows, cols = kat["rows"], kat["cols"]
    t = np.array([{0: 1, 1: -1, 2: 0}[i % 3] for i in range(rows * cols)], np.int8)
    x = (np.arange(cols, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    idx = oracle.ternary_sparse_indices(t, rows, cols)
    out = oracle.ternary_matmul_sparse_decode(*idx, kat["scale"], x, rows)
    ref = oracle.ternary_matmul_decode(t, kat["scale"], x, rows, cols)
    np.testing.assert_allclose(out, ref, rtol=0, atol=kat["tol"])


def test_blocked_vs_scalar_kat():
    kat = KATS["blocked_vs_scalar"]
    rows, cols, bs = kat["rows"], kat["cols"], kat["block_size"]
    w = (np.sin(np.arange(rows * cols, dtype=np.float32) * np.float32(1.618)) * np.float32(0.5)).astype(np.float32)
    nb = (cols + bs - 1) // bs
    scales = np.zeros(nb, np.float32)
    for b in range(nb):
        blk = w.reshape(rows, cols)[:, b * bs:(b + 1) * bs]
        s = np.float32(0)
        for v in blk.ravel():
            s = np.float32(s + np.float32(abs(v)))
        scales[b] = (s / np.float32(blk.size)) / np.float32(0.7978845608) if s > 0 else np.float32(1.0)
    t = np.zeros(rows * cols, np.int8)
    for r in range(rows):
        for b in range(nb):
            inv = np.float32(1.0) / scales[b]
            for j in range(b * bs, min((b + 1) * bs, cols)):
                v = np.float32(w[r * cols + j] * inv)
                t[r * cols + j] = int(np.clip(np.sign(v) * np.floor(abs(v) + 0.5), -1, 1))
    x = np.cos(np.arange(cols, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    out = oracle.ternary_matmul_blocked(t, scales, bs, x, rows, cols, 1)
    ref = np.zeros(rows, np.float32)
    for r in range(rows):
        for b in range(nb):
            for j in range(b * bs, min((b + 1) * bs, cols)):
                ref[r] = np.float32(ref[r] + np.float32(scales[b] * np.float32(t[r * cols + j])) * x[j])
    np.testing.assert_allclose(out, ref, rtol=0, atol=kat["tol"])


def test_ternary_linear_bias_kat():
    """ternary_linear.rs:308-324 (test_with_bias): the 2x3 layer
    [1, -1, 0.5, -0.5, 1, 1] quantises (absmean, ternary.rs:31-57) to
    [[1, -1, 0], [0, 1, 1]], so input [1, 2, 3] gives -alpha + 0.1 and
    5 alpha + 0.2, each product and sum rounded to f32 once."""
    t, alpha = oracle.quantize_ternary(np.array([1.0, -1.0, 0.5, -0.5, 1.0, 1.0], np.float32))
    np.testing.assert_array_equal(t, [1, -1, 0, 0, 1, 1])
    bias = np.array([0.1, 0.2], np.float32)
    x = np.array([1.0, 2.0, 3.0], np.float32)
    want = np.array([np.float32(-alpha) + bias[0], np.float32(alpha * np.float32(5.0)) + bias[1]], np.float32)
    for path in (0, 2):  # forward, forward_decode
        out = oracle.ternary_linear_forward(t, alpha, bias, x, 2, 3, 1, path)
        np.testing.assert_array_equal(out.ravel(), want)
        nob = oracle.ternary_linear_forward(t, alpha, None, x, 2, 3, 1, path)
        np.testing.assert_array_equal(nob.ravel(), [-alpha, np.float32(alpha * np.float32(5.0))])


def test_ternary_linear_paths_agree_with_bias():
    """forward / forward_packed / forward_decode with the same bias
    (ternary_linear.rs:258-306 pin the paths against each other without a
    bias; in_cols % 4 == 0 so the packed path's flat byte addressing is
    row-aligned), and seq tokens each get the bias once (:326-352)."""
    rng = np.random.default_rng(7)
    R, C, S = 6, 12, 3
    t = rng.integers(-1, 2, size=(R, C)).astype(np.int8)
    x = rng.standard_normal((S, C)).astype(np.float32)
    bias = rng.standard_normal(R).astype(np.float32)
    f = oracle.ternary_linear_forward(t, 0.37, bias, x, R, C, S, 0)
    p = oracle.ternary_linear_forward(t, 0.37, bias, x, R, C, S, 1)
    np.testing.assert_allclose(p, f, atol=1e-5, rtol=0)
    nob = oracle.ternary_linear_forward(t, 0.37, None, x, R, C, S, 0)
    np.testing.assert_array_equal(f, nob + bias[None, :])
    for s in range(S):
        d = oracle.ternary_linear_forward(t, 0.37, bias, x[s], R, C, 1, 2)
        np.testing.assert_allclose(d.ravel(), f[s], atol=1e-5, rtol=0)


def test_prune_fp32_kat():
    """prune_fp32_to_sparse_ternary (sparse_ternary.rs:523-544
    test_prune_fp32_to_sparse): top-2 by |v| per group, decompressed."""
    kat = KATS["prune_fp32"]
    w = np.array(kat["weights"], np.float32)
    pats, signs, scale = oracle.prune_sparse24(w, kat["rows"], kat["cols"])
    dec = oracle.sparse24_cpu_to_ternary(pats, signs, kat["rows"], kat["cols"])
    np.testing.assert_array_equal(dec, kat["expected_decompressed"])
    # the absmean of the fp32 values, ternary.rs:15 ABSMEAN_NORM
    assert abs(float(scale) - np.abs(w.astype(np.float64)).mean() / 0.7978845608) <= 1e-6 * float(scale)


def _quantization_cos(w, r):
    w = w.astype(np.float64)
    r = r.astype(np.float64)
    return float((w @ r) / (np.linalg.norm(w) * np.linalg.norm(r)))


def test_blocked_vs_per_tensor_kat():
    """ternary.rs:845-873 test_blocked_vs_per_tensor: bimodal weights (i *
    0.001 - 0.128 for i < 256, i * 0.01 - 2.56 above), block 64: the blocked
    round trip's cosine is at least the per-tensor one minus 0.01."""
    i = np.arange(512, dtype=np.float32)
    w = np.where(i < 256, i * np.float32(0.001) - np.float32(0.128),
                 i * np.float32(0.01) - np.float32(2.56)).astype(np.float32)
    q_t, s_t = oracle.quantize_ternary(w)
    r_t = s_t * q_t.astype(np.float32)
    q_b, s_b = oracle.quantize_ternary_blocked(w, 64)
    assert s_b.size == 8
    r_b = oracle.dequantize_ternary_blocked(q_b, s_b, 64)
    assert _quantization_cos(w, r_b) >= _quantization_cos(w, r_t) - 0.01
