"""The reference's other ternary matmul forms on the GPU against the oracle:
column-block scales (ternary_matmul_blocked, ternary.rs:541-579), index-list
decode (ternary_matmul_sparse_decode with ternary_sparse_indices,
ternary.rs:647-707) and tensor statistics (ternary_stats, ternary.rs:725-746).
Dyadic inputs with power-of-two scales make every partial sum exact, so there
the GPU equals the oracle bit for bit; random inputs within 1e-3."""
import numpy as np
import pytest
import torch

import ferrisres_amd as frx
import oracle
from ferrisres_amd import synth
from _gpu import DEV, assert_close_f32, dev_bf16, dev_f32, dev_u32, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "GPU tests need a gfx950 device"
    c = frx.Context(0)
    yield c
    c.close()


def _dyadic(rng, n):
    return (rng.integers(-64, 65, size=n) / 8).astype(np.float32)


@pytest.mark.parametrize("M,K,N,bs", [(1, 4096, 256, 64), (3, 1024, 130, 100), (20, 512, 96, 32), (1, 2048, 64, 2048)])
def test_blocked_linear(ctx, M, K, N, bs):
    rng = np.random.default_rng(M * 7 + K)
    t = rng.integers(-1, 2, size=(N, K)).astype(np.int8)
    nb = (K + bs - 1) // bs
    w = dev_u32(oracle.pack_rows_u32(t))
    # power-of-two block scales + dyadic activations: exact
    sc = (2.0 ** rng.integers(-3, 3, size=nb)).astype(np.float32)
    x = _dyadic(rng, M * K).reshape(M, K)
    y = torch.empty((M, N), dtype=torch.float32, device=DEV)
    ctx.ternary_linear_blocked(w, dev_f32(sc), bs, dev_f32(x), y)
    torch.cuda.synchronize()
    ref = oracle.ternary_matmul_blocked(t, sc, bs, x, N, K, M).reshape(M, N)
    np.testing.assert_array_equal(host(y), ref)
    # random scales and bf16 activations
    sc = rng.uniform(0.01, 0.05, size=nb).astype(np.float32)
    xf, xb = synth.activations(f"blocked/{M}x{K}x{N}", "x", M, K)
    y = torch.empty((M, N), dtype=torch.float32, device=DEV)
    ctx.ternary_linear_blocked(w, dev_f32(sc), bs, dev_bf16(xb), y)
    torch.cuda.synchronize()
    ref = oracle.ternary_matmul_blocked(t, sc, bs, synth.bf16_bits_to_f32(xb), N, K, M).reshape(M, N)
    assert_close_f32(host(y), ref)


@pytest.mark.parametrize("M,K,N", [(1, 4096, 300), (4, 1000, 77), (1, 16, 3)])
@pytest.mark.parametrize("xt", ["f32", "bf16"])
def test_index_list_decode(ctx, M, K, N, xt):
    rng = np.random.default_rng(K + N)
    t = rng.integers(-1, 2, size=(N, K)).astype(np.int8)
    t[0, :] = 0  # an empty row: both lists empty
    po, pi, no, ni = frx.ternary_sparse_indices(t)
    d = [dev_u32(a) for a in (po, pi, no, ni)]
    if xt == "f32":
        x = _dyadic(rng, M * K).reshape(M, K)
        xd = dev_f32(x)
    else:
        xf, xb = synth.activations(f"idx/{K}x{N}", "x", M, K)
        x, xd = synth.bf16_bits_to_f32(xb), dev_bf16(xb)
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device=DEV)
    ctx.ternary_sparse_decode(*d, 0.5, xd, y)
    torch.cuda.synchronize()
    ref = np.stack([oracle.ternary_matmul_sparse_decode(po, pi[:po[-1]], no, ni[:no[-1]], 0.5, x[m], N)
                    for m in range(M)])
    if xt == "f32":
        np.testing.assert_array_equal(host(y), ref)
    else:
        assert_close_f32(host(y), ref)
    assert (host(y)[:, 0] == 0).all()


@pytest.mark.parametrize("N,K", [(11008, 4096), (3, 16), (257, 1040)])
def test_stats_counts(ctx, N, K):
    t = np.random.default_rng(N).integers(-1, 2, size=(N, K)).astype(np.int8)
    words = oracle.pack_rows_u32(t)
    if N == 3:  # code 3 (never packed) counts as zero, as TERNARY_DECODE
        words[0, 0] = 0xFFFFFFFF
        t[0, :16] = 0
    counts = torch.zeros(3, dtype=torch.int64, device=DEV)
    ctx.ternary_stats(dev_u32(words), K, counts)
    torch.cuda.synchronize()
    ref, ratios, _ = oracle.ternary_stats(t)
    np.testing.assert_array_equal(counts.cpu().numpy().astype(np.uint64), ref)


def test_variant_shape_errors(ctx):
    w = dev_u32(np.zeros((4, 1), np.uint32))
    with pytest.raises(frx.FrxError) as e:
        ctx.ternary_linear_blocked(w, dev_f32(np.ones(1, np.float32)), 0, dev_f32(np.ones((1, 16), np.float32)),
                                   torch.empty((1, 4), dtype=torch.float32, device=DEV))
    assert e.value.kind == "Shape"
    with pytest.raises(frx.FrxError) as e:
        ctx.ternary_stats(dev_u32(np.zeros(4, np.uint32)), 20, torch.zeros(3, dtype=torch.int64, device=DEV))
    assert e.value.kind == "Shape"


def _linear_from_u8(ctx, packed_u8, N, K, alpha, x, xt):
    """The reference's u8 packing (pack_ternary, ternary.rs:146-163) as
    uploaded by the drop-in: repacked to u32 words (ternary.rs:1317-1328,
    row-aligned for K % 16 == 0) and one scale broadcast over the rows."""
    w = frx.repack_u8_to_u32(packed_u8, N * K).reshape(N, K // 16)
    M = x.shape[0]
    xd = dev_bf16(synth.f32_to_bf16_bits(x)) if xt == "bf16" else dev_f32(x)
    y = torch.empty((M, N), dtype=torch.float32, device=DEV)
    ctx.ternary_linear(dev_u32(w), dev_f32(np.full(N, alpha, np.float32)), xd, y)
    torch.cuda.synchronize()
    return host(y)


@pytest.mark.parametrize("form,M,K,N", [("decode", 1, 4096, 11008), ("decode", 1, 2048, 2048),
                                        ("packed", 4, 1024, 300), ("packed", 16, 2048, 512),
                                        ("packed", 40, 4096, 256), ("packed_parallel", 1, 11008, 4096),
                                        ("packed_parallel", 1, 4096, 1000)])
def test_reference_cpu_matmul_forms(ctx, form, M, K, N):
    """ternary_matmul_decode (ternary.rs:591-633), ternary_matmul_packed
    (:401-464) and ternary_matmul_packed_parallel (:471-539) on the GPU: the
    same u8-packed weights and alpha through frx_ternary_linear. Dyadic
    activations and a power-of-two alpha: bit for bit; normal f32 and bf16
    activations: within 1e-3."""
    rng = np.random.default_rng(hash((form, M, K, N)) % 2 ** 32)
    t = rng.integers(-1, 2, size=(N, K)).astype(np.int8)
    pk = oracle.pack_ternary(t)

    def ref(x, alpha):
        if form == "decode":
            return oracle.ternary_matmul_decode(t, alpha, x[0], N, K)[None, :]
        if form == "packed":
            return oracle.ternary_matmul_packed(pk, alpha, x, N, K, M).reshape(M, N)
        return oracle.ternary_matmul_packed_parallel(pk, alpha, x[0], N, K)[None, :]

    xd = _dyadic(rng, M * K).reshape(M, K)
    for xt in ("bf16", "f32"):
        np.testing.assert_array_equal(_linear_from_u8(ctx, pk, N, K, 0.25, xd, xt), ref(xd, 0.25))
    xn = synth.normal(synth.seed_of(f"forms/{form}/{M}x{K}x{N}", "x"), M * K).reshape(M, K).astype(np.float32)
    assert_close_f32(_linear_from_u8(ctx, pk, N, K, 0.0371, xn, "f32"), ref(xn, np.float32(0.0371)))
    xb = synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(xn))
    assert_close_f32(_linear_from_u8(ctx, pk, N, K, 0.0371, xb, "bf16"), ref(xb, np.float32(0.0371)))
