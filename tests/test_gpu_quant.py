"""On-device ternary quantisation (frx_quantize_ternary) against the CPU
oracle: quantize_ternary (src/model/ternary.rs:31-57) and the on-the-fly
rule of BitLinear::forward_ste (src/training/shadow_weights.rs:203-231),
applied to each row. Scales and codes must be bit-identical (the sum of
|w| runs left to right in f32 on both sides); packed words must equal
pack_ternary followed by pack_ternary_u32 of the oracle's codes."""
import numpy as np
import pytest
import torch

import ferrisres_amd as frx
import oracle
from ferrisres_amd import synth
from _gpu import dev_bf16, dev_f32, host

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
RULES = {frx.QUANT_ABSMEAN: oracle.quantize_ternary, frx.QUANT_STE: oracle.quantize_ste}


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "GPU tests need a gfx950 device"
    c = frx.Context(0)
    yield c
    c.close()


def _quantize(ctx, w_dev, rule):
    N, K = w_dev.shape
    packed = torch.full((N, K // 16), -1, dtype=torch.int32, device=DEV)
    scale = torch.full((N,), float("nan"), dtype=torch.float32, device=DEV)
    ctx.quantize_ternary(w_dev, rule, packed, scale)
    torch.cuda.synchronize()
    return packed.cpu().numpy().view(np.uint32), host(scale)


def _codes(packed):
    shifts = 2 * np.arange(16, dtype=np.uint32)
    c = (packed[..., None] >> shifts) & 3
    return c.reshape(packed.shape[0], -1).astype(np.int8) - 1


def _check_rows(w_f32, packed, scale, rule):
    for r in range(w_f32.shape[0]):
        q, a = RULES[rule](w_f32[r])
        assert np.array_equal(np.float32(scale[r]).view(np.uint32), np.float32(a).view(np.uint32)) or (
            np.isnan(scale[r]) and np.isnan(a)), f"row {r}: scale {scale[r]!r} vs {a!r}"
        np.testing.assert_array_equal(_codes(packed[r:r + 1])[0], q, err_msg=f"row {r}")


@pytest.mark.parametrize("N,K", [(1, 16), (7, 64), (300, 4096), (33, 11008), (5, 2048 + 16)])
@pytest.mark.parametrize("rule", [frx.QUANT_ABSMEAN, frx.QUANT_STE])
@pytest.mark.parametrize("wt", ["f32", "bf16"])
def test_quantize_rows_match_oracle(ctx, N, K, rule, wt):
    w = synth.normal(synth.seed_of(f"quant/{N}x{K}", "w"), N * K, std=0.02).reshape(N, K)
    if wt == "bf16":
        bits = synth.f32_to_bf16_bits(w)
        w_f32, w_dev = synth.bf16_bits_to_f32(bits), dev_bf16(bits)
    else:
        w_f32, w_dev = w.astype(np.float32), dev_f32(w)
    packed, scale = _quantize(ctx, w_dev, rule)
    _check_rows(w_f32, packed, scale, rule)


@pytest.mark.parametrize("rule", [frx.QUANT_ABSMEAN, frx.QUANT_STE])
def test_quantize_special_rows(ctx, rule):
    """All-zero, negative-zero, tiny, huge (sum overflows to inf), NaN and
    inf rows, the +-0.5 boundaries of both rules, a constant row."""
    K = 64
    norm = np.float32(0.7978845608)
    rows = np.zeros((10, K), np.float32)
    rows[1] = -0.0
    rows[2] = 1e-12
    rows[3] = 3e38
    rows[4] = np.linspace(-1, 1, K)
    rows[4, 7] = np.nan
    rows[5] = np.linspace(-1, 1, K)
    rows[5, 9] = np.inf
    rows[6, :4] = [0.5, -0.5, 1.5, -1.5]  # STE: alpha = 4/64
    rows[7, :4] = [0.5, -0.5, 1.5, np.float32(4) * norm - np.float32(2.5)]
    rows[7] *= np.float32(16)  # quantize_ternary: alpha = 16 * 4 * norm / 64 / norm = 1
    rows[8] = -0.125
    rows[9] = np.linspace(-3, 3, K)
    packed, scale = _quantize(ctx, dev_f32(rows), rule)
    _check_rows(rows, packed, scale, rule)


def test_quantize_whole_tensor_matches_reference_packing(ctx):
    """N = 1 with K = n is the reference's call on a whole tensor: one alpha
    and the flat packing of pack_ternary + pack_ternary_u32."""
    n = 65536
    w = synth.normal(synth.seed_of("quant/flat", "w"), n, std=1.0).astype(np.float32)
    packed, scale = _quantize(ctx, dev_f32(w.reshape(1, n)), frx.QUANT_ABSMEAN)
    q, a = oracle.quantize_ternary(w)
    assert np.float32(scale[0]).view(np.uint32) == np.float32(a).view(np.uint32)
    ref_words = oracle.pack_ternary_u32(oracle.pack_ternary(q), n)
    np.testing.assert_array_equal(packed.reshape(-1), ref_words)


def test_quantized_weights_feed_the_linear(ctx):
    """Quantise on the device, then run frx_ternary_linear on the result:
    equals the oracle matmul of the oracle's codes and scales."""
    N, K, M = 96, 1024, 3
    w = synth.normal(synth.seed_of("quant/chain", "w"), N * K, std=0.02).reshape(N, K)
    packed = torch.empty((N, K // 16), dtype=torch.int32, device=DEV)
    scale = torch.empty((N,), dtype=torch.float32, device=DEV)
    ctx.quantize_ternary(dev_f32(w), frx.QUANT_ABSMEAN, packed, scale)
    xf, xb = synth.activations("quant/chain", "x", M, K)
    y = torch.empty((M, N), dtype=torch.float32, device=DEV)
    ctx.ternary_linear(packed, scale, dev_bf16(xb), y)
    torch.cuda.synchronize()
    codes = np.stack([oracle.quantize_ternary(w[r].astype(np.float32))[0] for r in range(N)])
    scales = np.array([oracle.quantize_ternary(w[r].astype(np.float32))[1] for r in range(N)], np.float32)
    ref = oracle.ternary_matmul_u32(synth.pack_rows_u32(codes), scales, xf, M, K, N)
    from _gpu import assert_close_f32
    assert_close_f32(host(y), ref)


def test_quantize_shape_errors(ctx):
    w = dev_f32(np.zeros((4, 40), np.float32))  # K = 40 is not a multiple of 16
    packed = torch.empty((4, 3), dtype=torch.int32, device=DEV)
    scale = torch.empty((4,), dtype=torch.float32, device=DEV)
    with pytest.raises(frx.FrxError) as ei:
        ctx.quantize_ternary(w, frx.QUANT_ABSMEAN, packed, scale)
    assert ei.value.kind == "Shape"


# ---- quantize_ternary_blocked / dequantize_ternary_blocked ------------------

@pytest.mark.parametrize("n,block", [(512, 64), (1000, 64), (37, 8), (4096, 4096), (45056, 1000),
                                     (11008 * 16, 4096), (100, 128), (17, 1)])
@pytest.mark.parametrize("wt", ["f32", "bf16"])
def test_quantize_blocked_matches_oracle(ctx, n, block, wt):
    """frx_quantize_ternary_blocked = quantize_ternary_blocked
    (ternary.rs:76-110): scales bit-identical, packed words equal to
    pack_ternary + pack_ternary_u32 of the oracle's codes (zero padding past
    n), ragged last blocks included; the device dequantise equals the
    oracle's dequantize_ternary_blocked bit for bit."""
    rng = np.random.default_rng(n + block)
    w = (rng.standard_normal(n) * np.where(np.arange(n) % 700 < 350, 0.02, 1.0)).astype(np.float32)
    w[::29] = 0.0
    if wt == "bf16":
        bits = synth.f32_to_bf16_bits(w)
        w, w_dev = synth.bf16_bits_to_f32(bits), dev_bf16(bits)
    else:
        w_dev = dev_f32(w)
    q, sc = oracle.quantize_ternary_blocked(w, block)
    packed = torch.full((-(-n // 16),), -1, dtype=torch.int32, device=DEV)
    scales = torch.full((sc.size,), float("nan"), dtype=torch.float32, device=DEV)
    ctx.quantize_ternary_blocked(w_dev, block, packed, scales)
    out = torch.full((n,), float("nan"), dtype=torch.float32, device=DEV)
    ctx.dequantize_ternary_blocked(packed, scales, n, block, out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(scales).view(np.uint32), sc.view(np.uint32))
    ref_words = oracle.pack_ternary_u32(oracle.pack_ternary(q), n)
    np.testing.assert_array_equal(packed.cpu().numpy().view(np.uint32), ref_words)
    deq = oracle.dequantize_ternary_blocked(q, sc, block)
    np.testing.assert_array_equal(host(out).view(np.uint32), deq.view(np.uint32))


def test_quantize_blocked_equals_row_view(ctx):
    """With block_size % 16 == 0 dividing n, the blocked call is
    frx_quantize_ternary on the [n/block][block] view, word for word."""
    n, block = 64 * 4096, 4096
    w = synth.normal(synth.seed_of("quant/blocked_view", "w"), n, std=0.02)
    w_dev = dev_f32(w)
    packed = torch.zeros((n // 16,), dtype=torch.int32, device=DEV)
    scales = torch.zeros((n // block,), dtype=torch.float32, device=DEV)
    ctx.quantize_ternary_blocked(w_dev, block, packed, scales)
    p2, s2 = _quantize(ctx, w_dev.view(n // block, block), frx.QUANT_ABSMEAN)
    np.testing.assert_array_equal(packed.cpu().numpy().view(np.uint32), p2.ravel())
    np.testing.assert_array_equal(host(scales), s2)


# ---- prune_fp32_to_sparse_ternary -----------------------------------------------

def _prune_dev(ctx, w_dev, per_row=False):
    N, K = w_dev.shape
    ng = N * K // 4
    pats = torch.full(((ng + 1) // 2,), 0xEE, dtype=torch.uint8, device=DEV)
    signs = torch.full(((ng + 3) // 4,), 0xEE, dtype=torch.uint8, device=DEV)
    meta = torch.full((N, -(-(K // 4) // 6)), -1, dtype=torch.int32, device=DEV)
    scale = torch.full((N,), float("nan"), dtype=torch.float32, device=DEV)
    ctx.prune_sparse24(w_dev, scale, pats, signs, meta, per_row=per_row)
    torch.cuda.synchronize()
    return pats.cpu().numpy(), signs.cpu().numpy(), meta.cpu().numpy().view(np.uint32), host(scale)


@pytest.mark.parametrize("N,K", [(2, 4), (1, 12), (3, 20), (64, 256), (257, 4096), (5, 2052)])
@pytest.mark.parametrize("wt", ["f32", "bf16"])
def test_prune_sparse24_matches_oracle(ctx, N, K, wt):
    """frx_prune_sparse24 = prune_fp32_to_sparse_ternary
    (sparse_ternary.rs:598-663): CPU-layout patterns and signs bit-exact
    (odd group counts share no byte between threads), the GPU layout equal
    to the transcoder's output of the oracle's CPU layout, and the tensor
    scale bit-identical on every row. Ties, zeros and mixed-sign groups are
    forced into the input."""
    rng = np.random.default_rng(N * 7 + K)
    w = rng.standard_normal(N * K).astype(np.float32) * 0.05
    w[rng.random(w.size) < 0.1] = 0.0
    t = rng.random(w.size) < 0.1
    w[t] = np.float32(0.03) * np.sign(rng.standard_normal(t.sum())).astype(np.float32)
    if wt == "bf16":
        bits = synth.f32_to_bf16_bits(w)
        w, w_dev = synth.bf16_bits_to_f32(bits), dev_bf16(bits.reshape(N, K))
    else:
        w_dev = dev_f32(w.reshape(N, K))
    pats, signs, meta, scale = _prune_dev(ctx, w_dev)
    rp, rs, rsc = oracle.prune_sparse24(w, N, K)
    np.testing.assert_array_equal(pats, rp)
    np.testing.assert_array_equal(signs, rs)
    np.testing.assert_array_equal(meta.ravel(), frx.sparse24_cpu_to_gpu(rp, rs, N, K).ravel())
    assert (scale.view(np.uint32) == np.float32(rsc).view(np.uint32)).all()
    # per-row scales: each row as its own tensor
    _, _, meta_r, scale_r = _prune_dev(ctx, w_dev, per_row=True)
    np.testing.assert_array_equal(meta_r, meta)
    for r in range(N):
        assert scale_r[r].view(np.uint32) == np.float32(oracle.prune_sparse24(w[r * K:(r + 1) * K], 1, K)[2]).view(
            np.uint32)


def test_prune_sparse24_kat_and_matmul(ctx):
    """The reference's KAT (sparse_ternary.rs:523-544) through the device
    prune, and the pruned 2:4 matrix multiplied on the GPU equals the oracle's
    2:4 matmul of the same pruned matrix (the producer feeds the kernels)."""
    import json
    import os
    kat = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))["prune_fp32"]
    w = np.array(kat["weights"], np.float32)
    pats, signs, meta, scale = _prune_dev(ctx, dev_f32(w.reshape(kat["rows"], kat["cols"])))
    dec = oracle.sparse24_cpu_to_ternary(pats, signs, kat["rows"], kat["cols"])
    np.testing.assert_array_equal(dec, kat["expected_decompressed"])
    N, K, M = 256, 1024, 8
    wf = synth.normal(synth.seed_of("prune/mm", "w"), N * K, std=0.02).reshape(N, K)
    pats, signs, meta, scale = _prune_dev(ctx, dev_f32(wf), per_row=True)
    xf, xb = synth.activations("prune/mm", "x", M, K)
    y = torch.empty((M, N), dtype=torch.float32, device=DEV)
    from _gpu import dev_u32, assert_close_f32
    ctx.sparse24_ternary_linear(dev_u32(meta), dev_f32(scale), dev_bf16(xb), y)
    torch.cuda.synchronize()
    ref = oracle.sparse24_gpu_matmul(meta, scale, xf, M, K, N)
    assert_close_f32(host(y), np.asarray(ref).reshape(M, N))
