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
