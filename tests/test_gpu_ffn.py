"""Dense ternary FFN (gate/up/activation/down) and its gated first half on
the GPU against the oracle (dense FFN branch of cpu_block_attn_res.rs:
2317-2326 with per-row scales). Outputs within 1e-3; the decode path
(M <= 16: fused gate/up launch + fp32-input down GEMV) and the GEMM path
(M > 16) at the LLaMA-7B FFN shape and small ragged shapes."""
import numpy as np
import pytest
import torch

import ferrisres_amd as frx
import oracle
from ferrisres_amd import synth
from _gpu import DEV, assert_bf16_within_1ulp, assert_close_f32, dev_bf16, dev_f32, dev_u32, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "GPU tests need a gfx950 device"
    c = frx.Context(0)
    yield c
    c.close()


def make_ffn(name, M, H, I):
    xf, xb = synth.activations(name, "x", M, H)
    mats = {}
    for mat, (n, k) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
        t = synth.ternary_uniform(name, mat, n, k)
        mats[mat] = (synth.pack_rows_u32(t), synth.row_scales(name, "s" + mat, n, samples=256))
    return xf, xb, mats


def ref_ffn(xf, mats, gelu):
    return oracle.ffn_forward(xf, mats["gate"][0], mats["gate"][1], mats["up"][0], mats["up"][1],
                              mats["down"][0], mats["down"][1], gelu=gelu)


def ref_glu(xf, mats, gelu):
    g = oracle.ternary_matmul_u32(mats["gate"][0], mats["gate"][1], xf, xf.shape[0], xf.shape[1],
                                  mats["gate"][0].shape[0])
    u = oracle.ternary_matmul_u32(mats["up"][0], mats["up"][1], xf, xf.shape[0], xf.shape[1],
                                  mats["up"][0].shape[0])
    g = g.reshape(xf.shape[0], -1).astype(np.float32)
    u = u.reshape(xf.shape[0], -1).astype(np.float32)
    a = np.array([oracle.gelu_tanh(v) for v in g.ravel()], np.float32).reshape(g.shape) if gelu \
        else (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32)
    return a * u


def run_ffn(ctx, xf, xb, mats, act, xt="bf16", yt="f32"):
    M, H = xf.shape
    d = {k: (dev_u32(v[0]), dev_f32(v[1])) for k, v in mats.items()}
    x = dev_bf16(xb) if xt == "bf16" else dev_f32(xf)
    y = torch.empty((M, H), dtype=torch.float32 if yt == "f32" else torch.bfloat16, device=DEV)
    ctx.ternary_ffn(x, d["gate"][0], d["gate"][1], d["up"][0], d["up"][1], d["down"][0], d["down"][1], y, act=act)
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("M", [1, 4, 16])
def test_ffn_decode_llama7b_shape(ctx, M):
    xf, xb, mats = make_ffn(f"ffn/dec{M}", M, 4096, 11008)
    xw = synth.bf16_bits_to_f32(xb)  # the oracle consumes the bf16 inputs widened
    y = run_ffn(ctx, xf, xb, mats, frx.ACT_SILU)
    assert_close_f32(host(y), ref_ffn(xw, mats, False))


@pytest.mark.parametrize("M,H,I", [(1, 64, 96), (3, 128, 48), (7, 96, 272), (16, 256, 160),
                                   (17, 64, 96), (40, 128, 256)])
@pytest.mark.parametrize("act", [frx.ACT_SILU, frx.ACT_GELU_TANH])
def test_ffn_small_parity(ctx, M, H, I, act):
    xf, xb, mats = make_ffn(f"ffn/s{M}_{H}_{I}", M, H, I)
    xw = synth.bf16_bits_to_f32(xb)
    y = run_ffn(ctx, xf, xb, mats, act)
    assert_close_f32(host(y), ref_ffn(xw, mats, act == frx.ACT_GELU_TANH))


@pytest.mark.parametrize("M", [2, 24])
def test_ffn_f32_in_bf16_out(ctx, M):
    xf, xb, mats = make_ffn(f"ffn/f32_{M}", M, 128, 208)
    y = run_ffn(ctx, xf, xb, mats, frx.ACT_SILU, xt="f32", yt="bf16")
    ref = ref_ffn(xf, mats, False)
    assert_bf16_within_1ulp(y.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("M,H,I", [(1, 4096, 11008), (4, 256, 96), (33, 128, 160)])
@pytest.mark.parametrize("act", [frx.ACT_SILU, frx.ACT_GELU_TANH])
def test_glu_parity(ctx, M, H, I, act):
    xf, xb, mats = make_ffn(f"glu/{M}_{H}_{I}", M, H, I)
    xw = synth.bf16_bits_to_f32(xb)
    d = {k: (dev_u32(v[0]), dev_f32(v[1])) for k, v in mats.items() if k != "down"}
    h = torch.empty((M, I), dtype=torch.float32, device=DEV)
    ctx.ternary_glu(dev_bf16(xb), d["gate"][0], d["gate"][1], d["up"][0], d["up"][1], h, act=act)
    torch.cuda.synchronize()
    assert_close_f32(host(h), ref_glu(xw, mats, act == frx.ACT_GELU_TANH))


def test_ffn_equals_composition(ctx):
    """The fused path equals glu followed by the fp32-input linear."""
    M, H, I = 4, 256, 320
    xf, xb, mats = make_ffn("ffn/comp", M, H, I)
    d = {k: (dev_u32(v[0]), dev_f32(v[1])) for k, v in mats.items()}
    x = dev_bf16(xb)
    y = torch.empty((M, H), dtype=torch.float32, device=DEV)
    ctx.ternary_ffn(x, d["gate"][0], d["gate"][1], d["up"][0], d["up"][1], d["down"][0], d["down"][1], y)
    h = torch.empty((M, I), dtype=torch.float32, device=DEV)
    ctx.ternary_glu(x, d["gate"][0], d["gate"][1], d["up"][0], d["up"][1], h)
    y2 = torch.empty((M, H), dtype=torch.float32, device=DEV)
    ctx.ternary_linear(d["down"][0], d["down"][1], h, y2)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)


def test_ffn_shape_errors(ctx):
    M, H, I = 2, 64, 96
    xf, xb, mats = make_ffn("ffn/err", M, H, I)
    d = {k: (dev_u32(v[0]), dev_f32(v[1])) for k, v in mats.items()}
    x = dev_f32(np.zeros((M, 72), np.float32))  # H = 72 is not a multiple of 16
    y = torch.empty((M, 72), dtype=torch.float32, device=DEV)
    with pytest.raises(frx.FrxError) as ei:
        ctx.ternary_ffn(x, d["gate"][0], d["gate"][1], d["up"][0], d["up"][1], d["down"][0], d["down"][1], y)
    assert ei.value.kind == "Shape"
