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


@pytest.mark.parametrize("M,H,I", [(1, 64, 96), (3, 128, 48), (7, 96, 272), (9, 272, 208),
                                   (16, 256, 160), (17, 64, 96), (40, 128, 256)])
@pytest.mark.parametrize("act", [frx.ACT_SILU, frx.ACT_GELU_TANH])
def test_ffn_small_parity(ctx, M, H, I, act):
    xf, xb, mats = make_ffn(f"ffn/s{M}_{H}_{I}", M, H, I)
    xw = synth.bf16_bits_to_f32(xb)
    y = run_ffn(ctx, xf, xb, mats, act)
    assert_close_f32(host(y), ref_ffn(xw, mats, act == frx.ACT_GELU_TANH))


@pytest.mark.parametrize("H,I", [(64, 64), (1024, 2816), (2048, 5632), (128, 16384), (16384, 128),
                                 (4160, 8256), (4096, 11008), (12352, 8256)])
@pytest.mark.parametrize("act", [frx.ACT_SILU, frx.ACT_GELU_TANH])
def test_ffn_single_token_rows(ctx, H, I, act):
    """One bf16 token in the default mode: gate/up/act by whole rows into bf16
    hi/lo planes of h, then the down rows over both planes (H and I multiples
    of 64 up to 16384: one to four 4096-column windows on either side; the
    down launch at I = 16384 holds 74 KB of LDS)."""
    xf, xb, mats = make_ffn(f"ffn/rows{H}_{I}", 1, H, I)
    xw = synth.bf16_bits_to_f32(xb)
    ref = ref_ffn(xw, mats, act == frx.ACT_GELU_TANH)
    assert_close_f32(host(run_ffn(ctx, xf, xb, mats, act)), ref)
    yb = run_ffn(ctx, xf, xb, mats, act, yt="bf16")
    assert_bf16_within_1ulp(yb.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("H,I", [(64, 64), (1024, 2816), (4096, 11008), (128, 14336), (14336, 128),
                                 (2112, 4160)])
@pytest.mark.parametrize("act", [frx.ACT_SILU, frx.ACT_GELU_TANH])
def test_ffn_two_tokens_rows(ctx, H, I, act):
    """Two bf16 tokens in the default mode: gate/up/act in the 4-segment
    kernel into bf16 hi/lo planes of h, then the down launch with the two
    tokens' hi and lo planes as its four token columns (H and I multiples of
    64 up to 14336: one to fourteen 1024-column windows, split over two
    waves above one)."""
    xf, xb, mats = make_ffn(f"ffn/rows2_{H}_{I}", 2, H, I)
    xw = synth.bf16_bits_to_f32(xb)
    ref = ref_ffn(xw, mats, act == frx.ACT_GELU_TANH)
    assert_close_f32(host(run_ffn(ctx, xf, xb, mats, act)), ref)
    yb = run_ffn(ctx, xf, xb, mats, act, yt="bf16")
    assert_bf16_within_1ulp(yb.view(torch.int16).cpu().numpy().view(np.uint16), ref)


def test_ffn_single_token_rows_matches_one_launch(ctx):
    """The rows path (default at M = 1) and the one-launch kernel agree to
    fp32 rounding (different summation orders)."""
    xf, xb, mats = make_ffn("ffn/rows_vs_one", 1, 4096, 11008)
    y_rows = host(run_ffn(ctx, xf, xb, mats, frx.ACT_SILU))
    ctx.set_ffn_mode(frx.FFN_ONE_LAUNCH)
    try:
        y_one = host(run_ffn(ctx, xf, xb, mats, frx.ACT_SILU))
        ctx.synchronize()
    finally:
        ctx.set_ffn_mode(frx.FFN_AUTO)
    rms = float(np.sqrt(np.mean(y_one.astype(np.float64) ** 2)))
    assert np.max(np.abs(y_rows - y_one)) <= 1e-4 * rms


@pytest.mark.parametrize("M", [3, 4, 5, 7, 8, 16])
@pytest.mark.parametrize("H,I", [(4096, 11008), (2112, 4160), (320, 1088)])
def test_ffn_bf16_in_bf16_out_3_to_16_tokens(ctx, M, H, I):
    """bf16 x and bf16 y at 3-16 tokens (the dense FFN branch,
    cpu_block_attn_res.rs:2317-2326): the gate/up/act launch writing h as
    bf16 hi/lo planes (the 4-segment kernel at 3-4 tokens, operand-load and
    staged kernels above) and the down GEMV over both planes with a bf16
    epilogue (split-K at I >= 8192, whole-K below), at LLaMA-7B and ragged
    shapes; within 1 bf16 ulp of bf16(reference), and the f32 output within
    1e-3."""
    xf, xb, mats = make_ffn(f"ffn/bf16out{M}_{H}_{I}", M, H, I)
    xw = synth.bf16_bits_to_f32(xb)
    ref = ref_ffn(xw, mats, False)
    yb = run_ffn(ctx, xf, xb, mats, frx.ACT_SILU, yt="bf16")
    assert_bf16_within_1ulp(yb.view(torch.int16).cpu().numpy().view(np.uint16), ref)
    assert_close_f32(host(run_ffn(ctx, xf, xb, mats, frx.ACT_SILU)), ref)


@pytest.mark.parametrize("H,I", [(1024, 16448), (2048, 28672), (16384, 20480)])
@pytest.mark.parametrize("act", [frx.ACT_SILU, frx.ACT_GELU_TANH])
def test_ffn_single_token_long_intermediate(ctx, H, I, act):
    """One bf16 token with an intermediate longer than 16384 (LLaMA-70B:
    I = 28672): gate/up/act into h's bf16 hi/lo planes (rows kernel), then
    the split-K down launch over both planes; f32 and bf16 outputs against
    the reference FFN."""
    xf, xb, mats = make_ffn(f"ffn/long{H}_{I}", 1, H, I)
    xw = synth.bf16_bits_to_f32(xb)
    ref = ref_ffn(xw, mats, act == frx.ACT_GELU_TANH)
    assert_close_f32(host(run_ffn(ctx, xf, xb, mats, act)), ref)
    yb = run_ffn(ctx, xf, xb, mats, act, yt="bf16")
    assert_bf16_within_1ulp(yb.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("M,H,I", [(17, 1024, 2816), (40, 4096, 11008), (300, 512, 1344)])
@pytest.mark.parametrize("xt", ["bf16", "f32"])
def test_ffn_prefill_tokens(ctx, M, H, I, xt):
    """Above 16 tokens: gate and up as linears (split over K where the tiles
    leave compute units idle), the activation product in fp32, h as bf16
    hi | lo rows and the down projection over both halves; bf16 output within
    1 ulp, f32 within 1e-3 of the reference FFN."""
    xf, xb, mats = make_ffn(f"ffn/prefill{M}_{H}_{I}", M, H, I)
    xin = synth.bf16_bits_to_f32(xb) if xt == "bf16" else xf
    ref = ref_ffn(xin, mats, False)
    assert_close_f32(host(run_ffn(ctx, xf, xb, mats, frx.ACT_SILU, xt=xt)), ref)
    yb = run_ffn(ctx, xf, xb, mats, frx.ACT_SILU, xt=xt, yt="bf16")
    assert_bf16_within_1ulp(yb.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("M", [2, 24])
def test_ffn_f32_in_bf16_out(ctx, M):
    xf, xb, mats = make_ffn(f"ffn/f32_{M}", M, 128, 208)
    y = run_ffn(ctx, xf, xb, mats, frx.ACT_SILU, xt="f32", yt="bf16")
    ref = ref_ffn(xf, mats, False)
    assert_bf16_within_1ulp(y.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("M,H,I", [(1, 4096, 11008), (4, 256, 96), (12, 272, 208), (33, 128, 160)])
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
    """Where h stays fp32 (three tokens, two-launch mode) the fused path
    equals glu followed by the fp32-input linear bit for bit."""
    M, H, I = 3, 256, 320
    xf, xb, mats = make_ffn("ffn/comp", M, H, I)
    d = {k: (dev_u32(v[0]), dev_f32(v[1])) for k, v in mats.items()}
    x = dev_bf16(xb)
    y = torch.empty((M, H), dtype=torch.float32, device=DEV)
    ctx.set_ffn_mode(frx.FFN_TWO_LAUNCH)
    try:
        ctx.ternary_ffn(x, d["gate"][0], d["gate"][1], d["up"][0], d["up"][1], d["down"][0], d["down"][1], y)
    finally:
        ctx.set_ffn_mode(frx.FFN_AUTO)
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


# ---- one-launch decode FFN (M <= 3) -------------------------------------------

@pytest.fixture
def one_launch(ctx):
    ctx.set_ffn_mode(frx.FFN_ONE_LAUNCH)  # fails the call instead of falling back
    yield ctx
    ctx.set_ffn_mode(frx.FFN_AUTO)


@pytest.mark.parametrize("M", [1, 2, 3])
@pytest.mark.parametrize("act", [frx.ACT_SILU, frx.ACT_GELU_TANH])
def test_ffn_one_launch_llama7b(one_launch, M, act):
    ctx = one_launch
    xf, xb, mats = make_ffn(f"ffn1/dec{M}", M, 4096, 11008)
    xw = synth.bf16_bits_to_f32(xb)
    ref = ref_ffn(xw, mats, act == frx.ACT_GELU_TANH)
    y = run_ffn(ctx, xf, xb, mats, act)
    ctx.synchronize()  # raises if the grid barrier timed out
    assert_close_f32(host(y), ref)
    yb = run_ffn(ctx, xf, xb, mats, act, yt="bf16")
    ctx.synchronize()
    assert_bf16_within_1ulp(yb.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("M,H,I", [(1, 64, 64), (2, 128, 192), (3, 256, 320), (1, 4096, 64),
                                   (3, 64, 11008), (2, 1024, 2816), (1, 2048, 5632), (3, 4032, 11520)])
def test_ffn_one_launch_shapes(one_launch, M, H, I):
    ctx = one_launch
    xf, xb, mats = make_ffn(f"ffn1/s{M}_{H}_{I}", M, H, I)
    xw = synth.bf16_bits_to_f32(xb)
    y = run_ffn(ctx, xf, xb, mats, frx.ACT_SILU)
    ctx.synchronize()
    assert_close_f32(host(y), ref_ffn(xw, mats, False))


@pytest.mark.parametrize("M", [1, 3])
def test_ffn_one_launch_f32_in(one_launch, M):
    ctx = one_launch
    xf, xb, mats = make_ffn(f"ffn1/f32_{M}", M, 512, 1344)
    y = run_ffn(ctx, xf, xb, mats, frx.ACT_GELU_TANH, xt="f32", yt="f32")
    ctx.synchronize()
    assert_close_f32(host(y), ref_ffn(xf, mats, True))


def test_ffn_one_launch_matches_two_launch(ctx):
    """Both executions of the decode FFN agree (different summation orders,
    so within fp32 rounding, not bit for bit)."""
    xf, xb, mats = make_ffn("ffn1/both", 2, 4096, 11008)
    ctx.set_ffn_mode(frx.FFN_TWO_LAUNCH)
    try:
        y2 = run_ffn(ctx, xf, xb, mats, frx.ACT_SILU)
    finally:
        ctx.set_ffn_mode(frx.FFN_AUTO)
    ctx.set_ffn_mode(frx.FFN_ONE_LAUNCH)
    try:
        y1 = run_ffn(ctx, xf, xb, mats, frx.ACT_SILU)
    finally:
        ctx.set_ffn_mode(frx.FFN_AUTO)
    ctx.synchronize()
    a, b = host(y1), host(y2)
    assert np.max(np.abs(a - b)) <= 1e-4 * max(1e-30, float(np.sqrt(np.mean(b.astype(np.float64) ** 2))))


def test_ffn_one_launch_repeat_and_graph(one_launch):
    """Back-to-back launches (the barrier epoch advances every launch) and
    replays of a captured launch, each checked, with eager work between."""
    ctx = one_launch
    M, H, I = 1, 1024, 2816
    cases = [make_ffn(f"ffn1/rep{i}", M, H, I) for i in range(3)]
    refs = [ref_ffn(synth.bf16_bits_to_f32(xb), mats, False) for _, xb, mats in cases]
    dev = [({k: (dev_u32(v[0]), dev_f32(v[1])) for k, v in mats.items()}, dev_bf16(xb)) for _, xb, mats in cases]
    ys = [torch.empty((M, H), dtype=torch.float32, device=DEV) for _ in cases]

    def call(i):
        d, x = dev[i]
        ctx.ternary_ffn(x, d["gate"][0], d["gate"][1], d["up"][0], d["up"][1], d["down"][0], d["down"][1], ys[i])

    for rep in range(40):
        call(rep % 3)
    ctx.synchronize()
    for i in range(3):
        assert_close_f32(host(ys[i]), refs[i])

    s = torch.cuda.Stream()
    ctx.set_stream(s)
    try:
        with torch.cuda.stream(s):
            call(0)  # workspace and barrier words exist before capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            call(1)
        torch.cuda.synchronize()
        for rep in range(4):
            ys[1].fill_(float("nan"))
            with torch.cuda.stream(s):
                g.replay()
                call(2)  # an eager launch between replays
            torch.cuda.synchronize()
            ctx.synchronize()
            assert_close_f32(host(ys[1]), refs[1])
            assert_close_f32(host(ys[2]), refs[2])
    finally:
        ctx.set_stream(None)


def test_ffn_one_launch_unsupported(one_launch):
    ctx = one_launch
    xf, xb, mats = make_ffn("ffn1/unsup", 4, 128, 192)  # M = 4 > 3
    d = {k: (dev_u32(v[0]), dev_f32(v[1])) for k, v in mats.items()}
    y = torch.empty((4, 128), dtype=torch.float32, device=DEV)
    with pytest.raises(frx.FrxError) as ei:
        ctx.ternary_ffn(dev_bf16(xb), d["gate"][0], d["gate"][1], d["up"][0], d["up"][1], d["down"][0],
                        d["down"][1], y)
    assert ei.value.kind == "Unsupported"
