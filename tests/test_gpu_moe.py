"""MoE ternary expert layer on the GPU against the oracle (the GPU-path MoE
glue, cpu_block_attn_res.rs:1148-1184, and TernaryMoELayer::forward,
ternary_moe.rs:145-223, with per-row scales; their GeLU experts differ:
gelu(g)*u in the glue, gelu(g) alone in TernaryMoELayer). Routing indices
must be bit-exact; outputs within 1e-3."""
import numpy as np
import pytest
import torch

import ferrisres_amd as frx
import oracle
from ferrisres_amd import synth
from _gpu import assert_bf16_within_1ulp, assert_close_f32, dev_bf16, dev_f32, dev_u32, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "GPU tests need a gfx950 device"
    c = frx.Context(0)
    yield c
    c.close()


def make_moe(name, T, H, I, E):
    xf, xb = synth.activations(name, "x", T, H)
    rf, rb = synth.activations(name, "router", E, H, std=0.02)
    ex = {}
    for e in range(E):
        for mat, (n, k) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
            t = synth.ternary_uniform(name, f"{mat}{e}", n, k)
            ex[(mat, e)] = (synth.pack_rows_u32(t), synth.row_scales(name, f"s{mat}{e}", n, samples=256))
    return xf, xb, rf, rb, ex


def run_gpu(ctx, xf, xb, rf, rb, ex, E, top_k, act, xt="bf16", yt="f32", rt=None, no_up=False):
    T, H = xf.shape
    rt = xt if rt is None else rt
    dw = {k: (dev_u32(v[0]), dev_f32(v[1])) for k, v in ex.items()}
    x = dev_bf16(xb) if xt == "bf16" else dev_f32(xf)
    r = dev_bf16(rb) if rt == "bf16" else dev_f32(rf)
    y = torch.empty((T, H), dtype=torch.float32 if yt == "f32" else torch.bfloat16, device="cuda:0")
    idx = torch.zeros((T, top_k), dtype=torch.int32, device="cuda:0")
    w = torch.zeros((T, top_k), dtype=torch.float32, device="cuda:0")
    g = lambda m, i: [dw[(m, e)][i] for e in range(E)]  # noqa: E731
    up_w, up_s = (None, None) if no_up else (g("up", 0), g("up", 1))
    ctx.moe_ternary_ffn(x, r, g("gate", 0), g("gate", 1), up_w, up_s, g("down", 0), g("down", 1),
                        y, top_k=top_k, act=act, topk_idx=idx, topk_w=w)
    torch.cuda.synchronize()
    return y, idx.cpu().numpy().astype(np.uint32), w.cpu().numpy()


def run_oracle(xf, rf, ex, E, top_k, gelu, tokens=None, routing=0):
    x = xf if tokens is None else xf[tokens]
    g = lambda m, i: [ex[(m, e)][i] for e in range(E)]  # noqa: E731
    return oracle.moe_forward(x, rf, g("gate", 0), g("gate", 1), g("up", 0), g("up", 1), g("down", 0),
                              g("down", 1), top_k, gelu, routing=routing)


@pytest.mark.parametrize("T,H,I,E,k", [(40, 128, 256, 8, 2), (7, 64, 96, 4, 1), (130, 256, 160, 16, 2),
                                       (64, 128, 128, 6, 3), (50, 320, 192, 5, 2), (300, 192, 448, 3, 2),
                                       (200, 128, 192, 2, 1), (97, 64, 128, 1, 1)])
@pytest.mark.parametrize("act", [frx.ACT_SILU, frx.ACT_GELU_TANH, frx.ACT_GELU_TANH_GATE])
def test_moe_small_parity(ctx, T, H, I, E, k, act):
    name = f"moe/{T}x{H}x{I}x{E}"
    xf, xb, rf, rb, ex = make_moe(name, T, H, I, E)
    y, idx, w = run_gpu(ctx, xf, xb, rf, rb, ex, E, k, act)
    ref, ridx, rw = run_oracle(xf, rf, ex, E, k, act)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(w, rw, rtol=0, atol=1e-6)
    assert_close_f32(host(y), ref)


@pytest.mark.parametrize("T,H,I,E,k,act,xt", [
    (1, 2048, 5632, 16, 2, frx.ACT_SILU, "bf16"), (1, 2048, 5632, 16, 2, frx.ACT_SILU, "f32"),
    (2, 128, 192, 5, 2, frx.ACT_GELU_TANH, "bf16"), (1, 256, 320, 8, 4, frx.ACT_SILU, "f32"),
    (3, 64, 128, 4, 1, frx.ACT_GELU_TANH_GATE, "bf16"), (4, 128, 64, 3, 1, frx.ACT_SILU, "f32")])
def test_moe_decode_rows_parity(ctx, T, H, I, E, k, act, xt):
    """A few routed rows (T * top_k <= 4, decode): one GEMV per routed row for
    gate/up and for down (two K parts), no grouping. Routing bit-exact,
    outputs within 1e-3, f32 and bf16 outputs."""
    name = f"moe/dec/{T}x{H}x{I}x{E}x{k}"
    xf, xb, rf, rb, ex = make_moe(name, T, H, I, E)
    if xt == "f32":
        xf = synth.normal(synth.seed_of(name, "xf32"), T * H).reshape(T, H)
    y, idx, w = run_gpu(ctx, xf, xb, rf, rb, ex, E, k, act, xt=xt, no_up=act == frx.ACT_GELU_TANH_GATE)
    ref, ridx, rw = run_oracle(xf, rf, ex, E, k, act)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(w, rw, rtol=0, atol=1e-6)
    assert_close_f32(host(y), ref)
    yb, _, _ = run_gpu(ctx, xf, xb, rf, rb, ex, E, k, act, xt=xt, yt="bf16", no_up=act == frx.ACT_GELU_TANH_GATE)
    assert_bf16_within_1ulp(yb.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("T", [1, 40])
def test_moe_unaligned_tokens_and_router(ctx, T):
    """x and the router one bf16 element into larger buffers (element-aligned,
    not 16-byte aligned): the router then runs without its LDS DMA of the
    router rows, and the experts without the pipelined engines or the decode
    GEMVs. Routing is bit-exact against the oracle and the aligned call, the
    output within 1e-3."""
    H, I, E, k = 256, 192, 8, 2
    name = f"moe/unaligned/{T}"
    xf, xb, rf, rb, ex = make_moe(name, T, H, I, E)
    y0, idx0, w0 = run_gpu(ctx, xf, xb, rf, rb, ex, E, k, frx.ACT_SILU)
    xbuf = torch.zeros(T * H + 8, dtype=torch.bfloat16, device="cuda:0")
    rbuf = torch.zeros(E * H + 8, dtype=torch.bfloat16, device="cuda:0")
    xbuf[1:1 + T * H] = dev_bf16(xb).reshape(-1)
    rbuf[1:1 + E * H] = dev_bf16(rb).reshape(-1)
    x, r = xbuf[1:1 + T * H].view(T, H), rbuf[1:1 + E * H].view(E, H)
    assert x.data_ptr() % 16 != 0 and r.data_ptr() % 16 != 0
    dw = {key: (dev_u32(v[0]), dev_f32(v[1])) for key, v in ex.items()}
    g = lambda m, i: [dw[(m, e)][i] for e in range(E)]  # noqa: E731
    y = torch.empty((T, H), dtype=torch.float32, device="cuda:0")
    idx = torch.zeros((T, k), dtype=torch.int32, device="cuda:0")
    w = torch.zeros((T, k), dtype=torch.float32, device="cuda:0")
    ctx.moe_ternary_ffn(x, r, g("gate", 0), g("gate", 1), g("up", 0), g("up", 1), g("down", 0), g("down", 1),
                        y, top_k=k, act=frx.ACT_SILU, topk_idx=idx, topk_w=w)
    torch.cuda.synchronize()
    ref, ridx, rw = run_oracle(xf, rf, ex, E, k, frx.ACT_SILU)
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.uint32), ridx)
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.uint32), idx0)
    np.testing.assert_array_equal(w.cpu().numpy(), w0)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=0, atol=1e-6)
    assert_close_f32(host(y), ref)
    assert_close_f32(host(y0), ref)


def test_moe_f32_inputs(ctx):
    xf, xb, rf, rb, ex = make_moe("moe/f32", 33, 128, 192, 5)
    xf = synth.normal(99, 33 * 128).reshape(33, 128)
    rf = synth.normal(98, 5 * 128, 0.05).reshape(5, 128)
    y, idx, w = run_gpu(ctx, xf, None, rf, None, ex, 5, 2, frx.ACT_SILU, xt="f32")
    ref, ridx, rw = run_oracle(xf, rf, ex, 5, 2, False)
    np.testing.assert_array_equal(idx, ridx)
    assert_close_f32(host(y), ref)


@pytest.mark.parametrize("xt,rt", [("f32", "bf16"), ("bf16", "f32")])
def test_moe_mixed_input_dtypes(ctx, xt, rt):
    """f32 tokens with bf16 router weights (the resident router, separate
    multiply and add) and bf16 tokens with f32 router weights (the chunked
    router); routing indices bit-exact."""
    T, H, I, E, k = 40, 256, 192, 6, 2
    xf, xb, rf, rb, ex = make_moe(f"moe/mix_{xt}_{rt}", T, H, I, E)
    if xt == "f32":
        xf, xb = synth.normal(97, T * H).reshape(T, H), None
    if rt == "f32":
        rf, rb = synth.normal(96, E * H, 0.05).reshape(E, H), None
    y, idx, w = run_gpu(ctx, xf, xb, rf, rb, ex, E, k, frx.ACT_SILU, xt=xt, rt=rt)
    ref, ridx, rw = run_oracle(xf, rf, ex, E, k, False)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(w, rw, rtol=0, atol=1e-6)
    assert_close_f32(host(y), ref)


def test_moe_config_shape(ctx):
    """512 tokens, H=2048, I=5632, 16 experts, top-2: routing for all tokens
    is checked bit-exactly, outputs for 24 sampled tokens in full."""
    T, H, I, E, k = 512, 2048, 5632, 16, 2
    xf, xb, rf, rb, ex = make_moe("moe/config", T, H, I, E)
    y, idx, w = run_gpu(ctx, xf, xb, rf, rb, ex, E, k, frx.ACT_SILU)
    ridx, rw, _ = oracle.moe_route(xf, rf, k)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(w, rw, rtol=0, atol=1e-6)
    tok = np.array([0, 1, 2, 63, 64, 100, 127, 128, 200, 255, 256, 300, 333, 400, 401, 450, 480, 500, 505,
                    508, 509, 510, 511, 17])
    ref, _, _ = run_oracle(xf, rf, ex, E, k, False, tokens=tok)
    assert_close_f32(host(y)[tok], ref)
    assert np.isfinite(host(y)).all()


@pytest.mark.parametrize("T,H,I,E,k", [(512, 2048, 5632, 16, 2), (70, 256, 320, 6, 2)])
def test_moe_f32_tokens_engine2(ctx, T, H, I, E, k):
    """Genuine f32 tokens (the reference's dtype; the lo half matters): the
    router reads them as f32 (bit-exact routing), the gate/up GEMM takes
    them as bf16 hi | lo rows in one K loop of 2H columns. Sampled tokens in
    full within 1e-3."""
    name = f"moe/f32e2/{T}x{H}"
    _, _, rf, rb, ex = make_moe(name, T, H, I, E)
    xf = synth.normal(synth.seed_of(name, "xf32"), T * H).reshape(T, H)
    y, idx, w = run_gpu(ctx, xf, None, rf, rb, ex, E, k, frx.ACT_SILU, xt="f32")
    ridx, rw, _ = oracle.moe_route(xf, rf, k)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(w, rw, rtol=0, atol=1e-6)
    tok = np.arange(T) if T <= 70 else np.array([0, 1, 63, 64, 127, 255, 256, 300, 400, 511])
    ref, _, _ = run_oracle(xf, rf, ex, E, k, False, tokens=tok)
    assert_close_f32(host(y)[tok], ref)


def test_moe_gelu_gate_only_config_shape(ctx):
    """TernaryMoELayer's GeLU experts (h = gelu_tanh(g) with the literal
    0.7978845608, no up projection; ternary_moe.rs:193-200) at 512 tokens,
    H=2048, I=5632, 16 experts, top-2, called without up matrices: routing
    for all tokens bit-exact, 16 sampled tokens in full within 1e-3."""
    T, H, I, E, k = 512, 2048, 5632, 16, 2
    xf, xb, rf, rb, ex = make_moe("moe/config", T, H, I, E)
    y, idx, w = run_gpu(ctx, xf, xb, rf, rb, ex, E, k, frx.ACT_GELU_TANH_GATE, no_up=True)
    ridx, rw, _ = oracle.moe_route(xf, rf, k)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(w, rw, rtol=0, atol=1e-6)
    tok = np.array([0, 5, 63, 64, 127, 128, 255, 256, 300, 383, 384, 447, 448, 500, 510, 511])
    g = lambda m, i: [ex[(m, e)][i] for e in range(E)]  # noqa: E731
    ref, _, _ = oracle.moe_forward(xf[tok], rf, g("gate", 0), g("gate", 1), None, None, g("down", 0),
                                   g("down", 1), k, 2)
    assert_close_f32(host(y)[tok], ref)
    # the glue's GeLU (gelu(g) * u) is a different function
    ref_glue, _, _ = run_oracle(xf, rf, ex, E, k, 1, tokens=tok[:2])
    assert np.abs(ref_glue - ref[:2]).max() > 1e-2 * np.abs(ref[:2]).max()


@pytest.mark.parametrize("T,H,I,E,k,xt", [(40, 128, 256, 8, 2, "bf16"), (33, 128, 192, 5, 2, "f32"),
                                          (50, 320, 192, 5, 2, "bf16")])
def test_moe_gelu_gate_only_without_up(ctx, T, H, I, E, k, xt):
    """FRX_ACT_GELU_TANH_GATE with the up arrays NULL equals the call with up
    matrices given (they are not read), on both grouped-GEMM engines."""
    xf, xb, rf, rb, ex = make_moe(f"moe/gate_only/{T}x{H}x{I}", T, H, I, E)
    if xt == "f32":
        xf, xb = synth.normal(95, T * H).reshape(T, H), None
    a = run_gpu(ctx, xf, xb, rf, rb, ex, E, k, frx.ACT_GELU_TANH_GATE, xt=xt, no_up=True)
    b = run_gpu(ctx, xf, xb, rf, rb, ex, E, k, frx.ACT_GELU_TANH_GATE, xt=xt)
    np.testing.assert_array_equal(host(a[0]), host(b[0]))
    ref, ridx, _ = run_oracle(xf, rf, ex, E, k, 2)
    np.testing.assert_array_equal(a[1], ridx)
    assert_close_f32(host(a[0]), ref)


def test_moe_routing_deterministic_and_repeatable(ctx):
    xf, xb, rf, rb, ex = make_moe("moe/rep", 96, 128, 128, 8)
    a = run_gpu(ctx, xf, xb, rf, rb, ex, 8, 2, frx.ACT_SILU)
    b = run_gpu(ctx, xf, xb, rf, rb, ex, 8, 2, frx.ACT_SILU)
    np.testing.assert_array_equal(host(a[0]), host(b[0]))
    np.testing.assert_array_equal(a[1], b[1])


def test_moe_shape_errors(ctx):
    xf, xb, rf, rb, ex = make_moe("moe/err", 4, 64, 64, 2)
    with pytest.raises(frx.FrxError) as e:
        run_gpu(ctx, xf, xb, rf, rb, ex, 2, 3, frx.ACT_SILU)  # top_k > E
    assert e.value.kind == "Shape"


def test_moe_nonfinite_tokens_route_like_the_reference(ctx):
    """A token whose activations hold NaN or +-inf makes every routing
    probability of that token NaN (or leaves them finite for -inf logits);
    the reference's stable sort then keeps expert order 0..k-1
    (ternary_moe.rs:175, partial_cmp().unwrap_or(Equal)). Indices must be in
    range and equal to the oracle's for every token, finite or not."""
    T, H, I, E, k = 24, 128, 128, 8, 2
    xf, xb, rf, rb, ex = make_moe("moe/nonfinite", T, H, I, E)
    xf = xf.copy()
    xf[3, 5] = np.nan
    xf[7, :] = np.inf
    xf[11, 0] = -np.inf
    xf[12, 17] = np.inf
    y, idx, w = run_gpu(ctx, xf, None, rf, None, ex, E, k, frx.ACT_SILU, xt="f32")
    ridx, rw, _ = oracle.moe_route(xf, rf, k)
    assert (idx < E).all()
    np.testing.assert_array_equal(idx, ridx)
    finite = [t for t in range(T) if np.isfinite(xf[t]).all()]
    np.testing.assert_allclose(w[finite], rw[finite], rtol=0, atol=1e-6)
    ref, _, _ = run_oracle(xf, rf, ex, E, k, False, tokens=np.array(finite))
    assert_close_f32(host(y)[finite], ref)


@pytest.mark.parametrize("T,H,I,E,k,xt", [(40, 128, 256, 8, 2, "bf16"), (33, 192, 128, 5, 3, "f32"),
                                          (7, 64, 96, 4, 4, "bf16")])
def test_moe_cpu_moe_layer_routing(ctx, T, H, I, E, k, xt):
    """CpuMoELayer semantics (cpu_moe.rs:146-201, 365-400): router read as
    [H, E], experts ranked by logit, weights exp(l - l_max) over the top k.
    The router's values are the same as the [E, H] layer's, transposed."""
    name = f"moe/cpu/{T}x{H}x{I}x{E}"
    xf, xb, rf, rb, ex = make_moe(name, T, H, I, E)
    rf_he = np.ascontiguousarray(rf.T)
    rb_he = np.ascontiguousarray(rb.T) if rb is not None else None
    if xt == "f32":
        xf = synth.normal(77, T * H).reshape(T, H)
    ctx.set_moe_routing(frx.MOE_CPU_MOE_LAYER)
    try:
        y, idx, w = run_gpu(ctx, xf, xb, rf_he, rb_he, ex, E, k, frx.ACT_SILU, xt=xt)
    finally:
        ctx.set_moe_routing(frx.MOE_TERNARY_MOE_LAYER)
    ref, ridx, rw = run_oracle(xf, rf_he, ex, E, k, False, routing=1)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(w, rw, rtol=0, atol=1e-6)
    assert_close_f32(host(y), ref)


def test_moe_cpu_moe_layer_underflow_ranking_and_skip(ctx):
    """Logits far apart: the runner-up weight underflows below 1e-8 and is
    skipped, so the second expert's NaN down scale never reaches the output;
    the experts whose probabilities underflow to 0 are still ranked by
    logit. The [E, H] routing, by contrast, adds the NaN expert."""
    T, H, I, E, k = 4, 64, 64, 3, 3
    xf, xb, rf, rb, ex = make_moe("moe/cpu/skip", T, H, I, E)
    xf = np.zeros((T, H), np.float32)
    xf[:, 0] = 1.0
    r_he = np.zeros((H, E), np.float32)
    r_he[0] = [0.0, -150.0, -120.0]
    ex = dict(ex)
    ex[("down", 1)] = (ex[("down", 1)][0], np.full(H, np.nan, np.float32))
    ctx.set_moe_routing(frx.MOE_CPU_MOE_LAYER)
    try:
        y, idx, w = run_gpu(ctx, xf, None, r_he, None, ex, E, k, frx.ACT_SILU, xt="f32", rt="f32")
    finally:
        ctx.set_moe_routing(frx.MOE_TERNARY_MOE_LAYER)
    ref, ridx, rw = run_oracle(xf, r_he, ex, E, k, False, routing=1)
    assert (ridx == np.array([0, 2, 1], np.uint32)).all()
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_array_equal(w, rw)
    assert np.isfinite(host(y)).all()
    assert_close_f32(host(y), ref)
    y0, idx0, _ = run_gpu(ctx, xf, None, np.ascontiguousarray(r_he.T), None, ex, E, k, frx.ACT_SILU, xt="f32",
                          rt="f32")
    assert list(idx0[0]) == [0, 1, 2]
    assert not np.isfinite(host(y0)).all()


def test_moe_routing_mode_rejects_unknown(ctx):
    with pytest.raises(frx.FrxError) as e:
        ctx.set_moe_routing(7)
    assert e.value.kind == "Unsupported"


KATS = __import__("json").load(open(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden",
                                                                "reference_kats.json")))


@pytest.mark.parametrize("kat", KATS["routing"], ids=lambda k: k["source"].split()[-1])
@pytest.mark.parametrize("xt", ["f32", "bf16"])
def test_routing_kats_through_the_gpu_router(ctx, kat, xt):
    """The reference's routing known-answer tests (kernel_tests.rs) through
    the device router: H padded to 16 with the logits in the first E
    activations and the router [E][16] the identity on them, so the router
    GEMV yields the KAT's logits (bf16 x: the logits rounded to bf16, which
    keeps their order). Indices must be the KAT's; weights softmax over the
    selected logits within the KAT's tolerance; every token routes alike."""
    logits = np.array(kat["logits"], np.float32)
    E, k, H, I, T = logits.size, kat["top_k"], 16, 16, 3
    xf = np.zeros((T, H), np.float32)
    xf[:, :E] = logits
    if xt == "bf16":
        xf = synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(xf))
    rf = np.zeros((E, H), np.float32)
    rf[np.arange(E), np.arange(E)] = 1.0
    ex = {}
    for e in range(E):
        for mat, (n, kk) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
            t = synth.ternary_uniform("moe/kat", f"{mat}{e}", n, kk)
            ex[(mat, e)] = (synth.pack_rows_u32(t), synth.row_scales("moe/kat", f"s{mat}{e}", n, samples=16))
    y, idx, w = run_gpu(ctx, xf, synth.f32_to_bf16_bits(xf), rf, synth.f32_to_bf16_bits(rf), ex, E, k,
                        frx.ACT_SILU, xt=xt, rt="f32")
    for t in range(T):
        assert list(idx[t]) == kat["expected_idx"]
        sel = xf[t, kat["expected_idx"]].astype(np.float64)
        np.testing.assert_allclose(w[t], np.exp(sel) / np.exp(sel).sum(), atol=kat["weight_tol"], rtol=0)
        if "sum_tol" in kat:
            assert abs(float(w[t].sum()) - 1.0) < kat["sum_tol"]
    ref, _, _ = run_oracle(xf, rf, ex, E, k, False)
    assert_close_f32(host(y), ref)


def make_lora(name, H, I, E, rank, skip):
    """Random f32 LoRA adapters (A ~ N(0, 0.1), B ~ N(0, 0.1)) for every
    (projection, expert) except those in `skip` (no adapter there)."""
    shapes = {"gate": ((rank, H), (I, rank)), "up": ((rank, H), (I, rank)), "down": ((rank, I), (H, rank))}
    host_l = {"rank": rank, "scaling": 2.0}
    dev_l = {}
    for proj, (sa, sb) in shapes.items():
        a_l, b_l = [], []
        for e in range(E):
            if (proj, e) in skip:
                a_l.append(None)
                b_l.append(None)
                continue
            a_l.append(synth.normal(synth.seed_of(name, f"la_{proj}{e}"), sa[0] * sa[1], 0.1).reshape(sa))
            b_l.append(synth.normal(synth.seed_of(name, f"lb_{proj}{e}"), sb[0] * sb[1], 0.1).reshape(sb))
        host_l["a_" + proj], host_l["b_" + proj] = a_l, b_l
        dev_l["a_" + proj] = [None if m is None else dev_f32(m) for m in a_l]
        dev_l["b_" + proj] = [None if m is None else dev_f32(m) for m in b_l]
    return host_l, dev_l


@pytest.mark.parametrize("T,H,I,E,k,xt,routing", [(40, 128, 256, 8, 2, "bf16", 0), (50, 320, 192, 5, 2, "bf16", 1),
                                                  (33, 192, 128, 5, 3, "f32", 0), (7, 64, 96, 4, 1, "bf16", 1),
                                                  (300, 192, 448, 3, 2, "bf16", 0)])
def test_moe_lora_parity(ctx, T, H, I, E, k, xt, routing):
    """LoRA adapters on the experts (CpuMoELayer::expert_forward_*_with_lora,
    cpu_moe.rs:321-363; LoraLayer::forward, lora.rs:138-167), on some experts
    and projections only: gated/upped gain scaling * B (A x) before the
    activation, the down output scaling * B (A h). Both GEMM engines (bf16 x
    with H, I multiples of 64; f32 x or I % 64 != 0), one and two K parts of
    the down GEMM, both routing modes; routing bit-exact, outputs within
    1e-3 of the oracle."""
    name = f"moe/lora/{T}x{H}x{I}x{E}"
    xf, xb, rf, rb, ex = make_moe(name, T, H, I, E)
    if xt == "f32":
        xf = synth.normal(91, T * H).reshape(T, H)
    if routing == 1:
        rf, rb = np.ascontiguousarray(rf.T), np.ascontiguousarray(rb.T)
    skip = {("gate", 1), ("up", 0), ("down", 2), ("up", E - 1)}
    hl, dl = make_lora(name, H, I, E, 8, skip)
    ctx.set_moe_routing(routing)
    ctx.set_moe_lora(8, 2.0, E, **dl)
    try:
        y, idx, w = run_gpu(ctx, xf, xb, rf, rb, ex, E, k, frx.ACT_SILU, xt=xt)
    finally:
        ctx.set_moe_lora(None)
        ctx.set_moe_routing(frx.MOE_TERNARY_MOE_LAYER)
    g = lambda m, i: [ex[(m, e)][i] for e in range(E)]  # noqa: E731
    ref, ridx, rw = oracle.moe_forward_lora(xf, rf, g("gate", 0), g("gate", 1), g("up", 0), g("up", 1),
                                            g("down", 0), g("down", 1), k, hl, routing=routing)
    np.testing.assert_array_equal(idx, ridx)
    assert_close_f32(host(y), ref)
    plain, _, _ = run_oracle(xf, rf, ex, E, k, False, routing=routing)
    assert np.abs(ref - plain).max() > 1e-2 * np.abs(plain).max()  # the adapters change the output


def test_moe_lora_cleared_and_shape_checks(ctx):
    """Removing the adapters restores the plain layer bit for bit; a rank
    outside [1, 64] and an expert count that differs from the call's are
    shape errors."""
    T, H, I, E, k = 40, 128, 256, 8, 2
    xf, xb, rf, rb, ex = make_moe("moe/lora/clear", T, H, I, E)
    a = run_gpu(ctx, xf, xb, rf, rb, ex, E, k, frx.ACT_SILU)
    _, dl = make_lora("moe/lora/clear", H, I, E, 4, set())
    ctx.set_moe_lora(4, 1.0, E, **dl)
    ctx.set_moe_lora(None)
    b = run_gpu(ctx, xf, xb, rf, rb, ex, E, k, frx.ACT_SILU)
    np.testing.assert_array_equal(host(a[0]), host(b[0]))
    for rank in (0, 65):
        with pytest.raises(frx.FrxError):
            ctx.set_moe_lora(rank, 1.0, E, **dl)
    ctx.set_moe_lora(4, 1.0, E, **dl)
    try:
        with pytest.raises(frx.FrxError):
            run_gpu(ctx, xf[:, :], xb, rf[:4], rb[:4], {kk: v for kk, v in ex.items() if kk[1] < 4}, 4, k,
                    frx.ACT_SILU)
    finally:
        ctx.set_moe_lora(None)


def test_moe_lora_graph_keeps_its_adapters(ctx):
    """A graph captured with rank-8 adapters keeps reading the table it was
    captured with after frx_set_moe_lora installs rank-2 adapters (each call
    builds its own table): its replays equal the eager rank-8 output bit for
    bit while eager calls between them use rank 2; then the retired tables
    are released."""
    T, H, I, E, k = 40, 128, 256, 8, 2
    name = "moe/lora/graph"
    xf, xb, rf, rb, ex = make_moe(name, T, H, I, E)
    h8, d8 = make_lora(name, H, I, E, 8, set())
    h2, d2 = make_lora(name + "/r2", H, I, E, 2, {("down", 3)})
    dw = {kk: (dev_u32(v[0]), dev_f32(v[1])) for kk, v in ex.items()}
    g = lambda m, i: [dw[(m, e)][i] for e in range(E)]  # noqa: E731
    x, r = dev_bf16(xb), dev_bf16(rb)
    y8 = torch.empty((T, H), dtype=torch.float32, device="cuda:0")
    yg = torch.empty((T, H), dtype=torch.float32, device="cuda:0")
    y2 = torch.empty((T, H), dtype=torch.float32, device="cuda:0")
    c = frx.Context(0)
    s = torch.cuda.Stream()
    c.set_stream(s)
    try:
        def call(y):
            c.moe_ternary_ffn(x, r, g("gate", 0), g("gate", 1), g("up", 0), g("up", 1), g("down", 0),
                              g("down", 1), y, top_k=k)
        c.set_moe_lora(8, 2.0, E, **d8)
        with torch.cuda.stream(s):
            call(y8)  # workspace exists before capture
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            call(yg)
        torch.cuda.synchronize()
        c.set_moe_lora(2, 2.0, E, **d2)
        for rep in range(3):
            yg.fill_(float("nan"))
            y2.fill_(float("nan"))
            with torch.cuda.stream(s):
                graph.replay()
                call(y2)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(host(yg), host(y8))
            ex_h = lambda m, i: [ex[(m, e)][i] for e in range(E)]  # noqa: E731
            ref2, _, _ = oracle.moe_forward_lora(xf, rf, ex_h("gate", 0), ex_h("gate", 1), ex_h("up", 0),
                                                 ex_h("up", 1), ex_h("down", 0), ex_h("down", 1), k, h2)
            assert_close_f32(host(y2), ref2)
        del graph
        torch.cuda.synchronize()
        assert c.workspace_stats()[1] > 0  # the rank-8 table is retired, not freed
        c.release_retired()
        assert c.workspace_stats()[1] == 0
    finally:
        c.set_stream(None)
        c.close()


def test_moe_decode_rows_repeat_and_graph(ctx):
    """The decode path (GEMVs per routed row, routing order): back-to-back
    calls with different tokens, then replays of a captured call with eager
    calls between, each equal to its first eager run bit for bit."""
    H, I, E, k = 256, 320, 8, 2
    name = "moe/dec/graph"
    _, _, rf, rb, ex = make_moe(name, 1, H, I, E)
    dw = {kk: (dev_u32(v[0]), dev_f32(v[1])) for kk, v in ex.items()}
    g = lambda m, i: [dw[(m, e)][i] for e in range(E)]  # noqa: E731
    r = dev_bf16(rb)
    xs = [dev_bf16(synth.activations(f"{name}/{i}", "x", 1, H)[1]) for i in range(3)]
    ys = [torch.empty((1, H), dtype=torch.float32, device="cuda:0") for _ in range(3)]
    s = torch.cuda.Stream()
    ctx.set_stream(s)
    try:
        def call(i):
            ctx.moe_ternary_ffn(xs[i], r, g("gate", 0), g("gate", 1), g("up", 0), g("up", 1), g("down", 0),
                                g("down", 1), ys[i], top_k=k)
        with torch.cuda.stream(s):
            for i in range(3):
                call(i)
        torch.cuda.synchronize()
        refs = [host(y).copy() for y in ys]
        for i in range(3):
            ref, _, _ = run_oracle(synth.bf16_bits_to_f32(synth.activations(f"{name}/{i}", "x", 1, H)[1]), rf, ex,
                                   E, k, False)
            assert_close_f32(refs[i], ref)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            call(0)
        torch.cuda.synchronize()
        for rep in range(4):
            for y in ys:
                y.fill_(float("nan"))
            with torch.cuda.stream(s):
                graph.replay()
                call(1)
                call(2)
            torch.cuda.synchronize()
            for i in range(3):
                np.testing.assert_array_equal(host(ys[i]), refs[i])
    finally:
        ctx.set_stream(None)
