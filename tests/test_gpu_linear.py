"""Dense ternary linear on the GPU (decode GEMV for M <= 16, MFMA GEMM
above) against the CPU oracle (kernels/ternary_matmul.rs:233-265 semantics).

Tolerance (fp32 accumulate vs the reference's f32): elementwise
|y - ref| <= 1e-3 * max(|ref|, rms(ref)) and normwise 1e-3; bf16 outputs
within 1 bf16 ulp of bf16(ref). Dyadic inputs make every partial sum exact,
so there the GPU must equal the reference bit for bit."""
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


def _case(name, M, K, N, seed_x="x"):
    t = synth.ternary_uniform(name, "w", N, K)
    w = synth.pack_rows_u32(t)
    s = synth.row_scales(name, "s", N, samples=256)
    xf, xb = synth.activations(name, seed_x, M, K)
    return t, w, s, xf, xb


def _run(ctx, w, s, xf, xb, xt, yt):
    M, K = xf.shape
    N = w.shape[0]
    x = dev_bf16(xb) if xt == "bf16" else dev_f32(xf)
    y = torch.empty((M, N), dtype=torch.bfloat16 if yt == "bf16" else torch.float32, device="cuda:0")
    y.fill_(float("nan"))
    ctx.ternary_linear(dev_u32(w), dev_f32(s), x, y)
    torch.cuda.synchronize()
    return y


SHAPES = [(1, 256, 64), (2, 512, 100), (3, 512, 100), (16, 1024, 48), (1, 2064, 33), (5, 4096, 130),
          (8, 11008, 72), (9, 2064, 33), (12, 4096, 130), (10, 1040, 8200),
          (17, 256, 64), (64, 1040, 200), (130, 512, 136), (257, 128, 19)]


@pytest.mark.parametrize("M,K,N", SHAPES)
@pytest.mark.parametrize("xt,yt", [("bf16", "f32"), ("f32", "f32"), ("bf16", "bf16"), ("f32", "bf16")])
def test_dense_parity_random(ctx, M, K, N, xt, yt):
    name = f"dense/{M}x{K}x{N}"
    t, w, s, xf, xb = _case(name, M, K, N)
    if xt == "f32":  # genuine f32 activations (exercise the hi/lo split)
        xf = synth.normal(synth.seed_of(name, "xf32"), M * K).reshape(M, K)
    ref = oracle.ternary_matmul_u32(w, s, xf, M, K, N)
    y = _run(ctx, w, s, xf, xb, xt, yt)
    if yt == "f32":
        assert_close_f32(host(y), ref)
    else:
        assert_bf16_within_1ulp(y.view(torch.int16).cpu().numpy().view(np.uint16), ref)


def _dyadic_case(M, K, N, seed):
    rng = np.random.default_rng(seed)
    t = rng.integers(-1, 2, size=(N, K)).astype(np.int8)
    x = (rng.integers(-64, 65, size=(M, K)) / 8.0).astype(np.float32)
    s = (2.0 ** rng.integers(-4, 2, size=N)).astype(np.float32)
    return t, synth.pack_rows_u32(t), s, x, synth.f32_to_bf16_bits(x)


@pytest.mark.parametrize("M,K,N", [(1, 4096, 11008), (1, 11008, 4096), (4, 4096, 11008), (4, 11008, 4096),
                                   (16, 4096, 11008), (16, 11008, 4096), (7, 2048, 2048), (300, 4096, 1000),
                                   (2048, 4096, 4096), (2048, 4096, 11008)])
def test_dense_bit_exact_on_dyadic_inputs(ctx, M, K, N):
    """bf16 and f32 activations (the f32 drop-in path of TernaryMatMulOp,
    split into bf16 hi/lo planes) at the decode shapes and token counts."""
    t, w, s, x, xb = _dyadic_case(M, K, N, M + K + N)
    ref = (x @ t.T.astype(np.float32)) * s[None, :]
    for xt in ("bf16", "f32"):
        y = host(_run(ctx, w, s, x, xb, xt, "f32"))
        np.testing.assert_array_equal(y, ref)


@pytest.mark.parametrize("K,N", [(64, 1), (64, 17), (4160, 35), (8192, 20), (12352, 9), (16384, 50),
                                 (16448, 5)])
@pytest.mark.parametrize("yt", ["f32", "bf16"])
def test_single_token_rows(ctx, K, N, yt):
    """One bf16 token: whole rows per wave for K % 64 == 0 up to 16384 (one
    to four 1 KB windows per row, the last one partial at 4160 and 12352;
    rows past N in the last workgroup), the 16-row tiles at 16448."""
    name = f"rows/{K}x{N}"
    t, w, s, xf, xb = _case(name, 1, K, N)
    ref = oracle.ternary_matmul_u32(w, s, xf, 1, K, N)
    y = _run(ctx, w, s, xf, xb, "bf16", yt)
    if yt == "f32":
        assert_close_f32(host(y), ref)
    else:
        assert_bf16_within_1ulp(y.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("K,N", [(2048, 16385), (4160, 16401), (8256, 16384), (12352, 16390)])
def test_single_token_rows_tall(ctx, K, N):
    """From N = 16384 rows, above one window, persistent waves walk row
    groups with the next group's words in flight (two, three and four
    windows, the last one partial; ragged last group); the one-window case
    stays on the one-shot kernel. f32 and bf16 outputs."""
    t, w, s, xf, xb = _case(f"rows/tall/{K}x{N}", 1, K, N)
    ref = oracle.ternary_matmul_u32(w, s, xf, 1, K, N)
    assert_close_f32(host(_run(ctx, w, s, xf, xb, "bf16", "f32")), ref)
    yb = _run(ctx, w, s, xf, xb, "bf16", "bf16")
    assert_bf16_within_1ulp(yb.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("K,N", [(8192, 28672), (8192, 57344)])
def test_single_token_tall_llama70b_bit_exact_on_dyadic_inputs(ctx, K, N):
    """The LLaMA-70B gate projection [28672, 8192] and gate + up stacked
    [57344, 8192] at one token (the persistent kernel, bf16 and f32 outputs):
    every output equals the exact sum (bf16: its round-to-nearest-even)."""
    t, w, s, x, xb = _dyadic_case(1, K, N, K + N)
    ref = (x @ t.T.astype(np.float32)) * s[None, :]
    np.testing.assert_array_equal(host(_run(ctx, w, s, x, xb, "bf16", "f32")), ref)
    yb = _run(ctx, w, s, x, xb, "bf16", "bf16")
    np.testing.assert_array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), synth.f32_to_bf16_bits(ref))


@pytest.mark.parametrize("K,N", [(4160, 300), (12352, 40), (4096, 64), (4160, 16390)])
def test_single_token_rows_bit_exact_on_dyadic_inputs(ctx, K, N):
    t, w, s, x, xb = _dyadic_case(1, K, N, K + N)
    ref = (x @ t.T.astype(np.float32)) * s[None, :]
    y = host(_run(ctx, w, s, x, xb, "bf16", "f32"))
    np.testing.assert_array_equal(y, ref)


@pytest.mark.parametrize("M,K,N", [(2, 64, 9), (3, 1024, 70), (4, 2048, 33), (2, 4096, 300), (3, 4160, 20),
                                   (4, 8192, 17), (4, 11008, 100), (2, 12352, 40), (4, 14336, 8),
                                   (3, 14400, 8)])
@pytest.mark.parametrize("yt", ["f32", "bf16"])
def test_two_to_four_tokens_rows(ctx, M, K, N, yt):
    """2 <= B <= 4 bf16 tokens: 4 rows x 4 segments per MFMA for K % 64 == 0
    up to 14336 (1 to 14 windows of 1024 codes, rounded up to the
    instantiated counts; rows past N in the last workgroup), the 16-row
    tiles at 14400."""
    name = f"rows4/{M}x{K}x{N}"
    t, w, s, xf, xb = _case(name, M, K, N)
    ref = oracle.ternary_matmul_u32(w, s, xf, M, K, N)
    y = _run(ctx, w, s, xf, xb, "bf16", yt)
    if yt == "f32":
        assert_close_f32(host(y), ref)
    else:
        assert_bf16_within_1ulp(y.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("M,K,N", [(4, 4160, 64), (2, 11008, 48), (3, 4096, 130)])
def test_two_to_four_tokens_bit_exact_on_dyadic_inputs(ctx, M, K, N):
    t, w, s, x, xb = _dyadic_case(M, K, N, M * K + N)
    ref = (x @ t.T.astype(np.float32)) * s[None, :]
    y = host(_run(ctx, w, s, x, xb, "bf16", "f32"))
    np.testing.assert_array_equal(y, ref)


@pytest.mark.parametrize("M,K,N", [(8, 16, 5), (11, 272, 17), (16, 4112, 700), (13, 8208, 33), (16, 12288, 1100),
                                   (9, 16384, 40), (16, 4096, 16400), (16, 11008, 9000)])
@pytest.mark.parametrize("yt", ["f32", "bf16"])
def test_eight_to_sixteen_tokens_staged(ctx, M, K, N, yt):
    """8 <= B <= 16 bf16 tokens through the per-wave staged activations: K
    from one word to 64 quads (partial last quads), N below one tile, ragged
    last tiles, more than 64 rows per CU (extra workgroups), and the
    two-tile limit above 32 quads."""
    name = f"xs/{M}x{K}x{N}"
    t, w, s, xf, xb = _case(name, M, K, N)
    ref = oracle.ternary_matmul_u32(w, s, xf, M, K, N)
    y = _run(ctx, w, s, xf, xb, "bf16", yt)
    if yt == "f32":
        assert_close_f32(host(y), ref)
    else:
        assert_bf16_within_1ulp(y.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("M,K,N", [(16, 4096, 11008), (12, 12352, 300), (8, 2048, 64)])
def test_eight_to_sixteen_tokens_bit_exact_on_dyadic_inputs(ctx, M, K, N):
    t, w, s, x, xb = _dyadic_case(M, K, N, M * K + N + 1)
    ref = (x @ t.T.astype(np.float32)) * s[None, :]
    y = host(_run(ctx, w, s, x, xb, "bf16", "f32"))
    np.testing.assert_array_equal(y, ref)


def test_single_token_unaligned_weights(ctx):
    """Packed weights 4 bytes past a 16-byte boundary take the 16-row tiles
    (dword loads); both placements match the oracle."""
    K, N = 4096, 300
    t, w, s, xf, xb = _case("rows/unaligned", 1, K, N)
    ref = oracle.ternary_matmul_u32(w, s, xf, 1, K, N)
    buf = torch.zeros(w.size + 4, dtype=torch.int32, device="cuda:0")
    buf[1:1 + w.size] = torch.from_numpy(w.reshape(-1).view(np.int32)).to("cuda:0")
    w_un = buf[1:1 + w.size].view(N, K // 16)
    assert w_un.data_ptr() % 16 == 4
    y = torch.empty((1, N), dtype=torch.float32, device="cuda:0")
    ctx.ternary_linear(w_un, dev_f32(s), dev_bf16(xb), y)
    torch.cuda.synchronize()
    assert_close_f32(host(y), ref)
    assert_close_f32(host(_run(ctx, w, s, xf, xb, "bf16", "f32")), ref)


@pytest.mark.parametrize("B", [1, 4, 16])
@pytest.mark.parametrize("K,N", [(4096, 11008), (11008, 4096)])
def test_decode_gemv_config_shapes(ctx, B, K, N):
    """LLaMA-7B FFN decode shapes, bf16 x, fp32 accumulate (f32 and bf16 out)."""
    name = f"decode/{K}x{N}"
    t, w, s, xf, xb = _case(name, B, K, N, seed_x=f"x{B}")
    ref = oracle.ternary_matmul_u32(w, s, xf, B, K, N)
    assert_close_f32(host(_run(ctx, w, s, xf, xb, "bf16", "f32")), ref)
    yb = _run(ctx, w, s, xf, xb, "bf16", "bf16")
    assert_bf16_within_1ulp(yb.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("N", [4096, 11008])
def test_prefill_gemm_config_shapes_sampled(ctx, N):
    """X[2048,4096] bf16 x W[N,4096]: output rows depend only on their own
    token, so 12 sampled tokens are checked against the oracle in full."""
    M, K = 2048, 4096
    name = f"prefill/{N}"
    t, w, s, xf, xb = _case(name, M, K, N)
    y = host(_run(ctx, w, s, xf, xb, "bf16", "f32"))
    rows = np.array([0, 1, 15, 16, 127, 128, 1000, 1023, 1024, 2000, 2046, 2047])
    ref = oracle.ternary_matmul_u32(w, s, xf[rows], len(rows), K, N)
    assert_close_f32(y[rows], ref)
    assert np.isfinite(y).all()


def test_deterministic_across_runs(ctx):
    t, w, s, xf, xb = _case("det", 16, 4096, 1024)
    a = host(_run(ctx, w, s, xf, xb, "bf16", "f32"))
    b = host(_run(ctx, w, s, xf, xb, "bf16", "f32"))
    np.testing.assert_array_equal(a, b)
    t, w, s, xf, xb = _case("det2", 300, 1024, 256)
    a = host(_run(ctx, w, s, xf, xb, "bf16", "f32"))
    b = host(_run(ctx, w, s, xf, xb, "bf16", "f32"))
    np.testing.assert_array_equal(a, b)


def test_code3_decodes_to_zero_on_gpu(ctx):
    K, N = 64, 16
    rng = np.random.default_rng(0)
    w = rng.integers(0, 2 ** 32, size=(N, K // 16), dtype=np.uint64).astype(np.uint32)  # codes 0..3
    s = np.ones(N, np.float32)
    x = (rng.integers(-8, 9, size=(2, K)) / 4.0).astype(np.float32)
    ref = oracle.ternary_matmul_u32(w, s, x, 2, K, N)
    y = host(_run(ctx, w, s, x, synth.f32_to_bf16_bits(x), "f32", "f32"))
    np.testing.assert_array_equal(y, ref)
    y = host(_run(ctx, w, s, np.repeat(x, 10, 0), synth.f32_to_bf16_bits(np.repeat(x, 10, 0)), "f32", "f32"))
    np.testing.assert_array_equal(y, np.repeat(ref, 10, 0))


def test_shape_errors_are_statuses(ctx):
    w = dev_u32(np.zeros((4, 1), np.uint32))
    s = dev_f32(np.ones(4, np.float32))
    x = dev_f32(np.ones((1, 20), np.float32))
    y = torch.empty((1, 4), dtype=torch.float32, device="cuda:0")
    with pytest.raises(frx.FrxError) as e:
        ctx.ternary_linear(w, s, x, y)  # K = 20 is not a multiple of 16
    assert e.value.kind == "Shape"


# ---- TernaryLinear with a bias (frx_ternary_linear_bias) --------------------

def _run_bias(ctx, w, s, bias, x, xb, xt, yt):
    M, K = x.shape
    N = w.shape[0]
    xd = dev_bf16(xb) if xt == "bf16" else dev_f32(x)
    y = torch.empty((M, N), dtype=torch.bfloat16 if yt == "bf16" else torch.float32, device="cuda:0")
    y.fill_(float("nan"))
    ctx.ternary_linear(dev_u32(w), dev_f32(s), xd, y, bias=None if bias is None else dev_f32(bias))
    torch.cuda.synchronize()
    return y


# Every kernel family of the linear path: one token (balanced rows; whole
# rows per wave, one-shot and persistent; 16-row tiles above 16384 columns),
# 2-4 tokens, 5-7 tokens (16-row tiles), 8-16 tokens (staged activations;
# above 16384 columns the per-lane operand loads, 16- and 32-row tiles), the
# MFMA GEMM (K % 64 == 0 and not).
BIAS_SHAPES = [(1, 2048, 2048), (1, 4096, 11008), (1, 11008, 4096), (1, 8256, 9000), (1, 4160, 16401),
               (1, 16448, 40), (3, 4096, 300), (4, 11008, 4096), (6, 2048, 130), (16, 4096, 11008),
               (16, 11008, 4096), (9, 16400, 40), (9, 16400, 8170), (64, 1040, 200), (300, 4096, 1000),
               (2048, 4096, 4096)]


@pytest.mark.parametrize("M,K,N", BIAS_SHAPES)
def test_linear_bias_bit_exact_on_dyadic_inputs(ctx, M, K, N):
    """y = (alpha * W x) + bias (ternary_linear.rs:94-115) with dyadic x and
    codes, so every sum is exact; alpha and bias are random f32, which fixes
    both roundings (the product, then the addition): a fused multiply-add
    in an epilogue would differ in the last bit. The reference's layer has
    one alpha for all rows. Against the oracle's TernaryLinear forward where
    it finishes in seconds, else against the same two f32 operations on the
    exact sums."""
    t, w, _, x, xb = _dyadic_case(M, K, N, 7 * M + K + N)
    rng = np.random.default_rng(M + K + 3 * N)
    alpha = np.float32(rng.uniform(0.25, 2.0))
    s = np.full(N, alpha, np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    if M * K * N <= 2e8:
        ref = oracle.ternary_linear_forward(t, alpha, bias, x, N, K, M, 0)
    else:
        ref = ((x @ t.T.astype(np.float32)) * alpha).astype(np.float32) + bias[None, :]
    for xt in ("bf16", "f32"):
        y = host(_run_bias(ctx, w, s, bias, x, xb, xt, "f32"))
        np.testing.assert_array_equal(y, ref)
    yb = _run_bias(ctx, w, s, bias, x, xb, "bf16", "bf16").view(torch.int16).cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(yb, synth.f32_to_bf16_bits(ref))


@pytest.mark.parametrize("M,K,N", [(1, 2048, 2048), (4, 4096, 11008), (16, 11008, 4096), (2048, 2048, 2048)])
def test_linear_bias_random_inputs(ctx, M, K, N):
    """Normal f32 activations (hi/lo split) and bf16 activations with a
    bias, against the oracle's TernaryLinear forward (rows sampled at
    M = 2048), at the tolerance of the bias-free linear tests."""
    name = f"bias/{M}x{K}x{N}"
    t, w, _, xf, xb = _case(name, M, K, N)
    alpha = np.float32(0.0371)
    s = np.full(N, alpha, np.float32)
    bias = synth.normal(synth.seed_of(name, "bias"), N).astype(np.float32)
    rows = np.arange(M) if M <= 16 else np.array([0, 1, 127, 128, 1000, 2047])
    ref = oracle.ternary_linear_forward(t, alpha, bias, xf[rows], N, K, len(rows), 0)
    assert_close_f32(host(_run_bias(ctx, w, s, bias, xf, xb, "bf16", "f32"))[rows], ref)
    x32 = synth.normal(synth.seed_of(name, "xf32"), M * K).reshape(M, K).astype(np.float32)
    ref32 = oracle.ternary_linear_forward(t, alpha, bias, x32[rows], N, K, len(rows), 0)
    assert_close_f32(host(_run_bias(ctx, w, s, bias, x32, xb, "f32", "f32"))[rows], ref32)


def test_linear_bias_none_is_plain_linear(ctx):
    t, w, s, xf, xb = _case("bias/none", 5, 1024, 96)
    a = host(_run_bias(ctx, w, s, None, xf, xb, "bf16", "f32"))
    b = host(_run(ctx, w, s, xf, xb, "bf16", "f32"))
    np.testing.assert_array_equal(a, b)
    zero = np.zeros(96, np.float32)
    c = host(_run_bias(ctx, w, s, zero, xf, xb, "bf16", "f32"))
    np.testing.assert_array_equal(c, b)


def test_forced_status_for_caller_fallback(ctx):
    """frx_force_status makes every compute call fail with the chosen
    FerrisResError variant before touching its arguments (the output keeps
    its contents), synchronize still works, and 0 clears it."""
    t, w, s, xf, xb = _case("forced", 2, 256, 32)
    y = torch.full((2, 32), 7.0, dtype=torch.float32, device="cuda:0")
    wd, sd, xd = dev_u32(w), dev_f32(s), dev_bf16(xb)
    for status, kind in ((5, "OOM"), (1, "Gpu"), (6, "Unsupported")):
        ctx.force_status(status)
        with pytest.raises(frx.FrxError) as e:
            ctx.ternary_linear(wd, sd, xd, y)
        assert e.value.kind == kind and "forced" in str(e.value)
        ctx.synchronize()
    assert (host(y) == 7.0).all()
    with pytest.raises(frx.FrxError) as e:
        ctx.force_status(9)
    assert e.value.kind == "Unsupported"
    ctx.force_status(0)
    ctx.ternary_linear(wd, sd, xd, y)
    torch.cuda.synchronize()
    assert_close_f32(host(y), oracle.ternary_matmul_u32(w, s, synth.bf16_bits_to_f32(xb), 2, 256, 32))


@pytest.mark.parametrize("M", [1, 4, 16, 40])
@pytest.mark.parametrize("xt,yt", [("bf16", "bf16"), ("f32", "f32")])
def test_unaligned_subslices_are_staged(ctx, M, xt, yt):
    """x, scale and y as sub-slices at element offsets that are not 16-byte
    aligned (a caller slicing a larger tensor, as the reference's &[f32]
    slices allow): the call stages them through an aligned workspace and
    gives the aligned call's output bit for bit; the 2:4 GEMM as well."""
    K, N = 1024, 200
    t, w, s, xf, xb = _case(f"unaligned/{M}", M, K, N)
    xe = 1  # one element past a 16-byte boundary
    if xt == "bf16":
        big = torch.zeros(M * K + 8, dtype=torch.int16, device="cuda:0")
        big[xe:xe + M * K] = torch.from_numpy(xb.reshape(-1).view(np.int16)).to("cuda:0")
        x_un = big[xe:xe + M * K].view(torch.bfloat16).view(M, K)
    else:
        big = torch.zeros(M * K + 8, dtype=torch.float32, device="cuda:0")
        big[xe:xe + M * K] = torch.from_numpy(xf.reshape(-1)).to("cuda:0")
        x_un = big[xe:xe + M * K].view(M, K)
    assert x_un.data_ptr() % 16 != 0
    sbig = torch.zeros(N + 4, dtype=torch.float32, device="cuda:0")
    sbig[1:1 + N] = dev_f32(s)
    s_un = sbig[1:1 + N]
    ydt = torch.bfloat16 if yt == "bf16" else torch.float32
    ybig = torch.full((M * N + 8,), float("nan"), dtype=ydt, device="cuda:0")
    y_un = ybig[3:3 + M * N].view(M, N)
    assert y_un.data_ptr() % 16 != 0 and s_un.data_ptr() % 16 != 0
    ctx.ternary_linear(dev_u32(w), s_un, x_un, y_un)
    ref = _run(ctx, w, s, xf, xb, xt, yt)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(y_un), host(ref))
    assert torch.isnan(ybig[:3].float()).all() and torch.isnan(ybig[3 + M * N:].float()).all()
    # 2:4 on the same sub-slices
    t24 = synth.sparse24_uniform(f"unaligned24/{M}", "w", N, K)
    meta = frx.pack_sparse24_gpu(t24)
    y24 = torch.empty((M, N), dtype=ydt, device="cuda:0")
    ctx.sparse24_ternary_linear(dev_u32(meta), s_un, x_un, y_un)
    ctx.sparse24_ternary_linear(dev_u32(meta), dev_f32(s), x_un.contiguous().clone(), y24)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(y_un), host(y24))


def test_workspaces_grow_geometrically(ctx):
    """Rising sizes through a workspace-backed entry point (the column-block
    linear's prescaled activations, M*K*4 bytes) make O(log) allocations,
    retire less than twice the live bytes, and frx_release_retired frees the
    retired ones; results stay correct after the release."""
    c = frx.Context(0)
    try:
        K, N, bs = 1024, 64, 128
        t, w, s, _, _ = _case("ws/grow", 1, K, N)
        wd = dev_u32(w)
        bsc = dev_f32(np.linspace(0.5, 1.5, K // bs).astype(np.float32))
        for M in range(1, 161, 3):
            x = torch.randn((M, K), dtype=torch.float32, device="cuda:0")
            y = torch.empty((M, N), dtype=torch.float32, device="cuda:0")
            c.ternary_linear_blocked(wd, bsc, bs, x, y)
        torch.cuda.synchronize()
        live, retired, allocs = c.workspace_stats()
        assert allocs <= 16, allocs
        assert retired < 2 * live, (retired, live)
        c.release_retired()
        assert c.workspace_stats()[1] == 0
        xf = synth.normal(5, 160 * K).reshape(160, K)
        y = torch.empty((160, N), dtype=torch.float32, device="cuda:0")
        c.ternary_linear_blocked(wd, bsc, bs, dev_f32(xf), y)
        torch.cuda.synchronize()
        ref = oracle.ternary_matmul_blocked(t.astype(np.int8), host(bsc), bs, xf, N, K, 160)
        assert_close_f32(host(y), np.asarray(ref).reshape(160, N))
    finally:
        c.close()


@pytest.mark.parametrize("M,K,Ns,xt,yt", [
    (1, 4096, (11008, 11008), "bf16", "bf16"),      # LLaMA-7B gate + up
    (1, 4096, (4096, 4096, 4096), "bf16", "f32"),   # Q / K / V
    (1, 2048, (4096, 1024, 512, 33), "f32", "bf16"),
    (1, 11008, (4096, 300), "bf16", "f32"),
    (4, 4096, (1024, 2048), "bf16", "bf16"),        # per-matrix launches
    (40, 1024, (256, 100, 64), "bf16", "f32"),      # prefill: per-matrix GEMMs
])
def test_linear_group_equals_separate_calls(ctx, M, K, Ns, xt, yt):
    """frx_ternary_linear_group (the Q/K/V and gate/up calls on one x,
    cpu_block_attn_res.rs:2254-2263, :2319-2320): each output equals the
    separate frx_ternary_linear call bit for bit (every row is one wave's
    chain in both, whatever launch it is part of) and the oracle within
    1e-3."""
    name = f"group/{M}x{K}x{'_'.join(map(str, Ns))}"
    xf, xb = synth.activations(name, "x", M, K)
    if xt == "f32":
        xf = synth.normal(synth.seed_of(name, "xf"), M * K).reshape(M, K)
    x = dev_bf16(xb) if xt == "bf16" else dev_f32(xf)
    ydt = torch.bfloat16 if yt == "bf16" else torch.float32
    ws, ss, refs, ts = [], [], [], []
    for i, n in enumerate(Ns):
        t = synth.ternary_uniform(name, f"w{i}", n, K)
        w = synth.pack_rows_u32(t)
        s = synth.row_scales(name, f"s{i}", n, samples=256)
        ws.append(dev_u32(w))
        ss.append(dev_f32(s))
        refs.append(np.asarray(oracle.ternary_matmul_u32(w, s, xf, M, K, n)).reshape(M, n))
    ys = [torch.full((M, n), float("nan"), dtype=ydt, device="cuda:0") for n in Ns]
    ctx.ternary_linear_group(x, ws, ss, ys)
    sep = [torch.empty((M, n), dtype=ydt, device="cuda:0") for n in Ns]
    for w, s, y in zip(ws, ss, sep):
        ctx.ternary_linear(w, s, x, y)
    torch.cuda.synchronize()
    for y, y2, ref in zip(ys, sep, refs):
        np.testing.assert_array_equal(host(y), host(y2))
        if yt == "bf16":
            assert_bf16_within_1ulp(y.view(torch.int16).cpu().numpy().view(np.uint16), ref)
        else:
            assert_close_f32(host(y), ref)


def test_linear_group_errors(ctx):
    x = torch.zeros((1, 64), dtype=torch.bfloat16, device="cuda:0")
    w = torch.zeros((8, 4), dtype=torch.int32, device="cuda:0")
    s = torch.zeros(8, dtype=torch.float32, device="cuda:0")
    y = torch.zeros((1, 8), dtype=torch.float32, device="cuda:0")
    with pytest.raises(frx.FrxError) as e:
        ctx.ternary_linear_group(x, [w] * 5, [s] * 5, [y] * 5)
    assert e.value.kind == "Shape"
    with pytest.raises(frx.FrxError) as e:
        ctx.ternary_linear_group(x, [], [], [])
    assert e.value.kind == "Shape"


@pytest.mark.parametrize("M,K,N", [(2, 4096, 11008), (4, 11008, 4096), (16, 11008, 4096), (16, 4096, 11008),
                                   (5, 1040, 300), (8, 256, 130), (16, 2064, 33), (3, 16, 7)])
@pytest.mark.parametrize("xt,yt", [("f32", "f32"), ("bf16", "bf16"), ("f32", "bf16")])
def test_split_k_gemv_parity(ctx, M, K, N, xt, yt):
    """The split-K decode GEMV (frx_set_gemv_split ALWAYS: 128-row tiles x
    1024-column slices, fp32 partials added in slice order) against the
    oracle, K not a multiple of 256 and ragged N included; with a bias; and
    the whole-K kernels (NEVER) on the same inputs."""
    name = f"splitk/{M}x{K}x{N}"
    t, w, s, xf, xb = _case(name, M, K, N)
    if xt == "f32":
        xf = synth.normal(synth.seed_of(name, "xf"), M * K).reshape(M, K)
    ref = np.asarray(oracle.ternary_matmul_u32(w, s, xf, M, K, N)).reshape(M, N)
    bias = synth.normal(synth.seed_of(name, "b"), N, 0.1)
    outs = {}
    try:
        for mode in (frx.GEMV_SPLIT_ALWAYS, frx.GEMV_SPLIT_NEVER):
            ctx.set_gemv_split(mode)
            y = _run(ctx, w, s, xf, xb, xt, yt)
            yb = torch.empty_like(y)
            x = dev_bf16(xb) if xt == "bf16" else dev_f32(xf)
            ctx.ternary_linear(dev_u32(w), dev_f32(s), x, yb, bias=dev_f32(bias))
            torch.cuda.synchronize()
            outs[mode] = (y, yb)
    finally:
        ctx.set_gemv_split(frx.GEMV_SPLIT_AUTO)
    for mode, (y, yb) in outs.items():
        refb = (ref * 1.0 + bias[None, :]).astype(np.float32)
        if yt == "bf16":
            assert_bf16_within_1ulp(y.view(torch.int16).cpu().numpy().view(np.uint16), ref)
            assert_bf16_within_1ulp(yb.view(torch.int16).cpu().numpy().view(np.uint16), refb)
        else:
            assert_close_f32(host(y), ref)
            assert_close_f32(host(yb), refb)


@pytest.mark.parametrize("M,K,N", [(16, 11008, 4096), (7, 4096, 1100), (2, 1024, 200)])
def test_split_k_gemv_bit_exact_on_dyadic_inputs(ctx, M, K, N):
    """Dyadic activations make every partial sum exact: the split-K kernel
    equals the f64 product bit for bit, bf16 and f32 activations."""
    t, w, s, x, xb = _dyadic_case(M, K, N, 7 * M + K + N)
    ref = (x @ t.T.astype(np.float32)) * s[None, :]
    try:
        ctx.set_gemv_split(frx.GEMV_SPLIT_ALWAYS)
        np.testing.assert_array_equal(host(_run(ctx, w, s, x, xb, "bf16", "f32")), ref)
        np.testing.assert_array_equal(host(_run(ctx, w, s, x, xb, "f32", "f32")), ref)
    finally:
        ctx.set_gemv_split(frx.GEMV_SPLIT_AUTO)


def test_stream_switch_orders_workspace_use():
    """frx_set_stream makes the new stream wait for the work already enqueued
    on the previous one, so two split-K calls on one context, the second on
    another stream right after the switch, do not share the partial-sum
    workspace and counters at the same time: both outputs stay exact."""
    c = frx.Context(0)
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    try:
        c.set_gemv_split(frx.GEMV_SPLIT_ALWAYS)
        cases = [_dyadic_case(16, 11008, 4096, 91), _dyadic_case(16, 11008, 4096, 92)]
        dev = [(dev_u32(w), dev_f32(s), dev_f32(x)) for (t, w, s, x, xb) in cases]
        refs = [(x @ t.T.astype(np.float32)) * s[None, :] for (t, w, s, x, xb) in cases]
        torch.cuda.synchronize()
        for rep in range(3):
            ys = [torch.full((16, 4096), float("nan"), device="cuda:0") for _ in cases]
            torch.cuda.synchronize()
            for i, (st, (w, s, x)) in enumerate(zip((sa, sb), dev)):
                c.set_stream(st)
                with torch.cuda.stream(st):
                    c.ternary_linear(w, s, x, ys[i])
            torch.cuda.synchronize()
            for y, ref in zip(ys, refs):
                np.testing.assert_array_equal(host(y), ref)
            c.set_stream(sa)
    finally:
        c.close()


@pytest.mark.parametrize("M,K,N", [(5, 28672, 8192), (16, 28672, 8192), (3, 16448, 4096), (8, 14336, 4096),
                                   (16, 14336, 3072)])
def test_auto_split_bf16_bit_exact_on_dyadic_inputs(ctx, M, K, N):
    """bf16 activations at 3-16 tokens over long rows take the split-K GEMV
    under FRX_GEMV_SPLIT_AUTO (the LLaMA-70B down projection 8192 x 28672
    among them): dyadic inputs, exact sums, f32 and bf16 outputs."""
    t, w, s, x, xb = _dyadic_case(M, K, N, 5 * M + K + N)
    ref = (x @ t.T.astype(np.float32)) * s[None, :]
    np.testing.assert_array_equal(host(_run(ctx, w, s, x, xb, "bf16", "f32")), ref)
    yb = _run(ctx, w, s, x, xb, "bf16", "bf16")
    np.testing.assert_array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), synth.f32_to_bf16_bits(ref))


@pytest.mark.parametrize("K,N", [(28672, 8192), (16448, 3000)])
def test_auto_split_one_f32_token_long_rows(ctx, K, N):
    """One f32 token past 16384 columns takes the split-K GEMV under
    FRX_GEMV_SPLIT_AUTO: dyadic inputs give the exact sums, with and without
    a bias (added after the scale)."""
    t, w, s, x, xb = _dyadic_case(1, K, N, K + 3 * N)
    ref = (x @ t.T.astype(np.float32)) * s[None, :]
    np.testing.assert_array_equal(host(_run(ctx, w, s, x, xb, "f32", "f32")), ref)
    bias = (np.arange(N) % 7 - 3).astype(np.float32) / 4
    y = torch.full((1, N), float("nan"), device="cuda:0")
    ctx.ternary_linear(dev_u32(w), dev_f32(s), dev_f32(x), y, bias=dev_f32(bias))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(y), ref + bias[None, :])


@pytest.mark.parametrize("K,N", [(16448, 37), (20480, 1001), (24576, 64), (24640, 515), (32768, 300)])
@pytest.mark.parametrize("yt", ["f32", "bf16"])
def test_single_token_long_rows(ctx, K, N, yt):
    """One bf16 token over rows of 16448 to 32768 codes: two passes of three
    or four 1 KB windows per row (the last window partial at 16448, 20480
    and 24640; passes past K multiply staged zeros), rows past N in the last
    workgroup, against the oracle."""
    t, w, s, xf, xb = _case(f"rows/long/{K}x{N}", 1, K, N)
    ref = oracle.ternary_matmul_u32(w, s, xf, 1, K, N)
    y = _run(ctx, w, s, xf, xb, "bf16", yt)
    if yt == "f32":
        assert_close_f32(host(y), ref)
    else:
        assert_bf16_within_1ulp(y.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("K,N", [(28672, 8192), (20544, 3000)])
def test_single_token_long_rows_bit_exact_on_dyadic_inputs(ctx, K, N):
    """The LLaMA-70B down projection [8192, 28672] at one bf16 token: exact
    sums, f32 and bf16 outputs, and with a bias."""
    t, w, s, x, xb = _dyadic_case(1, K, N, 2 * K + N)
    ref = (x @ t.T.astype(np.float32)) * s[None, :]
    np.testing.assert_array_equal(host(_run(ctx, w, s, x, xb, "bf16", "f32")), ref)
    yb = _run(ctx, w, s, x, xb, "bf16", "bf16")
    np.testing.assert_array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), synth.f32_to_bf16_bits(ref))
    bias = (np.arange(N) % 5 - 2).astype(np.float32) / 8
    y = torch.full((1, N), float("nan"), device="cuda:0")
    ctx.ternary_linear(dev_u32(w), dev_f32(s), dev_bf16(xb), y, bias=dev_f32(bias))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(y), ref + bias[None, :])


@pytest.mark.parametrize("M,K,N", [(17, 4096, 11008), (32, 11008, 4096), (64, 4096, 4096), (100, 2048, 5632),
                                   (256, 4096, 11008), (500, 1024, 1028)])
def test_split_k_gemm_bit_exact_on_dyadic_inputs(ctx, M, K, N):
    """17 to a few hundred bf16 tokens, where 64-token tiles leave compute
    units idle: the GEMM splits K into parts whose fp32 partials are added in
    part order. Dyadic inputs: exact sums, f32 and bf16 outputs, and a bias."""
    t, w, s, x, xb = _dyadic_case(M, K, N, 3 * M + K + N)
    ref = (x @ t.T.astype(np.float32)) * s[None, :]
    np.testing.assert_array_equal(host(_run(ctx, w, s, x, xb, "bf16", "f32")), ref)
    yb = _run(ctx, w, s, x, xb, "bf16", "bf16")
    np.testing.assert_array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), synth.f32_to_bf16_bits(ref))
    bias = (np.arange(N) % 9 - 4).astype(np.float32) / 16
    y = torch.full((M, N), float("nan"), device="cuda:0")
    ctx.ternary_linear(dev_u32(w), dev_f32(s), dev_bf16(xb), y, bias=dev_f32(bias))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(y), ref + bias[None, :])


@pytest.mark.parametrize("M,K,N", [(24, 4096, 11008), (130, 11008, 4096)])
def test_split_k_gemm_random_parity(ctx, M, K, N):
    t, w, s, xf, xb = _case(f"gemmsk/{M}x{K}x{N}", M, K, N)
    ref = oracle.ternary_matmul_u32(w, s, xf, M, K, N)
    assert_close_f32(host(_run(ctx, w, s, xf, xb, "bf16", "f32")), ref)
    yb = _run(ctx, w, s, xf, xb, "bf16", "bf16")
    assert_bf16_within_1ulp(yb.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("M,K,N", [(17, 4096, 11008), (300, 1024, 1000), (2048, 4096, 4096), (64, 11008, 4096)])
def test_f32_prefill_planes_bit_exact_on_dyadic_inputs(ctx, M, K, N):
    """f32 activations above 16 tokens: split once into bf16 hi | lo rows and
    multiplied by the bf16 engine over both halves (split over K at small
    token counts). Dyadic inputs are exact in the hi half."""
    t, w, s, x, xb = _dyadic_case(M, K, N, 11 * M + K + N)
    ref = (x @ t.T.astype(np.float32)) * s[None, :]
    np.testing.assert_array_equal(host(_run(ctx, w, s, x, xb, "f32", "f32")), ref)
    yb = _run(ctx, w, s, x, xb, "f32", "bf16")
    np.testing.assert_array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), synth.f32_to_bf16_bits(ref))


@pytest.mark.parametrize("M,K,N", [(40, 2048, 3000), (17, 11008, 4096), (700, 4096, 1100)])
def test_f32_prefill_planes_random_parity(ctx, M, K, N):
    """Genuine f32 activations (the lo half matters) above 16 tokens against
    the oracle, f32 and bf16 outputs."""
    name = f"f32planes/{M}x{K}x{N}"
    t, w, s, xf, xb = _case(name, M, K, N)
    xf = synth.normal(synth.seed_of(name, "xf32"), M * K).reshape(M, K)
    ref = oracle.ternary_matmul_u32(w, s, xf, M, K, N)
    assert_close_f32(host(_run(ctx, w, s, xf, xb, "f32", "f32")), ref)
    yb = _run(ctx, w, s, xf, xb, "f32", "bf16")
    assert_bf16_within_1ulp(yb.view(torch.int16).cpu().numpy().view(np.uint16), ref)
