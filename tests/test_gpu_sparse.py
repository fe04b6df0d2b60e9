"""2:4 sparse ternary linear on the GPU against the oracle's restatement of
the WGSL 2:4 kernel (kernels/sparse_ternary.rs:321-360), in the GPU 5-bit
layout. Same tolerances as the dense path."""
import json
import os

import numpy as np
import pytest
import torch

import ferrisres_amd as frx
import oracle
from ferrisres_amd import synth
from _gpu import assert_bf16_within_1ulp, assert_close_f32, dev_bf16, dev_f32, dev_u32, host

pytestmark = pytest.mark.gpu
KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "GPU tests need a gfx950 device"
    c = frx.Context(0)
    yield c
    c.close()


def _run(ctx, meta, s, xf, xb, xt, yt):
    M, K = xf.shape
    N = meta.shape[0]
    x = dev_bf16(xb) if xt == "bf16" else dev_f32(xf)
    y = torch.empty((M, N), dtype=torch.bfloat16 if yt == "bf16" else torch.float32, device="cuda:0")
    ctx.sparse24_ternary_linear(dev_u32(meta), dev_f32(s), x, y)
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("kat", KATS["sparse24_gpu"], ids=lambda k: k["source"].split()[-1])
def test_reference_kats_on_gpu(ctx, kat):
    w = np.array(kat["weights"], np.int8).reshape(kat["rows"], kat["cols"])
    meta, sc = frx.pack_sparse24_gpu(w, with_scales=True)
    x = np.array(kat["input"], np.float32).reshape(kat["seq"], kat["cols"])
    y = host(_run(ctx, meta, sc, x, None, "f32", "f32"))
    np.testing.assert_allclose(y.ravel(), kat["expected"], atol=kat["tol"], rtol=0)


@pytest.mark.parametrize("M,K,N", [(1, 96, 8), (4, 1024, 100), (16, 2048, 64), (1, 4100, 37), (33, 512, 130),
                                   (128, 4096, 256)])
@pytest.mark.parametrize("xt,yt", [("bf16", "f32"), ("f32", "f32"), ("bf16", "bf16")])
def test_sparse_parity_random(ctx, M, K, N, xt, yt):
    name = f"sp24/{M}x{K}x{N}"
    t = synth.sparse24_uniform(name, "w", N, K)
    meta = frx.pack_sparse24_gpu(t)
    s = synth.row_scales(name, "s", N, samples=256)
    xf, xb = synth.activations(name, "x", M, K)
    if xt == "f32":
        xf = synth.normal(7, M * K).reshape(M, K)
    ref = oracle.sparse24_gpu_matmul(meta, s, xf, M, K, N)
    y = _run(ctx, meta, s, xf, xb, xt, yt)
    if yt == "f32":
        assert_close_f32(host(y), ref)
    else:
        assert_bf16_within_1ulp(y.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("M,K,N,xt", [(1, 100, 12, "bf16"), (2, 388, 260, "bf16"), (1, 4100, 1028, "bf16"),
                                      (2, 6004, 516, "bf16"), (1, 388, 260, "f32"), (3, 4100, 8196, "f32"),
                                      (4, 8188, 4100, "f32")])
@pytest.mark.parametrize("yt", ["f32", "bf16"])
def test_sparse_decode_gemv_ragged(ctx, M, K, N, xt, yt):
    """The one-token table GEMV (1-2 bf16 tokens; 3-4 f32 tokens over >= 32 M
    codes) on ragged shapes: rows whose word count is not a multiple of 4 (a
    row's last 16-byte metadata load runs into the next row, whose words are
    cleared), a last chunk shorter than 16 words, a last row block shorter
    than 256 rows, and chunk counts on both sides of the fused reduction's
    limit (6004 columns: 16 chunks, added by the separate launch)."""
    name = f"sp24/gemv/{M}x{K}x{N}"
    t = synth.sparse24_uniform(name, "w", N, K)
    meta = frx.pack_sparse24_gpu(t)
    s = synth.row_scales(name, "s", N, samples=256)
    xf, xb = synth.activations(name, "x", M, K)
    if xt == "f32":
        xf = synth.normal(11, M * K).reshape(M, K)
    ref = oracle.sparse24_gpu_matmul(meta, s, xf, M, K, N)
    y = _run(ctx, meta, s, xf, xb, xt, yt)
    if yt == "f32":
        assert_close_f32(host(y), ref)
    else:
        assert_bf16_within_1ulp(y.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("M,K,N", [(2048, 4096, 4096), (2048, 4096, 11008), (16, 4096, 11008), (64, 11008, 512)])
def test_sparse_bit_exact_on_dyadic(ctx, M, K, N):
    """Whole output, bit for bit (dyadic x, power-of-two scales: every
    partial sum exact), including the full 2048 x 4096 x 11008 prefill."""
    rng = np.random.default_rng(M + N)
    t = synth.sparse24_uniform(f"dy/{M}", "w", N, K)
    meta = frx.pack_sparse24_gpu(t)
    x = (rng.integers(-64, 65, size=(M, K)) / 8.0).astype(np.float32)
    s = (2.0 ** rng.integers(-4, 2, size=N)).astype(np.float32)
    ref = (x @ t.T.astype(np.float32)) * s[None, :]
    y = host(_run(ctx, meta, s, x, synth.f32_to_bf16_bits(x), "bf16", "f32"))
    np.testing.assert_array_equal(y, ref)


def test_cpu_layout_through_transcoder(ctx):
    rows, cols = 64, 512
    t = synth.sparse24_uniform("tc", "w", rows, cols)
    p, sg = oracle.sparse24_cpu_from_ternary(t, rows, cols)
    meta = frx.sparse24_cpu_to_gpu(p, sg, rows, cols)
    x = synth.normal(3, 8 * cols).reshape(8, cols)
    s = np.full(rows, 0.03, np.float32)
    ref = oracle.sparse24_cpu_matmul(p, sg, 0.03, rows, cols, x, 8).reshape(8, rows)
    assert_close_f32(host(_run(ctx, meta, s, x, None, "f32", "f32")), ref)


def test_sparse_raw_metadata_patterns_6_7(ctx):
    """Raw metadata words: every 5-bit code including patterns 6 and 7
    (read as 5 by the reference) and set bits 30-31 (not part of any
    group). The prefill path (bf16, K % 64 == 0) against the oracle."""
    M, K, N = 64, 512, 256
    rng = np.random.default_rng(67)
    wpr = (K // 4 + 5) // 6
    meta = rng.integers(0, 2**32, size=(N, wpr), dtype=np.uint64).astype(np.uint32)
    s = (rng.random(N) * 0.05 + 0.01).astype(np.float32)
    xf, xb = synth.activations("sp24/raw", "x", M, K)
    xw = synth.bf16_bits_to_f32(xb)
    ref = oracle.sparse24_gpu_matmul(meta, s, xw, M, K, N)
    y = _run(ctx, meta, s, xf, xb, "bf16", "f32")
    assert_close_f32(host(y), ref)


def test_sparse_prefill_11008_sampled(ctx):
    """2:4 prefill at X[2048, 4096] x W[11008, 4096]: every output row of
    eight sampled tokens against the oracle (each row depends only on its
    token)."""
    M, K, N = 2048, 4096, 11008
    name = "sp24/prefill11008"
    t = synth.sparse24_uniform(name, "w", N, K)
    meta = frx.pack_sparse24_gpu(t)
    s = synth.row_scales(name, "s", N, samples=256)
    xf, xb = synth.activations(name, "x", M, K)
    y = host(_run(ctx, meta, s, xf, xb, "bf16", "f32"))
    rows = np.array([0, 1, 127, 128, 1000, 1919, 2046, 2047])
    xw = synth.bf16_bits_to_f32(xb)[rows]
    ref = oracle.sparse24_gpu_matmul(meta, s, np.ascontiguousarray(xw), len(rows), K, N)
    assert_close_f32(y[rows], ref.reshape(len(rows), N))


@pytest.mark.parametrize("M,K,N", [(1, 4096, 11008), (5, 11008, 4096), (16, 4096, 11008), (17, 11008, 4096),
                                   (200, 4096, 4096), (3, 2048, 300), (1600, 16384, 2048), (2, 4100, 1000),
                                   (4, 11008, 4096)])
def test_sparse_split_k_bit_exact_on_dyadic(ctx, M, K, N):
    """Decode and small prefill, where 64-token tiles leave compute units
    idle: K is split into parts of whole 64-column steps (each reading its
    own metadata windows) whose fp32 partials are added in part order. Dyadic
    inputs: every sum exact, the same bits as the unsplit kernels (split mode
    NEVER) and as the dense product, f32 and bf16 outputs."""
    rng = np.random.default_rng(5 * M + K + N)
    t = synth.sparse24_uniform(f"dysk/{M}x{K}x{N}", "w", N, K)
    meta = frx.pack_sparse24_gpu(t)
    x = (rng.integers(-64, 65, size=(M, K)) / 8.0).astype(np.float32)
    s = (2.0 ** rng.integers(-4, 2, size=N)).astype(np.float32)
    ref = (x @ t.T.astype(np.float32)) * s[None, :]
    xb = synth.f32_to_bf16_bits(x)
    np.testing.assert_array_equal(host(_run(ctx, meta, s, x, xb, "bf16", "f32")), ref)
    yb = _run(ctx, meta, s, x, xb, "bf16", "bf16")
    np.testing.assert_array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), synth.f32_to_bf16_bits(ref))
    ctx.set_gemv_split(frx.GEMV_SPLIT_NEVER)
    try:
        y0 = host(_run(ctx, meta, s, x, xb, "bf16", "f32"))
    finally:
        ctx.set_gemv_split(frx.GEMV_SPLIT_AUTO)
    np.testing.assert_array_equal(y0, ref)


@pytest.mark.parametrize("M,K,N", [(1, 4096, 512), (2, 4100, 512), (7, 4096, 512), (48, 4096, 512),
                                   (600, 4096, 512), (1024, 1024, 4096)])
def test_sparse_split_k_raw_metadata(ctx, M, K, N):
    """Raw metadata words (patterns 6 and 7, stray bits 30-31) through the
    split path (windows that straddle words at every step phase) and, from
    512 tokens, the prepared form (split and whole-K), against the oracle."""
    rng = np.random.default_rng(91 + M)
    wpr = (K // 4 + 5) // 6
    meta = rng.integers(0, 2**32, size=(N, wpr), dtype=np.uint64).astype(np.uint32)
    s = (rng.random(N) * 0.05 + 0.01).astype(np.float32)
    xf, xb = synth.activations(f"sp24/rawsk{M}", "x", M, K)
    ref = oracle.sparse24_gpu_matmul(meta, s, synth.bf16_bits_to_f32(xb), M, K, N)
    assert_close_f32(host(_run(ctx, meta, s, xf, xb, "bf16", "f32")), ref)


def _prepare(ctx, meta, K):
    N = meta.shape[0]
    prep = torch.empty((N, K // 16), dtype=torch.int32, device="cuda:0")
    ctx.sparse24_prepare(dev_u32(meta), K, prep)
    return prep


@pytest.mark.parametrize("M,K,N", [(1, 4096, 11008), (16, 1024, 300), (64, 4096, 4096), (700, 2048, 1000),
                                   (2048, 4096, 4096)])
def test_prepared_linear_bit_exact_on_dyadic(ctx, M, K, N):
    """frx_sparse24_prepare + frx_sparse24_prepared_linear: dyadic inputs give
    the exact product, and the same bits as frx_sparse24_ternary_linear,
    bf16 and f32 outputs."""
    rng = np.random.default_rng(7 * M + K + N)
    t = synth.sparse24_uniform(f"prep/{M}x{K}x{N}", "w", N, K)
    meta = frx.pack_sparse24_gpu(t)
    x = (rng.integers(-64, 65, size=(M, K)) / 8.0).astype(np.float32)
    s = (2.0 ** rng.integers(-4, 2, size=N)).astype(np.float32)
    ref = (x @ t.T.astype(np.float32)) * s[None, :]
    xb = dev_bf16(synth.f32_to_bf16_bits(x))
    prep = _prepare(ctx, meta, K)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda:0")
    ctx.sparse24_prepared_linear(prep, dev_f32(s), xb, y)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(y), ref)
    yb = torch.empty((M, N), dtype=torch.bfloat16, device="cuda:0")
    ctx.sparse24_prepared_linear(prep, dev_f32(s), xb, yb)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), synth.f32_to_bf16_bits(ref))


@pytest.mark.parametrize("M", [3, 130, 1024])
def test_prepared_linear_raw_metadata(ctx, M):
    """Raw metadata words (patterns 6 and 7, stray bits 30-31) through the
    prepared form, against the oracle and against the 5-bit entry."""
    K, N = 2048, 768
    rng = np.random.default_rng(5 + M)
    wpr = (K // 4 + 5) // 6
    meta = rng.integers(0, 2**32, size=(N, wpr), dtype=np.uint64).astype(np.uint32)
    s = (rng.random(N) * 0.05 + 0.01).astype(np.float32)
    xf, xb = synth.activations(f"sp24/prepraw{M}", "x", M, K)
    ref = oracle.sparse24_gpu_matmul(meta, s, synth.bf16_bits_to_f32(xb), M, K, N)
    prep = _prepare(ctx, meta, K)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda:0")
    ctx.sparse24_prepared_linear(prep, dev_f32(s), dev_bf16(xb), y)
    torch.cuda.synchronize()
    assert_close_f32(host(y), ref)
    y5 = host(_run(ctx, meta, s, xf, xb, "bf16", "f32"))
    if M > 16:
        np.testing.assert_array_equal(host(y), y5)


def test_prepared_entry_errors(ctx):
    """K % 64 != 0 and f32 activations are refused with a status, before any
    launch; the context stays usable."""
    N, K = 64, 256
    t = synth.sparse24_uniform("prep/err", "w", N, K)
    meta = dev_u32(frx.pack_sparse24_gpu(t))
    bad = torch.empty((N, 96 // 16), dtype=torch.int32, device="cuda:0")
    with pytest.raises(frx.FrxError) as e:
        ctx.sparse24_prepare(dev_u32(frx.pack_sparse24_gpu(synth.sparse24_uniform("prep/err96", "w", N, 96))), 96,
                             bad)
    assert e.value.kind == "Shape"
    prep = _prepare(ctx, frx.pack_sparse24_gpu(t), K)
    s = dev_f32(np.full(N, 0.5, np.float32))
    y = torch.empty((2, N), dtype=torch.float32, device="cuda:0")
    with pytest.raises(frx.FrxError) as e:
        ctx.sparse24_prepared_linear(prep, s, torch.zeros((2, K), dtype=torch.float32, device="cuda:0"), y)
    assert e.value.kind == "Unsupported"
    ctx.sparse24_prepared_linear(prep, s, torch.zeros((2, K), dtype=torch.bfloat16, device="cuda:0"), y)
    torch.cuda.synchronize()
    assert float(y.abs().max()) == 0.0
    del meta


@pytest.mark.parametrize("M,K,N", [(1, 4096, 11008), (7, 2048, 1000), (130, 4096, 512), (700, 1024, 2048),
                                   (300, 1024, 11008), (2048, 1024, 2048), (4, 4096, 11008), (3, 11008, 4096)])
def test_sparse_f32_activations_bit_exact_on_dyadic(ctx, M, K, N):
    """f32 activations (the reference's dtype) split once into bf16 hi | lo
    rows and multiplied on the sparse pipe over both halves: split over K,
    whole-K, and from 512 tokens over the prepared form. Dyadic x lies in
    the hi half: exact products and sums, f32 and bf16 outputs."""
    rng = np.random.default_rng(3 * M + K + N)
    t = synth.sparse24_uniform(f"f32sp/{M}x{K}x{N}", "w", N, K)
    meta = frx.pack_sparse24_gpu(t)
    x = (rng.integers(-64, 65, size=(M, K)) / 8.0).astype(np.float32)
    s = (2.0 ** rng.integers(-4, 2, size=N)).astype(np.float32)
    ref = (x @ t.T.astype(np.float32)) * s[None, :]
    np.testing.assert_array_equal(host(_run(ctx, meta, s, x, None, "f32", "f32")), ref)
    yb = _run(ctx, meta, s, x, None, "f32", "bf16")
    np.testing.assert_array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), synth.f32_to_bf16_bits(ref))


@pytest.mark.parametrize("M,K,N", [(3, 4096, 4096), (64, 2048, 3000), (600, 2048, 1024), (4, 4096, 11008),
                                   (1, 4100, 1000)])
def test_sparse_f32_activations_random_parity(ctx, M, K, N):
    """Genuine f32 activations (the lo half matters) against the oracle's
    sequential f32 sums, f32 and bf16 outputs."""
    name = f"sp24f32/{M}x{K}x{N}"
    t = synth.sparse24_uniform(name, "w", N, K)
    meta = frx.pack_sparse24_gpu(t)
    s = synth.row_scales(name, "s", N, samples=256)
    xf = synth.normal(synth.seed_of(name, "xf32"), M * K).reshape(M, K)
    ref = oracle.sparse24_gpu_matmul(meta, s, xf, M, K, N)
    assert_close_f32(host(_run(ctx, meta, s, xf, None, "f32", "f32")), ref)
    yb = _run(ctx, meta, s, xf, None, "f32", "bf16")
    assert_bf16_within_1ulp(yb.view(torch.int16).cpu().numpy().view(np.uint16), ref)


def test_sparse_decode_paths_repeat_and_graph(ctx):
    """The decode GEMV (chunk sums added by the last-arriving chunk, its
    arrival counters left zero by every launch; and with a separate
    reduction over long rows) and the split-K engine: back-to-back launches
    of different shapes, then replays of captured launches with eager
    launches between, every result equal to its first eager run bit for
    bit."""
    shapes = [(1, 4096, 11008), (1, 11008, 4096), (2, 4096, 4096), (16, 4096, 4096)]
    cases = []
    for M, K, N in shapes:
        name = f"sp24/graph/{M}x{K}x{N}"
        t = synth.sparse24_uniform(name, "w", N, K)
        meta = dev_u32(frx.pack_sparse24_gpu(t))
        s = dev_f32(synth.row_scales(name, "s", N, samples=256))
        _, xb = synth.activations(name, "x", M, K)
        cases.append((meta, s, dev_bf16(xb), torch.empty((M, N), dtype=torch.float32, device="cuda:0")))

    def call(i):
        meta, s, x, y = cases[i]
        ctx.sparse24_ternary_linear(meta, s, x, y)

    for i in range(len(cases)):
        call(i)
    torch.cuda.synchronize()
    refs = [host(c[3]).copy() for c in cases]
    for rep in range(12):
        call(rep % len(cases))
    torch.cuda.synchronize()
    for i, c in enumerate(cases):
        np.testing.assert_array_equal(host(c[3]), refs[i])
    st = torch.cuda.Stream()
    ctx.set_stream(st)
    try:
        graphs = []
        for i in range(3):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=st):
                call(i)
            graphs.append(g)
        torch.cuda.synchronize()
        for rep in range(4):
            for i, g in enumerate(graphs):
                cases[i][3].fill_(float("nan"))
                with torch.cuda.stream(st):
                    g.replay()
                    call(3)  # an eager launch between replays
            torch.cuda.synchronize()
            ctx.synchronize()
            for i in range(4):
                np.testing.assert_array_equal(host(cases[i][3]), refs[i])
    finally:
        ctx.set_stream(None)
