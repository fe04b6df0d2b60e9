"""frx_ternary_ffn_noalloc (intermediate in the library's fixed per-GPU
scratch array, no device allocation) against frx_ternary_ffn in two-launch
execution with the whole-K decode GEMVs (FRX_GEMV_SPLIT_NEVER: the split-K
down launch needs a workspace, so the no-allocation entry never takes it),
which runs the same kernels on a context-owned workspace: the
outputs must be identical bit for bit, and both within 1e-3 of the oracle
(dense FFN branch of cpu_block_attn_res.rs:2317-2326 with per-row scales).
Two calls in a row on one GPU, the second smaller, then a graph-captured call
replayed several times against eager results, then the size limit."""
import numpy as np
import pytest
import torch

import ferrisres_amd as frx
import oracle
from ferrisres_amd import synth
from _gpu import DEV, assert_close_f32, dev_bf16, dev_f32, dev_u32, host

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 4 << 20  # FRX_NOALLOC_SCRATCH_BYTES


def _ffn_case(name, M, H, I, xt):
    xf, xb = synth.activations(name, "x", M, H)
    mats = {}
    for mat, (n, k) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
        t = synth.ternary_uniform(name, mat, n, k)
        mats[mat] = (synth.pack_rows_u32(t), synth.row_scales(name, "s" + mat, n, samples=256))
    d = {k: (dev_u32(v[0]), dev_f32(v[1])) for k, v in mats.items()}
    x = dev_bf16(xb) if xt == "bf16" else dev_f32(xf)
    ref = oracle.ffn_forward(synth.bf16_bits_to_f32(xb) if xt == "bf16" else xf,
                             mats["gate"][0], mats["gate"][1], mats["up"][0], mats["up"][1],
                             mats["down"][0], mats["down"][1], gelu=False)
    return x, d, ref


def _args(d):
    return (d["gate"][0], d["gate"][1], d["up"][0], d["up"][1], d["down"][0], d["down"][1])


@pytest.fixture(scope="module")
def ctxs():
    assert torch.cuda.is_available(), "GPU tests need a gfx950 device"
    ref = frx.Context(0)
    ref.set_ffn_mode(frx.FFN_TWO_LAUNCH)
    ref.set_gemv_split(frx.GEMV_SPLIT_NEVER)
    na = frx.Context(0)
    yield ref, na
    na.close()
    ref.close()


# (M, H, I, x dtype): bf16 planes path (M=4), one-token rows path, the
# fp32-h path (M=3 with f32 x), the GEMM path (M=20: h and the up
# projection both in the scratch array)
CASES = [(4, 4096, 11008, "bf16"), (1, 1024, 2048, "bf16"), (3, 512, 1040, "f32"), (20, 256, 1024, "bf16")]


def test_noalloc_equals_allocating_ffn_two_calls_in_a_row(ctxs):
    ref_ctx, na = ctxs
    for (M, H, I, xt) in CASES:
        print(f"noalloc FFN case M={M} H={H} I={I} x={xt}", flush=True)
        x, d, ref = _ffn_case(f"noalloc/{M}x{H}x{I}", M, H, I, xt)
        y_ref = torch.empty((M, H), dtype=torch.float32, device=DEV)
        y_na = torch.full((M, H), float("nan"), dtype=torch.float32, device=DEV)
        ref_ctx.ternary_ffn(x, *_args(d), y_ref)
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        na.ternary_ffn_noalloc(x, *_args(d), y_na)
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free0, "the no-allocation FFN changed free device memory"
        a, b = host(y_ref), host(y_na)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), \
            f"M={M}: {(a != b).sum()} outputs differ from frx_ternary_ffn"
        assert_close_f32(b, ref.reshape(M, H))


def test_noalloc_graph_replays_match_eager(ctxs):
    ref_ctx, na = ctxs
    M, H, I = 1, 2048, 4096
    print(f"noalloc FFN graph case M={M} H={H} I={I}", flush=True)
    names = [f"noalloc/graph{r}" for r in range(3)]
    cases = [_ffn_case(n, M, H, I, "bf16") for n in names]
    x0, d, _ = cases[0]
    x = x0.clone()
    y = torch.empty((M, H), dtype=torch.float32, device=DEV)
    s = torch.cuda.Stream()
    na.set_stream(s)
    with torch.cuda.stream(s):
        na.ternary_ffn_noalloc(x, *_args(d), y)  # eager first call
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        na.ternary_ffn_noalloc(x, *_args(d), y)
    torch.cuda.synchronize()
    for r in range(3):
        xr = cases[r][0]
        with torch.cuda.stream(s):
            x.copy_(xr)
            g.replay()
        torch.cuda.synchronize()
        got = host(y).copy()
        y_e = torch.empty_like(y)
        ref_ctx.ternary_ffn(xr, *_args(d), y_e)
        torch.cuda.synchronize()
        assert np.array_equal(got.view(np.uint32), host(y_e).view(np.uint32)), f"replay {r} differs from eager"
    na.set_stream(None)
    del g


def test_noalloc_rejects_shapes_beyond_the_scratch(ctxs):
    _, na = ctxs
    M, H = 16, 64
    I = SCRATCH_BYTES // (4 * M) + 16  # M*I*4 just above the array
    x = torch.zeros((M, H), dtype=torch.bfloat16, device=DEV)
    w = torch.zeros((I, H // 16), dtype=torch.int32, device=DEV)
    wd = torch.zeros((H, I // 16), dtype=torch.int32, device=DEV)
    s = torch.zeros(I, dtype=torch.float32, device=DEV)
    sd = torch.zeros(H, dtype=torch.float32, device=DEV)
    y = torch.empty((M, H), dtype=torch.float32, device=DEV)
    with pytest.raises(frx.FrxError) as ei:
        na.ternary_ffn_noalloc(x, w, s, w, s, wd, sd, y)
    assert ei.value.kind == "Unsupported" and "scratch" in str(ei.value)
