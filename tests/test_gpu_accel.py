"""Host-slice accelerator API (GpuMatmulAccelerator analogue,
src/model/gpu_forward.rs:1146-1328) on the GPU."""
import numpy as np
import pytest
import torch

import ferrisres_amd as frx
import oracle
from ferrisres_amd import synth
from _gpu import assert_close_f32, dev_f32, dev_u32

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "GPU tests need a gfx950 device"
    c = frx.Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("seq,K,N", [(1, 2048, 2048), (5, 512, 300), (40, 256, 64)])
def test_gpu_ternary_matmul_host_slices(ctx, seq, K, N):
    """Config #1 shape first: x[1,2048] f32 x W[2048,2048], per-row scales."""
    name = f"accel/{seq}x{K}x{N}"
    t = synth.ternary_uniform(name, "w", N, K)
    w = synth.pack_rows_u32(t)
    s = synth.row_scales(name, "s", N)
    x = synth.normal(synth.seed_of(name, "x"), seq * K)
    out = ctx.gpu_ternary_matmul(w.ravel(), s, x, seq, K, N)
    ref = oracle.ternary_matmul_u32(w, s, x.reshape(seq, K), seq, K, N)
    assert_close_f32(out.reshape(seq, N), ref)
    out2 = ctx.gpu_ternary_matmul_vram(dev_u32(w), dev_f32(s), x, seq, K, N)
    np.testing.assert_array_equal(out2, out)


def test_gpu_sparse_ternary_matmul_host_slices(ctx):
    t = synth.sparse24_uniform("accel/sp", "w", 96, 256)
    meta, sc = frx.pack_sparse24_gpu(t, with_scales=True)
    x = synth.normal(5, 3 * 256)
    out = ctx.gpu_sparse_ternary_matmul(meta.ravel(), sc, x, 3, 256, 96)
    ref = oracle.sparse24_gpu_matmul(meta, sc, x.reshape(3, 256), 3, 256, 96)
    assert_close_f32(out.reshape(3, 96), ref)


def test_reference_pipeline_gpu_packed(ctx):
    """CpuLinear::gpu_packed (per-tensor scale broadcast) -> GPU matmul equals
    the per-tensor CPU matmul (ternary.rs:292-328)."""
    rng = np.random.default_rng(1)
    t = rng.integers(-1, 2, size=(64, 256)).astype(np.int8)
    w, s = frx.gpu_packed(t, 0.0625)
    x = synth.normal(11, 2 * 256)
    out = ctx.gpu_ternary_matmul(w.ravel(), s, x, 2, 256, 64)
    ref = oracle.ternary_matmul_i8(t, 0.0625, x, 64, 256, 2)
    assert_close_f32(out.reshape(2, 64), ref.reshape(2, 64))


def test_empty_shape_is_an_error(ctx):
    with pytest.raises(frx.FrxError) as e:
        ctx.gpu_ternary_matmul(np.zeros(1, np.uint32), np.ones(1, np.float32), np.zeros(0, np.float32), 0, 16, 1)
    assert e.value.kind == "Shape"
