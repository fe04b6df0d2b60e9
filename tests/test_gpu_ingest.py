"""Weight ingest on the GPU: resident uploads of the dense packed layout and
of .stm 2:4 expert images (src/model/expert_loader.rs:6-152), and the device
CPU->GPU 2:4 transcoder, checked bit-exactly against the host packers and
through the matmul against the oracle."""
import ctypes
import struct

import numpy as np
import pytest
import torch

import ferrisres_amd as frx
import oracle
from ferrisres_amd import synth
from _gpu import DEV, assert_close_f32, dev_f32, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "GPU tests need a gfx950 device"
    c = frx.Context(0)
    yield c
    c.close()


def read_device(buf, dtype, count):
    """Copies count elements of a library-owned device buffer to the host."""
    t = torch.empty(count, dtype=dtype, device=DEV)
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hip.hipMemcpy(ctypes.c_void_p(t.data_ptr()), ctypes.c_void_p(buf.data_ptr()),
                         t.numel() * t.element_size(), 3) == 0  # device to device
    torch.cuda.synchronize()
    return t.cpu().numpy()


def stm_image(patterns, signs, rows, cols, scale):
    """An .stm file image as write_stm_file lays it out (expert_loader.rs:45-60)."""
    hdr = struct.pack("<IIIfII", 0x53544D31, rows, cols, scale, len(patterns), len(signs))
    return hdr + bytes(patterns) + bytes(signs)


@pytest.mark.parametrize("per_row", [True, False])
def test_upload_ternary_dense(ctx, per_row):
    N, K, M = 300, 512, 5
    t = synth.ternary_uniform("ingest", "w", N, K)
    packed = oracle.pack_ternary(t.ravel())
    rs = synth.row_scales("ingest", "s", N, samples=64) if per_row else None
    w, s = ctx.upload_ternary(packed, N, K, row_scales=rs, tensor_scale=0.0375)
    try:
        words = read_device(w, torch.int32, N * K // 16).view(np.uint32)
        np.testing.assert_array_equal(words, oracle.pack_rows_u32(t).ravel())
        sc = read_device(s, torch.float32, N)
        np.testing.assert_array_equal(sc, rs if per_row else np.full(N, 0.0375, np.float32))
        x = synth.normal(5, M * K).reshape(M, K)
        y = torch.empty((M, N), dtype=torch.float32, device=DEV)
        ctx.ternary_linear(w, s, dev_f32(x), y)
        torch.cuda.synchronize()
        ref = oracle.ternary_matmul_u32(oracle.pack_rows_u32(t), sc, x, M, K, N).reshape(M, N)
        assert_close_f32(host(y), ref)
    finally:
        w.close()
        s.close()


def test_upload_ternary_rejects_unaligned_k(ctx):
    with pytest.raises(frx.FrxError) as e:
        ctx.upload_ternary(np.zeros(10, np.uint8), 2, 20)
    assert e.value.kind == "Shape"


@pytest.mark.parametrize("rows,cols", [(64, 512), (37, 1000), (1, 4)])
def test_device_transcoder_matches_host(ctx, rows, cols):
    rng = np.random.default_rng(rows + cols)
    ng = rows * cols // 4
    p = rng.integers(0, 256, size=(ng + 1) // 2, dtype=np.uint8)
    s = rng.integers(0, 256, size=(ng + 3) // 4, dtype=np.uint8)
    ref = frx.sparse24_cpu_to_gpu(p, s, rows, cols)
    meta = torch.full(ref.shape, -1, dtype=torch.int32, device=DEV)
    ctx.sparse24_cpu_to_gpu_device(torch.from_numpy(p).to(DEV), torch.from_numpy(s).to(DEV), rows, cols, meta)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(meta.cpu().numpy().view(np.uint32), ref)


def test_upload_stm_end_to_end(ctx):
    """An .stm expert built from a 2:4 matrix: uploaded, transcoded on the
    device, multiplied; equals the reference CPU 2:4 matmul
    (sparse_ternary.rs:203-252, per-tensor scale)."""
    rows, cols, M = 256, 1024, 7
    t = synth.sparse24_uniform("stm", "w", rows, cols)
    p, s = oracle.sparse24_cpu_from_ternary(t, rows, cols)
    img = stm_image(p, s, rows, cols, 0.04)
    meta, sc, N, K = ctx.upload_stm(img)
    try:
        assert (N, K) == (rows, cols)
        np.testing.assert_array_equal(read_device(meta, torch.int32, meta.nbytes // 4).view(np.uint32),
                                      frx.sparse24_cpu_to_gpu(p, s, rows, cols).ravel())
        x = synth.normal(9, M * cols).reshape(M, cols)
        y = torch.empty((M, rows), dtype=torch.float32, device=DEV)
        ctx.sparse24_ternary_linear(meta, sc, dev_f32(x), y)
        torch.cuda.synchronize()
        ref = oracle.sparse24_cpu_matmul(p, s, 0.04, rows, cols, x, M).reshape(M, rows)
        assert_close_f32(host(y), ref)
    finally:
        meta.close()
        sc.close()


@pytest.mark.parametrize("case", ["short", "magic", "truncated", "cols", "arrays"])
def test_upload_stm_rejects_bad_images(ctx, case):
    rows, cols = 8, 64
    ng = rows * cols // 4
    p, s = bytes((ng + 1) // 2), bytes((ng + 3) // 4)
    img = stm_image(p, s, rows, cols, 1.0)
    if case == "short":
        img = img[:20]
    elif case == "magic":
        img = b"XTM1" + img[4:]
    elif case == "truncated":
        img = img[:-1]
    elif case == "cols":
        img = stm_image(p, s, rows, 66, 1.0)
    else:
        img = stm_image(p[:-1], s, rows, cols, 1.0)
    with pytest.raises(frx.FrxError) as e:
        ctx.upload_stm(img)
    assert e.value.kind == "Shape"
