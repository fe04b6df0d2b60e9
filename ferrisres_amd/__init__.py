"""ferrisres_amd — MI355X (gfx950) ternary linear backend for FerrisRes.

The compute lives in the C-ABI library ``libfrx_ternary.so`` (HIP kernels,
header ``include/frx_ternary.h``). This module is a thin ctypes binding used
by the tests and the benchmark: it loads the library (failing loudly if it is
missing — there is no CPU fallback), maps ``frx_status`` codes to exceptions
named after the reference's ``FerrisResError`` variants (src/error.rs:4-22),
and passes torch device tensors as raw pointers.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfrx_ternary.so")

FRX_F32, FRX_BF16 = 0, 1
ACT_SILU, ACT_GELU_TANH, ACT_GELU_TANH_GATE = 0, 1, 2
GEMV_SPLIT_AUTO, GEMV_SPLIT_ALWAYS, GEMV_SPLIT_NEVER = 0, 1, 2
FFN_AUTO, FFN_ONE_LAUNCH, FFN_TWO_LAUNCH = 0, 1, 2
MOE_TERNARY_MOE_LAYER, MOE_CPU_MOE_LAYER = 0, 1
QUANT_ABSMEAN, QUANT_STE = 0, 1

_STATUS = {
    0: "Ok", 1: "Gpu", 2: "Shape", 3: "Device", 4: "Shader", 5: "OOM", 6: "Unsupported",
}


class FrxError(RuntimeError):
    """A non-OK frx_status; ``kind`` is the FerrisResError variant name."""

    def __init__(self, status: int, message: str):
        self.status = status
        self.kind = _STATUS.get(status, f"Unknown({status})")
        super().__init__(f"{self.kind} error: {message}")


_lib = None


class MoeLora(ctypes.Structure):
    """frx_moe_lora (include/frx_ternary.h)."""
    _fields_ = [("rank", ctypes.c_uint32), ("scaling", ctypes.c_float),
                ("a_gate", ctypes.c_void_p), ("b_gate", ctypes.c_void_p),
                ("a_up", ctypes.c_void_p), ("b_up", ctypes.c_void_p),
                ("a_down", ctypes.c_void_p), ("b_down", ctypes.c_void_p)]

_u32p = ctypes.POINTER(ctypes.c_uint32)
_f32p = ctypes.POINTER(ctypes.c_float)
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_u32 = ctypes.c_uint32
_int = ctypes.c_int

# name -> (restype, argtypes)
_SIGS = {
    "frx_create": (_int, [_int, ctypes.POINTER(_vp)]),
    "frx_destroy": (None, [_vp]),
    "frx_set_stream": (_int, [_vp, _vp]),
    "frx_synchronize": (_int, [_vp]),
    "frx_last_error": (ctypes.c_char_p, [_vp]),
    "frx_status_string": (ctypes.c_char_p, [_int]),
    "frx_version": (ctypes.c_char_p, []),
    "frx_ternary_linear": (_int, [_vp, _vp, _vp, _vp, _int, _vp, _int, _u32, _u32, _u32]),
    "frx_ternary_linear_bias": (_int, [_vp, _vp, _vp, _vp, _vp, _int, _vp, _int, _u32, _u32, _u32]),
    "frx_sparse24_ternary_linear": (_int, [_vp, _vp, _vp, _vp, _int, _vp, _int, _u32, _u32, _u32]),
    "frx_sparse24_prepare": (_int, [_vp, _vp, _u32, _u32, _vp]),
    "frx_sparse24_prepared_linear": (_int, [_vp, _vp, _vp, _vp, _int, _vp, _int, _u32, _u32, _u32]),
    "frx_ternary_linear_blocked": (_int, [_vp, _vp, _vp, _u32, _vp, _int, _vp, _int, _u32, _u32, _u32]),
    "frx_ternary_sparse_decode": (_int, [_vp, _vp, _vp, _vp, _vp, ctypes.c_float, _vp, _int, _vp, _int,
                                         _u32, _u32, _u32]),
    "frx_ternary_stats": (_int, [_vp, _vp, _u32, _u32, _vp]),
    "frx_ternary_sparse_indices": (_int, [_vp, _u32, _u32, _vp, _vp, _vp, _vp]),
    "frx_moe_ternary_ffn": (_int, [_vp, _vp, _int, _vp, _int, _vp, _vp, _vp, _vp, _vp, _vp,
                                   _u32, _u32, _u32, _u32, _u32, _int, _vp, _int, _vp, _vp]),
    "frx_ternary_glu": (_int, [_vp, _vp, _int, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _int, _vp]),
    "frx_ternary_ffn": (_int, [_vp, _vp, _int, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32,
                               _int, _vp, _int]),
    "frx_ternary_ffn_noalloc": (_int, [_vp, _vp, _int, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32,
                                       _int, _vp, _int]),
    "frx_set_ffn_mode": (_int, [_vp, _int]),
    "frx_set_moe_routing": (_int, [_vp, _int]),
    "frx_set_moe_lora": (_int, [_vp, _vp, _u32]),
    "frx_force_status": (_int, [_vp, _int]),
    "frx_upload_ternary": (_int, [_vp, _vp, _u32, _u32, _vp, ctypes.c_float, ctypes.POINTER(_vp),
                                  ctypes.POINTER(_vp)]),
    "frx_upload_stm": (_int, [_vp, _vp, _sz, ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_u32),
                              ctypes.POINTER(_u32)]),
    "frx_sparse24_cpu_to_gpu_device": (_int, [_vp, _vp, _vp, _u32, _u32, _vp]),
    "frx_quantize_ternary": (_int, [_vp, _vp, _int, _u32, _u32, _int, _vp, _vp]),
    "frx_quantize_ternary_blocked": (_int, [_vp, _vp, _int, _sz, _u32, _vp, _vp]),
    "frx_dequantize_ternary_blocked": (_int, [_vp, _vp, _vp, _sz, _u32, _vp]),
    "frx_prune_sparse24": (_int, [_vp, _vp, _int, _u32, _u32, _int, _vp, _vp, _vp, _vp]),
    "frx_ternary_linear_group": (_int, [_vp, _vp, _int, _u32, _u32, _u32, _vp, _vp, _vp, _vp, _int]),
    "frx_set_gemv_split": (_int, [_vp, _int]),
    "frx_workspace_stats": (_int, [_vp, ctypes.POINTER(_sz), ctypes.POINTER(_sz), ctypes.POINTER(_u32)]),
    "frx_release_retired": (_int, [_vp]),
    "frx_free": (_int, [_vp, _vp]),
    "frx_pack_ternary_u8": (_int, [_vp, _sz, _vp]),
    "frx_unpack_ternary_u8": (_int, [_vp, _sz, _vp]),
    "frx_repack_u8_to_u32": (_int, [_vp, _sz, _vp]),
    "frx_gpu_packed": (_int, [_vp, _u32, _u32, ctypes.c_float, _vp, _vp]),
    "frx_pack_sparse24_gpu": (_int, [_vp, _u32, _u32, _vp, _vp]),
    "frx_sparse24_cpu_to_gpu": (_int, [_vp, _vp, _u32, _u32, _vp]),
    "frx_gpu_ternary_matmul": (_int, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "frx_gpu_ternary_matmul_vram": (_int, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "frx_gpu_sparse_ternary_matmul": (_int, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
}


def lib():
    """Loads libfrx_ternary.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                "(there is no CPU fallback)")
        h = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def exported_symbols():
    return list(_SIGS)


def _np_ptr(a: np.ndarray):
    return a.ctypes.data_as(_vp)


def _check(status: int, ctx=None):
    if status != 0:
        msg = ""
        if ctx is not None:
            raw = lib().frx_last_error(ctx)
            msg = raw.decode() if raw else ""
        if not msg:
            msg = lib().frx_status_string(status).decode()
        raise FrxError(status, msg)


# ---- host packers (no GPU) -------------------------------------------------

def pack_ternary_u8(values: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(values, dtype=np.int8).ravel()
    out = np.zeros((v.size + 3) // 4, dtype=np.uint8)
    _check(lib().frx_pack_ternary_u8(_np_ptr(v), v.size, _np_ptr(out)))
    return out


def unpack_ternary_u8(packed: np.ndarray, n: int) -> np.ndarray:
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.zeros(n, dtype=np.int8)
    _check(lib().frx_unpack_ternary_u8(_np_ptr(p), n, _np_ptr(out)))
    return out


def repack_u8_to_u32(packed: np.ndarray, n_values: int) -> np.ndarray:
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    if p.size < (n_values + 3) // 4:
        raise ValueError("packed buffer shorter than ceil(n_values/4)")
    out = np.zeros((n_values + 15) // 16, dtype=np.uint32)
    _check(lib().frx_repack_u8_to_u32(_np_ptr(p), n_values, _np_ptr(out)))
    return out


def gpu_packed(values: np.ndarray, tensor_scale: float):
    v = np.ascontiguousarray(values, dtype=np.int8)
    n, k = v.shape
    w = np.zeros(n * k // 16, dtype=np.uint32)
    s = np.zeros(n, dtype=np.float32)
    _check(lib().frx_gpu_packed(_np_ptr(v), n, k, ctypes.c_float(tensor_scale), _np_ptr(w), _np_ptr(s)))
    return w.reshape(n, k // 16), s


def ternary_sparse_indices(values: np.ndarray):
    """frx_ternary_sparse_indices (ternary_sparse_indices, ternary.rs:681-707)
    as CSR arrays (pos_off, pos_idx, neg_off, neg_idx) for an i8 [N][K]."""
    v = np.ascontiguousarray(values, dtype=np.int8)
    n, k = v.shape
    po = np.zeros(n + 1, np.uint32)
    no = np.zeros(n + 1, np.uint32)
    _check(lib().frx_ternary_sparse_indices(_np_ptr(v), n, k, _np_ptr(po), None, _np_ptr(no), None))
    pi = np.zeros(max(int(po[-1]), 1), np.uint32)
    ni = np.zeros(max(int(no[-1]), 1), np.uint32)
    _check(lib().frx_ternary_sparse_indices(_np_ptr(v), n, k, _np_ptr(po), _np_ptr(pi), _np_ptr(no), _np_ptr(ni)))
    return po, pi, no, ni


def pack_sparse24_gpu(w: np.ndarray, with_scales: bool = False):
    v = np.ascontiguousarray(w, dtype=np.int8)
    n, k = v.shape
    wpr = ((k + 3) // 4 + 5) // 6
    meta = np.zeros(n * wpr, dtype=np.uint32)
    sc = np.zeros(n, dtype=np.float32)
    _check(lib().frx_pack_sparse24_gpu(_np_ptr(v), n, k, _np_ptr(meta),
                                       _np_ptr(sc) if with_scales else None))
    meta = meta.reshape(n, wpr)
    return (meta, sc) if with_scales else meta


def sparse24_cpu_to_gpu(patterns: np.ndarray, signs: np.ndarray, n: int, k: int) -> np.ndarray:
    p = np.ascontiguousarray(patterns, dtype=np.uint8)
    s = np.ascontiguousarray(signs, dtype=np.uint8)
    wpr = (k // 4 + 5) // 6
    meta = np.zeros(n * wpr, dtype=np.uint32)
    _check(lib().frx_sparse24_cpu_to_gpu(_np_ptr(p), _np_ptr(s), n, k, _np_ptr(meta)))
    return meta.reshape(n, wpr)


# ---- device context ----------------------------------------------------------

def _dtype_code(t) -> int:
    import torch
    if t.dtype == torch.float32:
        return FRX_F32
    if t.dtype == torch.bfloat16:
        return FRX_BF16
    raise TypeError(f"unsupported dtype {t.dtype}")


def _numel(t):
    if hasattr(t, "numel"):
        return int(t.numel())
    return int(np.prod(t.shape))


def _shape_err(msg):
    return FrxError(2, msg)


def _shape2(t, name):
    if len(t.shape) != 2:
        raise _shape_err(f"{name} must be 2-D, got shape {tuple(t.shape)}")
    return int(t.shape[0]), int(t.shape[1])


def _rows(t, words_per_row, name):
    """Rows of a packed matrix whose rows hold words_per_row u32 words."""
    n = _numel(t)
    if words_per_row <= 0 or n % words_per_row:
        raise _shape_err(f"{name} holds {n} words, not a multiple of {words_per_row} per row")
    return n // words_per_row


def _expect_numel(t, n, name):
    if t is not None and _numel(t) < n:
        raise _shape_err(f"{name} holds {_numel(t)} elements, needs {n}")


def _expect_shape(t, shape, name):
    if tuple(int(d) for d in t.shape) != tuple(shape):
        raise _shape_err(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")


def _ptr(t):
    """Device address of a tensor, a DeviceBuffer or a raw integer address."""
    if t is None:
        return None
    if isinstance(t, int):
        return _vp(t)
    return _vp(t.data_ptr())


class DeviceBuffer:
    """Device memory allocated by the library (frx_upload_*); released with
    frx_free on close() or when the owning context closes it. data_ptr()
    gives the address, so it can be passed wherever a tensor is."""

    def __init__(self, ctx, addr: int, nbytes: int, shape):
        self._ctx, self.addr, self.nbytes, self.shape = ctx, addr, nbytes, tuple(shape)

    def data_ptr(self) -> int:
        return self.addr

    def close(self):
        if self.addr:
            _check(lib().frx_free(self._ctx._h, _vp(self.addr)), self._ctx._h)
            self.addr = 0


class Context:
    """Owns an frx_ctx bound to one device and (optionally) a torch stream."""

    def __init__(self, device: int = 0, stream=None):
        h = _vp()
        _check(lib().frx_create(device, ctypes.byref(h)))
        self._h = h
        if stream is not None:
            self.set_stream(stream)

    def close(self):
        if getattr(self, "_h", None):
            lib().frx_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_stream(self, stream):
        raw = stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream or 0)
        _check(lib().frx_set_stream(self._h, _vp(raw)), self._h)

    def synchronize(self):
        _check(lib().frx_synchronize(self._h), self._h)

    # TernaryMatMulOp::dispatch analogue; all tensors on the device.
    def ternary_linear(self, w, scale, x, y, bias=None):
        """frx_ternary_linear; with bias ([N] f32) frx_ternary_linear_bias
        (TernaryLinear::forward with a bias, ternary_linear.rs:94-115)."""
        M, K = _shape2(x, "x")
        N = _rows(w, K // 16, "w") if K % 16 == 0 else int(w.shape[0])
        _expect_numel(scale, N, "scale")
        _expect_shape(y, (M, N), "y")
        if bias is not None:
            _expect_numel(bias, N, "bias")
            if _dtype_code(bias) != FRX_F32:
                raise TypeError("bias must be float32")
            _check(lib().frx_ternary_linear_bias(self._h, _ptr(w), _ptr(scale), _ptr(bias), _ptr(x),
                                                 _dtype_code(x), _ptr(y), _dtype_code(y), M, K, N), self._h)
            return y
        _check(lib().frx_ternary_linear(self._h, _ptr(w), _ptr(scale), _ptr(x), _dtype_code(x),
                                        _ptr(y), _dtype_code(y), M, K, N), self._h)
        return y

    def ternary_linear_group(self, x, ws, scales, ys):
        """frx_ternary_linear_group: y_i = x W_i^T * s_i for up to four
        matrices with the same K against one x (one launch at one token)."""
        M, K = _shape2(x, "x")
        count = len(ws)
        if not (len(scales) == len(ys) == count):
            raise _shape_err("ws, scales and ys must have the same length")
        Ns = []
        for i, (w, sc, y) in enumerate(zip(ws, scales, ys)):
            n = _rows(w, K // 16, f"w[{i}]") if K % 16 == 0 else int(w.shape[0])
            _expect_numel(sc, n, f"scale[{i}]")
            _expect_shape(y, (M, n), f"y[{i}]")
            Ns.append(n)
        arr = lambda ts: (_vp * max(count, 1))(*[t.data_ptr() for t in ts])  # noqa: E731
        ydt = _dtype_code(ys[0]) if ys else FRX_F32
        if any(_dtype_code(y) != ydt for y in ys):
            raise TypeError("all outputs of a group must have the same dtype")
        _check(lib().frx_ternary_linear_group(self._h, _ptr(x), _dtype_code(x), M, K, count, arr(ws), arr(scales),
                                              (_u32 * max(count, 1))(*Ns), arr(ys), ydt), self._h)
        return ys

    def sparse24_ternary_linear(self, meta, scale, x, y):
        M, K = _shape2(x, "x")
        N = _rows(meta, ((K + 3) // 4 + 5) // 6, "meta")
        _expect_numel(scale, N, "scale")
        _expect_shape(y, (M, N), "y")
        _check(lib().frx_sparse24_ternary_linear(self._h, _ptr(meta), _ptr(scale), _ptr(x),
                                                 _dtype_code(x), _ptr(y), _dtype_code(y), M, K, N),
               self._h)
        return y

    def sparse24_prepare(self, meta, K: int, prepared):
        """frx_sparse24_prepare: 2:4 metadata [N][ceil(ceil(K/4)/6)] u32 into
        its prepared form [N][K/16] u32 (K % 64 == 0)."""
        N = _rows(meta, ((K + 3) // 4 + 5) // 6, "meta")
        _expect_numel(prepared, N * (K // 16), "prepared")
        _check(lib().frx_sparse24_prepare(self._h, _ptr(meta), K, N, _ptr(prepared)), self._h)
        return prepared

    def sparse24_prepared_linear(self, prepared, scale, x, y):
        """frx_sparse24_prepared_linear: the 2:4 linear over prepared
        metadata (bf16 x)."""
        M, K = _shape2(x, "x")
        N = _rows(prepared, K // 16, "prepared")
        _expect_numel(scale, N, "scale")
        _expect_shape(y, (M, N), "y")
        _check(lib().frx_sparse24_prepared_linear(self._h, _ptr(prepared), _ptr(scale), _ptr(x), _dtype_code(x),
                                                  _ptr(y), _dtype_code(y), M, K, N), self._h)
        return y

    def ternary_linear_blocked(self, w, block_scales, block_size: int, x, y):
        """frx_ternary_linear_blocked (ternary_matmul_blocked, ternary.rs:541-579)."""
        M, K = _shape2(x, "x")
        N = _rows(w, K // 16, "w")
        if block_size > 0:
            _expect_numel(block_scales, (K + block_size - 1) // block_size, "block_scales")
        _expect_shape(y, (M, N), "y")
        _check(lib().frx_ternary_linear_blocked(self._h, _ptr(w), _ptr(block_scales), block_size, _ptr(x),
                                                _dtype_code(x), _ptr(y), _dtype_code(y), M, K, N), self._h)
        return y

    def ternary_sparse_decode(self, pos_off, pos_idx, neg_off, neg_idx, scale: float, x, y):
        """frx_ternary_sparse_decode (ternary_matmul_sparse_decode, ternary.rs:647-673)."""
        M, K = _shape2(x, "x")
        N = y.shape[-1]
        _expect_shape(y, (M, N), "y")
        _expect_numel(pos_off, N + 1, "pos_off")
        _expect_numel(neg_off, N + 1, "neg_off")
        _check(lib().frx_ternary_sparse_decode(self._h, _ptr(pos_off), _ptr(pos_idx), _ptr(neg_off), _ptr(neg_idx),
                                               ctypes.c_float(scale), _ptr(x), _dtype_code(x), _ptr(y),
                                               _dtype_code(y), M, K, N), self._h)
        return y

    def ternary_stats(self, w, K: int, counts):
        """frx_ternary_stats: counts (3 x u64 on the device) of -1, 0, +1 codes."""
        N = _rows(w, K // 16, "w")
        _expect_numel(counts, 3, "counts")
        _check(lib().frx_ternary_stats(self._h, _ptr(w), N, K, _ptr(counts)), self._h)
        return counts

    def moe_ternary_ffn(self, x, router, w_gate, s_gate, w_up, s_up, w_down, s_down, y,
                        top_k: int, act: int = ACT_SILU, topk_idx=None, topk_w=None):
        T, H = _shape2(x, "x")
        E = len(w_gate)
        _expect_numel(router, E * H, "router")
        I = _rows(w_gate[0], H // 16, "w_gate[0]") if H % 16 == 0 else int(w_gate[0].shape[0])
        _expect_shape(y, (T, H), "y")
        arr = lambda ts: None if ts is None else (_vp * E)(*[t.data_ptr() for t in ts])  # noqa: E731
        _check(lib().frx_moe_ternary_ffn(
            self._h, _ptr(x), _dtype_code(x), _ptr(router), _dtype_code(router),
            arr(w_gate), arr(s_gate), arr(w_up), arr(s_up), arr(w_down), arr(s_down),
            T, H, I, E, top_k, act, _ptr(y), _dtype_code(y), _ptr(topk_idx), _ptr(topk_w)),
            self._h)
        return y

    def ternary_glu(self, x, w_gate, s_gate, w_up, s_up, h, act: int = ACT_SILU):
        """h (fp32) = act(x Wg^T s_gate) * (x Wu^T s_up)."""
        M, H = x.shape
        I = w_gate.shape[0]
        _check(lib().frx_ternary_glu(self._h, _ptr(x), _dtype_code(x), _ptr(w_gate), _ptr(s_gate),
                                     _ptr(w_up), _ptr(s_up), M, H, I, act, _ptr(h)), self._h)
        return h

    def ternary_ffn(self, x, w_gate, s_gate, w_up, s_up, w_down, s_down, y, act: int = ACT_SILU):
        """Dense FFN: y = (act(x Wg^T s_gate) * (x Wu^T s_up)) Wd^T s_down."""
        M, H = x.shape
        I = w_gate.shape[0]
        _check(lib().frx_ternary_ffn(self._h, _ptr(x), _dtype_code(x), _ptr(w_gate), _ptr(s_gate),
                                     _ptr(w_up), _ptr(s_up), _ptr(w_down), _ptr(s_down), M, H, I,
                                     act, _ptr(y), _dtype_code(y)), self._h)
        return y

    def ternary_ffn_noalloc(self, x, w_gate, s_gate, w_up, s_up, w_down, s_down, y, act: int = ACT_SILU):
        """frx_ternary_ffn_noalloc: the dense FFN with its intermediate in the
        library's fixed per-GPU scratch array (no device allocation)."""
        M, H = x.shape
        I = w_gate.shape[0]
        _check(lib().frx_ternary_ffn_noalloc(self._h, _ptr(x), _dtype_code(x), _ptr(w_gate), _ptr(s_gate),
                                             _ptr(w_up), _ptr(s_up), _ptr(w_down), _ptr(s_down), M, H, I,
                                             act, _ptr(y), _dtype_code(y)), self._h)
        return y

    # Weight ingest: resident device copies in the GPU layout.
    def upload_ternary(self, packed_u8: np.ndarray, N: int, K: int, row_scales=None, tensor_scale: float = 1.0):
        """frx_upload_ternary: pack_ternary bytes [N*K/4] -> (w [N][K/16] u32,
        scales [N] f32) on the device, as DeviceBuffers."""
        p = np.ascontiguousarray(packed_u8, dtype=np.uint8)
        rs = None if row_scales is None else np.ascontiguousarray(row_scales, dtype=np.float32)
        w, sc = _vp(), _vp()
        _check(lib().frx_upload_ternary(self._h, p.ctypes.data_as(_vp), N, K,
                                        None if rs is None else rs.ctypes.data_as(_vp),
                                        ctypes.c_float(tensor_scale), ctypes.byref(w), ctypes.byref(sc)), self._h)
        return DeviceBuffer(self, w.value, N * K // 4, (N, K // 16)), DeviceBuffer(self, sc.value, 4 * N, (N,))

    def upload_stm(self, image: bytes):
        """frx_upload_stm: an .stm file image -> (meta [N][ceil(K/24)] u32,
        scales [N] f32) on the device, plus (N, K)."""
        buf = np.frombuffer(bytes(image), dtype=np.uint8)
        m, sc, n, k = _vp(), _vp(), _u32(), _u32()
        _check(lib().frx_upload_stm(self._h, buf.ctypes.data_as(_vp), buf.size, ctypes.byref(m),
                                    ctypes.byref(sc), ctypes.byref(n), ctypes.byref(k)), self._h)
        N, K = n.value, k.value
        wpr = (K // 4 + 5) // 6
        return (DeviceBuffer(self, m.value, 4 * N * wpr, (N, wpr)), DeviceBuffer(self, sc.value, 4 * N, (N,)), N, K)

    def sparse24_cpu_to_gpu_device(self, patterns, signs, N: int, K: int, meta):
        """frx_sparse24_cpu_to_gpu_device on device tensors (stream-ordered)."""
        _check(lib().frx_sparse24_cpu_to_gpu_device(self._h, _ptr(patterns), _ptr(signs), N, K, _ptr(meta)),
               self._h)
        return meta

    def quantize_ternary(self, w, rule: int, packed, scale):
        """frx_quantize_ternary: each row of w [N][K] (f32 or bf16 device
        tensor) quantised on its own (QUANT_ABSMEAN: quantize_ternary,
        ternary.rs:31-57; QUANT_STE: BitLinear::forward_ste,
        shadow_weights.rs:203-231) into packed [N][K/16] u32 codes and
        scale [N] f32. Stream-ordered."""
        N, K = w.shape
        _check(lib().frx_quantize_ternary(self._h, _ptr(w), _dtype_code(w), N, K, rule, _ptr(packed),
                                          _ptr(scale)), self._h)
        return packed, scale

    def quantize_ternary_blocked(self, w, block_size: int, packed, scales):
        """frx_quantize_ternary_blocked: the flat tensor w (f32 or bf16
        device tensor, n values) in blocks of block_size values, each with
        its own absmean alpha (quantize_ternary_blocked, ternary.rs:76-110),
        into packed [ceil(n/16)] u32 codes and scales [ceil(n/block)] f32."""
        n = int(w.numel())
        _expect_numel(packed, -(-n // 16), "packed")
        _expect_numel(scales, -(-n // block_size) if block_size else 0, "scales")
        _check(lib().frx_quantize_ternary_blocked(self._h, _ptr(w), _dtype_code(w), n, block_size, _ptr(packed),
                                                  _ptr(scales)), self._h)
        return packed, scales

    def dequantize_ternary_blocked(self, packed, scales, n: int, block_size: int, out):
        """frx_dequantize_ternary_blocked: out[i] = scales[i / block] *
        dec(code i) (dequantize_ternary_blocked, ternary.rs:113-128)."""
        _expect_numel(out, n, "out")
        _check(lib().frx_dequantize_ternary_blocked(self._h, _ptr(packed), _ptr(scales), n, block_size,
                                                    _ptr(out)), self._h)
        return out

    def prune_sparse24(self, w, scale, patterns=None, signs=None, meta=None, per_row: bool = False):
        """frx_prune_sparse24: prune_fp32_to_sparse_ternary
        (sparse_ternary.rs:598-663) of w [N][K] (f32 or bf16 device tensor)
        into the CPU layout (patterns, signs) and / or the GPU layout (meta
        [N][ceil(K/24)]), scale [N] f32 (the tensor scale on every row, or
        one per row)."""
        N, K = _shape2(w, "w")
        _expect_numel(scale, N, "scale")
        _check(lib().frx_prune_sparse24(self._h, _ptr(w), _dtype_code(w), N, K, int(per_row), _ptr(patterns),
                                        _ptr(signs), _ptr(meta), _ptr(scale)), self._h)
        return patterns, signs, meta, scale

    def set_gemv_split(self, mode: int):
        """frx_set_gemv_split: GEMV_SPLIT_AUTO, _ALWAYS or _NEVER (the
        split-K decode GEMV at 2-16 tokens)."""
        _check(lib().frx_set_gemv_split(self._h, mode), self._h)

    def workspace_stats(self):
        """frx_workspace_stats: (live bytes, retired bytes, allocations)."""
        live, ret, n = _sz(0), _sz(0), _u32(0)
        _check(lib().frx_workspace_stats(self._h, ctypes.byref(live), ctypes.byref(ret), ctypes.byref(n)), self._h)
        return int(live.value), int(ret.value), int(n.value)

    def release_retired(self):
        """frx_release_retired: frees workspaces replaced by larger ones."""
        _check(lib().frx_release_retired(self._h), self._h)

    def set_moe_routing(self, routing: int):
        """frx_set_moe_routing: MOE_TERNARY_MOE_LAYER (router [E,H], default)
        or MOE_CPU_MOE_LAYER (CpuMoELayer: router [H,E], top-k by logit)."""
        _check(lib().frx_set_moe_routing(self._h, routing), self._h)

    def set_moe_lora(self, rank=None, scaling=0.0, experts=0, a_gate=None, b_gate=None, a_up=None, b_up=None,
                     a_down=None, b_down=None):
        """frx_set_moe_lora: per-expert LoRA adapters of the MoE experts
        (lists of ``experts`` f32 device tensors or None; a list may be None).
        rank=None removes the adapters."""
        if rank is None:
            _check(lib().frx_set_moe_lora(self._h, None, 0), self._h)
            return
        for name, lst in (("a_gate", a_gate), ("b_gate", b_gate), ("a_up", a_up), ("b_up", b_up),
                          ("a_down", a_down), ("b_down", b_down)):
            for t in (lst or []):
                if t is not None and (t.dtype.__str__() != "torch.float32" or not t.is_contiguous()):
                    raise ValueError(f"{name}: LoRA matrices are contiguous float32 device tensors")
        keep = []

        def arr(lst):
            if lst is None:
                return None
            if len(lst) != experts:
                raise ValueError("one LoRA matrix (or None) per expert")
            a = (_vp * experts)(*[None if t is None else t.data_ptr() for t in lst])
            keep.append(a)
            return ctypes.cast(a, _vp)
        cfg = MoeLora(int(rank), float(scaling), arr(a_gate), arr(b_gate), arr(a_up), arr(b_up), arr(a_down),
                      arr(b_down))
        _check(lib().frx_set_moe_lora(self._h, ctypes.byref(cfg), int(experts)), self._h)

    def force_status(self, status: int):
        """frx_force_status: every compute / upload call on this context
        returns ``status`` (raised here as FrxError) until it is set to 0."""
        _check(lib().frx_force_status(self._h, status), self._h)

    def set_ffn_mode(self, mode: int):
        """frx_set_ffn_mode: FFN_AUTO, FFN_ONE_LAUNCH or FFN_TWO_LAUNCH."""
        _check(lib().frx_set_ffn_mode(self._h, mode), self._h)

    # GpuMatmulAccelerator analogues: host numpy in, host numpy out.
    def gpu_ternary_matmul(self, packed_weights: np.ndarray, scales: np.ndarray,
                           inp: np.ndarray, seq_len: int, in_cols: int, out_rows: int):
        w = np.ascontiguousarray(packed_weights, dtype=np.uint32)
        s = np.ascontiguousarray(scales, dtype=np.float32)
        x = np.ascontiguousarray(inp, dtype=np.float32)
        out = np.zeros(seq_len * out_rows, dtype=np.float32)
        _check(lib().frx_gpu_ternary_matmul(self._h, _np_ptr(w), _np_ptr(s), _np_ptr(x),
                                            seq_len, in_cols, out_rows, _np_ptr(out)), self._h)
        return out

    def gpu_ternary_matmul_vram(self, w_dev, s_dev, inp: np.ndarray, seq_len: int, in_cols: int,
                                out_rows: int):
        x = np.ascontiguousarray(inp, dtype=np.float32)
        out = np.zeros(seq_len * out_rows, dtype=np.float32)
        _check(lib().frx_gpu_ternary_matmul_vram(self._h, _ptr(w_dev), _ptr(s_dev), _np_ptr(x),
                                                 seq_len, in_cols, out_rows, _np_ptr(out)), self._h)
        return out

    def gpu_sparse_ternary_matmul(self, meta: np.ndarray, scales: np.ndarray, inp: np.ndarray,
                                  seq_len: int, in_cols: int, out_rows: int):
        m = np.ascontiguousarray(meta, dtype=np.uint32)
        s = np.ascontiguousarray(scales, dtype=np.float32)
        x = np.ascontiguousarray(inp, dtype=np.float32)
        out = np.zeros(seq_len * out_rows, dtype=np.float32)
        _check(lib().frx_gpu_sparse_ternary_matmul(self._h, _np_ptr(m), _np_ptr(s), _np_ptr(x),
                                                   seq_len, in_cols, out_rows, _np_ptr(out)),
               self._h)
        return out
