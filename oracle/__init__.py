"""CPU oracle for the ternary linear path — TEST INFRASTRUCTURE ONLY.

Wraps oracle/libfrx_oracle.so (plain-C restatement of the reference's loops,
see frx_oracle.c) with numpy in/out. Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg may import this package, and only as the
checker or the timed CPU baseline; the product library never uses it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfrx_oracle.so")

_lib = None
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_f = ctypes.c_float


def build():
    r = subprocess.run(["make", "-C", HERE, "-s"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + r.stderr)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        h = ctypes.CDLL(LIB_PATH)
        sig = {
            "frxo_pack_ternary": (None, [_vp, _sz, _vp]),
            "frxo_unpack_ternary": (None, [_vp, _sz, _vp]),
            "frxo_pack_ternary_u32": (None, [_vp, _sz, _sz, _vp]),
            "frxo_pack_rows_u32": (None, [_vp, _sz, _sz, _vp]),
            "frxo_ternary_matmul_u32": (None, [_vp, _vp, _vp, _sz, _sz, _sz, _vp]),
            "frxo_ternary_matmul_i8": (None, [_vp, _f, _vp, _sz, _sz, _sz, _vp]),
            "frxo_ternary_matmul_decode": (None, [_vp, _f, _vp, _sz, _sz, _vp]),
            "frxo_ternary_matmul_packed": (None, [_vp, _f, _vp, _sz, _sz, _sz, _vp]),
            "frxo_ternary_matmul_packed_rows": (None, [_vp, _f, _vp, _sz, _sz, _sz, _sz, _vp]),
            "frxo_ternary_linear_forward": (None, [_vp, _vp, _f, _vp, _vp, _sz, _sz, _sz, ctypes.c_int, _vp]),
            "frxo_ternary_matmul_blocked": (None, [_vp, _vp, _sz, _vp, _sz, _sz, _sz, _vp]),
            "frxo_ternary_sparse_indices": (None, [_vp, _sz, _sz, _vp, _vp, _vp, _vp]),
            "frxo_ternary_matmul_sparse_decode": (None, [_vp, _vp, _vp, _vp, _f, _vp, _sz, _vp]),
            "frxo_ternary_stats": (_f, [_vp, _sz, _vp, _vp]),
            "frxo_moe_route_cpu_layer": (None, [_vp, _vp, _sz, _sz, _sz, _sz, _vp, _vp]),
            "frxo_moe_forward_routed": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz,
                                               ctypes.c_int, ctypes.c_int, _vp, _vp, _vp]),
            "frxo_bench_ternary_matmul": (None, [_vp, _vp, _f, _sz, _sz, _sz, _vp]),
            "frxo_quantize_ternary": (_f, [_vp, _sz, _vp]),
            "frxo_quantize_ternary_blocked": (None, [_vp, _sz, _sz, _vp, _vp]),
            "frxo_dequantize_ternary_blocked": (_sz, [_vp, _sz, _vp, _sz, _sz, _vp]),
            "frxo_prune_sparse24": (_f, [_vp, _sz, _sz, _vp, _vp]),
            "frxo_quantize_ste": (_f, [_vp, _sz, _vp]),
            "frxo_pack_sparse24_gpu": (ctypes.c_int, [_vp, _sz, _sz, _vp, _vp]),
            "frxo_sparse24_gpu_matmul": (None, [_vp, _vp, _vp, _sz, _sz, _sz, _vp]),
            "frxo_sparse24_gpu_decode": (None, [_vp, _sz, _sz, _vp]),
            "frxo_sparse24_cpu_from_ternary": (None, [_vp, _sz, _sz, _vp, _vp]),
            "frxo_sparse24_cpu_to_ternary": (None, [_vp, _vp, _sz, _sz, _vp]),
            "frxo_sparse24_cpu_matmul": (None, [_vp, _vp, _f, _sz, _sz, _vp, _sz, _vp]),
            "frxo_sparse24_cpu_matmul_decode": (None, [_vp, _vp, _f, _sz, _sz, _vp, _vp]),
            "frxo_moe_route": (None, [_vp, _vp, _sz, _sz, _sz, _sz, _vp, _vp, _vp]),
            "frxo_moe_forward": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                        _sz, _sz, _sz, _sz, _sz, ctypes.c_int, _vp, _vp, _vp]),
            "frxo_lora_forward": (None, [_vp, _vp, _sz, _sz, _sz, _f, _vp, _vp]),
            "frxo_moe_forward_lora": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz,
                                             ctypes.c_int, ctypes.c_int, _sz, _f, _vp, _vp, _vp, _vp, _vp, _vp,
                                             _vp, _vp, _vp]),
            "frxo_gelu_tanh": (_f, [_f]),
            "frxo_gelu_tanh_lit": (_f, [_f]),
            "frxo_ffn_forward": (None, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp,
                                        ctypes.c_int, _vp]),
            "frxo_time_packed_parallel": (ctypes.c_double, [_vp, _f, _vp, _sz, _sz, ctypes.c_int,
                                                            ctypes.c_int, _vp, _vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def _p(a):
    return a.ctypes.data_as(_vp)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def pack_ternary(values):
    v = _c(values, np.int8).ravel()
    out = np.zeros((v.size + 3) // 4, np.uint8)
    lib().frxo_pack_ternary(_p(v), v.size, _p(out))
    return out


def unpack_ternary(packed, n):
    p = _c(packed, np.uint8)
    out = np.zeros(n, np.int8)
    lib().frxo_unpack_ternary(_p(p), n, _p(out))
    return out


def pack_ternary_u32(packed_u8, total_values):
    p = _c(packed_u8, np.uint8)
    out = np.zeros((total_values + 15) // 16, np.uint32)
    lib().frxo_pack_ternary_u32(_p(p), p.size, total_values, _p(out))
    return out


def pack_rows_u32(values):
    v = _c(values, np.int8)
    rows, cols = v.shape
    out = np.zeros((rows, (cols + 15) // 16), np.uint32)
    lib().frxo_pack_rows_u32(_p(v), rows, cols, _p(out))
    return out


def ternary_matmul_u32(packed, scales, inp, seq, in_cols, out_rows):
    w = _c(packed, np.uint32)
    s = _c(scales, np.float32)
    x = _c(inp, np.float32)
    out = np.zeros(seq * out_rows, np.float32)
    lib().frxo_ternary_matmul_u32(_p(w), _p(s), _p(x), seq, in_cols, out_rows, _p(out))
    return out.reshape(seq, out_rows)


def ternary_matmul_i8(ternary, scale, inp, out_rows, in_cols, seq):
    t = _c(ternary, np.int8)
    x = _c(inp, np.float32)
    out = np.zeros(seq * out_rows, np.float32)
    lib().frxo_ternary_matmul_i8(_p(t), scale, _p(x), out_rows, in_cols, seq, _p(out))
    return out


def ternary_matmul_decode(ternary, scale, inp, out_rows, in_cols):
    t = _c(ternary, np.int8)
    x = _c(inp, np.float32)
    out = np.zeros(out_rows, np.float32)
    lib().frxo_ternary_matmul_decode(_p(t), scale, _p(x), out_rows, in_cols, _p(out))
    return out


def ternary_matmul_packed(packed, scale, inp, out_rows, in_cols, seq):
    p = _c(packed, np.uint8)
    x = _c(inp, np.float32)
    out = np.zeros(seq * out_rows, np.float32)
    lib().frxo_ternary_matmul_packed(_p(p), scale, _p(x), out_rows, in_cols, seq, _p(out))
    return out


def ternary_linear_forward(ternary, scale, bias, inp, out_rows, in_cols, seq, path=0):
    """TernaryLinear forward (path 0), forward_packed (1) or forward_decode (2)
    with an optional bias [out_rows] (None: no bias)."""
    t = _c(ternary, np.int8)
    pk = pack_ternary(t) if path == 1 else np.zeros(1, np.uint8)
    b = None if bias is None else _c(bias, np.float32)
    x = _c(inp, np.float32)
    n = 1 if path == 2 else seq
    out = np.zeros(n * out_rows, np.float32)
    lib().frxo_ternary_linear_forward(_p(t), _p(pk), scale, None if b is None else _p(b), _p(x),
                                      out_rows, in_cols, n, path, _p(out))
    return out.reshape(n, out_rows)


def ternary_matmul_packed_parallel(packed, scale, inp, out_rows, in_cols):
    p = _c(packed, np.uint8)
    x = _c(inp, np.float32)
    out = np.zeros(out_rows, np.float32)
    lib().frxo_ternary_matmul_packed_rows(_p(p), scale, _p(x), out_rows, in_cols, 0, out_rows, _p(out))
    return out


def ternary_matmul_blocked(ternary, scales, block_size, inp, out_rows, in_cols, seq):
    t = _c(ternary, np.int8)
    s = _c(scales, np.float32)
    x = _c(inp, np.float32)
    out = np.zeros(seq * out_rows, np.float32)
    lib().frxo_ternary_matmul_blocked(_p(t), _p(s), block_size, _p(x), out_rows, in_cols, seq, _p(out))
    return out


def bench_ternary_matmul(a, weights, scale, m, n, k):
    aa = _c(a, np.float32)
    w = _c(weights, np.int8)
    out = np.zeros(m * n, np.float32)
    lib().frxo_bench_ternary_matmul(_p(aa), _p(w), scale, m, n, k, _p(out))
    return out


def quantize_ternary(weights):
    w = _c(weights, np.float32).ravel()
    out = np.zeros(w.size, np.int8)
    alpha = lib().frxo_quantize_ternary(_p(w), w.size, _p(out))
    return out, np.float32(alpha)


def quantize_ternary_blocked(weights, block_size):
    """quantize_ternary_blocked (ternary.rs:76-110): (codes i8 [n], scales
    f32 [ceil(n / block_size)])."""
    w = _c(weights, np.float32).ravel()
    out = np.zeros(w.size, np.int8)
    scales = np.zeros(-(-w.size // block_size), np.float32)
    lib().frxo_quantize_ternary_blocked(_p(w), w.size, block_size, _p(out), _p(scales))
    return out, scales


def dequantize_ternary_blocked(ternary, scales, block_size):
    """dequantize_ternary_blocked (ternary.rs:113-128)."""
    t = _c(ternary, np.int8).ravel()
    sc = _c(scales, np.float32).ravel()
    out = np.zeros(t.size, np.float32)
    n = lib().frxo_dequantize_ternary_blocked(_p(t), t.size, _p(sc), sc.size, block_size, _p(out))
    return out[:n]


def prune_sparse24(weights, rows, cols):
    """prune_fp32_to_sparse_ternary (sparse_ternary.rs:598-663): CPU-layout
    (patterns, signs, scale)."""
    w = _c(weights, np.float32).ravel()
    ng = rows * cols // 4
    pats = np.zeros((ng + 1) // 2, np.uint8)
    signs = np.zeros((ng + 3) // 4, np.uint8)
    scale = lib().frxo_prune_sparse24(_p(w), rows, cols, _p(pats), _p(signs))
    return pats, signs, np.float32(scale)


def quantize_ste(weights):
    """BitLinear::forward_ste's quantisation (shadow_weights.rs:203-231):
    (codes i8, alpha)."""
    w = _c(weights, np.float32).reshape(-1)
    out = np.zeros(w.size, np.int8)
    a = lib().frxo_quantize_ste(_p(w), w.size, _p(out))
    return out, np.float32(a)


def pack_sparse24_gpu(weights):
    w = _c(weights, np.int8)
    rows, cols = w.shape
    wpr = ((cols + 3) // 4 + 5) // 6
    meta = np.zeros((rows, wpr), np.uint32)
    sc = np.zeros(rows, np.float32)
    rc = lib().frxo_pack_sparse24_gpu(_p(w), rows, cols, _p(meta), _p(sc))
    if rc != 0:
        raise ValueError("Each group must have exactly 2 non-zero values")
    return meta, sc


def sparse24_gpu_matmul(meta, scales, inp, seq, cols, rows):
    m = _c(meta, np.uint32)
    s = _c(scales, np.float32)
    x = _c(inp, np.float32)
    out = np.zeros(seq * rows, np.float32)
    lib().frxo_sparse24_gpu_matmul(_p(m), _p(s), _p(x), seq, cols, rows, _p(out))
    return out.reshape(seq, rows)


def sparse24_gpu_decode(meta, rows, cols):
    m = _c(meta, np.uint32)
    out = np.zeros((rows, cols), np.int8)
    lib().frxo_sparse24_gpu_decode(_p(m), rows, cols, _p(out))
    return out


def sparse24_cpu_from_ternary(ternary, rows, cols):
    t = _c(ternary, np.int8)
    ng = rows * cols // 4
    pats = np.zeros((ng + 1) // 2, np.uint8)
    signs = np.zeros((ng + 3) // 4, np.uint8)
    lib().frxo_sparse24_cpu_from_ternary(_p(t), rows, cols, _p(pats), _p(signs))
    return pats, signs


def sparse24_cpu_to_ternary(pats, signs, rows, cols):
    out = np.zeros(rows * cols, np.int8)
    lib().frxo_sparse24_cpu_to_ternary(_p(_c(pats, np.uint8)), _p(_c(signs, np.uint8)), rows, cols, _p(out))
    return out


def sparse24_cpu_matmul(pats, signs, scale, rows, cols, inp, seq):
    x = _c(inp, np.float32)
    out = np.zeros(seq * rows, np.float32)
    lib().frxo_sparse24_cpu_matmul(_p(_c(pats, np.uint8)), _p(_c(signs, np.uint8)), scale, rows, cols,
                                   _p(x), seq, _p(out))
    return out


def sparse24_cpu_matmul_decode(pats, signs, scale, rows, cols, inp):
    x = _c(inp, np.float32)
    out = np.zeros(rows, np.float32)
    lib().frxo_sparse24_cpu_matmul_decode(_p(_c(pats, np.uint8)), _p(_c(signs, np.uint8)), scale, rows,
                                          cols, _p(x), _p(out))
    return out


def ternary_sparse_indices(ternary, out_rows, in_cols):
    """ternary.rs:681-707 as CSR arrays (pos_off, pos_idx, neg_off, neg_idx)."""
    t = _c(ternary, np.int8)
    po = np.zeros(out_rows + 1, np.uint32)
    no = np.zeros(out_rows + 1, np.uint32)
    lib().frxo_ternary_sparse_indices(_p(t), out_rows, in_cols, _p(po), None, _p(no), None)
    pi = np.zeros(max(int(po[-1]), 1), np.uint32)
    ni = np.zeros(max(int(no[-1]), 1), np.uint32)
    lib().frxo_ternary_sparse_indices(_p(t), out_rows, in_cols, _p(po), _p(pi), _p(no), _p(ni))
    return po, pi[:int(po[-1])], no, ni[:int(no[-1])]


def ternary_matmul_sparse_decode(pos_off, pos_idx, neg_off, neg_idx, scale, x, out_rows):
    """ternary.rs:647-673."""
    po, no = _c(pos_off, np.uint32), _c(neg_off, np.uint32)
    pi = _c(pos_idx if len(pos_idx) else np.zeros(1), np.uint32)
    ni = _c(neg_idx if len(neg_idx) else np.zeros(1), np.uint32)
    xx = _c(x, np.float32)
    out = np.zeros(out_rows, np.float32)
    lib().frxo_ternary_matmul_sparse_decode(_p(po), _p(pi), _p(no), _p(ni), scale, _p(xx), out_rows, _p(out))
    return out


def ternary_stats(ternary):
    """ternary.rs:725-746: (counts [neg1, zero, pos1], ratios, compression)."""
    t = _c(ternary, np.int8).ravel()
    counts = np.zeros(3, np.uint64)
    ratios = np.zeros(3, np.float32)
    comp = lib().frxo_ternary_stats(_p(t), t.size, _p(counts), _p(ratios))
    return counts, ratios, float(comp)


def moe_route(x, router, top_k):
    xx = _c(x, np.float32)
    r = _c(router, np.float32)
    T, H = xx.shape
    E = r.shape[0]
    idx = np.zeros((T, top_k), np.uint32)
    w = np.zeros((T, top_k), np.float32)
    probs = np.zeros((T, E), np.float32)
    lib().frxo_moe_route(_p(xx), _p(r), T, H, E, top_k, _p(idx), _p(w), _p(probs))
    return idx, w, probs


def moe_route_cpu_layer(x, router_he, top_k):
    """CpuMoELayer routing (cpu_moe.rs:146,365-400) with the router [H][E]."""
    xx = _c(x, np.float32)
    r = _c(router_he, np.float32)
    T, H = xx.shape
    E = r.shape[1]
    idx = np.zeros((T, top_k), np.uint32)
    w = np.zeros((T, top_k), np.float32)
    lib().frxo_moe_route_cpu_layer(_p(xx), _p(r), T, H, E, top_k, _p(idx), _p(w))
    return idx, w


def moe_forward(x, router, w_gate, s_gate, w_up, s_up, w_down, s_down, top_k, gelu=False, routing=0):
    """Expert weights: lists of u32 [rows][cols/16] arrays and f32 scale arrays.
    gelu: 0 (False) silu(g)*u, 1 (True) gelu_tanh(g)*u, 2 TernaryMoELayer's
    gelu_tanh(g) without the up projection (w_up / s_up may then be None)."""
    if int(gelu) == 2 and w_up is None:
        w_up, s_up = w_gate, s_gate  # not read
    xx = _c(x, np.float32)
    r = _c(router, np.float32)
    T, H = xx.shape
    E = len(w_gate)
    if r.shape != ((H, E) if routing == 1 else (E, H)):
        raise ValueError(f"router shape {r.shape} does not match H={H}, E={E}, routing={routing}")
    I = w_gate[0].shape[0]
    keep = [_c(a, np.uint32) for a in (*w_gate, *w_up, *w_down)] + \
           [_c(a, np.float32) for a in (*s_gate, *s_up, *s_down)]

    def arr(lst):
        return (_vp * E)(*[a.ctypes.data for a in lst])
    wg, wu, wd = keep[0:E], keep[E:2 * E], keep[2 * E:3 * E]
    sg, su, sd = keep[3 * E:4 * E], keep[4 * E:5 * E], keep[5 * E:6 * E]
    out = np.zeros((T, H), np.float32)
    idx = np.zeros((T, top_k), np.uint32)
    w = np.zeros((T, top_k), np.float32)
    lib().frxo_moe_forward_routed(_p(xx), _p(r), arr(wg), arr(sg), arr(wu), arr(su), arr(wd), arr(sd),
                                  T, H, I, E, top_k, int(gelu), int(routing), _p(out), _p(idx), _p(w))
    return out, idx, w


def lora_forward(a, b, scaling, x):
    """LoraLayer::forward (lora.rs:138-167) of one position: A [rank][in],
    B [out][rank], x [in] -> [out]."""
    aa = _c(a, np.float32)
    bb = _c(b, np.float32)
    xx = _c(x, np.float32)
    rank, n_in = aa.shape
    n_out = bb.shape[0]
    out = np.zeros(n_out, np.float32)
    lib().frxo_lora_forward(_p(aa), _p(bb), rank, n_in, n_out, scaling, _p(xx), _p(out))
    return out


def moe_forward_lora(x, router, w_gate, s_gate, w_up, s_up, w_down, s_down, top_k, lora, gelu=False, routing=0):
    """moe_forward with LoRA adapters (CpuMoELayer, cpu_moe.rs:321-363).
    lora: dict with rank, scaling and per-expert lists a_gate, b_gate, a_up,
    b_up, a_down, b_down (entries None where an expert has no adapter)."""
    xx = _c(x, np.float32)
    r = _c(router, np.float32)
    T, H = xx.shape
    E = len(w_gate)
    I = w_gate[0].shape[0]
    keep = [_c(a, np.uint32) for a in (*w_gate, *w_up, *w_down)] + \
           [_c(a, np.float32) for a in (*s_gate, *s_up, *s_down)]

    def arr(lst):
        return (_vp * E)(*[a.ctypes.data for a in lst])
    wg, wu, wd = keep[0:E], keep[E:2 * E], keep[2 * E:3 * E]
    sg, su, sd = keep[3 * E:4 * E], keep[4 * E:5 * E], keep[5 * E:6 * E]
    lk = {}
    for name in ("a_gate", "b_gate", "a_up", "b_up", "a_down", "b_down"):
        mats = [None if m is None else _c(m, np.float32) for m in lora[name]]
        lk[name] = mats
    def larr(name):
        return (_vp * E)(*[None if m is None else m.ctypes.data for m in lk[name]])
    out = np.zeros((T, H), np.float32)
    idx = np.zeros((T, top_k), np.uint32)
    w = np.zeros((T, top_k), np.float32)
    lib().frxo_moe_forward_lora(_p(xx), _p(r), arr(wg), arr(sg), arr(wu), arr(su), arr(wd), arr(sd), T, H, I, E,
                                top_k, int(gelu), int(routing), int(lora["rank"]), float(lora["scaling"]),
                                larr("a_gate"), larr("b_gate"), larr("a_up"), larr("b_up"), larr("a_down"),
                                larr("b_down"), _p(out), _p(idx), _p(w))
    return out, idx, w


def ffn_forward(x, w_gate, s_gate, w_up, s_up, w_down, s_down, gelu=False):
    """Dense FFN (gate/up u32 matmuls, activation, product, down matmul), f32."""
    xx = _c(x, np.float32)
    M, H = xx.shape
    I = w_gate.shape[0]
    arrs = [_c(a, np.uint32) for a in (w_gate, w_up, w_down)] + \
           [_c(a, np.float32) for a in (s_gate, s_up, s_down)]
    out = np.zeros((M, H), np.float32)
    lib().frxo_ffn_forward(_p(xx), M, H, I, _p(arrs[0]), _p(arrs[3]), _p(arrs[1]), _p(arrs[4]),
                           _p(arrs[2]), _p(arrs[5]), int(gelu), _p(out))
    return out


def gelu_tanh(x):
    return lib().frxo_gelu_tanh(float(x))


def gelu_tanh_lit(x):
    return lib().frxo_gelu_tanh_lit(float(x))


def time_packed_parallel(packed, scale, inp, out_rows, in_cols, threads, reps, pct=None):
    """Median seconds per call over `reps` calls (and the output); a
    2-element float64 `pct` receives the 10th and 90th percentiles."""
    p = _c(packed, np.uint8)
    x = _c(inp, np.float32)
    out = np.zeros(out_rows, np.float32)
    q = None if pct is None else _p(pct)
    t = lib().frxo_time_packed_parallel(_p(p), scale, _p(x), out_rows, in_cols, threads, reps, _p(out), q)
    return t, out
