"""Pins the oracle beyond the reference KATs: exact-arithmetic identities,
float64 brute force, independent numpy restatements and layout round trips.
Each check is chosen so a plausible mistake (dropped term, wrong sign or
index, transposed operand, wrong code table) fails it."""
import numpy as np
import pytest

import oracle
from ferrisres_amd import synth


def _dyadic(rng, shape):
    # small integers / 8: every partial sum of <= 2^16 terms is exact in f32
    return (rng.integers(-64, 65, size=shape) / 8.0).astype(np.float32)


def _dense_f64(t, x, scales):
    return (x.astype(np.float64) @ t.astype(np.float64).T) * scales.astype(np.float64)[None, :]


@pytest.mark.parametrize("m,k,n", [(1, 16, 8), (3, 48, 5), (7, 256, 33), (2, 1024, 64)])
def test_u32_matmul_exact_on_dyadic(m, k, n):
    rng = np.random.default_rng(m * 1000 + k + n)
    t = rng.integers(-1, 2, size=(n, k)).astype(np.int8)
    x = _dyadic(rng, (m, k))
    sc = (2.0 ** rng.integers(-3, 3, size=n)).astype(np.float32)  # exact scales
    out = oracle.ternary_matmul_u32(oracle.pack_rows_u32(t), sc, x, m, k, n)
    np.testing.assert_array_equal(out, _dense_f64(t, x, sc).astype(np.float32))


def test_u32_matmul_code3_decodes_to_zero():
    # word with code 3 everywhere plus a single +1 at column 5
    w = np.full((1, 1), 0xFFFFFFFF, np.uint32)
    w[0, 0] &= ~np.uint32(3 << 10)
    w[0, 0] |= np.uint32(2 << 10)
    x = np.arange(16, dtype=np.float32)[None, :] + 1
    out = oracle.ternary_matmul_u32(w, np.ones(1, np.float32), x, 1, 16, 1)
    assert out[0, 0] == 6.0


@pytest.mark.parametrize("seed", [1, 2])
def test_u32_matmul_random_vs_f64(seed):
    rng = np.random.default_rng(seed)
    m, k, n = 4, 2048, 96
    t = rng.integers(-1, 2, size=(n, k)).astype(np.int8)
    x = rng.standard_normal((m, k)).astype(np.float32)
    sc = np.abs(rng.standard_normal(n)).astype(np.float32) * 0.02
    out = oracle.ternary_matmul_u32(oracle.pack_rows_u32(t), sc, x, m, k, n).astype(np.float64)
    ref = _dense_f64(t, x, sc)
    rms = np.sqrt((ref ** 2).mean())
    assert np.abs(out - ref).max() <= 1e-5 * rms


def test_all_cpu_matmul_variants_agree_exactly_on_dyadic():
    rng = np.random.default_rng(7)
    n, k = 24, 64
    t = rng.integers(-1, 2, size=(n, k)).astype(np.int8)
    x = _dyadic(rng, (1, k))
    scale = np.float32(0.5)
    ref = _dense_f64(t, x, np.full(n, scale, np.float32)).astype(np.float32).ravel()
    u32 = oracle.ternary_matmul_u32(oracle.pack_rows_u32(t), np.full(n, scale, np.float32), x, 1, k, n).ravel()
    i8 = oracle.ternary_matmul_i8(t, scale, x, n, k, 1)
    dec = oracle.ternary_matmul_decode(t, scale, x, n, k)
    packed = oracle.pack_ternary(t)
    pk = oracle.ternary_matmul_packed(packed, scale, x, n, k, 1)
    pp = oracle.ternary_matmul_packed_parallel(packed, scale, x, n, k)
    bench = oracle.bench_ternary_matmul(x, t, scale, 1, n, k)
    for got in (u32, i8, dec, pk, pp, bench):
        np.testing.assert_array_equal(got, ref)


def test_blocked_matmul_vs_f64():
    rng = np.random.default_rng(3)
    n, k, bs = 8, 40, 16
    t = rng.integers(-1, 2, size=(n, k)).astype(np.int8)
    x = _dyadic(rng, (2, k))
    sc = np.array([0.5, 0.25, 2.0], np.float32)
    out = oracle.ternary_matmul_blocked(t, sc, bs, x, n, k, 2).reshape(2, n)
    ref = np.zeros((2, n))
    for b in range(3):
        c0, c1 = b * bs, min(k, (b + 1) * bs)
        ref += sc[b] * (x[:, c0:c1].astype(np.float64) @ t[:, c0:c1].T.astype(np.float64))
    np.testing.assert_array_equal(out, ref.astype(np.float32))


def test_pack_u8_bit_spec():
    rng = np.random.default_rng(11)
    v = rng.integers(-1, 2, size=1001).astype(np.int8)
    p = oracle.pack_ternary(v)
    code = np.where(v == -1, 0, np.where(v == 1, 2, 1))
    for i in range(v.size):
        assert (p[i // 4] >> (2 * (i % 4))) & 3 == code[i]
    # padding bits of the last byte are zero
    assert p[-1] >> (2 * (v.size % 4)) == 0


def test_pack_u8_out_of_range_is_zero_code():
    p = oracle.pack_ternary(np.array([5, -7, 1, -1], np.int8))
    assert p[0] == (1 | (1 << 2) | (2 << 4) | (0 << 6))


@pytest.mark.parametrize("n_values", [1, 15, 16, 17, 100, 4096])
def test_pack_u32_closed_form(n_values):
    rng = np.random.default_rng(n_values)
    v = rng.integers(-1, 2, size=n_values).astype(np.int8)
    p8 = oracle.pack_ternary(v)
    w = oracle.pack_ternary_u32(p8, n_values)
    assert w.size == (n_values + 15) // 16
    for i in range(w.size):
        for j in range(4):
            b = p8[4 * i + j] if 4 * i + j < p8.size else 0
            assert (int(w[i]) >> (8 * j)) & 0xFF == b


def test_flat_u32_equals_row_aligned_when_k_mod_16():
    rng = np.random.default_rng(5)
    t = rng.integers(-1, 2, size=(12, 64)).astype(np.int8)
    flat = oracle.pack_ternary_u32(oracle.pack_ternary(t), t.size).reshape(12, 4)
    np.testing.assert_array_equal(flat, oracle.pack_rows_u32(t))
    np.testing.assert_array_equal(flat, synth.pack_rows_u32(t))


def _quantize_restated(w):
    s = np.float32(0)
    for v in w.astype(np.float32):
        s = np.float32(s + np.float32(abs(v)))
    alpha = np.float32(np.float32(s / np.float32(w.size)) / np.float32(0.7978845608)) if s > 0 else np.float32(1)
    inv = np.float32(np.float32(1) / alpha)
    q = np.trunc(np.abs(w * inv) + np.float32(0.5)) * np.sign(w * inv)  # round half away from zero
    return np.clip(q, -1, 1).astype(np.int8), alpha


def test_quantize_ternary_vs_restatement_and_kats():
    rng = np.random.default_rng(9)
    w = (rng.standard_normal(777) * 0.3).astype(np.float32)
    q, a = oracle.quantize_ternary(w)
    q2, a2 = _quantize_restated(w)
    assert a == a2
    np.testing.assert_array_equal(q, q2)
    # ternary.rs:778-795 KATs
    q0, _ = oracle.quantize_ternary(np.zeros(16, np.float32))
    assert (q0 == 0).all()
    qs, _ = oracle.quantize_ternary(np.array([-3.0, -0.5, -0.01, 0.01, 0.5, 3.0], np.float32))
    assert qs[0] == -1 and qs[5] == 1 and qs[2] == qs[3]


def test_sparse24_gpu_roundtrip_and_dense_equivalence():
    t = synth.sparse24_uniform("test", "w", 37, 96)
    meta, sc = oracle.pack_sparse24_gpu(t)
    assert meta.shape == (37, (96 // 4 + 5) // 6)
    np.testing.assert_array_equal(oracle.sparse24_gpu_decode(meta, 37, 96), t)
    # the GPU test packer's scale is mean |nonzero| = 1 for +-1 weights
    np.testing.assert_array_equal(sc, np.ones(37, np.float32))
    rng = np.random.default_rng(2)
    x = _dyadic(rng, (3, 96))
    s = (2.0 ** rng.integers(-2, 2, size=37)).astype(np.float32)
    sp = oracle.sparse24_gpu_matmul(meta, s, x, 3, 96, 37)
    de = oracle.ternary_matmul_u32(oracle.pack_rows_u32(t), s, x, 3, 96, 37)
    np.testing.assert_array_equal(sp, de)


def test_sparse24_gpu_pattern_clamp():
    # pattern id 7 decodes as pattern 5 (positions 2,3) in the WGSL kernel
    meta = np.array([[7 | (0b01 << 3)]], np.uint32)
    d = oracle.sparse24_gpu_decode(meta, 1, 4)
    np.testing.assert_array_equal(d[0], [0, 0, -1, 1])


def _from_ternary_restated(t):
    out = np.zeros_like(t)
    for g in range(t.size // 4):
        v = t[4 * g:4 * g + 4]
        order = sorted(range(4), key=lambda i: -abs(int(v[i])))  # stable
        pos0 = order[0]
        pos1 = order[1] if (v[order[1]] != 0 or v[order[0]] != 0) else 1
        p0, p1 = min(pos0, pos1), max(pos0, pos1)
        out[4 * g + p0] = 1 if v[p0] >= 0 else -1
        out[4 * g + p1] = 1 if v[p1] >= 0 else -1
    return out


def test_sparse24_cpu_from_ternary_vs_restatement():
    rng = np.random.default_rng(4)
    t = rng.integers(-1, 2, size=(16, 32)).astype(np.int8)
    p, s = oracle.sparse24_cpu_from_ternary(t, 16, 32)
    d = oracle.sparse24_cpu_to_ternary(p, s, 16, 32)
    np.testing.assert_array_equal(d, _from_ternary_restated(t.ravel()))
    t24 = synth.sparse24_uniform("test", "cpu", 16, 32)
    p, s = oracle.sparse24_cpu_from_ternary(t24, 16, 32)
    np.testing.assert_array_equal(oracle.sparse24_cpu_to_ternary(p, s, 16, 32), t24.ravel())


def test_sparse24_cpu_matmul_vs_dense():
    t24 = synth.sparse24_uniform("test", "cpum", 8, 64)
    p, s = oracle.sparse24_cpu_from_ternary(t24, 8, 64)
    rng = np.random.default_rng(8)
    x = _dyadic(rng, (2, 64))
    out = oracle.sparse24_cpu_matmul(p, s, 0.5, 8, 64, x, 2)
    ref = oracle.ternary_matmul_i8(t24, 0.5, x, 8, 64, 2)
    np.testing.assert_array_equal(out, ref)


def _softmax_route_f64(x, r, k):
    logits = x.astype(np.float64) @ r.astype(np.float64).T
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    idx = np.argsort(-p, axis=1, kind="stable")[:, :k]
    w = np.take_along_axis(p, idx, 1)
    return idx, w / w.sum(1, keepdims=True)


def test_moe_route_vs_bruteforce():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((64, 32)).astype(np.float32)
    r = (rng.standard_normal((6, 32)) * 0.5).astype(np.float32)
    idx, w, probs = oracle.moe_route(x, r, 2)
    i2, w2 = _softmax_route_f64(x, r, 2)
    np.testing.assert_array_equal(idx, i2)
    np.testing.assert_allclose(w, w2, atol=1e-6)
    np.testing.assert_allclose(w.sum(1), 1.0, atol=1e-6)
    np.testing.assert_allclose(probs.sum(1), 1.0, atol=1e-6)


def test_moe_route_ties_keep_lower_index():
    x = np.ones((1, 4), np.float32)
    r = np.array([[0.25] * 4, [0.5] * 4, [0.5] * 4, [0.25] * 4], np.float32)
    idx, w, _ = oracle.moe_route(x, r, 3)
    assert list(idx[0]) == [1, 2, 0]


def _gpu_rank_rule(probs, k):
    """The device router's ranking: a lane's rank is the number of experts
    with a greater probability plus the lower-indexed experts it ties with,
    where an unordered pair (NaN) counts as a tie. Returns [T][k] indices, or
    None for a token whose ranks are not a permutation."""
    T, E = probs.shape
    out = np.zeros((T, k), np.uint32)
    for t in range(T):
        slots = [None] * E
        for e in range(E):
            pe = probs[t, e]
            rank = 0
            for j in range(E):
                pj = probs[t, j]
                tie = not (pj < pe) and not (pj > pe)
                rank += (pj > pe) or (tie and j < e)
            if slots[rank] is not None:
                return None
            slots[rank] = e
        out[t] = slots[:k]
    return out


def test_moe_route_nonfinite_tokens_and_gpu_rank_rule():
    """NaN and +inf in a token's activations make all of its probabilities
    NaN (the exp sum is NaN); the oracle's stable sort then keeps experts in
    index order, as the reference's sort_by(partial_cmp().unwrap_or(Equal))
    does. The device router's rank rule must give the same indices and a
    permutation for every token, finite ones included."""
    rng = np.random.default_rng(31)
    T, H, E, k = 12, 16, 6, 3
    x = rng.standard_normal((T, H)).astype(np.float32)
    r = (rng.standard_normal((E, H)) * 0.5).astype(np.float32)
    x[2, 3] = np.nan
    x[4, :] = np.inf
    x[5, 0] = -np.inf
    x[6, 1] = np.inf
    idx, w, probs = oracle.moe_route(x, r, k)
    for t in (2, 4, 6):
        assert np.isnan(probs[t]).all(), t
        assert list(idx[t]) == list(range(k)), t
    np.testing.assert_array_equal(_gpu_rank_rule(probs, k), idx)
    # the rule without the tie clause for NaN leaves slots unwritten
    nan_row = np.full((1, E), np.nan, np.float32)
    assert _gpu_rank_rule(nan_row, k) is not None


def _cpu_layer_route_f64(x, r_he, k):
    """CpuMoELayer ranking (cpu_moe.rs:365-400) in float64: experts sorted
    by logit (stable), weights exp(l - l_max) over the top k, normalised."""
    logits = x.astype(np.float64) @ r_he.astype(np.float64)
    idx = np.argsort(-logits, axis=1, kind="stable")[:, :k]
    top = np.take_along_axis(logits, idx, 1)
    w = np.exp(top - top[:, :1])
    return idx, w / w.sum(1, keepdims=True)


def test_moe_route_cpu_layer_vs_bruteforce():
    rng = np.random.default_rng(41)
    x = rng.standard_normal((64, 32)).astype(np.float32)
    r = (rng.standard_normal((32, 7)) * 0.5).astype(np.float32)  # [H][E]
    idx, w = oracle.moe_route_cpu_layer(x, r, 3)
    i2, w2 = _cpu_layer_route_f64(x, r, 3)
    np.testing.assert_array_equal(idx, i2)
    np.testing.assert_allclose(w, w2, atol=1e-6)
    # on distinct probabilities the softmax router over the transposed matrix
    # ranks the same way and its renormalised top-k probabilities are the
    # same weights, up to rounding
    i3, w3, _ = oracle.moe_route(x, np.ascontiguousarray(r.T), 3)
    np.testing.assert_array_equal(idx, i3)
    np.testing.assert_allclose(w, w3, atol=1e-6)


def test_moe_route_cpu_layer_ranks_underflowed_probabilities_by_logit():
    # logits 0, -150, -120: both small probabilities underflow to 0, so the
    # softmax router ties them (index order) while CpuMoELayer ranks by logit
    x = np.ones((1, 1), np.float32)
    r = np.array([[0.0, -150.0, -120.0]], np.float32)  # [H=1][E=3]
    idx, w = oracle.moe_route_cpu_layer(x, r, 3)
    i3, _, _ = oracle.moe_route(x, np.ascontiguousarray(r.T), 3)
    assert list(idx[0]) == [0, 2, 1]
    assert list(i3[0]) == [0, 1, 2]
    assert list(w[0]) == [1.0, 0.0, 0.0]


def test_moe_route_cpu_layer_ties_and_nan():
    # ties keep the lower index (a stable sort); a NaN logit puts the token's
    # experts in index order
    x = np.ones((2, 4), np.float32)
    x[1, 2] = np.nan
    r = np.array([[0.25, 0.5, 0.5, 0.25]] * 4, np.float32)  # [H][E]: logits 1, 2, 2, 1
    idx, w = oracle.moe_route_cpu_layer(x, r, 3)
    assert list(idx[0]) == [1, 2, 0]
    np.testing.assert_allclose(w[0], np.array([1, 1, np.exp(-1)]) / (2 + np.exp(-1)), rtol=1e-6)
    assert list(idx[1]) == [0, 1, 2]


def test_moe_forward_cpu_layer_skips_negligible_experts():
    """cpu_moe.rs:172: an expert whose weight is below 1e-8 is skipped, so a
    NaN produced by that expert alone does not reach the output."""
    rng = np.random.default_rng(43)
    T, H, I, E, k = 3, 16, 32, 3, 2
    x = rng.standard_normal((T, H)).astype(np.float32)
    r = np.zeros((H, E), np.float32)
    r[0, 0] = 40.0 / x[:, 0].max()  # expert 0 dominates by more than ln(1e8) for token argmax
    t_dom = int(np.argmax(x[:, 0]))
    mk = lambda n, kk: rng.integers(-1, 2, size=(n, kk)).astype(np.int8)  # noqa: E731
    wg = [mk(I, H) for _ in range(E)]
    wu = [mk(I, H) for _ in range(E)]
    wd = [mk(H, I) for _ in range(E)]
    pk = lambda m: oracle.pack_rows_u32(m)  # noqa: E731
    sg = [np.full(I, 0.5, np.float32) for _ in range(E)]
    su = [np.full(I, 0.25, np.float32) for _ in range(E)]
    sd = [np.full(H, 0.125, np.float32) for _ in range(E)]
    # a NaN down scale on experts 1 and 2: their output is NaN everywhere
    sd[1][:] = np.nan
    sd[2][:] = np.nan
    out, idx, w = oracle.moe_forward(x, r, [pk(m) for m in wg], sg, [pk(m) for m in wu], su,
                                     [pk(m) for m in wd], sd, k, routing=1)
    assert idx[t_dom, 0] == 0 and w[t_dom, 1] < 1e-8
    assert np.isfinite(out[t_dom]).all()
    assert not np.isfinite(out).all()  # the other tokens use the NaN experts
    # the default (GPU-path glue) routing adds every selected expert
    out0, _, _ = oracle.moe_forward(x, np.ascontiguousarray(r.T), [pk(m) for m in wg], sg,
                                    [pk(m) for m in wu], su, [pk(m) for m in wd], sd, k)
    assert not np.isfinite(out0[t_dom]).all()


def _moe_f64(x, r, wg, sg, wu, su, wd, sd, k, gelu):
    idx, w = _softmax_route_f64(x, r, k)
    out = np.zeros((x.shape[0], x.shape[1]))
    for t in range(x.shape[0]):
        for j in range(k):
            e = idx[t, j]
            g = (wg[e].astype(np.float64) @ x[t]) * sg[e]
            u = (wu[e].astype(np.float64) @ x[t]) * su[e]
            if gelu:
                a = 0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * (g + 0.044715 * g ** 3)))
            else:
                a = g / (1 + np.exp(-g))
            h = a if gelu == 2 else a * u  # 2: TernaryMoELayer's GeLU, no up product
            out[t] += w[t, j] * ((wd[e].astype(np.float64) @ h) * sd[e])
    return out, idx


@pytest.mark.parametrize("gelu", [0, 1, 2])
def test_moe_forward_vs_f64(gelu):
    """Activation codes: 0 silu(g)*u, 1 gelu(g)*u (the model glue,
    cpu_block_attn_res.rs:1176-1178), 2 gelu(g) alone (TernaryMoELayer,
    ternary_moe.rs:193-200)."""
    rng = np.random.default_rng(21 + gelu)
    T, H, I, E, k = 9, 32, 48, 4, 2
    x = rng.standard_normal((T, H)).astype(np.float32)
    r = (rng.standard_normal((E, H)) * 0.3).astype(np.float32)
    mk = lambda n, kk: rng.integers(-1, 2, size=(n, kk)).astype(np.int8)  # noqa: E731
    wg = [mk(I, H) for _ in range(E)]
    wu = [mk(I, H) for _ in range(E)]
    wd = [mk(H, I) for _ in range(E)]
    sc = lambda n: (np.abs(rng.standard_normal(n)) * 0.1 + 0.05).astype(np.float32)  # noqa: E731
    sg = [sc(I) for _ in range(E)]
    su = [sc(I) for _ in range(E)]
    sd = [sc(H) for _ in range(E)]
    pk = oracle.pack_rows_u32
    out, idx, w = oracle.moe_forward(x, r, [pk(a) for a in wg], sg, [pk(a) for a in wu], su,
                                     [pk(a) for a in wd], sd, k, gelu)
    ref, idx2 = _moe_f64(x, r, wg, sg, wu, su, wd, sd, k, gelu)
    np.testing.assert_array_equal(idx, idx2)
    rms = np.sqrt((ref ** 2).mean())
    assert np.abs(out - ref).max() <= 1e-5 * rms


def test_gelu_tanh_vs_f64():
    for v in [-3.0, -0.5, 0.0, 0.3, 2.0]:
        ref = 0.5 * v * (1 + np.tanh(np.sqrt(2 / np.pi) * (v + 0.044715 * v ** 3)))
        assert abs(oracle.gelu_tanh(v) - ref) <= 1e-6 * max(1.0, abs(ref))
        assert abs(oracle.gelu_tanh_lit(v) - ref) <= 1e-6 * max(1.0, abs(ref))


def test_gelu_tanh_special_values():
    """GeLU-tanh fixed points: gelu(0) = 0 exactly, gelu(x) -> x for large x
    and -> -0 for large negative x (tanh saturates to +-1 in f32), and
    gelu(-x) = gelu(x) - x (odd tanh) to f32 rounding."""
    for f in (oracle.gelu_tanh, oracle.gelu_tanh_lit):
        assert f(0.0) == 0.0
        assert f(20.0) == 20.0
        assert f(-20.0) == 0.0
        for v in (0.25, 1.0, 1.7, 3.0):
            assert abs(f(-v) - (f(v) - v)) <= 4e-7 * max(1.0, v)


def test_moe_forward_gate_only_does_not_read_up():
    """Activation 2 (TernaryMoELayer's GeLU) never reads W_up: garbage up
    matrices give the same output bit for bit as None."""
    rng = np.random.default_rng(5)
    T, H, I, E, k = 6, 32, 48, 3, 2
    x = rng.standard_normal((T, H)).astype(np.float32)
    r = (rng.standard_normal((E, H)) * 0.3).astype(np.float32)
    pk = oracle.pack_rows_u32
    wg = [pk(rng.integers(-1, 2, (I, H)).astype(np.int8)) for _ in range(E)]
    wd = [pk(rng.integers(-1, 2, (H, I)).astype(np.int8)) for _ in range(E)]
    sg = [np.full(I, 0.1, np.float32)] * E
    sd = [np.full(H, 0.1, np.float32)] * E
    wu = [pk(rng.integers(-1, 2, (I, H)).astype(np.int8)) for _ in range(E)]
    su = [np.full(I, 7.0, np.float32)] * E
    a, _, _ = oracle.moe_forward(x, r, wg, sg, None, None, wd, sd, k, 2)
    b, _, _ = oracle.moe_forward(x, r, wg, sg, wu, su, wd, sd, k, 2)
    np.testing.assert_array_equal(a, b)
    c, _, _ = oracle.moe_forward(x, r, wg, sg, wu, su, wd, sd, k, 1)
    assert np.abs(c - a).max() > 1e-2 * np.abs(a).max()


@pytest.mark.parametrize("gelu", [False, True])
def test_ffn_oracle_matches_float64(gelu):
    """Dense FFN oracle (cpu_block_attn_res.rs:2317-2326) = gate/up u32
    matmuls, activation, product, down matmul; checked against a float64
    restatement on small shapes, and SiLU != GeLU."""
    rng = np.random.default_rng(7)
    M, H, I = 3, 48, 80
    tg, tu = (rng.integers(-1, 2, (I, H)).astype(np.int8) for _ in range(2))
    td = rng.integers(-1, 2, (H, I)).astype(np.int8)
    sg, su = (rng.random(I).astype(np.float32) * 0.1 + 0.01 for _ in range(2))
    sd = rng.random(H).astype(np.float32) * 0.1 + 0.01
    x = rng.standard_normal((M, H)).astype(np.float32)
    y = oracle.ffn_forward(x, synth.pack_rows_u32(tg), sg, synth.pack_rows_u32(tu), su,
                           synth.pack_rows_u32(td), sd, gelu=gelu)
    g = (x.astype(np.float64) @ tg.T.astype(np.float64)) * sg
    u = (x.astype(np.float64) @ tu.T.astype(np.float64)) * su
    if gelu:
        a = 0.5 * g * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (g + 0.044715 * g ** 3)))
    else:
        a = g / (1.0 + np.exp(-g))
    ref = ((a * u) @ td.T.astype(np.float64)) * sd
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()
    other = oracle.ffn_forward(x, synth.pack_rows_u32(tg), sg, synth.pack_rows_u32(tu), su,
                               synth.pack_rows_u32(td), sd, gelu=not gelu)
    assert np.abs(other - y).max() > 1e-3 * np.abs(y).max()


def test_quantize_ste_closed_cases():
    """BitLinear::forward_ste (shadow_weights.rs:203-231): alpha = mean|w|,
    strict +-0.5 thresholds on w / alpha (unlike round(), which takes +-0.5
    away from zero), all zero below alpha = 1e-10."""
    q, a = oracle.quantize_ste(np.array([0.5, -0.5, 1.5, -1.5], np.float32))  # alpha = 1
    assert a == 1.0 and q.tolist() == [0, 0, 1, -1]
    q, a = oracle.quantize_ste(np.array([0.6, -0.4], np.float32))  # alpha = 0.5: t = 1.2, -0.8
    assert a == np.float32(0.5) and q.tolist() == [1, -1]
    q, a = oracle.quantize_ste(np.full(16, -0.25, np.float32))  # constant row: its sign
    assert a == np.float32(0.25) and (q == -1).all()
    for row in (np.zeros(8, np.float32), np.full(8, 1e-11, np.float32)):
        q, a = oracle.quantize_ste(row)
        assert a < 1e-10 and (q == 0).all()
    q, a = oracle.quantize_ste(np.array([1.0, np.nan, -3.0], np.float32))  # NaN mean: every t is NaN
    assert np.isnan(a) and (q == 0).all()
    # quantize_ternary rounds +-0.5 away from zero: with |w| summing to
    # 4 * ABSMEAN_NORM exactly, alpha = 1 and w * (1 / alpha) = w
    norm = np.float32(0.7978845608)
    w = np.array([0.5, -0.5, 1.5, np.float32(4) * norm - np.float32(2.5)], np.float32)
    qt, at = oracle.quantize_ternary(w)
    assert at == 1.0 and qt.tolist() == [1, -1, 1, 1]


def test_sparse_index_decode_exact_on_dyadic_and_vs_f64():
    rng = np.random.default_rng(41)
    rows, cols = 37, 200
    t = rng.integers(-1, 2, size=rows * cols).astype(np.int8)
    xd = (rng.integers(-64, 65, size=cols) / 8).astype(np.float32)
    idx = oracle.ternary_sparse_indices(t, rows, cols)
    # every +1 and -1 is listed once, in column order
    po, pi, no, ni = idx
    assert po[-1] == (t == 1).sum() and no[-1] == (t == -1).sum()
    for r in range(rows):
        assert (np.diff(pi[po[r]:po[r + 1]].astype(np.int64)) > 0).all()
    exact = t.reshape(rows, cols).astype(np.float64) @ xd.astype(np.float64) * 0.25
    np.testing.assert_array_equal(oracle.ternary_matmul_sparse_decode(*idx, 0.25, xd, rows), exact.astype(np.float32))
    x = rng.standard_normal(cols).astype(np.float32)
    ref = t.reshape(rows, cols).astype(np.float64) @ x.astype(np.float64) * 0.7
    np.testing.assert_allclose(oracle.ternary_matmul_sparse_decode(*idx, 0.7, x, rows), ref, rtol=1e-5, atol=1e-5)


def test_ternary_stats_counts_every_value_once():
    rng = np.random.default_rng(42)
    t = rng.integers(-1, 2, size=10007).astype(np.int8)
    counts, ratios, _ = oracle.ternary_stats(t)
    assert list(counts) == [(t == -1).sum(), (t == 0).sum(), (t == 1).sum()]
    np.testing.assert_allclose(ratios.sum(), 1.0, atol=1e-6)


def test_lora_forward_closed_form_and_vs_f64():
    """LoraLayer::forward (lora.rs:138-167): rank 1 with A = e_0 and B = ones
    is scaling * x[0] in every output, exactly; random adapters match float64."""
    rng = np.random.default_rng(41)
    x = rng.standard_normal(24).astype(np.float32)
    a = np.zeros((1, 24), np.float32)
    a[0, 0] = 1.0
    out = oracle.lora_forward(a, np.ones((7, 1), np.float32), 0.5, x)
    np.testing.assert_array_equal(out, np.full(7, np.float32(0.5) * x[0], np.float32))
    a = rng.standard_normal((8, 96)).astype(np.float32)
    b = rng.standard_normal((40, 8)).astype(np.float32)
    x = rng.standard_normal(96).astype(np.float32)
    ref = 2.0 * (b.astype(np.float64) @ (a.astype(np.float64) @ x))
    assert np.abs(oracle.lora_forward(a, b, 2.0, x) - ref).max() <= 1e-5 * np.abs(ref).max()
    # rank 0 rows of B: the output is zero
    np.testing.assert_array_equal(oracle.lora_forward(a, np.zeros((5, 8), np.float32), 3.0, x), np.zeros(5))


def _moe_lora_f64(x, r, wg, sg, wu, su, wd, sd, k, lora):
    idx, w = _softmax_route_f64(x, r, k)
    out = np.zeros((x.shape[0], x.shape[1]))
    sc = lora["scaling"]
    lo = lambda n, e, v: (sc * (lora["b_" + n][e].astype(np.float64) @  # noqa: E731
                                (lora["a_" + n][e].astype(np.float64) @ v))
                          if lora["a_" + n][e] is not None else 0.0)
    for t in range(x.shape[0]):
        for j in range(k):
            e = idx[t, j]
            g = (wg[e].astype(np.float64) @ x[t]) * sg[e] + lo("gate", e, x[t])
            u = (wu[e].astype(np.float64) @ x[t]) * su[e] + lo("up", e, x[t])
            h = g / (1 + np.exp(-g)) * u
            out[t] += w[t, j] * ((wd[e].astype(np.float64) @ h) * sd[e] + lo("down", e, h))
    return out, idx


def test_moe_forward_lora_vs_f64_and_without_adapters():
    """The MoE forward with LoRA adapters (cpu_moe.rs:321-363) against a
    float64 composition, adapters on some experts and projections only; with
    no adapters it equals moe_forward bit for bit."""
    rng = np.random.default_rng(43)
    T, H, I, E, k, rank = 7, 32, 48, 4, 2, 4
    x = rng.standard_normal((T, H)).astype(np.float32)
    r = (rng.standard_normal((E, H)) * 0.3).astype(np.float32)
    mk = lambda n, kk: rng.integers(-1, 2, size=(n, kk)).astype(np.int8)  # noqa: E731
    wg, wu, wd = [mk(I, H) for _ in range(E)], [mk(I, H) for _ in range(E)], [mk(H, I) for _ in range(E)]
    sc = lambda n: (np.abs(rng.standard_normal(n)) * 0.1 + 0.05).astype(np.float32)  # noqa: E731
    sg, su, sd = [sc(I) for _ in range(E)], [sc(I) for _ in range(E)], [sc(H) for _ in range(E)]
    f = lambda *s: (rng.standard_normal(s) * 0.2).astype(np.float32)  # noqa: E731
    lora = {"rank": rank, "scaling": 2.0,
            "a_gate": [f(rank, H), None, f(rank, H), f(rank, H)], "b_gate": [f(I, rank), None, f(I, rank), f(I, rank)],
            "a_up": [None, f(rank, H), f(rank, H), None], "b_up": [None, f(I, rank), f(I, rank), None],
            "a_down": [f(rank, I), f(rank, I), None, f(rank, I)], "b_down": [f(H, rank), f(H, rank), None, f(H, rank)]}
    pk = oracle.pack_rows_u32
    args = (x, r, [pk(a) for a in wg], sg, [pk(a) for a in wu], su, [pk(a) for a in wd], sd, k)
    out, idx, w = oracle.moe_forward_lora(*args, lora)
    ref, idx2 = _moe_lora_f64(x, r, wg, sg, wu, su, wd, sd, k, lora)
    np.testing.assert_array_equal(idx, idx2)
    assert np.abs(out - ref).max() <= 1e-5 * np.sqrt((ref ** 2).mean())
    plain, _, _ = oracle.moe_forward(*args)
    assert np.abs(out - plain).max() > 1e-2 * np.abs(plain).max()  # the adapters matter here
    none = {**lora, **{n: [None] * E for n in ("a_gate", "b_gate", "a_up", "b_up", "a_down", "b_down")}}
    np.testing.assert_array_equal(oracle.moe_forward_lora(*args, none)[0], plain)


@pytest.mark.parametrize("n,block", [(512, 64), (1000, 64), (37, 8), (96, 96), (100, 128), (4096, 1000)])
def test_quantize_blocked_reduces_to_per_block_quantize(n, block):
    """quantize_ternary_blocked (ternary.rs:76-110) = quantize_ternary on
    each block of block_size values (the last block shorter), bit for bit;
    dequantize_ternary_blocked is alpha * q per block (exact)."""
    rng = np.random.default_rng(n + block)
    w = (rng.standard_normal(n) * np.where(np.arange(n) % 300 < 150, 0.02, 1.5)).astype(np.float32)
    w[::17] = 0.0
    q, sc = oracle.quantize_ternary_blocked(w, block)
    assert sc.size == -(-n // block)
    for b in range(sc.size):
        qb, ab = oracle.quantize_ternary(w[b * block:(b + 1) * block])
        np.testing.assert_array_equal(q[b * block:(b + 1) * block], qb)
        assert sc[b].view(np.uint32) == np.float32(ab).view(np.uint32)
        seg = w[b * block:(b + 1) * block].astype(np.float64)
        assert abs(sc[b] - np.abs(seg).mean() / 0.7978845608) <= 1e-5 * sc[b]
    r = oracle.dequantize_ternary_blocked(q, sc, block)
    np.testing.assert_array_equal(r, np.repeat(sc, block)[:n] * q.astype(np.float32))
    # an all-zero block takes alpha = 1 and codes 0
    z = np.zeros(2 * block, np.float32)
    z[block:] = 1.0
    qz, sz = oracle.quantize_ternary_blocked(z, block)
    assert sz[0] == 1.0 and (qz[:block] == 0).all()


def _prune_bruteforce(w, rows, cols):
    """Kept positions and magnitude-ordered values of each group: the top 2
    by |v|, the lower index first among equals (float64 brute force)."""
    out = []
    g = w.reshape(-1, 4).astype(np.float64)
    for v in g:
        order = sorted(range(4), key=lambda i: (-abs(v[i]), i))
        out.append((order[0], order[1], v[order[0]], v[order[1]]))
    return out


@pytest.mark.parametrize("rows,cols,seed", [(1, 4, 0), (3, 8, 1), (16, 64, 2), (5, 12, 3), (64, 256, 4)])
def test_prune_sparse24_vs_bruteforce(rows, cols, seed):
    """prune_fp32_to_sparse_ternary (sparse_ternary.rs:598-663): the kept
    positions are the stable top 2 by |v| (checked with ties forced), the
    sign of each kept position is the sign of the value the reference's
    sign bit names (bit 0: the larger |v|, bit 1: the second), and the
    scale is the float64 absmean within f32 rounding of the sequential sum."""
    rng = np.random.default_rng(seed)
    w = rng.standard_normal(rows * cols).astype(np.float32)
    w[rng.random(w.size) < 0.15] = 0.0
    ties = rng.random(w.size) < 0.2
    w[ties] = np.float32(0.5) * np.sign(w[ties])  # equal magnitudes, mixed signs
    pats, signs, scale = oracle.prune_sparse24(w, rows, cols)
    dec = oracle.sparse24_cpu_to_ternary(pats, signs, rows, cols).reshape(-1, 4)
    for g, (pa, pb, va, vb) in enumerate(_prune_bruteforce(w, rows, cols)):
        lo, hi = min(pa, pb), max(pa, pb)
        kept = [i for i in range(4) if dec[g][i] != 0]
        assert kept == [lo, hi], g
        # bit 0 (read as the lower position) carries sign(va), bit 1 sign(vb)
        assert dec[g][lo] == (1 if va >= 0 else -1), g
        assert dec[g][hi] == (1 if vb >= 0 else -1), g
    ref = np.abs(w.astype(np.float64)).mean() / 0.7978845608
    assert abs(float(scale) - ref) <= 1e-5 * ref


def test_prune_sparse24_sign_order_and_special_values():
    """Closed cases of the reference's packing order: when the larger |v| is
    at the higher position, its sign lands on the lower position (the
    reference packs signs in magnitude order, :642-644); all-zero groups keep
    positions (0, 1) with + signs (0.0 >= 0); -0.0 counts as +; the scale of
    an all-zero matrix is 1."""
    w = np.array([0.1, -0.5, 0.0, 3.0,      # larger at pos 3 (+), second at pos 1 (-)
                  -3.0, 0.0, 0.5, 0.1,      # larger at pos 0 (-), second at pos 2 (+)
                  0.0, 0.0, 0.0, 0.0,       # all zero
                  -0.0, -0.0, 0.25, 0.0],   # one nonzero, then the first -0.0
                 np.float32)
    pats, signs, scale = oracle.prune_sparse24(w, 1, 16)
    dec = oracle.sparse24_cpu_to_ternary(pats, signs, 1, 16).reshape(4, 4)
    np.testing.assert_array_equal(dec[0], [0, 1, 0, -1])
    np.testing.assert_array_equal(dec[1], [-1, 0, 1, 0])
    np.testing.assert_array_equal(dec[2], [1, 1, 0, 0])
    np.testing.assert_array_equal(dec[3], [1, 0, 1, 0])
    z = np.zeros(8, np.float32)
    assert oracle.prune_sparse24(z, 2, 4)[2] == np.float32(1.0)
