// frx_moe.hip — MoE ternary expert layer on gfx950.
//
// Semantics: the model's GPU-path MoE glue, src/model/cpu_block_attn_res.rs
// :1148-1184, and TernaryMoELayer::forward, src/model/ternary_moe.rs:145-223,
// with per-row scales. Their routing is the same; their GeLU experts differ
// (the glue: gelu(g) * u; TernaryMoELayer: gelu(g) alone, ternary_moe.rs:
// 193-200), selected by the activation code (moe_act). The reference runs it
// as host loops over tokens and
// experts with 3 GEMV dispatches per (token, expert); here it is five
// launches:
//   1. router_topk   one lane per (token, expert): logits (sequential f32
//                    sums, bit-identical to the reference), softmax, stable
//                    descending sort of the probabilities, top-k, weights.
//   2. group         one workgroup: per-expert histogram, exclusive scan and
//                    a stable scatter of the (token, k) assignments into
//                    expert-sorted rows, plus the M-tile schedule (tiles
//                    sized to each expert's tokens).
//   3. gateup        grouped GEMM over the tile schedule: gathered token rows
//                    x W_gate[e] and x W_up[e] in one workgroup, SwiGLU or
//                    GeLU-tanh epilogue (moe_act), h stored as bf16 hi/lo
//                    planes.
//   4. down          grouped GEMM h x W_down[e] (hi and lo planes in one K
//                    loop, on separate waves that share the weight tile),
//                    fp32 rows.
//   5. combine       out[t] = sum_k w[t,k] * d[row(t,k)] in k order from 0.0,
//                    exactly the reference's accumulation (deterministic).
#include "frx_gemm2.hpp"
#include "frx_gemm_core.hpp"
#include "frx_internal.hpp"

namespace frx {

constexpr int MOE_MAXE = 64;
constexpr int MOE_BM = 64;   // tokens per grouped-GEMM tile
constexpr int MOE_BN = 128;  // weight rows per tile

static inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

size_t moe_workspace_bytes(int T, int H, int I, int E, int top_k) {
  const size_t A = (size_t)T * top_k;
  const size_t max_tiles = (A + MOE_BM - 1) / MOE_BM + E;
  size_t b = 0;
  b += align256(A * 4) * 2;             // idx, wts
  b += align256((size_t)E * 4);         // counts
  b += align256((size_t)(E + 1) * 4);   // offsets
  b += align256(A * 4) * 3;             // perm_token, inv, row_expert
  b += align256(A * 4 * 3 * MOE_LORA_MAXR);  // LoRA A x (gate, up) and A h (down)
  b += align256(max_tiles * 16);        // tiles
  b += align256(4);                     // ntiles
  b += align256(A * I * 2) * 2;         // h planes
  b += align256(A * H * 4) * 2;         // dout, dout_lo
  b += align256((size_t)T * H * 4);     // f32 x as bf16 hi | lo rows
  return b;
}

void moe_workspace_carve(void *base, int T, int H, int I, int E, int top_k,
                         MoeWorkspace *ws) {
  const size_t A = (size_t)T * top_k;
  const size_t max_tiles = (A + MOE_BM - 1) / MOE_BM + E;
  char *p = reinterpret_cast<char *>(base);
  auto take = [&](size_t n) { char *r = p; p += align256(n); return r; };
  ws->idx = reinterpret_cast<uint32_t *>(take(A * 4));
  ws->wts = reinterpret_cast<float *>(take(A * 4));
  ws->counts = reinterpret_cast<int *>(take((size_t)E * 4));
  ws->offsets = reinterpret_cast<int *>(take((size_t)(E + 1) * 4));
  ws->perm_token = reinterpret_cast<int *>(take(A * 4));
  ws->inv = reinterpret_cast<int *>(take(A * 4));
  ws->row_expert = reinterpret_cast<int *>(take(A * 4));
  ws->lora_ax = reinterpret_cast<float *>(take(A * 4 * 3 * MOE_LORA_MAXR));
  ws->lora_ah = ws->lora_ax + A * 2 * MOE_LORA_MAXR;
  ws->tiles = reinterpret_cast<int *>(take(max_tiles * 16));
  ws->ntiles = reinterpret_cast<int *>(take(4));
  ws->h_hi = reinterpret_cast<uint16_t *>(take(A * I * 2));
  ws->h_lo = reinterpret_cast<uint16_t *>(take(A * I * 2));
  ws->dout = reinterpret_cast<float *>(take(A * H * 4));
  ws->dout_lo = reinterpret_cast<float *>(take(A * H * 4));
  ws->x2 = reinterpret_cast<uint16_t *>(take((size_t)T * H * 4));
}

template <typename T>
__device__ __forceinline__ float ld_f32(const T *p, long i);
template <>
__device__ __forceinline__ float ld_f32<float>(const float *p, long i) { return p[i]; }
template <>
__device__ __forceinline__ float ld_f32<uint16_t>(const uint16_t *p, long i) {
  return __uint_as_float((uint32_t)p[i] << 16);
}

// ---- 1. router + softmax + stable top-k -----------------------------------
// ternary_moe.rs:152-183 / cpu_block_attn_res.rs:1150-1166. The logit of
// expert e is a left-to-right f32 sum of x[j]*r[e][j], each product rounded
// to f32 before its add, so it is bit-identical to the reference for the
// same inputs (bf16 x and r: the product is exact, and a fused multiply-add
// rounds once to that same sum; otherwise a separate multiply and add); exp is
// evaluated in double and rounded to f32 (correctly rounded except in
// vanishingly rare near-halfway cases), division is IEEE.
#pragma clang fp contract(off)
// 8 consecutive elements as f32 (16-byte bf16 load or two 16-byte f32 loads).
__device__ __forceinline__ void ld8(const uint16_t *p, float v[8]) {
  const u32x4 a = *reinterpret_cast<const u32x4 *>(p);
  const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
  }
}
__device__ __forceinline__ void ld8(const float *p, float v[8]) {
  const float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

constexpr int RT_CHMAX = 256;  // router columns staged per chunk (at most)

// One wave per workgroup (RT_NT threads); each thread stages RT_SP units of
// 8 columns per chunk.
constexpr int RT_NT = 64, RT_SP = 8;

// Chunk width so that one pass of RT_NT threads x RT_SP units of 8 columns
// covers every staged row (tokens of the block + experts): a multiple of 8.
static inline int router_chunk(int rows) {
  int ch = (RT_NT * RT_SP / rows) * 8;
  return ch > RT_CHMAX ? RT_CHMAX : ch;
}

// Softmax and stable top-k in LDS, one EP-lane group per token (lane
// (tl, e) holds the logit of expert e for token t). A lane's rank among the
// probabilities (greater, or equal with a lower index) reproduces the stable
// descending sort of the reference; the two reductions (sum of exps in
// expert order, sum of the top-k in sorted order) stay sequential on one
// lane, as in the reference. logit: 4 * RT_NT floats of LDS.
// by_logit (CpuMoELayer::top_k_select_with_probs, src/model/cpu_moe.rs:
// 365-400): the experts are ranked by logit instead of probability and the
// weights are exp(l_k - l_max) over the selected logits, divided by their
// sum in rank order when it is positive.
__device__ __forceinline__ void router_softmax_topk(float sum, float *logit, int tid, int e, int tl, int t,
                                                    int T, int E, int EP, int top_k,
                                                    uint32_t *__restrict__ idx_out, float *__restrict__ w_out,
                                                    uint32_t *__restrict__ user_idx, float *__restrict__ user_w,
                                                    int by_logit) {
  float *pbuf = logit + RT_NT;             // [RT_NT] probabilities
  float *tsum = pbuf + RT_NT;              // [RT_NT/EP] per-token sums
  int *order = reinterpret_cast<int *>(tsum + RT_NT);  // [RT_NT/EP][EP]
  logit[tid] = sum;
  __syncthreads();
  const float *lg = logit + tl * EP;
  const bool live = e < E && t < T;
  float mx = -INFINITY;
  for (int i = 0; i < E; i++) mx = fmaxf(mx, lg[i]);
  const float ex = live ? (float)exp((double)__fsub_rn(lg[e], mx)) : 0.0f;
  pbuf[tid] = ex;
  __syncthreads();
  if (e == 0) {
    float se = 0.0f;
    for (int i = 0; i < E; i++) se = __fadd_rn(se, pbuf[tl * EP + i]);
    tsum[tl] = se;
  }
  __syncthreads();
  const float pe = live ? __fdiv_rn(ex, tsum[tl]) : 0.0f;
  __syncthreads();
  pbuf[tid] = pe;
  __syncthreads();
  if (live) {
    // Unordered pairs (NaN) count as ties, broken by index, as the
    // reference's sort_by(partial_cmp().unwrap_or(Equal)) keeps them. Within
    // a token the probabilities are either all NaN (a NaN or +inf logit
    // makes the exp sum NaN) or all ordered, so the ranks are a permutation
    // of 0..E-1 in both cases and every slot below top_k is written. Ranked
    // by logit, a NaN logit ties with every expert; ties break by index.
    int rank = 0;
    const float ve = by_logit ? lg[e] : pe;
    for (int j = 0; j < E; j++) {
      const float vj = by_logit ? lg[j] : pbuf[tl * EP + j];
      const bool tie = !(vj < ve) && !(vj > ve);
      rank += (vj > ve) || (tie && j < e);
    }
    if (by_logit) {
      // a NaN among the logits makes the rank relation intransitive: fall
      // back to index order for the whole token
      bool any_nan = false;
      for (int j = 0; j < E; j++) any_nan |= lg[j] != lg[j];
      if (any_nan) rank = e;
    }
    if (rank < top_k) order[tl * EP + rank] = e;
  }
  __syncthreads();
  if (by_logit) {
    // weights: exp(l_k - l_max) over the top-k logits (rank order), as pbuf
    if (live) {
      int r = -1;
      for (int i = 0; i < top_k; i++) r = order[tl * EP + i] == e ? i : r;
      if (r >= 0) pbuf[tid] = (float)exp((double)__fsub_rn(lg[e], lg[order[tl * EP]]));
    }
    __syncthreads();
  }
  if (e == 0 && t < T) {
    float ts = 0.0f;
    for (int i = 0; i < top_k; i++) ts = __fadd_rn(ts, pbuf[tl * EP + order[tl * EP + i]]);
    tsum[tl] = ts;
  }
  __syncthreads();
  if (e < top_k && t < T) {
    const int oi = order[tl * EP + e];
    const int ei = (unsigned)oi < (unsigned)E ? oi : 0;  // the ranks above fill every slot; kept in range regardless
    const float ts = tsum[tl];
    const float wi = (by_logit && !(ts > 0.0f)) ? pbuf[tl * EP + ei] : __fdiv_rn(pbuf[tl * EP + ei], ts);
    idx_out[t * top_k + e] = (uint32_t)ei;
    w_out[t * top_k + e] = wi;
    if (user_idx) user_idx[t * top_k + e] = (uint32_t)ei;
    if (user_w) user_w[t * top_k + e] = wi;
  }
}

// RT_NT threads = (RT_NT/EP) tokens x EP expert lanes (EP = E rounded up to
// a power of two). A (token, expert) lane's logit is a chain of H dependent
// adds, so the kernel time is one chain's latency: one wave per workgroup
// spreads the chains over as many SIMDs as possible. Chunks of CH columns of
// the block's token rows and of all router rows are staged in LDS as f32
// (double-buffered: the next chunk's global loads are in flight while the
// current one is summed); each lane runs the reference's sequential dot
// product.
template <typename XT, typename RT>
__global__ __launch_bounds__(RT_NT) void moe_router_kernel(
    const XT *__restrict__ x, const RT *__restrict__ router, int T, int H,
    int E, int EP, int top_k, int CH, uint32_t *__restrict__ idx_out,
    float *__restrict__ w_out, uint32_t *__restrict__ user_idx,
    float *__restrict__ user_w, int by_logit) {
  const int RS = CH + 4;  // padded row stride (floats)
  extern __shared__ __align__(16) float rsm[];
  const int tid = threadIdx.x, e = tid % EP, tl = tid / EP;
  const int TPB = RT_NT / EP;
  const int t = blockIdx.x * TPB + tl;
  const int rows = TPB + E;  // staged rows: tokens then experts
  // the two chunk buffers, indexed off the __shared__ base so that reads
  // stay LDS instructions (a pointer picked from an array would turn them
  // into generic FLAT loads)
  auto buf = [&](int i) { return rsm + i * rows * RS; };
  float *logit = rsm + 2 * rows * RS;
  const int nch = (H + CH - 1) / CH;
  // each thread stages 8 consecutive columns of one row per pass. The loads
  // are unconditional (out-of-range units read a valid clamped address and
  // are zeroed when stored): a load under a divergent branch makes the
  // compiler wait for it on the spot, which serialises the chunk's loads.
  const int units = rows * (CH / 8);
  constexpr int NVX = sizeof(XT) == 2 ? 1 : 2, NVR = sizeof(RT) == 2 ? 1 : 2;  // 16-byte loads per unit
  constexpr bool SAME = sizeof(XT) == sizeof(RT);
  constexpr bool EXACT_PRODUCT = sizeof(XT) == 2 && sizeof(RT) == 2;
  // same element size: one load from the selected row; otherwise both
  // candidates are loaded and the store picks one
  struct Raw {
    u32x4 a[RT_SP][NVX], b[RT_SP][SAME ? 1 : NVR];
    bool ok[RT_SP], tok[RT_SP];
  };
  auto gload = [&](int c, Raw &raw) {
#pragma unroll
    for (int i = 0; i < RT_SP; i++) {
      const int u = tid + i * RT_NT;
      const int rr = u / (CH / 8), col = c * CH + (u % (CH / 8)) * 8;
      const int tt = blockIdx.x * TPB + rr;
      const bool tok = rr < TPB;
      raw.ok[i] = u < units && col < H && (!tok || tt < T);
      raw.tok[i] = tok;
      const int cc = raw.ok[i] ? col : 0;
      const u32x4 *xs = reinterpret_cast<const u32x4 *>(x + (long)min(tt, T - 1) * H + cc);
      const u32x4 *rs = reinterpret_cast<const u32x4 *>(router + (long)min(max(rr - TPB, 0), E - 1) * H + cc);
      if constexpr (SAME) {
        const u32x4 *src = tok ? xs : rs;
#pragma unroll
        for (int v = 0; v < NVX; v++) raw.a[i][v] = src[v];
      } else {
#pragma unroll
        for (int v = 0; v < NVX; v++) raw.a[i][v] = xs[v];
#pragma unroll
        for (int v = 0; v < NVR; v++) raw.b[i][v] = rs[v];
      }
    }
  };
  // 8 elements (one 16-byte bf16 load or two 16-byte f32 loads) as f32,
  // zero when m == 0
  auto cvt8 = [](const u32x4 *r, int nv, uint32_t m, float v8[8]) {
    if (nv == 1) {
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint32_t w = r[0][q] & m;
        v8[2 * q] = __uint_as_float(w << 16);
        v8[2 * q + 1] = __uint_as_float(w & 0xFFFF0000u);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; q++) {
        v8[q] = __uint_as_float(r[0][q] & m);
        v8[4 + q] = __uint_as_float(r[1][q] & m);
      }
    }
  };
  auto sstore = [&](float *b, const Raw &raw) {
#pragma unroll
    for (int i = 0; i < RT_SP; i++) {
      const int u = tid + i * RT_NT;
      if (u < units) {
        const int rr = u / (CH / 8), cc = (u % (CH / 8)) * 8;
        const uint32_t m = raw.ok[i] ? 0xFFFFFFFFu : 0u;
        float v8[8];
        if constexpr (SAME) {
          cvt8(raw.a[i], NVX, m, v8);
        } else {
          float va[8], vb[8];
          cvt8(raw.a[i], NVX, m, va);
          cvt8(raw.b[i], NVR, m, vb);
#pragma unroll
          for (int q = 0; q < 8; q++) v8[q] = raw.tok[i] ? va[q] : vb[q];
        }
        float4 *d = reinterpret_cast<float4 *>(b + rr * RS + cc);
        d[0] = make_float4(v8[0], v8[1], v8[2], v8[3]);
        d[1] = make_float4(v8[4], v8[5], v8[6], v8[7]);
      }
    }
  };
  float sum = 0.0f;
  // Staged data of two chunks sits in registers: chunk c + 2 is loaded while
  // chunk c is summed and chunk c + 1 (loaded during chunk c - 1) is stored.
  Raw r0, r1;
  gload(0, r0);
  gload(min(1, nch - 1), r1);
  sstore(buf(0), r0);
  __syncthreads();
  // (loads and calls are unconditional inside the loop: a conditionally
  // loaded register set makes the compiler wait for every load at the merge)
  auto chunk = [&](int c, const Raw &rnext, Raw &rfree) {
    gload(min(c + 2, nch - 1), rfree);
    if (e < E && t < T) {
#pragma clang fp contract(off)
      const float *xr = buf(c & 1) + tl * RS;
      const float *rr = buf(c & 1) + (TPB + e) * RS;
      const int ncol = min(CH, H - c * CH);  // multiple of 8
      // One step of the chain: sum = fl(sum + fl(x * r)). With bf16 x and r
      // the product is exact in f32 (8-bit significands), so a fused
      // multiply-add rounds once to the same value and halves the issue.
      auto step = [&](float xe, float re) {
        if constexpr (EXACT_PRODUCT) sum = __fmaf_rn(xe, re, sum);
        else sum = sum + xe * re;
      };
      // 24-column blocks, the LDS reads of block b + 1 issued before the
      // dependent steps of block b (two register sets, unrolled by two so
      // they alternate without copies; the read-ahead past the last block
      // re-reads that block). 24 columns are 12 reads, so a block's reads can
      // all be outstanding within the 4-bit LDS wait counter while the
      // previous block is consumed.
      constexpr int BQ = 6;  // 16-byte reads per row and block
      const int nblk = ncol / (4 * BQ);
      auto rd = [&](int b, f32x4 *xv, f32x4 *rv) {
        const int j = min(b, max(nblk - 1, 0)) * (4 * BQ);
#pragma unroll
        for (int q = 0; q < BQ; q++) {
          xv[q] = *reinterpret_cast<const f32x4 *>(xr + j + 4 * q);
          rv[q] = *reinterpret_cast<const f32x4 *>(rr + j + 4 * q);
        }
      };
      auto run = [&](const f32x4 *xv, const f32x4 *rv) {
#pragma unroll
        for (int q = 0; q < BQ; q++) {
#pragma unroll
          for (int i = 0; i < 4; i++) step(xv[q][i], rv[q][i]);
        }
      };
      // (the scheduling barriers keep each read-ahead in front of the chain
      // it overlaps; left alone, the scheduler sinks the reads below the
      // chain and every block starts with an LDS round trip)
      f32x4 xa[BQ], ra[BQ], xb[BQ], rb[BQ];
      rd(0, xa, ra);
      int b = 0;
      for (; b + 2 <= nblk; b += 2) {
        rd(b + 1, xb, rb);
        __builtin_amdgcn_sched_barrier(0);
        run(xa, ra);
        __builtin_amdgcn_sched_barrier(0);
        rd(b + 2, xa, ra);
        __builtin_amdgcn_sched_barrier(0);
        run(xb, rb);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (b < nblk) run(xa, ra);
      int j = nblk * (4 * BQ);
      for (; j < ncol; j += 8) {
        f32x4 xv[2], rv[2];
#pragma unroll
        for (int q = 0; q < 2; q++) {
          xv[q] = *reinterpret_cast<const f32x4 *>(xr + j + 4 * q);
          rv[q] = *reinterpret_cast<const f32x4 *>(rr + j + 4 * q);
        }
#pragma unroll
        for (int q = 0; q < 2; q++) {
#pragma unroll
          for (int i = 0; i < 4; i++) step(xv[q][i], rv[q][i]);
        }
      }
    }
    if (c + 1 < nch) sstore(buf((c + 1) & 1), rnext);
    __syncthreads();
  };
  int c = 0;
  for (; c + 1 < nch; c += 2) {
    chunk(c, r1, r0);
    chunk(c + 1, r0, r1);
  }
  if (c < nch) chunk(c, r1, r0);
  router_softmax_topk(sum, logit, tid, e, tl, t, T, E, EP, top_k, idx_out, w_out, user_idx, user_w, by_logit);
}

// Resident variant for bf16 router weights when the block's data fits LDS
// (E = 16, H = 2048: 100 KB). Measured on the chunked kernel above, staging
// (per-chunk global loads, conversion, LDS writes) cost as much as the
// dependent chains and did not overlap them: one wave does both. Here the
// router rows arrive by LDS DMA as bf16 (no registers, no VALU) in
// 512-column chunks: the first together with the block's token rows (once,
// as f32), the others while the chains run on the chunks before them; a
// router value is widened from its bf16 pair with one shift or mask, which
// fits the latency of the dependent add. Row strides are padded by 16 bytes
// so the 16 experts' (and the tokens') 16-byte reads hit disjoint banks.
static inline int router_res_row_bytes(int H) { return (H * 2 + 1023) / 1024 * 1024 + 16; }
static inline size_t router_res_lds(int H, int E, int tpb) {
  return (size_t)tpb * (H + 4) * 4 + (size_t)E * router_res_row_bytes(H) + 4 * RT_NT * 4;
}

template <typename XT>
__global__ __launch_bounds__(RT_NT) void moe_router_res_kernel(
    const XT *__restrict__ x, const uint16_t *__restrict__ router, int T, int H, int E, int EP,
    int top_k, int RSB, uint32_t *__restrict__ idx_out, float *__restrict__ w_out,
    uint32_t *__restrict__ user_idx, float *__restrict__ user_w, int by_logit) {
  extern __shared__ __align__(16) uint32_t smr[];
  const int tid = threadIdx.x, e = tid % EP, tl = tid / EP;
  const int TPB = RT_NT / EP;
  const int t = blockIdx.x * TPB + tl;
  const int XS = H + 4;                                   // token row stride (floats)
  float *xs = reinterpret_cast<float *>(smr);             // [TPB][XS] f32
  uint32_t *rs = smr + TPB * XS;                           // [E][RSB / 4] bf16 pairs
  float *logit = reinterpret_cast<float *>(rs + E * (RSB >> 2));
  static_assert(RT_NT == 64, "one wave per workgroup: LDS order needs no barrier");
  // 1. router rows by LDS DMA in 1 KB instructions, column-chunk order (the
  //    512 columns j of every row, then j + 1, ...): chunk 0 now, the rest
  //    after the token rows, so that the chains start on chunk 0 while the
  //    later chunks land (lanes past a row's end fill that row's padding;
  //    past the matrix the descriptor returns zeros)
  const int ipr = (H * 2 + 1023) >> 10;
  const __amdgpu_buffer_rsrc_t rr = buffer_rsrc(router, (uint32_t)E * (uint32_t)H * 2u);
  auto dma_chunk = [&](int j) {
    for (int row = 0; row < E; row++)
      lds_load16(rr, rs + row * (RSB >> 2) + j * 256, (uint32_t)row * (uint32_t)H * 2u + (uint32_t)j * 1024u + 16u * tid,
                 0u);
  };
  dma_chunk(0);
  // 2. the block's token rows as f32 (zeros for tokens past T): UB 8-column
  //    units per lane in flight per batch (one batch at H = 2048, E = 16);
  //    loads are unconditional from clamped addresses. Vector loads complete
  //    in issue order, so converting them waits for chunk 0 as well.
  {
    constexpr int NV = sizeof(XT) == 2 ? 1 : 2;  // 16-byte loads per unit
    constexpr int UB = sizeof(XT) == 2 ? 16 : 8;
    const int upr = H >> 3, units = TPB * upr;
    for (int u0 = 0; u0 < units; u0 += UB * RT_NT) {
      u32x4 raw[UB][NV];
#pragma unroll
      for (int q = 0; q < UB; q++) {
        const int u = min(u0 + q * RT_NT + tid, units - 1), rrow = u / upr, c = (u - rrow * upr) * 8;
        const int tt = min(blockIdx.x * TPB + rrow, T - 1);
        const u32x4 *src = reinterpret_cast<const u32x4 *>(x + (size_t)tt * H + c);
#pragma unroll
        for (int v = 0; v < NV; v++) raw[q][v] = src[v];
      }
#pragma unroll
      for (int q = 0; q < UB; q++) {
        const int u = u0 + q * RT_NT + tid;
        if (u < units) {
          const int rrow = u / upr, c = (u - rrow * upr) * 8;
          const uint32_t m = blockIdx.x * TPB + rrow < T ? 0xFFFFFFFFu : 0u;
          float v8[8];
          if constexpr (NV == 1) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
              const uint32_t w = raw[q][0][k] & m;
              v8[2 * k] = __uint_as_float(w << 16);
              v8[2 * k + 1] = __uint_as_float(w & 0xFFFF0000u);
            }
          } else {
#pragma unroll
            for (int k = 0; k < 4; k++) {
              v8[k] = __uint_as_float(raw[q][0][k] & m);
              v8[4 + k] = __uint_as_float(raw[q][1][k] & m);
            }
          }
          float4 *d = reinterpret_cast<float4 *>(xs + rrow * XS + c);
          d[0] = make_float4(v8[0], v8[1], v8[2], v8[3]);
          d[1] = make_float4(v8[4], v8[5], v8[6], v8[7]);
        }
      }
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the token rows are in LDS
  for (int j = 1; j < ipr; j++) dma_chunk(j);
  // chunk c has landed once at most (ipr - 1 - c) * E DMA instructions are
  // outstanding (rounded down to a multiple of 16 for the immediate wait:
  // waiting longer is safe); nothing else is in flight during the chains
  int landed = 1;  // chunk 0 landed before the token rows were converted
  auto ensure_chunk = [&](int c) {
    if (c < landed) return;  // wave-uniform
    const int rem = (ipr - 1 - c) * E;
    if (rem >= 48) wait_vmcnt<48>();
    else if (rem >= 32) wait_vmcnt<32>();
    else if (rem >= 16) wait_vmcnt<16>();
    else wait_vmcnt<0>();
    landed = c + 1;
  };
  // 3. one dependent chain per lane (left to right, as the reference)
  float sum = 0.0f;
  if (e < E && t < T) {
#pragma clang fp contract(off)
    const float *xr = xs + tl * XS;
    const uint32_t *rw = rs + e * (RSB >> 2);
    constexpr bool EXACT_PRODUCT = sizeof(XT) == 2;  // bf16 x bf16: exact in f32
    auto step = [&](float xe, float re) {
      if constexpr (EXACT_PRODUCT) sum = __fmaf_rn(xe, re, sum);
      else sum = sum + xe * re;
    };
    // 32-column blocks: 8 token reads + 4 router reads (12, within the LDS
    // wait counter), read one block ahead of the chain
    const int nblk = H >> 5;
    auto rd = [&](int b, f32x4 *xv, u32x4 *rv) {
      const int j = min(b, max(nblk - 1, 0)) * 32;
      ensure_chunk(j >> 9);
#pragma unroll
      for (int q = 0; q < 8; q++) xv[q] = *reinterpret_cast<const f32x4 *>(xr + j + 4 * q);
#pragma unroll
      for (int q = 0; q < 4; q++) rv[q] = *reinterpret_cast<const u32x4 *>(rw + (j >> 1) + 4 * q);
    };
    auto run = [&](const f32x4 *xv, const u32x4 *rv) {
#pragma unroll
      for (int q = 0; q < 4; q++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {  // router columns 8q + 2i, 8q + 2i + 1
          const uint32_t d = rv[q][i];
          step(xv[2 * q + (i >> 1)][(2 * i) & 3], __uint_as_float(d << 16));
          step(xv[2 * q + (i >> 1)][(2 * i + 1) & 3], __uint_as_float(d & 0xFFFF0000u));
        }
      }
    };
    f32x4 xa[8], xb[8];
    u32x4 ra[4], rb[4];
    rd(0, xa, ra);
    int b = 0;
    for (; b + 2 <= nblk; b += 2) {
      rd(b + 1, xb, rb);
      __builtin_amdgcn_sched_barrier(0);
      run(xa, ra);
      __builtin_amdgcn_sched_barrier(0);
      rd(b + 2, xa, ra);
      __builtin_amdgcn_sched_barrier(0);
      run(xb, rb);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (b < nblk) run(xa, ra);
    ensure_chunk(ipr - 1);
    for (int j = nblk * 32; j < H; j += 8) {  // H % 32 columns, 8 at a time
      const f32x4 x0 = *reinterpret_cast<const f32x4 *>(xr + j), x1 = *reinterpret_cast<const f32x4 *>(xr + j + 4);
      const u32x4 r = *reinterpret_cast<const u32x4 *>(rw + (j >> 1));
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const f32x4 &xv = i < 2 ? x0 : x1;
        step(xv[(2 * i) & 3], __uint_as_float(r[i] << 16));
        step(xv[(2 * i + 1) & 3], __uint_as_float(r[i] & 0xFFFF0000u));
      }
    }
  }
  wait_vmcnt<0>();  // every DMA landed (lanes without a chain skip the waits above)
  router_softmax_topk(sum, logit, tid, e, tl, t, T, E, EP, top_k, idx_out, w_out, user_idx, user_w, by_logit);
}

// Two-wave variant of the resident router (bf16 router weights): wave 1
// brings the router rows by LDS DMA and widens them to f32, 256 columns at a
// time, into a two-slot ring; wave 0 converts the token rows and runs the
// chains on the widened chunks, one chunk behind (one block barrier per
// chunk). A chain step is then one fused multiply-add (or multiply and add)
// and half a 16-byte read, the widening runs beside it on another SIMD.
constexpr int RP_CW = 256;  // columns per widened chunk
static inline size_t router_pair_lds(int H, int E, int tpb) {
  return (size_t)tpb * (H + 4) * 4 + (size_t)E * router_res_row_bytes(H) + (size_t)2 * E * (RP_CW + 4) * 4 +
         2 * 4 * RT_NT * 4;
}
template <typename XT>
__global__ __launch_bounds__(2 * RT_NT) void moe_router_pair_kernel(
    const XT *__restrict__ x, const uint16_t *__restrict__ router, int T, int H, int E, int EP,
    int top_k, int RSB, uint32_t *__restrict__ idx_out, float *__restrict__ w_out,
    uint32_t *__restrict__ user_idx, float *__restrict__ user_w, int by_logit) {
  extern __shared__ __align__(16) uint32_t smr[];
  const int tid = threadIdx.x & 63, wave = threadIdx.x >> 6, e = tid % EP, tl = tid / EP;
  const int TPB = RT_NT / EP;
  const int t = blockIdx.x * TPB + tl;
  const int XS = H + 4, RW = RP_CW + 4;
  float *xs = reinterpret_cast<float *>(smr);                  // [TPB][XS] f32
  uint32_t *rs = smr + TPB * XS;                                 // [E][RSB / 4] bf16 pairs (DMA)
  float *ring = reinterpret_cast<float *>(rs + E * (RSB >> 2));  // [2][E][RW] f32
  float *logit = ring + 2 * E * RW;                              // [2][4 RT_NT] (one per wave)
  const int ipr = (H * 2 + 1023) >> 10;    // 1 KB DMA instructions per row
  const int nch = (H + RP_CW - 1) / RP_CW;  // widened chunks
  if (wave == 1) {
    // every router row by LDS DMA, 1 KB instructions in column-block order
    const __amdgpu_buffer_rsrc_t rr = buffer_rsrc(router, (uint32_t)E * (uint32_t)H * 2u);
    for (int j = 0; j < ipr; j++)
      for (int row = 0; row < E; row++)
        lds_load16(rr, rs + row * (RSB >> 2) + j * 256,
                   (uint32_t)row * (uint32_t)H * 2u + (uint32_t)j * 1024u + 16u * tid, 0u);
  } else {
    // the block's token rows as f32 (zeros for tokens past T)
    constexpr int NV = sizeof(XT) == 2 ? 1 : 2;
    constexpr int UB = sizeof(XT) == 2 ? 16 : 8;
    const int upr = H >> 3, units = TPB * upr;
    for (int u0 = 0; u0 < units; u0 += UB * RT_NT) {
      u32x4 raw[UB][NV];
#pragma unroll
      for (int q = 0; q < UB; q++) {
        const int u = min(u0 + q * RT_NT + tid, units - 1), rrow = u / upr, c = (u - rrow * upr) * 8;
        const int tt = min(blockIdx.x * TPB + rrow, T - 1);
        const u32x4 *src = reinterpret_cast<const u32x4 *>(x + (size_t)tt * H + c);
#pragma unroll
        for (int v = 0; v < NV; v++) raw[q][v] = src[v];
      }
#pragma unroll
      for (int q = 0; q < UB; q++) {
        const int u = u0 + q * RT_NT + tid;
        if (u < units) {
          const int rrow = u / upr, c = (u - rrow * upr) * 8;
          const uint32_t m = blockIdx.x * TPB + rrow < T ? 0xFFFFFFFFu : 0u;
          float v8[8];
          if constexpr (NV == 1) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
              const uint32_t w = raw[q][0][k] & m;
              v8[2 * k] = __uint_as_float(w << 16);
              v8[2 * k + 1] = __uint_as_float(w & 0xFFFF0000u);
            }
          } else {
#pragma unroll
            for (int k = 0; k < 4; k++) {
              v8[k] = __uint_as_float(raw[q][0][k] & m);
              v8[4 + k] = __uint_as_float(raw[q][1][k] & m);
            }
          }
          float4 *d = reinterpret_cast<float4 *>(xs + rrow * XS + c);
          d[0] = make_float4(v8[0], v8[1], v8[2], v8[3]);
          d[1] = make_float4(v8[4], v8[5], v8[6], v8[7]);
        }
      }
    }
  }
  float sum = 0.0f;
  for (int c = 0; c < nch; c++) {
    float *slot = ring + (c & 1) * E * RW;
    if (wave == 1) {
      // chunk c lies in 1 KB column block jc: wait until at most the DMA
      // instructions of the blocks after jc are outstanding (rounded down
      // to the immediate waits; waiting longer is safe)
      const int jc = (c * RP_CW) >> 9, rem = (ipr - 1 - jc) * E;
      if (rem >= 48) wait_vmcnt<48>();
      else if (rem >= 32) wait_vmcnt<32>();
      else if (rem >= 16) wait_vmcnt<16>();
      else wait_vmcnt<0>();
      for (int u = tid; u < E * (RP_CW / 8); u += RT_NT) {
        const int row = u / (RP_CW / 8), c8 = (u % (RP_CW / 8)) * 8, col = c * RP_CW + c8;
        u32x4 r = (u32x4){0u, 0u, 0u, 0u};
        if (col < H) r = *reinterpret_cast<const u32x4 *>(rs + row * (RSB >> 2) + (col >> 1));
        float4 *d = reinterpret_cast<float4 *>(slot + row * RW + c8);
        d[0] = make_float4(__uint_as_float(r[0] << 16), __uint_as_float(r[0] & 0xFFFF0000u),
                           __uint_as_float(r[1] << 16), __uint_as_float(r[1] & 0xFFFF0000u));
        d[1] = make_float4(__uint_as_float(r[2] << 16), __uint_as_float(r[2] & 0xFFFF0000u),
                           __uint_as_float(r[3] << 16), __uint_as_float(r[3] & 0xFFFF0000u));
      }
    }
    __syncthreads();  // chunk c widened; chunk c - 1 consumed, its slot free again
    if (wave == 0 && e < E && t < T) {
#pragma clang fp contract(off)
      const int c0 = c * RP_CW, n = min(RP_CW, H - c0);
      const float *xr = xs + tl * XS + c0, *rw = slot + e * RW;
      constexpr bool EXACT_PRODUCT = sizeof(XT) == 2;  // bf16 x bf16: exact in f32
      auto step = [&](float xe, float re) {
        if constexpr (EXACT_PRODUCT) sum = __fmaf_rn(xe, re, sum);
        else sum = sum + xe * re;
      };
      const int nb = n >> 5;
      auto rd = [&](int b, f32x4 *xv, f32x4 *rv) {
        const int j = min(b, max(nb - 1, 0)) * 32;
#pragma unroll
        for (int q = 0; q < 8; q++) {
          xv[q] = *reinterpret_cast<const f32x4 *>(xr + j + 4 * q);
          rv[q] = *reinterpret_cast<const f32x4 *>(rw + j + 4 * q);
        }
      };
      auto run = [&](const f32x4 *xv, const f32x4 *rv) {
#pragma unroll
        for (int q = 0; q < 8; q++)
#pragma unroll
          for (int i = 0; i < 4; i++) step(xv[q][i], rv[q][i]);
      };
      // the next block's 16 reads go out before the current block's 32
      // steps; the scheduling barriers keep the compiler from sinking them
      // next to their use, where each group of 4 steps would wait out the
      // LDS latency (2048 columns: 10.8 -> 9.1 us of chain)
      f32x4 xa[8], xb[8], ra[8], rb[8];
      rd(0, xa, ra);
      int b = 0;
      for (; b + 2 <= nb; b += 2) {
        rd(b + 1, xb, rb);
        __builtin_amdgcn_sched_barrier(0);
        run(xa, ra);
        __builtin_amdgcn_sched_barrier(0);
        rd(b + 2, xa, ra);
        __builtin_amdgcn_sched_barrier(0);
        run(xb, rb);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (b < nb) run(xa, ra);
      for (int j = nb * 32; j < n; j += 4) {  // n % 32 columns, 4 at a time (H % 16 == 0)
        const f32x4 xv = *reinterpret_cast<const f32x4 *>(xr + j), rv = *reinterpret_cast<const f32x4 *>(rw + j);
#pragma unroll
        for (int i = 0; i < 4; i++) step(xv[i], rv[i]);
      }
    }
  }
  // wave 1 joins the softmax's barriers on its own LDS, as no token (t = T)
  router_softmax_topk(sum, logit + wave * 4 * RT_NT, tid, e, tl, wave == 0 ? t : T, T, E, EP, top_k, idx_out, w_out,
                      user_idx, user_w, by_logit);
}
#pragma clang fp contract(on)

// ---- 2. histogram / scan / stable scatter / tile schedule -----------------
// Exclusive prefix sum of v over the 64 lanes of a wave: shifts by 1, 2, 4
// and 8 within each row of 16 lanes, then row 0's total into row 1 and row
// 2's into row 3 (row_bcast:15), then rows 0-1's total into rows 2-3
// (row_bcast:31). Lanes without a source add 0.
__device__ __forceinline__ int wave_excl_scan(int v) {
  int x = v;
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return x - v;
}

// Tiles: 4 ints each, (expert, first row within the expert, rows, token
// blocks). An expert's rows are split into ceil(rows / bm_max) tiles of
// equal height (the last one shorter); token blocks = max(fm_min,
// ceil(rows / 16)) is the number of 16-row MFMA blocks a tile multiplies.
// The list runs by descending token blocks so that the largest tiles are
// dispatched first.
__global__ __launch_bounds__(1024) void moe_group_kernel(
    const uint32_t *__restrict__ idx, int A, int top_k, int E, int bm_max, int fm_min,
    int *__restrict__ counts, int *__restrict__ offsets,
    int *__restrict__ perm_token, int *__restrict__ inv,
    int *__restrict__ tiles, int *__restrict__ ntiles, int *__restrict__ row_expert) {
  __shared__ int wave_cnt[16][MOE_MAXE];
  __shared__ int base[MOE_MAXE];
  __shared__ int offs[MOE_MAXE + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid < MOE_MAXE) base[tid] = 0;
  __syncthreads();
  // Pass 1: rank of each assignment within its expert, in (t, k) order (the
  // last chunk's expert and rank stay in registers for pass 2).
  int e_last = -1, r_last = 0;
  for (int c0 = 0; c0 < A; c0 += 1024) {
    const int a = c0 + tid;
    const int e = a < A ? (int)idx[a] : -1;
    e_last = e;
    int rank = 0;
    for (int ee = 0; ee < E; ee++) {
      const unsigned long long m = __ballot(e == ee);
      if (lane == 0) wave_cnt[wave][ee] = __popcll(m);
      if (e == ee) rank = __popcll(m & ((1ull << lane) - 1ull));
    }
    __syncthreads();
    if (e >= 0) {
      int before = base[e];
      for (int w = 0; w < wave; w++) before += wave_cnt[w][e];
      r_last = before + rank;  // position within the expert (fixed below)
      if (c0 + 1024 < A) inv[a] = r_last;
    }
    __syncthreads();
    if (tid < E) {
      int s = 0;
      for (int w = 0; w < 16; w++) s += wave_cnt[w][tid];
      base[tid] += s;
    }
    __syncthreads();
  }
  if (wave == 0) {
    // lane ee: expert ee's offset (exclusive scan of the counts) and tiles
    const int c = lane < E ? base[lane] : 0;
    const int off = wave_excl_scan(c);
    if (lane < E) {
      offs[lane] = off;
      counts[lane] = c;
      offsets[lane] = off;
    }
    if (lane == 63) {
      offs[E] = off + c;
      offsets[E] = off + c;
    }
    // n tiles: n - 1 of `rows` rows, the last of c - (n - 1) rows
    // (rows <= bm_max and (n - 1) * rows < c: every tile is non-empty)
    const int n = (c + bm_max - 1) / bm_max, rows = n ? (c + n - 1) / n : 0;
    const int fa = max(fm_min, (rows + 15) / 16), fb = max(fm_min, (c - (n - 1) * rows + 15) / 16);
    const int fm_top = max(fm_min, (bm_max + 15) / 16);
    int nt = 0;
    for (int f = fm_top; f >= fm_min; f--) {
      const int na = (n > 1 && fa == f) ? n - 1 : 0, nb = (n > 0 && fb == f) ? 1 : 0;
      const int before = wave_excl_scan(na + nb);
      int pos = nt + before;
      for (int i = 0; i < n; i++) {
        const int fi = i < n - 1 ? fa : fb;
        if (fi != f) continue;
        tiles[4 * pos] = lane;
        tiles[4 * pos + 1] = i * rows;
        tiles[4 * pos + 2] = min(rows, c - i * rows);
        tiles[4 * pos + 3] = f;
        pos++;
      }
      nt += __shfl(before + na + nb, 63);
    }
    if (lane == 0) *ntiles = nt;
  }
  __syncthreads();
  // Pass 2: final rows.
  const int a_last = (A - 1) / 1024 * 1024 + tid;  // this thread's assignment of the last chunk
  for (int a = tid; a < A; a += 1024) {
    const bool reg = a == a_last;
    const int e = reg ? e_last : (int)idx[a];
    const int pos = offs[e] + (reg ? r_last : inv[a]);
    inv[a] = pos;
    perm_token[pos] = a / top_k;
    row_expert[pos] = e;
  }
}

// ---- LoRA adapters of the experts --------------------------------------------
// CpuMoELayer::expert_forward_*_with_lora (src/model/cpu_moe.rs:281-363) with
// LoraLayer::forward (src/training/lora.rs:138-167): lora(v) = scaling *
// B (A v). Per expert-sorted row a, this kernel writes A v for the adapter
// kinds [kind0, kind0 + nk) (0 gate, 1 up: v = x of the row's token; 2 down:
// v = h = hi + lo of the row) to out[a][(k - kind0) * rank + r], zeros where
// the row's expert has no adapter of that kind. One workgroup per row, one
// wave per rank index at a time, lane-strided dot products reduced across
// the wave. The epilogues of the grouped GEMMs add scaling * B (A v).
template <typename XT>
__global__ __launch_bounds__(256) void moe_lora_a_kernel(
    const float *const *__restrict__ tbl, int rank, const XT *__restrict__ x, const int *__restrict__ perm_token,
    const int *__restrict__ row_expert, const uint16_t *__restrict__ hh, const uint16_t *__restrict__ hl,
    long hstride, int D, int kind0, int nk, float *__restrict__ out, int out_stride) {
  const int a = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = row_expert[a];
  for (int k = kind0; k < kind0 + nk; k++) {
    const float *Am = tbl[(2 * k) * MOE_MAXE + e], *Bm = tbl[(2 * k + 1) * MOE_MAXE + e];
    for (int r = wave; r < rank; r += 4) {
      float sum = 0.f;
      if (Am && Bm) {
        if (k < 2) {
          const long t = perm_token[a];
          for (int d = lane; d < D; d += 64) sum += Am[(long)r * D + d] * ld_f32(x, t * D + d);
        } else {
          for (int d = lane; d < D; d += 64) {
            const float h = __uint_as_float((uint32_t)hh[a * hstride + d] << 16) +
                            __uint_as_float((uint32_t)hl[a * hstride + d] << 16);
            sum += Am[(long)r * D + d] * h;
          }
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o);
      }
      if (lane == 0) out[(long)a * out_stride + (k - kind0) * rank + r] = sum;
    }
  }
}

// scaling * sum_r B[n][r] * av[r] (0 without the adapter's B matrix).
__device__ __forceinline__ float lora_b(const float *Bm, int n, int rank, const float *av, float scaling) {
  if (!Bm) return 0.f;
  float s = 0.f;
  for (int r = 0; r < rank; r++) s += Bm[(long)n * rank + r] * av[r];
  return s * scaling;
}

// ---- 3. grouped gate/up GEMM + activation -----------------------------------
struct GateUpArgs {
  const uint32_t *wg[MOE_MAXE];
  const uint32_t *wu[MOE_MAXE];
  const float *sg[MOE_MAXE];
  const float *su[MOE_MAXE];
};


template <int XS>
__global__ __launch_bounds__(256) void moe_gateup_kernel(
    const GateUpArgs args, const void *__restrict__ x, int H, int I,
    const int *__restrict__ tiles, const int *__restrict__ ntiles,
    const int *__restrict__ counts, const int *__restrict__ offsets,
    const int *__restrict__ perm_token, uint16_t *__restrict__ h_hi,
    uint16_t *__restrict__ h_lo, int act, const float *const *__restrict__ ltbl, int lrank, float lscale,
    const float *__restrict__ lax) {
  using Core = GemmCore<MOE_BM, MOE_BN, 1, 4, XS, 2>;
  __shared__ __align__(16) uint32_t lds[Core::LDS_DWORDS];
  const int tile = blockIdx.y;
  if (tile >= *ntiles) return;
  const int e = tiles[4 * tile], mstart = tiles[4 * tile + 1];
  const int mcount = tiles[4 * tile + 2];
  const int row0 = offsets[e] + mstart;
  const int n0 = blockIdx.x * MOE_BN;
  XDesc xd{x, nullptr, perm_token + row0, 0, H, 1};
  const uint32_t *Wm[2] = {args.wg[e], args.wu[e]};
  const int wvec = ((H >> 4) % 4 == 0);
  f32x4 acc[2][Core::FN][Core::FM];
  Core::run(lds, xd, mcount, Wm, n0, I, H, wvec, acc);
#pragma unroll
  for (int fn = 0; fn < Core::FN; fn++) {
    const int n = n0 + Core::rowoff(fn);
    if (n >= I) continue;
    const int nok = min(4, I - n);
    const f32x4 sg = load_scale4(args.sg[e], n, nok) * 0.5f;
    const f32x4 su = load_scale4(args.su[e], n, nok) * 0.5f;
#pragma unroll
    for (int fm = 0; fm < Core::FM; fm++) {
      const int m = Core::tok(fm);
      if (m >= mcount) continue;
      f32x4 g = acc[0][fn][fm] * sg, u = acc[1][fn][fm] * su;
      if (ltbl) {  // LoRA: gated += lora_gate(x), upped += lora_up(x)
        const float *av = lax + (long)(row0 + m) * (2 * MOE_LORA_MAXR);
        const float *Bg = ltbl[1 * MOE_MAXE + e], *Bu = ltbl[3 * MOE_MAXE + e];
        for (int j = 0; j < nok; j++) {
          g[j] += lora_b(Bg, n + j, lrank, av, lscale);
          u[j] += lora_b(Bu, n + j, lrank, av + lrank, lscale);
        }
      }
      float hv[4];
      for (int j = 0; j < 4; j++) hv[j] = moe_act(act, g[j], u[j]);
      uint32_t hh[4], hl[4];
      for (int j = 0; j < 4; j++) split_bf16(hv[j], hh[j], hl[j]);
      const long o = (long)(row0 + m) * I + n;
      if (nok == 4) {
        *reinterpret_cast<u32x2 *>(h_hi + o) = (u32x2){hh[0] | (hh[1] << 16), hh[2] | (hh[3] << 16)};
        *reinterpret_cast<u32x2 *>(h_lo + o) = (u32x2){hl[0] | (hl[1] << 16), hl[2] | (hl[3] << 16)};
      } else {
        for (int j = 0; j < nok; j++) {
          h_hi[o + j] = (uint16_t)hh[j];
          h_lo[o + j] = (uint16_t)hl[j];
        }
      }
    }
  }
}

// ---- 4. grouped down GEMM ---------------------------------------------------
struct DownArgs {
  const uint32_t *wd[MOE_MAXE];
  const float *sd[MOE_MAXE];
};

__global__ __launch_bounds__(256) void moe_down_kernel(
    const DownArgs args, const uint16_t *__restrict__ h_hi,
    const uint16_t *__restrict__ h_lo, int H, int I,
    const int *__restrict__ tiles, const int *__restrict__ ntiles,
    const int *__restrict__ counts, const int *__restrict__ offsets,
    float *__restrict__ dout, const float *const *__restrict__ ltbl, int lrank, float lscale,
    const float *__restrict__ lah) {
  using Core = GemmCore<MOE_BM, MOE_BN, 1, 4, XS_BF16X2, 1>;
  __shared__ __align__(16) uint32_t lds[Core::LDS_DWORDS];
  const int tile = blockIdx.y;
  if (tile >= *ntiles) return;
  const int e = tiles[4 * tile], mstart = tiles[4 * tile + 1];
  const int mcount = tiles[4 * tile + 2];
  const int row0 = offsets[e] + mstart;
  const int n0 = blockIdx.x * MOE_BN;
  XDesc xd{h_hi, h_lo, nullptr, (long)row0, I, 1};
  const uint32_t *Wm[1] = {args.wd[e]};
  const int wvec = ((I >> 4) % 4 == 0);
  f32x4 acc[1][Core::FN][Core::FM];
  Core::run(lds, xd, mcount, Wm, n0, H, I, wvec, acc);
#pragma unroll
  for (int fn = 0; fn < Core::FN; fn++) {
    const int n = n0 + Core::rowoff(fn);
    if (n >= H) continue;
    const int nok = min(4, H - n);
    const f32x4 sd = load_scale4(args.sd[e], n, nok) * 0.5f;
#pragma unroll
    for (int fm = 0; fm < Core::FM; fm++) {
      const int m = Core::tok(fm);
      if (m >= mcount) continue;
      f32x4 v = acc[0][fn][fm] * sd;
      if (ltbl) {  // LoRA: down += lora_down(h)
        const float *av = lah + (long)(row0 + m) * MOE_LORA_MAXR;
        for (int j = 0; j < nok; j++) v[j] += lora_b(ltbl[5 * MOE_MAXE + e], n + j, lrank, av, lscale);
      }
      YStore<float>::store4(dout + (long)(row0 + m) * H + n, v, nok);
    }
  }
}

// ---- 3b/4b. the grouped GEMMs on the pipelined engine -------------------------
// bf16 activations, H % 64 == 0, I % 64 == 0, 16-byte aligned weights. A tile
// holds up to MOE3_BM expert-sorted token rows (the schedule of
// moe_group_kernel with bm_max = MOE3_BM) and multiplies 4, 5 or 6 blocks of
// 16 tokens, chosen per tile at run time, so that an expert with up to 96
// tokens streams its weights once and pads to 16 rows at most.
constexpr int MOE3_BM = 96;
constexpr int MOE3_FMIN = 4;  // the engine's operand schedule needs 4 token blocks
// gate/up: one 256-row weight tile holds 128 gate rows and the same 128 up
// rows (frx_gemm2.hpp dual weights), token rows gathered through
// perm_token; the epilogue writes h = act(g) * u as bf16 hi | lo halves of
// one row of h2 [A][2 I].
constexpr int MOE_GU_BN = 256;
constexpr int MOE_NS = 4;  // pipeline stages of the gate/up K loop
using MoeGateUpCore = Gemm2<MOE3_BM, MOE_GU_BN, 1, 4, MOE_NS, true>;
// down: the X stage holds a tile's rows twice (DUALX), as their hi halves
// (stage rows 0..95, waves 0 and 2) and their lo halves (rows 96..191, waves
// 1 and 3); each pair of waves shares 64 weight rows, so one K loop covers
// both planes of h and the lo waves hand their sums to the hi waves at the
// end: d = 0.5 s (acc_hi + acc_lo), fp32 rows of dout.
constexpr int MOE3_DBN = 128;
constexpr int MOE3_DNS = 3;
using MoeDownCore = Gemm2<2 * MOE3_BM, MOE3_DBN, 2, 2, MOE3_DNS, false, true>;
static_assert(MoeGateUpCore::FM == 6 && MoeDownCore::FM == 6, "token blocks per tile");

template <int F>
__device__ __forceinline__ void gateup_tile(uint32_t *lds, const GateUpArgs &args, const uint16_t *x, int ldx, int T,
                                            int H, int I, int e, int mcount, int row0, const int *perm_token,
                                            uint16_t *h2, int act, const MoeLora &lora, const float *lax) {
  using Core = MoeGateUpCore;
  const int n0 = blockIdx.x * (MOE_GU_BN / 2), nc = min(MOE_GU_BN / 2, I - n0);
  f32x4 acc[Core::FN][F];
  // ldx = 2 H: x rows are an fp32 activation as bf16 hi | lo halves, one K
  // loop of 2 H columns whose weight columns wrap at H
  Core::template run<F>(lds, x, (uint32_t)T * (uint32_t)ldx * 2u, perm_token + row0, mcount,
                        args.wg[e] + (size_t)n0 * (H >> 4), nc, ldx, acc, args.wu[e] + (size_t)n0 * (H >> 4), H,
                        ldx);
  // Epilogue: the fragments go to LDS in passes of up to PB token blocks (row
  // pitch MOE_GU_BN + 16 floats); each thread then owns 4 gate columns (and
  // the same 4 up columns MOE_GU_BN / 2 further) of a run of tokens per pass.
  constexpr int PF = MOE_GU_BN + 16, PB = 3;
  static_assert(PB * 16 * PF <= Core::LDS_DWORDS, "epilogue staging");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, g = lane >> 4;
  float *st = reinterpret_cast<float *>(lds);
  constexpr int CT = MOE_GU_BN / 8, RT = 256 / CT;  // column threads, rows per iteration
  const int c = threadIdx.x % CT, rr = threadIdx.x / CT;
  f32x4 sgv, suv;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int n = n0 + min(4 * c + j, nc - 1);
    sgv[j] = 0.5f * args.sg[e][n];  // 0.5 undoes the 2*dec(c) operand encoding
    suv[j] = 0.5f * args.su[e][n];
  }
#pragma unroll
  for (int f0 = 0; f0 < F; f0 += PB) {
#pragma unroll
    for (int fn = 0; fn < Core::FN; fn++)
#pragma unroll
      for (int fi = 0; fi < PB; fi++)
        if (f0 + fi < F)
          *reinterpret_cast<f32x4 *>(st + (fi * 16 + l16) * PF + wave * Core::TN + fn * 16 + 4 * g) =
              acc[fn][f0 + fi];
    __syncthreads();
    const int rows = min(PB, F - f0) * 16;
    for (int lr = rr; lr < rows; lr += RT) {
      const int m = f0 * 16 + lr;
      if (m >= mcount || 4 * c >= nc) continue;
      f32x4 gv = *reinterpret_cast<const f32x4 *>(st + lr * PF + 4 * c) * sgv;
      f32x4 uv = *reinterpret_cast<const f32x4 *>(st + lr * PF + MOE_GU_BN / 2 + 4 * c) * suv;
      if (lora.tbl) {  // LoRA: gated += lora_gate(x), upped += lora_up(x)
        const float *av = lax + (long)(row0 + m) * (2 * MOE_LORA_MAXR);
        const float *Bg = lora.tbl[1 * MOE_MAXE + e], *Bu = lora.tbl[3 * MOE_MAXE + e];
        for (int j = 0; j < 4 && 4 * c + j < nc; j++) {
          gv[j] += lora_b(Bg, n0 + 4 * c + j, lora.rank, av, lora.scaling);
          uv[j] += lora_b(Bu, n0 + 4 * c + j, lora.rank, av + lora.rank, lora.scaling);
        }
      }
      uint32_t hh[4], hl[4];
#pragma unroll
      for (int j = 0; j < 4; j++) split_bf16(moe_act(act, gv[j], uv[j]), hh[j], hl[j]);
      uint16_t *d = h2 + (size_t)(row0 + m) * (2 * (size_t)I) + n0 + 4 * c;
      if (4 * c + 4 <= nc) {
        *reinterpret_cast<u32x2 *>(d) = (u32x2){hh[0] | (hh[1] << 16), hh[2] | (hh[3] << 16)};
        *reinterpret_cast<u32x2 *>(d + I) = (u32x2){hl[0] | (hl[1] << 16), hl[2] | (hl[3] << 16)};
      } else {
        for (int j = 0; j < nc - 4 * c; j++) {
          d[j] = (uint16_t)hh[j];
          d[I + j] = (uint16_t)hl[j];
        }
      }
    }
    __syncthreads();
  }
}

// grid (ceil(I / 128), tile slots); slots past *ntiles exit at once.
__global__ __launch_bounds__(256) void moe_gateup3_kernel(
    const GateUpArgs args, const uint16_t *__restrict__ x, int ldx, int T, int H, int I,
    const int *__restrict__ tiles, const int *__restrict__ ntiles,
    const int *__restrict__ offsets, const int *__restrict__ perm_token,
    uint16_t *__restrict__ h2, int act, const MoeLora lora, const float *__restrict__ lax) {
  extern __shared__ __align__(16) uint32_t lds[];
  const int tile = blockIdx.y;
  if (tile >= *ntiles) return;  // whole workgroup
  const int e = tiles[4 * tile], row0 = offsets[e] + tiles[4 * tile + 1];
  const int mcount = tiles[4 * tile + 2], f = tiles[4 * tile + 3];
  if (f <= 4) gateup_tile<4>(lds, args, x, ldx, T, H, I, e, mcount, row0, perm_token, h2, act, lora, lax);
  else if (f == 5) gateup_tile<5>(lds, args, x, ldx, T, H, I, e, mcount, row0, perm_token, h2, act, lora, lax);
  else gateup_tile<6>(lds, args, x, ldx, T, H, I, e, mcount, row0, perm_token, h2, act, lora, lax);
}

template <int F>
__device__ __forceinline__ void down_tile(uint32_t *lds, const DownArgs &args, const uint16_t *h2, int H, int I,
                                          int ks, int part, int nt, int e, int mcount, int row0, float *dout,
                                          const MoeLora &lora, const float *lah) {
  using Core = MoeDownCore;
  const int n0 = nt * MOE3_DBN, nc = min(MOE3_DBN, H - n0);
  const int k0 = part * ks;
  f32x4 acc[Core::FN][F];
  // X = the tile's rows of h2 from column k0; stage rows >= 96 read the same
  // rows I columns further (the lo halves)
  Core::template run<F>(lds, h2 + (size_t)row0 * (2 * (size_t)I) + k0,
                        (uint32_t)mcount * (uint32_t)I * 4u - (uint32_t)k0 * 2u, nullptr, mcount,
                        args.wd[e] + (size_t)n0 * (I >> 4) + (k0 >> 4), nc, ks, acc, nullptr, I, 2 * I,
                        (uint32_t)I * 2u);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, wm = wave % 2, wn = wave / 2;
  // lane-linear exchange slots: [wn][fn][fm][lane] of 16 bytes (48 KB)
  f32x4 *xs = reinterpret_cast<f32x4 *>(lds);
  if (wm == 1) {
#pragma unroll
    for (int fn = 0; fn < Core::FN; fn++)
#pragma unroll
      for (int fm = 0; fm < F; fm++) xs[((wn * Core::FN + fn) * F + fm) * 64 + lane] = acc[fn][fm];
  }
  __syncthreads();
  if (wm == 0) {
    const int l16 = lane & 15, g = lane >> 4;
#pragma unroll
    for (int fn = 0; fn < Core::FN; fn++) {
      const int nl = wn * Core::TN + fn * 16 + 4 * g;
      if (nl >= nc) continue;
      const int nok = min(4, nc - nl);
      const f32x4 sd = load_scale4(args.sd[e], n0 + nl, nok) * 0.5f;
#pragma unroll
      for (int fm = 0; fm < F; fm++) {
        const int m = fm * 16 + l16;
        f32x4 v = (acc[fn][fm] + xs[((wn * Core::FN + fn) * F + fm) * 64 + lane]) * sd;
        if (m >= mcount) continue;
        if (lora.tbl && part == 0) {  // LoRA: down += lora_down(h), in the first K part only
          const float *av = lah + (long)(row0 + m) * MOE_LORA_MAXR;
          for (int j = 0; j < nok; j++)
            v[j] += lora_b(lora.tbl[5 * MOE_MAXE + e], n0 + nl + j, lora.rank, av, lora.scaling);
        }
        YStore<float>::store4(dout + (size_t)(row0 + m) * H + n0 + nl, v, nok);
      }
    }
  }
}

// 1-D grid of 8 * slots * NTN * KP workgroups (NTN = ceil(H / 128) column
// tiles, KP = I / ks K parts). Workgroup L runs on XCD L % 8 (the dispatch
// order of the 8 XCDs); each XCD takes the tiles t with t % 8 == its index
// and all NTN * KP items of such a tile, so a tile's h rows are fetched into
// one L2. Part p of the K range writes its own fp32 rows (dout, dout_lo);
// the combine adds them in a fixed order.
__global__ __launch_bounds__(256) void moe_down3_kernel(
    const DownArgs args, const uint16_t *__restrict__ h2, int H, int I, int ks, int ntn, int kp,
    const int *__restrict__ tiles, const int *__restrict__ ntiles, const int *__restrict__ offsets,
    float *__restrict__ dout, float *__restrict__ dout_lo, const MoeLora lora, const float *__restrict__ lah) {
  extern __shared__ __align__(16) uint32_t lds[];
  const int L = blockIdx.x, xcd = L & 7, j = L >> 3, per = ntn * kp;
  const int tile = xcd + 8 * (j / per);
  if (tile >= *ntiles) return;  // whole workgroup
  const int item = j % per, nt = item % ntn, part = item / ntn;
  const int e = tiles[4 * tile], row0 = offsets[e] + tiles[4 * tile + 1];
  const int mcount = tiles[4 * tile + 2], f = tiles[4 * tile + 3];
  float *out = part == 0 ? dout : dout_lo;
  if (f <= 4) down_tile<4>(lds, args, h2, H, I, ks, part, nt, e, mcount, row0, out, lora, lah);
  else if (f == 5) down_tile<5>(lds, args, h2, H, I, ks, part, nt, e, mcount, row0, out, lora, lah);
  else down_tile<6>(lds, args, h2, H, I, ks, part, nt, e, mcount, row0, out, lora, lah);
}

// ---- 3c/4c. decode: a few routed rows ------------------------------------------
// With T * top_k <= MOE_DEC_MAXA routed rows (decode: one token, top-2) the
// grouped GEMMs leave almost every workgroup empty and run each expert's K
// loop on one tile, latency-bound. These two kernels are GEMVs per routed
// row instead, in routing order (row a = token a / top_k, its j-th expert),
// so the group kernel is not needed: the combine reads row a for assignment
// a (inv = identity, written here). Weights stream once per routed row (top-k
// experts of one token are distinct).
//
// MFMA GEMV: a wave multiplies 16 weight rows by the row's activation; lane
// (i, g) loads 16 bytes of row i (4 code words = 64 consecutive columns, the
// g-th 64 of each 256), unpacks each word into two 8-column operands, and
// the B operand of lane group g is the activation at the same columns (every
// B column holds the same activation, so any output column is the result).
// fp32 activations are multiplied as bf16 hi and lo planes (two MFMAs).
constexpr int MOE_DEC_ROWS = 64;  // weight rows of each matrix per workgroup

// The activation slice [0, n) of one row into LDS as bf16 hi (and, for f32,
// lo) planes, zero-padded to np columns; n and np multiples of 8, src 16-byte
// aligned. Each thread moves 8 columns per unit and issues the loads of up
// to 4 units before converting any.
template <typename XT>
__device__ __forceinline__ void dec_stage_row(const XT *src, int n, int np, uint16_t *hi, uint16_t *lo) {
  constexpr int U = 4;
  const int step = (int)blockDim.x * 8;
  for (int c0 = (int)threadIdx.x * 8; c0 < np; c0 += step * U) {
    u32x4 raw[U][sizeof(XT) == 2 ? 1 : 2];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int c = c0 + u * step;
#pragma unroll
      for (int v = 0; v < (sizeof(XT) == 2 ? 1 : 2); v++) {
        raw[u][v] = (u32x4){0u, 0u, 0u, 0u};
        if (c < n) raw[u][v] = *reinterpret_cast<const u32x4 *>(src + c + 4 * v);
      }
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int c = c0 + u * step;
      if (c >= np) break;
      if constexpr (sizeof(XT) == 2) {
        *reinterpret_cast<u32x4 *>(hi + c) = raw[u][0];
      } else {
        u32x4 h, l;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const float a = __uint_as_float(raw[u][q >> 1][2 * (q & 1)]);
          const float b = __uint_as_float(raw[u][q >> 1][2 * (q & 1) + 1]);
          uint32_t hq, lq;
          split2_bf16(a, b, hq, lq);
          h[q] = hq;
          l[q] = lq;
        }
        *reinterpret_cast<u32x4 *>(hi + c) = h;
        *reinterpret_cast<u32x4 *>(lo + c) = l;
      }
    }
  }
}

// acc[f] += W[row f][0 .. kl) . act for NF 16-row fragments (rows clamped by
// the caller), kl % 64 == 0. The weight loads of CH 256-column blocks of
// every fragment are issued before any is used (the first batch before the
// activation is staged: stage() fills LDS and meets the block barrier), so
// a wave waits one memory round trip per batch rather than per block.
template <bool LO, int NF, int CH, typename Stage>
__device__ __forceinline__ void dec_gemv(const uint32_t *const (&wrow)[NF], int kl, const uint16_t *hi,
                                         const uint16_t *lo, f32x4 (&acc)[NF], Stage stage) {
  const int g = (threadIdx.x & 63) >> 4;
  u32x4 wq[NF][CH];
  // independent accumulation chains (the two word halves, each plane)
  f32x4 part[NF][LO ? 4 : 2];
#pragma unroll
  for (int f = 0; f < NF; f++)
#pragma unroll
    for (int q = 0; q < (LO ? 4 : 2); q++) part[f][q] = (f32x4){0.f, 0.f, 0.f, 0.f};
  auto fetch = [&](int c00) {
#pragma unroll
    for (int f = 0; f < NF; f++)
#pragma unroll
      for (int c = 0; c < CH; c++) {
        const int col = c00 + 256 * c + 64 * g;
        wq[f][c] = (u32x4){0x55555555u, 0x55555555u, 0x55555555u, 0x55555555u};  // code 1: zero
        if (col < kl) wq[f][c] = *reinterpret_cast<const u32x4 *>(wrow[f] + (col >> 4));
      }
  };
  fetch(0);
  stage();
  for (int c00 = 0; c00 < kl; c00 += 256 * CH) {
    if (c00 > 0) fetch(c00);
#pragma unroll
    for (int c = 0; c < CH; c++) {
      const int col = c00 + 256 * c + 64 * g;  // past kl: zero weights, zero-padded activation
#pragma unroll
      for (int w = 0; w < 4; w++) {
        const int cc = col + 16 * w;
        const u32x4 b0 = *reinterpret_cast<const u32x4 *>(hi + cc), b1 = *reinterpret_cast<const u32x4 *>(hi + cc + 8);
        u32x4 l0, l1;
        if constexpr (LO) {
          l0 = *reinterpret_cast<const u32x4 *>(lo + cc);
          l1 = *reinterpret_cast<const u32x4 *>(lo + cc + 8);
        }
#pragma unroll
        for (int f = 0; f < NF; f++) {
          u32x4 a0, a1;
          unpack16_nat(wq[f][c][w], a0, a1);
          part[f][0] = mfma16(a0, b0, part[f][0]);
          part[f][1] = mfma16(a1, b1, part[f][1]);
          if constexpr (LO) {
            part[f][2] = mfma16(a0, l0, part[f][2]);
            part[f][3] = mfma16(a1, l1, part[f][3]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int f = 0; f < NF; f++) {
    acc[f] = acc[f] + part[f][0] + part[f][1];
    if constexpr (LO) acc[f] = acc[f] + part[f][2] + part[f][3];
  }
}

// Columns of LDS staging for a row of n activations: whole 256-column
// blocks of the CH-block batches (the batch past the end reads zeros).
__host__ __device__ constexpr int dec_pad(int n, int ch) { return (n + 256 * ch - 1) / (256 * ch) * (256 * ch); }
// The two K halves of a workgroup: [0, kc) and [kc, n), kc a multiple of 64,
// and the staged columns both halves read (each reads whole batches).
__host__ __device__ constexpr int dec_half(int n) { return (n / 2 + 63) / 64 * 64; }
__host__ __device__ constexpr int dec_pad2(int n, int ch) {
  return dec_pad(dec_half(n), ch) > dec_half(n) + dec_pad(n - dec_half(n), ch)
             ? dec_pad(dec_half(n), ch)
             : dec_half(n) + dec_pad(n - dec_half(n), ch);
}
constexpr int MOE_DEC_GU_CH = 4, MOE_DEC_DN_CH = 6;

// grid (ceil(I / 64), A), 8 waves: waves 0-1 (and 4-5) gate rows n0 .. n0 +
// 63, waves 2-3 (6-7) the same up rows; waves 0-3 multiply the first K half,
// 4-7 the second, and add their sums through LDS (first half + second);
// h[a][n] = act(g, u) as fp32 rows [A][I].
template <typename XT>
__global__ __launch_bounds__(512) void moe_dec_gateup_kernel(const GateUpArgs args, const XT *__restrict__ x, int H,
                                                             int I, int top_k, const uint32_t *__restrict__ idx,
                                                             float *__restrict__ h, int *__restrict__ inv, int act) {
  extern __shared__ __align__(16) uint16_t dsm[];
  const int kc = dec_half(H), hp = dec_pad2(H, MOE_DEC_GU_CH);
  uint16_t *xh = dsm, *xl = dsm + hp;
  float *gu = reinterpret_cast<float *>(dsm + 2 * hp);  // [2][64]
  f32x4 *red = reinterpret_cast<f32x4 *>(gu + 2 * MOE_DEC_ROWS);  // [4 waves][2][64 lanes]
  const int a = blockIdx.y, t = a / top_k, e = (int)idx[a];
  if (blockIdx.x == 0 && threadIdx.x == 0) inv[a] = a;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kh = wave >> 2, wl = wave & 3, mat = wl >> 1;
  const int n0 = blockIdx.x * MOE_DEC_ROWS;
  const int ko = kh ? kc : 0, kl = kh ? H - kc : kc;
  const uint32_t *W = mat ? args.wu[e] : args.wg[e];
  const uint32_t *wrow[2];
#pragma unroll
  for (int f = 0; f < 2; f++)
    wrow[f] = W + (size_t)min(n0 + (wl & 1) * 32 + f * 16 + (lane & 15), I - 1) * (H >> 4) + (ko >> 4);
  f32x4 acc[2] = {(f32x4){0.f, 0.f, 0.f, 0.f}, (f32x4){0.f, 0.f, 0.f, 0.f}};
  auto stage = [&]() {
    dec_stage_row<XT>(x + (size_t)t * H, H, hp, xh, xl);
    __syncthreads();
  };
  if (W) {
    dec_gemv<sizeof(XT) == 4, 2, MOE_DEC_GU_CH>(wrow, kl, xh + ko, xl + ko, acc, stage);
  } else {  // gate-only experts: no up rows
    stage();
  }
  if (kh) {
#pragma unroll
    for (int f = 0; f < 2; f++) red[(wl * 2 + f) * 64 + lane] = acc[f];
  }
  __syncthreads();
  if (!kh && (lane & 15) == 0) {
#pragma unroll
    for (int f = 0; f < 2; f++) {
      const f32x4 v = acc[f] + red[(wl * 2 + f) * 64 + lane];
#pragma unroll
      for (int j = 0; j < 4; j++) gu[mat * 64 + (wl & 1) * 32 + f * 16 + 4 * (lane >> 4) + j] = v[j];
    }
  }
  __syncthreads();
  const int n = n0 + (int)threadIdx.x;
  if (threadIdx.x < MOE_DEC_ROWS && n < I) {
    const float gv = gu[threadIdx.x] * (0.5f * args.sg[e][n]);  // 0.5 undoes the 2*dec(c) encoding
    const float uv = args.wu[e] ? gu[64 + threadIdx.x] * (0.5f * args.su[e][n]) : 0.f;
    h[(size_t)a * I + n] = moe_act(act, gv, uv);
  }
}

// grid (ceil(H / 64), 2, A), 8 waves: rows n0 .. n0 + 63 of W_down[e] over
// K part part (columns [part ks, part ks + ks)), waves 0-3 its first half and
// 4-7 its second (added through LDS), h as bf16 hi and lo planes; part 0 ->
// dout, part 1 -> dout_lo (the combine adds them).
// cnt != nullptr: the combine runs here too. Each workgroup stores its 64
// columns device-coherent and counts itself in for (column block, token);
// the last of the token's 2 top_k workgroups adds the routes as the combine
// kernel does (acc from 0, k = 0, 1, ..., d = part 0 + part 1, d * w rounded
// before the add, CpuMoELayer's skip of |w| < 1e-8) and writes y, then
// resets the counter for the next launch.
__global__ __launch_bounds__(512) void moe_dec_down_kernel(const DownArgs args, const float *__restrict__ h, int H,
                                                           int I, int ks, const uint32_t *__restrict__ idx,
                                                           float *__restrict__ dout, float *__restrict__ dout_lo,
                                                           unsigned *__restrict__ cnt, const float *__restrict__ wts,
                                                           int top_k, int skip_small, void *__restrict__ y,
                                                           int y_bf16) {
  extern __shared__ __align__(16) uint16_t dsm[];
  const int kp = dec_pad2(ks, MOE_DEC_DN_CH);
  uint16_t *hh = dsm, *hl = dsm + kp;
  f32x4 *red = reinterpret_cast<f32x4 *>(dsm + 2 * kp);  // [4 waves][64 lanes]
  const int a = blockIdx.z, part = blockIdx.y, e = (int)idx[a];
  const int k0 = part * ks, kl = max(0, min(ks, I - k0));
  const int kc = dec_half(kl);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kh = wave >> 2, wl = wave & 3;
  const int ko = kh ? kc : 0, kw = kh ? kl - kc : kc;
  const int n0 = blockIdx.x * MOE_DEC_ROWS;
  const uint32_t *wrow[1] = {args.wd[e] + (size_t)min(n0 + wl * 16 + (lane & 15), H - 1) * (I >> 4) +
                             ((k0 + ko) >> 4)};
  f32x4 acc[1] = {(f32x4){0.f, 0.f, 0.f, 0.f}};
  auto stage = [&]() {
    dec_stage_row<float>(h + (size_t)a * I + k0, kl, dec_pad2(kl, MOE_DEC_DN_CH), hh, hl);
    __syncthreads();
  };
  dec_gemv<true, 1, MOE_DEC_DN_CH>(wrow, kw, hh + ko, hl + ko, acc, stage);
  if (kh) red[wl * 64 + lane] = acc[0];
  __syncthreads();
  constexpr int SC1 = 16;  // cache policy: performed at the point of coherence of all XCDs
  constexpr uint32_t OOB = 0x80000000u;
  if (!kh && (lane & 15) == 0) {
    const f32x4 v = acc[0] + red[wl * 64 + lane];
    const __amdgpu_buffer_rsrc_t orr = buffer_rsrc((part == 0 ? dout : dout_lo) + (size_t)a * H, (uint32_t)H * 4u);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = n0 + wl * 16 + 4 * (lane >> 4) + j;
      const float o = n < H ? v[j] * (0.5f * args.sd[e][n]) : 0.f;
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(o), orr, n < H ? (uint32_t)n * 4u : OOB, 0, SC1);
    }
  }
  if (!cnt) return;  // a separate launch combines
  __shared__ int last;
  const int t = a / top_k;
  wait_vmcnt<0>();
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned *c = cnt + blockIdx.x * MOE_DEC_MAXA + t;
    const unsigned old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old == 2u * (unsigned)top_k - 1u;
    if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last || threadIdx.x >= MOE_DEC_ROWS) return;
  const int n = n0 + (int)threadIdx.x;
  if (n >= H) return;
  const __amdgpu_buffer_rsrc_t d0r = buffer_rsrc(dout, (uint32_t)(gridDim.z * H) * 4u);
  const __amdgpu_buffer_rsrc_t d1r = buffer_rsrc(dout_lo, (uint32_t)(gridDim.z * H) * 4u);
  float d0[MOE_DEC_MAXA], d1[MOE_DEC_MAXA];
#pragma unroll
  for (int k = 0; k < MOE_DEC_MAXA; k++) {
    const uint32_t off = k < top_k ? ((uint32_t)(t * top_k + k) * (uint32_t)H + (uint32_t)n) * 4u : OOB;
    d0[k] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(d0r, off, 0, SC1));
    d1[k] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(d1r, off, 0, SC1));
  }
  float accy = 0.0f;
#pragma unroll
  for (int k = 0; k < MOE_DEC_MAXA; k++) {
#pragma clang fp contract(off)
    if (k >= top_k) break;
    const float w = wts[t * top_k + k];
    if (skip_small && fabsf(w) < 1e-8f) continue;  // src/model/cpu_moe.rs:172
    const float d = d0[k] + d1[k];
    const float prod = d * w;
    accy = accy + prod;
  }
  if (y_bf16) reinterpret_cast<uint16_t *>(y)[(size_t)t * H + n] = (uint16_t)bf16_rne(accy);
  else reinterpret_cast<float *>(y)[(size_t)t * H + n] = accy;
}

// ---- 5. combine ---------------------------------------------------------------
// cpu_block_attn_res.rs:1179 `expert_outputs[t*hd+d] += w * down[d]`, k order.
// dout_lo != nullptr: the down rows arrive as two partials (the engine-2 K
// parts), d = dout + dout_lo.
template <typename YT>
__global__ __launch_bounds__(256) void moe_combine_kernel(
    const float *__restrict__ dout, const float *__restrict__ dout_lo, const float *__restrict__ wts,
    const int *__restrict__ inv, int H, int top_k, YT *__restrict__ y, int skip_small) {
  // The token's routes are read once; then per group of up to CK routes all
  // of their rows (and the second K part) are loaded before any is added, so
  // a thread waits one memory round trip per group rather than per route.
  // The additions keep the reference's order: acc from 0, k = 0, 1, ...
  constexpr int CK = 4, CJ = 2;  // routes per group, column quads per thread
  __shared__ float sw[64];
  __shared__ long so[64];
  const int t = blockIdx.x;
  if ((int)threadIdx.x < top_k) {
    sw[threadIdx.x] = wts[t * top_k + threadIdx.x];
    so[threadIdx.x] = (long)inv[t * top_k + threadIdx.x] * H;
  }
  __syncthreads();
  for (int j0 = threadIdx.x * 4; j0 < H; j0 += 1024 * CJ) {  // H % 16 == 0
    f32x4 acc[CJ];
#pragma unroll
    for (int c = 0; c < CJ; c++) acc[c] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < top_k; k0 += CK) {
      f32x4 d[CK][CJ];
#pragma unroll
      for (int q = 0; q < CK; q++)
#pragma unroll
        for (int c = 0; c < CJ; c++) {
          const int j = j0 + c * 1024;
          d[q][c] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
          if (k0 + q < top_k && j < H) {
            const long o = so[k0 + q] + j;
            d[q][c] = *reinterpret_cast<const f32x4 *>(dout + o);
            if (dout_lo) d[q][c] = d[q][c] + *reinterpret_cast<const f32x4 *>(dout_lo + o);
          }
        }
#pragma unroll
      for (int q = 0; q < CK; q++) {
#pragma clang fp contract(off)
        if (k0 + q >= top_k) break;
        const float w = sw[k0 + q];
        // CpuMoELayer skips experts whose weight is below 1e-8 in magnitude
        // (src/model/cpu_moe.rs:172)
        if (skip_small && fabsf(w) < 1e-8f) continue;
#pragma unroll
        for (int c = 0; c < CJ; c++) {
          const f32x4 prod = d[q][c] * w;
          acc[c] = acc[c] + prod;
        }
      }
    }
#pragma unroll
    for (int c = 0; c < CJ; c++)
      if (j0 + c * 1024 < H) YStore<YT>::store4(y + (long)t * H + j0 + c * 1024, acc[c], 4);
  }
}
#pragma clang fp contract(on)

hipError_t launch_moe(const void *x, int xt_bf16, const void *router,
                      int rt_bf16, const uint32_t *const *w_gate,
                      const float *const *s_gate, const uint32_t *const *w_up,
                      const float *const *s_up, const uint32_t *const *w_down,
                      const float *const *s_down, int T, int H, int I, int E,
                      int top_k, int act, void *y, int yt_bf16,
                      uint32_t *topk_idx, float *topk_w, const MoeWorkspace &ws,
                      int routing, const MoeLora &lora, hipStream_t stream) {
  const int A = T * top_k;
  // 1. router
  int EP = 1;
  while (EP < E) EP *= 2;
  const int tpb = RT_NT / EP;
  const dim3 rg((T + tpb - 1) / tpb);
  const int rch = router_chunk(tpb + E);
  const size_t rlds = (size_t)(2 * (tpb + E) * (rch + 4) + 4 * RT_NT) * 4;
  {
    static std::atomic<uint64_t> done[4];
    const void *fns[4] = {reinterpret_cast<const void *>(&moe_router_kernel<uint16_t, uint16_t>),
                          reinterpret_cast<const void *>(&moe_router_kernel<uint16_t, float>),
                          reinterpret_cast<const void *>(&moe_router_kernel<float, uint16_t>),
                          reinterpret_cast<const void *>(&moe_router_kernel<float, float>)};
    const int v = (xt_bf16 ? 0 : 2) + (rt_bf16 ? 0 : 1);
    const hipError_t e = opt_in_lds(fns[v], 160 * 1024, done[v]);
    if (e != hipSuccess) return e;
  }
  const size_t res_lds = router_res_lds(H, E, tpb);
  const size_t pair_lds = router_pair_lds(H, E, tpb);
  // the resident kernels bring the router rows by LDS DMA, in whole 16-byte
  // pieces
  const bool r16 = (reinterpret_cast<uintptr_t>(router) & 15) == 0;
  if (rt_bf16 && r16 && H % 16 == 0 && pair_lds <= 160 * 1024) {
    static std::atomic<uint64_t> done_p[2];
    const void *fn = xt_bf16 ? reinterpret_cast<const void *>(&moe_router_pair_kernel<uint16_t>)
                             : reinterpret_cast<const void *>(&moe_router_pair_kernel<float>);
    const hipError_t e = opt_in_lds(fn, 160 * 1024, done_p[xt_bf16 ? 0 : 1]);
    if (e != hipSuccess) return e;
    const int rsb = router_res_row_bytes(H);
    if (xt_bf16)
      hipLaunchKernelGGL((moe_router_pair_kernel<uint16_t>), rg, dim3(2 * RT_NT), pair_lds, stream,
                         (const uint16_t *)x, (const uint16_t *)router, T, H, E, EP, top_k, rsb, ws.idx, ws.wts,
                         topk_idx, topk_w, routing);
    else
      hipLaunchKernelGGL((moe_router_pair_kernel<float>), rg, dim3(2 * RT_NT), pair_lds, stream, (const float *)x,
                         (const uint16_t *)router, T, H, E, EP, top_k, rsb, ws.idx, ws.wts, topk_idx, topk_w,
                         routing);
  } else if (rt_bf16 && r16 && res_lds <= 160 * 1024) {
    static std::atomic<uint64_t> done_res[2];
    const void *fn = xt_bf16 ? reinterpret_cast<const void *>(&moe_router_res_kernel<uint16_t>)
                             : reinterpret_cast<const void *>(&moe_router_res_kernel<float>);
    const hipError_t e = opt_in_lds(fn, 160 * 1024, done_res[xt_bf16 ? 0 : 1]);
    if (e != hipSuccess) return e;
    const int rsb = router_res_row_bytes(H);
    if (xt_bf16)
      hipLaunchKernelGGL((moe_router_res_kernel<uint16_t>), rg, dim3(RT_NT), res_lds, stream, (const uint16_t *)x,
                         (const uint16_t *)router, T, H, E, EP, top_k, rsb, ws.idx, ws.wts, topk_idx, topk_w, routing);
    else
      hipLaunchKernelGGL((moe_router_res_kernel<float>), rg, dim3(RT_NT), res_lds, stream, (const float *)x,
                         (const uint16_t *)router, T, H, E, EP, top_k, rsb, ws.idx, ws.wts, topk_idx, topk_w, routing);
  } else if (xt_bf16 && rt_bf16)
    hipLaunchKernelGGL((moe_router_kernel<uint16_t, uint16_t>), rg, dim3(RT_NT), rlds, stream,
                       (const uint16_t *)x, (const uint16_t *)router, T, H, E, EP, top_k, rch, ws.idx, ws.wts, topk_idx, topk_w, routing);
  else if (xt_bf16)
    hipLaunchKernelGGL((moe_router_kernel<uint16_t, float>), rg, dim3(RT_NT), rlds, stream,
                       (const uint16_t *)x, (const float *)router, T, H, E, EP, top_k, rch, ws.idx, ws.wts, topk_idx, topk_w, routing);
  else if (rt_bf16)
    hipLaunchKernelGGL((moe_router_kernel<float, uint16_t>), rg, dim3(RT_NT), rlds, stream,
                       (const float *)x, (const uint16_t *)router, T, H, E, EP, top_k, rch, ws.idx, ws.wts, topk_idx, topk_w, routing);
  else
    hipLaunchKernelGGL((moe_router_kernel<float, float>), rg, dim3(RT_NT), rlds, stream,
                       (const float *)x, (const float *)router, T, H, E, EP, top_k, rch, ws.idx, ws.wts, topk_idx, topk_w, routing);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  // engine 2 (pipelined MFMA GEMMs): H and I multiples of 64, 16-byte
  // aligned weights, bf16 x or f32 x (8-byte aligned, split into bf16 hi | lo
  // rows for the gate/up GEMM); otherwise the register-staged engine 1
  bool engine2 = (xt_bf16 || (reinterpret_cast<uintptr_t>(x) & 7) == 0) && H % 64 == 0 && I % 64 == 0;
  for (int i = 0; i < E && engine2; i++)
    engine2 = ((reinterpret_cast<uintptr_t>(w_gate[i]) | reinterpret_cast<uintptr_t>(w_up[i]) |
                reinterpret_cast<uintptr_t>(w_down[i])) & 15) == 0;
  DownArgs da;
  for (int i = 0; i < MOE_MAXE; i++) {
    da.wd[i] = i < E ? w_down[i] : nullptr;
    da.sd[i] = i < E ? s_down[i] : nullptr;
  }
  GateUpArgs ga;
  for (int i = 0; i < MOE_MAXE; i++) {
    const bool v = i < E;
    ga.wg[i] = v ? w_gate[i] : nullptr;
    ga.wu[i] = v ? w_up[i] : nullptr;
    ga.sg[i] = v ? s_gate[i] : nullptr;
    ga.su[i] = v ? s_up[i] : nullptr;
  }
  if (engine2 && A <= MOE_DEC_MAXA && !lora.tbl && H <= 8192 && I <= 16384 &&  // LDS <= 40 KB
      (reinterpret_cast<uintptr_t>(x) & 15) == 0) {
    // decode: GEMVs per routed row (no grouping), down in two K parts
    const int ks = (I / 2 + 63) / 64 * 64;
    const size_t gl = (size_t)dec_pad2(H, MOE_DEC_GU_CH) * 4 + 2 * MOE_DEC_ROWS * 4 + 4 * 2 * 64 * 16;
    const size_t dl = (size_t)dec_pad2(ks, MOE_DEC_DN_CH) * 4 + 4 * 64 * 16;
    if (xt_bf16)
      hipLaunchKernelGGL((moe_dec_gateup_kernel<uint16_t>), dim3((I + MOE_DEC_ROWS - 1) / MOE_DEC_ROWS, A), dim3(512),
                         gl, stream, ga, (const uint16_t *)x, H, I, top_k, ws.idx, (float *)ws.h_hi, ws.inv, act);
    else
      hipLaunchKernelGGL((moe_dec_gateup_kernel<float>), dim3((I + MOE_DEC_ROWS - 1) / MOE_DEC_ROWS, A), dim3(512),
                         gl, stream, ga, (const float *)x, H, I, top_k, ws.idx, (float *)ws.h_hi, ws.inv, act);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    // with arrival counters the down launch also combines (one launch fewer)
    hipLaunchKernelGGL(moe_dec_down_kernel, dim3((H + MOE_DEC_ROWS - 1) / MOE_DEC_ROWS, 2, A), dim3(512), dl, stream,
                       da, (const float *)ws.h_hi, H, I, ks, ws.idx, ws.dout, ws.dout_lo, ws.cnt, ws.wts, top_k,
                       routing, y, yt_bf16);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    if (ws.cnt) return hipSuccess;
    if (yt_bf16)
      hipLaunchKernelGGL((moe_combine_kernel<uint16_t>), dim3(T), dim3(256), 0, stream, ws.dout, ws.dout_lo, ws.wts,
                         ws.inv, H, top_k, (uint16_t *)y, routing);
    else
      hipLaunchKernelGGL((moe_combine_kernel<float>), dim3(T), dim3(256), 0, stream, ws.dout, ws.dout_lo, ws.wts,
                         ws.inv, H, top_k, (float *)y, routing);
    return hipGetLastError();
  }
  // 2. group
  const int bm_max = engine2 ? MOE3_BM : MOE_BM;
  hipLaunchKernelGGL(moe_group_kernel, dim3(1), dim3(1024), 0, stream, ws.idx, A, top_k, E, bm_max,
                     engine2 ? MOE3_FMIN : 1, ws.counts, ws.offsets, ws.perm_token, ws.inv, ws.tiles, ws.ntiles,
                     ws.row_expert);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  // LoRA A x of the gate and up adapters, per expert-sorted row
  if (lora.tbl) {
    if (xt_bf16)
      hipLaunchKernelGGL((moe_lora_a_kernel<uint16_t>), dim3(A), dim3(256), 0, stream, lora.tbl, lora.rank,
                         (const uint16_t *)x, ws.perm_token, ws.row_expert, nullptr, nullptr, 0L, H, 0, 2,
                         ws.lora_ax, 2 * MOE_LORA_MAXR);
    else
      hipLaunchKernelGGL((moe_lora_a_kernel<float>), dim3(A), dim3(256), 0, stream, lora.tbl, lora.rank,
                         (const float *)x, ws.perm_token, ws.row_expert, nullptr, nullptr, 0L, H, 0, 2, ws.lora_ax,
                         2 * MOE_LORA_MAXR);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  // LoRA A h of the down adapter (h as bf16 hi + lo, row stride hs)
  auto lora_down_a = [&](const uint16_t *hh, const uint16_t *hl, long hs) -> hipError_t {
    if (!lora.tbl) return hipSuccess;
    hipLaunchKernelGGL((moe_lora_a_kernel<uint16_t>), dim3(A), dim3(256), 0, stream, lora.tbl, lora.rank,
                       (const uint16_t *)nullptr, ws.perm_token, ws.row_expert, hh, hl, hs, I, 2, 1, ws.lora_ah,
                       MOE_LORA_MAXR);
    return hipGetLastError();
  };
  // 3. gate/up
  const int max_tiles = (A + bm_max - 1) / bm_max + E;
  bool two_parts = false;  // engine-2 down GEMM in two K parts (dout, dout_lo)
  if (engine2) {
    const int gu_lds = MoeGateUpCore::LDS_DWORDS * 4, dn_lds = MoeDownCore::LDS_DWORDS * 4;
    static std::atomic<uint64_t> done_gu, done_dn;
    if ((err = opt_in_lds(reinterpret_cast<const void *>(&moe_gateup3_kernel), gu_lds, done_gu)) != hipSuccess)
      return err;
    if ((err = opt_in_lds(reinterpret_cast<const void *>(&moe_down3_kernel), dn_lds, done_dn)) != hipSuccess)
      return err;
    const uint16_t *xg = reinterpret_cast<const uint16_t *>(x);
    if (!xt_bf16) {
      if ((err = launch_to_planes(reinterpret_cast<const float *>(x), ws.x2, T, H, stream)) != hipSuccess) return err;
      xg = ws.x2;
    }
    const dim3 g1((I + MOE_GU_BN / 2 - 1) / (MOE_GU_BN / 2), max_tiles);
    hipLaunchKernelGGL(moe_gateup3_kernel, g1, dim3(256), gu_lds, stream, ga, xg, xt_bf16 ? H : 2 * H, T, H, I,
                       ws.tiles, ws.ntiles, ws.offsets, ws.perm_token, ws.h_hi, act, lora, ws.lora_ax);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    if ((err = lora_down_a(ws.h_hi, ws.h_hi + I, 2L * I)) != hipSuccess) return err;
    // two K parts when each is a whole number of 64-column steps: twice the
    // workgroups (two per CU at the 512-token, 16-expert layer)
    const int ks = I % 128 == 0 ? I / 2 : I, kp = I / ks;
    const int ntn = (H + MOE3_DBN - 1) / MOE3_DBN;
    const int slots = (max_tiles + 7) / 8 * 8;
    hipLaunchKernelGGL(moe_down3_kernel, dim3(slots * ntn * kp), dim3(256), dn_lds, stream, da,
                       (const uint16_t *)ws.h_hi, H, I, ks, ntn, kp, ws.tiles, ws.ntiles, ws.offsets, ws.dout,
                       ws.dout_lo, lora, ws.lora_ah);
    two_parts = kp == 2;
    if ((err = hipGetLastError()) != hipSuccess) return err;
  } else {
    dim3 g1((I + MOE_BN - 1) / MOE_BN, max_tiles);
    if (xt_bf16)
      hipLaunchKernelGGL((moe_gateup_kernel<XS_BF16>), g1, dim3(256), 0, stream, ga, x, H, I,
                         ws.tiles, ws.ntiles, ws.counts, ws.offsets, ws.perm_token, ws.h_hi, ws.h_lo, act,
                         lora.tbl, lora.rank, lora.scaling, (const float *)ws.lora_ax);
    else
      hipLaunchKernelGGL((moe_gateup_kernel<XS_F32>), g1, dim3(256), 0, stream, ga, x, H, I,
                         ws.tiles, ws.ntiles, ws.counts, ws.offsets, ws.perm_token, ws.h_hi, ws.h_lo, act,
                         lora.tbl, lora.rank, lora.scaling, (const float *)ws.lora_ax);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    if ((err = lora_down_a(ws.h_hi, ws.h_lo, (long)I)) != hipSuccess) return err;
    // 4. down
    dim3 g2((H + MOE_BN - 1) / MOE_BN, max_tiles);
    hipLaunchKernelGGL(moe_down_kernel, g2, dim3(256), 0, stream, da, ws.h_hi, ws.h_lo, H, I,
                       ws.tiles, ws.ntiles, ws.counts, ws.offsets, ws.dout, lora.tbl, lora.rank, lora.scaling,
                       (const float *)ws.lora_ah);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  // 5. combine
  if (yt_bf16)
    hipLaunchKernelGGL((moe_combine_kernel<uint16_t>), dim3(T), dim3(256), 0, stream, ws.dout,
                       two_parts ? ws.dout_lo : nullptr, ws.wts, ws.inv, H, top_k, (uint16_t *)y, routing);
  else
    hipLaunchKernelGGL((moe_combine_kernel<float>), dim3(T), dim3(256), 0, stream, ws.dout,
                       two_parts ? ws.dout_lo : nullptr, ws.wts, ws.inv, H, top_k, (float *)y, routing);
  return hipGetLastError();
}

}  // namespace frx
