// frx_moe.hip — MoE ternary expert layer on gfx950.
//
// Semantics: the model's GPU-path MoE glue, src/model/cpu_block_attn_res.rs
// :1148-1184 (= TernaryMoELayer::forward, src/model/ternary_moe.rs:145-223,
// with per-row scales). The reference runs it as host loops over tokens and
// experts with 3 GEMV dispatches per (token, expert); here it is five
// launches:
//   1. router_topk   one wave per token: logits (sequential f32 sums, no
//                    FMA, bit-identical to the reference), softmax, stable
//                    descending sort of the probabilities, top-k, weights.
//   2. group         one workgroup: per-expert histogram, exclusive scan and
//                    a stable scatter of the (token, k) assignments into
//                    expert-sorted rows, plus the M-tile schedule.
//   3. gateup        grouped GEMM over the tile schedule: gathered token rows
//                    x W_gate[e] and x W_up[e] in one workgroup, SwiGLU (or
//                    GeLU-tanh) epilogue, h stored as bf16 hi/lo planes.
//   4. down          grouped GEMM h x W_down[e] (hi and lo planes: two MFMAs
//                    per operand), fp32 rows.
//   5. combine       out[t] = sum_k w[t,k] * d[row(t,k)] in k order from 0.0,
//                    exactly the reference's accumulation (deterministic).
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
  b += align256(A * 4) * 2;             // perm_token, inv
  b += align256(max_tiles * 8);         // tiles
  b += align256(4);                     // ntiles
  b += align256(A * I * 2) * 2;         // h planes
  b += align256(A * H * 4);             // dout
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
  ws->tiles = reinterpret_cast<int *>(take(max_tiles * 8));
  ws->ntiles = reinterpret_cast<int *>(take(4));
  ws->h_hi = reinterpret_cast<uint16_t *>(take(A * I * 2));
  ws->h_lo = reinterpret_cast<uint16_t *>(take(A * I * 2));
  ws->dout = reinterpret_cast<float *>(take(A * H * 4));
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
// expert e is a left-to-right f32 sum of x[j]*r[e][j] with no contraction,
// so it is bit-identical to the reference for the same inputs; exp is
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

// Chunk width so that one pass of 256 threads x 4 units of 8 columns covers
// every staged row (tokens of the block + experts): a multiple of 8.
static inline int router_chunk(int rows) {
  int ch = (1024 / rows) * 8;
  return ch > RT_CHMAX ? RT_CHMAX : ch;
}

// 256 threads = (256/EP) tokens x EP expert lanes (EP = E rounded up to a
// power of two). Chunks of RT_CH columns of the block's token rows and of
// all router rows are staged in LDS as f32 (double-buffered: the next
// chunk's global loads are in flight while the current one is summed); each
// (token, expert) lane then runs the reference's sequential dot product.
template <typename XT, typename RT>
__global__ __launch_bounds__(256) void moe_router_kernel(
    const XT *__restrict__ x, const RT *__restrict__ router, int T, int H,
    int E, int EP, int top_k, int CH, uint32_t *__restrict__ idx_out,
    float *__restrict__ w_out, uint32_t *__restrict__ user_idx,
    float *__restrict__ user_w) {
  const int RS = CH + 4;  // padded row stride (floats)
  extern __shared__ __align__(16) float rsm[];
  const int tid = threadIdx.x, e = tid % EP, tl = tid / EP;
  const int TPB = 256 / EP;
  const int t = blockIdx.x * TPB + tl;
  const int rows = TPB + E;  // staged rows: tokens then experts
  float *buf[2] = {rsm, rsm + rows * RS};
  float *logit = rsm + 2 * rows * RS;
  const int nch = (H + CH - 1) / CH;
  // each thread stages 8 consecutive columns of one row per pass
  const int units = rows * (CH / 8);
  float stage[4][8];
  auto gload = [&](int c) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int u = tid + i * 256;
      const int rr = u / (CH / 8), col = c * CH + (u % (CH / 8)) * 8;
      const bool ok = u < units && col < H;
      if (ok && rr < TPB) {
        const int tt = blockIdx.x * TPB + rr;
        if (tt < T) ld8(x + (long)tt * H + col, stage[i]);
        else for (int k = 0; k < 8; k++) stage[i][k] = 0.f;
      } else if (ok) {
        ld8(router + (long)(rr - TPB) * H + col, stage[i]);
      } else {
        for (int k = 0; k < 8; k++) stage[i][k] = 0.f;
      }
    }
  };
  auto sstore = [&](float *b) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int u = tid + i * 256;
      if (u < units) {
        const int rr = u / (CH / 8), cc = (u % (CH / 8)) * 8;
        float4 *d = reinterpret_cast<float4 *>(b + rr * RS + cc);
        d[0] = make_float4(stage[i][0], stage[i][1], stage[i][2], stage[i][3]);
        d[1] = make_float4(stage[i][4], stage[i][5], stage[i][6], stage[i][7]);
      }
    }
  };
  float sum = 0.0f;
  gload(0);
  sstore(buf[0]);
  __syncthreads();
  for (int c = 0; c < nch; c++) {
    if (c + 1 < nch) gload(c + 1);
    if (e < E && t < T) {
#pragma clang fp contract(off)
      const float *xr = buf[c & 1] + tl * RS;
      const float *rr = buf[c & 1] + (TPB + e) * RS;
      const int ncol = min(CH, H - c * CH);  // multiple of 8
      int j = 0;
      // 32 columns of LDS reads issued ahead of each run of dependent adds
      for (; j + 32 <= ncol; j += 32) {
        f32x4 xv[8], rv[8];
#pragma unroll
        for (int q = 0; q < 8; q++) {
          xv[q] = *reinterpret_cast<const f32x4 *>(xr + j + 4 * q);
          rv[q] = *reinterpret_cast<const f32x4 *>(rr + j + 4 * q);
        }
#pragma unroll
        for (int q = 0; q < 8; q++) {
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float pr = xv[q][i] * rv[q][i];
            sum = sum + pr;
          }
        }
      }
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
          for (int i = 0; i < 4; i++) {
            const float pr = xv[q][i] * rv[q][i];
            sum = sum + pr;
          }
        }
      }
    }
    if (c + 1 < nch) sstore(buf[(c + 1) & 1]);
    __syncthreads();
  }
  // Softmax and stable top-k in LDS, one EP-lane group per token. A lane's
  // rank among the probabilities (greater, or equal with a lower index)
  // reproduces the stable descending sort of the reference; the two
  // reductions (sum of exps in expert order, sum of the top-k in sorted
  // order) stay sequential on one lane, as in the reference.
  float *pbuf = logit + 256;             // [256] probabilities
  float *tsum = pbuf + 256;              // [256/EP] per-token sums
  int *order = reinterpret_cast<int *>(tsum + 256);  // [256/EP][EP]
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
    int rank = 0;
    for (int j = 0; j < E; j++) {
      const float pj = pbuf[tl * EP + j];
      rank += (pj > pe) || (pj == pe && j < e);
    }
    if (rank < top_k) order[tl * EP + rank] = e;
  }
  __syncthreads();
  if (e == 0 && t < T) {
    float ts = 0.0f;
    for (int i = 0; i < top_k; i++) ts = __fadd_rn(ts, pbuf[tl * EP + order[tl * EP + i]]);
    tsum[tl] = ts;
  }
  __syncthreads();
  if (e < top_k && t < T) {
    const int ei = order[tl * EP + e];
    const float wi = __fdiv_rn(pbuf[tl * EP + ei], tsum[tl]);
    idx_out[t * top_k + e] = (uint32_t)ei;
    w_out[t * top_k + e] = wi;
    if (user_idx) user_idx[t * top_k + e] = (uint32_t)ei;
    if (user_w) user_w[t * top_k + e] = wi;
  }
}

// ---- 2. histogram / scan / stable scatter / tile schedule -----------------
__global__ __launch_bounds__(1024) void moe_group_kernel(
    const uint32_t *__restrict__ idx, int A, int top_k, int E, int bm,
    int *__restrict__ counts, int *__restrict__ offsets,
    int *__restrict__ perm_token, int *__restrict__ inv,
    int *__restrict__ tiles, int *__restrict__ ntiles) {
  __shared__ int wave_cnt[16][MOE_MAXE];
  __shared__ int base[MOE_MAXE];
  __shared__ int offs[MOE_MAXE + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid < MOE_MAXE) base[tid] = 0;
  __syncthreads();
  // Pass 1: rank of each assignment within its expert, in (t, k) order.
  for (int c0 = 0; c0 < A; c0 += 1024) {
    const int a = c0 + tid;
    const int e = a < A ? (int)idx[a] : -1;
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
      inv[a] = before + rank;  // position within the expert (fixed below)
    }
    __syncthreads();
    if (tid < E) {
      int s = 0;
      for (int w = 0; w < 16; w++) s += wave_cnt[w][tid];
      base[tid] += s;
    }
    __syncthreads();
  }
  if (tid == 0) {
    int run = 0, nt = 0;
    for (int ee = 0; ee < E; ee++) {
      offs[ee] = run;
      counts[ee] = base[ee];
      offsets[ee] = run;
      for (int m0 = 0; m0 < base[ee]; m0 += bm) {
        tiles[2 * nt] = ee;
        tiles[2 * nt + 1] = m0;
        nt++;
      }
      run += base[ee];
    }
    offs[E] = run;
    offsets[E] = run;
    *ntiles = nt;
  }
  __syncthreads();
  // Pass 2: final rows.
  for (int a = tid; a < A; a += 1024) {
    const int e = (int)idx[a];
    const int pos = offs[e] + inv[a];
    inv[a] = pos;
    perm_token[pos] = a / top_k;
  }
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
    uint16_t *__restrict__ h_lo, int gelu) {
  using Core = GemmCore<MOE_BM, MOE_BN, 1, 4, XS, 2>;
  __shared__ __align__(16) uint32_t lds[Core::LDS_DWORDS];
  const int tile = blockIdx.y;
  if (tile >= *ntiles) return;
  const int e = tiles[2 * tile], mstart = tiles[2 * tile + 1];
  const int mcount = min(MOE_BM, counts[e] - mstart);
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
      const f32x4 g = acc[0][fn][fm] * sg, u = acc[1][fn][fm] * su;
      float hv[4];
      for (int j = 0; j < 4; j++) {
        const float a = gelu ? act_gelu_tanh(g[j]) : act_silu(g[j]);
        hv[j] = a * u[j];
      }
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
    float *__restrict__ dout) {
  using Core = GemmCore<MOE_BM, MOE_BN, 1, 4, XS_BF16X2, 1>;
  __shared__ __align__(16) uint32_t lds[Core::LDS_DWORDS];
  const int tile = blockIdx.y;
  if (tile >= *ntiles) return;
  const int e = tiles[2 * tile], mstart = tiles[2 * tile + 1];
  const int mcount = min(MOE_BM, counts[e] - mstart);
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
      if (m < mcount)
        YStore<float>::store4(dout + (long)(row0 + m) * H + n, acc[0][fn][fm] * sd, nok);
    }
  }
}

// ---- 5. combine ---------------------------------------------------------------
// cpu_block_attn_res.rs:1179 `expert_outputs[t*hd+d] += w * down[d]`, k order.
template <typename YT>
__global__ __launch_bounds__(256) void moe_combine_kernel(
    const float *__restrict__ dout, const float *__restrict__ wts,
    const int *__restrict__ inv, int H, int top_k, YT *__restrict__ y) {
  const int t = blockIdx.x;
  for (int j = threadIdx.x * 4; j < H; j += 1024) {  // H % 16 == 0
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k = 0; k < top_k; k++) {
#pragma clang fp contract(off)
      const float w = wts[t * top_k + k];
      const f32x4 d = *reinterpret_cast<const f32x4 *>(dout + (long)inv[t * top_k + k] * H + j);
      const f32x4 prod = d * w;
      acc = acc + prod;
    }
    YStore<YT>::store4(y + (long)t * H + j, acc, 4);
  }
}
#pragma clang fp contract(on)

hipError_t launch_moe(const void *x, int xt_bf16, const void *router,
                      int rt_bf16, const uint32_t *const *w_gate,
                      const float *const *s_gate, const uint32_t *const *w_up,
                      const float *const *s_up, const uint32_t *const *w_down,
                      const float *const *s_down, int T, int H, int I, int E,
                      int top_k, int gelu, void *y, int yt_bf16,
                      uint32_t *topk_idx, float *topk_w, const MoeWorkspace &ws,
                      hipStream_t stream) {
  const int A = T * top_k;
  // 1. router
  int EP = 1;
  while (EP < E) EP *= 2;
  const dim3 rg((T + 256 / EP - 1) / (256 / EP));
  const int rch = router_chunk(256 / EP + E);
  const size_t rlds = (size_t)(2 * (256 / EP + E) * (rch + 4) + 4 * 256) * 4;
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
  if (xt_bf16 && rt_bf16)
    hipLaunchKernelGGL((moe_router_kernel<uint16_t, uint16_t>), rg, dim3(256), rlds, stream,
                       (const uint16_t *)x, (const uint16_t *)router, T, H, E, EP, top_k, rch, ws.idx, ws.wts, topk_idx, topk_w);
  else if (xt_bf16)
    hipLaunchKernelGGL((moe_router_kernel<uint16_t, float>), rg, dim3(256), rlds, stream,
                       (const uint16_t *)x, (const float *)router, T, H, E, EP, top_k, rch, ws.idx, ws.wts, topk_idx, topk_w);
  else if (rt_bf16)
    hipLaunchKernelGGL((moe_router_kernel<float, uint16_t>), rg, dim3(256), rlds, stream,
                       (const float *)x, (const uint16_t *)router, T, H, E, EP, top_k, rch, ws.idx, ws.wts, topk_idx, topk_w);
  else
    hipLaunchKernelGGL((moe_router_kernel<float, float>), rg, dim3(256), rlds, stream,
                       (const float *)x, (const float *)router, T, H, E, EP, top_k, rch, ws.idx, ws.wts, topk_idx, topk_w);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  // 2. group
  hipLaunchKernelGGL(moe_group_kernel, dim3(1), dim3(1024), 0, stream, ws.idx, A, top_k, E,
                     MOE_BM, ws.counts, ws.offsets, ws.perm_token, ws.inv, ws.tiles, ws.ntiles);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  // 3. gate/up
  const int max_tiles = (A + MOE_BM - 1) / MOE_BM + E;
  GateUpArgs ga;
  for (int i = 0; i < MOE_MAXE; i++) {
    const bool v = i < E;
    ga.wg[i] = v ? w_gate[i] : nullptr;
    ga.wu[i] = v ? w_up[i] : nullptr;
    ga.sg[i] = v ? s_gate[i] : nullptr;
    ga.su[i] = v ? s_up[i] : nullptr;
  }
  dim3 g1((I + MOE_BN - 1) / MOE_BN, max_tiles);
  if (xt_bf16)
    hipLaunchKernelGGL((moe_gateup_kernel<XS_BF16>), g1, dim3(256), 0, stream, ga, x, H, I,
                       ws.tiles, ws.ntiles, ws.counts, ws.offsets, ws.perm_token, ws.h_hi, ws.h_lo, gelu);
  else
    hipLaunchKernelGGL((moe_gateup_kernel<XS_F32>), g1, dim3(256), 0, stream, ga, x, H, I,
                       ws.tiles, ws.ntiles, ws.counts, ws.offsets, ws.perm_token, ws.h_hi, ws.h_lo, gelu);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  // 4. down
  DownArgs da;
  for (int i = 0; i < MOE_MAXE; i++) {
    da.wd[i] = i < E ? w_down[i] : nullptr;
    da.sd[i] = i < E ? s_down[i] : nullptr;
  }
  dim3 g2((H + MOE_BN - 1) / MOE_BN, max_tiles);
  hipLaunchKernelGGL(moe_down_kernel, g2, dim3(256), 0, stream, da, ws.h_hi, ws.h_lo, H, I,
                     ws.tiles, ws.ntiles, ws.counts, ws.offsets, ws.dout);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  // 5. combine
  if (yt_bf16)
    hipLaunchKernelGGL((moe_combine_kernel<uint16_t>), dim3(T), dim3(256), 0, stream, ws.dout,
                       ws.wts, ws.inv, H, top_k, (uint16_t *)y);
  else
    hipLaunchKernelGGL((moe_combine_kernel<float>), dim3(T), dim3(256), 0, stream, ws.dout,
                       ws.wts, ws.inv, H, top_k, (float *)y);
  return hipGetLastError();
}

}  // namespace frx
