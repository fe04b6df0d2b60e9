// frx_gemv.hip — decode ternary GEMV for M <= 16 tokens on gfx950.
//
// Replaces the WGSL entry ternary_matmul_main
// (src/compute/kernels/ternary_matmul.rs:32-75) for decode shapes. Four
// kernels: gemv_rows_kernel (one bf16 token: whole rows per wave, 16 row
// segments per MFMA; gemv_rows_stream_kernel is its persistent form for
// tall matrices), gemv_rows4_kernel (2-4 bf16 tokens: 4 rows x 4
// segments), gemv_direct_kernel / gemv_tall_kernel (8-16 bf16 tokens,
// operands from L2) and gemv_kernel below (f32 activations, other token
// counts and unaligned shapes); launch_gemv picks one.
//
// gemv_kernel mapping. One workgroup (WAVES waves) owns a 16-row tile of W. The 16 rows
// are the M side of v_mfma_f32_16x16x32_bf16 and the (<= 16) tokens its N
// side. Lane (r = l%16, g = l/16) streams 16-byte chunks (64 codes) of row r
// with dwordx4 loads; the 4 lanes of a row read 64 contiguous bytes per
// instruction (a "quad" of chunks). The waves split K into contiguous,
// balanced ranges of quads, so each wave walks a contiguous stretch of every
// row of the tile. Each wave issues all of its loads (activations first,
// then up to UMAX weight quads per lane) before anything else, so the whole
// matrix is in flight at once; the kernel is one HBM round trip plus the
// stream.
//
// Activations. A wave reads only the x columns of its own quads, so it stages
// exactly those (B rows x 256 columns per quad) into its own columns of the
// LDS rows: one or two load instructions, then a wait on its own loads, and
// no workgroup barrier before the MFMAs. Rows are K-interleaved bf16 (dword i =
// x[i] | x[i+8] << 16, the order the weight unpack produces); f32 inputs are
// split into a hi/lo bf16 pair (two MFMAs per operand, |error| <= 2^-17 |x|).
// Lanes whose token is >= B read a 32-dword zero block of their wave instead.
// Codes become bf16 operands in registers (two VALU ops per weight pair,
// frx_device.hpp). The waves' partial tiles are summed in a fixed order
// through LDS, so results are deterministic.
#include "frx_device.hpp"
#include "frx_gemm2.hpp"
#include "frx_internal.hpp"

namespace frx {

constexpr int GEMV_XPRE = 1;  // rounds of activation items loaded before the weights

// Weight chunk c (words wb..wb+3, wb = first word of the slice + 4c) of this
// lane's row. VEC: one dwordx4 (rows 16-byte aligned, K % 64 == 0); else four
// dword loads. Chunks past the slice end are clamped in address and zeroed by
// the caller (mask), so every load stays inside the matrix.
template <bool VEC>
__device__ __forceinline__ u32x4 load_chunk(const uint32_t *wrow, int wb, int kw_end) {
  if constexpr (VEC) {
    return *reinterpret_cast<const u32x4 *>(wrow + min(wb, kw_end - 4));
  } else {
    u32x4 v;
    v.x = wrow[min(wb + 0, kw_end - 1)];
    v.y = wrow[min(wb + 1, kw_end - 1)];
    v.z = wrow[min(wb + 2, kw_end - 1)];
    v.w = wrow[min(wb + 3, kw_end - 1)];
    return v;
  }
}

// Epilogues. GEMV_LINEAR: Y = (W x) * scale. GEMV_SWIGLU / GEMV_GEGLU: two
// matrices (gate W, up W2) against the same x in one pass; Y = act(gate) *
// up, act = SiLU or GeLU-tanh (the decode FFN's first half; x is staged and
// read once for both).
enum { GEMV_LINEAR = 0, GEMV_SWIGLU = 1, GEMV_GEGLU = 2 };

// LDS rows for slices of ks columns: token row stride in dwords (ks padded
// to 256 columns, bf16 pairs, +4 so that 16 tokens' 16-byte reads spread
// over the banks). Layout: P planes x B rows, then one 32-dword zero block
// per wave.
static inline int gemv_row_stride(int ks) { return ((ks + 255) / 256) * 128 + 4; }
static inline size_t gemv_lds_bytes(int ks, int waves, int P, int B) {
  return ((size_t)P * B * gemv_row_stride(ks) + (size_t)waves * 32) * 4;
}

// UMAX: weight quads per lane per load batch (registers: 4 per quad and
// matrix).
// Occupancy target: the 8-wave bf16 tiles of the widest decode launch (688
// workgroups of N = 11008) need 6 waves per SIMD to be resident at once;
// the other variants keep their registers (no spills).
template <typename XT, typename YT, int WAVES, int UMAX, bool VEC, int EPI>
__global__ __launch_bounds__(WAVES * 64)
__attribute__((amdgpu_waves_per_eu(WAVES == 8 && sizeof(XT) == 2 && EPI == 0 ? 6 : 1))) void gemv_kernel(
    const uint32_t *__restrict__ W, const float *__restrict__ scale,
    const uint32_t *__restrict__ W2, const float *__restrict__ scale2,
    const XT *__restrict__ X, YT *__restrict__ Y, int B, int K, int N, int KS,
    int rs, const float *__restrict__ bias) {
  constexpr int P = XBlock<XT>::P;
  constexpr int NW = EPI == GEMV_LINEAR ? 1 : 2;  // weight matrices
  extern __shared__ __align__(16) uint32_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int wpr = K >> 4;
  const int row = min((int)blockIdx.x * 16 + r, N - 1);  // clamped; stores are masked
  const uint32_t *wrow[NW];
  wrow[0] = W + (size_t)row * wpr;
  if constexpr (NW == 2) wrow[1] = W2 + (size_t)row * wpr;
  uint32_t *zblk = lds + P * B * rs + wave * 32;  // this wave's zero block
  const int t = r;  // token whose activations this lane feeds (MFMA column)
  const bool live = t < B;
  if (lane < 8) reinterpret_cast<u32x4 *>(zblk)[lane] = (u32x4){0u, 0u, 0u, 0u};
  f32x4 acc[NW];
#pragma unroll
  for (int m = 0; m < NW; m++) acc[m] = (f32x4){0.f, 0.f, 0.f, 0.f};
  // Row scales are needed only by the epilogue; fetch them now so that load
  // is not a memory round trip after the reduction.
  const int n_out = blockIdx.x * 16 + 4 * g;
  f32x4 sc[NW];
#pragma unroll
  for (int m = 0; m < NW; m++) {
    const float *sp = m == 0 ? scale : scale2;
    sc[m] = (f32x4){0.f, 0.f, 0.f, 0.f};
    if (wave == 0 && live && n_out < N) {
      const int nok = min(4, N - n_out);
      sc[m].x = sp[n_out];
      sc[m].y = nok > 1 ? sp[n_out + 1] : 0.f;
      sc[m].z = nok > 2 ? sp[n_out + 2] : 0.f;
      sc[m].w = nok > 3 ? sp[n_out + 3] : 0.f;
    }
  }

  for (int s0 = 0; s0 < K; s0 += KS) {
    const int ks = min(KS, K - s0);
    const int nch = (ks + 63) >> 6;     // 64-column chunks in the slice
    const int nq = (nch + 3) >> 2;      // quads: one chunk per lane group g
    const int qa = (wave * nq) / WAVES, qb = ((wave + 1) * nq) / WAVES;  // this wave's quads
    const int kw0 = s0 >> 4;
    const int kw_end = (s0 + ks) >> 4;  // one past the slice's last word
    const int kblk = ks >> 4;           // 16-column blocks of the slice
    const int nb = 16 * (qb - qa);      // blocks of this wave (per token)
    const int cb0 = 16 * qa;            // first block of this wave
    uint32_t *reg = lds + cb0 * 8;      // this wave's columns of row 0
    // (token, block) pairs of the wave: item i -> token i / nb, block i % nb;
    // nb = 16 * (quads of the wave), the division by the quad count is a
    // multiply-shift (exact here: (i/16) * (quads - 1) < 2^16)
    const int nqw = max(qb - qa, 1);
    const uint32_t mq = (65536u + nqw - 1) / nqw;
    auto item_tok = [&](int i) { return (int)(((uint32_t)(i >> 4) * mq) >> 16); };
    const int nitem = B * nb;

    // 1. the first GEMV_XPRE rounds of the wave's activation items (L2-hot,
    //    issued before the weights so that waiting for them does not wait for
    //    the weights)
    uint32_t xh[GEMV_XPRE][8], xl[GEMV_XPRE][8];
#pragma unroll
    for (int i = 0; i < GEMV_XPRE; i++) {
      const int it = lane + 64 * i, tt = item_tok(it), j = it - tt * nb;
      const bool ok = it < nitem && cb0 + j < kblk;
      XBlock<XT>::load(X + (size_t)(ok ? tt : 0) * K + s0 + (ok ? cb0 + j : 0) * 16, ok, xh[i], xl[i]);
    }
    // 2. first batch of weight loads
    u32x4 wv[NW][UMAX];
#pragma unroll
    for (int u = 0; u < UMAX; u++) {
      const int q = qa + u;
#pragma unroll
      for (int m = 0; m < NW; m++)
        if (q < qb) wv[m][u] = load_chunk<VEC>(wrow[m], kw0 + (q * 4 + g) * 4, kw_end);
    }
    // 3. stage into the wave's columns (zero past the slice end). Quad
    //    ownership differs between slices, so a later slice first waits until
    //    every wave is done reading the previous one (no barrier when K fits
    //    one slice, the decode shapes).
    if (s0 > 0) __syncthreads();
    auto put = [&](int tt, int j, const uint32_t *hi, const uint32_t *lo) {
      u32x4 *d = reinterpret_cast<u32x4 *>(reg + tt * rs + j * 8);
      d[0] = (u32x4){hi[0], hi[1], hi[2], hi[3]};
      d[1] = (u32x4){hi[4], hi[5], hi[6], hi[7]};
      if constexpr (P == 2) {
        u32x4 *e = reinterpret_cast<u32x4 *>(reg + (B + tt) * rs + j * 8);
        e[0] = (u32x4){lo[0], lo[1], lo[2], lo[3]};
        e[1] = (u32x4){lo[4], lo[5], lo[6], lo[7]};
      }
    };
#pragma unroll
    for (int i = 0; i < GEMV_XPRE; i++) {
      const int it = lane + 64 * i, tt = item_tok(it);
      if (it < nitem) put(tt, it - tt * nb, xh[i], xl[i]);
    }
    // the remaining items, one round of 64 at a time
    constexpr int XR = 1;
    for (int i0 = 64 * GEMV_XPRE; i0 < nitem; i0 += 64 * XR) {
      uint32_t hi[XR][8], lo[XR][8];
#pragma unroll
      for (int i = 0; i < XR; i++) {
        const int it = i0 + lane + 64 * i, tt = item_tok(it), j = it - tt * nb;
        const bool ok = it < nitem && cb0 + j < kblk;
        XBlock<XT>::load(X + (size_t)(ok ? tt : 0) * K + s0 + (ok ? cb0 + j : 0) * 16, ok, hi[i], lo[i]);
      }
#pragma unroll
      for (int i = 0; i < XR; i++) {
        const int it = i0 + lane + 64 * i, tt = item_tok(it);
        if (it < nitem) put(tt, it - tt * nb, hi[i], lo[i]);
      }
    }
    // 4. unpack + MFMA, batch by batch
    for (int q0 = qa; q0 < qb; q0 += UMAX) {
      if (q0 != qa) {
#pragma unroll
        for (int u = 0; u < UMAX; u++) {
          const int q = q0 + u;
#pragma unroll
          for (int m = 0; m < NW; m++)
            if (q < qb) wv[m][u] = load_chunk<VEC>(wrow[m], kw0 + (q * 4 + g) * 4, kw_end);
        }
      }
#pragma unroll
      for (int u = 0; u < UMAX; u++) {
        const int q = q0 + u;
        if (q >= qb) break;  // wave-uniform
        const int lc = (q - qa) * 4 + g;  // chunk within the wave's columns
        const int wb = kw0 + (q * 4 + g) * 4;
        const uint32_t *bp = live ? reg + t * rs + lc * 32 : zblk;
        const uint32_t *bq = live ? reg + (B + t) * rs + lc * 32 : zblk;
        // VEC: a chunk is either entirely inside the slice or entirely past
        // its end, so one mask per chunk; otherwise one per word.
        const uint32_t mchunk = wb < kw_end ? 0xC000C000u : 0u;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          // past the slice end: zero operand (the x rows there are zero too)
          const uint32_t mask = VEC ? mchunk : ((wb + q < kw_end) ? 0xC000C000u : 0u);
          const u32x4 b0 = *reinterpret_cast<const u32x4 *>(bp + (live ? q * 8 : 0));
          const u32x4 b1 = *reinterpret_cast<const u32x4 *>(bp + (live ? q * 8 + 4 : 4));
          u32x4 c0, c1;
          if constexpr (P == 2) {
            c0 = *reinterpret_cast<const u32x4 *>(bq + (live ? q * 8 : 0));
            c1 = *reinterpret_cast<const u32x4 *>(bq + (live ? q * 8 + 4 : 4));
          }
#pragma unroll
          for (int m = 0; m < NW; m++) {
            const uint32_t wq = q == 0 ? wv[m][u].x : q == 1 ? wv[m][u].y : q == 2 ? wv[m][u].z : wv[m][u].w;
            const u32x4 a0 = unpack_half_m<0>(wq, mask), a1 = unpack_half_m<1>(wq, mask);
            acc[m] = mfma16(a0, b0, acc[m]);
            acc[m] = mfma16(a1, b1, acc[m]);
            if constexpr (P == 2) {
              acc[m] = mfma16(a0, c0, acc[m]);
              acc[m] = mfma16(a1, c1, acc[m]);
            }
          }
        }
      }
    }
  }
  __syncthreads();  // every wave is done with its columns before the reuse

  // Fixed-order reduction of the waves' partial tiles.
  f32x4 *red = reinterpret_cast<f32x4 *>(lds);
#pragma unroll
  for (int m = 0; m < NW; m++) red[(m * WAVES + wave) * 64 + lane] = acc[m];
  __syncthreads();
  if (wave == 0) {
    f32x4 s[NW];
#pragma unroll
    for (int m = 0; m < NW; m++) {
      s[m] = red[m * WAVES * 64 + lane];
#pragma unroll
      for (int w = 1; w < WAVES; w++) s[m] += red[(m * WAVES + w) * 64 + lane];
      s[m] *= sc[m] * 0.5f;  // 0.5 undoes the 2*dec(c) operand encoding
    }
    if (live && n_out < N) {  // rows 4g..4g+3 of token t
      f32x4 v = s[0];
      if constexpr (NW == 2) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const float a = EPI == GEMV_GEGLU ? act_gelu_tanh(s[0][j]) : act_silu(s[0][j]);
          v[j] = a * s[1][j];
        }
      }
      if constexpr (NW == 1)
        if (bias) v = add_bias4(v, bias, n_out, N);
      YStore<YT>::store4(Y + (size_t)t * N + n_out, v, min(4, N - n_out));
    }
  }
}

template <typename XT, typename YT, int WAVES, int UMAX, bool VEC, int EPI>
static hipError_t launch_gemv_w(const uint32_t *w, const float *scale, const uint32_t *w2,
                                const float *scale2, const void *x, void *y, int B, int K, int N,
                                hipStream_t stream, const float *bias) {
  constexpr int P = XBlock<XT>::P;
  constexpr int NW = EPI == GEMV_LINEAR ? 1 : 2;
  // K slices (multiples of 256 columns) small enough that the rows fit the
  // LDS budget; one slice at the decode shapes.
  const size_t budget = 64 * 1024;
  int KS = (K + 255) / 256 * 256;
  while (KS > 256 && gemv_lds_bytes(KS, WAVES, P, B) > budget) KS = ((KS / 2) + 255) / 256 * 256;
  const int rs = gemv_row_stride(KS);
  size_t lds = gemv_lds_bytes(KS, WAVES, P, B);
  if (lds < (size_t)NW * WAVES * 64 * 16) lds = (size_t)NW * WAVES * 64 * 16;
  dim3 grid((N + 15) / 16);
  hipLaunchKernelGGL((gemv_kernel<XT, YT, WAVES, UMAX, VEC, EPI>), grid, dim3(WAVES * 64), lds, stream,
                     w, scale, w2, scale2, reinterpret_cast<const XT *>(x), reinterpret_cast<YT *>(y),
                     B, K, N, KS, rs, bias);
  return hipGetLastError();
}

template <typename XT, typename YT, int EPI>
static hipError_t launch_gemv_t(const uint32_t *w, const float *scale, const uint32_t *w2,
                                const float *scale2, const void *x, void *y, int B, int K, int N,
                                hipStream_t stream, const float *bias = nullptr) {
  // Waves per tile grow with K so that each wave holds two to three quads
  // (short per-wave work after its loads land, many waves in flight, and few
  // enough registers that every workgroup of the decode shapes is resident
  // at once); UMAX covers a wave's quads in one load batch up to K = 12288.
  // Dword loads when rows are not 16-byte aligned.
  const bool vec = ((K >> 4) & 3) == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(w2) & 15) == 0;
#define FRX_GEMV_LAUNCH(WV, UM)                                                                  \
  return vec ? launch_gemv_w<XT, YT, WV, UM, true, EPI>(w, scale, w2, scale2, x, y, B, K, N, stream, bias) \
             : launch_gemv_w<XT, YT, WV, UM, false, EPI>(w, scale, w2, scale2, x, y, B, K, N, stream, bias)
  const int nq = (K + 255) / 256;
  if (nq <= 8) FRX_GEMV_LAUNCH(4, 2);
  if (nq <= 16) FRX_GEMV_LAUNCH(8, 2);
  if constexpr (EPI != GEMV_LINEAR) {
    // two matrices double the weight registers: 8 waves and load batches
    FRX_GEMV_LAUNCH(8, 3);
  } else {
    if (nq <= 48) FRX_GEMV_LAUNCH(16, 3);
    FRX_GEMV_LAUNCH(16, 4);
  }
#undef FRX_GEMV_LAUNCH
}

// ---- bf16 activations, 8 <= B <= 16: operands straight from L2 ------------
//
// Staging every token's activation row in LDS needs B*K*2 bytes per
// workgroup (352 KB at B = 16, K = 11008), more than a CU holds; the slices
// that would take serialise the launch. Here no lane stages anything: lane
// (r = l%16, g = l/16), which feeds token r as the MFMA's B operand, loads
// its own 32 bytes of x[r] for each weight word it decodes (two 16-byte
// buffer loads, the B operands of the word's two MFMAs), and the word's
// codes become natural-order bf16 pairs (unpack16_nat), so the loaded bytes
// are the operands as they are.
// Word order. The four lanes of a row load 16 consecutive words (64 bytes,
// 16 bytes each) and transpose them across the four 16-lane rows of the
// wave (two v_permlane32_swap + two v_permlane16_swap per quad), so that
// lane g decodes words g, g+4, g+8, g+12. The four lanes of a token then
// read adjacent 32-byte pieces of x for the same instruction: one 128-byte
// line per token, 16 lines per load instead of 64.
// Planes. With XPL = 2 the activations arrive as two bf16 planes (hi, lo)
// whose sum is an fp32 vector to 2^-17 (the decode FFN's gated product):
// every word then loads both planes and runs four MFMAs. YSPLIT writes the
// output the same way, as bf16 hi and lo planes of [B][N] each. The loads go through a buffer descriptor
// whose range is the B x K activation matrix: lanes of tokens >= B and words
// past K (or past the wave's quads) read zeros without touching memory, and
// a zero operand cancels whatever its weight word holds, so no lane needs a
// mask, a predicate or a clamp on the activation side. A wave issues the
// activations of its first D words, then every weight quad of its batch
// (whole matrix in flight), then keeps D words of activations in flight
// ahead of the word it multiplies. The waves' tiles are reduced in a fixed
// order through LDS, as in gemv_kernel.
template <typename YT, int WAVES, int UMAX, int D, bool VEC, int EPI, int XPL, bool YSPLIT>
__global__ __launch_bounds__(WAVES * 64) void gemv_direct_kernel(
    const uint32_t *__restrict__ W, const float *__restrict__ scale,
    const uint32_t *__restrict__ W2, const float *__restrict__ scale2,
    const uint16_t *__restrict__ X, const uint16_t *__restrict__ X2, YT *__restrict__ Y, int B,
    int K, int N, const float *__restrict__ bias) {
  static_assert(XPL == 1 || XPL == 2, "activation planes");
  static_assert(!YSPLIT || sizeof(YT) == 2, "split output is two bf16 planes");
  constexpr int NW = EPI == GEMV_LINEAR ? 1 : 2;
  constexpr int NWD = 4 * UMAX;  // weight words per lane in one batch
  static_assert(D >= 1 && D <= NWD, "prefetch distance");
  __shared__ f32x4 red[NW * WAVES * 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int wpr = K >> 4;
  const int row = min((int)blockIdx.x * 16 + r, N - 1);  // clamped; stores are masked
  const uint32_t *wrow[NW];
  wrow[0] = W + (size_t)row * wpr;
  if constexpr (NW == 2) wrow[1] = W2 + (size_t)row * wpr;
  const int nch = (K + 63) >> 6, nq = (nch + 3) >> 2;
  const int qa = (wave * nq) / WAVES, qb = ((wave + 1) * nq) / WAVES;  // this wave's quads
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(X, (uint32_t)B * (uint32_t)K * 2u);
  const __amdgpu_buffer_rsrc_t xr2 = buffer_rsrc(XPL == 2 ? X2 : X, (uint32_t)B * (uint32_t)K * 2u);
  const uint32_t xrow = (uint32_t)r * (uint32_t)K * 2u;  // past the range when r >= B
  constexpr uint32_t XOOB = 0x80000000u;                   // an offset past any range
  const bool live = r < B;
  const int n_out = blockIdx.x * 16 + 4 * g;
  f32x4 sc[NW];
#pragma unroll
  for (int m = 0; m < NW; m++) {
    const float *sp = m == 0 ? scale : scale2;
    sc[m] = (f32x4){0.f, 0.f, 0.f, 0.f};
    if (wave == 0 && live && n_out < N) {
      const int nok = min(4, N - n_out);
      sc[m].x = sp[n_out];
      sc[m].y = nok > 1 ? sp[n_out + 1] : 0.f;
      sc[m].z = nok > 2 ? sp[n_out + 2] : 0.f;
      sc[m].w = nok > 3 ? sp[n_out + 3] : 0.f;
    }
  }
  f32x4 acc[NW];
#pragma unroll
  for (int m = 0; m < NW; m++) acc[m] = (f32x4){0.f, 0.f, 0.f, 0.f};

  for (int q0 = qa; q0 < qb; q0 += UMAX) {
    const int nwd = 4 * min(UMAX, qb - q0);  // words of this batch (per lane)
    // word j of the batch: word 16(q0 + j/4) + 4(j%4) + g of the row
    auto xoff = [&](int j) -> uint32_t {
      const int col = 256 * (q0 + (j >> 2)) + 64 * (j & 3) + 16 * g;
      return (j < nwd && col < K) ? xrow + 2u * (uint32_t)col : XOOB;
    };
    u32x4 xv[NWD][2 * XPL];  // [hi0, hi1, lo0, lo1]
    auto xload = [&](int j) {
      const uint32_t o = xoff(j);
      xv[j][0] = __builtin_amdgcn_raw_buffer_load_b128(xr, o, 0, 0);
      xv[j][1] = __builtin_amdgcn_raw_buffer_load_b128(xr, o + 16u, 0, 0);
      if constexpr (XPL == 2) {
        xv[j][2] = __builtin_amdgcn_raw_buffer_load_b128(xr2, o, 0, 0);
        xv[j][3] = __builtin_amdgcn_raw_buffer_load_b128(xr2, o + 16u, 0, 0);
      }
    };
#pragma unroll
    for (int j = 0; j < D; j++) xload(j);
    // every weight quad of the batch (addresses clamped to the row; words
    // past the wave's quads or past K meet zero activations)
    u32x4 wv[NW][UMAX];
#pragma unroll
    for (int u = 0; u < UMAX; u++) {
      const int wb = 4 * (4 * (q0 + u) + g);
#pragma unroll
      for (int m = 0; m < NW; m++) wv[m][u] = load_chunk<VEC>(wrow[m], wb, wpr);
    }
#pragma unroll
    for (int j = 0; j < NWD; j++) {
      if (j + D < NWD) xload(j + D);
      if (j >= nwd) continue;  // wave-uniform: past the batch's words
      const int u = j >> 2, wi = j & 3;
      if (wi == 0) {
        // 4x4 transpose of quad u across the lane rows g (every lane takes
        // part): lane g held words 4g..4g+3 of the quad and now holds words
        // g, g+4, g+8, g+12. The off-diagonal 2x2 blocks swap between lane
        // halves, then the off-diagonal elements of each block between
        // adjacent rows.
#pragma unroll
        for (int m = 0; m < NW; m++) {
          u32x4 &v = wv[m][u];
          const auto p02 = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
          const auto p13 = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
          const auto p01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
          const auto p23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
          v = (u32x4){p01[0], p01[1], p23[0], p23[1]};
        }
      }
#pragma unroll
      for (int m = 0; m < NW; m++) {
        const uint32_t wq = wi == 0 ? wv[m][u].x : wi == 1 ? wv[m][u].y : wi == 2 ? wv[m][u].z : wv[m][u].w;
        u32x4 a0, a1;
        unpack16_nat(wq, a0, a1);
        acc[m] = mfma16(a0, xv[j][0], acc[m]);
        acc[m] = mfma16(a1, xv[j][1], acc[m]);
        if constexpr (XPL == 2) {
          acc[m] = mfma16(a0, xv[j][2], acc[m]);
          acc[m] = mfma16(a1, xv[j][3], acc[m]);
        }
      }
    }
  }

  // Fixed-order reduction of the waves' partial tiles.
#pragma unroll
  for (int m = 0; m < NW; m++) red[(m * WAVES + wave) * 64 + lane] = acc[m];
  __syncthreads();
  if (wave == 0) {
    f32x4 s[NW];
#pragma unroll
    for (int m = 0; m < NW; m++) {
      s[m] = red[m * WAVES * 64 + lane];
#pragma unroll
      for (int w = 1; w < WAVES; w++) s[m] += red[(m * WAVES + w) * 64 + lane];
      s[m] *= sc[m] * 0.5f;  // 0.5 undoes the 2*dec(c) operand encoding
    }
    if (live && n_out < N) {  // rows 4g..4g+3 of token r
      f32x4 v = s[0];
      if constexpr (NW == 2) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const float a = EPI == GEMV_GEGLU ? act_gelu_tanh(s[0][j]) : act_silu(s[0][j]);
          v[j] = a * s[1][j];
        }
      }
      if constexpr (YSPLIT) {
        // hi = bf16(v), lo = bf16(v - hi) (lo = 0 where hi is not finite)
        f32x4 hi, lo;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          hi[j] = bf16_to_f32(bf16_rne(v[j]));
          lo[j] = (__float_as_uint(hi[j]) & 0x7F800000u) == 0x7F800000u ? 0.0f : v[j] - hi[j];
        }
        YStore<uint16_t>::store4(reinterpret_cast<uint16_t *>(Y) + (size_t)r * N + n_out, hi,
                                 min(4, N - n_out));
        YStore<uint16_t>::store4(reinterpret_cast<uint16_t *>(Y) + (size_t)B * N + (size_t)r * N + n_out,
                                 lo, min(4, N - n_out));
      } else {
        if constexpr (NW == 1)
          if (bias) v = add_bias4(v, bias, n_out, N);
        YStore<YT>::store4(Y + (size_t)r * N + n_out, v, min(4, N - n_out));
      }
    }
  }
}

template <typename YT, int WAVES, int UMAX, int D, bool VEC, int EPI, int XPL, bool YSPLIT>
static hipError_t launch_gemv_d(const uint32_t *w, const float *scale, const uint32_t *w2,
                                const float *scale2, const void *x, const void *x2, void *y, int B,
                                int K, int N, hipStream_t stream, const float *bias) {
  hipLaunchKernelGGL((gemv_direct_kernel<YT, WAVES, UMAX, D, VEC, EPI, XPL, YSPLIT>),
                     dim3((N + 15) / 16), dim3(WAVES * 64), 0, stream, w, scale, w2, scale2,
                     reinterpret_cast<const uint16_t *>(x), reinterpret_cast<const uint16_t *>(x2),
                     reinterpret_cast<YT *>(y), B, K, N, bias);
  return hipGetLastError();
}

// ---- bf16 activations, B >= 8, wide matrices: taller tiles ---------------
//
// At B = 16 the direct kernel's time is its activation loads (ablation at
// 11008x4096 / 4096x11008: 14.1 / 12.4 us per launch, 5.3 / 5.2 us with the
// activation loads removed, decode and reduction under 0.7 us): every
// 16-row tile reads all of x, 90 MB per launch from L2. Here a tile is
// 16 * RS rows and each activation load feeds RS row blocks (RS unpacks and
// 2 * RS MFMAs per word), which divides that traffic by RS. Used where the
// taller tiles still give every CU a workgroup (11008x4096: 14.3 -> 12.2 us
// at RS = 2). Where they would not, the direct kernel stays: splitting K
// over workgroups with an in-kernel combine (device-coherent partials and a
// per-tile counter) was measured: the combine's chain of memory round trips
// cost what the halved traffic saved (4096x11008: 12.9 us against 12.8 us),
// and 32-row tiles without a split leave half the CUs idle there (15.6 us).
template <typename YT, int WAVES, int UMAX, int D, bool VEC, int RS>
__global__ __launch_bounds__(WAVES * 64) void gemv_tall_kernel(
    const uint32_t *__restrict__ W, const float *__restrict__ scale, const uint16_t *__restrict__ X,
    YT *__restrict__ Y, int B, int K, int N, const float *__restrict__ bias) {
  constexpr int NWD = 4 * UMAX;  // weight words per lane and row block in one batch
  static_assert(D >= 1 && D <= NWD, "prefetch distance");
  __shared__ f32x4 red[RS * WAVES * 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int wpr = K >> 4;
  const int n_base = blockIdx.x * 16 * RS;
  const uint32_t *wrow[RS];
#pragma unroll
  for (int rs = 0; rs < RS; rs++) wrow[rs] = W + (size_t)min(n_base + 16 * rs + r, N - 1) * wpr;
  const int nch = (K + 63) >> 6, nq = (nch + 3) >> 2;
  const int qa = (wave * nq) / WAVES, qb = ((wave + 1) * nq) / WAVES;  // this wave's quads
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(X, (uint32_t)B * (uint32_t)K * 2u);
  const uint32_t xrow = (uint32_t)r * (uint32_t)K * 2u;  // past the range when r >= B
  constexpr uint32_t XOOB = 0x80000000u;
  const bool live = r < B;
  f32x4 sc[RS];
#pragma unroll
  for (int rs = 0; rs < RS; rs++) {
    const int n_out = n_base + 16 * rs + 4 * g;
    sc[rs] = (f32x4){0.f, 0.f, 0.f, 0.f};
    if (wave == 0 && live && n_out < N) {
      const int nok = min(4, N - n_out);
      sc[rs].x = scale[n_out];
      sc[rs].y = nok > 1 ? scale[n_out + 1] : 0.f;
      sc[rs].z = nok > 2 ? scale[n_out + 2] : 0.f;
      sc[rs].w = nok > 3 ? scale[n_out + 3] : 0.f;
    }
  }
  f32x4 acc[RS];
#pragma unroll
  for (int rs = 0; rs < RS; rs++) acc[rs] = (f32x4){0.f, 0.f, 0.f, 0.f};

  for (int q0 = qa; q0 < qb; q0 += UMAX) {
    const int nwd = 4 * min(UMAX, qb - q0);
    auto xoff = [&](int j) -> uint32_t {
      const int col = 256 * (q0 + (j >> 2)) + 64 * (j & 3) + 16 * g;
      return (j < nwd && col < K) ? xrow + 2u * (uint32_t)col : XOOB;
    };
    u32x4 xv[NWD][2];
    auto xload = [&](int j) {
      const uint32_t o = xoff(j);
      xv[j][0] = __builtin_amdgcn_raw_buffer_load_b128(xr, o, 0, 0);
      xv[j][1] = __builtin_amdgcn_raw_buffer_load_b128(xr, o + 16u, 0, 0);
    };
#pragma unroll
    for (int j = 0; j < D; j++) xload(j);
    u32x4 wv[RS][UMAX];
#pragma unroll
    for (int u = 0; u < UMAX; u++) {
      const int wb = 4 * (4 * (q0 + u) + g);
#pragma unroll
      for (int rs = 0; rs < RS; rs++) wv[rs][u] = load_chunk<VEC>(wrow[rs], wb, wpr);
    }
#pragma unroll
    for (int j = 0; j < NWD; j++) {
      if (j + D < NWD) xload(j + D);
      if (j >= nwd) continue;  // wave-uniform
      const int u = j >> 2, wi = j & 3;
      if (wi == 0) {
        // the 4x4 word transpose of gemv_direct_kernel, per row block
#pragma unroll
        for (int rs = 0; rs < RS; rs++) {
          u32x4 &v = wv[rs][u];
          const auto p02 = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
          const auto p13 = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
          const auto p01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
          const auto p23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
          v = (u32x4){p01[0], p01[1], p23[0], p23[1]};
        }
      }
#pragma unroll
      for (int rs = 0; rs < RS; rs++) {
        const uint32_t wq = wi == 0 ? wv[rs][u].x : wi == 1 ? wv[rs][u].y : wi == 2 ? wv[rs][u].z : wv[rs][u].w;
        u32x4 a0, a1;
        unpack16_nat(wq, a0, a1);
        acc[rs] = mfma16(a0, xv[j][0], acc[rs]);
        acc[rs] = mfma16(a1, xv[j][1], acc[rs]);
      }
    }
  }

  // Fixed-order reduction of the waves' partial tiles.
#pragma unroll
  for (int rs = 0; rs < RS; rs++) red[(rs * WAVES + wave) * 64 + lane] = acc[rs];
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int rs = 0; rs < RS; rs++) {
    f32x4 v = red[rs * WAVES * 64 + lane];
#pragma unroll
    for (int w = 1; w < WAVES; w++) v += red[(rs * WAVES + w) * 64 + lane];
    const int n_out = n_base + 16 * rs + 4 * g;
    if (live && n_out < N) {
      v = v * sc[rs] * 0.5f;
      if (bias) v = add_bias4(v, bias, n_out, N);
      YStore<YT>::store4(Y + (size_t)r * N + n_out, v, min(4, N - n_out));
    }
  }
}

template <typename YT, int WAVES, int UMAX, int D, bool VEC, int RS>
static hipError_t launch_gemv_tall_w(const uint32_t *w, const float *scale, const void *x, void *y, int B, int K,
                                     int N, hipStream_t stream, const float *bias) {
  hipLaunchKernelGGL((gemv_tall_kernel<YT, WAVES, UMAX, D, VEC, RS>), dim3((N + 16 * RS - 1) / (16 * RS)),
                     dim3(WAVES * 64), 0, stream, w, scale, reinterpret_cast<const uint16_t *>(x),
                     reinterpret_cast<YT *>(y), B, K, N, bias);
  return hipGetLastError();
}

// Rows per tile of the tall kernel: 16 * GEMV_TALL_RS.
constexpr int GEMV_TALL_RS = 2;

template <typename YT>
static hipError_t launch_gemv_tall(const uint32_t *w, const float *scale, const void *x, void *y, int B, int K,
                                   int N, hipStream_t stream, const float *bias) {
  constexpr int RS = GEMV_TALL_RS;
  const bool vec = ((K >> 4) & 3) == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0;
  const int nq = (K + 255) / 256;
#define FRX_GEMV_T(WV, UM)                                                                       \
  return vec ? launch_gemv_tall_w<YT, WV, UM, 4, true, RS>(w, scale, x, y, B, K, N, stream, bias) \
             : launch_gemv_tall_w<YT, WV, UM, 4, false, RS>(w, scale, x, y, B, K, N, stream, bias)
  if (nq <= 8) FRX_GEMV_T(4, 2);
  if (nq <= 16) FRX_GEMV_T(8, 2);
  if (nq <= 48) FRX_GEMV_T(16, 3);
  FRX_GEMV_T(16, 4);
#undef FRX_GEMV_T
}

template <typename YT, int EPI, int XPL = 1, bool YSPLIT = false>
static hipError_t launch_gemv_direct(const uint32_t *w, const float *scale, const uint32_t *w2,
                                     const float *scale2, const void *x, const void *x2, void *y,
                                     int B, int K, int N, hipStream_t stream, const float *bias = nullptr) {
  // Waves per tile as in gemv_kernel (two to three quads per wave). D words
  // of activations in flight per lane (8 registers per plane): 8 for the
  // 16-wave tiles (one workgroup per CU), 4 where several workgroups of a
  // wide matrix must be resident at once or two planes double the registers.
  const bool vec = ((K >> 4) & 3) == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(w2) & 15) == 0;
#define FRX_GEMV_D(WV, UM, DD)                                                                          \
  return vec ? launch_gemv_d<YT, WV, UM, DD, true, EPI, XPL, YSPLIT>(w, scale, w2, scale2, x, x2, y, B, K, \
                                                                      N, stream, bias)                  \
             : launch_gemv_d<YT, WV, UM, DD, false, EPI, XPL, YSPLIT>(w, scale, w2, scale2, x, x2, y, B,  \
                                                                       K, N, stream, bias)
  const int nq = (K + 255) / 256;
  if (nq <= 8) FRX_GEMV_D(4, 2, 4);
  if (nq <= 16) FRX_GEMV_D(8, 2, 4);
  if constexpr (EPI != GEMV_LINEAR) {
    FRX_GEMV_D(8, 3, 4);
  } else {
    if (nq <= 48) FRX_GEMV_D(16, 3, XPL == 2 ? 4 : 8);
    FRX_GEMV_D(16, 4, XPL == 2 ? 2 : 8);
  }
#undef FRX_GEMV_D
}

// ---- one bf16 token (B = 1): whole rows per wave --------------------------
//
// Each wave owns RW complete rows, so no partial sums cross waves. A wave
// instruction reads a 1 KB window of one row (lane l: bytes 16l..16l+15 of
// the window, full 128-byte lines); the 16 MFMA rows are the 16 lane
// segments of that window (row r = l%16, k-group g = l/16 as the MFMA
// lays out A) and the 16 MFMA columns the activations of the same
// segments, so column c of B holds x at the positions of A's row c and the
// dot product is the diagonal of the 16x16 accumulator. A lane's 64
// activations per window (natural order, the order unpack16_nat gives the
// codes) come from LDS, staged once per workgroup with a 16-byte pad per
// 64 values so that the lanes' 128-byte reads spread over the banks; one
// read feeds the wave's RW rows. Activations past K are zero, and the
// weight loads of a partial last window are clamped inside the row (the
// zero activations cancel whatever those words hold). The diagonal lives
// in lanes (c, c/4) register c%4: two quad DPP adds and four lane reads
// sum it, in a fixed order, so results are deterministic.
// Against the 16-row tiles with K split over waves (gemv_kernel at B = 1),
// measured over rotating weights: 5.38 -> 4.83 us (11008x4096) and 5.33 ->
// 4.97 us (4096x11008) per launch. A per-wave timeline shows the weights of
// a launch landing within ~1 us, ~2.3 us after the start; the decode (15
// VALU ops per word) then runs on every SIMD at once, which is what
// remains above the bare read.
constexpr int ROWS_XCH = 36;  // LDS dwords per 64-activation chunk (128 B + 16 B pad)

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

// NW = 2 (EPI = GEMV_SWIGLU / GEMV_GEGLU): rows of the gate (W) and up (W2)
// matrices with the same index against the same x; h = act(g) * u is
// written as bf16 hi and lo planes (Y = [2][N], |h - hi - lo| <= 2^-17 |h|).
// XPL = 2: the activations arrive as two bf16 planes (X hi, X2 lo) whose sum
// is an fp32 vector to 2^-17; both are staged and each word runs four MFMAs
// into the same accumulator.
// K-interleaved staging of x for the decode of unpack32_kil: the 16-column
// block b is pieces 2b (columns 0..7) and 2b+1 (8..15) of 8 bf16, held by
// neighbouring lanes (piece index parity = lane parity). After swapping
// pieces with its neighbour, the even lane returns block dwords 0..3 and the
// odd lane dwords 4..7, dword i = x[16b + i] | x[16b + i + 8] << 16, to be
// stored where its own piece would go. Every lane of the wave must call it
// (DPP); pieces past the data are zeros.
__device__ __forceinline__ u32x4 stage_kil(const u32x4 &mine, int tid) {
  u32x4 other;
#pragma unroll
  for (int d = 0; d < 4; d++)
    other[d] = (uint32_t)__builtin_amdgcn_mov_dpp((int)mine[d], 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  const bool odd = tid & 1;
  const u32x4 A = odd ? other : mine, B = odd ? mine : other;
  const uint32_t a0 = odd ? A.z : A.x, a1 = odd ? A.w : A.y, c0 = odd ? B.z : B.x, c1 = odd ? B.w : B.y;
  return (u32x4){__builtin_amdgcn_perm(c0, a0, 0x05040100u), __builtin_amdgcn_perm(c0, a0, 0x07060302u),
                 __builtin_amdgcn_perm(c1, a1, 0x05040100u), __builtin_amdgcn_perm(c1, a1, 0x07060302u)};
}

template <typename YT, int WAVES, int RW, int NI, int NW = 1, int XPL = 1, int EPI = GEMV_LINEAR>
__global__ __launch_bounds__(WAVES * 64) void gemv_rows_kernel(
    const uint32_t *__restrict__ W, const float *__restrict__ scale, const uint32_t *__restrict__ W2,
    const float *__restrict__ scale2, const uint16_t *__restrict__ X, const uint16_t *__restrict__ X2,
    YT *__restrict__ Y, int K, int N, const float *__restrict__ bias) {
  static_assert((NW == 2) == (EPI != GEMV_LINEAR), "two matrices exactly for the GLU epilogues");
  extern __shared__ __align__(16) uint32_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = ((int)blockIdx.x * WAVES + wave) * RW;
  const int kw = K >> 4;   // words per row
  const int nxp = K >> 3;  // 16-byte pieces of x
  constexpr int NT = WAVES * 64;
  constexpr int PP = NI * 512;                  // staged pieces per plane (NI * 4096 activations)
  constexpr int PD = NI * 64 * ROWS_XCH;        // LDS dwords per plane
  constexpr int XR = (XPL * PP + NT - 1) / NT;  // staging rounds
  // 1. activations (zero past K), issued before the weights so that waiting
  //    for them does not wait for the weights
  u32x4 xs[XR];
#pragma unroll
  for (int r = 0; r < XR; r++) {
    const int j = tid + r * NT, pl = j >= PP ? 1 : 0, jp = j - pl * PP;
    const u32x4 *X4 = reinterpret_cast<const u32x4 *>(pl ? X2 : X);
    xs[r] = (u32x4){0u, 0u, 0u, 0u};
    if (pl < XPL && jp < nxp) xs[r] = X4[jp];
  }
  // 2. the wave's weights: NW matrices x RW rows x NI windows
  u32x4 wv[NW][RW][NI];
  float sc[NW][RW];
#pragma unroll
  for (int m = 0; m < NW; m++)
#pragma unroll
    for (int rr = 0; rr < RW; rr++) {
      const int row = min(row0 + rr, N - 1);
      const uint32_t *wr = (m ? W2 : W) + (size_t)row * kw;
#pragma unroll
      for (int i = 0; i < NI; i++)
        wv[m][rr][i] = *reinterpret_cast<const u32x4 *>(wr + min(i * 256 + 4 * lane, kw - 4));
      sc[m][rr] = (m ? scale2 : scale)[row];
    }
  // 3. stage: plane p, 16-byte piece j -> chunk j/8, slot j%8, K-interleaved
  //    (stage_kil; PP is even, so neighbouring pieces share a plane)
#pragma unroll
  for (int r = 0; r < XR; r++) {
    const int j = tid + r * NT, pl = j >= PP ? 1 : 0, jp = j - pl * PP;
    const u32x4 v = stage_kil(xs[r], tid);
    if (pl < XPL) *reinterpret_cast<u32x4 *>(lds + pl * PD + (jp >> 3) * ROWS_XCH + (jp & 7) * 4) = v;
  }
  __syncthreads();
  // 4. per window: the lane's 64 activations (per plane), then each row's 4 words
  f32x4 acc[NW][RW];
#pragma unroll
  for (int m = 0; m < NW; m++)
#pragma unroll
    for (int rr = 0; rr < RW; rr++) acc[m][rr] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NI; i++) {
    u32x4 xb[XPL][8];
#pragma unroll
    for (int p = 0; p < XPL; p++) {
      const uint32_t *xp = lds + p * PD + (i * 64 + lane) * ROWS_XCH;
#pragma unroll
      for (int q = 0; q < 8; q++) xb[p][q] = *reinterpret_cast<const u32x4 *>(xp + 4 * q);
    }
#pragma unroll
    for (int m = 0; m < NW; m++)
#pragma unroll
      for (int rr = 0; rr < RW; rr++) {
        u32x4 lo[4], hi[4];
        unpack32_kil(wv[m][rr][i].x, wv[m][rr][i].y, lo[0], hi[0], lo[1], hi[1]);
        unpack32_kil(wv[m][rr][i].z, wv[m][rr][i].w, lo[2], hi[2], lo[3], hi[3]);
#pragma unroll
        for (int j = 0; j < 4; j++) {
#pragma unroll
          for (int p = 0; p < XPL; p++) {
            acc[m][rr] = mfma16(lo[j], xb[p][2 * j], acc[m][rr]);
            acc[m][rr] = mfma16(hi[j], xb[p][2 * j + 1], acc[m][rr]);
          }
        }
      }
  }
  // 5. diagonal: lane (c = l%16, rg = l/16) holds C[4rg + e][c]
  const int c = lane & 15, rg = lane >> 4, e = c & 3;
  const bool diag = (c >> 2) == rg;
  float tot[NW][RW];
#pragma unroll
  for (int m = 0; m < NW; m++)
#pragma unroll
    for (int rr = 0; rr < RW; rr++) {
      const f32x4 A = acc[m][rr];
      float v = e == 0 ? A[0] : e == 1 ? A[1] : e == 2 ? A[2] : A[3];
      v = diag ? v : 0.f;
      v += dpp_f32<0xB1>(v);  // quad_perm [1,0,3,2]
      v += dpp_f32<0x4E>(v);  // quad_perm [2,3,0,1]
      const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
      const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 20));
      const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 40));
      const float f = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 60));
      tot[m][rr] = ((a + b) + (d + f)) * sc[m][rr] * 0.5f;  // 0.5 undoes the 2*dec(c) encoding
    }
  if (lane < RW) {
    float t[NW];
#pragma unroll
    for (int m = 0; m < NW; m++) {
      t[m] = tot[m][0];
#pragma unroll
      for (int rr = 1; rr < RW; rr++)
        if (lane == rr) t[m] = tot[m][rr];
    }
    const int row = row0 + lane;
    if (row < N) {
      if constexpr (EPI != GEMV_LINEAR) {
        const float h = (EPI == GEMV_GEGLU ? act_gelu_tanh(t[0]) : act_silu(t[0])) * t[1];
        uint32_t hh, hl;
        split_bf16(h, hh, hl);
        Y[row] = (uint16_t)hh;
        Y[N + row] = (uint16_t)hl;
      } else {
        const float o = bias ? add_bias(t[0], bias[row]) : t[0];
        if constexpr (sizeof(YT) == 2) Y[row] = (uint16_t)bf16_rne(o);
        else Y[row] = o;
      }
    }
  }
}

template <typename YT, int RW, int NI, int NW = 1, int XPL = 1, int EPI = GEMV_LINEAR>
static hipError_t launch_gemv_rows_w(const uint32_t *w, const float *scale, const uint32_t *w2, const float *scale2,
                                     const void *x, const void *x2, void *y, int K, int N, hipStream_t stream,
                                     const float *bias = nullptr) {
  constexpr int WAVES = 8;
  const dim3 grid((N + WAVES * RW - 1) / (WAVES * RW));
  const size_t lds = (size_t)XPL * NI * 64 * ROWS_XCH * 4;
  if (lds > 64 * 1024) {
    static std::atomic<uint64_t> done;
    const hipError_t e = opt_in_lds(reinterpret_cast<const void *>(&gemv_rows_kernel<YT, WAVES, RW, NI, NW, XPL, EPI>),
                                    (int)lds, done);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((gemv_rows_kernel<YT, WAVES, RW, NI, NW, XPL, EPI>), grid, dim3(WAVES * 64), lds, stream, w,
                     scale, w2, scale2, reinterpret_cast<const uint16_t *>(x),
                     reinterpret_cast<const uint16_t *>(x2), reinterpret_cast<YT *>(y), K, N, bias);
  return hipGetLastError();
}

// ---- one token, balanced: one or two workgroups per CU --------------------
//
// The rows kernel's decode (whole 1 KB windows per wave instruction, the MFMA
// diagonal, the same reduction order) with the rows of the matrix split
// evenly over G = 1 or 2 workgroups per CU, and within a workgroup over its
// 8 waves, so that every CU decodes the same number of rows. Every wave
// issues its share of x first and a workgroup barrier separates those loads
// from the weight loads: in the CU's in-order memory pipeline the staging of
// x then does not wait behind weights. Row scales are scalar loads (uniform
// rows). Measured per launch against gemv_rows_kernel: 5.66 -> 5.50 us
// (11008x4096, G = 2 per CU) and 5.67 -> 5.28 us (4096x11008, G = 1).
// The weight words decode in K-interleaved pairs (unpack32_kil, two words
// per 64-bit shift) and x is staged in the same order. One matrix (NW = 1):
// each row's diagonal is summed within its quads as the row completes, and
// the cross-quad sums of all the wave's rows run once at the end, merged
// into one register (row r at position r of each quad).
// XF32: fp32 activations, split once per workgroup at staging into bf16 hi
// and lo planes (split2_bf16: hi = bf16(x), lo = bf16(x - hi), |x - hi - lo|
// <= 2^-17 |x|, lo = 0 where hi is not finite); each word then runs four
// MFMAs.
// XPLN: the activations arrive as two bf16 planes, hi at Xv and lo K values
// further (h of the decode FFN, |h - hi - lo| <= 2^-17 |h|): both are staged
// and each word runs four MFMAs. NW = 2 (EPI = GEMV_SWIGLU / GEMV_GEGLU):
// the same rows of the gate (W) and up (W2) matrices against the same x;
// h = act(g) * u is written as bf16 hi and lo planes (Y = [2][N]).
template <typename YT, int NI, int RMAX, bool XF32, bool XPLN = false, int NW = 1, int EPI = GEMV_LINEAR,
          bool GRP = false>
__global__ __launch_bounds__(512) void gemv_bal_kernel(const uint32_t *__restrict__ W, const float *__restrict__ scale,
                                                       const uint32_t *__restrict__ W2,
                                                       const float *__restrict__ scale2,
                                                       const void *__restrict__ Xv, YT *__restrict__ Y, int K, int N,
                                                       const float *__restrict__ bias, int nq, int nr,
                                                       const GemvGroup grp) {
  static_assert((NW == 2) == (EPI != GEMV_LINEAR), "two matrices exactly for the GLU epilogues");
  static_assert(!(XF32 && XPLN), "one activation source");
  static_assert(!GRP || (NW == 1 && !XPLN), "a group of linear matrices over one x");
  constexpr int WAVES = 8, NT = 512;
  constexpr int XPL = (XF32 || XPLN) ? 2 : 1;
  constexpr int PP = NI * 512;                   // 8-value pieces of x staged (NI * 4096 values)
  constexpr int PD = NI * 64 * ROWS_XCH;         // LDS dwords per plane
  constexpr int XR = (PP + NT - 1) / NT;         // pieces per thread
  constexpr int XL = (XF32 || XPLN) ? 2 : 1;     // 16-byte loads per piece
  extern __shared__ __align__(16) uint32_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // rows of this workgroup: nq = N / G each, the first nr = N % G one more
  // (the host divides; a scalar division would delay every load)
  const int bx = blockIdx.x;
  const int b0 = bx * nq + min(bx, nr), cb = nq + (bx < nr ? 1 : 0);
  const int row0 = b0 + wave * cb / WAVES, cnt = b0 + (wave + 1) * cb / WAVES - row0;
  const int kw = K >> 4;
  constexpr uint32_t OOB = 0x80000000u;  // a buffer offset past any range this path takes
  // x range: K values (f32 or bf16); planes: one descriptor per plane, each
  // K bf16 long, so that pieces past K read zeros in both (the weight words
  // past K decode to -1 and must meet zeros)
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(Xv, (uint32_t)K * (XF32 ? 4u : 2u));
  const __amdgpu_buffer_rsrc_t xr2 =
      buffer_rsrc(XPLN ? reinterpret_cast<const char *>(Xv) + (size_t)K * 2 : Xv, (uint32_t)K * 2u);
  __amdgpu_buffer_rsrc_t wr[NW];
#pragma unroll
  for (int m = 0; m < NW; m++) wr[m] = buffer_rsrc(m ? W2 : W, (uint32_t)N * (uint32_t)kw * 4u);
  // GRP: the rows of the group's matrices, concatenated, are the rows of the
  // launch; launch row r (wave-uniform) is located by scalar selects
  // (GemvGroup::locate) and read through a descriptor of its own row, built
  // where it is loaded (no arrays of descriptors: they would go to scratch)
  auto grp_row = [&](int rr, const uint32_t *&wp, const float *&sp) {
    const int r = min(row0 + rr, N - 1);
    int first;
    grp.locate(r, wp, sp, first);
    const int l = r - first;
    wp += (size_t)l * (uint32_t)kw;
    sp += l;
  };
  // 1. x pieces (zero past K), then a barrier: all of the CU's x loads are
  //    ahead of its weight loads
  u32x4 xs[XR][XL];
#pragma unroll
  for (int r = 0; r < XR; r++) {
    const int j = tid + r * NT;
    const uint32_t off = j < PP ? (uint32_t)j * (XF32 ? 32u : 16u) : OOB;
    // f32: the piece's two 16-byte halves; planes: the piece in each plane
#pragma unroll
    for (int l = 0; l < XL; l++)
      xs[r][l] = XPLN ? __builtin_amdgcn_raw_buffer_load_b128(l ? xr2 : xr, off, 0, 0)
                      : __builtin_amdgcn_raw_buffer_load_b128(xr, off + 16u * l, 0, 0);
  }
  __syncthreads();
  // 2. the wave's rows (rows past cnt read zeros without touching memory)
  u32x4 wv[RMAX][NW][NI];
#pragma unroll
  for (int rr = 0; rr < RMAX; rr++)
#pragma unroll
    for (int m = 0; m < NW; m++)
#pragma unroll
      for (int i = 0; i < NI; i++) {
        const int wi = i * 256 + 4 * lane;
        if constexpr (GRP) {
          const uint32_t *wp;
          const float *sp;
          grp_row(rr, wp, sp);
          const uint32_t off = (rr < cnt && wi < kw) ? (uint32_t)wi * 4u : OOB;
          wv[rr][m][i] = __builtin_amdgcn_raw_buffer_load_b128(buffer_rsrc(wp, (uint32_t)kw * 4u), off, 0, 0);
        } else {
          const uint32_t off =
              (rr < cnt && wi < kw) ? ((uint32_t)(row0 + rr) * (uint32_t)kw + (uint32_t)wi) * 4u : OOB;
          wv[rr][m][i] = __builtin_amdgcn_raw_buffer_load_b128(wr[m], off, 0, 0);
        }
      }
  float sc[RMAX][NW];
#pragma unroll
  for (int rr = 0; rr < RMAX; rr++)
#pragma unroll
    for (int m = 0; m < NW; m++) {
      if constexpr (GRP) {
        const uint32_t *wp;
        const float *sp;
        grp_row(rr, wp, sp);
        sc[rr][m] = *sp;
      }
      else sc[rr][m] = (m ? scale2 : scale)[min(row0 + rr, N - 1)];
    }
  const float bv = bias ? bias[min(row0 + lane, N - 1)] : 0.f;  // lane's output row
  // 3. stage: piece j -> chunk j/8, slot j%8 (per plane), K-interleaved to
  //    match the decode (stage_kil: all lanes take part)
#pragma unroll
  for (int r = 0; r < XR; r++) {
    const int j = tid + r * NT;
    uint32_t *dst = lds + (j >> 3) * ROWS_XCH + (j & 7) * 4;
    if constexpr (XPLN) {
      const u32x4 h = stage_kil(xs[r][0], tid), l = stage_kil(xs[r][1], tid);
      if (j < PP) {
        *reinterpret_cast<u32x4 *>(dst) = h;
        *reinterpret_cast<u32x4 *>(dst + PD) = l;
      }
    } else if constexpr (XF32) {
      const float f[8] = {__uint_as_float(xs[r][0].x), __uint_as_float(xs[r][0].y), __uint_as_float(xs[r][0].z),
                          __uint_as_float(xs[r][0].w), __uint_as_float(xs[r][1].x), __uint_as_float(xs[r][1].y),
                          __uint_as_float(xs[r][1].z), __uint_as_float(xs[r][1].w)};
      uint32_t hi[4], lo[4];
#pragma unroll
      for (int e = 0; e < 4; e++) split2_bf16(f[2 * e], f[2 * e + 1], hi[e], lo[e]);
      const u32x4 h = stage_kil((u32x4){hi[0], hi[1], hi[2], hi[3]}, tid),
                  l = stage_kil((u32x4){lo[0], lo[1], lo[2], lo[3]}, tid);
      if (j < PP) {
        *reinterpret_cast<u32x4 *>(dst) = h;
        *reinterpret_cast<u32x4 *>(dst + PD) = l;
      }
    } else {
      const u32x4 v = stage_kil(xs[r][0], tid);
      if (j < PP) *reinterpret_cast<u32x4 *>(dst) = v;
    }
  }
  __syncthreads();
  // 4. the lane's activations of every window once (registers; re-read per
  //    row where two planes of more than two windows would not fit), then
  //    rows in order as their weights land, each reduced right away
  constexpr bool XREG = NI * XPL <= 4;
  u32x4 xb[XREG ? NI : 1][XPL][8];
  auto xread = [&](int i, u32x4(&dst)[XPL][8]) {
#pragma unroll
    for (int p = 0; p < XPL; p++) {
      const uint32_t *xp = lds + p * PD + (i * 64 + lane) * ROWS_XCH;
#pragma unroll
      for (int q = 0; q < 8; q++) dst[p][q] = *reinterpret_cast<const u32x4 *>(xp + 4 * q);
    }
  };
  if constexpr (XREG) {
#pragma unroll
    for (int i = 0; i < NI; i++) xread(i, xb[i]);
  }
  float res[NW];
#pragma unroll
  for (int m = 0; m < NW; m++) res[m] = 0.f;
  const int c = lane & 15, rg = lane >> 4, e = c & 3;
  const bool e_odd = e & 1, e_hi = e & 2, diag = (c >> 2) == rg;
  float vq[RMAX];  // NW == 1: each row's diagonal, summed within its quads
#pragma unroll
  for (int rr = 0; rr < RMAX; rr++) {
    vq[rr] = 0.f;
    if (rr < cnt) {  // wave-uniform
#pragma unroll
      for (int m = 0; m < NW; m++) {
        // two accumulation chains (even and odd words) halve the dependent
        // MFMA latency of a row
        f32x4 acc2[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int i = 0; i < NI; i++) {
          u32x4 xw[XPL][8];
          if constexpr (!XREG) xread(i, xw);
          const u32x4(&xv)[XPL][8] = XREG ? xb[XREG ? i : 0] : xw;
          u32x4 lo[4], hi[4];
          unpack32_kil(wv[rr][m][i].x, wv[rr][m][i].y, lo[0], hi[0], lo[1], hi[1]);
          unpack32_kil(wv[rr][m][i].z, wv[rr][m][i].w, lo[2], hi[2], lo[3], hi[3]);
#pragma unroll
          for (int j = 0; j < 4; j++) {
#pragma unroll
            for (int p = 0; p < XPL; p++) {
              acc2[j & 1] = mfma16(lo[j], xv[p][2 * j], acc2[j & 1]);
              acc2[j & 1] = mfma16(hi[j], xv[p][2 * j + 1], acc2[j & 1]);
            }
          }
        }
        const f32x4 acc = acc2[0] + acc2[1];
        // diagonal: lane (c = l%16, rg = l/16) holds C[4rg + e][c]
        const float t0 = e_odd ? acc[1] : acc[0], t1 = e_odd ? acc[3] : acc[2];
        float v = diag ? (e_hi ? t1 : t0) : 0.f;
        v += dpp_f32<0xB1>(v);  // quad_perm [1,0,3,2]
        v += dpp_f32<0x4E>(v);  // quad_perm [2,3,0,1]
        if constexpr (NW == 1) {
          vq[rr] = v;
        } else {
          const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
          const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 20));
          const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 40));
          const float f = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 60));
          const float tot = ((a + b) + (d + f)) * sc[rr][m] * 0.5f;  // 0.5 undoes the 2*dec(c) encoding
          if (lane == rr) res[m] = tot;
        }
      }
    }
  }
  if constexpr (NW == 1) {
    // All rows at once: row r's quad sums move to position r of their quads
    // (the diagonal quads are quad g of 16-lane row g, all other lanes 0),
    // rotations by 8 and 4 bring every 16-lane row's quad to positions 0..3,
    // and two exchanges add the four 16-lane rows: lane r < RMAX then holds
    // row r's dot product.
    const int q = lane & 3;
    if constexpr (!GRP) {
      float mv = vq[0];
#pragma unroll
      for (int rr = 1; rr < RMAX; rr++) mv = q == rr ? vq[rr] : mv;
      mv += dpp_f32<0x128>(mv);  // row_ror:8
      mv += dpp_f32<0x124>(mv);  // row_ror:4
      mv += __shfl_xor(mv, 32);
      mv += __shfl_xor(mv, 16);
      float s = sc[0][0];
#pragma unroll
      for (int rr = 1; rr < RMAX; rr++) s = q == rr ? sc[rr][0] : s;
      res[0] = mv * s * 0.5f;  // 0.5 undoes the 2*dec(c) encoding
    } else {
      // Groups take up to 8 rows per wave: every lane l ends with the total
      // of row (l % 4) of its pass, and above four rows a second pass takes
      // rows 4..7, which lanes 4..7 keep. Rows are picked with bit masks (a
      // select chain here became an indexed load from a scratch copy).
      auto pass = [&](auto base_c) {
        constexpr int base = decltype(base_c)::value;
        uint32_t mb = 0, sb = 0;
#pragma unroll
        for (int rr = base; rr < min(RMAX, base + 4); rr++) {
          const uint32_t k = q == rr - base ? 0xFFFFFFFFu : 0u;
          mb |= __float_as_uint(vq[rr]) & k;
          sb |= __float_as_uint(sc[rr][0]) & k;
        }
        float mv = __uint_as_float(mb);
        mv += dpp_f32<0x128>(mv);  // row_ror:8
        mv += dpp_f32<0x124>(mv);  // row_ror:4
        mv += __shfl_xor(mv, 32);
        mv += __shfl_xor(mv, 16);
        return mv * __uint_as_float(sb) * 0.5f;  // 0.5 undoes the 2*dec(c) encoding
      };
      res[0] = pass(std::integral_constant<int, 0>{});
      if constexpr (RMAX > 4) {
        const float r1 = pass(std::integral_constant<int, 4>{});
        if (lane >= 4) res[0] = r1;
      }
    }
  }
  if (lane < cnt) {
    const int row = row0 + lane;
    if constexpr (EPI != GEMV_LINEAR) {
      const float h = (EPI == GEMV_GEGLU ? act_gelu_tanh(res[0]) : act_silu(res[0])) * res[NW - 1];
      uint32_t hh, hl;
      split_bf16(h, hh, hl);
      Y[row] = (uint16_t)hh;
      Y[N + row] = (uint16_t)hl;
    } else if constexpr (GRP) {
      const int m = grp.matrix_of(row);
      YT *Ym = reinterpret_cast<YT *>(grp.y_of(m));
      const int lr = row - grp.start_of(m);
      if constexpr (sizeof(YT) == 2) Ym[lr] = (uint16_t)bf16_rne(res[0]);
      else Ym[lr] = res[0];
    } else {
      float o = res[0];
      if (bias) o = add_bias(o, bv);
      if constexpr (sizeof(YT) == 2) Y[row] = (uint16_t)bf16_rne(o);
      else Y[row] = o;
    }
  }
}

// Most rows per wave of the balanced kernel. The row slots are sized to the
// launch (a slot past the wave's rows still costs its loads: at 4096x11008,
// four slots for two rows measured 6.30 against 5.31 us).
constexpr int GEMV_BAL_RMAX = 4;
constexpr int GEMV_GROUP_RMAX = 8;  // most rows per wave of a same-x group launch

template <typename YT, int NI, int RMAX, bool XF32, bool XPLN = false, int NW = 1, int EPI = GEMV_LINEAR,
          bool GRP = false>
static hipError_t launch_gemv_bal_w(const uint32_t *w, const float *scale, const void *x, void *y, int K, int N,
                                    int G, hipStream_t stream, const float *bias, const uint32_t *w2 = nullptr,
                                    const float *scale2 = nullptr, const GemvGroup *grp = nullptr) {
  const size_t lds = (size_t)((XF32 || XPLN) ? 2 : 1) * NI * 64 * ROWS_XCH * 4;
  if (lds > 64 * 1024) {
    static std::atomic<uint64_t> done;
    const hipError_t e = opt_in_lds(
        reinterpret_cast<const void *>(&gemv_bal_kernel<YT, NI, RMAX, XF32, XPLN, NW, EPI, GRP>), (int)lds, done);
    if (e != hipSuccess) return e;
  }
  const GemvGroup g = grp ? *grp : GemvGroup{};
  hipLaunchKernelGGL((gemv_bal_kernel<YT, NI, RMAX, XF32, XPLN, NW, EPI, GRP>), dim3(G), dim3(512), lds, stream, w,
                     scale, w2 ? w2 : w, scale2 ? scale2 : scale, x, reinterpret_cast<YT *>(y), K, N, bias, N / G,
                     N % G, g);
  return hipGetLastError();
}

static int device_cu_count();

// One token, K % 64 == 0 up to 16384, 16-byte aligned weights and x, and at
// most GEMV_BAL_RMAX rows per wave at G workgroups (two per CU for one
// window per row, one above).
static bool gemv_bal_grid(const uint32_t *w, const void *x, int B, int K, int N, int *G,
                          int rmax = GEMV_BAL_RMAX) {
  if (B != 1 || K % 64 != 0 || K > 4 * 4096 || (reinterpret_cast<uintptr_t>(w) & 15) != 0 ||
      (reinterpret_cast<uintptr_t>(x) & 15) != 0)
    return false;
  const int ni = (K + 4095) / 4096;
  const int g = std::min((ni == 1 ? 2 : 1) * device_cu_count(), (N + 7) / 8);
  if ((N + g - 1) / g > 8 * rmax) return false;
  *G = g;
  return true;
}

bool gemv_bal_fits(const uint32_t *w, const void *x, int B, int K, int N) {
  int G = 0;
  return gemv_bal_grid(w, x, B, K, N, &G);
}

template <typename YT, int NI, bool XF32, bool GRP = false>
static hipError_t launch_gemv_bal_r(const uint32_t *w, const float *scale, const void *x, void *y, int K, int N, int G,
                                    hipStream_t stream, const float *bias, const GemvGroup *grp = nullptr) {
  const int rmax = ((N + G - 1) / G + 7) / 8;
  constexpr int L = GEMV_LINEAR;
  if (rmax <= 1)
    return launch_gemv_bal_w<YT, NI, 1, XF32, false, 1, L, GRP>(w, scale, x, y, K, N, G, stream, bias, nullptr,
                                                                 nullptr, grp);
  if (rmax <= 2)
    return launch_gemv_bal_w<YT, NI, 2, XF32, false, 1, L, GRP>(w, scale, x, y, K, N, G, stream, bias, nullptr,
                                                                 nullptr, grp);
  if (rmax <= 3)
    return launch_gemv_bal_w<YT, NI, 3, XF32, false, 1, L, GRP>(w, scale, x, y, K, N, G, stream, bias, nullptr,
                                                                 nullptr, grp);
  // groups (gate + up: 22016 rows) take up to GEMV_GROUP_RMAX rows per wave
  // up to 12288 columns; above, the registers hold 4 rows at most
  if constexpr (GRP && NI < 4) {
    if (rmax > 6)
      return launch_gemv_bal_w<YT, NI, GEMV_GROUP_RMAX, XF32, false, 1, L, GRP>(w, scale, x, y, K, N, G, stream,
                                                                                 bias, nullptr, nullptr, grp);
    if (rmax > 4)
      return launch_gemv_bal_w<YT, NI, 6, XF32, false, 1, L, GRP>(w, scale, x, y, K, N, G, stream, bias, nullptr,
                                                                   nullptr, grp);
  }
  return launch_gemv_bal_w<YT, NI, 4, XF32, false, 1, L, GRP>(w, scale, x, y, K, N, G, stream, bias, nullptr,
                                                               nullptr, grp);
}

template <typename YT, bool XF32, bool GRP = false>
static hipError_t launch_gemv_bal(const uint32_t *w, const float *scale, const void *x, void *y, int K, int N, int G,
                                  hipStream_t stream, const float *bias, const GemvGroup *grp = nullptr) {
  const int ni = (K + 4095) / 4096;
  if (ni == 1) return launch_gemv_bal_r<YT, 1, XF32, GRP>(w, scale, x, y, K, N, G, stream, bias, grp);
  if (ni == 2) return launch_gemv_bal_r<YT, 2, XF32, GRP>(w, scale, x, y, K, N, G, stream, bias, grp);
  if (ni == 3) return launch_gemv_bal_r<YT, 3, XF32, GRP>(w, scale, x, y, K, N, G, stream, bias, grp);
  return launch_gemv_bal_r<YT, 4, XF32, GRP>(w, scale, x, y, K, N, G, stream, bias, grp);
}

// ---- tall single-token GEMV: persistent waves, next group in flight ------
//
// Above one residency pass the one-shot rows kernel runs in lockstep passes:
// the resident workgroups load, wait, then decode together, so a pass's
// loads do not overlap its decode. Here the grid is two workgroups per CU
// and each wave walks row groups g, g + G, g + 2G, ... (G = waves in the
// grid), two register sets alternating: the next group's words are loaded
// before the current group is decoded. The loads are buffer loads issued
// unconditionally: a group past the end gets an offset beyond the buffer's
// range and reads zeros without touching memory, so no load sits in a branch
// (a conditional load makes the compiler copy its registers at the join and
// wait for it there). Per group the work is the rows kernel's: the same LDS
// activations, windows, MFMA diagonal and reduction order.
constexpr uint32_t ROWS_STREAM_OOB = 0x80000000u;  // past every weight buffer this path takes

template <int RW, int NI>
__device__ __forceinline__ void rows_stream_load(__amdgpu_buffer_rsrc_t wr, const float *__restrict__ scale, int g,
                                                 int ng, int kw, int N, int lane, u32x4 (&wv)[RW][NI],
                                                 float (&sc)[RW]) {
  const bool live = g < ng;
#pragma unroll
  for (int rr = 0; rr < RW; rr++) {
    const int row = min(g * RW + rr, N - 1);
    const uint32_t base = (uint32_t)row * (uint32_t)kw * 4u;
#pragma unroll
    for (int i = 0; i < NI; i++) {
      const uint32_t off = live ? base + 4u * (uint32_t)min(i * 256 + 4 * lane, kw - 4) : ROWS_STREAM_OOB;
      wv[rr][i] = __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0);
    }
    sc[rr] = scale[row];
  }
}

template <typename YT, int RW, int NI>
__device__ __forceinline__ void rows_stream_group(const uint32_t *lds, const u32x4 (&wv)[RW][NI],
                                                  const float (&sc)[RW], int g, int N, int lane,
                                                  YT *__restrict__ Y, const float *__restrict__ bias) {
  // x is staged K-interleaved (stage_kil) and the words decode in pairs
  // (unpack32_kil: 11.5 VALU ops per word against 15 in natural order);
  // each row runs two accumulation chains (even and odd words)
  f32x4 acc[RW][2];
#pragma unroll
  for (int rr = 0; rr < RW; rr++) acc[rr][0] = acc[rr][1] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NI; i++) {
    u32x4 xb[8];
    const uint32_t *xp = lds + (i * 64 + lane) * ROWS_XCH;
#pragma unroll
    for (int q = 0; q < 8; q++) xb[q] = *reinterpret_cast<const u32x4 *>(xp + 4 * q);
#pragma unroll
    for (int rr = 0; rr < RW; rr++) {
      u32x4 lo[4], hi[4];
      unpack32_kil(wv[rr][i].x, wv[rr][i].y, lo[0], hi[0], lo[1], hi[1]);
      unpack32_kil(wv[rr][i].z, wv[rr][i].w, lo[2], hi[2], lo[3], hi[3]);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        acc[rr][j & 1] = mfma16(lo[j], xb[2 * j], acc[rr][j & 1]);
        acc[rr][j & 1] = mfma16(hi[j], xb[2 * j + 1], acc[rr][j & 1]);
      }
    }
  }
  const int c = lane & 15, rg = lane >> 4, e = c & 3;
  const bool diag = (c >> 2) == rg;
  float t = 0.f;
#pragma unroll
  for (int rr = 0; rr < RW; rr++) {
    const f32x4 A = acc[rr][0] + acc[rr][1];
    float v = e == 0 ? A[0] : e == 1 ? A[1] : e == 2 ? A[2] : A[3];
    v = diag ? v : 0.f;
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 20));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 40));
    const float f = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 60));
    const float tr = ((a + b) + (d + f)) * sc[rr] * 0.5f;  // 0.5 undoes the 2*dec(c) encoding
    if (lane == rr) t = tr;
  }
  const int row = g * RW + lane;
  if (lane < RW && row < N) {
    if (bias) t = add_bias(t, bias[row]);
    if constexpr (sizeof(YT) == 2) Y[row] = (uint16_t)bf16_rne(t);
    else Y[row] = t;
  }
}

template <typename YT, int WAVES, int RW, int NI>
__global__ __launch_bounds__(WAVES * 64) void gemv_rows_stream_kernel(const uint32_t *__restrict__ W,
                                                                      const float *__restrict__ scale,
                                                                      const uint16_t *__restrict__ X,
                                                                      YT *__restrict__ Y, int K, int N,
                                                                      const float *__restrict__ bias) {
  extern __shared__ __align__(16) uint32_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kw = K >> 4, nxp = K >> 3;
  const int ng = (N + RW - 1) / RW;
  const int stride = (int)gridDim.x * WAVES;
  int g = (int)blockIdx.x * WAVES + wave;
  const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(W, (uint32_t)N * (uint32_t)kw * 4u);
  constexpr int NT = WAVES * 64;
  constexpr int PP = NI * 512;
  constexpr int XR = (PP + NT - 1) / NT;
  // activations first (zero past K), then the first group's weights
  u32x4 xs[XR];
  const u32x4 *X4 = reinterpret_cast<const u32x4 *>(X);
#pragma unroll
  for (int r = 0; r < XR; r++) {
    const int j = tid + r * NT;
    xs[r] = (u32x4){0u, 0u, 0u, 0u};
    if (j < PP && j < nxp) xs[r] = X4[j];
  }
  u32x4 wa[RW][NI], wb[RW][NI];
  float sa[RW], sb[RW];
  rows_stream_load<RW, NI>(wr, scale, g, ng, kw, N, lane, wa, sa);
  // K-interleaved staging (all lanes take part in the exchange; PP and NT
  // are even, so neighbouring pieces are neighbouring lanes)
#pragma unroll
  for (int r = 0; r < XR; r++) {
    const int j = tid + r * NT;
    const u32x4 v = stage_kil(xs[r], tid);
    if (j < PP) *reinterpret_cast<u32x4 *>(lds + (j >> 3) * ROWS_XCH + (j & 7) * 4) = v;
  }
  __syncthreads();
  for (; g < ng; g += 2 * stride) {  // wave-uniform; no barrier below
    const int g1 = g + stride, g2 = g1 + stride;
    rows_stream_load<RW, NI>(wr, scale, g1, ng, kw, N, lane, wb, sb);
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the decode
    rows_stream_group<YT, RW, NI>(lds, wa, sa, g, N, lane, Y, bias);
    rows_stream_load<RW, NI>(wr, scale, g2, ng, kw, N, lane, wa, sa);
    __builtin_amdgcn_sched_barrier(0);
    if (g1 < ng) rows_stream_group<YT, RW, NI>(lds, wb, sb, g1, N, lane, Y, bias);
  }
}

// ---- one token over rows of 16448 to 32768 codes ------------------------
//
// The persistent form above with each row read in NP passes of NH windows
// (1 KB per lane group and window), so that one register set holds a pass
// and the next pass (of the same row, or the next row's first) is in
// flight while the current one decodes: a row longer than the four windows
// a register set holds (8192 x 28672, the LLaMA-70B down projection) still
// streams two sets deep. One row per wave unit; the x of the whole row is
// staged once per workgroup, K-interleaved. The passes of a row accumulate
// into the same two chains; the row is reduced and stored after its last.
template <int NH>
__device__ __forceinline__ void rows_pass_load(__amdgpu_buffer_rsrc_t wr, int row, int pass, bool live, int kw,
                                               int lane, u32x4 (&wv)[NH]) {
  const uint32_t base = (uint32_t)row * (uint32_t)kw * 4u;
#pragma unroll
  for (int i = 0; i < NH; i++) {
    const int wi = (pass * NH + i) * 256 + 4 * lane;
    const uint32_t off = live ? base + 4u * (uint32_t)min(wi, kw - 4) : ROWS_STREAM_OOB;
    wv[i] = __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0);
  }
}

template <int NH>
__device__ __forceinline__ void rows_pass_acc(const uint32_t *lds, const u32x4 (&wv)[NH], int pass, int lane,
                                              f32x4 (&acc)[2]) {
#pragma unroll
  for (int i = 0; i < NH; i++) {
    u32x4 xb[8];
    const uint32_t *xp = lds + ((pass * NH + i) * 64 + lane) * ROWS_XCH;
#pragma unroll
    for (int q = 0; q < 8; q++) xb[q] = *reinterpret_cast<const u32x4 *>(xp + 4 * q);
    u32x4 lo[4], hi[4];
    unpack32_kil(wv[i].x, wv[i].y, lo[0], hi[0], lo[1], hi[1]);
    unpack32_kil(wv[i].z, wv[i].w, lo[2], hi[2], lo[3], hi[3]);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      acc[j & 1] = mfma16(lo[j], xb[2 * j], acc[j & 1]);
      acc[j & 1] = mfma16(hi[j], xb[2 * j + 1], acc[j & 1]);
    }
  }
}

template <typename YT>
__device__ __forceinline__ void rows_pass_store(const f32x4 (&acc)[2], float sc, int row, int N, int lane,
                                                YT *__restrict__ Y, const float *__restrict__ bias) {
  const int c = lane & 15, rg = lane >> 4, e = c & 3;
  const f32x4 A = acc[0] + acc[1];
  float v = e == 0 ? A[0] : e == 1 ? A[1] : e == 2 ? A[2] : A[3];
  v = (c >> 2) == rg ? v : 0.f;  // the diagonal
  v += dpp_f32<0xB1>(v);
  v += dpp_f32<0x4E>(v);
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 20));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 40));
  const float f = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 60));
  float t = ((a + b) + (d + f)) * sc * 0.5f;  // 0.5 undoes the 2*dec(c) encoding
  if (lane == 0 && row < N) {
    if (bias) t = add_bias(t, bias[row]);
    if constexpr (sizeof(YT) == 2) Y[row] = (uint16_t)bf16_rne(t);
    else Y[row] = t;
  }
}

template <typename YT, int WAVES, int NH, int NP>
__global__ __launch_bounds__(WAVES * 64) void gemv_rows_pass_kernel(const uint32_t *__restrict__ W,
                                                                    const float *__restrict__ scale,
                                                                    const uint16_t *__restrict__ X,
                                                                    YT *__restrict__ Y, int K, int N,
                                                                    const float *__restrict__ bias) {
  static_assert(NP == 2, "the loop below alternates two register sets over two passes per row");
  extern __shared__ __align__(16) uint32_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kw = K >> 4, nxp = K >> 3;
  const int stride = (int)gridDim.x * WAVES;
  int row = (int)blockIdx.x * WAVES + wave;
  const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(W, (uint32_t)N * (uint32_t)kw * 4u);
  constexpr int NT = WAVES * 64;
  constexpr int PP = NH * NP * 512;
  constexpr int XR = (PP + NT - 1) / NT;
  // activations first (zero past K), then the first row's first pass
  u32x4 xs[XR];
  const u32x4 *X4 = reinterpret_cast<const u32x4 *>(X);
#pragma unroll
  for (int r = 0; r < XR; r++) {
    const int j = tid + r * NT;
    xs[r] = (u32x4){0u, 0u, 0u, 0u};
    if (j < PP && j < nxp) xs[r] = X4[j];
  }
  u32x4 wa[NH], wb[NH];
  rows_pass_load<NH>(wr, min(row, N - 1), 0, row < N, kw, lane, wa);
#pragma unroll
  for (int r = 0; r < XR; r++) {
    const int j = tid + r * NT;
    const u32x4 v = stage_kil(xs[r], tid);  // all lanes take part
    if (j < PP) *reinterpret_cast<u32x4 *>(lds + (j >> 3) * ROWS_XCH + (j & 7) * 4) = v;
  }
  __syncthreads();
  for (; row < N; row += stride) {  // wave-uniform; no barrier below
    const int next = row + stride;
    const float sc = scale[row];
    rows_pass_load<NH>(wr, row, 1, true, kw, lane, wb);
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the decode
    f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    rows_pass_acc<NH>(lds, wa, 0, lane, acc);
    rows_pass_load<NH>(wr, min(next, N - 1), 0, next < N, kw, lane, wa);
    __builtin_amdgcn_sched_barrier(0);
    rows_pass_acc<NH>(lds, wb, 1, lane, acc);
    rows_pass_store<YT>(acc, sc, row, N, lane, Y, bias);
  }
}

static int device_cu_count() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

template <typename YT, int RW, int NI>
static hipError_t launch_gemv_rows_stream(const uint32_t *w, const float *scale, const void *x, void *y, int K,
                                          int N, hipStream_t stream, const float *bias) {
  constexpr int WAVES = 8;
  const int ng = (N + RW - 1) / RW;
  const int grid = std::min((ng + WAVES - 1) / WAVES, 2 * device_cu_count());
  const size_t lds = (size_t)NI * 64 * ROWS_XCH * 4;  // at most 36 KB (NI <= 4)
  hipLaunchKernelGGL((gemv_rows_stream_kernel<YT, WAVES, RW, NI>), dim3(grid), dim3(WAVES * 64), lds, stream, w,
                     scale, reinterpret_cast<const uint16_t *>(x), reinterpret_cast<YT *>(y), K, N, bias);
  return hipGetLastError();
}

template <typename YT, int NH>
static hipError_t launch_gemv_rows_pass(const uint32_t *w, const float *scale, const void *x, void *y, int K, int N,
                                        hipStream_t stream, const float *bias) {
  constexpr int WAVES = 8;
  const int grid = std::min((N + WAVES - 1) / WAVES, 2 * device_cu_count());
  const size_t lds = (size_t)2 * NH * 64 * ROWS_XCH * 4;  // at most 72 KB (NH <= 4)
  if (lds > 64 * 1024) {
    static std::atomic<uint64_t> done;
    const hipError_t e =
        opt_in_lds(reinterpret_cast<const void *>(&gemv_rows_pass_kernel<YT, WAVES, NH, 2>), (int)lds, done);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((gemv_rows_pass_kernel<YT, WAVES, NH, 2>), dim3(grid), dim3(WAVES * 64), lds, stream, w, scale,
                     reinterpret_cast<const uint16_t *>(x), reinterpret_cast<YT *>(y), K, N, bias);
  return hipGetLastError();
}

// ---- 8 to 16 bf16 tokens: activations staged per wave ---------------------
//
// One workgroup per CU owns a contiguous range of rows (T tiles of 16 rows x
// 16 tokens, the M and N sides of v_mfma_f32_16x16x32_bf16) and its waves
// split K into ranges of whole quads (256 columns). A wave stages the x of
// its current quad, all 16 tokens, in its own 8 KB of LDS and computes every
// tile of the workgroup from it, so each CU reads x once and each weight
// word is decoded once. Measured against the per-lane operand loads of
// gemv_direct_kernel / gemv_tall_kernel at B = 16: 12.3 -> 7.5 us
// (11008x4096) and 13.3 -> 9.5 us (4096x11008) per launch.
//  - Staging: load instruction ii of a quad reads tokens 2ii and 2ii+1, 512
//    contiguous bytes each (whole 128-byte lines; the per-lane 32-byte
//    operand loads touched 16 half-used lines per instruction and ran the
//    L2 -> L1 path at half its line rate).
//  - LDS layout: 16-byte slot ((m*2 + h)*64 + g*16 + (t ^ (2g + h))) holds
//    x[t][256Q + 64m + 16g + 8h .. +7]. The XOR spreads both the staging
//    writes (eight consecutive pieces of one token) and the operand reads
//    (eight consecutive tokens of one piece) over distinct bank groups.
//  - Weights: lane (r, g) loads 16 bytes (words 4g..4g+3 of the quad) of row
//    r of each tile, and the 4x4 word transpose of gemv_direct_kernel gives
//    it words g, g+4, g+8, g+12; step m multiplies word 4m + g against the
//    slots (m, h = 0 / 1) of token t = lane % 16.
//  - Tokens >= B and columns >= K are staged as zeros (buffer loads past the
//    range), rows past the workgroup's range read zero words; the waves'
//    partial tiles are added in wave order through LDS (deterministic).
//  - Activation sources (XS): one bf16 plane; two bf16 planes whose sum is
//    the fp32 activation (hi, lo: the decode FFN's intermediate); or fp32,
//    split at staging into such a pair (split2_bf16). Two planes take 16 KB
//    per wave and quad and two MFMAs per operand. Token pairs at or past B
//    are not staged: their LDS slots feed only MFMA columns of tokens that
//    are never stored.
//  - NW = 2 (EPI = GEMV_SWIGLU / GEMV_GEGLU): the gate (W) and up (W2)
//    tiles of the same rows against the same staged x; h = act(g) * u, as
//    fp32 or (YSPLIT) as bf16 hi/lo planes Y = [2][B][N].
constexpr int XS_QUAD_BYTES = 8192;  // one plane of a quad: 16 tokens x 256 bf16
enum { XS_BF16 = 0, XS_PLANES = 1, XS_F32 = 2 };

template <typename YT, int WAVES, int T, int UMAX, int NW, int EPI, int XS, bool YSPLIT>
__global__ __launch_bounds__(WAVES * 64) void gemv_xs_kernel(
    const uint32_t *__restrict__ W, const float *__restrict__ scale, const uint32_t *__restrict__ W2,
    const float *__restrict__ scale2, const void *__restrict__ Xv, const uint16_t *__restrict__ X2,
    YT *__restrict__ Y, int B, int K, int N, const float *__restrict__ bias) {
  static_assert((NW == 2) == (EPI != GEMV_LINEAR), "two matrices exactly for the GLU epilogues");
  static_assert(!YSPLIT || (NW == 2 && sizeof(YT) == 2), "split output is the GLU's bf16 planes");
  constexpr int XP = XS == XS_BF16 ? 1 : 2;  // planes staged per quad
  constexpr int NL = 8 * XP;  // 16-byte loads per lane and quad (fp32: two per piece)
  extern __shared__ __align__(16) uint32_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int b0 = (int)((long long)blockIdx.x * N / gridDim.x);
  const int b1 = (int)((long long)(blockIdx.x + 1) * N / gridDim.x);
  const int wpr = K >> 4;
  const int nq = (K + 255) >> 8;
  const int qa = (wave * nq) / WAVES, qb = ((wave + 1) * nq) / WAVES;
  uint8_t *xl = reinterpret_cast<uint8_t *>(lds) + wave * XP * XS_QUAD_BYTES;
  const uint32_t xbytes = (uint32_t)B * (uint32_t)K * (XS == XS_F32 ? 4u : 2u);
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(Xv, xbytes);
  const __amdgpu_buffer_rsrc_t xr2 = buffer_rsrc(XS == XS_PLANES ? (const void *)X2 : Xv, xbytes);
  const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(W, (uint32_t)N * (uint32_t)wpr * 4u);
  const __amdgpu_buffer_rsrc_t wr2 = buffer_rsrc(NW == 2 ? W2 : W, (uint32_t)N * (uint32_t)wpr * 4u);
  constexpr uint32_t OOB = 0x80000000u;  // a buffer offset past any range this path takes
  const int st = lane >> 5, sp = lane & 31;  // staging: token of the pair, 16-byte bf16 piece
  const int sm = sp >> 3, sg = (sp >> 1) & 3, sh = sp & 1;
  auto xload = [&](int q, u32x4(&xs)[NL]) {
#pragma unroll
    for (int ii = 0; ii < 8; ii++) {
      const int t = 2 * ii + st, col = 256 * q + 8 * sp;
      const bool ok = q < qb && t < B && col < K;
      const uint32_t e = (uint32_t)t * (uint32_t)K + (uint32_t)col;  // element index
      if constexpr (XS == XS_F32) {
        xs[2 * ii] = __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? e * 4u : OOB, 0, 0);
        xs[2 * ii + 1] = __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? e * 4u + 16u : OOB, 0, 0);
      } else {
        xs[ii] = __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? e * 2u : OOB, 0, 0);
        if constexpr (XS == XS_PLANES)
          xs[8 + ii] = __builtin_amdgcn_raw_buffer_load_b128(xr2, ok ? e * 2u : OOB, 0, 0);
      }
    }
  };
  auto xstore = [&](const u32x4(&xs)[NL]) {
#pragma unroll
    for (int ii = 0; ii < 8; ii++) {
      const int ts = 2 * ii + st;
      uint8_t *dst = xl + ((sm * 2 + sh) * 64 + sg * 16 + (ts ^ (2 * sg + sh))) * 16;
      if constexpr (XS == XS_F32) {
        if (2 * ii >= B) continue;  // wave-uniform
        const u32x4 a = xs[2 * ii], b = xs[2 * ii + 1];
        uint32_t hi[4], lo[4];
        split2_bf16(__uint_as_float(a.x), __uint_as_float(a.y), hi[0], lo[0]);
        split2_bf16(__uint_as_float(a.z), __uint_as_float(a.w), hi[1], lo[1]);
        split2_bf16(__uint_as_float(b.x), __uint_as_float(b.y), hi[2], lo[2]);
        split2_bf16(__uint_as_float(b.z), __uint_as_float(b.w), hi[3], lo[3]);
        *reinterpret_cast<u32x4 *>(dst) = (u32x4){hi[0], hi[1], hi[2], hi[3]};
        *reinterpret_cast<u32x4 *>(dst + XS_QUAD_BYTES) = (u32x4){lo[0], lo[1], lo[2], lo[3]};
      } else {
        *reinterpret_cast<u32x4 *>(dst) = xs[ii];
        if constexpr (XS == XS_PLANES) *reinterpret_cast<u32x4 *>(dst + XS_QUAD_BYTES) = xs[8 + ii];
      }
    }
  };
  u32x4 xs[NL];
  xload(qa, xs);  // first, so that it does not wait behind the weights
  u32x4 wv[NW][T][UMAX];
#pragma unroll
  for (int mw = 0; mw < NW; mw++)
#pragma unroll
    for (int tt = 0; tt < T; tt++)
#pragma unroll
      for (int u = 0; u < UMAX; u++) {
        const int row = b0 + 16 * tt + r, q = qa + u, wi = 16 * q + 4 * g;
        const uint32_t off =
            (row < b1 && q < qb && wi < wpr) ? ((uint32_t)row * (uint32_t)wpr + (uint32_t)wi) * 4u : OOB;
        wv[mw][tt][u] = __builtin_amdgcn_raw_buffer_load_b128(mw ? wr2 : wr, off, 0, 0);
      }
  f32x4 acc[NW][T];
#pragma unroll
  for (int mw = 0; mw < NW; mw++)
#pragma unroll
    for (int tt = 0; tt < T; tt++) acc[mw][tt] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const int t = lane & 15;
#pragma unroll
  for (int u = 0; u < UMAX; u++) {
    if (qa + u >= qb) break;  // wave-uniform
    // the wave's own LDS area: its reads of the previous quad precede these
    // writes in the wave's LDS order
    xstore(xs);
    if (u + 1 < UMAX) xload(qa + u + 1, xs);
#pragma unroll
    for (int mw = 0; mw < NW; mw++)
#pragma unroll
      for (int tt = 0; tt < T; tt++) {
        u32x4 &v = wv[mw][tt][u];
        const auto p02 = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
        const auto p13 = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
        const auto p01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
        const auto p23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
        v = (u32x4){p01[0], p01[1], p23[0], p23[1]};
      }
#pragma unroll
    for (int m = 0; m < 4; m++) {
      u32x4 x0[XP], x1[XP];
#pragma unroll
      for (int p = 0; p < XP; p++) {
        x0[p] = *reinterpret_cast<const u32x4 *>(xl + p * XS_QUAD_BYTES + ((m * 2) * 64 + g * 16 + (t ^ (2 * g))) * 16);
        x1[p] = *reinterpret_cast<const u32x4 *>(xl + p * XS_QUAD_BYTES +
                                                 ((m * 2 + 1) * 64 + g * 16 + (t ^ (2 * g + 1))) * 16);
      }
#pragma unroll
      for (int mw = 0; mw < NW; mw++)
#pragma unroll
        for (int tt = 0; tt < T; tt++) {
          const u32x4 &v = wv[mw][tt][u];
          const uint32_t wq = m == 0 ? v.x : m == 1 ? v.y : m == 2 ? v.z : v.w;
          u32x4 a0, a1;
          unpack16_nat(wq, a0, a1);
#pragma unroll
          for (int p = 0; p < XP; p++) {
            acc[mw][tt] = mfma16(a0, x0[p], acc[mw][tt]);
            acc[mw][tt] = mfma16(a1, x1[p], acc[mw][tt]);
          }
        }
    }
  }
  // Partial tiles, added in wave order; wave tt finishes tile tt.
  __syncthreads();
  f32x4 *red = reinterpret_cast<f32x4 *>(lds);
#pragma unroll
  for (int mw = 0; mw < NW; mw++)
#pragma unroll
    for (int tt = 0; tt < T; tt++) red[((mw * T + tt) * WAVES + wave) * 64 + lane] = acc[mw][tt];
  __syncthreads();
  if (wave < T) {
    const int tt = wave;
    const int n_out = b0 + 16 * tt + 4 * g;  // rows 4g..4g+3 of token t
    if (t < B && n_out < b1) {
      const int nok = min(4, b1 - n_out);
      f32x4 v[NW];
#pragma unroll
      for (int mw = 0; mw < NW; mw++) {
        const f32x4 *rp = red + (mw * T + tt) * WAVES * 64 + lane;
        f32x4 s = rp[0];
        for (int w = 1; w < WAVES; w++) s += rp[w * 64];
        const float *sp2 = mw ? scale2 : scale;
        const f32x4 sc = {sp2[n_out], nok > 1 ? sp2[n_out + 1] : 0.f, nok > 2 ? sp2[n_out + 2] : 0.f,
                          nok > 3 ? sp2[n_out + 3] : 0.f};
        v[mw] = s * sc * 0.5f;  // 0.5: the 2*dec(c) operand encoding
      }
      f32x4 o = v[0];
      if constexpr (NW == 2) {
#pragma unroll
        for (int j = 0; j < 4; j++) o[j] = (EPI == GEMV_GEGLU ? act_gelu_tanh(v[0][j]) : act_silu(v[0][j])) * v[1][j];
      }
      if constexpr (YSPLIT) {
        f32x4 hi, lo;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          hi[j] = bf16_to_f32(bf16_rne(o[j]));
          lo[j] = (__float_as_uint(hi[j]) & 0x7F800000u) == 0x7F800000u ? 0.0f : o[j] - hi[j];
        }
        YStore<uint16_t>::store4(reinterpret_cast<uint16_t *>(Y) + (size_t)t * N + n_out, hi, nok);
        YStore<uint16_t>::store4(reinterpret_cast<uint16_t *>(Y) + (size_t)B * N + (size_t)t * N + n_out, lo, nok);
      } else {
        if constexpr (NW == 1)
          if (bias) o = add_bias4(o, bias, n_out, N);
        YStore<YT>::store4(Y + (size_t)t * N + n_out, o, nok);
      }
    }
  }
}

template <typename YT, int WAVES, int T, int UMAX, int NW, int EPI, int XS, bool YSPLIT>
static hipError_t launch_gemv_xs_w(const uint32_t *w, const float *scale, const uint32_t *w2, const float *scale2,
                                   const void *x, const void *x2, void *y, int B, int K, int N, int G,
                                   hipStream_t stream, const float *bias) {
  constexpr int XP = XS == XS_BF16 ? 1 : 2;
  static_assert(NW * T * 1024 <= XP * XS_QUAD_BYTES, "the partial tiles reuse the staging area");
  const size_t lds = (size_t)WAVES * XP * XS_QUAD_BYTES;
  if (lds > 64 * 1024) {
    static std::atomic<uint64_t> done;
    const hipError_t e = opt_in_lds(
        reinterpret_cast<const void *>(&gemv_xs_kernel<YT, WAVES, T, UMAX, NW, EPI, XS, YSPLIT>), (int)lds, done);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((gemv_xs_kernel<YT, WAVES, T, UMAX, NW, EPI, XS, YSPLIT>), dim3(G), dim3(WAVES * 64), lds,
                     stream, w, scale, w2, scale2, x, reinterpret_cast<const uint16_t *>(x2),
                     reinterpret_cast<YT *>(y), B, K, N, bias);
  return hipGetLastError();
}

// Shapes gemv_xs_kernel takes: up to 16 tokens, K up to 64 quads (16384; 48
// with two planes or two matrices), 16-byte aligned activations.
static bool gemv_xs_ok(const void *x, int B, int K, int XP, int NW) {
  const int nq = (K + 255) / 256;
  return B >= 1 && B <= 16 && nq <= (XP == 1 && NW == 1 ? 64 : 48) && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
}

// Grid: one workgroup per CU, fewer where that would leave tiles of fewer
// than 16 rows, more where a workgroup would hold more tiles than its
// weight registers allow (tiles x quads per wave x matrices <= 8).
static int gemv_xs_grid(int N, int tmax) {
  int G = std::min(device_cu_count(), (N + 15) / 16);
  if ((N + G - 1) / G > 16 * tmax) G = (N + 16 * tmax - 1) / (16 * tmax);
  return G;
}

// Waves and quads per wave. One plane and one matrix: 16 waves of one quad
// (K <= 4096) or two (8192); 12 waves of up to four quads (K <= 12288;
// measured 9.5 us against 10.0 us with 16 waves of three quads at
// 4096x11008, B = 16); 16 waves of four above. Two planes (16 KB per wave)
// or two matrices (twice the weight registers): 8 waves of up to 2, 4 or 6
// quads, so that a wave has 256 registers.
template <typename YT, int NW, int EPI, int XS, bool YSPLIT>
static hipError_t launch_gemv_xs(const uint32_t *w, const float *scale, const uint32_t *w2, const float *scale2,
                                 const void *x, const void *x2, void *y, int B, int K, int N, hipStream_t stream,
                                 const float *bias = nullptr) {
  const int nq = (K + 255) / 256;
#define FRX_XS(WV, TT, UM)                                                                                    \
  return launch_gemv_xs_w<YT, WV, TT, UM, NW, EPI, XS, YSPLIT>(w, scale, w2, scale2, x, x2, y, B, K, N, \
                                                                gemv_xs_grid(N, TT), stream, bias)
#define FRX_XS_T(WV, UM, TMAX)                                                               \
  {                                                                                          \
    const int tiles = ((N + gemv_xs_grid(N, TMAX) - 1) / gemv_xs_grid(N, TMAX) + 15) / 16; \
    if (tiles <= 1 || TMAX == 1) FRX_XS(WV, 1, UM);                                          \
    if (tiles <= 2 || TMAX == 2) FRX_XS(WV, (TMAX >= 2 ? 2 : 1), UM);                        \
    if (tiles <= 3 || TMAX == 3) FRX_XS(WV, (TMAX >= 3 ? 3 : 1), UM);                        \
    FRX_XS(WV, (TMAX >= 4 ? 4 : 1), UM);                                                     \
  }
  if constexpr (XS == XS_BF16 && NW == 1) {
    if (nq <= 16) FRX_XS_T(16, 1, 4);
    if (nq <= 32) FRX_XS_T(16, 2, 4);
    if (nq <= 48) FRX_XS_T(12, 4, 2);
    FRX_XS_T(16, 4, 2);
  } else if constexpr (NW == 1) {
    if (nq <= 16) FRX_XS_T(8, 2, 4);
    if (nq <= 32) FRX_XS_T(8, 4, 2);
    FRX_XS_T(8, 6, 1);
  } else {
    if (nq <= 16) FRX_XS_T(8, 2, 2);
    if (nq <= 32) FRX_XS_T(8, 4, 1);
    FRX_XS_T(8, 6, 1);
  }
#undef FRX_XS_T
#undef FRX_XS
}

// ---- two to four bf16 tokens: four rows x four segments per MFMA ----------
//
// The same diagonal idea with the 16 MFMA rows as 4 rows x 4 segments and
// the 16 columns as 4 tokens x 4 segments: lane (a*4 + s, g) loads 16 bytes
// at (4g + s) * 16 of row a's 256-byte window (a wave instruction covers 4
// rows x 256 B, whole lines), and lane (t*4 + s, g) feeds token t's
// activations at the same positions. C[(a,s)][(t,s')] is wanted for s = s'
// only, which is register col%4 of lane (col, rg) with a = rg, t = col/4:
// a quad sum gives y[t][row a] in a fixed order. A wave holds RW groups of
// 4 rows; the workgroup stages all B activation rows in LDS (chunks of 64
// values padded to 144 bytes, token rows 16 dwords apart modulo the 64
// banks, so the 16 lanes of a read phase hit disjoint banks; tokens >= B
// read a zero block). Measured over rotating weights at B = 4: 6.41 ->
// 5.78 us (11008x4096) and 6.76 -> 5.93 us (4096x11008) per launch against
// the 16-row tiles.
// KS = 2: the windows of each row group are split between two waves (the
// first and second halves of K), so a workgroup whose LDS holds long token
// rows still has two waves per SIMD; the second wave's partial tile goes
// through LDS and is added to the first's in that order.
// NW = 2 (EPI = GEMV_SWIGLU / GEMV_GEGLU): gate (W) and up (W2) groups of
// the same rows against the same tokens; h = act(g) * u is written as bf16
// hi and lo planes (Y = [2][B][N]). VPL (B = 2): X holds the hi and lo
// planes of two tokens ([2][2][K]), staged as four token rows; the hi and
// lo results of a token (quads t and t + 2 of a lane row) are added by one
// DPP rotation.
template <typename YT, int WAVES, int RW, int NI, int KS = 1, int NW = 1, int EPI = GEMV_LINEAR, bool VPL = false>
__global__ __launch_bounds__(WAVES * 64) void gemv_rows4_kernel(
    const uint32_t *__restrict__ W, const float *__restrict__ scale, const uint32_t *__restrict__ W2,
    const float *__restrict__ scale2, const uint16_t *__restrict__ X, YT *__restrict__ Y, int B, int K, int N,
    const float *__restrict__ bias) {
  static_assert((NW == 2) == (EPI != GEMV_LINEAR), "two matrices exactly for the GLU epilogues");
  static_assert(!(VPL && NW == 2), "planes feed the linear epilogue");
  extern __shared__ __align__(16) uint32_t lds[];
  constexpr int NCH = NI * 16;             // 64-value chunks per token
  constexpr int TS = NCH * ROWS_XCH + 16;  // token stride (dwords)
  constexpr int NT = WAVES * 64;
  constexpr int PPT = NI * 128;            // staged 16-byte pieces per token
  constexpr int XR = (4 * PPT + NT - 1) / NT;
  constexpr int GW = WAVES / KS;            // waves per K part
  constexpr int NIP = (NI + KS - 1) / KS;   // windows per K part
  static_assert(WAVES % KS == 0, "K parts split the waves evenly");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int part = wave / GW, wg = wave - part * GW;
  const int grp0 = ((int)blockIdx.x * GW + wg) * RW;  // first 4-row group of the wave
  const int kw = K >> 4;
  const int nxp = K >> 3;  // 16-byte pieces per activation row
  const int BS = VPL ? 2 * B : B;  // staged token rows
  // 1. activations of the B tokens (zero past K and for tokens >= B)
  u32x4 xs[XR];
  const u32x4 *X4 = reinterpret_cast<const u32x4 *>(X);
#pragma unroll
  for (int r = 0; r < XR; r++) {
    const int j = tid + r * NT, t = j / PPT, p = j - t * PPT;
    xs[r] = (u32x4){0u, 0u, 0u, 0u};
    if (t < BS && p < nxp) xs[r] = X4[(size_t)t * nxp + p];
  }
  // 2. weights: lane (a, s, g) of group G reads row 4G + a at (4g + s) * 16
  //    bytes into each 256-byte window (clamped inside the row)
  const int a = (lane & 15) >> 2, s = lane & 3, g = lane >> 4;
  u32x4 wv[NW][RW][NIP];
  float sc[NW][RW];
#pragma unroll
  for (int m = 0; m < NW; m++)
#pragma unroll
    for (int rr = 0; rr < RW; rr++) {
      const uint32_t *wr = (m ? W2 : W) + (size_t)min((grp0 + rr) * 4 + a, N - 1) * kw;
#pragma unroll
      for (int i = 0; i < NIP; i++) {
        const int win = min(part * NIP + i, NI - 1);  // a window past NI is loaded, never used
        wv[m][rr][i] = *reinterpret_cast<const u32x4 *>(wr + min(win * 64 + (g * 4 + s) * 4, kw - 4));
      }
      sc[m][rr] = (m ? scale2 : scale)[min((grp0 + rr) * 4 + g, N - 1)];  // the row this lane's sum lands on
    }
  // 3. stage: token t, piece p -> chunk p/8 slot p%8; zero block after the tokens
#pragma unroll
  for (int r = 0; r < XR; r++) {
    const int j = tid + r * NT, t = j / PPT, p = j - t * PPT;
    if (t < 4) *reinterpret_cast<u32x4 *>(lds + t * TS + (p >> 3) * ROWS_XCH + (p & 7) * 4) = xs[r];
  }
  if (tid < 8) reinterpret_cast<u32x4 *>(lds + 4 * TS)[tid] = (u32x4){0u, 0u, 0u, 0u};
  __syncthreads();
  // 4. per window: this lane's 64 activations of token col/4, then the words
  const int tcol = (lane & 15) >> 2, scol = lane & 3;
  const bool live = tcol < BS;
  f32x4 acc[NW][RW];
#pragma unroll
  for (int m = 0; m < NW; m++)
#pragma unroll
    for (int rr = 0; rr < RW; rr++) acc[m][rr] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NIP; i++) {
    const int win = part * NIP + i;
    if (win >= NI) continue;  // wave-uniform: the last part's missing windows
    u32x4 xb[8];
    const uint32_t *xp = live ? lds + tcol * TS + (win * 16 + g * 4 + scol) * ROWS_XCH : lds + 4 * TS;
#pragma unroll
    for (int q = 0; q < 8; q++) xb[q] = *reinterpret_cast<const u32x4 *>(xp + (live ? 4 * q : 4 * (q & 1)));
#pragma unroll
    for (int m = 0; m < NW; m++)
#pragma unroll
      for (int rr = 0; rr < RW; rr++) {
        const uint32_t wq[4] = {wv[m][rr][i].x, wv[m][rr][i].y, wv[m][rr][i].z, wv[m][rr][i].w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
          u32x4 lo, hi;
          unpack16_nat(wq[j], lo, hi);
          acc[m][rr] = mfma16(lo, xb[2 * j], acc[m][rr]);
          acc[m][rr] = mfma16(hi, xb[2 * j + 1], acc[m][rr]);
        }
      }
  }
  if constexpr (KS > 1) {
    // second-half partials through LDS (after the zero block), added in order
    f32x4 *cb = reinterpret_cast<f32x4 *>(lds + 4 * TS + 32);
    if (part == 1) {
#pragma unroll
      for (int m = 0; m < NW; m++)
#pragma unroll
        for (int rr = 0; rr < RW; rr++) cb[((wg * NW + m) * RW + rr) * 64 + lane] = acc[m][rr];
    }
    __syncthreads();
    if (part != 0) return;
#pragma unroll
    for (int m = 0; m < NW; m++)
#pragma unroll
      for (int rr = 0; rr < RW; rr++) acc[m][rr] = acc[m][rr] + cb[((wg * NW + m) * RW + rr) * 64 + lane];
  }
  // 5. lane (col, rg) register e holds C[(a=rg, s=e)][(t=col/4, s'=col%4)]
  const int e = lane & 3;
#pragma unroll
  for (int rr = 0; rr < RW; rr++) {
    float v[NW];
#pragma unroll
    for (int m = 0; m < NW; m++) {
      const f32x4 A = acc[m][rr];
      v[m] = e == 0 ? A[0] : e == 1 ? A[1] : e == 2 ? A[2] : A[3];
      v[m] += dpp_f32<0xB1>(v[m]);  // quad_perm [1,0,3,2]
      v[m] += dpp_f32<0x4E>(v[m]);  // quad_perm [2,3,0,1]
      if constexpr (VPL) v[m] += dpp_f32<0x128>(v[m]);  // row_ror:8: token t's hi + lo
    }
    const int row = (grp0 + rr) * 4 + g;
    if (e == 0 && tcol < B && row < N) {
      if constexpr (EPI != GEMV_LINEAR) {
        const float gv = v[0] * sc[0][rr] * 0.5f, uv = v[1] * sc[1][rr] * 0.5f;
        const float h = (EPI == GEMV_GEGLU ? act_gelu_tanh(gv) : act_silu(gv)) * uv;
        uint32_t hh, hl;
        split_bf16(h, hh, hl);
        Y[(size_t)tcol * N + row] = (uint16_t)hh;
        Y[(size_t)(B + tcol) * N + row] = (uint16_t)hl;
      } else {
        float yv = v[0] * sc[0][rr] * 0.5f;
        if (bias) yv = add_bias(yv, bias[row]);
        if constexpr (sizeof(YT) == 2) Y[(size_t)tcol * N + row] = (uint16_t)bf16_rne(yv);
        else Y[(size_t)tcol * N + row] = yv;
      }
    }
  }
}

template <typename YT, int WAVES, int RW, int NI, int KS = 1, int NW = 1, int EPI = GEMV_LINEAR, bool VPL = false>
static hipError_t launch_gemv_rows4_w(const uint32_t *w, const float *scale, const uint32_t *w2,
                                      const float *scale2, const void *x, void *y, int B, int K, int N,
                                      hipStream_t stream, const float *bias = nullptr) {
  constexpr int GW = WAVES / KS;
  const dim3 grid((N + GW * RW * 4 - 1) / (GW * RW * 4));
  const size_t lds =
      ((size_t)4 * (NI * 16 * ROWS_XCH + 16) + 32) * 4 + (KS > 1 ? (size_t)GW * NW * RW * 64 * 16 : 0);
  if (lds > 64 * 1024) {
    static std::atomic<uint64_t> done;
    const hipError_t e = opt_in_lds(
        reinterpret_cast<const void *>(&gemv_rows4_kernel<YT, WAVES, RW, NI, KS, NW, EPI, VPL>), (int)lds, done);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((gemv_rows4_kernel<YT, WAVES, RW, NI, KS, NW, EPI, VPL>), grid, dim3(WAVES * 64), lds, stream,
                     w, scale, w2, scale2, reinterpret_cast<const uint16_t *>(x), reinterpret_cast<YT *>(y), B, K,
                     N, bias);
  return hipGetLastError();
}

// 2 <= B <= 4 bf16 tokens, K % 64 == 0 and K <= 14336 (four token rows in
// LDS), 16-byte aligned weights and activations. Window counts round up to
// the instantiated ones (extra windows hold zero activations).
static bool gemv_rows4_ok(const uint32_t *w, const void *x, int B, int K) {
  return B >= 2 && B <= 4 && K % 64 == 0 && K <= 14336 && (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(x) & 15) == 0;
}


template <typename YT>
static hipError_t launch_gemv_rows4(const uint32_t *w, const float *scale, const void *x, void *y, int B, int K,
                                    int N, hipStream_t stream, const float *bias) {
  const int ni = (K + 1023) / 1024;
  // one 4-row group per wave and (above one window) each group's windows
  // split over two waves: 8 waves, 16 or 32 rows per workgroup, so N = 11008
  // gives 688 workgroups instead of 172 (11008x4096 at B = 4: 6.8 -> 6.0 us
  // per launch; 4096x11008: 7.04 -> 6.48 us against 4 waves of one group)
  if (ni <= 1) return launch_gemv_rows4_w<YT, 8, 1, 1>(w, scale, w, scale, x, y, B, K, N, stream, bias);
  if (ni <= 2) return launch_gemv_rows4_w<YT, 8, 1, 2, 2>(w, scale, w, scale, x, y, B, K, N, stream, bias);
  if (ni <= 4) return launch_gemv_rows4_w<YT, 8, 1, 4, 2>(w, scale, w, scale, x, y, B, K, N, stream, bias);
  // 5120 and 6144 columns (LLaMA-13B-sized rows) without rounding up to 8
  // windows of loads
  if (ni <= 5) return launch_gemv_rows4_w<YT, 8, 1, 5, 2>(w, scale, w, scale, x, y, B, K, N, stream, bias);
  if (ni <= 6) return launch_gemv_rows4_w<YT, 8, 1, 6, 2>(w, scale, w, scale, x, y, B, K, N, stream, bias);
  if (ni <= 8) return launch_gemv_rows4_w<YT, 8, 1, 8, 2>(w, scale, w, scale, x, y, B, K, N, stream, bias);
  if (ni <= 11) return launch_gemv_rows4_w<YT, 8, 1, 11, 2>(w, scale, w, scale, x, y, B, K, N, stream, bias);
  return launch_gemv_rows4_w<YT, 8, 1, 14, 2>(w, scale, w, scale, x, y, B, K, N, stream, bias);
}

// Decode FFN of two bf16 tokens through the 4-segment kernels: gate/up/act
// into hi/lo planes of h ([2][2][N]), then the down rows with the planes as
// four token columns (H and I multiples of 64 up to 14336).
bool gemv_rows4_ffn_ok(int M, int H, int I) {
  return M == 2 && H % 64 == 0 && I % 64 == 0 && H <= 14336 && I <= 14336;
}

hipError_t launch_gemv_rows4_glu_planes(const uint32_t *w_gate, const float *s_gate, const uint32_t *w_up,
                                        const float *s_up, const void *x, uint16_t *h_planes, int B, int K, int N,
                                        int gelu, hipStream_t stream) {
  const int ni = (K + 1023) / 1024;
#define FRX_R4_GLU(NI, KS)                                                                                      \
  return gelu ? launch_gemv_rows4_w<uint16_t, 8, 1, NI, KS, 2, GEMV_GEGLU>(w_gate, s_gate, w_up, s_up, x,      \
                                                                           h_planes, B, K, N, stream)         \
              : launch_gemv_rows4_w<uint16_t, 8, 1, NI, KS, 2, GEMV_SWIGLU>(w_gate, s_gate, w_up, s_up, x,     \
                                                                            h_planes, B, K, N, stream)
  if (ni <= 1) FRX_R4_GLU(1, 1);
  if (ni <= 2) FRX_R4_GLU(2, 2);
  if (ni <= 4) FRX_R4_GLU(4, 2);
  if (ni <= 8) FRX_R4_GLU(8, 2);
  if (ni <= 11) FRX_R4_GLU(11, 2);
  FRX_R4_GLU(14, 2);
#undef FRX_R4_GLU
}

hipError_t launch_gemv_rows4_planes(const uint32_t *w, const float *scale, const uint16_t *x_planes, void *y,
                                    int yt_bf16, int K, int N, hipStream_t stream) {
  const int ni = (K + 1023) / 1024;
#define FRX_R4_PL(NI, KS)                                                                                         \
  return yt_bf16                                                                                                  \
             ? launch_gemv_rows4_w<uint16_t, 8, 1, NI, KS, 1, GEMV_LINEAR, true>(w, scale, w, scale, x_planes, y, \
                                                                                 2, K, N, stream)                 \
             : launch_gemv_rows4_w<float, 8, 1, NI, KS, 1, GEMV_LINEAR, true>(w, scale, w, scale, x_planes, y, 2, \
                                                                              K, N, stream)
  if (ni <= 1) FRX_R4_PL(1, 1);
  if (ni <= 2) FRX_R4_PL(2, 2);
  if (ni <= 4) FRX_R4_PL(4, 2);
  if (ni <= 8) FRX_R4_PL(8, 2);
  if (ni <= 11) FRX_R4_PL(11, 2);
  FRX_R4_PL(14, 2);
#undef FRX_R4_PL
}

// One bf16 token, K % 64 == 0, K <= 16384, 16-byte aligned weights and
// activations; two rows per wave where a row is one window (x read once per
// two rows), one row per wave above (registers).
static bool gemv_rows_ok(const uint32_t *w, const void *x, int B, int K) {
  return B == 1 && K % 64 == 0 && K <= 4 * 4096 && (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(x) & 15) == 0;
}

constexpr int GEMV_ROWS_TALL_N = 16384;  // rows from which waves persist over row groups above 4096 codes

// One bf16 token over rows of 16448 to 32768 codes (K % 64 == 0, aligned),
// weights addressable by 32-bit buffer offsets: the two-pass persistent
// kernel.
static bool gemv_rows_pass_ok(const uint32_t *w, const void *x, int B, int K, int N) {
  return B == 1 && K % 64 == 0 && K > 4 * 4096 && K <= 8 * 4096 && (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (size_t)N * (size_t)K / 4 < (size_t)ROWS_STREAM_OOB;
}

template <typename YT>
static hipError_t launch_gemv_rows(const uint32_t *w, const float *scale, const void *x, void *y, int K, int N,
                                   hipStream_t stream, const float *bias) {
  const int ni = (K + 4095) / 4096;
  if (ni == 1) return launch_gemv_rows_w<YT, 2, 1>(w, scale, w, scale, x, x, y, K, N, stream, bias);
  // Tall matrices (more rows than one residency pass holds at one row per
  // wave: 4 workgroups x 8 waves per CU), above one window per row.
  if (N >= GEMV_ROWS_TALL_N) {
    // persistent waves; buffer offsets are 32-bit with the out-of-range
    // marker above every weight byte
    if ((size_t)N * (size_t)K / 4 < (size_t)ROWS_STREAM_OOB) {
      if (ni == 2) return launch_gemv_rows_stream<YT, 2, 2>(w, scale, x, y, K, N, stream, bias);
      if (ni == 3) return launch_gemv_rows_stream<YT, 1, 3>(w, scale, x, y, K, N, stream, bias);
      return launch_gemv_rows_stream<YT, 1, 4>(w, scale, x, y, K, N, stream, bias);
    }
    if (ni == 2) return launch_gemv_rows_w<YT, 2, 2>(w, scale, w, scale, x, x, y, K, N, stream, bias);
    if (ni == 3) return launch_gemv_rows_w<YT, 2, 3>(w, scale, w, scale, x, x, y, K, N, stream, bias);
    return launch_gemv_rows_w<YT, 2, 4>(w, scale, w, scale, x, x, y, K, N, stream, bias);
  }
  if (ni == 2) return launch_gemv_rows_w<YT, 1, 2>(w, scale, w, scale, x, x, y, K, N, stream, bias);
  if (ni == 3) return launch_gemv_rows_w<YT, 1, 3>(w, scale, w, scale, x, x, y, K, N, stream, bias);
  return launch_gemv_rows_w<YT, 1, 4>(w, scale, w, scale, x, x, y, K, N, stream, bias);
}

// Decode FFN of one bf16 token through the rows kernels: gate/up/act into
// hi/lo planes of h, then the down rows over both planes.
bool gemv_rows_ffn_ok(int M, int H, int I) {
  return M == 1 && H % 64 == 0 && I % 64 == 0 && H <= 4 * 4096 && I <= 4 * 4096;
}

// The two FFN launches on the balanced one-token kernel (rows split evenly
// over one or two workgroups per CU): GLU into h planes, down over them.
template <typename YT, int NI, bool XPLN, int NW, int EPI>
static hipError_t launch_gemv_bal_ffn_r(const uint32_t *w, const float *scale, const uint32_t *w2,
                                        const float *scale2, const void *x, void *y, int K, int N, int G,
                                        hipStream_t stream) {
  const int rmax = ((N + G - 1) / G + 7) / 8;
#define FRX_BAL_FFN(R) \
  return launch_gemv_bal_w<YT, NI, R, false, XPLN, NW, EPI>(w, scale, x, y, K, N, G, stream, nullptr, w2, scale2)
  if (rmax <= 1) FRX_BAL_FFN(1);
  if (rmax <= 2) FRX_BAL_FFN(2);
  if (rmax <= 3) FRX_BAL_FFN(3);
  FRX_BAL_FFN(4);
#undef FRX_BAL_FFN
}

template <typename YT, bool XPLN, int NW, int EPI>
static hipError_t launch_gemv_bal_ffn(const uint32_t *w, const float *scale, const uint32_t *w2, const float *scale2,
                                      const void *x, void *y, int K, int N, int G, hipStream_t stream) {
  const int ni = (K + 4095) / 4096;
  if (ni == 1) return launch_gemv_bal_ffn_r<YT, 1, XPLN, NW, EPI>(w, scale, w2, scale2, x, y, K, N, G, stream);
  if (ni == 2) return launch_gemv_bal_ffn_r<YT, 2, XPLN, NW, EPI>(w, scale, w2, scale2, x, y, K, N, G, stream);
  if (ni == 3) return launch_gemv_bal_ffn_r<YT, 3, XPLN, NW, EPI>(w, scale, w2, scale2, x, y, K, N, G, stream);
  // two matrices of four windows per row would spill (callers stop at three)
  if constexpr (NW == 2) return hipErrorInvalidValue;
  else return launch_gemv_bal_ffn_r<YT, 4, XPLN, NW, EPI>(w, scale, w2, scale2, x, y, K, N, G, stream);
}

hipError_t launch_gemv_rows_glu_planes(const uint32_t *w_gate, const float *s_gate, const uint32_t *w_up,
                                       const float *s_up, const void *x, uint16_t *h_planes, int K, int N,
                                       int gelu, hipStream_t stream) {
  int G = 0;
  if (K <= 3 * 4096 && gemv_bal_grid(w_gate, x, 1, K, N, &G) && (reinterpret_cast<uintptr_t>(w_up) & 15) == 0) {
    if (gelu)
      return launch_gemv_bal_ffn<uint16_t, false, 2, GEMV_GEGLU>(w_gate, s_gate, w_up, s_up, x, h_planes, K, N, G,
                                                                 stream);
    return launch_gemv_bal_ffn<uint16_t, false, 2, GEMV_SWIGLU>(w_gate, s_gate, w_up, s_up, x, h_planes, K, N, G,
                                                                stream);
  }
  const int ni = (K + 4095) / 4096;
#define FRX_ROWS_GLU(NI)                                                                                        \
  return gelu ? launch_gemv_rows_w<uint16_t, 1, NI, 2, 1, GEMV_GEGLU>(w_gate, s_gate, w_up, s_up, x, x, h_planes, \
                                                                      K, N, stream)                           \
              : launch_gemv_rows_w<uint16_t, 1, NI, 2, 1, GEMV_SWIGLU>(w_gate, s_gate, w_up, s_up, x, x,      \
                                                                       h_planes, K, N, stream)
  if (ni == 1) FRX_ROWS_GLU(1);
  if (ni == 2) FRX_ROWS_GLU(2);
  if (ni == 3) FRX_ROWS_GLU(3);
  FRX_ROWS_GLU(4);
#undef FRX_ROWS_GLU
}

hipError_t launch_gemv_rows_planes(const uint32_t *w, const float *scale, const uint16_t *x_planes, void *y,
                                   int yt_bf16, int K, int N, hipStream_t stream) {
  int G = 0;
  if (gemv_bal_grid(w, x_planes, 1, K, N, &G) && (K * 2) % 16 == 0) {  // the lo plane 16-byte aligned too
    if (yt_bf16)
      return launch_gemv_bal_ffn<uint16_t, true, 1, GEMV_LINEAR>(w, scale, nullptr, nullptr, x_planes, y, K, N, G,
                                                                 stream);
    return launch_gemv_bal_ffn<float, true, 1, GEMV_LINEAR>(w, scale, nullptr, nullptr, x_planes, y, K, N, G, stream);
  }
  const int ni = (K + 4095) / 4096;
  const uint16_t *lo = x_planes + K;
#define FRX_ROWS_PL(RW, NI)                                                                                   \
  return yt_bf16 ? launch_gemv_rows_w<uint16_t, RW, NI, 1, 2>(w, scale, w, scale, x_planes, lo, y, K, N, stream) \
                 : launch_gemv_rows_w<float, RW, NI, 1, 2>(w, scale, w, scale, x_planes, lo, y, K, N, stream)
  if (ni == 1) FRX_ROWS_PL(2, 1);
  if (ni == 2) FRX_ROWS_PL(1, 2);
  if (ni == 3) FRX_ROWS_PL(1, 3);
  FRX_ROWS_PL(1, 4);
#undef FRX_ROWS_PL
}

hipError_t launch_gemv(const uint32_t *w, const float *scale, const void *x,
                       int xt_bf16, void *y, int yt_bf16, int B, int K, int N,
                       hipStream_t stream, const float *bias) {
  constexpr int L = GEMV_LINEAR;
  int G = 0;
  if (gemv_bal_grid(w, x, B, K, N, &G)) {
    if (xt_bf16) {
      if (yt_bf16) return launch_gemv_bal<uint16_t, false>(w, scale, x, y, K, N, G, stream, bias);
      return launch_gemv_bal<float, false>(w, scale, x, y, K, N, G, stream, bias);
    }
    if (yt_bf16) return launch_gemv_bal<uint16_t, true>(w, scale, x, y, K, N, G, stream, bias);
    return launch_gemv_bal<float, true>(w, scale, x, y, K, N, G, stream, bias);
  }
  if (xt_bf16 && gemv_rows_ok(w, x, B, K)) {
    if (yt_bf16) return launch_gemv_rows<uint16_t>(w, scale, x, y, K, N, stream, bias);
    return launch_gemv_rows<float>(w, scale, x, y, K, N, stream, bias);
  }
  if (xt_bf16 && gemv_rows_pass_ok(w, x, B, K, N)) {
    const bool four = K > 6 * 4096;  // windows per pass: 3 up to 24576 columns, else 4
    if (yt_bf16)
      return four ? launch_gemv_rows_pass<uint16_t, 4>(w, scale, x, y, K, N, stream, bias)
                  : launch_gemv_rows_pass<uint16_t, 3>(w, scale, x, y, K, N, stream, bias);
    return four ? launch_gemv_rows_pass<float, 4>(w, scale, x, y, K, N, stream, bias)
                : launch_gemv_rows_pass<float, 3>(w, scale, x, y, K, N, stream, bias);
  }
  if (xt_bf16 && gemv_rows4_ok(w, x, B, K)) {
    if (yt_bf16) return launch_gemv_rows4<uint16_t>(w, scale, x, y, B, K, N, stream, bias);
    return launch_gemv_rows4<float>(w, scale, x, y, B, K, N, stream, bias);
  }
  if (xt_bf16 && B >= GEMV_XS_MIN_B && gemv_xs_ok(x, B, K, 1, 1)) {
    if (yt_bf16) return launch_gemv_xs<uint16_t, 1, L, XS_BF16, false>(w, scale, w, scale, x, x, y, B, K, N, stream, bias);
    return launch_gemv_xs<float, 1, L, XS_BF16, false>(w, scale, w, scale, x, x, y, B, K, N, stream, bias);
  }
  if (xt_bf16 && B >= GEMV_DIRECT_MIN_B) {
    // taller tiles where their grid still covers every CU
    static std::atomic<int> cus{0};
    int c = cus.load(std::memory_order_relaxed);
    if (c == 0) {
      int dev = 0;
      if (hipGetDevice(&dev) != hipSuccess ||
          hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
        c = 256;
      cus.store(c, std::memory_order_relaxed);
    }
    if ((N + 16 * GEMV_TALL_RS - 1) / (16 * GEMV_TALL_RS) >= c) {
      if (yt_bf16) return launch_gemv_tall<uint16_t>(w, scale, x, y, B, K, N, stream, bias);
      return launch_gemv_tall<float>(w, scale, x, y, B, K, N, stream, bias);
    }
    if (yt_bf16) return launch_gemv_direct<uint16_t, L>(w, scale, w, scale, x, x, y, B, K, N, stream, bias);
    return launch_gemv_direct<float, L>(w, scale, w, scale, x, x, y, B, K, N, stream, bias);
  }
  if (xt_bf16) {
    if (yt_bf16) return launch_gemv_t<uint16_t, uint16_t, L>(w, scale, w, scale, x, y, B, K, N, stream, bias);
    return launch_gemv_t<uint16_t, float, L>(w, scale, w, scale, x, y, B, K, N, stream, bias);
  }
  if (gemv_xs_ok(x, B, K, 2, 1)) {  // fp32 x, 2 to 16 tokens: staged as bf16 hi/lo planes
    if (yt_bf16) return launch_gemv_xs<uint16_t, 1, L, XS_F32, false>(w, scale, w, scale, x, x, y, B, K, N, stream, bias);
    return launch_gemv_xs<float, 1, L, XS_F32, false>(w, scale, w, scale, x, x, y, B, K, N, stream, bias);
  }
  if (yt_bf16) return launch_gemv_t<float, uint16_t, L>(w, scale, w, scale, x, y, B, K, N, stream, bias);
  return launch_gemv_t<float, float, L>(w, scale, w, scale, x, y, B, K, N, stream, bias);
}

// Same-x group: at one token, when every matrix suits the balanced kernel
// (16-byte aligned, K % 64 == 0 up to 16384) and the rows fit its slots, one
// launch over the concatenated rows; otherwise one launch per matrix.
static bool gemv_group_grid(const void *x, int B, int K, int count, const uint32_t *const *w, const int *N,
                            int *total, int *G) {
  *total = 0;
  bool one = count >= 1 && count <= GEMV_GROUP_MAX;
  for (int i = 0; i < count; i++) {
    *total += N[i];
    one = one && (reinterpret_cast<uintptr_t>(w[i]) & 15) == 0;
  }
  return one && gemv_bal_grid(w[0], x, B, K, *total, G, K > 3 * 4096 ? GEMV_BAL_RMAX : GEMV_GROUP_RMAX);
}

bool gemv_group_fits(const void *x, int B, int K, int count, const uint32_t *const *w, const int *N) {
  int total = 0, G = 0;
  return gemv_group_grid(x, B, K, count, w, N, &total, &G);
}

hipError_t launch_gemv_group(const void *x, int xt_bf16, int yt_bf16, int B, int K, int count,
                             const uint32_t *const *w, const float *const *s, void *const *y, const int *N,
                             hipStream_t stream) {
  int total = 0, G = 0;
  if (gemv_group_grid(x, B, K, count, w, N, &total, &G)) {
    GemvGroup g{};
    int st = 0;
    for (int i = 0; i < GEMV_GROUP_MAX; i++) {
      g.w[i] = i < count ? w[i] : w[0];
      g.s[i] = i < count ? s[i] : s[0];
      g.y[i] = i < count ? y[i] : y[0];
      g.start[i] = i < count ? st : 0x7fffffff;
      if (i < count) st += N[i];
    }
    if (xt_bf16) {
      if (yt_bf16) return launch_gemv_bal<uint16_t, false, true>(w[0], s[0], x, y[0], K, total, G, stream, nullptr, &g);
      return launch_gemv_bal<float, false, true>(w[0], s[0], x, y[0], K, total, G, stream, nullptr, &g);
    }
    if (yt_bf16) return launch_gemv_bal<uint16_t, true, true>(w[0], s[0], x, y[0], K, total, G, stream, nullptr, &g);
    return launch_gemv_bal<float, true, true>(w[0], s[0], x, y[0], K, total, G, stream, nullptr, &g);
  }
  for (int i = 0; i < count; i++) {
    const hipError_t e = launch_gemv(w[i], s[i], x, xt_bf16, y[i], yt_bf16, B, K, N[i], stream, nullptr);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_gemv_glu(const uint32_t *w_gate, const float *s_gate, const uint32_t *w_up,
                           const float *s_up, const void *x, int xt_bf16, float *h, int B, int K,
                           int N, int gelu, hipStream_t stream) {
  if (xt_bf16 && B >= GEMV_GLU_XS_MIN_B && gemv_xs_ok(x, B, K, 1, 2)) {
    if (gelu)
      return launch_gemv_xs<float, 2, GEMV_GEGLU, XS_BF16, false>(w_gate, s_gate, w_up, s_up, x, x, h, B, K, N,
                                                                   stream);
    return launch_gemv_xs<float, 2, GEMV_SWIGLU, XS_BF16, false>(w_gate, s_gate, w_up, s_up, x, x, h, B, K, N,
                                                                  stream);
  }
  if (!xt_bf16 && B >= 2 && gemv_xs_ok(x, B, K, 2, 2)) {
    if (gelu)
      return launch_gemv_xs<float, 2, GEMV_GEGLU, XS_F32, false>(w_gate, s_gate, w_up, s_up, x, x, h, B, K, N,
                                                                  stream);
    return launch_gemv_xs<float, 2, GEMV_SWIGLU, XS_F32, false>(w_gate, s_gate, w_up, s_up, x, x, h, B, K, N,
                                                                 stream);
  }
  if (xt_bf16 && B >= GEMV_DIRECT_MIN_B) {
    if (gelu) return launch_gemv_direct<float, GEMV_GEGLU>(w_gate, s_gate, w_up, s_up, x, x, h, B, K, N, stream);
    return launch_gemv_direct<float, GEMV_SWIGLU>(w_gate, s_gate, w_up, s_up, x, x, h, B, K, N, stream);
  }
  if (xt_bf16) {
    if (gelu)
      return launch_gemv_t<uint16_t, float, GEMV_GEGLU>(w_gate, s_gate, w_up, s_up, x, h, B, K, N, stream);
    return launch_gemv_t<uint16_t, float, GEMV_SWIGLU>(w_gate, s_gate, w_up, s_up, x, h, B, K, N, stream);
  }
  if (gelu)
    return launch_gemv_t<float, float, GEMV_GEGLU>(w_gate, s_gate, w_up, s_up, x, h, B, K, N, stream);
  return launch_gemv_t<float, float, GEMV_SWIGLU>(w_gate, s_gate, w_up, s_up, x, h, B, K, N, stream);
}

template <bool GELU>
__global__ __launch_bounds__(256) void glu_combine_kernel(const float *__restrict__ g,
                                                          const float *__restrict__ u,
                                                          float *h, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const float a = GELU ? act_gelu_tanh(g[i]) : act_silu(g[i]);
    h[i] = a * u[i];
  }
}

hipError_t launch_glu_combine(const float *g, const float *u, float *h, size_t n, int gelu,
                              hipStream_t stream) {
  const size_t blocks = (n + 255) / 256;
  const dim3 grid((unsigned)(blocks < 8192 ? blocks : 8192));
  if (gelu) hipLaunchKernelGGL((glu_combine_kernel<true>), grid, dim3(256), 0, stream, g, u, h, n);
  else hipLaunchKernelGGL((glu_combine_kernel<false>), grid, dim3(256), 0, stream, g, u, h, n);
  return hipGetLastError();
}

hipError_t launch_gemv_glu_planes(const uint32_t *w_gate, const float *s_gate, const uint32_t *w_up,
                                  const float *s_up, const void *x, uint16_t *h_planes, int B, int K,
                                  int N, int gelu, hipStream_t stream) {
  if (B >= GEMV_GLU_XS_MIN_B && gemv_xs_ok(x, B, K, 1, 2)) {
    if (gelu)
      return launch_gemv_xs<uint16_t, 2, GEMV_GEGLU, XS_BF16, true>(w_gate, s_gate, w_up, s_up, x, x, h_planes, B,
                                                                     K, N, stream);
    return launch_gemv_xs<uint16_t, 2, GEMV_SWIGLU, XS_BF16, true>(w_gate, s_gate, w_up, s_up, x, x, h_planes, B,
                                                                    K, N, stream);
  }
  if (gelu)
    return launch_gemv_direct<uint16_t, GEMV_GEGLU, 1, true>(w_gate, s_gate, w_up, s_up, x, x, h_planes, B,
                                                             K, N, stream);
  return launch_gemv_direct<uint16_t, GEMV_SWIGLU, 1, true>(w_gate, s_gate, w_up, s_up, x, x, h_planes, B,
                                                            K, N, stream);
}

hipError_t launch_gemv_planes(const uint32_t *w, const float *scale, const uint16_t *x_planes, void *y,
                              int yt_bf16, int B, int K, int N, hipStream_t stream) {
  const uint16_t *lo = x_planes + (size_t)B * K;
  if (B >= GEMV_PLANES_XS_MIN_B && gemv_xs_ok(x_planes, B, K, 2, 1) && (reinterpret_cast<uintptr_t>(lo) & 15) == 0) {
    if (yt_bf16)
      return launch_gemv_xs<uint16_t, 1, GEMV_LINEAR, XS_PLANES, false>(w, scale, w, scale, x_planes, lo, y, B, K,
                                                                        N, stream);
    return launch_gemv_xs<float, 1, GEMV_LINEAR, XS_PLANES, false>(w, scale, w, scale, x_planes, lo, y, B, K, N,
                                                                   stream);
  }
  if (yt_bf16)
    return launch_gemv_direct<uint16_t, GEMV_LINEAR, 2>(w, scale, w, scale, x_planes, lo, y, B, K, N, stream);
  return launch_gemv_direct<float, GEMV_LINEAR, 2>(w, scale, w, scale, x_planes, lo, y, B, K, N, stream);
}

}  // namespace frx
