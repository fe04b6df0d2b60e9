// frx_gemv.hip — decode ternary GEMV for M <= 16 tokens on gfx950.
//
// Replaces the WGSL entry ternary_matmul_main
// (src/compute/kernels/ternary_matmul.rs:32-75) for decode shapes.
//
// Mapping. One workgroup (WAVES waves) owns a 16-row tile of W. The 16 rows
// are the M side of v_mfma_f32_16x16x32_bf16 and the (<= 16) tokens its N
// side. Lane (r = l%16, g = l/16) streams 16-byte chunks (64 codes) of row r
// with dwordx4 loads; the 4 lanes of a row read 64 contiguous bytes per
// instruction. The waves split K. Each wave issues all of its weight loads
// (up to UMAX per lane) before anything else, so the whole matrix is in
// flight at once; the kernel is a single HBM round trip plus the stream.
// Codes become bf16 operands in registers (two VALU ops per weight pair,
// frx_device.hpp); activations come from LDS in the matching K-interleaved
// order. Lanes whose token is >= B read a zero row, and the staged rows are
// zero-padded to a multiple of 256 columns, so operand reads never need a
// predicate. The waves' partial tiles are summed in a fixed order through
// LDS, so results are deterministic.
//
// Activations are staged per K-slice into LDS as bf16 (f32 inputs as a hi/lo
// bf16 pair: two MFMAs per operand, |error| <= 2^-17 |x|).
#include "frx_device.hpp"
#include "frx_internal.hpp"

namespace frx {

constexpr int GEMV_UMAX = 8;   // weight chunks per lane per batch
constexpr int GEMV_XBMAX = 2;  // activation blocks per thread loaded up front

// LDS row stride (dwords) for a slice of ks columns padded to 256: ks/2
// dwords rounded up to 128 plus 4, so 16 tokens' 16-byte reads hit disjoint
// banks.
static inline int gemv_row_stride(int ks) { return ((ks + 255) / 256) * 128 + 4; }

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

template <typename XT, typename YT, int WAVES, bool VEC>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(
    const uint32_t *__restrict__ W, const float *__restrict__ scale,
    const XT *__restrict__ X, YT *__restrict__ Y, int B, int K, int N, int KS,
    int rs) {
  constexpr int P = XBlock<XT>::P;
  constexpr int NT = WAVES * 64;
  extern __shared__ __align__(16) uint32_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int wpr = K >> 4;
  const int row = min((int)blockIdx.x * 16 + r, N - 1);  // clamped; stores are masked
  const uint32_t *wrow = W + (size_t)row * wpr;
  const int t = r;  // token whose activations this lane feeds (MFMA column)
  const int zrow = P * B;  // all-zero LDS row for lanes with t >= B
  const uint32_t *bp0 = lds + (t < B ? t : zrow) * rs;
  const uint32_t *bq0 = lds + (t < B ? B + t : zrow) * rs;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  // Row scales are needed only by the epilogue; fetch them now so that load
  // is not a memory round trip after the reduction.
  const int n_out = blockIdx.x * 16 + 4 * g;
  f32x4 sc = {0.f, 0.f, 0.f, 0.f};
  if (wave == 0 && t < B && n_out < N) {
    const int nok = min(4, N - n_out);
    sc.x = scale[n_out];
    sc.y = nok > 1 ? scale[n_out + 1] : 0.f;
    sc.z = nok > 2 ? scale[n_out + 2] : 0.f;
    sc.w = nok > 3 ? scale[n_out + 3] : 0.f;
  }

  for (int s0 = 0; s0 < K; s0 += KS) {
    const int ks = min(KS, K - s0);
    const int nch = (ks + 63) >> 6;     // 64-column chunks in the slice
    const int nsteps = (nch + 3) >> 2;  // a wave step covers 4 chunks
    const int kw0 = s0 >> 4;
    const int kw_end = (s0 + ks) >> 4;  // one past the slice's last word
    const int nblk = (ks + 255) / 256 * 16;  // 16-column x blocks, padded to 256 cols
    const int kblk = ks >> 4;
    const int nbtot = (B + 1) * nblk;        // + the zero row

    // 1. activation loads for the first XBMAX blocks of this thread (L2-hot,
    //    issued first so that waiting for them does not wait for the weights)
    uint32_t xh[GEMV_XBMAX][8], xl[GEMV_XBMAX][8];
#pragma unroll
    for (int i = 0; i < GEMV_XBMAX; i++) {
      const int bi = tid + i * NT;
      const int tt = bi / nblk, cb = bi - tt * nblk;
      const bool ok = bi < nbtot && tt < B && cb < kblk;
      XBlock<XT>::load(X + (size_t)(ok ? tt : 0) * K + s0 + (ok ? cb : 0) * 16, ok, xh[i], xl[i]);
    }
    // 2. first batch of weight loads
    u32x4 wv[GEMV_UMAX];
#pragma unroll
    for (int u = 0; u < GEMV_UMAX; u++) {
      const int st = wave + WAVES * u;
      if (st < nsteps) wv[u] = load_chunk<VEC>(wrow, kw0 + (st * 4 + g) * 4, kw_end);
    }
    // 3. stage the slice's activations into LDS (every wave takes part)
    if (s0 > 0) __syncthreads();  // previous slice fully consumed
    auto put = [&](int bi, const uint32_t *hi, const uint32_t *lo) {
      const int tt = bi / nblk, cb = bi - tt * nblk;
      const int rh = tt < B ? tt : zrow;
      u32x4 *d = reinterpret_cast<u32x4 *>(lds + rh * rs + cb * 8);
      d[0] = (u32x4){hi[0], hi[1], hi[2], hi[3]};
      d[1] = (u32x4){hi[4], hi[5], hi[6], hi[7]};
      if constexpr (P == 2) {
        if (tt < B) {
          u32x4 *e = reinterpret_cast<u32x4 *>(lds + (B + tt) * rs + cb * 8);
          e[0] = (u32x4){lo[0], lo[1], lo[2], lo[3]};
          e[1] = (u32x4){lo[4], lo[5], lo[6], lo[7]};
        }
      }
    };
#pragma unroll
    for (int i = 0; i < GEMV_XBMAX; i++) {
      const int bi = tid + i * NT;
      if (bi < nbtot) put(bi, xh[i], xl[i]);
    }
    for (int bi = tid + GEMV_XBMAX * NT; bi < nbtot; bi += NT) {  // large B x K
      const int tt = bi / nblk, cb = bi - tt * nblk;
      const bool ok = tt < B && cb < kblk;
      uint32_t hi[8], lo[8];
      XBlock<XT>::load(X + (size_t)(ok ? tt : 0) * K + s0 + (ok ? cb : 0) * 16, ok, hi, lo);
      put(bi, hi, lo);
    }
    __syncthreads();
    // 3. unpack + MFMA, batch by batch
    for (int st0 = wave; st0 < nsteps; st0 += WAVES * GEMV_UMAX) {
      if (st0 != wave) {
#pragma unroll
        for (int u = 0; u < GEMV_UMAX; u++) {
          const int st = st0 + WAVES * u;
          if (st < nsteps) wv[u] = load_chunk<VEC>(wrow, kw0 + (st * 4 + g) * 4, kw_end);
        }
      }
#pragma unroll
      for (int u = 0; u < GEMV_UMAX; u++) {
        const int st = st0 + WAVES * u;
        if (st >= nsteps) break;  // wave-uniform
        const int c = st * 4 + g;
        const int wb = kw0 + c * 4;
        const uint32_t *bp = bp0 + c * 32;
        const uint32_t *bq = bq0 + c * 32;
        const uint32_t wq[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
        // VEC: a chunk is either entirely inside the slice or entirely past
        // its end, so one mask per chunk; otherwise one per word.
        const uint32_t mchunk = wb < kw_end ? 0xC000C000u : 0u;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          // past the slice end: zero operand (the x rows there are zero too)
          const uint32_t mask = VEC ? mchunk : ((wb + q < kw_end) ? 0xC000C000u : 0u);
          const u32x4 b0 = *reinterpret_cast<const u32x4 *>(bp + q * 8);
          const u32x4 b1 = *reinterpret_cast<const u32x4 *>(bp + q * 8 + 4);
          const u32x4 a0 = unpack_half_m<0>(wq[q], mask), a1 = unpack_half_m<1>(wq[q], mask);
          acc = mfma16(a0, b0, acc);
          acc = mfma16(a1, b1, acc);
          if constexpr (P == 2) {
            const u32x4 c0 = *reinterpret_cast<const u32x4 *>(bq + q * 8);
            const u32x4 c1 = *reinterpret_cast<const u32x4 *>(bq + q * 8 + 4);
            acc = mfma16(a0, c0, acc);
            acc = mfma16(a1, c1, acc);
          }
        }
      }
    }
  }
  __syncthreads();

  // Fixed-order reduction of the waves' partial tiles.
  f32x4 *red = reinterpret_cast<f32x4 *>(lds);
  red[wave * 64 + lane] = acc;
  __syncthreads();
  if (wave == 0) {
    f32x4 s = red[lane];
#pragma unroll
    for (int w = 1; w < WAVES; w++) s += red[w * 64 + lane];
    if (t < B && n_out < N) {  // rows 4g..4g+3 of token t
      const f32x4 v = s * (sc * 0.5f);
      YStore<YT>::store4(Y + (size_t)t * N + n_out, v, min(4, N - n_out));
    }
  }
}

template <typename XT, typename YT, int WAVES, bool VEC>
static hipError_t launch_gemv_w(const uint32_t *w, const float *scale,
                                const void *x, void *y, int B, int K, int N,
                                hipStream_t stream) {
  constexpr int P = XBlock<XT>::P;
  const int budget = 56 * 1024;
  int KS = K;
  while (KS > 256 && (size_t)(P * B + 1) * gemv_row_stride(KS) * 4 > (size_t)budget)
    KS = ((KS / 2) + 255) / 256 * 256;
  const int rs = gemv_row_stride(KS);
  size_t lds = (size_t)(P * B + 1) * rs * 4;
  if (lds < (size_t)WAVES * 64 * 16) lds = (size_t)WAVES * 64 * 16;
  dim3 grid((N + 15) / 16);
  hipLaunchKernelGGL((gemv_kernel<XT, YT, WAVES, VEC>), grid, dim3(WAVES * 64), lds, stream, w, scale,
                     reinterpret_cast<const XT *>(x), reinterpret_cast<YT *>(y), B, K, N, KS, rs);
  return hipGetLastError();
}

template <typename XT, typename YT>
static hipError_t launch_gemv_t(const uint32_t *w, const float *scale,
                                const void *x, void *y, int B, int K, int N,
                                hipStream_t stream) {
  // 8 waves when one batch of 4 waves could not cover K (more loads in
  // flight); dword loads when rows are not 16-byte aligned.
  const bool vec = ((K >> 4) & 3) == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0;
  if (K > 4 * GEMV_UMAX * 256) {
    if (vec) return launch_gemv_w<XT, YT, 8, true>(w, scale, x, y, B, K, N, stream);
    return launch_gemv_w<XT, YT, 8, false>(w, scale, x, y, B, K, N, stream);
  }
  if (vec) return launch_gemv_w<XT, YT, 4, true>(w, scale, x, y, B, K, N, stream);
  return launch_gemv_w<XT, YT, 4, false>(w, scale, x, y, B, K, N, stream);
}

hipError_t launch_gemv(const uint32_t *w, const float *scale, const void *x,
                       int xt_bf16, void *y, int yt_bf16, int B, int K, int N,
                       hipStream_t stream) {
  if (xt_bf16) {
    if (yt_bf16) return launch_gemv_t<uint16_t, uint16_t>(w, scale, x, y, B, K, N, stream);
    return launch_gemv_t<uint16_t, float>(w, scale, x, y, B, K, N, stream);
  }
  if (yt_bf16) return launch_gemv_t<float, uint16_t>(w, scale, x, y, B, K, N, stream);
  return launch_gemv_t<float, float>(w, scale, x, y, B, K, N, stream);
}

}  // namespace frx
