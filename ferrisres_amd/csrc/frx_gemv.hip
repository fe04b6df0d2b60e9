// frx_gemv.hip — decode ternary GEMV for M <= 16 tokens on gfx950.
//
// Replaces the WGSL entry ternary_matmul_main
// (src/compute/kernels/ternary_matmul.rs:32-75) for decode shapes.
//
// Mapping. One workgroup (4 waves) owns a 16-row tile of W. The 16 rows are
// the M side of v_mfma_f32_16x16x32_bf16 and the (<= 16) tokens its N side.
// Lane (r = l%16, g = l/16) streams 16-byte chunks (64 codes) of row r with
// dwordx4 loads; the 4 lanes of a row read 64 contiguous bytes per
// instruction. Each lane turns its codes into bf16 operands in registers
// (two VALU ops per weight pair, see frx_device.hpp), the activations come
// from LDS in the matching K-interleaved order, and the MFMA does the
// multiply-adds. The four waves split K; their partial tiles are summed in a
// fixed order through LDS, so results are deterministic.
//
// Activations are staged per K-slice into LDS as bf16 (f32 inputs as a hi/lo
// bf16 pair: two MFMAs per operand, |error| <= 2^-17 |x|).
#include "frx_device.hpp"
#include "frx_internal.hpp"

namespace frx {

// LDS row stride (dwords) for a slice of ks columns: ks/2 dwords rounded up
// to a multiple of 64 plus 4, so 16 tokens' 16-byte reads hit disjoint banks.
static inline int gemv_row_stride(int ks) { return ((ks / 2 + 63) / 64) * 64 + 4; }

template <typename XT, typename YT>
__global__ __launch_bounds__(256) void gemv_kernel(
    const uint32_t *__restrict__ W, const float *__restrict__ scale,
    const XT *__restrict__ X, YT *__restrict__ Y, int B, int K, int N, int KS,
    int rs, int vec_ok) {
  constexpr int P = XBlock<XT>::P;
  extern __shared__ __align__(16) uint32_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int row = blockIdx.x * 16 + r;
  const int wpr = K >> 4;
  const bool row_ok = row < N;
  const uint32_t *wrow = W + (size_t)(row_ok ? row : 0) * wpr;
  const int t = r;  // token whose activations this lane feeds (MFMA column)
  const bool t_ok = t < B;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};

  for (int s0 = 0; s0 < K; s0 += KS) {
    const int ks = min(KS, K - s0);
    const int nblk = ks >> 4;
    // Stage x[:, s0:s0+ks] into LDS (interleaved bf16; lo plane after hi).
    for (int bi = tid; bi < B * nblk; bi += 256) {
      const int tt = bi / nblk, cb = bi - tt * nblk;
      uint32_t hi[8], lo[8];
      XBlock<XT>::load(X + (size_t)tt * K + s0 + cb * 16, true, hi, lo);
      u32x4 *d = reinterpret_cast<u32x4 *>(lds + tt * rs + cb * 8);
      d[0] = (u32x4){hi[0], hi[1], hi[2], hi[3]};
      d[1] = (u32x4){hi[4], hi[5], hi[6], hi[7]};
      if constexpr (P == 2) {
        u32x4 *e = reinterpret_cast<u32x4 *>(lds + (B + tt) * rs + cb * 8);
        e[0] = (u32x4){lo[0], lo[1], lo[2], lo[3]};
        e[1] = (u32x4){lo[4], lo[5], lo[6], lo[7]};
      }
    }
    __syncthreads();

    const int nch = (ks + 63) >> 6;     // 64-column chunks in the slice
    const int nsteps = (nch + 3) >> 2;  // a wave step covers 4 chunks
    for (int st0 = wave; st0 < nsteps; st0 += 16) {
      uint32_t wv[4][4];
      // Issue all loads of the batch first (up to 4 dwordx4 per lane).
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int st = st0 + 4 * u;
        const int c = st * 4 + g;
        const int cw = c * 4;  // first word of the chunk within the slice
        const int wb = (s0 >> 4) + cw;
        if (st < nsteps && row_ok && vec_ok && c * 64 + 64 <= ks) {
          u32x4 v = *reinterpret_cast<const u32x4 *>(wrow + wb);
          wv[u][0] = v.x; wv[u][1] = v.y; wv[u][2] = v.z; wv[u][3] = v.w;
        } else {
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const bool ok = st < nsteps && row_ok && (c * 64 + 16 * q < ks);
            wv[u][q] = ok ? wrow[wb + q] : 0xFFFFFFFFu;  // ~0 -> zero operand
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int st = st0 + 4 * u;
        if (st >= nsteps) break;  // wave-uniform
        const int c = st * 4 + g;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const uint32_t nw = ~wv[u][q];
          const bool bok = t_ok && (c * 64 + 16 * q < ks);
          const uint32_t *bp = lds + t * rs + (c * 4 + q) * 8;
          const u32x4 z = {0u, 0u, 0u, 0u};
          u32x4 b0 = bok ? *reinterpret_cast<const u32x4 *>(bp) : z;
          u32x4 b1 = bok ? *reinterpret_cast<const u32x4 *>(bp + 4) : z;
          const u32x4 a0 = unpack_half<0>(nw), a1 = unpack_half<1>(nw);
          acc = mfma16(a0, b0, acc);
          acc = mfma16(a1, b1, acc);
          if constexpr (P == 2) {
            const uint32_t *bq = bp + B * rs;
            u32x4 c0 = bok ? *reinterpret_cast<const u32x4 *>(bq) : z;
            u32x4 c1 = bok ? *reinterpret_cast<const u32x4 *>(bq + 4) : z;
            acc = mfma16(a0, c0, acc);
            acc = mfma16(a1, c1, acc);
          }
        }
      }
    }
    __syncthreads();
  }

  // Fixed-order reduction of the four waves' partial tiles.
  f32x4 *red = reinterpret_cast<f32x4 *>(lds);
  red[wave * 64 + lane] = acc;
  __syncthreads();
  if (wave == 0) {
    f32x4 s = red[lane];
    s += red[64 + lane];
    s += red[128 + lane];
    s += red[192 + lane];
    const int n = blockIdx.x * 16 + 4 * g;  // rows 4g..4g+3, token t
    if (t_ok && n < N) {
      const int nok = min(4, N - n);
      f32x4 sc;
      sc.x = scale[n];
      sc.y = nok > 1 ? scale[n + 1] : 0.f;
      sc.z = nok > 2 ? scale[n + 2] : 0.f;
      sc.w = nok > 3 ? scale[n + 3] : 0.f;
      const f32x4 v = s * (sc * 0.5f);
      YStore<YT>::store4(Y + (size_t)t * N + n, v, nok);
    }
  }
}

template <typename XT, typename YT>
static hipError_t launch_gemv_t(const uint32_t *w, const float *scale,
                                const void *x, void *y, int B, int K, int N,
                                hipStream_t stream) {
  constexpr int P = XBlock<XT>::P;
  const int budget = 48 * 1024;
  int KS = K;
  while (KS > 128 && (size_t)P * B * gemv_row_stride(KS) * 4 > (size_t)budget)
    KS = ((KS / 2) + 127) / 128 * 128;
  const int rs = gemv_row_stride(KS);
  size_t lds = (size_t)P * B * rs * 4;
  if (lds < 4096) lds = 4096;
  const int vec_ok = ((K >> 4) % 4 == 0) && ((reinterpret_cast<uintptr_t>(w) & 15) == 0);
  dim3 grid((N + 15) / 16);
  hipLaunchKernelGGL((gemv_kernel<XT, YT>), grid, dim3(256), lds, stream, w,
                     scale, reinterpret_cast<const XT *>(x),
                     reinterpret_cast<YT *>(y), B, K, N, KS, rs, vec_ok);
  return hipGetLastError();
}

hipError_t launch_gemv(const uint32_t *w, const float *scale, const void *x,
                       int xt_bf16, void *y, int yt_bf16, int B, int K, int N,
                       hipStream_t stream) {
  if (xt_bf16) {
    if (yt_bf16)
      return launch_gemv_t<uint16_t, uint16_t>(w, scale, x, y, B, K, N, stream);
    return launch_gemv_t<uint16_t, float>(w, scale, x, y, B, K, N, stream);
  }
  if (yt_bf16)
    return launch_gemv_t<float, uint16_t>(w, scale, x, y, B, K, N, stream);
  return launch_gemv_t<float, float>(w, scale, x, y, B, K, N, stream);
}

}  // namespace frx
