// frx_gemv_sk.hip — decode ternary GEMV for 2-16 tokens with K split over
// workgroups (tall row tiles, short column slices) and an ordered combine.
//
// Same semantics as the WGSL entry ternary_matmul_main
// (src/compute/kernels/ternary_matmul.rs:32-75): y[m][n] = scale[n] *
// sum_k dec(W[n][k]) x[m][k].
//
// Why a split. At 16 tokens the activations outweigh the weights a compute
// unit reads: a 16-row tile over the whole of K = 11008 multiplies 44 KB of
// weights against 16 x 11008 activations (352 KB as bf16, 704 KB as f32),
// and every tile of the launch streams all of them through its L1 and LDS.
// Here a workgroup owns 128 rows (eight waves of 16) and a slice of at most
// SK_NC 256-column chunks (as few as keep the grid within two workgroups per
// compute unit): the activations of the slice are staged once in LDS for
// all 128 rows, which cuts the activation stream per weight byte by 8x; the
// slices of a row tile run on other compute units and write fp32 partial
// tiles part[s][16][Np] with device-coherent stores. The last slice of a row
// tile to finish (a per-tile counter, agent-scope atomic) adds the slices of
// each output in slice order (deterministic whatever the arrival order),
// applies the row scale (and bias) and converts; no second launch and no
// workgroup waits for another.
//
// Operands. Lane (i = l % 16, g = l / 16) of a wave loads 16 bytes (words
// 4g .. 4g + 3, 64 codes) of its row i per chunk and decodes them in natural
// order (unpack16_nat): word q gives the A operands of MFMAs 2q and 2q + 1.
// MFMA m of a chunk therefore sums columns 64g + 8m .. 64g + 8m + 7 for lane
// group g; the B operand of lane (token j, g) is the 16 bytes of x[j] at
// those columns, read from the staged slice in natural order. f32
// activations are split into bf16 hi and lo planes at staging (|x - hi -
// lo| <= 2^-17 |x|) and each operand runs two MFMAs; bf16 planes given by
// the caller (the FFN's h) are staged as they are. Columns past K and
// tokens past B are staged as zeros, which cancel whatever the weight words
// hold there.
#include "frx_device.hpp"
#include "frx_gemm2.hpp"
#include "frx_internal.hpp"

namespace frx {

constexpr int SK_WAVES = 8;                  // waves per workgroup, 16 rows each
constexpr int SK_ROWS = SK_WAVES * 16;       // rows per workgroup
constexpr int SK_NC = 4;                     // 256-column chunks per slice at most
constexpr int SK_XS = SK_NC * 256 + 8;       // bf16 per staged token row (16-byte pad)
constexpr int SK_PIECES = 16 * SK_NC * 32;   // 8-column pieces of a slice (16 tokens)

constexpr int SK_CPOL_SC1 = 16;  // cache policy: performed at the point of coherence of all XCDs
constexpr int SK_CG = 16;        // partial slices loaded before they are added

// XS: 0 bf16 x; 1 f32 x (split into planes); 2 bf16 planes (X hi, X2 lo).
template <typename YT, int XS>
__global__ __launch_bounds__(SK_WAVES * 64) void gemv_sk_kernel(const uint32_t *__restrict__ W,
                                                                const float *__restrict__ scale,
                                                                const float *__restrict__ bias,
                                                                const void *__restrict__ X,
                                                                const void *__restrict__ X2,
                                                                float *__restrict__ part,
                                                                unsigned *__restrict__ counters,
                                                                YT *__restrict__ Y, int B, int K, int N,
                                                                int Np, int ncs, int S) {
  constexpr int P = XS == 0 ? 1 : 2;
  __shared__ __align__(16) uint16_t xs[P][16][SK_XS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int s = blockIdx.y;
  const int nch = (K + 255) >> 8;
  const int c0 = s * ncs, nc = min(ncs, nch - c0);
  const int k0 = c0 * 256;
  const int kw = K >> 4;
  constexpr uint32_t OOB = 0x80000000u;  // past every range this kernel takes
  // 1. activation pieces of the slice (token t, 8 columns), zero past B or K:
  //    issued first, since vector loads complete in issue order
  constexpr int XR = SK_PIECES / (SK_WAVES * 64);
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(X, (uint32_t)B * (uint32_t)K * (XS == 1 ? 4u : 2u));
  const __amdgpu_buffer_rsrc_t xr2 = buffer_rsrc(XS == 2 ? X2 : X, (uint32_t)B * (uint32_t)K * 2u);
  u32x4 xv[XR][XS == 0 ? 1 : 2];
#pragma unroll
  for (int r = 0; r < XR; r++) {
    const int pc = tid + r * SK_WAVES * 64;
    const int t = pc / (SK_NC * 32), col = k0 + (pc % (SK_NC * 32)) * 8;
    const bool ok = t < B && col < K;
    const uint32_t e = (uint32_t)t * (uint32_t)K + (uint32_t)col;  // element index
    if constexpr (XS == 1) {
#pragma unroll
      for (int l = 0; l < 2; l++) xv[r][l] = __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? e * 4u + 16u * l : OOB, 0, 0);
    } else if constexpr (XS == 2) {
      xv[r][0] = __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? e * 2u : OOB, 0, 0);
      xv[r][1] = __builtin_amdgcn_raw_buffer_load_b128(xr2, ok ? e * 2u : OOB, 0, 0);
    } else {
      xv[r][0] = __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? e * 2u : OOB, 0, 0);
    }
  }
  // 2. the wave's weight words, every chunk of the slice (rows past N and
  //    chunks past the slice read zeros)
  const int i = lane & 15, g = lane >> 4;
  const int row = blockIdx.x * SK_ROWS + wave * 16 + i;
  const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(W, (uint32_t)N * (uint32_t)kw * 4u);
  u32x4 wv[SK_NC];
#pragma unroll
  for (int c = 0; c < SK_NC; c++) {
    const uint32_t off =
        (c < nc && row < N) ? ((uint32_t)row * (uint32_t)kw + (uint32_t)(c0 + c) * 16u + 4u * g) * 4u : OOB;
    wv[c] = __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0);
  }
  // 3. stage the activations (natural order; f32 split into planes)
#pragma unroll
  for (int r = 0; r < XR; r++) {
    const int pc = tid + r * SK_WAVES * 64;
    const int t = pc / (SK_NC * 32), o = (pc % (SK_NC * 32)) * 8;
    if constexpr (XS == 1) {
      const u32x4 a = xv[r][0], b = xv[r][1];
      uint32_t hi[4], lo[4];
      split2_bf16(__uint_as_float(a.x), __uint_as_float(a.y), hi[0], lo[0]);
      split2_bf16(__uint_as_float(a.z), __uint_as_float(a.w), hi[1], lo[1]);
      split2_bf16(__uint_as_float(b.x), __uint_as_float(b.y), hi[2], lo[2]);
      split2_bf16(__uint_as_float(b.z), __uint_as_float(b.w), hi[3], lo[3]);
      *reinterpret_cast<u32x4 *>(&xs[0][t][o]) = (u32x4){hi[0], hi[1], hi[2], hi[3]};
      *reinterpret_cast<u32x4 *>(&xs[P - 1][t][o]) = (u32x4){lo[0], lo[1], lo[2], lo[3]};
    } else {
#pragma unroll
      for (int p = 0; p < P; p++) *reinterpret_cast<u32x4 *>(&xs[p][t][o]) = xv[r][p];
    }
  }
  __syncthreads();
  // 4. chunks in order as their words land: 8 MFMAs (x P planes) each
  f32x4 acc2[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  // B operand of lane (token l % 16, g): the token's staged row at 64 g
  const uint16_t *xrow[P];
#pragma unroll
  for (int p = 0; p < P; p++) xrow[p] = &xs[p][lane & 15][64 * g];
#pragma unroll
  for (int c = 0; c < SK_NC; c++) {
    if (c < nc) {  // workgroup-uniform
#pragma unroll
      for (int q = 0; q < 4; q++) {
        u32x4 lo, hi;
        unpack16_nat(wv[c][q], lo, hi);
#pragma unroll
        for (int p = 0; p < P; p++) {
          const u32x4 xa = *reinterpret_cast<const u32x4 *>(xrow[p] + c * 256 + 16 * q);
          const u32x4 xb = *reinterpret_cast<const u32x4 *>(xrow[p] + c * 256 + 16 * q + 8);
          acc2[q & 1] = mfma16(lo, xa, acc2[q & 1]);
          acc2[q & 1] = mfma16(hi, xb, acc2[q & 1]);
        }
      }
    }
  }
  const f32x4 acc = acc2[0] + acc2[1];
  // 5. partial tile: lane (token j = l % 16, g) holds rows 4g .. 4g + 3 of
  //    the wave's 16 for token j (unscaled, 2 * the dot product), stored
  //    device-coherent so that the workgroup that adds the slices (on any
  //    XCD) reads them from the point of coherence, not from its own L2
  const __amdgpu_buffer_rsrc_t pr = buffer_rsrc(part, (uint32_t)S * 16u * (uint32_t)Np * 4u);
  {
    const int j = lane & 15, r0 = blockIdx.x * SK_ROWS + wave * 16 + 4 * g;
    const uint32_t off = (j < B && r0 < Np) ? (((uint32_t)s * 16u + (uint32_t)j) * (uint32_t)Np + (uint32_t)r0) * 4u
                                            : OOB;
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc), pr, off, 0, SK_CPOL_SC1);
  }
  // 6. the last slice of this row tile to arrive adds all slices in slice
  //    order (a per-tile counter, reset by that workgroup for the next launch)
  __shared__ int last;
  wait_vmcnt<0>();  // this wave's partial stores are complete
  __syncthreads();
  if (tid == 0) {
    const unsigned old = __hip_atomic_fetch_add(counters + blockIdx.x, 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    last = old == (unsigned)S - 1u;
    if (last) __hip_atomic_store(counters + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last) return;  // workgroup-uniform
  // unit u = (token t, rows 4c .. 4c + 3 of the tile): 32 units per token
  for (int u = tid; u < B * (SK_ROWS / 4); u += SK_WAVES * 64) {
    const int t = u / (SK_ROWS / 4), n = blockIdx.x * SK_ROWS + (u % (SK_ROWS / 4)) * 4;
    if (n >= N) continue;
    f32x4 sum = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < S; s0 += SK_CG) {
      f32x4 v[SK_CG];
#pragma unroll
      for (int k = 0; k < SK_CG; k++) {
        const uint32_t off = s0 + k < S ? (((uint32_t)(s0 + k) * 16u + (uint32_t)t) * (uint32_t)Np + (uint32_t)n) * 4u
                                        : OOB;
        v[k] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, off, 0, SK_CPOL_SC1));
      }
#pragma unroll
      for (int k = 0; k < SK_CG; k++)
        if (s0 + k < S) sum = (s0 + k == 0) ? v[k] : sum + v[k];
    }
    const int nok = min(4, N - n);
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int nn = min(n + e, N - 1);
      o[e] = sum[e] * (0.5f * scale[nn]);  // 0.5 undoes the 2*dec(c) encoding
      if (bias) o[e] = add_bias(o[e], bias[nn]);
    }
    YStore<YT>::store4(Y + (size_t)t * N + n, o, nok);
  }
}

// Chunks per slice: the fewest (most slices, most workgroups) that keep the
// grid within two workgroups per compute unit, at most SK_NC.
static int gemv_sk_chunks(int K, int N, int cus) {
  const int nch = (K + 255) / 256, tiles = (N + SK_ROWS - 1) / SK_ROWS;
  for (int ncs = 1; ncs < SK_NC; ncs++)
    if ((size_t)tiles * ((nch + ncs - 1) / ncs) <= (size_t)2 * cus) return ncs;
  return SK_NC;
}

size_t gemv_sk_workspace_bytes(int K, int N, int cus) {
  const int ncs = gemv_sk_chunks(K, N, cus);
  const int S = ((K + 255) / 256 + ncs - 1) / ncs;
  const size_t Np = (size_t)(N + 3) / 4 * 4;
  return (size_t)S * 16 * Np * 4;
}

hipError_t launch_gemv_sk(const uint32_t *w, const float *scale, const void *x, const void *x2, int xs,
                          void *y, int yt_bf16, int B, int K, int N, float *part, unsigned *counters,
                          const float *bias, int cus, hipStream_t stream) {
  const int ncs = gemv_sk_chunks(K, N, cus);
  const int S = ((K + 255) / 256 + ncs - 1) / ncs;
  const int Np = (N + 3) / 4 * 4;
  const dim3 grid((unsigned)((N + SK_ROWS - 1) / SK_ROWS), (unsigned)S);
  const dim3 block(SK_WAVES * 64);
#define FRX_SK(YT, XSV)                                                                                     \
  hipLaunchKernelGGL((gemv_sk_kernel<YT, XSV>), grid, block, 0, stream, w, scale, bias, x, x2, part, counters, \
                     reinterpret_cast<YT *>(y), B, K, N, Np, ncs, S)
  if (yt_bf16) {
    if (xs == 1) FRX_SK(uint16_t, 1);
    else if (xs == 2) FRX_SK(uint16_t, 2);
    else FRX_SK(uint16_t, 0);
  } else {
    if (xs == 1) FRX_SK(float, 1);
    else if (xs == 2) FRX_SK(float, 2);
    else FRX_SK(float, 0);
  }
#undef FRX_SK
  return hipGetLastError();
}

}  // namespace frx
