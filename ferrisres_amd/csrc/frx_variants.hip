// frx_variants.hip — the reference's other ternary matmul forms on gfx950:
// index-list decode (ternary_matmul_sparse_decode), tensor statistics
// (ternary_stats), column-block scales (ternary_matmul_blocked, via an
// activation prescale feeding the dense kernels), and the [H, E] router
// layout of CpuMoELayer (transposed into the [E, H] layout the MoE kernels
// read).
#include "frx_device.hpp"
#include "frx_internal.hpp"

namespace frx {

// ---- index-list decode (src/model/ternary.rs:647-707) ----------------------
// y[m][r] = scale * (sum over pos list of x[m][j] - sum over neg list of
// x[m][j]). One wave per (row, token): lanes stride over each list in order,
// then a fixed-order wave reduction (DPP within rows of 16 lanes, then the
// four row sums added in lane order), so results are deterministic. Gathers
// of x hit L2: the lists are the only HBM stream (4 bytes per nonzero).
template <int CTRL>
__device__ __forceinline__ float dpp_sum_step(float v) {
  return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float wave_sum_fixed(float v) {
  v = dpp_sum_step<0xB1>(v);   // quad_perm [1,0,3,2]
  v = dpp_sum_step<0x4E>(v);   // quad_perm [2,3,0,1]
  v = dpp_sum_step<0x124>(v);  // row_ror:4
  v = dpp_sum_step<0x128>(v);  // row_ror:8
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (a + b) + (c + d);
}

template <typename XT>
__device__ __forceinline__ float load_act(const XT *x, size_t i);
template <>
__device__ __forceinline__ float load_act<float>(const float *x, size_t i) { return x[i]; }
template <>
__device__ __forceinline__ float load_act<uint16_t>(const uint16_t *x, size_t i) { return bf16_to_f32(x[i]); }

template <typename XT, typename YT>
__global__ __launch_bounds__(256) void index_decode_kernel(const uint32_t *__restrict__ pos_off,
                                                           const uint32_t *__restrict__ pos_idx,
                                                           const uint32_t *__restrict__ neg_off,
                                                           const uint32_t *__restrict__ neg_idx, float scale,
                                                           const XT *__restrict__ X, YT *__restrict__ Y, int K,
                                                           int N) {
  const int lane = threadIdx.x & 63;
  const int row = (int)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int m = (int)blockIdx.y;
  if (row >= N) return;  // whole waves leave together
  const XT *xr = X + (size_t)m * K;
  float sp = 0.0f, sn = 0.0f;
  for (uint32_t i = pos_off[row] + lane; i < pos_off[row + 1]; i += 64) sp += load_act(xr, pos_idx[i]);
  for (uint32_t i = neg_off[row] + lane; i < neg_off[row + 1]; i += 64) sn += load_act(xr, neg_idx[i]);
  const float s = wave_sum_fixed(sp) - wave_sum_fixed(sn);
  if (lane == 0) {
    const float y = scale * s;
    if constexpr (sizeof(YT) == 2) Y[(size_t)m * N + row] = (uint16_t)bf16_rne(y);
    else Y[(size_t)m * N + row] = y;
  }
}

hipError_t launch_index_decode(const uint32_t *pos_off, const uint32_t *pos_idx, const uint32_t *neg_off,
                               const uint32_t *neg_idx, float scale, const void *x, int xt_bf16, void *y,
                               int yt_bf16, int M, int K, int N, hipStream_t stream) {
  const dim3 grid((N + 3) / 4, M), block(256);
#define FRX_IDX(XT, YT)                                                                                       \
  hipLaunchKernelGGL((index_decode_kernel<XT, YT>), grid, block, 0, stream, pos_off, pos_idx, neg_off, neg_idx, \
                     scale, reinterpret_cast<const XT *>(x), reinterpret_cast<YT *>(y), K, N)
  if (xt_bf16 && yt_bf16) FRX_IDX(uint16_t, uint16_t);
  else if (xt_bf16) FRX_IDX(uint16_t, float);
  else if (yt_bf16) FRX_IDX(float, uint16_t);
  else FRX_IDX(float, float);
#undef FRX_IDX
  return hipGetLastError();
}

// ---- statistics of a packed tensor (src/model/ternary.rs:725-746) ---------
// Counts of -1 (code 0), 0 (codes 1 and 3, as TERNARY_DECODE) and +1 (code 2)
// over the N*K codes of a [N][K/16] u32 matrix. A first launch clears the
// three counters; the second adds per-wave popcounts with 64-bit atomics
// (integer sums, so the result does not depend on the order).
__global__ void stats_clear_kernel(unsigned long long *counts) {
  if (threadIdx.x < 3) counts[threadIdx.x] = 0ull;
}

__global__ __launch_bounds__(256) void stats_kernel(const uint32_t *__restrict__ W, size_t nwords,
                                                    unsigned long long *__restrict__ counts) {
  unsigned long long neg = 0, pos = 0;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < nwords; i += (size_t)gridDim.x * 256) {
    const uint32_t w = W[i];
    const uint32_t lo = w & 0x55555555u, hi = (w >> 1) & 0x55555555u;
    neg += (unsigned)__builtin_popcount(~lo & ~hi & 0x55555555u);  // code 0
    pos += (unsigned)__builtin_popcount(~lo & hi);                  // code 2
  }
  // wave sums, then one atomic per wave
  for (int off = 32; off > 0; off >>= 1) {
    neg += __shfl_down(neg, off);
    pos += __shfl_down(pos, off);
  }
  if ((threadIdx.x & 63) == 0) {
    atomicAdd(&counts[0], neg);
    atomicAdd(&counts[2], pos);
  }
}

__global__ void stats_zero_count_kernel(unsigned long long *counts, unsigned long long n) {
  if (threadIdx.x == 0) counts[1] = n - counts[0] - counts[2];
}

hipError_t launch_stats(const uint32_t *w, size_t nwords, unsigned long long *counts, hipStream_t stream) {
  hipLaunchKernelGGL(stats_clear_kernel, dim3(1), dim3(64), 0, stream, counts);
  const size_t blocks = (nwords + 255) / 256;
  hipLaunchKernelGGL(stats_kernel, dim3((unsigned)(blocks < 2048 ? (blocks ? blocks : 1) : 2048)), dim3(256), 0,
                     stream, w, nwords, counts);
  hipLaunchKernelGGL(stats_zero_count_kernel, dim3(1), dim3(64), 0, stream, counts,
                     (unsigned long long)nwords * 16ull);
  return hipGetLastError();
}

// ---- column-block scales (src/model/ternary.rs:541-579) --------------------
// xs[m][k] = x[m][k] * scales[k / block_size] in fp32; the dense kernels then
// run xs against the codes with unit row scales. Every element is one
// multiply, so the sum is the reference's up to the order of the adds.
template <typename XT>
__global__ __launch_bounds__(256) void block_prescale_kernel(const XT *__restrict__ x,
                                                             const float *__restrict__ scales, int block_size,
                                                             float *__restrict__ xs, int K, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const int k = (int)(i % (size_t)K);
    xs[i] = load_act(x, i) * scales[k / block_size];
  }
}

__global__ __launch_bounds__(256) void fill_kernel(float *__restrict__ p, float v, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = v;
}

hipError_t launch_block_prescale(const void *x, int xt_bf16, const float *scales, int block_size, float *xs, int M,
                                 int K, hipStream_t stream) {
  const size_t n = (size_t)M * K;
  const size_t blocks = (n + 255) / 256;
  const dim3 grid((unsigned)(blocks < 4096 ? blocks : 4096));
  if (xt_bf16)
    hipLaunchKernelGGL((block_prescale_kernel<uint16_t>), grid, dim3(256), 0, stream,
                       reinterpret_cast<const uint16_t *>(x), scales, block_size, xs, K, n);
  else
    hipLaunchKernelGGL((block_prescale_kernel<float>), grid, dim3(256), 0, stream, reinterpret_cast<const float *>(x),
                       scales, block_size, xs, K, n);
  return hipGetLastError();
}

hipError_t launch_fill(float *p, float v, size_t n, hipStream_t stream) {
  const size_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)(blocks < 4096 ? (blocks ? blocks : 1) : 4096)), dim3(256), 0, stream,
                     p, v, n);
  return hipGetLastError();
}

// ---- router layout [H][E] -> [E][H] (CpuMoELayer, src/model/cpu_moe.rs:146) --
template <typename RT>
__global__ __launch_bounds__(256) void router_transpose_kernel(const RT *__restrict__ src, RT *__restrict__ dst,
                                                               int H, int E) {
  const size_t n = (size_t)H * E;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const int e = (int)(i / (size_t)H), h = (int)(i % (size_t)H);
    dst[i] = src[(size_t)h * E + e];
  }
}

hipError_t launch_router_transpose(const void *src, int rt_bf16, void *dst, int H, int E, hipStream_t stream) {
  const size_t n = (size_t)H * E, blocks = (n + 255) / 256;
  const dim3 grid((unsigned)(blocks < 1024 ? blocks : 1024));
  if (rt_bf16)
    hipLaunchKernelGGL((router_transpose_kernel<uint16_t>), grid, dim3(256), 0, stream,
                       reinterpret_cast<const uint16_t *>(src), reinterpret_cast<uint16_t *>(dst), H, E);
  else
    hipLaunchKernelGGL((router_transpose_kernel<float>), grid, dim3(256), 0, stream,
                       reinterpret_cast<const float *>(src), reinterpret_cast<float *>(dst), H, E);
  return hipGetLastError();
}

}  // namespace frx
