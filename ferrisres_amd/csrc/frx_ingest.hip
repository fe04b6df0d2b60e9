// frx_ingest.hip — weight ingest on the device: the CPU 2:4 layout
// (SparseTernaryMatrix, src/model/sparse_ternary.rs:52-70: pattern nibbles,
// sign pairs with bit 1 = +1, groups numbered flat over the matrix) to the
// GPU 5-bit layout (src/compute/kernels/sparse_ternary.rs:254-318: six groups
// per row word, bits[2:0] pattern, bit 3 / bit 4 set = the lower / higher
// nonzero is -1). One thread per GPU word; bit-exact with the host
// transcoder frx_sparse24_cpu_to_gpu. Patterns 6 and 7, which the CPU layout
// can hold but no packer writes, become pattern 0 as in to_ternary
// (sparse_ternary.rs:172-176).
#include "frx_internal.hpp"

namespace frx {

__global__ __launch_bounds__(256) void sp24_cpu_to_gpu_kernel(const uint8_t *__restrict__ patterns,
                                                              const uint8_t *__restrict__ signs, uint32_t N,
                                                              uint32_t gpr, uint32_t wpr,
                                                              uint32_t *__restrict__ meta) {
  const size_t wid = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (wid >= (size_t)N * wpr) return;
  const size_t r = wid / wpr;
  const uint32_t w = (uint32_t)(wid - r * wpr);
  uint32_t word = 0;
  for (uint32_t q = 0; q < 6; q++) {
    const uint32_t g = w * 6 + q;
    if (g >= gpr) break;
    const size_t gi = r * gpr + g;
    uint32_t pat = (patterns[gi >> 1] >> (4 * (gi & 1))) & 7u;
    if (pat > 5u) pat = 0u;
    const uint32_t sb = (signs[gi >> 2] >> (2 * (gi & 3))) & 3u;
    word |= (pat | (((~sb) & 3u) << 3)) << (5 * q);
  }
  meta[wid] = word;
}

hipError_t launch_sp24_cpu_to_gpu(const uint8_t *patterns, const uint8_t *signs, int N, int K, uint32_t *meta,
                                  hipStream_t stream) {
  const uint32_t gpr = (uint32_t)K / 4, wpr = (gpr + 5) / 6;
  const size_t words = (size_t)N * wpr;
  if (words == 0) return hipSuccess;
  const size_t blocks = (words + 255) / 256;
  hipLaunchKernelGGL(sp24_cpu_to_gpu_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, patterns, signs,
                     (uint32_t)N, gpr, wpr, meta);
  return hipGetLastError();
}

// ---- on-device quantisation: f32 or bf16 weights -> packed codes + scales --
//
// quantize_ternary (src/model/ternary.rs:31-57: alpha = mean|w| /
// ABSMEAN_NORM, 1 for an all-zero input; q = clamp(round(w * (1 / alpha)),
// -1, 1), round half away from zero; used by BitLinear::requantize,
// src/training/shadow_weights.rs:152-160) and the on-the-fly rule of
// BitLinear::forward_ste (shadow_weights.rs:203-231: alpha = mean|w|; q = +1
// where w / alpha > 0.5, -1 where < -0.5, else 0; all 0 when alpha < 1e-10),
// each applied to every row of W [N][K] on its own; a single row of n values
// is the reference's call on a whole tensor. bf16 weights (bf16 shadows) are
// widened exactly, as P::to_f32 does.
// Scale. The reference sums |w| left to right in f32, and that order fixes
// the rounding, so one lane adds its row in exactly that order from LDS while
// the rest of its wave stages the next 1024 values with coalesced loads; one
// workgroup (one wave) per row. Codes: one thread per u32 word, -1 / 0 / +1
// -> codes 0 / 1 / 2, sixteen per word LSB first (pack_ternary with
// pack_ternary_u32's word order, ternary.rs:134-163,1317-1328).
constexpr float QUANT_ABSMEAN_NORM = 0.7978845608f;  // sqrt(2 / pi), ternary.rs:15
constexpr uint32_t QUANT_CHUNK = 1024;               // values per staged chunk

__device__ __forceinline__ float quant_widen(const float *p, size_t i) { return p[i]; }
__device__ __forceinline__ float quant_widen(const uint16_t *p, size_t i) {
  return __uint_as_float((uint32_t)p[i] << 16);
}

template <typename WT>
__global__ __launch_bounds__(64) void quant_scale_kernel(const WT *__restrict__ W, uint32_t K, int rule,
                                                        float *__restrict__ scale) {
  __shared__ __align__(16) float buf[2][QUANT_CHUNK];
  const int lane = threadIdx.x;
  const WT *row = W + (size_t)blockIdx.x * K;
  const uint32_t nch = (K + QUANT_CHUNK - 1) / QUANT_CHUNK;
  float v[QUANT_CHUNK / 64];
  auto load = [&](uint32_t c) {
#pragma unroll
    for (uint32_t j = 0; j < QUANT_CHUNK / 64; j++) {
      const uint32_t i = c * QUANT_CHUNK + j * 64 + (uint32_t)lane;
      v[j] = i < K ? quant_widen(row, i) : 0.0f;
    }
  };
  auto store = [&](uint32_t c) {
#pragma unroll
    for (uint32_t j = 0; j < QUANT_CHUNK / 64; j++) buf[c & 1][j * 64 + lane] = v[j];
  };
  load(0);
  store(0);
  __syncthreads();
  float sum = 0.0f;
  for (uint32_t c = 0; c < nch; c++) {
    if (c + 1 < nch) load(c + 1);  // in flight during the additions
    if (lane == 0) {
      const uint32_t n = min(QUANT_CHUNK, K - c * QUANT_CHUNK);
      const float *b = buf[c & 1];
      for (uint32_t i = 0; i < n; i++) sum = sum + fabsf(b[i]);  // adds only: nothing to contract
    }
    if (c + 1 < nch) store(c + 1);  // the other buffer (read during the previous chunk)
    __syncthreads();
  }
  if (lane == 0) {
    const float mean = sum / (float)K;
    // quantize_ternary: sum_abs > 0 (false for NaN) selects the absmean
    scale[blockIdx.x] = rule == 0 ? (sum > 0.0f ? mean / QUANT_ABSMEAN_NORM : 1.0f) : mean;
  }
}

template <typename WT>
__global__ __launch_bounds__(256) void quant_pack_kernel(const WT *__restrict__ W, uint32_t N, uint32_t K, int rule,
                                                        const float *__restrict__ scale,
                                                        uint32_t *__restrict__ packed) {
  const size_t wid = (size_t)blockIdx.x * 256 + threadIdx.x;
  const uint32_t wpr = K / 16;
  if (wid >= (size_t)N * wpr) return;
  const float alpha = scale[wid / wpr];
  const float inv = 1.0f / alpha;
  uint32_t word = 0;
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const float w = quant_widen(W, wid * 16 + j);
    int q;
    if (rule == 0) {
      // (w * inv).round() as i32, clamped: NaN -> 0, +-inf saturate
      const float r = roundf(w * inv);
      q = r >= 1.0f ? 1 : r <= -1.0f ? -1 : 0;
    } else {
      const float t = w / alpha;  // NaN compares false -> 0
      q = alpha < 1e-10f ? 0 : t > 0.5f ? 1 : t < -0.5f ? -1 : 0;
    }
    word |= (uint32_t)(q + 1) << (2 * j);
  }
  packed[wid] = word;
}

hipError_t launch_quantize(const void *w, int wt_bf16, int N, int K, int rule, uint32_t *packed, float *scale,
                           hipStream_t stream) {
  if (N == 0) return hipSuccess;
  if (wt_bf16)
    hipLaunchKernelGGL(quant_scale_kernel<uint16_t>, dim3((unsigned)N), dim3(64), 0, stream,
                       reinterpret_cast<const uint16_t *>(w), (uint32_t)K, rule, scale);
  else
    hipLaunchKernelGGL(quant_scale_kernel<float>, dim3((unsigned)N), dim3(64), 0, stream,
                       reinterpret_cast<const float *>(w), (uint32_t)K, rule, scale);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t words = (size_t)N * (K / 16);
  const unsigned blocks = (unsigned)((words + 255) / 256);
  if (wt_bf16)
    hipLaunchKernelGGL(quant_pack_kernel<uint16_t>, dim3(blocks), dim3(256), 0, stream,
                       reinterpret_cast<const uint16_t *>(w), (uint32_t)N, (uint32_t)K, rule, scale, packed);
  else
    hipLaunchKernelGGL(quant_pack_kernel<float>, dim3(blocks), dim3(256), 0, stream,
                       reinterpret_cast<const float *>(w), (uint32_t)N, (uint32_t)K, rule, scale, packed);
  return hipGetLastError();
}

}  // namespace frx
