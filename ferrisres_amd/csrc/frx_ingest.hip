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

// Scale of one block: block b covers values [b * block, min(n, (b + 1) *
// block)) of the flat array (a row of W [N][K] is a block of K; the whole
// tensor is one block of n; quantize_ternary_blocked's blocks are ragged at
// the end). One workgroup (one wave) per block.
template <typename WT>
__global__ __launch_bounds__(64) void quant_scale_kernel(const WT *__restrict__ W, size_t n, size_t block,
                                                        int rule, float *__restrict__ scale) {
  __shared__ __align__(16) float buf[2][QUANT_CHUNK];
  const int lane = threadIdx.x;
  const size_t start = (size_t)blockIdx.x * block;
  const size_t len = min(block, n - start);
  const WT *row = W + start;
  const size_t nch = (len + QUANT_CHUNK - 1) / QUANT_CHUNK;
  float v[QUANT_CHUNK / 64];
  auto load = [&](size_t c) {
#pragma unroll
    for (uint32_t j = 0; j < QUANT_CHUNK / 64; j++) {
      const size_t i = c * QUANT_CHUNK + j * 64 + (uint32_t)lane;
      v[j] = i < len ? quant_widen(row, i) : 0.0f;
    }
  };
  auto store = [&](size_t c) {
#pragma unroll
    for (uint32_t j = 0; j < QUANT_CHUNK / 64; j++) buf[c & 1][j * 64 + lane] = v[j];
  };
  load(0);
  store(0);
  __syncthreads();
  float sum = 0.0f;
  for (size_t c = 0; c < nch; c++) {
    if (c + 1 < nch) load(c + 1);  // in flight during the additions
    if (lane == 0) {
      const uint32_t m = (uint32_t)min((size_t)QUANT_CHUNK, len - c * QUANT_CHUNK);
      const float *b = buf[c & 1];
      for (uint32_t i = 0; i < m; i++) sum = sum + fabsf(b[i]);  // adds only: nothing to contract
    }
    if (c + 1 < nch) store(c + 1);  // the other buffer (read during the previous chunk)
    __syncthreads();
  }
  if (lane == 0) {
    const float mean = sum / (float)len;  // len as f32, as `block.len() as f32`
    // quantize_ternary: sum_abs > 0 (false for NaN) selects the absmean
    scale[blockIdx.x] = rule == 0 ? (sum > 0.0f ? mean / QUANT_ABSMEAN_NORM : 1.0f) : mean;
  }
}

// Codes of 16 consecutive values of the flat array per thread (one u32 word
// of pack_ternary_u32); value i uses the scale of block i / block. Values past
// n are the zero padding bits of pack_ternary (code 0b00).
template <typename WT>
__global__ __launch_bounds__(256) void quant_pack_kernel(const WT *__restrict__ W, size_t n, size_t block, int rule,
                                                        const float *__restrict__ scale,
                                                        uint32_t *__restrict__ packed) {
  const size_t wid = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (wid * 16 >= n) return;
  size_t b_cur = ~(size_t)0;
  float alpha = 1.0f, inv = 1.0f;
  uint32_t word = 0;
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const size_t i = wid * 16 + j;
    if (i >= n) break;
    const size_t b = i / block;
    if (b != b_cur) {
      b_cur = b;
      alpha = scale[b];
      inv = 1.0f / alpha;
    }
    const float w = quant_widen(W, i);
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

hipError_t launch_quantize_flat(const void *w, int wt_bf16, size_t n, size_t block, int rule, uint32_t *packed,
                                float *scale, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const size_t nb = (n + block - 1) / block;
  if (wt_bf16)
    hipLaunchKernelGGL(quant_scale_kernel<uint16_t>, dim3((unsigned)nb), dim3(64), 0, stream,
                       reinterpret_cast<const uint16_t *>(w), n, block, rule, scale);
  else
    hipLaunchKernelGGL(quant_scale_kernel<float>, dim3((unsigned)nb), dim3(64), 0, stream,
                       reinterpret_cast<const float *>(w), n, block, rule, scale);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (!packed) return hipSuccess;
  const size_t words = (n + 15) / 16;
  const unsigned blocks = (unsigned)((words + 255) / 256);
  if (wt_bf16)
    hipLaunchKernelGGL(quant_pack_kernel<uint16_t>, dim3(blocks), dim3(256), 0, stream,
                       reinterpret_cast<const uint16_t *>(w), n, block, rule, scale, packed);
  else
    hipLaunchKernelGGL(quant_pack_kernel<float>, dim3(blocks), dim3(256), 0, stream,
                       reinterpret_cast<const float *>(w), n, block, rule, scale, packed);
  return hipGetLastError();
}

hipError_t launch_quantize(const void *w, int wt_bf16, int N, int K, int rule, uint32_t *packed, float *scale,
                           hipStream_t stream) {
  return launch_quantize_flat(w, wt_bf16, (size_t)N * (size_t)K, (size_t)K, rule, packed, scale, stream);
}

// ---- dequantize_ternary_blocked (ternary.rs:113-128) ------------------------
// out[i] = scales[i / block] * dec(code i) over the flat packed codes
// (alpha * {-1, 0, +1}, one IEEE product: exact). Codes 0b01 and 0b11 are 0
// (TERNARY_DECODE, ternary.rs:136-140).
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t *__restrict__ packed,
                                                     const float *__restrict__ scales, size_t n, size_t block,
                                                     float *__restrict__ out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const uint32_t c = (packed[i >> 4] >> (2 * (i & 15))) & 3u;
  const float d = c == 0 ? -1.0f : c == 2 ? 1.0f : 0.0f;
  out[i] = scales[i / block] * d;
}

hipError_t launch_dequantize(const uint32_t *packed, const float *scales, size_t n, size_t block, float *out,
                             hipStream_t stream) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, packed, scales, n,
                     block, out);
  return hipGetLastError();
}

// ---- prune_fp32_to_sparse_ternary (sparse_ternary.rs:598-663) -----------------
// One group of four values: the two largest |v| by the reference's stable
// sort_by (an insertion sort on four elements: a value moves left only past
// a strictly smaller |v|, so ties keep the lower position and a NaN moves
// past nothing). pat = pattern of the ordered positions; s0 / s1 = 1 when the
// LARGEST / second largest value is >= 0: the reference packs the sign bits
// in magnitude order (:642-644) while decoding reads bit 0 as the lower
// position's sign, and this keeps that.
__device__ __forceinline__ void prune_group(const float v[4], uint32_t &pat, uint32_t &s0, uint32_t &s1) {
  int idx[4] = {0, 1, 2, 3};
#pragma unroll
  for (int i = 1; i < 4; i++) {
#pragma unroll
    for (int j = i; j > 0; j--) {
      // adjacent swap while the later element is strictly larger in |v|
      if (fabsf(v[idx[j]]) > fabsf(v[idx[j - 1]])) {
        const int t = idx[j];
        idx[j] = idx[j - 1];
        idx[j - 1] = t;
      } else {
        break;
      }
    }
  }
  const int a = idx[0], b = idx[1];
  const int p0 = min(a, b), p1 = max(a, b);
  // SPARSE_PATTERN (sparse_ternary.rs:27-34): (0,1)(0,2)(0,3)(1,2)(1,3)(2,3)
  pat = p0 == 0 ? (uint32_t)(p1 - 1) : p0 == 1 ? (uint32_t)(p1 + 1) : 5u;
  s0 = v[a] >= 0.0f ? 1u : 0u;
  s1 = v[b] >= 0.0f ? 1u : 0u;
}

template <typename WT>
__device__ __forceinline__ void load_group(const WT *w, size_t g, float v[4]) {
#pragma unroll
  for (int j = 0; j < 4; j++) v[j] = quant_widen(w, 4 * g + j);
}

// CPU layout: thread t owns flat groups 4t .. 4t+3, i.e. pattern bytes 2t
// and 2t+1 and sign byte t, so no byte is shared between threads.
template <typename WT>
__global__ __launch_bounds__(256) void prune_cpu_kernel(const WT *__restrict__ w, size_t ng,
                                                       uint8_t *__restrict__ patterns,
                                                       uint8_t *__restrict__ signs) {
  const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (4 * t >= ng) return;
  uint32_t pb[2] = {0, 0}, sb = 0;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const size_t g = 4 * t + q;
    if (g >= ng) break;
    float v[4];
    load_group(w, g, v);
    uint32_t pat, s0, s1;
    prune_group(v, pat, s0, s1);
    pb[q >> 1] |= pat << (4 * (q & 1));
    sb |= (s0 | (s1 << 1)) << (2 * q);
  }
  patterns[2 * t] = (uint8_t)pb[0];
  if (2 * t + 1 < (ng + 1) / 2) patterns[2 * t + 1] = (uint8_t)pb[1];
  signs[t] = (uint8_t)sb;
}

// GPU layout: one thread per row word (six groups, bit 3 / bit 4 set when
// the lower / higher position decodes to -1), the same bits the transcoder
// writes from the CPU layout.
template <typename WT>
__global__ __launch_bounds__(256) void prune_gpu_kernel(const WT *__restrict__ w, uint32_t N, uint32_t gpr,
                                                       uint32_t wpr, uint32_t *__restrict__ meta) {
  const size_t wid = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (wid >= (size_t)N * wpr) return;
  const size_t r = wid / wpr;
  const uint32_t j = (uint32_t)(wid - r * wpr);
  uint32_t word = 0;
  for (uint32_t q = 0; q < 6; q++) {
    const uint32_t g = j * 6 + q;
    if (g >= gpr) break;
    float v[4];
    load_group(w, r * gpr + g, v);
    uint32_t pat, s0, s1;
    prune_group(v, pat, s0, s1);
    word |= (pat | ((s0 ^ 1u) << 3) | ((s1 ^ 1u) << 4)) << (5 * q);
  }
  meta[wid] = word;
}

__global__ void broadcast_first_kernel(float *__restrict__ v, uint32_t n) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x + 1;
  if (i < n) v[i] = v[0];
}

template <typename WT>
static hipError_t launch_prune_t(const WT *w, int N, int K, int per_row, uint8_t *patterns, uint8_t *signs,
                                 uint32_t *meta, float *scale, hipStream_t stream) {
  const size_t n = (size_t)N * (size_t)K;
  if (n == 0) return hipSuccess;
  const size_t ng = n / 4;
  if (patterns) {
    const size_t threads = (ng + 3) / 4;
    hipLaunchKernelGGL(prune_cpu_kernel<WT>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, w, ng,
                       patterns, signs);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (meta) {
    const uint32_t gpr = (uint32_t)K / 4, wpr = (gpr + 5) / 6;
    const size_t words = (size_t)N * wpr;
    hipLaunchKernelGGL(prune_gpu_kernel<WT>, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, stream, w,
                       (uint32_t)N, gpr, wpr, meta);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  // the reference's per-tensor absmean (rule 0 of the quantiser), or one
  // per row; the tensor scale is then copied to every row
  hipError_t e = launch_quantize_flat(w, sizeof(WT) == 2, n, per_row ? (size_t)K : n, 0, nullptr, scale, stream);
  if (e != hipSuccess || per_row || N <= 1) return e;
  hipLaunchKernelGGL(broadcast_first_kernel, dim3((unsigned)((N - 1 + 255) / 256)), dim3(256), 0, stream, scale,
                     (uint32_t)N);
  return hipGetLastError();
}

hipError_t launch_prune_sparse24(const void *w, int wt_bf16, int N, int K, int per_row, uint8_t *patterns,
                                 uint8_t *signs, uint32_t *meta, float *scale, hipStream_t stream) {
  if (wt_bf16)
    return launch_prune_t(reinterpret_cast<const uint16_t *>(w), N, K, per_row, patterns, signs, meta, scale,
                          stream);
  return launch_prune_t(reinterpret_cast<const float *>(w), N, K, per_row, patterns, signs, meta, scale, stream);
}

}  // namespace frx
