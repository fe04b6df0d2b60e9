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

}  // namespace frx
