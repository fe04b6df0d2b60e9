// frx_bench_read.hip — measurement helper for bench.py (libfrx_bench.so), not
// part of the ternary path.
//
// frxb_read: a plain streaming read of a buffer, the ceiling a decode GEMV
// launch of the same bytes can approach. Two workgroups of 8 waves per
// compute unit; each wave streams its own contiguous share of the buffer in
// 1 KB units (16 bytes per lane), eight units in flight per lane, and
// XOR-folds the words (one store, under a condition the data never meets,
// keeps the loads live). Units past a wave's share are not loaded (a
// wave-uniform branch), so a wave whose share is under eight units issues
// no extra reads. No decode,
// no arithmetic, no reduction: what is left of a launch is dispatch, the
// first HBM round trip and the streaming.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int RD_WAVES = 8, RD_UNITS = 8;
constexpr size_t RD_MAX = 0x80000000u;  // bytes read at most (unit indices fit 32 bits)

__global__ __launch_bounds__(RD_WAVES * 64) void read_kernel(const u32x4 *__restrict__ p, uint32_t nu,
                                                            uint32_t *__restrict__ sink) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t waves = gridDim.x * RD_WAVES, t = blockIdx.x * RD_WAVES + wave;
  const uint32_t a = (uint32_t)((uint64_t)t * nu / waves), b = (uint32_t)((uint64_t)(t + 1) * nu / waves);
  uint32_t acc = 0;
  for (uint32_t u0 = a; u0 < b; u0 += RD_UNITS) {
    u32x4 v[RD_UNITS];
#pragma unroll
    for (int u = 0; u < RD_UNITS; u++) {
      v[u] = (u32x4){0u, 0u, 0u, 0u};
      if (u0 + u < b) v[u] = p[(size_t)(u0 + u) * 64 + lane];  // wave-uniform
    }
#pragma unroll
    for (int u = 0; u < RD_UNITS; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}
}  // namespace

extern "C" {
// Reads `bytes` (a multiple of 1024, under 2 GiB) at the 16-byte aligned device address p
// on `stream`; sink: device buffer of at least frxb_read_grid() words.
int frxb_read_grid(void) {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  return 2 * cus;
}

int frxb_read(const void *p, size_t bytes, uint32_t *sink, void *stream) {
  if (!p || !sink || bytes == 0 || (bytes & 1023) != 0 || bytes >= RD_MAX ||
      (reinterpret_cast<uintptr_t>(p) & 15) != 0)
    return 1;
  hipLaunchKernelGGL(read_kernel, dim3(frxb_read_grid()), dim3(RD_WAVES * 64), 0,
                     reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const u32x4 *>(p),
                     (uint32_t)(bytes / 1024), sink);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
}
