// frx_bench_read.hip — measurement helpers for bench.py (libfrx_bench.so), not
// part of the ternary path.
//
// frxb_read: a plain streaming read of a buffer, the ceiling a decode GEMV
// launch of the same bytes can approach. Two workgroups of 8 waves per
// compute unit; each wave streams its own contiguous share of the buffer in
// 1 KB units (16 bytes per lane), issuing up to RD_UNITS = 28 units before it
// consumes any: every share up to 28 units (buffers up to 112 MiB on 256
// compute units: the whole weight-size sweep) is one batch with all of its
// loads in flight at once, and larger shares drain only every 28 units. 28
// units (112 VGPRs) keep both workgroups of a compute unit resident.
// Units past the share are not loaded (wave-uniform branches). The words
// are XOR-folded (one store, under a condition the data never meets, keeps
// the loads live). No decode, no arithmetic, no reduction: what is left of
// a launch is dispatch, the first HBM round trip and the streaming.
//
// frxb_mfma: back-to-back v_mfma_f32_16x16x32_bf16 on register operands,
// eight independent accumulators per wave, four waves per compute unit (one
// per SIMD) or eight: the matrix pipe's sustained rate on this device at
// its clock under this load, with no memory traffic at all.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
constexpr int RD_WAVES = 8, RD_UNITS = 28;
constexpr size_t RD_MAX = 0x80000000u;  // bytes read at most (unit indices fit 32 bits)

__global__ __launch_bounds__(RD_WAVES * 64) void read_kernel(const u32x4 *__restrict__ p, uint32_t nu,
                                                            uint32_t *__restrict__ sink) {
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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

template <int NACC>
__global__ __launch_bounds__(512) void mfma_kernel(int iters, float *__restrict__ sink) {
  const int lane = threadIdx.x & 63;
  bf16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    a[i] = (__bf16)(float)((lane + i) & 7);
    b[i] = (__bf16)(float)((lane * 3 + i) & 7);
  }
  f32x4 acc[NACC];
#pragma unroll
  for (int j = 0; j < NACC; j++) acc[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int j = 0; j < NACC; j++) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[j], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NACC; j++) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  if (s == -1.0f) sink[blockIdx.x] = s;
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

// `iters` x 8 MFMAs (16x16x32 bf16, 16384 flop each) per wave, one
// workgroup per compute unit of waves_per_cu (4 or 8) waves; returns 0 when
// launched. Flops = CUs * waves_per_cu * iters * 8 * 16384. sink: at least
// frxb_read_grid() floats.
int frxb_mfma(int iters, int waves_per_cu, float *sink, void *stream) {
  if (iters <= 0 || !sink || (waves_per_cu != 4 && waves_per_cu != 8)) return 1;
  const int g = frxb_read_grid() / 2;
  hipLaunchKernelGGL((mfma_kernel<8>), dim3(g), dim3(64 * waves_per_cu), 0, reinterpret_cast<hipStream_t>(stream),
                     iters, sink);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
}
