// frx_device.hpp — device-side building blocks shared by the gfx950 kernels.
//
// Operand encoding. A 2-bit code c in {0:-1, 1:0, 2:+1, 3:0}
// (src/model/ternary.rs:134-140) maps to the bf16 bit pattern
// ((~c) & 3) << 14:
//     c=0 -> 0xC000 = -2.0    c=1 -> 0x8000 = -0.0
//     c=2 -> 0x4000 = +2.0    c=3 -> 0x0000 = +0.0
// i.e. exactly 2*dec(c), code 3 included. Products with bf16 activations are
// exact in the MFMA's fp32 datapath; the factor 2 is removed by scaling the
// per-row scale by 0.5 in the epilogue (exact: a power of two).
//
// K-interleave. Inside a 16-code word, codes i and i+8 sit at bits 2i and
// 2i+16, so one shift and one AND place both in the sign/exponent bits of the
// two bf16 halves of a dword:  pair_i = (~w << (14 - 2i)) & 0xC000C000.
// The MFMA sums over k, so any k order is valid as long as both operands use
// the same one: activations are staged with the matching order, i.e. within
// each 16-column block dword i holds (x[i], x[i+8]).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace frx {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4 mfma16(const u32x4 &a, const u32x4 &b,
                                        const f32x4 &c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
      __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
      0);
}

// Pairs 4h..4h+3 of an inverted 16-code word as MFMA bf16 operand dwords.
template <int H>
__device__ __forceinline__ u32x4 unpack_half(uint32_t nw) {
  u32x4 r;
  r.x = (nw << (14 - 2 * (4 * H + 0))) & 0xC000C000u;
  r.y = (nw << (14 - 2 * (4 * H + 1))) & 0xC000C000u;
  r.z = (nw << (14 - 2 * (4 * H + 2))) & 0xC000C000u;
  r.w = (nw << (14 - 2 * (4 * H + 3))) & 0xC000C000u;
  return r;
}

// Same pairs from the raw (non-inverted) word: ~(w << s) & mask equals
// (~w << s) & mask for s <= 14 because the mask keeps only bits 14-15 and
// 30-31; mask = 0xC000C000, or 0 to zero the operand. One shift plus one
// three-input bit op (v_bitop3) per pair.
template <int H>
__device__ __forceinline__ u32x4 unpack_half_m(uint32_t w, uint32_t mask) {
  u32x4 r;
  r.x = ~(w << (14 - 2 * (4 * H + 0))) & mask;
  r.y = ~(w << (14 - 2 * (4 * H + 1))) & mask;
  r.z = ~(w << (14 - 2 * (4 * H + 2))) & mask;
  r.w = ~(w << (14 - 2 * (4 * H + 3))) & mask;
  return r;
}

// Round-to-nearest-even f32 -> bf16 (NaN stays NaN).
__device__ __forceinline__ uint32_t bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

// bf16_rne without a branch (select instead of early return), for unrolled
// epilogues where a per-value branch would multiply the code size.
__device__ __forceinline__ uint32_t bf16_rne_nb(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  return (u & 0x7FFFFFFFu) > 0x7F800000u ? ((u >> 16) | 0x40u) : r;
}

__device__ __forceinline__ float bf16_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// Split f32 into bf16 hi + lo with |x - hi - lo| <= 2^-17 |x| (hi carries
// infinities, lo is then 0).
__device__ __forceinline__ void split_bf16(float x, uint32_t &hi,
                                           uint32_t &lo) {
  hi = bf16_rne(x);
  float r = x - bf16_to_f32(hi);
  lo = ((hi & 0x7F80u) == 0x7F80u) ? 0u : bf16_rne(r);
}

// split_bf16 of two values at once, packed: hi = (bf16(a), bf16(b)), lo =
// (bf16(a - hi_a), bf16(b - hi_b)), a lo half zero where its hi half is not
// finite. The rounding is the hardware's packed f32 -> bf16 conversion
// (round to nearest even, as bf16_rne), about five VALU ops a value.
__device__ __forceinline__ void split2_bf16(float a, float b, uint32_t &hi, uint32_t &lo) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  hi = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
  const float ha = __uint_as_float(hi << 16), hb = __uint_as_float(hi & 0xFFFF0000u);
  const float ra = __builtin_isfinite(ha) ? a - ha : 0.0f;
  const float rb = __builtin_isfinite(hb) ? b - hb : 0.0f;
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){ra, rb}, bf16x2));
}

// Two 16-code words at once: the interleaved pairs of w0 (lo0 = pairs 0..3,
// hi0 = pairs 4..7) and of w1, pair i = ~(w << (14 - 2i)) & 0xC000C000. The
// words shift together as one 64-bit value (v_lshlrev_b64, full rate): the
// bits w0 pushes into w1's half land in bits 0..13, which the mask clears.
// 7 shifts and 16 three-input bit ops per 32 weights.
__device__ __forceinline__ void unpack32_kil(uint32_t w0, uint32_t w1, u32x4 &lo0, u32x4 &hi0, u32x4 &lo1,
                                             u32x4 &hi1) {
  const uint64_t p = ((uint64_t)w1 << 32) | w0;
  uint32_t d0[8], d1[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    uint64_t q = p;
    // the shift stays one 64-bit op (left to the compiler it becomes a
    // 32-bit shift plus a funnel shift per pair)
    if (i < 7) asm("v_lshlrev_b64 %0, %1, %2" : "=v"(q) : "n"(14 - 2 * i), "v"(p));
    d0[i] = ~(uint32_t)q & 0xC000C000u;
    d1[i] = ~(uint32_t)(q >> 32) & 0xC000C000u;
  }
  lo0 = (u32x4){d0[0], d0[1], d0[2], d0[3]};
  hi0 = (u32x4){d0[4], d0[5], d0[6], d0[7]};
  lo1 = (u32x4){d1[0], d1[1], d1[2], d1[3]};
  hi1 = (u32x4){d1[4], d1[5], d1[6], d1[7]};
}

// Natural bf16 dwords n[0..7] of a 16-column block (x0..x15) -> interleaved
// dwords d[i] = x[i] | x[i+8] << 16.
// One byte permute per output dword.
__device__ __forceinline__ void interleave16(const uint32_t n[8],
                                             uint32_t d[8]) {
#pragma unroll
  for (int j = 0; j < 4; j++) {
    d[2 * j] = __builtin_amdgcn_perm(n[j + 4], n[j], 0x05040100u);
    d[2 * j + 1] = __builtin_amdgcn_perm(n[j + 4], n[j], 0x07060302u);
  }
}

// Loads one 16-column block of activations and produces the interleaved
// bf16 dwords (hi plane; lo plane when the source is f32).
template <typename XT>
struct XBlock;

template <>
struct XBlock<uint16_t> {
  static constexpr int P = 1;
  static constexpr int NV = 2;  // 16-byte loads per block
  // Unconditional raw load of a block (src must be a valid block address);
  // finish() turns it into the staged dwords, zero when !ok. Split so that a
  // kernel can issue further loads before it consumes these.
  __device__ __forceinline__ static void load_raw(const uint16_t *src, u32x4 v[NV]) {
    const u32x4 *s = reinterpret_cast<const u32x4 *>(src);
    v[0] = s[0];
    v[1] = s[1];
  }
  __device__ __forceinline__ static void finish(const u32x4 v[NV], bool ok, uint32_t hi[8],
                                                uint32_t lo[8]) {
    (void)lo;
    const uint32_t m = ok ? 0xFFFFFFFFu : 0u;
    uint32_t n[8] = {v[0].x & m, v[0].y & m, v[0].z & m, v[0].w & m,
                     v[1].x & m, v[1].y & m, v[1].z & m, v[1].w & m};
    interleave16(n, hi);
  }
  __device__ __forceinline__ static void load(const uint16_t *src,
                                              bool ok, uint32_t hi[8],
                                              uint32_t lo[8]) {
    (void)lo;
    uint32_t n[8];
    if (ok) {
      const u32x4 *s = reinterpret_cast<const u32x4 *>(src);
      u32x4 a = s[0], b = s[1];
      n[0] = a.x; n[1] = a.y; n[2] = a.z; n[3] = a.w;
      n[4] = b.x; n[5] = b.y; n[6] = b.z; n[7] = b.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) n[i] = 0;
    }
    interleave16(n, hi);
  }
};

template <>
struct XBlock<float> {
  static constexpr int P = 2;
  static constexpr int NV = 4;
  __device__ __forceinline__ static void load_raw(const float *src, u32x4 v[NV]) {
    const u32x4 *s = reinterpret_cast<const u32x4 *>(src);
#pragma unroll
    for (int q = 0; q < 4; q++) v[q] = s[q];
  }
  __device__ __forceinline__ static void finish(const u32x4 v[NV], bool ok, uint32_t hi[8],
                                                uint32_t lo[8]) {
    uint32_t h[16], l[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const float f[4] = {__uint_as_float(v[q].x), __uint_as_float(v[q].y), __uint_as_float(v[q].z),
                          __uint_as_float(v[q].w)};
#pragma unroll
      for (int e = 0; e < 4; e++) split_bf16(ok ? f[e] : 0.0f, h[4 * q + e], l[4 * q + e]);
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
      hi[i] = h[i] | (h[i + 8] << 16);
      lo[i] = l[i] | (l[i + 8] << 16);
    }
  }
  __device__ __forceinline__ static void load(const float *src, bool ok,
                                              uint32_t hi[8], uint32_t lo[8]) {
    uint32_t h[16], l[16];
    if (ok) {
      const float4 *s = reinterpret_cast<const float4 *>(src);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        float4 v = s[q];
        split_bf16(v.x, h[4 * q + 0], l[4 * q + 0]);
        split_bf16(v.y, h[4 * q + 1], l[4 * q + 1]);
        split_bf16(v.z, h[4 * q + 2], l[4 * q + 2]);
        split_bf16(v.w, h[4 * q + 3], l[4 * q + 3]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; i++) h[i] = l[i] = 0;
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
      hi[i] = h[i] | (h[i + 8] << 16);
      lo[i] = l[i] | (l[i + 8] << 16);
    }
  }
};

// FFN activations, fp32 (the reference's f32 formulas: SiLU g/(1+e^-g),
// ternary_moe.rs:204, cpu_block_attn_res.rs:2323; GeLU-tanh,
// gemma_mapper.rs:2073-2077).
__device__ __forceinline__ float act_silu(float g) { return g / (1.0f + expf(-g)); }
// GeLU-tanh with the constant c given: 0.5 x (1 + tanh(c (x + 0.044715 x^3))).
__device__ __forceinline__ float gelu_tanh_c(float x, float c) {
  const float inner = c * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}
// gemma_mapper.rs:2073-2077: c = (2 / PI).sqrt() evaluated in f32, which is
// 0x3F4C4229, one ulp below the nearest f32 to sqrt(2/pi).
__device__ __forceinline__ float act_gelu_tanh(float x) { return gelu_tanh_c(x, __uint_as_float(0x3F4C4229u)); }
// ternary_moe.rs:196-199: the literal 0.7978845608 (0x3F4C422A).
__device__ __forceinline__ float act_gelu_tanh_lit(float x) { return gelu_tanh_c(x, 0.7978845608f); }

// Expert activation of the MoE kernels, by frx_activation: 0 silu(g) * u,
// 1 gelu_tanh(g) * u (the model glue, CpuMoELayer), 2 gelu_tanh(g) alone
// (TernaryMoELayer::forward with use_gelu, ternary_moe.rs:193-200).
__device__ __forceinline__ float moe_act(int act, float g, float u) {
  if (act == 2) return act_gelu_tanh_lit(g);
  return (act == 1 ? act_gelu_tanh(g) : act_silu(g)) * u;
}

// Output bias, added to the scaled f32 result as a separate rounding step:
// the layer computes y = (alpha * sum) + bias in two f32 operations, so the
// product must not fuse with the addition into one multiply-add.
__device__ __forceinline__ float add_bias(float v, float b) {
#pragma clang fp contract(off)
  return v + b;
}

// Bias of output rows n..n+3 (rows past N read row N-1; their stores are
// masked).
__device__ __forceinline__ f32x4 add_bias4(f32x4 v, const float *bias, int n, int N) {
#pragma unroll
  for (int j = 0; j < 4; j++) v[j] = add_bias(v[j], bias[min(n + j, N - 1)]);
  return v;
}

// Output stores of 4 consecutive columns.
template <typename YT>
struct YStore;

template <>
struct YStore<float> {
  __device__ __forceinline__ static void store4(float *dst, f32x4 v, int n_ok) {
    if (n_ok >= 4 && ((reinterpret_cast<uintptr_t>(dst) & 15) == 0)) {
      *reinterpret_cast<float4 *>(dst) = make_float4(v.x, v.y, v.z, v.w);
    } else {
      if (n_ok > 0) dst[0] = v.x;
      if (n_ok > 1) dst[1] = v.y;
      if (n_ok > 2) dst[2] = v.z;
      if (n_ok > 3) dst[3] = v.w;
    }
  }
};

template <>
struct YStore<uint16_t> {
  __device__ __forceinline__ static void store4(uint16_t *dst, f32x4 v,
                                                int n_ok) {
    uint32_t a = bf16_rne(v.x), b = bf16_rne(v.y), c = bf16_rne(v.z),
             d = bf16_rne(v.w);
    if (n_ok >= 4 && ((reinterpret_cast<uintptr_t>(dst) & 7) == 0)) {
      u32x2 p;
      p.x = a | (b << 16);
      p.y = c | (d << 16);
      *reinterpret_cast<u32x2 *>(dst) = p;
    } else {
      uint16_t *o = reinterpret_cast<uint16_t *>(dst);
      if (n_ok > 0) o[0] = (uint16_t)a;
      if (n_ok > 1) o[1] = (uint16_t)b;
      if (n_ok > 2) o[2] = (uint16_t)c;
      if (n_ok > 3) o[3] = (uint16_t)d;
    }
  }
};

}  // namespace frx
