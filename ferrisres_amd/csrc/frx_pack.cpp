// frx_pack.cpp — host-side packers of libfrx_ternary.so (no GPU needed).
// Bit-exact with the reference packers; each cites the function it mirrors.
#include <string.h>

#include "../../include/frx_ternary.h"

namespace {
// src/model/ternary.rs:134-140
inline uint8_t encode(int8_t v) { return v == -1 ? 0u : v == 1 ? 2u : 1u; }
const int8_t kDecode[4] = {-1, 0, 1, 0};
// src/compute/kernels/sparse_ternary.rs:20-27 / src/model/sparse_ternary.rs:27-34
const uint8_t kPattern[6][2] = {{0, 1}, {0, 2}, {0, 3}, {1, 2}, {1, 3}, {2, 3}};
int pattern_of(int a, int b) {
  for (int p = 0; p < 6; p++)
    if (kPattern[p][0] == a && kPattern[p][1] == b) return p;
  return -1;
}
}  // namespace

extern "C" {

// pack_ternary, src/model/ternary.rs:146-163
frx_status frx_pack_ternary_u8(const int8_t *values, size_t n, uint8_t *out) {
  if ((!values || !out) && n) return FRX_ERR_SHAPE;
  memset(out, 0, (n + 3) / 4);
  for (size_t i = 0; i < n; i++) out[i >> 2] |= (uint8_t)(encode(values[i]) << ((i & 3) * 2));
  return FRX_OK;
}

// unpack_ternary, src/model/ternary.rs:168-179
frx_status frx_unpack_ternary_u8(const uint8_t *packed, size_t n, int8_t *out) {
  if ((!packed || !out) && n) return FRX_ERR_SHAPE;
  for (size_t i = 0; i < n; i++) out[i] = kDecode[(packed[i >> 2] >> ((i & 3) * 2)) & 3];
  return FRX_OK;
}

// pack_ternary_u32, src/model/ternary.rs:1317-1328 (flat, little endian)
frx_status frx_repack_u8_to_u32(const uint8_t *packed, size_t n_values, uint32_t *out) {
  if ((!packed || !out) && n_values) return FRX_ERR_SHAPE;
  const size_t nbytes = (n_values + 3) / 4, words = (n_values + 15) / 16;
  for (size_t i = 0; i < words; i++) {
    uint32_t w = 0;
    for (size_t b = 0; b < 4; b++) {
      const size_t idx = 4 * i + b;
      w |= (uint32_t)(idx < nbytes ? packed[idx] : 0u) << (8 * b);
    }
    out[i] = w;
  }
  return FRX_OK;
}

// gpu_packed, src/model/cpu_linear.rs:164-169 / cpu_moe.rs:73-78: the flat
// u8 pack regrouped into u32 words (row aligned because K % 16 == 0) and the
// tensor scale broadcast to every row.
frx_status frx_gpu_packed(const int8_t *values, uint32_t N, uint32_t K, float tensor_scale, uint32_t *w_out,
                          float *scales_out) {
  if (!values || !w_out || !scales_out) return FRX_ERR_SHAPE;
  if (K % 16 != 0) return FRX_ERR_SHAPE;
  const size_t n = (size_t)N * K, words = n / 16;
  for (size_t i = 0; i < words; i++) {
    uint32_t w = 0;
    for (int b = 0; b < 16; b++) w |= (uint32_t)encode(values[16 * i + b]) << (2 * b);
    w_out[i] = w;
  }
  for (uint32_t r = 0; r < N; r++) scales_out[r] = tensor_scale;
  return FRX_OK;
}

// pack_sparse_ternary, src/compute/kernels/sparse_ternary.rs:254-318
frx_status frx_pack_sparse24_gpu(const int8_t *w, uint32_t N, uint32_t K, uint32_t *meta, float *scales) {
  if (!w || !meta) return FRX_ERR_SHAPE;
  const size_t gpr = (K + 3) / 4, wpr = (gpr + 5) / 6;
  memset(meta, 0, (size_t)N * wpr * 4);
  for (size_t r = 0; r < N; r++) {
    float row_sum = 0.0f;
    size_t row_count = 0;
    for (size_t g = 0; g < gpr; g++) {
      int pos[2] = {0, 0}, n = 0;
      int8_t val[2] = {0, 0};
      for (int i = 0; i < 4; i++) {
        const size_t col = g * 4 + i;
        if (col >= K) continue;
        const int8_t v = w[r * K + col];
        if (v != 0) {
          if (n < 2) {
            pos[n] = i;
            val[n] = v;
          }
          n++;
          row_sum += v < 0 ? (float)-v : (float)v;
          row_count++;
        }
      }
      if (n != 2) return FRX_ERR_SHAPE;
      const int pat = pattern_of(pos[0], pos[1]);
      if (pat < 0) return FRX_ERR_SHAPE;
      const uint32_t sg = (val[0] < 0 ? 1u : 0u) | ((val[1] < 0 ? 1u : 0u) << 1);
      meta[r * wpr + g / 6] |= ((uint32_t)pat | (sg << 3)) << ((g % 6) * 5);
    }
    if (scales) scales[r] = row_count > 0 ? row_sum / (float)row_count : 1.0f;
  }
  return FRX_OK;
}

// CPU SparseTernaryMatrix layout (src/model/sparse_ternary.rs:52-70: flat
// group index r*K/4+g, pattern nibble at bits 0-2 / 4-6, sign pair at
// 2*(g%4) with bit 1 = +1) -> GPU layout (row-aligned words of six 5-bit
// groups, bit 1 = -1). Pattern ids 6/7 (never produced) become pattern 0,
// as SparseTernaryMatrix::to_ternary decodes them (sparse_ternary.rs:172-176),
// so both layouts decode to the same matrix.
frx_status frx_sparse24_cpu_to_gpu(const uint8_t *patterns, const uint8_t *signs, uint32_t N, uint32_t K,
                                   uint32_t *meta) {
  if (!patterns || !signs || !meta) return FRX_ERR_SHAPE;
  if (K % 4 != 0) return FRX_ERR_SHAPE;
  const size_t gpr = K / 4, wpr = (gpr + 5) / 6;
  memset(meta, 0, (size_t)N * wpr * 4);
  for (size_t r = 0; r < N; r++) {
    for (size_t g = 0; g < gpr; g++) {
      const size_t gi = r * gpr + g;
      uint32_t pat = (gi % 2 == 0) ? (patterns[gi / 2] & 7u) : ((patterns[gi / 2] >> 4) & 7u);
      if (pat > 5u) pat = 0u;  // to_ternary's fallback (sparse_ternary.rs:172-176)
      const uint32_t sb = (signs[gi / 4] >> ((gi % 4) * 2)) & 3u;
      const uint32_t neg = (~sb) & 3u;  // polarity flip: CPU 1 = +1, GPU 1 = -1
      meta[r * wpr + g / 6] |= (pat | (neg << 3)) << ((g % 6) * 5);
    }
  }
  return FRX_OK;
}

// ternary_sparse_indices (src/model/ternary.rs:681-707) as CSR arrays: the
// +1 and -1 columns of each row in column order; offsets only when the index
// arrays are NULL.
frx_status frx_ternary_sparse_indices(const int8_t *values, uint32_t N, uint32_t K, uint32_t *pos_off,
                                      uint32_t *pos_idx, uint32_t *neg_off, uint32_t *neg_idx) {
  if (!values || !pos_off || !neg_off) return FRX_ERR_SHAPE;
  if ((size_t)N * K > 0xFFFFFFFFull) return FRX_ERR_SHAPE;
  uint32_t np = 0, nn = 0;
  for (size_t r = 0; r < N; r++) {
    pos_off[r] = np;
    neg_off[r] = nn;
    const int8_t *row = values + r * K;
    for (uint32_t j = 0; j < K; j++) {
      if (row[j] == 1) {
        if (pos_idx) pos_idx[np] = j;
        np++;
      } else if (row[j] == -1) {
        if (neg_idx) neg_idx[nn] = j;
        nn++;
      }
    }
  }
  pos_off[N] = np;
  neg_off[N] = nn;
  return FRX_OK;
}

}  // extern "C"
