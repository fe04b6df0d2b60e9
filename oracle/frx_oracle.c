/*
 * frx_oracle.c — CPU restatement of FerrisRes's 1.58-bit ternary linear path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker and the timed CPU baseline).
 * The product library libfrx_ternary.so never links or calls this file.
 *
 * Build: gcc -O2 -std=c11 -ffp-contract=off -fno-fast-math (oracle/Makefile).
 * -ffp-contract=off matters: Rust never contracts a*b+c into an FMA, so the
 * restatement must not either, or the rounding sequence diverges.
 *
 * Parity pinning. Each function below names the checks that pin it (tests in
 * tests/test_oracle_*.py): the reference's own known-answer tests (KATs,
 * transcribed as data into tests/golden/reference_kats.json), closed-form
 * invariants, and brute force in float64 on small inputs. The reference is
 * Rust and no Rust toolchain exists here, so the reference itself cannot be
 * built or run; the bit-level f32 rounding sequence
 * of the Rust build is therefore matched by construction (same loop order,
 * same libm) and pinned only by the KATs, which the reference checks at 1e-5.
 */
#include "frx_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ternary.rs:134-140 — {-1 -> 0b00, 0 -> 0b01, +1 -> 0b10}; 0b11 decodes 0. */
static const uint8_t TERNARY_ENCODE[3] = {0x0, 0x1, 0x2};
static const int8_t TERNARY_DECODE[4] = {-1, 0, 1, 0};

/* ternary.rs:15 */
#define ABSMEAN_NORM 0.7978845608f

/*
 * ternary.rs:146-163 pack_ternary. Value i goes to byte i/4 at bit 2*(i%4);
 * out-of-range values are packed as code 01 (zero). `out` holds (n+3)/4
 * bytes. Pinned by: KATs ternary.rs:797-822 (roundtrip, 3-value, single
 * values) and :951-959 (1024-value cycle); bit-spec property test.
 */
void frxo_pack_ternary(const int8_t *values, size_t n, uint8_t *out) {
  size_t packed_len = (n + 3) / 4;
  memset(out, 0, packed_len);
  for (size_t i = 0; i < n; i++) {
    int8_t v = values[i];
    uint8_t code;
    if (v == -1)
      code = TERNARY_ENCODE[0];
    else if (v == 0)
      code = TERNARY_ENCODE[1];
    else if (v == 1)
      code = TERNARY_ENCODE[2];
    else
      code = TERNARY_ENCODE[1];
    out[i / 4] |= (uint8_t)(code << ((i % 4) * 2));
  }
}

/* ternary.rs:168-179 unpack_ternary (LUT decode, 0b11 -> 0). Pinned as above. */
void frxo_unpack_ternary(const uint8_t *packed, size_t n, int8_t *out) {
  for (size_t i = 0; i < n; i++) {
    uint8_t code = (packed[i / 4] >> ((i % 4) * 2)) & 0x3;
    out[i] = TERNARY_DECODE[code];
  }
}

/*
 * ternary.rs:1317-1328 pack_ternary_u32: little-endian regroup of 4 bytes
 * into one u32 (16 codes), flat over the tensor, missing bytes read as 0.
 * Pinned by: KAT kernels/ternary_matmul.rs:362-381 (17 values, code per
 * index) via the pack_rows_u32 equivalence when cols % 16 == 0, and the
 * closed form (byte j of word i == packed_u8[4i+j]).
 */
void frxo_pack_ternary_u32(const uint8_t *packed_u8, size_t packed_len,
                           size_t total_values, uint32_t *out) {
  size_t words = (total_values + 15) / 16;
  for (size_t i = 0; i < words; i++) {
    uint32_t w = 0;
    for (size_t b = 0; b < 4; b++) {
      size_t idx = i * 4 + b;
      uint32_t byte = idx < packed_len ? packed_u8[idx] : 0u;
      w |= byte << (8 * b);
    }
    out[i] = w;
  }
}

/*
 * kernels/ternary_matmul.rs:268-292 (test packer): row-aligned u32 packing,
 * cols_packed = ceil(cols/16) words per row, unused trailing codes are 00.
 * Values outside {-1,0,1} pack as code 3. Pinned by KAT :362-381.
 */
void frxo_pack_rows_u32(const int8_t *values, size_t rows, size_t cols,
                        uint32_t *out) {
  size_t cp = (cols + 15) / 16;
  for (size_t r = 0; r < rows; r++) {
    for (size_t p = 0; p < cp; p++) {
      uint32_t word = 0;
      for (size_t b = 0; b < 16; b++) {
        size_t col = p * 16 + b;
        if (col >= cols) break;
        int8_t v = values[r * cols + col];
        uint32_t code = v == -1 ? 0u : v == 0 ? 1u : v == 1 ? 2u : 3u;
        word |= code << (b * 2);
      }
      out[r * cp + p] = word;
    }
  }
}

/*
 * kernels/ternary_matmul.rs:233-265 (ternary_matmul_ref), identical to the
 * model's CPU fallback cpu_block_attn_res.rs:2373-2398 and to the WGSL
 * kernel :50-74: one sequential f32 accumulator per (s, r); code 0 -> sum -=
 * x, code 2 -> sum += x, codes 1/3 skipped; out = sum * scale[r].
 * Pinned by: KATs kernels/ternary_matmul.rs:294-360 (identity, negate,
 * scaled, batch); dyadic-input exactness (all partial sums exact in f32 ->
 * equals float64 brute force bit-for-bit); float64 brute force on random
 * small shapes.
 */
void frxo_ternary_matmul_u32(const uint32_t *packed, const float *scales,
                             const float *input, size_t seq, size_t in_cols,
                             size_t out_rows, float *out) {
  size_t cp = (in_cols + 15) / 16;
  for (size_t s = 0; s < seq; s++) {
    for (size_t r = 0; r < out_rows; r++) {
      float sum = 0.0f;
      for (size_t p = 0; p < cp; p++) {
        uint32_t word = packed[r * cp + p];
        for (size_t b = 0; b < 16; b++) {
          size_t col = p * 16 + b;
          if (col >= in_cols) break;
          uint32_t code = (word >> (b * 2)) & 3u;
          float x = input[s * in_cols + col];
          if (code == 0u)
            sum -= x;
          else if (code == 2u)
            sum += x;
        }
      }
      out[s * out_rows + r] = sum * scales[r];
    }
  }
}

/*
 * ternary.rs:292-328 ternary_matmul: split positive/negative accumulators,
 * out = scale * (pos - neg). Pinned by KATs ternary.rs:963-1019 (identity,
 * scale -2 -> -20, 2x3 batch -> all -1) and :1255-1261 (all zeros).
 */
void frxo_ternary_matmul_i8(const int8_t *ternary, float scale,
                            const float *input, size_t out_rows,
                            size_t in_cols, size_t seq, float *out) {
  for (size_t s = 0; s < seq; s++) {
    const float *xr = input + s * in_cols;
    for (size_t r = 0; r < out_rows; r++) {
      const int8_t *wr = ternary + r * in_cols;
      float pos = 0.0f, neg = 0.0f;
      for (size_t j = 0; j < in_cols; j++) {
        int8_t w = wr[j];
        float v = xr[j];
        pos += w > 0 ? v : 0.0f;
        neg += w < 0 ? v : 0.0f;
      }
      out[s * out_rows + r] = scale * (pos - neg);
    }
  }
}

/*
 * ternary.rs:591-633 ternary_matmul_decode: sum += (w as f32) * x in column
 * order (the x8 unroll does not change the order), out = scale * sum.
 * Used by TernaryMoELayer (ternary_moe.rs:56). Pinned by KATs
 * ternary.rs:1177-1205 (decode == general within 1e-5) and :1263-1297.
 */
void frxo_ternary_matmul_decode(const int8_t *ternary, float scale,
                                const float *input, size_t out_rows,
                                size_t in_cols, float *out) {
  for (size_t r = 0; r < out_rows; r++) {
    const int8_t *wr = ternary + r * in_cols;
    float sum = 0.0f;
    for (size_t j = 0; j < in_cols; j++) sum += (float)wr[j] * input[j];
    out[r] = scale * sum;
  }
}

/*
 * ternary_linear.rs:94-165 TernaryLinear::forward / forward_packed /
 * forward_decode: the layer's matmul, then out[s*out_rows + r] += bias[r]
 * for every token s (bias NULL: a layer without bias). path 0 = forward
 * (ternary_matmul on the i8 values), 1 = forward_packed (the u8 packing of
 * the same values), 2 = forward_decode (seq must be 1).
 * Pinned by the hand-computed KAT of test_ternary_linear_bias_kat (2x3
 * layer, bias [0.1, 0.2]), by bias NULL == the matmul alone, and by the
 * three paths agreeing with bias (ternary_linear.rs:258-306).
 */
void frxo_ternary_linear_forward(const int8_t *ternary, const uint8_t *packed, float scale,
                                 const float *bias, const float *input, size_t out_rows,
                                 size_t in_cols, size_t seq, int path, float *out) {
  if (path == 2) {
    seq = 1;
    frxo_ternary_matmul_decode(ternary, scale, input, out_rows, in_cols, out);
  } else if (path == 1) {
    frxo_ternary_matmul_packed(packed, scale, input, out_rows, in_cols, seq, out);
  } else {
    frxo_ternary_matmul_i8(ternary, scale, input, out_rows, in_cols, seq, out);
  }
  if (!bias) return;
  for (size_t s = 0; s < seq; s++)
    for (size_t r = 0; r < out_rows; r++) out[s * out_rows + r] += bias[r];
}

/*
 * ternary.rs:401-464 ternary_matmul_packed (u8 layout, per-tensor scale).
 * The byte index is (r*in_cols + 4q)/4 exactly as in the reference, so rows
 * with in_cols % 4 != 0 reproduce the reference's flat addressing.
 * Pinned by KATs ternary.rs:1058-1095 (== unpacked) and :1299-1312 (1x6 ->
 * -3.0).
 */
void frxo_ternary_matmul_packed(const uint8_t *packed, float scale,
                                const float *input, size_t out_rows,
                                size_t in_cols, size_t seq, float *out) {
  size_t full_quads = in_cols / 4, rem = in_cols % 4;
  for (size_t s = 0; s < seq; s++) {
    const float *xr = input + s * in_cols;
    for (size_t r = 0; r < out_rows; r++) {
      size_t row_offset = r * in_cols;
      float sum = 0.0f;
      for (size_t q = 0; q < full_quads; q++) {
        uint8_t pb = packed[(row_offset + q * 4) / 4];
        for (size_t bp = 0; bp < 4; bp++) {
          float sign = (float)TERNARY_DECODE[(pb >> (bp * 2)) & 3];
          sum += sign * xr[q * 4 + bp];
        }
      }
      if (rem > 0) {
        uint8_t pb = packed[(row_offset + full_quads * 4) / 4];
        for (size_t bp = 0; bp < rem; bp++) {
          float sign = (float)TERNARY_DECODE[(pb >> (bp * 2)) & 3];
          sum += sign * xr[full_quads * 4 + bp];
        }
      }
      out[s * out_rows + r] = scale * sum;
    }
  }
}

/*
 * ternary.rs:471-529 ternary_matmul_packed_parallel, the model's CPU decode
 * path (CS-3), for rows [row_begin, row_end) of a single token. Per byte:
 * sum += s0*x0 + s1*x1 + s2*x2 + s3*x3 (Rust evaluates the right side left to
 * right before adding it to sum). Row r starts at byte r*ceil(in_cols/4).
 * Pinned by: equality with frxo_ternary_matmul_u32 on dyadic inputs (exact
 * arithmetic) and 1e-5 agreement on random inputs.
 */
void frxo_ternary_matmul_packed_rows(const uint8_t *packed, float scale,
                                     const float *input, size_t out_rows,
                                     size_t in_cols, size_t row_begin,
                                     size_t row_end, float *out) {
  (void)out_rows;
  size_t full_quads = in_cols / 4, rem = in_cols % 4;
  size_t stride = (in_cols + 3) / 4;
  for (size_t row = row_begin; row < row_end; row++) {
    size_t start = row * stride;
    float sum = 0.0f;
    for (size_t q = 0; q < full_quads; q++) {
      uint8_t pb = packed[start + q];
      float s0 = (float)TERNARY_DECODE[pb & 3];
      float s1 = (float)TERNARY_DECODE[(pb >> 2) & 3];
      float s2 = (float)TERNARY_DECODE[(pb >> 4) & 3];
      float s3 = (float)TERNARY_DECODE[(pb >> 6) & 3];
      size_t base = q * 4;
      float t = s0 * input[base];
      t = t + s1 * input[base + 1];
      t = t + s2 * input[base + 2];
      t = t + s3 * input[base + 3];
      sum += t;
    }
    if (rem > 0) {
      uint8_t pb = packed[start + full_quads];
      size_t base = full_quads * 4;
      for (size_t bp = 0; bp < rem; bp++)
        sum += (float)TERNARY_DECODE[(pb >> (bp * 2)) & 3] * input[base + bp];
    }
    out[row] = scale * sum;
  }
}

/* ternary.rs:541-579 ternary_matmul_blocked (column-block scales). Pinned by
 * KAT ternary.rs:1097-1175 (== dequantised reference within 1e-4). */
void frxo_ternary_matmul_blocked(const int8_t *ternary, const float *scales,
                                 size_t block_size, const float *input,
                                 size_t out_rows, size_t in_cols, size_t seq,
                                 float *out) {
  size_t nb = (in_cols + block_size - 1) / block_size;
  for (size_t s = 0; s < seq; s++) {
    const float *xr = input + s * in_cols;
    for (size_t r = 0; r < out_rows; r++) {
      const int8_t *wr = ternary + r * in_cols;
      float sum = 0.0f;
      for (size_t b = 0; b < nb; b++) {
        size_t c0 = b * block_size;
        size_t c1 = c0 + block_size < in_cols ? c0 + block_size : in_cols;
        float bs = 0.0f;
        for (size_t j = c0; j < c1; j++) bs += (float)wr[j] * xr[j];
        sum += scales[b] * bs;
      }
      out[s * out_rows + r] = sum;
    }
  }
}

/*
 * ternary.rs:681-707 ternary_sparse_indices: per row, the column indices of
 * +1 entries (pos) and of -1 entries (neg), in column order; other values
 * are in neither list. Returned as CSR arrays: pos_off[r]..pos_off[r+1] index
 * pos_idx (same for neg). With pos_idx/neg_idx NULL only the offsets (the
 * list sizes) are filled. Pinned by KAT ternary.rs:1238-1254.
 */
void frxo_ternary_sparse_indices(const int8_t *ternary, size_t out_rows,
                                 size_t in_cols, uint32_t *pos_off,
                                 uint32_t *pos_idx, uint32_t *neg_off,
                                 uint32_t *neg_idx) {
  uint32_t np = 0, nn = 0;
  for (size_t r = 0; r < out_rows; r++) {
    pos_off[r] = np;
    neg_off[r] = nn;
    const int8_t *row = ternary + r * in_cols;
    for (size_t j = 0; j < in_cols; j++) {
      if (row[j] == 1) {
        if (pos_idx) pos_idx[np] = (uint32_t)j;
        np++;
      } else if (row[j] == -1) {
        if (neg_idx) neg_idx[nn] = (uint32_t)j;
        nn++;
      }
    }
  }
  pos_off[out_rows] = np;
  neg_off[out_rows] = nn;
}

/*
 * ternary.rs:647-673 ternary_matmul_sparse_decode: per row, sum += x[j] over
 * the pos list in order, then sum -= x[j] over the neg list in order; out =
 * scale * sum. Pinned by KAT ternary.rs:1208-1236 (equals the decode matmul)
 * and exactness on dyadic inputs.
 */
void frxo_ternary_matmul_sparse_decode(const uint32_t *pos_off,
                                       const uint32_t *pos_idx,
                                       const uint32_t *neg_off,
                                       const uint32_t *neg_idx, float scale,
                                       const float *input, size_t out_rows,
                                       float *out) {
  for (size_t r = 0; r < out_rows; r++) {
    float sum = 0.0f;
    for (uint32_t i = pos_off[r]; i < pos_off[r + 1]; i++) sum += input[pos_idx[i]];
    for (uint32_t i = neg_off[r]; i < neg_off[r + 1]; i++) sum -= input[neg_idx[i]];
    out[r] = scale * sum;
  }
}

/*
 * ternary.rs:725-746 ternary_stats: counts of -1 and +1, zeros = n - both,
 * ratios count as f32 / n as f32, compression 32 / 2. out: [num_neg1,
 * num_zero, num_pos1] and ratios[3] in the same order; returns the
 * compression ratio. Pinned by KAT ternary.rs:894-904.
 */
float frxo_ternary_stats(const int8_t *ternary, size_t n, uint64_t counts[3],
                         float ratios[3]) {
  uint64_t neg = 0, pos = 0;
  for (size_t i = 0; i < n; i++) {
    if (ternary[i] == -1) neg++;
    if (ternary[i] == 1) pos++;
  }
  counts[0] = neg;
  counts[1] = n - neg - pos;
  counts[2] = pos;
  for (int i = 0; i < 3; i++) ratios[i] = (float)counts[i] / (float)n;
  return 32.0f / 2.0f;
}

/*
 * benches/ternary_bench.rs:87-106 (the criterion bench's inline i8 loop):
 * weights indexed [col*k + ki] (i.e. W is [n x k] row-major), branchy
 * add/sub, c = sum * scale. Pinned by equality with frxo_ternary_matmul_u32
 * on dyadic inputs.
 */
void frxo_bench_ternary_matmul(const float *a, const int8_t *weights,
                               float scale, size_t m, size_t n, size_t k,
                               float *out) {
  for (size_t row = 0; row < m; row++) {
    for (size_t col = 0; col < n; col++) {
      float sum = 0.0f;
      for (size_t ki = 0; ki < k; ki++) {
        int8_t w = weights[col * k + ki];
        if (w > 0)
          sum += a[row * k + ki];
        else if (w < 0)
          sum -= a[row * k + ki];
      }
      out[row * n + col] = sum * scale;
    }
  }
}

/* Rust `f32 as i32` saturates and maps NaN to 0. */
static int32_t rust_f32_to_i32(float v) {
  if (v != v) return 0;
  if (v >= 2147483647.0f) return 2147483647;
  if (v <= -2147483648.0f) return (int32_t)(-2147483647 - 1);
  return (int32_t)v;
}

/*
 * ternary.rs:31-57 quantize_ternary: alpha = (sum|W| / n) / ABSMEAN_NORM
 * (1.0 when all zero), W_q = clamp(round(W / alpha)) with round half away
 * from zero (C roundf == Rust f32::round). Returns alpha. Pinned by KATs
 * ternary.rs:752-795 (values in {-1,0,1}, zero weights, sign preservation)
 * and a float64 restatement.
 */
float frxo_quantize_ternary(const float *weights, size_t n, int8_t *out) {
  if (n == 0) return 0.0f;
  float sum_abs = 0.0f;
  for (size_t i = 0; i < n; i++) sum_abs += fabsf(weights[i]);
  float alpha = sum_abs > 0.0f ? (sum_abs / (float)n) / ABSMEAN_NORM : 1.0f;
  float inv = 1.0f / alpha;
  for (size_t i = 0; i < n; i++) {
    int32_t r = rust_f32_to_i32(roundf(weights[i] * inv));
    out[i] = (int8_t)(r < -1 ? -1 : r > 1 ? 1 : r);
  }
  return alpha;
}

/*
 * ternary.rs:76-110 quantize_ternary_blocked: blocks of block_size values
 * (the last one shorter when block_size does not divide n), each quantised
 * as quantize_ternary with its own alpha = (sum|block| / len) / ABSMEAN_NORM
 * (1.0 when the sum is not > 0); scales[b] receives block b's alpha, out the
 * codes in order. Pinned by its reduction to frxo_quantize_ternary on each
 * block (itself pinned by KATs and float64) and by the round trip of
 * dequantize below.
 */
void frxo_quantize_ternary_blocked(const float *weights, size_t n, size_t block_size, int8_t *out,
                                   float *scales) {
  size_t nb = (n + block_size - 1) / block_size;
  for (size_t b = 0; b < nb; b++) {
    size_t start = b * block_size, end = start + block_size < n ? start + block_size : n;
    float sum_abs = 0.0f;
    for (size_t i = start; i < end; i++) sum_abs += fabsf(weights[i]);
    float alpha = sum_abs > 0.0f ? (sum_abs / (float)(end - start)) / ABSMEAN_NORM : 1.0f;
    scales[b] = alpha;
    float inv = 1.0f / alpha;
    for (size_t i = start; i < end; i++) {
      int32_t r = rust_f32_to_i32(roundf(weights[i] * inv));
      out[i] = (int8_t)(r < -1 ? -1 : r > 1 ? 1 : r);
    }
  }
}

/*
 * ternary.rs:113-128 dequantize_ternary_blocked: for each of the n_scales
 * blocks, out[i] = alpha * (ternary[i] as f32) over the block's range (the
 * output ends with the last scale's block). Returns the number of values
 * written. Pinned by closed form: alpha * {-1, 0, +1} is exact.
 */
size_t frxo_dequantize_ternary_blocked(const int8_t *ternary, size_t n, const float *scales, size_t n_scales,
                                       size_t block_size, float *out) {
  size_t w = 0;
  for (size_t b = 0; b < n_scales; b++) {
    size_t start = b * block_size, end = start + block_size < n ? start + block_size : n;
    for (size_t i = start; i < end; i++) out[w++] = scales[b] * (float)ternary[i];
  }
  return w;
}

/*
 * shadow_weights.rs:203-231 BitLinear::forward_ste, the on-the-fly
 * quantisation: alpha = sum|w| / n (left-to-right f32 sum), then per value
 * normalized = w / alpha; +1 if > 0.5, -1 if < -0.5, else 0; all 0 when
 * alpha < 1e-10. Returns alpha. Pinned by closed cases in the tests: the
 * +-0.5 boundaries map to 0 (strict comparisons, unlike round()), a constant
 * row maps to its sign, tiny and zero rows to 0.
 */
float frxo_quantize_ste(const float *weights, size_t n, int8_t *out) {
  if (n == 0) return 0.0f;
  float sum = 0.0f;
  for (size_t i = 0; i < n; i++) sum += fabsf(weights[i]);
  const float alpha = sum / (float)n;
  for (size_t i = 0; i < n; i++) {
    if (alpha < 1e-10f) {
      out[i] = 0;
    } else {
      const float t = weights[i] / alpha;
      out[i] = t > 0.5f ? 1 : t < -0.5f ? -1 : 0;
    }
  }
  return alpha;
}

/* ---- 2:4 sparse ---------------------------------------------------------- */

/* kernels/sparse_ternary.rs:45-52 and sparse_ternary.rs:27-34 (same LUT). */
static const uint8_t PATTERN_POS[6][2] = {{0, 1}, {0, 2}, {0, 3},
                                          {1, 2}, {1, 3}, {2, 3}};

static int find_pattern(int a, int b) {
  for (int p = 0; p < 6; p++)
    if (PATTERN_POS[p][0] == a && PATTERN_POS[p][1] == b) return p;
  return -1;
}

/*
 * kernels/sparse_ternary.rs:254-318 pack_sparse_ternary (GPU 5-bit layout):
 * groups_per_row = ceil(cols/4), words_per_row = ceil(groups/6); group g of
 * row r lives in word r*wpr + g/6 at bit 5*(g%6): bits[2:0] pattern,
 * bit 3 = 1 iff the lower nonzero is -1, bit 4 = 1 iff the higher is -1.
 * scales[r] = mean |nonzero| of the row (1.0 if none). Returns 0, or -1
 * where the reference asserts (a group without exactly two nonzeros).
 * Pinned by KATs kernels/sparse_ternary.rs:362-436 through the matmul below,
 * and by decode(pack(W)) == W on random 2:4 matrices.
 */
int frxo_pack_sparse24_gpu(const int8_t *weights, size_t rows, size_t cols,
                           uint32_t *packed, float *scales) {
  size_t gpr = (cols + 3) / 4, wpr = (gpr + 5) / 6;
  memset(packed, 0, rows * wpr * sizeof(uint32_t));
  for (size_t r = 0; r < rows; r++) {
    float row_sum = 0.0f;
    size_t row_count = 0;
    scales[r] = 1.0f;
    for (size_t g = 0; g < gpr; g++) {
      int pos[4], n = 0;
      int8_t val[4];
      for (int i = 0; i < 4; i++) {
        size_t col = g * 4 + (size_t)i;
        if (col < cols) {
          int8_t v = weights[r * cols + col];
          if (v != 0) {
            if (n < 4) {
              pos[n] = i;
              val[n] = v;
            }
            n++;
            row_sum += fabsf((float)v);
            row_count++;
          }
        }
      }
      if (n != 2) return -1;
      int pat = find_pattern(pos[0], pos[1]);
      if (pat < 0) return -1;
      uint32_t sa = val[0] < 0 ? 1u : 0u, sb = val[1] < 0 ? 1u : 0u;
      uint32_t grp = (uint32_t)pat | ((sa | (sb << 1)) << 3);
      packed[r * wpr + g / 6] |= grp << ((g % 6) * 5);
    }
    if (row_count > 0) scales[r] = row_sum / (float)row_count;
  }
  return 0;
}

/*
 * kernels/sparse_ternary.rs:321-360 sparse_ternary_matmul_ref (== WGSL
 * :54-112): pattern clamped to <= 5, sign bit 1 -> -1.0, sum += sign * x in
 * group order (lower position first), out = sum * scale[r]. Pinned by KATs
 * kernels/sparse_ternary.rs:362-436 (3,4,6,7 / -3,-4 / -2.0 / 3,7) and by
 * equality with the dense u32 matmul on the decoded matrix (dyadic inputs).
 */
void frxo_sparse24_gpu_matmul(const uint32_t *packed, const float *scales,
                              const float *input, size_t seq, size_t cols,
                              size_t rows, float *out) {
  size_t gpr = (cols + 3) / 4, wpr = (gpr + 5) / 6;
  for (size_t s = 0; s < seq; s++) {
    for (size_t r = 0; r < rows; r++) {
      float sum = 0.0f;
      for (size_t g = 0; g < gpr; g++) {
        uint32_t gp = (packed[r * wpr + g / 6] >> ((g % 6) * 5)) & 0x1Fu;
        uint32_t pat = gp & 7u;
        if (pat > 5u) pat = 5u;
        uint32_t sg = (gp >> 3) & 3u;
        size_t ca = g * 4 + PATTERN_POS[pat][0];
        size_t cb = g * 4 + PATTERN_POS[pat][1];
        float sa = (sg & 1u) ? -1.0f : 1.0f;
        float sb = (sg & 2u) ? -1.0f : 1.0f;
        if (ca < cols) sum += sa * input[s * cols + ca];
        if (cb < cols) sum += sb * input[s * cols + cb];
      }
      out[s * rows + r] = sum * scales[r];
    }
  }
}

/* Dense i8 view of the GPU 2:4 layout (the WGSL decode, :87-107). */
void frxo_sparse24_gpu_decode(const uint32_t *packed, size_t rows, size_t cols,
                              int8_t *out) {
  size_t gpr = (cols + 3) / 4, wpr = (gpr + 5) / 6;
  memset(out, 0, rows * cols);
  for (size_t r = 0; r < rows; r++) {
    for (size_t g = 0; g < gpr; g++) {
      uint32_t gp = (packed[r * wpr + g / 6] >> ((g % 6) * 5)) & 0x1Fu;
      uint32_t pat = gp & 7u;
      if (pat > 5u) pat = 5u;
      uint32_t sg = (gp >> 3) & 3u;
      size_t ca = g * 4 + PATTERN_POS[pat][0];
      size_t cb = g * 4 + PATTERN_POS[pat][1];
      if (ca < cols) out[r * cols + ca] = (sg & 1u) ? -1 : 1;
      if (cb < cols) out[r * cols + cb] = (sg & 2u) ? -1 : 1;
    }
  }
}

/*
 * sparse_ternary.rs:78-144 SparseTernaryMatrix::from_ternary (CPU layout):
 * per group keep the two largest |v| (stable sort, so ties keep the lower
 * position), an all-zero group becomes positions (0,1); pattern nibbles two
 * per byte (even group -> bits 0-2, odd -> bits 4-6), sign pairs four per
 * byte at 2*(g%4) with bit=1 meaning +1 (v >= 0). cols % 4 == 0.
 * Pinned by KATs sparse_ternary.rs:327-393 and :418-432.
 */
void frxo_sparse24_cpu_from_ternary(const int8_t *ternary, size_t rows,
                                    size_t cols, uint8_t *patterns,
                                    uint8_t *signs) {
  size_t ng = rows * cols / 4;
  memset(patterns, 0, (ng + 1) / 2);
  memset(signs, 0, (ng + 3) / 4);
  for (size_t g = 0; g < ng; g++) {
    const int8_t *v = ternary + g * 4;
    int idx[4] = {0, 1, 2, 3};
    /* stable insertion sort by |v| descending */
    for (int i = 1; i < 4; i++) {
      int cur = idx[i], j = i - 1;
      int ca = abs(v[cur]);
      while (j >= 0 && abs(v[idx[j]]) < ca) {
        idx[j + 1] = idx[j];
        j--;
      }
      idx[j + 1] = cur;
    }
    int pos0 = idx[0];
    int pos1 = (v[idx[1]] != 0 || v[idx[0]] != 0) ? idx[1] : 1;
    int p0 = pos0 < pos1 ? pos0 : pos1, p1 = pos0 < pos1 ? pos1 : pos0;
    int pat = find_pattern(p0, p1);
    if (g % 2 == 0)
      patterns[g / 2] |= (uint8_t)(pat & 7);
    else
      patterns[g / 2] |= (uint8_t)((pat & 7) << 4);
    uint8_t s0 = v[p0] >= 0 ? 1 : 0, s1 = v[p1] >= 0 ? 1 : 0;
    signs[g / 4] |= (uint8_t)((s0 | (s1 << 1)) << ((g % 4) * 2));
  }
}

/*
 * sparse_ternary.rs:598-663 prune_fp32_to_sparse_ternary (CPU layout): per
 * group of 4 f32 values, the two largest |v| by Rust's stable sort_by with
 * b.abs().partial_cmp(a.abs()).unwrap_or(Equal). On 4 elements that sort is
 * an insertion sort (Rust's merge sort below its insertion threshold, from
 * 1.75 on): an element moves left past its neighbour only while its |v| is
 * strictly greater, so ties keep the lower position and a NaN moves past
 * nothing and lets nothing past it. Positions are then ordered (p0 < p1) for
 * the pattern, but the sign bits are taken in magnitude order: bit 0 =
 * (val0 >= 0) of the LARGEST |v|, bit 1 = (val1 >= 0) of the second, exactly
 * as the reference packs them (:642-644). Decoding reads bit 0 as the sign
 * of the lower position, so a group whose larger |v| sits at the higher
 * position and whose two signs differ decodes with the signs exchanged; this
 * restatement keeps that. NaN >= 0 is false (sign -1); -0.0 >= 0 is true.
 * scale = (sum|w| / n) / ABSMEAN_NORM with sum|w| left to right in f32 over
 * all rows*cols values, 1.0 when the sum is not > 0. cols % 4 == 0.
 * Pinned by the KAT sparse_ternary.rs:523-544 (tests/golden), brute force of
 * the kept positions (top-2 by |v|, lower index on ties) and of the absmean
 * scale in float64. The exchanged-sign case is covered by no reference
 * fixture (parity unpinned for it beyond this reading of :626-644).
 */
float frxo_prune_sparse24(const float *weights, size_t rows, size_t cols, uint8_t *patterns,
                          uint8_t *signs) {
  size_t ng = rows * cols / 4;
  memset(patterns, 0, (ng + 1) / 2);
  memset(signs, 0, (ng + 3) / 4);
  for (size_t g = 0; g < ng; g++) {
    const float *v = weights + g * 4;
    int idx[4] = {0, 1, 2, 3};
    for (int i = 1; i < 4; i++) {
      int cur = idx[i], j = i;
      while (j > 0 && fabsf(v[cur]) > fabsf(v[idx[j - 1]])) {
        idx[j] = idx[j - 1];
        j--;
      }
      idx[j] = cur;
    }
    int pos0 = idx[0], pos1 = idx[1];
    float val0 = v[pos0], val1 = v[pos1];
    int p0 = pos0 < pos1 ? pos0 : pos1, p1 = pos0 < pos1 ? pos1 : pos0;
    int pat = find_pattern(p0, p1);
    if (g % 2 == 0)
      patterns[g / 2] |= (uint8_t)(pat & 7);
    else
      patterns[g / 2] |= (uint8_t)((pat & 7) << 4);
    uint8_t s0 = val0 >= 0.0f ? 1 : 0, s1 = val1 >= 0.0f ? 1 : 0;
    signs[g / 4] |= (uint8_t)((s0 | (s1 << 1)) << ((g % 4) * 2));
  }
  float sum_abs = 0.0f;
  for (size_t i = 0; i < rows * cols; i++) sum_abs += fabsf(weights[i]);
  return sum_abs > 0.0f ? (sum_abs / (float)(rows * cols)) / ABSMEAN_NORM : 1.0f;
}

/* sparse_ternary.rs:159-190 to_ternary (pattern > 5 falls back to 0). */
void frxo_sparse24_cpu_to_ternary(const uint8_t *patterns,
                                  const uint8_t *signs, size_t rows,
                                  size_t cols, int8_t *out) {
  size_t ng = rows * cols / 4;
  memset(out, 0, rows * cols);
  for (size_t g = 0; g < ng; g++) {
    int pat = g % 2 == 0 ? (patterns[g / 2] & 7) : ((patterns[g / 2] >> 4) & 7);
    if (pat > 5) pat = 0;
    int sb = (signs[g / 4] >> ((g % 4) * 2)) & 3;
    out[g * 4 + PATTERN_POS[pat][0]] = (sb & 1) ? 1 : -1;
    out[g * 4 + PATTERN_POS[pat][1]] = (sb & 2) ? 1 : -1;
  }
}

/*
 * sparse_ternary.rs:203-252 sparse_ternary_matmul (per-tensor scale):
 * sum += s0*x[p0]; sum += s1*x[p1] per group, out = scale * sum. Patterns 6
 * and 7 index out of the LUT in the reference (a panic); callers must not
 * pass them. :255-320 (_decode) has the same accumulation order.
 * Pinned by KATs sparse_ternary.rs:418-468 (16.0 known output, decode ==
 * general) and equality with the dense i8 matmul of to_ternary().
 */
void frxo_sparse24_cpu_matmul(const uint8_t *patterns, const uint8_t *signs,
                              float scale, size_t rows, size_t cols,
                              const float *input, size_t seq, float *out) {
  size_t ngr = cols / 4;
  for (size_t s = 0; s < seq; s++) {
    const float *xr = input + s * cols;
    for (size_t r = 0; r < rows; r++) {
      float sum = 0.0f;
      for (size_t g = 0; g < ngr; g++) {
        size_t gi = r * ngr + g;
        int pat = gi % 2 == 0 ? (patterns[gi / 2] & 7) : ((patterns[gi / 2] >> 4) & 7);
        if (pat > 5) pat = 5; /* reference panics; never produced by packers */
        int sb = (signs[gi / 4] >> ((gi % 4) * 2)) & 3;
        float s0 = (sb & 1) ? 1.0f : -1.0f, s1 = (sb & 2) ? 1.0f : -1.0f;
        sum += s0 * xr[g * 4 + PATTERN_POS[pat][0]];
        sum += s1 * xr[g * 4 + PATTERN_POS[pat][1]];
      }
      out[s * rows + r] = scale * sum;
    }
  }
}

void frxo_sparse24_cpu_matmul_decode(const uint8_t *patterns,
                                     const uint8_t *signs, float scale,
                                     size_t rows, size_t cols,
                                     const float *input, float *out) {
  frxo_sparse24_cpu_matmul(patterns, signs, scale, rows, cols, input, 1, out);
}

/* ---- MoE ------------------------------------------------------------------ */

/* gemma_mapper.rs:2073-2077 gelu_tanh. */
float frxo_gelu_tanh(float x) {
  const float pi = 3.14159265358979323846f;
  float c = sqrtf(2.0f / pi);
  float t = 0.044715f * x;
  t = t * x;
  t = t * x;
  float inner = c * (x + t);
  return (0.5f * x) * (1.0f + tanhf(inner));
}

/*
 * The GeLU of TernaryMoELayer::forward, src/model/ternary_moe.rs:196-199:
 * tanh_arg = 0.7978845608 * (x + 0.044715 * x * x * x) with the f32 literal
 * 0.7978845608 (one ulp above the f32 sqrt(2/pi) of frxo_gelu_tanh), then
 * 0.5 * x * (1.0 + tanh_arg.tanh()), each operation rounded to f32 left to
 * right as Rust evaluates it.
 */
float frxo_gelu_tanh_lit(float x) {
  float t = 0.044715f * x;
  t = t * x;
  t = t * x;
  float inner = 0.7978845608f * (x + t);
  return (0.5f * x) * (1.0f + tanhf(inner));
}

/* Expert activation by code: 0 silu(g) * u, 1 gelu_tanh(g) * u,
 * 2 gelu_tanh_lit(g) (no up product). */
static float moe_act(int act, float g, float u) {
  if (act == 2) return frxo_gelu_tanh_lit(g);
  float a = act == 1 ? frxo_gelu_tanh(g) : g / (1.0f + expf(-g));
  return a * u;
}

/*
 * Routing of the GPU-path MoE glue, cpu_block_attn_res.rs:1150-1166 (same as
 * TernaryMoELayer::forward, ternary_moe.rs:152-183): logits[e] = sequential
 * sum_j x[j]*router[e*H+j] (router is [E,H]); softmax over all E (max, exp,
 * sequential sum, divide); stable sort by probability descending; keep the
 * first top_k; weight_k = p_k / sum(p_top) (sum in sorted order).
 * Pinned by routing KATs tests/kernel_tests.rs:360-405 and :660-735 (on
 * logits), a brute-force argsort on tiny E, sum(w) == 1 within 1e-6.
 */
void frxo_moe_route(const float *x, const float *router, size_t tokens,
                    size_t hidden, size_t experts, size_t top_k,
                    uint32_t *topk_idx, float *topk_w, float *probs_out) {
  float *p = (float *)malloc(experts * sizeof(float));
  size_t *order = (size_t *)malloc(experts * sizeof(size_t));
  for (size_t t = 0; t < tokens; t++) {
    const float *xr = x + t * hidden;
    for (size_t e = 0; e < experts; e++) {
      float dot = 0.0f;
      for (size_t d = 0; d < hidden; d++) dot += xr[d] * router[e * hidden + d];
      p[e] = dot;
    }
    float mx = -INFINITY;
    for (size_t e = 0; e < experts; e++) mx = fmaxf(mx, p[e]);
    float se = 0.0f;
    for (size_t e = 0; e < experts; e++) {
      p[e] = expf(p[e] - mx);
      se += p[e];
    }
    for (size_t e = 0; e < experts; e++) p[e] /= se;
    if (probs_out)
      for (size_t e = 0; e < experts; e++) probs_out[t * experts + e] = p[e];
    for (size_t e = 0; e < experts; e++) order[e] = e;
    for (size_t i = 1; i < experts; i++) {
      size_t cur = order[i];
      size_t j = i;
      while (j > 0 && p[order[j - 1]] < p[cur]) {
        order[j] = order[j - 1];
        j--;
      }
      order[j] = cur;
    }
    size_t k = top_k < experts ? top_k : experts;
    float tsum = 0.0f;
    for (size_t i = 0; i < k; i++) tsum += p[order[i]];
    for (size_t i = 0; i < k; i++) {
      topk_idx[t * top_k + i] = (uint32_t)order[i];
      topk_w[t * top_k + i] = p[order[i]] / tsum;
    }
  }
  free(p);
  free(order);
}

/*
 * cpu_moe.rs:365-400 top_k_select_with_probs on logits computed as
 * cpu_moe.rs:146 does, with the router read as [H][E]: l_e = sum_h x_h *
 * R[h*E+e] (sequential in h; the reference's matrixmultiply::sgemm adds in
 * its own blocked order, which is not restated), experts sorted by logit
 * descending (stable, so ties keep index order), w_k = expf(l_k - l_max) for
 * the top-k in rank order, divided by their sum when the sum is > 0. A NaN
 * logit (a panic in the reference's unwrap) puts the token's experts in
 * index order.
 */
void frxo_moe_route_cpu_layer(const float *x, const float *router_he, size_t tokens, size_t hidden,
                              size_t experts, size_t top_k, uint32_t *topk_idx, float *topk_w) {
  float *l = (float *)malloc(experts * sizeof(float));
  size_t *order = (size_t *)malloc(experts * sizeof(size_t));
  for (size_t t = 0; t < tokens; t++) {
    const float *xr = x + t * hidden;
    int any_nan = 0;
    for (size_t e = 0; e < experts; e++) {
      float dot = 0.0f;
      for (size_t h = 0; h < hidden; h++) dot += xr[h] * router_he[h * experts + e];
      l[e] = dot;
      any_nan |= dot != dot;
    }
    for (size_t e = 0; e < experts; e++) order[e] = e;
    if (!any_nan) {
      for (size_t i = 1; i < experts; i++) {
        size_t cur = order[i];
        size_t j = i;
        while (j > 0 && l[order[j - 1]] < l[cur]) {
          order[j] = order[j - 1];
          j--;
        }
        order[j] = cur;
      }
    }
    const size_t k = top_k < experts ? top_k : experts;
    const float max_l = l[order[0]];
    float top_sum = 0.0f;
    for (size_t i = 0; i < k; i++) {
      const float ev = expf(l[order[i]] - max_l);
      top_sum += ev;
      topk_idx[t * top_k + i] = (uint32_t)order[i];
      topk_w[t * top_k + i] = ev;
    }
    if (top_sum > 0.0f)
      for (size_t i = 0; i < k; i++) topk_w[t * top_k + i] /= top_sum;
  }
  free(l);
  free(order);
}

/*
 * MoE forward of the GPU-path glue, cpu_block_attn_res.rs:1148-1184, and of
 * TernaryMoELayer::forward (ternary_moe.rs:145-223), with per-row scales:
 * per token, route (above), then for each selected expert in sorted order:
 * g = W_gate x, u = W_up x (u32 matmul), h by the activation code use_gelu:
 *   0: silu(g) * u, silu = g / (1 + exp(-g))  (both; ternary_moe.rs:202-204)
 *   1: gelu_tanh(g) * u                       (the glue, :1176-1178)
 *   2: gelu_tanh_lit(g), no up projection      (TernaryMoELayer, :193-200;
 *      w_up / s_up are not read and may be NULL)
 * then d = W_down h, out += w_k * d (out starts at 0.0). Pinned by: the
 * decomposition MoE = sum_k w_k FFN_e(x) where each matmul is the pinned u32
 * matmul, a float64 restatement on tiny shapes, and the reference's shape /
 * non-zero / GeLU != SwiGLU tests (ternary_moe.rs:311-443).
 */
/* routing 0: TernaryMoELayer / GPU glue; 1: CpuMoELayer (router [H][E],
 * frxo_moe_route_cpu_layer, experts with |w| < 1e-8 skipped as
 * cpu_moe.rs:172 does). */
void frxo_moe_forward_routed(const float *x, const float *router,
                             const uint32_t *const *w_gate,
                             const float *const *s_gate,
                             const uint32_t *const *w_up, const float *const *s_up,
                             const uint32_t *const *w_down,
                             const float *const *s_down, size_t tokens, size_t hidden,
                             size_t inter, size_t experts, size_t top_k, int use_gelu,
                             int routing, float *out, uint32_t *topk_idx, float *topk_w);

void frxo_moe_forward(const float *x, const float *router,
                      const uint32_t *const *w_gate,
                      const float *const *s_gate,
                      const uint32_t *const *w_up, const float *const *s_up,
                      const uint32_t *const *w_down,
                      const float *const *s_down, size_t tokens, size_t hidden,
                      size_t inter, size_t experts, size_t top_k, int use_gelu,
                      float *out, uint32_t *topk_idx, float *topk_w) {
  frxo_moe_forward_routed(x, router, w_gate, s_gate, w_up, s_up, w_down, s_down, tokens, hidden, inter, experts,
                          top_k, use_gelu, 0, out, topk_idx, topk_w);
}

/*
 * LoraLayer::forward for one position, src/training/lora.rs:138-167:
 * ax[r] = sum_d A[r][d] * in[d] (A: [rank][in]), then
 * out[o] = (sum_r B[o][r] * ax[r]) * scaling (B: [out][rank]), both sums
 * left to right in f32 from 0.0, the product rounded before its add.
 */
void frxo_lora_forward(const float *a, const float *b, size_t rank, size_t in_f, size_t out_f, float scaling,
                       const float *input, float *out) {
  float *ax = (float *)malloc((rank ? rank : 1) * sizeof(float));
  for (size_t r = 0; r < rank; r++) {
    float sum = 0.0f;
    for (size_t d = 0; d < in_f; d++) sum += a[r * in_f + d] * input[d];
    ax[r] = sum;
  }
  for (size_t o = 0; o < out_f; o++) {
    float sum = 0.0f;
    for (size_t r = 0; r < rank; r++) sum += b[o * rank + r] * ax[r];
    out[o] = sum * scaling;
  }
  free(ax);
}

/*
 * The MoE forward with LoRA adapters on the experts, as
 * CpuMoELayer::expert_forward_packed_parallel_with_lora
 * (src/model/cpu_moe.rs:321-363): gated = W_gate x (+ lora_gate(x)),
 * activation, upped = W_up x (+ lora_up(x)), combined = act(gated) * upped,
 * down = W_down combined (+ lora_down(combined)); then the routed combine of
 * frxo_moe_forward_routed. lora_*[e] may be NULL (no adapter on that expert
 * and projection). Adapter shapes: gate/up A [rank][hidden], B [inter][rank];
 * down A [rank][inter], B [hidden][rank].
 */
void frxo_moe_forward_lora(const float *x, const float *router, const uint32_t *const *w_gate,
                           const float *const *s_gate, const uint32_t *const *w_up, const float *const *s_up,
                           const uint32_t *const *w_down, const float *const *s_down, size_t tokens,
                           size_t hidden, size_t inter, size_t experts, size_t top_k, int use_gelu, int routing,
                           size_t rank, float scaling, const float *const *a_gate, const float *const *b_gate,
                           const float *const *a_up, const float *const *b_up, const float *const *a_down,
                           const float *const *b_down, float *out, uint32_t *topk_idx, float *topk_w) {
  if (routing == 1)
    frxo_moe_route_cpu_layer(x, router, tokens, hidden, experts, top_k, topk_idx, topk_w);
  else
    frxo_moe_route(x, router, tokens, hidden, experts, top_k, topk_idx, topk_w, NULL);
  float *g = (float *)malloc(inter * sizeof(float));
  float *u = (float *)malloc(inter * sizeof(float));
  float *l = (float *)malloc((inter > hidden ? inter : hidden) * sizeof(float));
  float *d = (float *)malloc(hidden * sizeof(float));
  size_t k = top_k < experts ? top_k : experts;
  for (size_t t = 0; t < tokens; t++) {
    const float *xr = x + t * hidden;
    float *orow = out + t * hidden;
    for (size_t j = 0; j < hidden; j++) orow[j] = 0.0f;
    for (size_t i = 0; i < k; i++) {
      uint32_t e = topk_idx[t * top_k + i];
      float w = topk_w[t * top_k + i];
      if (routing == 1 && fabsf(w) < 1e-8f) continue;
      frxo_ternary_matmul_u32(w_gate[e], s_gate[e], xr, 1, hidden, inter, g);
      if (a_gate && a_gate[e] && b_gate[e]) {
        frxo_lora_forward(a_gate[e], b_gate[e], rank, hidden, inter, scaling, xr, l);
        for (size_t j = 0; j < inter; j++) g[j] += l[j];
      }
      if (use_gelu == 2) {
        for (size_t j = 0; j < inter; j++) g[j] = frxo_gelu_tanh_lit(g[j]);
      } else {
        for (size_t j = 0; j < inter; j++) g[j] = use_gelu ? frxo_gelu_tanh(g[j]) : g[j] / (1.0f + expf(-g[j]));
        frxo_ternary_matmul_u32(w_up[e], s_up[e], xr, 1, hidden, inter, u);
        if (a_up && a_up[e] && b_up[e]) {
          frxo_lora_forward(a_up[e], b_up[e], rank, hidden, inter, scaling, xr, l);
          for (size_t j = 0; j < inter; j++) u[j] += l[j];
        }
        for (size_t j = 0; j < inter; j++) g[j] = g[j] * u[j];
      }
      frxo_ternary_matmul_u32(w_down[e], s_down[e], g, 1, inter, hidden, d);
      if (a_down && a_down[e] && b_down[e]) {
        frxo_lora_forward(a_down[e], b_down[e], rank, inter, hidden, scaling, g, l);
        for (size_t j = 0; j < hidden; j++) d[j] += l[j];
      }
      for (size_t j = 0; j < hidden; j++) orow[j] += w * d[j];
    }
  }
  free(g);
  free(u);
  free(l);
  free(d);
}

void frxo_moe_forward_routed(const float *x, const float *router,
                             const uint32_t *const *w_gate,
                             const float *const *s_gate,
                             const uint32_t *const *w_up, const float *const *s_up,
                             const uint32_t *const *w_down,
                             const float *const *s_down, size_t tokens, size_t hidden,
                             size_t inter, size_t experts, size_t top_k, int use_gelu,
                             int routing, float *out, uint32_t *topk_idx, float *topk_w) {
  if (routing == 1)
    frxo_moe_route_cpu_layer(x, router, tokens, hidden, experts, top_k, topk_idx, topk_w);
  else
    frxo_moe_route(x, router, tokens, hidden, experts, top_k, topk_idx, topk_w, NULL);
  float *g = (float *)malloc(inter * sizeof(float));
  float *u = (float *)malloc(inter * sizeof(float));
  float *d = (float *)malloc(hidden * sizeof(float));
  size_t k = top_k < experts ? top_k : experts;
  for (size_t t = 0; t < tokens; t++) {
    const float *xr = x + t * hidden;
    float *orow = out + t * hidden;
    for (size_t j = 0; j < hidden; j++) orow[j] = 0.0f;
    for (size_t i = 0; i < k; i++) {
      uint32_t e = topk_idx[t * top_k + i];
      float w = topk_w[t * top_k + i];
      if (routing == 1 && fabsf(w) < 1e-8f) continue;
      frxo_ternary_matmul_u32(w_gate[e], s_gate[e], xr, 1, hidden, inter, g);
      if (use_gelu != 2) frxo_ternary_matmul_u32(w_up[e], s_up[e], xr, 1, hidden, inter, u);
      for (size_t j = 0; j < inter; j++) g[j] = moe_act(use_gelu, g[j], use_gelu == 2 ? 0.0f : u[j]);
      frxo_ternary_matmul_u32(w_down[e], s_down[e], g, 1, inter, hidden, d);
      for (size_t j = 0; j < hidden; j++) orow[j] += w * d[j];
    }
  }
  free(g);
  free(u);
  free(d);
}

/*
 * Dense FFN of one layer, cpu_block_attn_res.rs:2317-2326 (decode) and
 * :1185-1194 (prefill): gated = W_gate x, upped = W_up x (the u32 matmul,
 * per-row scales), gated = gelu_tanh(gated) or gated / (1 + exp(-gated))
 * (:2323), combined = gated * upped, out = W_down combined, all in f32 over
 * all seq tokens. Pinned by its decomposition into the pinned u32 matmul and
 * the activation (checked against float64 on tiny shapes in the tests).
 */
void frxo_ffn_forward(const float *x, size_t seq, size_t hidden, size_t inter,
                      const uint32_t *w_gate, const float *s_gate,
                      const uint32_t *w_up, const float *s_up,
                      const uint32_t *w_down, const float *s_down, int use_gelu,
                      float *out) {
  float *g = (float *)malloc(seq * inter * sizeof(float));
  float *u = (float *)malloc(seq * inter * sizeof(float));
  frxo_ternary_matmul_u32(w_gate, s_gate, x, seq, hidden, inter, g);
  frxo_ternary_matmul_u32(w_up, s_up, x, seq, hidden, inter, u);
  for (size_t i = 0; i < seq * inter; i++) {
    float a = use_gelu ? frxo_gelu_tanh(g[i]) : g[i] / (1.0f + expf(-g[i]));
    g[i] = a * u[i];
  }
  frxo_ternary_matmul_u32(w_down, s_down, g, seq, inter, hidden, out);
  free(g);
  free(u);
}

/* ---- timed multi-threaded CPU baseline ------------------------------------ */

typedef struct {
  const uint8_t *packed;
  float scale;
  const float *input;
  size_t out_rows, in_cols, batch;
  float *out;
  int tid, nthreads, reps;
  pthread_barrier_t *bar;
  double *times;
} pp_arg;

static double now_s(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

static void *pp_worker(void *p) {
  pp_arg *a = (pp_arg *)p;
  size_t nchunks = (a->out_rows + a->batch - 1) / a->batch;
  for (int rep = 0; rep < a->reps; rep++) {
    pthread_barrier_wait(a->bar);
    double t0 = now_s();
    for (size_t c = (size_t)a->tid; c < nchunks; c += (size_t)a->nthreads) {
      size_t r0 = c * a->batch;
      size_t r1 = r0 + a->batch < a->out_rows ? r0 + a->batch : a->out_rows;
      frxo_ternary_matmul_packed_rows(a->packed, a->scale, a->input,
                                      a->out_rows, a->in_cols, r0, r1, a->out);
    }
    pthread_barrier_wait(a->bar);
    if (a->tid == 0) a->times[rep] = now_s() - t0;
  }
  return NULL;
}

static int cmp_double(const void *x, const void *y) {
  double a = *(const double *)x, b = *(const double *)y;
  return a < b ? -1 : a > b;
}

/*
 * Times ternary_matmul_packed_parallel (ternary.rs:471-529): rows split into
 * ceil(N / max(N/32,1)) row batches spread over `threads` workers (rayon's
 * par_chunks_mut split, statically round-robined). Returns the median wall
 * time in seconds over `reps` calls; when `pct` is not NULL it receives the
 * 10th and 90th percentile (nearest rank) in pct[0], pct[1].
 */
double frxo_time_packed_parallel(const uint8_t *packed, float scale,
                                 const float *input, size_t out_rows,
                                 size_t in_cols, int threads, int reps,
                                 float *out, double *pct) {
  if (threads < 1) threads = 1;
  if (reps < 1) reps = 1;
  pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
  pp_arg *args = (pp_arg *)malloc(sizeof(pp_arg) * (size_t)threads);
  double *times = (double *)malloc(sizeof(double) * (size_t)reps);
  pthread_barrier_t bar;
  pthread_barrier_init(&bar, NULL, (unsigned)threads);
  size_t batch = out_rows / 32 > 0 ? out_rows / 32 : 1;
  for (int i = 0; i < threads; i++) {
    pp_arg a = {packed, scale, input, out_rows, in_cols, batch, out,
                i,      threads, reps, &bar, times};
    args[i] = a;
  }
  for (int i = 1; i < threads; i++) pthread_create(&th[i], NULL, pp_worker, &args[i]);
  pp_worker(&args[0]);
  for (int i = 1; i < threads; i++) pthread_join(th[i], NULL);
  pthread_barrier_destroy(&bar);
  qsort(times, (size_t)reps, sizeof(double), cmp_double);
  double med = times[reps / 2];
  if (pct) {
    pct[0] = times[(reps - 1) / 10];
    pct[1] = times[(9 * (reps - 1) + 9) / 10];
  }
  free(th);
  free(args);
  free(times);
  return med;
}
