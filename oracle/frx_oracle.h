/*
 * frx_oracle.h — CPU restatement of FerrisRes's 1.58-bit ternary linear path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * kernels in libfrx_ternary.so. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker or the
 * timed CPU baseline; the product path never calls it.
 *
 * Every function restates a reference function loop-for-loop (same
 * accumulation order, no FMA contraction: build with -ffp-contract=off), and
 * cites the file:line it follows (paths relative to the FerrisRes tree).
 *
 * Parity pinning (which checks pin each function) is documented per function
 * in frx_oracle.c.
 */
#ifndef FRX_ORACLE_H
#define FRX_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- dense 2-bit packing --------------------------------------------- */
void frxo_pack_ternary(const int8_t *values, size_t n, uint8_t *out);
void frxo_unpack_ternary(const uint8_t *packed, size_t n, int8_t *out);
void frxo_pack_ternary_u32(const uint8_t *packed_u8, size_t packed_len,
                           size_t total_values, uint32_t *out);
void frxo_pack_rows_u32(const int8_t *values, size_t rows, size_t cols,
                        uint32_t *out);

/* ---- dense matmuls ----------------------------------------------------- */
void frxo_ternary_matmul_u32(const uint32_t *packed, const float *scales,
                             const float *input, size_t seq, size_t in_cols,
                             size_t out_rows, float *out);
void frxo_ternary_matmul_i8(const int8_t *ternary, float scale,
                            const float *input, size_t out_rows,
                            size_t in_cols, size_t seq, float *out);
void frxo_ternary_matmul_decode(const int8_t *ternary, float scale,
                                const float *input, size_t out_rows,
                                size_t in_cols, float *out);
void frxo_ternary_matmul_packed(const uint8_t *packed, float scale,
                                const float *input, size_t out_rows,
                                size_t in_cols, size_t seq, float *out);
/* ternary_linear.rs:94-165: matmul (path 0 i8, 1 packed u8, 2 decode) + bias */
void frxo_ternary_linear_forward(const int8_t *ternary, const uint8_t *packed, float scale,
                                 const float *bias, const float *input, size_t out_rows,
                                 size_t in_cols, size_t seq, int path, float *out);
void frxo_ternary_matmul_packed_rows(const uint8_t *packed, float scale,
                                     const float *input, size_t out_rows,
                                     size_t in_cols, size_t row_begin,
                                     size_t row_end, float *out);
void frxo_ternary_matmul_blocked(const int8_t *ternary, const float *scales,
                                 size_t block_size, const float *input,
                                 size_t out_rows, size_t in_cols, size_t seq,
                                 float *out);
void frxo_ternary_sparse_indices(const int8_t *ternary, size_t out_rows,
                                 size_t in_cols, uint32_t *pos_off,
                                 uint32_t *pos_idx, uint32_t *neg_off,
                                 uint32_t *neg_idx);
void frxo_ternary_matmul_sparse_decode(const uint32_t *pos_off,
                                       const uint32_t *pos_idx,
                                       const uint32_t *neg_off,
                                       const uint32_t *neg_idx, float scale,
                                       const float *input, size_t out_rows,
                                       float *out);
float frxo_ternary_stats(const int8_t *ternary, size_t n, uint64_t counts[3],
                         float ratios[3]);
void frxo_bench_ternary_matmul(const float *a, const int8_t *weights,
                               float scale, size_t m, size_t n, size_t k,
                               float *out);
float frxo_quantize_ternary(const float *weights, size_t n, int8_t *out);
float frxo_quantize_ste(const float *weights, size_t n, int8_t *out);

/* ---- 2:4 sparse, GPU (WGSL) layout ------------------------------------- */
int frxo_pack_sparse24_gpu(const int8_t *weights, size_t rows, size_t cols,
                           uint32_t *packed, float *scales);
void frxo_sparse24_gpu_matmul(const uint32_t *packed, const float *scales,
                              const float *input, size_t seq, size_t cols,
                              size_t rows, float *out);

/* ---- 2:4 sparse, CPU (SparseTernaryMatrix) layout ---------------------- */
void frxo_sparse24_cpu_from_ternary(const int8_t *ternary, size_t rows,
                                    size_t cols, uint8_t *patterns,
                                    uint8_t *signs);
void frxo_sparse24_cpu_to_ternary(const uint8_t *patterns,
                                  const uint8_t *signs, size_t rows,
                                  size_t cols, int8_t *out);
void frxo_sparse24_cpu_matmul(const uint8_t *patterns, const uint8_t *signs,
                              float scale, size_t rows, size_t cols,
                              const float *input, size_t seq, float *out);
void frxo_sparse24_cpu_matmul_decode(const uint8_t *patterns,
                                     const uint8_t *signs, float scale,
                                     size_t rows, size_t cols,
                                     const float *input, float *out);
void frxo_sparse24_gpu_decode(const uint32_t *packed, size_t rows, size_t cols,
                              int8_t *out);

/* ---- MoE (per-row-scale ternary SwiGLU / GeLU experts) ----------------- */
void frxo_moe_route(const float *x, const float *router, size_t tokens,
                    size_t hidden, size_t experts, size_t top_k,
                    uint32_t *topk_idx, float *topk_w, float *probs_out);
void frxo_moe_route_cpu_layer(const float *x, const float *router_he, size_t tokens, size_t hidden,
                              size_t experts, size_t top_k, uint32_t *topk_idx, float *topk_w);
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
                      float *out, uint32_t *topk_idx, float *topk_w);
void frxo_lora_forward(const float *a, const float *b, size_t rank, size_t in_f, size_t out_f, float scaling,
                       const float *input, float *out);
void frxo_moe_forward_lora(const float *x, const float *router, const uint32_t *const *w_gate,
                           const float *const *s_gate, const uint32_t *const *w_up, const float *const *s_up,
                           const uint32_t *const *w_down, const float *const *s_down, size_t tokens,
                           size_t hidden, size_t inter, size_t experts, size_t top_k, int use_gelu, int routing,
                           size_t rank, float scaling, const float *const *a_gate, const float *const *b_gate,
                           const float *const *a_up, const float *const *b_up, const float *const *a_down,
                           const float *const *b_down, float *out, uint32_t *topk_idx, float *topk_w);
float frxo_gelu_tanh(float x);
float frxo_prune_sparse24(const float *weights, size_t rows, size_t cols, uint8_t *patterns,
                          uint8_t *signs);
void frxo_quantize_ternary_blocked(const float *weights, size_t n, size_t block_size, int8_t *out,
                                   float *scales);
size_t frxo_dequantize_ternary_blocked(const int8_t *ternary, size_t n, const float *scales, size_t n_scales,
                                       size_t block_size, float *out);
float frxo_gelu_tanh_lit(float x);
void frxo_ffn_forward(const float *x, size_t seq, size_t hidden, size_t inter,
                      const uint32_t *w_gate, const float *s_gate,
                      const uint32_t *w_up, const float *s_up,
                      const uint32_t *w_down, const float *s_down, int use_gelu,
                      float *out);

/* ---- multi-threaded CPU baseline (ternary.rs packed-parallel shape) ---- */
double frxo_time_packed_parallel(const uint8_t *packed, float scale,
                                 const float *input, size_t out_rows,
                                 size_t in_cols, int threads, int reps,
                                 float *out, double *pct);

#ifdef __cplusplus
}
#endif
#endif
