/* Host code of libfrx_ternary under AddressSanitizer and UBSan: this file,
 * the oracle (oracle/frx_oracle.c) and the host sources frx_pack.cpp and
 * frx_api.cpp are built with -fsanitize=address,undefined (host code only;
 * the kernels are linked uninstrumented) and run on the CPU.
 *
 *  - Every host packer against the oracle on random and edge-case shapes,
 *    with exact-size heap buffers so that any read or write past an end is
 *    reported: pack/unpack u8, the u32 repack, gpu_packed, the 2:4 GPU packer,
 *    the CPU->GPU 2:4 transcoder and the CSR index lists.
 *  - Every argument check of the host packers (null pointers, zero and
 *    misaligned sizes) returns its status.
 *  - Every context entry point with a null context returns FRX_ERR_DEVICE
 *    without dereferencing anything; with "--device" (a GPU present) the
 *    validation of each compute entry point on a real context (shape, dtype,
 *    alignment errors) and frx_force_status, none of which launches a kernel.
 * Prints "asan_check ok" and exits 0 when every check passes. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "frx_ternary.h"
#include "frx_oracle.h"

static int failures = 0;
#define EXPECT(cond)                                                       \
  do {                                                                     \
    if (!(cond)) {                                                         \
      fprintf(stderr, "%s:%d: expected %s\n", __FILE__, __LINE__, #cond); \
      failures++;                                                          \
    }                                                                      \
  } while (0)

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint64_t rnd(void) { /* splitmix64 */
  uint64_t z = (rng_state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static void *xmalloc(size_t n) { /* exact size, never 0 bytes */
  void *p = malloc(n ? n : 1);
  if (!p) abort();
  return p;
}

static void random_ternary(int8_t *v, size_t n) {
  for (size_t i = 0; i < n; i++) v[i] = (int8_t)((int)(rnd() % 3) - 1);
}

/* two nonzeros per group of 4 (the 2:4 packers' precondition) */
static void random_24(int8_t *v, size_t rows, size_t cols) {
  static const int pos[6][2] = {{0, 1}, {0, 2}, {0, 3}, {1, 2}, {1, 3}, {2, 3}};
  for (size_t r = 0; r < rows; r++)
    for (size_t g = 0; g < cols / 4; g++) {
      int8_t *q = v + r * cols + 4 * g;
      memset(q, 0, 4);
      const int p = (int)(rnd() % 6);
      q[pos[p][0]] = (rnd() & 1) ? 1 : -1;
      q[pos[p][1]] = (rnd() & 1) ? 1 : -1;
    }
}

static void check_dense_packers(size_t n) {
  int8_t *v = xmalloc(n);
  random_ternary(v, n);
  const size_t nb = (n + 3) / 4;
  uint8_t *a = xmalloc(nb), *b = xmalloc(nb);
  EXPECT(frx_pack_ternary_u8(v, n, a) == FRX_OK);
  frxo_pack_ternary(v, n, b);
  EXPECT(memcmp(a, b, nb) == 0);
  int8_t *back = xmalloc(n);
  EXPECT(frx_unpack_ternary_u8(a, n, back) == FRX_OK);
  EXPECT(memcmp(back, v, n) == 0);
  const size_t nw = (n + 15) / 16;
  uint32_t *wa = xmalloc(nw * 4), *wb = xmalloc(nw * 4);
  EXPECT(frx_repack_u8_to_u32(a, n, wa) == FRX_OK);
  frxo_pack_ternary_u32(b, nb, n, wb);
  EXPECT(memcmp(wa, wb, nw * 4) == 0);
  free(v), free(a), free(b), free(back), free(wa), free(wb);
}

static void check_gpu_packed(uint32_t N, uint32_t K) {
  int8_t *v = xmalloc((size_t)N * K);
  random_ternary(v, (size_t)N * K);
  uint32_t *w = xmalloc((size_t)N * K / 16 * 4), *wo = xmalloc((size_t)N * K / 16 * 4);
  float *s = xmalloc((size_t)N * 4);
  EXPECT(frx_gpu_packed(v, N, K, 0.75f, w, s) == FRX_OK);
  frxo_pack_rows_u32(v, N, K, wo);
  EXPECT(memcmp(w, wo, (size_t)N * K / 16 * 4) == 0);
  for (uint32_t r = 0; r < N; r++) EXPECT(s[r] == 0.75f);
  free(v), free(w), free(wo), free(s);
}

static void check_sparse24(uint32_t N, uint32_t K) {
  int8_t *v = xmalloc((size_t)N * K);
  random_24(v, N, K);
  const size_t wpr = ((size_t)K / 4 + 5) / 6;
  uint32_t *m = xmalloc((size_t)N * wpr * 4), *mo = xmalloc((size_t)N * wpr * 4), *mt = xmalloc((size_t)N * wpr * 4);
  float *s = xmalloc((size_t)N * 4), *so = xmalloc((size_t)N * 4);
  EXPECT(frx_pack_sparse24_gpu(v, N, K, m, s) == FRX_OK);
  EXPECT(frxo_pack_sparse24_gpu(v, N, K, mo, so) == 0);
  EXPECT(memcmp(m, mo, (size_t)N * wpr * 4) == 0);
  EXPECT(memcmp(s, so, (size_t)N * 4) == 0);
  /* CPU layout -> GPU layout decodes to the same matrix */
  const size_t ng = (size_t)N * K / 4;
  uint8_t *pat = xmalloc((ng + 1) / 2), *sg = xmalloc((ng + 3) / 4);
  frxo_sparse24_cpu_from_ternary(v, N, K, pat, sg);
  EXPECT(frx_sparse24_cpu_to_gpu(pat, sg, N, K, mt) == FRX_OK);
  int8_t *d1 = xmalloc((size_t)N * K), *d2 = xmalloc((size_t)N * K);
  frxo_sparse24_gpu_decode(mt, N, K, d1);
  frxo_sparse24_cpu_to_ternary(pat, sg, N, K, d2);
  EXPECT(memcmp(d1, d2, (size_t)N * K) == 0);
  free(v), free(m), free(mo), free(mt), free(s), free(so), free(pat), free(sg), free(d1), free(d2);
}

static void check_indices(uint32_t N, uint32_t K) {
  int8_t *v = xmalloc((size_t)N * K);
  random_ternary(v, (size_t)N * K);
  uint32_t *po = xmalloc(((size_t)N + 1) * 4), *no = xmalloc(((size_t)N + 1) * 4);
  EXPECT(frx_ternary_sparse_indices(v, N, K, po, NULL, no, NULL) == FRX_OK);
  const size_t np = po[N], nn = no[N];
  uint32_t *pi = xmalloc(np * 4), *ni = xmalloc(nn * 4);
  EXPECT(frx_ternary_sparse_indices(v, N, K, po, pi, no, ni) == FRX_OK);
  uint32_t *po2 = xmalloc(((size_t)N + 1) * 4), *no2 = xmalloc(((size_t)N + 1) * 4);
  uint32_t *pi2 = xmalloc(np * 4), *ni2 = xmalloc(nn * 4);
  frxo_ternary_sparse_indices(v, N, K, po2, pi2, no2, ni2);
  EXPECT(memcmp(po, po2, ((size_t)N + 1) * 4) == 0 && memcmp(no, no2, ((size_t)N + 1) * 4) == 0);
  EXPECT((np == 0 || memcmp(pi, pi2, np * 4) == 0) && (nn == 0 || memcmp(ni, ni2, nn * 4) == 0));
  free(v), free(po), free(no), free(pi), free(ni), free(po2), free(no2), free(pi2), free(ni2);
}

static void check_host_errors(void) {
  uint8_t b[4];
  int8_t v[16] = {0};
  uint32_t w[4];
  float s[4];
  EXPECT(frx_pack_ternary_u8(NULL, 4, b) == FRX_ERR_SHAPE);
  EXPECT(frx_pack_ternary_u8(v, 4, NULL) == FRX_ERR_SHAPE);
  EXPECT(frx_unpack_ternary_u8(NULL, 4, v) == FRX_ERR_SHAPE);
  EXPECT(frx_repack_u8_to_u32(NULL, 4, w) == FRX_ERR_SHAPE);
  EXPECT(frx_gpu_packed(v, 1, 15, 1.0f, w, s) == FRX_ERR_SHAPE); /* K % 16 */
  EXPECT(frx_gpu_packed(NULL, 1, 16, 1.0f, w, s) == FRX_ERR_SHAPE);
  EXPECT(frx_pack_sparse24_gpu(v, 1, 6, w, s) != FRX_OK); /* K % 4 */
  EXPECT(frx_sparse24_cpu_to_gpu(b, b, 1, 6, w) == FRX_ERR_SHAPE);
  EXPECT(frx_sparse24_cpu_to_gpu(NULL, b, 1, 8, w) == FRX_ERR_SHAPE);
  EXPECT(frx_ternary_sparse_indices(NULL, 1, 4, w, NULL, w, NULL) == FRX_ERR_SHAPE);
}

static void check_null_context(void) {
  const frx_status D = FRX_ERR_DEVICE;
  EXPECT(frx_ternary_linear(NULL, NULL, NULL, NULL, FRX_F32, NULL, FRX_F32, 1, 16, 1) == D);
  EXPECT(frx_ternary_linear_bias(NULL, NULL, NULL, NULL, NULL, FRX_F32, NULL, FRX_F32, 1, 16, 1) == D);
  EXPECT(frx_ternary_linear_group(NULL, NULL, FRX_F32, 1, 16, 1, NULL, NULL, NULL, NULL, FRX_F32) == D);
  EXPECT(frx_quantize_ternary_blocked(NULL, NULL, FRX_F32, 16, 16, NULL, NULL) == D);
  EXPECT(frx_dequantize_ternary_blocked(NULL, NULL, NULL, 16, 16, NULL) == D);
  EXPECT(frx_prune_sparse24(NULL, NULL, FRX_F32, 1, 4, 0, NULL, NULL, NULL, NULL) == D);
  EXPECT(frx_workspace_stats(NULL, NULL, NULL, NULL) == D);
  EXPECT(frx_release_retired(NULL) == D);
  EXPECT(frx_sparse24_ternary_linear(NULL, NULL, NULL, NULL, FRX_F32, NULL, FRX_F32, 1, 16, 1) == D);
  EXPECT(frx_ternary_linear_blocked(NULL, NULL, NULL, 16, NULL, FRX_F32, NULL, FRX_F32, 1, 16, 1) == D);
  EXPECT(frx_ternary_sparse_decode(NULL, NULL, NULL, NULL, NULL, 1.0f, NULL, FRX_F32, NULL, FRX_F32, 1, 16, 1) == D);
  EXPECT(frx_ternary_stats(NULL, NULL, 1, 16, NULL) == D);
  EXPECT(frx_moe_ternary_ffn(NULL, NULL, FRX_F32, NULL, FRX_F32, NULL, NULL, NULL, NULL, NULL, NULL, 1, 16, 16, 2,
                             1, FRX_ACT_SILU, NULL, FRX_F32, NULL, NULL) == D);
  EXPECT(frx_ternary_glu(NULL, NULL, FRX_F32, NULL, NULL, NULL, NULL, 1, 16, 16, FRX_ACT_SILU, NULL) == D);
  EXPECT(frx_ternary_ffn(NULL, NULL, FRX_F32, NULL, NULL, NULL, NULL, NULL, NULL, 1, 16, 16, FRX_ACT_SILU, NULL,
                         FRX_F32) == D);
  EXPECT(frx_ternary_ffn_noalloc(NULL, NULL, FRX_F32, NULL, NULL, NULL, NULL, NULL, NULL, 1, 16, 16, FRX_ACT_SILU,
                                 NULL, FRX_F32) == D);
  EXPECT(frx_set_moe_routing(NULL, FRX_MOE_CPU_MOE_LAYER) == D);
  EXPECT(frx_set_ffn_mode(NULL, FRX_FFN_AUTO) == D);
  EXPECT(frx_force_status(NULL, FRX_ERR_OOM) == D);
  EXPECT(frx_upload_ternary(NULL, NULL, 1, 16, NULL, 1.0f, NULL, NULL) == D);
  EXPECT(frx_upload_stm(NULL, NULL, 0, NULL, NULL, NULL, NULL) == D);
  EXPECT(frx_sparse24_cpu_to_gpu_device(NULL, NULL, NULL, 1, 16, NULL) == D);
  EXPECT(frx_quantize_ternary(NULL, NULL, FRX_F32, 1, 16, FRX_QUANT_ABSMEAN, NULL, NULL) == D);
  EXPECT(frx_free(NULL, NULL) == D);
  EXPECT(frx_gpu_ternary_matmul(NULL, NULL, NULL, NULL, 1, 16, 1, NULL) == D);
  EXPECT(frx_gpu_ternary_matmul_vram(NULL, NULL, NULL, NULL, 1, 16, 1, NULL) == D);
  EXPECT(frx_gpu_sparse_ternary_matmul(NULL, NULL, NULL, NULL, 1, 16, 1, NULL) == D);
  EXPECT(frx_synchronize(NULL) == D);
  EXPECT(frx_set_stream(NULL, NULL) == D);
  EXPECT(strcmp(frx_last_error(NULL), "") == 0);
  frx_destroy(NULL);
}

/* With a device: argument validation of the compute entry points on a real
 * context. Every call below is rejected before any launch. */
static void check_validation(void) {
  frx_ctx *ctx = NULL;
  if (frx_create(0, &ctx) != FRX_OK || !ctx) {
    fprintf(stderr, "frx_create(0) failed\n");
    failures++;
    return;
  }
  /* 16-byte aligned host addresses stand in for device pointers: they are
   * never dereferenced, the calls fail validation first */
  static _Alignas(16) uint32_t dummy[64];
  const uint32_t *w = dummy;
  const float *f = (const float *)dummy;
  void *y = dummy;
  EXPECT(frx_ternary_linear(ctx, w, f, f, FRX_F32, y, FRX_F32, 0, 16, 1) == FRX_ERR_SHAPE);   /* M = 0 */
  EXPECT(frx_ternary_linear(ctx, w, f, f, FRX_F32, y, FRX_F32, 1, 20, 1) == FRX_ERR_SHAPE);   /* K % 16 */
  EXPECT(frx_ternary_linear(ctx, NULL, f, f, FRX_F32, y, FRX_F32, 1, 16, 1) == FRX_ERR_SHAPE);
  EXPECT(frx_ternary_linear(ctx, w, f, f, (frx_dtype)7, y, FRX_F32, 1, 16, 1) == FRX_ERR_UNSUPPORTED);
  /* x not aligned to its element size (sub-slices at element offsets are
   * staged, not rejected) */
  EXPECT(frx_ternary_linear(ctx, w, f, (const char *)f + 2, FRX_F32, y, FRX_F32, 1, 16, 1) == FRX_ERR_SHAPE);
  EXPECT(frx_ternary_linear(ctx, w, f, f, FRX_F32, (char *)y + 1, FRX_BF16, 1, 16, 1) == FRX_ERR_SHAPE);
  /* weights of 4 GiB or more */
  EXPECT(frx_ternary_linear(ctx, w, f, f, FRX_F32, y, FRX_F32, 1, 0x10000, 0x40000) == FRX_ERR_SHAPE);
  EXPECT(strlen(frx_last_error(ctx)) > 0);
  EXPECT(frx_ternary_linear(ctx, w, f, f, FRX_F32, y, FRX_F32, 0x10000, 0x10000, 1) == FRX_ERR_SHAPE); /* > 2^31 */
  EXPECT(frx_ternary_linear_bias(ctx, w, f, f, f, FRX_F32, y, FRX_F32, 1, 24, 1) == FRX_ERR_SHAPE);
  EXPECT(frx_sparse24_ternary_linear(ctx, w, f, f, FRX_F32, y, FRX_F32, 1, 6, 1) == FRX_ERR_SHAPE);
  EXPECT(frx_ternary_linear_blocked(ctx, w, f, 0, f, FRX_F32, y, FRX_F32, 1, 16, 1) != FRX_OK);
  {
    const uint32_t *gw[5] = {w, w, w, w, w};
    const float *gs[5] = {f, f, f, f, f};
    void *gy[5] = {y, y, y, y, y};
    const uint32_t gn[5] = {1, 1, 1, 1, 1};
    EXPECT(frx_ternary_linear_group(ctx, f, FRX_F32, 1, 16, 0, gw, gs, gn, gy, FRX_F32) == FRX_ERR_SHAPE);
    EXPECT(frx_ternary_linear_group(ctx, f, FRX_F32, 1, 16, 5, gw, gs, gn, gy, FRX_F32) == FRX_ERR_SHAPE);
    EXPECT(frx_ternary_linear_group(ctx, f, FRX_F32, 1, 20, 2, gw, gs, gn, gy, FRX_F32) == FRX_ERR_SHAPE);
    EXPECT(frx_ternary_linear_group(ctx, f, FRX_F32, 1, 16, 2, NULL, gs, gn, gy, FRX_F32) == FRX_ERR_SHAPE);
  }
  EXPECT(frx_ternary_glu(ctx, f, FRX_F32, w, f, w, f, 1, 20, 16, FRX_ACT_SILU, y) == FRX_ERR_SHAPE);
  EXPECT(frx_ternary_ffn(ctx, f, FRX_F32, w, f, w, f, w, f, 1, 16, 20, FRX_ACT_SILU, y, FRX_F32) == FRX_ERR_SHAPE);
  EXPECT(frx_ternary_ffn(ctx, f, FRX_F32, w, f, w, f, w, f, 1, 16, 16, (frx_activation)5, y, FRX_F32) != FRX_OK);
  const uint32_t *wp[2] = {w, w};
  const float *sp[2] = {f, f};
  EXPECT(frx_moe_ternary_ffn(ctx, f, FRX_F32, f, FRX_F32, wp, sp, wp, sp, wp, sp, 1, 16, 16, 2, 3, FRX_ACT_SILU, y,
                             FRX_F32, NULL, NULL) == FRX_ERR_SHAPE); /* top_k > E */
  EXPECT(frx_moe_ternary_ffn(ctx, f, FRX_F32, f, FRX_F32, wp, sp, wp, sp, wp, sp, 1, 20, 16, 2, 1, FRX_ACT_SILU, y,
                             FRX_F32, NULL, NULL) == FRX_ERR_SHAPE); /* H % 16 */
  EXPECT(frx_moe_ternary_ffn(ctx, f, FRX_F32, f, FRX_F32, wp, sp, wp, sp, wp, sp, 1, 16, 16, 2, 1,
                             (frx_activation)7, y, FRX_F32, NULL, NULL) == FRX_ERR_UNSUPPORTED);
  EXPECT(frx_ternary_ffn(ctx, f, FRX_F32, w, f, w, f, w, f, 1, 16, 16, FRX_ACT_GELU_TANH_GATE, y, FRX_F32) ==
         FRX_ERR_UNSUPPORTED); /* the MoE layer's activation only */
  EXPECT(frx_prune_sparse24(ctx, f, FRX_F32, 1, 6, 0, NULL, NULL, (uint32_t *)y, (float *)y) == FRX_ERR_SHAPE);
  EXPECT(frx_prune_sparse24(ctx, f, FRX_F32, 1, 8, 0, (uint8_t *)y, NULL, NULL, (float *)y) == FRX_ERR_SHAPE);
  EXPECT(frx_quantize_ternary_blocked(ctx, f, FRX_F32, 16, 0, (uint32_t *)y, (float *)y) == FRX_ERR_SHAPE);
  EXPECT(frx_quantize_ternary_blocked(ctx, f, FRX_F32, 0, 0, NULL, NULL) == FRX_OK); /* empty: nothing */
  EXPECT(frx_dequantize_ternary_blocked(ctx, w, f, 16, 0, (float *)y) == FRX_ERR_SHAPE);
  {
    size_t live = 1, retired = 1;
    uint32_t allocs = 1;
    EXPECT(frx_workspace_stats(ctx, &live, &retired, &allocs) == FRX_OK);
    EXPECT(live == 0 && retired == 0 && allocs == 0);
    EXPECT(frx_release_retired(ctx) == FRX_OK);
  }
  EXPECT(frx_set_ffn_mode(ctx, (frx_ffn_mode)9) == FRX_ERR_UNSUPPORTED);
  EXPECT(frx_set_moe_routing(ctx, (frx_moe_routing)9) == FRX_ERR_UNSUPPORTED);
  /* forced status: returned before any argument is read */
  EXPECT(frx_force_status(ctx, FRX_ERR_OOM) == FRX_OK);
  EXPECT(frx_ternary_linear(ctx, NULL, NULL, NULL, FRX_F32, NULL, FRX_F32, 0, 0, 0) == FRX_ERR_OOM);
  EXPECT(strstr(frx_last_error(ctx), "forced") != NULL);
  EXPECT(frx_synchronize(ctx) == FRX_OK);
  EXPECT(frx_force_status(ctx, (frx_status)42) == FRX_ERR_UNSUPPORTED);
  EXPECT(frx_force_status(ctx, FRX_OK) == FRX_OK);
  EXPECT(frx_ternary_linear(ctx, NULL, NULL, NULL, FRX_F32, NULL, FRX_F32, 0, 0, 0) == FRX_ERR_SHAPE);
  frx_destroy(ctx);
}

int main(int argc, char **argv) {
  const int device = argc > 1 && strcmp(argv[1], "--device") == 0;
  static const size_t ns[] = {0, 1, 2, 3, 4, 5, 7, 15, 16, 17, 31, 33, 63, 64, 65, 1000, 4099};
  for (size_t i = 0; i < sizeof(ns) / sizeof(ns[0]); i++) check_dense_packers(ns[i]);
  for (int i = 0; i < 40; i++) check_dense_packers((size_t)(rnd() % 5000));
  static const uint32_t gp[][2] = {{1, 16}, {3, 32}, {17, 48}, {64, 256}, {5, 4096}};
  for (size_t i = 0; i < sizeof(gp) / sizeof(gp[0]); i++) check_gpu_packed(gp[i][0], gp[i][1]);
  static const uint32_t sp[][2] = {{1, 4}, {1, 24}, {2, 28}, {3, 100}, {7, 96}, {16, 1024}, {5, 4100}};
  for (size_t i = 0; i < sizeof(sp) / sizeof(sp[0]); i++) check_sparse24(sp[i][0], sp[i][1]);
  static const uint32_t ix[][2] = {{1, 1}, {1, 7}, {4, 33}, {30, 100}, {64, 512}};
  for (size_t i = 0; i < sizeof(ix) / sizeof(ix[0]); i++) check_indices(ix[i][0], ix[i][1]);
  check_host_errors();
  check_null_context();
  if (device) check_validation();
  if (failures) {
    fprintf(stderr, "%d check(s) failed\n", failures);
    return 1;
  }
  printf("asan_check ok%s\n", device ? " (device validation)" : "");
  return 0;
}
