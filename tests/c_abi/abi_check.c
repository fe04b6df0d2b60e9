/* Compiled by gcc as C99 against include/frx_ternary.h and linked with
 * libfrx_ternary.so: the header's declarations must match what the library
 * exports, and the host-side entry points must behave as declared without a
 * GPU (packers bit-exact on a small case, every error path a status). */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "frx_ternary.h"

static int failures = 0;
#define EXPECT(cond)                                              \
  do {                                                            \
    if (!(cond)) {                                                \
      fprintf(stderr, "%s:%d: expected %s\n", __FILE__, __LINE__, #cond); \
      failures++;                                                 \
    }                                                             \
  } while (0)

/* Every declared function, taken by address with its declared type. */
typedef frx_status (*linear_fn)(frx_ctx *, const uint32_t *, const float *, const void *, frx_dtype, void *,
                                frx_dtype, uint32_t, uint32_t, uint32_t);
typedef frx_status (*linear_bias_fn)(frx_ctx *, const uint32_t *, const float *, const float *, const void *,
                                     frx_dtype, void *, frx_dtype, uint32_t, uint32_t, uint32_t);
typedef frx_status (*ffn_fn)(frx_ctx *, const void *, frx_dtype, const uint32_t *, const float *,
                             const uint32_t *, const float *, const uint32_t *, const float *, uint32_t, uint32_t,
                             uint32_t, frx_activation, void *, frx_dtype);

int main(void) {
  linear_fn lin = frx_ternary_linear;
  linear_fn sp = frx_sparse24_ternary_linear;
  linear_bias_fn lin_b = frx_ternary_linear_bias;
  ffn_fn ffn = frx_ternary_ffn;
  ffn_fn ffn_na = frx_ternary_ffn_noalloc;
  (void)lin;
  (void)sp;
  (void)lin_b;
  (void)ffn;
  (void)ffn_na;

  /* pack_ternary: values -1,0,+1,0,+1 -> codes 00,01,10,01 | 10 */
  const int8_t vals[5] = {-1, 0, 1, 0, 1};
  uint8_t packed[2] = {0xFF, 0xFF};
  EXPECT(frx_pack_ternary_u8(vals, 5, packed) == FRX_OK);
  EXPECT(packed[0] == (uint8_t)(0x0 | (0x1 << 2) | (0x2 << 4) | (0x1 << 6)));
  EXPECT(packed[1] == 0x2);
  int8_t back[5];
  EXPECT(frx_unpack_ternary_u8(packed, 5, back) == FRX_OK);
  EXPECT(memcmp(back, vals, 5) == 0);
  uint32_t words[1] = {0};
  EXPECT(frx_repack_u8_to_u32(packed, 5, words) == FRX_OK);
  EXPECT(words[0] == ((uint32_t)packed[0] | ((uint32_t)packed[1] << 8)));

  /* gpu_packed: one 1x16 row, tensor scale broadcast */
  int8_t row[16];
  for (int i = 0; i < 16; i++) row[i] = (int8_t)((i % 3) - 1);
  uint32_t w16 = 0;
  float sc = 0.0f;
  EXPECT(frx_gpu_packed(row, 1, 16, 0.5f, &w16, &sc) == FRX_OK);
  EXPECT(sc == 0.5f);
  for (int i = 0; i < 16; i++) EXPECT(((w16 >> (2 * i)) & 3u) == (uint32_t)(row[i] + 1));

  /* 2:4 packer: a group with three nonzeros is a shape error */
  const int8_t bad24[4] = {1, -1, 1, 0};
  uint32_t meta[1];
  EXPECT(frx_pack_sparse24_gpu(bad24, 1, 4, meta, NULL) == FRX_ERR_SHAPE);
  const int8_t ok24[4] = {1, 0, 0, -1};
  EXPECT(frx_pack_sparse24_gpu(ok24, 1, 4, meta, NULL) == FRX_OK);

  /* error paths without a context or a GPU */
  EXPECT(frx_ternary_linear(NULL, NULL, NULL, NULL, FRX_F32, NULL, FRX_F32, 1, 16, 1) == FRX_ERR_DEVICE);
  EXPECT(frx_ternary_linear_bias(NULL, NULL, NULL, NULL, NULL, FRX_F32, NULL, FRX_F32, 1, 16, 1) == FRX_ERR_DEVICE);
  EXPECT(frx_synchronize(NULL) == FRX_ERR_DEVICE);
  EXPECT(frx_force_status(NULL, FRX_ERR_OOM) == FRX_ERR_DEVICE);
  EXPECT(frx_set_stream(NULL, NULL) == FRX_ERR_DEVICE);
  EXPECT(strcmp(frx_last_error(NULL), "") == 0);
  EXPECT(strcmp(frx_status_string(FRX_ERR_SHAPE), "shape error") == 0);
  EXPECT(strncmp(frx_version(), "frx_ternary", 11) == 0);
  frx_ctx *ctx = NULL;
  EXPECT(frx_create(0, NULL) == FRX_ERR_DEVICE);
  const frx_status st = frx_create(-1, &ctx);
  EXPECT(st == FRX_ERR_DEVICE && ctx == NULL);
  EXPECT(frx_pack_ternary_u8(NULL, 4, packed) == FRX_ERR_SHAPE);

  if (failures) {
    fprintf(stderr, "%d ABI check(s) failed\n", failures);
    return 1;
  }
  printf("abi_check ok\n");
  return 0;
}
