// frx_internal.hpp — launchers shared between the kernel files and the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace frx {

// Opts kernel `fn` in to `bytes` of dynamic LDS on the current device (the
// attribute is needed above 64 KB), once per device; `done` holds one bit per
// device id. Concurrent first calls may both set it, which is harmless.
inline hipError_t opt_in_lds(const void *fn, int bytes, std::atomic<uint64_t> &done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = dev < 64 ? (uint64_t)1 << dev : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
  e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_acq_rel);
  return e;
}

// Token counts from which the bf16 decode GEMVs leave the 16-row tiles
// with x staged in LDS (gemv_kernel) for the kernels built for many tokens,
// measured per step at the LLaMA-7B decode shapes (11008x4096 / 4096x11008,
// rotating weights, graph-replayed):
//  - linear: the per-wave staged kernel (gemv_xs_kernel) from 5 tokens
//    (B = 5, 6, 7: 7.44 / 8.26, 7.62 / 9.60, 9.19 / 9.73 us with the 16-row
//    tiles against 6.39 / 8.14, 6.57 / 8.31, 6.74 / 8.45 us staged); 2-4
//    tokens take the 4-segment rows kernel before either.
//  - the FFN's gate/up launch (h as bf16 planes): per-lane operand loads
//    (gemv_direct_kernel) below 8 tokens, staged from 8 (FFN step at 4-7
//    tokens 25.2-28.3 us direct against 26.1-28.4 us staged);
//  - the FFN's down launch over those planes: staged from 6 tokens (FFN step
//    at 6 / 7 tokens 26.6 / 28.3 us with operand loads, 25.9 / 26.4 us
//    staged; at 4 / 5 tokens 25.2 / 25.2 against 25.7 / 25.2 us).
constexpr int GEMV_XS_MIN_B = 5;
constexpr int GEMV_GLU_XS_MIN_B = 8;
constexpr int GEMV_PLANES_XS_MIN_B = 6;
// The operand-load kernels (gemv_direct_kernel, gemv_tall_kernel) serve from
// 8 tokens where the staged kernel does not fit (K above its quad limit).
constexpr int GEMV_DIRECT_MIN_B = 8;

// Up to GEMV_GROUP_MAX matrices with the same K against one x, launched as
// one GEMV over their concatenated rows (frx_ternary_linear_group).
constexpr int GEMV_GROUP_MAX = 4;
struct GemvGroup {
  const uint32_t *w[GEMV_GROUP_MAX];
  const float *s[GEMV_GROUP_MAX];
  void *y[GEMV_GROUP_MAX];
  int start[GEMV_GROUP_MAX];  // first row of each matrix in the launch; 0x7fffffff past the group
  // matrix holding launch row r (r below the total)
  __host__ __device__ __forceinline__ int matrix_of(int r) const {
    int m = 0;
#pragma unroll
    for (int i = 1; i < GEMV_GROUP_MAX; i++) m += r >= start[i] ? 1 : 0;
    return m;
  }
  // members by a run-time index through selects with constant indices (an
  // indexed access to the by-value kernel argument would copy it to scratch)
  template <typename T>
  __host__ __device__ __forceinline__ static T pick(const T (&a)[GEMV_GROUP_MAX], int m) {
    static_assert(GEMV_GROUP_MAX == 4, "select chain");
    return m == 0 ? a[0] : m == 1 ? a[1] : m == 2 ? a[2] : a[3];
  }
  __host__ __device__ __forceinline__ const uint32_t *w_of(int m) const { return pick(w, m); }
  __host__ __device__ __forceinline__ const float *s_of(int m) const { return pick(s, m); }
  __host__ __device__ __forceinline__ void *y_of(int m) const { return pick(y, m); }
  __host__ __device__ __forceinline__ int start_of(int m) const { return pick(start, m); }
  // weights, scales and first launch row of the matrix holding launch row r,
  // as a chain of selects on r (the starts ascend, so the last start <= r
  // wins): a wave-uniform r gives scalar selects and no branches (a select
  // on the matrix index became a branch per candidate and delayed the
  // issue of each row's loads: 8.2 -> 7.3 us per gate + up group launch)
  __host__ __device__ __forceinline__ void locate(int r, const uint32_t *&wp, const float *&sp, int &first) const {
    wp = w[0];
    sp = s[0];
    first = 0;
#pragma unroll
    for (int i = 1; i < GEMV_GROUP_MAX; i++) {
      const bool in = r >= start[i];
      wp = in ? w[i] : wp;
      sp = in ? s[i] : sp;
      first = in ? start[i] : first;
    }
  }
};
// The group runs as one balanced launch (one token, aligned operands, K %
// 64 == 0 up to 16384, rows within the slots); else launch_gemv_group runs
// one launch per matrix.
bool gemv_group_fits(const void *x, int B, int K, int count, const uint32_t *const *w, const int *N);
hipError_t launch_gemv_group(const void *x, int xt_bf16, int yt_bf16, int B, int K, int count,
                             const uint32_t *const *w, const float *const *s, void *const *y, const int *N,
                             hipStream_t stream);

// Decode GEMV for 2-16 tokens with K split over workgroups (frx_gemv_sk.hip):
// 128-row tiles x slices of up to 1024 columns write fp32 partials into
// `part` (gemv_sk_workspace_bytes); the last slice of each row tile adds
// them in slice order. counters: one zero-initialised word per 128-row tile
// (GEMV_SK_MAX_TILES at most), left zero by every launch. xs: 0 bf16 x, 1
// f32 x, 2 bf16 planes (x hi, x2 lo). K % 16 == 0, x 16-byte aligned,
// B * K * 4 < 2^32.
constexpr int GEMV_SK_MAX_TILES = 65536;
// Split-K dense GEMM (frx_gemm.hip) for 17 to a few hundred bf16 tokens,
// where 64-token tiles give fewer workgroups than compute units: S parts of
// kp columns (K % 64 == 0, N % 4 == 0, 16-byte aligned weights and x),
// fp32 partials in `part` (gemm_splitk_workspace_bytes), then an ordered
// reduction with the scale and bias.
// halves = 2: x is an fp32 activation as bf16 hi | lo rows ([M][2K]), S
// counts the parts of both halves.
bool gemm_splitk_plan(int M, int K, int N, int cus, int *S, int *kp, int halves = 1);
size_t gemm_splitk_workspace_bytes(int M, int N, int S);
hipError_t launch_gemm_splitk(const uint32_t *w, const float *scale, const void *x, void *y, int yt_bf16, int M, int K,
                              int N, int S, int kp, float *part, hipStream_t stream, const float *bias, int halves = 1);
// The split for 2:4 weights (GPU layout), any token count from 1, bf16 x.
// halves = 2: x2 [M][2K] bf16 hi | lo rows (an fp32 activation), parts over
// both halves.
bool gemm_sp_splitk_plan(int M, int K, int N, int cus, int *S, int *sp, int halves = 1);
hipError_t launch_gemm_sp_splitk(const uint32_t *meta, const float *scale, const void *x, void *y, int yt_bf16, int M,
                                 int K, int N, int S, int sp, float *part, hipStream_t stream, const float *bias,
                                 int prepared, int halves = 1);
// Whole-K 2:4 GEMM over x2 = [M][2K] bf16 hi | lo rows (5-bit or prepared
// metadata), one K loop of 2K columns.
hipError_t launch_gemm_sp_planes(const uint32_t *meta, int prepared, const float *scale, const uint16_t *x2, void *y,
                                 int yt_bf16, int M, int K, int N, hipStream_t stream);
// 1-2 tokens (3-4 fp32 tokens) over 2:4 metadata (GPU 5-bit layout, K % 4
// == 0, N % 4 == 0): S chunk partials of M * N fp32 in part, added in order
// into y by the last chunk of each 256-row block (counters: the split-K
// GEMV's, zero between launches).
bool sp24_gemv_plan(int M, int K, int N, int xt_bf16, int *S);
hipError_t launch_sp24_gemv(const uint32_t *meta, const float *scale, const void *x, int xt_bf16, void *y,
                            int yt_bf16, int M, int K, int N, int S, float *part, unsigned *counters,
                            hipStream_t stream);
// 2:4 metadata (GPU 5-bit layout) -> its prepared form, [N][K/16] words
// (K % 64 == 0), and the whole-K GEMM over it (bf16 x, aligned).
hipError_t launch_sp24_prepare(const uint32_t *meta, uint32_t *out, int N, int K, hipStream_t stream);
hipError_t launch_gemm_sp_prepared(const uint32_t *prep, const float *scale, const void *x, void *y, int yt_bf16,
                                   int M, int K, int N, hipStream_t stream, const float *bias);
// Whole-K GEMM over x2 = [M][2K] bf16 hi | lo rows (K % 64 == 0, aligned).
hipError_t launch_gemm_planes(const uint32_t *w, const float *scale, const uint16_t *x2, void *y, int yt_bf16, int M,
                              int K, int N, hipStream_t stream, const float *bias);
// x [M][K] f32 -> [M][2K] bf16 hi | lo rows (K even).
hipError_t launch_to_planes(const float *x, uint16_t *x2, int M, int K, hipStream_t stream);
// The balanced one-token kernel takes this launch (one token, K % 64 == 0
// up to 16384, aligned operands, rows within its per-wave slots).
bool gemv_bal_fits(const uint32_t *w, const void *x, int B, int K, int N);
size_t gemv_sk_workspace_bytes(int K, int N, int cus);
hipError_t launch_gemv_sk(const uint32_t *w, const float *scale, const void *x, const void *x2, int xs,
                          void *y, int yt_bf16, int B, int K, int N, float *part, unsigned *counters,
                          const float *bias, int cus, hipStream_t stream);

// Decode GEMV, B <= 16 tokens (frx_gemv.hip).
// One bf16 token through the whole-rows kernels (M == 1, H and I multiples
// of 64 up to 16384): gate/up/act into bf16 hi/lo planes h_planes [2][N],
// then the linear rows over both planes (x_planes [2][K]).
bool gemv_rows_ffn_ok(int M, int H, int I);
hipError_t launch_gemv_rows_glu_planes(const uint32_t *w_gate, const float *s_gate, const uint32_t *w_up,
                                       const float *s_up, const void *x, uint16_t *h_planes, int K, int N,
                                       int gelu, hipStream_t stream);
hipError_t launch_gemv_rows_planes(const uint32_t *w, const float *scale, const uint16_t *x_planes, void *y,
                                   int yt_bf16, int K, int N, hipStream_t stream);
// Two bf16 tokens through the 4-segment kernels (M == 2, H and I multiples of
// 64 up to 14336): gate/up/act into bf16 hi/lo planes h_planes [2][2][N],
// then the linear rows over both planes of both tokens (x_planes [2][2][K]).
bool gemv_rows4_ffn_ok(int M, int H, int I);
hipError_t launch_gemv_rows4_glu_planes(const uint32_t *w_gate, const float *s_gate, const uint32_t *w_up,
                                        const float *s_up, const void *x, uint16_t *h_planes, int B, int K, int N,
                                        int gelu, hipStream_t stream);
hipError_t launch_gemv_rows4_planes(const uint32_t *w, const float *scale, const uint16_t *x_planes, void *y,
                                    int yt_bf16, int K, int N, hipStream_t stream);
// bias: optional per-row f32 bias [N] added to every token's output after
// the scale (null: none).
hipError_t launch_gemv(const uint32_t *w, const float *scale, const void *x,
                       int xt_bf16, void *y, int yt_bf16, int B, int K, int N,
                       hipStream_t stream, const float *bias = nullptr);
// Decode FFN first half, B <= 16 tokens (frx_gemv.hip): h[B][N] (fp32) =
// act(gate) * up with gate/up = (W x) * scale for two [N][K] matrices.
hipError_t launch_gemv_glu(const uint32_t *w_gate, const float *s_gate, const uint32_t *w_up,
                           const float *s_up, const void *x, int xt_bf16, float *h, int B, int K,
                           int N, int gelu, hipStream_t stream);
// The same with bf16 activations, h written as two bf16 planes (hi [B][N]
// then lo [B][N], hi + lo = h to 2^-17), B <= 16 (frx_gemv.hip).
hipError_t launch_gemv_glu_planes(const uint32_t *w_gate, const float *s_gate, const uint32_t *w_up,
                                  const float *s_up, const void *x, uint16_t *h_planes, int B, int K,
                                  int N, int gelu, hipStream_t stream);
// Decode GEMV over activations given as bf16 hi/lo planes (hi [B][K] then
// lo [B][K]), B <= 16 (frx_gemv.hip).
hipError_t launch_gemv_planes(const uint32_t *w, const float *scale, const uint16_t *x_planes, void *y,
                              int yt_bf16, int B, int K, int N, hipStream_t stream);
// h[i] = act(g[i]) * u[i], n elements, fp32 (in place allowed: h == g).
hipError_t launch_glu_combine(const float *g, const float *u, float *h, size_t n, int gelu,
                              hipStream_t stream);
// 2:4 decode GEMV, B <= 16 tokens (frx_gemv.hip).
hipError_t launch_gemv_sp24(const uint32_t *meta, const float *scale,
                            const void *x, int xt_bf16, void *y, int yt_bf16,
                            int B, int K, int N, hipStream_t stream);
// Dense / 2:4 GEMM, any M (frx_gemm.hip). sp24 selects the metadata layout.
hipError_t launch_gemm(const uint32_t *w, const float *scale, const void *x,
                       int xt_bf16, void *y, int yt_bf16, int M, int K, int N,
                       int sp24, hipStream_t stream, const float *bias = nullptr);

// One-launch decode FFN, M <= 3 tokens (frx_ffn.hip). ffn1_supported says
// whether the shape fits the kernel on a device with `cus` compute units and
// returns its grid and dynamic LDS. hs: ffn1_h_bytes(B, I) of device memory
// for h; bar: ffn1_barrier_bytes() of zero-initialised device memory owned
// by the caller (one per stream of launches).
bool ffn1_supported(int B, int H, int I, int xt_bf16, int cus, int *grid, size_t *lds);
size_t ffn1_h_bytes(int B, int I);
size_t ffn1_barrier_bytes();
size_t ffn1_error_word();
hipError_t launch_ffn1(const void *x, int xt_bf16, const uint32_t *wg, const float *sg, const uint32_t *wu,
                       const float *su, const uint32_t *wd, const float *sd, uint32_t *hs, void *y,
                       int yt_bf16, unsigned *bar, int B, int H, int I, int gelu, int G, size_t lds,
                       hipStream_t stream);

// CPU 2:4 layout -> GPU 5-bit layout on the device (frx_ingest.hip); K % 4 == 0.
// Per-row ternary quantisation (rule 0: quantize_ternary, 1: the STE rule of
// BitLinear::forward_ste) of W [N][K] (f32, or bf16 when wt_bf16), K % 16 ==
// 0: scale [N], packed [N][K/16].
hipError_t launch_quantize_flat(const void *w, int wt_bf16, size_t n, size_t block, int rule, uint32_t *packed,
                                float *scale, hipStream_t stream);
hipError_t launch_dequantize(const uint32_t *packed, const float *scales, size_t n, size_t block, float *out,
                             hipStream_t stream);
hipError_t launch_prune_sparse24(const void *w, int wt_bf16, int N, int K, int per_row, uint8_t *patterns,
                                 uint8_t *signs, uint32_t *meta, float *scale, hipStream_t stream);
hipError_t launch_quantize(const void *w, int wt_bf16, int N, int K, int rule, uint32_t *packed, float *scale,
                           hipStream_t stream);
hipError_t launch_sp24_cpu_to_gpu(const uint8_t *patterns, const uint8_t *signs, int N, int K, uint32_t *meta,
                                  hipStream_t stream);

// The reference's other matmul forms (frx_variants.hip).
// Index-list decode: y[m][r] = scale * (sum of x[m][pos] - sum of x[m][neg])
// over the CSR lists of row r.
hipError_t launch_index_decode(const uint32_t *pos_off, const uint32_t *pos_idx, const uint32_t *neg_off,
                               const uint32_t *neg_idx, float scale, const void *x, int xt_bf16, void *y,
                               int yt_bf16, int M, int K, int N, hipStream_t stream);
// counts[0..2] (device) = number of -1, 0, +1 codes in nwords packed words.
hipError_t launch_stats(const uint32_t *w, size_t nwords, unsigned long long *counts, hipStream_t stream);
// xs[m][k] = x[m][k] * scales[k / block_size] (fp32).
hipError_t launch_block_prescale(const void *x, int xt_bf16, const float *scales, int block_size, float *xs, int M,
                                 int K, hipStream_t stream);
hipError_t launch_fill(float *p, float v, size_t n, hipStream_t stream);
// [H][E] router -> [E][H].
hipError_t launch_router_transpose(const void *src, int rt_bf16, void *dst, int H, int E, hipStream_t stream);

// MoE pipeline (frx_moe.hip).
// Most routed rows (tokens x top_k) of the MoE decode path.
constexpr int MOE_DEC_MAXA = 4;

struct MoeWorkspace {
  uint32_t *idx;       // [T*k] selected experts (sorted order per token)
  float *wts;          // [T*k] routing weights
  int *counts;         // [E] tokens per expert
  int *offsets;        // [E+1] exclusive scan of counts
  int *perm_token;     // [T*k] token of each expert-sorted row
  int *row_expert;     // [T*k] expert of each expert-sorted row
  float *lora_ax;      // [T*k][2 * MOE_LORA_MAXR] LoRA A x of the gate and up adapters
  float *lora_ah;      // [T*k][MOE_LORA_MAXR] LoRA A h of the down adapter
  int *inv;            // [T*k] expert-sorted row of assignment t*k+j
  int *tiles;          // [4*max_tiles] (expert, first row, rows, token blocks)
                       // per M tile
  int *ntiles;         // [1]
  uint16_t *h_hi;      // [T*k][I] SwiGLU output, bf16 hi plane; the bf16
                       // engine-2 path uses h_hi.. as [T*k][2I] (hi | lo
                       // halves per row; h_lo follows h_hi contiguously)
  uint16_t *h_lo;      // [T*k][I] lo plane
  float *dout;         // [T*k][H] down-projection rows
  float *dout_lo;      // [T*k][H] second partial (engine-2 path: the second
                       // K part)
  uint16_t *x2;        // [T][2H] f32 x as bf16 hi | lo rows (engine-2 path)
  unsigned *cnt = nullptr;  // decode path: (column block, token) arrival
                            // counters, zero between launches; null: the
                            // combine runs as a launch of its own
};
// Largest LoRA rank of the MoE adapters.
constexpr int MOE_LORA_MAXR = 64;
// LoRA adapters of the MoE experts: tbl is a device array of 6 x 64
// pointers, [2 k] = A and [2 k + 1] = B of kind k (0 gate, 1 up, 2 down) at
// index 64 * slot + expert; nullptr tbl: no adapters.
struct MoeLora {
  const float *const *tbl = nullptr;
  int rank = 0;
  float scaling = 0.f;
};
size_t moe_workspace_bytes(int T, int H, int I, int E, int top_k);
void moe_workspace_carve(void *base, int T, int H, int I, int E, int top_k,
                         MoeWorkspace *ws);
hipError_t launch_moe(const void *x, int xt_bf16, const void *router,
                      int rt_bf16, const uint32_t *const *w_gate,
                      const float *const *s_gate, const uint32_t *const *w_up,
                      const float *const *s_up, const uint32_t *const *w_down,
                      const float *const *s_down, int T, int H, int I, int E,
                      int top_k, int act, void *y, int yt_bf16,
                      uint32_t *topk_idx, float *topk_w, const MoeWorkspace &ws,
                      int routing, const MoeLora &lora, hipStream_t stream);

}  // namespace frx
