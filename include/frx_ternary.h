/*
 * frx_ternary.h — C ABI of the MI355X (gfx950) ternary linear backend for
 * FerrisRes. Library: ferrisres_amd/libfrx_ternary.so.
 *
 * Weight layouts are the reference's, unchanged:
 *  - dense: row-major [N][K/16] u32, 16 two-bit codes per word, LSB first,
 *    codes {0b00:-1, 0b01:0, 0b10:+1, 0b11:0}
 *    (src/compute/kernels/ternary_matmul.rs:3-11, src/model/ternary.rs:134-140);
 *    one f32 scale per output row (ternary_matmul.rs:27,74).
 *  - 2:4 sparse: per row ceil(ceil(K/4)/6) u32 words, six 5-bit groups per
 *    word, group = pattern[2:0] | sign_lo[3] | sign_hi[4], sign bit 1 = -1
 *    (src/compute/kernels/sparse_ternary.rs:7-10,71-108).
 *
 * Conventions:
 *  - GPU entry points take device pointers owned by the caller, enqueue work
 *    on the context's stream and never synchronise (the reference records
 *    into a caller-owned CommandEncoder, kernels/ternary_matmul.rs:167-225).
 *  - Errors are returned, never raised: the enum is 1:1 with
 *    FerrisResError (src/error.rs:4-22). frx_last_error() gives the message.
 *  - y[m][n] = scale[n] * sum_k dec(W[n][k]) * x[m][k] (fp32 accumulation).
 */
#ifndef FRX_TERNARY_H
#define FRX_TERNARY_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct frx_ctx frx_ctx;

/* 1:1 with FerrisResError::{Gpu, Shape, Device, Shader, OOM, Unsupported}
 * (src/error.rs:4-22). */
typedef enum frx_status {
  FRX_OK = 0,
  FRX_ERR_GPU = 1,
  FRX_ERR_SHAPE = 2,
  FRX_ERR_DEVICE = 3,
  FRX_ERR_SHADER = 4,
  FRX_ERR_OOM = 5,
  FRX_ERR_UNSUPPORTED = 6,
  FRX_STATUS_RANGE_ = 0x7fffffff /* range sentinel, never returned */
} frx_status;

/* Each argument enum carries a sentinel at INT_MAX so that any int a caller
 * passes (a value from a newer header, or a corrupt one) is a valid value of
 * the type in C++ as well as C; the library rejects it with a status. */
typedef enum frx_dtype { FRX_F32 = 0, FRX_BF16 = 1, FRX_DTYPE_RANGE_ = 0x7fffffff } frx_dtype;

/* Expert / FFN activation. FRX_ACT_SILU and FRX_ACT_GELU_TANH gate the up
 * projection: h = act(g) * u (the dense FFN branch,
 * src/model/cpu_block_attn_res.rs:2319-2324, the MoE glue :1176-1178 and
 * CpuMoELayer, src/model/cpu_moe.rs:337-352; GeLU-tanh as
 * gemma_mapper::gelu_tanh, src/model/gemma_mapper.rs:2073-2077, with
 * c = sqrt(2/pi) evaluated in f32). FRX_ACT_GELU_TANH_GATE is
 * TernaryMoELayer::forward's use_gelu branch (src/model/ternary_moe.rs:
 * 193-200): h = gelu_tanh(g) with the literal c = 0.7978845608 and no up
 * product; frx_moe_ternary_ffn only. */
typedef enum frx_activation {
  FRX_ACT_SILU = 0,
  FRX_ACT_GELU_TANH = 1,
  FRX_ACT_GELU_TANH_GATE = 2,
  FRX_ACT_RANGE_ = 0x7fffffff
} frx_activation;
/* How frx_ternary_ffn runs at decode sizes (see frx_set_ffn_mode). */
typedef enum frx_ffn_mode {
  FRX_FFN_AUTO = 0,        /* M <= 4: two whole-row launches where the
                              shape allows, else the one-launch kernel at
                              M <= 3 where it allows; otherwise two */
  FRX_FFN_ONE_LAUNCH = 1,  /* one launch or FRX_ERR_UNSUPPORTED */
  FRX_FFN_TWO_LAUNCH = 2,  /* gate/up/act launch + down launch */
  FRX_FFN_MODE_RANGE_ = 0x7fffffff
} frx_ffn_mode;

/* Decode GEMV kernels at 2-16 tokens (see frx_set_gemv_split). */
typedef enum frx_gemv_split {
  FRX_GEMV_SPLIT_AUTO = 0,   /* split K where it measured faster: f32 x above 4096 columns (one
                                token: where the balanced kernel does not apply); bf16 x from 5
                                tokens at 14336 columns and from 3 tokens above 16384, at least
                                3072 rows */
  FRX_GEMV_SPLIT_ALWAYS = 1, /* split K at every 2-16 token call */
  FRX_GEMV_SPLIT_NEVER = 2,  /* whole-K kernels only */
  FRX_GEMV_SPLIT_RANGE_ = 0x7fffffff
} frx_gemv_split;

/* Routing semantics of frx_moe_ternary_ffn (see frx_set_moe_routing). */
typedef enum frx_moe_routing {
  FRX_MOE_TERNARY_MOE_LAYER = 0, /* TernaryMoELayer and the GPU-path glue */
  FRX_MOE_CPU_MOE_LAYER = 1,     /* CpuMoELayer */
  FRX_MOE_ROUTING_RANGE_ = 0x7fffffff
} frx_moe_routing;

/* ---- context -------------------------------------------------------------
 * Replaces the Arc<Device>/Arc<Queue> pair ops are built from
 * (TernaryMatMulOp::new, src/compute/kernels/ternary_matmul.rs:84-155).
 * One context per (thread, stream); contexts are independent. */
frx_status frx_create(int device, frx_ctx **out);
void frx_destroy(frx_ctx *ctx);
/* Caller-owned hipStream_t (NULL = the device's null stream); the analogue of
 * the caller-owned CommandEncoder in TernaryMatMulOp::dispatch. Switching to
 * another stream makes it wait, on the device, for the work already enqueued
 * on the previous one (the context's workspaces serve one stream at a time);
 * not while either stream is being captured into a graph. frx_destroy waits
 * for the context's stream before it frees the workspaces. */
frx_status frx_set_stream(frx_ctx *ctx, void *hip_stream);
/* Waits for all work enqueued on the context's stream. Returns FRX_ERR_GPU
 * if a one-launch FFN since the last call timed out at its grid barrier
 * (see frx_ternary_ffn). */
frx_status frx_synchronize(frx_ctx *ctx);
/* Message of the last failed call on this context ("" if none). */
const char *frx_last_error(const frx_ctx *ctx);
const char *frx_status_string(frx_status s);
/* Library version string ("frx_ternary <major>.<minor>.<patch> gfx950"). */
const char *frx_version(void);

/* ---- dense ternary linear --------------------------------------------------
 * Replaces TernaryMatMulOp::dispatch(encoder, ternary, scales, input, output,
 * seq_len, in_cols, out_rows) (src/compute/kernels/ternary_matmul.rs:167-225),
 * WGSL entry ternary_matmul_main (:32-75).
 *   w     [N][K/16] u32      scale [N] f32
 *   x     [M][K]  xt         y     [M][N] yt
 * M = seq_len, K = in_cols, N = out_rows. Requires K % 16 == 0 (the u32
 * repack of ternary.rs:1317-1328 is row-aligned only then), M, N >= 1,
 * N*K/4 bytes of weights below 4 GiB, and pointers aligned to their element
 * size. M <= 16 runs the decode GEMV kernel, larger M the MFMA GEMM kernel.
 * The kernels read x and scale and write y 16 bytes at a time: a sub-slice
 * at another offset is copied into an aligned context workspace on the
 * stream (x and scale before the launch, y back after it; allocated on the
 * first such call at a larger size, which must not be under graph
 * capture). */
frx_status frx_ternary_linear(frx_ctx *ctx, const uint32_t *w,
                              const float *scale, const void *x, frx_dtype xt,
                              void *y, frx_dtype yt, uint32_t M, uint32_t K,
                              uint32_t N);

/* ---- dense ternary linear with bias ----------------------------------------
 * Replaces TernaryLinear::forward / forward_packed / forward_decode with a
 * bias (src/model/ternary_linear.rs:94-165): output = ternary_matmul(...)
 * and then output[s][r] += bias[r] for every token s.
 *   bias  [N] f32 device pointer, or NULL (then exactly frx_ternary_linear)
 * y[m][n] = (scale[n] * sum_k dec(W[n][k]) x[m][k]) + bias[n], the product
 * and the addition each rounded to f32 as the reference does (no fused
 * multiply-add), then converted to yt. The bias is added inside the GEMV /
 * GEMM epilogue (no extra launch). Same requirements as frx_ternary_linear;
 * bias needs no particular alignment. */
frx_status frx_ternary_linear_bias(frx_ctx *ctx, const uint32_t *w,
                                   const float *scale, const float *bias,
                                   const void *x, frx_dtype xt, void *y,
                                   frx_dtype yt, uint32_t M, uint32_t K,
                                   uint32_t N);

/* ---- same-x group of dense ternary linears -----------------------------------
 * Several matrices with the same in_cols applied to one x: the decode step's
 * Q/K/V projections (src/model/cpu_block_attn_res.rs:2254-2263) and the
 * FFN's gate and up projections (:2319-2320), which the reference issues as
 * separate gpu_ternary_matmul_vram calls on the same input. For each
 * i < count: y[i] = x W[i]^T * scale[i], exactly frx_ternary_linear(w[i],
 * scale[i], x, y[i], M, K, N[i]).
 *   x [M][K] xt; w[i] [N[i]][K/16] u32; scale[i] [N[i]] f32; y[i] [M][N[i]]
 *   yt. w, scale, N and y are host arrays of count entries (device pointers
 *   in w, scale and y); 1 <= count <= 4.
 * At one token (bf16 or f32 x, K % 64 == 0 up to 16384, 16-byte aligned
 * weights, x, scales and outputs) the group is one launch over the
 * matrices' concatenated rows, so x is read once and the launch's fixed
 * cost is paid once; otherwise each matrix runs as frx_ternary_linear. */
frx_status frx_ternary_linear_group(frx_ctx *ctx, const void *x, frx_dtype xt, uint32_t M,
                                    uint32_t K, uint32_t count, const uint32_t *const *w,
                                    const float *const *scale, const uint32_t *N, void *const *y,
                                    frx_dtype yt);

/* ---- dense ternary linear with column-block scales --------------------------
 * Replaces ternary_matmul_blocked (src/model/ternary.rs:541-579): each block
 * of block_size input columns has its own scale, shared by all rows, and
 * there is no per-row scale:
 *   y[m][n] = sum_b block_scales[b] * sum_{k in block b} dec(W[n][k]) x[m][k]
 *   block_scales [ceil(K / block_size)] f32 (device). Same layouts and
 * requirements as frx_ternary_linear. The activations are prescaled per
 * element in fp32 (a context workspace of M*K*4 bytes, allocated on the
 * first call at a larger size) and run through the dense kernels. */
frx_status frx_ternary_linear_blocked(frx_ctx *ctx, const uint32_t *w,
                                      const float *block_scales,
                                      uint32_t block_size, const void *x,
                                      frx_dtype xt, void *y, frx_dtype yt,
                                      uint32_t M, uint32_t K, uint32_t N);

/* ---- index-list decode -------------------------------------------------------
 * Replaces ternary_matmul_sparse_decode (src/model/ternary.rs:647-673) with
 * the lists of ternary_sparse_indices (:681-707) as CSR arrays (device):
 * row r's +1 columns are pos_idx[pos_off[r] .. pos_off[r+1]), its -1 columns
 * neg_idx[neg_off[r] .. neg_off[r+1]).
 *   y[m][r] = scale * (sum_pos x[m][j] - sum_neg x[m][j])
 * x [M][K] xt, y [M][N] yt; every index must be < K. */
frx_status frx_ternary_sparse_decode(frx_ctx *ctx, const uint32_t *pos_off,
                                     const uint32_t *pos_idx,
                                     const uint32_t *neg_off,
                                     const uint32_t *neg_idx, float scale,
                                     const void *x, frx_dtype xt, void *y,
                                     frx_dtype yt, uint32_t M, uint32_t K,
                                     uint32_t N);

/* ---- statistics of a packed matrix -------------------------------------------
 * Replaces the counts of ternary_stats (src/model/ternary.rs:725-746) for a
 * matrix already on the device in the dense layout [N][K/16] u32:
 * counts[0] = number of -1 codes, counts[1] = zeros (codes 0b01 and 0b11),
 * counts[2] = +1 codes (device array of 3 u64, stream-ordered). The ratios
 * are counts / (N*K) and the compression ratio is 16, as in the reference. */
frx_status frx_ternary_stats(frx_ctx *ctx, const uint32_t *w, uint32_t N,
                             uint32_t K, unsigned long long *counts);

/* ---- 2:4 sparse ternary linear ---------------------------------------------
 * Replaces SparseTernaryMatMulOp::dispatch (src/compute/kernels/
 * sparse_ternary.rs:194-247), WGSL entry sparse_ternary_matmul_main (:54-112).
 *   meta [N][ceil(ceil(K/4)/6)] u32, scale [N] f32. Requires K % 4 == 0.
 * With K % 64 == 0 both dtypes of x run on the sparse matrix pipe (f32 x as
 * bf16 hi | lo rows in a context workspace); below 512 tokens the K range is
 * split over workgroups where the token tiles leave compute units idle
 * (fp32 partials in a context workspace, added in a fixed order). */
frx_status frx_sparse24_ternary_linear(frx_ctx *ctx, const uint32_t *meta,
                                       const float *scale, const void *x,
                                       frx_dtype xt, void *y, frx_dtype yt,
                                       uint32_t M, uint32_t K, uint32_t N);

/* ---- 2:4 metadata in its prepared form --------------------------------------
 * No counterpart in the reference (its WGSL kernel decodes the 5-bit groups
 * per use). For callers that keep 2:4 weights resident and run prefill-sized
 * batches: the GPU 5-bit layout re-encoded once so that each (row, 64-column
 * step, 16-column quarter) is one u32 from which the sparse matrix pipe's
 * operands decode in 9 ops (position nibbles as the pipe's index, the 8 sign
 * bits gathered), instead of a window funnel and a lookup per group.
 *   meta [N][ceil(ceil(K/4)/6)] u32 -> prepared [N][K/16] u32 (device,
 *   16-byte aligned), K % 64 == 0; patterns 6 and 7 read as 5 and bits
 *   30-31 of a word are ignored, as in frx_sparse24_ternary_linear.
 * frx_sparse24_ternary_linear prepares into a context workspace by itself
 * from 512 tokens; a caller that prepares at upload saves that pass
 * (10.6 us at 11008 x 4096). */
frx_status frx_sparse24_prepare(frx_ctx *ctx, const uint32_t *meta, uint32_t K,
                                uint32_t N, uint32_t *prepared);

/* frx_sparse24_ternary_linear over prepared metadata (frx_sparse24_prepare):
 * the same products on the sparse matrix pipe, equal to it up to fp32
 * summation order (bit for bit where both take the same engine, i.e. bf16 x
 * with K % 64 == 0 at more than 16 tokens or where the K split applies).
 * x must be FRX_BF16 (FRX_ERR_UNSUPPORTED otherwise); y f32 or bf16. */
frx_status frx_sparse24_prepared_linear(frx_ctx *ctx, const uint32_t *prepared,
                                        const float *scale, const void *x,
                                        frx_dtype xt, void *y, frx_dtype yt,
                                        uint32_t M, uint32_t K, uint32_t N);

/* ---- MoE ternary expert layer -----------------------------------------------
 * Replaces the GPU-path MoE glue of the model (router, softmax, stable top-k,
 * per-expert ternary FFN, weighted sum; src/model/cpu_block_attn_res.rs:
 * 1148-1184 and :2284-2316) and TernaryMoELayer::forward
 * (src/model/ternary_moe.rs:145-223), with per-row scales. Their routing is
 * the same; their experts differ only for GeLU: the glue computes
 * gelu(g) * u (act = FRX_ACT_GELU_TANH), TernaryMoELayer gelu(g) alone
 * (act = FRX_ACT_GELU_TANH_GATE). With SiLU both are silu(g) * u. Routing
 * is done on the device (router GEMV, softmax, stable sort, per-expert
 * histogram and scan, token permutation); the experts run as grouped ternary
 * GEMMs.
 *   x [T][H] xt; router [E][H] rt (row e = expert e, ternary_moe.rs:157)
 *   w_gate[e], w_up[e]: [I][H/16] u32, s_gate[e], s_up[e]: [I] f32
 *   w_down[e]: [H][I/16] u32, s_down[e]: [H] f32   (device pointers; the
 *   pointer arrays themselves are host arrays of length E)
 *   y [T][H] yt; topk_idx [T][top_k] u32 and topk_w [T][top_k] f32 (device,
 *   may be NULL).
 * With FRX_ACT_GELU_TANH_GATE the up projection is not used: w_up and s_up
 * may be NULL (the arrays or their entries).
 * Requires H % 16 == 0, I % 16 == 0, 1 <= top_k <= E <= 64.
 * Workspace is allocated on the context on first use and grown on the first
 * call at a larger size (not under graph capture); a replaced workspace is
 * kept until frx_destroy, so graphs captured at smaller sizes stay valid. */
frx_status frx_moe_ternary_ffn(
    frx_ctx *ctx, const void *x, frx_dtype xt, const void *router,
    frx_dtype rt, const uint32_t *const *w_gate, const float *const *s_gate,
    const uint32_t *const *w_up, const float *const *s_up,
    const uint32_t *const *w_down, const float *const *s_down, uint32_t T,
    uint32_t H, uint32_t I, uint32_t E, uint32_t top_k, frx_activation act,
    void *y, frx_dtype yt, uint32_t *topk_idx, float *topk_w);

/* ---- gated pair (first half of the dense FFN) -------------------------------
 * Replaces the gate and up gpu_ternary_matmul_vram calls plus the host
 * activation and product of the dense FFN branch
 * (src/model/cpu_block_attn_res.rs:2319-2324):
 *   h = act(x Wg^T * s_gate) * (x Wu^T * s_up),  h [M][I] f32 (device)
 * Same arguments as frx_ternary_ffn below. M <= 16 is one launch that reads x
 * once for both matrices; larger M runs two GEMMs and an element-wise
 * combine (up projection in a context workspace, allocated on first use). */
frx_status frx_ternary_glu(frx_ctx *ctx, const void *x, frx_dtype xt,
                           const uint32_t *w_gate, const float *s_gate,
                           const uint32_t *w_up, const float *s_up,
                           uint32_t M, uint32_t H, uint32_t I,
                           frx_activation act, float *h);

/* ---- dense ternary FFN ------------------------------------------------------
 * Replaces the dense FFN branch of the decode step
 * (src/model/cpu_block_attn_res.rs:2317-2326; prefill forward: :1185-1194):
 * three ternary matmul calls (gate, up, down) with the activation and the
 * product on the host.
 *   y = ((act(x Wg^T * s_gate)) * (x Wu^T * s_up)) Wd^T * s_down
 *   act = SiLU g/(1+e^-g) (FRX_ACT_SILU) or GeLU-tanh (FRX_ACT_GELU_TANH).
 *   x [M][H] xt; w_gate, w_up [I][H/16] u32, s_gate, s_up [I] f32;
 *   w_down [H][I/16] u32, s_down [H] f32; y [M][H] yt (device pointers).
 * Requires H % 16 == 0, I % 16 == 0. The intermediate h = act(g) * u
 * ([M][I]) lives in a context workspace of M*I*4 bytes. Paths, by M and the
 * dtype of x (FRX_FFN_AUTO):
 *  - bf16 x, M = 1 (H, I multiples of 64 up to 16384) or M = 2 to 4 (up to
 *    14336), 16-byte aligned weights: two launches that read whole weight
 *    rows per wave (4 row segments per MFMA from 2 tokens); h as bf16 hi +
 *    lo planes, |h - hi - lo| <= 2^-17 |h|. At M = 3 and 4 the down launch
 *    is the split-K GEMV over both planes (frx_set_gemv_split) where I >=
 *    8192.
 *  - bf16 x, 5 <= M <= 16: gate/up/act launch writing h as bf16 hi + lo
 *    planes (2^-17), then the down GEMV over both planes (split-K where
 *    I >= 8192).
 *  - M = 3 in FRX_FFN_ONE_LAUNCH mode (H <= 4096, I <= 11520, multiples of
 *    64, 16-byte aligned weights): one launch with a grid barrier between
 *    the halves; h as bf16 hi + lo planes (2^-17). Other M <= 3 shapes that
 *    the paths above do not take run it in FRX_FFN_AUTO too.
 *  - f32 x at M <= 16, and every other shape at M <= 16: h in fp32, then the
 *    down GEMV with fp32 input, as the reference keeps it.
 *  - M > 16: gate and up GEMMs (the up projection in a second context
 *    workspace), an element-wise fp32 combine, then the down GEMM.
 * Workspaces grow on the first call at a larger size, and that first call
 * must not be under graph capture. A workspace replaced by a larger one is
 * kept until frx_destroy, so graphs captured at smaller sizes stay valid.
 * The one-launch kernel needs all its workgroups (one per CU) resident at
 * once; if another kernel holds CUs so that they are not, its barrier times
 * out, the outputs are invalid and the next frx_synchronize returns
 * FRX_ERR_GPU. Callers that share the GPU with concurrent kernels select
 * FRX_FFN_TWO_LAUNCH. */
frx_status frx_ternary_ffn(frx_ctx *ctx, const void *x, frx_dtype xt,
                           const uint32_t *w_gate, const float *s_gate,
                           const uint32_t *w_up, const float *s_up,
                           const uint32_t *w_down, const float *s_down,
                           uint32_t M, uint32_t H, uint32_t I,
                           frx_activation act, void *y, frx_dtype yt);

/* ---- dense ternary FFN without allocation ------------------------------------
 * No counterpart in the reference. For callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc. Same arguments, semantics and kernels as frx_ternary_ffn
 * in FRX_FFN_TWO_LAUNCH execution with FRX_GEMV_SPLIT_NEVER (whatever
 * frx_set_ffn_mode and frx_set_gemv_split selected: the split-K down launch
 * needs a context workspace), but
 * the intermediate lives in a fixed device array of the library
 * (FRX_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends) and the
 * call allocates nothing. It needs M*I*4 bytes of that array (rounded up to
 * 256) for M <= 16 and twice that above; larger shapes return
 * FRX_ERR_UNSUPPORTED. Every call on a GPU shares that GPU's array: calls
 * that overlap on one GPU (other streams, other contexts, other threads)
 * race on it, and must be serialised by the caller. */
#define FRX_NOALLOC_SCRATCH_BYTES (4u << 20)
frx_status frx_ternary_ffn_noalloc(frx_ctx *ctx, const void *x, frx_dtype xt,
                                   const uint32_t *w_gate, const float *s_gate,
                                   const uint32_t *w_up, const float *s_up,
                                   const uint32_t *w_down, const float *s_down,
                                   uint32_t M, uint32_t H, uint32_t I,
                                   frx_activation act, void *y, frx_dtype yt);

/* Selects the routing semantics of frx_moe_ternary_ffn on this context
 * (default FRX_MOE_TERNARY_MOE_LAYER: router [E][H], softmax over all
 * experts, stable top-k by probability, weights renormalised over the top-k;
 * src/model/ternary_moe.rs:145-223). FRX_MOE_CPU_MOE_LAYER follows
 * CpuMoELayer (src/model/cpu_moe.rs:146-201,365-400): the router is read as
 * [H][E] (transposed into a context workspace of H*E elements on the device,
 * allocated on the first call at a larger size), the top-k is ranked by
 * logit (ties by index; a NaN logit puts the token's experts in index
 * order), the weights are exp(l - l_max) over the selected logits divided by
 * their sum, and experts whose weight is below 1e-8 in magnitude are
 * skipped. The logits are sequential f32 dot products over H; the
 * reference's matrixmultiply::sgemm sums in an order this library does not
 * reproduce. CpuMoELayer's LoRA adapters are set with frx_set_moe_lora. */
frx_status frx_set_moe_routing(frx_ctx *ctx, frx_moe_routing routing);

/* LoRA adapters on the MoE experts: CpuMoELayer::expert_forward_*_with_lora
 * (src/model/cpu_moe.rs:281-363) with LoraLayer::forward
 * (src/training/lora.rs:138-167), for LoraManager::forward's per-expert
 * modules "moe.expert.{e}.gate/up/down" (src/training/lora.rs:447-457):
 *   gated = W_gate x + scaling * B_gate (A_gate x)   (before the activation)
 *   upped = W_up x   + scaling * B_up (A_up x)
 *   down  = W_down h + scaling * B_down (A_down h),  h = act(gated) * upped
 * for each expert and projection whose A and B are both non-NULL. Device
 * f32, row-major: A_gate, A_up [rank][H]; B_gate, B_up [I][rank]; A_down
 * [rank][I]; B_down [H][rank]. Each member below is a host array of
 * `experts` device pointers (the array itself may be NULL: no adapter of
 * that projection). The pointer arrays are copied by this call
 * (synchronously); the matrices are read by every later
 * frx_moe_ternary_ffn on the context, whose expert count must then equal
 * `experts` (FRX_ERR_SHAPE otherwise), until frx_set_moe_lora(ctx, NULL, 0)
 * removes them. Each call builds a new device table of the pointers and
 * retires the previous one (frx_release_retired frees it): launches already
 * enqueued and graphs captured earlier keep the adapters and rank they were
 * captured with, and read those matrices on every replay, so a caller that
 * changes, removes or frees adapters must recapture such graphs. 1 <= rank <= 64, 1 <= experts <= 64. Both routing modes. The
 * low-rank sums run in another order than the reference's sequential f32
 * loops (outputs within 1e-3). */
typedef struct frx_moe_lora {
  uint32_t rank;
  float scaling; /* LoraConfig alpha / rank */
  const float *const *a_gate;
  const float *const *b_gate;
  const float *const *a_up;
  const float *const *b_up;
  const float *const *a_down;
  const float *const *b_down;
} frx_moe_lora;
frx_status frx_set_moe_lora(frx_ctx *ctx, const frx_moe_lora *lora, uint32_t experts);

/* Device memory held by the context's workspaces (no counterpart in the
 * reference, whose wgpu buffers are allocated per call): live_bytes in the
 * current workspaces, retired_bytes in workspaces replaced by larger ones
 * (kept because graphs captured at the smaller size still address them),
 * allocations = device allocations made so far. Workspaces grow by at
 * least 1.5x, so rising sizes make O(log) allocations and the retired bytes
 * of a workspace stay below twice its current size. Any pointer may be
 * NULL. */
frx_status frx_workspace_stats(frx_ctx *ctx, size_t *live_bytes, size_t *retired_bytes,
                               uint32_t *allocations);
/* Frees the retired workspaces (and LoRA tables replaced by
 * frx_set_moe_lora) after waiting for the context stream. Only for callers
 * that know no captured graph still uses them. */
frx_status frx_release_retired(frx_ctx *ctx);

/* Forced failure, for testing a caller's fallback path (no counterpart in
 * the reference; its callers fall back to the CPU on any FerrisResError,
 * src/model/cpu_block_attn_res.rs:1004-1031). While status != FRX_OK, every
 * compute and upload entry point on this context returns that status, with
 * a message, before reading its arguments or touching the device;
 * frx_synchronize, frx_free, frx_set_* and frx_destroy still work. FRX_OK
 * clears it. A status outside frx_status is FRX_ERR_UNSUPPORTED. */
frx_status frx_force_status(frx_ctx *ctx, frx_status status);

/* Selects the decode GEMV of frx_ternary_linear / _bias / _group at 2-16
 * tokens (and at one f32 token above 16384 columns) on this context (default
 * FRX_GEMV_SPLIT_AUTO). No counterpart in the
 * reference. The split-K kernel gives each workgroup 128 weight rows and a
 * slice of 256 to 1024 columns, stages that slice of the activations once
 * for all 128 rows, and writes fp32 partial sums to a context workspace of
 * at most ceil(K/256) * 16 * N4 * 4 bytes (N4 = N rounded up to a multiple
 * of 4), plus 256 KiB of tile counters (both allocated on the first split
 * call at a larger size, not under graph capture). The last slice of a row
 * tile to finish adds the slices of each output in slice order, in the same
 * launch. Results differ from the whole-K kernels only in fp32 summation
 * order. */
frx_status frx_set_gemv_split(frx_ctx *ctx, frx_gemv_split mode);

/* Selects the execution of frx_ternary_ffn on this context (default
 * FRX_FFN_AUTO). No counterpart in the reference, whose FFN is three
 * separate matmul calls. */
frx_status frx_set_ffn_mode(frx_ctx *ctx, frx_ffn_mode mode);

/* ---- weight ingest (resident upload, done once) ----------------------------
 * Replaces GpuVramCache::upload / GpuWeightCache::build
 * (src/model/cpu_block_attn_res.rs:3005-3171) and the .stm expert files of
 * expert_loader.rs:6-152: weights reach the device once, in the GPU layout,
 * and are then passed to the entry points above as device pointers.
 * Buffers returned through w_dev / meta_dev / s_dev are allocated by the
 * library and released with frx_free. Synchronous (load time). */

/* Dense [N][K] ternary matrix from pack_ternary bytes (4 codes per byte,
 * src/model/ternary.rs:146-163), K % 16 == 0: *w_dev receives the u32 words
 * [N][K/16] of pack_ternary_u32 (ternary.rs:1317-1328; on a little-endian
 * device the same bytes), *s_dev the per-row scales (row_scales[N], or
 * tensor_scale on every row when row_scales is NULL, as gpu_packed() does,
 * src/model/cpu_linear.rs:164-169). */
frx_status frx_upload_ternary(frx_ctx *ctx, const uint8_t *packed, uint32_t N, uint32_t K,
                              const float *row_scales, float tensor_scale, uint32_t **w_dev,
                              float **s_dev);
/* 2:4 matrix from an .stm file image (expert_loader.rs:6-16,63-106: magic
 * 0x53544D31 "STM1", rows, cols, scale f32, pattern bytes, sign bytes, then
 * the CPU-layout patterns and signs; little-endian). The arrays go to the
 * device and are transcoded there into the GPU 5-bit layout (*meta_dev
 * [N][ceil(K/24)]); *s_dev holds the tensor scale on every row; *N, *K
 * receive rows and cols (may be NULL). FRX_ERR_SHAPE for an image shorter
 * than the header, a wrong magic or truncated arrays (the reference's
 * InvalidData cases), cols % 4 != 0, or arrays too short for rows x cols. */
frx_status frx_upload_stm(frx_ctx *ctx, const void *image, size_t len, uint32_t **meta_dev,
                          float **s_dev, uint32_t *N, uint32_t *K);
/* CPU 2:4 layout (patterns, signs; device pointers) -> GPU layout (meta,
 * device) on the context's stream; bit-exact with frx_sparse24_cpu_to_gpu.
 * Requires K % 4 == 0. No synchronisation, no allocation. */
frx_status frx_sparse24_cpu_to_gpu_device(frx_ctx *ctx, const uint8_t *patterns,
                                          const uint8_t *signs, uint32_t N, uint32_t K,
                                          uint32_t *meta);
/* ---- on-device quantisation (training-side producer of the layout) ----------
 * Replaces quantize_ternary (src/model/ternary.rs:31-57, used by
 * quantize_ste / TernarySteResult::requantize :237-258 and
 * BitLinear::requantize, src/training/shadow_weights.rs:152-160) and the
 * on-the-fly quantisation of BitLinear::forward_ste (shadow_weights.rs:
 * 203-231), applied to every row of W [N][K] on its own (N = 1 with K = n
 * is the reference's call on a whole n-value tensor):
 *   FRX_QUANT_ABSMEAN: alpha = mean|w| / sqrt(2/pi) (1 when sum|w| is not
 *     > 0), q = clamp(round_half_away(w * (1 / alpha)), -1, 1);
 *   FRX_QUANT_STE: alpha = mean|w|, q = +1 where w / alpha > 0.5, -1 where
 *     < -0.5, else 0; every q = 0 when alpha < 1e-10.
 * sum|w| is accumulated left to right in f32, as in the reference, so alpha
 * and every code are bit-identical to the reference applied to that row.
 * w: [N][K] f32, or bf16 (bf16 shadow weights, widened exactly); packed:
 * [N][K/16] u32 codes (q + 1, 16 per word LSB first: pack_ternary then
 * pack_ternary_u32); scale: [N] f32 alpha (the dequantised row is
 * alpha * q). Device pointers, stream-ordered, no allocation. Requires
 * K % 16 == 0 and K > 0. */
typedef enum frx_quant_rule {
  FRX_QUANT_ABSMEAN = 0,
  FRX_QUANT_STE = 1,
  FRX_QUANT_RULE_RANGE_ = 0x7fffffff
} frx_quant_rule;
frx_status frx_quantize_ternary(frx_ctx *ctx, const void *w, frx_dtype wt, uint32_t N, uint32_t K,
                                frx_quant_rule rule, uint32_t *packed, float *scale);

/* Replaces quantize_ternary_blocked (src/model/ternary.rs:76-110): the flat
 * n-value tensor w is cut into blocks of block_size values (the last one
 * shorter when block_size does not divide n) and each block is quantised as
 * quantize_ternary with its own alpha (FRX_QUANT_ABSMEAN above; sum|w|
 * left to right in f32 within the block, len as f32), so alpha and every
 * code are bit-identical to the reference.
 *   w [n] f32 or bf16 (device); packed [ceil(n/16)] u32: the codes of
 *   pack_ternary then pack_ternary_u32 over the flat tensor (zero padding
 *   bits past n); scales [ceil(n/block_size)] f32.
 * n = 0 writes nothing (the reference returns empty vectors). A row-aligned
 * matrix view needs block_size % 16 == 0 and block_size dividing n; then
 * this equals frx_quantize_ternary on [n/block_size][block_size]. Stream-
 * ordered, no allocation. */
frx_status frx_quantize_ternary_blocked(frx_ctx *ctx, const void *w, frx_dtype wt, size_t n,
                                        uint32_t block_size, uint32_t *packed, float *scales);
/* Replaces dequantize_ternary_blocked (src/model/ternary.rs:113-128):
 * out[i] = scales[i / block_size] * dec(code i) for i < n, over the flat
 * packed codes of frx_quantize_ternary_blocked (one f32 product each: exact;
 * codes 0b01 and 0b11 give alpha * 0). packed [ceil(n/16)] u32, scales
 * [ceil(n/block_size)] f32, out [n] f32 (device). */
frx_status frx_dequantize_ternary_blocked(frx_ctx *ctx, const uint32_t *packed, const float *scales,
                                          size_t n, uint32_t block_size, float *out);
/* Replaces prune_fp32_to_sparse_ternary (src/model/sparse_ternary.rs:598-663),
 * the producer of 2:4 expert weights (quantized_model.rs:191,
 * expert_loader.rs:380-390): per group of 4 values the two largest |w|
 * (ties to the lower position, as the reference's stable sort) become
 * +-1, the other two 0. Sign bits are packed as the reference packs them:
 * bit 0 from the larger |w|, bit 1 from the second, and read back as the
 * signs of the lower and higher positions (so a group whose larger |w| sits
 * at the higher position with the two signs different decodes with them
 * exchanged, exactly as the reference's SparseTernaryMatrix does).
 *   w [N][K] f32 or bf16 (device), K % 4 == 0.
 *   patterns [ceil(N*K/8)] u8, signs [ceil(N*K/16)] u8: the CPU layout
 *     SparseTernaryMatrix holds (both NULL: not written);
 *   meta [N][ceil(K/24)] u32: the same matrix in the GPU 5-bit layout, as
 *     frx_sparse24_cpu_to_gpu would transcode it (NULL: not written);
 *   scale [N] f32: per_row = 0 gives the reference's tensor scale
 *     (sum|w| / (N*K)) / 0.7978845608 (1 when the sum is not > 0), summed
 *     left to right over the whole tensor on one lane, on every row;
 *     per_row != 0 takes each row as its own tensor.
 * Stream-ordered, no allocation. */
frx_status frx_prune_sparse24(frx_ctx *ctx, const void *w, frx_dtype wt, uint32_t N, uint32_t K,
                              int per_row, uint8_t *patterns, uint8_t *signs, uint32_t *meta,
                              float *scale);

/* Releases a buffer returned by frx_upload_ternary / frx_upload_stm. */
frx_status frx_free(frx_ctx *ctx, void *dev_ptr);

/* ---- host-side packers (no GPU) --------------------------------------------*/
/* pack_ternary (src/model/ternary.rs:146-163): out has (n+3)/4 bytes. */
frx_status frx_pack_ternary_u8(const int8_t *values, size_t n, uint8_t *out);
/* ternary_sparse_indices (src/model/ternary.rs:681-707) as CSR arrays:
 * values [N][K] i8; pos_off, neg_off [N + 1]; pos_idx, neg_idx receive the
 * column indices of +1 and -1 entries in column order. With pos_idx and
 * neg_idx NULL only the offsets are written (pos_off[N], neg_off[N] give
 * the list lengths to allocate). */
frx_status frx_ternary_sparse_indices(const int8_t *values, uint32_t N,
                                      uint32_t K, uint32_t *pos_off,
                                      uint32_t *pos_idx, uint32_t *neg_off,
                                      uint32_t *neg_idx);
/* unpack_ternary (src/model/ternary.rs:168-179). */
frx_status frx_unpack_ternary_u8(const uint8_t *packed, size_t n, int8_t *out);
/* pack_ternary_u32 (src/model/ternary.rs:1317-1328): n_values codes read from
 * ceil(n_values/4) bytes; out has ceil(n_values/16) words. */
frx_status frx_repack_u8_to_u32(const uint8_t *packed, size_t n_values,
                                uint32_t *out);
/* gpu_packed() (src/model/cpu_linear.rs:164-169, cpu_moe.rs:73-78): i8 [N][K]
 * -> u32 [N][K/16] plus per-row scales filled with the tensor scale. */
frx_status frx_gpu_packed(const int8_t *values, uint32_t N, uint32_t K,
                          float tensor_scale, uint32_t *w_out,
                          float *scales_out);
/* GPU 2:4 packer (src/compute/kernels/sparse_ternary.rs:254-318, test-only
 * in the reference): every group of 4 must hold exactly two nonzeros
 * (FRX_ERR_SHAPE otherwise). scales may be NULL; when given it receives the
 * reference's per-row absmean of the nonzeros. */
frx_status frx_pack_sparse24_gpu(const int8_t *w, uint32_t N, uint32_t K,
                                 uint32_t *meta, float *scales);
/* Bit-exact transcoder from the CPU SparseTernaryMatrix layout (pattern
 * nibbles + sign pairs, bit 1 = +1; src/model/sparse_ternary.rs:52-70) to the
 * GPU 5-bit layout (sign bit 1 = -1). Requires K % 4 == 0. Patterns 6 and 7
 * (never written by a packer) become pattern 0, as in to_ternary
 * (sparse_ternary.rs:172-176), so decoding either layout gives the same
 * matrix. */
frx_status frx_sparse24_cpu_to_gpu(const uint8_t *patterns,
                                   const uint8_t *signs, uint32_t N,
                                   uint32_t K, uint32_t *meta);

/* ---- host-slice accelerator API ------------------------------------------
 * Replaces GpuMatmulAccelerator (src/model/gpu_forward.rs:1146-1328): host
 * inputs, synchronous, host f32 output [seq][out_rows]. Device memory is
 * owned by the context and reused across calls. */
/* gpu_ternary_matmul (gpu_forward.rs:1154-1237): uploads weights per call. */
frx_status frx_gpu_ternary_matmul(frx_ctx *ctx, const uint32_t *packed_weights,
                                  const float *scales, const float *input,
                                  size_t seq_len, size_t in_cols,
                                  size_t out_rows, float *out);
/* gpu_ternary_matmul_vram (gpu_forward.rs:1245-1297): weights already on the
 * device (w_dev, s_dev device pointers); only the input is uploaded. */
frx_status frx_gpu_ternary_matmul_vram(frx_ctx *ctx, const uint32_t *w_dev,
                                       const float *s_dev, const float *input,
                                       size_t seq_len, size_t in_cols,
                                       size_t out_rows, float *out);
/* gpu_sparse_ternary_matmul (gpu_forward.rs:1299-1327; a zero-returning stub
 * in the reference): host 2:4 metadata in the GPU layout + per-row scales. */
frx_status frx_gpu_sparse_ternary_matmul(frx_ctx *ctx, const uint32_t *meta,
                                         const float *scales,
                                         const float *input, size_t seq_len,
                                         size_t in_cols, size_t out_rows,
                                         float *out);

#ifdef __cplusplus
}
#endif
#endif /* FRX_TERNARY_H */
