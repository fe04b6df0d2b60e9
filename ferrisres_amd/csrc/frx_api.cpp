// frx_api.cpp — C ABI of libfrx_ternary.so (declared in include/frx_ternary.h).
//
// Host-side mirror of the reference's ternary operator surface:
//  - frx_ternary_linear / frx_sparse24_ternary_linear = TernaryMatMulOp /
//    SparseTernaryMatMulOp::dispatch (device buffers, stream-ordered, no sync)
//  - frx_gpu_* = GpuMatmulAccelerator::gpu_*_matmul (host slices in, owned
//    host result out, synchronous; src/model/gpu_forward.rs:1146-1328)
//  - frx_moe_ternary_ffn = the model's GPU MoE glue.
//  - frx_ternary_ffn = the dense FFN branch of the model's decode step
//    (gate/up projections, activation, product, down projection).
// Every failure is returned as a status (FerrisResError mapping) with a
// message in the context; nothing aborts. There is no CPU fallback: a call
// either runs the HIP kernels or fails.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "../../include/frx_ternary.h"
#include "frx_internal.hpp"
#include "frx_policy.hpp"

// Device scratch of frx_ternary_ffn_noalloc: one array per GPU, held until
// the process ends. Its host-side name is only a handle: kernels and copies
// get the device address from hipGetSymbolAddress (noalloc_scratch_ptr).
// Every call on a GPU shares that GPU's array; calls that overlap on one GPU
// race on it.
static __device__ __align__(256) unsigned char
    frx_noalloc_scratch[FRX_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
void *g_noalloc_ptr[kMaxDevices];  // device address of frx_noalloc_scratch per device
hipError_t g_noalloc_err[kMaxDevices];
bool g_noalloc_done[kMaxDevices];

// Resolves the scratch array's device address on `device` once (that device
// current while it runs) and returns the cached result after that.
hipError_t noalloc_scratch_ptr(int device, void **out) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if (!g_noalloc_done[device]) {
    int prev = 0;
    hipError_t e = hipGetDevice(&prev);
    if (e == hipSuccess) e = hipSetDevice(device);
    void *p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(frx_noalloc_scratch));
    if (prev != device) (void)hipSetDevice(prev);
    g_noalloc_ptr[device] = e == hipSuccess ? p : nullptr;
    g_noalloc_err[device] = e;
    g_noalloc_done[device] = true;
  }
  *out = g_noalloc_ptr[device];
  return g_noalloc_err[device];
}
}  // namespace

struct frx_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  hipEvent_t handoff = nullptr;  // orders a new stream after the previous one (frx_set_stream)
  char err[512] = {0};
  // Workspaces replaced by larger ones stay allocated until frx_destroy: a
  // graph captured at a smaller size still holds their addresses.
  std::vector<void *> retired;
  size_t retired_bytes = 0;
  size_t live_bytes = 0;    // bytes of the current (not retired) context buffers
  uint32_t allocations = 0;  // device allocations made by this context
  void *noalloc = nullptr;  // device address of frx_noalloc_scratch on this device
  hipError_t noalloc_err = hipSuccess;
  // growable device scratch for the host-slice API and the MoE workspace
  void *scratch = nullptr;
  size_t scratch_bytes = 0;
  void *moe_ws = nullptr;
  size_t moe_ws_bytes = 0;
  void *ffn_ws = nullptr;  // dense FFN intermediate h (fp32)
  size_t ffn_ws_bytes = 0;
  void *glu_ws = nullptr;  // up projection of the GEMM-path GLU (fp32)
  size_t glu_ws_bytes = 0;
  void *blk_ws = nullptr;  // prescaled activations of the column-block linear (fp32)
  size_t blk_ws_bytes = 0;
  void *unit_ws = nullptr;  // unit row scales of the column-block linear
  size_t unit_ws_bytes = 0;
  void *stage_ws = nullptr;  // 16-byte aligned copies of unaligned x / scale / y
  size_t stage_ws_bytes = 0;
  void *sk_ws = nullptr;  // fp32 partial tiles of the split-K decode GEMV
  size_t sk_ws_bytes = 0;
  void *gk_ws = nullptr;  // fp32 K parts of the split-K GEMM
  size_t gk_ws_bytes = 0;
  void *xpl_ws = nullptr;  // f32 activations as bf16 hi | lo rows (GEMM above 16 tokens)
  size_t xpl_ws_bytes = 0;
  void *spp_ws = nullptr;  // 2:4 metadata in its prepared form (GEMM above a few tokens)
  size_t spp_ws_bytes = 0;
  unsigned *sk_cnt = nullptr;  // its per-row-tile arrival counters (zero between launches)
  int gemv_split = FRX_GEMV_SPLIT_AUTO;
  unsigned *ffn_bar = nullptr;  // grid-barrier words of the one-launch FFN
  int ffn_mode = FRX_FFN_AUTO;
  int moe_routing = FRX_MOE_TERNARY_MOE_LAYER;
  // MoE LoRA adapters: device table of 6 x 64 pointers (frx_set_moe_lora)
  const float **lora_tbl = nullptr;
  uint32_t lora_rank = 0, lora_experts = 0;
  float lora_scaling = 0.f;
  bool lora_on = false;
  void *router_ws = nullptr;  // [E][H] copy of a [H][E] router (CpuMoELayer routing)
  size_t router_ws_bytes = 0;
  int cus = 0;  // compute units of the device
  frx_status forced = FRX_OK;  // frx_force_status: returned by every compute / upload call
};

static frx_status fail(frx_ctx *ctx, frx_status st, const char *fmt, ...) {
  if (ctx) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(ctx->err, sizeof(ctx->err), fmt, ap);
    va_end(ap);
  }
  return st;
}

static frx_status hip_fail(frx_ctx *ctx, hipError_t e, const char *what) {
  const frx_status st = (e == hipErrorOutOfMemory) ? FRX_ERR_OOM : FRX_ERR_GPU;
  return fail(ctx, st, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

// Makes the context's device current for the calling thread; every entry
// point that takes a context starts here. work: a compute or upload call,
// which returns the status forced by frx_force_status instead (before
// reading any argument or touching the device).
static frx_status enter(frx_ctx *ctx, bool work = true) {
  if (!ctx) return FRX_ERR_DEVICE;
  ctx->err[0] = 0;
  if (work && ctx->forced != FRX_OK)
    return fail(ctx, ctx->forced, "status %d forced by frx_force_status", (int)ctx->forced);
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return fail(ctx, FRX_ERR_DEVICE, "hipSetDevice(%d): %s", ctx->device, hipGetErrorString(e));
  return FRX_OK;
}

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

static size_t a256(size_t v) { return (v + 255) & ~(size_t)255; }

extern "C" {

const char *frx_version(void) { return "frx_ternary 0.1.0 gfx950"; }

const char *frx_status_string(frx_status s) {
  switch (s) {
    case FRX_OK: return "ok";
    case FRX_ERR_GPU: return "GPU error";
    case FRX_ERR_SHAPE: return "shape error";
    case FRX_ERR_DEVICE: return "device error";
    case FRX_ERR_SHADER: return "kernel error";
    case FRX_ERR_OOM: return "out of memory";
    case FRX_ERR_UNSUPPORTED: return "unsupported";
  }
  return "unknown status";
}

frx_status frx_create(int device, frx_ctx **out) {
  if (!out) return FRX_ERR_DEVICE;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return FRX_ERR_DEVICE;
  if (device < 0 || device >= n) return FRX_ERR_DEVICE;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return FRX_ERR_DEVICE;
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return FRX_ERR_UNSUPPORTED;
  frx_ctx *c = new frx_ctx();
  c->device = device;
  c->cus = prop.multiProcessorCount;
  c->noalloc_err = noalloc_scratch_ptr(device, &c->noalloc);
  *out = c;
  return FRX_OK;
}

void frx_destroy(frx_ctx *ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  // the buffers below may still be read by work enqueued on the context's
  // stream (which frx_set_stream ordered after any earlier stream's)
  (void)hipStreamSynchronize(ctx->stream);
  if (ctx->handoff) (void)hipEventDestroy(ctx->handoff);
  if (ctx->scratch) (void)hipFree(ctx->scratch);
  if (ctx->moe_ws) (void)hipFree(ctx->moe_ws);
  if (ctx->lora_tbl) (void)hipFree(ctx->lora_tbl);
  if (ctx->ffn_ws) (void)hipFree(ctx->ffn_ws);
  if (ctx->glu_ws) (void)hipFree(ctx->glu_ws);
  if (ctx->blk_ws) (void)hipFree(ctx->blk_ws);
  if (ctx->router_ws) (void)hipFree(ctx->router_ws);
  if (ctx->unit_ws) (void)hipFree(ctx->unit_ws);
  if (ctx->stage_ws) (void)hipFree(ctx->stage_ws);
  if (ctx->sk_ws) (void)hipFree(ctx->sk_ws);
  if (ctx->gk_ws) (void)hipFree(ctx->gk_ws);
  if (ctx->xpl_ws) (void)hipFree(ctx->xpl_ws);
  if (ctx->spp_ws) (void)hipFree(ctx->spp_ws);
  if (ctx->sk_cnt) (void)hipFree(ctx->sk_cnt);
  if (ctx->ffn_bar) (void)hipFree(ctx->ffn_bar);
  for (void *p : ctx->retired) (void)hipFree(p);
  delete ctx;
}

frx_status frx_set_stream(frx_ctx *ctx, void *hip_stream) {
  if (!ctx) return FRX_ERR_DEVICE;
  const hipStream_t next = reinterpret_cast<hipStream_t>(hip_stream);
  if (next == ctx->stream) return FRX_OK;
  // The context's workspaces serve one stream at a time: the new stream
  // waits (on the device, without blocking the host) for the work already
  // enqueued on the previous one. Streams under graph capture are left as
  // they are (an event would join the capture).
  hipStreamCaptureStatus a = hipStreamCaptureStatusNone, b = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(ctx->stream, &a);
  if (e == hipSuccess) e = hipStreamIsCapturing(next, &b);
  if (e == hipSuccess && a == hipStreamCaptureStatusNone && b == hipStreamCaptureStatusNone) {
    if (!ctx->handoff) e = hipEventCreateWithFlags(&ctx->handoff, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(ctx->handoff, ctx->stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(next, ctx->handoff, 0);
  }
  if (e != hipSuccess) return hip_fail(ctx, e, "stream hand-off");
  ctx->stream = next;
  return FRX_OK;
}

frx_status frx_synchronize(frx_ctx *ctx) {
  frx_status st = enter(ctx, false);
  if (st != FRX_OK) return st;
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
  if (ctx->ffn_bar) {
    // A one-launch FFN whose grid barrier timed out (its workgroups were not
    // all resident at once) raised the error word: report it and reset the
    // barrier words for the next launch.
    unsigned err = 0;
    e = hipMemcpy(&err, ctx->ffn_bar + frx::ffn1_error_word(), sizeof(err), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(ctx, e, "FFN barrier state read");
    if (err) {
      // reset on the context's stream and wait for it, so that the next
      // one-launch FFN on this stream sees the cleared words
      e = hipMemsetAsync(ctx->ffn_bar, 0, frx::ffn1_barrier_bytes(), ctx->stream);
      if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
      if (e != hipSuccess) return hip_fail(ctx, e, "FFN barrier reset");
      return fail(ctx, FRX_ERR_GPU,
                  "one-launch FFN: grid barrier timed out (workgroups not co-resident); "
                  "outputs of FFN calls since the last synchronize are invalid");
    }
  }
  return FRX_OK;
}

frx_status frx_set_ffn_mode(frx_ctx *ctx, frx_ffn_mode mode) {
  if (!ctx) return FRX_ERR_DEVICE;
  ctx->err[0] = 0;
  if (mode != FRX_FFN_AUTO && mode != FRX_FFN_ONE_LAUNCH && mode != FRX_FFN_TWO_LAUNCH)
    return fail(ctx, FRX_ERR_UNSUPPORTED, "unknown FFN mode %d", (int)mode);
  ctx->ffn_mode = mode;
  return FRX_OK;
}

frx_status frx_set_gemv_split(frx_ctx *ctx, frx_gemv_split mode) {
  if (!ctx) return FRX_ERR_DEVICE;
  ctx->err[0] = 0;
  if (mode != FRX_GEMV_SPLIT_AUTO && mode != FRX_GEMV_SPLIT_ALWAYS && mode != FRX_GEMV_SPLIT_NEVER)
    return fail(ctx, FRX_ERR_UNSUPPORTED, "unknown split mode %d", (int)mode);
  ctx->gemv_split = mode;
  return FRX_OK;
}

frx_status frx_set_moe_routing(frx_ctx *ctx, frx_moe_routing routing) {
  if (!ctx) return FRX_ERR_DEVICE;
  ctx->err[0] = 0;
  if (routing != FRX_MOE_TERNARY_MOE_LAYER && routing != FRX_MOE_CPU_MOE_LAYER)
    return fail(ctx, FRX_ERR_UNSUPPORTED, "unknown MoE routing %d", (int)routing);
  ctx->moe_routing = routing;
  return FRX_OK;
}

frx_status frx_set_moe_lora(frx_ctx *ctx, const frx_moe_lora *lora, uint32_t experts) {
  if (!ctx) return FRX_ERR_DEVICE;
  ctx->err[0] = 0;
  if (!lora) {
    ctx->lora_on = false;
    return FRX_OK;
  }
  if (lora->rank == 0 || lora->rank > (uint32_t)frx::MOE_LORA_MAXR)
    return fail(ctx, FRX_ERR_SHAPE, "LoRA rank=%u must be in [1, %d]", lora->rank, frx::MOE_LORA_MAXR);
  if (experts == 0 || experts > 64) return fail(ctx, FRX_ERR_SHAPE, "LoRA experts=%u must be in [1, 64]", experts);
  const float *host[6 * 64] = {nullptr};
  const float *const *src[6] = {lora->a_gate, lora->b_gate, lora->a_up, lora->b_up, lora->a_down, lora->b_down};
  for (int k = 0; k < 6; k++)
    for (uint32_t e = 0; e < experts && src[k]; e++) host[k * 64 + e] = src[k][e];
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "LoRA setup");
  // Every call gets a table of its own: launches already enqueued, and
  // graphs captured with the previous adapters, keep reading the previous
  // table (retired like a replaced workspace) with the rank they were
  // launched with, so no launch sees a table and a rank that do not match.
  const float **tbl = nullptr;
  e = hipMalloc(reinterpret_cast<void **>(&tbl), sizeof(host));
  if (e != hipSuccess) return hip_fail(ctx, e, "LoRA table allocation");
  ctx->allocations++;
  if ((e = hipMemcpy(tbl, host, sizeof(host), hipMemcpyHostToDevice)) != hipSuccess) {
    (void)hipFree(tbl);
    return hip_fail(ctx, e, "LoRA table copy");
  }
  if (ctx->lora_tbl) {
    ctx->retired.push_back(ctx->lora_tbl);
    ctx->retired_bytes += sizeof(host);
  } else {
    ctx->live_bytes += sizeof(host);
  }
  ctx->lora_tbl = tbl;
  ctx->lora_rank = lora->rank;
  ctx->lora_scaling = lora->scaling;
  ctx->lora_experts = experts;
  ctx->lora_on = true;
  return FRX_OK;
}

frx_status frx_force_status(frx_ctx *ctx, frx_status status) {
  if (!ctx) return FRX_ERR_DEVICE;
  ctx->err[0] = 0;
  if ((int)status < (int)FRX_OK || (int)status > (int)FRX_ERR_UNSUPPORTED)
    return fail(ctx, FRX_ERR_UNSUPPORTED, "unknown status %d", (int)status);
  ctx->forced = status;
  return FRX_OK;
}

const char *frx_last_error(const frx_ctx *ctx) { return ctx ? ctx->err : ""; }

static frx_status check_linear(frx_ctx *ctx, const void *w, const void *scale,
                               const void *x, frx_dtype xt, const void *y,
                               frx_dtype yt, uint32_t M, uint32_t K,
                               uint32_t N, bool sparse) {
  if (!w || !scale || !x || !y) return fail(ctx, FRX_ERR_SHAPE, "null buffer pointer");
  if (M == 0 || K == 0 || N == 0) return fail(ctx, FRX_ERR_SHAPE, "empty shape M=%u K=%u N=%u", M, K, N);
  if (!sparse && K % 16 != 0)
    return fail(ctx, FRX_ERR_SHAPE, "in_cols=%u must be a multiple of 16 for the row-aligned u32 layout", K);
  if (sparse && K % 4 != 0) return fail(ctx, FRX_ERR_SHAPE, "in_cols=%u must be a multiple of 4 for 2:4", K);
  if ((xt != FRX_F32 && xt != FRX_BF16) || (yt != FRX_F32 && yt != FRX_BF16))
    return fail(ctx, FRX_ERR_UNSUPPORTED, "dtype must be FRX_F32 or FRX_BF16");
  const uintptr_t xa = xt == FRX_BF16 ? 1 : 3, ya = yt == FRX_BF16 ? 1 : 3;
  if ((reinterpret_cast<uintptr_t>(x) & xa) || (reinterpret_cast<uintptr_t>(y) & ya) ||
      (reinterpret_cast<uintptr_t>(scale) & 3) || (reinterpret_cast<uintptr_t>(w) & 3))
    return fail(ctx, FRX_ERR_SHAPE, "x, y, scale and weights must be aligned to their element size");
  if ((size_t)M * K > (size_t)0x7FFFFFFF || (size_t)M * N > (size_t)0x7FFFFFFF)
    return fail(ctx, FRX_ERR_SHAPE, "M*K or M*N exceeds 2^31 elements");
  // the kernels address the weights through 32-bit buffer ranges
  const size_t wbytes = sparse ? (size_t)N * (((size_t)K / 4 + 5) / 6) * 4 : (size_t)N * K / 4;
  if (wbytes > (size_t)0xFFFFFFF0u)
    return fail(ctx, FRX_ERR_SHAPE, "weight matrix of %zu bytes exceeds 4 GiB (N=%u K=%u)", wbytes, N, K);
  return FRX_OK;
}

static frx_status ensure_buffer(frx_ctx *ctx, void **buf, size_t *have, size_t need, const char *what);

// x, scale and y as the kernels take them: 16-byte aligned. A caller's sub-
// slice at another offset is copied into the context's staging workspace
// (x and scale before the launch, y back after it), on the context stream.
struct Staged {
  const void *x;
  const float *scale;
  void *y;
  void *y_user = nullptr;
  size_t y_bytes = 0;
};

static frx_status stage_linear(frx_ctx *ctx, const void *x, frx_dtype xt, const float *scale, void *y,
                               frx_dtype yt, uint32_t M, uint32_t K, uint32_t N, Staged *out) {
  out->x = x;
  out->scale = scale;
  out->y = y;
  const bool sx = !aligned16(x), ss = !aligned16(scale), sy = !aligned16(y);
  if (!sx && !ss && !sy) return FRX_OK;
  const size_t xb = (size_t)M * K * (xt == FRX_BF16 ? 2 : 4), sb = (size_t)N * 4;
  const size_t yb = (size_t)M * N * (yt == FRX_BF16 ? 2 : 4);
  const size_t need = (sx ? a256(xb) : 0) + (ss ? a256(sb) : 0) + (sy ? a256(yb) : 0);
  frx_status st = ensure_buffer(ctx, &ctx->stage_ws, &ctx->stage_ws_bytes, need, "staging workspace allocation");
  if (st != FRX_OK) return st;
  char *base = reinterpret_cast<char *>(ctx->stage_ws);
  hipError_t e = hipSuccess;
  if (sx) {
    e = hipMemcpyAsync(base, x, xb, hipMemcpyDeviceToDevice, ctx->stream);
    out->x = base;
    base += a256(xb);
  }
  if (ss && e == hipSuccess) {
    e = hipMemcpyAsync(base, scale, sb, hipMemcpyDeviceToDevice, ctx->stream);
    out->scale = reinterpret_cast<const float *>(base);
    base += a256(sb);
  }
  if (sy) {
    out->y = base;
    out->y_user = y;
    out->y_bytes = yb;
  }
  if (e != hipSuccess) return hip_fail(ctx, e, "staging copy");
  return FRX_OK;
}

static hipError_t unstage_linear(frx_ctx *ctx, const Staged &sg) {
  if (!sg.y_user) return hipSuccess;
  return hipMemcpyAsync(sg.y_user, sg.y, sg.y_bytes, hipMemcpyDeviceToDevice, ctx->stream);
}

// Split-K decode GEMV (frx_gemv_sk.hip): chosen where it measured faster
// than the whole-K kernels (below); the f32 stream each compute unit pulls
// through L1 bounds those (4096x11008, 2 / 4 / 8 / 16 tokens: 11.2 / 11.8 /
// 13.8 / 17.8 us whole-K against 9.9 / 10.0 / 10.3 / 11.8 us split).
// frx_set_gemv_split forces either.
static bool use_split(const frx_ctx *ctx, const uint32_t *w, const void *x, uint32_t M, uint32_t K, uint32_t N,
                      frx_dtype xt) {
  // one f32 token that the balanced kernel does not take (past its 16384
  // columns, or more rows than its slots): the 16-row tiles that would run
  // instead stream all of x per tile (8192 x 28672: 40.7 -> 26.5 us split)
  if (M == 1 && xt == FRX_F32 && ctx->gemv_split != FRX_GEMV_SPLIT_NEVER &&
      !frx::gemv_bal_fits(w, x, 1, (int)K, (int)N) && (size_t)K * 4 < ((size_t)1 << 32) &&
      (N + 127) / 128 <= (uint32_t)frx::GEMV_SK_MAX_TILES)
    return true;
  if (M < 2 || M > 16 || ctx->gemv_split == FRX_GEMV_SPLIT_NEVER) return false;
  if ((size_t)M * K * 4 >= ((size_t)1 << 32) || (N + 127) / 128 > (uint32_t)frx::GEMV_SK_MAX_TILES) return false;
  if (ctx->gemv_split == FRX_GEMV_SPLIT_ALWAYS) return true;
  // where it measured faster: f32 x above 4096 columns (every whole-K tile
  // streams all of x: 13824 x 5120, B = 16: 23.0 -> 15.4 us; at 4096 the
  // whole-K kernels stay ahead); bf16 x from 5 tokens at 14336 columns and from 3
  // tokens above 16384 (8192 x 28672, B = 16: 38.1 -> 26.8 us), with enough
  // 128-row tiles to fill the grid (at N = 2048 the slices get too thin)
  if (xt == FRX_F32) return K > 4096;
  return N >= 3072 && ((M >= 5 && K >= 14336) || (M >= 3 && K > 16384));
}

// The split-K GEMV's tile counters: allocated and zeroed once per context
// (the first split-K call, not under graph capture); every launch leaves
// them zero.
static frx_status ensure_sk_counters(frx_ctx *ctx) {
  if (ctx->sk_cnt) return FRX_OK;
  void *p = nullptr;
  const size_t bytes = (size_t)frx::GEMV_SK_MAX_TILES * 4;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) return hip_fail(ctx, e, "split-K counter allocation");
  e = hipMemset(p, 0, bytes);
  // the legacy stream of hipMemset does not order against a non-blocking
  // caller stream: wait for it here (first use only)
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    (void)hipFree(p);
    return hip_fail(ctx, e, "split-K counter initialisation");
  }
  ctx->allocations++;
  ctx->live_bytes += bytes;
  ctx->sk_cnt = reinterpret_cast<unsigned *>(p);
  return FRX_OK;
}

// y = x W^T * scale (+ bias) for x2 = [M][2K] bf16 hi | lo rows (an fp32
// activation), M > 16: K split over workgroups where the tiles leave compute
// units idle (and the call may allocate), else one pass over both halves.
static frx_status gemm_planes_auto(frx_ctx *ctx, const uint32_t *w, const float *scale, const float *bias,
                                   const uint16_t *x2, void *y, frx_dtype yt, uint32_t M, uint32_t K, uint32_t N,
                                   bool may_alloc) {
  frx_status st;
  hipError_t e;
  int S = 0, kp = 0;
  if (may_alloc && ctx->gemv_split != FRX_GEMV_SPLIT_NEVER &&
      frx::gemm_splitk_plan((int)M, (int)K, (int)N, ctx->cus, &S, &kp, 2)) {
    if ((st = ensure_buffer(ctx, &ctx->gk_ws, &ctx->gk_ws_bytes, frx::gemm_splitk_workspace_bytes((int)M, (int)N, S),
                            "split-K GEMM workspace allocation")) != FRX_OK)
      return st;
    e = frx::launch_gemm_splitk(w, scale, x2, y, yt == FRX_BF16, (int)M, (int)K, (int)N, S, kp,
                                reinterpret_cast<float *>(ctx->gk_ws), ctx->stream, bias, 2);
  } else {
    e = frx::launch_gemm_planes(w, scale, x2, y, yt == FRX_BF16, (int)M, (int)K, (int)N, ctx->stream, bias);
  }
  if (e != hipSuccess) return hip_fail(ctx, e, "ternary_linear launch");
  return FRX_OK;
}

// y = x W^T * scale (+ bias) on aligned operands: the split-K GEMV where
// use_split picks it (allocating its workspace on first use), else the
// decode GEMVs up to 16 tokens and the GEMM above.
static frx_status gemv_auto(frx_ctx *ctx, const uint32_t *w, const float *scale, const float *bias, const void *x,
                            frx_dtype xt, void *y, frx_dtype yt, uint32_t M, uint32_t K, uint32_t N) {
  frx_status st;
  hipError_t e;
  if (use_split(ctx, w, x, M, K, N, xt)) {
    if ((st = ensure_buffer(ctx, &ctx->sk_ws, &ctx->sk_ws_bytes,
                            frx::gemv_sk_workspace_bytes((int)K, (int)N, ctx->cus),
                            "split-K workspace allocation")) != FRX_OK)
      return st;
    if ((st = ensure_sk_counters(ctx)) != FRX_OK) return st;
    e = frx::launch_gemv_sk(w, scale, x, nullptr, xt == FRX_BF16 ? 0 : 1, y, yt == FRX_BF16, (int)M, (int)K, (int)N,
                            reinterpret_cast<float *>(ctx->sk_ws), ctx->sk_cnt, bias, ctx->cus, ctx->stream);
  } else if (M <= 16) {
    e = frx::launch_gemv(w, scale, x, xt == FRX_BF16, y, yt == FRX_BF16, (int)M, (int)K, (int)N, ctx->stream, bias);
  } else if (xt == FRX_F32 && K % 64 == 0 && aligned16(w) && aligned16(x) && (size_t)M * K * 4 < ((size_t)1 << 31)) {
    // f32 activations, 17 tokens and more: split once into bf16 hi | lo rows
    // (the same bytes), then the bf16 engine over both halves
    if ((st = ensure_buffer(ctx, &ctx->xpl_ws, &ctx->xpl_ws_bytes, a256((size_t)M * K * 4),
                            "activation planes workspace allocation")) != FRX_OK)
      return st;
    uint16_t *x2 = reinterpret_cast<uint16_t *>(ctx->xpl_ws);
    e = frx::launch_to_planes(reinterpret_cast<const float *>(x), x2, (int)M, (int)K, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "activation planes launch");
    return gemm_planes_auto(ctx, w, scale, bias, x2, y, yt, M, K, N, true);
  } else {
    int S = 0, kp = 0;
    if (ctx->gemv_split != FRX_GEMV_SPLIT_NEVER && xt == FRX_BF16 && aligned16(w) && aligned16(x) &&
        (size_t)M * K * 2 < ((size_t)1 << 31) && frx::gemm_splitk_plan((int)M, (int)K, (int)N, ctx->cus, &S, &kp)) {
      // 17 to a few hundred tokens: K split over workgroups so that the
      // grid covers the compute units
      if ((st = ensure_buffer(ctx, &ctx->gk_ws, &ctx->gk_ws_bytes, frx::gemm_splitk_workspace_bytes((int)M, (int)N, S),
                              "split-K GEMM workspace allocation")) != FRX_OK)
        return st;
      e = frx::launch_gemm_splitk(w, scale, x, y, yt == FRX_BF16, (int)M, (int)K, (int)N, S, kp,
                                  reinterpret_cast<float *>(ctx->gk_ws), ctx->stream, bias);
    } else {
      e = frx::launch_gemm(w, scale, x, xt == FRX_BF16, y, yt == FRX_BF16, (int)M, (int)K, (int)N, 0, ctx->stream,
                           bias);
    }
  }
  if (e != hipSuccess) return hip_fail(ctx, e, "ternary_linear launch");
  return FRX_OK;
}

static frx_status ternary_linear_run(frx_ctx *ctx, const uint32_t *w, const float *scale, const float *bias,
                                     const void *x, frx_dtype xt, void *y, frx_dtype yt, uint32_t M, uint32_t K,
                                     uint32_t N) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if ((st = check_linear(ctx, w, scale, x, xt, y, yt, M, K, N, false)) != FRX_OK) return st;
  Staged sg;
  if ((st = stage_linear(ctx, x, xt, scale, y, yt, M, K, N, &sg)) != FRX_OK) return st;
  if ((st = gemv_auto(ctx, w, sg.scale, bias, sg.x, xt, sg.y, yt, M, K, N)) != FRX_OK) return st;
  const hipError_t e = unstage_linear(ctx, sg);
  if (e != hipSuccess) return hip_fail(ctx, e, "ternary_linear launch");
  return FRX_OK;
}

frx_status frx_ternary_linear(frx_ctx *ctx, const uint32_t *w,
                              const float *scale, const void *x, frx_dtype xt,
                              void *y, frx_dtype yt, uint32_t M, uint32_t K,
                              uint32_t N) {
  return ternary_linear_run(ctx, w, scale, nullptr, x, xt, y, yt, M, K, N);
}

frx_status frx_ternary_linear_bias(frx_ctx *ctx, const uint32_t *w, const float *scale, const float *bias,
                                   const void *x, frx_dtype xt, void *y, frx_dtype yt, uint32_t M, uint32_t K,
                                   uint32_t N) {
  return ternary_linear_run(ctx, w, scale, bias, x, xt, y, yt, M, K, N);
}

frx_status frx_ternary_linear_group(frx_ctx *ctx, const void *x, frx_dtype xt, uint32_t M, uint32_t K,
                                    uint32_t count, const uint32_t *const *w, const float *const *scale,
                                    const uint32_t *N, void *const *y, frx_dtype yt) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if (!w || !scale || !N || !y) return fail(ctx, FRX_ERR_SHAPE, "null pointer array");
  if (count == 0 || count > (uint32_t)frx::GEMV_GROUP_MAX)
    return fail(ctx, FRX_ERR_SHAPE, "count=%u must be in [1, %d]", count, frx::GEMV_GROUP_MAX);
  bool aligned = aligned16(x);
  size_t rows = 0;
  for (uint32_t i = 0; i < count; i++) {
    if ((st = check_linear(ctx, w[i], scale[i], x, xt, y[i], yt, M, K, N[i], false)) != FRX_OK) return st;
    aligned = aligned && aligned16(scale[i]) && aligned16(y[i]);
    rows += N[i];
  }
  if (rows > (size_t)0x7FFFFFFF) return fail(ctx, FRX_ERR_SHAPE, "too many rows in the group");
  hipError_t e = hipSuccess;
  int n[frx::GEMV_GROUP_MAX];
  for (uint32_t i = 0; i < count; i++) n[i] = (int)N[i];
  if (M == 1 && aligned && frx::gemv_group_fits(x, 1, (int)K, (int)count, w, n)) {
    e = frx::launch_gemv_group(x, xt == FRX_BF16, yt == FRX_BF16, (int)M, (int)K, (int)count, w, scale, y, n,
                               ctx->stream);
  } else {
    // several tokens, prefill, shapes past the one-launch group, or
    // sub-slices that need staging: one linear per matrix
    for (uint32_t i = 0; i < count; i++)
      if ((st = ternary_linear_run(ctx, w[i], scale[i], nullptr, x, xt, y[i], yt, M, K, N[i])) != FRX_OK) return st;
  }
  if (e != hipSuccess) return hip_fail(ctx, e, "ternary_linear_group launch");
  return FRX_OK;
}

// Token count from which a 2:4 linear decodes its metadata once into the
// prepared form (one pass over the matrix, 10.6 us at 11008 x 4096) before
// the GEMM: at 512 tokens and more the cheaper operand decode repays it
// (4096 x 11008 at 2048 tokens: 160 -> 145 us; at 256 tokens it is even).
constexpr uint32_t SP24_PREP_MIN_TOKENS = 512;

frx_status frx_sparse24_ternary_linear(frx_ctx *ctx, const uint32_t *meta,
                                       const float *scale, const void *x,
                                       frx_dtype xt, void *y, frx_dtype yt,
                                       uint32_t M, uint32_t K, uint32_t N) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if ((st = check_linear(ctx, meta, scale, x, xt, y, yt, M, K, N, true)) != FRX_OK) return st;
  Staged sg;
  if ((st = stage_linear(ctx, x, xt, scale, y, yt, M, K, N, &sg)) != FRX_OK) return st;
  hipError_t e = hipSuccess;
  int S = 0, sp = 0;
  if (frx::sp24_gemv_plan((int)M, (int)K, (int)N, xt == FRX_BF16, &S)) {
    // decode: the metadata read once by a table-driven GEMV
    if ((st = ensure_buffer(ctx, &ctx->gk_ws, &ctx->gk_ws_bytes, frx::gemm_splitk_workspace_bytes((int)M, (int)N, S),
                            "split-K GEMM workspace allocation")) != FRX_OK)
      return st;
    if ((st = ensure_sk_counters(ctx)) != FRX_OK) return st;
    e = frx::launch_sp24_gemv(meta, sg.scale, sg.x, xt == FRX_BF16, sg.y, yt == FRX_BF16, (int)M, (int)K, (int)N, S,
                              reinterpret_cast<float *>(ctx->gk_ws), ctx->sk_cnt, ctx->stream);
    if (e == hipSuccess) e = unstage_linear(ctx, sg);
    if (e != hipSuccess) return hip_fail(ctx, e, "sparse24_ternary_linear launch");
    return FRX_OK;
  }
  // f32 x runs as bf16 hi | lo rows ([M][2K], |x - hi - lo| <= 2^-17 |x|)
  // through the same sparse engine, both halves against the same weights
  const bool planes = xt == FRX_F32 && aligned16(sg.x) && K % 64 == 0 && (size_t)M * K * 4 < ((size_t)1 << 31);
  const bool engine =
      planes || (xt == FRX_BF16 && aligned16(sg.x) && K % 64 == 0 && (size_t)M * K * 2 < ((size_t)1 << 31));
  const int halves = planes ? 2 : 1;
  const bool split = engine && ctx->gemv_split != FRX_GEMV_SPLIT_NEVER &&
                     frx::gemm_sp_splitk_plan((int)M, (int)K, (int)N, ctx->cus, &S, &sp, halves);
  const uint32_t *wm = meta;
  const void *xin = sg.x;
  int prepared = 0;
  if (planes) {
    if ((st = ensure_buffer(ctx, &ctx->xpl_ws, &ctx->xpl_ws_bytes, a256((size_t)M * K * 4),
                            "activation planes allocation")) != FRX_OK)
      return st;
    e = frx::launch_to_planes(reinterpret_cast<const float *>(sg.x), reinterpret_cast<uint16_t *>(ctx->xpl_ws),
                              (int)M, (int)K, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "sparse24_ternary_linear planes");
    xin = ctx->xpl_ws;
  }
  if (engine && M >= SP24_PREP_MIN_TOKENS) {
    // the metadata decoded once into its prepared form for every token tile
    if ((st = ensure_buffer(ctx, &ctx->spp_ws, &ctx->spp_ws_bytes, (size_t)N * K / 4,
                            "2:4 prepared metadata allocation")) != FRX_OK)
      return st;
    e = frx::launch_sp24_prepare(meta, reinterpret_cast<uint32_t *>(ctx->spp_ws), (int)N, (int)K, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "sparse24_ternary_linear prepare");
    wm = reinterpret_cast<const uint32_t *>(ctx->spp_ws);
    prepared = 1;
  }
  if (split) {
    // decode and small prefill: K split over workgroups on the sparse pipe
    if ((st = ensure_buffer(ctx, &ctx->gk_ws, &ctx->gk_ws_bytes, frx::gemm_splitk_workspace_bytes((int)M, (int)N, S),
                            "split-K GEMM workspace allocation")) != FRX_OK)
      return st;
    e = frx::launch_gemm_sp_splitk(wm, sg.scale, xin, sg.y, yt == FRX_BF16, (int)M, (int)K, (int)N, S, sp,
                                   reinterpret_cast<float *>(ctx->gk_ws), ctx->stream, nullptr, prepared, halves);
  } else if (planes) {
    e = frx::launch_gemm_sp_planes(wm, prepared, sg.scale, reinterpret_cast<const uint16_t *>(xin), sg.y,
                                   yt == FRX_BF16, (int)M, (int)K, (int)N, ctx->stream);
  } else if (prepared) {
    e = frx::launch_gemm_sp_prepared(wm, sg.scale, sg.x, sg.y, yt == FRX_BF16, (int)M, (int)K, (int)N, ctx->stream,
                                     nullptr);
  } else {
    e = frx::launch_gemm(meta, sg.scale, sg.x, xt == FRX_BF16, sg.y, yt == FRX_BF16, (int)M, (int)K, (int)N, 1,
                         ctx->stream);
  }
  if (e == hipSuccess) e = unstage_linear(ctx, sg);
  if (e != hipSuccess) return hip_fail(ctx, e, "sparse24_ternary_linear launch");
  return FRX_OK;
}

frx_status frx_sparse24_prepare(frx_ctx *ctx, const uint32_t *meta, uint32_t K, uint32_t N, uint32_t *prepared) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if (!meta || !prepared) return fail(ctx, FRX_ERR_SHAPE, "null buffer pointer");
  if (K == 0 || N == 0 || K % 64 != 0)
    return fail(ctx, FRX_ERR_SHAPE, "prepared 2:4 form needs K a positive multiple of 64 (K=%u N=%u)", K, N);
  if ((reinterpret_cast<uintptr_t>(meta) & 3) || !aligned16(prepared))
    return fail(ctx, FRX_ERR_SHAPE, "meta must be 4-byte and prepared 16-byte aligned");
  if ((size_t)N * K / 4 > (size_t)0xFFFFFFF0u)
    return fail(ctx, FRX_ERR_SHAPE, "prepared matrix of %zu bytes exceeds 4 GiB", (size_t)N * K / 4);
  const hipError_t e = frx::launch_sp24_prepare(meta, prepared, (int)N, (int)K, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "sparse24_prepare launch");
  return FRX_OK;
}

frx_status frx_sparse24_prepared_linear(frx_ctx *ctx, const uint32_t *prepared, const float *scale, const void *x,
                                        frx_dtype xt, void *y, frx_dtype yt, uint32_t M, uint32_t K, uint32_t N) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if ((st = check_linear(ctx, prepared, scale, x, xt, y, yt, M, K, N, false)) != FRX_OK) return st;
  if (K % 64 != 0) return fail(ctx, FRX_ERR_SHAPE, "prepared 2:4 form needs K a multiple of 64 (K=%u)", K);
  if (xt != FRX_BF16) return fail(ctx, FRX_ERR_UNSUPPORTED, "the prepared 2:4 linear takes bf16 activations");
  if (!aligned16(prepared)) return fail(ctx, FRX_ERR_SHAPE, "prepared must be 16-byte aligned");
  if ((size_t)M * K * 2 >= ((size_t)1 << 31))
    return fail(ctx, FRX_ERR_UNSUPPORTED, "x of %zu bytes exceeds 2 GiB", (size_t)M * K * 2);
  Staged sg;
  if ((st = stage_linear(ctx, x, xt, scale, y, yt, M, K, N, &sg)) != FRX_OK) return st;
  hipError_t e;
  int S = 0, sp = 0;
  if (ctx->gemv_split != FRX_GEMV_SPLIT_NEVER && frx::gemm_sp_splitk_plan((int)M, (int)K, (int)N, ctx->cus, &S, &sp)) {
    if ((st = ensure_buffer(ctx, &ctx->gk_ws, &ctx->gk_ws_bytes, frx::gemm_splitk_workspace_bytes((int)M, (int)N, S),
                            "split-K GEMM workspace allocation")) != FRX_OK)
      return st;
    e = frx::launch_gemm_sp_splitk(prepared, sg.scale, sg.x, sg.y, yt == FRX_BF16, (int)M, (int)K, (int)N, S, sp,
                                   reinterpret_cast<float *>(ctx->gk_ws), ctx->stream, nullptr, 1);
  } else {
    e = frx::launch_gemm_sp_prepared(prepared, sg.scale, sg.x, sg.y, yt == FRX_BF16, (int)M, (int)K, (int)N,
                                     ctx->stream, nullptr);
  }
  if (e == hipSuccess) e = unstage_linear(ctx, sg);
  if (e != hipSuccess) return hip_fail(ctx, e, "sparse24_prepared_linear launch");
  return FRX_OK;
}

// Grows a context-owned device buffer. The buffer it replaces is retired,
// not freed: a graph captured at a smaller size still writes to it, so it
// stays allocated until frx_release_retired or frx_destroy. Sizes grow
// geometrically (frx::grow_bytes: at least 1.5x the old size), so rising
// requests make O(log) allocations and the retired buffers of one workspace
// total less than twice its current size. The first call at a larger size
// allocates and must not be under graph capture.
static frx_status ensure_buffer(frx_ctx *ctx, void **buf, size_t *have, size_t need, const char *what) {
  if (need <= *have) return FRX_OK;
  const size_t bytes = frx::grow_bytes(*have, need);
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e == hipErrorOutOfMemory && bytes > a256(need)) {
    (void)hipGetLastError();  // the geometric size did not fit: take what was asked
    e = hipMalloc(&p, a256(need));
    if (e == hipSuccess) {
      ctx->allocations++;
      if (*buf) {
        ctx->retired.push_back(*buf);
        ctx->retired_bytes += *have;
        ctx->live_bytes -= *have;
      }
      *buf = p;
      *have = a256(need);
      ctx->live_bytes += *have;
      return FRX_OK;
    }
  }
  if (e != hipSuccess) return hip_fail(ctx, e, what);
  ctx->allocations++;
  if (*buf) {
    ctx->retired.push_back(*buf);
    ctx->retired_bytes += *have;
    ctx->live_bytes -= *have;
  }
  *buf = p;
  *have = bytes;
  ctx->live_bytes += bytes;
  return FRX_OK;
}

frx_status frx_workspace_stats(frx_ctx *ctx, size_t *live_bytes, size_t *retired_bytes, uint32_t *allocations) {
  if (!ctx) return FRX_ERR_DEVICE;
  ctx->err[0] = 0;
  if (live_bytes) *live_bytes = ctx->live_bytes;
  if (retired_bytes) *retired_bytes = ctx->retired_bytes;
  if (allocations) *allocations = ctx->allocations;
  return FRX_OK;
}

frx_status frx_release_retired(frx_ctx *ctx) {
  frx_status st = enter(ctx, false);
  if (st != FRX_OK) return st;
  // launches already enqueued on the context stream may still use them
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "release wait");
  for (void *p : ctx->retired) (void)hipFree(p);
  ctx->retired.clear();
  ctx->retired_bytes = 0;
  return FRX_OK;
}

frx_status frx_moe_ternary_ffn(
    frx_ctx *ctx, const void *x, frx_dtype xt, const void *router,
    frx_dtype rt, const uint32_t *const *w_gate, const float *const *s_gate,
    const uint32_t *const *w_up, const float *const *s_up,
    const uint32_t *const *w_down, const float *const *s_down, uint32_t T,
    uint32_t H, uint32_t I, uint32_t E, uint32_t top_k, frx_activation act,
    void *y, frx_dtype yt, uint32_t *topk_idx, float *topk_w) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  // TernaryMoELayer's GeLU experts read no up projection: w_up / s_up may be
  // NULL, and the gate matrices stand in for them in the kernels' operands
  const bool gate_only = act == FRX_ACT_GELU_TANH_GATE;
  if (gate_only) {
    if (!w_up) w_up = w_gate;
    if (!s_up) s_up = s_gate;
  }
  if (!x || !router || !w_gate || !s_gate || !w_up || !s_up || !w_down || !s_down || !y)
    return fail(ctx, FRX_ERR_SHAPE, "null pointer argument");
  if (T == 0 || H == 0 || I == 0 || E == 0) return fail(ctx, FRX_ERR_SHAPE, "empty shape");
  if (E > 64) return fail(ctx, FRX_ERR_SHAPE, "num_experts=%u exceeds 64", E);
  if (top_k == 0 || top_k > E) return fail(ctx, FRX_ERR_SHAPE, "top_k=%u must be in [1, %u]", top_k, E);
  if (H % 16 != 0 || I % 16 != 0)
    return fail(ctx, FRX_ERR_SHAPE, "hidden=%u and intermediate=%u must be multiples of 16", H, I);
  if ((xt != FRX_F32 && xt != FRX_BF16) || (rt != FRX_F32 && rt != FRX_BF16) || (yt != FRX_F32 && yt != FRX_BF16))
    return fail(ctx, FRX_ERR_UNSUPPORTED, "dtype must be FRX_F32 or FRX_BF16");
  if (act != FRX_ACT_SILU && act != FRX_ACT_GELU_TANH && act != FRX_ACT_GELU_TANH_GATE)
    return fail(ctx, FRX_ERR_UNSUPPORTED, "activation");
  std::vector<const uint32_t *> wu_sub;
  std::vector<const float *> su_sub;
  if (gate_only) {
    wu_sub.assign(w_up, w_up + E);
    su_sub.assign(s_up, s_up + E);
    for (uint32_t e = 0; e < E; e++) {
      if (!wu_sub[e]) wu_sub[e] = w_gate[e];
      if (!su_sub[e]) su_sub[e] = s_gate[e];
    }
    w_up = wu_sub.data();
    s_up = su_sub.data();
  }
  for (uint32_t e = 0; e < E; e++)
    if (!w_gate[e] || !s_gate[e] || !w_up[e] || !s_up[e] || !w_down[e] || !s_down[e])
      return fail(ctx, FRX_ERR_SHAPE, "null weight pointer for expert %u", e);
  if ((size_t)T * top_k * I > (size_t)0x7FFFFFFF) return fail(ctx, FRX_ERR_SHAPE, "T*top_k*I too large");
  if (ctx->lora_on && ctx->lora_experts != E)
    return fail(ctx, FRX_ERR_SHAPE, "LoRA adapters were set for %u experts, the call has %u", ctx->lora_experts, E);
  const size_t need = frx::moe_workspace_bytes((int)T, (int)H, (int)I, (int)E, (int)top_k);
  if ((st = ensure_buffer(ctx, &ctx->moe_ws, &ctx->moe_ws_bytes, need, "MoE workspace allocation")) != FRX_OK)
    return st;
  frx::MoeWorkspace ws;
  frx::moe_workspace_carve(ctx->moe_ws, (int)T, (int)H, (int)I, (int)E, (int)top_k, &ws);
  // a few routed rows (the decode path): its down launch also combines,
  // through the context's arrival counters
  if ((size_t)T * top_k <= (size_t)frx::MOE_DEC_MAXA) {
    if ((st = ensure_sk_counters(ctx)) != FRX_OK) return st;
    ws.cnt = ctx->sk_cnt;
  }
  const void *router_eh = router;
  if (ctx->moe_routing == FRX_MOE_CPU_MOE_LAYER) {
    // CpuMoELayer reads its router as [H][E]; the kernels read [E][H]
    const size_t rb = (size_t)H * E * (rt == FRX_BF16 ? 2 : 4);
    if ((st = ensure_buffer(ctx, &ctx->router_ws, &ctx->router_ws_bytes, a256(rb), "router workspace allocation")) !=
        FRX_OK)
      return st;
    hipError_t e = frx::launch_router_transpose(router, rt == FRX_BF16, ctx->router_ws, (int)H, (int)E, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "router transpose launch");
    router_eh = ctx->router_ws;
  }
  frx::MoeLora lora;
  if (ctx->lora_on) {
    lora.tbl = ctx->lora_tbl;
    lora.rank = (int)ctx->lora_rank;
    lora.scaling = ctx->lora_scaling;
  }
  hipError_t e = frx::launch_moe(x, xt == FRX_BF16, router_eh, rt == FRX_BF16, w_gate, s_gate, w_up, s_up, w_down,
                                 s_down, (int)T, (int)H, (int)I, (int)E, (int)top_k, (int)act, y,
                                 yt == FRX_BF16, topk_idx, topk_w, ws, ctx->moe_routing, lora, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "moe launch");
  return FRX_OK;
}


static frx_status check_ffn(frx_ctx *ctx, const void *x, frx_dtype xt, const void *w_gate,
                            const float *s_gate, const void *w_up, const float *s_up, uint32_t M,
                            uint32_t H, uint32_t I, frx_activation act) {
  if (!x || !w_gate || !s_gate || !w_up || !s_up) return fail(ctx, FRX_ERR_SHAPE, "null pointer argument");
  if (M == 0 || H == 0 || I == 0) return fail(ctx, FRX_ERR_SHAPE, "empty shape M=%u H=%u I=%u", M, H, I);
  if (H % 16 != 0 || I % 16 != 0)
    return fail(ctx, FRX_ERR_SHAPE, "hidden=%u and intermediate=%u must be multiples of 16", H, I);
  if (xt != FRX_F32 && xt != FRX_BF16) return fail(ctx, FRX_ERR_UNSUPPORTED, "dtype must be FRX_F32 or FRX_BF16");
  if (act != FRX_ACT_SILU && act != FRX_ACT_GELU_TANH) return fail(ctx, FRX_ERR_UNSUPPORTED, "activation");
  if (!aligned16(x) || !aligned16(s_gate) || !aligned16(s_up))
    return fail(ctx, FRX_ERR_UNSUPPORTED, "x and scales must be 16-byte aligned device pointers");
  if ((size_t)M * H > (size_t)0x7FFFFFFF || (size_t)M * I > (size_t)0x3FFFFFFF)
    return fail(ctx, FRX_ERR_SHAPE, "M*H or M*I too large");
  return FRX_OK;
}

// h = act(g) * u into an fp32 [M][I] buffer. M <= 16: one launch; larger M:
// two GEMMs (g into h, u into u_ws, or into the context's workspace when
// u_ws is null) and a combine.
static frx_status glu_into(frx_ctx *ctx, const void *x, frx_dtype xt, const uint32_t *w_gate,
                           const float *s_gate, const uint32_t *w_up, const float *s_up, uint32_t M,
                           uint32_t H, uint32_t I, bool gelu, float *h, float *u_ws) {
  hipError_t e;
  if (M <= 16) {
    e = frx::launch_gemv_glu(w_gate, s_gate, w_up, s_up, x, xt == FRX_BF16, h, (int)M, (int)H, (int)I, gelu,
                             ctx->stream);
  } else {
    float *u = u_ws;
    if (!u) {
      // the allocating entries: gate and up as linears (split over K where
      // the tiles leave compute units idle; f32 x as bf16 hi | lo rows)
      const size_t ub = a256((size_t)M * I * 4);
      frx_status st = ensure_buffer(ctx, &ctx->glu_ws, &ctx->glu_ws_bytes, ub, "GLU workspace allocation");
      if (st != FRX_OK) return st;
      u = reinterpret_cast<float *>(ctx->glu_ws);
      if ((st = gemv_auto(ctx, w_gate, s_gate, nullptr, x, xt, h, FRX_F32, M, H, I)) != FRX_OK) return st;
      if ((st = gemv_auto(ctx, w_up, s_up, nullptr, x, xt, u, FRX_F32, M, H, I)) != FRX_OK) return st;
      e = frx::launch_glu_combine(h, u, h, (size_t)M * I, gelu, ctx->stream);
    } else {
      e = frx::launch_gemm(w_gate, s_gate, x, xt == FRX_BF16, h, 0, (int)M, (int)H, (int)I, 0, ctx->stream);
      if (e == hipSuccess)
        e = frx::launch_gemm(w_up, s_up, x, xt == FRX_BF16, u, 0, (int)M, (int)H, (int)I, 0, ctx->stream);
      if (e == hipSuccess) e = frx::launch_glu_combine(h, u, h, (size_t)M * I, gelu, ctx->stream);
    }
  }
  if (e != hipSuccess) return hip_fail(ctx, e, "gate/up launch");
  return FRX_OK;
}

frx_status frx_ternary_glu(frx_ctx *ctx, const void *x, frx_dtype xt, const uint32_t *w_gate,
                           const float *s_gate, const uint32_t *w_up, const float *s_up, uint32_t M,
                           uint32_t H, uint32_t I, frx_activation act, float *h) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if ((st = check_ffn(ctx, x, xt, w_gate, s_gate, w_up, s_up, M, H, I, act)) != FRX_OK) return st;
  if (!h) return fail(ctx, FRX_ERR_SHAPE, "null output pointer");
  if (!aligned16(h)) return fail(ctx, FRX_ERR_UNSUPPORTED, "h must be a 16-byte aligned device pointer");
  return glu_into(ctx, x, xt, w_gate, s_gate, w_up, s_up, M, H, I, act == FRX_ACT_GELU_TANH, h, nullptr);
}

// Token counts from which the unfused FFN writes h as bf16 hi/lo planes for
// the unstaged down GEMV (below: fp32 h, staged down).
static constexpr int FFN_PLANES_MIN_M = 4;

static frx_status check_ffn_down(frx_ctx *ctx, const uint32_t *w_down, const float *s_down, void *y,
                                 frx_dtype yt) {
  if (!w_down || !s_down || !y) return fail(ctx, FRX_ERR_SHAPE, "null pointer argument");
  if (yt != FRX_F32 && yt != FRX_BF16) return fail(ctx, FRX_ERR_UNSUPPORTED, "dtype must be FRX_F32 or FRX_BF16");
  if (!aligned16(y) || !aligned16(s_down))
    return fail(ctx, FRX_ERR_UNSUPPORTED, "y and scales must be 16-byte aligned device pointers");
  return FRX_OK;
}

// The dense FFN with its intermediate in `ws` (at least M*I*4 bytes, 256-byte
// aligned). u_ws: the GEMM path's up projection (M > 16; null = the
// context's workspace). allow_one: the one-launch kernel may run (it needs
// the context's barrier words).
// The down launch over h's bf16 planes [2][M][I] at 3-16 tokens: the split-K
// GEMV (planes staged once per 128-row tile and column slice) where it
// measured faster, i.e. I >= 8192, and only where the call may allocate its
// workspace; else the planes kernels of frx_gemv.hip.
static frx_status ffn_down_planes(frx_ctx *ctx, const uint32_t *w_down, const float *s_down, const uint16_t *hp,
                                  void *y, frx_dtype yt, uint32_t M, uint32_t H, uint32_t I, bool may_alloc) {
  const bool split = may_alloc && ctx->gemv_split != FRX_GEMV_SPLIT_NEVER &&
                     (ctx->gemv_split == FRX_GEMV_SPLIT_ALWAYS || I >= 8192) &&
                     (H + 127) / 128 <= (uint32_t)frx::GEMV_SK_MAX_TILES && (size_t)M * I * 4 < ((size_t)1 << 32);
  hipError_t e;
  if (split) {
    frx_status st = ensure_buffer(ctx, &ctx->sk_ws, &ctx->sk_ws_bytes,
                                  frx::gemv_sk_workspace_bytes((int)I, (int)H, ctx->cus), "split-K workspace allocation");
    if (st != FRX_OK) return st;
    if ((st = ensure_sk_counters(ctx)) != FRX_OK) return st;
    e = frx::launch_gemv_sk(w_down, s_down, hp, hp + (size_t)M * I, 2, y, yt == FRX_BF16, (int)M, (int)I, (int)H,
                            reinterpret_cast<float *>(ctx->sk_ws), ctx->sk_cnt, nullptr, ctx->cus, ctx->stream);
  } else {
    e = frx::launch_gemv_planes(w_down, s_down, hp, y, yt == FRX_BF16, (int)M, (int)I, (int)H, ctx->stream);
  }
  if (e != hipSuccess) return hip_fail(ctx, e, "ffn down launch");
  return FRX_OK;
}

static frx_status ffn_run(frx_ctx *ctx, const void *x, frx_dtype xt, const uint32_t *w_gate, const float *s_gate,
                          const uint32_t *w_up, const float *s_up, const uint32_t *w_down, const float *s_down,
                          uint32_t M, uint32_t H, uint32_t I, frx_activation act, void *y, frx_dtype yt, void *ws,
                          float *u_ws, bool allow_one) {
  hipError_t e;
  const bool two_only = ctx->ffn_mode == FRX_FFN_TWO_LAUNCH || !allow_one;
  // the one-launch kernel's context (allow_one) is the allocating entry point
  const bool may_alloc = allow_one;
  if ((!allow_one || ctx->ffn_mode != FRX_FFN_ONE_LAUNCH) && xt == FRX_BF16 && aligned16(w_gate) &&
      aligned16(w_up) && aligned16(w_down) && frx::gemv_rows_ffn_ok((int)M, (int)H, (int)I)) {
    // one token: gate/up/act into bf16 hi/lo planes of h (the first 4*I
    // bytes of the workspace), then the down rows over both planes
    uint16_t *hp = reinterpret_cast<uint16_t *>(ws);
    e = frx::launch_gemv_rows_glu_planes(w_gate, s_gate, w_up, s_up, x, hp, (int)H, (int)I,
                                         act == FRX_ACT_GELU_TANH, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "ffn gate/up launch");
    e = frx::launch_gemv_rows_planes(w_down, s_down, hp, y, yt == FRX_BF16, (int)I, (int)H, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "ffn down launch");
    return FRX_OK;
  }
  if ((!allow_one || ctx->ffn_mode != FRX_FFN_ONE_LAUNCH) && xt == FRX_BF16 && aligned16(w_gate) &&
      aligned16(w_up) && aligned16(w_down) && frx::gemv_rows4_ffn_ok((int)M, (int)H, (int)I)) {
    // two tokens: the same in the 4-segment kernels, the down launch taking
    // h's hi and lo planes of both tokens as its four token columns
    uint16_t *hp = reinterpret_cast<uint16_t *>(ws);
    e = frx::launch_gemv_rows4_glu_planes(w_gate, s_gate, w_up, s_up, x, hp, (int)M, (int)H, (int)I,
                                          act == FRX_ACT_GELU_TANH, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "ffn gate/up launch");
    e = frx::launch_gemv_rows4_planes(w_down, s_down, hp, y, yt == FRX_BF16, (int)I, (int)H, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "ffn down launch");
    return FRX_OK;
  }
  if (may_alloc && ctx->ffn_mode != FRX_FFN_ONE_LAUNCH && ctx->gemv_split != FRX_GEMV_SPLIT_NEVER &&
      xt == FRX_BF16 && M == 1 && aligned16(w_gate) && aligned16(w_up) && aligned16(w_down) && H % 64 == 0 &&
      H <= 16384 && I % 64 == 0 && I > 16384) {
    // one token over an intermediate longer than the rows kernels take
    // (LLaMA-70B: I = 28672): gate/up/act in the rows kernel into h's bf16
    // planes, then the split-K down launch over both planes
    uint16_t *hp = reinterpret_cast<uint16_t *>(ws);
    e = frx::launch_gemv_rows_glu_planes(w_gate, s_gate, w_up, s_up, x, hp, (int)H, (int)I,
                                         act == FRX_ACT_GELU_TANH, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "ffn gate/up launch");
    return ffn_down_planes(ctx, w_down, s_down, hp, y, yt, M, H, I, may_alloc);
  }
  if (ctx->ffn_mode != FRX_FFN_ONE_LAUNCH && xt == FRX_BF16 && aligned16(w_gate) && aligned16(w_up) &&
      aligned16(w_down) && (M == 3 || M == 4) && frx::gemv_rows4_ffn_ok(2, (int)H, (int)I)) {
    // three or four tokens: gate/up/act in the 4-segment kernel into h's
    // planes [2][M][I], then the down launch over both planes (LLaMA-7B
    // shapes, M = 4: 25.7 us with the operand-load kernels, 19.6 us so)
    uint16_t *hp = reinterpret_cast<uint16_t *>(ws);
    e = frx::launch_gemv_rows4_glu_planes(w_gate, s_gate, w_up, s_up, x, hp, (int)M, (int)H, (int)I,
                                          act == FRX_ACT_GELU_TANH, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "ffn gate/up launch");
    return ffn_down_planes(ctx, w_down, s_down, hp, y, yt, M, H, I, may_alloc);
  }
  int grid = 0;
  size_t lds = 0;
  const bool one = !two_only && aligned16(w_gate) && aligned16(w_up) && aligned16(w_down) &&
                   frx::ffn1_supported((int)M, (int)H, (int)I, xt == FRX_BF16, ctx->cus, &grid, &lds);
  if (allow_one && ctx->ffn_mode == FRX_FFN_ONE_LAUNCH && !one)
    return fail(ctx, FRX_ERR_UNSUPPORTED,
                "one-launch FFN: unsupported shape M=%u H=%u I=%u (M <= 3, H <= 4096, I <= 11520, "
                "multiples of 64, 16-byte aligned weights)", M, H, I);
  if (one) {
    if (!ctx->ffn_bar) {
      void *p = nullptr;
      e = hipMalloc(&p, frx::ffn1_barrier_bytes());
      if (e != hipSuccess) return hip_fail(ctx, e, "FFN barrier allocation");
      e = hipMemset(p, 0, frx::ffn1_barrier_bytes());
      // the legacy stream of hipMemset does not order against a non-blocking
      // caller stream: wait for it here (first use only)
      if (e == hipSuccess) e = hipDeviceSynchronize();
      if (e != hipSuccess) {
        (void)hipFree(p);
        return hip_fail(ctx, e, "FFN barrier initialisation");
      }
      ctx->ffn_bar = reinterpret_cast<unsigned *>(p);
    }
    e = frx::launch_ffn1(x, xt == FRX_BF16, w_gate, s_gate, w_up, s_up, w_down, s_down,
                         reinterpret_cast<uint32_t *>(ws), y, yt == FRX_BF16, ctx->ffn_bar, (int)M, (int)H, (int)I,
                         act == FRX_ACT_GELU_TANH, grid, lds, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "one-launch FFN");
    return FRX_OK;
  }
  if (xt == FRX_BF16 && (int)M >= FFN_PLANES_MIN_M && M <= 16) {
    // h as bf16 hi/lo planes (the same M*I*4 bytes), consumed by the down
    // GEMV without staging: at these M the fp32 rows of h do not fit LDS.
    uint16_t *hp = reinterpret_cast<uint16_t *>(ws);
    e = frx::launch_gemv_glu_planes(w_gate, s_gate, w_up, s_up, x, hp, (int)M, (int)H, (int)I,
                                    act == FRX_ACT_GELU_TANH, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "ffn gate/up launch");
    return ffn_down_planes(ctx, w_down, s_down, hp, y, yt, M, H, I, may_alloc);
  }
  float *h = reinterpret_cast<float *>(ws);
  frx_status st = glu_into(ctx, x, xt, w_gate, s_gate, w_up, s_up, M, H, I, act == FRX_ACT_GELU_TANH, h, u_ws);
  if (st != FRX_OK) return st;
  if (M > 16 && I % 64 == 0 && aligned16(w_down)) {
    // h as bf16 hi | lo rows in the up projection's buffer (no longer
    // read), then the bf16 engine over both halves
    uint16_t *h2 = reinterpret_cast<uint16_t *>(u_ws ? u_ws : reinterpret_cast<float *>(ctx->glu_ws));
    e = frx::launch_to_planes(h, h2, (int)M, (int)I, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "ffn planes launch");
    return gemm_planes_auto(ctx, w_down, s_down, nullptr, h2, y, yt, M, I, H, may_alloc);
  }
  // fp32 h: the allocating entry takes the split-K down launch where it is
  // faster (long rows of h)
  if (may_alloc) return gemv_auto(ctx, w_down, s_down, nullptr, h, FRX_F32, y, yt, M, I, H);
  if (M <= 16)
    e = frx::launch_gemv(w_down, s_down, h, 0, y, yt == FRX_BF16, (int)M, (int)I, (int)H, ctx->stream);
  else
    e = frx::launch_gemm(w_down, s_down, h, 0, y, yt == FRX_BF16, (int)M, (int)I, (int)H, 0, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "ffn down launch");
  return FRX_OK;
}

frx_status frx_ternary_ffn(frx_ctx *ctx, const void *x, frx_dtype xt, const uint32_t *w_gate,
                           const float *s_gate, const uint32_t *w_up, const float *s_up,
                           const uint32_t *w_down, const float *s_down, uint32_t M, uint32_t H,
                           uint32_t I, frx_activation act, void *y, frx_dtype yt) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if ((st = check_ffn(ctx, x, xt, w_gate, s_gate, w_up, s_up, M, H, I, act)) != FRX_OK) return st;
  if ((st = check_ffn_down(ctx, w_down, s_down, y, yt)) != FRX_OK) return st;
  if ((st = ensure_buffer(ctx, &ctx->ffn_ws, &ctx->ffn_ws_bytes, a256((size_t)M * I * 4),
                          "FFN workspace allocation")) != FRX_OK)
    return st;
  return ffn_run(ctx, x, xt, w_gate, s_gate, w_up, s_up, w_down, s_down, M, H, I, act, y, yt, ctx->ffn_ws, nullptr,
                 true);
}

frx_status frx_ternary_ffn_noalloc(frx_ctx *ctx, const void *x, frx_dtype xt, const uint32_t *w_gate,
                                   const float *s_gate, const uint32_t *w_up, const float *s_up,
                                   const uint32_t *w_down, const float *s_down, uint32_t M, uint32_t H,
                                   uint32_t I, frx_activation act, void *y, frx_dtype yt) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if ((st = check_ffn(ctx, x, xt, w_gate, s_gate, w_up, s_up, M, H, I, act)) != FRX_OK) return st;
  if ((st = check_ffn_down(ctx, w_down, s_down, y, yt)) != FRX_OK) return st;
  if (ctx->noalloc_err != hipSuccess || !ctx->noalloc)
    return fail(ctx, FRX_ERR_GPU, "no-allocation FFN: scratch address unavailable: %s",
                hipGetErrorString(ctx->noalloc_err));
  const size_t hb = a256((size_t)M * I * 4);
  const size_t need = M > 16 ? 2 * hb : hb;  // h, and the GEMM path's up projection
  if (need > FRX_NOALLOC_SCRATCH_BYTES)
    return fail(ctx, FRX_ERR_UNSUPPORTED,
                "no-allocation FFN: M=%u I=%u needs %zu bytes of scratch, the maximum is %u "
                "(M*I*4 bytes for M <= 16, twice that above)",
                M, I, need, (unsigned)FRX_NOALLOC_SCRATCH_BYTES);
  char *base = reinterpret_cast<char *>(ctx->noalloc);
  return ffn_run(ctx, x, xt, w_gate, s_gate, w_up, s_up, w_down, s_down, M, H, I, act, y, yt, base,
                 M > 16 ? reinterpret_cast<float *>(base + hb) : nullptr, false);
}

// ---- the reference's other matmul forms --------------------------------------

frx_status frx_ternary_linear_blocked(frx_ctx *ctx, const uint32_t *w, const float *block_scales,
                                      uint32_t block_size, const void *x, frx_dtype xt, void *y, frx_dtype yt,
                                      uint32_t M, uint32_t K, uint32_t N) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if (!block_scales) return fail(ctx, FRX_ERR_SHAPE, "null block scales");
  if (block_size == 0) return fail(ctx, FRX_ERR_SHAPE, "block_size must be positive");
  if ((st = check_linear(ctx, w, block_scales, x, xt, y, yt, M, K, N, false)) != FRX_OK) return st;
  if ((st = ensure_buffer(ctx, &ctx->blk_ws, &ctx->blk_ws_bytes, a256((size_t)M * K * 4),
                          "block-scale workspace allocation")) != FRX_OK)
    return st;
  if (ctx->unit_ws_bytes < (size_t)N * 4) {
    if ((st = ensure_buffer(ctx, &ctx->unit_ws, &ctx->unit_ws_bytes, a256((size_t)N * 4),
                            "unit scale allocation")) != FRX_OK)
      return st;
    hipError_t e = frx::launch_fill(reinterpret_cast<float *>(ctx->unit_ws), 1.0f, ctx->unit_ws_bytes / 4,
                                    ctx->stream);
    // wait for the fill: a later call may run on another stream (frx_set_stream)
    // and must not read the scales before they are written
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "unit scale fill");
  }
  float *xs = reinterpret_cast<float *>(ctx->blk_ws);
  const float *ones = reinterpret_cast<const float *>(ctx->unit_ws);
  Staged sg;  // xs and ones are aligned workspaces: at most y is staged
  if ((st = stage_linear(ctx, xs, FRX_F32, ones, y, yt, M, K, N, &sg)) != FRX_OK) return st;
  hipError_t e = frx::launch_block_prescale(x, xt == FRX_BF16, block_scales, (int)block_size, xs, (int)M, (int)K,
                                            ctx->stream);
  if (e == hipSuccess) {
    if (M <= 16)
      e = frx::launch_gemv(w, ones, xs, 0, sg.y, yt == FRX_BF16, (int)M, (int)K, (int)N, ctx->stream);
    else
      e = frx::launch_gemm(w, ones, xs, 0, sg.y, yt == FRX_BF16, (int)M, (int)K, (int)N, 0, ctx->stream);
  }
  if (e == hipSuccess) e = unstage_linear(ctx, sg);
  if (e != hipSuccess) return hip_fail(ctx, e, "column-block linear launch");
  return FRX_OK;
}

frx_status frx_ternary_sparse_decode(frx_ctx *ctx, const uint32_t *pos_off, const uint32_t *pos_idx,
                                     const uint32_t *neg_off, const uint32_t *neg_idx, float scale, const void *x,
                                     frx_dtype xt, void *y, frx_dtype yt, uint32_t M, uint32_t K, uint32_t N) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if (!pos_off || !pos_idx || !neg_off || !neg_idx || !x || !y)
    return fail(ctx, FRX_ERR_SHAPE, "null buffer pointer");
  if (M == 0 || K == 0 || N == 0) return fail(ctx, FRX_ERR_SHAPE, "empty shape M=%u K=%u N=%u", M, K, N);
  if ((xt != FRX_F32 && xt != FRX_BF16) || (yt != FRX_F32 && yt != FRX_BF16))
    return fail(ctx, FRX_ERR_UNSUPPORTED, "dtype must be FRX_F32 or FRX_BF16");
  if (M > 65535) return fail(ctx, FRX_ERR_SHAPE, "M=%u exceeds 65535 tokens", M);
  hipError_t e = frx::launch_index_decode(pos_off, pos_idx, neg_off, neg_idx, scale, x, xt == FRX_BF16, y,
                                          yt == FRX_BF16, (int)M, (int)K, (int)N, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "index-list decode launch");
  return FRX_OK;
}

frx_status frx_ternary_stats(frx_ctx *ctx, const uint32_t *w, uint32_t N, uint32_t K, unsigned long long *counts) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if (!w || !counts) return fail(ctx, FRX_ERR_SHAPE, "null buffer pointer");
  if (N == 0 || K == 0) return fail(ctx, FRX_ERR_SHAPE, "empty shape N=%u K=%u", N, K);
  if (K % 16 != 0) return fail(ctx, FRX_ERR_SHAPE, "K=%u must be a multiple of 16", K);
  hipError_t e = frx::launch_stats(w, (size_t)N * (K / 16), counts, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "statistics launch");
  return FRX_OK;
}

// ---- host-slice accelerator API (GpuMatmulAccelerator) --------------------

// The host-slice calls synchronise before they return, so nothing in flight
// uses the old scratch when it grows: it is freed at once.
static frx_status ensure_scratch(frx_ctx *ctx, size_t bytes) {
  if (bytes <= ctx->scratch_bytes) return FRX_OK;
  if (ctx->scratch) {
    (void)hipFree(ctx->scratch);
    ctx->scratch = nullptr;
    ctx->scratch_bytes = 0;
  }
  hipError_t e = hipMalloc(&ctx->scratch, bytes);
  if (e != hipSuccess) return hip_fail(ctx, e, "device scratch allocation");
  ctx->scratch_bytes = bytes;
  return FRX_OK;
}

// Host-slice linear: w / s are host arrays (uploaded per call) when
// upload_w is set, else device pointers.
static frx_status host_linear(frx_ctx *ctx, bool upload_w, const uint32_t *w, const float *s,
                              const float *input, size_t seq, size_t in_cols, size_t out_rows,
                              float *out, bool sparse) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if (!input || !out) return fail(ctx, FRX_ERR_SHAPE, "null host buffer");
  if (!w || !s) return fail(ctx, FRX_ERR_SHAPE, upload_w ? "null host weights or scales" : "null device weight buffer");
  const uint32_t *w_host = upload_w ? w : nullptr, *w_dev = upload_w ? nullptr : w;
  const float *s_host = upload_w ? s : nullptr, *s_dev = upload_w ? nullptr : s;
  if (seq == 0 || in_cols == 0 || out_rows == 0) return fail(ctx, FRX_ERR_SHAPE, "empty shape");
  if (seq > 0xFFFFFFFFu || in_cols > 0xFFFFFFFFu || out_rows > 0xFFFFFFFFu)
    return fail(ctx, FRX_ERR_SHAPE, "dimension exceeds 32 bits");
  size_t wwords = 0;
  if (w_host) {
    if (sparse) {
      const size_t gpr = (in_cols + 3) / 4;
      wwords = out_rows * ((gpr + 5) / 6);
    } else {
      wwords = out_rows * ((in_cols + 15) / 16);
    }
  }
  const size_t bw = a256(wwords * 4), bs = w_host ? a256(out_rows * 4) : 0;
  const size_t bx = a256(seq * in_cols * 4), by = a256(seq * out_rows * 4);
  if ((st = ensure_scratch(ctx, bw + bs + bx + by)) != FRX_OK) return st;
  char *base = reinterpret_cast<char *>(ctx->scratch);
  uint32_t *dw = w_host ? reinterpret_cast<uint32_t *>(base) : const_cast<uint32_t *>(w_dev);
  float *ds = w_host ? reinterpret_cast<float *>(base + bw) : const_cast<float *>(s_dev);
  float *dx = reinterpret_cast<float *>(base + bw + bs);
  float *dy = reinterpret_cast<float *>(base + bw + bs + bx);
  hipError_t e;
  if (w_host) {
    if ((e = hipMemcpyAsync(dw, w_host, wwords * 4, hipMemcpyHostToDevice, ctx->stream)) != hipSuccess)
      return hip_fail(ctx, e, "weight upload");
    if ((e = hipMemcpyAsync(ds, s_host, out_rows * 4, hipMemcpyHostToDevice, ctx->stream)) != hipSuccess)
      return hip_fail(ctx, e, "scale upload");
  }
  if ((e = hipMemcpyAsync(dx, input, seq * in_cols * 4, hipMemcpyHostToDevice, ctx->stream)) != hipSuccess)
    return hip_fail(ctx, e, "input upload");
  st = sparse ? frx_sparse24_ternary_linear(ctx, dw, ds, dx, FRX_F32, dy, FRX_F32, (uint32_t)seq,
                                            (uint32_t)in_cols, (uint32_t)out_rows)
              : frx_ternary_linear(ctx, dw, ds, dx, FRX_F32, dy, FRX_F32, (uint32_t)seq, (uint32_t)in_cols,
                                   (uint32_t)out_rows);
  if (st != FRX_OK) return st;
  if ((e = hipMemcpyAsync(out, dy, seq * out_rows * 4, hipMemcpyDeviceToHost, ctx->stream)) != hipSuccess)
    return hip_fail(ctx, e, "output readback");
  if ((e = hipStreamSynchronize(ctx->stream)) != hipSuccess) return hip_fail(ctx, e, "synchronize");
  return FRX_OK;
}

frx_status frx_gpu_ternary_matmul(frx_ctx *ctx, const uint32_t *packed_weights,
                                  const float *scales, const float *input,
                                  size_t seq_len, size_t in_cols,
                                  size_t out_rows, float *out) {
  return host_linear(ctx, true, packed_weights, scales, input, seq_len, in_cols, out_rows, out, false);
}

frx_status frx_gpu_ternary_matmul_vram(frx_ctx *ctx, const uint32_t *w_dev,
                                       const float *s_dev, const float *input,
                                       size_t seq_len, size_t in_cols,
                                       size_t out_rows, float *out) {
  return host_linear(ctx, false, w_dev, s_dev, input, seq_len, in_cols, out_rows, out, false);
}

frx_status frx_gpu_sparse_ternary_matmul(frx_ctx *ctx, const uint32_t *meta,
                                         const float *scales,
                                         const float *input, size_t seq_len,
                                         size_t in_cols, size_t out_rows,
                                         float *out) {
  return host_linear(ctx, true, meta, scales, input, seq_len, in_cols, out_rows, out, true);
}

// ---- weight ingest (resident upload, done once) ----------------------------

// Device allocation that frx_free releases; on failure nothing is left
// allocated.
static frx_status dev_alloc(frx_ctx *ctx, void **p, size_t bytes, const char *what) {
  *p = nullptr;
  const hipError_t e = hipMalloc(p, bytes ? bytes : 4);
  if (e != hipSuccess) {
    *p = nullptr;
    return hip_fail(ctx, e, what);
  }
  return FRX_OK;
}

static frx_status upload_scales(frx_ctx *ctx, const float *row_scales, float tensor_scale, uint32_t N,
                                float **s_dev) {
  frx_status st = dev_alloc(ctx, reinterpret_cast<void **>(s_dev), (size_t)N * 4, "scale allocation");
  if (st != FRX_OK) return st;
  std::vector<float> bc;
  const float *src = row_scales;
  if (!src) {  // gpu_packed(): the tensor scale on every row
    bc.assign(N, tensor_scale);
    src = bc.data();
  }
  const hipError_t e = hipMemcpy(*s_dev, src, (size_t)N * 4, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(*s_dev);
    *s_dev = nullptr;
    return hip_fail(ctx, e, "scale upload");
  }
  return FRX_OK;
}

frx_status frx_upload_ternary(frx_ctx *ctx, const uint8_t *packed, uint32_t N, uint32_t K,
                              const float *row_scales, float tensor_scale, uint32_t **w_dev, float **s_dev) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if (!packed || !w_dev || !s_dev) return fail(ctx, FRX_ERR_SHAPE, "null pointer argument");
  *w_dev = nullptr;
  *s_dev = nullptr;
  if (N == 0 || K == 0) return fail(ctx, FRX_ERR_SHAPE, "empty shape N=%u K=%u", N, K);
  if (K % 16 != 0) return fail(ctx, FRX_ERR_SHAPE, "K=%u must be a multiple of 16 for row-aligned u32 words", K);
  const size_t bytes = (size_t)N * K / 4;
  if ((st = dev_alloc(ctx, reinterpret_cast<void **>(w_dev), bytes, "weight allocation")) != FRX_OK) return st;
  // pack_ternary_u32 regroups 4 bytes little-endian into a word: on this
  // little-endian device the u32 layout is the u8 stream itself.
  hipError_t e = hipMemcpy(*w_dev, packed, bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(*w_dev);
    *w_dev = nullptr;
    return hip_fail(ctx, e, "weight upload");
  }
  if ((st = upload_scales(ctx, row_scales, tensor_scale, N, s_dev)) != FRX_OK) {
    (void)hipFree(*w_dev);
    *w_dev = nullptr;
  }
  return st;
}

frx_status frx_quantize_ternary(frx_ctx *ctx, const void *w, frx_dtype wt, uint32_t N, uint32_t K,
                                frx_quant_rule rule, uint32_t *packed, float *scale) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if (!w || !packed || !scale) return fail(ctx, FRX_ERR_SHAPE, "null pointer argument");
  if (K == 0 || K % 16 != 0) return fail(ctx, FRX_ERR_SHAPE, "K=%u must be a positive multiple of 16", K);
  if (wt != FRX_F32 && wt != FRX_BF16) return fail(ctx, FRX_ERR_UNSUPPORTED, "dtype must be FRX_F32 or FRX_BF16");
  if (rule != FRX_QUANT_ABSMEAN && rule != FRX_QUANT_STE) return fail(ctx, FRX_ERR_UNSUPPORTED, "quantisation rule");
  if (N > 0x7FFFFFFFu || K > 0x7FFFFFF0u) return fail(ctx, FRX_ERR_SHAPE, "N=%u K=%u too large", N, K);
  const hipError_t e =
      frx::launch_quantize(w, wt == FRX_BF16, (int)N, (int)K, (int)rule, packed, scale, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "quantise launch");
  return FRX_OK;
}

frx_status frx_quantize_ternary_blocked(frx_ctx *ctx, const void *w, frx_dtype wt, size_t n, uint32_t block_size,
                                        uint32_t *packed, float *scales) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if (n == 0) return FRX_OK;  // the reference returns two empty vectors
  if (!w || !packed || !scales) return fail(ctx, FRX_ERR_SHAPE, "null pointer argument");
  if (block_size == 0) return fail(ctx, FRX_ERR_SHAPE, "block_size must be positive");
  if (wt != FRX_F32 && wt != FRX_BF16) return fail(ctx, FRX_ERR_UNSUPPORTED, "dtype must be FRX_F32 or FRX_BF16");
  if ((n + block_size - 1) / block_size > 0x7FFFFFFFu || n > ((size_t)1 << 40))
    return fail(ctx, FRX_ERR_SHAPE, "n=%zu with block_size=%u: too many blocks", n, block_size);
  const hipError_t e =
      frx::launch_quantize_flat(w, wt == FRX_BF16, n, block_size, 0, packed, scales, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "blocked quantise launch");
  return FRX_OK;
}

frx_status frx_dequantize_ternary_blocked(frx_ctx *ctx, const uint32_t *packed, const float *scales, size_t n,
                                          uint32_t block_size, float *out) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if (n == 0) return FRX_OK;
  if (!packed || !scales || !out) return fail(ctx, FRX_ERR_SHAPE, "null pointer argument");
  if (block_size == 0) return fail(ctx, FRX_ERR_SHAPE, "block_size must be positive");
  if (n > ((size_t)1 << 40)) return fail(ctx, FRX_ERR_SHAPE, "n=%zu too large", n);
  const hipError_t e = frx::launch_dequantize(packed, scales, n, block_size, out, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "dequantise launch");
  return FRX_OK;
}

frx_status frx_prune_sparse24(frx_ctx *ctx, const void *w, frx_dtype wt, uint32_t N, uint32_t K, int per_row,
                              uint8_t *patterns, uint8_t *signs, uint32_t *meta, float *scale) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if (!w || !scale) return fail(ctx, FRX_ERR_SHAPE, "null pointer argument");
  if (!patterns != !signs) return fail(ctx, FRX_ERR_SHAPE, "patterns and signs must both be given or both NULL");
  if (N == 0 || K == 0) return fail(ctx, FRX_ERR_SHAPE, "empty matrix N=%u K=%u", N, K);
  if (K % 4 != 0) return fail(ctx, FRX_ERR_SHAPE, "K=%u must be a multiple of 4 for 2:4", K);
  if (wt != FRX_F32 && wt != FRX_BF16) return fail(ctx, FRX_ERR_UNSUPPORTED, "dtype must be FRX_F32 or FRX_BF16");
  if (N > 0x7FFFFFFFu || K > 0x7FFFFFF0u || (size_t)N * K > ((size_t)1 << 38))
    return fail(ctx, FRX_ERR_SHAPE, "N=%u K=%u too large", N, K);
  const hipError_t e = frx::launch_prune_sparse24(w, wt == FRX_BF16, (int)N, (int)K, per_row != 0, patterns, signs,
                                                  meta, scale, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "2:4 prune launch");
  return FRX_OK;
}

frx_status frx_sparse24_cpu_to_gpu_device(frx_ctx *ctx, const uint8_t *patterns, const uint8_t *signs,
                                          uint32_t N, uint32_t K, uint32_t *meta) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if (!patterns || !signs || !meta) return fail(ctx, FRX_ERR_SHAPE, "null pointer argument");
  if (K % 4 != 0) return fail(ctx, FRX_ERR_SHAPE, "K=%u must be a multiple of 4", K);
  if ((size_t)N * K > (size_t)0x7FFFFFFF * 4) return fail(ctx, FRX_ERR_SHAPE, "matrix too large");
  const hipError_t e = frx::launch_sp24_cpu_to_gpu(patterns, signs, (int)N, (int)K, meta, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "2:4 transcode launch");
  return FRX_OK;
}

// .stm image: magic "STM1", rows, cols, scale (f32), pattern bytes, sign
// bytes, then the two arrays; little-endian (expert_loader.rs:6-16,63-106).
frx_status frx_upload_stm(frx_ctx *ctx, const void *image, size_t len, uint32_t **meta_dev, float **s_dev,
                          uint32_t *N_out, uint32_t *K_out) {
  frx_status st = enter(ctx);
  if (st != FRX_OK) return st;
  if (!image || !meta_dev || !s_dev) return fail(ctx, FRX_ERR_SHAPE, "null pointer argument");
  *meta_dev = nullptr;
  *s_dev = nullptr;
  constexpr size_t HDR = 24;
  if (len < HDR) return fail(ctx, FRX_ERR_SHAPE, "STM image too small: %zu bytes", len);
  const uint8_t *b = reinterpret_cast<const uint8_t *>(image);
  auto u32 = [&](size_t o) { uint32_t v; memcpy(&v, b + o, 4); return v; };
  if (u32(0) != 0x53544D31u) return fail(ctx, FRX_ERR_SHAPE, "invalid STM magic 0x%08X", u32(0));
  const uint32_t rows = u32(4), cols = u32(8);
  float scale;
  memcpy(&scale, b + 12, 4);
  const size_t pb = u32(16), sb = u32(20);
  if (len < HDR + pb + sb) return fail(ctx, FRX_ERR_SHAPE, "STM data truncated: expected %zu bytes, got %zu", HDR + pb + sb, len);
  if (rows == 0 || cols == 0 || cols % 4 != 0)
    return fail(ctx, FRX_ERR_SHAPE, "STM shape rows=%u cols=%u (cols must be a multiple of 4)", rows, cols);
  const size_t ng = (size_t)rows * cols / 4;
  if (pb < (ng + 1) / 2 || sb < (ng + 3) / 4)
    return fail(ctx, FRX_ERR_SHAPE, "STM arrays too short for %u x %u (%zu pattern, %zu sign bytes)", rows, cols, pb, sb);
  const size_t wpr = ((size_t)cols / 4 + 5) / 6;
  void *tmp = nullptr;
  if ((st = dev_alloc(ctx, &tmp, pb + sb, "STM staging allocation")) != FRX_OK) return st;
  if ((st = dev_alloc(ctx, reinterpret_cast<void **>(meta_dev), (size_t)rows * wpr * 4, "2:4 metadata allocation")) !=
      FRX_OK) {
    (void)hipFree(tmp);
    return st;
  }
  hipError_t e = hipMemcpy(tmp, b + HDR, pb + sb, hipMemcpyHostToDevice);
  const uint8_t *dp = reinterpret_cast<const uint8_t *>(tmp);
  if (e == hipSuccess) e = frx::launch_sp24_cpu_to_gpu(dp, dp + pb, (int)rows, (int)cols, *meta_dev, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  (void)hipFree(tmp);
  if (e != hipSuccess) {
    (void)hipFree(*meta_dev);
    *meta_dev = nullptr;
    return hip_fail(ctx, e, "STM upload / transcode");
  }
  if ((st = upload_scales(ctx, nullptr, scale, rows, s_dev)) != FRX_OK) {
    (void)hipFree(*meta_dev);
    *meta_dev = nullptr;
    return st;
  }
  if (N_out) *N_out = rows;
  if (K_out) *K_out = cols;
  return FRX_OK;
}

frx_status frx_free(frx_ctx *ctx, void *dev_ptr) {
  frx_status st = enter(ctx, false);
  if (st != FRX_OK) return st;
  if (!dev_ptr) return FRX_OK;
  const hipError_t e = hipFree(dev_ptr);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipFree");
  return FRX_OK;
}

}  // extern "C"
