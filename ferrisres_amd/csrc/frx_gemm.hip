// frx_gemm.hip — prefill ternary GEMM (dense and 2:4) on gfx950 MFMA.
//
// Replaces ternary_matmul_main / sparse_ternary_matmul_main
// (src/compute/kernels/ternary_matmul.rs:32-75,
// src/compute/kernels/sparse_ternary.rs:54-112) for M > 16 tokens. The WGSL
// kernels launch one thread per output with a 1-D grid, which cannot even be
// dispatched at 2048 x 4096 (over 65,535 workgroups); here each workgroup
// owns a 128 x 128 output tile (see frx_gemm_core.hpp).
#include <type_traits>

#include "frx_gemm2.hpp"
#include "frx_gemm_core.hpp"
#include "frx_internal.hpp"

namespace frx {

// XCD-aware tile order: hardware deals workgroup ids round-robin over the 8
// XCDs (id % 8); renumber so that each XCD receives a contiguous run of tiles
// in (m-tile, n-tile) row-major order (neighbouring N tiles of one M tile
// share that XCD's L2). Bijective for any tile count.
__device__ __forceinline__ void xcd_tile(int &nt, int &mt) {
  const int gx = gridDim.x, total = gx * gridDim.y;
  const int bid = blockIdx.y * gx + blockIdx.x;
  const int q = total / 8, r = total % 8, xcd = bid % 8, kx = bid / 8;
  const int lin = xcd < r ? xcd * (q + 1) + kx : r * (q + 1) + (xcd - r) * q + kx;
  nt = lin % gx;
  mt = lin / gx;
}


template <int BM, int BN, int WM, int WN, int XS, int WF, typename YT>
__global__ __launch_bounds__(WM *WN * 64) void gemm_kernel(
    const uint32_t *__restrict__ W, const float *__restrict__ scale,
    const void *__restrict__ X, YT *__restrict__ Y, int M, int K, int N,
    int wvec, const float *__restrict__ bias) {
  using Core = GemmCore<BM, BN, WM, WN, XS, 1, WF>;
  __shared__ __align__(16) uint32_t lds[Core::LDS_DWORDS];
  int nt, mt;
  xcd_tile(nt, mt);
  const int n0 = nt * BN, m0 = mt * BM;
  constexpr int ES = XS == XS_F32 ? 4 : 2;
  XDesc xd{X, nullptr, nullptr, (long)m0, K, ((K * ES) % 16) == 0};
  const uint32_t *Wm[1] = {W};
  f32x4 acc[1][Core::FN][Core::FM];
  Core::run(lds, xd, min(BM, M - m0), Wm, n0, N, K, wvec, acc);
  // 2*dec(c) encoding for dense codes (frx_device.hpp): halve the scale.
  const float half = 0.5f;
#pragma unroll
  for (int fn = 0; fn < Core::FN; fn++) {
    const int n = n0 + Core::rowoff(fn);
    if (n >= N) continue;
    const int nok = min(4, N - n);
    const f32x4 sc = load_scale4(scale, n, nok) * half;
#pragma unroll
    for (int fm = 0; fm < Core::FM; fm++) {
      const int m = m0 + Core::tok(fm);
      if (m < M) {
        f32x4 v = acc[0][fn][fm] * sc;
        if (bias) v = add_bias4(v, bias, n, N);
        YStore<YT>::store4(Y + (size_t)m * N + n, v, nok);
      }
    }
  }
}

// bf16 activations, K % 64 == 0: the pipelined engine (frx_gemm2.hpp).
template <int BM, int BN, int WM, int WN, int NS, typename YT>
__global__ __launch_bounds__(WM *WN * 64) void gemm2_kernel(
    const uint32_t *__restrict__ W, const float *__restrict__ scale,
    const uint16_t *__restrict__ X, YT *__restrict__ Y, int M, int K, int N,
    const float *__restrict__ bias) {
  using Core = Gemm2<BM, BN, WM, WN, NS, false>;
  extern __shared__ __align__(16) uint32_t lds[];  // Core::LDS_DWORDS
  int nt, mt;
  xcd_tile(nt, mt);
  const int n0 = nt * BN, m0 = mt * BM;
  f32x4 acc[Core::FN][Core::FM];
  const int m_count = min(BM, M - m0), n_count = min(BN, N - n0);
  Core::run(lds, X + (size_t)m0 * K, (uint32_t)m_count * (uint32_t)K * 2u, nullptr, m_count,
            W + (size_t)n0 * (K >> 4), n_count, K, acc);
  Core::template store_tile<YT>(lds, acc, scale, Y, (size_t)N, m0, m_count, n0, n_count, bias);
}

// 2:4 weights (GPU 5-bit layout, or PREP: its prepared form, [N][K/16]
// words), bf16 activations, K % 64 == 0: the pipelined engine on the sparse
// matrix pipe.
// HV = 2: X is an fp32 activation as bf16 hi | lo halves of each row
// ([M][2K]); one K loop of 2K columns multiplies both by the same weights.
template <int BM, int BN, int WM, int WN, int NS, typename YT, bool PREP, int HV>
__global__ __launch_bounds__(WM *WN * 64) void gemm2sp_kernel(
    const uint32_t *__restrict__ meta, const float *__restrict__ scale,
    const uint16_t *__restrict__ X, YT *__restrict__ Y, int M, int K, int N,
    const float *__restrict__ bias) {
  using Core = Gemm2<BM, BN, WM, WN, NS, false>;
  extern __shared__ __align__(16) uint32_t lds[];
  int nt, mt;
  xcd_tile(nt, mt);
  const int n0 = nt * BN, m0 = mt * BM;
  const int wpr = ((K >> 2) + 5) / 6, ldx = HV * K;
  f32x4 acc[Core::FN][Core::FM];
  const int m_count = min(BM, M - m0), n_count = min(BN, N - n0);
  Core::template run_sp<PREP, HV == 2>(lds, X + (size_t)m0 * ldx, (uint32_t)m_count * (uint32_t)ldx * 2u, m_count,
                                       meta + (size_t)n0 * (PREP ? K >> 4 : wpr), n_count, K, wpr, acc, 0,
                                       HV * (K >> 6), ldx);
  Core::template store_tile<YT>(lds, acc, scale, Y, (size_t)N, m0, m_count, n0, n_count, bias);
}

// The prepared form of 2:4 metadata (K % 64 == 0): word j of row n covers
// groups 16 (j / 4) + 4 (j % 4) .. + 3 (sp24p_word), [N][K/16] words.
// One thread per (row, step): the step's 16 groups lie in the 4-word window
// from word floor(16 s / 6) of the row (6 groups of 5 bits per word, bits
// 30-31 belong to no group); its 4 prepared words are one 16-byte store.
__global__ void sp24_prepare_kernel(const uint32_t *__restrict__ meta, u32x4 *__restrict__ out, int N, int K) {
  const uint32_t wpr = ((uint32_t)(K >> 2) + 5u) / 6u, nks = (uint32_t)K >> 6;
  const uint32_t total = (uint32_t)N * nks;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
    const uint32_t n = i / nks, st = i - n * nks;
    const uint32_t q0 = (16u * st) / 6u, r = 16u * st - 6u * q0;
    const uint32_t *row = meta + (size_t)n * wpr;
    uint32_t w[4];
#pragma unroll
    for (int u = 0; u < 4; u++) w[u] = row[min(q0 + (uint32_t)u, wpr - 1u)] & 0x3FFFFFFFu;
    u32x4 o;
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const uint32_t l0 = r + 4u * g, jw = l0 / 6u, sh = 5u * (l0 - 6u * jw);
      const uint32_t lo = jw == 0 ? w[0] : jw == 1 ? w[1] : w[2];
      const uint32_t hi = jw == 0 ? w[1] : jw == 1 ? w[2] : w[3];
      const uint32_t F = (lo >> sh) | (sh > 10u ? hi << (30u - sh) : 0u);
      o[g] = sp24p_word(F);
    }
    out[i] = o;
  }
}

// Split-K dense GEMM for launches with fewer tiles than compute units (17
// to a few hundred tokens): workgroup (nt, mt, s) multiplies K columns
// [s kp, (s + 1) kp) of its tile with the pipelined engine and stores the
// raw fp32 accumulators to part[s][M][N]; gemm_splitk_reduce adds the parts
// in order s = 0, 1, ... and applies the scale (and bias).
// HV = 2: X rows are an fp32 activation as bf16 hi | lo halves ([M][2K]);
// parts 0 .. S/2 - 1 run over the hi half and S/2 .. S - 1 over the lo half,
// each against the same weight columns.
template <int BM, int BN, int WM, int WN, int NS, int HV>
__global__ __launch_bounds__(WM *WN * 64) void gemm2_splitk_kernel(
    const uint32_t *__restrict__ W, const uint16_t *__restrict__ X, float *__restrict__ part, int M, int K, int N,
    int kp) {
  using Core = Gemm2<BM, BN, WM, WN, NS, false>;
  extern __shared__ __align__(16) uint32_t lds[];
  const int nt = blockIdx.x, mt = blockIdx.y, s = blockIdx.z;
  const int sh = (int)gridDim.z / HV, half = s / sh, j = s - half * sh;
  const int n0 = nt * BN, m0 = mt * BM, k0 = j * kp, kl = min(kp, K - k0);
  const int ldx = HV * K;  // X row stride (elements)
  f32x4 acc[Core::FN][Core::FM];
  const int m_count = min(BM, M - m0), n_count = min(BN, N - n0);
  // X from row m0, column half K + k0; W from row n0, word k0 / 16 (row
  // stride K / 16 words): the engine's K loop runs kl columns
  const uint32_t xo = (uint32_t)(half * K + k0);
  Core::run(lds, X + (size_t)m0 * ldx + xo, (uint32_t)m_count * (uint32_t)ldx * 2u - xo * 2u, nullptr, m_count,
            W + (size_t)n0 * (K >> 4) + (k0 >> 4), n_count, kl, acc, nullptr, K, ldx);
  Core::template store_tile<float, true>(lds, acc, nullptr, part + (size_t)s * M * N, (size_t)N, m0, m_count, n0,
                                         n_count, nullptr);
}

// The same split over 2:4 weights (GPU 5-bit layout, wpr words per row):
// part s multiplies steps [s sp, (s + 1) sp) on the sparse matrix pipe.
// HV = 2: X rows are bf16 hi | lo halves ([M][2K]); parts 0 .. S/2 - 1 run
// over the hi half and S/2 .. S - 1 over the lo half.
template <int BM, int BN, int WM, int WN, int NS, bool PREP, int HV>
__global__ __launch_bounds__(WM *WN * 64) void gemm2sp_splitk_kernel(
    const uint32_t *__restrict__ meta, const uint16_t *__restrict__ X, float *__restrict__ part, int M, int K, int N,
    int sp) {
  using Core = Gemm2<BM, BN, WM, WN, NS, false>;
  extern __shared__ __align__(16) uint32_t lds[];
  const int nt = blockIdx.x, mt = blockIdx.y, s = blockIdx.z;
  const int sh = (int)gridDim.z / HV, half = s / sh, j = s - half * sh;
  const int n0 = nt * BN, m0 = mt * BM;
  const int nks = K >> 6, s0 = j * sp, ns = min(sp, nks - s0);
  const int wpr = ((K >> 2) + 5) / 6, ldx = HV * K;
  f32x4 acc[Core::FN][Core::FM];
  const int m_count = min(BM, M - m0), n_count = min(BN, N - n0);
  const uint32_t xo = (uint32_t)(half * K);  // the half's first column
  Core::template run_sp<PREP>(lds, X + (size_t)m0 * ldx + xo, (uint32_t)m_count * (uint32_t)ldx * 2u - xo * 2u,
                              m_count, meta + (size_t)n0 * (PREP ? K >> 4 : wpr), n_count, K, wpr, acc, s0, ns,
                              ldx);
  Core::template store_tile<float, true>(lds, acc, nullptr, part + (size_t)s * M * N, (size_t)N, m0, m_count, n0,
                                         n_count, nullptr);
}

// Whole-K GEMM over an fp32 activation stored as bf16 hi | lo halves of
// each row ([M][2K]): one pass of 2K columns in which the weight columns
// wrap at K (the engine's wk), i.e. acc = W x_hi + W x_lo.
template <int BM, int BN, int WM, int WN, int NS, typename YT>
__global__ __launch_bounds__(WM *WN * 64) void gemm2_planes_kernel(
    const uint32_t *__restrict__ W, const float *__restrict__ scale, const uint16_t *__restrict__ X,
    YT *__restrict__ Y, int M, int K, int N, const float *__restrict__ bias) {
  using Core = Gemm2<BM, BN, WM, WN, NS, false>;
  extern __shared__ __align__(16) uint32_t lds[];
  int nt, mt;
  xcd_tile(nt, mt);
  const int n0 = nt * BN, m0 = mt * BM;
  f32x4 acc[Core::FN][Core::FM];
  const int m_count = min(BM, M - m0), n_count = min(BN, N - n0);
  Core::run(lds, X + (size_t)m0 * 2 * K, (uint32_t)m_count * (uint32_t)K * 4u, nullptr, m_count,
            W + (size_t)n0 * (K >> 4), n_count, 2 * K, acc, nullptr, K, 2 * K);
  Core::template store_tile<YT>(lds, acc, scale, Y, (size_t)N, m0, m_count, n0, n_count, bias);
}

// x [M][K] f32 -> x2 [M][2K] bf16: hi = bf16(x), lo = bf16(x - hi) (split2_bf16,
// |x - hi - lo| <= 2^-17 |x|), two values per thread.
__global__ __launch_bounds__(256) void to_planes_kernel(const float *__restrict__ x, uint16_t *__restrict__ x2,
                                                        int M, int K) {
  const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 2;  // K even
  if (i >= (size_t)M * K) return;
  const size_t m = i / (size_t)K, k = i - m * (size_t)K;
  const float2 v = *reinterpret_cast<const float2 *>(x + i);
  uint32_t hi, lo;
  split2_bf16(v.x, v.y, hi, lo);
  *reinterpret_cast<uint32_t *>(x2 + m * 2 * K + k) = hi;
  *reinterpret_cast<uint32_t *>(x2 + m * 2 * K + K + k) = lo;
}

hipError_t launch_to_planes(const float *x, uint16_t *x2, int M, int K, hipStream_t stream) {
  const size_t pairs = (size_t)M * K / 2;
  hipLaunchKernelGGL(to_planes_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, stream, x, x2, M, K);
  return hipGetLastError();
}

template <typename YT>
__global__ __launch_bounds__(256) void gemm_splitk_reduce(const float *__restrict__ part, int S, int M, int N,
                                                          const float *__restrict__ scale,
                                                          const float *__restrict__ bias, YT *__restrict__ Y) {
  const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;  // N % 4 == 0
  const size_t MN = (size_t)M * N;
  if (i >= MN) return;
  f32x4 sum = *reinterpret_cast<const f32x4 *>(part + i);
  // eight parts' loads in flight at a time, added in part order
  for (int s0 = 1; s0 < S; s0 += 8) {
    f32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; u++)
      if (s0 + u < S) v[u] = *reinterpret_cast<const f32x4 *>(part + (size_t)(s0 + u) * MN + i);
#pragma unroll
    for (int u = 0; u < 8; u++)
      if (s0 + u < S) sum = sum + v[u];
  }
  const int n = (int)(i % (size_t)N);
  f32x4 o;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    o[e] = sum[e] * (0.5f * scale[n + e]);  // 0.5 undoes the 2*dec(c) encoding
    if (bias) o[e] = add_bias(o[e], bias[n + e]);
  }
  YStore<YT>::store4(Y + i, o, 4);
}

constexpr int GEMM_SK_BM = 64;

// The split: 64-token tiles; when they leave at least half of the compute
// units idle, S K parts (whole 64-column steps) bring the grid to about two
// workgroups per CU. (With more tiles the fp32 parts cost more than the
// idle units: 11008 x 4096 at 256 tokens, 172 tiles, 40.2 us whole against
// 46.9 us in three parts; 4096 x 11008 at 512 tokens, 128 tiles, 91.8 us
// whole against 54.5 us in four.)
bool gemm_splitk_plan(int M, int K, int N, int cus, int *S, int *kp, int halves) {
  if (M <= 16 || K % 64 != 0 || N % 4 != 0) return false;
  const long tiles = (long)((M + GEMM_SK_BM - 1) / GEMM_SK_BM) * ((N + 255) / 256);
  if (2 * tiles > cus) return false;
  const int nks = K / 64;
  // at least 8 steps of 64 columns per part: shorter parts are mostly the
  // pipeline's fill and drain, and their fp32 partials outweigh the weights
  int s = (int)std::min<long>((2L * cus + tiles * halves - 1) / (tiles * halves), nks / 8);
  if (s < 1 || halves * s < 2) return false;
  const int steps = (nks + s - 1) / s;
  *kp = steps * 64;
  *S = halves * ((K + *kp - 1) / *kp);
  return true;
}


size_t gemm_splitk_workspace_bytes(int M, int N, int S) { return (size_t)S * M * N * 4; }

constexpr int GEMM_SPSK_BM = 64;  // 4 token blocks, the fewest the sparse schedule takes

// 2:4 weights, 1 token and more, where 64-token tiles leave at least half of
// the compute units idle, or at rows of 16384 codes and more any of them
// (there a second workgroup per CU outweighs the partials' traffic: 8192 x
// 28672 at 512 tokens 283 -> 242 us; at 11008 x 4096, 256 tokens, 47 ->
// 53 us): parts of at least 8 steps (4 for bf16 decode), about two
// workgroups per CU.
bool gemm_sp_splitk_plan(int M, int K, int N, int cus, int *S, int *sp, int halves) {
  if (M < 1 || K % 64 != 0 || N % 4 != 0) return false;
  const long tiles = (long)((M + GEMM_SPSK_BM - 1) / GEMM_SPSK_BM) * ((N + 255) / 256);
  if (2 * tiles > cus && (tiles > cus || K < 16384)) return false;
  const int nks = K / 64;
  // bf16 decode (16 tokens at most): parts of 4 steps (11008 x 4096 at one
  // token 18.2 -> 16.6 us; the two halves of f32 tokens keep 8)
  const int mins = M <= 16 && halves == 1 ? 4 : 8;
  const int s = (int)std::min<long>((2L * cus + tiles * halves - 1) / (tiles * halves), nks / mins);
  if (s < 1 || halves * s < 2) return false;
  *sp = (nks + s - 1) / s;
  *S = halves * ((nks + *sp - 1) / *sp);
  return true;
}

template <bool PREP, int HV>
static hipError_t launch_gemm2sp_parts(const uint32_t *meta, const void *x, int M, int K, int N, int S, int sp,
                                       float *part, hipStream_t stream) {
  constexpr int BM = GEMM_SPSK_BM, BN = 256, WM = 1, WN = 4, NS = 4;
  using Core = Gemm2<BM, BN, WM, WN, NS, false>;
  constexpr int lds = Core::LDS_DWORDS * 4;
  static std::atomic<uint64_t> done;
  hipError_t e =
      opt_in_lds(reinterpret_cast<const void *>(&gemm2sp_splitk_kernel<BM, BN, WM, WN, NS, PREP, HV>), lds, done);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((gemm2sp_splitk_kernel<BM, BN, WM, WN, NS, PREP, HV>),
                     dim3((N + BN - 1) / BN, (M + BM - 1) / BM, S), dim3(WM * WN * 64), lds, stream, meta,
                     reinterpret_cast<const uint16_t *>(x), part, M, K, N, sp);
  return hipGetLastError();
}

// ---- 2:4 decode GEMV over the 5-bit layout (1-4 tokens, VALU) ----------------
// The metadata is read once at 1.25 bits per weight. A workgroup owns 256
// rows (one per lane) and a chunk of W metadata words of each row (6 groups
// of 4 columns per word). It first tabulates, for each group of the chunk
// and each of the 32 five-bit codes, the value the group adds:
// 2 (s0 x[4g + p0] + s1 x[4g + p1]) (pattern > 5 read as 5, sign bits 3 and
// 4; twice the sum, the 2 dec(c) scale of the other kernels). A code then
// costs one LDS read and one add per token; the lanes of a wave read the same
// group's 32 entries at a time, one bank each. The chunks' sums go to
// part[chunk][M][N] and are added in chunk order: by the last chunk of each
// row block to arrive (up to SPV_FUSED_MAX chunks), else by
// gemm_splitk_reduce in a second launch.
template <int MT>
__host__ __device__ constexpr int spv_words() { return 16; }  // LDS <= 54 KB at 4 tokens
// Most chunks that the last-arriving workgroup adds itself, all loads in
// flight at once; above, a second launch does (4096 x 11008, 29 chunks:
// 12.9 against 10.8 us with 8 loads in flight, 11.5 against 10.4 with all
// 29; a limit of 32 also slowed the shapes of 11 chunks, 9.3 -> 9.5 us).
constexpr int SPV_FUSED_MAX = 12;

template <typename XT, int MT, typename YT, bool XMAP>
__global__ __launch_bounds__(256) void sp24_gemv_kernel(const uint32_t *__restrict__ meta, const XT *__restrict__ x,
                                                        float *__restrict__ part, unsigned *__restrict__ counters,
                                                        const float *__restrict__ scale, YT *__restrict__ Y, int M,
                                                        int N, int K, int S) {
  constexpr int W = spv_words<MT>(), G = 6 * W;
  static_assert(W == 16, "one metadata load per 16 lanes and row");
  __shared__ float xs[MT][4 * G];
  __shared__ float tab[MT][G * 32];
  __shared__ uint32_t mw[256][W + 1];  // the block's rows' words (padded: conflict-free row reads)
  // XMAP: a one-dimensional grid, workgroup i dispatched to XCD i % 8, and
  // every chunk of a row block on the XCD of that block (rb % 8), so the
  // 128-byte lines that neighbouring chunks of a row share are fetched into
  // one L2 (with the chunks of a block spread over the XCDs, 11008 x 4096
  // fetched 3x its metadata bytes, 1.07x so); slots past the row blocks exit
  // at once. Otherwise grid (row blocks, chunks).
  const int nrb = (N + 255) >> 8, slot = (int)(blockIdx.x >> 3);
  const int rb = XMAP ? (slot / S) * 8 + (int)(blockIdx.x & 7) : (int)blockIdx.x;
  const int chunk = XMAP ? slot % S : (int)blockIdx.y;
  if (XMAP && rb >= nrb) return;  // whole workgroup
  const int wpr = ((K >> 2) + 5) / 6;
  const int w0 = chunk * W, nw = min(W, wpr - w0);
  const int c0 = 24 * w0;  // first column of the chunk
  // the chunk's activations first, then its metadata: vector loads complete
  // in issue order, so the tabulation waits only for the activations and
  // runs while the metadata streams in (11008 x 4096, one token: the table
  // was ready only after all 16 KB of a workgroup's metadata had landed)
  constexpr int XPT = (MT * 4 * G + 255) / 256;  // activations per thread
  float xv[XPT];
#pragma unroll
  for (int q = 0; q < XPT; q++) {
    const int i = (int)threadIdx.x + 256 * q, m = i / (4 * G), c = i - m * 4 * G;
    xv[q] = 0.f;
    if (i < MT * 4 * G && m < M && c0 + c < K) {
      if constexpr (sizeof(XT) == 2) xv[q] = __uint_as_float((uint32_t)x[(size_t)m * K + c0 + c] << 16);
      else xv[q] = x[(size_t)m * K + c0 + c];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // 16-byte loads (dword-aligned: rows are wpr words long): load i of thread
  // t is words 4 (t % 4) .. + 3 of row 64 i + t / 4, 64 contiguous bytes per
  // row and 16 rows per wave instruction; words past the row's end belong to
  // the next row and are cleared, past the matrix the descriptor reads zeros
  const int r0 = rb * 256, lq = threadIdx.x & 3, lr = threadIdx.x >> 2;
  const __amdgpu_buffer_rsrc_t mr = buffer_rsrc(meta, (uint32_t)N * (uint32_t)wpr * 4u);
  u32x4 wl[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = min(r0 + 64 * i + lr, N - 1);
    wl[i] = __builtin_amdgcn_raw_buffer_load_b128(mr, ((uint32_t)r * (uint32_t)wpr + (uint32_t)(w0 + 4 * lq)) * 4u, 0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int q = 0; q < XPT; q++) {
    const int i = (int)threadIdx.x + 256 * q, m = i / (4 * G), c = i - m * 4 * G;
    if (i < MT * 4 * G) xs[m][c] = xv[q];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < MT * G * 32; i += 256) {
    const int m = i / (G * 32), r = i - m * G * 32, gl = r >> 5, code = r & 31;
    const uint32_t nib = __builtin_amdgcn_ubfe(0xEEED9C84u, (uint32_t)(code & 7) << 2, 4);
    const float a = xs[m][4 * gl + (nib & 3)], b = xs[m][4 * gl + (nib >> 2)];
    tab[m][r] = 2.0f * ((code & 8 ? -a : a) + (code & 16 ? -b : b));
  }
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int k = 0; k < 4; k++) mw[64 * i + lr][4 * lq + k] = 4 * lq + k < nw ? wl[i][k] : 0u;
  __syncthreads();
  const int row = r0 + (int)threadIdx.x;
  uint32_t wq[W];
#pragma unroll
  for (int w = 0; w < W; w++) wq[w] = mw[threadIdx.x][w];
  // two chains per token (even and odd words), added at the end
  float acc[MT][2];
#pragma unroll
  for (int m = 0; m < MT; m++) acc[m][0] = acc[m][1] = 0.f;
#pragma unroll
  for (int w = 0; w < W; w++) {
    if (w >= nw) break;
#pragma unroll
    for (int q = 0; q < 6; q++) {
      const uint32_t code = (wq[w] >> (5 * q)) & 31u;
#pragma unroll
      for (int m = 0; m < MT; m++) acc[m][w & 1] += tab[m][(w * 6 + q) * 32 + code];
    }
  }
  // the chunk's sums, stored device-coherent (the workgroup that adds the
  // chunks may run on another XCD); the last chunk of this row block to
  // arrive adds them in chunk order (a per-block counter, reset by that
  // workgroup for the next launch)
  constexpr int SC1 = 16;  // cache policy: performed at the point of coherence of all XCDs
  constexpr uint32_t OOB = 0x80000000u;
  const __amdgpu_buffer_rsrc_t pr = buffer_rsrc(part, (uint32_t)S * (uint32_t)M * (uint32_t)N * 4u);
#pragma unroll
  for (int m = 0; m < MT; m++) {
    const uint32_t off =
        (m < M && row < N) ? (((uint32_t)chunk * (uint32_t)M + (uint32_t)m) * (uint32_t)N + (uint32_t)row) * 4u : OOB;
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[m][0] + acc[m][1]), pr, off, 0, SC1);
  }
  if (!counters) return;  // a separate launch adds the chunks
  __shared__ int last;
  wait_vmcnt<0>();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned old = __hip_atomic_fetch_add(counters + rb, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old == (unsigned)S - 1u;
    if (last) __hip_atomic_store(counters + rb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last || row >= N) return;
  const float sc = 0.5f * scale[row];  // 0.5 undoes the 2 dec(c) scale of the table
#pragma unroll
  for (int m = 0; m < MT; m++) {
    if (m >= M) break;
    // every chunk's partial in flight at once (the fused path takes up to
    // SPV_FUSED_MAX chunks): one round trip to the point of coherence
    float sum = 0.f;
    for (int c0 = 0; c0 < S; c0 += SPV_FUSED_MAX) {
      float v[SPV_FUSED_MAX];
#pragma unroll
      for (int k = 0; k < SPV_FUSED_MAX; k++) {
        const uint32_t off = c0 + k < S ? (((uint32_t)(c0 + k) * (uint32_t)M + (uint32_t)m) * (uint32_t)N +
                                           (uint32_t)row) * 4u
                                        : OOB;
        v[k] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(pr, off, 0, SC1));
      }
#pragma unroll
      for (int k = 0; k < SPV_FUSED_MAX; k++)
        if (c0 + k < S) sum = (c0 + k == 0) ? v[k] : sum + v[k];
    }
    const float o = sum * sc;
    if constexpr (sizeof(YT) == 4) Y[(size_t)m * N + row] = o;
    else Y[(size_t)m * N + row] = (uint16_t)bf16_rne(o);
  }
}

// 1-2 tokens, or 3-4 fp32 tokens over matrices of 32 M codes and more with
// rows up to 16384 (bf16 ones are faster on the sparse pipe, split over K:
// 16.8 against about 21 us at 11008 x 4096; fp32 ones there run twice, as hi
// and lo: 28 against 21.5 us; at 4096 x 4096 and 8192 x 28672 the split
// stays ahead: 16.3 / 68 against 17.3 / 84 us)
bool sp24_gemv_plan(int M, int K, int N, int xt_bf16, int *S) {
  if (M < 1 || K % 4 != 0 || N % 4 != 0 || (N + 255) / 256 > GEMV_SK_MAX_TILES) return false;
  if (M > 2 && (xt_bf16 || M > 4 || K > 16384 || (long)N * K < (1L << 25))) return false;
  const int wpr = ((K >> 2) + 5) / 6, w = M <= 2 ? spv_words<2>() : spv_words<4>();
  if ((long)N * wpr * 4 >= (1L << 32)) return false;  // the metadata's buffer range
  *S = (wpr + w - 1) / w;
  return true;
}

hipError_t launch_sp24_gemv(const uint32_t *meta, const float *scale, const void *x, int xt_bf16, void *y,
                            int yt_bf16, int M, int K, int N, int S, float *part, unsigned *counters,
                            hipStream_t stream) {
  // the XCD-grouped order for 1-2 tokens where the plain order spreads a row
  // block's chunks (with nrb % 8 == 0 it already keeps them on one XCD); at
  // 3-4 tokens (about 66 KB of LDS, two workgroups per CU) grouping 43 row
  // blocks put 66 workgroups on the 64 slots of some XCDs (11008 x 4096, 4
  // f32 tokens: 20.5 -> 28.2 us)
  const int nrb = (N + 255) / 256;
  const bool xmap = M <= 2 && nrb % 8 != 0;
  const dim3 g = xmap ? dim3(8 * S * ((nrb + 7) / 8)) : dim3(nrb, S);
  auto run = [&](auto xp, auto yp) {
    using XT = std::remove_const_t<std::remove_pointer_t<decltype(xp)>>;
    using YT = std::remove_pointer_t<decltype(yp)>;
    if (M == 1 && xmap)
      hipLaunchKernelGGL((sp24_gemv_kernel<XT, 1, YT, true>), g, dim3(256), 0, stream, meta, xp, part, counters, scale,
                         yp, M, N, K, S);
    else if (M == 1)
      hipLaunchKernelGGL((sp24_gemv_kernel<XT, 1, YT, false>), g, dim3(256), 0, stream, meta, xp, part, counters,
                         scale, yp, M, N, K, S);
    else if (M == 2 && xmap)
      hipLaunchKernelGGL((sp24_gemv_kernel<XT, 2, YT, true>), g, dim3(256), 0, stream, meta, xp, part, counters, scale,
                         yp, M, N, K, S);
    else if (M == 2)
      hipLaunchKernelGGL((sp24_gemv_kernel<XT, 2, YT, false>), g, dim3(256), 0, stream, meta, xp, part, counters,
                         scale, yp, M, N, K, S);
    else
      hipLaunchKernelGGL((sp24_gemv_kernel<XT, 4, YT, false>), g, dim3(256), 0, stream, meta, xp, part, counters,
                         scale, yp, M, N, K, S);
  };
  auto runx = [&](auto yp) {
    if (xt_bf16) run(reinterpret_cast<const uint16_t *>(x), yp);
    else run(reinterpret_cast<const float *>(x), yp);
  };
  const bool fused = S <= SPV_FUSED_MAX;
  if (!fused) counters = nullptr;
  if (yt_bf16) runx(reinterpret_cast<uint16_t *>(y));
  else runx(reinterpret_cast<float *>(y));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || fused) return e;
  const size_t quads = (size_t)M * N / 4;
  const dim3 gr((unsigned)((quads + 255) / 256));
  if (yt_bf16)
    hipLaunchKernelGGL(gemm_splitk_reduce<uint16_t>, gr, dim3(256), 0, stream, part, S, M, N, scale, nullptr,
                       reinterpret_cast<uint16_t *>(y));
  else
    hipLaunchKernelGGL(gemm_splitk_reduce<float>, gr, dim3(256), 0, stream, part, S, M, N, scale, nullptr,
                       reinterpret_cast<float *>(y));
  return hipGetLastError();
}

hipError_t launch_sp24_prepare(const uint32_t *meta, uint32_t *out, int N, int K, hipStream_t stream) {
  const size_t total = (size_t)N * (K >> 6);
  const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 65536);
  hipLaunchKernelGGL(sp24_prepare_kernel, dim3(blocks), dim3(256), 0, stream, meta, reinterpret_cast<u32x4 *>(out),
                     N, K);
  return hipGetLastError();
}

hipError_t launch_gemm_sp_splitk(const uint32_t *meta, const float *scale, const void *x, void *y, int yt_bf16, int M,
                                 int K, int N, int S, int sp, float *part, hipStream_t stream, const float *bias,
                                 int prepared, int halves) {
  hipError_t e;
  if (halves == 2)
    e = prepared ? launch_gemm2sp_parts<true, 2>(meta, x, M, K, N, S, sp, part, stream)
                 : launch_gemm2sp_parts<false, 2>(meta, x, M, K, N, S, sp, part, stream);
  else
    e = prepared ? launch_gemm2sp_parts<true, 1>(meta, x, M, K, N, S, sp, part, stream)
                 : launch_gemm2sp_parts<false, 1>(meta, x, M, K, N, S, sp, part, stream);
  if (e != hipSuccess) return e;
  const size_t quads = (size_t)M * N / 4;
  const dim3 g((unsigned)((quads + 255) / 256));
  if (yt_bf16)
    hipLaunchKernelGGL(gemm_splitk_reduce<uint16_t>, g, dim3(256), 0, stream, part, S, M, N, scale, bias,
                       reinterpret_cast<uint16_t *>(y));
  else
    hipLaunchKernelGGL(gemm_splitk_reduce<float>, g, dim3(256), 0, stream, part, S, M, N, scale, bias,
                       reinterpret_cast<float *>(y));
  return hipGetLastError();
}

hipError_t launch_gemm_splitk(const uint32_t *w, const float *scale, const void *x, void *y, int yt_bf16, int M, int K,
                              int N, int S, int kp, float *part, hipStream_t stream, const float *bias, int halves) {
  constexpr int BM = GEMM_SK_BM, BN = 256, WM = 1, WN = 4, NS = 4;
  using Core = Gemm2<BM, BN, WM, WN, NS, false>;
  constexpr int lds = Core::LDS_DWORDS * 4;
  const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM, S);
  hipError_t e;
  if (halves == 2) {
    static std::atomic<uint64_t> done2;
    e = opt_in_lds(reinterpret_cast<const void *>(&gemm2_splitk_kernel<BM, BN, WM, WN, NS, 2>), lds, done2);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((gemm2_splitk_kernel<BM, BN, WM, WN, NS, 2>), grid, dim3(WM * WN * 64), lds, stream, w,
                       reinterpret_cast<const uint16_t *>(x), part, M, K, N, kp);
  } else {
    static std::atomic<uint64_t> done;
    e = opt_in_lds(reinterpret_cast<const void *>(&gemm2_splitk_kernel<BM, BN, WM, WN, NS, 1>), lds, done);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((gemm2_splitk_kernel<BM, BN, WM, WN, NS, 1>), grid, dim3(WM * WN * 64), lds, stream, w,
                       reinterpret_cast<const uint16_t *>(x), part, M, K, N, kp);
  }
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const size_t quads = (size_t)M * N / 4;
  const dim3 g((unsigned)((quads + 255) / 256));
  if (yt_bf16)
    hipLaunchKernelGGL(gemm_splitk_reduce<uint16_t>, g, dim3(256), 0, stream, part, S, M, N, scale, bias,
                       reinterpret_cast<uint16_t *>(y));
  else
    hipLaunchKernelGGL(gemm_splitk_reduce<float>, g, dim3(256), 0, stream, part, S, M, N, scale, bias,
                       reinterpret_cast<float *>(y));
  return hipGetLastError();
}

// Pipeline stages of the K loop.
constexpr int GEMM2_NS = 4;
// One wave per SIMD, each over the tile's tokens x 64 rows. Waves split
// 2 x 2 over tokens and rows instead (half the activation reads from LDS,
// twice each wave's weight decode) measured slower at 2048 x 4096 x 4096 /
// 11008: dense 76 / 184 us against 65 / 175 us, 2:4 87 / 195 us against
// 71 / 157 us.
constexpr int GEMM2_WM = 1, GEMM2_WN = 4;
// Tokens per tile of the 2:4 launches with at least one 128-token tile per
// compute unit (64 measured slower there: 83 / 203 us against 71 / 158 us at
// 2048 x 4096 x 4096 / 11008).
constexpr int GEMM2SP_BM = 128;

// Compute units of the current device (queried once).
static int device_cus() {
  static std::atomic<int> cus{0};
  int c = cus.load(std::memory_order_relaxed);
  if (c == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
      c = 256;
    cus.store(c, std::memory_order_relaxed);
  }
  return c;
}

// The planes GEMM over x2 = [M][2K] bf16 (an fp32 activation as hi | lo).
hipError_t launch_gemm_planes(const uint32_t *w, const float *scale, const uint16_t *x2, void *y, int yt_bf16, int M,
                              int K, int N, hipStream_t stream, const float *bias) {
  constexpr int BN = 256, WM = GEMM2_WM, WN = GEMM2_WN, NS = GEMM2_NS;
  const long tiles128 = (long)((M + 127) / 128) * ((N + BN - 1) / BN);
  const bool small = tiles128 <= device_cus();
#define FRX_PLANES(BM, YT)                                                                                    \
  {                                                                                                           \
    using Core = Gemm2<BM, BN, WM, WN, NS, false>;                                                            \
    constexpr int lds = Core::LDS_DWORDS * 4;                                                                 \
    static std::atomic<uint64_t> done;                                                                        \
    const hipError_t e =                                                                                      \
        opt_in_lds(reinterpret_cast<const void *>(&gemm2_planes_kernel<BM, BN, WM, WN, NS, YT>), lds, done);  \
    if (e != hipSuccess) return e;                                                                            \
    hipLaunchKernelGGL((gemm2_planes_kernel<BM, BN, WM, WN, NS, YT>), dim3((N + BN - 1) / BN, (M + BM - 1) / BM), \
                       dim3(WM * WN * 64), lds, stream, w, scale, x2, reinterpret_cast<YT *>(y), M, K, N, bias);   \
    return hipGetLastError();                                                                                 \
  }
  if (small) {
    if (yt_bf16) FRX_PLANES(64, uint16_t)
    FRX_PLANES(64, float)
  }
  if (yt_bf16) FRX_PLANES(128, uint16_t)
  FRX_PLANES(128, float)
#undef FRX_PLANES
}

template <int BM, typename YT, int BN = 256>
static hipError_t launch_gemm2_bm(const uint32_t *w, const float *scale, const void *x, void *y,
                                  int M, int K, int N, hipStream_t stream, const float *bias) {
  constexpr int WM = GEMM2_WM, WN = GEMM2_WN, NS = GEMM2_NS;
  using Core = Gemm2<BM, BN, WM, WN, NS, false>;
  constexpr int lds = Core::LDS_DWORDS * 4;
  static std::atomic<uint64_t> done;
  const hipError_t e =
      opt_in_lds(reinterpret_cast<const void *>(&gemm2_kernel<BM, BN, WM, WN, NS, YT>), lds, done);
  if (e != hipSuccess) return e;
  dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
  hipLaunchKernelGGL((gemm2_kernel<BM, BN, WM, WN, NS, YT>), grid, dim3(WM * WN * 64), lds, stream, w,
                     scale, reinterpret_cast<const uint16_t *>(x), reinterpret_cast<YT *>(y), M, K, N, bias);
  return hipGetLastError();
}

// Dense tiles: 128 tokens x 256 rows, or 64 x 256 when the 128-token grid
// would give each CU at most one workgroup: the 64-token tile (48 KB of LDS,
// 64 accumulation registers per lane) runs two workgroups per CU, so each
// SIMD interleaves two waves (2048 x 4096 x 4096: 64 us against 70 us; at
// N = 11008 the 128-token tile stays ahead, 175 against 198 us). A 128 x 128
// tile there (half the decode per MFMA, twice the activation reads from LDS)
// measured 66.1 against 63.8 us.
template <typename YT>
static hipError_t launch_gemm2_t(const uint32_t *w, const float *scale, const void *x, void *y,
                                 int M, int K, int N, hipStream_t stream, const float *bias) {
  const long tiles128 = (long)((M + 127) / 128) * ((N + 255) / 256);
  if (tiles128 <= device_cus()) return launch_gemm2_bm<64, YT>(w, scale, x, y, M, K, N, stream, bias);
  return launch_gemm2_bm<128, YT>(w, scale, x, y, M, K, N, stream, bias);
}

template <int BM, typename YT, bool PREP, int HV>
static hipError_t launch_gemm2sp_bm(const uint32_t *meta, const float *scale, const void *x, void *y,
                                    int M, int K, int N, hipStream_t stream, const float *bias) {
  constexpr int BN = 256, WM = GEMM2_WM, WN = GEMM2_WN, NS = GEMM2_NS;
  using Core = Gemm2<BM, BN, WM, WN, NS, false>;
  constexpr int lds = Core::LDS_DWORDS * 4;
  static std::atomic<uint64_t> done;
  const hipError_t e =
      opt_in_lds(reinterpret_cast<const void *>(&gemm2sp_kernel<BM, BN, WM, WN, NS, YT, PREP, HV>), lds, done);
  if (e != hipSuccess) return e;
  dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
  hipLaunchKernelGGL((gemm2sp_kernel<BM, BN, WM, WN, NS, YT, PREP, HV>), grid, dim3(WM * WN * 64), lds, stream,
                     meta, scale, reinterpret_cast<const uint16_t *>(x), reinterpret_cast<YT *>(y), M, K, N, bias);
  return hipGetLastError();
}

// 64-token tiles while even those do not outnumber the compute units (at
// 11008 x 4096, 512 tokens: 344 tiles of 64 took 72 us, 172 of 128 64 us).
template <typename YT, bool PREP, int HV = 1>
static hipError_t launch_gemm2sp_t(const uint32_t *meta, const float *scale, const void *x, void *y,
                                   int M, int K, int N, hipStream_t stream, const float *bias) {
  const long tiles128 = (long)((M + GEMM2SP_BM - 1) / GEMM2SP_BM) * ((N + 255) / 256);
  if (2 * tiles128 <= device_cus())
    return launch_gemm2sp_bm<64, YT, PREP, HV>(meta, scale, x, y, M, K, N, stream, bias);
  return launch_gemm2sp_bm<GEMM2SP_BM, YT, PREP, HV>(meta, scale, x, y, M, K, N, stream, bias);
}

hipError_t launch_gemm_sp_prepared(const uint32_t *prep, const float *scale, const void *x, void *y, int yt_bf16,
                                   int M, int K, int N, hipStream_t stream, const float *bias) {
  if (yt_bf16) return launch_gemm2sp_t<uint16_t, true>(prep, scale, x, y, M, K, N, stream, bias);
  return launch_gemm2sp_t<float, true>(prep, scale, x, y, M, K, N, stream, bias);
}

hipError_t launch_gemm_sp_planes(const uint32_t *meta, int prepared, const float *scale, const uint16_t *x2, void *y,
                                 int yt_bf16, int M, int K, int N, hipStream_t stream) {
  if (prepared) {
    if (yt_bf16) return launch_gemm2sp_t<uint16_t, true, 2>(meta, scale, x2, y, M, K, N, stream, nullptr);
    return launch_gemm2sp_t<float, true, 2>(meta, scale, x2, y, M, K, N, stream, nullptr);
  }
  if (yt_bf16) return launch_gemm2sp_t<uint16_t, false, 2>(meta, scale, x2, y, M, K, N, stream, nullptr);
  return launch_gemm2sp_t<float, false, 2>(meta, scale, x2, y, M, K, N, stream, nullptr);
}

template <int XS, int WF, typename YT>
static hipError_t launch_gemm_t(const uint32_t *w, const float *scale,
                                const void *x, void *y, int M, int K, int N,
                                hipStream_t stream, const float *bias) {
  constexpr int BM = 128, BN = 128, WM = 2, WN = 2;
  const int wvec = ((K >> 4) % 4 == 0) && ((reinterpret_cast<uintptr_t>(w) & 15) == 0);
  dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
  hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, XS, WF, YT>), grid,
                     dim3(WM * WN * 64), 0, stream, w, scale, x,
                     reinterpret_cast<YT *>(y), M, K, N, wvec, bias);
  return hipGetLastError();
}

template <int WF>
static hipError_t launch_gemm_wf(const uint32_t *w, const float *scale,
                                 const void *x, int xt_bf16, void *y,
                                 int yt_bf16, int M, int K, int N,
                                 hipStream_t stream, const float *bias) {
  if (xt_bf16) {
    if (yt_bf16) return launch_gemm_t<XS_BF16, WF, uint16_t>(w, scale, x, y, M, K, N, stream, bias);
    return launch_gemm_t<XS_BF16, WF, float>(w, scale, x, y, M, K, N, stream, bias);
  }
  if (yt_bf16) return launch_gemm_t<XS_F32, WF, uint16_t>(w, scale, x, y, M, K, N, stream, bias);
  return launch_gemm_t<XS_F32, WF, float>(w, scale, x, y, M, K, N, stream, bias);
}

hipError_t launch_gemm(const uint32_t *w, const float *scale, const void *x,
                       int xt_bf16, void *y, int yt_bf16, int M, int K, int N,
                       int sp24, hipStream_t stream, const float *bias) {
  if (!sp24 && xt_bf16 && K % 64 == 0 && M > 16 && (reinterpret_cast<uintptr_t>(w) & 15) == 0) {
    if (yt_bf16) return launch_gemm2_t<uint16_t>(w, scale, x, y, M, K, N, stream, bias);
    return launch_gemm2_t<float>(w, scale, x, y, M, K, N, stream, bias);
  }
  if (sp24 && xt_bf16 && K % 64 == 0 && M > 16) {
    if (yt_bf16) return launch_gemm2sp_t<uint16_t, false>(w, scale, x, y, M, K, N, stream, bias);
    return launch_gemm2sp_t<float, false>(w, scale, x, y, M, K, N, stream, bias);
  }
  if (sp24) return launch_gemm_wf<WF_SP24>(w, scale, x, xt_bf16, y, yt_bf16, M, K, N, stream, bias);
  return launch_gemm_wf<WF_DENSE>(w, scale, x, xt_bf16, y, yt_bf16, M, K, N, stream, bias);
}

}  // namespace frx
