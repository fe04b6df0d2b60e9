// frx_ffn.hip — the whole decode FFN of a layer in one launch, M <= 3 tokens.
//
//   y = ((act(x Wg^T * s_gate)) * (x Wu^T * s_up)) Wd^T * s_down
//
// Replaces the dense FFN branch of the reference's decode step
// (src/model/cpu_block_attn_res.rs:2317-2326: three ternary matmul calls and
// the activation product on the host).
//
// Why one launch. A decode GEMV is a few µs of streaming behind a fixed
// per-launch cost (dispatch, ramp-up, drain) of about 2 µs on MI355X; the
// FFN's three matrices (34 MB at LLaMA-7B shapes) cost that three times when
// launched separately. Here every matrix byte is requested at kernel start:
// one workgroup per CU, each owning up to FFN1_T1 gate/up tile pairs (16 rows
// of both matrices) and one 16-row tile of the down matrix, loads all of its
// weights into registers, computes its part of h = act(g) * u, publishes it,
// meets the other workgroups at a grid barrier, and finishes its down tile
// with weights that arrived while the barrier was pending.
//
// Phases of a workgroup (16 waves):
//  1. Loads: x columns of each wave's gate/up quads (LDS staging, as in the
//     decode GEMV), the gate/up weight quads of every tile pair, then (waves
//     1..15 only) the down quads. Wave 0 holds no down weights, so its later
//     wait for its own stores does not wait for them.
//  2. Gate/up MFMAs (waves split K), fixed-order reduction through LDS,
//     row scales; wave 0 forms h = act(g) * u for its tiles and stores it as
//     the bf16 hi/lo planes the down MFMAs consume (dword i of a 16-column
//     block = (h[i], h[i+8]), |h - hi - lo| <= 2^-17 |h|).
//  3. Grid barrier (wave 0). h moves through device-coherent (sc1) stores
//     and loads, which bypass the per-XCD L2s, so the barrier needs no L2
//     writeback or invalidate. Arrivals count on one counter per XCD group
//     (workgroup id % 8), the last arrival of a group counts on a top
//     counter, and the last top arrival publishes the launch's epoch in the
//     `go` word that every workgroup polls. The epoch is go + 1 read at
//     kernel start, so the words never need resetting; the counters return
//     to zero at every barrier. The poll is bounded: on time-out it raises
//     the error word and carries on (results are then invalid; the host
//     reports it at the next synchronize).
//  4. Down MFMAs (waves 1..15 split K = I) on the staged h, fixed-order
//     reduction, row scales, y stores.
// All workgroups must be resident at once: the host launches at most one per
// CU and checks the occupancy.
#include <algorithm>

#include "frx_device.hpp"
#include "frx_internal.hpp"

namespace frx {

constexpr int FFN1_WAVES = 16;
constexpr int FFN1_T1 = 3;  // gate/up tile pairs per workgroup (max)
constexpr int FFN1_Q1 = 1;  // gate/up quads (256 columns) per wave: H <= 4096
constexpr int FFN1_Q2 = 3;  // down quads per wave (waves 1..15): I <= 11520
constexpr int FFN1_BMAX = 3;

// Barrier words (uint32 offsets into the context's barrier buffer).
constexpr int FFN1_BAR_TOP = 512, FFN1_BAR_GO = 576, FFN1_BAR_ERR = 640;
constexpr int FFN1_BAR_WORDS = 1024;
constexpr int FFN1_SPIN_LIMIT = 1 << 18;

// Buffer load / store of 16 bytes with the device-coherent cache policy
// (sc1: the access is performed at the point of coherence shared by all
// XCDs).
constexpr int CPOL_SC1 = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t ffn1_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

template <int N>
__device__ __forceinline__ void ffn1_wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

__device__ __forceinline__ unsigned ld_coherent(const unsigned *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent(unsigned *p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave-level arrival + wait (called by one whole wave, after its stores of
// the data to publish have completed).
__device__ __forceinline__ void ffn1_grid_barrier(unsigned *bar, unsigned target, unsigned G) {
  const int lane = threadIdx.x & 63;
  if (lane == 0) {
    const unsigned x = blockIdx.x & 7, gs = (G - x + 7) / 8;
    const unsigned old = __hip_atomic_fetch_add(bar + 64 * x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == gs - 1) {
      st_coherent(bar + 64 * x, 0u);
      const unsigned ng = G < 8 ? G : 8;
      const unsigned o2 = __hip_atomic_fetch_add(bar + FFN1_BAR_TOP, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (o2 == ng - 1) {
        st_coherent(bar + FFN1_BAR_TOP, 0u);
        ffn1_wait_vmcnt<0>();  // counters reset before the release
        st_coherent(bar + FFN1_BAR_GO, target);
      }
    }
  }
  int spins = 0;
  while (ld_coherent(bar + FFN1_BAR_GO) != target) {
    if (++spins > FFN1_SPIN_LIMIT) {
      if (lane == 0) st_coherent(bar + FFN1_BAR_ERR, 1u);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// LDS layout (dwords): per-wave zero blocks [0, 512), reduced gate/up tiles S
// [512, 2048), then one region reused phase by phase: x rows (gate/up), the
// gate/up partial tiles, h rows (down), the down partial tiles.
constexpr int FFN1_S_OFF = 512, FFN1_U_OFF = 2048;
static inline int ffn1_row_stride(int k) { return ((k + 255) / 256) * 128 + 4; }
static inline size_t ffn1_lds_bytes(int B, int H, int I, int P1) {
  size_t u = (size_t)P1 * B * ffn1_row_stride(H);
  const size_t red1 = (size_t)2 * FFN1_T1 * FFN1_WAVES * 64 * 4;
  const size_t h2 = (size_t)2 * B * ffn1_row_stride(I);
  const size_t red2 = (size_t)FFN1_WAVES * 64 * 4;
  if (red1 > u) u = red1;
  if (h2 > u) u = h2;
  if (red2 > u) u = red2;
  return (FFN1_U_OFF + u) * 4;
}

template <typename XT, typename YT, bool GELU>
__global__ __launch_bounds__(FFN1_WAVES * 64) void ffn1_kernel(
    const XT *__restrict__ X, const uint32_t *__restrict__ Wg, const float *__restrict__ sg,
    const uint32_t *__restrict__ Wu, const float *__restrict__ su, const uint32_t *__restrict__ Wd,
    const float *__restrict__ sd, uint32_t *hs, YT *__restrict__ Y, unsigned *bar, int B, int H,
    int I, int rs1, int rs2) {
  constexpr int P1 = XBlock<XT>::P;
  extern __shared__ __align__(16) uint32_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4, t = r;
  const bool live = t < B;
  const int G = gridDim.x, b = blockIdx.x;
  const int nt1 = I >> 4, nt2 = H >> 4;
  uint32_t *zblk = lds + wave * 32;
  uint32_t *U = lds + FFN1_U_OFF;
  f32x4 *S = reinterpret_cast<f32x4 *>(lds + FFN1_S_OFF);
  if (lane < 8) reinterpret_cast<u32x4 *>(zblk)[lane] = (u32x4){0u, 0u, 0u, 0u};

  // Every load below is issued unconditionally, in straight-line code, so
  // that the compiler's wait counts stay exact (a load skipped on some path
  // makes it wait for every outstanding load at the merge): out-of-range
  // tiles and quads are clamped to this workgroup's own data (L2 hits).
  // this launch's epoch (wave 0 publishes and polls)
  const unsigned target = ld_coherent(bar + FFN1_BAR_GO) + 1u;

  // tile pairs of this workgroup: b, b + G, b + 2G (< nt1)
  int np1 = 0;
#pragma unroll
  for (int i = 0; i < FFN1_T1; i++) np1 += (b + i * G < nt1) ? 1 : 0;
  const bool has_down = b < nt2;

  // scales for the epilogues: wave w < 2*np1 reduces (tile w/2, matrix w%2);
  // wave 0 also finishes the down tile
  const int tile_w = min(b + min(wave >> 1, FFN1_T1 - 1) * G, nt1 - 1);
  const f32x4 sc1 = *reinterpret_cast<const f32x4 *>(((wave & 1) ? su : sg) + tile_w * 16 + 4 * g);
  const f32x4 sc2 = *reinterpret_cast<const f32x4 *>(sd + min(b, nt2 - 1) * 16 + 4 * g);

  // ---- gate/up: this wave's quads of the H columns --------------------------
  const int wpr1 = H >> 4;
  const int nq1 = (H + 255) >> 8;
  const int qa1 = (wave * nq1) / FFN1_WAVES, qb1 = ((wave + 1) * nq1) / FFN1_WAVES;
  const int kblk1 = H >> 4;
  const int nb1 = 16 * (qb1 - qa1), cb1 = 16 * qa1;
  uint32_t *reg1 = U + cb1 * 8;
  const int nitem1 = B * nb1;  // <= 48: one round of 64 lanes
  const int x_tt = nb1 > 0 ? lane / nb1 : 0, x_j = lane - x_tt * nb1;
  const bool x_ok = lane < nitem1 && cb1 + x_j < kblk1;
  u32x4 xraw[XBlock<XT>::NV];
  XBlock<XT>::load_raw(X + (size_t)(x_ok ? x_tt : 0) * H + (x_ok ? cb1 + x_j : 0) * 16, xraw);
  __builtin_amdgcn_sched_barrier(0);  // x first: its staging must not wait for the weights
  u32x4 w1[FFN1_T1][2][FFN1_Q1];
#pragma unroll
  for (int i = 0; i < FFN1_T1; i++) {
    const int tile = min(b + min(i, max(np1 - 1, 0)) * G, nt1 - 1);
#pragma unroll
    for (int m = 0; m < 2; m++) {
      const uint32_t *wrow = (m ? Wu : Wg) + (size_t)(tile * 16 + r) * wpr1;
#pragma unroll
      for (int u = 0; u < FFN1_Q1; u++) {
        const int q = min(qa1 + u, nq1 - 1);
        w1[i][m][u] = *reinterpret_cast<const u32x4 *>(wrow + min((q * 4 + g) * 4, wpr1 - 4));
      }
    }
  }
  // stage x into the wave's columns. Unconditional: lanes without an item
  // write their zeros into the wave's zero block, so that the x loads stay
  // ahead of the weight loads (a conditional use would let the compiler sink
  // them behind the weights, and the staging would wait for all of them).
  {
    uint32_t xh[8], xl[8];
    XBlock<XT>::finish(xraw, x_ok, xh, xl);
    const bool mine = lane < nitem1;
    u32x4 *d = reinterpret_cast<u32x4 *>(mine ? reg1 + x_tt * rs1 + x_j * 8 : zblk);
    d[0] = (u32x4){xh[0], xh[1], xh[2], xh[3]};
    d[1] = (u32x4){xh[4], xh[5], xh[6], xh[7]};
    if constexpr (P1 == 2) {
      u32x4 *e = reinterpret_cast<u32x4 *>(mine ? reg1 + (B + x_tt) * rs1 + x_j * 8 : zblk);
      e[0] = (u32x4){xl[0], xl[1], xl[2], xl[3]};
      e[1] = (u32x4){xl[4], xl[5], xl[6], xl[7]};
    }
  }

  // gate/up MFMAs
  f32x4 acc1[FFN1_T1][2];
#pragma unroll
  for (int i = 0; i < FFN1_T1; i++) acc1[i][0] = acc1[i][1] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < FFN1_Q1; u++) {
    const int q = qa1 + u;
    if (q >= qb1) break;  // wave-uniform
    const int lc = (q - qa1) * 4 + g;
    const uint32_t mchunk = (q * 4 + g) * 4 < wpr1 ? 0xC000C000u : 0u;
    const uint32_t *bp = live ? reg1 + t * rs1 + lc * 32 : zblk;
    const uint32_t *bq = live ? reg1 + (B + t) * rs1 + lc * 32 : zblk;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const u32x4 b0 = *reinterpret_cast<const u32x4 *>(bp + (live ? k * 8 : 0));
      const u32x4 b1 = *reinterpret_cast<const u32x4 *>(bp + (live ? k * 8 + 4 : 4));
      u32x4 c0, c1;
      if constexpr (P1 == 2) {
        c0 = *reinterpret_cast<const u32x4 *>(bq + (live ? k * 8 : 0));
        c1 = *reinterpret_cast<const u32x4 *>(bq + (live ? k * 8 + 4 : 4));
      }
#pragma unroll
      for (int i = 0; i < FFN1_T1; i++) {
        if (i >= np1) break;  // workgroup-uniform
#pragma unroll
        for (int m = 0; m < 2; m++) {
          const u32x4 wq4 = w1[i][m][u];
          const uint32_t wq = k == 0 ? wq4.x : k == 1 ? wq4.y : k == 2 ? wq4.z : wq4.w;
          const u32x4 a0 = unpack_half_m<0>(wq, mchunk), a1 = unpack_half_m<1>(wq, mchunk);
          acc1[i][m] = mfma16(a0, b0, acc1[i][m]);
          acc1[i][m] = mfma16(a1, b1, acc1[i][m]);
          if constexpr (P1 == 2) {
            acc1[i][m] = mfma16(a0, c0, acc1[i][m]);
            acc1[i][m] = mfma16(a1, c1, acc1[i][m]);
          }
        }
      }
    }
  }
  // ---- down: waves 1..15 split the I columns --------------------------------
  // Issued once this wave's gate/up MFMAs are done, so that the gate/up
  // bytes (which the h exchange waits on) are not queued behind down bytes;
  // the down weights stream while h is exchanged. Wave 0 publishes h and must
  // not wait for down weights then: its slots read 16 bytes of x instead
  // (cached).
  const int wpr2 = I >> 4;
  const int nq2 = (I + 255) >> 8;
  const int qa2 = wave > 0 ? ((wave - 1) * nq2) / (FFN1_WAVES - 1) : 0;
  const int qb2 = wave > 0 ? (wave * nq2) / (FFN1_WAVES - 1) : 0;
  u32x4 w2[FFN1_Q2];
  {
    const uint32_t *wrow = wave > 0 ? Wd + (size_t)(min(b, nt2 - 1) * 16 + r) * wpr2
                                    : reinterpret_cast<const uint32_t *>(X);
#pragma unroll
    for (int u = 0; u < FFN1_Q2; u++) {
      const int q = min(qa2 + u, nq2 - 1);
      const int off = wave > 0 ? min((q * 4 + g) * 4, wpr2 - 4) : 0;
      w2[u] = *reinterpret_cast<const u32x4 *>(wrow + off);
    }
  }
  __syncthreads();  // x rows dead: the region now holds the partial tiles
  f32x4 *R1 = reinterpret_cast<f32x4 *>(U);
#pragma unroll
  for (int i = 0; i < FFN1_T1; i++)
    if (i < np1) {
      R1[((i * 2 + 0) * FFN1_WAVES + wave) * 64 + lane] = acc1[i][0];
      R1[((i * 2 + 1) * FFN1_WAVES + wave) * 64 + lane] = acc1[i][1];
    }
  __syncthreads();
  if (wave < 2 * np1) {  // wave = 2 * tile + matrix
    f32x4 s = R1[(wave * FFN1_WAVES) * 64 + lane];
#pragma unroll
    for (int v = 1; v < FFN1_WAVES; v++) s += R1[(wave * FFN1_WAVES + v) * 64 + lane];
    S[wave * 64 + lane] = s * (sc1 * 0.5f);  // 0.5 undoes the 2*dec(c) encoding
  }
  __syncthreads();

  // h = act(g) * u: waves 0..np1-1 (one per tile), one (row group, token)
  // per lane, into LDS (the partial tiles are dead)
  float *HF = reinterpret_cast<float *>(U);  // [tile][token][16 rows]
  if (wave < np1) {
    const int gg = lane >> 4, tt = lane & 15;
    if (tt < B) {
      const f32x4 gv = S[(wave * 2 + 0) * 64 + lane];
      const f32x4 uv = S[(wave * 2 + 1) * 64 + lane];
      f32x4 hv;
#pragma unroll
      for (int j = 0; j < 4; j++) hv[j] = (GELU ? act_gelu_tanh(gv[j]) : act_silu(gv[j])) * uv[j];
      *reinterpret_cast<f32x4 *>(HF + (wave * 16 + tt) * 16 + 4 * gg) = hv;
    }
  }
  __syncthreads();

  // ---- wave 0: publish h, grid barrier ---------------------------------------
  if (wave == 0) {
    const int i = lane >> 4, tt = lane & 15;  // (tile, token) per lane
    if (i < np1 && tt < B) {
      float v[16];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const f32x4 hq = *reinterpret_cast<const f32x4 *>(HF + (i * 16 + tt) * 16 + 4 * q);
#pragma unroll
        for (int j = 0; j < 4; j++) v[4 * q + j] = hq[j];
      }
      uint32_t hb[16], lb[16];
#pragma unroll
      for (int j = 0; j < 16; j++) split_bf16(v[j], hb[j], lb[j]);
      u32x4 hv[2], lv[2];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        hv[0][j] = hb[j] | (hb[j + 8] << 16);
        hv[1][j] = hb[j + 4] | (hb[j + 12] << 16);
        lv[0][j] = lb[j] | (lb[j + 8] << 16);
        lv[1][j] = lb[j + 4] | (lb[j + 12] << 16);
      }
      // planes: hs[(token * 2 + plane) * I/2 + block * 8 + dword]
      const int blk = b + i * G;
      const uint32_t plane = (uint32_t)I * 2u;  // bytes per plane
      const __amdgpu_buffer_rsrc_t rs = ffn1_rsrc(hs, (uint32_t)B * 2u * plane);
      const int off = tt * 2 * (int)plane + blk * 32;
      __builtin_amdgcn_raw_buffer_store_b128(hv[0], rs, off, 0, CPOL_SC1);
      __builtin_amdgcn_raw_buffer_store_b128(hv[1], rs, off + 16, 0, CPOL_SC1);
      __builtin_amdgcn_raw_buffer_store_b128(lv[0], rs, off + (int)plane, 0, CPOL_SC1);
      __builtin_amdgcn_raw_buffer_store_b128(lv[1], rs, off + (int)plane + 16, 0, CPOL_SC1);
    }
    ffn1_wait_vmcnt<0>();  // this wave's h stores have completed
    ffn1_grid_barrier(bar, target, (unsigned)G);
  }
  __syncthreads();  // every wave: h of all workgroups is published

  // ---- down: stage this wave's h columns, MFMAs -------------------------------
  // four independent accumulators (one per word of a chunk): a single
  // accumulator would chain every MFMA of the wave on the previous one
  f32x4 acc2[4];
#pragma unroll
  for (int k = 0; k < 4; k++) acc2[k] = (f32x4){0.f, 0.f, 0.f, 0.f};
  if (has_down && qb2 > qa2) {
    const int kblk2 = I >> 4;
    const int nb2 = 16 * (qb2 - qa2), cb2 = 16 * qa2;
    uint32_t *reg2 = U + cb2 * 8;
    const int nitem2 = 2 * B * nb2;  // (row = plane * B + token, block) pairs
    const uint32_t plane = (uint32_t)I * 2u;
    const __amdgpu_buffer_rsrc_t rs = ffn1_rsrc(hs, (uint32_t)B * 2u * plane);
    constexpr int R2MAX = (2 * FFN1_BMAX * 16 * FFN1_Q2 + 63) / 64;
    u32x4 hv[R2MAX][2];
#pragma unroll
    for (int k = 0; k < R2MAX; k++) {
      const int it = lane + 64 * k, row = it / nb2, j = it - row * nb2;
      if (it < nitem2 && cb2 + j < kblk2) {
        const int tt = row % B, pl = row / B;
        const int off = (tt * 2 + pl) * (int)plane + (cb2 + j) * 32;
        hv[k][0] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, CPOL_SC1);
        hv[k][1] = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16, 0, CPOL_SC1);
      } else {
        hv[k][0] = hv[k][1] = (u32x4){0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int k = 0; k < R2MAX; k++) {
      const int it = lane + 64 * k, row = it / nb2, j = it - row * nb2;
      if (it < nitem2) {
        u32x4 *d = reinterpret_cast<u32x4 *>(reg2 + row * rs2 + j * 8);
        d[0] = hv[k][0];
        d[1] = hv[k][1];
      }
    }
#pragma unroll
    for (int u = 0; u < FFN1_Q2; u++) {
      const int q = qa2 + u;
      if (q >= qb2) break;  // wave-uniform
      const int lc = (q - qa2) * 4 + g;
      const uint32_t mchunk = (q * 4 + g) * 4 < wpr2 ? 0xC000C000u : 0u;
      const uint32_t *bp = live ? reg2 + t * rs2 + lc * 32 : zblk;
      const uint32_t *bq = live ? reg2 + (B + t) * rs2 + lc * 32 : zblk;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const u32x4 b0 = *reinterpret_cast<const u32x4 *>(bp + (live ? k * 8 : 0));
        const u32x4 b1 = *reinterpret_cast<const u32x4 *>(bp + (live ? k * 8 + 4 : 4));
        const u32x4 c0 = *reinterpret_cast<const u32x4 *>(bq + (live ? k * 8 : 0));
        const u32x4 c1 = *reinterpret_cast<const u32x4 *>(bq + (live ? k * 8 + 4 : 4));
        const uint32_t wq = k == 0 ? w2[u].x : k == 1 ? w2[u].y : k == 2 ? w2[u].z : w2[u].w;
        const u32x4 a0 = unpack_half_m<0>(wq, mchunk), a1 = unpack_half_m<1>(wq, mchunk);
        acc2[k] = mfma16(a0, b0, acc2[k]);
        acc2[k] = mfma16(a1, b1, acc2[k]);
        acc2[k] = mfma16(a0, c0, acc2[k]);
        acc2[k] = mfma16(a1, c1, acc2[k]);
      }
    }
  }
  __syncthreads();  // h rows dead: the region now holds the down partials
  f32x4 *R2 = reinterpret_cast<f32x4 *>(U);
  R2[wave * 64 + lane] = (acc2[0] + acc2[1]) + (acc2[2] + acc2[3]);
  __syncthreads();
  if (wave == 0 && has_down) {
    f32x4 s = R2[64 + lane];
#pragma unroll
    for (int v = 2; v < FFN1_WAVES; v++) s += R2[v * 64 + lane];
    s *= sc2 * 0.5f;
    if (live) YStore<YT>::store4(Y + (size_t)t * H + b * 16 + 4 * g, s, 4);
  }
}

bool ffn1_supported(int B, int H, int I, int xt_bf16, int cus, int *grid, size_t *lds) {
  if (B < 1 || B > FFN1_BMAX || H % 64 || I % 64 || H < 64 || I < 64) return false;
  const int nt1 = I / 16, nt2 = H / 16;
  const int nq1 = (H + 255) / 256, nq2 = (I + 255) / 256;
  if ((nq1 + FFN1_WAVES - 1) / FFN1_WAVES > FFN1_Q1) return false;
  if ((nq2 + FFN1_WAVES - 2) / (FFN1_WAVES - 1) > FFN1_Q2) return false;
  const int G = std::max((nt1 + FFN1_T1 - 1) / FFN1_T1, nt2);
  if (G > cus) return false;
  const size_t bytes = ffn1_lds_bytes(B, H, I, xt_bf16 ? 1 : 2);
  if (bytes > 160 * 1024) return false;
  *grid = G;
  *lds = bytes;
  return true;
}

size_t ffn1_h_bytes(int B, int I) { return (size_t)B * 2 * I * 2; }
size_t ffn1_barrier_bytes() { return FFN1_BAR_WORDS * 4; }
size_t ffn1_error_word() { return FFN1_BAR_ERR; }

template <typename XT, typename YT, bool GELU>
static hipError_t launch_ffn1_t(const void *x, const uint32_t *wg, const float *sg, const uint32_t *wu,
                                const float *su, const uint32_t *wd, const float *sd, uint32_t *hs, void *y,
                                unsigned *bar, int B, int H, int I, int G, size_t lds, hipStream_t stream) {
  static std::atomic<uint64_t> done{0};
  const void *fn = reinterpret_cast<const void *>(&ffn1_kernel<XT, YT, GELU>);
  hipError_t e = opt_in_lds(fn, (int)lds, done);
  if (e != hipSuccess) return e;
  int per_cu = 0;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, FFN1_WAVES * 64, lds);
  if (e != hipSuccess) return e;
  if (per_cu < 1) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((ffn1_kernel<XT, YT, GELU>), dim3(G), dim3(FFN1_WAVES * 64), lds, stream,
                     reinterpret_cast<const XT *>(x), wg, sg, wu, su, wd, sd, hs, reinterpret_cast<YT *>(y),
                     bar, B, H, I, ffn1_row_stride(H), ffn1_row_stride(I));
  return hipGetLastError();
}

hipError_t launch_ffn1(const void *x, int xt_bf16, const uint32_t *wg, const float *sg, const uint32_t *wu,
                       const float *su, const uint32_t *wd, const float *sd, uint32_t *hs, void *y,
                       int yt_bf16, unsigned *bar, int B, int H, int I, int gelu, int G, size_t lds,
                       hipStream_t stream) {
#define FRX_FFN1(XT, YT)                                                                                 \
  return gelu ? launch_ffn1_t<XT, YT, true>(x, wg, sg, wu, su, wd, sd, hs, y, bar, B, H, I, G, lds, stream) \
              : launch_ffn1_t<XT, YT, false>(x, wg, sg, wu, su, wd, sd, hs, y, bar, B, H, I, G, lds, stream)
  if (xt_bf16) {
    if (yt_bf16) FRX_FFN1(uint16_t, uint16_t);
    FRX_FFN1(uint16_t, float);
  }
  if (yt_bf16) FRX_FFN1(float, uint16_t);
  FRX_FFN1(float, float);
#undef FRX_FFN1
}

}  // namespace frx
