// frx_gemm2.hpp — pipelined MFMA tile engine for bf16-activation ternary GEMMs.
//
// C[BN weight rows][BM tokens] += dec(W)[n][k] * X[m][k], one workgroup tile,
// v_mfma_f32_16x16x32_bf16 with A = weight rows, B = tokens, fp32 acc.
//
// Data movement. Both tiles go global -> LDS with buffer_load_dwordx4 ... lds
// (no VGPR staging, no VALU work per element) through an NS-stage ring, so
// the loads of step s+NS-1 are in flight while step s is multiplied. One
// vmcnt wait + barrier per 64-column step. Buffer (MUBUF) rather than global
// (FLAT) LDS DMA: the compiler treats a FLAT access that may touch LDS as
// unordered with LDS reads and would make every LDS wait of the step a full
// lgkmcnt(0); with MUBUF the operand reads get partial waits. Each lane's
// byte offset inside a tile is fixed for the whole K loop; the step's column
// advance goes in the scalar soffset. The buffer's num_records is the tile's
// valid byte range, so the hardware range check bounds every load.
//  - X stage: BM rows x 64 bf16 (128 B per row) in natural order, 16-byte
//    chunks XOR-swizzled (xswz) so the 16 rows of an MFMA operand read hit
//    disjoint bank groups.
//  - W stage: BN rows x 4 words (the reference's packed u32 words).
// Operands. Lane (i = l%16, g = l/16) of MFMA half h covers columns
// 16g + 8h .. 16g + 8h + 7 of the step, in natural order: the X operand is
// one 16-byte LDS read; the two W operands of a lane are the 16 codes of
// weight word g of its row, turned into bf16 pairs (c, c+1) by four masked
// shifted copies and one byte permute per pair (unpack16_nat, about 0.94
// VALU ops per weight), the same 2*dec(c) encoding as frx_device.hpp. Each
// W operand feeds TM/16 MFMAs.
#pragma once
#include "frx_device.hpp"

namespace frx {

typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

// Four natural-order operand pairs from the byte pair (b0, b0+1) of word w,
// i.e. codes 4*b0 .. 4*b0+7. sel0 / sel1 place byte b0 / b0+1 at bytes 1
// and 3 of a dword (v_perm_b32 selectors). Returns dwords (c0,c1) (c2,c3)
// (c4,c5) (c6,c7) with bf16 bits ((~c)&3)<<14 in each half.
__device__ __forceinline__ u32x4 unpack8_nat(uint32_t w, uint32_t sel0, uint32_t sel1) {
  const uint32_t y0 = __builtin_amdgcn_perm(w, w, sel0);
  const uint32_t y1 = __builtin_amdgcn_perm(w, w, sel1);
  const u16x2 s_lo = {6, 4}, s_hi = {2, 0};
  u32x4 r;
  r.x = ~__builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, y0) << s_lo) & 0xC000C000u;
  r.y = ~__builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, y0) << s_hi) & 0xC000C000u;
  r.z = ~__builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, y1) << s_lo) & 0xC000C000u;
  r.w = ~__builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, y1) << s_hi) & 0xC000C000u;
  return r;
}

// A whole 16-code word as two natural-order operands: lo = codes 0..7 as
// pairs (0,1) (2,3) (4,5) (6,7), hi = codes 8..15. m_r = ~(w << (6 - 2r)) &
// 0xC0C0C0C0 holds code 4b + r (inverted) in the top two bits of byte b;
// dword j (codes 2j, 2j+1) is one byte permute: byte j/2 of m_{2(j%2)} as
// its byte 1, of m_{2(j%2)+1} as its byte 3, zeros elsewhere (selector
// 0x0C). 15 VALU ops per 16 weights, the same 2*dec(c) bf16 encoding.
__device__ __forceinline__ void unpack16_nat(uint32_t w, u32x4 &lo, u32x4 &hi) {
  const uint32_t m0 = ~(w << 6) & 0xC0C0C0C0u, m1 = ~(w << 4) & 0xC0C0C0C0u;
  const uint32_t m2 = ~(w << 2) & 0xC0C0C0C0u, m3 = ~w & 0xC0C0C0C0u;
  uint32_t d[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint32_t b = (uint32_t)(j >> 1);
    const uint32_t sel = 0x0Cu | (b << 8) | (0x0Cu << 16) | ((4u + b) << 24);
    d[j] = (j & 1) ? __builtin_amdgcn_perm(m3, m2, sel) : __builtin_amdgcn_perm(m1, m0, sel);
  }
  lo = (u32x4){d[0], d[1], d[2], d[3]};
  hi = (u32x4){d[4], d[5], d[6], d[7]};
}

typedef __attribute__((address_space(3))) void *lds_ptr_t;

// gfx950 raw buffer descriptor word 3 (32-bit data format, no swizzle, no
// stride): byte offsets are range-checked against num_records.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// 16 bytes per lane from rsrc at voffset + soffset into LDS: lane l's bytes
// land at ldst + 16 * l (M0 holds the wave's LDS base).
// acc += A * B with the accumulator tied to one accumulation register. The
// builtin's untied form lets the register allocator write each product to a
// fresh register and copy it back every step (tens of copies per step in a
// pipelined loop). Operand producers are kept at least four MFMAs ahead by
// the schedule below, and accumulation into the same register needs no wait
// states, so no hazard padding is needed inside the loop; readers of the
// results after the loop get explicit padding (mfma_drain).
__device__ __forceinline__ void mfma16_acc(f32x4 &acc, const u32x4 &a, const u32x4 &b) {
  asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// Wait states between the last MFMA writing an accumulator and any other
// instruction reading it (more than the longest XDL write-to-read hazard).
__device__ __forceinline__ void mfma_drain() {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
}

typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));

// acc += A * B on the 2:4 sparse matrix pipe (twice the dense rate), tied
// like mfma16_acc. A (16 weight rows x 64 columns, two nonzeros per group
// of 4) arrives compressed: lane (i = l%16, kg = l/16) holds row i's values
// for groups 4 kg .. 4 kg + 3 as 8 bf16 (two per group, lower position
// first) and, in bits 2s+1:2s of idx, the position (0..3) inside its group
// of compressed value s. B is 16 bf16 per lane: columns 8 kg .. 8 kg + 7 and
// 32 + 8 kg .. 32 + 8 kg + 7 of the step for token l%16, i.e. the dense
// engine's two X operands of the step.
__device__ __forceinline__ void smfmac16_acc(f32x4 &acc, const u32x4 &a, const u32x8 &b, uint32_t idx) {
  asm("v_smfmac_f32_16x16x64_bf16 %0, %1, %2, %3" : "+a"(acc) : "v"(a), "v"(b), "v"(idx));
}

// Four 2:4 groups in the GPU 5-bit layout (bits 2:0 pattern, pattern > 5
// read as 5; bit 3 / bit 4 set: the lower / higher nonzero is -1;
// src/compute/kernels/sparse_ternary.rs:87-107) as a compressed smfmac A
// operand. F holds the groups at bits 5q. Values are +-2 (bf16 0x4000 /
// 0xC000, the 2*dec encoding of the dense path); the position nibble of a
// pattern is p0 | p1 << 2, looked up in a constant (pattern p at bits 4p:
// (0,1) (0,2) (0,3) (1,2) (1,3) (2,3), then 5 twice).
__device__ __forceinline__ void sp24_operand(uint32_t F, u32x4 &a, uint32_t &idx) {
  uint32_t ix = 0;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const uint32_t c = __builtin_amdgcn_ubfe(F, 5 * q, 5);
    ix |= __builtin_amdgcn_ubfe(0xEEED9C84u, c << 2, 4) << (4 * q);
    a[q] = (((c << 12) | (c << 27)) & 0x80008000u) | 0x40004000u;
  }
  idx = ix;
}

// The prepared form of four 2:4 groups (16 s + 4 g + q, q = 0..3, of one
// row): position nibble q at bits 4q (q < 3) and 16 (q = 3), sign of the
// lower / higher nonzero of group q at bit 12 + q / 28 + q. One word per
// (row, step, lane group) decodes in 9 ops instead of the 5-bit layout's
// window funnel and per-group lookups. F: the four 5-bit groups at bits 5q.
// The signs (bits 5q + 3 and 5q + 4 of F) are gathered by one multiply:
// bit 5q times 2^(12 - 4q') lands on 16 distinct positions, the q' = q ones
// on 12 + q, so nothing carries into them.
__device__ __forceinline__ uint32_t sp24p_word(uint32_t F) {
  uint32_t d = 0;
#pragma unroll
  for (int q = 0; q < 4; q++)
    d |= __builtin_amdgcn_ubfe(0xEEED9C84u, __builtin_amdgcn_ubfe(F, 5 * q, 3) << 2, 4) << (q < 3 ? 4 * q : 16);
  const uint32_t sa = (((F >> 3) & 0x8421u) * 0x1111u) & 0xF000u;
  const uint32_t sb = (((F >> 4) & 0x8421u) * 0x1111u) & 0xF000u;
  return d | sa | (sb << 16);
}
__device__ __forceinline__ void sp24p_operand(uint32_t d, u32x4 &a, uint32_t &idx) {
#pragma unroll
  for (int q = 0; q < 4; q++) a[q] = ((d << (3 - q)) & 0x80008000u) | 0x40004000u;
  idx = (d & 0xFFFu) | ((d >> 4) & 0xF000u);
}

__device__ __forceinline__ void lds_load4(__amdgpu_buffer_rsrc_t r, uint32_t *ldst,
                                          uint32_t voffset, uint32_t soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)ldst, 4, voffset, soffset, 0, 0);
}

__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, uint32_t *ldst,
                                           uint32_t voffset, uint32_t soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)ldst, 16, voffset, soffset, 0, 0);
}

// s_waitcnt with only the vector-memory counter limited to n (gfx9 encoding:
// vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14; expcnt and lgkmcnt left
// at their maxima, i.e. not waited on).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Requires K % 64 == 0 (whole 16-byte W chunks per row and step). GATHER:
// tile row m reads X row rowidx[m] (the indices are read once into
// registers, so the pipelined loop issues no other vector-memory ops and the
// explicit vmcnt accounting below stays exact).
// Workgroup barrier without the memory fence of __syncthreads(): the fence
// would make the compiler drain every in-flight global->LDS load (vmcnt(0))
// at each step. Completion of the stage about to be read is established by
// the explicit wait_vmcnt before the barrier, and LDS reads of a stage finish
// (their results feed MFMAs) before the barrier that precedes its reuse.
__device__ __forceinline__ void barrier_nofence() { __builtin_amdgcn_s_barrier(); }

// X-stage swizzle: 16-byte chunk c of stage row r sits at chunk c ^ xswz(r).
// An MFMA operand read has lanes 0..15 on rows r0..r0+15 (r0 % 16 == 0) at
// one chunk. xswz takes 8 distinct values on rows r0..r0+7 and on
// r0+8..r0+15, and (r % 2, xswz(r)) 16 distinct pairs over the 16 rows, so
// the read spreads over all banks whether the LDS serves 8 lanes (128 bytes)
// or 16 lanes (256 bytes) of a 16-byte read per pass.
__device__ __forceinline__ uint32_t xswz(int r) { return (uint32_t)((r & 7) ^ ((r >> 3) & 1)); }

// DUALX: X-stage rows [BM/2, BM) are the rows [0, BM/2) again, read at a
// second column offset (xoff2 bytes further along each row): one stage then
// holds two column ranges of the same token rows, e.g. the hi and lo bf16
// halves of an fp32 activation stored as [rows][2 K].
template <int BM, int BN, int WM, int WN, int NS, bool GATHER, bool DUALX = false>
struct Gemm2 {
  static constexpr int NT = WM * WN * 64;
  static constexpr int WAVES = WM * WN;
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int FM = TM / 16, FN = TN / 16;
  static constexpr int XSTAGE = BM * 32;  // dwords (BM rows x 128 B)
  static constexpr int WSTAGE = BN * 4;   // dwords (BN rows x 16 B)
  static constexpr int STAGE = XSTAGE + WSTAGE;
  static constexpr int LDS_DWORDS = NS * STAGE;
  static constexpr int XI = BM / 8;    // 1 KB load instructions per X stage
  static_assert(XI % WAVES == 0, "X loads must split evenly over the waves");
  // W stage: 1 KB (16-byte DMA, 64 rows) instructions when they split evenly
  // over the waves, else 256-byte (4-byte DMA: lane l loads word l % 4 of row
  // l / 4) instructions; both fill rows of 4 words.
  static constexpr bool W4 = (BN / 64) % WAVES != 0;
  static constexpr int WROWS = W4 ? 16 : 64;  // rows per W load instruction
  static constexpr int WI = BN / WROWS;
  static_assert(WI % WAVES == 0, "W loads must split evenly over the waves");
  static constexpr int XPW = XI / WAVES, WPW = WI / WAVES;
  static constexpr int LPW = XPW + WPW;  // load instructions per wave per stage
  static_assert(TM % 16 == 0 && TN % 16 == 0, "wave tile must be 16-aligned");

  // Per-lane byte offsets of the XPW X and WPW W load instructions of this
  // wave inside their buffers, fixed for the whole K loop. X rows past
  // m_count are clamped to the last valid row and W rows past n_count to the
  // last valid row (their outputs are discarded by the caller). Non-gather X
  // offsets are relative to the tile's first row; gather offsets to row 0.
  // ldx: X row stride (elements); wk: columns of W (its row length; the K
  // loop may run past it, see run). Dual weights: W-stage rows [BN/2, BN)
  // come from a second matrix (rows n - BN/2), each of n_count valid rows.
  __device__ __forceinline__ static void lane_offsets(uint32_t (&xv)[XPW], uint32_t (&wv)[WPW],
                                                      const int *rowidx, int m_count,
                                                      int n_count, int ldx, int wk, bool dual,
                                                      uint32_t xoff2) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < XPW; i++) {
      const int r = (wave * XPW + i) * 8 + (lane >> 3);
      const int second = DUALX && r >= BM / 2;
      const int rm = min(second ? r - BM / 2 : r, m_count - 1);
      const uint32_t gr = GATHER ? (uint32_t)rowidx[rm] : (uint32_t)rm;
      const uint32_t c = (lane & 7) ^ xswz(r);  // swizzled source chunk
      xv[i] = gr * (uint32_t)ldx * 2u + 16u * c + (second ? xoff2 : 0u);
    }
#pragma unroll
    for (int i = 0; i < WPW; i++) {
      int n = (wave * WPW + i) * WROWS + (W4 ? lane >> 2 : lane);
      if (dual && n >= BN / 2) n -= BN / 2;
      n = min(n, n_count - 1);
      wv[i] = ((uint32_t)n * (uint32_t)(wk >> 4) + (W4 ? (uint32_t)(lane & 3) : 0u)) * 4u;
    }
  }

  // k0: X column of the stage; kw0: its W column.
  __device__ __forceinline__ static void issue(uint32_t *stage, __amdgpu_buffer_rsrc_t xr,
                                               const __amdgpu_buffer_rsrc_t (&wr)[WPW], const uint32_t (&xv)[XPW],
                                               const uint32_t (&wv)[WPW], int k0, int kw0) {
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < XPW; i++) lds_load16(xr, stage + (wave * XPW + i) * 256, xv[i], 2u * k0);
#pragma unroll
    for (int i = 0; i < WPW; i++) {
      if constexpr (W4) lds_load4(wr[i], stage + XSTAGE + (wave * WPW + i) * 64, wv[i], (uint32_t)kw0 >> 2);
      else lds_load16(wr[i], stage + XSTAGE + (wave * WPW + i) * 256, wv[i], (uint32_t)kw0 >> 2);
    }
  }

  __device__ __forceinline__ static u32x4 xread(const uint32_t *stage, int r, int c) {
    return *reinterpret_cast<const u32x4 *>(stage + r * 32 + ((c ^ xswz(r)) * 4));
  }

  // X operand i of a step (i = h * F + fm, F token blocks multiplied):
  // tokens r0 + 16 fm, columns 16 g + 8 h .. +7 (the codes of weight word g
  // of the step, half h).
  template <int F>
  __device__ __forceinline__ static u32x4 xop(const uint32_t *stage, int r0, int g, int i) {
    return xread(stage, r0 + (i % F) * 16, 2 * g + i / F);
  }

  static constexpr int XD = 4;  // X operand reads run this many MFMA groups ahead

  // Waits until at most n of this wave's stage load groups are in flight
  // (n clamped to N; s_waitcnt takes an immediate, hence the chain).
  template <int N>
  __device__ __forceinline__ static void wait_stages(int n) {
    if constexpr (N == 0) {
      wait_vmcnt<0>();
    } else {
      if (n >= N) wait_vmcnt<N * LPW>();
      else wait_stages<N - 1>(n);
    }
  }

  // The K loop, software-pipelined so that the matrix pipe never waits on
  // the rest of the step. With one wave per SIMD nothing else hides latency,
  // so the instruction order is fixed with scheduling fences.
  //
  // Step t multiplies stage t in two halves of 32 columns (h = 0, 1), one
  // X-operand read two tiles ahead of its MFMAs. Between the halves each wave
  // waits for its own loads of stage t+1 and the block meets at a barrier;
  // after it, interleaved with the second half's MFMAs, the wave issues the
  // loads of stage t+NS-1 (into the slot of stage t-1, whose last reads fed
  // MFMAs before the barrier), reads stage t+1's weight words and first two
  // X operands, and unpacks stage t+1's first-half weight operands. The first
  // half's MFMAs likewise cover the unpack of the second half's operands.
  // Stage t+1 is issued in step t+2-NS, i.e. NS-2 steps of latency cover.
  //
  // W2 != nullptr: dual weights (W-stage rows BN/2.. from W2). wk: W's
  // columns, K <= 2 wk; past wk the loop multiplies X's columns by W again
  // (W column k - wk), which runs an fp32 activation stored as bf16 hi | lo
  // halves of one row in a single pass (K = 2 wk). ldx: X row stride in
  // elements (default K). F: the token blocks of each wave that are
  // multiplied (the first F of its FM; the stage holds all BM rows, rows
  // past F blocks are loaded and left unread). xoff2: see DUALX.
  template <int F = FM>
  __device__ static void run(uint32_t *lds, const uint16_t *X, uint32_t xbytes, const int *rowidx,
                             int m_count, const uint32_t *W, int n_count, int K,
                             f32x4 (&acc)[FN][F], const uint32_t *W2 = nullptr, int wk = 0, int ldx = 0,
                             uint32_t xoff2 = 0) {
    static_assert(NS >= 3, "the ring needs a stage being read, one landing and one free");
    static_assert(F >= 4 && XD <= F && F <= FM, "operand schedule");
    if (wk == 0) wk = K;
    if (ldx == 0) ldx = K;
    const bool dual = W2 != nullptr;
    uint32_t xv[XPW], wv[WPW];
    lane_offsets(xv, wv, rowidx, m_count, n_count, ldx, wk, dual, xoff2);
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(X, xbytes);
    __amdgpu_buffer_rsrc_t wr[WPW];
    {
      const int wave = threadIdx.x >> 6;
#pragma unroll
      for (int i = 0; i < WPW; i++) {
        const bool second = dual && (wave * WPW + i) * WROWS >= BN / 2;
        wr[i] = buffer_rsrc(second ? W2 : W, (uint32_t)n_count * (uint32_t)(wk >> 4) * 4u);
      }
    }
#pragma unroll
    for (int fn = 0; fn < FN; fn++)
#pragma unroll
      for (int fm = 0; fm < F; fm++) acc[fn][fm] = (f32x4){0.f, 0.f, 0.f, 0.f};
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave % WM, wn = wave / WM;
    const int l16 = lane & 15, g = lane >> 4;
    const int r0 = wm * TM + l16;
    // weight word g of fragment fn's row in a stage (both halves of the step)
    const int wofs = XSTAGE + (wn * TN + l16) * 4 + g;
    const int nks = (K + 63) >> 6;

    // One stage is issued per step, always: past the last stage the last
    // stage's columns are loaded again (valid addresses) into the slot that
    // is free anyway and never read. The wait counts stay uniform and the
    // step has no branch; control flow among the MFMAs makes the register
    // allocator shuttle the accumulators between register files.
#pragma unroll
    for (int s = 0; s < NS - 1; s++) {
      const int k0 = min(s, nks - 1) * 64;
      issue(lds + s * STAGE, xr, wr, xv, wv, k0, k0 >= wk ? k0 - wk : k0);
    }
    wait_vmcnt<(NS - 2) * LPW>();  // stage 0 landed
    barrier_nofence();

    // operands of step 0
    u32x4 a0[FN], a1[FN], bn[XD];
    {
      uint32_t wq[FN];
#pragma unroll
      for (int fn = 0; fn < FN; fn++) wq[fn] = lds[wofs + fn * 64];
#pragma unroll
      for (int d = 0; d < XD; d++) bn[d] = xop<F>(lds, r0, g, d);
#pragma unroll
      for (int fn = 0; fn < FN; fn++) unpack16_nat(wq[fn], a0[fn], a1[fn]);
    }

    for (int t = 0; t < nks; t++) {
      const uint32_t *cur = lds + (t % NS) * STAGE;
      const uint32_t *nxt = lds + ((t + 1) % NS) * STAGE;
      u32x4 b[2 * F];
#pragma unroll
      for (int d = 0; d < XD; d++) b[d] = bn[d];
      __builtin_amdgcn_sched_barrier(0);
      // first half: the low 8 codes of each weight word
#pragma unroll
      for (int fm = 0; fm < F; fm++) {
        const int q = fm;
        b[q + XD] = xop<F>(cur, r0, g, q + XD);
#pragma unroll
        for (int fn = 0; fn < FN; fn++) mfma16_acc(acc[fn][fm], a0[fn], b[q]);
        __builtin_amdgcn_sched_barrier(0);
      }
      // stage t+1 landed for every wave (the NS-3 stages issued after it may
      // stay in flight)
      wait_vmcnt<(NS - 3) * LPW>();
      barrier_nofence();
      __builtin_amdgcn_sched_barrier(0);
      // second half: the high 8 codes, plus the next stage's loads and operands
      uint32_t wqn[FN];
      u32x4 a0n[FN], a1n[FN];
#pragma unroll
      for (int fm = 0; fm < F; fm++) {
        const int q = F + fm;
        if (q + XD < 2 * F) b[q + XD] = xop<F>(cur, r0, g, q + XD);
        else bn[q + XD - 2 * F] = xop<F>(nxt, r0, g, q + XD - 2 * F);
        if (fm == 0) {
#pragma unroll
          for (int fn = 0; fn < FN; fn++) wqn[fn] = nxt[wofs + fn * 64];
        }
#pragma unroll
        for (int fn = 0; fn < FN; fn++) mfma16_acc(acc[fn][fm], a1[fn], b[q]);
        if (fm == 0) {
          const int k0 = min(t + NS - 1, nks - 1) * 64;
          issue(lds + ((t + NS - 1) % NS) * STAGE, xr, wr, xv, wv, k0, k0 >= wk ? k0 - wk : k0);
        }
        if (fm >= 2 && fm - 2 < FN) unpack16_nat(wqn[fm - 2], a0n[fm - 2], a1n[fm - 2]);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int fn = F - 2; fn < FN; fn++) unpack16_nat(wqn[fn], a0n[fn], a1n[fn]);
#pragma unroll
      for (int fn = 0; fn < FN; fn++) {
        a0[fn] = a0n[fn];
        a1[fn] = a1n[fn];
      }
    }
    mfma_drain();
    // every load has landed and every read is done before the epilogue
    // reuses the ring
    wait_vmcnt<0>();
    barrier_nofence();
  }

  // ---- 2:4 sparse weights (GPU 5-bit layout, wpr words per row) ------------
  // A step's 16 groups per row lie in the 4-word window that starts at word
  // floor(16 s / 6) of the row (6 groups per word). Rows are only 4-byte
  // aligned, so the window moves with 4-byte LDS DMA: lane l of a 256-byte
  // instruction loads word l % 4 of row l / 4, which keeps the dense W-stage
  // layout (rows of 4 words).
  static constexpr int SWI = BN * 4 / 64;
  static_assert(SWI % WAVES == 0, "sparse W loads must split evenly over the waves");
  static constexpr int SWPW = SWI / WAVES;
  static constexpr int SLPW = XPW + SWPW;

  __device__ __forceinline__ static uint32_t sp_window_bytes(int s) { return 4u * (uint32_t)((16 * s) / 6); }

  // s: the X step (64 columns), sw: the metadata step
  __device__ __forceinline__ static void issue_sp(uint32_t *stage, __amdgpu_buffer_rsrc_t xr,
                                                  __amdgpu_buffer_rsrc_t wr, const uint32_t (&xv)[XPW],
                                                  const uint32_t (&wv)[SWPW], int s, int sw) {
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < XPW; i++) lds_load16(xr, stage + (wave * XPW + i) * 256, xv[i], 128u * (uint32_t)s);
#pragma unroll
    for (int i = 0; i < SWPW; i++)
      lds_load4(wr, stage + XSTAGE + (wave * SWPW + i) * 64, wv[i], sp_window_bytes(sw));
  }

  // The A operands of fragment rows wn*TN + fn*16 + l16 for step s from the
  // W stage at ws (lane kg = g takes groups 16 s + 4 g .. + 3).
  __device__ __forceinline__ static void sp_read(const uint32_t *ws, int s, int wrow, int g,
                                                 uint32_t (&wa)[FN], uint32_t (&wb)[FN], int &o5) {
    const int l0 = (4 * s) % 6 + 4 * g;  // first group, relative to the window
    const int jw = l0 / 6;
    o5 = 5 * (l0 - 6 * jw);
#pragma unroll
    for (int fn = 0; fn < FN; fn++) {
      wa[fn] = ws[(wrow + fn * 16) * 4 + jw];
      wb[fn] = ws[(wrow + fn * 16) * 4 + jw + 1];
    }
  }
  __device__ __forceinline__ static void sp_decode(uint32_t wa, uint32_t wb, int o5, u32x4 &a, uint32_t &idx) {
    const uint32_t F = (((wa & 0x3FFFFFFFu) >> o5) | (wb << (30 - o5))) & 0xFFFFFu;
    sp24_operand(F, a, idx);
  }

  // B operand of token block fm in a stage: columns 8 g .. 8 g + 7 and
  // 32 + 8 g .. 32 + 8 g + 7 (the sparse operand layout).
  __device__ __forceinline__ static u32x8 xop_sp(const uint32_t *stage, int r0, int g, int fm) {
    const u32x4 lo = xread(stage, r0 + fm * 16, g), hi = xread(stage, r0 + fm * 16, 4 + g);
    return (u32x8){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
  }

  static constexpr int XDS = 2;  // sparse: B operands read this many token blocks ahead
  // More weight fragments per wave than second-half token blocks after the
  // window read: the next step's operands are decoded in place, each right
  // after its fragment's last sparse MFMA of the step (one operand set in
  // registers; 2048 x 4096 x {4096, 11008} over prepared metadata 52.0 /
  // 124.0 -> 50.5 / 120.5 us against a second set filled over the half).
  static constexpr bool SP_INPLACE = FN > FM - FM / 2 - 1;

  // The 2:4 K loop: the schedule of run() with one sparse MFMA per
  // (row block, token block) and step; the first half of a step covers token
  // blocks 0 .. FM/2-1, the second half the rest plus the next stage's loads,
  // window reads and operand decode. Requires K % 64 == 0.
  // s0 / nsteps: the steps (64 columns each) multiplied, default all of K;
  // X and W stay addressed from column 0 (a step's metadata window depends
  // on its absolute index).
  // PREP: W is the prepared form of the metadata (sp24p_operand: one word
  // per row, step and lane group, [N][K/16] words like the dense codes), so
  // the stage loads are the dense engine's and a fragment's operand is one
  // LDS word; wpr is unused.
  // ldx: X row stride in elements (default K). WRAP: X has 2K columns (an
  // fp32 activation as bf16 hi | lo halves of each row) and steps K/64 ..
  // 2K/64 - 1 multiply them by the weight steps 0 .. K/64 - 1 again.
  template <bool PREP = false, bool WRAP = false>
  __device__ static void run_sp(uint32_t *lds, const uint16_t *X, uint32_t xbytes, int m_count,
                                const uint32_t *W, int n_count, int K, int wpr, f32x4 (&acc)[FN][FM], int s0 = 0,
                                int nsteps = -1, int ldx = 0) {
    static_assert(NS >= 3 && FM % 2 == 0 && FM / 2 >= XDS, "sparse schedule");
    constexpr int LP = PREP ? LPW : SLPW;  // load instructions per wave per stage
    constexpr int WL = PREP ? WPW : SWPW;
    if (ldx == 0) ldx = K;
    const int nkw = K >> 6;  // weight steps
    auto wstep = [&](int s) { return WRAP && s >= nkw ? s - nkw : s; };
    uint32_t xv[XPW], wv[WL];
    __amdgpu_buffer_rsrc_t wr[PREP ? WPW : 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if constexpr (PREP) {
      lane_offsets(xv, wv, nullptr, m_count, n_count, ldx, K, false, 0u);
#pragma unroll
      for (int i = 0; i < WPW; i++) wr[i] = buffer_rsrc(W, (uint32_t)n_count * (uint32_t)(K >> 4) * 4u);
    } else {
#pragma unroll
      for (int i = 0; i < XPW; i++) {
        const int r = (wave * XPW + i) * 8 + (lane >> 3);
        const int rm = min(r, m_count - 1);
        const uint32_t c = (lane & 7) ^ xswz(r);
        xv[i] = (uint32_t)rm * (uint32_t)ldx * 2u + 16u * c;
      }
#pragma unroll
      for (int i = 0; i < SWPW; i++) {
        const int n = min((wave * SWPW + i) * 16 + (lane >> 2), n_count - 1);
        wv[i] = ((uint32_t)n * (uint32_t)wpr + (uint32_t)(lane & 3)) * 4u;
      }
      wr[0] = buffer_rsrc(W, (uint32_t)n_count * (uint32_t)wpr * 4u);
    }
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(X, xbytes);
    auto load = [&](uint32_t *stage, int s) {
      if constexpr (PREP) issue(stage, xr, wr, xv, wv, 64 * s, 64 * wstep(s));
      else issue_sp(stage, xr, wr[0], xv, wv, s, wstep(s));
    };
#pragma unroll
    for (int fn = 0; fn < FN; fn++)
#pragma unroll
      for (int fm = 0; fm < FM; fm++) acc[fn][fm] = (f32x4){0.f, 0.f, 0.f, 0.f};
    const int wm = wave % WM, wn = wave / WM;
    const int l16 = lane & 15, g = lane >> 4;
    const int r0 = wm * TM + l16;
    const int wrow = wn * TN + l16;
    const int nks = nsteps < 0 ? (K + 63) >> 6 : nsteps;
    // the fragment words of step s from its W stage, and their operands
    auto wread = [&](const uint32_t *ws, int s, uint32_t (&wa)[FN], uint32_t (&wb)[FN], int &o5) {
      if constexpr (PREP) {
#pragma unroll
        for (int fn = 0; fn < FN; fn++) wa[fn] = ws[(wrow + fn * 16) * 4 + g];
      } else {
        sp_read(ws, s, wrow, g, wa, wb, o5);
      }
    };
    auto decode = [&](uint32_t wa, uint32_t wb, int o5, u32x4 &a, uint32_t &ix) {
      if constexpr (PREP) sp24p_operand(wa, a, ix);
      else sp_decode(wa, wb, o5, a, ix);
    };

#pragma unroll
    for (int s = 0; s < NS - 1; s++) load(lds + s * STAGE, s0 + min(s, nks - 1));
    wait_vmcnt<(NS - 2) * LP>();
    barrier_nofence();

    u32x4 a[FN];
    uint32_t ix[FN];
    u32x8 bn[XDS];
    {
      uint32_t wa[FN], wb[FN];
      int o5 = 0;
      wread(lds + XSTAGE, wstep(s0), wa, wb, o5);
#pragma unroll
      for (int d = 0; d < XDS; d++) bn[d] = xop_sp(lds, r0, g, d);
#pragma unroll
      for (int fn = 0; fn < FN; fn++) decode(wa[fn], wb[fn], o5, a[fn], ix[fn]);
    }

    for (int t = 0; t < nks; t++) {
      const uint32_t *cur = lds + (t % NS) * STAGE;
      const uint32_t *nxt = lds + ((t + 1) % NS) * STAGE;
      u32x8 b[FM];
#pragma unroll
      for (int d = 0; d < XDS; d++) b[d] = bn[d];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int fm = 0; fm < FM / 2; fm++) {
        b[fm + XDS] = xop_sp(cur, r0, g, fm + XDS);
#pragma unroll
        for (int fn = 0; fn < FN; fn++) smfmac16_acc(acc[fn][fm], a[fn], b[fm], ix[fn]);
        __builtin_amdgcn_sched_barrier(0);
      }
      wait_vmcnt<(NS - 3) * LP>();
      barrier_nofence();
      __builtin_amdgcn_sched_barrier(0);
      uint32_t wa[FN], wb[FN];
      int o5 = 0;
      u32x4 an[FN];
      uint32_t ixn[FN];
#pragma unroll
      for (int fm = FM / 2; fm < FM; fm++) {
        if (fm + XDS < FM) b[fm + XDS] = xop_sp(cur, r0, g, fm + XDS);
        else bn[fm + XDS - FM] = xop_sp(nxt, r0, g, fm + XDS - FM);
        if (fm == FM / 2) wread(nxt + XSTAGE, wstep(s0 + t + 1), wa, wb, o5);
        if (SP_INPLACE && fm == FM - 1) {
          // the next step's operands decoded into a[fn] right after its last
          // use (more fragments than decode slots: no second operand set)
#pragma unroll
          for (int fn = 0; fn < FN; fn++) {
            smfmac16_acc(acc[fn][fm], a[fn], b[fm], ix[fn]);
            decode(wa[fn], wb[fn], o5, a[fn], ix[fn]);
          }
        } else {
#pragma unroll
          for (int fn = 0; fn < FN; fn++) smfmac16_acc(acc[fn][fm], a[fn], b[fm], ix[fn]);
        }
        if (fm == FM / 2) load(lds + ((t + NS - 1) % NS) * STAGE, s0 + min(t + NS - 1, nks - 1));
        if (!SP_INPLACE && fm > FM / 2 && fm - FM / 2 - 1 < FN) {
          const int fn = fm - FM / 2 - 1;
          decode(wa[fn], wb[fn], o5, an[fn], ixn[fn]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (!SP_INPLACE) {
#pragma unroll
        for (int fn = FM / 2 - 1; fn < FN; fn++) decode(wa[fn], wb[fn], o5, an[fn], ixn[fn]);
#pragma unroll
        for (int fn = 0; fn < FN; fn++) {
          a[fn] = an[fn];
          ix[fn] = ixn[fn];
        }
      }
    }
    mfma_drain();
    wait_vmcnt<0>();
    barrier_nofence();
  }

  // Epilogue: Y[m][n] = acc * 0.5 * scale[n] for the tile's m_count x n_count
  // valid outputs (0.5 undoes the 2*dec(c) operand encoding). The raw fp32
  // accumulators go to the LDS ring straight from the accumulation registers,
  // in P passes of BM/P tokens (row = token, weight rows contiguous, rows
  // padded by 16 floats so that the fragment writes of 16 tokens spread over
  // all banks). The block then writes whole 16-byte chunks of output rows
  // with a rolled loop in which each thread owns one column chunk (its scales
  // load once). Stores cover full cache lines and the code stays compact: a
  // fully unrolled per-fragment store sequence is tens of KB that each
  // workgroup runs once, and fetching it costs more than the stores.
  // RAW: the accumulators as they are (scale unused), e.g. the fp32 partial
  // sums of a K part that a later launch scales.
  template <typename YT, bool RAW = false>
  __device__ static void store_tile(uint32_t *lds, const f32x4 (&acc)[FN][FM],
                                    const float *scale, YT *Y, size_t ldy, int m0, int m_count,
                                    int n0, int n_count, const float *bias = nullptr) {
    constexpr int ES = sizeof(YT);
    constexpr int PF = BN + 16;  // LDS row pitch in floats
    constexpr int P = (BM / 2) * PF * 4 <= LDS_DWORDS * 4 ? 2 : 4;
    static_assert(FM % P == 0 && (BM / P) * PF * 4 <= LDS_DWORDS * 4, "epilogue staging");
    constexpr int FMP = FM / P, RP = BM / P, TMP = TM / P;
    constexpr int CE = 16 / ES;   // output elements per 16-byte chunk
    constexpr int CR = BN / CE;   // chunks per output row
    static_assert(NT % CR == 0, "each thread owns one column chunk");
    constexpr int RI = NT / CR;   // rows per iteration
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave % WM, wn = wave / WM, l16 = lane & 15, g = lane >> 4;
    float *st = reinterpret_cast<float *>(lds);
    const int c = threadIdx.x % CR, r0 = threadIdx.x / CR;
    const int nl = c * CE;
    float sc[CE];
#pragma unroll
    for (int e = 0; e < CE; e++) sc[e] = RAW ? 1.0f : 0.5f * scale[n0 + min(nl + e, n_count - 1)];
    float bv[CE];  // row bias (added after the scale, its own rounding)
#pragma unroll
    for (int e = 0; e < CE; e++) bv[e] = bias ? bias[n0 + min(nl + e, n_count - 1)] : 0.f;
    const bool vec = ((reinterpret_cast<uintptr_t>(Y) | (ldy * ES) | ((size_t)n0 * ES)) & 15) == 0;
    const bool full = vec && nl + CE <= n_count;
#pragma unroll
    for (int p = 0; p < P; p++) {
#pragma unroll
      for (int fn = 0; fn < FN; fn++)
#pragma unroll
        for (int fmi = 0; fmi < FMP; fmi++)
          *reinterpret_cast<f32x4 *>(st + (wm * TMP + fmi * 16 + l16) * PF + wn * TN + fn * 16 + 4 * g) =
              acc[fn][p * FMP + fmi];
      __syncthreads();
      for (int lr = r0; lr < RP; lr += RI) {
        const int m = (lr / TMP) * TM + p * TMP + lr % TMP;  // token within the tile
        if (m >= m_count || nl >= n_count) continue;
        const float *src = st + lr * PF + nl;
        float v[CE];
#pragma unroll
        for (int e = 0; e < CE; e += 4) {
          const f32x4 q = *reinterpret_cast<const f32x4 *>(src + e);
          v[e] = q.x * sc[e];
          v[e + 1] = q.y * sc[e + 1];
          v[e + 2] = q.z * sc[e + 2];
          v[e + 3] = q.w * sc[e + 3];
        }
        if (bias) {
#pragma unroll
          for (int e = 0; e < CE; e++) v[e] = add_bias(v[e], bv[e]);
        }
        YT *d = Y + (size_t)(m0 + m) * ldy + n0 + nl;
        if constexpr (ES == 4) {
          if (full) {
            *reinterpret_cast<f32x4 *>(d) = (f32x4){v[0], v[1], v[2], v[3]};
          } else {
            for (int e = 0; e < CE && nl + e < n_count; e++) d[e] = v[e];
          }
        } else {
          uint32_t h[CE];
#pragma unroll
          for (int e = 0; e < CE; e++) h[e] = bf16_rne_nb(v[e]);
          if (full) {
            *reinterpret_cast<u32x4 *>(d) = (u32x4){h[0] | (h[1] << 16), h[2] | (h[3] << 16),
                                                   h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
          } else {
            for (int e = 0; e < CE && nl + e < n_count; e++) d[e] = (uint16_t)h[e];
          }
        }
      }
      __syncthreads();
    }
  }

  __device__ __forceinline__ static int tok(int fm) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    return (wave % WM) * TM + fm * 16 + (lane & 15);
  }
  __device__ __forceinline__ static int rowoff(int fn) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    return (wave / WM) * TN + fn * 16 + 4 * (lane >> 4);
  }
};

}  // namespace frx
