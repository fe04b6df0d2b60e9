// frx_gemm_core.hpp — MFMA tile engine for ternary-weight GEMMs on gfx950.
//
// C[BN rows of W][BM tokens] += dec(W)[n][k] * X[m][k] for one workgroup tile,
// with v_mfma_f32_16x16x32_bf16 (A = weight rows, B = tokens, fp32 acc).
//
// Per K-step of 64 columns, double-buffered in LDS:
//  - X tile [P planes][BM tokens][64 cols] bf16, K-interleaved per 16-column
//    block (dword i = x[i] | x[i+8] << 16), row stride 36 dwords so the 16
//    token rows of one 16-byte read hit disjoint banks.
//  - W tile [NW matrices][BN rows][4 words] packed u32, exactly the
//    reference layout; each wave unpacks its rows' words to bf16 operands in
//    registers (frx_device.hpp), so the unpacked tile never exists in memory.
// Global loads for step s+1 are issued before the MFMAs of step s and land
// in the other LDS buffer afterwards (one barrier per step).
//
// X sources: XS_BF16 (one plane), XS_F32 (split into hi/lo planes at
// staging), XS_BF16X2 (two precomputed bf16 planes). Rows may be gathered
// through an index list (MoE token permutation).
#pragma once
#include "frx_device.hpp"

namespace frx {

enum { XS_BF16 = 0, XS_F32 = 1, XS_BF16X2 = 2 };
enum { WF_DENSE = 0, WF_SP24 = 1 };

// 2:4 group field (5 bits: pattern[2:0], sign_lo[3], sign_hi[4], sign 1 =
// -1; src/compute/kernels/sparse_ternary.rs:84-100) -> one byte of four dense
// 2-bit codes. Pattern values 6, 7 clamp to 5 as in the WGSL (:91).
__host__ __device__ constexpr uint32_t sp24_code_byte(uint32_t f) {
  uint32_t p = f & 7u;
  if (p > 5u) p = 5u;
  const uint32_t a = (0x940u >> (2 * p)) & 3u;  // lower position per pattern
  const uint32_t b = (0xFB9u >> (2 * p)) & 3u;  // higher position
  const uint32_t ca = ((f >> 3) & 1u) ? 0u : 2u;
  const uint32_t cb = ((f >> 4) & 1u) ? 0u : 2u;
  uint32_t byte = 0x55u;  // four zero codes
  byte = (byte & ~(3u << (2 * a))) | (ca << (2 * a));
  byte = (byte & ~(3u << (2 * b))) | (cb << (2 * b));
  return byte;
}

// Transcodes 8 consecutive 2:4 groups starting at bit 5*PH of word w[0] into
// two dense code words (32 columns). LUT = 32 code bytes in LDS.
template <int PH>
__device__ __forceinline__ void sp24_transcode8(const uint32_t w[3],
                                                const uint8_t *lut,
                                                int valid, uint32_t &c0,
                                                uint32_t &c1) {
  uint32_t out[2] = {0u, 0u};
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int pos = PH + j;
    const uint32_t f = (w[pos / 6] >> (5 * (pos % 6))) & 31u;
    const uint32_t byte = j < valid ? (uint32_t)lut[f] : 0x55u;
    out[j >> 2] |= byte << (8 * (j & 3));
  }
  c0 = out[0];
  c1 = out[1];
}

struct XDesc {
  const void *x0;     // bf16 or f32 rows (hi plane for XS_BF16X2)
  const void *x1;     // lo plane for XS_BF16X2
  const int *rowidx;  // optional: global row of tile row m = rowidx[m]
  long row0;          // used when rowidx == nullptr: global row = row0 + m
  int ldx;            // row stride in elements
  int xvec;           // rows are 16-byte aligned (vector loads allowed)
};

template <int BM, int BN, int WM, int WN, int XS, int NW, int WF = WF_DENSE>
struct GemmCore {
  static constexpr int NT = WM * WN * 64;
  static constexpr int P = XS == XS_BF16 ? 1 : 2;
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int FM = TM / 16, FN = TN / 16;
  static constexpr int RS = 36;  // dwords per token row per plane
  static constexpr int XPLANE = BM * RS;
  static constexpr int XSTAGE = P * XPLANE;
  static constexpr int WSTAGE = NW * BN * 4;
  static constexpr int STAGE = XSTAGE + WSTAGE;
  static constexpr int LUT_DWORDS = WF == WF_SP24 ? 8 : 0;
  static constexpr int LDS_DWORDS = 2 * STAGE + LUT_DWORDS;
  static constexpr int XB = (BM * 4 + NT - 1) / NT;       // X blocks / thread
  // dense: one thread per W row (4 words); 2:4: two threads per row (3
  // metadata words each, transcoded to 2 code words).
  static constexpr int WROWS = WF == WF_DENSE ? NW * BN : 2 * NW * BN;
  static constexpr int WB = (WROWS + NT - 1) / NT;
  static constexpr int XREG = XS == XS_F32 ? 16 : (XS == XS_BF16X2 ? 16 : 8);
  static_assert(TM % 16 == 0 && TN % 16 == 0, "wave tile must be 16-aligned");

  struct Regs {
    uint32_t x[XB][XREG];
    uint32_t w[WB][4];
    int wk;          // K-step start column of the loaded data (2:4 phase)
    int wvalid[WB];  // 2:4: groups of this half inside the row
  };

  __device__ __forceinline__ static long xrow(const XDesc &xd, int m) {
    return xd.rowidx ? (long)xd.rowidx[m] : xd.row0 + m;
  }

  // Global -> registers for the K-step starting at column k0.
  __device__ __forceinline__ static void load(Regs &R, const XDesc &xd,
                                              int m_count,
                                              const uint32_t *const *Wm,
                                              int n0, int N, int K, int k0,
                                              int wvec) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < XB; i++) {
      const int b = tid + i * NT;
      const int m = b >> 2, blk = b & 3;
      const int col = k0 + blk * 16;
      const bool ok = (b < BM * 4) && (m < m_count) && (col < K);
      if (ok && (col + 16 > K || !xd.xvec)) {
        // partial block (K % 16 != 0) or unaligned rows: element-wise, zero
        // beyond K
        const long gr = xrow(xd, m);
        const int nv = K - col;
        if constexpr (XS == XS_BF16) {
          const uint16_t *s = reinterpret_cast<const uint16_t *>(xd.x0) + gr * xd.ldx + col;
#pragma unroll
          for (int j = 0; j < 8; j++) {
            uint32_t lo = 2 * j < nv ? s[2 * j] : 0u, hi = 2 * j + 1 < nv ? s[2 * j + 1] : 0u;
            R.x[i][j] = lo | (hi << 16);
          }
        } else if constexpr (XS == XS_F32) {
          const uint32_t *s = reinterpret_cast<const uint32_t *>(xd.x0) + gr * xd.ldx + col;
#pragma unroll
          for (int j = 0; j < 16; j++) R.x[i][j] = j < nv ? s[j] : 0u;
        } else {
          const uint16_t *s = reinterpret_cast<const uint16_t *>(xd.x0) + gr * xd.ldx + col;
          const uint16_t *t = reinterpret_cast<const uint16_t *>(xd.x1) + gr * xd.ldx + col;
#pragma unroll
          for (int j = 0; j < 8; j++) {
            R.x[i][j] = (2 * j < nv ? s[2 * j] : 0u) | ((2 * j + 1 < nv ? s[2 * j + 1] : 0u) << 16);
            R.x[i][8 + j] = (2 * j < nv ? t[2 * j] : 0u) | ((2 * j + 1 < nv ? t[2 * j + 1] : 0u) << 16);
          }
        }
      } else if (ok) {
        const long gr = xrow(xd, m);
        if constexpr (XS == XS_BF16) {
          const u32x4 *s = reinterpret_cast<const u32x4 *>(
              reinterpret_cast<const uint16_t *>(xd.x0) + gr * xd.ldx + col);
          u32x4 a = s[0], c = s[1];
          R.x[i][0] = a.x; R.x[i][1] = a.y; R.x[i][2] = a.z; R.x[i][3] = a.w;
          R.x[i][4] = c.x; R.x[i][5] = c.y; R.x[i][6] = c.z; R.x[i][7] = c.w;
        } else if constexpr (XS == XS_F32) {
          const u32x4 *s = reinterpret_cast<const u32x4 *>(
              reinterpret_cast<const float *>(xd.x0) + gr * xd.ldx + col);
#pragma unroll
          for (int q = 0; q < 4; q++) {
            u32x4 a = s[q];
            R.x[i][4 * q + 0] = a.x; R.x[i][4 * q + 1] = a.y;
            R.x[i][4 * q + 2] = a.z; R.x[i][4 * q + 3] = a.w;
          }
        } else {
          const u32x4 *s = reinterpret_cast<const u32x4 *>(
              reinterpret_cast<const uint16_t *>(xd.x0) + gr * xd.ldx + col);
          const u32x4 *t = reinterpret_cast<const u32x4 *>(
              reinterpret_cast<const uint16_t *>(xd.x1) + gr * xd.ldx + col);
          u32x4 a = s[0], c = s[1], d = t[0], e = t[1];
          R.x[i][0] = a.x; R.x[i][1] = a.y; R.x[i][2] = a.z; R.x[i][3] = a.w;
          R.x[i][4] = c.x; R.x[i][5] = c.y; R.x[i][6] = c.z; R.x[i][7] = c.w;
          R.x[i][8] = d.x; R.x[i][9] = d.y; R.x[i][10] = d.z; R.x[i][11] = d.w;
          R.x[i][12] = e.x; R.x[i][13] = e.y; R.x[i][14] = e.z; R.x[i][15] = e.w;
        }
      } else {
#pragma unroll
        for (int j = 0; j < XREG; j++) R.x[i][j] = 0u;
      }
    }
    R.wk = k0;
    if constexpr (WF == WF_SP24) {
      const int gpr = (K + 3) >> 2, wpr = (gpr + 5) / 6;
#pragma unroll
      for (int i = 0; i < WB; i++) {
        const int rt = tid + i * NT;
        const int rr = rt >> 1, hf = rt & 1;
        const int mat = rr / BN, n = n0 + (rr - mat * BN);
        const bool rok = (rt < WROWS) && (n < N);
        const int G0 = (k0 >> 2) + 8 * hf;  // first group of this half
        const int w0 = G0 / 6;
        const uint32_t *src = rok ? Wm[mat] + (size_t)n * wpr : nullptr;
#pragma unroll
        for (int q = 0; q < 3; q++)
          R.w[i][q] = (rok && w0 + q < wpr) ? src[w0 + q] : 0u;
        R.w[i][3] = 0u;
        R.wvalid[i] = rok ? min(8, max(0, gpr - G0)) : 0;
      }
      return;
    }
    const int wpr = K >> 4, kw = k0 >> 4;
#pragma unroll
    for (int i = 0; i < WB; i++) {
      const int rr = tid + i * NT;
      const int mat = rr / BN, n = n0 + (rr - mat * BN);
      const bool rok = (rr < NW * BN) && (n < N);
      const uint32_t *src = rok ? Wm[mat] + (size_t)n * wpr + kw : nullptr;
      if (rok && wvec && kw + 4 <= wpr) {
        u32x4 v = *reinterpret_cast<const u32x4 *>(src);
        R.w[i][0] = v.x; R.w[i][1] = v.y; R.w[i][2] = v.z; R.w[i][3] = v.w;
      } else {
#pragma unroll
        for (int q = 0; q < 4; q++)
          R.w[i][q] = (rok && kw + q < wpr) ? src[q] : 0xFFFFFFFFu;
      }
    }
  }

  // Registers -> LDS stage buffer (interleave / split on the way).
  __device__ __forceinline__ static void store(const Regs &R, uint32_t *buf,
                                               const uint32_t *lut32) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < XB; i++) {
      const int b = tid + i * NT;
      if (b >= BM * 4) break;
      const int m = b >> 2, blk = b & 3;
      uint32_t *d0 = buf + m * RS + blk * 8;
      if constexpr (XS == XS_BF16) {
        uint32_t d[8];
        interleave16(R.x[i], d);
        reinterpret_cast<u32x4 *>(d0)[0] = (u32x4){d[0], d[1], d[2], d[3]};
        reinterpret_cast<u32x4 *>(d0)[1] = (u32x4){d[4], d[5], d[6], d[7]};
      } else if constexpr (XS == XS_F32) {
        uint32_t h[16], l[16];
#pragma unroll
        for (int j = 0; j < 16; j++) split_bf16(__uint_as_float(R.x[i][j]), h[j], l[j]);
        uint32_t dh[8], dl[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
          dh[j] = h[j] | (h[j + 8] << 16);
          dl[j] = l[j] | (l[j + 8] << 16);
        }
        reinterpret_cast<u32x4 *>(d0)[0] = (u32x4){dh[0], dh[1], dh[2], dh[3]};
        reinterpret_cast<u32x4 *>(d0)[1] = (u32x4){dh[4], dh[5], dh[6], dh[7]};
        uint32_t *d1 = d0 + XPLANE;
        reinterpret_cast<u32x4 *>(d1)[0] = (u32x4){dl[0], dl[1], dl[2], dl[3]};
        reinterpret_cast<u32x4 *>(d1)[1] = (u32x4){dl[4], dl[5], dl[6], dl[7]};
      } else {
        uint32_t dh[8], dl[8];
        interleave16(&R.x[i][0], dh);
        interleave16(&R.x[i][8], dl);
        reinterpret_cast<u32x4 *>(d0)[0] = (u32x4){dh[0], dh[1], dh[2], dh[3]};
        reinterpret_cast<u32x4 *>(d0)[1] = (u32x4){dh[4], dh[5], dh[6], dh[7]};
        uint32_t *d1 = d0 + XPLANE;
        reinterpret_cast<u32x4 *>(d1)[0] = (u32x4){dl[0], dl[1], dl[2], dl[3]};
        reinterpret_cast<u32x4 *>(d1)[1] = (u32x4){dl[4], dl[5], dl[6], dl[7]};
      }
    }
    uint32_t *wb = buf + XSTAGE;
    if constexpr (WF == WF_SP24) {
      const uint8_t *lut = reinterpret_cast<const uint8_t *>(lut32);
#pragma unroll
      for (int i = 0; i < WB; i++) {
        const int rt = tid + i * NT;
        if (rt >= WROWS) break;
        const int rr = rt >> 1, hf = rt & 1;
        const int G0 = (R.wk >> 2) + 8 * hf;
        const int valid = R.wvalid[i];
        uint32_t c0, c1;
        switch (G0 % 6) {
          case 0: sp24_transcode8<0>(R.w[i], lut, valid, c0, c1); break;
          case 2: sp24_transcode8<2>(R.w[i], lut, valid, c0, c1); break;
          default: sp24_transcode8<4>(R.w[i], lut, valid, c0, c1); break;
        }
        reinterpret_cast<u32x2 *>(wb + rr * 4 + 2 * hf)[0] = (u32x2){c0, c1};
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < WB; i++) {
      const int rr = tid + i * NT;
      if (rr >= NW * BN) break;
      reinterpret_cast<u32x4 *>(wb + rr * 4)[0] =
          (u32x4){R.w[i][0], R.w[i][1], R.w[i][2], R.w[i][3]};
    }
  }

  // MFMAs for one LDS stage.
  __device__ __forceinline__ static void compute(const uint32_t *buf,
                                                 f32x4 (&acc)[NW][FN][FM]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave % WM, wn = wave / WM;
    const int l16 = lane & 15, g = lane >> 4;
    uint32_t nw[NW][FN];
    const uint32_t *wb = buf + XSTAGE;
#pragma unroll
    for (int mat = 0; mat < NW; mat++)
#pragma unroll
      for (int fn = 0; fn < FN; fn++)
        nw[mat][fn] = wb[(mat * BN + wn * TN + fn * 16 + l16) * 4 + g];
#pragma unroll
    for (int h = 0; h < 2; h++) {
      u32x4 bx[P][FM];
#pragma unroll
      for (int p = 0; p < P; p++)
#pragma unroll
        for (int fm = 0; fm < FM; fm++)
          bx[p][fm] = *reinterpret_cast<const u32x4 *>(
              buf + p * XPLANE + (wm * TM + fm * 16 + l16) * RS + g * 8 + h * 4);
#pragma unroll
      for (int mat = 0; mat < NW; mat++)
#pragma unroll
        for (int fn = 0; fn < FN; fn++) {
          const u32x4 a = h == 0 ? unpack_half_m<0>(nw[mat][fn], 0xC000C000u)
                                 : unpack_half_m<1>(nw[mat][fn], 0xC000C000u);
#pragma unroll
          for (int fm = 0; fm < FM; fm++)
#pragma unroll
            for (int p = 0; p < P; p++)
              acc[mat][fn][fm] = mfma16(a, bx[p][fm], acc[mat][fn][fm]);
        }
    }
  }

  __device__ static void run(uint32_t *lds, const XDesc &xd, int m_count,
                             const uint32_t *const *Wm, int n0, int N, int K,
                             int wvec, f32x4 (&acc)[NW][FN][FM]) {
#pragma unroll
    for (int mat = 0; mat < NW; mat++)
#pragma unroll
      for (int fn = 0; fn < FN; fn++)
#pragma unroll
        for (int fm = 0; fm < FM; fm++) acc[mat][fn][fm] = (f32x4){0.f, 0.f, 0.f, 0.f};
    const int nks = (K + 63) >> 6;
    uint32_t *lut = lds + 2 * STAGE;
    if constexpr (WF == WF_SP24) {
      if (threadIdx.x < 8) {
        uint32_t v = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) v |= sp24_code_byte(4 * threadIdx.x + j) << (8 * j);
        lut[threadIdx.x] = v;
      }
      __syncthreads();
    }
    Regs R;
    load(R, xd, m_count, Wm, n0, N, K, 0, wvec);
    store(R, lds, lut);
    __syncthreads();
    for (int s = 0; s < nks; s++) {
      uint32_t *cur = lds + (s & 1) * STAGE;
      uint32_t *nxt = lds + ((s + 1) & 1) * STAGE;
      const bool more = s + 1 < nks;
      if (more) load(R, xd, m_count, Wm, n0, N, K, (s + 1) * 64, wvec);
      compute(cur, acc);
      if (more) store(R, nxt, lut);
      __syncthreads();
    }
  }

  // Epilogue coordinates of accumulator (mat, fn, fm), register j:
  //   token  m = wm*TM + fm*16 + lane%16
  //   row    n = n0 + wn*TN + fn*16 + 4*(lane/16) + j
  __device__ __forceinline__ static int tok(int fm) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    return (wave % WM) * TM + fm * 16 + (lane & 15);
  }
  __device__ __forceinline__ static int rowoff(int fn) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    return (wave / WM) * TN + fn * 16 + 4 * (lane >> 4);
  }
};

__device__ __forceinline__ f32x4 load_scale4(const float *s, int n, int nok) {
  f32x4 v;
  v.x = s[n];
  v.y = nok > 1 ? s[n + 1] : 0.f;
  v.z = nok > 2 ? s[n + 2] : 0.f;
  v.w = nok > 3 ? s[n + 3] : 0.f;
  return v;
}

}  // namespace frx
