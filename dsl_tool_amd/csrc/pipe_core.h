// Pipelined GEMM mainloop for gfx950 (shared by the dense and grouped
// kernels): C[M,N] = A[M,K] . W[N,K]^T with both operands packed K-major
// (FP8: 1 byte per element, FP4: 2 per byte).
//
// Data path
//   * K advances in stages of SKB bytes per row (64 or 128; FP8: SKB
//     elements, FP4: 2*SKB).  NS stages form a ring in LDS.  128-byte stages
//     read whole 128-byte cache lines per row, which halves the L2 -> L1
//     traffic of 64-byte stages (the L1 cannot keep the other half of a
//     line until the next stage needs it).
//   * Every stage is copied global -> LDS by the direct-to-LDS load
//     (global_load_lds_dwordx4: 16 bytes per lane, the wave's 64 lanes fill
//     1 KB of LDS contiguously), so no VGPRs hold in-flight tiles.  The
//     loads of stage ks+NS-1 are issued right after the barrier that opens
//     stage ks, which leaves NS-1 stages in flight behind the MFMAs.
//   * The loads are issued from inline asm: the compiler then does not
//     track them as LDS writes (it would put a vmcnt(0) in front of every
//     LDS read); completion is waited for explicitly with s_waitcnt vmcnt
//     before the barrier that publishes a stage to the workgroup.
//   * LDS rows are SKB bytes of 16-byte chunks, XOR-swizzled (swz below).
//   * MXFP4 scales (SKB/16 E8M0 bytes per row per stage) ride along in the
//     same ring via 4-byte direct loads and go straight into the scaled MFMA.
//
// Operand layout of v_mfma_scale_f32_32x32x64_f8f6f4 used here: lane l
// supplies row l%32 of its operand and K half h = l/32 (FP8: 32 bytes,
// FP4: 16 bytes = 32 elements = one E8M0 block); output register i of lane
// l is C[8*(i/4) + 4*h + i%4][l%32].
#pragma once

#include "gemm_core.h"

#pragma clang diagnostic ignored "-Winline-asm"

namespace dsl {

namespace pipe {

DSL_DEV uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// 16 bytes per lane from `src` into LDS at m0 + lane*16.  gfx9 needs one
// wait state between an SALU write of m0 and an LDS-DMA instruction that
// reads it (the compiler's hazard recognizer cannot see into inline asm),
// hence the s_nop.
DSL_DEV void dma16(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src),
               "s"(lds)
               : "memory", "m0");
}
// 4 bytes per lane from `src` into LDS at m0 + lane*4.
DSL_DEV void dma4(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src),
               "s"(lds)
               : "memory", "m0");
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8], vmcnt[5:4] in bits [15:14]).
template <int N>
DSL_DEV void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// LDS row swizzle: chunk c of row r lives in slot c ^ swz<SKB>(r).
//
// gfx950 serves a 16-byte read (ds_read_b128) in four cycles over 64 banks
// of 4 bytes, all 64 lanes each cycle: in cycle t lane l reads dword
// (t + f(l)) & 3 of its 16 bytes, with f(l) = (l >> 4) ^ (bit 2 ^ bit 3 of l).
// That model reproduces the bank-conflict counts measured for about 80
// read patterns (SQ_LDS_BANK_CONFLICT).  Under it, the earlier 128-byte swizzle
// (r >> 1) & 7 served the 32x32 fragments (lane = row, 2 chunks per row)
// without conflicts but doubled the cycles of the 16x16x128 fragments (lane
// l & 15 = row, 4 chunks per row in one read) and of the one-chunk FP4
// fragments.  The 128-byte swizzle below, r1 * 1 ^ r2 * 4 ^ r3 * 7 ^ r4 * 2
// (r_b = bit b of the row), leaves all of the pipelined kernels' readers
// conflict-free: 32x32 FP8 (chunks 4k + 2h, +1), FP4 (2k + h), and 16x16x128
// (2g, 2g + 1) at every 16-row base.  With 64-byte rows four rows share a
// 256-byte bank line and (r >> 2) & 3 spreads them.
template <int SKB>
DSL_DEV int swz(int row) {
  if constexpr (SKB == 64) return (row >> 2) & 3;
  return ((row >> 1) & 1) ^ (((row >> 2) & 1) * 4) ^ (((row >> 3) & 1) * 7) ^ (((row >> 4) & 1) * 2);
}

// FP4 x FP4 32x32x64 scaled MFMA; OPS picks the scale byte of sa / sb.
template <int OPS>
DSL_DEV v16f mfma_fp4(const v4i &a, const v4i &b, const v16f &c, int sa, int sb) {
  const v8i a8 = {a[0], a[1], a[2], a[3], 0, 0, 0, 0};
  const v8i b8 = {b[0], b[1], b[2], b[3], 0, 0, 0, 0};
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, c, 4, 4, OPS, sa, OPS, sb);
}

}  // namespace pipe

template <int MODE_, int BM_, int BN_, int WGM_, int WGN_, int NS_, int SKB_ = 64, int OCC_ = 0,
          int PF_ = 0>
struct PipeCfg {
  static constexpr int MODE = MODE_, BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_, NS = NS_;
  static constexpr bool PF = PF_ != 0;                      // fragment prefetch schedule
  static constexpr int SKB = SKB_;                          // stage bytes per row
  static constexpr int NW = WGM * WGN, NT = NW * 64;
  static constexpr int OCC = OCC_ > 0 ? OCC_ : (NW >= 8 ? 2 : 1);   // waves per SIMD
  static constexpr int WM = BM / WGM, WN = BN / WGN, TM = WM / 32, TN = WN / 32;
  static constexpr bool MX = MODE == MODE_MXFP4;
  static constexpr bool NV = MODE == MODE_NVFP4;
  static constexpr bool FP4 = MX || NV;
  static constexpr bool BF16 = MODE == MODE_BF16;           // 64-byte k-step = 32 bf16 of K
  static constexpr bool BLOCK = mode_grouped_k(MODE);       // one 128-K scale group per stage
  static constexpr bool GCOL = MODE == MODE_FP8_GCOL;       // ... with a weight scale per column
  static constexpr int CH = SKB / 16, RPI = 1024 / SKB;     // chunks per row, rows per DMA
  // MFMA steps per stage: 32x32x64 for FP8 / MXFP4; for NVFP4 a "step" is a
  // quad of four 32x32x16 fp16 MFMAs over 64 elements (32 bytes)
  static constexpr int KSTEPS = MX ? SKB / 32 : (NV ? SKB / 32 : SKB / 64);
  // scale words (4 bytes) per row per stage: E8M0 per 32, E4M3 per 16, fp32
  // per 128-K group (the block-scaled prefetch kernel keeps its activation
  // scales in a separate ring, SA_RING below, instead)
  static constexpr int SCW = MX ? SKB / 64 : (NV ? SKB / 32 : ((BLOCK && !PF) ? 1 : 0));
  static constexpr int A_BYTES = BM * SKB, B_BYTES = BN * SKB;
  // GCOL: the stage's weight scales sb[grp][n0 .. n0 + BN) ride along too
  static constexpr int SA_BYTES = BM * 4 * SCW, SB_BYTES = (FP4 || GCOL) ? BN * 4 * SCW : 0;
  static constexpr int STAGE = A_BYTES + B_BYTES + SA_BYTES + SB_BYTES;
  // block-scaled prefetch kernel: two slots of 4 groups x BM rows of fp32
  // activation scales, [slot][row][4 groups], plus a 1 KB dummy target
  static constexpr int SA_SET = BM * 16, SA_RING = (BLOCK && PF) ? 2 * SA_SET + 1024 : 0;
  static constexpr int LDS = NS * STAGE + SA_RING;
  static constexpr int A_DMA = A_BYTES / 1024, B_DMA = B_BYTES / 1024;
  static constexpr int SA_DMA = SA_BYTES / 256, SB_DMA = SB_BYTES / 256;
  static constexpr int DATA_DMA = A_DMA + B_DMA, SC_DMA = SA_DMA + SB_DMA;
  static constexpr int TOTAL_DMA = DATA_DMA + SC_DMA;
  // DMA instructions per wave per stage: an equal share of the operand data
  // and a round-robin share of the scale words, so waves issue D or D-1
  static constexpr int DD = DATA_DMA / NW, DS = (SC_DMA + NW - 1) / NW;
  static constexpr int D = DD + DS;
  // block scales: one fp32 per row per 128-K group; with 64-byte stages a
  // group spans two stages and both carry its scale words
  static constexpr int SC_SHIFT = (BLOCK && SKB == 64) ? 1 : 0;
  static_assert(SKB == 64 || SKB == 128, "stage width");
  static_assert(DATA_DMA % NW == 0, "operand DMA work must split evenly over the waves");
  static_assert(BM % 64 == 0 && BN % 64 == 0 && WM % 32 == 0 && WN % 32 == 0, "tile shape");
  static_assert(LDS <= 160 * 1024, "LDS budget");
  static_assert(NS >= 2 && (NS - 1) * D < 64, "ring depth / vmcnt range");
  static_assert(!PF || !NV, "the prefetch schedule covers FP8 and MXFP4");
  static_assert(!BLOCK || SKB == 128 || PF, "64-byte block-scaled stages use the prefetch schedule");
  static_assert(!GCOL || !PF, "per-column weight scales use the per-stage partial kernel");
};

namespace pipe {

// Direct-to-LDS copy plan of one thread: Cfg::DD operand-data DMA
// instructions (16 bytes per lane) and up to Cfg::DS scale-word DMA
// instructions (4 bytes per lane) per stage, all wave-uniform: their stage-0
// sources, LDS offsets within a stage and source advance per stage.
// `full` tells whether this wave issues all D of them (scale words are dealt
// round-robin, so some waves may issue D-1): its vmcnt waits count with it.
template <class Cfg>
struct Ring {
  const uint8_t *src[Cfg::D];
  uint32_t dst[Cfg::D];
  int step[Cfg::D];
  bool has[Cfg::D];     // scale-word slot used by this wave
  bool full;

  DSL_DEV void init(const GemmArgs &p, int m0, int n0, int wave, int lane) {
    constexpr int SKB = Cfg::SKB;
    full = true;
#pragma unroll
    for (int j = 0; j < Cfg::D; ++j) {
      src[j] = p.a;
      dst[j] = 0;
      step[j] = 0;
      has[j] = j < Cfg::DD;
      if (j < Cfg::DD) {
        const int i = wave * Cfg::DD + j;
        const bool isA = i < Cfg::A_DMA;
        const int lrow = (isA ? i : i - Cfg::A_DMA) * Cfg::RPI + lane / Cfg::CH;
        const int chunk = (lane % Cfg::CH) ^ swz<SKB>(lrow);
        const int lim = isA ? p.M - 1 : p.N - 1;
        int grow = (isA ? m0 : n0) + lrow;
        grow = grow > lim ? lim : grow;    // rows past the edge re-read the last row
        src[j] = (isA ? p.a : p.b) + (int64_t)grow * p.Kb + chunk * 16;
        dst[j] = i * 1024;
        step[j] = SKB;
      } else {
        const int si = (j - Cfg::DD) * Cfg::NW + wave;
        if (si >= Cfg::SC_DMA) {
          full = false;
          continue;
        }
        has[j] = true;
        const bool isA = si < Cfg::SA_DMA;
        const int rows = isA ? Cfg::BM : Cfg::BN;
        const int sidx = isA ? si : si - Cfg::SA_DMA;
        const int word = sidx / (rows / 64), rblk = sidx % (rows / 64);
        const int lrow = rblk * 64 + lane;
        const int lim = isA ? p.M - 1 : p.N - 1;
        int grow = (isA ? m0 : n0) + lrow;
        grow = grow > lim ? lim : grow;
        if constexpr (Cfg::GCOL) {
          if (isA) {                       // fp32 sa[row][K/128]: one float per row per group
            src[j] = reinterpret_cast<const uint8_t *>(static_cast<const float *>(p.sa) +
                                                       (int64_t)grow * (p.K / 128));
            step[j] = 4;
          } else {                         // fp32 sb[K/128][N]: the tile's columns of a group
            src[j] = reinterpret_cast<const uint8_t *>(static_cast<const float *>(p.sb) + grow);
            step[j] = 4 * p.N;
          }
        } else if constexpr (Cfg::BLOCK) { // fp32 sa[row][K/128]: one float per row per group
          src[j] = reinterpret_cast<const uint8_t *>(static_cast<const float *>(p.sa) +
                                                     (int64_t)grow * (p.K / 128));
          step[j] = 4;
        } else if constexpr (Cfg::MX) {    // E8M0 [row][K/32]: SKB/16 bytes per row per stage
          src[j] = static_cast<const uint8_t *>(isA ? p.sa : p.sb) + (int64_t)grow * (p.K / 32) +
                   word * 4;
          step[j] = SKB / 16;
        } else {                           // E4M3 [row][K/16]: SKB/8 bytes per row per stage
          src[j] = static_cast<const uint8_t *>(isA ? p.sa : p.sb) + (int64_t)grow * (p.K / 16) +
                   word * 4;
          step[j] = SKB / 8;
        }
        dst[j] = Cfg::A_BYTES + Cfg::B_BYTES + (isA ? 0 : Cfg::SA_BYTES) +
                 (word * rows + rblk * 64) * 4;
      }
    }
  }

  // DMA instruction j of stage ks
  DSL_DEV void issue_one(int j, int ks, uint32_t lds0) const {
    const uint32_t base = lds0 + (uint32_t)((ks % Cfg::NS) * Cfg::STAGE);
    if (j < Cfg::DD) dma16(src[j] + (int64_t)ks * step[j], base + dst[j]);
    else if (has[j]) dma4(src[j] + (int64_t)(ks >> Cfg::SC_SHIFT) * step[j], base + dst[j]);
  }
  // The same copies for a caller that issues stages strictly in order: the
  // source pointers advance in place, so no 64-bit `src + ks*step`
  // temporaries are live where the copies are issued (between MFMA rows).
  DSL_DEV void issue_next(int ks, uint32_t lds0) {
    static_assert(Cfg::SC_SHIFT == 0, "one scale step per stage");
    const uint32_t base = lds0 + (uint32_t)((ks % Cfg::NS) * Cfg::STAGE);
#pragma unroll
    for (int j = 0; j < Cfg::D; ++j) {
      if (j < Cfg::DD) {
        dma16(src[j], base + dst[j]);
        src[j] += step[j];
      } else if (has[j]) {
        dma4(src[j], base + dst[j]);
        src[j] += step[j];
      }
    }
  }
  // copies j0 .. j1-1 of stage ks, in place like issue_next (a caller that
  // spreads a stage over several calls issues every j once per stage)
  DSL_DEV void issue_range(int ks, uint32_t lds0, int j0, int j1) {
    const uint32_t base = lds0 + (uint32_t)((ks % Cfg::NS) * Cfg::STAGE);
#pragma unroll
    for (int j = 0; j < Cfg::D; ++j) {
      if (j < j0 || j >= j1) continue;
      if (j < Cfg::DD) {
        dma16(src[j], base + dst[j]);
        src[j] += step[j];
      } else if (has[j]) {
        dma4(src[j], base + dst[j]);
        src[j] += step[j];
      }
    }
  }
  DSL_DEV void issue(int ks, uint32_t lds0) const {
#pragma unroll
    for (int j = 0; j < Cfg::D; ++j) issue_one(j, ks, lds0);
  }
};

// Output staging for the epilogue: a BM x BN bf16 tile in LDS (the ring is
// idle by then), row-major, 16-byte chunk c of row r stored at chunk
// c ^ (r % CPR), so that fragment writes spread over the banks whether a
// write instruction covers a few rows (32x32 and 16x16 layouts: rows r, r+4,
// ...) or 32 rows of one column group (the transposed layout).  The tile
// then leaves LDS in 16-byte chunks, 8 consecutive bf16 of one row per
// lane: whole rows per store instruction instead of 2-byte scattered stores.
template <int BM, int BN>
struct OutStage {
  static constexpr int CPR = BN / 8;
  static_assert(CPR >= 8 && (CPR & (CPR - 1)) == 0, "power-of-two chunks per staged row");
  static DSL_DEV int off(int row, int col) {
    return row * BN + ((((col >> 3) ^ (row & (CPR - 1))) << 3) | (col & 7));
  }
  // copy the staged tile to C rows m0.., columns n0.. (clipped to M x N)
  template <int NT>
  static DSL_DEV void store(const GemmArgs &p, int m0, int n0, const uint16_t *stg) {
    const bool vec = (p.ldc % 8) == 0 && (reinterpret_cast<uintptr_t>(p.c) & 15) == 0;
    static_assert((BM * CPR) % NT == 0, "whole passes");
#pragma unroll
    for (int it = 0; it < BM * CPR / NT; ++it) {
      const int idx = it * NT + (int)threadIdx.x;
      const int row = idx / CPR, ch = idx % CPR;
      const int grow = m0 + row, gcol = n0 + ch * 8;
      if (grow >= p.M || gcol >= p.N) continue;
      const uint4 v = *reinterpret_cast<const uint4 *>(stg + row * BN + ((ch ^ (row & (CPR - 1))) << 3));
      uint16_t *dst = static_cast<uint16_t *>(p.c) + (int64_t)grow * p.ldc + gcol;
      if (vec && gcol + 8 <= p.N) {
        *reinterpret_cast<uint4 *>(dst) = v;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t w = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
          if (gcol + e < p.N) dst[e] = (uint16_t)(w >> (16 * (e & 1)));
        }
      }
    }
  }
};

// fp32 output staging (the same idea at 4 bytes per element): a BM x BN fp32
// tile in LDS, 16-byte chunk c of row r at chunk c ^ (r % CPR), leaving in
// 16-byte stores; with p.accumulate the store adds to C (one writer per
// element).
template <int BM, int BN>
struct OutStageF32 {
  static constexpr int CPR = BN / 4;
  static_assert(CPR >= 8 && (CPR & (CPR - 1)) == 0, "power-of-two chunks per staged row");
  static DSL_DEV int off(int row, int col) {
    return row * BN + ((((col >> 2) ^ (row & (CPR - 1))) << 2) | (col & 3));
  }
  template <int NT>
  static DSL_DEV void store(const GemmArgs &p, int m0, int n0, const float *stg) {
    const bool vec = (p.ldc % 4) == 0 && (reinterpret_cast<uintptr_t>(p.c) & 15) == 0;
    static_assert((BM * CPR) % NT == 0, "whole passes");
#pragma unroll
    for (int it = 0; it < BM * CPR / NT; ++it) {
      const int idx = it * NT + (int)threadIdx.x;
      const int row = idx / CPR, ch = idx % CPR;
      const int grow = m0 + row, gcol = n0 + ch * 4;
      if (grow >= p.M || gcol >= p.N) continue;
      float4 v = *reinterpret_cast<const float4 *>(stg + row * BN + ((ch ^ (row & (CPR - 1))) << 2));
      float *dst = static_cast<float *>(p.c) + (int64_t)grow * p.ldc + gcol;
      if (vec && gcol + 4 <= p.N) {
        if (p.accumulate) {
          const float4 o = *reinterpret_cast<const float4 *>(dst);
          v.x += o.x;
          v.y += o.y;
          v.z += o.z;
          v.w += o.w;
        }
        *reinterpret_cast<float4 *>(dst) = v;
      } else {
        const float e4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (gcol + e < p.N) dst[e] = p.accumulate ? dst[e] + e4[e] : e4[e];
      }
    }
  }
};

}  // namespace pipe

// Operand fragments of one K-step (64 K for FP8, 64 K = 32 bytes for FP4)
// of one wave, read from the stage at `st` by load() and consumed by mma().
// Splitting the two lets the mainloop read the next stage's fragments while
// the MFMAs of the current one run.
template <class Cfg, bool FP4 = Cfg::FP4>
struct KFrag;

// FP8: 32 bytes of K per lane (two 16-byte chunks) for every 32-row tile.
template <class Cfg>
struct KFrag<Cfg, false> {
  v8i a[Cfg::TM], b[Cfg::TN];
  static DSL_DEV v8i ld(const uint8_t *base, int row, int k, int h) {
    constexpr int SKB = Cfg::SKB;
    const int s = pipe::swz<SKB>(row), c0 = 4 * k + 2 * h;
    const v4i lo = *reinterpret_cast<const v4i *>(base + row * SKB + ((c0 ^ s) << 4));
    const v4i hi = *reinterpret_cast<const v4i *>(base + row * SKB + (((c0 + 1) ^ s) << 4));
    return (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
  DSL_DEV void load_a(const uint8_t *st, int k, int t, int wm, int r32, int h) {
    a[t] = ld(st, wm * Cfg::WM + t * 32 + r32, k, h);
  }
  DSL_DEV void load_b(const uint8_t *st, int k, int wn, int r32, int h) {
#pragma unroll
    for (int t = 0; t < Cfg::TN; ++t) b[t] = ld(st + Cfg::A_BYTES, wn * Cfg::WN + t * 32 + r32, k, h);
  }
  DSL_DEV void load(const uint8_t *st, int k, int wm, int wn, int r32, int h) {
    load_b(st, k, wn, r32, h);
#pragma unroll
    for (int t = 0; t < Cfg::TM; ++t) load_a(st, k, t, wm, r32, h);
  }
  // bf16: the lane's 32 bytes are 16 bf16 of K, two 32x32x16 MFMAs (first
  // and second 16-byte chunk; the same K order for A and W)
  static DSL_DEV v16f mma_bf16(const v8i &x, const v8i &y, v16f c) {
    const v8bf x0 = __builtin_bit_cast(v8bf, (v4i){x[0], x[1], x[2], x[3]});
    const v8bf x1 = __builtin_bit_cast(v8bf, (v4i){x[4], x[5], x[6], x[7]});
    const v8bf y0 = __builtin_bit_cast(v8bf, (v4i){y[0], y[1], y[2], y[3]});
    const v8bf y1 = __builtin_bit_cast(v8bf, (v4i){y[4], y[5], y[6], y[7]});
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x0, y0, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(x1, y1, c, 0, 0, 0);
  }
  // TR: operands swapped, see mma_row_t
  template <bool TR = false>
  DSL_DEV void mma_row(int, int i, v16f (&acc)[Cfg::TM][Cfg::TN]) const {
    if constexpr (TR) {
      mma_row_t(i, acc);
      return;
    }
#pragma unroll
    for (int j = 0; j < Cfg::TN; ++j) {
      if constexpr (Cfg::BF16)
        acc[i][j] = mma_bf16(a[i], b[j], acc[i][j]);
      else
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[i], b[j], acc[i][j], 0, 0,
                                                                    0, 0, 0, 0);
    }
  }
  // operands swapped (W tile in the first slot): acc[i][j] holds C^T, so
  // lane l owns output row 32i + l%32 and register r the column
  // 32j + 8(r/4) + 4h + r%4
  DSL_DEV void mma_row_t(int i, v16f (&acc)[Cfg::TM][Cfg::TN]) const {
#pragma unroll
    for (int j = 0; j < Cfg::TN; ++j) {
      if constexpr (Cfg::BF16)
        acc[i][j] = mma_bf16(b[j], a[i], acc[i][j]);
      else
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b[j], a[i], acc[i][j], 0, 0,
                                                                    0, 0, 0, 0);
    }
  }
  template <bool TR = false>
  DSL_DEV void mma(int k, v16f (&acc)[Cfg::TM][Cfg::TN]) const {
#pragma unroll
    for (int i = 0; i < Cfg::TM; ++i) mma_row<TR>(k, i, acc);
  }
};

// MXFP4: one 16-byte chunk (32 elements = one E8M0 block) per lane and tile.
// Scales: [word][row] u32 after the two data tiles; byte j of the permuted
// word is the E8M0 of block 2*j + h of the word's 4 blocks of this row.
template <class Cfg>
struct KFrag<Cfg, true> {
  v4i a[Cfg::TM], b[Cfg::TN];
  int as[Cfg::TM], bs[Cfg::TN];
  DSL_DEV void load_a(const uint8_t *st, int k, int t, int wm, int r32, int h) {
    const uint8_t *sSa = st + Cfg::A_BYTES + Cfg::B_BYTES;
    const int row = wm * Cfg::WM + t * 32 + r32;
    a[t] = *reinterpret_cast<const v4i *>(st + row * Cfg::SKB +
                                          (((2 * k + h) ^ pipe::swz<Cfg::SKB>(row)) << 4));
    const uint32_t w = *reinterpret_cast<const uint32_t *>(sSa + ((k >> 1) * Cfg::BM + row) * 4);
    as[t] = (int)__builtin_amdgcn_perm(w, w, h ? 0x02000301u : 0x03010200u);
  }
  DSL_DEV void load_b(const uint8_t *st, int k, int wn, int r32, int h) {
    const uint8_t *sB = st + Cfg::A_BYTES;
    const uint8_t *sSb = st + Cfg::A_BYTES + Cfg::B_BYTES + Cfg::SA_BYTES;
#pragma unroll
    for (int t = 0; t < Cfg::TN; ++t) {
      const int row = wn * Cfg::WN + t * 32 + r32;
      b[t] = *reinterpret_cast<const v4i *>(sB + row * Cfg::SKB +
                                            (((2 * k + h) ^ pipe::swz<Cfg::SKB>(row)) << 4));
      const uint32_t w = *reinterpret_cast<const uint32_t *>(sSb + ((k >> 1) * Cfg::BN + row) * 4);
      bs[t] = (int)__builtin_amdgcn_perm(w, w, h ? 0x02000301u : 0x03010200u);
    }
  }
  DSL_DEV void load(const uint8_t *st, int k, int wm, int wn, int r32, int h) {
    load_b(st, k, wn, r32, h);
#pragma unroll
    for (int t = 0; t < Cfg::TM; ++t) load_a(st, k, t, wm, r32, h);
  }
  // TR: W tile (and its scales) in the first operand slot, acc holds C^T
  template <bool TR = false>
  DSL_DEV void mma_row(int k, int i, v16f (&acc)[Cfg::TM][Cfg::TN]) const {
#pragma unroll
    for (int j = 0; j < Cfg::TN; ++j) {
      if constexpr (TR)
        acc[i][j] = (k & 1) ? pipe::mfma_fp4<1>(b[j], a[i], acc[i][j], bs[j], as[i])
                            : pipe::mfma_fp4<0>(b[j], a[i], acc[i][j], bs[j], as[i]);
      else
        acc[i][j] = (k & 1) ? pipe::mfma_fp4<1>(a[i], b[j], acc[i][j], as[i], bs[j])
                            : pipe::mfma_fp4<0>(a[i], b[j], acc[i][j], as[i], bs[j]);
    }
  }
  template <bool TR = false>
  DSL_DEV void mma(int k, v16f (&acc)[Cfg::TM][Cfg::TN]) const {
#pragma unroll
    for (int i = 0; i < Cfg::TM; ++i) mma_row<TR>(k, i, acc);
  }
};

// NVFP4 quad k: lane half h holds the 32 elements [64k + 32h, +32) of its row
// (one 16-byte chunk), taken as four 8-element K-steps i; K-step i of both
// operands covers elements 64k + 32h + 8i.. for lane half h, so A and W see
// the same K order and each lane's 8 elements lie in one 16-element E4M3
// block (2h + i/2 of the quad's four).  Elements are dequantized to fp16
// exactly (E2M1 x E4M3 has <= 5 significant bits) and multiplied by fp16
// MFMAs; the fp32 global scales apply in the epilogue.  Scales: [word][row]
// u32 after the data tiles, word k holds the quad's four E4M3 bytes.  (A
// free function with local arrays: as struct members the scale arrays were
// left in private memory by the compiler.)
template <class Cfg, bool TR = false>
DSL_DEV void nv_kstep(const uint8_t *st, int k, int wm, int wn, int r32, int h,
                      v16f (&acc)[Cfg::TM][Cfg::TN]) {
  constexpr int SKB = Cfg::SKB;
  const uint8_t *sA = st, *sB = st + Cfg::A_BYTES;
  const uint8_t *sSa = st + Cfg::A_BYTES + Cfg::B_BYTES;
  const uint8_t *sSb = sSa + Cfg::SA_BYTES;
  v4i araw[Cfg::TM], braw[Cfg::TN];
  _Float16 asc[Cfg::TM][2], bsc[Cfg::TN][2];
#pragma unroll
  for (int t = 0; t < Cfg::TN; ++t) {
    const int row = wn * Cfg::WN + t * 32 + r32;
    braw[t] = *reinterpret_cast<const v4i *>(sB + row * SKB + (((2 * k + h) ^ pipe::swz<SKB>(row)) << 4));
    const uint32_t w = *reinterpret_cast<const uint32_t *>(sSb + (k * Cfg::BN + row) * 4);
    bsc[t][0] = e4m3_to_f16((w >> (16 * h)) & 0xFF);
    bsc[t][1] = e4m3_to_f16((w >> (16 * h + 8)) & 0xFF);
  }
#pragma unroll
  for (int t = 0; t < Cfg::TM; ++t) {
    const int row = wm * Cfg::WM + t * 32 + r32;
    araw[t] = *reinterpret_cast<const v4i *>(sA + row * SKB + (((2 * k + h) ^ pipe::swz<SKB>(row)) << 4));
    const uint32_t w = *reinterpret_cast<const uint32_t *>(sSa + (k * Cfg::BM + row) * 4);
    asc[t][0] = e4m3_to_f16((w >> (16 * h)) & 0xFF);
    asc[t][1] = e4m3_to_f16((w >> (16 * h + 8)) & 0xFF);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v8h af[Cfg::TM], bf[Cfg::TN];
#pragma unroll
    for (int t = 0; t < Cfg::TN; ++t) bf[t] = fp4x8_to_f16((uint32_t)braw[t][i], bsc[t][i >> 1]);
#pragma unroll
    for (int t = 0; t < Cfg::TM; ++t) af[t] = fp4x8_to_f16((uint32_t)araw[t][i], asc[t][i >> 1]);
#pragma unroll
    for (int x = 0; x < Cfg::TM; ++x)
#pragma unroll
      for (int y = 0; y < Cfg::TN; ++y)
        acc[x][y] = TR ? __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[y], af[x], acc[x][y], 0, 0, 0)
                       : __builtin_amdgcn_mfma_f32_32x32x16_f16(af[x], bf[y], acc[x][y], 0, 0, 0);
  }
}

// All K-steps of one stage, for the prefetch schedule (FP8 / MXFP4).
template <class Cfg>
struct StageFrag {
  KFrag<Cfg> f[Cfg::KSTEPS];
  DSL_DEV void load(const uint8_t *st, int wm, int wn, int r32, int h) {
#pragma unroll
    for (int k = 0; k < Cfg::KSTEPS; ++k) f[k].load(st, k, wm, wn, r32, h);
  }
  template <bool TR = false>
  DSL_DEV void mma(v16f (&acc)[Cfg::TM][Cfg::TN]) const {
#pragma unroll
    for (int k = 0; k < Cfg::KSTEPS; ++k) f[k].template mma<TR>(k, acc);
  }
  // MFMAs of this stage, with the next stage's fragments read into `nxt`
  // as this stage's registers free up: next B first (its own registers),
  // then each A row right after the MFMAs that consume this stage's copy.
  // When `issue` is set, the DMA instructions of stage `ks_issue` are spread
  // over the MFMA rows, so that the MFMA pipe is already busy while the
  // vector-memory queue accepts them.
  template <bool TR = false>
  DSL_DEV void mma_prefetch(v16f (&acc)[Cfg::TM][Cfg::TN], StageFrag &nxt, const uint8_t *st_next,
                            int wm, int wn, int r32, int h, const pipe::Ring<Cfg> &ring,
                            bool issue, int ks_issue, uint32_t lds0) const {
    constexpr int R = Cfg::KSTEPS * Cfg::TM, D = Cfg::D;
#pragma unroll
    for (int k = 0; k < Cfg::KSTEPS; ++k) nxt.f[k].load_b(st_next, k, wn, r32, h);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < Cfg::KSTEPS; ++k)
#pragma unroll
      for (int i = 0; i < Cfg::TM; ++i) {
        const int t = k * Cfg::TM + i;
        f[k].template mma_row<TR>(k, i, acc);
        if (issue) {
#pragma unroll
          for (int j = t * D / R; j < (t + 1) * D / R; ++j) ring.issue_one(j, ks_issue, lds0);
        }
        nxt.f[k].load_a(st_next, k, i, wm, r32, h);
        __builtin_amdgcn_sched_barrier(0);
      }
  }
};

namespace pipe {

// s_waitcnt vmcnt(n * D) for a run-time n in [0, NMAX].
template <int D, int NMAX>
DSL_DEV void wait_stages(int n) {
  if constexpr (NMAX <= 0) {
    wait_vmcnt<0>();
  } else {
    if (n >= NMAX) wait_vmcnt<NMAX * D>();
    else wait_stages<D, NMAX - 1>(n);
  }
}

// s_waitcnt vmcnt(n * cnt) where cnt is D or D-1 (`full` selects D).
template <int D, int NMAX>
DSL_DEV void wait_stages_of(int n, bool full) {
  if constexpr (D > 1) {
    if (!full) {
      wait_stages<D - 1, NMAX>(n);
      return;
    }
  }
  wait_stages<D, NMAX>(n);
}

// Every LDS read this wave issued has returned (its data is in registers).
DSL_DEV void wait_lds() { __builtin_amdgcn_s_waitcnt((15 << 0) | (7 << 4) | (0 << 8) | (3 << 14)); }

}  // namespace pipe

// One stage of the prefetch schedule (ks + 1 < nks): `cur` holds stage ks in
// registers, `nxt` receives stage ks+1.  STEADY: stage ks+NS exists (the
// next stage is issued and NS-2 stages follow stage ks+1); without it the
// step checks at run time.  The steady form has no branch between the MFMA
// rows, which keeps the compiler from sinking work across them.
template <class Cfg, bool STEADY, bool TR = false>
DSL_DEV void pf_step(int ks, int nks, const pipe::Ring<Cfg> &ring, uint32_t lds0,
                     const uint8_t *smem, const StageFrag<Cfg> &cur, StageFrag<Cfg> &nxt, int wm,
                     int wn, int r32, int h, v16f (&acc)[Cfg::TM][Cfg::TN]) {
  constexpr int NS = Cfg::NS, D = Cfg::D;
  if constexpr (STEADY) {
    pipe::wait_stages_of<D, NS - 2>(NS - 2, ring.full);
  } else {
    // issued so far: stages 0 .. min(ks+NS-1, nks-1); stage ks+1 has landed
    // once at most the stages after it are outstanding
    const int last = (ks + NS - 1 < nks - 1) ? ks + NS - 1 : nks - 1;
    pipe::wait_stages_of<D, NS - 2>(last - (ks + 1), ring.full);
  }
  pipe::wait_lds();
  __syncthreads();
  cur.template mma_prefetch<TR>(acc, nxt, smem + ((ks + 1) % NS) * Cfg::STAGE, wm, wn, r32, h, ring,
                   STEADY || ks + NS < nks, ks + NS, lds0);
}

// One BM x BN output tile over all of K: ring set-up, prologue, and the
// stage loop.  `p` describes the operands the tile reads (A rows m0.., W
// rows n0.., p.M / p.N bound the rows that exist; rows past them re-read
// the last row).  The caller zeroes nothing: acc is initialised here.  On
// return every wave has finished reading LDS only once it passes a barrier,
// so a caller that reuses `smem` for another tile must __syncthreads() first.
//
// Cfg::PF selects the schedule:
//   * PF = 0: a wave reads a stage's fragments after the barrier that
//     publishes it and feeds them straight to the MFMAs; the loads of stage
//     ks+NS-1 go out after that barrier (NS-2 stages in flight during the
//     MFMAs).
//   * PF = 1: fragments are double-buffered in registers.  After the barrier
//     that publishes stage ks+1 (and certifies that every wave holds stage
//     ks in registers), a wave refills the slot of stage ks with stage
//     ks+NS, issues the LDS reads of stage ks+1 and then the MFMAs of stage
//     ks, so the LDS latency hides behind the MFMAs and NS-1 stages are in
//     flight.  Requires an even stage count Kb / SKB >= 2.
template <class Cfg, bool TR = false>
DSL_DEV void pipe_mainloop(const GemmArgs &p, int m0, int n0, uint8_t *smem, int wave, int lane,
                           v16f (&acc)[Cfg::TM][Cfg::TN]) {
  constexpr int NS = Cfg::NS, D = Cfg::D;
  const uint32_t lds0 = pipe::lds_addr(smem);
  pipe::Ring<Cfg> ring;
  ring.init(p, m0, n0, wave, lane);
  const int nks = p.Kb / Cfg::SKB;
  const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
  const int r32 = lane & 31, h = lane >> 5;
#pragma unroll
  for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  if constexpr (!Cfg::PF) {
#pragma unroll
    for (int s = 0; s < NS - 1; ++s)
      if (s < nks) ring.issue(s, lds0);
    for (int ks = 0; ks < nks; ++ks) {
      // this wave's loads of stage ks have landed once at most the later
      // stages' loads are outstanding; the barrier then publishes stage ks to
      // every wave and certifies that stage ks-1's slot is no longer read
      // (issued so far: stages 0 .. min(ks+NS-2, nks-1))
      const int pending = (nks - 1 - ks < NS - 2) ? nks - 1 - ks : NS - 2;
      pipe::wait_stages_of<D, NS - 2>(pending, ring.full);
      __syncthreads();
      if (ks + NS - 1 < nks) ring.issue(ks + NS - 1, lds0);
      const uint8_t *st = smem + (ks % NS) * Cfg::STAGE;
#pragma unroll
      for (int k = 0; k < Cfg::KSTEPS; ++k) {
        if constexpr (Cfg::NV) {
          nv_kstep<Cfg, TR>(st, k, wm, wn, r32, h, acc);
        } else {
          KFrag<Cfg> f;
          f.load(st, k, wm, wn, r32, h);
          f.template mma<TR>(k, acc);
        }
      }
    }
  } else {
#pragma unroll
    for (int s = 0; s < NS; ++s)
      if (s < nks) ring.issue(s, lds0);
    // stages issued after the prologue: 0 .. min(NS, nks) - 1
    pipe::wait_stages_of<D, NS - 1>((nks < NS ? nks : NS) - 1, ring.full);
    __syncthreads();
    StageFrag<Cfg> f0, f1;
    f0.load(smem, wm, wn, r32, h);
    // steady state in pairs (f0 -> f1 -> f0), every step with a next stage;
    // the MFMAs of the last stage are peeled so that no branch carries
    // MFMAs (the accumulators would be copied at the join)
    // (nks is even and >= 2: a precondition of this schedule)
    int ks = 0;
    for (; ks + NS + 1 < nks; ks += 2) {
      pf_step<Cfg, true, TR>(ks, nks, ring, lds0, smem, f0, f1, wm, wn, r32, h, acc);
      pf_step<Cfg, true, TR>(ks + 1, nks, ring, lds0, smem, f1, f0, wm, wn, r32, h, acc);
    }
    for (; ks + 2 < nks; ks += 2) {
      pf_step<Cfg, false, TR>(ks, nks, ring, lds0, smem, f0, f1, wm, wn, r32, h, acc);
      pf_step<Cfg, false, TR>(ks + 1, nks, ring, lds0, smem, f1, f0, wm, wn, r32, h, acc);
    }
    pf_step<Cfg, false, TR>(ks, nks, ring, lds0, smem, f0, f1, wm, wn, r32, h, acc);
    f1.template mma<TR>(acc);
  }
}

}  // namespace dsl
