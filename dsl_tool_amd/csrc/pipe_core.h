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

// LDS row swizzle: chunk c of row r lives in slot c ^ swz<SKB>(r).  With
// 64-byte rows four rows share a 256-byte bank line, with 128-byte rows two;
// either way the 16 lanes that read one logical chunk of 16 consecutive rows
// land on 16 distinct 16-byte bank groups.
template <int SKB>
DSL_DEV int swz(int row) { return SKB == 64 ? (row >> 2) & 3 : (row >> 1) & 7; }

// FP4 x FP4 32x32x64 scaled MFMA; OPS picks the scale byte of sa / sb.
template <int OPS>
DSL_DEV v16f mfma_fp4(const v4i &a, const v4i &b, const v16f &c, int sa, int sb) {
  const v8i a8 = {a[0], a[1], a[2], a[3], 0, 0, 0, 0};
  const v8i b8 = {b[0], b[1], b[2], b[3], 0, 0, 0, 0};
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, c, 4, 4, OPS, sa, OPS, sb);
}

}  // namespace pipe

template <int MODE_, int BM_, int BN_, int WGM_, int WGN_, int NS_, int SKB_ = 64, int OCC_ = 0>
struct PipeCfg {
  static constexpr int MODE = MODE_, BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_, NS = NS_;
  static constexpr int SKB = SKB_;                          // stage bytes per row
  static constexpr int NW = WGM * WGN, NT = NW * 64;
  static constexpr int OCC = OCC_ > 0 ? OCC_ : (NW >= 8 ? 2 : 1);   // waves per SIMD
  static constexpr int WM = BM / WGM, WN = BN / WGN, TM = WM / 32, TN = WN / 32;
  static constexpr bool MX = MODE == MODE_MXFP4;
  static constexpr bool NV = MODE == MODE_NVFP4;
  static constexpr bool FP4 = MX || NV;
  static constexpr bool BLOCK = MODE == MODE_FP8_BLOCK;     // one 128-K scale group per stage
  static constexpr int CH = SKB / 16, RPI = 1024 / SKB;     // chunks per row, rows per DMA
  // MFMA steps per stage: 32x32x64 for FP8 / MXFP4; for NVFP4 a "step" is a
  // quad of four 32x32x16 fp16 MFMAs over 64 elements (32 bytes)
  static constexpr int KSTEPS = MX ? SKB / 32 : (NV ? SKB / 32 : SKB / 64);
  // scale words (4 bytes) per row per stage: E8M0 per 32, E4M3 per 16, fp32 per 128-K group
  static constexpr int SCW = MX ? SKB / 64 : (NV ? SKB / 32 : (BLOCK ? 1 : 0));
  static constexpr int A_BYTES = BM * SKB, B_BYTES = BN * SKB;
  static constexpr int SA_BYTES = BM * 4 * SCW, SB_BYTES = FP4 ? BN * 4 * SCW : 0;
  static constexpr int STAGE = A_BYTES + B_BYTES + SA_BYTES + SB_BYTES;
  static constexpr int LDS = NS * STAGE;
  static constexpr int A_DMA = A_BYTES / 1024, B_DMA = B_BYTES / 1024;
  static constexpr int SA_DMA = SA_BYTES / 256, SB_DMA = SB_BYTES / 256;
  static constexpr int TOTAL_DMA = A_DMA + B_DMA + SA_DMA + SB_DMA;
  static constexpr int D = (TOTAL_DMA + NW - 1) / NW;      // DMA instructions per wave per stage
  static_assert(SKB == 64 || SKB == 128, "stage width");
  static_assert(!BLOCK || SKB == 128, "block scales need one 128-K group per stage");
  // an uneven split leaves waves with different DMA counts; only a 2-stage
  // ring (always vmcnt(0)) is independent of the per-wave count
  static_assert(TOTAL_DMA % NW == 0 || NS == 2, "DMA work must split evenly over the waves");
  static_assert(BM % 64 == 0 && BN % 64 == 0 && WM % 32 == 0 && WN % 32 == 0, "tile shape");
  static_assert(LDS <= 160 * 1024, "LDS budget");
  static_assert(NS >= 2 && (NS - 2) * D < 64, "ring depth / vmcnt range");
};

namespace pipe {

// Direct-to-LDS copy plan of one thread: D wave-uniform DMA instructions
// per stage (operand data, then scale words), their stage-0 sources, LDS
// offsets within a stage and source advance per stage.
template <class Cfg>
struct Ring {
  const uint8_t *src[Cfg::D];
  uint32_t dst[Cfg::D];
  int step[Cfg::D];
  int kind[Cfg::D];     // 0: none, 1: 16-byte data, 2: 4-byte scale word

  DSL_DEV void init(const GemmArgs &p, int m0, int n0, int wave, int lane) {
    constexpr int SKB = Cfg::SKB;
#pragma unroll
    for (int j = 0; j < Cfg::D; ++j) {
      const int i = wave * Cfg::D + j;
      src[j] = p.a;
      dst[j] = 0;
      step[j] = 0;
      kind[j] = 0;
      if (i < Cfg::A_DMA + Cfg::B_DMA) {
        const bool isA = i < Cfg::A_DMA;
        const int lrow = (isA ? i : i - Cfg::A_DMA) * Cfg::RPI + lane / Cfg::CH;
        const int chunk = (lane % Cfg::CH) ^ swz<SKB>(lrow);
        const int lim = isA ? p.M - 1 : p.N - 1;
        int grow = (isA ? m0 : n0) + lrow;
        grow = grow > lim ? lim : grow;    // rows past the edge re-read the last row
        src[j] = (isA ? p.a : p.b) + (int64_t)grow * p.Kb + chunk * 16;
        dst[j] = i * 1024;
        step[j] = SKB;
        kind[j] = 1;
      } else if (i < Cfg::TOTAL_DMA) {
        const int si = i - Cfg::A_DMA - Cfg::B_DMA;
        const bool isA = si < Cfg::SA_DMA;
        const int rows = isA ? Cfg::BM : Cfg::BN;
        const int sidx = isA ? si : si - Cfg::SA_DMA;
        const int word = sidx / (rows / 64), rblk = sidx % (rows / 64);
        const int lrow = rblk * 64 + lane;
        const int lim = isA ? p.M - 1 : p.N - 1;
        int grow = (isA ? m0 : n0) + lrow;
        grow = grow > lim ? lim : grow;
        if constexpr (Cfg::BLOCK) {        // fp32 sa[row][K/128]: one float per row per stage
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
        kind[j] = 2;
      }
    }
  }

  DSL_DEV void issue(int ks, uint32_t lds0) const {
    const uint32_t base = lds0 + (uint32_t)((ks % Cfg::NS) * Cfg::STAGE);
#pragma unroll
    for (int j = 0; j < Cfg::D; ++j) {
      const uint8_t *s = src[j] + (int64_t)ks * step[j];
      if (kind[j] == 1) dma16(s, base + dst[j]);
      else if (kind[j] == 2) dma4(s, base + dst[j]);
    }
  }
};

}  // namespace pipe

// One K-step (64 K for FP8, 64 K = 32 bytes for FP4) of MFMAs from the
// stage at `st`.
template <class Cfg>
DSL_DEV void mma_kstep(const uint8_t *st, int k, int wm, int wn, int r32, int h,
                       v16f (&acc)[Cfg::TM][Cfg::TN]) {
  constexpr int SKB = Cfg::SKB;
  const uint8_t *sA = st, *sB = st + Cfg::A_BYTES;
  if constexpr (!Cfg::FP4) {
    auto ld = [&](const uint8_t *base, int row) {
      const int s = pipe::swz<SKB>(row), c0 = 4 * k + 2 * h;
      const v4i lo = *reinterpret_cast<const v4i *>(base + row * SKB + ((c0 ^ s) << 4));
      const v4i hi = *reinterpret_cast<const v4i *>(base + row * SKB + (((c0 + 1) ^ s) << 4));
      return (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    v8i af[Cfg::TM], bf[Cfg::TN];
#pragma unroll
    for (int t = 0; t < Cfg::TN; ++t) bf[t] = ld(sB, wn * Cfg::WN + t * 32 + r32);
#pragma unroll
    for (int t = 0; t < Cfg::TM; ++t) af[t] = ld(sA, wm * Cfg::WM + t * 32 + r32);
#pragma unroll
    for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[i], bf[j], acc[i][j], 0, 0,
                                                                    0, 0, 0, 0);
  } else if constexpr (Cfg::NV) {
    // NVFP4 quad k: lane half h holds the 32 elements [64k + 32h, +32) of its
    // row (one 16-byte chunk), taken as four 8-element K-steps i; K-step i
    // of both operands covers elements 64k + 32h + 8i.. for lane half h, so
    // A and W see the same K order and each lane's 8 elements lie in one
    // 16-element E4M3 block (2h + i/2 of the quad's four).  Elements are
    // dequantized to fp16 exactly (E2M1 x E4M3 has <= 5 significant bits)
    // and multiplied by fp16 MFMAs; the fp32 global scales apply in the
    // epilogue.  Scales: [word][row] u32 after the data tiles, word k holds
    // the quad's four E4M3 bytes.
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
      for (int a = 0; a < Cfg::TM; ++a)
#pragma unroll
        for (int b = 0; b < Cfg::TN; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[a], bf[b], acc[a][b], 0, 0, 0);
    }
  } else {
    // scales: [word][row] u32 after the two data tiles; byte j of the permuted
    // word is the E8M0 of block 2*j + h of the word's 4 blocks of this row
    const uint8_t *sSa = st + Cfg::A_BYTES + Cfg::B_BYTES;
    const uint8_t *sSb = sSa + Cfg::SA_BYTES;
    const uint32_t sel = h ? 0x02000301u : 0x03010200u;
    const int word = k >> 1;
    v4i af[Cfg::TM], bf[Cfg::TN];
    int as[Cfg::TM], bs[Cfg::TN];
#pragma unroll
    for (int t = 0; t < Cfg::TN; ++t) {
      const int row = wn * Cfg::WN + t * 32 + r32;
      bf[t] = *reinterpret_cast<const v4i *>(sB + row * SKB + (((2 * k + h) ^ pipe::swz<SKB>(row)) << 4));
      const uint32_t w = *reinterpret_cast<const uint32_t *>(sSb + (word * Cfg::BN + row) * 4);
      bs[t] = (int)__builtin_amdgcn_perm(w, w, sel);
    }
#pragma unroll
    for (int t = 0; t < Cfg::TM; ++t) {
      const int row = wm * Cfg::WM + t * 32 + r32;
      af[t] = *reinterpret_cast<const v4i *>(sA + row * SKB + (((2 * k + h) ^ pipe::swz<SKB>(row)) << 4));
      const uint32_t w = *reinterpret_cast<const uint32_t *>(sSa + (word * Cfg::BM + row) * 4);
      as[t] = (int)__builtin_amdgcn_perm(w, w, sel);
    }
#pragma unroll
    for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::TN; ++j)
        acc[i][j] = (k & 1) ? pipe::mfma_fp4<1>(af[i], bf[j], acc[i][j], as[i], bs[j])
                            : pipe::mfma_fp4<0>(af[i], bf[j], acc[i][j], as[i], bs[j]);
  }
}

// One BM x BN output tile over all of K: ring set-up, prologue, and the
// stage loop.  `p` describes the operands the tile reads (A rows m0.., W
// rows n0.., p.M / p.N bound the rows that exist; rows past them re-read
// the last row).  The caller zeroes nothing: acc is initialised here.  On
// return every wave has finished reading LDS only once it passes a barrier,
// so a caller that reuses `smem` for another tile must __syncthreads() first.
template <class Cfg>
DSL_DEV void pipe_mainloop(const GemmArgs &p, int m0, int n0, uint8_t *smem, int wave, int lane,
                           v16f (&acc)[Cfg::TM][Cfg::TN]) {
  constexpr int NS = Cfg::NS, D = Cfg::D, SKB = Cfg::SKB;
  const uint32_t lds0 = pipe::lds_addr(smem);
  pipe::Ring<Cfg> ring;
  ring.init(p, m0, n0, wave, lane);
  const int nks = p.Kb / SKB;
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nks) ring.issue(s, lds0);

  const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
  const int r32 = lane & 31, h = lane >> 5;
#pragma unroll
  for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  for (int ks = 0; ks < nks; ++ks) {
    // this wave's loads of stage ks have landed once at most the later
    // stages' loads are outstanding; the barrier then publishes stage ks to
    // every wave and certifies that stage ks-1's slot is no longer read
    if (ks + NS - 2 < nks) pipe::wait_vmcnt<(NS - 2) * D>();
    else pipe::wait_vmcnt<0>();
    __syncthreads();
    if (ks + NS - 1 < nks) ring.issue(ks + NS - 1, lds0);
    const uint8_t *st = smem + (ks % NS) * Cfg::STAGE;
#pragma unroll
    for (int k = 0; k < Cfg::KSTEPS; ++k) mma_kstep<Cfg>(st, k, wm, wn, r32, h, acc);
  }
}

}  // namespace dsl
