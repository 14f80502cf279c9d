// Persistent pipelined GEMM for gfx950 (FP8 per-tensor, FP8 1x128/128x128
// block-scaled, MXFP4): C[M,N] = A[M,K] . W[N,K]^T, both operands K-major.
//
// One workgroup per CU walks its output tiles (tile v = blockIdx.x +
// r * gridDim.x in the XCD-aware order of tile_coords), 256x256 with 8 waves
// (2 x 4, each 128 x 64, 32x32x64 MFMAs with the W tile in the first operand
// slot, so a lane owns one output row).
//
// Data path.  K advances in 64-byte steps, but operands move in pairs of
// steps: a pair is 128 bytes of K for every row of the tile, and each
// direct-to-LDS load (global_load_lds_dwordx4) copies 8 rows x 128 bytes,
// i.e. whole 128-byte lines.  With 64-byte rows the L1 sends one 64-byte
// request to L2 per half line and cannot keep the other half until the next
// step, so the same bytes cost twice the requests; the L1's outstanding
// requests are what limit the copy rate, so whole lines double it.  Two pair
// slots form the ring in LDS: pair q+2 is copied into the slot of pair q
// during the second step of pair q+1, one step after the barrier that
// certifies pair q read, and waited for two steps later.  A barrier is
// needed only at the start of the second step of a pair (it publishes the
// next pair and frees the previous slot), so there is one per 128 K.  The
// ring runs on across tile boundaries: the first pairs of tile r+1 are
// copied during the last steps of tile r.
//
// Fragments: W fragments double-buffered by step parity, A rows reloaded in
// place right after the MFMAs that consume them (they are not read again
// until the next step), which keeps the 128 fp32 accumulators, both
// fragment sets and the copy plan within 256 VGPRs.
//
// Scales move 16 bytes per row at a time, in a ring of their own: one
// "quad" holds a row's scales for QP pairs (FP8 block: four fp32 group
// scales, QP = 4; MXFP4: sixteen E8M0 bytes, QP = 2), so one
// global_load_lds_dwordx4 per 64 rows fetches QP pairs' worth.  Per-pair
// 4-byte loads would touch one cache line per row for every pair (50% more
// L1 requests than the operands for FP8 block, 200% for MXFP4).  Two quad
// slots alternate; quad c+2 is copied with the first pair of that quad,
// after every wave has read quad c.
//
// FP8 block: a pair is exactly one 128-K scale group.  The accumulator is
// kept in units of the current group's scale s_g(m) = sa[m][g] * sb[n/128][g]
// and multiplied by s_g / s_{g+1} at each group boundary; the epilogue
// multiplies by the last s_g.  This is the group-partial sum of
// cuda/gemm/fp8_gemm.cu:84-97 up to fp32 rounding.
//
// MXFP4: each 64-byte step is two 32x32x64 FP4 MFMAs per tile, the E8M0
// block scales of W and A go into the MFMA's scale operands (exact powers
// of two), cuda/gemm/fp4_gemm.cu semantics.
//
// NVFP4: the E4M3 block scales (one per 16 elements) are not powers of two,
// so operands are dequantized in registers: each 8-element group becomes
// 8 fp16 values (hardware E2M1 -> fp16 and E4M3 -> fp16 conversions, then
// one packed fp16 multiply per 2 values; E2M1 x E4M3 has at most 6
// significant bits, so the fp16 values are exact) and feeds 32x32x16 fp16
// MFMAs; the fp32 global scales apply in the epilogue.
//
// Epilogue: each wave converts its accumulators (v_cvt_pk_bf16_f32),
// regroups them across lanes (v_permlane32_swap, v_permlane16_swap) and
// stores 16 bytes per lane, 16 rows x 64 contiguous bytes per store, straight
// from registers.  Stores share vmcnt with the ring's loads; the next pair
// wait (vmcnt(0)) also waits for them.
#include <type_traits>

#include "pipe_core.h"

namespace dsl {

template <int MODE_, bool GROUPED_ = false, bool GATHER_ = false>
struct PersCfg {
  static constexpr int MODE = MODE_;
  static constexpr bool GROUPED = GROUPED_;    // FP8 grouped (MoE) tile walk
  static constexpr bool GATHER = GATHER_;      // grouped: A rows through a row table
  static constexpr int BM = 256, BN = 256, WGM = 2, WGN = 4;
  static constexpr int NW = WGM * WGN, NT = NW * 64, OCC = 2;
  static constexpr int WM = BM / WGM, WN = BN / WGN, TM = WM / 32, TN = WN / 32;
  static constexpr bool BLOCK = MODE == MODE_FP8_BLOCK;
  static constexpr bool MX = MODE == MODE_MXFP4;
  static constexpr bool NV = MODE == MODE_NVFP4;
  static constexpr bool BF16 = MODE == MODE_BF16;
  static constexpr bool SCALED = BLOCK || MX || NV;
  static constexpr int PKB = 128;                      // K bytes per pair (per row)
  static constexpr int CH = PKB / 16, RPI = 1024 / PKB;  // chunks per row, rows per DMA
  static constexpr int A_BYTES = BM * PKB, B_BYTES = BN * PKB;
  static constexpr int PAIR = A_BYTES + B_BYTES;
  // scale quads: 16 bytes per row cover QP pairs
  static constexpr int QP = BLOCK ? 4 : (MX ? 2 : 1);
  static constexpr int SQA = SCALED ? BM * 16 : 0;                  // [row][16 B]
  static constexpr int SQB = BLOCK ? 1024 : (SCALED ? BN * 16 : 0); // block: [2 blocks][16 B] (+copies)
  static constexpr int SQ = SQA + SQB;
  // grouped: per-tile epilogue scales sx[256] and sw[256] (fp32) in a ring
  // of three slots (the slot of tile t is refilled with tile t+3's first
  // pair, after tile t's epilogue even when a tile is a single pair)
  static constexpr int ES = GROUPED ? 2 * 256 * 4 : 0, NES = 3;
  // gather: the A-row tables (256 int32) of two tiles
  static constexpr int TAB = GATHER ? 256 * 4 : 0;
  static constexpr int TAB_OFF = 2 * PAIR + 2 * SQ + NES * ES;
  static constexpr int LDS = TAB_OFF + 2 * TAB;
  static constexpr int A_DMA = A_BYTES / 1024, B_DMA = B_BYTES / 1024;
  static constexpr int SA_DMA = SQA / 1024, SB_DMA = SQB / 1024;
  static constexpr int DATA_DMA = A_DMA + B_DMA, SC_DMA = SA_DMA + SB_DMA;
  static constexpr int DD = DATA_DMA / NW, DS = (SC_DMA + NW - 1) / NW, D = DD + DS;
  static_assert(DATA_DMA % NW == 0 && A_DMA % DD == 0, "whole waves per operand");
  static_assert(DS <= 1, "at most one scale DMA per wave and quad");
  static_assert(LDS <= 160 * 1024, "LDS budget");
  static_assert(!BLOCK || (WN <= 128 && 128 % WN == 0), "one weight-scale block per wave");
  static_assert(!GROUPED || MODE == MODE_FP8_TENSOR, "grouped: FP8 with row x channel scales");
  static_assert(!GROUPED || NW == 8, "grouped: one epilogue-scale DMA per wave");
  static_assert(!GATHER || (GROUPED && A_DMA == 4 * DD), "gather: A copied by waves 0-3");
};

// One output tile as the kernel sees it: where its A and W rows start, how
// many of them exist, and where it lands in C.
struct TileRef {
  const uint8_t *a, *b;   // first A / W row of the tile (row stride Kb)
  const uint8_t *a2, *b2; // the same rows of the second K segment (BF16; row stride Kb2)
  int arows, brows;       // rows that exist from there on (>= 1)
  int m0, n0;             // tile origin in C (dense: also in the scale matrices)
  int mend;               // C rows below mend exist (dense: M; grouped: the group's end)
  int e;                  // grouped: the tile's group
};

namespace pers {

// Pair-slot row swizzle: chunk c of row r lives in slot c ^ pair_swz(r).
// Its readers (32x32 fragments: lane = row, chunks 4p + 2h and 4p + 2h + 1,
// or 4h + 2p + kk for MXFP4) are conflict-free with it on gfx950.  It is
// linear in the row bits and uses only bits 1-3, so the copy plan forms
// pair_swz(wrow + j*RPI + vsub) as pair_swz(wrow + vsub) ^ pair_swz(j*RPI).
DSL_DEV int pair_swz(int row) { return (row >> 1) & 7; }

// Direct-to-LDS loads in the saddr form: a wave-uniform 64-bit base (SGPRs)
// plus a 32-bit per-lane offset (one VGPR).
DSL_DEV void dma16(const uint8_t *base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff),
               "s"(base), "s"(lds)
               : "memory", "m0");
}
// dma4 (64 lanes x 4 bytes) when the wave-uniform `on` is non-zero (see
// dma16_if below).
DSL_DEV void dma4_if(int on, const uint8_t *base, uint32_t voff, uint32_t lds) {
  asm volatile(
      "s_cmp_eq_u32 %3, 0\n\t"
      "s_cbranch_scc1 .Ldma4_skip_%=\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %0, %1\n"
      ".Ldma4_skip_%=:" ::"v"(voff),
      "s"(base), "s"(lds), "s"(on)
      : "memory", "m0", "scc");
}

// dma16 when the wave-uniform `on` is non-zero.  The test is a branch
// inside the asm, so the compiler sees straight-line code: a branch in the
// source splits the step into basic blocks, and the compiler then gathers
// all of the step's copies ahead of its MFMAs.
DSL_DEV void dma16_if(int on, const uint8_t *base, uint32_t voff, uint32_t lds) {
  asm volatile(
      "s_cmp_eq_u32 %3, 0\n\t"
      "s_cbranch_scc1 .Ldma_skip_%=\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1\n"
      ".Ldma_skip_%=:" ::"v"(voff),
      "s"(base), "s"(lds), "s"(on)
      : "memory", "m0", "scc");
}

// Lane id from v_mbcnt in volatile asm, so that the compiler cannot merge it
// with an earlier copy and keep that live.
DSL_DEV int lane_id() {
  int x;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(x));
  return x;
}

// Copy plan of one thread for the tile at (m0, n0): DD operand DMAs per pair
// (8 rows x 128 bytes each) and, for waves below SC_DMA, one scale DMA per
// quad (64 rows x 16 bytes).  A wave's operand DMAs all read the same
// operand (waves below A_DMA/DD copy A, the others W), so one uniform base
// serves them; the lane offsets are formed at issue time from the lane's row
// and chunk (a few VALU ops beside the MFMAs instead of DD live registers).
// `full`: this wave has a scale DMA.
template <class Cfg>
struct Ring {
  const uint8_t *dbase;          // operand rows of the tile, pair 0
  const uint8_t *dbase2;         // second K segment's rows (pairs nk1 ..), BF16
  const uint8_t *sbase;          // scale rows of the tile, quad 0
  int wrow;                      // the wave's first tile row (uniform)
  int lim;                       // last valid tile row of the operand (uniform)
  int kb;
  int kb2, nk1;                  // second segment: row stride, first pair
  int rmask;                     // second segment: pair index mask (W2 repeating), else all ones
  uint32_t vsub;                 // lane's row within one DMA
  uint32_t vchunk;               // lane's chunk byte offset for even DMAs
  uint32_t soff;                 // lane's scale offset
  int wave;
  bool full;
  bool isA;                      // this wave copies A
  uint32_t grw[Cfg::GATHER ? Cfg::DD : 1];   // gather, A waves: x row of the lane's DMA j

  DSL_DEV void target(const TileRef &tr, int kb_, int wave_, int lane, int kb2_ = 0,
                      int ldb2_ = 0, int rep2_ = 0) {
    wave = wave_;
    nk1 = kb_ / Cfg::PKB;
    full = Cfg::DS > 0 && wave < Cfg::SC_DMA;
    isA = wave * Cfg::DD < Cfg::A_DMA;
    kb2 = isA || ldb2_ == 0 ? kb2_ : ldb2_;
    rmask = isA || rep2_ == 0 ? 0x7fffffff : rep2_ - 1;
    lim = (isA ? tr.arows : tr.brows) - 1;
    kb = kb_;
    wrow = (isA ? wave * Cfg::DD : wave * Cfg::DD - Cfg::A_DMA) * Cfg::RPI;
    dbase = isA ? tr.a : tr.b;
    dbase2 = isA ? tr.a2 : tr.b2;
    vsub = lane / Cfg::CH;
    // DMA j covers tile rows wrow + j*RPI + vsub; RPI is even, so the row
    // swizzle only depends on vsub and the parity of wrow/RPI + j
    vchunk = (uint32_t)(((lane % Cfg::CH) ^ pair_swz(wrow + (int)vsub)) * 16);
    sbase = tr.a;
    soff = 0;
  }
  // scale plan of a dense scaled tile at (m0, n0)
  DSL_DEV void target_scales(const GemmArgs &p, int m0, int n0, int lane) {
    if constexpr (Cfg::SCALED) {
      // bytes per scale row: fp32 per 128-K group, E8M0 per 32 elements or
      // E4M3 per 16
      const int64_t rowb = Cfg::BLOCK ? (int64_t)(p.K / 128) * 4
                                      : (Cfg::MX ? (int64_t)(p.K / 32) : (int64_t)(p.K / 16));
      if (wave < Cfg::SA_DMA) {
        int grow = m0 + wave * 64 + lane;
        grow = grow < p.M ? grow : p.M - 1;
        sbase = static_cast<const uint8_t *>(p.sa) + m0 * rowb;
        soff = (uint32_t)((grow - m0) * rowb);
      } else if (Cfg::BLOCK) {
        // lanes 0 / 1: the tile's two 128-column blocks (others repeat them)
        const int nbb = (p.N + 127) / 128, b0 = n0 / 128;
        int blk = b0 + (lane & 1);
        blk = blk < nbb ? blk : nbb - 1;
        sbase = static_cast<const uint8_t *>(p.sb) + b0 * rowb;
        soff = (uint32_t)((blk - b0) * rowb);
      } else {
        int grow = n0 + (wave - Cfg::SA_DMA) * 64 + lane;
        grow = grow < p.N ? grow : p.N - 1;
        sbase = static_cast<const uint8_t *>(p.sb) + n0 * rowb;
        soff = (uint32_t)((grow - n0) * rowb);
      }
    }
  }

  // operand DMA j of tile-local pair q into the pair slot at `slot`
  DSL_DEV void issue_data(int j, int q, uint32_t slot) const {
    int r = (int)vsub + (wrow + j * Cfg::RPI);
    r = r < lim ? r : lim;           // rows past the edge re-read the last row
    // swz(wrow + j*RPI + vsub) = swz(wrow + vsub) ^ swz(j*RPI): the row
    // offset j*RPI only flips bit 2 of the swizzle, by the parity of j
    const uint32_t ch = vchunk ^ (uint32_t)(pair_swz(j * Cfg::RPI) * 16);
    // r < 256 and Kb < 2^24 (checked at launch): a full-rate 24-bit multiply
    if constexpr (Cfg::BF16) {
      // pairs from nk1 on come from the second segment (selects, no branch)
      const bool s2 = q >= nk1;
      const uint8_t *base =
          s2 ? dbase2 + (int64_t)((q - nk1) & rmask) * Cfg::PKB : dbase + (int64_t)q * Cfg::PKB;
      dma16(base, __umul24((uint32_t)r, (uint32_t)(s2 ? kb2 : kb)) + ch,
            slot + (uint32_t)((wave * Cfg::DD + j) * 1024));
    } else if constexpr (Cfg::GATHER) {
      // A: the row table's x row (dbase is x itself); W: the tile's rows
      const uint32_t rr = isA ? grw[j] : (uint32_t)r;
      dma16(dbase + (int64_t)q * Cfg::PKB, __umul24(rr, (uint32_t)kb) + ch,
            slot + (uint32_t)((wave * Cfg::DD + j) * 1024));
    } else {
      dma16(dbase + (int64_t)q * Cfg::PKB, __umul24((uint32_t)r, (uint32_t)kb) + ch,
            slot + (uint32_t)((wave * Cfg::DD + j) * 1024));
    }
  }
  // gather, A waves, first tile: the x rows straight from the row table in
  // memory (before any copy is in flight)
  DSL_DEV void gather_rows_global(const int32_t *arow, int m0, int last, int xrows) {
    if constexpr (Cfg::GATHER) {
#pragma unroll
      for (int j = 0; j < Cfg::DD; ++j) {
        int r = wrow + j * Cfg::RPI + (int)vsub;
        r = r < last ? r : last;
        const uint32_t v = (uint32_t)arow[m0 + r];
        grw[j] = v < (uint32_t)xrows ? v : (uint32_t)(xrows - 1);
      }
    }
  }
  // gather, A waves: the x rows of the lane's DMAs from a tile's row table
  // (clamped to the group's rows when it was copied; x rows to xrows - 1)
  DSL_DEV void gather_rows(const int32_t *tab, int xrows) {
    if constexpr (Cfg::GATHER) {
#pragma unroll
      for (int j = 0; j < Cfg::DD; ++j) {
        const uint32_t v = (uint32_t)tab[wrow + j * Cfg::RPI + (int)vsub];
        grw[j] = v < (uint32_t)xrows ? v : (uint32_t)(xrows - 1);
      }
    }
  }
  // the wave's scale DMA of tile-local quad c into the quad slot at
  // `sslot`, when `on` (uniform)
  DSL_DEV void issue_scales(int on, int c, uint32_t sslot) const {
    const uint32_t dst = (uint32_t)(wave * 1024);   // SA parts, then SB right after
    dma16_if(on, sbase + (int64_t)c * 16, soff, sslot + dst);
  }
};

// Operand fragments of one 64-byte step (half p of a pair slot) of one wave:
// lane l holds row l%32 of each 32-row tile and 32 bytes of K, the layout
// of v_mfma_scale_f32_32x32x64_f8f6f4.  FP8: one MFMA per tile, K half
// h = l/32 (two 16-byte chunks 4p+2h, 4p+2h+1).
//
// MXFP4: two MFMAs per tile and step (kk = 0, 1); lane half h holds chunk
// 4h + 2p + kk of the pair = 32 elements = one E8M0 block.  Over the pair's
// four MFMAs (p, kk) the two lane halves cover blocks {2p+kk, 4+2p+kk}, all
// eight once, in the same order for A and W (a permutation of the K sum).
// With that order lane half h takes all its scales from word h of the
// row's two pair words, byte 2p + kk: the MFMA's op_sel selects it, so the
// word goes to the MFMA as read, once per pair.
//
// Scale words are read two 32-row tiles at a time: lane half h reads the
// whole 16-byte quad entry of its row in tile t + h (64 lanes, 64
// consecutive entries, 1 KB contiguous: no bank conflicts), and one
// v_permlane32_swap of the pair's two words leaves tile t's word in one
// register and tile t+1's in the other, for both lane halves.  Reading one
// 4-byte word per lane from 32 rows 16 bytes apart instead puts 4 lanes on
// each bank (8 rows per 128 bytes) for the tile's word alone.
template <class Cfg, int KIND = Cfg::MX ? 1 : (Cfg::NV ? 2 : 0)>
struct Frag {
  v8i a[Cfg::TM], b[Cfg::TN];
  static DSL_DEV v8i ld(const uint8_t *base, int row, int p, int h) {
    const int s = pair_swz(row), c0 = 4 * p + 2 * h;
    const v4i lo = *reinterpret_cast<const v4i *>(base + row * Cfg::PKB + ((c0 ^ s) << 4));
    const v4i hi = *reinterpret_cast<const v4i *>(base + row * Cfg::PKB + (((c0 + 1) ^ s) << 4));
    return (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
  DSL_DEV void load_a(const uint8_t *slot, const uint8_t *, int, int p, int i, int wm, int r32,
                      int h) {
    a[i] = ld(slot, wm * Cfg::WM + i * 32 + r32, p, h);
  }
  DSL_DEV void load_b(const uint8_t *slot, const uint8_t *, int, int p, int wn, int r32, int h) {
#pragma unroll
    for (int j = 0; j < Cfg::TN; ++j) b[j] = ld(slot + Cfg::A_BYTES, wn * Cfg::WN + j * 32 + r32, p, h);
  }
  DSL_DEV void share_scales(const Frag &) {}
};

template <class Cfg>
struct Frag<Cfg, 1> {
  v4i a[Cfg::TM][2], b[Cfg::TN][2];
  int as[Cfg::TM], bs[Cfg::TN];     // scale word h of the row's pair
  static DSL_DEV v4i ld(const uint8_t *base, int row, int c) {
    return *reinterpret_cast<const v4i *>(base + row * Cfg::PKB + ((c ^ pair_swz(row)) << 4));
  }
  // sq: quad slot; qw: first scale word of the pair in the row's 16 bytes
  // (2 x quad-local pair index).  The scale word is read with half 0.
  static_assert(Cfg::TM % 2 == 0 && Cfg::TN == 2, "scale words are read two tiles at a time");
  // words qw, qw + 1 (the pair's h = 0 / h = 1 words) of the quad entries of
  // tiles t (first) and t + 1 (second) of a 64-row span starting at row0,
  // for the calling lane's half
  static DSL_DEV void scale_pair(const uint8_t *sqrows, int row0, int qw, int r32, int h, int &first,
                                 int &second) {
    const v4i e = *reinterpret_cast<const v4i *>(sqrows + (row0 + h * 32 + r32) * 16);
    const int x = qw ? e[2] : e[0], y = qw ? e[3] : e[1];
    const auto s = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)y, false, false);
    first = (int)s[0];
    second = (int)s[1];
  }
  // The pair's scale words of tiles i-1 and i are read with odd i (half 0
  // only), after the MFMAs of both rows are issued.
  DSL_DEV void load_a(const uint8_t *slot, const uint8_t *sq, int qw, int p, int i, int wm,
                      int r32, int h) {
    const int row = wm * Cfg::WM + i * 32 + r32;
    a[i][0] = ld(slot, row, 4 * h + 2 * p);
    a[i][1] = ld(slot, row, 4 * h + 2 * p + 1);
    if (p == 0 && (i & 1)) scale_pair(sq, wm * Cfg::WM + (i - 1) * 32, qw, r32, h, as[i - 1], as[i]);
  }
  DSL_DEV void load_b(const uint8_t *slot, const uint8_t *sq, int qw, int p, int wn, int r32,
                      int h) {
#pragma unroll
    for (int j = 0; j < Cfg::TN; ++j) {
      const int row = wn * Cfg::WN + j * 32 + r32;
      b[j][0] = ld(slot + Cfg::A_BYTES, row, 4 * h + 2 * p);
      b[j][1] = ld(slot + Cfg::A_BYTES, row, 4 * h + 2 * p + 1);
    }
    if (p == 0) scale_pair(sq + Cfg::SQA, wn * Cfg::WN, qw, r32, h, bs[0], bs[1]);
  }
  // half 1 of a pair uses the scale words read with its half 0
  DSL_DEV void share_scales(const Frag &half0) {
#pragma unroll
    for (int j = 0; j < Cfg::TN; ++j) bs[j] = half0.bs[j];
  }
};

// NVFP4: the FP8 fragment layout (lane half h holds the 64 elements
// [64h, 64h+64) of the half as four u32 words, word s = elements 8s..8s+7,
// block s/2 of the lane's four) plus the lane's four E4M3 block-scale bytes
// (bytes 8p + 4h .. +3 of the row's 16 scale bytes of the pair).  K-step s
// of the 32x32x16 fp16 MFMA takes word s from both lane halves, the same
// element order for A and W.
template <class Cfg>
struct Frag<Cfg, 2> {
  v8i a[Cfg::TM], b[Cfg::TN];
  int as[Cfg::TM], bs[Cfg::TN];
  static DSL_DEV v8i ld(const uint8_t *base, int row, int p, int h) {
    return Frag<Cfg, 0>::ld(base, row, p, h);
  }
  DSL_DEV void load_a(const uint8_t *slot, const uint8_t *sq, int, int p, int i, int wm, int r32,
                      int h) {
    const int row = wm * Cfg::WM + i * 32 + r32;
    a[i] = ld(slot, row, p, h);
    as[i] = *reinterpret_cast<const int *>(sq + row * 16 + 8 * p + 4 * h);
  }
  DSL_DEV void load_b(const uint8_t *slot, const uint8_t *sq, int, int p, int wn, int r32, int h) {
#pragma unroll
    for (int j = 0; j < Cfg::TN; ++j) {
      const int row = wn * Cfg::WN + j * 32 + r32;
      b[j] = ld(slot + Cfg::A_BYTES, row, p, h);
      bs[j] = *reinterpret_cast<const int *>(sq + Cfg::SQA + row * 16 + 8 * p + 4 * h);
    }
  }
  DSL_DEV void share_scales(const Frag &) {}
};

// fp16 block scale (both halves of the result) of block `blk` (0..3) of a
// lane's E4M3 scale word
DSL_DEV v2h nv_scale2(int word, int blk) {
  const uint32_t w = blk >= 2 ? (uint32_t)word >> 16 : (uint32_t)word;
  const v2h t = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false);
  const _Float16 s = (blk & 1) ? t[1] : t[0];
  return (v2h){s, s};
}
// 8 E2M1 codes (low nibble first) times an fp16 scale, as 8 fp16 values
DSL_DEV v8h nv_deq(uint32_t w, v2h s2) {
  const v2h p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 0) * s2;
  const v2h p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 1) * s2;
  const v2h p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 2) * s2;
  const v2h p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 3) * s2;
  return (v8h){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// NVFP4 part i of a step: K-steps 2i and 2i+1 (block i of each lane's four)
// for all rows; W fragments are dequantized once per K-step.  With
// `last`, each A row is handed to `reload` right after its last MFMA of
// the step.  FRESH: the first MFMA of each tile (part 0, K-step 0) starts
// from zero instead of the accumulator.
template <class Cfg, bool FRESH, class Reload>
DSL_DEV void nv_part(int i, const Frag<Cfg> &fa, const Frag<Cfg> &fb,
                     v16f (&acc)[Cfg::TM][Cfg::TN], bool last, Reload &&reload) {
  const v16f zero = {};
  v2h sa[Cfg::TM], sb[Cfg::TN];
#pragma unroll
  for (int j = 0; j < Cfg::TN; ++j) sb[j] = nv_scale2(fb.bs[j], i);
#pragma unroll
  for (int r = 0; r < Cfg::TM; ++r) sa[r] = nv_scale2(fa.as[r], i);
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int st = 2 * i + u;
    v8h bq[Cfg::TN];
#pragma unroll
    for (int j = 0; j < Cfg::TN; ++j) bq[j] = nv_deq((uint32_t)fb.b[j][st], sb[j]);
#pragma unroll
    for (int r = 0; r < Cfg::TM; ++r) {
      const v8h aq = nv_deq((uint32_t)fa.a[r][st], sa[r]);
#pragma unroll
      for (int j = 0; j < Cfg::TN; ++j)
        acc[r][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
            bq[j], aq, (FRESH && i == 0 && u == 0) ? zero : acc[r][j], 0, 0, 0);
      if (last && u == 1) reload(r);
    }
  }
}

// MFMAs of row i for half P of a pair: W fragments from fb, A from fa
// (operands swapped).  FRESH: the tile's first MFMAs start from zero, so
// the epilogue does not clear the accumulators.
template <class Cfg, int P, bool FRESH = false>
DSL_DEV void mma_row(const Frag<Cfg> &fa, const Frag<Cfg> &fb, int i, v16f (&acc)[Cfg::TM][Cfg::TN]) {
  const v16f zero = {};
  if constexpr (Cfg::MX) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int j = 0; j < Cfg::TN; ++j) {
        const v4i &w4 = fb.b[j][kk], &a4 = fa.a[i][kk];
        const v8i w8 = {w4[0], w4[1], w4[2], w4[3], 0, 0, 0, 0};
        const v8i a8 = {a4[0], a4[1], a4[2], a4[3], 0, 0, 0, 0};
        acc[i][j] = kk == 0 ? __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                                  w8, a8, FRESH ? zero : acc[i][j], 4, 4, 2 * P, fb.bs[j], 2 * P,
                                  fa.as[i])
                            : __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                                  w8, a8, acc[i][j], 4, 4, 2 * P + 1, fb.bs[j], 2 * P + 1,
                                  fa.as[i]);
      }
  } else if constexpr (Cfg::BF16) {
    // the lane's 32 bytes are 16 bf16 of K: two 32x32x16 MFMAs, first and
    // second 16-byte chunk (the same K order for A and W)
#pragma unroll
    for (int j = 0; j < Cfg::TN; ++j) {
      const v8i &w = fb.b[j], &a = fa.a[i];
      const v8bf w0 = __builtin_bit_cast(v8bf, (v4i){w[0], w[1], w[2], w[3]});
      const v8bf w1 = __builtin_bit_cast(v8bf, (v4i){w[4], w[5], w[6], w[7]});
      const v8bf a0 = __builtin_bit_cast(v8bf, (v4i){a[0], a[1], a[2], a[3]});
      const v8bf a1 = __builtin_bit_cast(v8bf, (v4i){a[4], a[5], a[6], a[7]});
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w0, a0, FRESH ? zero : acc[i][j], 0, 0, 0);
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w1, a1, acc[i][j], 0, 0, 0);
    }
  } else {
#pragma unroll
    for (int j = 0; j < Cfg::TN; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
          fb.b[j], fa.a[i], FRESH ? zero : acc[i][j], 0, 0, 0, 0, 0, 0);
  }
}

}  // namespace pers

// Group g's row range with the offsets clamped into [0, rows] and made
// non-decreasing, so malformed tables can never address outside X / Y.
DSL_DEV int2 group_rows_of(const int32_t *off, int g, int rows) {
  int lo = off[g], hi = off[g + 1];
  lo = lo < 0 ? 0 : (lo > rows ? rows : lo);
  hi = hi < lo ? lo : (hi > rows ? rows : hi);
  return make_int2(lo, hi);
}

// Args: GemmArgs (dense) or GroupedArgs (Cfg::GROUPED).
template <class Cfg, class Args>
__global__ __launch_bounds__(Cfg::NT) __attribute__((amdgpu_waves_per_eu(Cfg::OCC, Cfg::OCC)))
void gemm_persist_kernel(const Args p) {
  constexpr int TM = Cfg::TM, TN = Cfg::TN;
  constexpr bool GR = Cfg::GROUPED;
  __shared__ __align__(16) uint8_t smem[Cfg::LDS];
  __shared__ int s_pre[GR ? kMaxGroups + 1 : 1];   // grouped: tile prefix per group
  __shared__ int s_off[GR ? kMaxGroups + 1 : 1];   // grouped: row offsets clamped to [0, rows]
  __shared__ int s_part[GR ? Cfg::NT : 1];
  const int b = blockIdx.x, grid = gridDim.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
  const int r32 = lane & 31, h = lane >> 5;
  const uint32_t lds0 = pipe::lds_addr(smem);
  const int nbn = (p.N + Cfg::BN - 1) / Cfg::BN;

  // per-tensor scales first: no global load may follow the DMA asm
  float s1 = 1.f, s2 = 1.f;
  int kb, my_tiles, ntiles;
  int xbase = 0, xstride = grid;   // local tile t is logical tile xbase + t * xstride
  if constexpr (!GR) {
    if constexpr (Cfg::MODE == MODE_FP8_TENSOR || Cfg::NV) {
      s1 = *p.ga;
      s2 = *p.gb;
    }
    kb = p.Kb;
    ntiles = ((p.M + Cfg::BM - 1) / Cfg::BM) * nbn;
    xbase = b;
    my_tiles = (ntiles - b + grid - 1) / grid;   // >= 1: grid <= ntiles
  } else {
    kb = p.K;
    // tile prefix over the groups (ceil(n_g / BM) * nbn tiles each), built
    // by every workgroup from the device offset table
    const int per = (p.G + Cfg::NT - 1) / Cfg::NT;
    const int g0 = tid * per, g1 = min(p.G, g0 + per);
    int local = 0;
    for (int gi = g0; gi < g1; ++gi) {
      const int2 gr = group_rows_of(p.offsets, gi, p.rows);
      local += ((gr.y - gr.x + Cfg::BM - 1) / Cfg::BM) * nbn;
    }
    s_part[tid] = local;
    __syncthreads();
    for (int off = 1; off < Cfg::NT; off <<= 1) {
      const int v = tid >= off ? s_part[tid - off] : 0;
      __syncthreads();
      s_part[tid] += v;
      __syncthreads();
    }
    int run = s_part[tid] - local;
    for (int gi = g0; gi < g1; ++gi) {
      s_pre[gi] = run;
      const int2 gr = group_rows_of(p.offsets, gi, p.rows);
      run += ((gr.y - gr.x + Cfg::BM - 1) / Cfg::BM) * nbn;
    }
    // the tile walk reads group rows from LDS: a global load after the
    // first copy would wait for every copy in flight (vmcnt is in order)
    for (int gi = tid; gi <= p.G; gi += Cfg::NT) {
      const int o = p.offsets[gi];
      s_off[gi] = o < 0 ? 0 : (o > p.rows ? p.rows : o);
    }
    if (tid == Cfg::NT - 1) s_pre[p.G] = s_part[Cfg::NT - 1];
    __syncthreads();
    ntiles = __builtin_amdgcn_readfirstlane(s_pre[p.G]);
    // XCD-aware order: dispatch ids go round-robin over the 8 XCDs, so XCD
    // x takes the contiguous logical range [x*q + min(x, rem), ...), in
    // which consecutive tiles share a group's W panels
    if (grid % 8 == 0) {
      const int x = b & 7, q = ntiles >> 3, rem = ntiles & 7;
      const int size = q + (x < rem ? 1 : 0), j0 = b >> 3;
      xbase = x * q + (x < rem ? x : rem) + j0;
      xstride = grid >> 3;
      my_tiles = size > j0 ? (size - j0 + xstride - 1) / xstride : 0;
    } else {
      xbase = b;
      my_tiles = b < ntiles ? (ntiles - b + grid - 1) / grid : 0;
    }
  }
  if (my_tiles <= 0) return;                      // before any copy is issued
  int kb2 = 0, ldb2 = 0, rep2 = 0;
  if constexpr (Cfg::BF16) {
    kb2 = p.Kb2;
    ldb2 = p.ldb2;
    rep2 = p.rep2;
  }
  const int nkp = (kb + kb2) / Cfg::PKB;          // pairs per tile, >= 1

  auto tile_ref = [&](int t) __attribute__((always_inline)) {
    TileRef tr;
    if constexpr (!GR) {
      int tm, tn;
      tile_coords(xbase + t * xstride, (p.M + Cfg::BM - 1) / Cfg::BM, nbn, tm, tn);
      tr.m0 = tm * Cfg::BM;
      tr.n0 = tn * Cfg::BN;
      tr.a = p.a + (int64_t)tr.m0 * kb;
      tr.b = p.b + (int64_t)tr.n0 * kb;
      tr.a2 = tr.b2 = nullptr;
      if constexpr (Cfg::BF16) {
        tr.a2 = p.a2 + (int64_t)tr.m0 * kb2;
        tr.b2 = p.b2 + (int64_t)tr.n0 * (ldb2 ? ldb2 : kb2);
      }
      tr.arows = p.M - tr.m0;
      tr.mend = p.M;
      tr.e = 0;
    } else {
      const int id = xbase + t * xstride;
      int l = 0, u = p.G - 1;              // largest group e with s_pre[e] <= id
      while (l < u) {
        const int mid = (l + u + 1) >> 1;
        if (s_pre[mid] <= id) l = mid;
        else u = mid - 1;
      }
      const int e = __builtin_amdgcn_readfirstlane(l);
      const int in = id - s_pre[e];
      const int mt = in / nbn, nt = in - mt * nbn;
      // the rows of group_rows_of(), from the clamped copy in LDS
      const int lo = s_off[e], hi0 = s_off[e + 1], hi = hi0 < lo ? lo : hi0;
      tr.m0 = __builtin_amdgcn_readfirstlane(lo + mt * Cfg::BM);
      tr.n0 = nt * Cfg::BN;
      tr.mend = __builtin_amdgcn_readfirstlane(hi);
      tr.a = Cfg::GATHER ? p.x : p.x + (int64_t)tr.m0 * kb;   // gather: rows from the table
      tr.b = p.w + ((int64_t)e * p.N + tr.n0) * kb;
      tr.a2 = tr.b2 = nullptr;
      tr.arows = tr.mend - tr.m0;
      tr.e = e;
    }
    tr.brows = p.N - tr.n0;
    return tr;
  };

  // issue cursor: the next pair to copy is pair iq of local tile it, global
  // pair number ig (its slot: ig % 2).  Past the workgroup's last pair the
  // cursor stays on it, so every step copies a pair (into a slot nobody reads
  // again) and all steps have the same shape; those repeats copy no scales.
  // iqc counts the quads begun (their slot: iqc % 2); grouped: ies is the
  // epilogue-scale slot of tile it.
  pers::Ring<Cfg> ring;
  int it = 0, iq = 0, ig = 0, iqc = -1, ies = 0;
  TileRef itr = tile_ref(0);
  auto retarget = [&]() __attribute__((always_inline)) {
    ring.target(itr, kb, wave, lane, kb2, ldb2, rep2);
    if constexpr (Cfg::SCALED) ring.target_scales(p, itr.m0, itr.n0, lane);
  };
  // gather: waves 0-3 copy tile t's row table (256 x rows, clamped to its
  // group's rows) into table slot t % 2, a tile ahead of its use
  auto copy_table = [&](int t) __attribute__((always_inline)) {
    if constexpr (Cfg::GATHER) {
      const TileRef nt = tile_ref(t);
      const int last = nt.mend - nt.m0 - 1;
      int k = wave * 64 + pers::lane_id();
      k = k < last ? k : last;
      pers::dma4_if(__builtin_amdgcn_readfirstlane((int)(wave < 4)),
                    reinterpret_cast<const uint8_t *>(p.arow + nt.m0), (uint32_t)k * 4u,
                    lds0 + (uint32_t)(Cfg::TAB_OFF + (t & 1) * Cfg::TAB + wave * 256));
    }
  };
  retarget();
  if constexpr (Cfg::GATHER) {
    if (ring.isA) ring.gather_rows_global(p.arow, itr.m0, itr.mend - itr.m0 - 1, p.xrows);
    if (my_tiles > 1) {
      copy_table(1);
      if (nkp == 1) {            // tile 1's first pair is copied in the prologue
        pipe::wait_vmcnt<0>();
        __syncthreads();
      }
    }
  }
  auto issue_pair_prep = [&]() __attribute__((always_inline)) {
    if (iq == nkp && it + 1 < my_tiles) {
      iq = 0;
      ++it;
      ies = ies == Cfg::NES - 1 ? 0 : ies + 1;
      itr = tile_ref(it);
      retarget();
      if constexpr (Cfg::GATHER) {
        // the table copied a tile ago (waited for and published by the
        // barrier before this point); then the next tile's
        if (ring.isA)
          ring.gather_rows(reinterpret_cast<const int32_t *>(smem + Cfg::TAB_OFF + (it & 1) * Cfg::TAB),
                           p.xrows);
        if (it + 1 < my_tiles) copy_table(it + 1);
      }
    }
  };
  auto slot_of = [&](int gp) __attribute__((always_inline)) { return lds0 + (uint32_t)((gp & 1) * Cfg::PAIR); };
  uint8_t *const squad = smem + 2 * Cfg::PAIR;   // the two scale-quad slots
  // issue the operand DMAs of the cursor's pair, spread over rows i of a
  // step (all of them when i < 0), and its scale quad if it begins one
  auto issue_part = [&](int i, int qq, uint32_t islot, bool quad) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < Cfg::DD; ++j)
      if (i < 0 || (j >= i * Cfg::DD / TM && j < (i + 1) * Cfg::DD / TM)) ring.issue_data(j, qq, islot);
    if constexpr (Cfg::SCALED) {
      if (i < 0 || i == TM - 1)
        ring.issue_scales(__builtin_amdgcn_readfirstlane((int)(quad && ring.full)), qq / Cfg::QP,
                          pipe::lds_addr(squad) + (uint32_t)((iqc & 1) * Cfg::SQ));
    }
    if constexpr (GR) {
      // a tile's first pair also brings its epilogue scales: waves 0-3 the
      // 256 row scales sx, waves 4-7 the 256 channel scales sw of its group
      if (i < 0 || i == TM - 1) {
        const bool rows = wave < 4;
        const int w4 = rows ? wave : wave - 4;
        const int last = (rows ? itr.mend - itr.m0 : p.N - itr.n0) - 1;
        int k = w4 * 64 + pers::lane_id();
        k = k < last ? k : last;
        const float *src = rows ? p.sx + itr.m0 : p.sw + (int64_t)itr.e * p.N + itr.n0;
        pers::dma4_if(__builtin_amdgcn_readfirstlane((int)(qq == 0 && iq < nkp)),
                      reinterpret_cast<const uint8_t *>(src), (uint32_t)k * 4u,
                      lds0 + (uint32_t)(2 * Cfg::PAIR + 2 * Cfg::SQ + ies * Cfg::ES + wave * 256));
      }
    }
  };

  // block scale of a lane's row i in the wave's column block for tile-local
  // pair q, from the quad slot `sq`
  auto block_scale = [&](const uint8_t *sq, int q, int i) __attribute__((always_inline)) {
    const float *sa = reinterpret_cast<const float *>(sq);
    const float *sb = reinterpret_cast<const float *>(sq + Cfg::SQA);
    const int g4 = q % Cfg::QP;
    return sa[(wm * Cfg::WM + i * 32 + r32) * 4 + g4] * sb[((wn * Cfg::WN) / 128) * 4 + g4];
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  float sc[TM];           // block: s_g(row) of the group the accumulator is expressed in
  float rt[TM];           // block: s_g / s_{g+1} at a group boundary
#pragma unroll
  for (int i = 0; i < TM; ++i) sc[i] = rt[i] = 1.f;

  // ---- epilogue of local tile t: convert, scale, store from registers.
  // Lane (r32, h) stores, for each of its rows, 4 consecutive columns per
  // (j, q): col = n0 + wn*WN + 32j + 8q + 4h.  Tiles whose columns all exist
  // (all but a ragged last column of tiles) take the wide-store path, where
  // rows past the end (a group's or the matrix's last partial tile) are
  // masked per lane; the rest check every element.
  int ces = 0;                     // grouped: epilogue-scale slot of the tile being finished
  auto epilogue = [&](int t) __attribute__((always_inline)) {
    // the lane's coordinates are formed afresh (opaque to CSE): values kept
    // from the prologue would be live across the whole loop and spill
    const int eln = pers::lane_id();
    const int r32 = eln & 31, h = eln >> 5;
    const TileRef tr = tile_ref(t);
    const int m0 = tr.m0, n0 = tr.n0, mend = tr.mend;
    void *cout;
    int64_t ldc;
    if constexpr (GR) {
      cout = p.y;
      ldc = p.ldy;
    } else {
      cout = p.c;
      ldc = p.ldc;
    }
    const int c0 = n0 + wn * Cfg::WN + 4 * h;
    const bool wide = n0 + Cfg::BN <= p.N && (ldc % (p.out_f32 ? 4 : 8)) == 0 &&
                      (reinterpret_cast<uintptr_t>(cout) & 15) == 0;
    const float *esx = reinterpret_cast<const float *>(smem + 2 * Cfg::PAIR + 2 * Cfg::SQ + ces * Cfg::ES);
    const float *esw = esx + 256;
    auto val = [&](int i, int j, int r) __attribute__((always_inline)) {
      float x = acc[i][j][r];
      if constexpr (GR) {
        // (acc * sx[row]) * sw[g, col], the grouped epilogue
        x = (x * esx[wm * Cfg::WM + i * 32 + r32]) *
            esw[wn * Cfg::WN + j * 32 + 8 * (r >> 2) + 4 * h + (r & 3)];
      } else if constexpr (Cfg::MODE == MODE_FP8_TENSOR || Cfg::NV) {
        x = (x * s1) * s2;   // the reference's order, triton/gemm/gemm_kernels.py:97
      } else if constexpr (Cfg::BLOCK) {
        x = x * sc[i];
      }
      return x;
    };
    if (wide) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int64_t row = m0 + wm * Cfg::WM + i * 32 + r32;
        if (p.out_f32) {
          float *dst = static_cast<float *>(cout) + row * ldc + c0;
          if (row < mend) {
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
              for (int q = 0; q < 4; ++q)
                *reinterpret_cast<float4 *>(dst + j * 32 + q * 8) =
                    make_float4(val(i, j, 4 * q), val(i, j, 4 * q + 1), val(i, j, 4 * q + 2),
                                val(i, j, 4 * q + 3));
          }
        } else {
          // Lane (h, r32) holds columns 8q + 4h .. +3 (q = 0..3) of row r32
          // of each 32x32 block.  Two lane exchanges regroup them so that
          // lane (h, g, r16), r32 = 16g + r16, holds the 8 columns 8(h+2g)
          // .. +7 of rows r16 (X) and 16 + r16 (Y): each store then writes
          // 16 rows x 64 contiguous bytes instead of 32 rows x 16 bytes.
          const int r16 = r32 & 15, seg = h + 2 * (r32 >> 4);
          const int rowx = m0 + wm * Cfg::WM + i * 32 + r16;     // X's row; Y's is rowx + 16
          uint16_t *dst = static_cast<uint16_t *>(cout) + (int64_t)rowx * ldc + n0 +
                          wn * Cfg::WN + 8 * seg;
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            uint32_t P[4][2];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              P[q][0] = pack_bf16x2(val(i, j, 4 * q), val(i, j, 4 * q + 1));
              P[q][1] = pack_bf16x2(val(i, j, 4 * q + 2), val(i, j, 4 * q + 3));
            }
            // upper half of the first operand <-> lower half of the second:
            // lane h=0 ends with columns 8q0 .. +7, lane h=1 with 8q0+8 .. +7
            uint32_t U[4], W[4];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
              const auto u = __builtin_amdgcn_permlane32_swap(P[0][k], P[1][k], false, false);
              const auto w = __builtin_amdgcn_permlane32_swap(P[2][k], P[3][k], false, false);
              U[k] = u[0];
              U[2 + k] = u[1];
              W[k] = w[0];
              W[2 + k] = w[1];
            }
            // odd 16-lane groups of U <-> even groups of W
            uint4 X, Y;
            {
              const auto t0 = __builtin_amdgcn_permlane16_swap(U[0], W[0], false, false);
              const auto t1 = __builtin_amdgcn_permlane16_swap(U[1], W[1], false, false);
              const auto t2 = __builtin_amdgcn_permlane16_swap(U[2], W[2], false, false);
              const auto t3 = __builtin_amdgcn_permlane16_swap(U[3], W[3], false, false);
              X = make_uint4(t0[0], t1[0], t2[0], t3[0]);
              Y = make_uint4(t0[1], t1[1], t2[1], t3[1]);
            }
            if (rowx < mend) *reinterpret_cast<uint4 *>(dst + j * 32) = X;
            if (rowx + 16 < mend) *reinterpret_cast<uint4 *>(dst + 16 * ldc + j * 32) = Y;
          }
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = m0 + wm * Cfg::WM + i * 32 + r32;
        if (row >= mend) continue;
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int col = c0 + j * 32 + 8 * (r >> 2) + (r & 3);
            if (col >= p.N) continue;
            const float v = val(i, j, r);
            if (p.out_f32) static_cast<float *>(cout)[(int64_t)row * ldc + col] = v;
            else static_cast<uint16_t *>(cout)[(int64_t)row * ldc + col] = f32_to_bf16(v);
          }
      }
    }
    // the next tile's fragment loads stay below the stores: hoisted into
    // the epilogue they would be live beside the accumulators
    __builtin_amdgcn_sched_barrier(0);
    ces = ces == Cfg::NES - 1 ? 0 : ces + 1;
  };

  // issue the cursor's pair (rows i of a step, or all when i < 0)
  auto issue_next = [&](int i, bool &quad, int &qq, uint32_t &islot) __attribute__((always_inline)) {
    issue_pair_prep();
    quad = iq < nkp && iq % Cfg::QP == 0;
    if (quad) ++iqc;
    qq = iq < nkp ? iq : nkp - 1;
    islot = slot_of(ig);
    if (i < 0) issue_part(-1, qq, islot, quad);
  };

  // ---- prologue: pairs 0 and 1 (pair 1 never begins a quad: quads are
  // whole and QP >= 2), then the fragments of step 0
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    bool quad;
    int qq;
    uint32_t islot;
    issue_next(-1, quad, qq, islot);
    ++iq;
    ++ig;
  }
  pipe::wait_vmcnt<Cfg::DD>();                // pair 0 landed, pair 1 may be in flight
  __syncthreads();
  // compute cursor: the pair whose half 0 was read last is tile-local pair
  // cq, in quad slot cqc % 2
  int cq = 0, cqc = 0;
  pers::Frag<Cfg> fa, fb[2];
  fb[0].load_b(smem, squad, 0, 0, wn, r32, h);
#pragma unroll
  for (int i = 0; i < TM; ++i) fa.load_a(smem, squad, 0, 0, i, wm, r32, h);
  if constexpr (Cfg::BLOCK) {
#pragma unroll
    for (int i = 0; i < TM; ++i) sc[i] = block_scale(squad, 0, i);
  }

  // First step of local pair gp: MFMAs of its half 0 (fragments in fb[0] /
  // fa), reads of its half 1 from the same slot (landed and published with
  // the pair).
  // RESCALE (block, not on a tile's first pair): the accumulator still
  // carries the previous group's scale; each row is brought to this group's
  // right before its first MFMA of the group, overlapping the MFMAs of the
  // row before and reading results that completed a step ago.
  // FRESH (a tile's first pair): the MFMAs start from zero.
  auto step0 = [&](auto tag, int gp) __attribute__((always_inline)) {
    constexpr bool RESCALE = Cfg::BLOCK && decltype(tag)::value == 1;
    constexpr bool FRESH = decltype(tag)::value == 2;
    const uint8_t *st = smem + (gp & 1) * Cfg::PAIR;
    const uint8_t *sq = squad + (cqc & 1) * Cfg::SQ;
    const int sw = (cq % Cfg::QP) * 2;              // MX: the pair's scale words
    fb[1].load_b(st, sq, sw, 1, wn, r32, h);
    fb[1].share_scales(fb[0]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      if constexpr (Cfg::NV) {
        pers::nv_part<Cfg, FRESH>(i, fa, fb[0], acc, i == TM - 1,
                           [&](int r) __attribute__((always_inline)) { fa.load_a(st, sq, sw, 1, r, wm, r32, h); });
      } else {
        if constexpr (RESCALE) {
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] *= rt[i];
        }
        pers::mma_row<Cfg, 0, FRESH>(fa, fb[0], i, acc);
        fa.load_a(st, sq, sw, 1, i, wm, r32, h);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Second step of local pair gp: wait for pair gp+1 (the only pair in
  // flight), barrier (publishes it; every wave has read pair gp), copy pair
  // gp+2 into the slot of pair gp during the MFMAs of half 1, read half 0 of
  // pair gp+1.  KIND 1: the group ends (block: rescale to the next group's
  // scale); KIND 2: the tile ends (epilogue, then the next tile's step 0).
  auto step1 = [&](auto kind_tag, int gp) __attribute__((always_inline)) {
    constexpr int KIND = decltype(kind_tag)::value;
    pipe::wait_vmcnt<0>();
    pipe::wait_lds();
    __syncthreads();
    const uint8_t *stn = smem + ((gp + 1) & 1) * Cfg::PAIR;
    bool quad;
    int qq;
    uint32_t islot;
    // grouped: the whole of pair gp+2 is issued here, right after the
    // barrier, so its copies get the most lead over the misses that a
    // group's W panels take (dense: spread over the MFMA rows below)
    issue_next(GR ? -1 : 0, quad, qq, islot);
    // the compute cursor moves to pair gp+1 (the next tile's first pair
    // after KIND 2)
    cq = KIND == 2 ? 0 : cq + 1;
    if (cq % Cfg::QP == 0) ++cqc;
    const uint8_t *sqn = squad + (cqc & 1) * Cfg::SQ;
    const int sw = (cq % Cfg::QP) * 2;              // MX: the pair's scale words
    if constexpr (KIND != 2) fb[0].load_b(stn, sqn, sw, 0, wn, r32, h);
    float sn[TM];
    if constexpr (Cfg::BLOCK) {
#pragma unroll
      for (int i = 0; i < TM; ++i) sn[i] = block_scale(sqn, cq, i);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      if constexpr (Cfg::NV) {
        pers::nv_part<Cfg, false>(i, fa, fb[1], acc, KIND != 2 && i == TM - 1,
                           [&](int r) __attribute__((always_inline)) { fa.load_a(stn, sqn, sw, 0, r, wm, r32, h); });
        issue_part(i, qq, islot, quad);
      } else {
        pers::mma_row<Cfg, 1>(fa, fb[1], i, acc);
        if constexpr (!GR) issue_part(i, qq, islot, quad);
        if constexpr (KIND != 2) fa.load_a(stn, sqn, sw, 0, i, wm, r32, h);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (Cfg::BLOCK && KIND == 1) {
      // the group ends: factors that bring the accumulator from this
      // group's scale to the next group's, applied by the next step0
#pragma unroll
      for (int u = 0; u < TM; ++u) {
        rt[u] = sc[u] * __builtin_amdgcn_rcpf(sn[u]);
        sc[u] = sn[u];
      }
    }
    ++iq;
    ++ig;
    if constexpr (KIND == 2) {
      epilogue(gp / nkp);
      if constexpr (Cfg::BLOCK) {
#pragma unroll
        for (int i = 0; i < TM; ++i) sc[i] = sn[i];   // the next tile's first group
      }
      fb[0].load_b(stn, sqn, sw, 0, wn, r32, h);
#pragma unroll
      for (int i = 0; i < TM; ++i) fa.load_a(stn, sqn, sw, 0, i, wm, r32, h);
    }
  };

  // Tiles, each a run of pairs; the tile's last pair is peeled, so no branch
  // carries MFMAs (the accumulators would be copied at the join).
  using K1 = std::integral_constant<int, 1>;
  using K2 = std::integral_constant<int, 2>;
  using Rescale = std::integral_constant<int, 1>;
  using Fresh = std::integral_constant<int, 2>;
  int gp = 0;
  for (int t = 0; t < my_tiles; ++t) {
    step0(Fresh{}, gp);
    for (int q = 0; q + 1 < nkp; ++q) {
      step1(K1{}, gp);
      ++gp;
      step0(Rescale{}, gp);
    }
    step1(K2{}, gp);
    ++gp;
  }
  // the ring's last copies target LDS this workgroup still owns: let them
  // land before the workgroup ends
  pipe::wait_vmcnt<0>();
}

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

template <int MODE>
static hipError_t launch_persist_mode(const GemmArgs &p, hipStream_t st) {
  using Cfg = PersCfg<MODE>;
  const int ntiles = ((p.M + Cfg::BM - 1) / Cfg::BM) * ((p.N + Cfg::BN - 1) / Cfg::BN);
  int grid = device_cu_count();
  if (grid > ntiles) grid = ntiles;
  gemm_persist_kernel<Cfg, GemmArgs><<<grid, Cfg::NT, 0, st>>>(p);
  return hipGetLastError();
}

bool persist_supported(int mode, int M, int N, int K, int Kb, bool scales16) {
  (void)M;
  (void)N;
  if (Kb % 128 != 0 || Kb < 128) return false;          // whole pairs of 64-byte steps
  if (Kb >= (1 << 24)) return false;                     // 24-bit row offsets
  if (mode == MODE_FP8_TENSOR || mode == MODE_BF16) return true;
  // scaled modes: whole 16-byte scale quads per row, 16-byte aligned rows
  if (mode == MODE_FP8_BLOCK || mode == MODE_MXFP4) return scales16 && K % 512 == 0;
  if (mode == MODE_NVFP4) return scales16 && K % 256 == 0;   // 16 scale bytes per row and pair
  return false;
}

hipError_t launch_gemm_persist(int mode, const GemmArgs &p, hipStream_t st) {
  switch (mode) {
    case MODE_FP8_TENSOR: return launch_persist_mode<MODE_FP8_TENSOR>(p, st);
    case MODE_FP8_BLOCK: return launch_persist_mode<MODE_FP8_BLOCK>(p, st);
    case MODE_MXFP4: return launch_persist_mode<MODE_MXFP4>(p, st);
    case MODE_NVFP4: return launch_persist_mode<MODE_NVFP4>(p, st);
    case MODE_BF16: return launch_persist_mode<MODE_BF16>(p, st);
    default: return hipErrorInvalidValue;
  }
}

bool grouped_persist_supported(const GroupedArgs &p) {
  return p.K % 128 == 0 && p.K >= 128 && p.K < (1 << 24) && p.G >= 1 && p.G <= kMaxGroups;
}

// The device-side tile count is not known here: the grid is one workgroup
// per CU (at most the tile-count upper bound); workgroups without a tile
// return before issuing anything.
template <class Cfg>
static hipError_t launch_grouped_persist_cfg(const GroupedArgs &p, hipStream_t st) {
  const int nbn = (p.N + Cfg::BN - 1) / Cfg::BN;
  const int64_t upper = ((int64_t)(p.rows + Cfg::BM - 1) / Cfg::BM + p.G) * nbn;
  int64_t grid = device_cu_count();
  if (grid > upper) grid = upper;
  if (grid < 1) grid = 1;
  gemm_persist_kernel<Cfg, GroupedArgs><<<(unsigned)grid, Cfg::NT, 0, st>>>(p);
  return hipGetLastError();
}

hipError_t launch_grouped_persist(const GroupedArgs &p, hipStream_t st) {
  if (p.arow) {
    // x rows are addressed by 32-bit offsets row * K
    if (p.xrows < 1 || (int64_t)p.xrows * p.K >= ((int64_t)1 << 32) || p.xrows >= (1 << 24))
      return hipErrorInvalidValue;
    return launch_grouped_persist_cfg<PersCfg<MODE_FP8_TENSOR, true, true>>(p, st);
  }
  return launch_grouped_persist_cfg<PersCfg<MODE_FP8_TENSOR, true>>(p, st);
}

}  // namespace dsl
