// Tile machinery shared by the dense and grouped GEMM kernels.
//
// One workgroup computes a BM x BN output tile with WGM x WGN waves; each
// wave owns a (BM/WGM) x (BN/WGN) sub-tile made of 16x16 MFMA tiles.
// K advances in "stages" of 128 bytes per operand row (FP8: 128 elements,
// one 16x16x128 MFMA step; FP4: 256 elements, two steps).  Stages are
// double-buffered in LDS; global loads of stage s+1 are issued before the
// MFMAs of stage s and written to LDS after them, with one barrier per
// stage.  LDS rows are 128 B (eight 16-B chunks); chunk c of row r lives at
// chunk slot c ^ (r & 7) so that lanes reading the same logical chunk of
// consecutive rows hit different banks.
//
// Scale handling per mode:
//   FP8_TENSOR  unscaled fp8 MFMA over all K, (acc * sa) * sb in the epilogue;
//   FP8_BLOCK   one fresh MFMA partial per 128-K group, folded into the fp32
//               accumulator as acc += part * (sa[m,g] * sb[n/128,g]);
//   FP8_GCOL    the same with one weight scale per column: sb[g,n];
//   MXFP4       E8M0 bytes go straight into v_mfma_scale_f32_16x16x128_f8f6f4;
//   NVFP4       E2M1 -> fp16 (hardware convert), times the E4M3 block scale
//               in fp16 (exact), fp16 MFMA; global scales in the epilogue;
//   BF16        unscaled bf16 MFMA (a stage is 64 elements of K).
#pragma once

#include "common.h"
#include "launch.h"

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

namespace dsl {

template <int MODE, int BM_, int BN_, int WGM_, int WGN_>
struct TileCfg {
  static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_;
  static constexpr int NT = WGM * WGN * 64;
  static constexpr int WM = BM / WGM, WN = BN / WGN;
  static constexpr int TM = WM / 16, TN = WN / 16;
  static constexpr int A_CH = (BM * 8 + NT - 1) / NT;           // 16-B chunks / thread / stage
  static constexpr int B_CH = (BN * 8 + NT - 1) / NT;
  static constexpr int SCB = MODE == MODE_MXFP4 ? 8 : (MODE == MODE_NVFP4 ? 16 : 0);
  static constexpr int SBN = BN >= 128 ? BN / 128 : 1;           // FP8_BLOCK weight scales / stage
  static constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128;
  static constexpr int SA_BYTES = mode_grouped_k(MODE) ? BM * 4 : BM * SCB;
  static constexpr int SB_BYTES = MODE == MODE_FP8_BLOCK ? 16 * ((SBN * 4 + 15) / 16)
                                  : (MODE == MODE_FP8_GCOL ? BN * 4 : BN * SCB);
  static constexpr int OFF_B = 2 * A_BYTES;
  static constexpr int OFF_SA = OFF_B + 2 * B_BYTES;
  static constexpr int OFF_SB = OFF_SA + 2 * SA_BYTES;
  static constexpr int LDS = OFF_SB + 2 * SB_BYTES;
  static_assert(WM % 16 == 0 && WN % 16 == 0, "wave tile must be a multiple of 16");
  static_assert(NT >= BM && NT >= BN, "one thread per row loads the stage's scales");
  static_assert(MODE != MODE_FP8_BLOCK || WN <= 128, "block scales assume WN <= 128");
};

// Operand rows of one output tile.
struct TileView {
  const uint8_t *a;     // row m0 of A
  const uint8_t *b;     // row n0 of B
  int a_rows, b_rows;   // valid rows (<= BM / BN)
  int Kb, K;            // bytes per packed row, K in elements
  const void *sa;       // MX/NV: scale row m0; FP8_BLOCK / GCOL: float row m0 ([.][nkg])
  const void *sb;       // MX/NV: scale row n0; FP8_BLOCK: float row n0/128; GCOL: &sb[0][n0]
  int64_t sa_ld, sb_ld; // scale row pitch (elements; GCOL sb: N, one row per group)
};

DSL_DEV int swz(int row, int ch) { return (ch ^ (row & 7)) << 4; }

template <class Cfg> struct StageRegs {
  uint4 a[Cfg::A_CH];
  uint4 b[Cfg::B_CH];
  uint4 sa, sb;         // scale staging (MX: .x/.y, NV: all four, BLOCK: .x as float bits)
};

// ------------------------------------------------------------ global load --
template <int MODE, class Cfg>
DSL_DEV void stage_load(const TileView &tv, int ks, StageRegs<Cfg> &r) {
  const int tid = threadIdx.x;
  const int kb0 = ks * 128;
#pragma unroll
  for (int j = 0; j < Cfg::A_CH; ++j) {
    const int i = tid + j * Cfg::NT, row = i >> 3, kb = kb0 + ((i & 7) << 4);
    r.a[j] = (i < Cfg::BM * 8 && row < tv.a_rows && kb < tv.Kb)
                 ? *reinterpret_cast<const uint4 *>(tv.a + (int64_t)row * tv.Kb + kb)
                 : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < Cfg::B_CH; ++j) {
    const int i = tid + j * Cfg::NT, row = i >> 3, kb = kb0 + ((i & 7) << 4);
    r.b[j] = (i < Cfg::BN * 8 && row < tv.b_rows && kb < tv.Kb)
                 ? *reinterpret_cast<const uint4 *>(tv.b + (int64_t)row * tv.Kb + kb)
                 : make_uint4(0, 0, 0, 0);
  }
  if constexpr (MODE == MODE_MXFP4 || MODE == MODE_NVFP4) {
    // SCB scale bytes per row per stage; blocks past K get code 0x7F/0x38 (1.0).
    constexpr int SCB = Cfg::SCB;
    const int nblk = MODE == MODE_MXFP4 ? tv.K / 32 : tv.K / 16;
    const uint8_t one = MODE == MODE_MXFP4 ? 0x7F : 0x38;
    const int blk0 = ks * SCB;
    auto load_row = [&](const uint8_t *base, int64_t ld, int row, int rows) -> uint4 {
      uint8_t v[16];
#pragma unroll
      for (int t = 0; t < SCB; ++t) {
        const int blk = blk0 + t;
        v[t] = (row < rows && blk < nblk) ? base[(int64_t)row * ld + blk] : one;
      }
#pragma unroll
      for (int t = SCB; t < 16; ++t) v[t] = 0;
      uint4 o;
      o.x = v[0] | (v[1] << 8) | (v[2] << 16) | ((uint32_t)v[3] << 24);
      o.y = v[4] | (v[5] << 8) | (v[6] << 16) | ((uint32_t)v[7] << 24);
      o.z = v[8] | (v[9] << 8) | (v[10] << 16) | ((uint32_t)v[11] << 24);
      o.w = v[12] | (v[13] << 8) | (v[14] << 16) | ((uint32_t)v[15] << 24);
      return o;
    };
    if (tid < Cfg::BM)
      r.sa = load_row(static_cast<const uint8_t *>(tv.sa), tv.sa_ld, tid, tv.a_rows);
    if (tid < Cfg::BN)
      r.sb = load_row(static_cast<const uint8_t *>(tv.sb), tv.sb_ld, tid, tv.b_rows);
  } else if constexpr (MODE == MODE_FP8_GCOL) {
    if (tid < Cfg::BM)
      r.sa.x = tid < tv.a_rows
                   ? f2u(static_cast<const float *>(tv.sa)[(int64_t)tid * tv.sa_ld + ks])
                   : 0u;
    if (tid < Cfg::BN)
      r.sb.x = tid < tv.b_rows
                   ? f2u(static_cast<const float *>(tv.sb)[(int64_t)ks * tv.sb_ld + tid])
                   : 0u;
  } else if constexpr (MODE == MODE_FP8_BLOCK) {
    if (tid < Cfg::BM)
      r.sa.x = tid < tv.a_rows
                   ? f2u(static_cast<const float *>(tv.sa)[(int64_t)tid * tv.sa_ld + ks])
                   : 0u;
    if (tid < Cfg::SBN) {
      const int nrow_blocks = (tv.b_rows + 127) / 128;
      r.sb.x = tid < nrow_blocks
                   ? f2u(static_cast<const float *>(tv.sb)[(int64_t)tid * tv.sb_ld + ks])
                   : 0u;
    }
  }
}

// ------------------------------------------------------------- LDS store --
template <int MODE, class Cfg>
DSL_DEV void stage_store(uint8_t *smem, int buf, const StageRegs<Cfg> &r) {
  const int tid = threadIdx.x;
  uint8_t *sA = smem + buf * Cfg::A_BYTES;
  uint8_t *sB = smem + Cfg::OFF_B + buf * Cfg::B_BYTES;
#pragma unroll
  for (int j = 0; j < Cfg::A_CH; ++j) {
    const int i = tid + j * Cfg::NT, row = i >> 3, ch = i & 7;
    if (i < Cfg::BM * 8) *reinterpret_cast<uint4 *>(sA + row * 128 + swz(row, ch)) = r.a[j];
  }
#pragma unroll
  for (int j = 0; j < Cfg::B_CH; ++j) {
    const int i = tid + j * Cfg::NT, row = i >> 3, ch = i & 7;
    if (i < Cfg::BN * 8) *reinterpret_cast<uint4 *>(sB + row * 128 + swz(row, ch)) = r.b[j];
  }
  uint8_t *sSa = smem + Cfg::OFF_SA + buf * Cfg::SA_BYTES;
  uint8_t *sSb = smem + Cfg::OFF_SB + buf * Cfg::SB_BYTES;
  if constexpr (MODE == MODE_MXFP4) {
    // bytes b0..b7 (blocks of this stage) -> [b0 b4 b1 b5 b2 b6 b3 b7]: lane
    // group g reads a u16 holding its blocks for sub-steps 0 and 1.
    auto perm = [](uint4 v) {
      return make_uint2(__builtin_amdgcn_perm(v.y, v.x, 0x05010400u),
                        __builtin_amdgcn_perm(v.y, v.x, 0x07030602u));
    };
    if (tid < Cfg::BM) *reinterpret_cast<uint2 *>(sSa + tid * 8) = perm(r.sa);
    if (tid < Cfg::BN) *reinterpret_cast<uint2 *>(sSb + tid * 8) = perm(r.sb);
  } else if constexpr (MODE == MODE_NVFP4) {
    // 16 group scales -> lane group g gets [2g, 2g+1, 8+2g, 9+2g] as one u32.
    auto perm = [](uint4 v) {
      uint4 o;
      o.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
      o.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
      o.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
      o.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
      return o;
    };
    if (tid < Cfg::BM) *reinterpret_cast<uint4 *>(sSa + tid * 16) = perm(r.sa);
    if (tid < Cfg::BN) *reinterpret_cast<uint4 *>(sSb + tid * 16) = perm(r.sb);
  } else if constexpr (MODE == MODE_FP8_BLOCK) {
    if (tid < Cfg::BM) reinterpret_cast<uint32_t *>(sSa)[tid] = r.sa.x;
    if (tid < Cfg::SBN) reinterpret_cast<uint32_t *>(sSb)[tid] = r.sb.x;
  } else if constexpr (MODE == MODE_FP8_GCOL) {
    if (tid < Cfg::BM) reinterpret_cast<uint32_t *>(sSa)[tid] = r.sa.x;
    if (tid < Cfg::BN) reinterpret_cast<uint32_t *>(sSb)[tid] = r.sb.x;
  }
}

// ----------------------------------------------------------- MFMA helpers --
DSL_DEV v4f mfma_fp8(const v8i &a, const v8i &b, const v4f &c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// bf16: the lane's 32 bytes are 16 elements of K, fed as two 16x16x32
// MFMAs (first and second 16-byte chunk; the same K order for A and W).
DSL_DEV v4f mfma_bf16(const v8i &a, const v8i &b, const v4f &c) {
  const v8bf a0 = __builtin_bit_cast(v8bf, (v4i){a[0], a[1], a[2], a[3]});
  const v8bf a1 = __builtin_bit_cast(v8bf, (v4i){a[4], a[5], a[6], a[7]});
  const v8bf b0 = __builtin_bit_cast(v8bf, (v4i){b[0], b[1], b[2], b[3]});
  const v8bf b1 = __builtin_bit_cast(v8bf, (v4i){b[4], b[5], b[6], b[7]});
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1, __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0, c, 0, 0, 0), 0, 0, 0);
}

template <int OPS>
DSL_DEV v4f mfma_mx(const v4i &a, const v4i &b, const v4f &c, int sa, int sb) {
  const v8i a8 = {a[0], a[1], a[2], a[3], 0, 0, 0, 0};
  const v8i b8 = {b[0], b[1], b[2], b[3], 0, 0, 0, 0};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8, b8, c, 4, 4, OPS, sa, OPS, sb);
}

// 8 E2M1 codes (one u32, even element in the low nibble) times an E4M3
// block scale, as 8 fp16 values (exact).
DSL_DEV v8h fp4x8_to_f16(uint32_t w, _Float16 s) {
  const v2h s2 = {s, s};
  v2h p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 0) * s2;
  v2h p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 1) * s2;
  v2h p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 2) * s2;
  v2h p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 3) * s2;
  return (v8h){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

DSL_DEV _Float16 e4m3_to_f16(uint32_t code) { return (_Float16)e4m3_decode((uint8_t)code); }

// ---------------------------------------------------------------- compute --
template <int MODE, class Cfg>
DSL_DEV void stage_compute(const uint8_t *smem, int buf, v4f (&acc)[Cfg::TM][Cfg::TN]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
  const int r16 = lane & 15, g = lane >> 4;
  const uint8_t *sA = smem + buf * Cfg::A_BYTES;
  const uint8_t *sB = smem + Cfg::OFF_B + buf * Cfg::B_BYTES;
  const uint8_t *sSa = smem + Cfg::OFF_SA + buf * Cfg::SA_BYTES;
  const uint8_t *sSb = smem + Cfg::OFF_SB + buf * Cfg::SB_BYTES;
  const int arow0 = wm * Cfg::WM + r16, brow0 = wn * Cfg::WN + r16;

  if constexpr (MODE == MODE_FP8_TENSOR || mode_grouped_k(MODE) || MODE == MODE_BF16) {
    v8i bop[Cfg::TN];
#pragma unroll
    for (int tn = 0; tn < Cfg::TN; ++tn) {
      const int row = brow0 + tn * 16;
      const uint8_t *rp = sB + row * 128;
      const v4i lo = *reinterpret_cast<const v4i *>(rp + swz(row, 2 * g));
      const v4i hi = *reinterpret_cast<const v4i *>(rp + swz(row, 2 * g + 1));
      bop[tn] = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
    float sbv = 0.f, sbc[Cfg::TN];   // BLOCK: the wave's 128-column block; GCOL: per column
    if constexpr (MODE == MODE_FP8_BLOCK)
      sbv = reinterpret_cast<const float *>(sSb)[(wn * Cfg::WN) / 128];
    if constexpr (MODE == MODE_FP8_GCOL) {
#pragma unroll
      for (int tn = 0; tn < Cfg::TN; ++tn) sbc[tn] = reinterpret_cast<const float *>(sSb)[brow0 + tn * 16];
    }
#pragma unroll
    for (int tm = 0; tm < Cfg::TM; ++tm) {
      const int row = arow0 + tm * 16;
      const uint8_t *rp = sA + row * 128;
      const v4i lo = *reinterpret_cast<const v4i *>(rp + swz(row, 2 * g));
      const v4i hi = *reinterpret_cast<const v4i *>(rp + swz(row, 2 * g + 1));
      const v8i aop = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      if constexpr (MODE == MODE_FP8_TENSOR) {
#pragma unroll
        for (int tn = 0; tn < Cfg::TN; ++tn) acc[tm][tn] = mfma_fp8(aop, bop[tn], acc[tm][tn]);
      } else if constexpr (MODE == MODE_BF16) {
#pragma unroll
        for (int tn = 0; tn < Cfg::TN; ++tn) acc[tm][tn] = mfma_bf16(aop, bop[tn], acc[tm][tn]);
      } else {
        const v4f sa4 = *reinterpret_cast<const v4f *>(
            reinterpret_cast<const float *>(sSa) + wm * Cfg::WM + tm * 16 + 4 * g);
        const v4f s4 = sa4 * sbv;
        const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int tn = 0; tn < Cfg::TN; ++tn) {
          const v4f part = mfma_fp8(aop, bop[tn], zero);
          if constexpr (MODE == MODE_FP8_GCOL) acc[tm][tn] = part * (sa4 * sbc[tn]) + acc[tm][tn];
          else acc[tm][tn] = part * s4 + acc[tm][tn];
        }
      }
    }
  } else if constexpr (MODE == MODE_MXFP4) {
    v4i bop0[Cfg::TN], bop1[Cfg::TN];
    int bsc[Cfg::TN];
#pragma unroll
    for (int tn = 0; tn < Cfg::TN; ++tn) {
      const int row = brow0 + tn * 16;
      const uint8_t *rp = sB + row * 128;
      bop0[tn] = *reinterpret_cast<const v4i *>(rp + swz(row, g));
      bop1[tn] = *reinterpret_cast<const v4i *>(rp + swz(row, 4 + g));
      bsc[tn] = *reinterpret_cast<const uint16_t *>(sSb + row * 8 + 2 * g);
    }
#pragma unroll
    for (int tm = 0; tm < Cfg::TM; ++tm) {
      const int row = arow0 + tm * 16;
      const uint8_t *rp = sA + row * 128;
      const v4i a0 = *reinterpret_cast<const v4i *>(rp + swz(row, g));
      const v4i a1 = *reinterpret_cast<const v4i *>(rp + swz(row, 4 + g));
      const int asc = *reinterpret_cast<const uint16_t *>(sSa + row * 8 + 2 * g);
#pragma unroll
      for (int tn = 0; tn < Cfg::TN; ++tn) {
        acc[tm][tn] = mfma_mx<0>(a0, bop0[tn], acc[tm][tn], asc, bsc[tn]);
        acc[tm][tn] = mfma_mx<1>(a1, bop1[tn], acc[tm][tn], asc, bsc[tn]);
      }
    }
  } else {  // MODE_NVFP4: fp16 MFMA 16x16x32 on dequantized operands
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      v8h bop[Cfg::TN][4];
#pragma unroll
      for (int tn = 0; tn < Cfg::TN; ++tn) {
        const int row = brow0 + tn * 16;
        const v4i raw = *reinterpret_cast<const v4i *>(sB + row * 128 + swz(row, 4 * q + g));
        const uint32_t sw = *reinterpret_cast<const uint32_t *>(sSb + row * 16 + 4 * g);
        const _Float16 s0 = e4m3_to_f16((sw >> (16 * q)) & 0xFF);
        const _Float16 s1 = e4m3_to_f16((sw >> (16 * q + 8)) & 0xFF);
        bop[tn][0] = fp4x8_to_f16((uint32_t)raw[0], s0);
        bop[tn][1] = fp4x8_to_f16((uint32_t)raw[1], s0);
        bop[tn][2] = fp4x8_to_f16((uint32_t)raw[2], s1);
        bop[tn][3] = fp4x8_to_f16((uint32_t)raw[3], s1);
      }
#pragma unroll
      for (int tm = 0; tm < Cfg::TM; ++tm) {
        const int row = arow0 + tm * 16;
        const v4i raw = *reinterpret_cast<const v4i *>(sA + row * 128 + swz(row, 4 * q + g));
        const uint32_t sw = *reinterpret_cast<const uint32_t *>(sSa + row * 16 + 4 * g);
        const _Float16 s0 = e4m3_to_f16((sw >> (16 * q)) & 0xFF);
        const _Float16 s1 = e4m3_to_f16((sw >> (16 * q + 8)) & 0xFF);
        v8h aop[4];
        aop[0] = fp4x8_to_f16((uint32_t)raw[0], s0);
        aop[1] = fp4x8_to_f16((uint32_t)raw[1], s0);
        aop[2] = fp4x8_to_f16((uint32_t)raw[2], s1);
        aop[3] = fp4x8_to_f16((uint32_t)raw[3], s1);
#pragma unroll
        for (int tn = 0; tn < Cfg::TN; ++tn)
#pragma unroll
          for (int t = 0; t < 4; ++t)
            acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop[t], bop[tn][t], acc[tm][tn], 0, 0, 0);
      }
    }
  }
}

// --------------------------------------------------------------- mainloop --
template <int MODE, class Cfg>
DSL_DEV void tile_mainloop(const TileView &tv, int ks0, int ks1, uint8_t *smem,
                           v4f (&acc)[Cfg::TM][Cfg::TN]) {
#pragma unroll
  for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::TN; ++j) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};
  if (ks0 >= ks1) return;
  StageRegs<Cfg> r;
  stage_load<MODE, Cfg>(tv, ks0, r);
  stage_store<MODE, Cfg>(smem, 0, r);
  __syncthreads();
  for (int ks = ks0; ks < ks1; ++ks) {
    const int buf = (ks - ks0) & 1;
    const bool more = ks + 1 < ks1;
    if (more) stage_load<MODE, Cfg>(tv, ks + 1, r);
    stage_compute<MODE, Cfg>(smem, buf, acc);
    if (more) stage_store<MODE, Cfg>(smem, buf ^ 1, r);
    __syncthreads();
  }
}

// XCD-aware tile order: dispatch ids go round-robin over the 8 XCDs, so
// give each XCD a contiguous range of logical tiles, then raster the
// logical ids in groups of GROUP_M tile-rows (neighbours share A/B panels
// inside one XCD's L2).
DSL_DEV void tile_coords(int bid, int nbm, int nbn, int &tm, int &tn) {
  const int nb = nbm * nbn;
  const int x = bid & 7, local = bid >> 3;
  const int q = nb >> 3, rem = nb & 7;
  const int id = x * q + (x < rem ? x : rem) + local;
  constexpr int GROUP_M = 8;
  const int width = GROUP_M * nbn;
  const int group = id / width, first = group * GROUP_M;
  const int gsz = (nbm - first) < GROUP_M ? (nbm - first) : GROUP_M;
  const int in = id - group * width;
  tm = first + in % gsz;
  tn = in / gsz;
}

}  // namespace dsl
