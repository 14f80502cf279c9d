// Streaming quantized GEMMs for gfx950 at skinny and mid M (M <= 1024; the
// router takes it while ceil(M/64) * N stays small):
// C[M,N] = A[M,K] . W[N,K]^T, FP8 per-tensor, FP8 1x128/128x128 block,
// MXFP4, NVFP4 and bf16, one launch, deterministic.  BASELINE config 1 (M=128,
// N=K=4096) and the decode shapes (M=16) run here.
//
// At these shapes the work per W byte is small (M flops per byte) and the
// output has too few large tiles to fill 256 CUs, so the kernel is laid out
// for streaming W once with every CU busy:
//   * a workgroup owns BM = 16*TMA activation rows and BN = 16*TN W rows of
//     C over all of K, TN chosen so that about a CU's worth of workgroups
//     cover C (the per-CU traffic (BM + BN) x K is then near its least);
//   * its four waves split that range into contiguous runs of CHUNK-byte
//     chunks.  For each chunk a wave streams its TN W tiles and then its TMA
//     activation tiles (16 rows x CHUNK bytes each, one direct-to-LDS load
//     per 1 KB) through NR private LDS regions, NR-1 items in flight behind
//     the one being consumed.  W tiles go into registers; each activation
//     tile is multiplied against them as it is read.  A wave waits for its
//     own loads only (no barrier until the final reduction);
//   * the waves' partial tiles are summed through LDS in a fixed order and
//     laid out row-major in LDS for 16-byte stores;
//   * one launch, no workspace, no atomics: the same bytes on every run;
//   * the M blocks of one W slice are launched 8 apart (same XCD, about the
//     same time), so the second reader finds the slice in that XCD's L2; W
//     loads carry the non-temporal hint, activations stay cached.
//
// MFMA: v_mfma_scale_f32_16x16x128_f8f6f4 (bf16: two v_mfma_f32_16x16x32_bf16),
// activation tile in the first operand: output register i of lane l is
// C[4*(l/16) + i][l%16], rows from the activation tile, columns from the W
// tile.  FP8 / bf16: lane group g holds 16-byte chunks g and g+4 of each
// 128-byte step; MXFP4: 512-element superblocks whose step j gives lane
// group g the 32-element block 4g+j (one u32 of 4 E8M0 bytes per lane and
// superblock, op_sel j picks the byte).  A and W share the order, so the
// sum is unchanged.  FP8 block: each 128-byte step is one 128-K group,
// folded as acc += part * (sa[m][grp] * sb[n/128][grp]), the group-partial
// form of cuda/gemm/fp8_gemm.cu:84-97; FP8 groupwise with per-column weight
// scales (that function's own layout sb[grp][n]) folds sa[m][grp] *
// sb[grp][n], one weight scale per lane (its output column) and group.  NVFP4: its E4M3 scales (one per
// 16 elements) are not powers of two, so both operands are dequantized
// exactly to fp16 (E2M1 x E4M3 has at most 6 significant bits) and go to
// v_mfma_f32_16x16x32_f16; a lane takes one 16-byte chunk per 128-element
// superblock, whose four words feed four MFMA steps; the fp32 global scales
// apply in the epilogue.
// LDS rows are CHUNK bytes; row r's 16-byte chunk c sits in slot c ^ r
// (r < 16), so the 16 lanes that read one logical chunk of 16 rows hit
// distinct bank groups.
#include <cstdlib>

#include "stream_core.h"

namespace dsl {

template <int MODE_, int TMA_, int TN_, int CHUNK_, int NR_>
struct StreamCfg {
  static constexpr int MODE = MODE_;
  static constexpr int TMA = TMA_, TN = TN_;         // 16-row activation / W tiles
  static constexpr int BM = 16 * TMA, BN = 16 * TN;
  static constexpr int NW = 4, NT = NW * 64;         // waves split K
  static constexpr bool MX = MODE == MODE_MXFP4;
  static constexpr bool BLOCK = mode_grouped_k(MODE);   // fp32 scales per 128-K group
  static constexpr bool GCOL = MODE == MODE_FP8_GCOL;   // ... per W row (output column)
  static constexpr bool NV = MODE == MODE_NVFP4;
  static constexpr int CHUNK = CHUNK_;               // bytes of one row per item
  static constexpr int STEPS = CHUNK / 128;          // 128-byte MFMA steps (FP8 block: groups)
  static constexpr int SBK = CHUNK / 256;            // MXFP4 512-element superblocks
  static constexpr int NSB = CHUNK / 64;             // NVFP4 128-element superblocks
  static constexpr int SPR = CHUNK / 16;             // 16-byte slots per row
  static constexpr int RPD = 1024 / CHUNK;           // rows per direct load
  static constexpr int DATA_DMA = 16 / RPD;          // direct loads per 16-row item
  // scale bytes per row per chunk: E8M0 per 32 elements, fp32 per 128-K
  // group, E4M3 per 16 elements
  static constexpr int SROW = MX ? CHUNK / 16 : (BLOCK ? 4 * STEPS : (NV ? CHUNK / 8 : 0));
  static constexpr bool SC16 = SROW >= 16;           // scales move 16 (else 4) bytes per lane
  static constexpr int AUX = SROW ? (SC16 ? 1024 : 256) : 0;
  static constexpr int DPI = DATA_DMA + (AUX ? 1 : 0);   // direct loads per item
  static constexpr int REGION = 16 * CHUNK + AUX;
  static constexpr int NR = NR_;                     // regions per wave
  static constexpr int P = TN + TMA;                 // items per chunk: W tiles, then A tiles
  static constexpr int RING = NW * NR * REGION;
  static constexpr int RED = NW * TN * TMA * 64 * 16;   // the waves' partial tiles
  static constexpr int TLD = BN + 4;                 // row pitch (floats) of the summed tile
  static constexpr int TILE = BM * TLD * 4;
  static constexpr int LDS = RING > RED + TILE ? RING : RED + TILE;
  static constexpr int CPT = BM * BN / NT;           // output columns per thread
  static_assert(CHUNK == 256 || CHUNK == 512, "chunk bytes");
  static_assert(!MX || CHUNK >= 256, "whole MXFP4 superblocks");
  static_assert(LDS <= 160 * 1024, "LDS budget");
  static_assert(NR >= 2 && (NR - 1) * DPI < 64, "vmcnt range");
  static_assert(CPT >= 1 && BN % CPT == 0, "epilogue mapping");
};

template <class Cfg>
struct StreamRegs {
  v8i wf[Cfg::TN][Cfg::STEPS];      // FP8 / bf16 W fragments of the current chunk
  v4i wq[Cfg::TN][Cfg::SBK][4];     // MXFP4 W fragments (16 bytes per step)
  int ws[Cfg::TN][Cfg::SBK];        // MXFP4 W E8M0 words
  float sb[Cfg::GCOL ? Cfg::TN : 1][Cfg::STEPS];   // FP8 block / groupwise: weight scales
                                                   // of the chunk's groups (GCOL: the lane's column)
  v4i wn[Cfg::TN][Cfg::NSB];        // NVFP4: the lane's 16-byte W chunk of each superblock
  uint32_t wsn[Cfg::TN][Cfg::NSB];  // NVFP4: that chunk's two E4M3 block scales (low 16 bits)
  v4f acc[Cfg::TN][Cfg::TMA];
};

// One workgroup's tile: C rows [m0, m0 + BM) x columns [n0, n0 + BN) of the
// problem p over all of K.  gsx / gsw (grouped FP8): the output is (acc *
// gsx[row]) * gsw[col] instead of the per-tensor scaling.  GATHER: row m of
// the problem reads activation row arow[m] (clamped to [0, xrows)) of p.a;
// each lane's row offsets are loaded once, before the first copy.
template <class Cfg, bool GATHER = false>
DSL_DEV void stream_tile(const GemmArgs &p, const int m0, const int n0, const float *gsx,
                         const float *gsw, const int *arow = nullptr, int xrows = 0) {
  constexpr int TMA = Cfg::TMA, TN = Cfg::TN, NW = Cfg::NW, P = Cfg::P, DPI = Cfg::DPI;
  constexpr int NR = Cfg::NR, CHUNK = Cfg::CHUNK, SROW = Cfg::SROW;
  __shared__ __align__(16) uint8_t lds[Cfg::LDS];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int nchunks = p.Kb / CHUNK;
  const int c_begin = nchunks * wave / NW, c_end = nchunks * (wave + 1) / NW;
  const int nitems = (c_end - c_begin) * P;
  uint8_t *my = lds + wave * NR * Cfg::REGION;
  const uint32_t R0 = dec::lds_addr(my);
  const int nkg = p.K / 128;                 // FP8 block: scale groups per row
  const int64_t sld = p.K / 32;              // MXFP4: E8M0 bytes per row
  // GATHER: the activation row each of the lane's direct loads reads, per
  // activation tile, as loaded; clamped and scaled to a byte offset only
  // where an activation copy is issued, so that the prologue's W copies
  // (issued first) do not wait for these loads
  int tokv[GATHER ? Cfg::TMA : 1][Cfg::DATA_DMA];
  if constexpr (GATHER) {
    const int sub = lane / Cfg::SPR;
#pragma unroll
    for (int t = 0; t < Cfg::TMA; ++t)
#pragma unroll
      for (int j = 0; j < Cfg::DATA_DMA; ++j)
        tokv[t][j] = arow[min(m0 + t * 16 + Cfg::RPD * j + sub, p.M - 1)];
  }

  // item it: chunk c_begin + it / P; kind it % P (< TN: W tile, else
  // activation tile kind - TN); region it % NR
  auto issue = [&](int it) {
    const int ch = c_begin + it / P, kind = it % P;
    const uint32_t dst = R0 + (uint32_t)((it % NR) * Cfg::REGION);
    const int64_t kb0 = (int64_t)ch * CHUNK;
    const bool isW = kind < TN;
    const int rbase = isW ? n0 + kind * 16 : m0 + (kind - TN) * 16;
    const int rlim = isW ? p.N - 1 : p.M - 1;
    const uint8_t *src = isW ? p.b : p.a;
    const int sub = lane / Cfg::SPR, slot = lane % Cfg::SPR;
#pragma unroll
    for (int j = 0; j < Cfg::DATA_DMA; ++j) {  // rows RPD*j + sub
      const int r = Cfg::RPD * j + sub;
      const int row = min(rbase + r, rlim);    // rows past the edge re-read the last row
      int64_t roff = (int64_t)row * p.Kb;
      if constexpr (GATHER) {
        if (!isW) {                            // the activation tile's gathered row
          uint32_t tok = (uint32_t)tokv[0][j];
#pragma unroll
          for (int t = 1; t < Cfg::TMA; ++t)
            if (kind - TN == t) tok = (uint32_t)tokv[t][j];
          // entries outside [0, xrows), negative ones included, read row
          // xrows - 1 (xrows * Kb < 2^32)
          roff = (tok >= (uint32_t)xrows ? (uint32_t)xrows - 1 : tok) * (uint32_t)p.Kb;
        }
      }
      const uint8_t *s = src + roff + kb0 + ((slot ^ r) << 4);
      if (isW) dec::dma16_nt(s, dst + j * 1024);
      else dec::dma16(s, dst + j * 1024);
    }
    if constexpr (Cfg::AUX) {
      // the item's scales, row r at aux + r*SROW: 16-byte parts (lanes past
      // 16 rows repeat) or, with 8 bytes per row, 4-byte words
      constexpr int PARTS = Cfg::SC16 ? SROW / 16 : SROW / 4;
      const int sr = (lane / PARTS) & 15, part = lane % PARTS;
      const int row = isW ? (Cfg::BLOCK ? n0 : min(rbase + sr, rlim)) : min(rbase + sr, rlim);
      const uint8_t *sc;
      if constexpr (Cfg::GCOL) {
        if (isW) {
          // sb[grp][n] of the tile's 16 columns and the chunk's STEPS groups:
          // lane -> column lane % 16, group lane / 16 (repeated past STEPS),
          // stored [group][column]; 16 lanes read 64 contiguous bytes
          const int col = min(rbase + (lane & 15), rlim);
          const int grp = ch * Cfg::STEPS + ((lane >> 4) & (Cfg::STEPS - 1));
          dec::dma4(static_cast<const float *>(p.sb) + (int64_t)grp * p.N + col, dst + 16 * CHUNK);
          return;
        }
      }
      if constexpr (Cfg::MX) {
        sc = static_cast<const uint8_t *>(isW ? p.sb : p.sa) + row * sld + kb0 / 16;
      } else if constexpr (Cfg::NV) {   // E4M3 per 16 elements: K/16 bytes per row
        sc = static_cast<const uint8_t *>(isW ? p.sb : p.sa) + row * (int64_t)(p.K / 16) + kb0 / 8;
      } else {   // fp32 group scales of the chunk: sa[row][.], sb[n0/128][.]
        sc = reinterpret_cast<const uint8_t *>(
            isW ? static_cast<const float *>(p.sb) + (int64_t)(row / 128) * nkg
                : static_cast<const float *>(p.sa) + (int64_t)row * nkg) +
             (int64_t)ch * Cfg::STEPS * 4;
      }
      if constexpr (Cfg::SC16) dec::dma16(sc + part * 16, dst + 16 * CHUNK);
      else dec::dma4(sc + part * 4, dst + 16 * CHUNK);
    }
  };

  StreamRegs<Cfg> st;
#pragma unroll
  for (int t = 0; t < TN; ++t)
#pragma unroll
    for (int a = 0; a < TMA; ++a) st.acc[t][a] = (v4f){0.f, 0.f, 0.f, 0.f};

  auto chunk16 = [&](const uint8_t *base, int c) {      // row r16's logical chunk c
    return *reinterpret_cast<const v4i *>(base + r16 * CHUNK + ((c ^ r16) << 4));
  };

  auto consume = [&](auto kind_tag, const uint8_t *base) {
    constexpr int KIND = decltype(kind_tag)::value;
    const uint8_t *aux = base + 16 * CHUNK;
    if constexpr (KIND < TN) {                  // W tile -> registers
      if constexpr (Cfg::MX) {
#pragma unroll
        for (int b = 0; b < Cfg::SBK; ++b) {
#pragma unroll
          for (int j = 0; j < 4; ++j) st.wq[KIND][b][j] = chunk16(base, b * 16 + 4 * g + j);
          st.ws[KIND][b] = *reinterpret_cast<const int *>(aux + r16 * SROW + b * 16 + g * 4);
        }
      } else if constexpr (Cfg::NV) {
        // superblock b: lane group g takes 16-byte chunk 4b + g and its two
        // block scales (kept packed; dequantized per activation tile)
#pragma unroll
        for (int b = 0; b < Cfg::NSB; ++b) {
          const int c = 4 * b + g;
          st.wn[KIND][b] = chunk16(base, c);
          st.wsn[KIND][b] = *reinterpret_cast<const uint16_t *>(aux + r16 * SROW + 2 * c);
        }
      } else {
#pragma unroll
        for (int s = 0; s < Cfg::STEPS; ++s) {
          const v4i lo = chunk16(base, s * 8 + g), hi = chunk16(base, s * 8 + g + 4);
          st.wf[KIND][s] = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
        if constexpr (Cfg::GCOL) {
#pragma unroll
          for (int s = 0; s < Cfg::STEPS; ++s)
            st.sb[KIND][s] = reinterpret_cast<const float *>(aux)[s * 16 + r16];
        } else if constexpr (Cfg::BLOCK) {
#pragma unroll
          for (int s = 0; s < Cfg::STEPS; ++s) st.sb[0][s] = reinterpret_cast<const float *>(aux)[s];
        }
      }
    } else {                                    // activation tile x the W tiles
      constexpr int A = KIND - TN;
      if constexpr (Cfg::NV) {
        // word s of a lane's chunk holds elements 8s .. 8s+7 of it (block
        // s / 2); MFMA step s of superblock b sums word s of chunk 4b + g
        // over the lane groups g: the same permutation of K for A and W
#pragma unroll
        for (int b = 0; b < Cfg::NSB; ++b) {
          const int c = 4 * b + g;
          const v4i ad = chunk16(base, c);
          const v2h as2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(
              (uint32_t)*reinterpret_cast<const uint16_t *>(aux + r16 * SROW + 2 * c), 1.0f, false);
          v2h ws2[TN];
#pragma unroll
          for (int t = 0; t < TN; ++t)
            ws2[t] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(st.wsn[t][b], 1.0f, false);
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const v8h ah = fp4x8_to_f16((uint32_t)ad[s], as2[s >> 1]);
#pragma unroll
            for (int t = 0; t < TN; ++t) {
              const v8h wh = fp4x8_to_f16((uint32_t)st.wn[t][b][s], ws2[t][s >> 1]);
              st.acc[t][A] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, wh, st.acc[t][A], 0, 0, 0);
            }
          }
        }
      } else if constexpr (Cfg::MX) {
#pragma unroll
        for (int b = 0; b < Cfg::SBK; ++b) {
          const int asv = *reinterpret_cast<const int *>(aux + r16 * SROW + b * 16 + g * 4);
          v4i ad[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) ad[j] = chunk16(base, b * 16 + 4 * g + j);
#pragma unroll
          for (int t = 0; t < TN; ++t) {
            st.acc[t][A] = mfma_mx<0>(ad[0], st.wq[t][b][0], st.acc[t][A], asv, st.ws[t][b]);
            st.acc[t][A] = mfma_mx<1>(ad[1], st.wq[t][b][1], st.acc[t][A], asv, st.ws[t][b]);
            st.acc[t][A] = mfma_mx<2>(ad[2], st.wq[t][b][2], st.acc[t][A], asv, st.ws[t][b]);
            st.acc[t][A] = mfma_mx<3>(ad[3], st.wq[t][b][3], st.acc[t][A], asv, st.ws[t][b]);
          }
        }
      } else {
        float sa[4][Cfg::STEPS];                // FP8 block: rows 4g+i, the chunk's groups
        if constexpr (Cfg::BLOCK) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int s = 0; s < Cfg::STEPS; ++s)
              sa[i][s] = reinterpret_cast<const float *>(aux + (4 * g + i) * SROW)[s];
        }
#pragma unroll
        for (int s = 0; s < Cfg::STEPS; ++s) {
          const v4i lo = chunk16(base, s * 8 + g), hi = chunk16(base, s * 8 + g + 4);
          const v8i af = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
          for (int t = 0; t < TN; ++t) {
            if constexpr (Cfg::BLOCK) {
              const v4f zero = {0.f, 0.f, 0.f, 0.f};
              const v4f part = mfma_fp8(af, st.wf[t][s], zero);
              const v4f sc = (v4f){sa[0][s], sa[1][s], sa[2][s], sa[3][s]} *
                             st.sb[Cfg::GCOL ? t : 0][s];
              st.acc[t][A] = part * sc + st.acc[t][A];
            } else if constexpr (Cfg::MODE == MODE_BF16) {
              st.acc[t][A] = mfma_bf16(af, st.wf[t][s], st.acc[t][A]);
            } else {
              st.acc[t][A] = mfma_fp8(af, st.wf[t][s], st.acc[t][A]);
            }
          }
        }
      }
    }
  };

  // wait until at most `after` items (issued after the current one) are
  // outstanding: the current item has landed
  auto wait_item = [&](int after) {
    if (after >= NR - 1) {
      dec::wait_vm<(NR - 1) * DPI>();
    } else {
      dec::static_for<0, NR - 1>([&](auto q) {
        if (after == decltype(q)::value) dec::wait_vm<decltype(q)::value * DPI>();
      });
    }
  };

#pragma unroll
  for (int i = 0; i < NR - 1; ++i)
    if (i < nitems) issue(i);
  for (int base_it = 0; base_it < nitems; base_it += P) {
    auto step = [&](auto kind_tag) {
      constexpr int K = decltype(kind_tag)::value;
      const int it = base_it + K;
      // the region of item it-1 is free (its reads returned): refill it
      if (it + NR - 1 < nitems) issue(it + NR - 1);
      wait_item(nitems - 1 - it);
      consume(kind_tag, my + (it % NR) * Cfg::REGION);
      dec::wait_lds();
    };
    dec::static_for<0, P>(step);
  }

  // ---- sum the waves' partial tiles (wave order 0..3) into a row-major
  // tile T [BM][TLD] in LDS
  __syncthreads();                              // every wave is done with its regions
  float *red = reinterpret_cast<float *>(lds);  // [NW][TN][TMA][64 lanes][4]
  float *T = reinterpret_cast<float *>(lds + Cfg::RED);
#pragma unroll
  for (int t = 0; t < TN; ++t)
#pragma unroll
    for (int a = 0; a < TMA; ++a)
      *reinterpret_cast<v4f *>(red + (((wave * TN + t) * TMA + a) * 64 + lane) * 4) = st.acc[t][a];
  __syncthreads();
  for (int sl = threadIdx.x; sl < TN * TMA * 64; sl += Cfg::NT) {
    const int combo = sl >> 6, ln = sl & 63;   // combo = t * TMA + a
    v4f v = *reinterpret_cast<const v4f *>(red + (combo * 64 + ln) * 4);
#pragma unroll
    for (int w = 1; w < NW; ++w)
      v += *reinterpret_cast<const v4f *>(red + ((w * TN * TMA + combo) * 64 + ln) * 4);
    const int t = combo / TMA, a = combo % TMA;
    const int col = t * 16 + (ln & 15), row0 = a * 16 + 4 * (ln >> 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) T[(row0 + i) * Cfg::TLD + col] = v[i];
  }
  __syncthreads();

  constexpr int CPT = Cfg::CPT, GPR = Cfg::BN / CPT;
  if constexpr (Cfg::MODE == MODE_BF16) {
    if (p.lora_scales) {
      // LoRA: C^T, scaled per adapter column, as a bf16 hi + lo pair.
      // Thread -> tile column n (a row of the output) and CPT consecutive
      // tile rows, so that the NT / BN threads of one n cover its BM rows.
      constexpr int TPN = Cfg::NT / Cfg::BN, RPT = Cfg::BM / TPN;
      static_assert(TPN * RPT == Cfg::BM, "transposed epilogue mapping");
      const int tn = threadIdx.x / TPN, tm = (threadIdx.x % TPN) * RPT;
      const int ncol = n0 + tn;
      if (ncol >= p.N) return;
      uint16_t *orow = static_cast<uint16_t *>(p.c) + (int64_t)ncol * p.ldc;
      for (int i = 0; i < RPT && m0 + tm + i < p.M; ++i) {
        const int m = m0 + tm + i;
        const float v = T[(tm + i) * Cfg::TLD + tn] * p.lora_scales[m / p.lora_rank];
        const uint16_t h = f32_to_bf16(v);
        orow[m] = h;
        orow[p.M + m] = f32_to_bf16(v - bf16_to_f32(h));
      }
      if (m0 == 0 && tm == 0)
        for (int64_t c = 2 * (int64_t)p.M; c < p.ldc; ++c) orow[c] = 0;
      return;
    }
  }
  const int lrow = threadIdx.x / GPR, lcol = (threadIdx.x % GPR) * CPT;
  float v[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) v[c] = T[lrow * Cfg::TLD + lcol + c];

  const int row = m0 + lrow, col0 = n0 + lcol;
  if (row >= p.M) return;
  if (gsx) {                                 // grouped: (acc * sx[row]) * sw[col]
    const float sxr = gsx[row];
#pragma unroll
    for (int c = 0; c < CPT; ++c) v[c] = (v[c] * sxr) * gsw[col0 + c < p.N ? col0 + c : p.N - 1];
  } else if constexpr (Cfg::MODE == MODE_FP8_TENSOR || Cfg::NV) {   // NVFP4: the global scales
    const float s1 = *p.ga, s2 = *p.gb;
#pragma unroll
    for (int c = 0; c < CPT; ++c) v[c] = (v[c] * s1) * s2;
  }
  if (p.out_f32) {
    float *dst = static_cast<float *>(p.c) + (int64_t)row * p.ldc + col0;
    if (CPT % 4 == 0 && col0 + CPT <= p.N && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
#pragma unroll
      for (int c = 0; c + 3 < CPT; c += 4) {
        v4f o = (v4f){v[c], v[c + 1], v[c + 2], v[c + 3]};
        if (p.accumulate) o = *reinterpret_cast<const v4f *>(dst + c) + o;   // C += result
        *reinterpret_cast<v4f *>(dst + c) = o;
      }
    } else {
      for (int c = 0; c < CPT && col0 + c < p.N; ++c) dst[c] = p.accumulate ? dst[c] + v[c] : v[c];
    }
  } else {
    uint16_t *dst = static_cast<uint16_t *>(p.c) + (int64_t)row * p.ldc + col0;
    if (CPT % 8 == 0 && col0 + CPT <= p.N && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
#pragma unroll
      for (int c = 0; c + 7 < CPT; c += 8)
        *reinterpret_cast<uint4 *>(dst + c) =
            make_uint4(pack_bf16x2(v[c], v[c + 1]), pack_bf16x2(v[c + 2], v[c + 3]),
                       pack_bf16x2(v[c + 4], v[c + 5]), pack_bf16x2(v[c + 6], v[c + 7]));
    } else if (CPT == 4 && col0 + 4 <= p.N && (reinterpret_cast<uintptr_t>(dst) & 7) == 0) {
      *reinterpret_cast<uint2 *>(dst) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    } else {
      for (int c = 0; c < CPT && col0 + c < p.N; ++c) dst[c] = f32_to_bf16(v[c]);
    }
  }
}

template <class Cfg>
__global__ __launch_bounds__(Cfg::NT) void gemm_stream_kernel(const GemmArgs p) {
  // workgroup -> (M block, N block); the M blocks of one W slice are 8 apart
  const int nmb = (p.M + Cfg::BM - 1) / Cfg::BM;
  const int nnb = (p.N + Cfg::BN - 1) / Cfg::BN;
  const int local = blockIdx.x >> 3;
  const int mblk = local % nmb, nblk = (local / nmb) * 8 + (blockIdx.x & 7);
  if (nblk >= nnb) return;                   // whole workgroup: no barrier reached
  stream_tile<Cfg>(p, mblk * Cfg::BM, nblk * Cfg::BN, nullptr, nullptr);
}

// Grouped FP8 (MoE) on the streaming tiles: workgroup -> (BM-row block of one
// group's rows, BN-row slice of that group's W).  Each workgroup builds the
// groups' block prefix from the device offset table (clamped to [0, rows]
// and made non-decreasing, as the persistent grouped kernel does); blocks
// past the total exit before any load.  A group's W slice is streamed once
// per row block, so at decode sizes (a few rows per group) W is read once.
template <class Cfg, bool GATHER>
__global__ __launch_bounds__(Cfg::NT) void gemm_stream_grouped_kernel(const GroupedArgs gp) {
  __shared__ int s_pre[kMaxGroups + 1];      // row blocks before group e
  __shared__ int s_sum[Cfg::NW];
  const int tid = threadIdx.x;
  const int per = (gp.G + Cfg::NT - 1) / Cfg::NT;
  auto off_of = [&](int e) {                 // offsets clamped to [0, rows], non-decreasing use below
    int o = gp.offsets[e];
    return o < 0 ? 0 : (o > gp.rows ? gp.rows : o);
  };
  int mine = 0;
  for (int i = 0; i < per; ++i) {
    const int e = tid * per + i;
    if (e < gp.G) {
      const int lo = off_of(e), hi0 = off_of(e + 1), hi = hi0 < lo ? lo : hi0;
      mine += (hi - lo + Cfg::BM - 1) / Cfg::BM;
    }
  }
  // exclusive prefix of the threads' sums: a shuffle scan within each wave,
  // then the earlier waves' totals
  const int lane = tid & 63, wv = tid >> 6;
  int incl = mine;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int t = __shfl_up(incl, d, 64);
    if (lane >= d) incl += t;
  }
  if (lane == 63) s_sum[wv] = incl;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wv; ++w) base += s_sum[w];
  if (tid == Cfg::NT - 1) s_pre[gp.G] = base + incl;
  {
    int run = base + incl - mine;
    for (int i = 0; i < per; ++i) {
      const int e = tid * per + i;
      if (e < gp.G) {
        s_pre[e] = run;
        const int lo = off_of(e), hi0 = off_of(e + 1), hi = hi0 < lo ? lo : hi0;
        run += (hi - lo + Cfg::BM - 1) / Cfg::BM;
      }
    }
  }
  __syncthreads();
  const int nnb = (gp.N + Cfg::BN - 1) / Cfg::BN;
  const int id = blockIdx.x / nnb, nblk = blockIdx.x - id * nnb;
  if (id >= s_pre[gp.G]) return;             // whole workgroup, before any load
  int l = 0, u = gp.G - 1;                   // largest group e with s_pre[e] <= id
  while (l < u) {
    const int mid = (l + u + 1) >> 1;
    if (s_pre[mid] <= id) l = mid;
    else u = mid - 1;
  }
  const int e = __builtin_amdgcn_readfirstlane(l);
  const int lo = off_of(e), hi0 = off_of(e + 1), hi = hi0 < lo ? lo : hi0;
  GemmArgs q{};
  q.a = GATHER ? gp.x : gp.x + (int64_t)lo * gp.K;   // gathered rows index x itself
  q.b = gp.w + (int64_t)e * gp.N * gp.K;
  q.c = static_cast<uint8_t *>(gp.y) + (int64_t)lo * gp.ldy * (gp.out_f32 ? 4 : 2);
  q.M = hi - lo;
  q.N = gp.N;
  q.K = gp.K;
  q.Kb = gp.K;
  q.ldc = gp.ldy;
  q.out_f32 = gp.out_f32;
  stream_tile<Cfg, GATHER>(q, (id - s_pre[e]) * Cfg::BM, nblk * Cfg::BN, gp.sx + lo,
                           gp.sw + (int64_t)e * gp.N, GATHER ? gp.arow + lo : nullptr, gp.xrows);
}

// ---------------------------------------------------------------- plans --
namespace {

struct StreamPlan {
  int tma, tn;
};

// Activation tiles by M (16, 32 or 64 rows per workgroup; 256-byte chunks
// for the skinny ones, 512-byte chunks otherwise; rows of an odd number of
// 256-byte chunks take the 32-row tiles), and the most W tiles
// per workgroup (4, 2, 1) that still leave >= 192 workgroups: fewer but
// larger workgroups read A and W fewer times (measured at M = 96..256), as
// long as they cover most CUs.  DSL_GEMM_STREAM_TMA / DSL_GEMM_STREAM_TN
// override them (tuning).
StreamPlan plan_for(int mode, int M, int N, int Kb) {
  StreamPlan pl;
  pl.tma = M <= 16 ? 1 : ((M <= 32 || Kb % 512 != 0) ? 2 : 4);
  const char *et = getenv("DSL_GEMM_STREAM_TMA");
  const bool force_tma = et && (et[0] == '1' || et[0] == '2' || (et[0] == '4' && Kb % 512 == 0)) && !et[1];
  if (force_tma) pl.tma = et[0] - '0';
  const int64_t nmb = (M + 16 * pl.tma - 1) / (16 * pl.tma);
  pl.tn = 1;
  for (int tn = 4; tn >= 2; tn /= 2)
    if (nmb * ((N + 16 * tn - 1) / (16 * tn)) >= 192) {
      pl.tn = tn;
      break;
    }
  // 33..64 rows (FP8 per-tensor, bf16): two 32-row blocks of two W tiles
  // read (32 + 32) K-rows per workgroup against (64 + 16) for one 64-row
  // block, when that grid is one round of 192 or more workgroups (M=64
  // N=4096 K=4096: 7.4 against 8.1 us per-tensor, 11.3 against 12.2 bf16;
  // past one round, and in the block / MXFP4 forms, it measured slower)
  if (!force_tma && (mode == MODE_FP8_TENSOR || mode == MODE_BF16) && M > 32 && M <= 64 &&
      pl.tma == 4) {
    const int64_t g = (int64_t)((M + 31) / 32) * ((N + 31) / 32);
    if (g >= 192 && g <= device_cu_count()) pl.tma = pl.tn = 2;
  }
  const char *e = getenv("DSL_GEMM_STREAM_TN");
  if (e && (e[0] == '1' || e[0] == '2' || e[0] == '4') && !e[1]) pl.tn = e[0] - '0';
  if (pl.tn == 4 && mode_grouped_k(mode) && pl.tma == 4) pl.tn = 2;   // register budget
  if (pl.tn == 4 && mode == MODE_NVFP4 && pl.tma == 4) pl.tn = 2;      // register budget
  return pl;
}

template <int MODE, int TMA, int TN, int CHUNK>
hipError_t launch_cfg(const GemmArgs &p, hipStream_t st) {
  using Cfg = StreamCfg<MODE, TMA, TN, CHUNK, 4>;
  const int nmb = (p.M + Cfg::BM - 1) / Cfg::BM;
  const int nnb = (p.N + Cfg::BN - 1) / Cfg::BN;
  const int grid = 8 * nmb * ((nnb + 7) / 8);
  gemm_stream_kernel<Cfg><<<grid, Cfg::NT, 0, st>>>(p);
  return hipGetLastError();
}

template <int MODE, int TMA, int CHUNK>
hipError_t launch_tn(const GemmArgs &p, int tn, hipStream_t st) {
  if (tn == 1) return launch_cfg<MODE, TMA, 1, CHUNK>(p, st);
  // four W tiles beside four activation tiles exceed the registers of the
  // FP8 block and NVFP4 forms (plan_for never asks for them)
  constexpr bool four = !(TMA == 4 && (mode_grouped_k(MODE) || MODE == MODE_NVFP4));
  if constexpr (four) {
    if (tn == 4) return launch_cfg<MODE, TMA, 4, CHUNK>(p, st);
  }
  return launch_cfg<MODE, TMA, 2, CHUNK>(p, st);
}

template <int MODE>
hipError_t launch_mode(const GemmArgs &p, const StreamPlan &pl, hipStream_t st) {
  if (pl.tma == 1) return launch_tn<MODE, 1, 256>(p, pl.tn, st);
  if (pl.tma == 2) return launch_tn<MODE, 2, 256>(p, pl.tn, st);
  return launch_tn<MODE, 4, 512>(p, pl.tn, st);
}

template <int TMA, int TN, int CHUNK>
hipError_t launch_grouped_cfg(const GroupedArgs &gp, hipStream_t st) {
  using Cfg = StreamCfg<MODE_FP8_TENSOR, TMA, TN, CHUNK, 4>;
  const int64_t nnb = (gp.N + Cfg::BN - 1) / Cfg::BN;
  const int64_t blocks = (gp.rows + Cfg::BM - 1) / Cfg::BM + gp.G;   // >= sum of per-group blocks
  const int64_t grid = blocks * nnb;
  if (grid >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
  if (gp.arow)
    gemm_stream_grouped_kernel<Cfg, true><<<(unsigned)grid, Cfg::NT, 0, st>>>(gp);
  else
    gemm_stream_grouped_kernel<Cfg, false><<<(unsigned)grid, Cfg::NT, 0, st>>>(gp);
  return hipGetLastError();
}

}  // namespace

bool grouped_stream_supported(const GroupedArgs &gp) {
  if (gp.arow && (gp.xrows < 1 || (int64_t)gp.xrows * gp.K >= ((int64_t)1 << 32))) return false;
  return gp.G >= 1 && gp.G <= kMaxGroups && gp.K % 256 == 0 && gp.K >= 256 && gp.N >= 1;
}

// Row blocks of 16 or 32 rows by the groups' average size (the router sends
// averages below 48 here); four 16-row W tiles per workgroup.  Measured
// (64 experts, N=1536 K=2048, 3 weight copies rotated): 16-row blocks up to
// 4 rows per group on average, 32-row blocks above (32 tokens x top-8:
// 31.5 against 33.7 us; 64 tokens: 34.9 against 37.6); two W tiles per
// workgroup were 12-22% slower (32 tokens 37.6 us, 128 tokens 56.2 against
// 41.6), one W tile or 512-byte chunks slower still, and 64-row blocks
// 30-90% slower.  Against the persistent kernel the crossover stays at 48
// rows per group (384 tokens: 62.2 against 62.7 us).
hipError_t launch_grouped_stream(const GroupedArgs &gp, hipStream_t st) {
  if (!grouped_stream_supported(gp)) return hipErrorInvalidValue;
  if (gp.rows / gp.G <= 4) return launch_grouped_cfg<1, 4, 256>(gp, st);
  return launch_grouped_cfg<2, 4, 256>(gp, st);
}

bool stream_supported(int mode, int M, int N, int K, int Kb, bool scales16) {
  if (M < 1 || M > 1024 || N < 1) return false;
  if (Kb % 256 != 0) return false;   // 512-byte chunks where they fit, else 256
  if (mode == MODE_FP8_TENSOR || mode == MODE_BF16) return true;
  // block scales and E8M0 rows move by 16-byte direct loads (K % 512)
  if (mode_grouped_k(mode) || mode == MODE_MXFP4) return scales16 && K % 512 == 0;
  // E4M3 rows (K/16 bytes) move by 16-byte direct loads
  if (mode == MODE_NVFP4) return scales16 && K % 256 == 0;
  return false;
}

hipError_t launch_gemm_stream(int mode, const GemmArgs &p, hipStream_t st) {
  if (p.lora_scales && (mode != MODE_BF16 || p.lora_rank < 1 || p.ldc < 2 * (int64_t)p.M))
    return hipErrorInvalidValue;
  if (p.accumulate && (!p.out_f32 || p.lora_scales)) return hipErrorInvalidValue;
  const StreamPlan pl = plan_for(mode, p.M, p.N, p.Kb);
  switch (mode) {
    case MODE_FP8_TENSOR: return launch_mode<MODE_FP8_TENSOR>(p, pl, st);
    case MODE_FP8_BLOCK: return launch_mode<MODE_FP8_BLOCK>(p, pl, st);
    case MODE_FP8_GCOL: return launch_mode<MODE_FP8_GCOL>(p, pl, st);
    case MODE_MXFP4: return launch_mode<MODE_MXFP4>(p, pl, st);
    case MODE_BF16: return launch_mode<MODE_BF16>(p, pl, st);
    case MODE_NVFP4: return launch_mode<MODE_NVFP4>(p, pl, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace dsl
