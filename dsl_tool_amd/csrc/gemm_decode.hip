// Skinny-M ("decode") quantized GEMMs for gfx950: C[M,N] = A[M,K] . W[N,K]^T
// with few activation rows, bound by streaming W from HBM.
//
// gemm_decode_kernel (FP8 per-tensor, FP8 1x128/128x128 block, FP8 1x128
// groups with a weight scale per output column, MXFP4, bf16; M <= 32)
//   One workgroup owns 32 rows of W (two 16-row MFMA tiles) over the whole
//   of K; its four waves split K into contiguous ranges of whole 1 KB chunks
//   (1 KB of every row: 1024 FP8 or 2048 FP4 elements).  A wave streams a
//   sequence of "items" through two LDS regions: for each of its chunks, the
//   activation tiles (16 rows x 1 KB each) and then the two W tiles.  Each
//   item is 16 direct-to-LDS loads (one row's 1 KB per instruction, i.e.
//   eight whole 128-byte lines) plus, for block-scaled FP8 and MXFP4, one
//   more load of the item's scales.  Item i goes into region i % 2 as soon
//   as item i-2 has left it, so two items (32 KB) are always in flight per
//   wave and every wave waits for its own loads only (no barrier until the
//   final reduction).  Activation tiles are moved into registers and reused
//   for both W tiles, which halves the activation traffic of a 16-row
//   layout; W loads carry the non-temporal hint so the stream of W lines
//   does not evict the activations from L2.  The waves' partial tiles are
//   summed through LDS: one launch, no workspace, no atomics.
//
//   MFMA: v_mfma_scale_f32_16x16x128_f8f6f4.  Lane l supplies row l%16 of
//   its operand; lane group g = l/16 supplies a quarter of the step's K.
//   Output register i of lane l is C[4*g + i][l%16] (rows: activations,
//   columns: W rows).
//     FP8 tensor / block: a step is 128 K bytes; group g holds the 16-byte
//       chunks g and 4+g of the step (the same K order for A and W, so the
//       sum is unchanged; for block scales a step is exactly one 128-K scale
//       group, folded as acc += part * sa[m][grp] * sb[n/128][grp], the
//       group-partial form of cuda/gemm/fp8_gemm.cu:84-97; with per-column
//       weight scales sb[grp][n], each lane's column scale of the group).
//     bf16: as FP8 per-tensor with 64 elements per 128-byte step; the lane's
//       32 bytes feed two v_mfma_f32_16x16x32_bf16 (first and second chunk).
//     MXFP4: K is taken in 512-element superblocks of 4 steps; at step j of
//       a superblock group g holds the 32-element block 4g+j, so a lane's data
//       for the superblock is 64 contiguous bytes and its 4 E8M0 scale bytes
//       are one aligned u32 (opsel j picks the byte).  A and W use the same
//       permutation of K, which leaves every block paired with its own scale.
//   LDS: row r's 16-byte chunk c lives in slot c ^ r (r < 16), so the 16
//   lanes reading one logical chunk of the 16 rows hit 16 distinct bank
//   groups.
//
// gemv_nvfp4_kernel (NVFP4, M <= 4)
//   One wave owns RPW consecutive W rows over all of K (2, 4 or 8 by the
//   number of activation rows and K).  Lane l holds bytes
//   [16l, 16l+16) of every 1 KB chunk of a row (32 E2M1 codes = two 16-element
//   E4M3 blocks), so each load instruction reads one row's 1 KB
//   contiguously.  The E4M3 scales of the wave's rows are contiguous in
//   memory and arrive in LDS by 1 KB direct loads (a 2-byte load per lane
//   would cost a whole instruction per 128 bytes); the activations and their
//   scales are loaded once per workgroup into LDS and dequantized exactly to
//   fp16 (E2M1 x E4M3 has at most 5 significant bits), held in registers for
//   all of K.  W codes are converted to fp16 with unit scale and multiplied
//   by fp16 dot products with fp32 accumulation per 16-element block; each
//   block's E4M3 scale (hardware OCP E4M3 -> f32 conversion, exact) applies
//   once per block.  Each row's 64 lane partials are summed across the wave;
//   the fp32 global scales apply last, as in the dense NVFP4 kernel.
#include "stream_core.h"

namespace dsl {


template <int MODE_, int TMA_>
struct DecodeCfg {
  static constexpr int MODE = MODE_;
  static constexpr int TMA = TMA_;                  // 16-row activation tiles (M <= 16*TMA)
  static constexpr int TN = 2;                      // 16-row W tiles per workgroup
  static constexpr int NW = 4, NT = NW * 64;        // waves split K
  static constexpr bool MX = MODE == MODE_MXFP4;
  static constexpr bool BLOCK = mode_grouped_k(MODE);     // fp32 scales per 128-K group
  static constexpr bool GCOL = MODE == MODE_FP8_GCOL;     // ... per W row (output column)
  static constexpr int CHUNK = 1024;                // bytes of one row per item
  static constexpr int AUX = (MX || BLOCK) ? 1024 : 0;   // scale bytes per item (DMA target)
  // scale DMAs per item (GCOL: two 4-byte copies of the W tile's 16 x 8
  // column scales; activation items repeat their one copy, so that every
  // item is the same number of loads for the vmcnt count)
  static constexpr int ADMA = GCOL ? 2 : (AUX ? 1 : 0);
  static constexpr int DPI = 16 + ADMA;             // DMA instructions per item
  static constexpr int REGION = 16 * CHUNK + AUX;
  static constexpr int P = TMA + TN;                // items per chunk
  static_assert(2 * NW * REGION + NW * TN * TMA * 1024 <= 160 * 1024, "LDS budget");
};

// Register state of one wave: activation fragments of the current chunk,
// their block scales, and the accumulators.
template <class Cfg>
struct DecodeRegs {
  static constexpr int TMA = Cfg::TMA;
  v8i af[TMA][8];               // FP8: 8 steps of 32 bytes per lane
  v4f sa[TMA][8];               // FP8 block: sa[4g+i][group] of the 8 groups
  v4i ad[TMA][4][4];            // MXFP4: 4 superblocks x 4 steps of 16 bytes
  int as[TMA][4];               // MXFP4: E8M0 u32 per superblock
  v4f acc[Cfg::TN][TMA];
};

template <class Cfg>
__global__ __launch_bounds__(Cfg::NT) void gemm_decode_kernel(const GemmArgs p) {
  constexpr int TMA = Cfg::TMA, TN = Cfg::TN, NW = Cfg::NW, P = Cfg::P, DPI = Cfg::DPI;
  constexpr int CHUNK = Cfg::CHUNK;
  __shared__ __align__(16) uint8_t region[NW][2][Cfg::REGION];
  __shared__ __align__(16) float red[NW][TN][TMA][64][4];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int nb0 = blockIdx.x * 16 * TN;
  const int nchunks = p.Kb / CHUNK;
  const int c_begin = nchunks * wave / NW, c_end = nchunks * (wave + 1) / NW;
  const int nitems = (c_end - c_begin) * P;
  const uint32_t R0 = dec::lds_addr(region[wave][0]), R1 = dec::lds_addr(region[wave][1]);
  const int nkg = p.K / 128;              // FP8 block: scale groups per row
  const int64_t sld = p.K / 32;           // MXFP4: E8M0 bytes per row

  // item it: chunk c_begin + it / P; kind it % P (< TMA: activation tile,
  // else W tile kind - TMA); region it % 2
  auto issue = [&](int it) {
    const int ch = c_begin + it / P, kind = it % P;
    const uint32_t dst = (it & 1) ? R1 : R0;
    const int64_t kb0 = (int64_t)ch * CHUNK;
    const bool isA = kind < TMA;
    const int rbase = isA ? kind * 16 : nb0 + (kind - TMA) * 16;
    const int rlim = isA ? p.M - 1 : p.N - 1;
    const uint8_t *src = isA ? p.a : p.b;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = min(rbase + r, rlim);          // rows past the edge re-read the last row
      const uint8_t *s = src + (int64_t)row * p.Kb + kb0 + ((lane ^ r) << 4);
      if (isA) dec::dma16(s, dst + r * CHUNK);
      else dec::dma16_nt(s, dst + r * CHUNK);
    }
    if constexpr (Cfg::MX) {
      // 16 rows x 64 E8M0 bytes (4 superblocks x 16): lane -> row r =
      // lane/4, superblock (lane - r/4) % 4, so superblock b of row r sits
      // in 16-byte slot (b + r/4) % 4 of the row (mx_scale_word)
      const int row = min(rbase + (lane >> 2), rlim);
      const uint8_t *sc = static_cast<const uint8_t *>(isA ? p.sa : p.sb);
      dec::dma16(sc + row * sld + kb0 / 16 + ((((lane & 3) - (lane >> 4)) & 3) << 4),
                 dst + 16 * CHUNK);
    } else if constexpr (Cfg::GCOL) {
      if (isA) {
        // sa[row][8 groups of the chunk], as the block form (twice)
        const int row = min(rbase + ((lane >> 1) & 15), rlim);
        const float *sc = static_cast<const float *>(p.sa) + (int64_t)row * nkg + ch * 8 + ((lane & 1) << 2);
        dec::dma16(sc, dst + 16 * CHUNK);
        dec::dma16(sc, dst + 16 * CHUNK);
      } else {
        // sb[group][column] of the tile's 16 columns and the chunk's 8
        // groups, stored [group][column]: lane -> column lane % 16, group
        // 4d + lane / 16 (columns past the last clamped)
        const int col = min(rbase + (lane & 15), rlim);
#pragma unroll
        for (int d = 0; d < 2; ++d)
          dec::dma4(static_cast<const float *>(p.sb) + (int64_t)(ch * 8 + 4 * d + (lane >> 4)) * p.N + col,
                    dst + 16 * CHUNK + d * 256);
      }
    } else if constexpr (Cfg::BLOCK) {
      // activation tile: sa[row][8 groups of the chunk], 32 bytes per row
      // (lanes 32..63 repeat lanes 0..31); W tile: sb[n/128][8 groups]
      const float *sc;
      if (isA) {
        const int row = min(rbase + ((lane >> 1) & 15), rlim);
        sc = static_cast<const float *>(p.sa) + (int64_t)row * nkg;
      } else {
        const int sbrow = min(nb0, p.N - 1) / 128;   // both W tiles lie in one 128-row block
        sc = static_cast<const float *>(p.sb) + (int64_t)sbrow * nkg;
      }
      dec::dma16(sc + ch * 8 + ((lane & 1) << 2), dst + 16 * CHUNK);
    }
  };

  DecodeRegs<Cfg> st;
#pragma unroll
  for (int t = 0; t < TN; ++t)
#pragma unroll
    for (int a = 0; a < TMA; ++a) st.acc[t][a] = (v4f){0.f, 0.f, 0.f, 0.f};

  auto chunk16 = [&](const uint8_t *base, int c) {      // row r16's logical chunk c
    return *reinterpret_cast<const v4i *>(base + r16 * CHUNK + ((c ^ r16) << 4));
  };
  // MXFP4: the E8M0 word of lane group g in superblock b of row r16.  The
  // rotation by r16/4 puts the 64 lanes of one read on 64 distinct banks
  // (rows 64 bytes apart would otherwise put rows r, r+4, r+8, r+12 on one).
  auto mx_scale_word = [&](const uint8_t *aux, int b) {
    return *reinterpret_cast<const int *>(aux + r16 * 64 + (((b + (r16 >> 2)) & 3) << 4) + g * 4);
  };

  // consume item of kind KIND from `base`
  auto consume = [&](auto kind_tag, const uint8_t *base) {
    constexpr int KIND = decltype(kind_tag)::value;
    const uint8_t *aux = base + 16 * CHUNK;
    if constexpr (KIND < TMA) {
      if constexpr (Cfg::MX) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
#pragma unroll
          for (int j = 0; j < 4; ++j) st.ad[KIND][b][j] = chunk16(base, b * 16 + 4 * g + j);
          st.as[KIND][b] = mx_scale_word(aux, b);
        }
      } else {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const v4i lo = chunk16(base, s * 8 + g), hi = chunk16(base, s * 8 + g + 4);
          st.af[KIND][s] = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
        if constexpr (Cfg::BLOCK) {
          const float *sa = reinterpret_cast<const float *>(aux);   // [16 rows][8 groups]
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const v4f q0 = *reinterpret_cast<const v4f *>(sa + (4 * g + i) * 8);
            const v4f q1 = *reinterpret_cast<const v4f *>(sa + (4 * g + i) * 8 + 4);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
              st.sa[KIND][s][i] = q0[s];
              st.sa[KIND][s + 4][i] = q1[s];
            }
          }
        }
      }
    } else {
      constexpr int T = KIND - TMA;
      if constexpr (Cfg::MX) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int wsv = mx_scale_word(aux, b);
          v4i wd[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) wd[j] = chunk16(base, b * 16 + 4 * g + j);
#pragma unroll
          for (int a = 0; a < TMA; ++a) {
            st.acc[T][a] = mfma_mx<0>(st.ad[a][b][0], wd[0], st.acc[T][a], st.as[a][b], wsv);
            st.acc[T][a] = mfma_mx<1>(st.ad[a][b][1], wd[1], st.acc[T][a], st.as[a][b], wsv);
            st.acc[T][a] = mfma_mx<2>(st.ad[a][b][2], wd[2], st.acc[T][a], st.as[a][b], wsv);
            st.acc[T][a] = mfma_mx<3>(st.ad[a][b][3], wd[3], st.acc[T][a], st.as[a][b], wsv);
          }
        }
      } else {
        v4f sb0, sb1;
        float sbc[8];                  // GCOL: this lane's column scale per group
        if constexpr (Cfg::GCOL) {
#pragma unroll
          for (int s = 0; s < 8; ++s) sbc[s] = reinterpret_cast<const float *>(aux)[s * 16 + r16];
        } else if constexpr (Cfg::BLOCK) {
          sb0 = *reinterpret_cast<const v4f *>(aux);
          sb1 = *reinterpret_cast<const v4f *>(aux + 16);
        }
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const v4i lo = chunk16(base, s * 8 + g), hi = chunk16(base, s * 8 + g + 4);
          const v8i wf = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
          for (int a = 0; a < TMA; ++a) {
            if constexpr (Cfg::BLOCK) {
              const v4f zero = {0.f, 0.f, 0.f, 0.f};
              const v4f part = mfma_fp8(st.af[a][s], wf, zero);
              const float sbv = Cfg::GCOL ? sbc[s] : (s < 4 ? sb0[s & 3] : sb1[s & 3]);
              st.acc[T][a] = part * (st.sa[a][s] * sbv) + st.acc[T][a];
            } else if constexpr (Cfg::MODE == MODE_BF16) {
              st.acc[T][a] = mfma_bf16(st.af[a][s], wf, st.acc[T][a]);
            } else {
              st.acc[T][a] = mfma_fp8(st.af[a][s], wf, st.acc[T][a]);
            }
          }
        }
      }
    }
  };

  if (nitems > 0) issue(0);
  if (nitems > 1) issue(1);
  for (int base_it = 0; base_it < nitems; base_it += P) {
    // the P items of one chunk; item it = base_it + k sits in region it % 2
    auto step = [&](auto kind_tag) {
      constexpr int K = decltype(kind_tag)::value;
      const int it = base_it + K;
      // item it has landed once at most the one item issued after it is outstanding
      if (it + 1 < nitems) dec::wait_vm<DPI>();
      else dec::wait_vm<0>();
      const uint8_t *base = region[wave][it & 1];
      consume(kind_tag, base);
      dec::wait_lds();                 // region free: every LDS read of it has returned
      if (it + 2 < nitems) issue(it + 2);
    };
    dec::static_for<0, P>(step);
  }

  // ---- sum the waves' partial tiles and write the 16*TN columns
#pragma unroll
  for (int t = 0; t < TN; ++t)
#pragma unroll
    for (int a = 0; a < TMA; ++a) *reinterpret_cast<v4f *>(red[wave][t][a][lane]) = st.acc[t][a];
  __syncthreads();
  float s1 = 1.f, s2 = 1.f;
  if constexpr (Cfg::MODE == MODE_FP8_TENSOR) {
    s1 = *p.ga;
    s2 = *p.gb;
  }
  for (int o = threadIdx.x; o < TN * TMA * 256; o += Cfg::NT) {
    // output o: W tile t, activation tile a, lane ln, register i ->
    // row 16a + 4*(ln/16) + i, col nb0 + 16t + ln%16
    const int t = o / (TMA * 256), a = (o >> 8) % TMA, ln = (o >> 2) & 63, i = o & 3;
    const int row = a * 16 + 4 * (ln >> 4) + i, col = nb0 + t * 16 + (ln & 15);
    if (row >= p.M || col >= p.N) continue;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) v += red[w][t][a][ln][i];
    if constexpr (Cfg::MODE == MODE_FP8_TENSOR) v = (v * s1) * s2;
    if (p.out_f32) static_cast<float *>(p.c)[(int64_t)row * p.ldc + col] = v;
    else static_cast<uint16_t *>(p.c)[(int64_t)row * p.ldc + col] = f32_to_bf16(v);
  }
}

// ------------------------------------------------------- NVFP4 GEMV (M <= 4)
// 32 E2M1 codes (16 bytes) with their two E4M3 block scales (low byte: the
// first 16 codes) as 16 pairs of fp16 (exact: at most 5 significant bits).
DSL_DEV void nv_dequant32(const v4i &q, uint32_t sc2, v2h (&out)[16]) {
  const _Float16 s0 = e4m3_to_f16(sc2 & 0xFF), s1 = e4m3_to_f16((sc2 >> 8) & 0xFF);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const v8h h = fp4x8_to_f16((uint32_t)q[w], w < 2 ? s0 : s1);
#pragma unroll
    for (int e = 0; e < 4; ++e) out[4 * w + e] = (v2h){h[2 * e], h[2 * e + 1]};
  }
}

// acc += sum over the 32 elements of a[e] * (E2M1 code e x its block scale):
// per 16-element block, the dot products of the raw codes (converted to fp16
// with unit scale) accumulate in fp32 and the block scale, decoded exactly
// by the hardware OCP E4M3 -> f32 conversion, applies once.
template <int B>
DSL_DEV float nv_dot16(const v2h (&a)[16], const v4i &q, uint32_t sc2, float acc) {
  float part = 0.f;
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    const uint32_t word = (uint32_t)q[2 * B + w];
    const v2h *ap = &a[8 * B + 4 * w];
    part = __builtin_amdgcn_fdot2(ap[0], __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(word, 1.0f, 0), part, false);
    part = __builtin_amdgcn_fdot2(ap[1], __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(word, 1.0f, 1), part, false);
    part = __builtin_amdgcn_fdot2(ap[2], __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(word, 1.0f, 2), part, false);
    part = __builtin_amdgcn_fdot2(ap[3], __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(word, 1.0f, 3), part, false);
  }
  return __builtin_fmaf(__builtin_amdgcn_cvt_f32_fp8((int)sc2, B), part, acc);
}
DSL_DEV float nv_dot32(const v2h (&a)[16], const v4i &q, uint32_t sc2, float acc) {
  return nv_dot16<1>(a, q, sc2, nv_dot16<0>(a, q, sc2, acc));
}

DSL_DEV float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int MM, int NCH, int RPW>
__global__ __launch_bounds__(256) void gemv_nvfp4_kernel(const GemmArgs p) {
  constexpr int SROW = NCH * 128;                 // E4M3 scale bytes per row
  constexpr int WSB = RPW * SROW;                 // a wave's W scale bytes (contiguous rows)
  constexpr int WSD = (WSB + 1023) / 1024;        // its 1 KB scale DMAs
  constexpr int AD = MM * NCH;                    // activation data DMAs (1 KB each)
  constexpr int ASD = (MM * SROW + 1023) / 1024;  // activation scale DMAs
  __shared__ __align__(16) uint8_t a_lds[MM][NCH * 1024];
  __shared__ __align__(16) uint8_t as_lds[ASD * 1024];
  __shared__ __align__(16) uint8_t ws_lds[4][WSD * 1024];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int n0 = (blockIdx.x * 4 + wv) * RPW;
  const bool live = n0 < p.N;
  const int64_t sbytes = (int64_t)p.N * SROW;     // size of the W scale matrix

  // wave 0: the activations (data and scales) for the whole workgroup
  if (wv == 0) {
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      const int row = min(m, p.M - 1);
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        dec::dma16(p.a + (int64_t)row * p.Kb + c * 1024 + lane * 16,
                   dec::lds_addr(&a_lds[m][c * 1024]));
    }
#pragma unroll
    for (int j = 0; j < ASD; ++j) {
      // activation scale rows are contiguous; pieces past them re-read the last 16 bytes
      const int off = min(j * 1024 + lane * 16, p.M * SROW - 16);
      dec::dma16(static_cast<const uint8_t *>(p.sa) + off, dec::lds_addr(&as_lds[j * 1024]));
    }
  }
  // this wave's W scales (RPW contiguous rows), then its W rows into registers
  v4i wq[RPW][NCH];
  if (live) {
#pragma unroll
    for (int j = 0; j < WSD; ++j) {
      const int64_t off = min((int64_t)n0 * SROW + j * 1024 + lane * 16, sbytes - 16);
      dec::dma16(static_cast<const uint8_t *>(p.sb) + off, dec::lds_addr(&ws_lds[wv][j * 1024]));
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const int row = min(n0 + r, p.N - 1);
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        wq[r][c] = __builtin_nontemporal_load(
            reinterpret_cast<const v4i *>(p.b + (int64_t)row * p.Kb + c * 1024 + lane * 16));
    }
  }
  // the direct-to-LDS loads were issued before the W rows: they have landed
  // once at most the RPW*NCH row loads are outstanding
  if (live) dec::wait_vm<RPW * NCH>();
  else dec::wait_vm<0>();
  __syncthreads();
  if (!live) return;
  v2h a[MM][NCH][16];
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const v4i q = *reinterpret_cast<const v4i *>(&a_lds[m][c * 1024 + lane * 16]);
      const uint32_t s2 = *reinterpret_cast<const uint16_t *>(&as_lds[m * SROW + c * 128 + lane * 2]);
      nv_dequant32(q, s2, a[m][c]);
    }
  uint32_t ws[RPW][NCH];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      ws[r][c] = *reinterpret_cast<const uint16_t *>(&ws_lds[wv][r * SROW + c * 128 + lane * 2]);
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    float acc[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[m] = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int m = 0; m < MM; ++m) acc[m] = nv_dot32(a[m][c], wq[r][c], ws[r][c], acc[m]);
    const int col = n0 + r;
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      float v = wave_sum(acc[m]);
      if (lane == m && m < p.M && col < p.N) {
        v = (v * (*p.ga)) * (*p.gb);
        if (p.out_f32) static_cast<float *>(p.c)[(int64_t)m * p.ldc + col] = v;
        else static_cast<uint16_t *>(p.c)[(int64_t)m * p.ldc + col] = f32_to_bf16(v);
      }
    }
  }
}

template <int MM, int NCH>
static hipError_t launch_gemv_nv(const GemmArgs &p, hipStream_t st) {
  if constexpr (MM * NCH > 8) {
    return hipErrorInvalidValue;          // excluded by decode_supported (register budget)
  } else {
    // W rows per wave (measured at N=14336, K=4096): one activation row
    // wants more, smaller waves (RPW 2: 9.3 us against 9.7 with 4; K=16384:
    // 10.7 against 12.0), four rows want fewer, longer ones (RPW 8: 22.5
    // against 25.2), as long as the W and activation registers fit
    constexpr int RPW = MM == 1 ? 2 : ((MM * 16 + 32) * NCH <= 192 ? 8 : 4);
    const int waves = (p.N + RPW - 1) / RPW;
    gemv_nvfp4_kernel<MM, NCH, RPW><<<(waves + 3) / 4, 256, 0, st>>>(p);
    return hipGetLastError();
  }
}

template <int MM>
static hipError_t launch_gemv_nv_m(const GemmArgs &p, hipStream_t st) {
  switch (p.Kb / 1024) {
    case 1: return launch_gemv_nv<MM, 1>(p, st);
    case 2: return launch_gemv_nv<MM, 2>(p, st);
    case 4: return launch_gemv_nv<MM, 4>(p, st);
    default: return launch_gemv_nv<MM, 8>(p, st);
  }
}

template <int MODE, int TMA>
static hipError_t launch_decode_tma(const GemmArgs &p, hipStream_t st) {
  using Cfg = DecodeCfg<MODE, TMA>;
  const int grid = (p.N + 16 * Cfg::TN - 1) / (16 * Cfg::TN);
  gemm_decode_kernel<Cfg><<<grid, Cfg::NT, 0, st>>>(p);
  return hipGetLastError();
}

template <int MODE>
static hipError_t launch_decode_mode(const GemmArgs &p, hipStream_t st) {
  if (p.M <= 16) return launch_decode_tma<MODE, 1>(p, st);
  return launch_decode_tma<MODE, 2>(p, st);
}

bool decode_supported(int mode, int M, int K, int Kb, bool scales4, bool scales16) {
  if (M < 1 || Kb % 1024 != 0) return false;
  if (mode == MODE_NVFP4) {
    // GEMV: activations stay in registers for all of K (M * chunks <= 8);
    // scale rows move by 16-byte direct-to-LDS loads
    const int nch = Kb / 1024;
    return scales16 && M <= 4 && (nch == 1 || nch == 2 || nch == 4 || nch == 8) && M * nch <= 8;
  }
  if (M > 32) return false;
  if (mode == MODE_FP8_TENSOR || mode == MODE_BF16) return true;
  // block scales and E8M0 rows move by 16-byte direct loads
  if (mode_grouped_k(mode)) return scales16 && K % 512 == 0;
  if (mode == MODE_MXFP4) return scales16 && K % 512 == 0;
  return false;
}

hipError_t launch_gemm_decode(int mode, const GemmArgs &p, hipStream_t st) {
  switch (mode) {
    case MODE_FP8_TENSOR: return launch_decode_mode<MODE_FP8_TENSOR>(p, st);
    case MODE_FP8_BLOCK: return launch_decode_mode<MODE_FP8_BLOCK>(p, st);
    case MODE_FP8_GCOL: return launch_decode_mode<MODE_FP8_GCOL>(p, st);
    case MODE_MXFP4: return launch_decode_mode<MODE_MXFP4>(p, st);
    case MODE_BF16: return launch_decode_mode<MODE_BF16>(p, st);
    case MODE_NVFP4:
      switch (p.M) {
        case 1: return launch_gemv_nv_m<1>(p, st);
        case 2: return launch_gemv_nv_m<2>(p, st);
        case 3: return launch_gemv_nv_m<3>(p, st);
        default: return launch_gemv_nv_m<4>(p, st);
      }
    default: return hipErrorInvalidValue;
  }
}

}  // namespace dsl
