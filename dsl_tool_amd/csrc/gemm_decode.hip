// Skinny-M ("decode") quantized GEMM for gfx950: C[M,N] = A[M,K] . W[N,K]^T
// with M <= 32, bound by streaming W from HBM.
//
// One workgroup owns 16 rows of W (one MFMA tile of output columns) over
// the whole of K; its NW waves split K into contiguous ranges.  Each wave
// copies its 16 rows x K-range slab of W into a private LDS region with
// direct-to-LDS loads (one instruction = one row's next 1 KB, i.e. eight
// whole 128-byte lines, so every line is requested once and the copy runs
// at streaming efficiency), loads its activation fragments straight into
// registers (A is tiny and L2-resident), waits for its own loads only, and
// runs the MFMAs from LDS.  The waves' partial tiles are summed through LDS
// and written as bf16 / fp32 by the workgroup: one launch, no workspace, no
// atomics.  A K-range longer than one LDS chunk is processed chunk by chunk.
//
// MFMA: v_mfma_scale_f32_16x16x128_f8f6f4.  Lane l supplies row l%16 of its
// operand; lane group g = l/16 supplies a quarter of the step's K.  Output
// register i of lane l is C[4*g + i][l%16].
//   FP8 tensor / block: group g holds the 16-byte chunks g and 4+g of the
//     step's 128 K bytes (the same K order for A and W, so the sum is
//     unchanged; for block scales the step is exactly one 128-K scale group),
//     so each activation load instruction reads 64 contiguous bytes per row.
//   MXFP4: K is taken in 512-element superblocks of 4 steps; at step j of a
//     superblock group g holds the 32-element block 4g+j, so a lane's data
//     for the superblock is 64 contiguous bytes and its 4 E8M0 scale bytes
//     are one aligned u32 (opsel j picks the byte).  A and W use the same
//     permutation of K, which leaves every block paired with its own scale.
// LDS slab: row r's 16-byte chunk c lives in slot c ^ r (r < 16), so the 16
// lanes reading one logical chunk of the 16 rows hit 16 distinct bank groups.
#include "gemm_core.h"

#pragma clang diagnostic ignored "-Winline-asm"

#ifndef DSL_DECODE_TN
#define DSL_DECODE_TN 1
#endif

namespace dsl {

namespace dec {

DSL_DEV uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
// 16 bytes per lane from `src` into LDS at m0 + lane*16 (the s_nop covers
// the m0 -> LDS-DMA wait state the compiler cannot see inside the asm).
DSL_DEV void dma16(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src),
               "s"(lds)
               : "memory", "m0");
}

}  // namespace dec

template <int MODE_, int TMA_, int NW_, int TN_ = 1>
struct DecodeCfg {
  static constexpr int MODE = MODE_;
  static constexpr int TMA = TMA_;       // 16-row activation tiles (M <= 16*TMA)
  static constexpr int TN = TN_;         // 16-row W tiles per workgroup (and per wave)
  static constexpr int NW = NW_, NT = NW * 64;
  static constexpr bool MX = MODE == MODE_MXFP4;
  static constexpr int STEP_BYTES = MX ? 64 : 128;    // bytes of one W row per MFMA step
  static constexpr int CHUNK = 1024;                  // W bytes per row per LDS chunk
  static constexpr int CSTEPS = CHUNK / STEP_BYTES;   // MFMA steps per chunk
  static constexpr int SLAB = TN * (16 * CHUNK + (MX ? 16 * (CHUNK / 16) : 0));   // + E8M0
};

template <class Cfg>
__global__ __launch_bounds__(Cfg::NT) void gemm_decode_kernel(const GemmArgs p) {
  constexpr int TMA = Cfg::TMA, NW = Cfg::NW, CHUNK = Cfg::CHUNK, CSTEPS = Cfg::CSTEPS;
  constexpr int TN = Cfg::TN;
  constexpr int TSLAB = Cfg::SLAB / TN;  // one 16-row tile's slab
  __shared__ __align__(16) uint8_t slab[NW][Cfg::SLAB];
  __shared__ __align__(16) float red[NW][TN][TMA][64][4];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int nb0 = blockIdx.x * 16 * TN;

  // contiguous K-range of this wave, in whole chunks
  const int nchunks = p.Kb / CHUNK;
  const int c_begin = (int)((int64_t)nchunks * wave / NW);
  const int c_end = (int)((int64_t)nchunks * (wave + 1) / NW);

  uint8_t *ws = slab[wave];
  const uint32_t ws_lds = dec::lds_addr(ws);
  const int64_t sld = p.K / 32;          // E8M0 bytes per row (MX)

  v4f acc_all[TN][TMA];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
#pragma unroll
    for (int t = 0; t < TMA; ++t) acc_all[tn][t] = (v4f){0.f, 0.f, 0.f, 0.f};

  for (int ch = c_begin; ch < c_end; ++ch) {
    const int64_t kb0 = (int64_t)ch * CHUNK;           // first W byte of the chunk
    // ---- W slabs: TN x 16 rows x CHUNK bytes (+ MX scales), swizzled
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int nrow = min(nb0 + tn * 16 + r, p.N - 1);   // rows past N re-read the last row
        const int c = lane ^ r;                          // logical chunk stored in slot `lane`
        dec::dma16(p.b + (int64_t)nrow * p.Kb + kb0 + c * 16, ws_lds + tn * TSLAB + r * CHUNK);
      }
      if constexpr (Cfg::MX) {
        // CHUNK*2 elements / 32 = 64 scale bytes per row: lane -> row lane/4, 16 bytes lane%4
        const int nrow = min(nb0 + tn * 16 + (lane >> 2), p.N - 1);
        dec::dma16(static_cast<const uint8_t *>(p.sb) + (int64_t)nrow * sld + kb0 / 16 +
                       (lane & 3) * 16,
                   ws_lds + tn * TSLAB + 16 * CHUNK);
      }
    }

    // ---- activation fragments for the chunk, straight into registers
    if constexpr (!Cfg::MX) {
      v8i af[CSTEPS][TMA];
#pragma unroll
      for (int s = 0; s < CSTEPS; ++s)
#pragma unroll
        for (int t = 0; t < TMA; ++t) {
          const uint8_t *ap = p.a + (int64_t)min(t * 16 + r16, p.M - 1) * p.Kb + kb0 + s * 128 +
                              g * 16;
          const v4i lo = reinterpret_cast<const v4i *>(ap)[0];
          const v4i hi = reinterpret_cast<const v4i *>(ap)[4];
          af[s][t] = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
      float sbv[TN][CSTEPS];
      v4f sa4[CSTEPS][TMA];
      if constexpr (Cfg::MODE == MODE_FP8_BLOCK) {
        const int nkg = p.K / 128, kg0 = (int)(kb0 / 128);
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
          const int sbrow = min(nb0 + tn * 16, p.N - 1) / 128;
          const float *sbp = static_cast<const float *>(p.sb) + (int64_t)sbrow * nkg + kg0;
#pragma unroll
          for (int s = 0; s < CSTEPS; ++s) sbv[tn][s] = sbp[s];
        }
        const float *sa = static_cast<const float *>(p.sa);
#pragma unroll
        for (int t = 0; t < TMA; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float *rp = sa + (int64_t)min(t * 16 + 4 * g + i, p.M - 1) * nkg + kg0;
#pragma unroll
            for (int s = 0; s < CSTEPS; ++s) sa4[s][t][i] = rp[s];
          }
      }
      __builtin_amdgcn_s_waitcnt(0);                   // this wave's DMA and loads
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const uint8_t *wt = ws + tn * TSLAB;
        v4f (&acc)[TMA] = acc_all[tn];
#pragma unroll
        for (int s = 0; s < CSTEPS; ++s) {
          const int c0 = s * 8 + g;
          const v4i lo = *reinterpret_cast<const v4i *>(wt + r16 * CHUNK + ((c0 ^ r16) << 4));
          const v4i hi = *reinterpret_cast<const v4i *>(wt + r16 * CHUNK + (((c0 + 4) ^ r16) << 4));
          const v8i wf = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
          for (int t = 0; t < TMA; ++t) {
            if constexpr (Cfg::MODE == MODE_FP8_TENSOR) {
              acc[t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[s][t], wf, acc[t], 0,
                                                                        0, 0, 0, 0, 0);
            } else {
              const v4f zero = {0.f, 0.f, 0.f, 0.f};
              const v4f part = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[s][t], wf,
                                                                                zero, 0, 0, 0,
                                                                                0, 0, 0);
              acc[t] = part * (sa4[s][t] * sbv[tn][s]) + acc[t];
            }
          }
        }
      }
    } else {
      constexpr int NSB = CSTEPS / 4;                  // superblocks per chunk
      v4i ad[NSB][TMA][4];
      int as[NSB][TMA];
#pragma unroll
      for (int b = 0; b < NSB; ++b)
#pragma unroll
        for (int t = 0; t < TMA; ++t) {
          const int arow = min(t * 16 + r16, p.M - 1);
          const v4i *ap = reinterpret_cast<const v4i *>(p.a + (int64_t)arow * p.Kb + kb0 +
                                                        b * 256 + g * 64);
#pragma unroll
          for (int j = 0; j < 4; ++j) ad[b][t][j] = ap[j];
          as[b][t] = *reinterpret_cast<const int *>(static_cast<const uint8_t *>(p.sa) +
                                                    (int64_t)arow * sld + kb0 / 16 + b * 16 + g * 4);
        }
      __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const uint8_t *wt = ws + tn * TSLAB;
        const uint8_t *wsc = wt + 16 * CHUNK;
        v4f (&acc)[TMA] = acc_all[tn];
#pragma unroll
        for (int b = 0; b < NSB; ++b) {
          const int wsv = *reinterpret_cast<const int *>(wsc + r16 * 64 + b * 16 + g * 4);
          v4i wd[4];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            wd[j] = *reinterpret_cast<const v4i *>(wt + r16 * CHUNK +
                                                   (((b * 16 + 4 * g + j) ^ r16) << 4));
#pragma unroll
          for (int t = 0; t < TMA; ++t) {
            acc[t] = mfma_mx<0>(ad[b][t][0], wd[0], acc[t], as[b][t], wsv);
            acc[t] = mfma_mx<1>(ad[b][t][1], wd[1], acc[t], as[b][t], wsv);
            acc[t] = mfma_mx<2>(ad[b][t][2], wd[2], acc[t], as[b][t], wsv);
            acc[t] = mfma_mx<3>(ad[b][t][3], wd[3], acc[t], as[b][t], wsv);
          }
        }
      }
    }
  }

  // ---- sum the waves' partial tiles and write the 16*TN columns
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
#pragma unroll
    for (int t = 0; t < TMA; ++t) *reinterpret_cast<v4f *>(red[wave][tn][t][lane]) = acc_all[tn][t];
  __syncthreads();
  float s1 = 1.f, s2 = 1.f;
  if constexpr (Cfg::MODE == MODE_FP8_TENSOR) {
    s1 = *p.ga;
    s2 = *p.gb;
  }
  for (int o = threadIdx.x; o < TN * TMA * 256; o += Cfg::NT) {
    // output o: W tile tn, A tile t, lane ln, register i ->
    // row 16t + 4*(ln/16) + i, col 16tn + ln%16
    const int tn = o / (TMA * 256), t = (o >> 8) % TMA, ln = (o >> 2) & 63, i = o & 3;
    const int row = t * 16 + 4 * (ln >> 4) + i, col = nb0 + tn * 16 + (ln & 15);
    if (row >= p.M || col >= p.N) continue;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) v += red[w][tn][t][ln][i];
    if constexpr (Cfg::MODE == MODE_FP8_TENSOR) v = (v * s1) * s2;
    if (p.out_f32) static_cast<float *>(p.c)[(int64_t)row * p.ldc + col] = v;
    else static_cast<uint16_t *>(p.c)[(int64_t)row * p.ldc + col] = f32_to_bf16(v);
  }
}

template <int MODE, int TMA>
static hipError_t launch_decode_tma(const GemmArgs &p, hipStream_t st) {
  using Cfg = DecodeCfg<MODE, TMA, 4, DSL_DECODE_TN>;
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
  if (M > 32 || M < 1 || Kb % 1024 != 0) return false;
  if (mode == MODE_FP8_TENSOR) return true;
  if (mode == MODE_FP8_BLOCK) return scales4;
  if (mode == MODE_MXFP4) return scales16 && (K / 32) % 16 == 0;
  return false;
}

hipError_t launch_gemm_decode(int mode, const GemmArgs &p, hipStream_t st) {
  switch (mode) {
    case MODE_FP8_TENSOR: return launch_decode_mode<MODE_FP8_TENSOR>(p, st);
    case MODE_FP8_BLOCK: return launch_decode_mode<MODE_FP8_BLOCK>(p, st);
    default: return launch_decode_mode<MODE_MXFP4>(p, st);
  }
}

}  // namespace dsl
