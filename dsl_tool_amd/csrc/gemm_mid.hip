// Mid-M quantized GEMMs for gfx950 (32 < M <= 256; BASELINE config 1 is
// M=128, N=K=4096): C[M,N] = A[M,K] . W[N,K]^T, one launch, no workspace,
// deterministic.  FP8 per-tensor, FP8 1x128/128x128 block, MXFP4, bf16.
//
// At these shapes the work per byte of W is small (M flops per W byte) and
// the output has too few 256x256 tiles to fill 256 CUs, so the kernel is
// laid out for streaming W once while every CU works:
//   * a workgroup owns BM = 64 activation rows (four 16-row tiles) and
//     BN = 16*TN W rows (TN = 2, or 1 when that leaves fewer than 256
//     workgroups) over the whole of K.  Per CU that moves (64 + BN) rows of
//     K bytes through LDS, the least for a one-pass split of M x N over the
//     CUs (the L2 -> CU copy rate, ~64 B/clk per CU, is what bounds it);
//   * its four waves split K into contiguous ranges of 512-byte chunks.  A
//     wave streams, for each of its chunks, the TN W tiles and then the four
//     activation tiles (16 rows x 512 B each, eight direct-to-LDS loads of
//     two rows each) through four private LDS regions, three items in flight
//     behind the one being consumed.  W tiles go into registers; each
//     activation tile is multiplied against them as it is read.  No barrier
//     until the final reduction, so a wave waits for its own loads only;
//   * the waves' partial tiles are summed through LDS in a fixed order (wave
//     0 + 1 + 2 + 3), then scaled and stored: no atomics, no split-K fix-up,
//     the same bytes on every run;
//   * the M blocks of one W slice are launched 8 apart, i.e. on the same XCD
//     at about the same time, so the second reader of a W slice finds it in
//     that XCD's L2; W loads carry the non-temporal hint, the activations
//     (re-read by every workgroup, 64 x K bytes) stay cached.
//
// MFMA: v_mfma_scale_f32_16x16x128_f8f6f4 (bf16: two v_mfma_f32_16x16x32_bf16),
// activation tile in the first operand: output register i of lane l is
// C[4*(l/16) + i][l%16] with rows from the activation tile and columns from
// the W tile.  K order inside a chunk as in the skinny-M kernel
// (gemm_decode.hip): FP8 / bf16 lane group g holds 16-byte chunks g and g+4
// of each 128-byte step; MXFP4 takes 512-element superblocks whose step j
// gives lane group g the 32-element block 4g+j (one u32 of 4 E8M0 bytes per
// lane and superblock, op_sel j picks the byte).  A and W share the order.
// Block scales: each 128-byte step is one 128-K group, folded as
// acc += part * (sa[m][grp] * sb[n/128][grp]) (cuda/gemm/fp8_gemm.cu:84-97).
// LDS rows are 512 bytes; row r's 16-byte chunk c sits in slot c ^ r (r < 16),
// so the 16 lanes that read one logical chunk of 16 rows hit distinct banks.
#include "stream_core.h"

namespace dsl {

template <int MODE_, int TN_>
struct MidCfg {
  static constexpr int MODE = MODE_;
  static constexpr int TMA = 4;                      // 16-row activation tiles
  static constexpr int TN = TN_;                     // 16-row W tiles
  static constexpr int BM = 16 * TMA, BN = 16 * TN;
  static constexpr int NW = 4, NT = NW * 64;         // waves split K
  static constexpr bool MX = MODE == MODE_MXFP4;
  static constexpr bool BLOCK = MODE == MODE_FP8_BLOCK;
  static constexpr int CHUNK = 512;                  // bytes of one row per item
  static constexpr int STEPS = CHUNK / 128;          // 128-byte MFMA steps per item
  static constexpr int SBK = CHUNK / 256;            // MXFP4 512-element superblocks per item
  static constexpr int AUX = (MX || BLOCK) ? 1024 : 0;   // scale DMA target per item
  static constexpr int DPI = 8 + (AUX ? 1 : 0);      // DMA instructions per item
  static constexpr int REGION = 16 * CHUNK + AUX;
  static constexpr int NR = 4;                       // regions per wave: NR-1 items in flight
  static constexpr int P = TN + TMA;                 // items per chunk: W tiles, then A tiles
  static constexpr int RING = NW * NR * REGION;
  static constexpr int RED = NW * TN * TMA * 64 * 16;   // partial tiles of the four waves
  static constexpr int LDS = RING > RED ? RING : RED;
  static_assert(LDS <= 160 * 1024, "LDS budget");
  static_assert(NR == 4 && (NR - 1) * DPI < 64, "the main loop's waits are written for 4 regions");
};

template <class Cfg>
struct MidRegs {
  v8i wf[Cfg::TN][Cfg::STEPS];      // FP8 / bf16 W fragments of the current chunk
  v4i wq[Cfg::TN][Cfg::SBK][4];     // MXFP4 W fragments (16 bytes per step)
  int ws[Cfg::TN][Cfg::SBK];        // MXFP4 W E8M0 words
  v4f sb;                           // FP8 block: weight scales of the chunk's 4 groups
  v4f acc[Cfg::TN][Cfg::TMA];
};

template <class Cfg>
__global__ __launch_bounds__(Cfg::NT) void gemm_mid_kernel(const GemmArgs p) {
  constexpr int TMA = Cfg::TMA, TN = Cfg::TN, NW = Cfg::NW, P = Cfg::P, DPI = Cfg::DPI;
  constexpr int NR = Cfg::NR, CHUNK = Cfg::CHUNK;
  __shared__ __align__(16) uint8_t lds[Cfg::LDS];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  // workgroup -> (M block, N block); the M blocks of one W slice are 8 apart
  const int nmb = (p.M + Cfg::BM - 1) / Cfg::BM;
  const int nnb = (p.N + Cfg::BN - 1) / Cfg::BN;
  const int local = blockIdx.x >> 3;
  const int mblk = local % nmb, nblk = (local / nmb) * 8 + (blockIdx.x & 7);
  if (nblk >= nnb) return;                   // whole workgroup: no barrier reached
  const int m0 = mblk * Cfg::BM, n0 = nblk * Cfg::BN;
  const int nchunks = p.Kb / CHUNK;
  const int c_begin = nchunks * wave / NW, c_end = nchunks * (wave + 1) / NW;
  const int nitems = (c_end - c_begin) * P;
  uint8_t *my = lds + wave * NR * Cfg::REGION;
  const uint32_t R0 = dec::lds_addr(my);
  const int nkg = p.K / 128;                 // FP8 block: scale groups per row
  const int64_t sld = p.K / 32;              // MXFP4: E8M0 bytes per row

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
    const int half = lane >> 5, slot = lane & 31;
#pragma unroll
    for (int j = 0; j < 8; ++j) {              // rows 2j (lanes 0..31) and 2j+1
      const int r = 2 * j + half;
      const int row = min(rbase + r, rlim);    // rows past the edge re-read the last row
      const uint8_t *s = src + (int64_t)row * p.Kb + kb0 + ((slot ^ r) << 4);
      if (isW) dec::dma16_nt(s, dst + j * 1024);
      else dec::dma16(s, dst + j * 1024);
    }
    if constexpr (Cfg::MX) {
      // 16 rows x 32 E8M0 bytes: lane -> row (lane/2)%16, 16 bytes lane%2
      // (lanes 32..63 repeat lanes 0..31)
      const int row = min(rbase + ((lane >> 1) & 15), rlim);
      const uint8_t *sc = static_cast<const uint8_t *>(isW ? p.sb : p.sa);
      dec::dma16(sc + row * sld + kb0 / 16 + ((lane & 1) << 4), dst + 16 * CHUNK);
    } else if constexpr (Cfg::BLOCK) {
      // activation tile: sa[row][4 groups of the chunk], 16 bytes per row
      // (lanes 16..63 repeat lanes 0..15); W tile: sb[n0/128][4 groups]
      const float *sc = isW ? static_cast<const float *>(p.sb) + (int64_t)(n0 / 128) * nkg
                            : static_cast<const float *>(p.sa) +
                                  (int64_t)min(rbase + r16, rlim) * nkg;
      dec::dma16(sc + ch * 4, dst + 16 * CHUNK);
    }
  };

  MidRegs<Cfg> st;
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
          st.ws[KIND][b] = *reinterpret_cast<const int *>(aux + r16 * 32 + b * 16 + g * 4);
        }
      } else {
#pragma unroll
        for (int s = 0; s < Cfg::STEPS; ++s) {
          const v4i lo = chunk16(base, s * 8 + g), hi = chunk16(base, s * 8 + g + 4);
          st.wf[KIND][s] = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
        if constexpr (Cfg::BLOCK) st.sb = *reinterpret_cast<const v4f *>(aux);
      }
    } else {                                    // activation tile x the W tiles
      constexpr int A = KIND - TN;
      if constexpr (Cfg::MX) {
#pragma unroll
        for (int b = 0; b < Cfg::SBK; ++b) {
          const int asv = *reinterpret_cast<const int *>(aux + r16 * 32 + b * 16 + g * 4);
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
        v4f sa4[4];                             // FP8 block: rows 4g+i, the chunk's 4 groups
        if constexpr (Cfg::BLOCK) {
#pragma unroll
          for (int i = 0; i < 4; ++i) sa4[i] = *reinterpret_cast<const v4f *>(aux + (4 * g + i) * 16);
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
              const v4f sc = (v4f){sa4[0][s], sa4[1][s], sa4[2][s], sa4[3][s]} * st.sb[s];
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

#pragma unroll
  for (int i = 0; i < NR - 1; ++i)
    if (i < nitems) issue(i);
  for (int base_it = 0; base_it < nitems; base_it += P) {
    auto step = [&](auto kind_tag) {
      constexpr int K = decltype(kind_tag)::value;
      const int it = base_it + K;
      // the region of item it-1 is free (its reads returned): refill it
      if (it + NR - 1 < nitems) issue(it + NR - 1);
      // item it has landed once at most the items issued after it are outstanding
      const int after = nitems - 1 - it;
      if (after >= NR - 1) dec::wait_vm<(NR - 1) * DPI>();
      else if (after == 2) dec::wait_vm<2 * DPI>();
      else if (after == 1) dec::wait_vm<DPI>();
      else dec::wait_vm<0>();
      consume(kind_tag, my + (it % NR) * Cfg::REGION);
      dec::wait_lds();
    };
    dec::static_for<0, P>(step);
  }

  // ---- sum the waves' partial tiles (fixed order), scale, store
  __syncthreads();                              // every wave is done with its regions
  float *red = reinterpret_cast<float *>(lds);  // [NW][TN][TMA][64 lanes][4]
#pragma unroll
  for (int t = 0; t < TN; ++t)
#pragma unroll
    for (int a = 0; a < TMA; ++a)
      *reinterpret_cast<v4f *>(red + (((wave * TN + t) * TMA + a) * 64 + lane) * 4) = st.acc[t][a];
  __syncthreads();
  float s1 = 1.f, s2 = 1.f;
  if constexpr (Cfg::MODE == MODE_FP8_TENSOR) {
    s1 = *p.ga;
    s2 = *p.gb;
  }
  constexpr int CPT = Cfg::BM * Cfg::BN / Cfg::NT;   // consecutive columns per thread (8 / 4)
  constexpr int GPR = Cfg::BN / CPT;                 // threads per tile row
  const int lrow = threadIdx.x / GPR, lcol = (threadIdx.x % GPR) * CPT;
  const int row = m0 + lrow, col0 = n0 + lcol;
  if (row >= p.M) return;
  const int a = lrow >> 4, i = lrow & 3, lq = (lrow & 15) >> 2;
  float v[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int t = (lcol + c) >> 4, ln = 16 * lq + ((lcol + c) & 15);
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) s += red[(((w * TN + t) * TMA + a) * 64 + ln) * 4 + i];
    if constexpr (Cfg::MODE == MODE_FP8_TENSOR) s = (s * s1) * s2;
    v[c] = s;
  }
  if (p.out_f32) {
    float *dst = static_cast<float *>(p.c) + (int64_t)row * p.ldc + col0;
    if (col0 + CPT <= p.N && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
#pragma unroll
      for (int c = 0; c < CPT; c += 4)
        *reinterpret_cast<v4f *>(dst + c) = (v4f){v[c], v[c + 1], v[c + 2], v[c + 3]};
    } else {
      for (int c = 0; c < CPT && col0 + c < p.N; ++c) dst[c] = v[c];
    }
  } else {
    uint16_t *dst = static_cast<uint16_t *>(p.c) + (int64_t)row * p.ldc + col0;
    if (col0 + CPT <= p.N && (reinterpret_cast<uintptr_t>(dst) & (2 * CPT - 1)) == 0) {
      uint32_t w[CPT / 2];
#pragma unroll
      for (int c = 0; c < CPT; c += 2) w[c / 2] = pack_bf16x2(v[c], v[c + 1]);
      if constexpr (CPT == 8)
        *reinterpret_cast<uint4 *>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
      else
        *reinterpret_cast<uint2 *>(dst) = make_uint2(w[0], w[1]);
    } else {
      for (int c = 0; c < CPT && col0 + c < p.N; ++c) dst[c] = f32_to_bf16(v[c]);
    }
  }
}

template <int MODE, int TN>
static hipError_t launch_mid_tn(const GemmArgs &p, hipStream_t st) {
  using Cfg = MidCfg<MODE, TN>;
  const int nmb = (p.M + Cfg::BM - 1) / Cfg::BM;
  const int nnb = (p.N + Cfg::BN - 1) / Cfg::BN;
  const int grid = 8 * nmb * ((nnb + 7) / 8);
  gemm_mid_kernel<Cfg><<<grid, Cfg::NT, 0, st>>>(p);
  return hipGetLastError();
}

// W tiles per workgroup: two, unless that leaves fewer than 256 workgroups.
static int mid_tn(int M, int N) {
  const int nmb = (M + 63) / 64;
  return (int64_t)nmb * ((N + 31) / 32) >= 256 ? 2 : 1;
}

template <int MODE>
static hipError_t launch_mid_mode(const GemmArgs &p, hipStream_t st) {
  return mid_tn(p.M, p.N) == 2 ? launch_mid_tn<MODE, 2>(p, st) : launch_mid_tn<MODE, 1>(p, st);
}

bool mid_supported(int mode, int M, int N, int K, int Kb, bool scales16) {
  if (M <= 32 || M > 256 || N < 1 || Kb % 512 != 0) return false;
  if (mode == MODE_FP8_TENSOR || mode == MODE_BF16) return true;
  // block scales and E8M0 rows move by 16-byte direct loads
  if (mode == MODE_FP8_BLOCK || mode == MODE_MXFP4) return scales16;
  (void)K;
  return false;
}

hipError_t launch_gemm_mid(int mode, const GemmArgs &p, hipStream_t st) {
  switch (mode) {
    case MODE_FP8_TENSOR: return launch_mid_mode<MODE_FP8_TENSOR>(p, st);
    case MODE_FP8_BLOCK: return launch_mid_mode<MODE_FP8_BLOCK>(p, st);
    case MODE_MXFP4: return launch_mid_mode<MODE_MXFP4>(p, st);
    case MODE_BF16: return launch_mid_mode<MODE_BF16>(p, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace dsl
