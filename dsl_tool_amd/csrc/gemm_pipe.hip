// Dense pipelined GEMM kernels for gfx950 (FP8 per-tensor, FP8 block-scaled,
// MXFP4); the mainloop, DMA ring and LDS layout are described in pipe_core.h.
#include "pipe_core.h"

namespace dsl {

template <class Cfg>
__global__ __launch_bounds__(Cfg::NT) __attribute__((amdgpu_waves_per_eu(Cfg::OCC, Cfg::OCC)))
void gemm_pipe_kernel(const GemmArgs p) {
  __shared__ __align__(16) uint8_t smem[Cfg::LDS];
  const int nbm = (p.M + Cfg::BM - 1) / Cfg::BM, nbn = (p.N + Cfg::BN - 1) / Cfg::BN;
  int tmi, tni;
  tile_coords(blockIdx.x, nbm, nbn, tmi, tni);
  const int m0 = tmi * Cfg::BM, n0 = tni * Cfg::BN;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
  const int r32 = lane & 31, h = lane >> 5;
  v16f acc[Cfg::TM][Cfg::TN];
  pipe_mainloop<Cfg>(p, m0, n0, smem, wave, lane, acc);

  float s1 = 1.f, s2 = 1.f;
  constexpr bool GLOBAL = Cfg::MODE == MODE_FP8_TENSOR || Cfg::MODE == MODE_NVFP4;
  if constexpr (GLOBAL) {
    s1 = *p.ga;
    s2 = *p.gb;
  }
#pragma unroll
  for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::TN; ++j) {
      const int col = n0 + wn * Cfg::WN + j * 32 + r32;
      if (col >= p.N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * Cfg::WM + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (row >= p.M) continue;
        float v = acc[i][j][r];
        if constexpr (GLOBAL) v = (v * s1) * s2;
        if (p.out_f32) static_cast<float *>(p.c)[(int64_t)row * p.ldc + col] = v;
        else static_cast<uint16_t *>(p.c)[(int64_t)row * p.ldc + col] = f32_to_bf16(v);
      }
    }
}

// Block-scaled FP8 (1x128 activation groups, 128x128 weight blocks): one
// 16x16x128 MFMA per output tile per stage yields the group's partial sum,
// folded at once into the fp32 accumulator as acc += part * sa[m,g] * sb[n/128,g]
// (the group-partial form of cuda/gemm/fp8_gemm.cu:84-97).  Activation
// scales travel with the stage; the weight scale of the wave's 128-column
// block is one scalar load per stage.
template <class Cfg>
__global__ __launch_bounds__(Cfg::NT) __attribute__((amdgpu_waves_per_eu(Cfg::OCC, Cfg::OCC)))
void gemm_pipe_block_kernel(const GemmArgs p) {
  static_assert(Cfg::BLOCK && Cfg::WN <= 128 && 128 % Cfg::WN == 0, "block-scale tiling");
  constexpr int NS = Cfg::NS, D = Cfg::D, SKB = Cfg::SKB;
  constexpr int TM = Cfg::WM / 16, TN = Cfg::WN / 16;
  __shared__ __align__(16) uint8_t smem[Cfg::LDS];
  const int nbm = (p.M + Cfg::BM - 1) / Cfg::BM, nbn = (p.N + Cfg::BN - 1) / Cfg::BN;
  int tmi, tni;
  tile_coords(blockIdx.x, nbm, nbn, tmi, tni);
  const int m0 = tmi * Cfg::BM, n0 = tni * Cfg::BN;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lds0 = pipe::lds_addr(smem);
  pipe::Ring<Cfg> ring;
  ring.init(p, m0, n0, wave, lane);

  const int nks = p.Kb / SKB, nkg = p.K / 128;
  const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
  const int r16 = lane & 15, g = lane >> 4;
  int sbrow = (n0 + wn * Cfg::WN) / 128;
  const int sblim = (p.N + 127) / 128 - 1;
  sbrow = sbrow > sblim ? sblim : sbrow;
  const float *sbp = static_cast<const float *>(p.sb) + (int64_t)sbrow * nkg;

#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nks) ring.issue(s, lds0);

  v4f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};

  for (int ks = 0; ks < nks; ++ks) {
    const float sbv = sbp[ks];
    if (ks + NS - 2 < nks) pipe::wait_vmcnt<(NS - 2) * D>();
    else pipe::wait_vmcnt<0>();
    __syncthreads();
    if (ks + NS - 1 < nks) ring.issue(ks + NS - 1, lds0);
    const uint8_t *st = smem + (ks % NS) * Cfg::STAGE;
    const uint8_t *sA = st, *sB = st + Cfg::A_BYTES;
    const float *sSa = reinterpret_cast<const float *>(st + Cfg::A_BYTES + Cfg::B_BYTES);
    auto ld = [&](const uint8_t *base, int row) {
      const int s = pipe::swz<SKB>(row);
      const v4i lo = *reinterpret_cast<const v4i *>(base + row * SKB + (((2 * g) ^ s) << 4));
      const v4i hi = *reinterpret_cast<const v4i *>(base + row * SKB + (((2 * g + 1) ^ s) << 4));
      return (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    v8i bf[TN];
#pragma unroll
    for (int t = 0; t < TN; ++t) bf[t] = ld(sB, wn * Cfg::WN + t * 16 + r16);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int arow = wm * Cfg::WM + i * 16;
      const v8i af = ld(sA, arow + r16);
      const v4f s4 = *reinterpret_cast<const v4f *>(sSa + arow + 4 * g) * sbv;
      const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const v4f part = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af, bf[j], zero, 0, 0, 0,
                                                                          0, 0, 0);
        acc[i][j] = part * s4 + acc[i][j];
      }
    }
  }

#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + wn * Cfg::WN + j * 16 + r16;
      if (col >= p.N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * Cfg::WM + i * 16 + 4 * g + r;
        if (row >= p.M) continue;
        if (p.out_f32) static_cast<float *>(p.c)[(int64_t)row * p.ldc + col] = acc[i][j][r];
        else static_cast<uint16_t *>(p.c)[(int64_t)row * p.ldc + col] = f32_to_bf16(acc[i][j][r]);
      }
    }
}

template <class Cfg>
static hipError_t launch_pipe_cfg(const GemmArgs &p, hipStream_t st) {
  const int tiles = ((p.M + Cfg::BM - 1) / Cfg::BM) * ((p.N + Cfg::BN - 1) / Cfg::BN);
  if constexpr (Cfg::BLOCK) gemm_pipe_block_kernel<Cfg><<<tiles, Cfg::NT, 0, st>>>(p);
  else gemm_pipe_kernel<Cfg><<<tiles, Cfg::NT, 0, st>>>(p);
  return hipGetLastError();
}

// Dense FP8 (per-tensor) / MXFP4 GEMM through the LDS-DMA pipeline.
// Preconditions (checked by the caller): Kb % 128 == 0, mode FP8_TENSOR,
// FP8_BLOCK or MXFP4, ksplit == 1, 4-byte aligned scales.
hipError_t launch_gemm_pipe(int mode, const GemmArgs &p, int variant, hipStream_t st) {
  if (mode == MODE_FP8_BLOCK) {
    switch (variant) {
      case 0: return launch_pipe_cfg<PipeCfg<MODE_FP8_BLOCK, 256, 256, 2, 4, 2, 128>>(p, st);
      case 2: return launch_pipe_cfg<PipeCfg<MODE_FP8_BLOCK, 256, 256, 4, 2, 2, 128>>(p, st);
      default: return launch_pipe_cfg<PipeCfg<MODE_FP8_BLOCK, 128, 128, 2, 2, 2, 128, 2>>(p, st);
    }
  }
  if (mode == MODE_FP8_TENSOR) {
    switch (variant) {
      case 0: return launch_pipe_cfg<PipeCfg<MODE_FP8_TENSOR, 256, 256, 2, 4, 4, 64>>(p, st);
      case 2: return launch_pipe_cfg<PipeCfg<MODE_FP8_TENSOR, 256, 256, 2, 4, 2, 128>>(p, st);
      case 3: return launch_pipe_cfg<PipeCfg<MODE_FP8_TENSOR, 256, 128, 4, 2, 3, 128>>(p, st);
      default: return launch_pipe_cfg<PipeCfg<MODE_FP8_TENSOR, 128, 128, 2, 2, 4, 64>>(p, st);
    }
  }
  if (mode == MODE_NVFP4) {
    switch (variant) {
      case 1: return launch_pipe_cfg<PipeCfg<MODE_NVFP4, 128, 128, 2, 2, 4, 64, 2>>(p, st);
      case 2: return launch_pipe_cfg<PipeCfg<MODE_NVFP4, 256, 256, 2, 4, 4, 64>>(p, st);
      default: return launch_pipe_cfg<PipeCfg<MODE_NVFP4, 256, 256, 2, 4, 2, 128>>(p, st);
    }
  }
  switch (variant) {
    case 0: return launch_pipe_cfg<PipeCfg<MODE_MXFP4, 256, 256, 2, 4, 4, 64>>(p, st);
    case 2: return launch_pipe_cfg<PipeCfg<MODE_MXFP4, 256, 256, 2, 4, 2, 128>>(p, st);
    default: return launch_pipe_cfg<PipeCfg<MODE_MXFP4, 128, 128, 2, 2, 4, 64>>(p, st);
  }
}

}  // namespace dsl
