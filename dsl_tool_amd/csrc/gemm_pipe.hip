// Dense pipelined GEMM kernels for gfx950 (FP8 per-tensor, FP8 block-scaled,
// MXFP4, NVFP4, bf16); the mainloop, DMA ring and LDS layout are described in
// pipe_core.h.
#include <type_traits>

#include "pipe_core.h"

namespace dsl {

// TR (chosen by the launcher wherever the output tile can be staged in the
// idle ring): the W tile is the MFMAs' first operand, so a lane holds one
// output row and, per group of four registers, four adjacent columns; the
// epilogue writes those as one packed 8-byte bf16 (or one 16-byte fp32)
// staging store instead of four scattered ones.  Without staging room the
// fp32 output keeps the other layout, whose column-contiguous direct stores
// coalesce.
template <class Cfg, bool TR>
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
  pipe_mainloop<Cfg, TR>(p, m0, n0, smem, wave, lane, acc);

  float s1 = 1.f, s2 = 1.f;
  constexpr bool GLOBAL = Cfg::MODE == MODE_FP8_TENSOR || Cfg::MODE == MODE_NVFP4;
  if constexpr (GLOBAL) {
    s1 = *p.ga;
    s2 = *p.gb;
  }
  using Out = pipe::OutStage<Cfg::BM, Cfg::BN>;
  if constexpr (TR) {
    static_assert(Cfg::BM * Cfg::BN * 2 <= Cfg::LDS, "TR stages the bf16 tile in LDS");
    // lane: row 32i + l%32 of the wave's tile; registers 4q..4q+3: columns
    // 32j + 8q + 4h .. +3
    auto val = [&](int i, int j, int r) __attribute__((always_inline)) {
      float v = acc[i][j][r];
      if constexpr (GLOBAL) v = (v * s1) * s2;
      return v;
    };
    if (p.out_f32) {
      if constexpr (Cfg::BM * Cfg::BN * 4 <= Cfg::LDS) {
        using OutF = pipe::OutStageF32<Cfg::BM, Cfg::BN>;
        float *stg = reinterpret_cast<float *>(smem);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
          for (int j = 0; j < Cfg::TN; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int row = wm * Cfg::WM + i * 32 + r32;
              const int col = wn * Cfg::WN + j * 32 + 8 * q + 4 * h;
              *reinterpret_cast<float4 *>(stg + OutF::off(row, col)) =
                  make_float4(val(i, j, 4 * q), val(i, j, 4 * q + 1), val(i, j, 4 * q + 2),
                              val(i, j, 4 * q + 3));
            }
        __syncthreads();
        OutF::template store<Cfg::NT>(p, m0, n0, stg);
      } else {
        // no staging room (the launcher does not pick TR then): direct stores
#pragma unroll
        for (int i = 0; i < Cfg::TM; ++i) {
          const int row = m0 + wm * Cfg::WM + i * 32 + r32;
          if (row >= p.M) continue;
#pragma unroll
          for (int j = 0; j < Cfg::TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int col = n0 + wn * Cfg::WN + j * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
              if (col >= p.N) continue;
              float *d = static_cast<float *>(p.c) + (int64_t)row * p.ldc + col;
              *d = p.accumulate ? *d + val(i, j, r) : val(i, j, r);
            }
        }
      }
      return;
    }
    uint16_t *stg = reinterpret_cast<uint16_t *>(smem);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int row = wm * Cfg::WM + i * 32 + r32;
          const int col = wn * Cfg::WN + j * 32 + 8 * q + 4 * h;
          *reinterpret_cast<uint2 *>(stg + Out::off(row, col)) =
              make_uint2(pack_bf16x2(val(i, j, 4 * q), val(i, j, 4 * q + 1)),
                         pack_bf16x2(val(i, j, 4 * q + 2), val(i, j, 4 * q + 3)));
        }
    __syncthreads();
    Out::template store<Cfg::NT>(p, m0, n0, stg);
    return;
  }
  if constexpr (Cfg::BM * Cfg::BN * 2 <= Cfg::LDS) {
    if (!p.out_f32) {
      // bf16: stage the tile in the idle ring, then write whole rows
      uint16_t *stg = reinterpret_cast<uint16_t *>(smem);
      __syncthreads();
#pragma unroll
      for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::TN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = wm * Cfg::WM + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
            const int col = wn * Cfg::WN + j * 32 + r32;
            float v = acc[i][j][r];
            if constexpr (GLOBAL) v = (v * s1) * s2;
            stg[Out::off(row, col)] = f32_to_bf16(v);
          }
      __syncthreads();
      Out::template store<Cfg::NT>(p, m0, n0, stg);
      return;
    }
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
        if (p.out_f32) {
          float *d = static_cast<float *>(p.c) + (int64_t)row * p.ldc + col;
          *d = p.accumulate ? *d + v : v;      // C += result: one writer per element
        } else {
          static_cast<uint16_t *>(p.c)[(int64_t)row * p.ldc + col] = f32_to_bf16(v);
        }
      }
    }
}

// Block-scaled FP8 (1x128 activation groups, 128x128 weight blocks): one
// 16x16x128 MFMA per output tile per stage yields the group's partial sum,
// folded at once into the fp32 accumulator as acc += part * sa[m,g] * sb[n/128,g]
// (the group-partial form of cuda/gemm/fp8_gemm.cu:84-97).  The W fragment
// is the MFMA's first operand, so a lane holds one output row (m = lane % 16)
// and four consecutive columns (4 * (lane / 16) ..): one row scale per lane,
// and four adjacent bf16 results that leave as one 8-byte write.  Activation
// scales travel with the stage; the weight scale of the wave's 128-column
// block is one scalar load per stage.  With per-column weight scales
// (MODE_FP8_GCOL, sb[g][n] as fp8_gemm_groupwise_kernel reads them) the
// stage also carries the tile's BN weight scales of its group, and each
// lane folds part * (sa[m,g] * sb[g,n]) for its own four columns.
template <class Cfg>
__global__ __launch_bounds__(Cfg::NT) __attribute__((amdgpu_waves_per_eu(Cfg::OCC, Cfg::OCC)))
void gemm_pipe_block_kernel(const GemmArgs p) {
  static_assert(Cfg::BLOCK && (Cfg::GCOL || (Cfg::WN <= 128 && 128 % Cfg::WN == 0)),
                "block-scale tiling");
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

  // Eight waves (two per SIMD; waves w and w + 4 share one): a wave cannot
  // issue its MFMAs until its nine copies have gone out, and copies issue at
  // the L2-to-LDS rate (~16 cycles per 1 KB instruction per CU), so when both
  // waves of a SIMD issue theirs together after the barrier the matrix pipe
  // idles.  Waves 4-7 therefore issue after their first row of MFMAs, and
  // the ring advances its source pointers in place, which leaves no address
  // temporaries live there.
  constexpr bool STAGGER = Cfg::NW == 8;
  // Four waves (one per SIMD, groupwise per-column scales): the copies go
  // out spread over the MFMA rows, a share after each row, so the SIMD's
  // only wave is not held at a burst of nine before its first MFMA
  // (2048x7168x4096 78.9 -> 75.9 us, 1500x1000x1024 9.70 -> 9.29 same-box;
  // the 128x128 block tiles measured 10% slower that way and keep the burst)
  constexpr bool SPREAD = Cfg::NW == 4 && Cfg::GCOL;
  const bool late = STAGGER && wave >= 4;
  auto issue_stage = [&](int s) __attribute__((always_inline)) {
    if constexpr (STAGGER || SPREAD) ring.issue_next(s, lds0);
    else ring.issue(s, lds0);
  };
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nks) issue_stage(s);

  v4f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};

  for (int ks = 0; ks < nks; ++ks) {
    const float sbv = Cfg::GCOL ? 1.f : sbp[ks];
    if (ks + NS - 2 < nks) pipe::wait_vmcnt<(NS - 2) * D>();
    else pipe::wait_vmcnt<0>();
    __syncthreads();
    const uint8_t *st = smem + (ks % NS) * Cfg::STAGE;
    const uint8_t *sA = st, *sB = st + Cfg::A_BYTES;
    const float *sSa = reinterpret_cast<const float *>(st + Cfg::A_BYTES + Cfg::B_BYTES);
    v4f sbc[TN];                         // GCOL: the lane's four column scales per 16-column tile
    if constexpr (Cfg::GCOL) {
#pragma unroll
      for (int t = 0; t < TN; ++t)
        sbc[t] = *reinterpret_cast<const v4f *>(sSa + Cfg::BM + wn * Cfg::WN + t * 16 + 4 * g);
    }
    auto ld = [&](const uint8_t *base, int row) {
      const int s = pipe::swz<SKB>(row);
      const v4i lo = *reinterpret_cast<const v4i *>(base + row * SKB + (((2 * g) ^ s) << 4));
      const v4i hi = *reinterpret_cast<const v4i *>(base + row * SKB + (((2 * g + 1) ^ s) << 4));
      return (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    v8i bf[TN];
#pragma unroll
    for (int t = 0; t < TN; ++t) bf[t] = ld(sB, wn * Cfg::WN + t * 16 + r16);
    // the next row's A fragment is read while this row's MFMAs run
    v8i afn = ld(sA, wm * Cfg::WM + r16);
    // the next stage's copies go out after this stage's first fragment
    // reads, so that those are not queued behind the copy burst
    if (!SPREAD && !late && ks + NS - 1 < nks) issue_stage(ks + NS - 1);
    // Rows are software-pipelined: row i's MFMAs are issued before row
    // i-1's partials are scaled into the accumulator, so the matrix pipe
    // works while the VALU folds (issuing each fold right after its own
    // MFMA left the wave waiting on that MFMA's result).
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
    v4f part[2][TN];
    float srq[2];                        // the lane's row scale (times sb for 128x128 blocks)
#pragma unroll
    for (int i = 0; i <= TM; ++i) {
      if (i < TM) {
        const int arow = wm * Cfg::WM + i * 16;
        const v8i af = afn;
        if (i + 1 < TM) afn = ld(sA, arow + 16 + r16);
        srq[i & 1] = sSa[arow + r16] * sbv;
#pragma unroll
        for (int j = 0; j < TN; ++j)
          part[i & 1][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf[j], af, zero, 0, 0,
                                                                            0, 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (i == 0 && late && ks + NS - 1 < nks) issue_stage(ks + NS - 1);
      if constexpr (SPREAD) {
        if (i < TM && ks + NS - 1 < nks) ring.issue_range(ks + NS - 1, lds0, i * D / TM, (i + 1) * D / TM);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (i > 0) {
        const int ip = i - 1;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if constexpr (Cfg::GCOL)
            acc[ip][j] = part[ip & 1][j] * (sbc[j] * srq[ip & 1]) + acc[ip][j];
          else acc[ip][j] = part[ip & 1][j] * srq[ip & 1] + acc[ip][j];
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  using Out = pipe::OutStage<Cfg::BM, Cfg::BN>;
  if constexpr (Cfg::BM * Cfg::BN * 2 <= Cfg::LDS) {
    if (!p.out_f32) {
      uint16_t *stg = reinterpret_cast<uint16_t *>(smem);
      __syncthreads();
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int row = wm * Cfg::WM + i * 16 + r16;
          const int col = wn * Cfg::WN + j * 16 + 4 * g;   // four columns, 8-byte aligned
          *reinterpret_cast<uint2 *>(stg + Out::off(row, col)) =
              make_uint2(pack_bf16x2(acc[i][j][0], acc[i][j][1]), pack_bf16x2(acc[i][j][2], acc[i][j][3]));
        }
      __syncthreads();
      Out::template store<Cfg::NT>(p, m0, n0, stg);
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int row = m0 + wm * Cfg::WM + i * 16 + r16;
    if (row >= p.M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int col = n0 + wn * Cfg::WN + j * 16 + 4 * g + r;
        if (col >= p.N) continue;
        if (p.out_f32) static_cast<float *>(p.c)[(int64_t)row * p.ldc + col] = acc[i][j][r];
        else static_cast<uint16_t *>(p.c)[(int64_t)row * p.ldc + col] = f32_to_bf16(acc[i][j][r]);
      }
  }
}

// Block-scaled FP8 (1x128 activation groups, 128x128 weight blocks) on the
// prefetch schedule: 64-byte stages, two per 128-K group, 32x32x64 MFMAs
// with the operands swapped so that each lane owns one output row.  Instead
// of a separate partial sum per group, the accumulator is kept in units of
// the current group's scale s_g(m) = sa[m][g] * sb[n/128][g]: MFMAs add the
// group's raw products, and at each group boundary the accumulator is
// multiplied by s_g / s_g+1; the epilogue multiplies by the last group's
// scale.  This equals the sum over groups of partial(g) * s_g of
// cuda/gemm/fp8_gemm.cu:84-97 up to fp32 rounding.
//
// Activation scales sa[M][K/128] travel in their own LDS ring of two slots,
// each holding one set of 4 groups for the tile's BM rows ([row][4 groups],
// 16 bytes per row, so one 16-byte DMA per lane reads a row's 4 groups).
// Wave 0 issues exactly one scale DMA with every stage: with stage s it
// loads row block t = (s+6) % 8 (t < 4) of set (s+6) / 8, else a dummy copy
// into a 1 KB scratch area, so its vmcnt count per stage stays fixed.  Set q
// is first read in the step that consumes stage 8q-1 (whose wait covers all
// loads issued with stages <= 8q) and its slot was last read in the step of
// stage 8q-11 (before the step that issues stage 8q-6 with a 4-stage ring);
// set 0 goes out before the prologue.  The weight scale of a wave's
// 128-column block is picked per group with readlane from one VGPR.
template <class Cfg>
struct BlockScales {
  static_assert(Cfg::NS <= 4, "the scale ring schedule assumes a ring of at most 4 stages");
  uint32_t sa_lds;        // LDS address of the scale ring
  int nsets;              // ceil(K/128 / 4)
  DSL_DEV void init(const GemmArgs &p, uint32_t lds0) {
    sa_lds = lds0 + Cfg::NS * Cfg::STAGE;
    nsets = (p.K / 128 + 3) / 4;
  }
  // the scale DMA of row block t of set q (a dummy copy if t >= 4 or q is
  // past the last set)
  DSL_DEV void issue(const GemmArgs &p, int m0, int lane, int q, int t) const {
    const int nkg = p.K / 128;
    const bool real = t < 4 && q < nsets;
    const int tb = real ? t : 0, qb = real ? q : 0;
    int row = m0 + tb * 64 + lane;
    row = row < p.M ? row : p.M - 1;
    const float *src = static_cast<const float *>(p.sa) + (int64_t)row * nkg + qb * 4;
    const uint32_t dst = real ? sa_lds + (uint32_t)((q & 1) * Cfg::SA_SET + t * 1024)
                              : sa_lds + 2 * Cfg::SA_SET;
    pipe::dma16(src, dst);
  }
  DSL_DEV void issue_for_stage(const GemmArgs &p, int m0, int lane, int s) const {
    issue(p, m0, lane, (s + 6) >> 3, (s + 6) & 7);
  }
  // sa[row][g] from the ring (row within the tile)
  static DSL_DEV float get(const uint8_t *smem, int row, int g) {
    const float *ring = reinterpret_cast<const float *>(smem + Cfg::NS * Cfg::STAGE);
    return ring[((g >> 2) & 1) * (Cfg::SA_SET / 4) + row * 4 + (g & 3)];
  }
};

template <class Cfg, bool ISSUE>
DSL_DEV void block_pf_step(int ks, int nks, bool rescale, int g_next, float sb_next,
                           const GemmArgs &p, int m0, bool sa_wave, const BlockScales<Cfg> &bs,
                           const pipe::Ring<Cfg> &ring, uint32_t lds0, const uint8_t *smem,
                           const StageFrag<Cfg> &cur, StageFrag<Cfg> &nxt, int wm, int wn,
                           int lane, float (&sc)[Cfg::TM], v16f (&acc)[Cfg::TM][Cfg::TN]) {
  constexpr int NS = Cfg::NS, D = Cfg::D, TM = Cfg::TM, TN = Cfg::TN;
  const int r32 = lane & 31, h = lane >> 5;
  // wave 0 issues one scale DMA per stage on top of the ring's D; in the
  // steady state (ISSUE) NS-2 stages follow stage ks+1, in the tail fewer
  if constexpr (ISSUE) {
    pipe::wait_stages_of<D + 1, NS - 2>(NS - 2, sa_wave);
  } else {
    const int last = (ks + NS - 1 < nks - 1) ? ks + NS - 1 : nks - 1;
    pipe::wait_stages_of<D + 1, NS - 2>(last - (ks + 1), sa_wave);
  }
  pipe::wait_lds();
  __syncthreads();
  const uint8_t *stn = smem + ((ks + 1) % NS) * Cfg::STAGE;
  nxt.f[0].load_b(stn, 0, wn, r32, h);
  float sn[TM];
  if (rescale) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
      sn[i] = BlockScales<Cfg>::get(smem, wm * Cfg::WM + i * 32 + r32, g_next) * sb_next;
  }
  __builtin_amdgcn_sched_barrier(0);
  float rt[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    cur.f[0].mma_row_t(i, acc);
    if constexpr (ISSUE) {
      if (i == 0 && sa_wave) bs.issue_for_stage(p, m0, lane, ks + NS);
#pragma unroll
      for (int j = i * D / TM; j < (i + 1) * D / TM; ++j) ring.issue_one(j, ks + NS, lds0);
    }
    nxt.f[0].load_a(stn, 0, i, wm, r32, h);
    if (rescale) {
      if (i == 1) {
#pragma unroll
        for (int t = 0; t < TM; ++t) {
          rt[t] = sc[t] * __builtin_amdgcn_rcpf(sn[t]);
          sc[t] = sn[t];
        }
      }
      // row i-1 has had its last MFMA of the group issued one row ago
      if (i >= 1) {
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i - 1][j] *= rt[i - 1];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  if (rescale) {
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[TM - 1][j] *= rt[TM - 1];
  }
}

// Preconditions (checked by the launcher): K % 512 == 0, K / 128 <=
// kBlockPfMaxGroups, sa 16-byte aligned.
constexpr int kBlockPfMaxGroups = 512;

template <class Cfg>
__global__ __launch_bounds__(Cfg::NT) __attribute__((amdgpu_waves_per_eu(Cfg::OCC, Cfg::OCC)))
void gemm_pipe_block_pf_kernel(const GemmArgs p) {
  static_assert(Cfg::BLOCK && Cfg::PF && Cfg::SKB == 64 && Cfg::KSTEPS == 1, "block prefetch cfg");
  static_assert(Cfg::TM >= 2 && Cfg::WN <= 128 && 128 % Cfg::WN == 0, "block-scale tiling");
  static_assert(Cfg::SC_DMA == 0 && Cfg::BM == 4 * 64, "scale ring: four 64-row blocks");
  constexpr int NS = Cfg::NS, D = Cfg::D, TM = Cfg::TM, TN = Cfg::TN;
  __shared__ __align__(16) uint8_t smem[Cfg::LDS];
  const int nbm = (p.M + Cfg::BM - 1) / Cfg::BM, nbn = (p.N + Cfg::BN - 1) / Cfg::BN;
  int tmi, tni;
  tile_coords(blockIdx.x, nbm, nbn, tmi, tni);
  const int m0 = tmi * Cfg::BM, n0 = tni * Cfg::BN;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
  const int r32 = lane & 31, h = lane >> 5;
  const bool sa_wave = wave == 0;
  const uint32_t lds0 = pipe::lds_addr(smem);
  pipe::Ring<Cfg> ring;
  ring.init(p, m0, n0, wave, lane);
  BlockScales<Cfg> bs;
  bs.init(p, lds0);
  const int nks = p.Kb / Cfg::SKB, nkg = p.K / 128;   // nks even, >= 2
  int sbrow = (n0 + wn * Cfg::WN) / 128;
  const int sblim = (p.N + 127) / 128 - 1;
  sbrow = sbrow > sblim ? sblim : sbrow;
  // Weight scales of the tile's 128-column blocks go to LDS once, before
  // the first DMA: a global load inside the loop would be a vector load
  // (the DMA asm may write memory, so the compiler does not use the scalar
  // cache), and waiting for it would also drain the DMA ring.
  constexpr int NBB = Cfg::BN / 128 > 0 ? Cfg::BN / 128 : 1;
  __shared__ float sb_lds[NBB][kBlockPfMaxGroups];
  {
    const int nb0 = n0 / 128;
    for (int idx = threadIdx.x; idx < NBB * nkg; idx += Cfg::NT) {
      const int b = idx / nkg, g = idx - b * nkg;
      const int row = nb0 + b < sblim ? nb0 + b : sblim;
      sb_lds[b][g] = static_cast<const float *>(p.sb)[(int64_t)row * nkg + g];
    }
  }
  const float *sbw = sb_lds[sbrow - n0 / 128 < NBB ? sbrow - n0 / 128 : NBB - 1];
  auto sb_of = [&](int g) { return sbw[g]; };

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // prologue: scale set 0, then stages 0..NS-1 (each with its scale DMA)
  if (sa_wave) {
#pragma unroll
    for (int t = 0; t < 4; ++t) bs.issue(p, m0, lane, 0, t);
  }
#pragma unroll
  for (int s = 0; s < NS; ++s)
    if (s < nks) {
      if (sa_wave) bs.issue_for_stage(p, m0, lane, s);
      ring.issue(s, lds0);
    }
  pipe::wait_stages_of<D + 1, NS - 1>((nks < NS ? nks : NS) - 1, sa_wave);
  __syncthreads();
  StageFrag<Cfg> f0, f1;
  f0.load(smem, wm, wn, r32, h);
  float sc[TM];   // s_g(row) of the group the accumulator is expressed in
  {
    const float sb0 = sb_of(0);
#pragma unroll
    for (int i = 0; i < TM; ++i)
      sc[i] = BlockScales<Cfg>::get(smem, wm * Cfg::WM + i * 32 + r32, 0) * sb0;
  }
  // one pair of steps per group: the second step moves to the next group.
  // NS and nks are even, so both steps of a pair either issue their next
  // stage (steady state) or not (tail); keeping that a compile-time choice
  // leaves no branch between the MFMAs and the rescale that follows them.
  static_assert(NS % 2 == 0, "pairs of steps agree on issuing");
  auto pair = [&](auto issue_tag, int ks) {
    constexpr bool ISSUE = decltype(issue_tag)::value;
    const int gn = ks / 2 + 1;
    const float sb_next = sb_of(gn);
    block_pf_step<Cfg, ISSUE>(ks, nks, false, 0, 0.f, p, m0, sa_wave, bs, ring, lds0, smem, f0,
                              f1, wm, wn, lane, sc, acc);
    block_pf_step<Cfg, ISSUE>(ks + 1, nks, true, gn, sb_next, p, m0, sa_wave, bs, ring, lds0,
                              smem, f1, f0, wm, wn, lane, sc, acc);
  };
  int ks = 0;
  for (; ks + NS < nks && ks + 2 < nks; ks += 2) pair(std::true_type{}, ks);
  for (; ks + 2 < nks; ks += 2) pair(std::false_type{}, ks);
  block_pf_step<Cfg, false>(ks, nks, false, 0, 0.f, p, m0, sa_wave, bs, ring, lds0, smem, f0, f1,
                            wm, wn, lane, sc, acc);
#pragma unroll
  for (int i = 0; i < TM; ++i) f1.f[0].mma_row_t(i, acc);

  using Out = pipe::OutStage<Cfg::BM, Cfg::BN>;
  if (!p.out_f32) {
    uint16_t *stg = reinterpret_cast<uint16_t *>(smem);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int row = wm * Cfg::WM + i * 32 + r32;
          const int col = wn * Cfg::WN + j * 32 + 8 * q + 4 * h;
          const uint32_t lo = (uint32_t)f32_to_bf16(acc[i][j][4 * q] * sc[i]) |
                              ((uint32_t)f32_to_bf16(acc[i][j][4 * q + 1] * sc[i]) << 16);
          const uint32_t hi = (uint32_t)f32_to_bf16(acc[i][j][4 * q + 2] * sc[i]) |
                              ((uint32_t)f32_to_bf16(acc[i][j][4 * q + 3] * sc[i]) << 16);
          *reinterpret_cast<uint2 *>(stg + Out::off(row, col)) = make_uint2(lo, hi);
        }
    __syncthreads();
    Out::template store<Cfg::NT>(p, m0, n0, stg);
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int row = m0 + wm * Cfg::WM + i * 32 + r32;
    if (row >= p.M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int col = n0 + wn * Cfg::WN + j * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (col < p.N) static_cast<float *>(p.c)[(int64_t)row * p.ldc + col] = acc[i][j][r] * sc[i];
      }
  }
}

template <class Cfg>
static hipError_t launch_pipe_cfg(const GemmArgs &p, hipStream_t st) {
  const int tiles = ((p.M + Cfg::BM - 1) / Cfg::BM) * ((p.N + Cfg::BN - 1) / Cfg::BN);
  if constexpr (Cfg::BLOCK && Cfg::PF) gemm_pipe_block_pf_kernel<Cfg><<<tiles, Cfg::NT, 0, st>>>(p);
  else if constexpr (Cfg::BLOCK) gemm_pipe_block_kernel<Cfg><<<tiles, Cfg::NT, 0, st>>>(p);
  else if constexpr (Cfg::BM * Cfg::BN * 2 <= Cfg::LDS) {
    const bool staged = !p.out_f32 || Cfg::BM * Cfg::BN * 4 <= Cfg::LDS;
    if (staged) gemm_pipe_kernel<Cfg, true><<<tiles, Cfg::NT, 0, st>>>(p);
    else gemm_pipe_kernel<Cfg, false><<<tiles, Cfg::NT, 0, st>>>(p);
  } else {
    gemm_pipe_kernel<Cfg, false><<<tiles, Cfg::NT, 0, st>>>(p);
  }
  return hipGetLastError();
}

// Dense FP8 (per-tensor, block-scaled), MXFP4 and NVFP4 GEMM through the
// LDS-DMA pipeline.  Preconditions (checked by the caller): Kb % 128 == 0,
// ksplit == 1, 4-byte aligned scales.  Variant 0 is the default for large
// grids, 1 the 128x128 tile for mid-sized ones; the others are kept as
// alternatives for tuning (DSL_GEMM_PIPE).
hipError_t launch_gemm_pipe(int mode, const GemmArgs &p, int variant, hipStream_t st) {
  // C += result: fp32 output through the plain epilogue only
  if (p.accumulate && (!p.out_f32 || mode_grouped_k(mode))) return hipErrorInvalidValue;
  if (mode == MODE_FP8_GCOL) {
    // per-column weight scales: the per-stage partial kernel (4-byte
    // aligned scales, K % 128 == 0)
    if (variant == 0) return launch_pipe_cfg<PipeCfg<MODE_FP8_GCOL, 256, 256, 2, 4, 2, 128>>(p, st);
    return launch_pipe_cfg<PipeCfg<MODE_FP8_GCOL, 128, 128, 2, 2, 2, 128, 2>>(p, st);
  }
  // The 128x128 tiles run where one round of them holds the problem: one
  // workgroup per CU, so with four waves each SIMD holds a single wave and
  // nothing hides a stage's LDS-read latency.  FP8 per-tensor and bf16 take
  // the fragment prefetch schedule there (same-box A/B: per-tensor
  // 1024x4096x4096 23.4 -> 20.6 us, 1536x2048x4096 22.7 -> 19.3; bf16
  // 1536x2048x4096 38.5 -> 33.5, fp32 out 1024x4096x4096 43.5 -> 40.0);
  // MXFP4 takes eight waves of 64x32 instead, two per SIMD (768x4096x2048
  // 10.5 -> 9.3 us; with the prefetch schedule it gained less).
  if (mode == MODE_BF16)
    return launch_pipe_cfg<PipeCfg<MODE_BF16, 128, 128, 2, 2, 4, 64, 0, 1>>(p, st);
  if (mode == MODE_FP8_BLOCK) {
    const bool ring_ok = p.K % 512 == 0 && p.K / 128 <= kBlockPfMaxGroups &&
                         (reinterpret_cast<uintptr_t>(p.sa) & 15) == 0;
    switch (variant) {
      case 0:
        // prefetch kernel with the activation-scale ring: K % 512 == 0, at
        // most kBlockPfMaxGroups groups, 16-byte aligned sa
        if (ring_ok)
          return launch_pipe_cfg<PipeCfg<MODE_FP8_BLOCK, 256, 256, 2, 4, 4, 64, 0, 1>>(p, st);
        return launch_pipe_cfg<PipeCfg<MODE_FP8_BLOCK, 256, 256, 2, 4, 2, 128>>(p, st);
      case 2: return launch_pipe_cfg<PipeCfg<MODE_FP8_BLOCK, 256, 256, 4, 2, 2, 128>>(p, st);
      case 3: return launch_pipe_cfg<PipeCfg<MODE_FP8_BLOCK, 256, 256, 2, 4, 2, 128>>(p, st);
      default: return launch_pipe_cfg<PipeCfg<MODE_FP8_BLOCK, 128, 128, 2, 2, 2, 128, 2>>(p, st);
    }
  }
  if (mode == MODE_FP8_TENSOR) {
    switch (variant) {
      case 0: return launch_pipe_cfg<PipeCfg<MODE_FP8_TENSOR, 256, 256, 2, 4, 4, 64, 0, 1>>(p, st);
      case 2: return launch_pipe_cfg<PipeCfg<MODE_FP8_TENSOR, 256, 256, 2, 4, 4, 64>>(p, st);
      case 4: return launch_pipe_cfg<PipeCfg<MODE_FP8_TENSOR, 256, 256, 2, 2, 4, 64, 1, 1>>(p, st);
      case 3: return launch_pipe_cfg<PipeCfg<MODE_FP8_TENSOR, 256, 128, 4, 2, 3, 128>>(p, st);
      default: return launch_pipe_cfg<PipeCfg<MODE_FP8_TENSOR, 128, 128, 2, 2, 4, 64, 0, 1>>(p, st);
    }
  }
  if (mode == MODE_NVFP4) {
    switch (variant) {
      // eight waves of 64x32 (two per SIMD) where four left one wave per SIMD
      // alone with its fp16 dequantization: 1024x4096x4096 71.4 -> 67.2 us
      case 1: return launch_pipe_cfg<PipeCfg<MODE_NVFP4, 128, 128, 2, 4, 4, 64>>(p, st);
      case 2: return launch_pipe_cfg<PipeCfg<MODE_NVFP4, 256, 256, 2, 4, 4, 64>>(p, st);
      default: return launch_pipe_cfg<PipeCfg<MODE_NVFP4, 256, 256, 2, 4, 2, 128>>(p, st);
    }
  }
  switch (variant) {
    case 0: return launch_pipe_cfg<PipeCfg<MODE_MXFP4, 256, 256, 2, 4, 4, 64>>(p, st);
    case 2: return launch_pipe_cfg<PipeCfg<MODE_MXFP4, 256, 256, 2, 4, 2, 128>>(p, st);
    case 4: return launch_pipe_cfg<PipeCfg<MODE_MXFP4, 256, 256, 2, 2, 4, 64, 1, 1>>(p, st);
    case 5: return launch_pipe_cfg<PipeCfg<MODE_MXFP4, 256, 256, 2, 4, 4, 64, 0, 1>>(p, st);
    default: return launch_pipe_cfg<PipeCfg<MODE_MXFP4, 128, 128, 2, 4, 4, 64>>(p, st);
  }
}

}  // namespace dsl
