// Grouped FP8 GEMM for variable-size groups (MoE experts, LoRA adapters).
//
// Rows offsets[g]..offsets[g+1]-1 of X multiply W[g].  The group-offset
// table stays on the device: every workgroup of a persistent grid builds the
// per-group tile prefix (ceil(n_g/BM) * ceil(N/BN)) in LDS, then walks the
// flattened tile space with stride gridDim.x, locating each tile's group by
// binary search.  Empty groups own zero tiles and are never touched.
// Epilogue: y = (acc * sx[row]) * sw[g, col] (per-row activation scale,
// per-channel weight scale).
#include <cstdlib>
#include <cstring>

#include "gemm_core.h"
#include "pipe_core.h"

namespace dsl {

// Group g's row range with the offsets clamped into [0, rows] and made
// non-decreasing, so malformed tables can never address outside X / Y.
DSL_DEV int2 group_rows(const int32_t *off, int g, int rows) {
  int lo = off[g], hi = off[g + 1];
  lo = lo < 0 ? 0 : (lo > rows ? rows : lo);
  hi = hi < lo ? lo : (hi > rows ? rows : hi);
  return make_int2(lo, hi);
}

template <class Cfg>
__global__ __launch_bounds__(Cfg::NT) void grouped_fp8_kernel(const GroupedArgs p) {
  __shared__ __align__(16) uint8_t smem[Cfg::LDS];
  __shared__ int s_pre[kMaxGroups + 1];
  __shared__ int s_part[Cfg::NT];
  const int tid = threadIdx.x;
  const int nbn = (p.N + Cfg::BN - 1) / Cfg::BN;

  // ---- per-group tile prefix: each thread sums a contiguous run of groups,
  // then a Hillis-Steele scan over the per-thread totals.
  const int per = (p.G + Cfg::NT - 1) / Cfg::NT;
  const int g0 = tid * per, g1 = min(p.G, g0 + per);
  int local = 0;
  for (int gi = g0; gi < g1; ++gi) {
    const int2 gr = group_rows(p.offsets, gi, p.rows);
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
  int run = s_part[tid] - local;   // exclusive prefix of this thread's run
  for (int gi = g0; gi < g1; ++gi) {
    s_pre[gi] = run;
    const int2 gr = group_rows(p.offsets, gi, p.rows);
    run += ((gr.y - gr.x + Cfg::BM - 1) / Cfg::BM) * nbn;
  }
  if (tid == Cfg::NT - 1) s_pre[p.G] = s_part[Cfg::NT - 1];
  __syncthreads();
  const int total = s_pre[p.G];

  const int nks = (p.K + 127) / 128;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
  const int r16 = lane & 15, g = lane >> 4;

  for (int t = blockIdx.x; t < total; t += gridDim.x) {
    // largest group index e with s_pre[e] <= t (empty groups share a prefix
    // value with their successor, so the search lands on a non-empty group)
    int lo = 0, hi = p.G - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_pre[mid] <= t) lo = mid; else hi = mid - 1;
    }
    const int e = lo;
    const int in = t - s_pre[e];
    const int mt = in / nbn, nt = in - mt * nbn;
    const int2 gr = group_rows(p.offsets, e, p.rows);
    const int r0 = gr.x + mt * Cfg::BM;
    const int rows_e = gr.y - r0;
    const int n0 = nt * Cfg::BN;

    TileView tv;
    tv.a = p.x + (int64_t)r0 * p.K;
    tv.b = p.w + ((int64_t)e * p.N + n0) * p.K;
    tv.a_rows = min(Cfg::BM, rows_e);
    tv.b_rows = min(Cfg::BN, p.N - n0);
    tv.Kb = p.K;
    tv.K = p.K;
    tv.sa = tv.sb = nullptr;
    tv.sa_ld = tv.sb_ld = 0;

    v4f acc[Cfg::TM][Cfg::TN];
    tile_mainloop<MODE_FP8_TENSOR, Cfg>(tv, 0, nks, smem, acc);

#pragma unroll
    for (int tm = 0; tm < Cfg::TM; ++tm) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int lr = wm * Cfg::WM + tm * 16 + 4 * g + i;
        if (lr >= tv.a_rows) continue;
        const int row = r0 + lr;
        const float sx = p.sx[row];
#pragma unroll
        for (int tn = 0; tn < Cfg::TN; ++tn) {
          const int col = n0 + wn * Cfg::WN + tn * 16 + r16;
          if (col >= p.N) continue;
          const float v = (acc[tm][tn][i] * sx) * p.sw[(int64_t)e * p.N + col];
          if (p.out_f32) static_cast<float *>(p.y)[(int64_t)row * p.ldy + col] = v;
          else static_cast<uint16_t *>(p.y)[(int64_t)row * p.ldy + col] = f32_to_bf16(v);
        }
      }
    }
  }
}

// Pipelined variant: the same persistent walk over the device-side tile
// prefix, each tile computed by the LDS-DMA mainloop of pipe_core.h (FP8,
// 32x32x64 MFMA).  Rows past the group's end re-read its last row and are
// never stored.  Needs K % 64 == 0.
template <class Cfg>
__global__ __launch_bounds__(Cfg::NT) __attribute__((amdgpu_waves_per_eu(Cfg::OCC, Cfg::OCC)))
void grouped_pipe_kernel(const GroupedArgs p) {
  static_assert(Cfg::MODE == MODE_FP8_TENSOR, "grouped FP8 only");
  __shared__ __align__(16) uint8_t smem[Cfg::LDS];
  __shared__ int s_pre[kMaxGroups + 1];
  __shared__ int s_part[Cfg::NT];
  const int tid = threadIdx.x;
  const int nbn = (p.N + Cfg::BN - 1) / Cfg::BN;

  const int per = (p.G + Cfg::NT - 1) / Cfg::NT;
  const int g0 = tid * per, g1 = min(p.G, g0 + per);
  int local = 0;
  for (int gi = g0; gi < g1; ++gi) {
    const int2 gr = group_rows(p.offsets, gi, p.rows);
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
    const int2 gr = group_rows(p.offsets, gi, p.rows);
    run += ((gr.y - gr.x + Cfg::BM - 1) / Cfg::BM) * nbn;
  }
  if (tid == Cfg::NT - 1) s_pre[p.G] = s_part[Cfg::NT - 1];
  __syncthreads();
  const int total = s_pre[p.G];

  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
  const int r32 = lane & 31, h = lane >> 5;

  for (int t = blockIdx.x; t < total; t += gridDim.x) {
    int lo = 0, hi = p.G - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_pre[mid] <= t) lo = mid; else hi = mid - 1;
    }
    const int e = lo;
    const int in = t - s_pre[e];
    const int mt = in / nbn, nt = in - mt * nbn;
    const int2 gr = group_rows(p.offsets, e, p.rows);
    const int r0 = gr.x + mt * Cfg::BM;
    const int n0 = nt * Cfg::BN;

    GemmArgs sub;
    sub.a = p.x + (int64_t)r0 * p.K;
    sub.b = p.w + (int64_t)e * p.N * p.K;
    sub.c = p.y;
    sub.M = gr.y - r0;                   // rows of this group from r0 on
    sub.N = p.N;
    sub.K = p.K;
    sub.Kb = p.K;
    sub.ldc = p.ldy;
    sub.sa = sub.sb = nullptr;
    sub.ga = sub.gb = nullptr;
    sub.ws = nullptr;
    sub.ws_bytes = 0;
    sub.ksplit = 1;
    sub.out_f32 = p.out_f32;

    v16f acc[Cfg::TM][Cfg::TN];
    pipe_mainloop<Cfg>(sub, 0, n0, smem, wave, lane, acc);

#pragma unroll
    for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lr = wm * Cfg::WM + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (lr >= sub.M) continue;
        const int row = r0 + lr;
        const float sx = p.sx[row];
#pragma unroll
        for (int j = 0; j < Cfg::TN; ++j) {
          const int col = n0 + wn * Cfg::WN + j * 32 + r32;
          if (col >= p.N) continue;
          const float v = (acc[i][j][r] * sx) * p.sw[(int64_t)e * p.N + col];
          if (p.out_f32) static_cast<float *>(p.y)[(int64_t)row * p.ldy + col] = v;
          else static_cast<uint16_t *>(p.y)[(int64_t)row * p.ldy + col] = f32_to_bf16(v);
        }
      }
    __syncthreads();                     // the next tile's loads reuse smem
  }
}

template <class Cfg>
static void launch_grouped_cfg(const GroupedArgs &p, hipStream_t st) {
  const int nbn = (p.N + Cfg::BN - 1) / Cfg::BN;
  const int64_t upper = ((int64_t)(p.rows + Cfg::BM - 1) / Cfg::BM + p.G) * nbn;
  int64_t grid = device_cu_count();
  if (grid > upper) grid = upper;
  if (grid < 1) grid = 1;
  grouped_fp8_kernel<Cfg><<<(unsigned)grid, Cfg::NT, 0, st>>>(p);
}

template <class Cfg>
static void launch_grouped_pipe_cfg(const GroupedArgs &p, hipStream_t st) {
  const int nbn = (p.N + Cfg::BN - 1) / Cfg::BN;
  const int64_t upper = ((int64_t)(p.rows + Cfg::BM - 1) / Cfg::BM + p.G) * nbn;
  int64_t grid = device_cu_count();
  if (grid > upper) grid = upper;
  if (grid < 1) grid = 1;
  grouped_pipe_kernel<Cfg><<<(unsigned)grid, Cfg::NT, 0, st>>>(p);
}

hipError_t launch_grouped_fp8(GroupedArgs p, hipStream_t st) {
  if (p.rows == 0 || p.N == 0) return hipSuccess;
  const int avg = p.rows / (p.G > 0 ? p.G : 1);
  if (p.arow) {   // the gather form: streaming tiles at decode sizes, else the persistent kernel
    if (avg < 48 && grouped_stream_supported(p)) return launch_grouped_stream(p, st);
    return grouped_persist_supported(p) ? launch_grouped_persist(p, st) : hipErrorInvalidValue;
  }
  // DSL_GEMM_PERSIST=0 keeps the per-tile pipelined walk below (tuning)
  static const bool persist_on = [] {
    const char *e = getenv("DSL_GEMM_PERSIST");
    if (!e) return true;
    char v[8] = {0};
    for (int i = 0; i < 7 && e[i]; ++i) v[i] = (char)((e[i] >= 'A' && e[i] <= 'Z') ? e[i] + 32 : e[i]);
    return !(strcmp(v, "0") == 0 || strcmp(v, "off") == 0 || strcmp(v, "false") == 0);
  }();
  // Few rows per group (MoE decode): the streaming tiles read each group's W
  // once with its rows (64 experts, N=1536 K=2048, 32 tokens x top-8: 37.4
  // against 53.3 us); from 64 rows per group the tiles win again (512
  // tokens: 63.8 us persistent, 117.9 streaming).
  if (avg < 48 && grouped_stream_supported(p)) return launch_grouped_stream(p, st);
  // From there on the persistent 256x256 walk, also for groups well below
  // 256 rows: 64 experts, N=1536 K=2048, 1024 tokens x top-8 (128 rows per
  // expert): 67.6 against 110.2 us on the 128x256 pipelined tiles; 384
  // tokens: 63.8 against 71.9.
  if (persist_on && grouped_persist_supported(p)) return launch_grouped_persist(p, st);
  if (p.K % 64 == 0) {
    // DSL_GROUPED_TILE=256 / 128 forces the 256x256 / 128x256 tile (tuning)
    static const int forced = [] {
      const char *e = getenv("DSL_GROUPED_TILE");
      return e ? atoi(e) : 0;
    }();
    if (forced == 256 || (forced != 128 && avg >= 256))
      launch_grouped_pipe_cfg<PipeCfg<MODE_FP8_TENSOR, 256, 256, 2, 4, 4, 64>>(p, st);
    else
      launch_grouped_pipe_cfg<PipeCfg<MODE_FP8_TENSOR, 128, 256, 2, 4, 4, 64>>(p, st);
    return hipGetLastError();
  }
  launch_grouped_cfg<TileCfg<MODE_FP8_TENSOR, 128, 128, 2, 2>>(p, st);
  return hipGetLastError();
}

}  // namespace dsl
