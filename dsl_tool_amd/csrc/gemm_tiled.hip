// Dense quantized GEMM: C[M,N] = A[M,K] . W[N,K]^T on gfx950 MFMA.
// Variant selection (tile shape, split-K) lives in launch_gemm below.
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "gemm_core.h"

namespace dsl {

// Floats between consecutive split-K partial slices in the workspace: M*N
// rounded up to whole float4s, so that every slice starts 16-byte aligned.
__host__ __device__ inline int64_t splitk_slice(int64_t M, int64_t N) {
  return (M * N + 3) / 4 * 4;
}

template <int MODE, class Cfg>
__global__ __launch_bounds__(Cfg::NT) void gemm_tiled_kernel(const GemmArgs p) {
  __shared__ __align__(16) uint8_t smem[Cfg::LDS];
  const int nbm = (p.M + Cfg::BM - 1) / Cfg::BM, nbn = (p.N + Cfg::BN - 1) / Cfg::BN;
  int tmi, tni;
  tile_coords(blockIdx.x, nbm, nbn, tmi, tni);
  const int m0 = tmi * Cfg::BM, n0 = tni * Cfg::BN;

  TileView tv;
  tv.a = p.a + (int64_t)m0 * p.Kb;
  tv.b = p.b + (int64_t)n0 * p.Kb;
  tv.a_rows = min(Cfg::BM, p.M - m0);
  tv.b_rows = min(Cfg::BN, p.N - n0);
  tv.Kb = p.Kb;
  tv.K = p.K;
  tv.sa = tv.sb = nullptr;
  tv.sa_ld = tv.sb_ld = 0;
  if constexpr (MODE == MODE_MXFP4 || MODE == MODE_NVFP4) {
    const int64_t ld = MODE == MODE_MXFP4 ? p.K / 32 : p.K / 16;
    tv.sa = static_cast<const uint8_t *>(p.sa) + (int64_t)m0 * ld;
    tv.sb = static_cast<const uint8_t *>(p.sb) + (int64_t)n0 * ld;
    tv.sa_ld = tv.sb_ld = ld;
  } else if constexpr (MODE == MODE_FP8_BLOCK) {
    const int64_t nkg = (p.K + 127) / 128;
    tv.sa = static_cast<const float *>(p.sa) + (int64_t)m0 * nkg;
    tv.sb = static_cast<const float *>(p.sb) + (int64_t)(n0 / 128) * nkg;
    tv.sa_ld = tv.sb_ld = nkg;
  } else if constexpr (MODE == MODE_FP8_GCOL) {
    const int64_t nkg = (p.K + 127) / 128;
    tv.sa = static_cast<const float *>(p.sa) + (int64_t)m0 * nkg;
    tv.sb = static_cast<const float *>(p.sb) + n0;
    tv.sa_ld = nkg;
    tv.sb_ld = p.N;
  }

  const int nks = (p.Kb + 127) / 128;
  int ks0 = 0, ks1 = nks;
  if (p.ksplit > 1) {
    const int per = (nks + p.ksplit - 1) / p.ksplit;
    ks0 = blockIdx.y * per;
    ks1 = min(nks, ks0 + per);
  }

  v4f acc[Cfg::TM][Cfg::TN];
  tile_mainloop<MODE, Cfg>(tv, ks0, ks1, smem, acc);

  float s1 = 1.f, s2 = 1.f;
  if constexpr (MODE == MODE_FP8_TENSOR || MODE == MODE_NVFP4) {
    s1 = *p.ga;
    s2 = *p.gb;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
  const int r16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int tm = 0; tm < Cfg::TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < Cfg::TN; ++tn) {
      const int col = n0 + wn * Cfg::WN + tn * 16 + r16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = m0 + wm * Cfg::WM + tm * 16 + 4 * g + i;
        if (row < p.M && col < p.N) {
          float v = acc[tm][tn][i];
          if constexpr (MODE == MODE_FP8_TENSOR || MODE == MODE_NVFP4) v = (v * s1) * s2;
          if (p.ksplit > 1) {
            // this K split's own slice of the workspace: the finalize pass
            // adds the slices in split order, so every run sums alike
            p.ws[(int64_t)blockIdx.y * splitk_slice(p.M, p.N) + (int64_t)row * p.N + col] = v;
          } else if (p.out_f32) {
            float *d = static_cast<float *>(p.c) + (int64_t)row * p.ldc + col;
            *d = p.accumulate ? *d + v : v;
          }
          else
            static_cast<uint16_t *>(p.c)[(int64_t)row * p.ldc + col] = f32_to_bf16(v);
        }
      }
    }
}

// Split-K finalize: C (bf16, fp32, or fp32 += for accumulate) from the
// ksplit fp32 partial slices in ws ([ksplit][M][N], slice stride
// splitk_slice(M, N)), added in split order.  Rows over blockIdx.y
// (grid-stride), four columns per thread; `vec`: N % 4 == 0 and C rows
// aligned for 16-byte (fp32) / 8-byte (bf16) stores, so a thread moves its
// four columns with one load per slice and one store (no per-element index
// division).
__global__ void splitk_finalize_kernel(const float *__restrict__ ws, int ksplit,
                                       void *__restrict__ c, int M, int N, int64_t ldc,
                                       int out_f32, int accumulate, int vec) {
  const int col = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (col >= N) return;
  const int64_t slice = splitk_slice(M, N);
  for (int r = blockIdx.y; r < M; r += gridDim.y) {
    const float *src = ws + (int64_t)r * N + col;
    if (vec) {
      float4 v = *reinterpret_cast<const float4 *>(src);
      for (int s = 1; s < ksplit; ++s) {
        const float4 u = *reinterpret_cast<const float4 *>(src + s * slice);
        v = make_float4(v.x + u.x, v.y + u.y, v.z + u.z, v.w + u.w);
      }
      if (out_f32) {
        float4 *d = reinterpret_cast<float4 *>(static_cast<float *>(c) + r * ldc + col);
        if (accumulate) {
          const float4 o = *d;
          v = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
        }
        *d = v;
      } else {
        *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(c) + r * ldc + col) =
            make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
      }
    } else {
      for (int t = 0; t < 4 && col + t < N; ++t) {
        float v = src[t];
        for (int s = 1; s < ksplit; ++s) v += src[s * slice + t];
        if (out_f32) {
          float *d = static_cast<float *>(c) + r * ldc + col + t;
          *d = accumulate ? *d + v : v;
        } else {
          static_cast<uint16_t *>(c)[r * ldc + col + t] = f32_to_bf16(v);
        }
      }
    }
  }
}

// ----------------------------------------------------------------------------
// Variant selection.
// ----------------------------------------------------------------------------
namespace {

struct Plan {
  int variant;   // 0: 256x256 (8 waves)  1: 128x128 (4 waves)  2: 64x128  3: 16x256
  int bm, bn;
  int ksplit;
};

Plan plan_for(int M, int N, int Kb) {
  Plan pl;
  if (M <= 16) { pl.variant = 3; pl.bm = 16; pl.bn = 256; }
  else if (M <= 64) { pl.variant = 2; pl.bm = 64; pl.bn = 128; }
  else if (M <= 128 || N <= 128) { pl.variant = 1; pl.bm = 128; pl.bn = 128; }
  else { pl.variant = 0; pl.bm = 256; pl.bn = 256; }
  const int tiles = ((M + pl.bm - 1) / pl.bm) * ((N + pl.bn - 1) / pl.bn);
  const int nks = (Kb + 127) / 128;
  int ks = 1;
  if (tiles < 256) {
    ks = (256 + tiles - 1) / tiles;
    const int maxk = nks / 4 > 0 ? nks / 4 : 1;    // keep >= 4 stages per split
    if (ks > maxk) ks = maxk;
    if (ks > 16) ks = 16;
    if (ks < 1) ks = 1;
  }
  pl.ksplit = ks;
  return pl;
}

template <int MODE, class Cfg>
void launch_variant(const GemmArgs &p, hipStream_t st) {
  const int tiles = ((p.M + Cfg::BM - 1) / Cfg::BM) * ((p.N + Cfg::BN - 1) / Cfg::BN);
  dim3 grid(tiles, p.ksplit, 1);
  gemm_tiled_kernel<MODE, Cfg><<<grid, Cfg::NT, 0, st>>>(p);
}

template <int MODE>
void launch_mode(const Plan &pl, const GemmArgs &p, hipStream_t st) {
  switch (pl.variant) {
    case 0: launch_variant<MODE, TileCfg<MODE, 256, 256, 2, 4>>(p, st); break;
    case 1: launch_variant<MODE, TileCfg<MODE, 128, 128, 2, 2>>(p, st); break;
    case 2: launch_variant<MODE, TileCfg<MODE, 64, 128, 1, 4>>(p, st); break;
    default: launch_variant<MODE, TileCfg<MODE, 16, 256, 1, 4>>(p, st); break;
  }
}

}  // namespace

// True when environment variable `name` is "0", "off" or "false" (any case).
static bool env_off(const char *name) {
  const char *e = getenv(name);
  if (!e) return false;
  char buf[8] = {0};
  for (int i = 0; i < 7 && e[i]; ++i) buf[i] = (char)((e[i] >= 'A' && e[i] <= 'Z') ? e[i] + 32 : e[i]);
  return strcmp(buf, "0") == 0 || strcmp(buf, "off") == 0 || strcmp(buf, "false") == 0;
}

// Kernel path for a problem.  The choice depends on the shape and on the
// alignment of the scale pointers only, so the workspace query (which sees
// no pointers and assumes aligned scales) and the launch agree whenever the
// scales are aligned; with misaligned scales the launch may fall back to
// the register-staged kernels, split-K only if a workspace was passed.
//   DSL_GEMM_DECODE = 0/off    never use the skinny-M kernel
//   DSL_GEMM_STREAM = 0/off    never use the streaming kernel (M <= 256)
//   DSL_GEMM_SKINNY = stream   2 <= M <= 16 on the streaming kernel too
//                              (default: the skinny-M decode kernel there)
//   DSL_GEMM_PIPE   = 0/off    never use the LDS-DMA pipelined kernels
//   DSL_GEMM_PIPE   = 1..9     force that pipelined variant for large problems
//   DSL_GEMM_PERSIST = 0/off   use the per-tile pipelined kernels instead of
//                              the persistent one for large problems
enum { PATH_DECODE = 0, PATH_PIPE = 1, PATH_TILED = 2, PATH_PERSIST = 3, PATH_STREAM = 4 };
struct Route {
  int path;
  int variant;    // PATH_PIPE variant
  Plan tiled;     // PATH_TILED plan
};

constexpr int kAccShortK = 512;   // C += result with K up to this streams where it can

static bool stream_enabled() {
  static const bool on = !env_off("DSL_GEMM_STREAM");
  return on;
}

static Route route_for(int mode, int M, int N, int K, int Kb, bool sc4, bool sc16) {
  static const bool decode_on = !env_off("DSL_GEMM_DECODE");
  const bool stream_on = stream_enabled();
  const char *skinny = getenv("DSL_GEMM_SKINNY");      // read per launch (tests switch it)
  const bool skinny_stream = skinny && strcmp(skinny, "stream") == 0;
  const bool skinny_decode = skinny && strcmp(skinny, "decode") == 0;
  static const bool persist_on = !env_off("DSL_GEMM_PERSIST");
  static const int pipe_forced = [] {
    if (env_off("DSL_GEMM_PIPE")) return -2;
    const char *e = getenv("DSL_GEMM_PIPE");
    return (e && e[0] >= '1' && e[0] <= '9' && !e[1]) ? e[0] - '0' : -1;
  }();
  Route r{PATH_TILED, -1, plan_for(M, N, Kb)};
  bool streamable = stream_on && stream_supported(mode, M, N, K, Kb, sc16);
  // The streaming kernel's time grows with the number of 64-row activation
  // blocks times N (each block streams all of W, and each W slice re-reads
  // its activation rows), while the 128x128 / persistent tiles stay at about
  // one round up to a few thousand rows.  The edge is a span of
  // 2 * ceil(M/64) * N (thr2 below, in units of 4096), measured for each
  // mode (the crossover moves little with K: both sides scale with it).
  // NVFP4 (dequantized to fp16 in the tiles) streams up to 256 rows whatever
  // N, and above that below span 30 (M=768 N=4096: 61.8 against 76.5 us;
  // M=320 N=14336: 91.4 against 88.1).  Rows of an odd number of 256-byte
  // chunks stream in 32-row blocks: twice the blocks.
  const int64_t t128 = (int64_t)((M + 127) / 128) * ((N + 127) / 128);
  const bool bf16_pipe_round = mode == MODE_BF16 && pipe_forced != -2 && Kb % 128 == 0 && M > 64 &&
                               N > 64 && t128 >= 40 && t128 <= device_cu_count();
  if (streamable && !skinny_stream && M > 32 && (mode != MODE_NVFP4 || M > 256)) {
    const int bm = Kb % 512 == 0 ? 64 : 32;
    const int64_t span2 = 2 * (int64_t)((M + bm - 1) / bm) * N;   // twice the span
    // crossovers re-measured against the prefetching / eight-wave 128x128
    // tiles (same-box sweep, M = 256..1024, N = 2048..14336, K = 2048 and
    // 4096; streamed against the tiles at the first span past the edge):
    // per-tensor and MXFP4 stream up to span 8 x 4096 (10: 12.5 against
    // 9.5 us, MXFP4 13.2 against 8.8), FP8 block up to 10 (14: 20.6 against
    // 14.7), groupwise per-column up to 12 (14: 21.4 against 15.8), bf16
    // where one round of tiles holds it up to 8 (10: 20.8 against 18.0),
    // other bf16 below 30 (35: 53.5 against 45.4 on the persistent tiles).
    const int64_t thr2 = mode == MODE_FP8_GCOL ? 13
                         : mode_grouped_k(mode) ? 11
                         : (mode == MODE_BF16 ? (bf16_pipe_round ? 9 : 30)
                                              : (mode == MODE_NVFP4 ? 30 : 9));
    if (span2 >= thr2 * 4096) streamable = false;
  }
  // Skinny M (measured, graph timing over rotating weights): the streaming
  // kernel is the faster one for M <= 8 (FP8, MXFP4: 4-25%), for bf16 at
  // every M <= 16 (5-26%), and at M = 9..16 wherever the decode kernel's
  // 32-row grid leaves CUs idle or needs a second round (N = 4096: 5.3
  // against 6.1 us, N = 14336: 11.4 against 13.1).  The decode kernel keeps
  // 9 <= M <= 16 when that grid fills 7/8 of the CUs or more in one round
  // (N = 7168: 7.1 against 7.4 us, N = 8192).  NVFP4: the GEMV for M = 1,
  // the streaming kernel above that (N=14336 K=4096: M=1 8.4 against 9.4 us;
  // M=2 10.0 against 14.4; M=4 10.0 against 22.5: the GEMV's time grows with
  // M).  DSL_GEMM_SKINNY=stream|decode forces one of them (tests).
  bool prefer_stream;
  if (skinny_stream) {
    prefer_stream = true;
  } else if (skinny_decode) {
    prefer_stream = false;
  } else if (mode == MODE_NVFP4) {
    prefer_stream = M > 1;
  } else if (M <= 8 || M > 16 || mode == MODE_BF16) {
    prefer_stream = true;
  } else {
    const int64_t g = (N + 31) / 32, cus = device_cu_count();
    prefer_stream = !(8 * g >= 7 * cus && g <= cus);
  }
  if (decode_on && !(prefer_stream && streamable) && decode_supported(mode, M, K, Kb, sc4, sc16)) {
    r.path = PATH_DECODE;
    return r;
  }
  if (streamable) {
    r.path = PATH_STREAM;
    return r;
  }
  if (mode == MODE_BF16) {   // pipelined, persistent or register-staged tiles
    const int64_t t256 = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
    // one round of 128x128 pipelined tiles (40 to one per CU) beats a
    // partial round of 256x256 persistent tiles, which leaves 3/4 of the
    // CUs idle (M=1536 N=2048 K=4096: 44.2 against 84.0 us; M=1024 N=4096:
    // 54.7 against 73.9); past one round the persistent kernel (M=1536
    // N=4096: 95.4 against 100.4).  Then one partial round of the persistent
    // kernel beats the register-staged tiles from about a sixth of the CUs'
    // worth of 256x256 tiles (M=768 N=4096 K=4096: 77 against 102 us;
    // M=2048 N=7168: 104 against 220) and about 2.4M outputs (M=288 N=7168,
    // 56 tiles of which 28 hold 32 rows: 77 against 70 us; M=384: 78 against
    // 89)
    if (bf16_pipe_round) {
      r.path = PATH_PIPE;
      r.variant = 1;
    } else if (persist_on && 6 * t256 >= device_cu_count() && (int64_t)M * N >= 2400000 &&
               persist_supported(mode, M, N, K, Kb, sc16)) {
      r.path = PATH_PERSIST;
    }
    return r;
  }
  const bool pipe_ok = pipe_forced != -2 && Kb % 128 == 0 && (mode == MODE_FP8_TENSOR || sc4);
  if (pipe_ok) {
    const int64_t t256 = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
    // Rounds of tiles per CU: a round of 256x256 persistent tiles costs
    // about as much as 1.6 rounds of the 128x128 pipelined tiles (1.5-2 with
    // block scales), so the persistent kernel takes over once the 128x128
    // grid needs twice its rounds (three times with block scales); below
    // that the 128x128 tiles, down to 40 of them: one round of those beats
    // the register-staged split-K tiles by 1.3-4.6x (M=300 N=5000 K=4096:
    // 24 against 67 us; block 31 against 149).  Measured at N = 512..14336,
    // K = 4096 and 8192, M = 288..3072.  With the prefetching 128x128 tiles
    // FP8 per-tensor keeps two rounds of them too (same-box, M = 1536..4096,
    // N = 2048 and 4096, K = 2048 and 4096: 7-12% ahead of the persistent
    // kernel at six of seven shapes, 2048x4096x4096 41.1 against 42.2 us);
    // MXFP4 does not (two rounds: 33.9 against 28.1 us at 1536x4096x4096).
    const int64_t cus = device_cu_count();
    const int64_t r128 = (t128 + cus - 1) / cus, r256 = (t256 + cus - 1) / cus;
    const int rounds128 = (mode_grouped_k(mode) || mode == MODE_FP8_TENSOR) ? 3 : 2;
    const bool persist_wins = t256 >= 240 || r128 >= rounds128 * r256;
    if (persist_wins) {
      r.path = PATH_PIPE;
      r.variant = pipe_forced >= 0 ? pipe_forced : (t256 >= 240 ? 0 : 1);
      if (persist_on && pipe_forced < 0 && persist_supported(mode, M, N, K, Kb, sc16))
        r.path = PATH_PERSIST;
    } else if (M > 64 && N > 64 && t128 >= 40) {
      r.path = PATH_PIPE;
      r.variant = 1;
    }
  }
  return r;
}

bool gemm_routes_to_stream(int mode, int64_t M, int64_t N, int64_t K, bool or_pipe, bool accumulate) {
  const int Kb = (mode == MODE_MXFP4 || mode == MODE_NVFP4) ? (int)(K / 2)
                                                            : (mode == MODE_BF16 ? (int)(2 * K) : (int)K);
  int path = route_for(mode, (int)M, (int)N, (int)K, Kb, true, true).path;
  if (accumulate && K <= kAccShortK && stream_enabled() && stream_supported(mode, (int)M, (int)N, (int)K, Kb, true))
    path = PATH_STREAM;   // as launch_gemm routes C += result
  return path == PATH_STREAM || (or_pipe && path == PATH_PIPE && (!accumulate || !mode_grouped_k(mode)));
}

size_t gemm_workspace_bytes(int mode, int64_t M, int64_t N, int64_t K, bool accumulate) {
  const int Kb = (mode == MODE_MXFP4 || mode == MODE_NVFP4) ? (int)(K / 2)
                                                            : (mode == MODE_BF16 ? (int)(2 * K) : (int)K);
  Route r = route_for(mode, (int)M, (int)N, (int)K, Kb, true, true);
  if (accumulate) r.path = PATH_TILED;
  return (r.path == PATH_TILED && r.tiled.ksplit > 1)
             ? (size_t)r.tiled.ksplit * (size_t)splitk_slice(M, N) * sizeof(float)
             : 0;
}

hipError_t launch_gemm(int mode, GemmArgs p, hipStream_t st) {
  const uintptr_t sc = reinterpret_cast<uintptr_t>(p.sa) | reinterpret_cast<uintptr_t>(p.sb);
  if (p.Kb2 > 0) {   // a second K segment: the persistent BF16 kernel only
    if (mode != MODE_BF16 || p.accumulate || p.lora_scales || p.Kb % 128 != 0 ||
        p.Kb2 % 128 != 0 || !persist_supported(mode, p.M, p.N, p.K, p.Kb + p.Kb2, true))
      return hipErrorInvalidValue;
    // W2 read from a narrower B whose pairs repeat: whole pairs, a power of
    // two of them per row
    if (p.rep2 != 0 && ((p.rep2 & (p.rep2 - 1)) != 0 || p.ldb2 % 16 != 0 ||
                        p.ldb2 < p.rep2 * 128 || p.Kb2 % (p.rep2 * 128) != 0))
      return hipErrorInvalidValue;
    return launch_gemm_persist(mode, p, st);
  }
  if (p.rep2 != 0 || p.ldb2 != 0) return hipErrorInvalidValue;
  Route r = route_for(mode, p.M, p.N, p.K, p.Kb, (sc & 3) == 0, (sc & 15) == 0);
  if (p.lora_scales) {   // the LoRA epilogue: the streaming kernel only
    if (mode != MODE_BF16 || !stream_supported(mode, p.M, p.N, p.K, p.Kb, true) || p.accumulate)
      return hipErrorInvalidValue;
    return launch_gemm_stream(mode, p, st);
  }
  // C += result (fp32 out, one writer per element): the streaming kernel
  // where the router picks a skinny kernel or K is short (a LoRA adapter
  // add: W is then small enough to stream once per activation block), the
  // pipelined tiles where the router picks those (not block-scaled), else
  // the register-staged kernels
  if (p.accumulate) {
    if ((r.path == PATH_STREAM || r.path == PATH_DECODE || p.K <= kAccShortK) && p.out_f32 &&
        stream_enabled() && stream_supported(mode, p.M, p.N, p.K, p.Kb, (sc & 15) == 0))
      r.path = PATH_STREAM;
    else if (!(r.path == PATH_PIPE && p.out_f32 && !mode_grouped_k(mode)))
      r.path = PATH_TILED;
  }
  p.ksplit = 1;
  if (r.path == PATH_DECODE) return launch_gemm_decode(mode, p, st);
  if (r.path == PATH_STREAM) return launch_gemm_stream(mode, p, st);
  if (r.path == PATH_PIPE) return launch_gemm_pipe(mode, p, r.variant, st);
  if (r.path == PATH_PERSIST) return launch_gemm_persist(mode, p, st);
  const Plan pl = r.tiled;
  // split-K into as many [M][N] fp32 slices as the workspace holds (at most
  // the plan's split count; fewer than two: one pass over K)
  const size_t slice_bytes = (size_t)splitk_slice(p.M, p.N) * sizeof(float);
  const size_t fit = p.ws ? p.ws_bytes / slice_bytes : 0;
  p.ksplit = fit >= 2 ? (int)std::min<size_t>((size_t)pl.ksplit, fit) : 1;
  switch (mode) {
    case MODE_FP8_TENSOR: launch_mode<MODE_FP8_TENSOR>(pl, p, st); break;
    case MODE_FP8_BLOCK: launch_mode<MODE_FP8_BLOCK>(pl, p, st); break;
    case MODE_FP8_GCOL: launch_mode<MODE_FP8_GCOL>(pl, p, st); break;
    case MODE_MXFP4: launch_mode<MODE_MXFP4>(pl, p, st); break;
    case MODE_NVFP4: launch_mode<MODE_NVFP4>(pl, p, st); break;
    case MODE_BF16: launch_mode<MODE_BF16>(pl, p, st); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (p.ksplit > 1) {
    const int esz = p.out_f32 ? 4 : 2;
    const int vec = p.N % 4 == 0 && p.ldc % 4 == 0 &&
                    (reinterpret_cast<uintptr_t>(p.c) % (4 * esz)) == 0;
    const dim3 fgrid((unsigned)((p.N + 1023) / 1024), (unsigned)std::min(p.M, 4096));
    splitk_finalize_kernel<<<fgrid, 256, 0, st>>>(p.ws, p.ksplit, p.c, p.M, p.N, p.ldc,
                                                  p.out_f32, p.accumulate, vec);
    e = hipGetLastError();
  }
  return e;
}

}  // namespace dsl
