// Quantize/pack kernels: bf16 -> E4M3 (per-tensor, block-scaled),
// MXFP4 (E2M1 + E8M0 / 32), NVFP4 (E2M1 + E4M3 / 16 + fp32 global).
//
// All kernels read x[r*sr + c*sc] (bf16) and write K-major codes q[r*C + c]
// (FP8) or packed nibbles q[r*C/2 + c/2] (FP4).  Two code paths:
//   * vector path (sc == 1, C % 8 == 0, sr % 8 == 0, 16-B aligned x):
//     each thread owns 8 consecutive elements (one 16-B load); a "team" of
//     T threads owns one scale group and reduces its amax with lane shuffles;
//   * strided path (anything else, e.g. the reference's B[K,N] given as a
//     contiguous [K,N] tensor): one thread per scale group, threads ordered
//     so that the unit-stride axis is the fast one across lanes.
// Arithmetic is the bit-exact contract of include/dsl_gemm.h (fp32 scales,
// IEEE division x / scale, RNE encoders from common.h); the vector paths
// encode with the gfx950 hardware converters, which common.h shows equal to
// those encoders, dividing through the exact reciprocal with an exact
// fallback near rounding boundaries.
#include "common.h"
#include "launch.h"

namespace dsl {

DSL_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// Block-wide max; `sh` needs blockDim.x/64 floats.  Every thread gets it.
DSL_DEV float block_max(float v, float *sh) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, nw = blockDim.x >> 6;
  __syncthreads();
  if (l == 0) sh[w] = v;
  __syncthreads();
  float r = 0.f;
  for (int i = 0; i < nw; ++i) r = fmaxf(r, sh[i]);
  return r;
}

DSL_DEV void unpack8(const uint4 &v, float f[8]) {
  f[0] = u2f(v.x << 16); f[1] = u2f(v.x & 0xffff0000u);
  f[2] = u2f(v.y << 16); f[3] = u2f(v.y & 0xffff0000u);
  f[4] = u2f(v.z << 16); f[5] = u2f(v.z & 0xffff0000u);
  f[6] = u2f(v.w << 16); f[7] = u2f(v.w & 0xffff0000u);
}

DSL_DEV float amax8(const float f[8]) {
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) m = fmaxf(m, __builtin_fabsf(f[i]));
  return m;
}

DSL_DEV float load_bf16(const uint16_t *x, int64_t idx) { return bf16_to_f32(x[idx]); }

// Reduce the pass-1 partial maxima (n <= kMaxPartials) inside one block.
DSL_DEV float reduce_partials(const float *partial, int n, float *sh) {
  float m = 0.f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, partial[i]);
  return block_max(m, sh);
}

DSL_DEV float fp8_scale_of(float amax) {
  float s = amax / kE4M3Max;
  return s < kScaleFloor ? kScaleFloor : s;
}

DSL_DEV float nv_global_of(float amax) {
  float s = amax / kNvGlobalDiv;
  return s < kScaleFloor ? kScaleFloor : s;
}

// 8 values / s as E4M3 codes (2 x u32), with the hardware encoder (see
// e4m3_div_pk); rs = 1.0f / s.
DSL_DEV uint2 e4m3_div8(const float (&f)[8], float s, float rs) {
  const uint32_t lo = e4m3_div_pk(f[0], f[1], s, rs) | (e4m3_div_pk(f[2], f[3], s, rs) << 16);
  const uint32_t hi = e4m3_div_pk(f[4], f[5], s, rs) | (e4m3_div_pk(f[6], f[7], s, rs) << 16);
  return make_uint2(lo, hi);
}

// ---------------------------------------------------------------------------
// Pass 1 of the per-tensor / NVFP4 quantizers: per-block amax partials.
// ---------------------------------------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(256) void amax_partial_kernel(
    const uint16_t *__restrict__ x, int64_t rows, int64_t cols, int64_t sr, int64_t sc,
    float *__restrict__ partial) {
  __shared__ float sh[4];
  float m = 0.f;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  if (VEC) {
    const int64_t cpr = cols >> 3, total = rows * cpr;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
      const int64_t r = i / cpr, c8 = i - r * cpr;
      float f[8];
      unpack8(*reinterpret_cast<const uint4 *>(x + r * sr + c8 * 8), f);
      m = fmaxf(m, amax8(f));
    }
  } else {
    const int64_t total = rows * cols;
    const bool rfast = (sr == 1);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
      int64_t r, c;
      if (rfast) { c = i / rows; r = i - c * rows; } else { r = i / cols; c = i - r * cols; }
      m = fmaxf(m, __builtin_fabsf(load_bf16(x, r * sr + c * sc)));
    }
  }
  m = block_max(m, sh);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

// ---------------------------------------------------------------------------
// Per-tensor E4M3, pass 2.
// ---------------------------------------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(256) void quant_fp8_tensor_kernel(
    const uint16_t *__restrict__ x, int64_t rows, int64_t cols, int64_t sr, int64_t sc,
    const float *__restrict__ partial, int nparts, uint8_t *__restrict__ q,
    float *__restrict__ scale_out) {
  __shared__ float sh[4];
  const float scale = fp8_scale_of(reduce_partials(partial, nparts, sh));
  const float rscale = 1.0f / scale;
  if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  if (VEC) {
    const int64_t cpr = cols >> 3, total = rows * cpr;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
      const int64_t r = i / cpr, c8 = i - r * cpr;
      float f[8];
      unpack8(*reinterpret_cast<const uint4 *>(x + r * sr + c8 * 8), f);
      *reinterpret_cast<uint2 *>(q + r * cols + c8 * 8) = e4m3_div8(f, scale, rscale);
    }
  } else {
    const int64_t total = rows * cols;
    const bool rfast = (sr == 1);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
      int64_t r, c;
      if (rfast) { c = i / rows; r = i - c * rows; } else { r = i / cols; c = i - r * cols; }
      q[r * cols + c] = e4m3_encode(load_bf16(x, r * sr + c * sc) / scale);
    }
  }
}

// ---------------------------------------------------------------------------
// Row-group team kernels (vector path).  A team of T lanes (T | 64) owns one
// group of 8*T consecutive elements of a row.  KIND selects the format.
// ---------------------------------------------------------------------------
enum { KIND_FP8 = 0, KIND_MX = 1, KIND_NV = 2 };

template <int KIND, int T>
__global__ __launch_bounds__(256) void quant_rowgroup_kernel(
    const uint16_t *__restrict__ x, int64_t rows, int64_t cols, int64_t sr,
    uint8_t *__restrict__ q, void *__restrict__ scales,
    const float *__restrict__ partial, int nparts, float *__restrict__ global_out) {
  constexpr int G = 8 * T;                      // elements per group
  __shared__ float sh[4];
  float sg = 1.f;
  if (KIND == KIND_NV) {
    sg = nv_global_of(reduce_partials(partial, nparts, sh));
    if (blockIdx.x == 0 && threadIdx.x == 0) *global_out = sg;
  }
  const int64_t gpr = (cols + G - 1) / G;       // groups per row
  const int64_t ngroups = rows * gpr;
  const int lane = threadIdx.x % T;
  const int64_t team0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / T;
  const int64_t nteams = (int64_t)gridDim.x * blockDim.x / T;
  for (int64_t g = team0; g < ngroups; g += nteams) {   // uniform across a team
    const int64_t r = g / gpr, gi = g - r * gpr;
    const int64_t c = gi * G + (int64_t)lane * 8;
    const bool ok = c < cols;
    float f[8];
    if (ok) unpack8(*reinterpret_cast<const uint4 *>(x + r * sr + c), f);
    else {
#pragma unroll
      for (int j = 0; j < 8; ++j) f[j] = 0.f;
    }
    float m = amax8(f);
#pragma unroll
    for (int o = 1; o < T; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
    if (KIND == KIND_FP8) {
      const float s = fp8_scale_of(m);
      if (lane == 0) reinterpret_cast<float *>(scales)[g] = s;
      if (ok) *reinterpret_cast<uint2 *>(q + r * cols + c) = e4m3_div8(f, s, 1.0f / s);
    } else if (KIND == KIND_MX) {
      const int e = mx_exponent(m);
      const float mul = pow2_neg(e);
      if (lane == 0) reinterpret_cast<uint8_t *>(scales)[g] = (uint8_t)(e + 127);
      uint32_t p = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) p |= e2m1_pk(f[2 * j] * mul, f[2 * j + 1] * mul) << (8 * j);
      if (ok) *reinterpret_cast<uint32_t *>(q + ((r * cols + c) >> 1)) = p;
    } else {  // KIND_NV
      const uint8_t sb = e4m3_encode((m / 6.0f) / sg);
      const float d = e4m3_decode(sb) * sg;
      if (lane == 0) reinterpret_cast<uint8_t *>(scales)[g] = sb;
      uint32_t p = 0;
      if (d != 0.f) {
        const float rd = 1.0f / d;
#pragma unroll
        for (int j = 0; j < 4; ++j) p |= e2m1_div_pk(f[2 * j], f[2 * j + 1], d, rd) << (8 * j);
      }
      if (ok) *reinterpret_cast<uint32_t *>(q + ((r * cols + c) >> 1)) = p;
    }
  }
}

// ---------------------------------------------------------------------------
// Strided path: one thread per scale group (group_rows == 1 groups only).
// ---------------------------------------------------------------------------
template <int KIND>
__global__ __launch_bounds__(256) void quant_group_scalar_kernel(
    const uint16_t *__restrict__ x, int64_t rows, int64_t cols, int64_t sr, int64_t sc,
    int64_t gsize, uint8_t *__restrict__ q, void *__restrict__ scales,
    const float *__restrict__ partial, int nparts, float *__restrict__ global_out) {
  __shared__ float sh[4];
  float sg = 1.f;
  if (KIND == KIND_NV) {
    sg = nv_global_of(reduce_partials(partial, nparts, sh));
    if (blockIdx.x == 0 && threadIdx.x == 0) *global_out = sg;
  }
  const int64_t gpr = (cols + gsize - 1) / gsize;
  const int64_t ngroups = rows * gpr;
  const bool rfast = (sr == 1);
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < ngroups;
       t += (int64_t)gridDim.x * blockDim.x) {
    int64_t r, gi;
    if (rfast) { gi = t / rows; r = t - gi * rows; } else { r = t / gpr; gi = t - r * gpr; }
    const int64_t c0 = gi * gsize, c1 = (c0 + gsize < cols) ? c0 + gsize : cols;
    float m = 0.f;
    for (int64_t c = c0; c < c1; ++c) m = fmaxf(m, __builtin_fabsf(load_bf16(x, r * sr + c * sc)));
    const int64_t g = r * gpr + gi;
    if (KIND == KIND_FP8) {
      const float s = fp8_scale_of(m);
      reinterpret_cast<float *>(scales)[g] = s;
      for (int64_t c = c0; c < c1; ++c) q[r * cols + c] = e4m3_encode(load_bf16(x, r * sr + c * sc) / s);
    } else if (KIND == KIND_MX) {
      const int e = mx_exponent(m);
      const float mul = pow2_neg(e);
      reinterpret_cast<uint8_t *>(scales)[g] = (uint8_t)(e + 127);
      for (int64_t c = c0; c < c1; c += 2) {
        uint32_t lo = e2m1_encode(load_bf16(x, r * sr + c * sc) * mul);
        uint32_t hi = e2m1_encode(load_bf16(x, r * sr + (c + 1) * sc) * mul);
        q[(r * cols + c) >> 1] = (uint8_t)(lo | (hi << 4));
      }
    } else {
      const uint8_t sb = e4m3_encode((m / 6.0f) / sg);
      const float d = e4m3_decode(sb) * sg;
      reinterpret_cast<uint8_t *>(scales)[g] = sb;
      for (int64_t c = c0; c < c1; c += 2) {
        uint32_t lo = 0, hi = 0;
        if (d != 0.f) {
          lo = e2m1_encode(load_bf16(x, r * sr + c * sc) / d);
          hi = e2m1_encode(load_bf16(x, r * sr + (c + 1) * sc) / d);
        }
        q[(r * cols + c) >> 1] = (uint8_t)(lo | (hi << 4));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Tile kernel: one workgroup per group_rows x group_cols FP8 tile (128x128
// weight blocks, per-row / per-channel scales over long rows).
// ---------------------------------------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(256) void quant_fp8_tile_kernel(
    const uint16_t *__restrict__ x, int64_t rows, int64_t cols, int64_t sr, int64_t sc,
    int64_t gr, int64_t gc, uint8_t *__restrict__ q, float *__restrict__ scales) {
  __shared__ float sh[4];
  const int64_t ntc = (cols + gc - 1) / gc;
  const int64_t tr = blockIdx.x / ntc, tc = blockIdx.x - tr * ntc;
  const int64_t r0 = tr * gr, c0 = tc * gc;
  const int64_t nr = (r0 + gr < rows ? gr : rows - r0), nc = (c0 + gc < cols ? gc : cols - c0);
  float m = 0.f;
  if (VEC) {
    const int64_t cpr = nc >> 3, total = nr * cpr;
    for (int64_t i = threadIdx.x; i < total; i += blockDim.x) {
      const int64_t r = r0 + i / cpr, c = c0 + (i % cpr) * 8;
      float f[8];
      unpack8(*reinterpret_cast<const uint4 *>(x + r * sr + c), f);
      m = fmaxf(m, amax8(f));
    }
  } else {
    const int64_t total = nr * nc;
    for (int64_t i = threadIdx.x; i < total; i += blockDim.x) {
      int64_t r, c;
      if (sr == 1) { r = r0 + i % nr; c = c0 + i / nr; } else { r = r0 + i / nc; c = c0 + i % nc; }
      m = fmaxf(m, __builtin_fabsf(load_bf16(x, r * sr + c * sc)));
    }
  }
  const float s = fp8_scale_of(block_max(m, sh));
  const float rs = 1.0f / s;
  if (threadIdx.x == 0) scales[blockIdx.x] = s;
  if (VEC) {
    const int64_t cpr = nc >> 3, total = nr * cpr;
    for (int64_t i = threadIdx.x; i < total; i += blockDim.x) {
      const int64_t r = r0 + i / cpr, c = c0 + (i % cpr) * 8;
      float f[8];
      unpack8(*reinterpret_cast<const uint4 *>(x + r * sr + c), f);
      *reinterpret_cast<uint2 *>(q + r * cols + c) = e4m3_div8(f, s, rs);
    }
  } else {
    const int64_t total = nr * nc;
    for (int64_t i = threadIdx.x; i < total; i += blockDim.x) {
      int64_t r, c;
      if (sr == 1) { r = r0 + i % nr; c = c0 + i / nr; } else { r = r0 + i / nc; c = c0 + i % nc; }
      q[r * cols + c] = e4m3_encode(load_bf16(x, r * sr + c * sc) / s);
    }
  }
}

// ---------------------------------------------------------------------------
// Host launchers (validated by capi.hip before they are called).
// ---------------------------------------------------------------------------
static bool vec_ok(const void *x, int64_t cols, int64_t sr, int64_t sc) {
  return sc == 1 && (cols % 8) == 0 && (sr % 8) == 0 &&
         (reinterpret_cast<uintptr_t>(x) % 16) == 0;
}

static int grid_for(int64_t work, int per_block) {
  int64_t g = (work + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > 65535) g = 65535;
  return (int)g;
}

static int partial_blocks(int64_t elems) {
  int64_t g = (elems + 256 * 16 - 1) / (256 * 16);
  if (g < 1) g = 1;
  if (g > kMaxPartials) g = kMaxPartials;
  return (int)g;
}

hipError_t launch_amax_partials(const uint16_t *x, int64_t rows, int64_t cols, int64_t sr,
                                int64_t sc, float *partial, int *nparts, hipStream_t st) {
  const int g = partial_blocks(rows * cols);
  *nparts = g;
  if (vec_ok(x, cols, sr, sc))
    amax_partial_kernel<true><<<g, 256, 0, st>>>(x, rows, cols, sr, sc, partial);
  else
    amax_partial_kernel<false><<<g, 256, 0, st>>>(x, rows, cols, sr, sc, partial);
  return hipGetLastError();
}

hipError_t launch_quant_fp8_tensor(const uint16_t *x, int64_t rows, int64_t cols, int64_t sr,
                                   int64_t sc, uint8_t *q, float *scale, float *partial,
                                   hipStream_t st) {
  int np = 0;
  hipError_t e = launch_amax_partials(x, rows, cols, sr, sc, partial, &np, st);
  if (e != hipSuccess) return e;
  if (vec_ok(x, cols, sr, sc))
    quant_fp8_tensor_kernel<true><<<grid_for(rows * cols / 8, 256 * 4), 256, 0, st>>>(
        x, rows, cols, sr, sc, partial, np, q, scale);
  else
    quant_fp8_tensor_kernel<false><<<grid_for(rows * cols, 256 * 16), 256, 0, st>>>(
        x, rows, cols, sr, sc, partial, np, q, scale);
  return hipGetLastError();
}

template <int KIND, int T>
static void launch_team(const uint16_t *x, int64_t rows, int64_t cols, int64_t sr, uint8_t *q,
                        void *scales, const float *partial, int np, float *gout, hipStream_t st) {
  const int64_t threads = rows * ((cols + 8 * T - 1) / (8 * T)) * T;
  quant_rowgroup_kernel<KIND, T><<<grid_for(threads, 256 * 2), 256, 0, st>>>(
      x, rows, cols, sr, q, scales, partial, np, gout);
}

hipError_t launch_quant_fp8_blocks(const uint16_t *x, int64_t rows, int64_t cols, int64_t sr,
                                   int64_t sc, int64_t gr, int64_t gc, uint8_t *q,
                                   float *scales, hipStream_t st) {
  const bool vec = vec_ok(x, cols, sr, sc);
  if (gr == 1 && vec && (gc == 32 || gc == 64 || gc == 128 || gc == 256)) {
    switch (gc) {
      case 32: launch_team<KIND_FP8, 4>(x, rows, cols, sr, q, scales, nullptr, 0, nullptr, st); break;
      case 64: launch_team<KIND_FP8, 8>(x, rows, cols, sr, q, scales, nullptr, 0, nullptr, st); break;
      case 128: launch_team<KIND_FP8, 16>(x, rows, cols, sr, q, scales, nullptr, 0, nullptr, st); break;
      default: launch_team<KIND_FP8, 32>(x, rows, cols, sr, q, scales, nullptr, 0, nullptr, st); break;
    }
    return hipGetLastError();
  }
  if (gr == 1 && !vec && gc <= 256) {
    const int64_t ngroups = rows * ((cols + gc - 1) / gc);
    quant_group_scalar_kernel<KIND_FP8><<<grid_for(ngroups, 256), 256, 0, st>>>(
        x, rows, cols, sr, sc, gc, q, scales, nullptr, 0, nullptr);
    return hipGetLastError();
  }
  const int64_t tiles = ((rows + gr - 1) / gr) * ((cols + gc - 1) / gc);
  const bool tvec = vec && (gc % 8) == 0;
  if (tvec)
    quant_fp8_tile_kernel<true><<<(unsigned)tiles, 256, 0, st>>>(x, rows, cols, sr, sc, gr, gc, q, scales);
  else
    quant_fp8_tile_kernel<false><<<(unsigned)tiles, 256, 0, st>>>(x, rows, cols, sr, sc, gr, gc, q, scales);
  return hipGetLastError();
}

hipError_t launch_quant_mxfp4(const uint16_t *x, int64_t rows, int64_t cols, int64_t sr,
                              int64_t sc, uint8_t *q, uint8_t *e8m0, hipStream_t st) {
  if (vec_ok(x, cols, sr, sc)) {
    launch_team<KIND_MX, 4>(x, rows, cols, sr, q, e8m0, nullptr, 0, nullptr, st);
  } else {
    const int64_t ngroups = rows * (cols / 32);
    quant_group_scalar_kernel<KIND_MX><<<grid_for(ngroups, 256), 256, 0, st>>>(
        x, rows, cols, sr, sc, 32, q, e8m0, nullptr, 0, nullptr);
  }
  return hipGetLastError();
}

hipError_t launch_quant_nvfp4(const uint16_t *x, int64_t rows, int64_t cols, int64_t sr,
                              int64_t sc, uint8_t *q, uint8_t *e4m3s, float *gscale,
                              float *partial, hipStream_t st) {
  int np = 0;
  hipError_t e = launch_amax_partials(x, rows, cols, sr, sc, partial, &np, st);
  if (e != hipSuccess) return e;
  if (vec_ok(x, cols, sr, sc)) {
    launch_team<KIND_NV, 2>(x, rows, cols, sr, q, e4m3s, partial, np, gscale, st);
  } else {
    const int64_t ngroups = rows * (cols / 16);
    quant_group_scalar_kernel<KIND_NV><<<grid_for(ngroups, 256), 256, 0, st>>>(
        x, rows, cols, sr, sc, 16, q, e4m3s, partial, np, gscale);
  }
  return hipGetLastError();
}

}  // namespace dsl
