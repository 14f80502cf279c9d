// Quantize/pack kernels: bf16 or fp32 -> E4M3 (per-tensor, block-scaled),
// MXFP4 (E2M1 + E8M0 / 32), NVFP4 (E2M1 + E4M3 / 16 + fp32 global).
//
// All kernels read x[r*sr + c*sc] (bf16 or fp32) and write K-major codes
// q[r*C + c] (FP8) or packed nibbles q[r*C/2 + c/2] (FP4).  fp32 sources
// divide with the IEEE division: contiguous rows on the fp32 team kernel
// (quant_f32_rowgroup_kernel), anything else on the strided kernels.  bf16
// code paths, fastest first:
//   * packed path (sc == 1, sr == C, C % 8 == 0, 16-B aligned x, fewer than
//     2^31 chunks; row groups also need C % group == 0): the input is one run
//     of 16-byte chunks and group g is chunks [g*CG, (g+1)*CG), so indices
//     are 32-bit and division-free.  TL lanes share a group (amax by DPP),
//     each holding CG/TL chunks, and every lane keeps several groups' loads
//     in flight;
//   * register tile path (FP8 tiles up to 128x128, vector-aligned rows):
//     one workgroup holds its tile in registers, so x is read once;
//   * team path (vector-aligned rows, any C): a team of T lanes owns one
//     group of 8*T elements of a row;
//   * strided path (anything else, e.g. the reference's B[K,N] given as a
//     contiguous [K,N] tensor): one thread per scale group, threads ordered
//     so that the unit-stride axis is the fast one across lanes.
// Arithmetic is the bit-exact contract of include/dsl_gemm.h (fp32 scales,
// codes of the IEEE quotient x / scale, RNE).  The vector paths encode with
// the gfx950 converters and the corrected reciprocal quotient of common.h
// (quot), which give the same codes; the strided path divides and encodes in
// software.
#include <mutex>

#include "launch.h"
#include "quant_core.h"

namespace dsl {

// ---------------------------------------------------------------------------
// Pass 1 of the per-tensor / NVFP4 quantizers: per-block amax partials.
// ---------------------------------------------------------------------------
template <int V>
__global__ __launch_bounds__(256) void amax_packed_kernel(
    const uint4 *__restrict__ x, uint32_t nchunks, float *__restrict__ partial) {
  __shared__ float sh[4];
  float m = 0.f;
  for (uint32_t base = blockIdx.x * (256u * V); base < nchunks; base += gridDim.x * (256u * V)) {
    uint4 d[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {   // lanes past the end re-read the last chunk
      const uint32_t i = base + v * 256u + threadIdx.x;
      d[v] = x[i < nchunks ? i : nchunks - 1];
    }
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float f[8];
      unpack8(d[v], f);
      m = fmaxf(m, amax8(f));
    }
  }
  m = block_max(m, sh);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

// 8 consecutive source elements as fp32: one 16-byte load of bf16, or two of fp32.
DSL_DEV void load8(const uint16_t *p, float *f) { unpack8(*reinterpret_cast<const uint4 *>(p), f); }
DSL_DEV void load8(const float *p, float *f) {
  const float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
  f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
  f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}

// T = uint16_t (bf16 bits) or float; VEC: rows of whole 8-element chunks,
// 16-byte aligned.
template <bool VEC, typename T>
__global__ __launch_bounds__(256) void amax_partial_kernel(
    const T *__restrict__ x, int64_t rows, int64_t cols, int64_t sr, int64_t sc,
    float *__restrict__ partial) {
  __shared__ float sh[4];
  float m = 0.f;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  if constexpr (VEC) {
    const int64_t cpr = cols >> 3, total = rows * cpr;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
      const int64_t r = i / cpr, c8 = i - r * cpr;
      float f[8];
      load8(x + r * sr + c8 * 8, f);
      m = fmaxf(m, amax8(f));
    }
  } else {
    const int64_t total = rows * cols;
    const bool rfast = (sr == 1);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
      int64_t r, c;
      if (rfast) { c = i / rows; r = i - c * rows; } else { r = i / cols; c = i - r * cols; }
      m = fmaxf(m, __builtin_fabsf(load_in(x, r * sr + c * sc)));
    }
  }
  m = block_max(m, sh);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

// ---------------------------------------------------------------------------
// Packed path.  KIND selects the format; CG = chunks (8 elements) per scale
// group (1 for the per-tensor scale); TL lanes per group, lane k of a team
// holding chunks k, k+TL, ... of it (each load instruction reads whole
// contiguous runs); V groups per lane in flight.
// ---------------------------------------------------------------------------
enum { KIND_FP8 = 0, KIND_MX = 1, KIND_NV = 2, KIND_TENSOR = 3 };

template <int KIND, int CG, int TL, int V>
__global__ __launch_bounds__(256) void quant_packed_kernel(
    const uint4 *__restrict__ x, uint32_t ngroups, uint8_t *__restrict__ q,
    void *__restrict__ scales, const float *__restrict__ partial, int nparts,
    float *__restrict__ scale_out) {
  constexpr int U = CG / TL;           // chunks per lane per group
  constexpr uint32_t GB = 256 / TL;    // groups per block per set
  static_assert(CG % TL == 0, "team must divide the group");
  __shared__ float sh[4];
  float st = 1.f, rt = 1.f;            // per-tensor scale (FP8) / global scale (NVFP4)
  if constexpr (KIND == KIND_TENSOR || KIND == KIND_NV) {
    const float am = reduce_partials(partial, nparts, sh);
    st = KIND == KIND_TENSOR ? fp8_scale_of(am) : nv_global_of(am);
    rt = rcp_approx(st);
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = st;
  }
  const uint32_t k = threadIdx.x % TL;
  for (uint32_t base = blockIdx.x * (GB * V); base < ngroups; base += gridDim.x * (GB * V)) {
    // Lanes past the end read the last group (their team's result is not
    // stored), so the loads need no mask.
    uint4 d[V][U];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const uint32_t g = base + v * GB + threadIdx.x / TL;
      const uint32_t gl = g < ngroups ? g : ngroups - 1;
#pragma unroll
      for (int j = 0; j < U; ++j) d[v][j] = x[gl * CG + k + j * TL];
    }
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const uint32_t g = base + v * GB + threadIdx.x / TL;
      const bool ok = g < ngroups;
      float f[U * 8];
      float m = 0.f;
#pragma unroll
      for (int j = 0; j < U; ++j) {
        unpack8(d[v][j], f + 8 * j);
        m = fmaxf(m, amax8(f + 8 * j));
      }
      if constexpr (KIND != KIND_TENSOR) m = team_max<TL>(m);
      const uint32_t c0 = g * CG + k;
      if constexpr (KIND == KIND_FP8 || KIND == KIND_TENSOR) {
        float s = st, r = rt;
        if constexpr (KIND == KIND_FP8) {
          s = fp8_scale_of(m);
          r = rcp_approx(s);
          if (ok && k == 0) reinterpret_cast<float *>(scales)[g] = s;
        }
        if (ok) {
#pragma unroll
          for (int j = 0; j < U; ++j)
            *reinterpret_cast<uint2 *>(q + (size_t)(c0 + j * TL) * 8) = e4m3_quot8(f + 8 * j, s, r);
        }
      } else if constexpr (KIND == KIND_MX) {
        const int e = mx_exponent(m);
        const float mul = pow2_neg(e);
        if (ok && k == 0) reinterpret_cast<uint8_t *>(scales)[g] = (uint8_t)(e + 127);
        if (ok) {
#pragma unroll
          for (int j = 0; j < U; ++j)
            *reinterpret_cast<uint32_t *>(q + (size_t)(c0 + j * TL) * 4) = e2m1_mul8(f + 8 * j, mul);
        }
      } else {  // KIND_NV
        const uint32_t sb = nv_block_code(m, st, rt);
        const float dd = e4m3_value(sb) * st;
        const float rd = rcp_approx(dd);
        if (ok && k == 0) reinterpret_cast<uint8_t *>(scales)[g] = (uint8_t)sb;
        if (ok) {
#pragma unroll
          for (int j = 0; j < U; ++j)
            *reinterpret_cast<uint32_t *>(q + (size_t)(c0 + j * TL) * 4) =
                dd != 0.f ? e2m1_quot8(f + 8 * j, dd, rd) : 0u;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Per-tensor E4M3, pass 2 (non-packed input).
// ---------------------------------------------------------------------------
template <bool VEC, typename T>
__global__ __launch_bounds__(256) void quant_fp8_tensor_kernel(
    const T *__restrict__ x, int64_t rows, int64_t cols, int64_t sr, int64_t sc,
    const float *__restrict__ partial, int nparts, uint8_t *__restrict__ q,
    float *__restrict__ scale_out) {
  __shared__ float sh[4];
  const float am = reduce_partials(partial, nparts, sh);
  const float scale = VEC ? fp8_scale_of(am) : fp8_scale_ieee(am);
  const float rscale = rcp_approx(scale);
  if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  if constexpr (VEC) {
    const int64_t cpr = cols >> 3, total = rows * cpr;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
      const int64_t r = i / cpr, c8 = i - r * cpr;
      float f[8];
      unpack8(*reinterpret_cast<const uint4 *>(x + r * sr + c8 * 8), f);
      *reinterpret_cast<uint2 *>(q + r * cols + c8 * 8) = e4m3_quot8(f, scale, rscale);
    }
  } else {
    const int64_t total = rows * cols;
    const bool rfast = (sr == 1);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
      int64_t r, c;
      if (rfast) { c = i / rows; r = i - c * rows; } else { r = i / cols; c = i - r * cols; }
      q[r * cols + c] = e4m3_encode(__fdiv_rn(load_in(x, r * sr + c * sc), scale));
    }
  }
}

// ---------------------------------------------------------------------------
// Team path: a team of T lanes (T | 64) owns one group of 8*T consecutive
// elements of a row (rows with any stride, any C).
// ---------------------------------------------------------------------------
template <int KIND, int T>
__global__ __launch_bounds__(256) void quant_rowgroup_kernel(
    const uint16_t *__restrict__ x, int64_t rows, int64_t cols, int64_t sr,
    uint8_t *__restrict__ q, void *__restrict__ scales,
    const float *__restrict__ partial, int nparts, float *__restrict__ global_out) {
  constexpr int G = 8 * T;                      // elements per group
  __shared__ float sh[4];
  float sg = 1.f, rsg = 1.f;
  if (KIND == KIND_NV) {
    sg = nv_global_of(reduce_partials(partial, nparts, sh));
    rsg = rcp_approx(sg);
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
      if (ok) *reinterpret_cast<uint2 *>(q + r * cols + c) = e4m3_quot8(f, s, rcp_approx(s));
    } else if (KIND == KIND_MX) {
      const int e = mx_exponent(m);
      if (lane == 0) reinterpret_cast<uint8_t *>(scales)[g] = (uint8_t)(e + 127);
      if (ok) *reinterpret_cast<uint32_t *>(q + ((r * cols + c) >> 1)) = e2m1_mul8(f, pow2_neg(e));
    } else {  // KIND_NV
      const uint32_t sb = nv_block_code(m, sg, rsg);
      const float d = e4m3_value(sb) * sg;
      if (lane == 0) reinterpret_cast<uint8_t *>(scales)[g] = (uint8_t)sb;
      const uint32_t p = d != 0.f ? e2m1_quot8(f, d, rcp_approx(d)) : 0u;
      if (ok) *reinterpret_cast<uint32_t *>(q + ((r * cols + c) >> 1)) = p;
    }
  }
}

// ---------------------------------------------------------------------------
// fp32 rows (unit column stride, 16-byte aligned rows, C % 8 == 0): a team
// of T lanes (T | 64) owns one group of G = 8*T*U elements of a row, lane k
// holding the runs of 8 consecutive elements k, k + T, ... (two 16-byte
// loads each), so each load instruction of a wave reads whole contiguous
// runs.  KIND_TENSOR: every group uses the per-tensor scale of the partials.
// The scales and codes are those of the strided kernel below: IEEE
// quotients (__fdiv_rn; the reciprocal quotient is only shown exact for
// bf16 sources) encoded by the hardware converters, which return
// e4m3_encode / e2m1_encode of every finite fp32 input.
// ---------------------------------------------------------------------------
DSL_DEV uint2 e4m3_div8(const float *f, float s) {
  uint32_t lo = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(__fdiv_rn(f[0], s), __fdiv_rn(f[1], s), 0, false);
  lo = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(__fdiv_rn(f[2], s), __fdiv_rn(f[3], s), (int)lo, true);
  uint32_t hi = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(__fdiv_rn(f[4], s), __fdiv_rn(f[5], s), 0, false);
  hi = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(__fdiv_rn(f[6], s), __fdiv_rn(f[7], s), (int)hi, true);
  return make_uint2(lo, hi);
}

DSL_DEV uint32_t e2m1_div8(const float *f, float d) {
  uint32_t c = e2m1_pk_into<0>(0u, __fdiv_rn(f[0], d), __fdiv_rn(f[1], d));
  c = e2m1_pk_into<1>(c, __fdiv_rn(f[2], d), __fdiv_rn(f[3], d));
  c = e2m1_pk_into<2>(c, __fdiv_rn(f[4], d), __fdiv_rn(f[5], d));
  return e2m1_pk_into<3>(c, __fdiv_rn(f[6], d), __fdiv_rn(f[7], d));
}

template <int KIND, int T, int U>
__global__ __launch_bounds__(256) void quant_f32_rowgroup_kernel(
    const float *__restrict__ x, int64_t rows, int64_t cols, int64_t sr,
    uint8_t *__restrict__ q, void *__restrict__ scales,
    const float *__restrict__ partial, int nparts, float *__restrict__ scale_out) {
  constexpr int G = 8 * T * U;                  // elements per group
  static_assert(64 % T == 0, "teams within a wave");
  __shared__ float sh[4];
  float st = 1.f;                               // per-tensor scale / NVFP4 global scale
  if constexpr (KIND == KIND_TENSOR || KIND == KIND_NV) {
    const float am = reduce_partials(partial, nparts, sh);
    st = KIND == KIND_TENSOR ? fp8_scale_ieee(am) : nv_global_ieee(am);
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = st;
  }
  const int64_t gpr = (cols + G - 1) / G;       // groups per row
  const int64_t ngroups = rows * gpr;
  const int lane = threadIdx.x % T;
  const int64_t team0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / T;
  const int64_t nteams = (int64_t)gridDim.x * blockDim.x / T;
  for (int64_t g = team0; g < ngroups; g += nteams) {   // uniform across a team
    const int64_t r = g / gpr, gi = g - r * gpr;
    float f[U][8];
    float m = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = gi * G + (int64_t)(u * T + lane) * 8;
      if (c < cols) {
        load8(x + r * sr + c, f[u]);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) f[u][j] = 0.f;
      }
      m = fmaxf(m, amax8(f[u]));
    }
    if constexpr (KIND != KIND_TENSOR) {
#pragma unroll
      for (int o = 1; o < T; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
    }
    float s = st, d = 0.f, mul = 1.f;
    if constexpr (KIND == KIND_FP8) {
      s = fp8_scale_ieee(m);
      if (lane == 0) reinterpret_cast<float *>(scales)[g] = s;
    } else if constexpr (KIND == KIND_MX) {
      const int e = mx_exponent(m);
      mul = pow2_neg(e);
      if (lane == 0) reinterpret_cast<uint8_t *>(scales)[g] = (uint8_t)(e + 127);
    } else if constexpr (KIND == KIND_NV) {
      const uint8_t sb = e4m3_encode(__fdiv_rn(__fdiv_rn(m, 6.0f), st));
      d = e4m3_decode(sb) * st;
      if (lane == 0) reinterpret_cast<uint8_t *>(scales)[g] = sb;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = gi * G + (int64_t)(u * T + lane) * 8;
      if (c >= cols) continue;
      if constexpr (KIND == KIND_FP8 || KIND == KIND_TENSOR) {
        *reinterpret_cast<uint2 *>(q + r * cols + c) = e4m3_div8(f[u], s);
      } else if constexpr (KIND == KIND_MX) {
        *reinterpret_cast<uint32_t *>(q + ((r * cols + c) >> 1)) = e2m1_mul8(f[u], mul);
      } else {
        *reinterpret_cast<uint32_t *>(q + ((r * cols + c) >> 1)) = d != 0.f ? e2m1_div8(f[u], d) : 0u;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Strided path: one thread per scale group (group_rows == 1 groups only).
// ---------------------------------------------------------------------------
// Every division here is the IEEE one (__fdiv_rn), for bf16 and fp32 sources.
template <int KIND, typename T>
__global__ __launch_bounds__(256) void quant_group_scalar_kernel(
    const T *__restrict__ x, int64_t rows, int64_t cols, int64_t sr, int64_t sc,
    int64_t gsize, uint8_t *__restrict__ q, void *__restrict__ scales,
    const float *__restrict__ partial, int nparts, float *__restrict__ global_out) {
  __shared__ float sh[4];
  float sg = 1.f;
  if (KIND == KIND_NV) {
    sg = nv_global_ieee(reduce_partials(partial, nparts, sh));
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
    for (int64_t c = c0; c < c1; ++c) m = fmaxf(m, __builtin_fabsf(load_in(x, r * sr + c * sc)));
    const int64_t g = r * gpr + gi;
    if (KIND == KIND_FP8) {
      const float s = fp8_scale_ieee(m);
      reinterpret_cast<float *>(scales)[g] = s;
      for (int64_t c = c0; c < c1; ++c)
        q[r * cols + c] = e4m3_encode(__fdiv_rn(load_in(x, r * sr + c * sc), s));
    } else if (KIND == KIND_MX) {
      const int e = mx_exponent(m);
      const float mul = pow2_neg(e);
      reinterpret_cast<uint8_t *>(scales)[g] = (uint8_t)(e + 127);
      for (int64_t c = c0; c < c1; c += 2) {
        uint32_t lo = e2m1_encode(load_in(x, r * sr + c * sc) * mul);
        uint32_t hi = e2m1_encode(load_in(x, r * sr + (c + 1) * sc) * mul);
        q[(r * cols + c) >> 1] = (uint8_t)(lo | (hi << 4));
      }
    } else {
      const uint8_t sb = e4m3_encode(__fdiv_rn(__fdiv_rn(m, 6.0f), sg));
      const float d = e4m3_decode(sb) * sg;
      reinterpret_cast<uint8_t *>(scales)[g] = sb;
      for (int64_t c = c0; c < c1; c += 2) {
        uint32_t lo = 0, hi = 0;
        if (d != 0.f) {
          lo = e2m1_encode(__fdiv_rn(load_in(x, r * sr + c * sc), d));
          hi = e2m1_encode(__fdiv_rn(load_in(x, r * sr + (c + 1) * sc), d));
        }
        q[(r * cols + c) >> 1] = (uint8_t)(lo | (hi << 4));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Register tile path: one workgroup per gr x gc FP8 tile with gr, gc <= 128
// and gc % 8 == 0 (128x128 weight blocks).  Lane t holds chunk t % 16 of rows
// t / 16 + 16 j (j < 8) in registers, so the tile is read from HBM once.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void quant_fp8_tile_reg_kernel(
    const uint16_t *__restrict__ x, int64_t rows, int64_t cols, int64_t sr, int gr, int gc,
    uint8_t *__restrict__ q, float *__restrict__ scales) {
  __shared__ float sh[4];
  const int64_t ntc = (cols + gc - 1) / gc;
  const int64_t tr = blockIdx.x / ntc, tc = blockIdx.x - tr * ntc;
  const int64_t r0 = tr * gr, c0 = tc * gc;
  const int nr = (int)(r0 + gr < rows ? gr : rows - r0), nc = (int)(c0 + gc < cols ? gc : cols - c0);
  const int cc = threadIdx.x & 15, rr = threadIdx.x >> 4;
  const bool cok = cc * 8 < nc;
  uint4 d[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = rr + 16 * j;
    d[j] = (cok && r < nr) ? *reinterpret_cast<const uint4 *>(x + (r0 + r) * sr + c0 + cc * 8)
                           : make_uint4(0, 0, 0, 0);
  }
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float f[8];
    unpack8(d[j], f);
    m = fmaxf(m, amax8(f));
  }
  const float s = fp8_scale_of(block_max(m, sh));
  const float rs = rcp_approx(s);
  if (threadIdx.x == 0) scales[blockIdx.x] = s;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = rr + 16 * j;
    float f[8];
    unpack8(d[j], f);
    if (cok && r < nr) *reinterpret_cast<uint2 *>(q + (r0 + r) * cols + c0 + cc * 8) = e4m3_quot8(f, s, rs);
  }
}

// Wide row groups (1 x gc, gc up to 32768, e.g. one scale per row): one
// workgroup per group, thread t holding chunks t + 256 j of it in registers.
template <int CPL>
__global__ __launch_bounds__(256) void quant_fp8_wide_kernel(
    const uint16_t *__restrict__ x, int64_t cols, int64_t sr, int gc, uint8_t *__restrict__ q,
    float *__restrict__ scales) {
  __shared__ float sh[4];
  const int64_t gpr = (cols + gc - 1) / gc;
  const int64_t r = blockIdx.x / gpr, gi = blockIdx.x - r * gpr;
  const int64_t c0 = gi * gc;
  const int nch = (int)((c0 + gc < cols ? gc : cols - c0) >> 3);
  const uint16_t *xr = x + r * sr + c0;
  uint4 d[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = threadIdx.x + 256 * j;
    d[j] = c < nch ? reinterpret_cast<const uint4 *>(xr)[c] : make_uint4(0, 0, 0, 0);
  }
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    float f[8];
    unpack8(d[j], f);
    m = fmaxf(m, amax8(f));
  }
  const float s = fp8_scale_of(block_max(m, sh));
  const float rs = rcp_approx(s);
  if (threadIdx.x == 0) scales[blockIdx.x] = s;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = threadIdx.x + 256 * j;
    if (c < nch) {
      float f[8];
      unpack8(d[j], f);
      *reinterpret_cast<uint2 *>(q + r * cols + c0 + (int64_t)c * 8) = e4m3_quot8(f, s, rs);
    }
  }
}

// Row groups of 264..2048 elements: one wave per group (four per
// workgroup), lane l holding chunks l + 64 j, the amax by wave reduction
// alone.  A workgroup per group left 3/4 of its threads idle at 1 x 512 and
// waited on a barrier for each group.  Same arithmetic as the wide kernel,
// so the same codes and scales.
template <int CPL>
__global__ __launch_bounds__(256) void quant_fp8_wavegroup_kernel(
    const uint16_t *__restrict__ x, int64_t cols, int64_t sr, int gc, int64_t ngroups,
    uint8_t *__restrict__ q, float *__restrict__ scales) {
  const int64_t g = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (g >= ngroups) return;                       // whole waves: no barrier below
  const int lane = threadIdx.x & 63;
  const int64_t gpr = (cols + gc - 1) / gc;
  const int64_t r = g / gpr, gi = g - r * gpr;
  const int64_t c0 = gi * gc;
  const int nch = (int)((c0 + gc < cols ? gc : cols - c0) >> 3);
  const uint16_t *xr = x + r * sr + c0;
  uint4 d[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    d[j] = c < nch ? reinterpret_cast<const uint4 *>(xr)[c] : make_uint4(0, 0, 0, 0);
  }
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    float f[8];
    unpack8(d[j], f);
    m = fmaxf(m, amax8(f));
  }
  const float s = fp8_scale_of(wave_max(m));
  const float rs = rcp_approx(s);
  if (lane == 0) scales[g] = s;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    if (c < nch) {
      float f[8];
      unpack8(d[j], f);
      *reinterpret_cast<uint2 *>(q + r * cols + c0 + (int64_t)c * 8) = e4m3_quot8(f, s, rs);
    }
  }
}

// One workgroup per gr x gc FP8 tile of any size (two reads of the tile).
// VEC (16-byte bf16 rows) divides by the reciprocal quotient; the other path
// divides with __fdiv_rn and serves fp32 sources too (T = float).
template <bool VEC, typename T>
__global__ __launch_bounds__(256) void quant_fp8_tile_kernel(
    const T *__restrict__ x, int64_t rows, int64_t cols, int64_t sr, int64_t sc,
    int64_t gr, int64_t gc, uint8_t *__restrict__ q, float *__restrict__ scales) {
  __shared__ float sh[4];
  const int64_t ntc = (cols + gc - 1) / gc;
  const int64_t tr = blockIdx.x / ntc, tc = blockIdx.x - tr * ntc;
  const int64_t r0 = tr * gr, c0 = tc * gc;
  const int64_t nr = (r0 + gr < rows ? gr : rows - r0), nc = (c0 + gc < cols ? gc : cols - c0);
  float m = 0.f;
  if constexpr (VEC) {
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
      m = fmaxf(m, __builtin_fabsf(load_in(x, r * sr + c * sc)));
    }
  }
  const float am = block_max(m, sh);
  const float s = VEC ? fp8_scale_of(am) : fp8_scale_ieee(am);
  if (threadIdx.x == 0) scales[blockIdx.x] = s;
  if constexpr (VEC) {
    const float rs = rcp_approx(s);
    const int64_t cpr = nc >> 3, total = nr * cpr;
    for (int64_t i = threadIdx.x; i < total; i += blockDim.x) {
      const int64_t r = r0 + i / cpr, c = c0 + (i % cpr) * 8;
      float f[8];
      unpack8(*reinterpret_cast<const uint4 *>(x + r * sr + c), f);
      *reinterpret_cast<uint2 *>(q + r * cols + c) = e4m3_quot8(f, s, rs);
    }
  } else {
    const int64_t total = nr * nc;
    for (int64_t i = threadIdx.x; i < total; i += blockDim.x) {
      int64_t r, c;
      if (sr == 1) { r = r0 + i % nr; c = c0 + i / nr; } else { r = r0 + i / nc; c = c0 + i % nc; }
      q[r * cols + c] = e4m3_encode(__fdiv_rn(load_in(x, r * sr + c * sc), s));
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

// One run of 16-byte chunks with 32-bit chunk indices (group = elements per
// scale group; the input must hold whole groups).
static bool packed_ok(const void *x, int64_t rows, int64_t cols, int64_t sr, int64_t sc,
                      int64_t group) {
  return vec_ok(x, cols, sr, sc) && (sr == cols || rows == 1) && (cols % group) == 0 &&
         rows * cols / 8 < ((int64_t)1 << 31);
}

static int grid_for(int64_t work, int per_block) {
  int64_t g = (work + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > 65535) g = 65535;
  return (int)g;
}

// fp32 rows the vector fp32 kernels take: unit column stride, whole 8-element
// runs, 16-byte aligned rows.
static bool f32_vec_ok(const void *x, int64_t cols, int64_t sr, int64_t sc) {
  return sc == 1 && (cols % 8) == 0 && (sr % 4) == 0 &&
         (reinterpret_cast<uintptr_t>(x) % 16) == 0;
}

template <int KIND, int T, int U>
static void launch_f32_rows(const float *x, int64_t rows, int64_t cols, int64_t sr, uint8_t *q,
                            void *scales, const float *partial, int np, float *sout, hipStream_t st) {
  constexpr int G = 8 * T * U;
  const int64_t threads = rows * ((cols + G - 1) / G) * T;
  quant_f32_rowgroup_kernel<KIND, T, U><<<grid_for(threads, 256 * 2), 256, 0, st>>>(
      x, rows, cols, sr, q, scales, partial, np, sout);
}

template <int KIND, int CG, int TL, int V>
static void launch_packed(const uint16_t *x, int64_t rows, int64_t cols, uint8_t *q, void *scales,
                          const float *partial, int np, float *sout, hipStream_t st) {
  const uint32_t ngroups = (uint32_t)(rows * cols / (8 * CG));
  const int g = grid_for(ngroups, (256 / TL) * V);
  quant_packed_kernel<KIND, CG, TL, V><<<g, 256, 0, st>>>(
      reinterpret_cast<const uint4 *>(x), ngroups, q, scales, partial, np, sout);
}

static int partial_blocks(int64_t elems) {
  int64_t g = (elems + 256 * 16 - 1) / (256 * 16);
  if (g < 1) g = 1;
  if (g > kMaxPartials) g = kMaxPartials;
  return (int)g;
}

// fp32 sources (f32) always take the strided kernels.
static hipError_t launch_amax_partials(const void *xv, bool f32, int64_t rows, int64_t cols,
                                       int64_t sr, int64_t sc, float *partial, int *nparts,
                                       hipStream_t st) {
  if (f32) {
    *nparts = partial_blocks(rows * cols);
    if (f32_vec_ok(xv, cols, sr, sc))
      amax_partial_kernel<true, float><<<*nparts, 256, 0, st>>>(static_cast<const float *>(xv), rows,
                                                                  cols, sr, sc, partial);
    else
      amax_partial_kernel<false, float><<<*nparts, 256, 0, st>>>(static_cast<const float *>(xv), rows,
                                                                   cols, sr, sc, partial);
    return hipGetLastError();
  }
  const uint16_t *x = static_cast<const uint16_t *>(xv);
  if (packed_ok(x, rows, cols, sr, sc, 8)) {
    const uint32_t n = (uint32_t)(rows * cols / 8);
    const int g = (int)((n + 256 * 4 - 1) / (256 * 4) < kMaxPartials ? (n + 256 * 4 - 1) / (256 * 4)
                                                                      : kMaxPartials);
    *nparts = g < 1 ? 1 : g;
    amax_packed_kernel<4><<<*nparts, 256, 0, st>>>(reinterpret_cast<const uint4 *>(x), n, partial);
    return hipGetLastError();
  }
  const int g = partial_blocks(rows * cols);
  *nparts = g;
  if (vec_ok(x, cols, sr, sc))
    amax_partial_kernel<true, uint16_t><<<g, 256, 0, st>>>(x, rows, cols, sr, sc, partial);
  else
    amax_partial_kernel<false, uint16_t><<<g, 256, 0, st>>>(x, rows, cols, sr, sc, partial);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Library-held amax partials for the entry point that allocates nothing
// (dsl_quant_fp8_tensor_noalloc).  One copy per GPU, for the life of the
// process; pass 1 writes every partial that pass 2 reads, so nothing in it
// has to start at zero.  Host code reaches it through the address that
// hipGetSymbolAddress returns on each device, never through its name.
// ---------------------------------------------------------------------------
static __device__ __align__(256) float scratch[kMaxPartials];

float *quant_scratch(hipError_t *err) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static float *ptr[kMaxDevices] = {};
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess && (dev < 0 || dev >= kMaxDevices)) e = hipErrorInvalidDevice;
  if (e != hipSuccess) {
    *err = e;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));   // with `dev` current
    if (e != hipSuccess || !p) {
      *err = e != hipSuccess ? e : hipErrorInvalidSymbol;
      return nullptr;
    }
    ptr[dev] = static_cast<float *>(p);
  }
  *err = hipSuccess;
  return ptr[dev];
}

size_t quant_scratch_bytes() { return sizeof(scratch); }

__global__ void empty_scale_kernel(float *scale) { *scale = kScaleFloor; }

hipError_t launch_empty_scale(float *scale, hipStream_t st) {
  empty_scale_kernel<<<1, 1, 0, st>>>(scale);
  return hipGetLastError();
}

hipError_t launch_quant_fp8_tensor(const void *xv, bool f32, int64_t rows, int64_t cols,
                                   int64_t sr, int64_t sc, uint8_t *q, float *scale,
                                   float *partial, hipStream_t st) {
  int np = 0;
  hipError_t e = launch_amax_partials(xv, f32, rows, cols, sr, sc, partial, &np, st);
  if (e != hipSuccess) return e;
  if (f32) {
    if (f32_vec_ok(xv, cols, sr, sc))
      launch_f32_rows<KIND_TENSOR, 1, 1>(static_cast<const float *>(xv), rows, cols, sr, q, nullptr,
                                         partial, np, scale, st);
    else
      quant_fp8_tensor_kernel<false, float><<<grid_for(rows * cols, 256 * 16), 256, 0, st>>>(
          static_cast<const float *>(xv), rows, cols, sr, sc, partial, np, q, scale);
    return hipGetLastError();
  }
  const uint16_t *x = static_cast<const uint16_t *>(xv);
  if (packed_ok(x, rows, cols, sr, sc, 8))
    launch_packed<KIND_TENSOR, 1, 1, 4>(x, rows, cols, q, nullptr, partial, np, scale, st);
  else if (vec_ok(x, cols, sr, sc))
    quant_fp8_tensor_kernel<true, uint16_t><<<grid_for(rows * cols / 8, 256 * 4), 256, 0, st>>>(
        x, rows, cols, sr, sc, partial, np, q, scale);
  else
    quant_fp8_tensor_kernel<false, uint16_t><<<grid_for(rows * cols, 256 * 16), 256, 0, st>>>(
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

hipError_t launch_quant_fp8_blocks(const void *xv, bool f32, int64_t rows, int64_t cols,
                                   int64_t sr, int64_t sc, int64_t gr, int64_t gc, uint8_t *q,
                                   float *scales, hipStream_t st) {
  const int64_t tiles = ((rows + gr - 1) / gr) * ((cols + gc - 1) / gc);
  if (f32) {
    const float *xf = static_cast<const float *>(xv);
    if (gr == 1 && f32_vec_ok(xv, cols, sr, sc) &&
        (gc == 32 || gc == 64 || gc == 128 || gc == 256)) {
      switch (gc) {
        case 32: launch_f32_rows<KIND_FP8, 4, 1>(xf, rows, cols, sr, q, scales, nullptr, 0, nullptr, st); break;
        case 64: launch_f32_rows<KIND_FP8, 8, 1>(xf, rows, cols, sr, q, scales, nullptr, 0, nullptr, st); break;
        case 128: launch_f32_rows<KIND_FP8, 16, 1>(xf, rows, cols, sr, q, scales, nullptr, 0, nullptr, st); break;
        default: launch_f32_rows<KIND_FP8, 16, 2>(xf, rows, cols, sr, q, scales, nullptr, 0, nullptr, st); break;
      }
      return hipGetLastError();
    }
    if (gr == 1 && gc <= 256)
      quant_group_scalar_kernel<KIND_FP8, float><<<grid_for(tiles, 256), 256, 0, st>>>(
          xf, rows, cols, sr, sc, gc, q, scales, nullptr, 0, nullptr);
    else
      quant_fp8_tile_kernel<false, float><<<(unsigned)tiles, 256, 0, st>>>(xf, rows, cols, sr, sc, gr,
                                                                           gc, q, scales);
    return hipGetLastError();
  }
  const uint16_t *x = static_cast<const uint16_t *>(xv);
  const bool vec = vec_ok(x, cols, sr, sc);
  const bool row_team = gc == 32 || gc == 64 || gc == 128 || gc == 256;
  if (gr == 1 && row_team && packed_ok(x, rows, cols, sr, sc, gc)) {
    switch (gc) {
      case 32: launch_packed<KIND_FP8, 4, 4, 4>(x, rows, cols, q, scales, nullptr, 0, nullptr, st); break;
      case 64: launch_packed<KIND_FP8, 8, 4, 2>(x, rows, cols, q, scales, nullptr, 0, nullptr, st); break;
      case 128: launch_packed<KIND_FP8, 16, 8, 2>(x, rows, cols, q, scales, nullptr, 0, nullptr, st); break;
      default: launch_packed<KIND_FP8, 32, 8, 1>(x, rows, cols, q, scales, nullptr, 0, nullptr, st); break;
    }
    return hipGetLastError();
  }
  if (gr == 1 && vec && row_team) {
    switch (gc) {
      case 32: launch_team<KIND_FP8, 4>(x, rows, cols, sr, q, scales, nullptr, 0, nullptr, st); break;
      case 64: launch_team<KIND_FP8, 8>(x, rows, cols, sr, q, scales, nullptr, 0, nullptr, st); break;
      case 128: launch_team<KIND_FP8, 16>(x, rows, cols, sr, q, scales, nullptr, 0, nullptr, st); break;
      default: launch_team<KIND_FP8, 32>(x, rows, cols, sr, q, scales, nullptr, 0, nullptr, st); break;
    }
    return hipGetLastError();
  }
  if (gr == 1 && !vec && gc <= 256) {
    quant_group_scalar_kernel<KIND_FP8, uint16_t><<<grid_for(tiles, 256), 256, 0, st>>>(
        x, rows, cols, sr, sc, gc, q, scales, nullptr, 0, nullptr);
    return hipGetLastError();
  }
  const bool tvec = vec && (gc % 8) == 0;
  if (gr == 1 && tvec && gc > 256 && gc <= 2048) {
    const unsigned g = (unsigned)((tiles + 3) / 4);
    if (gc <= 512)
      quant_fp8_wavegroup_kernel<1><<<g, 256, 0, st>>>(x, cols, sr, (int)gc, tiles, q, scales);
    else if (gc <= 1024)
      quant_fp8_wavegroup_kernel<2><<<g, 256, 0, st>>>(x, cols, sr, (int)gc, tiles, q, scales);
    else
      quant_fp8_wavegroup_kernel<4><<<g, 256, 0, st>>>(x, cols, sr, (int)gc, tiles, q, scales);
    return hipGetLastError();
  }
  if (gr == 1 && tvec && gc > 128 && gc <= 32768) {
    const int per = (int)((gc / 8 + 255) / 256);
    const unsigned g = (unsigned)tiles;
    if (per <= 1) quant_fp8_wide_kernel<1><<<g, 256, 0, st>>>(x, cols, sr, (int)gc, q, scales);
    else if (per <= 2) quant_fp8_wide_kernel<2><<<g, 256, 0, st>>>(x, cols, sr, (int)gc, q, scales);
    else if (per <= 4) quant_fp8_wide_kernel<4><<<g, 256, 0, st>>>(x, cols, sr, (int)gc, q, scales);
    else if (per <= 8) quant_fp8_wide_kernel<8><<<g, 256, 0, st>>>(x, cols, sr, (int)gc, q, scales);
    else quant_fp8_wide_kernel<16><<<g, 256, 0, st>>>(x, cols, sr, (int)gc, q, scales);
    return hipGetLastError();
  }
  if (tvec && gr <= 128 && gc <= 128)
    quant_fp8_tile_reg_kernel<<<(unsigned)tiles, 256, 0, st>>>(x, rows, cols, sr, (int)gr, (int)gc, q, scales);
  else if (tvec)
    quant_fp8_tile_kernel<true, uint16_t><<<(unsigned)tiles, 256, 0, st>>>(x, rows, cols, sr, sc, gr, gc, q, scales);
  else
    quant_fp8_tile_kernel<false, uint16_t><<<(unsigned)tiles, 256, 0, st>>>(x, rows, cols, sr, sc, gr, gc, q, scales);
  return hipGetLastError();
}

hipError_t launch_quant_mxfp4(const void *xv, bool f32, int64_t rows, int64_t cols, int64_t sr,
                              int64_t sc, uint8_t *q, uint8_t *e8m0, hipStream_t st) {
  if (f32) {
    if (f32_vec_ok(xv, cols, sr, sc))
      launch_f32_rows<KIND_MX, 4, 1>(static_cast<const float *>(xv), rows, cols, sr, q, e8m0,
                                     nullptr, 0, nullptr, st);
    else
      quant_group_scalar_kernel<KIND_MX, float><<<grid_for(rows * (cols / 32), 256), 256, 0, st>>>(
          static_cast<const float *>(xv), rows, cols, sr, sc, 32, q, e8m0, nullptr, 0, nullptr);
    return hipGetLastError();
  }
  const uint16_t *x = static_cast<const uint16_t *>(xv);
  if (packed_ok(x, rows, cols, sr, sc, 32)) {
    launch_packed<KIND_MX, 4, 4, 4>(x, rows, cols, q, e8m0, nullptr, 0, nullptr, st);
  } else if (vec_ok(x, cols, sr, sc)) {
    launch_team<KIND_MX, 4>(x, rows, cols, sr, q, e8m0, nullptr, 0, nullptr, st);
  } else {
    const int64_t ngroups = rows * (cols / 32);
    quant_group_scalar_kernel<KIND_MX, uint16_t><<<grid_for(ngroups, 256), 256, 0, st>>>(
        x, rows, cols, sr, sc, 32, q, e8m0, nullptr, 0, nullptr);
  }
  return hipGetLastError();
}

hipError_t launch_quant_nvfp4(const void *xv, bool f32, int64_t rows, int64_t cols, int64_t sr,
                              int64_t sc, uint8_t *q, uint8_t *e4m3s, float *gscale,
                              float *partial, hipStream_t st) {
  int np = 0;
  hipError_t e = launch_amax_partials(xv, f32, rows, cols, sr, sc, partial, &np, st);
  if (e != hipSuccess) return e;
  if (f32) {
    if (f32_vec_ok(xv, cols, sr, sc))
      launch_f32_rows<KIND_NV, 2, 1>(static_cast<const float *>(xv), rows, cols, sr, q, e4m3s,
                                     partial, np, gscale, st);
    else
      quant_group_scalar_kernel<KIND_NV, float><<<grid_for(rows * (cols / 16), 256), 256, 0, st>>>(
          static_cast<const float *>(xv), rows, cols, sr, sc, 16, q, e4m3s, partial, np, gscale);
    return hipGetLastError();
  }
  const uint16_t *x = static_cast<const uint16_t *>(xv);
  if (packed_ok(x, rows, cols, sr, sc, 16)) {
    launch_packed<KIND_NV, 2, 1, 2>(x, rows, cols, q, e4m3s, partial, np, gscale, st);
  } else if (vec_ok(x, cols, sr, sc)) {
    launch_team<KIND_NV, 2>(x, rows, cols, sr, q, e4m3s, partial, np, gscale, st);
  } else {
    const int64_t ngroups = rows * (cols / 16);
    quant_group_scalar_kernel<KIND_NV, uint16_t><<<grid_for(ngroups, 256), 256, 0, st>>>(
        x, rows, cols, sr, sc, 16, q, e4m3s, partial, np, gscale);
  }
  return hipGetLastError();
}

}  // namespace dsl
