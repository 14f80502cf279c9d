// Fused quantize producers: RMSNorm and SwiGLU whose bf16 results are
// quantized in registers into FP8 1x128 groups or MXFP4 blocks, so the
// activation never makes the round trip bf16 -> HBM -> quantizer.
//
// Lanes hold whole 16-byte chunks (8 elements) and the lanes of one scale
// group sit in one DPP row (FP8 1x128: 16 chunks) or quad (MXFP4: 4), so the
// group amax is a team_max; see each kernel for its lane -> chunk map.
//
// Values are those of the unfused reference operators rounded to bf16:
//   RMSNorm (triton/normalization/norm_kernels.py:21-30):
//     ms = sum(x^2) / N, r = 1 / sqrt(ms + eps), y = (x * r) * w
//   SwiGLU (triton/activations/activation_kernels.py:28-36, input
//   [rows, 2H] = gate | up):  y = (g * sigmoid(g)) * u, sigmoid = 1/(1+e^-g)
// all in fp32 (the sigmoid from the hardware 2^x and reciprocal), then RNE
// to bf16 (the reference stores into an x-dtype tensor).  The quantization
// of those bf16 values is the contract of quant.hip, bit for bit.
#include "launch.h"
#include "quant_core.h"

namespace dsl {

DSL_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// y[e] rounded to bf16 (nearest even) and widened back, two at a time by
// the hardware pack (pack_bf16x2: the same bits as f32_to_bf16).
DSL_DEV void round_bf16x8(float *y) {
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const uint32_t pk = pack_bf16x2(y[e], y[e + 1]);
    y[e] = u2f(pk << 16);
    y[e + 1] = u2f(pk & 0xffff0000u);
  }
}

// 1 / (1 + e^-g) from the hardware 2^x and reciprocal (each within about an
// ulp): a few ulp of fp32 from the IEEE form, far below the bf16 rounding of
// the product; the SwiGLU test bounds the bf16 outcome.  Saturates cleanly:
// e^-g = inf gives 0, e^-g = 0 gives 1.
DSL_DEV float sigmoid_fast(float g) {
  const float e = __builtin_amdgcn_exp2f(-g * 1.44269504088896341f);
  return __builtin_amdgcn_rcpf(1.0f + e);
}

// Quantize 8 bf16-valued floats of chunk c of a row (team of TL lanes per
// group: FP8 1x128 -> 16 chunks per group, MXFP4 -> 4) and store codes and,
// from the team's first lane, the group scale.
template <int QF, int TL>
DSL_DEV void emit_chunk(const FusedArgs &p, int row, int c, bool ok, bool lead, const float *y) {
  const int ngr = QF == QF_FP8_G128 ? (p.cols + 127) / 128 : p.cols / 32;
  if constexpr (QF == QF_FP8_G128) {
    const float s = fp8_scale_of(team_max<TL>(amax8(y)));
    if (ok && lead) reinterpret_cast<float *>(p.scales)[(int64_t)row * ngr + (c >> 4)] = s;
    if (ok)
      *reinterpret_cast<uint2 *>(p.q + (int64_t)row * p.cols + (int64_t)c * 8) =
          e4m3_quot8(y, s, rcp_approx(s));
  } else {
    const int e = mx_exponent(team_max<TL>(amax8(y)));
    if (ok && lead)
      reinterpret_cast<uint8_t *>(p.scales)[(int64_t)row * ngr + (c >> 2)] = (uint8_t)(e + 127);
    if (ok)
      *reinterpret_cast<uint32_t *>(p.q + (int64_t)row * (p.cols / 2) + (int64_t)c * 4) =
          e2m1_mul8(y, pow2_neg(e));
  }
}

DSL_DEV void store_y(const FusedArgs &p, int row, int c, const float *y) {
  uint4 o;
  o.x = (f2u(y[0]) >> 16) | (f2u(y[1]) & 0xffff0000u);
  o.y = (f2u(y[2]) >> 16) | (f2u(y[3]) & 0xffff0000u);
  o.z = (f2u(y[4]) >> 16) | (f2u(y[5]) & 0xffff0000u);
  o.w = (f2u(y[6]) >> 16) | (f2u(y[7]) & 0xffff0000u);
  reinterpret_cast<uint4 *>(p.y + (int64_t)row * p.ldy)[c] = o;
}

// RMSNorm: one workgroup per row, thread t holding chunks t + 256 j in
// registers (the sum of squares needs the whole row before any output).
// A group's 16 (FP8) or 4 (MXFP4) chunks are consecutive threads of one wave.
template <int QF, int CPL, bool WF32>
__global__ __launch_bounds__(256) void rmsnorm_quant_kernel(const FusedArgs p) {
  __shared__ float sh[4];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int nch = p.cols >> 3;
  const uint16_t *xr = p.x + (int64_t)row * p.ldx;
  uint4 xa[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = tid + 256 * j;
    xa[j] = c < nch ? reinterpret_cast<const uint4 *>(xr)[c] : make_uint4(0, 0, 0, 0);
  }
  // the weights are loaded with the row (packed), so their latency hides
  // behind the row's instead of following the sum-of-squares barrier
  uint4 wa[CPL][WF32 ? 2 : 1];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = tid + 256 * j;
#pragma unroll
    for (int h = 0; h < (WF32 ? 2 : 1); ++h)
      wa[j][h] = c < nch ? reinterpret_cast<const uint4 *>(p.w)[(WF32 ? 2 : 1) * c + h]
                         : make_uint4(0, 0, 0, 0);
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    float f[8];
    unpack8(xa[j], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) sh[tid >> 6] = ss;
  __syncthreads();
  ss = (sh[0] + sh[1]) + (sh[2] + sh[3]);
  const float rinv = 1.0f / __builtin_sqrtf(ss / (float)p.cols + p.eps);
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = tid + 256 * j;
    const bool ok = c < nch;
    float y[8], w[8];
    unpack8(xa[j], y);
    if constexpr (WF32) {
      const uint4 a = wa[j][0], b = wa[j][WF32 ? 1 : 0];
      w[0] = __uint_as_float(a.x); w[1] = __uint_as_float(a.y);
      w[2] = __uint_as_float(a.z); w[3] = __uint_as_float(a.w);
      w[4] = __uint_as_float(b.x); w[5] = __uint_as_float(b.y);
      w[6] = __uint_as_float(b.z); w[7] = __uint_as_float(b.w);
    } else {
      unpack8(wa[j][0], w);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = (y[e] * rinv) * w[e];
    round_bf16x8(y);
    if (p.y && ok) store_y(p, row, c, y);
    if constexpr (QF == QF_FP8_G128) emit_chunk<QF, 16>(p, row, c, ok, (tid & 15) == 0, y);
    else emit_chunk<QF, 4>(p, row, c, ok, (tid & 3) == 0, y);
  }
}

// SwiGLU: elementwise, so the rows stream through like the packed quantizer:
// group g (row g / gpr, group g % gpr of it) is handled by a team of TL
// lanes, lane k holding chunks k, k + TL, ... (U = group chunks / TL), and
// each lane keeps V groups' loads in flight.
template <int QF, int TL, int V>
__global__ __launch_bounds__(256) void swiglu_quant_kernel(const FusedArgs p, uint32_t ngroups,
                                                           uint32_t gpr) {
  constexpr int CG = QF == QF_FP8_G128 ? 16 : 4;   // chunks per group
  constexpr int U = CG / TL;
  constexpr uint32_t GB = 256 / TL;                // groups per block per set
  const int nch = p.cols >> 3;
  const int k = threadIdx.x % TL;
  for (uint32_t base = blockIdx.x * (GB * V); base < ngroups; base += gridDim.x * (GB * V)) {
    uint4 ga[V][U], ua[V][U];
    int rows_[V], c0[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      uint32_t g = base + v * GB + threadIdx.x / TL;
      g = g < ngroups ? g : ngroups - 1;             // past the end: redo the last group
      rows_[v] = (int)(g / gpr);
      c0[v] = (int)(g - (uint32_t)rows_[v] * gpr) * CG + k;
      const uint16_t *xr = p.x + (int64_t)rows_[v] * p.ldx;
#pragma unroll
      for (int j = 0; j < U; ++j) {
        const int c = c0[v] + j * TL;
        const bool ok = c < nch;
        ga[v][j] = ok ? reinterpret_cast<const uint4 *>(xr)[c] : make_uint4(0, 0, 0, 0);
        ua[v][j] = ok ? reinterpret_cast<const uint4 *>(xr + p.cols)[c] : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const bool live = base + v * GB + threadIdx.x / TL < ngroups;
      float y[U][8];
      float m = 0.f;
#pragma unroll
      for (int j = 0; j < U; ++j) {
        float u[8];
        unpack8(ga[v][j], y[j]);
        unpack8(ua[v][j], u);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float g = y[j][e];
          y[j][e] = (g * sigmoid_fast(g)) * u[e];
        }
        round_bf16x8(y[j]);
        m = fmaxf(m, amax8(y[j]));
      }
      m = team_max<TL>(m);
      const int row = rows_[v];
#pragma unroll
      for (int j = 0; j < U; ++j) {
        const int c = c0[v] + j * TL;
        const bool ok = live && c < nch;
        if (p.y && ok) store_y(p, row, c, y[j]);
        if constexpr (QF == QF_FP8_G128) {
          const float s = fp8_scale_of(m);
          if (ok && k == 0 && j == 0)
            reinterpret_cast<float *>(p.scales)[(int64_t)row * gpr + (c >> 4)] = s;
          if (ok)
            *reinterpret_cast<uint2 *>(p.q + (int64_t)row * p.cols + (int64_t)c * 8) =
                e4m3_quot8(y[j], s, rcp_approx(s));
        } else {
          const int e = mx_exponent(m);
          if (ok && k == 0 && j == 0)
            reinterpret_cast<uint8_t *>(p.scales)[(int64_t)row * gpr + (c >> 2)] = (uint8_t)(e + 127);
          if (ok)
            *reinterpret_cast<uint32_t *>(p.q + (int64_t)row * (p.cols / 2) + (int64_t)c * 4) =
                e2m1_mul8(y[j], pow2_neg(e));
        }
      }
    }
  }
}

template <int QF, bool WF32>
static void launch_rmsnorm_w(const FusedArgs &p, hipStream_t st) {
  const int per = (p.cols / 8 + 255) / 256;
  const unsigned grid = (unsigned)p.rows;
  if (per <= 1) rmsnorm_quant_kernel<QF, 1, WF32><<<grid, 256, 0, st>>>(p);
  else if (per <= 2) rmsnorm_quant_kernel<QF, 2, WF32><<<grid, 256, 0, st>>>(p);
  else if (per <= 4) rmsnorm_quant_kernel<QF, 4, WF32><<<grid, 256, 0, st>>>(p);
  else if (per <= 8) rmsnorm_quant_kernel<QF, 8, WF32><<<grid, 256, 0, st>>>(p);
  else rmsnorm_quant_kernel<QF, 16, WF32><<<grid, 256, 0, st>>>(p);
}

template <int QF>
static void launch_rmsnorm(const FusedArgs &p, hipStream_t st) {
  if (p.w_f32) launch_rmsnorm_w<QF, true>(p, st);
  else launch_rmsnorm_w<QF, false>(p, st);
}

template <int QF, int TL, int V>
static void launch_swiglu(const FusedArgs &p, hipStream_t st) {
  const uint32_t gpr = QF == QF_FP8_G128 ? (uint32_t)((p.cols + 127) / 128) : (uint32_t)(p.cols / 32);
  const uint32_t ngroups = (uint32_t)p.rows * gpr;
  const uint32_t per_block = (256 / TL) * V;
  uint32_t grid = (ngroups + per_block - 1) / per_block;
  if (grid > 65535) grid = 65535;
  swiglu_quant_kernel<QF, TL, V><<<grid, 256, 0, st>>>(p, ngroups, gpr);
}

hipError_t launch_fused_quant(int prod, int qf, const FusedArgs &p, hipStream_t st) {
  if (p.rows == 0) return hipSuccess;
  if (prod == PROD_RMSNORM) {
    if (qf == QF_FP8_G128) launch_rmsnorm<QF_FP8_G128>(p, st);
    else launch_rmsnorm<QF_MXFP4>(p, st);
  } else {
    if (qf == QF_FP8_G128) launch_swiglu<QF_FP8_G128, 8, 2>(p, st);
    else launch_swiglu<QF_MXFP4, 4, 4>(p, st);
  }
  return hipGetLastError();
}

}  // namespace dsl
