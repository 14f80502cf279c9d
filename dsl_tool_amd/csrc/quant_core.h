// Device helpers shared by the quantizers (quant.hip) and the fused
// quantize producers (fused.hip): bf16 unpacking, group amax by lane teams,
// scales and encoders.
#pragma once

#include "common.h"

namespace dsl {

constexpr float kRcp448 = 1.0f / 448.0f;     // RN(1/448)
constexpr float kRcp6 = 1.0f / 6.0f;         // RN(1/6)
constexpr float kRcp2688 = 1.0f / 2688.0f;   // RN(1/2688)

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

template <int CTRL>
DSL_DEV float dpp_f(float v) {
  return u2f((uint32_t)__builtin_amdgcn_mov_dpp((int)f2u(v), CTRL, 0xf, 0xf, false));
}

// Max over aligned teams of TL lanes (TL = 1, 2, 4, 8, 16); every lane of a
// team gets it.  quad_perm [1,0,3,2] and [2,3,0,1] reduce a quad, the half-row
// mirror pairs quads, the row mirror pairs half rows.  All lanes must be
// active.
template <int TL>
DSL_DEV float team_max(float v) {
  static_assert(TL == 1 || TL == 2 || TL == 4 || TL == 8 || TL == 16, "team size");
  if constexpr (TL >= 2) v = fmaxf(v, dpp_f<0xb1>(v));
  if constexpr (TL >= 4) v = fmaxf(v, dpp_f<0x4e>(v));
  if constexpr (TL >= 8) v = fmaxf(v, dpp_f<0x141>(v));
  if constexpr (TL >= 16) v = fmaxf(v, dpp_f<0x140>(v));
  return v;
}

DSL_DEV void unpack8(const uint4 &v, float *f) {
  f[0] = u2f(v.x << 16); f[1] = u2f(v.x & 0xffff0000u);
  f[2] = u2f(v.y << 16); f[3] = u2f(v.y & 0xffff0000u);
  f[4] = u2f(v.z << 16); f[5] = u2f(v.z & 0xffff0000u);
  f[6] = u2f(v.w << 16); f[7] = u2f(v.w & 0xffff0000u);
}

DSL_DEV float amax8(const float *f) {
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) m = fmaxf(m, __builtin_fabsf(f[i]));
  return m;
}

DSL_DEV float load_bf16(const uint16_t *x, int64_t idx) { return bf16_to_f32(x[idx]); }

// One source element as fp32: bf16 bits (uint16_t) or fp32 (float).
DSL_DEV float load_in(const uint16_t *x, int64_t idx) { return bf16_to_f32(x[idx]); }
DSL_DEV float load_in(const float *x, int64_t idx) { return x[idx]; }

// The scales with the IEEE division itself (the strided kernels, which also
// serve fp32 sources: the reciprocal quotient below is only shown exact for
// bf16 amax values).
DSL_DEV float fp8_scale_ieee(float amax) {
  const float s = __fdiv_rn(amax, kE4M3Max);
  return s < kScaleFloor ? kScaleFloor : s;
}
DSL_DEV float nv_global_ieee(float amax) {
  const float s = __fdiv_rn(amax, kNvGlobalDiv);
  return s < kScaleFloor ? kScaleFloor : s;
}

// Reduce the pass-1 partial maxima (n <= kMaxPartials) inside one block.
DSL_DEV float reduce_partials(const float *partial, int n, float *sh) {
  float m = 0.f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, partial[i]);
  return block_max(m, sh);
}

// max(amax / 448, 1e-12) and max(amax / 2688, 1e-12); quot with the constant
// reciprocal is the IEEE quotient for every bf16 amax.
DSL_DEV float fp8_scale_of(float amax) {
  const float s = quot(amax, kE4M3Max, kRcp448);
  return s < kScaleFloor ? kScaleFloor : s;
}

DSL_DEV float nv_global_of(float amax) {
  const float s = quot(amax, kNvGlobalDiv, kRcp2688);
  return s < kScaleFloor ? kScaleFloor : s;
}

// NVFP4 block scale code e4m3((amax16 / 6) / sg) (rsg = rcp(sg)).
DSL_DEV uint32_t nv_block_code(float m, float sg, float rsg) {
  const float t = quot(m, 6.0f, kRcp6);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(quot(t, sg, rsg), 0.f, 0, false) & 0xffu;
}

DSL_DEV float e4m3_value(uint32_t code) { return __builtin_amdgcn_cvt_f32_fp8((int)code, 0); }

// 8 values / s as E4M3 codes (2 x u32); r = rcp(s).
DSL_DEV uint2 e4m3_quot8(const float *f, float s, float r) {
  return make_uint2(e4m3_quot4(f[0], f[1], f[2], f[3], s, r), e4m3_quot4(f[4], f[5], f[6], f[7], s, r));
}

}  // namespace dsl
