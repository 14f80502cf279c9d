// Shared definitions for the gfx950 quantized-GEMM library.
//
// Number formats (bit-exact contract, identical on host and device):
//   E4M3FN  bias 7, max 448, NaN = S.1111.111, RNE, |x| > 464 -> NaN
//           (the conversion the reference performs with __nv_fp8_e4m3,
//           cuda/gemm/fp8_gemm.cu:141-142, restated from the OCP FP8 spec).
//   E2M1    {0,.5,1,1.5,2,3,4,6}, bit 3 = sign (cuda/gemm/fp4_gemm.cu:30-33),
//           RNE with saturation to +-6, sign of zero kept; two codes per
//           byte with the even K index in the low nibble (fp4_gemm.cu:45-47).
//   E8M0    2^(code-127); MXFP4 exponent = clamp(floor(log2 amax)-2,-127,127).
//
// MFMA operand layouts (measured on gfx950 with an in-bounds probe):
//   v_mfma_scale_f32_16x16x128_f8f6f4
//     A/B lane l -> row (col) l%16, lane group g = l/16.
//     FP4: the lane's 16 bytes are K elements [32g, 32g+32) of the 128-K
//          step (even element in the low nibble); E8M0 scale byte of lane l
//          (op_sel picks the byte of the 32-bit operand) scales that block.
//     FP8: bytes 0..15 are K [16g, 16g+16), bytes 16..31 are K [64+16g, ..);
//          with unit scales any K order shared by A and B gives the same
//          sum, so FP8 here packs 32 contiguous K bytes per lane.
//     D:   lane l, register i -> C[4*(l/16)+i][l%16].
//   v_mfma_f32_16x16x32_bf16: lane l -> row l%16, K [(l/16)*8, +8);
//     D as above.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define DSL_HD __host__ __device__ __forceinline__
#define DSL_DEV __device__ __forceinline__

typedef int      v8i  __attribute__((ext_vector_type(8)));
typedef int      v4i  __attribute__((ext_vector_type(4)));
typedef int      v2i  __attribute__((ext_vector_type(2)));
typedef float    v4f  __attribute__((ext_vector_type(4)));
typedef float    v16f __attribute__((ext_vector_type(16)));
typedef __bf16   v8bf __attribute__((ext_vector_type(8)));
typedef __bf16   v2bf __attribute__((ext_vector_type(2)));

namespace dsl {

// ------------------------------------------------------------------ bits --
DSL_HD uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
DSL_HD float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

DSL_HD float bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

// float32 -> bf16 bits, round-to-nearest-even, NaN stays NaN.
DSL_HD uint16_t f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Two floats as packed bf16 (low half: a) by v_cvt_pk_bf16_f32, which rounds
// to nearest even exactly as f32_to_bf16 (checked on gfx950 over 16.7M
// patterns: ties, subnormals, infinities and NaNs all agree).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef float v2f_ __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f_){a, b}, v2bf));
}

// ------------------------------------------------------------------ E4M3 --
DSL_HD uint8_t e4m3_encode(float x) {
  uint32_t u = f2u(x);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t mag = u & 0x7fffffffu;
  if (mag >= 0x7f800000u) return (uint8_t)(sign | 0x7fu);          // inf / nan
  if (mag >= 0x3c800000u) {                                        // >= 2^-6
    uint32_t r = (mag + 0x7ffffu + ((mag >> 20) & 1u)) >> 20;      // RNE to 3 bits
    int code = (int)r - ((127 - 7) << 3);
    if (code >= 0x7f) return (uint8_t)(sign | 0x7fu);              // > 464 -> NaN
    return (uint8_t)(sign | (uint32_t)code);
  }
  float a = u2f(mag) * 512.0f;                                     // exact
  return (uint8_t)(sign | (uint32_t)__builtin_rintf(a));           // RNE, 0..8
}

DSL_HD float e4m3_decode(uint8_t c) {
  uint32_t s = (uint32_t)(c & 0x80) << 24;
  uint32_t e = (c >> 3) & 0xF, m = c & 7;
  if (e == 0) return u2f(s | f2u((float)m * 0.001953125f));        // m * 2^-9
  if (e == 15 && m == 7) return u2f(s | 0x7fc00000u);
  return u2f(s | ((e + 120u) << 23) | (m << 20));
}

// ------------------------------------------------------------------ E2M1 --
// Count of thresholds not exceeded; NaN exceeds none and saturates to 7.
DSL_HD uint32_t e2m1_encode(float v) {
  uint32_t s = (f2u(v) >> 28) & 0x8u;
  float a = __builtin_fabsf(v);
  uint32_t c = 7u - (uint32_t)(a <= 5.0f) - (uint32_t)(a < 3.5f) - (uint32_t)(a <= 2.5f)
             - (uint32_t)(a < 1.75f) - (uint32_t)(a <= 1.25f) - (uint32_t)(a < 0.75f)
             - (uint32_t)(a <= 0.25f);
  return s | c;
}

// ----------------------------------------------- hardware encoders (gfx950) --
// v_cvt_pk_fp8_f32 and v_cvt_scalef32_pk_fp4_f32 (scale 1.0) return exactly
// e4m3_encode / e2m1_encode of every finite fp32 input (checked on gfx950
// over all 2^32 patterns; E4M3 differs only in the sign of the NaN code).
//
// Quotients.  The contract encodes the IEEE quotient RN(x / s).  The vector
// paths form instead
//     q = x * r,   e = fma(q, s, -x),   q' = fma(-e, r, q)
// (one correction step after Markstein) with r = v_rcp_f32(s).  q' is not
// always RN(x / s) in fp32, but for every bf16 x and every scale these
// quantizers produce, its E4M3 / E2M1 code is the code of RN(x / s) whenever
// r is within 1 ulp of 1/s: tests/quot_exhaustive.c checks every bf16
// (amax, x) pair for E4M3 (s = amax / 448 with the floor) and every
// (global scale, block scale code, x) triple for NVFP4, with r at RN(1/s) and
// one ulp either side.  v_rcp_f32 is specified to 1 ulp, and on gfx950 it lies
// within 1 ulp of 1.0f / s for every normal s in [2^-125, 2^125] (measured).
// The same step with a constant r = RN(1/b) gives RN(a / b) exactly for every
// bf16 a and b = 448, 6, 2688 (also checked there), which yields the scales.
// A zero x keeps its sign: e = +0 and q' = q + (-0) = q.
// Inputs are finite; codes for NaN or infinite inputs are not specified.

DSL_DEV float quot(float x, float s, float r) {
  const float q = x * r;
  const float e = __builtin_fmaf(q, s, -x);
  return __builtin_fmaf(-e, r, q);
}

DSL_DEV float rcp_approx(float s) { return __builtin_amdgcn_rcpf(s); }

// E4M3 codes of x[i] / s for 4 values, byte i = element i.
DSL_DEV uint32_t e4m3_quot4(float x0, float x1, float x2, float x3, float s, float r) {
  uint32_t c = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(quot(x0, s, r), quot(x1, s, r), 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(quot(x2, s, r), quot(x3, s, r), (int)c, true);
}

// E2M1 codes of v0 (low nibble) and v1, as e2m1_encode, into byte `b` of `old`.
template <int B>
DSL_DEV uint32_t e2m1_pk_into(uint32_t old, float v0, float v1) {
  return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(old, v0, v1, 1.0f, B);
}
DSL_DEV uint32_t e2m1_pk(float v0, float v1) { return e2m1_pk_into<0>(0u, v0, v1) & 0xffu; }

// E2M1 codes of x[i] / d for 8 values (nibble i = element i); r = rcp(d).
DSL_DEV uint32_t e2m1_quot8(const float *x, float d, float r) {
  uint32_t c = e2m1_pk_into<0>(0u, quot(x[0], d, r), quot(x[1], d, r));
  c = e2m1_pk_into<1>(c, quot(x[2], d, r), quot(x[3], d, r));
  c = e2m1_pk_into<2>(c, quot(x[4], d, r), quot(x[5], d, r));
  return e2m1_pk_into<3>(c, quot(x[6], d, r), quot(x[7], d, r));
}

// E2M1 codes of x[i] * m for 8 values (m a power of two: exact).
DSL_DEV uint32_t e2m1_mul8(const float *x, float m) {
  uint32_t c = e2m1_pk_into<0>(0u, x[0] * m, x[1] * m);
  c = e2m1_pk_into<1>(c, x[2] * m, x[3] * m);
  c = e2m1_pk_into<2>(c, x[4] * m, x[5] * m);
  return e2m1_pk_into<3>(c, x[6] * m, x[7] * m);
}

// ------------------------------------------------------------------ E8M0 --
// MXFP4 shared exponent: clamp(floor(log2(amax)) - 2, -127, 127); amax == 0
// gives -127.  Integer exponent extraction (exact for subnormals).
DSL_HD int mx_exponent(float amax) {
  uint32_t u = f2u(amax) & 0x7fffffffu;
  if (u == 0) return -127;
  int ex = (int)(u >> 23);
  int fl = ex > 0 ? ex - 127 : (31 - __builtin_clz(u)) - 149;
  int e = fl - 2;
  return e < -127 ? -127 : (e > 127 ? 127 : e);
}

// 2^-e as float for e in [-127, 126].
DSL_HD float pow2_neg(int e) { return u2f((uint32_t)(127 - e) << 23); }

// ---------------------------------------------------------- constants ----
constexpr float kE4M3Max = 448.0f;
constexpr float kScaleFloor = 1e-12f;
constexpr float kNvGlobalDiv = 2688.0f;   // 448 * 6

}  // namespace dsl
