// LoRA fused GEMM: Y = X W^T + sum_l s_l (X A_l^T) B_l^T on the bf16 MFMA
// path (reference: lora_fused_gemm_kernel, cuda/gemm/grouped_gemm.cu:106-140,
// Y = X @ W + sum_l scale_l * X @ A_l @ B_l in fp32).
//
// T = X A^T for all adapters at once (A^T = [L*R][K], fp32; computed as
// T^T = A^T X^T on the streaming kernel when L*R <= 256, which reads X once
// in one launch and whose epilogue does the split below itself), then T*s is
// split into bf16 hi + lo (hi + lo carries 16 mantissa bits of T*s, so the
// low-rank term loses almost nothing to the bf16 MFMA).  The adapter term is
// then a K extension of the base GEMM: Y = [X | hi | lo] [W | B^T | B^T]^T,
// which the persistent kernel reads as a second K segment of each row, so Y
// is written once.  hi | lo and B^T | B^T are padded with zeros to a
// multiple of 64 columns (whole 128-byte pairs); when L*R is 64, 128 or 256
// the kernel reads B^T twice instead of a materialized B^T | B^T.  That one
// pass is for more than 256 tokens; up to 256 the base GEMM runs on its own
// kernel and the adapter term is added into the fp32 Y by a second launch
// (below: T from the vector ALUs).
#include "launch.h"
#include "common.h"
#include "quant_core.h"

namespace dsl {

// t32 [M][LR] -> t2 [M][ld2]: cols [0, LR) hi, [LR, 2 LR) lo, the rest 0.
__global__ __launch_bounds__(256) void lora_split_kernel(const float *__restrict__ t32, int M,
                                                         int LR, int ld2, int rank,
                                                         const float *__restrict__ scales,
                                                         uint16_t *__restrict__ t2) {
  const int64_t n = (int64_t)M * ld2;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / ld2;
    const int col = (int)(i - r * ld2);
    uint16_t o = 0;
    if (col < 2 * LR) {
      const int c = col < LR ? col : col - LR;
      const float v = t32[r * LR + c] * scales[c / rank];
      const uint16_t h = f32_to_bf16(v);
      o = col < LR ? h : f32_to_bf16(v - bf16_to_f32(h));
    }
    t2[i] = o;
  }
}

// b_t [N][LR] -> b2 [N][ld2] = b_t | b_t | 0.
__global__ __launch_bounds__(256) void lora_dup_kernel(const uint16_t *__restrict__ bt, int N,
                                                       int LR, int ld2,
                                                       uint16_t *__restrict__ b2) {
  const int64_t n = (int64_t)N * ld2;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / ld2;
    const int col = (int)(i - r * ld2);
    b2[i] = col < 2 * LR ? bt[r * LR + (col < LR ? col : col - LR)] : (uint16_t)0;
  }
}

// ---- few tokens: the adapter term on the vector ALUs ---------------------
// T = X A^T (times the adapter scale) and Y += T B^T are small next to the
// base GEMM when the tokens are few (2 M L R K and 2 M N L R flops), but the
// MFMA form of T^T runs the L R adapter rows as one row block, so one
// workgroup streams all of A^T.  Here T is split over its adapter rows and
// token blocks and each workgroup sums its full K in a fixed order.  Up to
// 256 tokens T is written as hi | lo for the MFMA add; for one or two tokens
// it stays fp32 and the add is lora_apply_kernel (no hi + lo split, no
// B^T | B^T copy).

// v = scales[r / rank] * sum_k x[m][k] a_t[r][k] for RB = 4 adapter rows
// and MB tokens per workgroup, stored as fp32 t[m][r], or (t2 != null) as
// bf16 hi | lo in t2[m][ld2] (hi at column r, lo at LR + r, the columns
// from 2 LR on zero) for the MFMA add.  Threads take 8-element segments of
// K (a 16-byte load per row); the 256 partial sums of each output are added
// through LDS in a fixed order.
template <int MB>
__global__ __launch_bounds__(256) void lora_t_kernel(const uint16_t *__restrict__ x,
                                                     const uint16_t *__restrict__ a_t, int M,
                                                     int K, int LR, int rank,
                                                     const float *__restrict__ scales,
                                                     float *__restrict__ t,
                                                     uint16_t *__restrict__ t2, int ld2) {
  constexpr int RB = 4, NO = RB * MB, TPO = 256 / NO;   // outputs, threads per output
  static_assert(NO <= 32 && TPO * NO == 256, "lora_t_kernel shape");
  __shared__ float red[NO][257];
  const int r0 = blockIdx.x * RB, m0 = blockIdx.y * MB;
  const int rows = M - m0 < MB ? M - m0 : MB;
  float acc[RB][MB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[rb][mb] = 0.f;
  // every load of a segment is issued before its multiplies (rows past M
  // re-read the last row; their sums are never stored)
  const uint16_t *xr[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) xr[mb] = x + (int64_t)(mb < rows ? m0 + mb : M - 1) * K;
  const int segs = K / 8;
  for (int sg = threadIdx.x; sg < segs; sg += 256) {
    uint4 av[RB], xv[MB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
      av[rb] = *reinterpret_cast<const uint4 *>(a_t + (int64_t)(r0 + rb) * K + sg * 8);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) xv[mb] = *reinterpret_cast<const uint4 *>(xr[mb] + sg * 8);
    float a[RB][8];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) unpack8(av[rb], a[rb]);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      float xf[8];
      unpack8(xv[mb], xf);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[rb][mb] = fmaf(a[rb][j], xf[j], acc[rb][mb]);
    }
  }
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) red[rb * MB + mb][threadIdx.x] = acc[rb][mb];
  __syncthreads();
  // TPO consecutive lanes per output, each over NO partials, then a
  // butterfly over those lanes (the same order on every run)
  const int o = threadIdx.x / TPO, part = threadIdx.x % TPO;
  float v = 0.f;
  for (int j = 0; j < NO; ++j) v += red[o][part * NO + j];
#pragma unroll
  for (int off = TPO / 2; off >= 1; off /= 2) v += __shfl_xor(v, off);
  const int rb = o / MB, mb = o % MB;
  if (part == 0 && mb < rows) {
    const int r = r0 + rb;
    const float sv = v * scales[r / rank];
    if (t2) {
      uint16_t *row = t2 + (int64_t)(m0 + mb) * ld2;
      const uint16_t h = f32_to_bf16(sv);
      row[r] = h;
      row[LR + r] = f32_to_bf16(sv - bf16_to_f32(h));
    } else {
      t[(int64_t)(m0 + mb) * LR + r] = sv;
    }
  }
  if (t2 && blockIdx.x == 0)   // the pad columns of this workgroup's rows
    for (int i = threadIdx.x; i < rows * (ld2 - 2 * LR); i += 256)
      t2[(int64_t)(m0 + i / (ld2 - 2 * LR)) * ld2 + 2 * LR + i % (ld2 - 2 * LR)] = 0;
}

// y[m][n] += sum_r t[m][r] b_t[n][r]: a thread per output column n, MB
// tokens per workgroup.  t's addresses are the same across a wave, so its
// values come in through scalar loads and feed the multiplies as scalar
// operands; the thread's B^T row is read 16 bytes at a time, a 64-column
// run of it ahead of its multiplies.  One writer per element.
template <int MB>
__global__ __launch_bounds__(256) void lora_apply_kernel(const float *__restrict__ t,
                                                         const uint16_t *__restrict__ b_t,
                                                         float *__restrict__ y, int M, int N,
                                                         int LR, int64_t ldy) {
  const int m0 = blockIdx.y * MB;
  const int rows = M - m0 < MB ? M - m0 : MB;
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  const float *tr[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) tr[mb] = t + (int64_t)(mb < rows ? m0 + mb : M - 1) * LR;
  float acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = 0.f;
  const uint16_t *brow = b_t + (int64_t)n * LR;
  for (int r0 = 0; r0 < LR; r0 += 64) {
    const int nr = LR - r0 < 64 ? LR - r0 : 64;   // a multiple of 8
    uint4 bv[8];
#pragma unroll
    for (int c = 0; c < 8; ++c)
      bv[c] = c * 8 < nr ? *reinterpret_cast<const uint4 *>(brow + r0 + c * 8) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      if (c * 8 >= nr) break;
      float b[8];
      unpack8(bv[c], b);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const float *tp = tr[mb] + r0 + c * 8;
        float a = acc[mb];
#pragma unroll
        for (int j = 0; j < 8; ++j) a = fmaf(tp[j], b[j], a);
        acc[mb] = a;
      }
    }
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
    if (mb < rows) {
      float *d = y + (int64_t)(m0 + mb) * ldy + n;
      *d = *d + acc[mb];
    }
}

static unsigned grid_of(int64_t n) {
  int64_t g = (n + 255) / 256;
  return (unsigned)(g < 1 ? 1 : (g > 8192 ? 8192 : g));
}

hipError_t launch_lora_split(const float *t32, int M, int LR, int ld2, int rank,
                             const float *scales, uint16_t *t2, hipStream_t st) {
  if (M == 0) return hipSuccess;
  lora_split_kernel<<<grid_of((int64_t)M * ld2), 256, 0, st>>>(t32, M, LR, ld2, rank, scales, t2);
  return hipGetLastError();
}

hipError_t launch_lora_dup(const uint16_t *bt, int N, int LR, int ld2, uint16_t *b2,
                           hipStream_t st) {
  if (N == 0) return hipSuccess;
  lora_dup_kernel<<<grid_of((int64_t)N * ld2), 256, 0, st>>>(bt, N, LR, ld2, b2);
  return hipGetLastError();
}

bool lora_valu_supported(int64_t M, int64_t K, int64_t LR) {
  return M >= 1 && K % 8 == 0 && LR % 8 == 0 && LR <= kLoraValuMaxLR && M < ((int64_t)1 << 31);
}

hipError_t launch_lora_t(const uint16_t *x, const uint16_t *a_t, int M, int K, int LR, int rank,
                         const float *scales, float *t, uint16_t *t2, int ld2, hipStream_t st) {
  if (!lora_valu_supported(M, K, LR) || rank < 1 || (t2 && ld2 < 2 * LR)) return hipErrorInvalidValue;
  const int mb = M <= 1 ? 1 : (M <= 2 ? 2 : (M <= 4 ? 4 : 8));
  const dim3 grid((unsigned)(LR / 4), (unsigned)((M + mb - 1) / mb));
  if (grid.y > 65535u) return hipErrorInvalidValue;
  switch (mb) {
    case 1: lora_t_kernel<1><<<grid, 256, 0, st>>>(x, a_t, M, K, LR, rank, scales, t, t2, ld2); break;
    case 2: lora_t_kernel<2><<<grid, 256, 0, st>>>(x, a_t, M, K, LR, rank, scales, t, t2, ld2); break;
    case 4: lora_t_kernel<4><<<grid, 256, 0, st>>>(x, a_t, M, K, LR, rank, scales, t, t2, ld2); break;
    default: lora_t_kernel<8><<<grid, 256, 0, st>>>(x, a_t, M, K, LR, rank, scales, t, t2, ld2); break;
  }
  return hipGetLastError();
}

hipError_t launch_lora_apply(const float *t, const uint16_t *b_t, float *y, int M, int N, int LR,
                             int64_t ldy, hipStream_t st) {
  if (!lora_valu_supported(M, 8, LR) || N < 1) return hipErrorInvalidValue;
  const int mb = M <= 1 ? 1 : (M <= 2 ? 2 : (M <= 4 ? 4 : (M <= 8 ? 8 : 16)));
  const dim3 grid((unsigned)((N + 255) / 256), (unsigned)((M + mb - 1) / mb));
  if (grid.y > 65535u) return hipErrorInvalidValue;
  switch (mb) {
    case 1: lora_apply_kernel<1><<<grid, 256, 0, st>>>(t, b_t, y, M, N, LR, ldy); break;
    case 2: lora_apply_kernel<2><<<grid, 256, 0, st>>>(t, b_t, y, M, N, LR, ldy); break;
    case 4: lora_apply_kernel<4><<<grid, 256, 0, st>>>(t, b_t, y, M, N, LR, ldy); break;
    case 8: lora_apply_kernel<8><<<grid, 256, 0, st>>>(t, b_t, y, M, N, LR, ldy); break;
    default: lora_apply_kernel<16><<<grid, 256, 0, st>>>(t, b_t, y, M, N, LR, ldy); break;
  }
  return hipGetLastError();
}

}  // namespace dsl
