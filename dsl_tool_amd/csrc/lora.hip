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
// the kernel reads B^T twice instead of a materialized B^T | B^T.
#include "launch.h"
#include "common.h"

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

}  // namespace dsl
