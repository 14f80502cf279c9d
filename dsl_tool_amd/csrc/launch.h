// Host-side launcher prototypes shared between the kernel translation units
// and the C ABI (capi.hip).  Launchers assume arguments were validated.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dsl {

constexpr int kMaxPartials = 1024;   // pass-1 amax partials (floats)

// ------------------------------------------------------------- quantize --
// x: bf16 bits (f32 false) or fp32 (f32 true) elements x[r*sr + c*sc].
hipError_t launch_quant_fp8_tensor(const void *x, bool f32, int64_t rows, int64_t cols,
                                   int64_t sr, int64_t sc, uint8_t *q, float *scale,
                                   float *partial, hipStream_t st);
hipError_t launch_quant_fp8_blocks(const void *x, bool f32, int64_t rows, int64_t cols,
                                   int64_t sr, int64_t sc, int64_t gr, int64_t gc, uint8_t *q,
                                   float *scales, hipStream_t st);
hipError_t launch_quant_mxfp4(const void *x, bool f32, int64_t rows, int64_t cols, int64_t sr,
                              int64_t sc, uint8_t *q, uint8_t *e8m0, hipStream_t st);
hipError_t launch_quant_nvfp4(const void *x, bool f32, int64_t rows, int64_t cols, int64_t sr,
                              int64_t sc, uint8_t *q, uint8_t *e4m3s, float *gscale,
                              float *partial, hipStream_t st);
// The scale an empty tensor quantizes to (amax 0: the 1e-12 floor), written
// to *scale by one thread.
hipError_t launch_empty_scale(float *scale, hipStream_t st);
// Device address of the library-held amax partials on the current device
// (looked up once per device); nullptr and *err set on failure.
float *quant_scratch(hipError_t *err);
size_t quant_scratch_bytes();

// ---------------------------------------------------------------- GEMMs --
// FP8_BLOCK: 1x128 activation groups and 128x128 weight blocks; FP8_GCOL:
// 1x128 activation groups and one weight scale per output column per
// 128-K group (the reference's groupwise layout sb[K/128][N]).
enum GemmMode {
  MODE_FP8_TENSOR = 0, MODE_FP8_BLOCK = 1, MODE_MXFP4 = 2, MODE_NVFP4 = 3, MODE_BF16 = 4,
  MODE_FP8_GCOL = 5
};
// Both FP8 modes whose scales change with every 128-K group.
constexpr bool mode_grouped_k(int mode) { return mode == MODE_FP8_BLOCK || mode == MODE_FP8_GCOL; }

// Compute units of the current device (cached per device; 256 if the query
// fails).
int device_cu_count();

struct GemmArgs {
  const uint8_t *a;      // [M][Kb] packed, K-major
  const uint8_t *b;      // [N][Kb] packed, K-major
  void *c;               // [M][ldc] bf16 or fp32
  int M, N, K;           // K in elements
  int Kb;                // bytes per packed row (FP8: K, FP4: K/2, BF16: 2K)
  int64_t ldc;
  const void *sa;        // FP8_BLOCK / GCOL: float [M][nkg]; MX: uint8 [M][K/32]; NV: uint8 [M][K/16]
  const void *sb;        // FP8_BLOCK: float [ceil(N/128)][nkg]; FP8_GCOL: float [nkg][N];
                         // MX/NV as sa for N
  const float *ga;       // FP8_TENSOR: scale_a; NV: global_a
  const float *gb;       // FP8_TENSOR: scale_b; NV: global_b
  float *ws;             // split-K: one fp32 [M][N] partial slice per K split
  size_t ws_bytes;       // bytes at ws; split-K runs only when it holds two slices or more
  int ksplit;            // >= 1
  int out_f32;
  int accumulate;        // fp32 out only: C += result (register-staged kernels)
  // BF16 on the persistent kernel only: a second K segment, C = A W^T +
  // A2 W2^T with A2 [M][Kb2], W2 [N][Kb2] (Kb2 % 128 == 0; 0: none)
  const uint8_t *a2, *b2;
  int Kb2;
  // ... and W2's own row stride in bytes (0: Kb2) and the period in 128-byte
  // pairs after which W2's columns repeat (0: none; else a power of two): W2
  // = [B | B] is then read from B itself
  int ldb2 = 0, rep2 = 0;
  // Streaming kernel only, BF16 (the LoRA adapter product T^T = A^T X^T):
  // v = C[m][n] * lora_scales[m / lora_rank] is stored transposed, as bf16
  // hi at c[n * ldc + m] and lo = bf16(v - hi) at c[n * ldc + M + m], and
  // columns [2M, ldc) of those rows are zeroed (no other output)
  const float *lora_scales = nullptr;
  int lora_rank = 1;
};

// LDS-DMA pipelined kernel (FP8_TENSOR / MXFP4, Kb % 64 == 0, no split-K);
// variant 0: 256x256 tile, 8 waves; 1: 128x128 tile, 4 waves.
hipError_t launch_gemm_pipe(int mode, const GemmArgs &p, int variant, hipStream_t st);

// Persistent pipelined kernel (Kb % 128 == 0; FP8_TENSOR and BF16; FP8_BLOCK
// and MXFP4 with 16-byte aligned scales and K % 512 == 0; NVFP4 with K % 256
// == 0): one workgroup per CU
// walks its 256x256 tiles with a ring of 128-byte-per-row pair slots running
// across tile boundaries.
bool persist_supported(int mode, int M, int N, int K, int Kb, bool scales16);
hipError_t launch_gemm_persist(int mode, const GemmArgs &p, hipStream_t st);

// Skinny-M kernels, one launch, no workspace (Kb % 1024 == 0):
//   M <= 32: FP8_TENSOR and BF16; FP8_BLOCK and MXFP4 with 16-byte aligned scales
//            and K % 512 == 0;
//   M <= 4:  NVFP4 GEMV with 16-byte aligned scales and M * Kb/1024 <= 8.
bool decode_supported(int mode, int M, int K, int Kb, bool scales4, bool scales16);
hipError_t launch_gemm_decode(int mode, const GemmArgs &p, hipStream_t st);

// Streaming kernel for M <= 1024 (gemm_stream.hip), one launch, no
// workspace, deterministic, Kb % 256 == 0: FP8_TENSOR and BF16; FP8_BLOCK,
// FP8_GCOL and MXFP4 with 16-byte aligned scales and K % 512 == 0; NVFP4
// with 16-byte aligned scales and K % 256 == 0.  The router takes it while
// ceil(M/64) * N stays below a per-mode edge (gemm_tiled.hip, route_for).
bool stream_supported(int mode, int M, int N, int K, int Kb, bool scales16);
hipError_t launch_gemm_stream(int mode, const GemmArgs &p, hipStream_t st);

// Picks a kernel variant for the shape and launches it (plus the split-K
// finalize kernel, which adds the slices in split order, when ksplit > 1).
hipError_t launch_gemm(int mode, GemmArgs args, hipStream_t st);
// Workspace the launcher will need for this shape (0 if none).
size_t gemm_workspace_bytes(int mode, int64_t M, int64_t N, int64_t K, bool accumulate = false);
// Whether launch_gemm takes the streaming kernel (or_pipe: or the pipelined
// tiles) for this shape (aligned scales; accumulate: C += result, fp32 out).
bool gemm_routes_to_stream(int mode, int64_t M, int64_t N, int64_t K, bool or_pipe = false,
                           bool accumulate = false);

constexpr int kMaxGroups = 2048;   // groups per grouped launch (LDS tables)

struct GroupedArgs {
  const uint8_t *x;      // [rows][K]
  const uint8_t *w;      // [G][N][K]
  void *y;               // [rows][ldy]
  const int32_t *offsets;// [G+1] device
  int G, rows, N, K;
  int64_t ldy;
  const float *sx;       // [rows]
  const float *sw;       // [G][N]
  int out_f32;
  // gather form: x is [xrows][K] and sorted row r reads x row arow[r]
  // (persistent kernel, and the grouped streaming tiles; launch_grouped_fp8
  // sends groups of fewer than 48 rows on average to the streaming tiles
  // when K % 256 == 0, the rest to the persistent kernel)
  const int32_t *arow = nullptr;
  int xrows = 0;
};
hipError_t launch_grouped_fp8(GroupedArgs args, hipStream_t st);
// Grouped FP8 on the persistent kernel (K % 128 == 0, K < 2^24).
bool grouped_persist_supported(const GroupedArgs &args);
hipError_t launch_grouped_persist(const GroupedArgs &args, hipStream_t st);
// Grouped FP8 on the streaming tiles (few rows per group; K % 256 == 0).
bool grouped_stream_supported(const GroupedArgs &args);
hipError_t launch_grouped_stream(const GroupedArgs &args, hipStream_t st);

// -------------------------------------------- fused quantize producers --
enum { PROD_RMSNORM = 0, PROD_SWIGLU = 1 };
enum { QF_FP8_G128 = 0, QF_MXFP4 = 1 };

struct FusedArgs {
  const uint16_t *x;     // RMSNorm: [rows][cols]; SwiGLU: [rows][2*cols] (gate | up)
  int64_t ldx;           // row stride of x (elements)
  const void *w;         // RMSNorm weight [cols], bf16 or fp32 (w_f32)
  bool w_f32;
  int rows, cols;        // cols = output row length (SwiGLU: hidden)
  float eps;
  uint8_t *q;            // FP8 [rows][cols] / MXFP4 [rows][cols/2]
  void *scales;          // FP8: float [rows][ceil(cols/128)]; MXFP4: E8M0 [rows][cols/32]
  uint16_t *y;           // optional bf16 output [rows][ldy] (nullptr: none)
  int64_t ldy;
};
// cols % 8 == 0 (MXFP4: % 32); RMSNorm: cols <= 32768 (one workgroup per row).
hipError_t launch_fused_quant(int prod, int qf, const FusedArgs &p, hipStream_t st);

// ------------------------------------------------------------ MoE glue --
// ids [n = tokens * topk] expert per assignment; offsets [E+1]; dest [n]
// (sorted row or -1); src_token [n] (token of each sorted row < offsets[E]);
// ws: moe_route_workspace_bytes.  E <= kMaxGroups.
size_t moe_route_workspace_bytes(int64_t assignments, int64_t num_experts);
hipError_t launch_moe_route(const int32_t *ids, int n, int topk, int E, int32_t *offsets,
                            int32_t *dest, int32_t *src_token, int32_t *ws, hipStream_t st);
// One workgroup per token; slots whose row is < 0 or >= rows are skipped;
// k_dim <= 32768.  tok_major: the codes go once to the token's row of qx
// ([tokens][k_dim]) and only the scales to the sorted rows.
hipError_t launch_moe_permute_quant(const uint16_t *x, int64_t ldx, int k_dim, int tokens,
                                    const int32_t *dest, int topk, int rows, uint8_t *qx, float *sx,
                                    bool tok_major, hipStream_t st);
// launch_moe_route and the tok_major launch_moe_permute_quant in one launch
// for decode-size batches: n <= moe_route_quant_max_assignments, E <= 2047,
// k_dim <= 2048, ldx % 8 == 0, tokens >= 1 (else hipErrorInvalidValue, and
// nothing is launched).  Same offsets, dest, src_token, codes and scales.
constexpr int moe_route_quant_max_assignments = 1024;
hipError_t launch_moe_route_quant(const int32_t *ids, int n, int topk, int E,
                                  const uint16_t *x, int64_t ldx, int k_dim, int tokens,
                                  int32_t *offsets, int32_t *dest, int32_t *src_token,
                                  uint8_t *qx, float *sx, hipStream_t st);
// n <= 32768; slots whose row is < 0 or >= rows_y are skipped.
hipError_t launch_moe_combine(const uint16_t *y, int rows_y, int64_t ldy, int n, const int32_t *dest,
                              const float *w, int tokens, int topk, void *out, int64_t ldo,
                              int out_f32, hipStream_t st);

// -------------------------------------------------------------- LoRA --
// LoRA with few tokens: T = s * X A^T and Y += T B^T on the vector ALUs in
// fp32 (lora.hip); L*R up to kLoraValuMaxLR.  launch_lora_split: t32
// [M][LR] fp32 -> t2 [M][ld2] bf16 with cols [0, LR) hi = bf16(t * s),
// [LR, 2 LR) lo = bf16(t * s - hi), the rest 0; s = scales[col / rank].
constexpr int kLoraValuMaxLR = 512;
bool lora_valu_supported(int64_t M, int64_t K, int64_t LR);
hipError_t launch_lora_t(const uint16_t *x, const uint16_t *a_t, int M, int K, int LR, int rank,
                         const float *scales, float *t, uint16_t *t2, int ld2, hipStream_t st);
hipError_t launch_lora_apply(const float *t, const uint16_t *b_t, float *y, int M, int N, int LR,
                             int64_t ldy, hipStream_t st);
hipError_t launch_lora_split(const float *t32, int M, int LR, int ld2, int rank,
                             const float *scales, uint16_t *t2, hipStream_t st);
// bt [N][LR] -> b2 [N][ld2] = bt | bt | 0.
hipError_t launch_lora_dup(const uint16_t *bt, int N, int LR, int ld2, uint16_t *b2,
                           hipStream_t st);

}  // namespace dsl
