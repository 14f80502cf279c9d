/*
 * dsl_gemm.h -- C ABI of the gfx950 (MI355X) quantized-GEMM library
 * (libdsl_gemm.so).  Plain pointers and sizes only; no torch or C++ types.
 *
 * Conventions for every entry point:
 *   - all data pointers are device pointers on the current HIP device;
 *   - `stream` is a hipStream_t (torch.cuda.current_stream().cuda_stream);
 *     work is enqueued asynchronously, nothing synchronises;
 *   - strides are in elements; packed operand rows are K-major bytes
 *     (FP8: K bytes per row, FP4: K/2 bytes per row);
 *   - the return value is DSL_OK (0) or a negative status; the message is
 *     available from dsl_last_error() (thread-local).  Validation happens
 *     before any launch, so an error return means nothing was enqueued.
 *     Nothing in the library calls exit() (the reference's CHECK_CUDA does,
 *     cuda/gemm/fp8_gemm.cu:17-25);
 *   - the library never allocates device memory: outputs and workspaces
 *     are passed in (sizes from the *_workspace_bytes queries).
 *
 * Reference interfaces replaced (the reference has no C ABI for this path;
 * these are the functions the Python callables registered as
 * gemm.fp8_gemm / gemm.grouped_gemm reach, dispatcher/registry.py:133-141):
 */
#ifndef DSL_GEMM_H
#define DSL_GEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  DSL_OK = 0,
  DSL_ERR_ARG = -1,          /* bad shape / stride / alignment / null pointer */
  DSL_ERR_UNSUPPORTED = -2,  /* valid request this build does not implement   */
  DSL_ERR_WORKSPACE = -3,    /* workspace missing or too small                */
  DSL_ERR_HIP = -4           /* HIP runtime error while launching             */
};

enum { DSL_OUT_BF16 = 0, DSL_OUT_F32 = 1 };
enum { DSL_SCALE_TENSOR = 0, DSL_SCALE_BLOCK128 = 1, DSL_SCALE_GROUP128 = 2 };
enum { DSL_FMT_MXFP4 = 0, DSL_FMT_NVFP4 = 1 };
enum { DSL_OP_FP8 = 0, DSL_OP_FP4 = 1, DSL_OP_GROUPED_FP8 = 2, DSL_OP_BF16 = 3 };
enum { DSL_QFMT_FP8_G128 = 0, DSL_QFMT_MXFP4 = 1 };
enum { DSL_W_BF16 = 0, DSL_W_F32 = 1 };
enum { DSL_IN_BF16 = 0, DSL_IN_F32 = 1 };

/* Last error message of the calling thread ("" when none). */
const char *dsl_last_error(void);

/* ABI version of this header (bumped on any signature change). */
int dsl_abi_version(void);

/* ------------------------------------------------------------ quantize --
 * Input x is a bf16 (x_dtype DSL_IN_BF16) or fp32 (DSL_IN_F32, the
 * reference's own input type, cuda/gemm/fp8_gemm.cu:118-144,
 * fp4_gemm.cu:49-90) matrix read as x[r*stride_row + c*stride_col], rows R,
 * cols C, with C the GEMM reduction axis (A[M,K] directly; the reference's
 * B[K,N] as its [N,K] view).  Outputs are K-major: q[r*C + c].  Codes are
 * those of the IEEE quotient x / scale for either source type.
 */

/* Per-tensor E4M3.  scale = max(amax/448, 1e-12); q = e4m3(x / scale).
 * Replaces quantize_to_fp8_kernel (cuda/gemm/fp8_gemm.cu:118-144).
 * Writes one float to *scale (1e-12 for an empty tensor, when scale is not
 * NULL).  Needs dsl_quant_workspace_bytes(R, C). */
int dsl_quant_fp8_tensor(const void *x, int64_t rows, int64_t cols,
                         int64_t stride_row, int64_t stride_col, int x_dtype,
                         uint8_t *q, float *scale,
                         void *workspace, size_t workspace_bytes, void *stream);

/* dsl_quant_fp8_tensor without the workspace argument and without any
 * allocation: the amax partials live in a library-held device array of
 * 4 KB per GPU (1024 floats, kept until the process ends), which covers
 * every size.  No counterpart in the reference; for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Results are identical to dsl_quant_fp8_tensor.
 * Every call on one GPU uses that GPU's array, so calls that overlap on one
 * GPU (different streams, threads or graph replays in flight together) race
 * and must be serialized by the caller.  The array used is the current
 * device's: the current device must be the device of `stream` and of the
 * data.  The first call on a device looks up the array's address
 * (hipGetSymbolAddress); that call may be made inside HIP graph capture. */
int dsl_quant_fp8_tensor_noalloc(const void *x, int64_t rows, int64_t cols,
                                 int64_t stride_row, int64_t stride_col, int x_dtype,
                                 uint8_t *q, float *scale, void *stream);

/* Block-scaled E4M3 over group_rows x group_cols tiles (1x128 activations,
 * 128x128 weights, 1xC per-row / per-channel).  scales is
 * [ceil(R/group_rows)][ceil(C/group_cols)] fp32, each max(amax/448, 1e-12).
 * Replaces the scale layout read by fp8_gemm_groupwise_kernel
 * (cuda/gemm/fp8_gemm.cu:67-99), which ships no quantizer of its own. */
int dsl_quant_fp8_blocks(const void *x, int64_t rows, int64_t cols,
                         int64_t stride_row, int64_t stride_col, int x_dtype,
                         int64_t group_rows, int64_t group_cols,
                         uint8_t *q, float *scales, void *stream);

/* MXFP4: per row and 32 K elements, E8M0 = clamp(floor(log2 amax)-2,
 * -127,127)+127, codes = e2m1_rne_sat(x * 2^-e).  q_packed [R][C/2] (low
 * nibble = even K), e8m0 [R][C/32].  C % 32 == 0.
 * Replaces quantize_fp32_to_nvfp4 (cuda/gemm/fp4_gemm.cu:49-90), whose
 * flat fp32 amax/6 scales are not MXFP4. */
int dsl_quant_mxfp4(const void *x, int64_t rows, int64_t cols,
                    int64_t stride_row, int64_t stride_col, int x_dtype,
                    uint8_t *q_packed, uint8_t *e8m0, void *stream);

/* NVFP4: s_g = max(amax_T/2688, 1e-12); per row and 16 K elements
 * s_b = e4m3((amax_16/6)/s_g); codes = e2m1_rne_sat(x / (f32(s_b)*s_g)),
 * all-zero codes where that denominator is 0.  q_packed [R][C/2],
 * e4m3_scales [R][C/16], *global_scale = s_g (1e-12 for an empty tensor,
 * when global_scale is not NULL).  C % 16 == 0.
 * Same reference function replaced as dsl_quant_mxfp4. */
int dsl_quant_nvfp4(const void *x, int64_t rows, int64_t cols,
                    int64_t stride_row, int64_t stride_col, int x_dtype,
                    uint8_t *q_packed, uint8_t *e4m3_scales, float *global_scale,
                    void *workspace, size_t workspace_bytes, void *stream);

/* Workspace bytes for the two-pass (global amax) quantizers. */
size_t dsl_quant_workspace_bytes(int64_t rows, int64_t cols);

/* --------------------------------------------------------------- GEMMs --
 * C[m, n] = sum_k A[m, k] * W[n, k] (the reference's A @ B with B = W^T),
 * A [M][K] and W [N][K] packed K-major, C [M][ldc] in bf16 or fp32.
 * m == 0 or n == 0 succeeds without reading any pointer (an empty scale
 * array may be NULL); the dimensions and mode are still checked.
 */

/* FP8 E4M3 GEMM.
 *   DSL_SCALE_TENSOR:   scale_a, scale_b -> one float each (device);
 *                       C = (acc * sa) * sb  (triton/gemm/gemm_kernels.py:97).
 *   DSL_SCALE_BLOCK128: scale_a [M][ceil(K/128)] (1x128 groups),
 *                       scale_b [ceil(N/128)][ceil(K/128)] (128x128 blocks);
 *                       C = sum_g (sum_{k in g} a*w) * sa[m,g] * sb[n/128,g]
 *                       (cuda/gemm/fp8_gemm.cu:84-97).  The large-M kernels
 *                       carry the sum in units of the current group's
 *                       sa*sb and rescale by the ratio of consecutive
 *                       groups, so every product sa[m,g]*sb[n/128,g] must be
 *                       a normal fp32 number: a zero or subnormal product
 *                       makes that row inf/NaN there.  The quantizers here
 *                       and the reference's floor each scale at 1e-12
 *                       (cuda/gemm/fp8_gemm.cu:134), whose products are
 *                       normal.
 *   DSL_SCALE_GROUP128: the reference groupwise layout with G = 128:
 *                       scale_a [M][ceil(K/128)], scale_b [ceil(K/128)][N]
 *                       (one weight scale per output column per group,
 *                       cuda/gemm/fp8_gemm.cu:67-75);
 *                       C = sum_g (sum_{k in g} a*w) * sa[m,g] * sb[g,n]
 *                       (cuda/gemm/fp8_gemm.cu:84-97).  A group size G that
 *                       is a multiple of 128 is the same sum with each scale
 *                       repeated over G/128 groups of 128.
 * K % 16 == 0.  Replaces fp8_gemm (triton/gemm/gemm_kernels.py:104-122),
 * fp8_gemm_per_tensor (cuda/gemm/fp8_gemm.cu:102-108) and
 * fp8_gemm_groupwise (cuda/gemm/fp8_gemm.cu:110-116). */
int dsl_fp8_gemm(const uint8_t *a, const uint8_t *b, void *c,
                 int64_t m, int64_t n, int64_t k, int64_t ldc, int out_dtype,
                 int scale_mode, const float *scale_a, const float *scale_b,
                 void *workspace, size_t workspace_bytes, void *stream);

/* FP4 (E2M1) GEMM.
 *   DSL_FMT_MXFP4: scale_a [M][K/32], scale_b [N][K/32] E8M0 bytes, fed to
 *                  the scaled MFMA; global_a/global_b unused (may be NULL).
 *   DSL_FMT_NVFP4: scale_a [M][K/16], scale_b [N][K/16] E4M3 bytes,
 *                  global_a/global_b -> one float each (device).
 * K % 32 == 0.  Replaces fp4_gemm / fp4_gemm_kernel
 * (cuda/gemm/fp4_gemm.cu:92-146). */
int dsl_fp4_gemm(const uint8_t *a, const uint8_t *b, void *c,
                 int64_t m, int64_t n, int64_t k, int64_t ldc, int out_dtype,
                 int fmt, const uint8_t *scale_a, const uint8_t *scale_b,
                 const float *global_a, const float *global_b,
                 void *workspace, size_t workspace_bytes, void *stream);

/* BF16 GEMM, fp32 accumulation: a [M][K] and b = W [N][K] bf16, both
 * K-major rows (the reference's B[K, N] is W^T: pass the storage of B.t()).
 * K % 8 == 0.  Replaces bf16_gemm / bf16_gemm_kernel
 * (triton/gemm/gemm_kernels.py:11-65, registered as gemm.bf16_gemm,
 * dispatcher/registry.py:134) and cuda/gemm/bf16_gemm.cu:41-143.
 * Needs dsl_gemm_workspace_bytes(DSL_OP_BF16, m, n, k). */
int dsl_bf16_gemm(const void *a, const void *b, void *c,
                  int64_t m, int64_t n, int64_t k, int64_t ldc, int out_dtype,
                  void *workspace, size_t workspace_bytes, void *stream);

/* Grouped FP8 GEMM over variable-size groups (MoE experts / LoRA adapters).
 * Rows group_offsets[g] .. group_offsets[g+1]-1 of x [total_rows][K]
 * multiply w[g] (w is [num_groups][N][K]); y [total_rows][ldy].
 * group_offsets is a device int32 array of num_groups+1 non-decreasing
 * entries, offsets[0] = 0, offsets[num_groups] = total_rows; empty groups
 * are skipped on the device.  The kernels clamp each entry into
 * [0, total_rows] and end a group no earlier than it starts, so a malformed
 * table never addresses outside x or y: rows no group covers are not
 * written, and groups that overlap after the clamp write their shared rows
 * in no defined order.  Per-row scale_x [total_rows] and per-channel
 * scale_w [num_groups][N]: y = acc * sx[r] * sw[g, n].
 * Replaces grouped_gemm (triton/gemm/gemm_kernels.py:164-182, fixed size)
 * and grouped_gemm_variable (cuda/gemm/grouped_gemm.cu:26-32, :150-156). */
int dsl_grouped_fp8_gemm(const uint8_t *x, const uint8_t *w, void *y,
                         const int32_t *group_offsets, int64_t num_groups,
                         int64_t total_rows, int64_t n, int64_t k, int64_t ldy,
                         int out_dtype, const float *scale_x, const float *scale_w,
                         void *stream);

/* ------------------------------------------- fused quantize producers --
 * The step before the GEMM with its output quantized in registers: the
 * bf16 result of the reference operator (fp32 math, RNE to bf16) goes
 * straight into activation codes, as dsl_quant_fp8_blocks(1, 128) /
 * dsl_quant_mxfp4 would encode it:
 *   DSL_QFMT_FP8_G128: q [rows][cols] E4M3, scales float [rows][ceil(cols/128)];
 *   DSL_QFMT_MXFP4:    q [rows][cols/2] packed E2M1, scales E8M0 [rows][cols/32].
 * y (optional, NULL for none) receives the bf16 values too, [rows][ldy].
 * cols % 8 == 0 (MXFP4: % 32), RMSNorm cols <= 32768; x, q, scales, y, weight
 * 16-byte aligned; ldx, ldy multiples of 8. */

/* RMSNorm: y = (x * (1 / sqrt(sum(x^2) / cols + eps))) * w, x [rows][ldx]
 * bf16, weight [cols] bf16 or fp32 (weight_dtype).  Replaces rmsnorm followed
 * by the activation quantizer (triton/normalization/norm_kernels.py:21-30,
 * :110-116, registered as normalization.rmsnorm, dispatcher/registry.py:146;
 * the sum's order is this build's). */
int dsl_rmsnorm_quant(const void *x, int64_t rows, int64_t cols, int64_t ldx,
                      const void *weight, int weight_dtype, float eps,
                      int qfmt, void *q, void *scales, void *y, int64_t ldy, void *stream);

/* SwiGLU: y = (g * (1 / (1 + exp(-g)))) * u with x [rows][ldx] bf16 holding
 * gate = x[:, :hidden], up = x[:, hidden:2*hidden].  Replaces swiglu followed
 * by the activation quantizer (triton/activations/activation_kernels.py:
 * 28-36, :105-115, registered as activations.swiglu, registry.py:158;
 * cuda/activations/fused_gated_activations.cu:75-90). */
int dsl_swiglu_quant(const void *x, int64_t rows, int64_t hidden, int64_t ldx,
                     int qfmt, void *q, void *scales, void *y, int64_t ldy, void *stream);

/* ---------------------------------------------------------------- LoRA --
 * y [m][ldy] fp32 = x w^T + sum_l scales[l] * (x a_l^T) b_l^T, bf16
 * operands, fp32 accumulation: x [m][k], w [n][k], a_t [num_loras*rank][k]
 * (row l*rank + r is column r of the reference's A_l [k][rank]), b_t
 * [n][num_loras*rank] (column l*rank + r is row r of B_l [rank][n]).  The
 * low-rank product t*s is carried as a bf16 pair (hi + lo), so the adapter
 * term keeps about 16 mantissa bits.  k % 8 == 0, rank*num_loras % 8 == 0.
 * Replaces lora_fused_gemm_kernel (cuda/gemm/grouped_gemm.cu:106-140).
 * Needs dsl_lora_gemm_workspace_bytes (256-byte aligned). */
size_t dsl_lora_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k, int64_t rank,
                                     int64_t num_loras);
int dsl_lora_gemm(const void *x, const void *w, const void *a_t, const void *b_t,
                  const float *scales, float *y, int64_t m, int64_t n, int64_t k,
                  int64_t rank, int64_t num_loras, int64_t ldy,
                  void *workspace, size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------ MoE glue --
 * The steps either side of dsl_grouped_fp8_gemm in an MoE layer.  The
 * reference has no counterpart (its grouped GEMM takes rows already sorted
 * by group with a host-built descriptor table, cuda/gemm/grouped_gemm.cu:
 * 26-32, :150-156); these build that input on the device and reduce its
 * output.  Assignment a = t * topk + j is token t's j-th routed expert.
 */

/* Workspace bytes dsl_moe_route needs. */
size_t dsl_moe_route_workspace_bytes(int64_t tokens, int64_t topk, int64_t num_experts);

/* topk_ids [tokens][topk] int32 -> offsets [num_experts+1] (the grouped
 * GEMM's group_offsets), dest [tokens*topk] (sorted row of each assignment,
 * -1 for ids outside [0, num_experts), which are dropped) and src_token
 * [tokens*topk] (token of sorted row r, for r < offsets[num_experts]).
 * Rows of one expert keep the assignment order (a stable counting sort). */
int dsl_moe_route(const int32_t *topk_ids, int64_t tokens, int64_t topk, int64_t num_experts,
                  int32_t *offsets, int32_t *dest, int32_t *src_token,
                  void *workspace, size_t workspace_bytes, void *stream);

/* Token t of x [tokens][ldx] bf16 quantized per row to E4M3 with scale
 * max(amax/448, 1e-12) (as dsl_quant_fp8_blocks with a 1 x k group) and
 * written to every sorted row d = dest[t*topk+j] with 0 <= d < rows: codes
 * to qx [rows][k], scale to sx [d].  With dest from dsl_moe_route, row r <
 * offsets[num_experts] then holds token src_token[r]; rows no slot names
 * are left untouched.  Each token is read once whatever topk is.
 * k % 8 == 0, k <= 32768. */
int dsl_moe_permute_quant(const void *x, int64_t tokens, int64_t k, int64_t ldx,
                          const int32_t *dest, int64_t topk, int64_t rows,
                          uint8_t *qx, float *sx, void *stream);

/* dsl_moe_permute_quant without the row copies: the codes of token t go
 * once to row t of qx [tokens][k], and only the scales to the sorted rows
 * (sx [d] for every d = dest[t*topk+j] with 0 <= d < rows).  The input of
 * dsl_moe_grouped_fp8_gemm. */
int dsl_moe_quant_tokens(const void *x, int64_t tokens, int64_t k, int64_t ldx,
                         const int32_t *dest, int64_t topk, int64_t rows,
                         uint8_t *qx, float *sx, void *stream);

/* dsl_moe_route followed by dsl_moe_quant_tokens, in one launch, for
 * decode-size batches: the same offsets [num_experts + 1], dest and
 * src_token [tokens * topk], token-major codes qx [tokens][k] and scales sx
 * at the sorted rows, bit for bit.  tokens * topk <= 1024, num_experts <=
 * 2047 and k <= 2048 (k % 8 == 0, ldx % 8 == 0); other sizes return
 * DSL_ERR_UNSUPPORTED and take the two calls.  Needs no workspace.  For
 * the MoE projection at decode size, where each of the two launches is
 * mostly latency. */
int dsl_moe_route_quant_tokens(const int32_t *topk_ids, int64_t tokens, int64_t topk,
                               int64_t num_experts, const void *x, int64_t k, int64_t ldx,
                               int32_t *offsets, int32_t *dest, int32_t *src_token, uint8_t *qx,
                               float *sx, void *stream);

/* dsl_grouped_fp8_gemm whose sorted row r reads x row src_token[r]: x is
 * the token-major [tokens][k] E4M3 of dsl_moe_quant_tokens (8x fewer bytes
 * than the permuted copy at topk = 8), sx the per-sorted-row scales it
 * wrote, src_token from dsl_moe_route (entries outside [0, tokens) are
 * clamped).  Same result as dsl_moe_permute_quant + dsl_grouped_fp8_gemm.
 * k % 128 == 0, tokens < 2^24, tokens * k < 2^32 (else
 * DSL_ERR_UNSUPPORTED). */
int dsl_moe_grouped_fp8_gemm(const uint8_t *x, int64_t tokens, const int32_t *src_token,
                             const uint8_t *w, void *y, const int32_t *offsets,
                             int64_t num_groups, int64_t total_rows, int64_t n, int64_t k,
                             int64_t ldy, int out_dtype, const float *sx, const float *sw,
                             void *stream);

/* out [tokens][ldo] = sum over j of topk_weights[t][j] * y[dest[t*topk+j]]
 * (y [rows][ldy] bf16, the grouped GEMM's output), in fp32 with slot order j
 * and a separate multiply and add per term, then bf16 or fp32.  Slots with
 * dest < 0 or >= rows are skipped.  n % 8 == 0, n <= 32768. */
int dsl_moe_combine(const void *y, int64_t rows, int64_t n, int64_t ldy, const int32_t *dest,
                    const float *topk_weights, int64_t tokens, int64_t topk,
                    void *out, int64_t ldo, int out_dtype, void *stream);

/* Workspace bytes dsl_fp8_gemm / dsl_fp4_gemm / dsl_bf16_gemm need for this
 * shape (op = DSL_OP_FP8, DSL_OP_FP4 or DSL_OP_BF16; for FP8 / FP4 the larger of the plans of the op's two
 * scale modes / FP4 formats; 0 when none is needed).  The kernel choice
 * depends on the shape and on the scale pointers' alignment; with scale
 * arrays that are not 16-byte aligned a launch may fall back to a kernel
 * that runs without split-K rather than ask for more workspace. */
size_t dsl_gemm_workspace_bytes(int op, int64_t m, int64_t n, int64_t k);

#ifdef __cplusplus
}
#endif

#endif /* DSL_GEMM_H */
