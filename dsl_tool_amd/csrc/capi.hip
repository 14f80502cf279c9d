// extern "C" entry points declared in include/dsl_gemm.h.
//
// Every entry validates its arguments on the host before enqueuing anything,
// never allocates device memory, never synchronises, never exits; failures
// return a negative status with a thread-local message.
#include <cstdarg>
#include <algorithm>
#include <cstdio>
#include <string>

#include "dsl_gemm.h"
#include "launch.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int ok() {
  g_err.clear();
  return DSL_OK;
}

int hip_status(hipError_t e, const char *what) {
  if (e == hipSuccess) return ok();
  return fail(DSL_ERR_HIP, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
}

bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Common checks of a bf16 / fp32 input matrix.
int check_input(const char *fn, const void *x, int64_t rows, int64_t cols, int64_t sr,
                int64_t sc, int x_dtype) {
  if (x_dtype != DSL_IN_BF16 && x_dtype != DSL_IN_F32)
    return fail(DSL_ERR_ARG, "%s: unknown x_dtype %d", fn, x_dtype);
  if (rows < 0 || cols < 0) return fail(DSL_ERR_ARG, "%s: negative shape (%lld, %lld)", fn,
                                        (long long)rows, (long long)cols);
  if (rows == 0 || cols == 0) return DSL_OK;
  if (!x) return fail(DSL_ERR_ARG, "%s: input pointer is NULL", fn);
  if (!aligned(x, x_dtype == DSL_IN_F32 ? 4 : 2))
    return fail(DSL_ERR_ARG, "%s: input must be aligned to its element size", fn);
  if (sr <= 0 || sc <= 0)
    return fail(DSL_ERR_ARG, "%s: strides must be positive (got %lld, %lld)", fn, (long long)sr,
                (long long)sc);
  if (rows >= (int64_t)1 << 31 || cols >= (int64_t)1 << 31)
    return fail(DSL_ERR_ARG, "%s: dimensions must be < 2^31", fn);
  return DSL_OK;
}

int check_out(const char *fn, const void *q, const char *name) {
  if (!q) return fail(DSL_ERR_ARG, "%s: %s is NULL", fn, name);
  if (!aligned(q, 16)) return fail(DSL_ERR_ARG, "%s: %s must be 16-byte aligned", fn, name);
  return DSL_OK;
}

int check_gemm_dims(const char *fn, int64_t m, int64_t n, int64_t k, int64_t ldc, int kmult,
                    int out_dtype) {
  if (m < 0 || n < 0 || k <= 0)
    return fail(DSL_ERR_ARG, "%s: need m >= 0, n >= 0, k > 0 (got %lld, %lld, %lld)", fn,
                (long long)m, (long long)n, (long long)k);
  if (m >= (int64_t)1 << 31 || n >= (int64_t)1 << 31 || k >= (int64_t)1 << 31)
    return fail(DSL_ERR_ARG, "%s: dimensions must be < 2^31", fn);
  if (k % kmult != 0)
    return fail(DSL_ERR_ARG, "%s: k=%lld must be a multiple of %d", fn, (long long)k, kmult);
  if (ldc < n) return fail(DSL_ERR_ARG, "%s: ldc=%lld < n=%lld", fn, (long long)ldc, (long long)n);
  if (out_dtype != DSL_OUT_BF16 && out_dtype != DSL_OUT_F32)
    return fail(DSL_ERR_ARG, "%s: unknown out_dtype %d", fn, out_dtype);
  return DSL_OK;
}

}  // namespace

extern "C" {

const char *dsl_last_error(void) { return g_err.c_str(); }

int dsl_abi_version(void) { return 10; }

size_t dsl_quant_workspace_bytes(int64_t rows, int64_t cols) {
  (void)rows;
  (void)cols;
  return (size_t)dsl::kMaxPartials * sizeof(float);
}

int dsl_quant_fp8_tensor(const void *x, int64_t rows, int64_t cols, int64_t sr, int64_t sc,
                         int x_dtype, uint8_t *q, float *scale, void *ws, size_t ws_bytes,
                         void *stream) {
  const char *fn = "dsl_quant_fp8_tensor";
  int rc = check_input(fn, x, rows, cols, sr, sc, x_dtype);
  if (rc) return rc;
  if (rows == 0 || cols == 0)   // no codes; the scale of amax 0, as the reference's
    return scale ? hip_status(dsl::launch_empty_scale(scale, static_cast<hipStream_t>(stream)), fn)
                 : ok();
  if ((rc = check_out(fn, q, "q"))) return rc;
  if (!scale) return fail(DSL_ERR_ARG, "%s: scale is NULL", fn);
  if (!ws || ws_bytes < dsl_quant_workspace_bytes(rows, cols))
    return fail(DSL_ERR_WORKSPACE, "%s: workspace of %zu bytes required", fn,
                dsl_quant_workspace_bytes(rows, cols));
  return hip_status(dsl::launch_quant_fp8_tensor(x, x_dtype == DSL_IN_F32, rows, cols, sr, sc, q,
                                                 scale, static_cast<float *>(ws),
                                                 static_cast<hipStream_t>(stream)),
                    fn);
}

int dsl_quant_fp8_tensor_noalloc(const void *x, int64_t rows, int64_t cols, int64_t sr,
                                 int64_t sc, int x_dtype, uint8_t *q, float *scale,
                                 void *stream) {
  const char *fn = "dsl_quant_fp8_tensor_noalloc";
  int rc = check_input(fn, x, rows, cols, sr, sc, x_dtype);
  if (rc) return rc;
  if (rows == 0 || cols == 0)   // no codes; the scale of amax 0, as the reference's
    return scale ? hip_status(dsl::launch_empty_scale(scale, static_cast<hipStream_t>(stream)), fn)
                 : ok();
  if ((rc = check_out(fn, q, "q"))) return rc;
  if (!scale) return fail(DSL_ERR_ARG, "%s: scale is NULL", fn);
  if (dsl_quant_workspace_bytes(rows, cols) > dsl::quant_scratch_bytes())
    return fail(DSL_ERR_WORKSPACE, "%s: %zu bytes of amax partials exceed the %zu held by the library",
                fn, dsl_quant_workspace_bytes(rows, cols), dsl::quant_scratch_bytes());
  hipError_t e = hipSuccess;
  float *partials = dsl::quant_scratch(&e);
  if (!partials) return hip_status(e, fn);
  return hip_status(dsl::launch_quant_fp8_tensor(x, x_dtype == DSL_IN_F32, rows, cols, sr, sc, q,
                                                 scale, partials, static_cast<hipStream_t>(stream)),
                    fn);
}

int dsl_quant_fp8_blocks(const void *x, int64_t rows, int64_t cols, int64_t sr, int64_t sc,
                         int x_dtype, int64_t gr, int64_t gc, uint8_t *q, float *scales,
                         void *stream) {
  const char *fn = "dsl_quant_fp8_blocks";
  int rc = check_input(fn, x, rows, cols, sr, sc, x_dtype);
  if (rc) return rc;
  if (gr <= 0 || gc <= 0)
    return fail(DSL_ERR_ARG, "%s: group sizes must be positive (got %lld x %lld)", fn,
                (long long)gr, (long long)gc);
  if (rows == 0 || cols == 0) return ok();
  if ((rc = check_out(fn, q, "q"))) return rc;
  if (!scales) return fail(DSL_ERR_ARG, "%s: scales is NULL", fn);
  return hip_status(dsl::launch_quant_fp8_blocks(x, x_dtype == DSL_IN_F32, rows, cols, sr, sc, gr,
                                                 gc, q, scales, static_cast<hipStream_t>(stream)),
                    fn);
}

int dsl_quant_mxfp4(const void *x, int64_t rows, int64_t cols, int64_t sr, int64_t sc,
                    int x_dtype, uint8_t *q, uint8_t *e8m0, void *stream) {
  const char *fn = "dsl_quant_mxfp4";
  int rc = check_input(fn, x, rows, cols, sr, sc, x_dtype);
  if (rc) return rc;
  if (cols % 32 != 0)
    return fail(DSL_ERR_ARG, "%s: cols=%lld must be a multiple of 32", fn, (long long)cols);
  if (rows == 0 || cols == 0) return ok();
  if ((rc = check_out(fn, q, "q_packed"))) return rc;
  if (!e8m0) return fail(DSL_ERR_ARG, "%s: e8m0 is NULL", fn);
  return hip_status(dsl::launch_quant_mxfp4(x, x_dtype == DSL_IN_F32, rows, cols, sr, sc,
                                            q, e8m0, static_cast<hipStream_t>(stream)),
                    fn);
}

int dsl_quant_nvfp4(const void *x, int64_t rows, int64_t cols, int64_t sr, int64_t sc,
                    int x_dtype, uint8_t *q, uint8_t *e4m3s, float *gscale, void *ws,
                    size_t ws_bytes, void *stream) {
  const char *fn = "dsl_quant_nvfp4";
  int rc = check_input(fn, x, rows, cols, sr, sc, x_dtype);
  if (rc) return rc;
  if (cols % 16 != 0)
    return fail(DSL_ERR_ARG, "%s: cols=%lld must be a multiple of 16", fn, (long long)cols);
  if (rows == 0 || cols == 0)   // no codes; the global scale of amax 0
    return gscale ? hip_status(dsl::launch_empty_scale(gscale, static_cast<hipStream_t>(stream)), fn)
                  : ok();
  if ((rc = check_out(fn, q, "q_packed"))) return rc;
  if (!e4m3s || !gscale) return fail(DSL_ERR_ARG, "%s: scale output is NULL", fn);
  if (!ws || ws_bytes < dsl_quant_workspace_bytes(rows, cols))
    return fail(DSL_ERR_WORKSPACE, "%s: workspace of %zu bytes required", fn,
                dsl_quant_workspace_bytes(rows, cols));
  return hip_status(dsl::launch_quant_nvfp4(x, x_dtype == DSL_IN_F32, rows, cols, sr, sc,
                                            q, e4m3s, gscale, static_cast<float *>(ws),
                                            static_cast<hipStream_t>(stream)),
                    fn);
}

size_t dsl_gemm_workspace_bytes(int op, int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0) return 0;
  // the op does not say which scale mode / FP4 format follows, so report
  // the larger of the two plans
  auto mx = [](size_t a, size_t b) { return a > b ? a : b; };
  if (op == DSL_OP_FP8)
    return mx(mx(dsl::gemm_workspace_bytes(dsl::MODE_FP8_TENSOR, m, n, k),
                 dsl::gemm_workspace_bytes(dsl::MODE_FP8_BLOCK, m, n, k)),
              dsl::gemm_workspace_bytes(dsl::MODE_FP8_GCOL, m, n, k));
  if (op == DSL_OP_FP4)
    return mx(dsl::gemm_workspace_bytes(dsl::MODE_MXFP4, m, n, k),
              dsl::gemm_workspace_bytes(dsl::MODE_NVFP4, m, n, k));
  if (op == DSL_OP_BF16) return dsl::gemm_workspace_bytes(dsl::MODE_BF16, m, n, k);
  return 0;
}

static int run_gemm(const char *fn, int mode, const uint8_t *a, const uint8_t *b, void *c,
                    int64_t m, int64_t n, int64_t k, int64_t ldc, int out_dtype, const void *sa,
                    const void *sb, const float *ga, const float *gb, void *ws, size_t ws_bytes,
                    void *stream) {
  if (m == 0 || n == 0) return ok();
  int rc;
  if ((rc = check_out(fn, a, "a")) || (rc = check_out(fn, b, "b"))) return rc;
  if (!c) return fail(DSL_ERR_ARG, "%s: c is NULL", fn);
  if (!aligned(c, out_dtype == DSL_OUT_F32 ? 4 : 2))
    return fail(DSL_ERR_ARG, "%s: c is misaligned", fn);
  const size_t need = dsl::gemm_workspace_bytes(mode, m, n, k);
  if (need && (!ws || ws_bytes < need || !aligned(ws, 16)))
    return fail(DSL_ERR_WORKSPACE, "%s: workspace of %zu bytes (16-B aligned) required", fn, need);
  dsl::GemmArgs p;
  p.a = a;
  p.b = b;
  p.c = c;
  p.M = (int)m;
  p.N = (int)n;
  p.K = (int)k;
  p.Kb = (mode == dsl::MODE_MXFP4 || mode == dsl::MODE_NVFP4) ? (int)(k / 2)
                                                                : (mode == dsl::MODE_BF16 ? (int)(2 * k) : (int)k);
  p.ldc = ldc;
  p.sa = sa;
  p.sb = sb;
  p.ga = ga;
  p.gb = gb;
  p.ws = static_cast<float *>(ws);
  p.ws_bytes = ws ? ws_bytes : 0;
  p.ksplit = 1;
  p.out_f32 = out_dtype == DSL_OUT_F32;
  p.accumulate = 0;
  p.a2 = p.b2 = nullptr;
  p.Kb2 = 0;
  return hip_status(dsl::launch_gemm(mode, p, static_cast<hipStream_t>(stream)), fn);
}

int dsl_fp8_gemm(const uint8_t *a, const uint8_t *b, void *c, int64_t m, int64_t n, int64_t k,
                 int64_t ldc, int out_dtype, int scale_mode, const float *scale_a,
                 const float *scale_b, void *ws, size_t ws_bytes, void *stream) {
  const char *fn = "dsl_fp8_gemm";
  int rc = check_gemm_dims(fn, m, n, k, ldc, 16, out_dtype);
  if (rc) return rc;
  if (scale_mode != DSL_SCALE_TENSOR && scale_mode != DSL_SCALE_BLOCK128 &&
      scale_mode != DSL_SCALE_GROUP128)
    return fail(DSL_ERR_ARG, "%s: unknown scale_mode %d", fn, scale_mode);
  // an empty product reads nothing (its block scale arrays may be empty, i.e. NULL)
  if (m == 0 || n == 0) return ok();
  if (!scale_a || !scale_b) return fail(DSL_ERR_ARG, "%s: scale pointers must not be NULL", fn);
  if (scale_mode == DSL_SCALE_TENSOR)
    return run_gemm(fn, dsl::MODE_FP8_TENSOR, a, b, c, m, n, k, ldc, out_dtype, nullptr, nullptr,
                    scale_a, scale_b, ws, ws_bytes, stream);
  if (scale_mode == DSL_SCALE_BLOCK128)
    return run_gemm(fn, dsl::MODE_FP8_BLOCK, a, b, c, m, n, k, ldc, out_dtype, scale_a, scale_b,
                    nullptr, nullptr, ws, ws_bytes, stream);
  if (scale_mode == DSL_SCALE_GROUP128) {
    if (!aligned(scale_a, 4) || !aligned(scale_b, 4))
      return fail(DSL_ERR_ARG, "%s: scale arrays must be 4-byte aligned", fn);
    return run_gemm(fn, dsl::MODE_FP8_GCOL, a, b, c, m, n, k, ldc, out_dtype, scale_a, scale_b,
                    nullptr, nullptr, ws, ws_bytes, stream);
  }
  return fail(DSL_ERR_ARG, "%s: unknown scale_mode %d", fn, scale_mode);
}

int dsl_fp4_gemm(const uint8_t *a, const uint8_t *b, void *c, int64_t m, int64_t n, int64_t k,
                 int64_t ldc, int out_dtype, int fmt, const uint8_t *scale_a,
                 const uint8_t *scale_b, const float *global_a, const float *global_b, void *ws,
                 size_t ws_bytes, void *stream) {
  const char *fn = "dsl_fp4_gemm";
  int rc = check_gemm_dims(fn, m, n, k, ldc, 32, out_dtype);
  if (rc) return rc;
  if (fmt != DSL_FMT_MXFP4 && fmt != DSL_FMT_NVFP4)
    return fail(DSL_ERR_ARG, "%s: unknown fmt %d", fn, fmt);
  // an empty product reads nothing (its scale arrays may be empty, i.e. NULL)
  if (m == 0 || n == 0) return ok();
  if (!scale_a || !scale_b) return fail(DSL_ERR_ARG, "%s: scale pointers must not be NULL", fn);
  if (fmt == DSL_FMT_MXFP4)
    return run_gemm(fn, dsl::MODE_MXFP4, a, b, c, m, n, k, ldc, out_dtype, scale_a, scale_b,
                    nullptr, nullptr, ws, ws_bytes, stream);
  if (fmt == DSL_FMT_NVFP4) {
    if (!global_a || !global_b)
      return fail(DSL_ERR_ARG, "%s: NVFP4 needs global_a and global_b", fn);
    return run_gemm(fn, dsl::MODE_NVFP4, a, b, c, m, n, k, ldc, out_dtype, scale_a, scale_b,
                    global_a, global_b, ws, ws_bytes, stream);
  }
  return fail(DSL_ERR_ARG, "%s: unknown fmt %d", fn, fmt);
}

int dsl_bf16_gemm(const void *a, const void *b, void *c, int64_t m, int64_t n, int64_t k,
                  int64_t ldc, int out_dtype, void *ws, size_t ws_bytes, void *stream) {
  const char *fn = "dsl_bf16_gemm";
  int rc = check_gemm_dims(fn, m, n, k, ldc, 8, out_dtype);
  if (rc) return rc;
  if (k >= (int64_t)1 << 30) return fail(DSL_ERR_ARG, "%s: k must be < 2^30", fn);
  return run_gemm(fn, dsl::MODE_BF16, static_cast<const uint8_t *>(a),
                  static_cast<const uint8_t *>(b), c, m, n, k, ldc, out_dtype, nullptr, nullptr,
                  nullptr, nullptr, ws, ws_bytes, stream);
}

int dsl_grouped_fp8_gemm(const uint8_t *x, const uint8_t *w, void *y, const int32_t *offsets,
                         int64_t num_groups, int64_t total_rows, int64_t n, int64_t k,
                         int64_t ldy, int out_dtype, const float *sx, const float *sw,
                         void *stream) {
  const char *fn = "dsl_grouped_fp8_gemm";
  if (num_groups <= 0 || num_groups > 2048)
    return fail(DSL_ERR_ARG, "%s: num_groups=%lld must be in [1, 2048]", fn,
                (long long)num_groups);
  int rc = check_gemm_dims(fn, total_rows, n, k, ldy, 16, out_dtype);
  if (rc) return rc;
  if (total_rows == 0 || n == 0) return ok();
  if ((rc = check_out(fn, x, "x")) || (rc = check_out(fn, w, "w"))) return rc;
  if (!y || !offsets || !sx || !sw) return fail(DSL_ERR_ARG, "%s: NULL pointer argument", fn);
  dsl::GroupedArgs p;
  p.x = x;
  p.w = w;
  p.y = y;
  p.offsets = offsets;
  p.G = (int)num_groups;
  p.rows = (int)total_rows;
  p.N = (int)n;
  p.K = (int)k;
  p.ldy = ldy;
  p.sx = sx;
  p.sw = sw;
  p.out_f32 = out_dtype == DSL_OUT_F32;
  return hip_status(dsl::launch_grouped_fp8(p, static_cast<hipStream_t>(stream)), fn);
}

static int run_fused(const char *fn, int prod, const void *x, int64_t rows, int64_t cols,
                     int64_t ldx, const void *w, int w_dtype, float eps, int qfmt, void *q,
                     void *scales, void *y, int64_t ldy, void *stream) {
  if (rows < 0 || cols <= 0)
    return fail(DSL_ERR_ARG, "%s: need rows >= 0 and cols > 0 (got %lld, %lld)", fn,
                (long long)rows, (long long)cols);
  if (rows >= (int64_t)1 << 31) return fail(DSL_ERR_ARG, "%s: rows must be < 2^31", fn);
  if (qfmt != DSL_QFMT_FP8_G128 && qfmt != DSL_QFMT_MXFP4)
    return fail(DSL_ERR_ARG, "%s: unknown qfmt %d", fn, qfmt);
  const int mult = qfmt == DSL_QFMT_MXFP4 ? 32 : 8;
  if (cols % mult != 0)
    return fail(DSL_ERR_ARG, "%s: cols=%lld must be a multiple of %d", fn, (long long)cols, mult);
  if (prod == dsl::PROD_RMSNORM && cols > 32768)
    return fail(DSL_ERR_UNSUPPORTED, "%s: cols=%lld > 32768 (one workgroup holds a row)", fn,
                (long long)cols);
  if (rows * ((cols + 127) / 128) >= ((int64_t)1 << 32) / 2)
    return fail(DSL_ERR_ARG, "%s: too many scale groups", fn);
  const int64_t need = prod == dsl::PROD_SWIGLU ? 2 * cols : cols;
  if (ldx < need || ldx % 8 != 0)
    return fail(DSL_ERR_ARG, "%s: ldx=%lld must be >= %lld and a multiple of 8", fn,
                (long long)ldx, (long long)need);
  if (rows == 0) return ok();
  int rc;
  if ((rc = check_out(fn, x, "x")) || (rc = check_out(fn, q, "q")) ||
      (rc = check_out(fn, scales, "scales")))
    return rc;
  if (prod == dsl::PROD_RMSNORM) {
    if ((rc = check_out(fn, w, "weight"))) return rc;
    if (w_dtype != DSL_W_BF16 && w_dtype != DSL_W_F32)
      return fail(DSL_ERR_ARG, "%s: unknown weight dtype %d", fn, w_dtype);
    if (!(eps >= 0.f)) return fail(DSL_ERR_ARG, "%s: eps must be >= 0", fn);
  }
  if (y) {
    if ((rc = check_out(fn, y, "y"))) return rc;
    if (ldy < cols || ldy % 8 != 0)
      return fail(DSL_ERR_ARG, "%s: ldy=%lld must be >= cols and a multiple of 8", fn,
                  (long long)ldy);
  }
  dsl::FusedArgs p;
  p.x = static_cast<const uint16_t *>(x);
  p.ldx = ldx;
  p.w = w;
  p.w_f32 = w_dtype == DSL_W_F32;
  p.rows = (int)rows;
  p.cols = (int)cols;
  p.eps = eps;
  p.q = static_cast<uint8_t *>(q);
  p.scales = scales;
  p.y = static_cast<uint16_t *>(y);
  p.ldy = ldy;
  return hip_status(dsl::launch_fused_quant(prod, qfmt == DSL_QFMT_MXFP4 ? dsl::QF_MXFP4
                                                                         : dsl::QF_FP8_G128,
                                            p, static_cast<hipStream_t>(stream)),
                    fn);
}

int dsl_rmsnorm_quant(const void *x, int64_t rows, int64_t cols, int64_t ldx, const void *weight,
                      int weight_dtype, float eps, int qfmt, void *q, void *scales, void *y,
                      int64_t ldy, void *stream) {
  return run_fused("dsl_rmsnorm_quant", dsl::PROD_RMSNORM, x, rows, cols, ldx, weight,
                   weight_dtype, eps, qfmt, q, scales, y, ldy, stream);
}

int dsl_swiglu_quant(const void *x, int64_t rows, int64_t hidden, int64_t ldx, int qfmt, void *q,
                     void *scales, void *y, int64_t ldy, void *stream) {
  return run_fused("dsl_swiglu_quant", dsl::PROD_SWIGLU, x, rows, hidden, ldx, nullptr,
                   DSL_W_BF16, 0.f, qfmt, q, scales, y, ldy, stream);
}

}  // extern "C"

namespace {

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct LoraPlan {
  int64_t ld2;                 // padded columns of hi | lo and of B^T | B^T
  bool tt;                     // T^T = A^T X^T on the streaming kernel, split in its epilogue
  bool one_pass;               // adapter term as a second K segment of the persistent kernel
  int rep;                     // ... reading B^T twice: its pairs per row (else 0: B^T | B^T copied)
  bool valu;                   // few tokens: fp32 T and the add on the vector ALUs
  bool vt;                     // T (as hi | lo) on the vector ALUs, the add on MFMA
  size_t t32, ws, t2, b2, total;
};

// Most tokens for the vector-ALU add (DSL_LORA_VALU_MAX_M overrides it, for
// tuning).
int64_t lora_valu_max_m() {
  static const int64_t v = [] {
    const char *e = getenv("DSL_LORA_VALU_MAX_M");
    return e ? (int64_t)atoll(e) : (int64_t)2;
  }();
  return v;
}

LoraPlan lora_plan(int64_t m, int64_t n, int64_t k, int64_t lr) {
  LoraPlan p;
  p.ld2 = (2 * lr + 63) / 64 * 64;
  // T^T = A^T X^T on the streaming kernel when the adapter columns are few
  // enough to be its skinny M; its epilogue writes hi | lo itself.
  p.tt = lr <= 256 && dsl::stream_supported(dsl::MODE_BF16, (int)lr, (int)m, (int)k, (int)(2 * k), true);
  // One pass (the adapter term as a second K segment of the persistent
  // kernel) unless both the base GEMM and the adapter add would take the
  // streaming kernel or the 128x128 pipelined tiles (up to 1024 rows at
  // small N, and where one round of 128x128 tiles holds the problem): then
  // the base GEMM takes its own kernel and the adapter term is added by a
  // second pass into the fp32 output (N=K=4096, 4 x rank 16: M=16 79.9 us
  // in one pass, the base GEMM alone 7.3; M=512 100.2 in one pass, 58.8 in
  // two; M=768, where the add would run on the register-staged tiles, 115.2
  // in two).
  const bool both_stream = dsl::gemm_routes_to_stream(dsl::MODE_BF16, m, n, k, true) &&
                           dsl::gemm_routes_to_stream(dsl::MODE_BF16, m, n, p.ld2, true, true);
  p.one_pass = dsl::persist_supported(dsl::MODE_BF16, (int)m, (int)n, (int)k, (int)(2 * (k + p.ld2)), true) &&
               (2 * k) % 128 == 0 && m > 256 && !both_stream;
  // hi | lo against B^T | B^T without the copy (one pass only): B^T's rows
  // must be whole pairs (64 bf16), a power of two of them, filling ld2 / 2
  // Up to 256 tokens T comes from the vector-ALU kernel, which splits A^T's
  // rows over workgroups (the streaming kernel's T^T runs the 64 adapter rows
  // as one row block: one workgroup streams all of A^T); for the fewest
  // tokens the add is on the vector ALUs too, in fp32.
  p.vt = !p.one_pass && m <= 256 && dsl::lora_valu_supported(m, k, lr);
  p.valu = p.vt && m <= lora_valu_max_m();
  if (p.vt) p.tt = false;
  if (p.valu) {
    p.tt = p.one_pass = false;
    p.rep = 0;
    p.t32 = align256((size_t)(m * lr) * 4);
    p.ws = align256(dsl::gemm_workspace_bytes(dsl::MODE_BF16, m, n, k));
    p.t2 = p.b2 = 0;
    p.total = p.t32 + p.ws;
    return p;
  }
  const int64_t pr = lr / 64;
  p.rep = (p.one_pass && lr % 64 == 0 && (pr & (pr - 1)) == 0 && p.ld2 == 2 * lr) ? (int)pr : 0;
  const size_t ws1 = dsl::gemm_workspace_bytes(dsl::MODE_BF16, m, lr, k);
  const size_t ws3 = dsl::gemm_workspace_bytes(dsl::MODE_BF16, m, n, k);
  const size_t ws4 = dsl::gemm_workspace_bytes(dsl::MODE_BF16, m, n, p.ld2, true);
  p.t32 = (p.tt || p.vt) ? 0 : align256((size_t)(m * lr) * 4);
  p.ws = align256(std::max(ws1, std::max(ws3, ws4)));
  p.t2 = align256((size_t)(m * p.ld2) * 2);
  p.b2 = p.rep ? 0 : align256((size_t)(n * p.ld2) * 2);
  p.total = p.t32 + p.ws + p.t2 + p.b2;
  return p;
}

dsl::GemmArgs bf16_args(const void *a, const void *b, void *c, int64_t m, int64_t n, int64_t k,
                        int64_t ldc, bool accumulate, void *ws, size_t ws_bytes) {
  dsl::GemmArgs p;
  p.a = static_cast<const uint8_t *>(a);
  p.b = static_cast<const uint8_t *>(b);
  p.c = c;
  p.M = (int)m;
  p.N = (int)n;
  p.K = (int)k;
  p.Kb = (int)(2 * k);
  p.ldc = ldc;
  p.sa = p.sb = nullptr;
  p.ga = p.gb = nullptr;
  p.ws = static_cast<float *>(ws);
  p.ws_bytes = ws_bytes;
  p.ksplit = 1;
  p.out_f32 = 1;
  p.accumulate = accumulate ? 1 : 0;
  p.a2 = p.b2 = nullptr;
  p.Kb2 = 0;
  return p;
}

}  // namespace

extern "C" {

size_t dsl_lora_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k, int64_t rank,
                                     int64_t num_loras) {
  if (m <= 0 || n <= 0 || k <= 0 || rank <= 0 || num_loras <= 0) return 0;
  return lora_plan(m, n, k, rank * num_loras).total;
}

int dsl_lora_gemm(const void *x, const void *w, const void *a_t, const void *b_t,
                  const float *scales, float *y, int64_t m, int64_t n, int64_t k, int64_t rank,
                  int64_t num_loras, int64_t ldy, void *ws, size_t ws_bytes, void *stream) {
  const char *fn = "dsl_lora_gemm";
  if (rank <= 0 || num_loras <= 0) return fail(DSL_ERR_ARG, "%s: rank and num_loras must be > 0", fn);
  const int64_t lr = rank * num_loras;
  int rc = check_gemm_dims(fn, m, n, k, ldy, 8, DSL_OUT_F32);
  if (rc) return rc;
  if (lr % 8 != 0 || lr >= ((int64_t)1 << 20))
    return fail(DSL_ERR_ARG, "%s: rank * num_loras = %lld must be a multiple of 8", fn, (long long)lr);
  if (m == 0 || n == 0) return ok();
  if ((rc = check_out(fn, x, "x")) || (rc = check_out(fn, w, "w")) || (rc = check_out(fn, a_t, "a_t")) ||
      (rc = check_out(fn, b_t, "b_t")))
    return rc;
  if (!scales || !y) return fail(DSL_ERR_ARG, "%s: NULL pointer argument", fn);
  if (!aligned(y, 4)) return fail(DSL_ERR_ARG, "%s: y is misaligned", fn);
  const LoraPlan pl = lora_plan(m, n, k, lr);
  if (!ws || ws_bytes < pl.total || !aligned(ws, 256))
    return fail(DSL_ERR_WORKSPACE, "%s: workspace of %zu bytes (256-B aligned) required", fn, pl.total);
  uint8_t *base = static_cast<uint8_t *>(ws);
  float *t32 = reinterpret_cast<float *>(base);
  void *gws = base + pl.t32;
  uint16_t *t2 = reinterpret_cast<uint16_t *>(base + pl.t32 + pl.ws);
  uint16_t *b2 = reinterpret_cast<uint16_t *>(base + pl.t32 + pl.ws + pl.t2);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (pl.valu) {   // few tokens: fp32 T*s, the base GEMM, then Y += T*s B^T
    e = dsl::launch_lora_t(static_cast<const uint16_t *>(x), static_cast<const uint16_t *>(a_t),
                           (int)m, (int)k, (int)lr, (int)rank, scales, t32, nullptr, 0, st);
    if (e == hipSuccess) e = dsl::launch_gemm(dsl::MODE_BF16, bf16_args(x, w, y, m, n, k, ldy, false, gws, pl.ws), st);
    if (e == hipSuccess)
      e = dsl::launch_lora_apply(t32, static_cast<const uint16_t *>(b_t), y, (int)m, (int)n, (int)lr,
                                 ldy, st);
    return hip_status(e, fn);
  }
  // T = X A^T.  With at most 256 adapter columns it is computed as
  // T^T = A^T X^T: the adapter rows are then the skinny M of the streaming
  // kernel, which reads X once in one launch and whose epilogue writes
  // hi | lo of T*s (transposed back) straight into t2; otherwise (and when
  // K does not suit that kernel) T comes from the register-staged tiles over
  // the workspace and a separate split pass.
  if (pl.vt) {
    e = dsl::launch_lora_t(static_cast<const uint16_t *>(x), static_cast<const uint16_t *>(a_t),
                           (int)m, (int)k, (int)lr, (int)rank, scales, nullptr, t2, (int)pl.ld2, st);
  } else if (pl.tt) {
    dsl::GemmArgs tg = bf16_args(a_t, x, t2, lr, m, k, pl.ld2, false, nullptr, 0);
    tg.out_f32 = 0;
    tg.lora_scales = scales;
    tg.lora_rank = (int)rank;
    e = dsl::launch_gemm(dsl::MODE_BF16, tg, st);
  } else {
    e = dsl::launch_gemm(dsl::MODE_BF16, bf16_args(x, a_t, t32, m, lr, k, lr, false, gws, pl.ws), st);
    if (e == hipSuccess)
      e = dsl::launch_lora_split(t32, (int)m, (int)lr, (int)pl.ld2, (int)rank, scales, t2, st);
  }
  if (e == hipSuccess && !pl.rep)
    e = dsl::launch_lora_dup(static_cast<const uint16_t *>(b_t), (int)n, (int)lr, (int)pl.ld2, b2, st);
  if (e != hipSuccess) return hip_status(e, fn);
  dsl::GemmArgs g = bf16_args(x, w, y, m, n, k, ldy, false, gws, pl.ws);
  if (pl.one_pass) {
    // one pass: the adapter columns are a second K segment of every row
    g.a2 = reinterpret_cast<const uint8_t *>(t2);
    g.Kb2 = (int)(2 * pl.ld2);
    if (pl.rep) {            // B^T | B^T read from B^T itself
      g.b2 = static_cast<const uint8_t *>(b_t);
      g.ldb2 = (int)(2 * lr);
      g.rep2 = pl.rep;
    } else {
      g.b2 = reinterpret_cast<const uint8_t *>(b2);
    }
    e = dsl::launch_gemm(dsl::MODE_BF16, g, st);
  } else {
    e = dsl::launch_gemm(dsl::MODE_BF16, g, st);
    if (e == hipSuccess)
      e = dsl::launch_gemm(dsl::MODE_BF16, bf16_args(t2, b2, y, m, n, pl.ld2, ldy, true, gws, pl.ws), st);
  }
  return hip_status(e, fn);
}

size_t dsl_moe_route_workspace_bytes(int64_t tokens, int64_t topk, int64_t num_experts) {
  // tokens == 0 still needs one block's histogram (the offsets are written)
  if (tokens < 0 || topk <= 0 || num_experts <= 0) return 0;
  return dsl::moe_route_workspace_bytes(tokens * topk, num_experts);
}

int dsl_moe_route(const int32_t *topk_ids, int64_t tokens, int64_t topk, int64_t num_experts,
                  int32_t *offsets, int32_t *dest, int32_t *src_token, void *ws, size_t ws_bytes,
                  void *stream) {
  const char *fn = "dsl_moe_route";
  if (tokens < 0 || topk <= 0 || num_experts <= 0 || num_experts > dsl::kMaxGroups)
    return fail(DSL_ERR_ARG, "%s: need tokens >= 0, topk > 0, 1 <= num_experts <= %d", fn,
                dsl::kMaxGroups);
  if (tokens * topk >= ((int64_t)1 << 31)) return fail(DSL_ERR_ARG, "%s: too many assignments", fn);
  if (!offsets) return fail(DSL_ERR_ARG, "%s: offsets is NULL", fn);
  const int64_t n = tokens * topk;
  if (n > 0 && (!topk_ids || !dest || !src_token))
    return fail(DSL_ERR_ARG, "%s: NULL pointer argument", fn);
  const size_t need = dsl::moe_route_workspace_bytes(n, num_experts);
  if (!ws || ws_bytes < need)
    return fail(DSL_ERR_WORKSPACE, "%s: workspace of %zu bytes required", fn, need);
  return hip_status(dsl::launch_moe_route(topk_ids, (int)n, (int)topk, (int)num_experts, offsets,
                                          dest, src_token, static_cast<int32_t *>(ws),
                                          static_cast<hipStream_t>(stream)),
                    fn);
}

static int run_moe_quant(const char *fn, const void *x, int64_t tokens, int64_t k, int64_t ldx,
                         const int32_t *dest, int64_t topk, int64_t rows, uint8_t *qx, float *sx,
                         bool tok_major, void *stream) {
  if (tokens < 0 || rows < 0 || k <= 0 || topk <= 0) return fail(DSL_ERR_ARG, "%s: bad sizes", fn);
  if (k % 8 != 0 || k > 32768)
    return fail(DSL_ERR_ARG, "%s: k=%lld must be a multiple of 8 and <= 32768", fn, (long long)k);
  if (ldx < k || ldx % 8 != 0) return fail(DSL_ERR_ARG, "%s: ldx must be >= k, a multiple of 8", fn);
  if (rows >= ((int64_t)1 << 31) || tokens >= ((int64_t)1 << 31) || tokens * topk >= ((int64_t)1 << 31))
    return fail(DSL_ERR_ARG, "%s: too many rows", fn);
  if (tokens == 0 || (rows == 0 && !tok_major)) return ok();
  int rc;
  if ((rc = check_out(fn, x, "x")) || (rc = check_out(fn, qx, "qx"))) return rc;
  if (!dest || (rows > 0 && !sx)) return fail(DSL_ERR_ARG, "%s: NULL pointer argument", fn);
  return hip_status(dsl::launch_moe_permute_quant(static_cast<const uint16_t *>(x), ldx, (int)k,
                                                  (int)tokens, dest, (int)topk, (int)rows, qx, sx,
                                                  tok_major, static_cast<hipStream_t>(stream)),
                    fn);
}

int dsl_moe_permute_quant(const void *x, int64_t tokens, int64_t k, int64_t ldx,
                          const int32_t *dest, int64_t topk, int64_t rows, uint8_t *qx, float *sx,
                          void *stream) {
  return run_moe_quant("dsl_moe_permute_quant", x, tokens, k, ldx, dest, topk, rows, qx, sx, false,
                       stream);
}

int dsl_moe_quant_tokens(const void *x, int64_t tokens, int64_t k, int64_t ldx,
                         const int32_t *dest, int64_t topk, int64_t rows, uint8_t *qx, float *sx,
                         void *stream) {
  return run_moe_quant("dsl_moe_quant_tokens", x, tokens, k, ldx, dest, topk, rows, qx, sx, true,
                       stream);
}

int dsl_moe_route_quant_tokens(const int32_t *topk_ids, int64_t tokens, int64_t topk,
                               int64_t num_experts, const void *x, int64_t k, int64_t ldx,
                               int32_t *offsets, int32_t *dest, int32_t *src_token, uint8_t *qx,
                               float *sx, void *stream) {
  const char *fn = "dsl_moe_route_quant_tokens";
  if (tokens < 0 || topk <= 0 || num_experts <= 0 || num_experts > dsl::kMaxGroups)
    return fail(DSL_ERR_ARG, "%s: need tokens >= 0, topk > 0, 1 <= num_experts <= %d", fn,
                dsl::kMaxGroups);
  if (k <= 0 || k % 8 != 0 || ldx < k || ldx % 8 != 0)
    return fail(DSL_ERR_ARG, "%s: k must be a positive multiple of 8, ldx >= k a multiple of 8", fn);
  if (tokens * topk >= ((int64_t)1 << 31)) return fail(DSL_ERR_ARG, "%s: too many assignments", fn);
  if (!offsets) return fail(DSL_ERR_ARG, "%s: offsets is NULL", fn);
  const int64_t n = tokens * topk;
  if (n > dsl::moe_route_quant_max_assignments || num_experts > 2047 || k > 2048)
    return fail(DSL_ERR_UNSUPPORTED,
                "%s: one launch covers tokens * topk <= %d, num_experts <= 2047, k <= 2048 "
                "(dsl_moe_route + dsl_moe_quant_tokens cover the rest)", fn,
                dsl::moe_route_quant_max_assignments);
  if (tokens == 0)   // no token: the zero offsets only (the one-wave route needs no workspace)
    return hip_status(dsl::launch_moe_route(topk_ids, 0, (int)topk, (int)num_experts, offsets,
                                            dest, src_token, nullptr,
                                            static_cast<hipStream_t>(stream)), fn);
  int rc;
  if ((rc = check_out(fn, x, "x")) || (rc = check_out(fn, qx, "qx"))) return rc;
  if (!topk_ids || !dest || !src_token || !sx) return fail(DSL_ERR_ARG, "%s: NULL pointer argument", fn);
  return hip_status(dsl::launch_moe_route_quant(topk_ids, (int)n, (int)topk, (int)num_experts,
                                                static_cast<const uint16_t *>(x), ldx, (int)k,
                                                (int)tokens, offsets, dest, src_token, qx, sx,
                                                static_cast<hipStream_t>(stream)),
                    fn);
}

int dsl_moe_grouped_fp8_gemm(const uint8_t *x, int64_t tokens, const int32_t *src_token,
                             const uint8_t *w, void *y, const int32_t *offsets, int64_t num_groups,
                             int64_t total_rows, int64_t n, int64_t k, int64_t ldy, int out_dtype,
                             const float *sx, const float *sw, void *stream) {
  const char *fn = "dsl_moe_grouped_fp8_gemm";
  if (num_groups <= 0 || num_groups > 2048)
    return fail(DSL_ERR_ARG, "%s: num_groups=%lld must be in [1, 2048]", fn,
                (long long)num_groups);
  int rc = check_gemm_dims(fn, total_rows, n, k, ldy, 16, out_dtype);
  if (rc) return rc;
  if (tokens < 0 || tokens >= ((int64_t)1 << 24))
    return fail(DSL_ERR_ARG, "%s: tokens=%lld must be in [0, 2^24)", fn, (long long)tokens);
  if (total_rows == 0 || n == 0) return ok();
  if (tokens == 0) return fail(DSL_ERR_ARG, "%s: rows to compute but no tokens", fn);
  if ((rc = check_out(fn, x, "x")) || (rc = check_out(fn, w, "w"))) return rc;
  if (!y || !offsets || !sx || !sw || !src_token)
    return fail(DSL_ERR_ARG, "%s: NULL pointer argument", fn);
  if (k % 128 != 0 || tokens * k >= ((int64_t)1 << 32))
    return fail(DSL_ERR_UNSUPPORTED, "%s: needs k %% 128 == 0 and tokens * k < 2^32", fn);
  dsl::GroupedArgs p;
  p.x = x;
  p.w = w;
  p.y = y;
  p.offsets = offsets;
  p.G = (int)num_groups;
  p.rows = (int)total_rows;
  p.N = (int)n;
  p.K = (int)k;
  p.ldy = ldy;
  p.sx = sx;
  p.sw = sw;
  p.out_f32 = out_dtype == DSL_OUT_F32;
  p.arow = src_token;
  p.xrows = (int)tokens;
  return hip_status(dsl::launch_grouped_fp8(p, static_cast<hipStream_t>(stream)), fn);
}

int dsl_moe_combine(const void *y, int64_t rows, int64_t n, int64_t ldy, const int32_t *dest,
                    const float *topk_weights, int64_t tokens, int64_t topk, void *out,
                    int64_t ldo, int out_dtype, void *stream) {
  const char *fn = "dsl_moe_combine";
  if (rows < 0 || tokens < 0 || topk <= 0 || n <= 0) return fail(DSL_ERR_ARG, "%s: bad sizes", fn);
  if (n % 8 != 0 || n > 32768)
    return fail(DSL_ERR_ARG, "%s: n=%lld must be a multiple of 8 and <= 32768", fn, (long long)n);
  if (ldy < n || ldy % 8 != 0 || ldo < n || ldo % 8 != 0)
    return fail(DSL_ERR_ARG, "%s: ldy / ldo must be >= n and multiples of 8", fn);
  if (out_dtype != DSL_OUT_BF16 && out_dtype != DSL_OUT_F32)
    return fail(DSL_ERR_ARG, "%s: unknown out_dtype %d", fn, out_dtype);
  if (rows >= ((int64_t)1 << 31) || tokens * topk >= ((int64_t)1 << 31))
    return fail(DSL_ERR_ARG, "%s: sizes must be < 2^31", fn);
  if (tokens == 0) return ok();
  int rc;
  if ((rc = check_out(fn, out, "out"))) return rc;
  if (rows > 0 && (rc = check_out(fn, y, "y"))) return rc;
  if (!dest || !topk_weights) return fail(DSL_ERR_ARG, "%s: NULL pointer argument", fn);
  return hip_status(dsl::launch_moe_combine(static_cast<const uint16_t *>(y), (int)rows, ldy, (int)n,
                                            dest, topk_weights, (int)tokens, (int)topk, out, ldo,
                                            out_dtype == DSL_OUT_F32,
                                            static_cast<hipStream_t>(stream)),
                    fn);
}

}  // extern "C"
