"""CPU: the C-ABI library loads, exports every function include/dsl_gemm.h
declares, and rejects bad arguments with a status code before it would
launch anything (no GPU is touched by any call here)."""
import ctypes
import os

import pytest

from dsl_tool_amd import _native as N

LIB = N.LIB_PATH


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built; run `python -m dsl_tool_amd.build`")
    return N.lib()


def test_library_exports_every_header_function(lib):
    declared = N.header_functions()
    assert declared, "no dsl_* functions found in include/dsl_gemm.h"
    raw = ctypes.CDLL(LIB)
    for name in declared:
        assert hasattr(raw, name), f"{name} declared in dsl_gemm.h but not exported"
    assert set(declared) == set(N.SIGNATURES), "ctypes signature table out of sync with header"


def test_abi_version(lib):
    assert lib.dsl_abi_version() == N.ABI_VERSION


def _err(lib):
    return lib.dsl_last_error().decode()


def test_fp8_gemm_argument_validation(lib):
    # k not a multiple of 16
    rc = lib.dsl_fp8_gemm(None, None, None, 16, 16, 15, 16, 0, 0, None, None, None, 0, None)
    assert rc == N.DSL_ERR_ARG and "multiple of 16" in _err(lib)
    # ldc < n
    rc = lib.dsl_fp8_gemm(None, None, None, 16, 32, 16, 16, 0, 0, None, None, None, 0, None)
    assert rc == N.DSL_ERR_ARG and "ldc" in _err(lib)
    # missing scales
    rc = lib.dsl_fp8_gemm(None, None, None, 16, 16, 16, 16, 0, 0, None, None, None, 0, None)
    assert rc == N.DSL_ERR_ARG and "scale" in _err(lib)
    # unknown scale mode (pointers are never dereferenced on the host)
    fake = 1 << 20
    rc = lib.dsl_fp8_gemm(fake, fake, fake, 16, 16, 16, 16, 0, 7, fake, fake, None, 0, None)
    assert rc == N.DSL_ERR_ARG and "scale_mode" in _err(lib)
    # misaligned operand
    rc = lib.dsl_fp8_gemm(fake + 1, fake, fake, 16, 16, 16, 16, 0, 0, fake, fake, None, 0, None)
    assert rc == N.DSL_ERR_ARG and "aligned" in _err(lib)
    # empty problem is a no-op success, also with the empty (NULL) scale
    # arrays of an empty block-scaled or FP4 operand; the mode is still checked
    assert lib.dsl_fp8_gemm(None, None, None, 0, 16, 16, 16, 0, 0, fake, fake, None, 0, None) == 0
    for mode in (N.SCALE_BLOCK128, N.SCALE_GROUP128):
        assert lib.dsl_fp8_gemm(None, None, None, 0, 16, 256, 16, 0, mode, None, None, None, 0,
                                None) == 0
        assert lib.dsl_fp8_gemm(None, None, None, 16, 0, 256, 0, 0, mode, None, None, None, 0,
                                None) == 0
    assert lib.dsl_fp4_gemm(None, None, None, 0, 16, 256, 16, 0, N.FMT_MXFP4, None, None, None,
                            None, None, 0, None) == 0
    rc = lib.dsl_fp8_gemm(None, None, None, 0, 16, 16, 16, 0, 7, None, None, None, 0, None)
    assert rc == N.DSL_ERR_ARG and "scale_mode" in _err(lib)
    # groupwise (per-column weight scales): 4-byte aligned scale arrays
    rc = lib.dsl_fp8_gemm(fake, fake, fake, 16, 16, 16, 16, 0, N.SCALE_GROUP128, fake + 2, fake,
                          None, 0, None)
    assert rc == N.DSL_ERR_ARG and "4-byte aligned" in _err(lib)
    # a register-staged shape (K % 128 != 0, few tiles) asks for a split-K
    # workspace, which covers the groupwise mode too; without one it is refused
    need = lib.dsl_gemm_workspace_bytes(N.OP_FP8, 70, 300, 1040)
    assert need >= 70 * 300 * 4
    rc = lib.dsl_fp8_gemm(fake, fake, fake, 70, 300, 1040, 300, 0, N.SCALE_GROUP128, fake, fake,
                          None, 0, None)
    assert rc == N.DSL_ERR_WORKSPACE


def test_bf16_gemm_argument_validation(lib):
    fake = 1 << 20
    rc = lib.dsl_bf16_gemm(fake, fake, fake, 16, 16, 12, 16, 0, None, 0, None)
    assert rc == N.DSL_ERR_ARG and "multiple of 8" in _err(lib)
    rc = lib.dsl_bf16_gemm(fake, fake, fake, 16, 32, 16, 16, 0, None, 0, None)
    assert rc == N.DSL_ERR_ARG and "ldc" in _err(lib)
    rc = lib.dsl_bf16_gemm(fake + 2, fake, fake, 16, 16, 16, 16, 0, None, 0, None)
    assert rc == N.DSL_ERR_ARG and "aligned" in _err(lib)
    rc = lib.dsl_bf16_gemm(fake, fake, fake, 16, 16, 16, 16, 5, None, 0, None)
    assert rc == N.DSL_ERR_ARG and "out_dtype" in _err(lib)
    # small M with K % 512 == 0 takes the one-launch decode kernel (no
    # workspace); other K split over a workspace, and without one the call is refused
    assert lib.dsl_gemm_workspace_bytes(N.OP_BF16, 16, 256, 4096) == 0
    need = lib.dsl_gemm_workspace_bytes(N.OP_BF16, 16, 256, 4104)
    assert need >= 16 * 256 * 4
    rc = lib.dsl_bf16_gemm(fake, fake, fake, 16, 256, 4104, 256, 0, None, 0, None)
    assert rc == N.DSL_ERR_WORKSPACE
    # large problems run on the persistent kernel without workspace
    assert lib.dsl_gemm_workspace_bytes(N.OP_BF16, 4096, 4096, 4096) == 0
    assert lib.dsl_bf16_gemm(None, None, None, 0, 16, 16, 16, 0, None, 0, None) == 0


def test_fused_producer_argument_validation(lib):
    fake = 1 << 20
    rc = lib.dsl_rmsnorm_quant(fake, 4, 40, 40, fake, N.W_BF16, 1e-6, N.QFMT_MXFP4, fake, fake,
                               None, 0, None)
    assert rc == N.DSL_ERR_ARG and "multiple of 32" in _err(lib)
    rc = lib.dsl_rmsnorm_quant(fake, 4, 65536, 65536, fake, N.W_BF16, 1e-6, N.QFMT_FP8_G128, fake,
                               fake, None, 0, None)
    assert rc == N.DSL_ERR_UNSUPPORTED
    rc = lib.dsl_swiglu_quant(fake, 4, 64, 100, N.QFMT_FP8_G128, fake, fake, None, 0, None)
    assert rc == N.DSL_ERR_ARG and "ldx" in _err(lib)
    rc = lib.dsl_swiglu_quant(fake, 4, 64, 128, 9, fake, fake, None, 0, None)
    assert rc == N.DSL_ERR_ARG and "qfmt" in _err(lib)
    rc = lib.dsl_rmsnorm_quant(fake, 4, 64, 64, fake + 2, N.W_BF16, 1e-6, N.QFMT_FP8_G128, fake,
                               fake, None, 0, None)
    assert rc == N.DSL_ERR_ARG and "weight" in _err(lib)
    assert lib.dsl_swiglu_quant(None, 0, 64, 128, 0, None, None, None, 0, None) == 0


def test_lora_argument_validation(lib):
    fake = 1 << 20
    rc = lib.dsl_lora_gemm(fake, fake, fake, fake, fake, fake, 64, 64, 64, 3, 1, 64, fake, 1 << 30, None)
    assert rc == N.DSL_ERR_ARG and "multiple of 8" in _err(lib)
    need = lib.dsl_lora_gemm_workspace_bytes(256, 256, 512, 16, 2)
    assert need >= 256 * 32 * 8
    rc = lib.dsl_lora_gemm(fake, fake, fake, fake, fake, fake, 256, 256, 512, 16, 2, 256, fake, need - 1, None)
    assert rc == N.DSL_ERR_WORKSPACE


def test_moe_glue_argument_validation(lib):
    fake = 1 << 20
    rc = lib.dsl_moe_route(fake, 16, 2, 4096, fake, fake, fake, fake, 1 << 20, None)
    assert rc == N.DSL_ERR_ARG and "num_experts" in _err(lib)
    need = lib.dsl_moe_route_workspace_bytes(4096, 8, 64)
    assert need >= 32 * 64 * 4
    rc = lib.dsl_moe_route(fake, 4096, 8, 64, fake, fake, fake, fake, need - 4, None)
    assert rc == N.DSL_ERR_WORKSPACE
    rc = lib.dsl_moe_permute_quant(fake, 16, 100, 104, fake, 2, 32, fake, fake, None)
    assert rc == N.DSL_ERR_ARG and "multiple of 8" in _err(lib)
    rc = lib.dsl_moe_combine(fake, 32, 64, 32, fake, fake, 16, 2, fake, 64, 0, None)
    assert rc == N.DSL_ERR_ARG and "ldy" in _err(lib)
    assert lib.dsl_moe_combine(None, 0, 64, 64, None, None, 0, 2, None, 64, 0, None) == 0
    # no tokens still needs one block's histogram when the route takes two passes
    assert lib.dsl_moe_route_workspace_bytes(0, 8, 1500) >= 1500 * 4
    rc = lib.dsl_moe_quant_tokens(fake, 16, 100, 104, fake, 2, 32, fake, fake, None)
    assert rc == N.DSL_ERR_ARG and "multiple of 8" in _err(lib)
    # the gather GEMM: whole 128-byte pairs of K, a row map, tokens < 2^24
    rc = lib.dsl_moe_grouped_fp8_gemm(fake, 64, fake, fake, fake, fake, 4, 128, 256, 192, 256, 0,
                                      fake, fake, None)
    assert rc == N.DSL_ERR_UNSUPPORTED and "128" in _err(lib)
    rc = lib.dsl_moe_grouped_fp8_gemm(fake, 64, None, fake, fake, fake, 4, 128, 256, 256, 256, 0,
                                      fake, fake, None)
    assert rc == N.DSL_ERR_ARG and "NULL" in _err(lib)
    rc = lib.dsl_moe_grouped_fp8_gemm(fake, 1 << 24, fake, fake, fake, fake, 4, 128, 256, 256, 256, 0,
                                      fake, fake, None)
    assert rc == N.DSL_ERR_ARG and "tokens" in _err(lib)


def test_workspace_query_matches_the_planned_path(lib):
    # skinny M with K a multiple of 1024 takes the single-pass decode kernel
    assert lib.dsl_gemm_workspace_bytes(N.OP_FP8, 16, 8192, 8192) == 0
    # FP4 reports the larger of the MXFP4 and NVFP4 plans: NVFP4 with M = 1
    # runs the GEMV kernel and larger skinny M the streaming kernel (no
    # workspace); a K neither skinny kernel takes (4352: not a multiple of
    # 512 elements) plans split-K over the register-staged tiles
    assert lib.dsl_gemm_workspace_bytes(N.OP_FP4, 1, 14336, 4096) == 0
    assert lib.dsl_gemm_workspace_bytes(N.OP_FP4, 8, 14336, 4096) == 0
    assert lib.dsl_gemm_workspace_bytes(N.OP_FP4, 8, 14336, 4352) >= 8 * 14336 * 4
    # large problems take the pipelined kernels, which need none either
    assert lib.dsl_gemm_workspace_bytes(N.OP_FP8, 8192, 8192, 8192) == 0
    # a skinny problem the decode kernel does not cover plans split-K and
    # then requires the workspace it reports
    need = lib.dsl_gemm_workspace_bytes(N.OP_FP8, 16, 8192, 8208)
    assert need >= 16 * 8192 * 4
    fake = 1 << 20
    rc = lib.dsl_fp8_gemm(fake, fake, fake, 16, 8192, 8208, 8192, 0, 0, fake, fake, None,
                          need - 4, None)
    assert rc == N.DSL_ERR_WORKSPACE


def test_fp4_gemm_argument_validation(lib):
    fake = 1 << 20
    rc = lib.dsl_fp4_gemm(fake, fake, fake, 4, 4, 48, 4, 0, N.FMT_MXFP4, fake, fake, None, None,
                          None, 0, None)
    assert rc == N.DSL_ERR_ARG and "multiple of 32" in _err(lib)
    rc = lib.dsl_fp4_gemm(fake, fake, fake, 4, 4, 64, 4, 0, N.FMT_NVFP4, fake, fake, None, None,
                          None, 0, None)
    assert rc == N.DSL_ERR_ARG and "global" in _err(lib)
    rc = lib.dsl_fp4_gemm(fake, fake, fake, 4, 4, 64, 4, 0, 9, fake, fake, None, None,
                          None, 0, None)
    assert rc == N.DSL_ERR_ARG and "fmt" in _err(lib)
    rc = lib.dsl_fp4_gemm(fake, fake, fake, 4, 4, 64, 4, 5, N.FMT_MXFP4, fake, fake, None, None,
                          None, 0, None)
    assert rc == N.DSL_ERR_ARG and "out_dtype" in _err(lib)


def test_grouped_gemm_argument_validation(lib):
    fake = 1 << 20
    rc = lib.dsl_grouped_fp8_gemm(fake, fake, fake, fake, 0, 8, 16, 16, 16, 0, fake, fake, None)
    assert rc == N.DSL_ERR_ARG and "num_groups" in _err(lib)
    rc = lib.dsl_grouped_fp8_gemm(fake, fake, fake, fake, 4096, 8, 16, 16, 16, 0, fake, fake,
                                  None)
    assert rc == N.DSL_ERR_ARG
    rc = lib.dsl_grouped_fp8_gemm(fake, fake, fake, None, 4, 8, 16, 16, 16, 0, fake, fake, None)
    assert rc == N.DSL_ERR_ARG and "NULL" in _err(lib)


def test_quantizer_argument_validation(lib):
    fake = 1 << 20
    rc = lib.dsl_quant_mxfp4(fake, 4, 48, 48, 1, 0, fake, fake, None)
    assert rc == N.DSL_ERR_ARG and "multiple of 32" in _err(lib)
    rc = lib.dsl_quant_nvfp4(fake, 4, 40, 40, 1, 0, fake, fake, fake, fake, 1 << 20, None)
    assert rc == N.DSL_ERR_ARG and "multiple of 16" in _err(lib)
    rc = lib.dsl_quant_fp8_tensor(fake, 4, 64, 64, 1, 0, fake, fake, fake, 4, None)
    assert rc == N.DSL_ERR_WORKSPACE
    rc = lib.dsl_quant_fp8_blocks(fake, 4, 64, 64, 1, 0, 0, 128, fake, fake, None)
    assert rc == N.DSL_ERR_ARG and "group" in _err(lib)
    rc = lib.dsl_quant_fp8_blocks(fake + 1, 4, 64, 64, 1, 0, 1, 128, fake, fake, None)
    assert rc == N.DSL_ERR_ARG and "aligned" in _err(lib)
    rc = lib.dsl_quant_fp8_blocks(fake, 4, 64, -3, 1, 0, 1, 128, fake, fake, None)
    assert rc == N.DSL_ERR_ARG and "stride" in _err(lib)
    # an empty input is a successful no-op
    assert lib.dsl_quant_mxfp4(None, 0, 64, 64, 1, 0, None, None, None) == 0


def test_error_message_is_cleared_on_success(lib):
    lib.dsl_quant_mxfp4(1 << 20, 4, 48, 48, 1, 0, 1 << 20, 1 << 20, None)
    assert _err(lib)
    assert lib.dsl_quant_mxfp4(None, 0, 64, 64, 1, 0, None, None, None) == 0
    assert _err(lib) == ""


def test_python_wrappers_raise_dslerror(lib):
    with pytest.raises(N.DslError) as ei:
        N.call("dsl_quant_mxfp4", 1 << 20, 4, 48, 48, 1, 0, 1 << 20, 1 << 20, None)
    assert ei.value.status == N.DSL_ERR_ARG


def test_quantizer_source_dtype_validation(lib):
    fake = 1 << 20
    rc = lib.dsl_quant_mxfp4(fake, 4, 64, 64, 1, 7, fake, fake, None)
    assert rc == N.DSL_ERR_ARG and "x_dtype" in _err(lib)
    # fp32 sources must be 4-byte aligned
    rc = lib.dsl_quant_fp8_blocks(fake + 2, 4, 64, 64, 1, N.IN_F32, 1, 128, fake, fake, None)
    assert rc == N.DSL_ERR_ARG and "aligned" in _err(lib)


def test_noalloc_quantizer_validation(lib):
    """Argument checks of the allocation-free quantizer run before any HIP
    call, so they are testable without a GPU."""
    fake = 1 << 20
    rc = lib.dsl_quant_fp8_tensor_noalloc(fake, 4, 64, 64, 1, 9, fake, fake, None)
    assert rc == N.DSL_ERR_ARG and "x_dtype" in _err(lib)
    rc = lib.dsl_quant_fp8_tensor_noalloc(fake, 4, 64, 64, 1, N.IN_BF16, fake, None, None)
    assert rc == N.DSL_ERR_ARG and "scale" in _err(lib)
    assert lib.dsl_quant_fp8_tensor_noalloc(None, 0, 64, 64, 1, N.IN_BF16, None, None, None) == 0
