"""Fused quantize producers on the GPU.

Two checks per case: the bf16 operator output y (returned with
return_y=True) against the oracle's RMSNorm / SwiGLU, within one bf16 ulp
(the fp32 sum order of RMSNorm and exp's last bit are not fixed by the
reference), and the codes and scales bit for bit against the oracle
quantizer applied to that same y.
"""
import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import fused as OF
from oracle import quant as OQ
from oracle import gemm as OG
from dsl_tool_amd import fused as FU
from dsl_tool_amd import gemm as G
from dsl_tool_amd import quant as Q
from dsl_tool_amd import workloads as W
from tests.util import assert_close, np_f32, np_u8

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ulp_diff(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in bf16 steps between two arrays of bf16 values (same sign)."""
    ia = F.f32_to_bf16_bits(a).astype(np.int32)
    ib = F.f32_to_bf16_bits(b).astype(np.int32)
    return np.abs(ia - ib)


def _check_values(y_gpu: np.ndarray, y_ref: np.ndarray, what: str):
    d = _ulp_diff(y_gpu, y_ref)
    assert d.max() <= 1, f"{what}: bf16 values off by {d.max()} ulp"
    assert (d > 0).mean() <= 2e-3, f"{what}: {(d > 0).mean():.2e} of values differ by one ulp"


def _check_codes(fmt, q, s, y):
    if fmt == "fp8":
        q_ref, s_ref = OQ.quant_fp8_blockwise(y, 1, 128)
        assert np.array_equal(np_f32(s), s_ref)
    else:
        q_ref, s_ref = OQ.quant_mxfp4(y)
        assert np.array_equal(np_u8(s), s_ref)
    assert np.array_equal(np_u8(q), q_ref)


RMS_SHAPES = [(64, 7168), (37, 4096), (5, 136), (3, 16384), (2, 32768), (2, 32), (1, 8)]


# MXFP4 takes whole 32-element blocks only (cols % 32 == 0): those shapes
# run FP8 alone
@pytest.mark.parametrize("rows,cols,fmt", [(r, c, f) for r, c in RMS_SHAPES for f in ("fp8", "mxfp4")
                                           if f == "fp8" or c % 32 == 0])
@pytest.mark.parametrize("wdt", [torch.bfloat16, torch.float32])
def test_rmsnorm_quant(rows, cols, fmt, wdt):
    x = W.randn_bf16((rows, cols), 300) * 3
    w = (1.0 + 0.1 * torch.randn(cols, generator=torch.Generator().manual_seed(301))).to(wdt)
    q, s, y = FU.rmsnorm_quant(x.to(DEV), w.to(DEV), 1e-6, fmt=fmt, return_y=True)
    y_gpu = np_f32(y)
    _check_values(y_gpu, OF.rmsnorm_bf16(x.float().numpy(), w.float().numpy(), 1e-6),
                  f"rmsnorm {rows}x{cols}")
    _check_codes(fmt, q, s, y_gpu)
    q2, s2 = FU.rmsnorm_quant(x.to(DEV), w.to(DEV), 1e-6, fmt=fmt)   # no y output
    assert torch.equal(q2, q) and torch.equal(s2, s)


SWIGLU_SHAPES = [(64, 7168), (37, 4096), (5, 136), (2, 16384), (1, 8)]


@pytest.mark.parametrize("rows,hidden,fmt", [(r, h, f) for r, h in SWIGLU_SHAPES for f in ("fp8", "mxfp4")
                                              if f == "fp8" or h % 32 == 0])
def test_swiglu_quant(rows, hidden, fmt):
    x = W.randn_bf16((rows, 2 * hidden), 310) * 4
    q, s, y = FU.swiglu_quant(x.to(DEV), fmt=fmt, return_y=True)
    y_gpu = np_f32(y)
    _check_values(y_gpu, OF.swiglu_bf16(x.float().numpy()), f"swiglu {rows}x{hidden}")
    _check_codes(fmt, q, s, y_gpu)


def test_producers_on_row_strided_inputs_and_zero_rows():
    wide = W.randn_bf16((16, 2 * 512 + 64), 320)
    xs = wide.to(DEV)[:, :1024]                      # SwiGLU input with a padded row stride
    q, s, y = FU.swiglu_quant(xs, return_y=True)
    _check_values(np_f32(y), OF.swiglu_bf16(wide[:, :1024].float().numpy()), "swiglu strided")
    _check_codes("fp8", q, s, np_f32(y))
    x = torch.zeros((4, 256), dtype=torch.bfloat16)
    x[1] = W.randn_bf16((1, 256), 321)[0]
    w = torch.ones(256, dtype=torch.bfloat16)
    q, s, y = FU.rmsnorm_quant(x.to(DEV), w.to(DEV), 1e-6, return_y=True)
    _check_codes("fp8", q, s, np_f32(y))
    assert not np_u8(q)[0].any() and np.all(np_f32(s)[0] == np.float32(1e-12))


def test_rmsnorm_quant_feeds_the_block_scaled_gemm():
    # rmsnorm_quant -> fp8_gemm on pre-quantized operands == oracle GEMM of the same codes
    x = W.randn_bf16((256, 1024), 330)
    w_norm = torch.ones(1024, dtype=torch.bfloat16)
    wt = W.randn_bf16((512, 1024), 331, 0.02)
    qa, sa = FU.rmsnorm_quant(x.to(DEV), w_norm.to(DEV))
    qw, sw = Q.quant_fp8_blocks(wt.to(DEV), 128, 128)
    c = G.fp8_gemm(qa.view(torch.float8_e4m3fn), qw.view(torch.float8_e4m3fn).t(), sa, sw)
    ref = OG.ref_fp8_groupwise(np_u8(qa), np_f32(sa), np_u8(qw), np_f32(sw))
    assert_close(c, ref, what="rmsnorm_quant -> fp8_gemm")


def test_producer_argument_errors():
    x = torch.zeros((4, 40), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        FU.rmsnorm_quant(x, torch.ones(40, device=DEV), fmt="mxfp4")   # 40 % 32
    with pytest.raises(TypeError):
        FU.swiglu_quant(x.float())
    with pytest.raises(ValueError):
        FU.rmsnorm_quant(x, torch.ones(41, device=DEV))
