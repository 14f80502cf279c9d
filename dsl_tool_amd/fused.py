"""Fused quantize producers: the step before the GEMM, quantized in registers.

* ``rmsnorm_quant(x, weight, eps=1e-6, fmt="fp8")`` -- RMSNorm
  (triton/normalization/norm_kernels.py:21-30, :110-116, registered as
  ``normalization.rmsnorm``) whose bf16 result is encoded straight into the
  activation format of the GEMM that follows;
* ``swiglu_quant(input, fmt="fp8")`` -- SwiGLU on ``input [B, 2H]`` = gate | up
  (triton/activations/activation_kernels.py:28-36, :105-115, registered as
  ``activations.swiglu``), likewise.

``fmt="fp8"``: E4M3 codes ``[rows, cols]`` uint8 with 1x128 group scales
``[rows, ceil(cols/128)]`` float32 (the activation side of the block-scaled
``fp8_gemm``); ``fmt="mxfp4"``: packed E2M1 ``[rows, cols/2]`` with E8M0
scales ``[rows, cols/32]``.  The codes are exactly what ``quant_fp8_blocks(y,
1, 128)`` / ``quant_mxfp4(y)`` give for the bf16 operator output ``y``;
``return_y=True`` also returns ``y``.  Everything runs in
``libdsl_gemm.so``; inputs must be CUDA bf16 tensors.
"""
from __future__ import annotations

import torch

from . import _native as N

_FMTS = {"fp8": N.QFMT_FP8_G128, "mxfp4": N.QFMT_MXFP4}


def _rows2d(x: torch.Tensor, name: str) -> torch.Tensor:
    if not isinstance(x, torch.Tensor) or x.dim() != 2:
        raise ValueError(f"{name}: expected a 2-D tensor")
    if x.device.type != "cuda":
        raise ValueError(f"{name}: tensor must be on a GPU device (got {x.device})")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"{name}: input must be bfloat16 (got {x.dtype})")
    return N.vec_rows(x, 8)


def _outputs(rows: int, cols: int, fmt: str, dev, return_y: bool):
    if fmt not in _FMTS:
        raise ValueError(f"fmt must be 'fp8' or 'mxfp4', got {fmt!r}")
    if fmt == "fp8":
        q = torch.empty((rows, cols), dtype=torch.uint8, device=dev)
        s = torch.empty((rows, -(-cols // 128)), dtype=torch.float32, device=dev)
    else:
        if cols % 32:
            raise ValueError(f"mxfp4 needs a row length that is a multiple of 32 (got {cols})")
        q = torch.empty((rows, cols // 2), dtype=torch.uint8, device=dev)
        s = torch.empty((rows, cols // 32), dtype=torch.uint8, device=dev)
    y = torch.empty((rows, cols), dtype=torch.bfloat16, device=dev) if return_y else None
    return q, s, y


def rmsnorm_quant(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6, *,
                  fmt: str = "fp8", return_y: bool = False):
    """RMSNorm of ``x [rows, cols]`` (bf16) with ``weight [cols]`` (bf16 or
    fp32), quantized.  Returns ``(q, scales)`` or ``(q, scales, y)``."""
    x = _rows2d(x, "rmsnorm_quant")
    rows, cols = x.shape
    if weight.dim() != 1 or weight.numel() != cols:
        raise ValueError(f"rmsnorm_quant: weight must be [{cols}]")
    if weight.device != x.device:
        raise ValueError("rmsnorm_quant: weight must be on the device of x")
    if weight.dtype not in (torch.bfloat16, torch.float32):
        weight = weight.float()
    weight = weight.contiguous()
    q, s, y = _outputs(rows, cols, fmt, x.device, return_y)
    with torch.cuda.device(x.device):
        N.call("dsl_rmsnorm_quant", N.ptr(x), rows, cols, x.stride(0), N.ptr(weight),
               N.W_F32 if weight.dtype == torch.float32 else N.W_BF16, float(eps), _FMTS[fmt],
               N.ptr(q), N.ptr(s), N.ptr(y), cols if y is not None else 0,
               N.stream_of(x.device))
    return (q, s, y) if return_y else (q, s)


def swiglu_quant(input: torch.Tensor, *, fmt: str = "fp8", return_y: bool = False):
    """SwiGLU of ``input [rows, 2H]`` (bf16; gate = first H, up = last H),
    quantized.  Returns ``(q, scales)`` or ``(q, scales, y)``."""
    x = _rows2d(input, "swiglu_quant")
    rows, two_h = x.shape
    if two_h % 2:
        raise ValueError("swiglu_quant: input must be [rows, 2*hidden]")
    hidden = two_h // 2
    q, s, y = _outputs(rows, hidden, fmt, x.device, return_y)
    with torch.cuda.device(x.device):
        N.call("dsl_swiglu_quant", N.ptr(x), rows, hidden, x.stride(0), _FMTS[fmt], N.ptr(q),
               N.ptr(s), N.ptr(y), hidden if y is not None else 0, N.stream_of(x.device))
    return (q, s, y) if return_y else (q, s)
