"""Quantize/pack operands on the GPU through the C ABI.

Each function takes a bf16 or fp32 operand ``x`` (fp16 is widened to fp32,
which is exact) whose LAST dimension is the GEMM
reduction axis K (``A[M, K]``; for weights pass ``W[N, K]``, which may be the
``.t()`` view of the reference's ``B[K, N]``) and returns K-major packed
codes plus scales, exactly as laid out in ``include/dsl_gemm.h``:

* ``quant_fp8_tensor(x)   -> (q uint8 [R, K], scale float32 [1])``
* ``quant_fp8_blocks(x, gr, gc) -> (q, scales float32 [ceil(R/gr), ceil(K/gc)])``
* ``quant_mxfp4(x)        -> (q uint8 [R, K/2], e8m0 uint8 [R, K/32])``
* ``quant_nvfp4(x)        -> (q uint8 [R, K/2], e4m3 uint8 [R, K/16], s_g float32 [1])``

Codes are raw bytes (``uint8``); ``.view(torch.float8_e4m3fn)`` gives the
torch fp8 view of E4M3 codes.
"""
from __future__ import annotations

import torch

from . import _native as N


def _check(x: torch.Tensor, name: str):
    """(x, x_dtype code): bf16 and fp32 are read as they are, fp16 is
    widened to fp32 (exact), so the codes are those of the source values
    (the reference quantizers read fp32, cuda/gemm/fp8_gemm.cu:118-144,
    cuda/gemm/fp4_gemm.cu:49-90)."""
    if not isinstance(x, torch.Tensor) or x.dim() != 2:
        raise ValueError(f"{name}: expected a 2-D tensor")
    if x.device.type != "cuda":
        raise ValueError(f"{name}: tensor must be on a GPU device (got {x.device})")
    if x.dtype == torch.bfloat16:
        return x, N.IN_BF16
    if x.dtype == torch.float32:
        return x, N.IN_F32
    if x.dtype == torch.float16:
        return x.float(), N.IN_F32
    raise TypeError(f"{name}: unsupported dtype {x.dtype} (bfloat16, float16 or float32)")


def _workspace(x: torch.Tensor) -> torch.Tensor:
    nbytes = N.lib().dsl_quant_workspace_bytes(x.shape[0], x.shape[1])
    return torch.empty(nbytes // 4, dtype=torch.float32, device=x.device)


def quant_fp8_tensor(x: torch.Tensor):
    x, xd = _check(x, "quant_fp8_tensor")
    R, C = x.shape
    q = torch.empty((R, C), dtype=torch.uint8, device=x.device)
    scale = torch.empty(1, dtype=torch.float32, device=x.device)
    ws = _workspace(x)
    with torch.cuda.device(x.device):
        N.call("dsl_quant_fp8_tensor", N.ptr(x), R, C, x.stride(0), x.stride(1), xd, N.ptr(q),
               N.ptr(scale), N.ptr(ws), ws.numel() * 4, N.stream_of(x.device))
    return q, scale


def quant_fp8_blocks(x: torch.Tensor, group_rows: int, group_cols: int):
    x, xd = _check(x, "quant_fp8_blocks")
    R, C = x.shape
    q = torch.empty((R, C), dtype=torch.uint8, device=x.device)
    scales = torch.empty((-(-R // group_rows), -(-C // group_cols)), dtype=torch.float32,
                         device=x.device)
    with torch.cuda.device(x.device):
        N.call("dsl_quant_fp8_blocks", N.ptr(x), R, C, x.stride(0), x.stride(1), xd, group_rows,
               group_cols, N.ptr(q), N.ptr(scales), N.stream_of(x.device))
    return q, scales


def quant_mxfp4(x: torch.Tensor):
    x, xd = _check(x, "quant_mxfp4")
    R, C = x.shape
    if C % 32:
        raise ValueError(f"quant_mxfp4: K={C} must be a multiple of 32")
    q = torch.empty((R, C // 2), dtype=torch.uint8, device=x.device)
    e8 = torch.empty((R, C // 32), dtype=torch.uint8, device=x.device)
    with torch.cuda.device(x.device):
        N.call("dsl_quant_mxfp4", N.ptr(x), R, C, x.stride(0), x.stride(1), xd, N.ptr(q), N.ptr(e8),
               N.stream_of(x.device))
    return q, e8


def quant_nvfp4(x: torch.Tensor):
    x, xd = _check(x, "quant_nvfp4")
    R, C = x.shape
    if C % 16:
        raise ValueError(f"quant_nvfp4: K={C} must be a multiple of 16")
    q = torch.empty((R, C // 2), dtype=torch.uint8, device=x.device)
    sb = torch.empty((R, C // 16), dtype=torch.uint8, device=x.device)
    sg = torch.empty(1, dtype=torch.float32, device=x.device)
    ws = _workspace(x)
    with torch.cuda.device(x.device):
        N.call("dsl_quant_nvfp4", N.ptr(x), R, C, x.stride(0), x.stride(1), xd, N.ptr(q), N.ptr(sb),
               N.ptr(sg), N.ptr(ws), ws.numel() * 4, N.stream_of(x.device))
    return q, sb, sg
