"""ctypes binding of ``libdsl_gemm.so`` (the C ABI in ``include/dsl_gemm.h``).

``torch`` is imported before the library is opened on purpose: torch ships
its own HIP runtime whose SONAME (``libamdhip64.so.7``) matches the one the
library links against, so the dynamic loader reuses torch's runtime and the
two share devices, streams and allocations.

There is no fallback: if the library is missing or fails to load, every
entry point raises ``DslLibraryError``.
"""
from __future__ import annotations

import ctypes
import os
import re
import threading

import torch  # noqa: F401  (must precede loading the HIP library, see above)

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "_lib", "libdsl_gemm.so")
HEADER_PATH = os.path.join(os.path.dirname(PKG_DIR), "include", "dsl_gemm.h")

DSL_OK = 0
DSL_ERR_ARG = -1
DSL_ERR_UNSUPPORTED = -2
DSL_ERR_WORKSPACE = -3
DSL_ERR_HIP = -4
OUT_BF16, OUT_F32 = 0, 1
SCALE_TENSOR, SCALE_BLOCK128, SCALE_GROUP128 = 0, 1, 2
FMT_MXFP4, FMT_NVFP4 = 0, 1
OP_FP8, OP_FP4, OP_GROUPED_FP8, OP_BF16 = 0, 1, 2, 3
QFMT_FP8_G128, QFMT_MXFP4 = 0, 1
W_BF16, W_F32 = 0, 1
IN_BF16, IN_F32 = 0, 1
ABI_VERSION = 10


class DslLibraryError(ImportError):
    """The HIP library is not built or cannot be loaded."""


class DslError(RuntimeError):
    """A library entry point returned a non-zero status."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn}: {message} (status {status})")
        self.status = status


_vp, _i64, _i32, _sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t

# name -> (restype, argtypes)
SIGNATURES = {
    "dsl_last_error": (ctypes.c_char_p, []),
    "dsl_abi_version": (_i32, []),
    "dsl_quant_fp8_tensor": (_i32, [_vp, _i64, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _sz, _vp]),
    "dsl_quant_fp8_tensor_noalloc": (_i32, [_vp, _i64, _i64, _i64, _i64, _i32, _vp, _vp, _vp]),
    "dsl_quant_fp8_blocks": (_i32, [_vp, _i64, _i64, _i64, _i64, _i32, _i64, _i64, _vp, _vp, _vp]),
    "dsl_quant_mxfp4": (_i32, [_vp, _i64, _i64, _i64, _i64, _i32, _vp, _vp, _vp]),
    "dsl_quant_nvfp4": (_i32, [_vp, _i64, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _sz, _vp]),
    "dsl_quant_workspace_bytes": (_sz, [_i64, _i64]),
    "dsl_fp8_gemm": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _i32, _vp, _vp,
                            _vp, _sz, _vp]),
    "dsl_fp4_gemm": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _i32, _vp, _vp,
                            _vp, _vp, _vp, _sz, _vp]),
    "dsl_bf16_gemm": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp, _sz, _vp]),
    "dsl_grouped_fp8_gemm": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i32,
                                    _vp, _vp, _vp]),
    "dsl_gemm_workspace_bytes": (_sz, [_i32, _i64, _i64, _i64]),
    "dsl_rmsnorm_quant": (_i32, [_vp, _i64, _i64, _i64, _vp, _i32, ctypes.c_float, _i32, _vp, _vp,
                                 _vp, _i64, _vp]),
    "dsl_swiglu_quant": (_i32, [_vp, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _i64, _vp]),
    "dsl_lora_gemm_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "dsl_lora_gemm": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp,
                             _sz, _vp]),
    "dsl_moe_route_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "dsl_moe_route": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _sz, _vp]),
    "dsl_moe_permute_quant": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _vp]),
    "dsl_moe_quant_tokens": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _vp]),
    "dsl_moe_route_quant_tokens": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _vp,
                                          _vp, _vp, _vp]),
    "dsl_moe_grouped_fp8_gemm": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                        _i64, _i32, _vp, _vp, _vp]),
    "dsl_moe_combine": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _i64, _i32, _vp]),
}

_lib = None
_lock = threading.Lock()


def header_functions(path: str = HEADER_PATH) -> list[str]:
    """Names of the functions declared in include/dsl_gemm.h."""
    text = open(path).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(dsl_\w+)\s*\(", text, re.M)))


def lib():
    """Load (once) and return the ctypes handle; raises DslLibraryError."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise DslLibraryError(
                    f"HIP library not built: {LIB_PATH} (run `python -m dsl_tool_amd.build`)")
            try:
                handle = ctypes.CDLL(LIB_PATH)
            except OSError as exc:
                raise DslLibraryError(f"cannot load {LIB_PATH}: {exc}") from exc
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            if handle.dsl_abi_version() != ABI_VERSION:
                raise DslLibraryError("libdsl_gemm.so ABI version mismatch; rebuild it")
            _lib = handle
    return _lib


def call(name: str, *args) -> None:
    """Call an entry point and raise DslError on a non-zero status."""
    handle = lib()
    rc = getattr(handle, name)(*args)
    if rc != DSL_OK:
        msg = handle.dsl_last_error().decode(errors="replace")
        raise DslError(name, rc, msg)


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def vec_rows(t: torch.Tensor, ld_mult: int | None = None) -> torch.Tensor:
    """``t`` in a layout the kernels read in 16-byte vectors: a 16-byte
    aligned start and either row-major contiguous storage (``ld_mult=None``,
    for entry points that take no row stride) or unit column stride with a
    row stride of at least one row and a multiple of ``ld_mult`` elements.
    The C ABI refuses anything else, so any other view (an odd storage
    offset, a transposed or padded one) is copied into fresh row-major
    storage, which the allocator aligns."""
    if ld_mult is None:
        ok = t.is_contiguous()
    else:
        ok = t.stride(-1) == 1 and t.stride(0) >= t.shape[-1] and t.stride(0) % ld_mult == 0
    if ok and t.data_ptr() % 16 == 0:
        return t
    out = torch.empty(t.shape, dtype=t.dtype, device=t.device)
    out.copy_(t)
    return out
