"""Pydantic request/response models of the REST service (same fields and
validation as the reference's dispatcher/schemas.py:15-136, with the
backend set extended by ``hip`` and the dtype set by ``uint8`` /
``float8_e8m0fnu`` for pre-quantized operands)."""
from __future__ import annotations

from typing import Any, Dict, List, Optional, Union

from pydantic import BaseModel, Field, field_validator

from .dispatcher import SUPPORTED_DTYPES

# "hip" is the only backend with entries in this build; the reference's
# names stay valid requests (they resolve to 404 kernel_not_found).
ALLOWED_BACKENDS = frozenset({"hip", "triton", "tilelang", "cuda"})


class TensorSpec(BaseModel):
    shape: List[int] = Field(..., description="Tensor shape, e.g. [128, 4096]")
    dtype: str = Field("bfloat16", description="float32|float16|bfloat16|fp8|uint8|e8m0|int32|...")
    data: Optional[str] = Field(None, description="Base64-encoded little-endian tensor bytes")
    fill: Optional[Union[str, float]] = Field(
        "random", description="When data is absent: 'zeros'|'ones'|'random'|<float>")

    @field_validator("dtype")
    @classmethod
    def _dtype(cls, v: str) -> str:
        if v.lower() not in SUPPORTED_DTYPES:
            raise ValueError(f"dtype '{v}' not supported. Choose from {sorted(SUPPORTED_DTYPES)}")
        return v.lower()

    @field_validator("shape")
    @classmethod
    def _shape(cls, v: list) -> list:
        if not v:
            raise ValueError("shape must be non-empty")
        if any(d <= 0 for d in v):
            raise ValueError("all shape dimensions must be > 0")
        return v


class KernelRunRequest(BaseModel):
    kernel_name: str = Field(..., description="e.g. 'gemm.fp8_gemm'",
                             examples=["gemm.fp8_gemm", "gemm.fp4_gemm", "gemm.grouped_gemm"])
    backend: str = Field(..., description="'hip'", examples=["hip"])
    inputs: List[TensorSpec] = Field(default_factory=list,
                                     description="Ordered input tensors (positional arguments)")
    params: Dict[str, Any] = Field(default_factory=dict,
                                   description="Scalar keyword arguments for the kernel")

    @field_validator("backend")
    @classmethod
    def _backend(cls, v: str) -> str:
        if v.lower() not in ALLOWED_BACKENDS:
            raise ValueError(f"backend '{v}' not recognised. Choose from {sorted(ALLOWED_BACKENDS)}")
        return v.lower()


class TensorOutput(BaseModel):
    shape: List[int]
    dtype: str
    data: str = Field(..., description="Base64-encoded output tensor bytes")


class KernelRunResponse(BaseModel):
    kernel_name: str
    backend: str
    elapsed_ms: float = Field(..., description="Wall-clock kernel time in ms (device synchronized)")
    device_info: str
    output: Union[TensorOutput, List[TensorOutput], Any]


class KernelSummary(BaseModel):
    kernel_name: str
    backend: str
    description: str


class KernelListResponse(BaseModel):
    count: int
    kernels: List[KernelSummary]


class KernelDetailResponse(BaseModel):
    kernel_name: str
    backend: str
    description: str
    input_schema: Dict[str, Any]
    output_schema: Dict[str, Any]
    backends_available: List[str]


class ErrorResponse(BaseModel):
    error: str
    detail: Optional[str] = None
    kernel_name: Optional[str] = None
    backend: Optional[str] = None
