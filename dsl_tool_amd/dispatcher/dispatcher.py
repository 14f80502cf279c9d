"""Kernel dispatcher: resolve ``(kernel_name, backend)``, build tensors from
JSON-safe specs, call the kernel, return JSON-safe results.

Same public API and wire format as the reference (dispatcher/dispatcher.py:
``deserialize_tensor`` :75-112, ``serialize_tensor`` :115-128,
``summarize_tensor`` :131-145, ``DispatchResult`` :152-185,
``KernelDispatcher.run / run_from_spec / list_kernels / list_backends /
kernel_info`` :192-344).  Tensor specs are positional arguments in order,
scalar params keyword arguments (:285-294).

Tensor spec::

    {"shape": [M, K], "dtype": "bfloat16",
     "data": "<base64 little-endian bytes>"          # optional, or
     "fill": "zeros" | "ones" | "random" | <float>}  # when data is absent

Differences from the reference, each a fix of a wire-format gap on the
quantized path (the reference cannot carry fp8 or packed fp4 operands):

* dtypes ``uint8`` and ``float8_e8m0fnu`` are accepted (packed E2M1 bytes,
  MX scales);
* ``fill: "random"`` for fp8 dtypes draws N(0,1) and casts (the reference
  calls ``torch.randint`` with an fp8 dtype, which raises);
* ``data`` for 1-byte dtypes carries the raw bytes, and outputs in those
  dtypes serialize as raw bytes (the reference's ``.numpy()`` fails on fp8);
* ``elapsed_ms`` synchronizes the device before reading the clock, so it is
  the kernel's wall time rather than its launch time.
"""
from __future__ import annotations

import base64
import logging
import time
from typing import Any, Dict, List, Optional

import numpy as np
import torch

from .registry import KernelEntry, get_registry

__all__ = ["KernelDispatcher", "DispatchResult", "deserialize_tensor", "serialize_tensor",
           "summarize_tensor"]

logger = logging.getLogger(__name__)

_DTYPE_MAP: Dict[str, torch.dtype] = {
    "float32": torch.float32, "fp32": torch.float32,
    "float16": torch.float16, "fp16": torch.float16,
    "bfloat16": torch.bfloat16, "bf16": torch.bfloat16,
    "float8_e4m3fn": torch.float8_e4m3fn, "fp8": torch.float8_e4m3fn,
    "float8_e8m0fnu": torch.float8_e8m0fnu, "e8m0": torch.float8_e8m0fnu,
    "uint8": torch.uint8, "int8": torch.int8,
    "int32": torch.int32, "int64": torch.int64,
}
SUPPORTED_DTYPES = frozenset(_DTYPE_MAP)

# numpy carrier of each dtype's wire bytes (bf16 travels as fp32 values, as
# in the reference; 1-byte float formats travel as their raw bytes)
_NP_CARRIER = {
    torch.float32: np.float32, torch.float16: np.float16, torch.bfloat16: np.float32,
    torch.float8_e4m3fn: np.uint8, torch.float8_e8m0fnu: np.uint8, torch.uint8: np.uint8,
    torch.int8: np.int8, torch.int32: np.int32, torch.int64: np.int64,
}
_RAW_BYTES = (torch.float8_e4m3fn, torch.float8_e8m0fnu)


def _resolve_dtype(name: str) -> torch.dtype:
    dt = _DTYPE_MAP.get(str(name).lower())
    if dt is None:
        raise ValueError(f"Unknown dtype '{name}'. Supported: {sorted(_DTYPE_MAP)}")
    return dt


def deserialize_tensor(spec: Dict[str, Any], device: str = "cuda") -> torch.Tensor:
    """Build a tensor on ``device`` from a JSON-safe spec."""
    shape = tuple(int(d) for d in spec["shape"])
    dtype = _resolve_dtype(spec.get("dtype", "bfloat16"))
    data = spec.get("data")
    if data is not None:
        raw = base64.b64decode(data)
        arr = np.frombuffer(raw, dtype=_NP_CARRIER[dtype])
        if arr.size != int(np.prod(shape, dtype=np.int64)):
            raise ValueError(f"data holds {arr.size} elements, shape {list(shape)} needs "
                             f"{int(np.prod(shape, dtype=np.int64))}")
        t = torch.from_numpy(arr.reshape(shape).copy())
        if dtype in _RAW_BYTES:
            t = t.view(dtype)
        elif t.dtype != dtype:
            t = t.to(dtype)
        return t.to(device)
    fill = spec.get("fill", "random")
    if fill is None or fill == "random":
        if dtype.is_floating_point:
            x = torch.randn(shape, dtype=torch.float32, device=device)
            return x.to(dtype)
        return torch.randint(0, 127, shape, dtype=dtype, device=device)
    if fill == "zeros":
        return torch.zeros(shape, dtype=torch.float32, device=device).to(dtype)
    if fill == "ones":
        return torch.ones(shape, dtype=torch.float32, device=device).to(dtype)
    return torch.full(shape, float(fill), dtype=torch.float32, device=device).to(dtype)


def serialize_tensor(t: torch.Tensor) -> Dict[str, Any]:
    """Tensor -> ``{"shape", "dtype", "data": base64}`` (bf16 as fp32 values)."""
    cpu = t.detach().cpu().contiguous()
    if cpu.dtype == torch.bfloat16:
        cpu = cpu.float()
    elif cpu.dtype in _RAW_BYTES:
        cpu = cpu.view(torch.uint8)
    return {"shape": list(t.shape), "dtype": str(t.dtype).replace("torch.", ""),
            "data": base64.b64encode(cpu.numpy().tobytes()).decode()}


def summarize_tensor(t: torch.Tensor) -> Dict[str, Any]:
    """Shape, dtype and value statistics of a tensor (no raw bytes)."""
    f = t.detach().cpu()
    f = f.view(torch.uint8).float() if f.dtype in _RAW_BYTES else f.float()
    n = f.numel()
    return {"shape": list(t.shape), "dtype": str(t.dtype).replace("torch.", ""), "numel": n,
            "min": round(f.min().item(), 6) if n else 0.0,
            "max": round(f.max().item(), 6) if n else 0.0,
            "mean": round(f.mean().item(), 6) if n else 0.0,
            "std": round(f.std().item(), 6) if n > 1 else 0.0}


class DispatchResult:
    def __init__(self, output: Any, kernel_name: str, backend: str, elapsed_ms: float,
                 device_info: str) -> None:
        self.output = output
        self.kernel_name = kernel_name
        self.backend = backend
        self.elapsed_ms = elapsed_ms
        self.device_info = device_info

    def to_dict(self) -> dict:
        out = self.output
        if isinstance(out, torch.Tensor):
            ser: Any = serialize_tensor(out)
        elif isinstance(out, (list, tuple)):
            ser = [serialize_tensor(o) if isinstance(o, torch.Tensor) else o for o in out]
        else:
            ser = out
        return {"kernel_name": self.kernel_name, "backend": self.backend,
                "elapsed_ms": round(self.elapsed_ms, 4), "device_info": self.device_info,
                "output": ser}


class KernelDispatcher:
    """Programmatic entry point (reference dispatcher.py:192-344).

    ``device`` falls back to ``"cpu"`` when no GPU is visible, as in the
    reference; the hip kernels then refuse the CPU tensors with an error.
    """

    def __init__(self, device: str = "cuda") -> None:
        self.device = device if torch.cuda.is_available() else "cpu"
        self._registry = get_registry(auto_load=True)
        if self.device == "cpu":
            logger.warning("no GPU visible: tensors are built on the CPU and the hip "
                           "kernels will refuse them")

    def run(self, kernel_name: str, backend: str, args: Optional[List[Any]] = None,
            kwargs: Optional[Dict[str, Any]] = None) -> DispatchResult:
        entry = self._resolve(kernel_name, backend)
        args = list(args or [])
        kwargs = dict(kwargs or {})
        info = self._device_info()
        t0 = time.perf_counter()
        try:
            out = entry.fn(*args, **kwargs)
            if self.device != "cpu" and torch.cuda.is_available():
                torch.cuda.synchronize()
        except Exception as exc:
            raise RuntimeError(f"Kernel '{kernel_name}' [{backend}] raised: {exc}") from exc
        ms = (time.perf_counter() - t0) * 1e3
        return DispatchResult(out, entry.kernel_name, entry.backend, ms, info)

    def run_from_spec(self, kernel_name: str, backend: str,
                      tensor_specs: Optional[List[Dict[str, Any]]] = None,
                      scalar_params: Optional[Dict[str, Any]] = None) -> DispatchResult:
        self._resolve(kernel_name, backend)      # unknown names fail before any allocation
        tensors = [deserialize_tensor(s, device=self.device) for s in (tensor_specs or [])]
        return self.run(kernel_name, backend, args=tensors, kwargs=scalar_params or {})

    def list_kernels(self) -> List[dict]:
        return self._registry.list_kernels()

    def list_backends(self, kernel_name: str) -> List[str]:
        return self._registry.list_backends_for(kernel_name)

    def kernel_info(self, kernel_name: str, backend: str) -> dict:
        e = self._resolve(kernel_name, backend)
        return {"kernel_name": e.kernel_name, "backend": e.backend,
                "description": e.description, "input_schema": e.input_schema,
                "output_schema": e.output_schema}

    def _resolve(self, kernel_name: str, backend: str) -> KernelEntry:
        entry = self._registry.get(kernel_name, backend)
        if entry is not None:
            return entry
        avail = self._registry.list_backends_for(kernel_name)
        if avail:
            raise KeyError(f"Backend '{backend}' not available for kernel '{kernel_name}'. "
                           f"Available backends: {avail}")
        raise KeyError(f"Unknown kernel '{kernel_name}'. Run list_kernels() to see all "
                       f"registered kernels.")

    def _device_info(self) -> str:
        if self.device == "cpu" or not torch.cuda.is_available():
            return "cpu"
        idx = torch.cuda.current_device()
        p = torch.cuda.get_device_properties(idx)
        return f"{p.name} ({p.total_memory // (1 << 20)} MB) [device:{idx}]"
