"""Kernel registry: ``(kernel_name, backend) -> callable``.

Same plugin surface as the reference (dispatcher/registry.py:26-122,
:329-336): ``KernelEntry``, ``KernelRegistry.register / get / list_kernels /
list_backends_for / load_all`` and the ``get_registry()`` singleton, with
names following ``<category>.<function>`` (registry.py:6-8) and keys
lower-cased.

This build registers one backend, ``hip``: the gfx950 quantized GEMMs of
``dsl_tool_amd.gemm`` under the reference's names ``gemm.fp8_gemm`` and
``gemm.grouped_gemm`` plus the new ``gemm.fp4_gemm``.  The callables are
registered whether or not the HIP library is built; calling one without it
raises ``DslLibraryError`` (no CPU fallback), which the dispatcher turns into
the same ``RuntimeError`` the reference raises for a failing kernel.

Unlike the reference (whose docstring promises thread safety without a lock),
registration and lookup here hold a lock, and the singleton is created
under it.
"""
from __future__ import annotations

import importlib
import importlib.util
import logging
import os
import threading
from dataclasses import dataclass, field
from typing import Callable, Dict, Optional, Tuple

logger = logging.getLogger(__name__)

BACKENDS = ("hip",)


@dataclass
class KernelEntry:
    """One registered (kernel, backend) pair (reference registry.py:26-34)."""
    kernel_name: str
    backend: str
    fn: Callable
    description: str = ""
    input_schema: dict = field(default_factory=dict)
    output_schema: dict = field(default_factory=dict)


class KernelRegistry:
    def __init__(self) -> None:
        self._store: Dict[Tuple[str, str], KernelEntry] = {}
        self._lock = threading.RLock()

    # ------------------------------------------------------------ register --
    def register(self, kernel_name: str, backend: str, fn: Callable, description: str = "",
                 input_schema: Optional[dict] = None,
                 output_schema: Optional[dict] = None) -> None:
        name, be = kernel_name.lower(), backend.lower()
        entry = KernelEntry(name, be, fn, description, dict(input_schema or {}),
                            dict(output_schema or {}))
        with self._lock:
            self._store[(name, be)] = entry
        logger.debug("registered %s [%s]", name, be)

    def get(self, kernel_name: str, backend: str) -> Optional[KernelEntry]:
        with self._lock:
            return self._store.get((kernel_name.lower(), backend.lower()))

    def list_kernels(self) -> list[dict]:
        with self._lock:
            entries = list(self._store.values())
        rows = [{"kernel_name": e.kernel_name, "backend": e.backend,
                 "description": e.description} for e in entries]
        return sorted(rows, key=lambda r: (r["kernel_name"], r["backend"]))

    def list_backends_for(self, kernel_name: str) -> list[str]:
        kn = kernel_name.lower()
        with self._lock:
            return sorted(b for (k, b) in self._store if k == kn)

    # -------------------------------------------------------------- loading --
    def _try_load_attr_from_file(self, file_path: str, attr: str) -> Optional[Callable]:
        """Load ``attr`` from a Python file given by absolute path (the
        reference's discovery hook, registry.py:99-111), for callers that
        register their own kernel files.  Failures are logged and give None."""
        try:
            mod_name = "_dsl_kernel_file_" + os.path.splitext(os.path.basename(file_path))[0]
            spec = importlib.util.spec_from_file_location(mod_name, file_path)
            if spec is None or spec.loader is None:
                return None
            mod = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(mod)
            return getattr(mod, attr, None)
        except Exception as exc:   # noqa: BLE001 -- a broken plugin file must not break startup
            logger.warning("could not load %s:%s: %s", file_path, attr, exc)
            return None

    def load_all(self, root: Optional[str] = None) -> None:
        """Register every backend this build ships (only ``hip``)."""
        self._register_hip(root)

    def _register_hip(self, root: Optional[str] = None) -> None:
        del root  # the hip kernels are a package module, not files under a root
        gemm = importlib.import_module("dsl_tool_amd.gemm")
        for name, attr, desc in HIP_GEMM_ENTRIES:
            self.register(name, "hip", getattr(gemm, attr), desc,
                          input_schema=gemm_input_schema(name),
                          output_schema=gemm_output_schema(name))
        for name, mod, attr, desc, ins, outs in HIP_EXTRA_ENTRIES:
            fn = getattr(importlib.import_module(mod), attr)
            self.register(name, "hip", fn, desc, input_schema=dict(ins), output_schema=dict(outs))


HIP_GEMM_ENTRIES = (
    ("gemm.bf16_gemm", "bf16_gemm",
     "BF16 GEMM (A[M,K] @ B[K,N], fp32 accumulation and output), gfx950 bf16 MFMA"),
    ("gemm.lora_fused_gemm", "lora_fused_gemm",
     "LoRA fused GEMM Y = X@W + Σ scale_l·X@A_l@B_l (bf16 MFMA, fp32 out)"),
    ("gemm.fp8_gemm", "fp8_gemm",
     "FP8 E4M3 GEMM (per-tensor or 1x128/128x128 block scales), gfx950 scaled MFMA"),
    ("gemm.fp4_gemm", "fp4_gemm",
     "FP4 E2M1 GEMM: MXFP4 (E8M0 / 32, scaled MFMA) or NVFP4 (E4M3 / 16 + fp32 global)"),
    ("gemm.grouped_gemm", "grouped_gemm",
     "Grouped FP8 GEMM for MoE / LoRA: fixed [G,M,K] or variable-size groups by offsets"),
)


# The step before the GEMM, quantized in registers (new names in the
# reference's <category>.<function> scheme, next to normalization.rmsnorm and
# activations.swiglu, dispatcher/registry.py:146,158).
_PRODUCER_OUT = {"q": "uint8 Tensor: E4M3 [rows, cols] (fmt 'fp8') | packed E2M1 [rows, cols/2] ('mxfp4')",
                 "scales": "fp32 [rows, ceil(cols/128)] ('fp8') | E8M0 uint8 [rows, cols/32] ('mxfp4')"}
HIP_EXTRA_ENTRIES = (
    ("normalization.rmsnorm_quant", "dsl_tool_amd.fused", "rmsnorm_quant",
     "RMSNorm y = w·x/√(mean(x²)+ε) quantized in registers to FP8 1x128 groups or MXFP4",
     {"x": "Tensor[batch, hidden] bf16", "weight": "Tensor[hidden] bf16/fp32",
      "eps": "float (default 1e-6)", "fmt": "str 'fp8' (default) | 'mxfp4'",
      "return_y": "bool: also return the bf16 RMSNorm output"}, _PRODUCER_OUT),
    ("activations.swiglu_quant", "dsl_tool_amd.fused", "swiglu_quant",
     "SwiGLU SiLU(gate)×up of input=[B,2H] quantized in registers to FP8 1x128 groups or MXFP4",
     {"input": "Tensor[batch, 2*hidden] bf16", "fmt": "str 'fp8' (default) | 'mxfp4'",
      "return_y": "bool: also return the bf16 SwiGLU output"}, _PRODUCER_OUT),
    # The step either side of gemm.grouped_gemm in an MoE layer: routing
    # tables, expert-ordered FP8 tokens, grouped GEMM, weighted combine.
    ("moe.routed_grouped_gemm", "dsl_tool_amd.moe", "routed_grouped_gemm",
     "MoE projection: route top-k ids, permute + FP8-quantize tokens, grouped FP8 GEMM, weighted combine",
     {"x": "Tensor[tokens, K] bf16", "topk_ids": "Tensor[tokens, topk] int32",
      "topk_weights": "Tensor[tokens, topk] fp32", "w": "Tensor[E, K, N] bf16",
      "out_dtype": "torch.bfloat16 (default) | torch.float32"},
     {"out": "Tensor[tokens, N]"}),
)


def gemm_input_schema(kernel_name: str) -> dict:
    """Documentation schema (the reference's _gemm_input_schema,
    registry.py:274-283, extended with this build's keyword arguments)."""
    s = {"A": "Tensor[M, K] bf16/fp16/fp32 (or pre-quantized, see kwargs)",
         "B": "Tensor[K, N] (pass W.t() for a K-major weight W[N, K])"}
    if kernel_name.endswith("lora_fused_gemm"):
        s = {"X": "Tensor[M, K] bf16", "W": "Tensor[K, N] bf16", "loraA": "Tensor[L, K, R] bf16",
             "loraB": "Tensor[L, R, N] bf16", "scales": "Tensor[L] fp32 | list of L floats"}
    elif kernel_name.endswith("bf16_gemm"):
        s = {"A": "Tensor[M, K] bf16", "B": "Tensor[K, N] bf16 (W.t() of a K-major W[N, K] is read in place)",
             "out_dtype": "torch.float32 (default) | torch.bfloat16"}
    elif kernel_name.endswith("fp8_gemm"):
        s.update({"scale_a": "float | Tensor[M, ceil(K/128)] fp32 | Tensor[M, ceil(K/G)] fp32 (groupwise)",
                  "scale_b": "float | Tensor[ceil(N/128), ceil(K/128)] fp32 (128x128 blocks) "
                             "| Tensor[ceil(K/G), N] fp32 (groupwise, per output column)",
                  "granularity": "str 'tensor' | 'block' | 'group' (bf16 inputs; "
                                 "pre-quantized: inferred from scale_b's shape)",
                  "group_size": "int G, a multiple of 128 (default 128; 'group' only)",
                  "out_dtype": "torch.bfloat16 (default) | torch.float32"})
    elif kernel_name.endswith("fp4_gemm"):
        s.update({"fmt": "str 'mxfp4' (default) | 'nvfp4'",
                  "scale_a": "uint8 Tensor (pre-packed inputs only)",
                  "scale_b": "uint8 Tensor (pre-packed inputs only)",
                  "global_a": "float (nvfp4, pre-packed)", "global_b": "float (nvfp4, pre-packed)"})
    elif kernel_name.endswith("grouped_gemm"):
        s = {"A": "Tensor[G, M, K] (fixed) | Tensor[T, K] rows sorted by group (variable) "
                  "| flat Tensor (descriptors)",
             "B": "Tensor[G, K, N] | flat Tensor (descriptors)",
             "num_groups": "int G (fixed) | int32 Tensor[G+1] group offsets (variable) | "
                           "int32 Tensor[G, 6] GemmProblem descriptors (M, N, K, A_offset, "
                           "B_offset, C_offset; per-group N and K)"}
    return s


def gemm_output_schema(kernel_name: str) -> dict:
    if kernel_name.endswith("grouped_gemm"):
        return {"C": "Tensor[G, M, N] | Tensor[T, N] | flat Tensor (descriptors), bf16 "
                     "(fp32 for fp32 inputs)"}
    if kernel_name.endswith("bf16_gemm"):
        return {"C": "Tensor[M, N] fp32 (out_dtype=torch.bfloat16 for bf16)"}
    if kernel_name.endswith("lora_fused_gemm"):
        return {"Y": "Tensor[M, N] fp32"}
    return {"C": "Tensor[M, N] bf16 (out_dtype=torch.float32 for the reference's fp32)"}


_registry: Optional[KernelRegistry] = None
_registry_lock = threading.Lock()


def get_registry(auto_load: bool = True) -> KernelRegistry:
    """The process-wide registry, created (and loaded) on first use."""
    global _registry
    with _registry_lock:
        if _registry is None:
            reg = KernelRegistry()
            if auto_load:
                reg.load_all()
            _registry = reg
    return _registry
