"""Value step of the fused quantize producers (CPU) -- TEST INFRASTRUCTURE ONLY.

The fused kernels quantize the bf16 result of the reference operator; these
functions restate that result.  Quantization itself is ``oracle.quant``.

* ``rmsnorm_bf16`` follows triton/normalization/norm_kernels.py:21-30:
  ``ms = sum(x^2) / N``, ``r = 1 / sqrt(ms + eps)``, ``y = (x * r) * w`` in
  fp32, stored as bf16 (RNE).  The reference's fp32 sum has no fixed order;
  here it is the correctly rounded fp32 value of the exact sum, so a GPU
  result may differ by one bf16 ulp where y sits next to a rounding boundary.
* ``swiglu_bf16`` follows triton/activations/activation_kernels.py:28-36:
  ``y = (g * sigmoid(g)) * u`` with ``sigmoid(g) = 1 / (1 + exp(-g))`` in
  fp32, gate = ``x[:, :H]``, up = ``x[:, H:2H]``, stored as bf16.

Pinned by float64 evaluations of the same formulas and closed forms
(tests/test_oracle.py).
"""
from __future__ import annotations

import numpy as np

from .formats import round_to_bf16

F32 = np.float32


def rmsnorm_bf16(x: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    x = np.asarray(x, F32)
    w = np.asarray(w, F32)
    n = x.shape[1]
    ss = (x.astype(np.float64) ** 2).sum(axis=1).astype(F32)
    ms = (ss / F32(n)).astype(F32)
    r = (F32(1.0) / np.sqrt((ms + F32(eps)).astype(F32))).astype(F32)
    y = ((x * r[:, None]).astype(F32) * w[None, :]).astype(F32)
    return round_to_bf16(y)


def swiglu_bf16(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, F32)
    h = x.shape[1] // 2
    g, u = x[:, :h], x[:, h:2 * h]
    with np.errstate(over="ignore"):
        sg = (F32(1.0) / (F32(1.0) + np.exp(-g).astype(F32))).astype(F32)
    y = ((g * sg).astype(F32) * u).astype(F32)
    return round_to_bf16(y)
