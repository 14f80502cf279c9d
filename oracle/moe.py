"""MoE glue around the grouped GEMM (CPU) -- TEST INFRASTRUCTURE ONLY.

The reference has no device-side MoE glue: its grouped GEMM consumes rows
already sorted by group plus a descriptor table (cuda/gemm/grouped_gemm.cu:
26-32, :77-104).  These functions define the build's glue contract:

* ``route``: a stable counting sort of the assignments a = t * topk + j by
  expert; ``offsets`` are the group offsets of the sorted rows, ``dest[a]``
  the sorted row of assignment a (-1 for ids outside [0, E), dropped), and
  ``src_token[r]`` the token of sorted row r.
* ``permute_quant``: sorted row r is token ``src_token[r]`` quantized per row
  (E4M3, scale max(amax/448, 1e-12): ``quant_fp8_blockwise`` with a 1 x K
  group).
* ``combine``: ``out[t] = sum_j w[t, j] * y[dest[t*topk + j]]`` in fp32, slot
  order j, one rounding per multiply and per add, then bf16.

Pinned by brute-force loops and closed forms (tests/test_oracle.py).
"""
from __future__ import annotations

import numpy as np

from .formats import round_to_bf16
from .quant import quant_fp8_blockwise

F32 = np.float32


def route(topk_ids: np.ndarray, num_experts: int):
    ids = np.asarray(topk_ids, np.int64).reshape(-1)
    topk = np.asarray(topk_ids).shape[1]
    valid = (ids >= 0) & (ids < num_experts)
    counts = np.bincount(ids[valid], minlength=num_experts)
    offsets = np.zeros(num_experts + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    key = np.where(valid, ids, num_experts)
    order = np.argsort(key, kind="stable")
    n_valid = int(valid.sum())
    dest = np.full(ids.shape, -1, np.int32)
    dest[order[:n_valid]] = np.arange(n_valid, dtype=np.int32)
    src_token = (order[:n_valid] // topk).astype(np.int32)
    return offsets, dest, src_token


def permute_quant(x: np.ndarray, src_token: np.ndarray):
    rows = np.asarray(x, F32)[np.asarray(src_token, np.int64)]
    q, s = quant_fp8_blockwise(rows, 1, rows.shape[1])
    return q, s[:, 0]


def combine(y: np.ndarray, dest: np.ndarray, w: np.ndarray, tokens: int, topk: int,
            out_bf16: bool = True):
    y = np.asarray(y, F32)
    w = np.asarray(w, F32).reshape(tokens, topk)
    d = np.asarray(dest).reshape(tokens, topk)
    out = np.zeros((tokens, y.shape[1]), F32)
    for j in range(topk):
        sel = (d[:, j] >= 0) & (d[:, j] < y.shape[0])
        term = (w[sel, j][:, None] * y[d[sel, j]]).astype(F32)
        out[sel] = (out[sel] + term).astype(F32)
    return round_to_bf16(out) if out_bf16 else out
