"""MoE glue on the GPU around the grouped FP8 GEMM.

An MoE FFN projection, on the device end to end:

    route = moe_route(topk_ids, E)                  # offsets, dest, src_token
    qx, sx = moe_permute_quant(x, route)            # tokens in expert order, E4M3 per row
    y = gemm.grouped_fp8_gemm_packed(qx, sx, qw, sw, route.offsets)
    out = moe_combine(y, route, topk_weights)       # weighted sum over each token's experts

``routed_grouped_gemm`` runs the four steps (registered as
``moe.routed_grouped_gemm``).  Where the persistent grouped kernel takes the
GEMM (groups averaging 48 rows or more, K % 128 == 0) the middle two are
``moe_quant_tokens`` (codes in token order, scales per sorted row) and
``moe_grouped_fp8_gemm``, which reads each sorted row's A through
``route.src_token``: the codes are written once per token instead of topk
times, with the same result bit for bit.  At decode size
(``tokens * topk <= 1024``, K <= 2048) ``moe_route_quant_tokens`` routes and
quantizes in one launch, again with the same tables, codes and scales.  The reference has no MoE glue; its grouped
GEMM takes rows already sorted by group (cuda/gemm/grouped_gemm.cu:26-32,
:77-104, triton/gemm/gemm_kernels.py:164-182).  Everything runs in
``libdsl_gemm.so``; the sorted order is a stable counting sort, so results
do not depend on scheduling.
"""
from __future__ import annotations

from typing import NamedTuple

import torch

from . import _native as N
from . import gemm as G
from . import quant as Q


class Route(NamedTuple):
    offsets: torch.Tensor     # int32 [E + 1]
    dest: torch.Tensor        # int32 [T * topk]: sorted row of assignment t*topk+j, -1 if dropped
    src_token: torch.Tensor   # int32 [T * topk]: token of sorted row r (r < offsets[E])
    tokens: int
    topk: int
    num_experts: int


def _gpu(t: torch.Tensor, name: str):
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be a tensor on a GPU device")


def moe_route(topk_ids: torch.Tensor, num_experts: int) -> Route:
    """Group offsets and row maps from ``topk_ids [T, topk]`` (expert ids)."""
    _gpu(topk_ids, "topk_ids")
    if topk_ids.dim() != 2:
        raise ValueError("topk_ids must be [tokens, topk]")
    ids = topk_ids.to(torch.int32).contiguous()
    T, k = ids.shape
    dev = ids.device
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    dest = torch.empty(T * k, dtype=torch.int32, device=dev)
    src = torch.empty(T * k, dtype=torch.int32, device=dev)
    nb = N.lib().dsl_moe_route_workspace_bytes(T, k, num_experts)
    ws = torch.empty(max(nb, 4) // 4, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        N.call("dsl_moe_route", N.ptr(ids), T, k, num_experts, N.ptr(offsets), N.ptr(dest),
               N.ptr(src), N.ptr(ws), ws.numel() * 4, N.stream_of(dev))
    return Route(offsets, dest, src, T, k, num_experts)


def moe_permute_quant(x: torch.Tensor, route: Route):
    """Token rows of ``x [T, K]`` (bf16) in expert order, E4M3 with one scale
    per row: ``(qx [T*topk, K] uint8, sx [T*topk] float32)``; rows past the
    routed total are unused.  Each token is quantized once and written to
    its ``topk`` sorted rows ``route.dest``."""
    _gpu(x, "x")
    if x.dtype != torch.bfloat16 or x.dim() != 2 or x.shape[0] != route.tokens:
        raise ValueError("x must be bf16 [tokens, K]")
    x = N.vec_rows(x, 8)
    T, K = x.shape
    rows = T * route.topk
    qx = torch.empty((rows, K), dtype=torch.uint8, device=x.device)
    sx = torch.empty(rows, dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        N.call("dsl_moe_permute_quant", N.ptr(x), T, K, x.stride(0), N.ptr(route.dest),
               route.topk, rows, N.ptr(qx), N.ptr(sx), N.stream_of(x.device))
    return qx, sx


def moe_quant_tokens(x: torch.Tensor, route: Route):
    """``x [T, K]`` (bf16) to E4M3 in token order, one scale per row:
    ``(qx [T, K] uint8, sx [T*topk] float32)`` where ``sx`` holds each
    token's scale at its sorted rows ``route.dest`` (the input of
    :func:`moe_grouped_fp8_gemm`; the codes are those of
    :func:`moe_permute_quant`, not copied per routed row)."""
    _gpu(x, "x")
    if x.dtype != torch.bfloat16 or x.dim() != 2 or x.shape[0] != route.tokens:
        raise ValueError("x must be bf16 [tokens, K]")
    x = N.vec_rows(x, 8)
    T, K = x.shape
    rows = T * route.topk
    qx = torch.empty((T, K), dtype=torch.uint8, device=x.device)
    sx = torch.empty(rows, dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        N.call("dsl_moe_quant_tokens", N.ptr(x), T, K, x.stride(0), N.ptr(route.dest),
               route.topk, rows, N.ptr(qx), N.ptr(sx), N.stream_of(x.device))
    return qx, sx


# one launch for route + per-token quantize (dsl_moe_route_quant_tokens)
ROUTE_QUANT_MAX_ASSIGNMENTS = 1024


def route_quant_applies(tokens: int, topk: int, num_experts: int, k: int) -> bool:
    """Whether :func:`moe_route_quant_tokens` takes one launch (decode-size
    batches); otherwise it runs :func:`moe_route` and :func:`moe_quant_tokens`."""
    return (1 <= tokens and tokens * topk <= ROUTE_QUANT_MAX_ASSIGNMENTS
            and num_experts <= 2047 and k <= 2048 and k % 8 == 0)


def moe_route_quant_tokens(topk_ids: torch.Tensor, x: torch.Tensor, num_experts: int):
    """:func:`moe_route` then :func:`moe_quant_tokens`: ``(route, qx, sx)``.
    For decode-size batches (``tokens * topk <= 1024``, K <= 2048) both run in
    one launch with the same results bit for bit; other sizes take the two
    calls."""
    _gpu(topk_ids, "topk_ids")
    _gpu(x, "x")
    if topk_ids.dim() != 2 or x.dim() != 2 or x.shape[0] != topk_ids.shape[0]:
        raise ValueError("topk_ids [tokens, topk] and x [tokens, K] must match")
    if x.dtype != torch.bfloat16:
        raise ValueError("x must be bf16 [tokens, K]")
    T, k = topk_ids.shape
    K = x.shape[1]
    x = N.vec_rows(x, 8)
    if not route_quant_applies(T, k, num_experts, K):
        route = moe_route(topk_ids, num_experts)
        qx, sx = moe_quant_tokens(x, route)
        return route, qx, sx
    ids = topk_ids.to(torch.int32).contiguous()
    dev = ids.device
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    dest = torch.empty(T * k, dtype=torch.int32, device=dev)
    src = torch.empty(T * k, dtype=torch.int32, device=dev)
    qx = torch.empty((T, K), dtype=torch.uint8, device=dev)
    sx = torch.empty(T * k, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        N.call("dsl_moe_route_quant_tokens", N.ptr(ids), T, k, num_experts, N.ptr(x), K,
               x.stride(0), N.ptr(offsets), N.ptr(dest), N.ptr(src), N.ptr(qx), N.ptr(sx),
               N.stream_of(dev))
    return Route(offsets, dest, src, T, k, num_experts), qx, sx


def moe_grouped_fp8_gemm(qx: torch.Tensor, sx: torch.Tensor, route: Route, qw: torch.Tensor,
                         sw: torch.Tensor, *, out_dtype=torch.bfloat16) -> torch.Tensor:
    """The grouped GEMM over the routed rows with A read through the row
    map: sorted row r multiplies token ``route.src_token[r]`` of the
    token-major codes ``qx [T, K]`` (from :func:`moe_quant_tokens`) with its
    expert's ``qw [E, N, K]``; ``y [T*topk, N]`` in sorted order, as
    ``grouped_fp8_gemm_packed`` over the permuted copy gives."""
    dev = G._require_gpu(qx, qw, sx, sw)
    qx, qw = N.vec_rows(G._u8(qx)), N.vec_rows(G._u8(qw))
    T, K = qx.shape
    E, Nn, K2 = qw.shape
    if K != K2 or T != route.tokens or E != route.num_experts:
        raise ValueError("qx [tokens, K] / qw [E, N, K] do not match the route")
    rows = T * route.topk
    sx = sx.reshape(-1).float().contiguous()
    sw = sw.reshape(E, Nn).float().contiguous()
    if sx.numel() != rows:
        raise ValueError("sx must have one entry per routed row")
    y = torch.empty((rows, Nn), dtype=G._as_dtype(out_dtype), device=dev)
    with torch.cuda.device(dev):
        N.call("dsl_moe_grouped_fp8_gemm", N.ptr(qx), T, N.ptr(route.src_token), N.ptr(qw),
               N.ptr(y), N.ptr(route.offsets), E, rows, Nn, K, y.stride(0), G._out_code(y.dtype),
               N.ptr(sx), N.ptr(sw), N.stream_of(dev))
    return y


def gather_applies(tokens: int, topk: int, num_experts: int, k: int) -> bool:
    """Whether the routed GEMM reads A through the row map: k % 128 == 0,
    tokens < 2^24 and tokens * k < 2^32.  Groups averaging 48 rows or more
    take the persistent grouped kernel, fewer the streaming grouped tiles
    (k % 256 == 0; else the persistent kernel again)."""
    return (k % 128 == 0 and 1 <= num_experts <= 2048
            and tokens < (1 << 24) and tokens * k < (1 << 32))


def moe_combine(y: torch.Tensor, route: Route, topk_weights: torch.Tensor, *,
                out_dtype=torch.bfloat16) -> torch.Tensor:
    """``out[t] = sum_j topk_weights[t, j] * y[dest[t*topk + j]]`` (fp32 sum)."""
    _gpu(y, "y")
    _gpu(topk_weights, "topk_weights")
    if y.dtype != torch.bfloat16 or y.dim() != 2 or y.stride(1) != 1:
        raise ValueError("y must be bf16 [rows, N] with unit column stride")
    w = topk_weights.to(torch.float32).contiguous()
    if tuple(w.shape) != (route.tokens, route.topk):
        raise ValueError(f"topk_weights must be [{route.tokens}, {route.topk}]")
    rows, n = y.shape
    out = torch.empty((route.tokens, n), dtype=out_dtype, device=y.device)
    with torch.cuda.device(y.device):
        N.call("dsl_moe_combine", N.ptr(y), rows, n, y.stride(0), N.ptr(route.dest), N.ptr(w),
               route.tokens, route.topk, N.ptr(out), n, G._out_code(out_dtype),
               N.stream_of(y.device))
    return out


def routed_grouped_gemm(x: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
                        w: torch.Tensor, *, out_dtype=torch.bfloat16) -> torch.Tensor:
    """MoE projection ``out[t] = sum_j w_tj * (x[t] @ W[e_tj])`` for
    ``x [T, K]`` bf16, ``topk_ids / topk_weights [T, topk]`` and expert
    weights ``w [E, K, N]`` (the reference's grouped B layout; bf16, quantized
    here per output channel) or pre-quantized ``(qw [E, N, K] uint8, sw [E, N])``.
    """
    if isinstance(w, (tuple, list)):
        qw, sw = w
        E = qw.shape[0]
    else:
        _gpu(w, "w")
        if w.dim() != 3:
            raise ValueError("w must be [E, K, N]")
        E, K, Nn = w.shape
        wt = w.transpose(1, 2).reshape(E * Nn, K)       # [E*N, K] K-major rows
        qw, sw = Q.quant_fp8_blocks(wt, 1, K)
        qw, sw = qw.reshape(E, Nn, K), sw.reshape(E, Nn)
    _gpu(topk_ids, "topk_ids")
    if topk_ids.dim() != 2:
        raise ValueError("topk_ids must be [tokens, topk]")
    T, topk = topk_ids.shape
    if gather_applies(T, topk, E, qw.shape[2]):
        # token-major codes, A rows through the row map: no permuted copy
        # (route and quantize in one launch at decode size)
        route, qx, sx = moe_route_quant_tokens(topk_ids, x, E)
        y = moe_grouped_fp8_gemm(qx, sx, route, qw, sw, out_dtype=torch.bfloat16)
    else:
        route = moe_route(topk_ids, E)
        qx, sx = moe_permute_quant(x, route)
        y = G.grouped_fp8_gemm_packed(qx, sx, qw, sw, route.offsets, out_dtype=torch.bfloat16)
    return moe_combine(y, route, topk_weights, out_dtype=out_dtype)
