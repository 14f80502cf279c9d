"""Reference GEMMs for the quantized path (CPU).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Orientation: A is [M, K], the weight operand is W[N, K] (K-major); the
reference's ``B[K, N]`` is ``W.t()`` (triton/gemm/gemm_kernels.py:104-108,
:117-119 are stride-generic, so passing ``W.t()`` is the same call).

The dense references dequantize both operands to fp32 and multiply with an
fp32 (or fp64) matmul, then round to bf16 -- the "dequantize -> fp32
matmul" oracle.  Mathematically this equals the reference's group-partial
form ``sum_g s_a s_b sum_{k in g} a b`` (cuda/gemm/fp8_gemm.cu:84-97,
fp4_gemm.cu:111-135); the two differ only by fp32 summation order, which the
1e-2 tolerance absorbs.  ``tiled_fp8_gemm`` restates the reference's own CPU
path (tilelang/gemm/gemm_kernels.py:96-113) tile for tile and is used as the
reference-structured CPU baseline.
"""
from __future__ import annotations

import numpy as np
import torch

from .formats import e2m1_decode, e4m3_decode, e8m0_decode, unpack_nibbles, round_to_bf16
from .quant import F32


def _mm(a: np.ndarray, w: np.ndarray, f64: bool = False) -> np.ndarray:
    """a[M,K] @ w[N,K].T on the CPU (torch, so the thread count is explicit)."""
    dt = torch.float64 if f64 else torch.float32
    ta = torch.from_numpy(np.ascontiguousarray(a)).to(dt)
    tw = torch.from_numpy(np.ascontiguousarray(w)).to(dt)
    return (ta @ tw.T).to(torch.float32).numpy()


# ----------------------------- dequantizers -------------------------------

def dequant_fp8_tensor(q, scale):
    return (e4m3_decode(q) * F32(scale)).astype(F32)


def dequant_fp8_blocks(q, scales, group_rows, group_cols):
    R, C = q.shape
    full = np.repeat(np.repeat(np.asarray(scales, F32), group_rows, axis=0),
                     group_cols, axis=1)[:R, :C]
    return (e4m3_decode(q) * full).astype(F32)


def dequant_mxfp4(packed, e8m0):
    v = e2m1_decode(unpack_nibbles(packed))
    R, C = v.shape
    s = np.repeat(e8m0_decode(e8m0), 32, axis=1)[:, :C]
    return (v * s).astype(F32)


def dequant_nvfp4(packed, sb_codes, s_g):
    v = e2m1_decode(unpack_nibbles(packed))
    R, C = v.shape
    s = np.repeat(e4m3_decode(sb_codes), 16, axis=1)[:, :C]
    return (v * s * F32(s_g)).astype(F32)


# ------------------------------ references --------------------------------

def ref_gemm_dequant(a_deq: np.ndarray, w_deq: np.ndarray, f64: bool = False) -> np.ndarray:
    """fp32 (or fp64) matmul of dequantized operands -> float32 holding bf16."""
    return round_to_bf16(_mm(a_deq, w_deq, f64))


def ref_fp8_per_tensor(qa, sa, qw, sw, f64=False):
    """C = (sum_k a*w) * sa * sb (triton/gemm/gemm_kernels.py:97 applies the
    scales after accumulation); bf16 result."""
    acc = _mm(e4m3_decode(qa), e4m3_decode(qw), f64)
    return round_to_bf16((acc * F32(sa) * F32(sw)).astype(F32))


def ref_fp8_groupwise(qa, sa, qw, sw, f64=False):
    """Activations 1x128, weights 128x128 (sa [M, K/128], sw [N/128, K/128])."""
    return ref_gemm_dequant(dequant_fp8_blocks(qa, sa, 1, 128),
                            dequant_fp8_blocks(qw, sw, 128, 128), f64)


def ref_fp8_groupwise_cols(qa, sa, qw, sb, group_size=128, f64=False):
    """The reference's own groupwise layout (cuda/gemm/fp8_gemm.cu:67-99):
    sa [M, ceil(K/G)] per activation row and K group, sb [ceil(K/G), N] per
    K group and output column (qw is W [N, K], so column n is row n of qw);
    C[m, n] = sum_g (sum_{k in g} a*w) * sa[m, g] * sb[g, n], the last group
    partial when G does not divide K (:84-86).  Computed as dequantize ->
    matmul: A with 1 x G groups, W with its column scales as 1 x G groups of
    its rows."""
    sb = np.asarray(sb, F32)
    return ref_gemm_dequant(dequant_fp8_blocks(qa, sa, 1, group_size),
                            dequant_fp8_blocks(qw, sb.T, 1, group_size), f64)


def ref_mxfp4(pa, ea, pw, ew, f64=False):
    return ref_gemm_dequant(dequant_mxfp4(pa, ea), dequant_mxfp4(pw, ew), f64)


def ref_nvfp4(pa, sba, ga, pw, sbw, gw, f64=False):
    return ref_gemm_dequant(dequant_nvfp4(pa, sba, ga), dequant_nvfp4(pw, sbw, gw), f64)


def ref_grouped_fp8(qx, sx, qw, sw, offsets, f64=False):
    """Grouped (MoE) FP8: rows offsets[e]:offsets[e+1] of X multiply W[e].

    Per-row activation scale sx[r], per-channel weight scale sw[e, n]:
    ``Y[r, n] = sx[r] * sw[e(r), n] * sum_k Q8 Q8``.  Follows the
    variable-size descriptor semantics of cuda/gemm/grouped_gemm.cu:26-32,
    :77-104 with the concatenated-rows layout; empty groups produce no rows.
    """
    qx = np.asarray(qx)
    G = len(offsets) - 1
    N = qw.shape[1]
    out = np.zeros((qx.shape[0], N), dtype=F32)
    xd = e4m3_decode(qx)
    for e in range(G):
        r0, r1 = int(offsets[e]), int(offsets[e + 1])
        if r1 == r0:
            continue
        acc = _mm(xd[r0:r1], e4m3_decode(qw[e]), f64)
        out[r0:r1] = acc * np.asarray(sx[r0:r1], F32)[:, None] * np.asarray(sw[e], F32)[None, :]
    return round_to_bf16(out.astype(F32))


def ref_bf16(a: np.ndarray, w: np.ndarray, f64: bool = True) -> np.ndarray:
    """C = A @ W.T for bf16 operands held in float32 arrays, float32 result.

    The reference accumulates bf16 tiles into an fp32 accumulator with
    ``tl.dot`` and returns fp32 (triton/gemm/gemm_kernels.py:31-37, :50).
    Each bf16 x bf16 product is exact in fp32, so the fp64 sum rounded once
    to fp32 is the exact result up to that rounding; an fp32 accumulator
    differs from it only by summation order.
    """
    return _mm(a, w, f64)


def ref_lora(x, w, a, b, scales) -> np.ndarray:
    """Y = X @ W + sum_l s_l * (X @ A_l) @ B_l in float64, as float32
    (cuda/gemm/grouped_gemm.cu:120-137).  x [M, K], w [N, K] (the reference's
    W [K, N] is w.T), a [L, K, R], b [L, R, N], scales [L]."""
    x64 = np.asarray(x, np.float64)
    y = x64 @ np.asarray(w, np.float64).T
    for l in range(np.asarray(a).shape[0]):
        y += float(scales[l]) * ((x64 @ np.asarray(a[l], np.float64)) @ np.asarray(b[l], np.float64))
    return y.astype(np.float32)


def tiled_bf16_gemm(a: np.ndarray, w: np.ndarray, block_m=128, block_n=128, block_k=32):
    """The reference's CPU path for bf16 restated: 128x128x32 tiles, fp32
    accumulation over K tiles (tilelang/gemm/gemm_kernels.py:75-95).
    a [M, K], w [N, K] float32 holding bf16; returns fp32 [M, N]."""
    ta = torch.from_numpy(np.ascontiguousarray(a, np.float32))
    tw = torch.from_numpy(np.ascontiguousarray(w, np.float32))
    M, K = ta.shape
    N = tw.shape[0]
    c = torch.zeros(M, N, dtype=torch.float32)
    for bm in range(0, M, block_m):
        for bn in range(0, N, block_n):
            acc = torch.zeros(min(block_m, M - bm), min(block_n, N - bn))
            for bk in range(0, K, block_k):
                acc += ta[bm:bm + block_m, bk:bk + block_k] @ tw[bn:bn + block_n, bk:bk + block_k].T
            c[bm:bm + block_m, bn:bn + block_n] = acc
    return c.numpy()


def tiled_fp8_gemm(a_codes, w_codes, sa, sw, block_m=64, block_n=64, block_k=32):
    """The reference's CPU path restated: 64x64x32 tiles, fp32 accumulation
    over K tiles, scales applied to each finished tile
    (tilelang/gemm/gemm_kernels.py:96-113).  Returns fp32 [M, N]."""
    a = torch.from_numpy(e4m3_decode(a_codes))
    w = torch.from_numpy(e4m3_decode(w_codes))
    M, K = a.shape
    N = w.shape[0]
    c = torch.zeros(M, N, dtype=torch.float32)
    for bm in range(0, M, block_m):
        for bn in range(0, N, block_n):
            acc = torch.zeros(min(block_m, M - bm), min(block_n, N - bn))
            for bk in range(0, K, block_k):
                acc += a[bm:bm + block_m, bk:bk + block_k] @ w[bn:bn + block_n, bk:bk + block_k].T
            c[bm:bm + block_m, bn:bn + block_n] = acc * float(sa) * float(sw)
    return c.numpy()


def tiled_grouped_fp8_gemm(qx, sx, qw, sw, offsets, block_m=64, block_n=64, block_k=32,
                           groups=None):
    """The reference's grouped CPU path restated (tilelang/gemm/gemm_kernels.py:
    116-133): per group, 64x64x32 tiles with fp32 accumulation over K tiles,
    here over the variable-size groups of cuda/gemm/grouped_gemm.cu:26-32
    (rows offsets[g]..offsets[g+1] of qx times W_g), each finished tile
    scaled per row and per channel as (acc * sx[r]) * sw[g, n].
    qx [T, K], qw [G, N, K] E4M3 codes, sx [T], sw [G, N]; `groups` limits
    the work to those group indices (rows of other groups stay 0).
    Returns fp32 [T, N]."""
    x = torch.from_numpy(e4m3_decode(qx))
    G, N, K = qw.shape
    c = torch.zeros(x.shape[0], N, dtype=torch.float32)
    sxt = torch.from_numpy(np.asarray(sx, np.float32))
    swt = torch.from_numpy(np.asarray(sw, np.float32))
    for g in (range(G) if groups is None else groups):
        r0, r1 = int(offsets[g]), int(offsets[g + 1])
        if r1 <= r0:
            continue
        w = torch.from_numpy(e4m3_decode(qw[g]))
        for bm in range(r0, r1, block_m):
            be = min(bm + block_m, r1)
            for bn in range(0, N, block_n):
                acc = torch.zeros(be - bm, min(block_n, N - bn))
                for bk in range(0, K, block_k):
                    acc += x[bm:be, bk:bk + block_k] @ w[bn:bn + block_n, bk:bk + block_k].T
                c[bm:be, bn:bn + block_n] = ((acc * sxt[bm:be, None])
                                             * swt[g, None, bn:bn + block_n])
    return c.numpy()


# ------------------------------ tolerance ---------------------------------

def rel_errors(c: np.ndarray, r: np.ndarray):
    """(max|C-R| / max|R|, max elementwise rel err over |R| >= 0.1*rms(R))."""
    c = np.asarray(c, np.float64)
    r = np.asarray(r, np.float64)
    denom = np.max(np.abs(r))
    glob = float(np.max(np.abs(c - r)) / denom) if denom > 0 else float(np.max(np.abs(c)))
    rms = np.sqrt(np.mean(r * r)) if r.size else 0.0
    mask = np.abs(r) >= 0.1 * rms
    if rms == 0 or not mask.any():
        return glob, 0.0
    elem = float(np.max(np.abs(c - r)[mask] / np.abs(r)[mask]))
    return glob, elem
