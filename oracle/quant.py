"""Quantize/pack contract for the quantized GEMM path (numpy, CPU).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Every quantizer takes the logical operand as a float32 array ``x[R, C]``
whose columns run along the GEMM reduction axis K (activations A[M,K] and
weights W[N,K] alike), and returns K-major codes, i.e. exactly the byte
arrays the HIP quantize kernels write.

Arithmetic order is part of the contract (it decides individual codes):
* scales are computed in fp32 (``np.float32`` scalars/arrays throughout);
* elements are divided by the fp32 scale in fp32 (``x / scale``), not
  multiplied by a reciprocal; MXFP4 multiplies by an exact power of two.
"""
from __future__ import annotations

import numpy as np

from .formats import (e2m1_encode, e4m3_encode, e4m3_decode, floor_log2,
                      pack_nibbles)

F32 = np.float32
SCALE_FLOOR = F32(1e-12)


def _amax(x: np.ndarray, axis=None) -> np.ndarray:
    return np.max(np.abs(x.astype(F32)), axis=axis).astype(F32)


# --------------------------------------------------------------------------
# FP8 E4M3
# --------------------------------------------------------------------------

def quant_fp8_per_tensor(x: np.ndarray):
    """Per-tensor E4M3: ``scale = max(amax/448, 1e-12)``, ``q = e4m3(x/scale)``.

    Follows cuda/gemm/fp8_gemm.cu:118-144 (amax, the 448 divisor, the 1e-12
    floor, divide-then-convert).  Returns (codes uint8 [R,C], scale float32).
    """
    x = np.asarray(x, dtype=F32)
    amax = _amax(x)
    scale = F32(amax / F32(448.0))
    if scale < SCALE_FLOOR:
        scale = SCALE_FLOOR
    q = e4m3_encode((x / scale).astype(F32))
    return q, F32(scale)


def quant_fp8_blockwise(x: np.ndarray, group_rows: int, group_cols: int):
    """Block-scaled E4M3 over tiles of ``group_rows x group_cols``.

    One fp32 scale per tile, ``max(amax_tile/448, 1e-12)``; partial edge
    tiles use the elements present.  Scale grid is
    ``[ceil(R/group_rows), ceil(C/group_cols)]``.  Cases on the path:
    * activations 1x128  -> scale_a[M, K/128]   (the reference's groupwise
      ``scale_a[row * num_groups + g]``, cuda/gemm/fp8_gemm.cu:74,87);
    * weights 128x128    -> scale_w[N/128, K/128] (``sb[g][n]`` constant over
      each 128-column block, cuda/gemm/fp8_gemm.cu:75,88);
    * per-row / per-channel: group_rows=1, group_cols=C.
    """
    x = np.asarray(x, dtype=F32)
    R, C = x.shape
    gr, gc = group_rows, group_cols
    nr, nc = -(-R // gr), -(-C // gc)
    pad = np.zeros((nr * gr, nc * gc), dtype=F32)
    pad[:R, :C] = np.abs(x)
    amax = pad.reshape(nr, gr, nc, gc).max(axis=(1, 3)).astype(F32)
    scale = (amax / F32(448.0)).astype(F32)
    scale = np.where(scale < SCALE_FLOOR, SCALE_FLOOR, scale).astype(F32)
    full = np.repeat(np.repeat(scale, gr, axis=0), gc, axis=1)[:R, :C]
    q = e4m3_encode((x / full).astype(F32))
    return q, scale


def dequant_fp8(q: np.ndarray, scale, group_rows: int = 0, group_cols: int = 0) -> np.ndarray:
    """codes * scale in fp32 (per-tensor when group sizes are 0)."""
    v = e4m3_decode(q)
    if group_rows == 0:
        return (v * F32(scale)).astype(F32)
    R, C = q.shape
    full = np.repeat(np.repeat(np.asarray(scale, F32), group_rows, axis=0),
                     group_cols, axis=1)[:R, :C]
    return (v * full).astype(F32)


# --------------------------------------------------------------------------
# MXFP4 (E2M1 + E8M0 per 32 along K)
# --------------------------------------------------------------------------

def quant_mxfp4(x: np.ndarray):
    """MXFP4 per OCP MX v1.0 with the shared exponent of BASELINE config 3.

    Per row and per 32 consecutive K elements:
    ``e = clamp(floor(log2(amax)) - 2, -127, 127)`` (amax == 0 -> e = -127),
    ``E8M0 = e + 127``, ``Q4 = e2m1_rne_sat(x * 2**-e)``.  Packing: two codes
    per byte, low nibble = even K index (cuda/gemm/fp4_gemm.cu:45-47, :88).
    Returns (packed uint8 [R, C/2], e8m0 uint8 [R, C/32]).
    """
    x = np.asarray(x, dtype=F32)
    R, C = x.shape
    assert C % 32 == 0, "MXFP4 needs K % 32 == 0"
    blocks = x.reshape(R, C // 32, 32)
    amax = _amax(blocks, axis=-1)
    e = floor_log2(amax) - 2
    e = np.clip(e, -127, 127)
    code = (e + 127).astype(np.uint8)
    mul = np.ldexp(np.ones_like(amax, dtype=F32), (-e).astype(np.int32)).astype(F32)
    v = (blocks * mul[..., None]).astype(F32)
    q = e2m1_encode(v).reshape(R, C)
    return pack_nibbles(q), code


# --------------------------------------------------------------------------
# NVFP4 (E2M1 + E4M3 per 16 along K + fp32 global)
# --------------------------------------------------------------------------

def quant_nvfp4(x: np.ndarray):
    """NVFP4 with the BASELINE config 4 scale rules.

    ``s_g = max(amax_T / 2688, 1e-12)`` (2688 = 448*6; the floor follows the
    reference's scale floors, cuda/gemm/fp8_gemm.cu:134, fp4_gemm.cu:70-71),
    per row and per 16 K: ``s_b = e4m3(amax_16 / 6 / s_g)`` computed as
    ``(amax_16 / 6) / s_g`` in fp32, then
    ``Q4 = e2m1_rne_sat(x / (f32(s_b) * s_g))`` with the denominator rounded
    to fp32 first.  A block whose denominator is 0 (s_b underflowed) gets
    all-zero codes.  Returns (packed uint8 [R, C/2], e4m3 uint8 [R, C/16],
    s_g float32).
    """
    x = np.asarray(x, dtype=F32)
    R, C = x.shape
    assert C % 16 == 0, "NVFP4 needs K % 16 == 0"
    amax_t = _amax(x)
    s_g = F32(amax_t / F32(2688.0))
    if s_g < SCALE_FLOOR:
        s_g = SCALE_FLOOR
    blocks = x.reshape(R, C // 16, 16)
    amax_b = _amax(blocks, axis=-1)
    s_b_code = e4m3_encode(((amax_b / F32(6.0)).astype(F32) / s_g).astype(F32))
    d = (e4m3_decode(s_b_code) * s_g).astype(F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        v = (blocks / d[..., None]).astype(F32)
    q = e2m1_encode(v)
    q = np.where((d == 0)[..., None], np.uint8(0), q).reshape(R, C)
    return pack_nibbles(q), s_b_code, F32(s_g)
