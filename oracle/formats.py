"""Bit-level number formats used on the quantized GEMM path (numpy, CPU).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Formats
-------
E4M3 (OCP "FN" variant): bias 7, 3 mantissa bits, max normal 448
    (S.1111.110), NaN = S.1111.111, no infinities, subnormal step 2**-9.
    The reference quantizes with ``__nv_fp8_e4m3(x / scale)``
    (cuda/gemm/fp8_gemm.cu:141-142); its semantics are restated here from the
    OCP spec: round-to-nearest-even, values >= 464 (exclusive tie) -> NaN,
    i.e. no saturation -- identical to torch's ``float8_e4m3fn`` cast.
E2M1: code -> value table {0, .5, 1, 1.5, 2, 3, 4, 6}, bit 3 = sign
    (cuda/gemm/fp4_gemm.cu:30-33); two codes per byte, low nibble = the
    element with the even index (cuda/gemm/fp4_gemm.cu:45-47, :88).
    Encoding is round-to-nearest-even with saturation to +-6 (OCP MX v1.0);
    the sign of zero is kept.  ``e2m1_encode_reference_ties`` restates the
    reference's first-index argmin search (cuda/gemm/fp4_gemm.cu:79-87)
    for a documented cross-check only.
E8M0: unsigned biased exponent, value 2**(code-127), 0xFF = NaN.
"""
from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0
E2M1_MAX = 6.0
E2M1_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                        -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
                       dtype=np.float32)


# --------------------------------------------------------------------------
# bf16 helpers (numpy has no bf16; bf16 = upper 16 bits of an fp32)
# --------------------------------------------------------------------------

def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> exact float32 values."""
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round-to-nearest-even (NaN kept quiet)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = rounded.astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return out


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> float32 holding the nearest-even bf16 value."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# --------------------------------------------------------------------------
# E4M3
# --------------------------------------------------------------------------

def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> E4M3FN code (uint8), RNE, NaN (0x7F|sign) for |x| > 464.

    Normal range (|x| >= 2**-6): round the fp32 mantissa to 3 bits with RNE on
    the integer bit pattern and re-bias the exponent (127 -> 7).  Subnormal
    range: RNE of |x| * 2**9 to an integer 0..8 (8 is the smallest normal,
    code 0x08, so the carry is automatically correct).
    Pinned against torch's float8_e4m3fn cast (tests/test_oracle.py, tests/golden/e4m3_bf16.npy).
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32)
    sign = ((bits >> 31).astype(np.uint8) << 7).astype(np.uint8)
    mag = (bits & 0x7FFFFFFF).astype(np.int64)
    a = np.abs(x)

    # normal path
    r = (mag + 0x7FFFF + ((mag >> 20) & 1)) >> 20      # exp32<<3 | mant3
    code_n = r - ((127 - 7) << 3)
    # subnormal path (np.rint is round-half-to-even)
    with np.errstate(over="ignore", invalid="ignore"):
        code_s = np.rint(a.astype(np.float64) * 512.0)
    code = np.where(a >= np.float32(2.0 ** -6), code_n, code_s)
    nan = ~np.isfinite(a) | (code >= 0x7F)
    code = np.where(nan, 0x7F, code)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


def e4m3_decode(code: np.ndarray) -> np.ndarray:
    """E4M3FN code -> float32 (exact)."""
    c = np.asarray(code, dtype=np.uint8).astype(np.int32)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 7
    val = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = np.where((e == 15) & (m == 7), np.nan, val)
    return (s * val).astype(np.float32)


# --------------------------------------------------------------------------
# E2M1
# --------------------------------------------------------------------------

def e2m1_encode(v: np.ndarray) -> np.ndarray:
    """float32 -> E2M1 code (uint8 in 0..15), RNE with saturation to +-6.

    Magnitude thresholds (ties go to the code with an even mantissa bit):
    <=0.25 -> 0, <0.75 -> 0.5, <=1.25 -> 1, <1.75 -> 1.5, <=2.5 -> 2,
    <3.5 -> 3, <=5 -> 4, else 6.  The sign bit is kept (so -0.1 -> 0x8).
    NaN maps to the saturated code (+-6); inputs on the path are finite.
    Pinned by exhaustive brute force over all bf16 patterns
    (tests/test_oracle.py, tests/golden/e2m1_bf16.npy).
    """
    v = np.ascontiguousarray(v, dtype=np.float32)
    sign = ((v.view(np.uint32) >> 31).astype(np.uint8) << 3).astype(np.uint8)
    a = np.abs(v)
    code = np.full(v.shape, 7, dtype=np.uint8)
    code = np.where(a <= 5.0, 6, code)
    code = np.where(a < 3.5, 5, code)
    code = np.where(a <= 2.5, 4, code)
    code = np.where(a < 1.75, 3, code)
    code = np.where(a <= 1.25, 2, code)
    code = np.where(a < 0.75, 1, code)
    code = np.where(a <= 0.25, 0, code)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


def e2m1_encode_reference_ties(v: np.ndarray) -> np.ndarray:
    """The reference's rounding: first index j minimising |LUT[j] - v| over the
    16-entry table (cuda/gemm/fp4_gemm.cu:79-87).  Ties go to the smaller
    magnitude and -0 becomes +0.  Cross-check only; not the build's contract.
    """
    v = np.asarray(v, dtype=np.float32)[..., None]
    err = np.abs(E2M1_VALUES[None, :] - v)
    return np.argmin(err, axis=-1).astype(np.uint8)


def e2m1_decode(code: np.ndarray) -> np.ndarray:
    return E2M1_VALUES[np.asarray(code, dtype=np.uint8) & 0xF]


def pack_nibbles(codes: np.ndarray) -> np.ndarray:
    """[..., 2n] E2M1 codes -> [..., n] bytes; low nibble = even index."""
    c = np.asarray(codes, dtype=np.uint8)
    assert c.shape[-1] % 2 == 0
    return (c[..., 0::2] & 0xF) | ((c[..., 1::2] & 0xF) << 4)


def unpack_nibbles(packed: np.ndarray) -> np.ndarray:
    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = p & 0xF
    out[..., 1::2] = p >> 4
    return out


# --------------------------------------------------------------------------
# E8M0
# --------------------------------------------------------------------------

def floor_log2(a: np.ndarray) -> np.ndarray:
    """floor(log2(a)) for finite a > 0 by integer exponent extraction
    (exact for fp32 subnormals too); returns int64.  a == 0 -> -1000."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.int64)
    exp = (u >> 23) & 0xFF
    mant = u & 0x7FFFFF
    normal = exp - 127
    # subnormal: value = mant * 2**-149 -> floor(log2) = bitlen(mant)-1-149
    bl = np.zeros_like(mant)
    m = mant.copy()
    for _ in range(23):
        nz = m > 0
        bl += nz
        m >>= 1
    sub = bl - 1 - 149
    out = np.where(exp > 0, normal, sub)
    return np.where(a == 0, -1000, out)


def e8m0_decode(code: np.ndarray) -> np.ndarray:
    c = np.asarray(code, dtype=np.uint8).astype(np.int32)
    val = np.exp2((c - 127).astype(np.float64)).astype(np.float32)
    return np.where(c == 255, np.float32(np.nan), val).astype(np.float32)
