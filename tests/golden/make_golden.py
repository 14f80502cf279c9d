"""Writes the golden fixtures in this directory.  Run from the repo root:

    python tests/golden/make_golden.py

The reference ships no golden vectors for the quantized GEMM path, so these
come from sources independent of ``oracle/``:

* ``e4m3_bf16.npy``   -- torch's ``Tensor.to(torch.float8_e4m3fn)`` of every
  bf16 bit pattern (a library routine, not the oracle's encoder);
* ``e2m1_bf16.npy``   -- brute-force nearest E2M1 value (exact rational distance to
  the eight magnitudes of cuda/gemm/fp4_gemm.cu:30-33, ties to the even
  mantissa code, saturation at 6, sign kept) for every bf16 pattern;
  0xFF marks NaN/Inf inputs;
* ``e8m0_bf16.npy``   -- the MXFP4 shared-exponent byte
  ``clamp(floor(log2 a) - 2, -127, 127) + 127`` from ``math.frexp`` for every
  positive finite bf16 amax; 0 for +-0, 0xFF for negative / non-finite;
* ``kat_gemm.npz``    -- small known-answer cases: seeded bf16 inputs, codes
  and scales from pure-Python scalar quantizers (written with ``math`` and
  loops, not numpy vector code), and float64 triple-loop GEMM outputs.
"""
from __future__ import annotations

import math
import os
import struct
from fractions import Fraction

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
E2M1_MAG = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


# ------------------------------------------------------------ scalar helpers --
def bf16_value(bits: int) -> float:
    return struct.unpack("<f", struct.pack("<I", (bits & 0xFFFF) << 16))[0]


def f32(x: float) -> float:
    """Round a Python float to the nearest fp32 value."""
    return struct.unpack("<f", struct.pack("<f", x))[0]


def e2m1_brute(v: float) -> int:
    if math.isnan(v) or math.isinf(v):
        return 0xFF
    sign = 8 if math.copysign(1.0, v) < 0 else 0
    a = Fraction(abs(v))                     # exact: float64 distances tie for huge |v|
    best, best_d = 0, None
    for code, mag in enumerate(E2M1_MAG):
        d = abs(Fraction(mag) - a)
        if best_d is None or d < best_d or (d == best_d and code % 2 == 0):
            best, best_d = code, d
    return sign | best


def e8m0_frexp(a: float) -> int:
    if math.isnan(a) or math.isinf(a) or a < 0:
        return 0xFF
    if a == 0:
        return 0
    _, e = math.frexp(a)          # a = m * 2**e, 0.5 <= m < 1
    x = (e - 1) - 2
    return max(-127, min(127, x)) + 127


def e4m3_torch(x: float) -> int:
    return int(torch.tensor([x], dtype=torch.float32).to(torch.float8_e4m3fn)
               .view(torch.uint8).item())


def e4m3_value(code: int) -> float:
    s = -1.0 if code & 0x80 else 1.0
    e, m = (code >> 3) & 0xF, code & 7
    if e == 0:
        return s * m * 2.0 ** -9
    if e == 15 and m == 7:
        return float("nan")
    return s * (1 + m / 8.0) * 2.0 ** (e - 7)


def e2m1_value(code: int) -> float:
    return (-1.0 if code & 8 else 1.0) * E2M1_MAG[code & 7]


# --------------------------------------------------------- scalar quantizers --
def q_fp8_tensor(x):
    amax = max(abs(v) for row in x for v in row)
    scale = max(f32(amax / 448.0), f32(1e-12))
    codes = [[e4m3_torch(f32(v / scale)) for v in row] for row in x]
    return codes, scale


def q_fp8_blocks(x, gr, gc):
    R, C = len(x), len(x[0])
    nr, nc = -(-R // gr), -(-C // gc)
    scales = [[0.0] * nc for _ in range(nr)]
    for i in range(nr):
        for j in range(nc):
            amax = max(abs(x[r][c]) for r in range(i * gr, min(R, (i + 1) * gr))
                       for c in range(j * gc, min(C, (j + 1) * gc)))
            scales[i][j] = max(f32(amax / 448.0), f32(1e-12))
    codes = [[e4m3_torch(f32(x[r][c] / scales[r // gr][c // gc])) for c in range(C)]
             for r in range(R)]
    return codes, scales


def q_mxfp4(x):
    codes, e8 = [], []
    for row in x:
        crow, erow = [], []
        for b in range(0, len(row), 32):
            blk = row[b:b + 32]
            code = e8m0_frexp(max(abs(v) for v in blk))
            e = code - 127
            erow.append(code)
            crow.extend(e2m1_brute(f32(v * 2.0 ** (-e))) for v in blk)
        codes.append(crow)
        e8.append(erow)
    return codes, e8


def q_nvfp4(x):
    amax_t = max(abs(v) for row in x for v in row)
    sg = max(f32(amax_t / 2688.0), f32(1e-12))
    codes, sb = [], []
    for row in x:
        crow, srow = [], []
        for b in range(0, len(row), 16):
            blk = row[b:b + 16]
            c = e4m3_torch(f32(f32(max(abs(v) for v in blk) / 6.0) / sg))
            srow.append(c)
            d = f32(e4m3_value(c) * sg)
            crow.extend(0 if d == 0 else e2m1_brute(f32(v / d)) for v in blk)
        codes.append(crow)
        sb.append(srow)
    return codes, sb, sg


def matmul64(a, w):
    """a[M][K] . w[N][K]^T in float64 by triple loop."""
    return [[math.fsum(a[m][k] * w[n][k] for k in range(len(a[0]))) for n in range(len(w))]
            for m in range(len(a))]


def pack(codes):
    return [[(r[i] & 0xF) | ((r[i + 1] & 0xF) << 4) for i in range(0, len(r), 2)] for r in codes]


# --------------------------------------------------------------------- main --
def seeded_bf16(shape, seed, std=1.0, outliers=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g, dtype=torch.float32) * std
    if outliers:
        idx = torch.randperm(x.numel(), generator=g)[:outliers]
        x.view(-1)[idx] *= 50.0
    return x.bfloat16()


def to_list(t):
    return t.float().tolist()


def main():
    bits = np.arange(65536, dtype=np.uint32)
    vals = [bf16_value(int(b)) for b in bits]
    e4m3 = torch.from_numpy((bits << 16).astype(np.uint32).view(np.float32)) \
        .to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.save(os.path.join(HERE, "e4m3_bf16.npy"), e4m3.astype(np.uint8))
    np.save(os.path.join(HERE, "e2m1_bf16.npy"), np.array([e2m1_brute(v) for v in vals], np.uint8))
    np.save(os.path.join(HERE, "e8m0_bf16.npy"), np.array([e8m0_frexp(v) for v in vals], np.uint8))

    kat = {}
    # FP8 per-tensor, M=3 N=5 K=32
    a, w = seeded_bf16((3, 32), 11), seeded_bf16((5, 32), 12, 0.02)
    qa, sa = q_fp8_tensor(to_list(a))
    qw, sw = q_fp8_tensor(to_list(w))
    acc = matmul64([[e4m3_value(c) for c in r] for r in qa], [[e4m3_value(c) for c in r] for r in qw])
    kat.update(fp8t_a=a.view(torch.int16).numpy(), fp8t_w=w.view(torch.int16).numpy(),
               fp8t_qa=np.array(qa, np.uint8), fp8t_sa=np.float32(sa),
               fp8t_qw=np.array(qw, np.uint8), fp8t_sw=np.float32(sw),
               fp8t_c=np.array(acc) * sa * sw)
    # FP8 block-scaled (1x128 activations, 128x128 weights), M=2 N=130 K=256, outliers
    a, w = seeded_bf16((2, 256), 21, outliers=3), seeded_bf16((130, 256), 22, 0.02)
    qa, sa = q_fp8_blocks(to_list(a), 1, 128)
    qw, sw = q_fp8_blocks(to_list(w), 128, 128)
    ad = [[e4m3_value(qa[m][k]) * sa[m][k // 128] for k in range(256)] for m in range(2)]
    wd = [[e4m3_value(qw[n][k]) * sw[n // 128][k // 128] for k in range(256)] for n in range(130)]
    kat.update(fp8b_a=a.view(torch.int16).numpy(), fp8b_w=w.view(torch.int16).numpy(),
               fp8b_qa=np.array(qa, np.uint8), fp8b_sa=np.array(sa, np.float32),
               fp8b_qw=np.array(qw, np.uint8), fp8b_sw=np.array(sw, np.float32),
               fp8b_c=np.array(matmul64(ad, wd)))
    # FP8 groupwise in the reference's own layout (cuda/gemm/fp8_gemm.cu:67-99):
    # sa [M][ceil(K/G)], sb [ceil(K/G)][N] (one scale per output column and
    # K group), G = 128 and 256, K = 320 so the last group is partial (:84-86);
    # C by the group-partial triple loop of that kernel, in float64
    a, w = seeded_bf16((3, 320), 23, outliers=4), seeded_bf16((5, 320), 24, 0.02)
    for G in (128, 256):
        qa, sa = q_fp8_blocks(to_list(a), 1, G)
        qw, swr = q_fp8_blocks(to_list(w), 1, G)          # [N][ceil(K/G)] per weight row
        ng = len(sa[0])
        sb = [[swr[n][g] for n in range(5)] for g in range(ng)]   # [ceil(K/G)][N]
        c = [[math.fsum(math.fsum(e4m3_value(qa[m][k]) * e4m3_value(qw[n][k])
                                  for k in range(g * G, min(g * G + G, 320))) * sa[m][g] * sb[g][n]
                        for g in range(ng)) for n in range(5)] for m in range(3)]
        kat.update({f"fp8g{G}_qa": np.array(qa, np.uint8), f"fp8g{G}_sa": np.array(sa, np.float32),
                    f"fp8g{G}_qw": np.array(qw, np.uint8), f"fp8g{G}_sb": np.array(sb, np.float32),
                    f"fp8g{G}_c": np.array(c)})
    kat.update(fp8g_a=a.view(torch.int16).numpy(), fp8g_w=w.view(torch.int16).numpy())
    # MXFP4, M=2 N=3 K=64, rows spanning a wide dynamic range
    a = (seeded_bf16((2, 64), 31).float() * torch.tensor([[2.0 ** -20], [2.0 ** 30]])).bfloat16()
    w = seeded_bf16((3, 64), 32, 0.02)
    qa, ea = q_mxfp4(to_list(a))
    qw, ew = q_mxfp4(to_list(w))
    ad = [[e2m1_value(qa[m][k]) * 2.0 ** (ea[m][k // 32] - 127) for k in range(64)] for m in range(2)]
    wd = [[e2m1_value(qw[n][k]) * 2.0 ** (ew[n][k // 32] - 127) for k in range(64)] for n in range(3)]
    kat.update(mx_a=a.view(torch.int16).numpy(), mx_w=w.view(torch.int16).numpy(),
               mx_qa=np.array(pack(qa), np.uint8), mx_ea=np.array(ea, np.uint8),
               mx_qw=np.array(pack(qw), np.uint8), mx_ew=np.array(ew, np.uint8),
               mx_c=np.array(matmul64(ad, wd)))
    # NVFP4, M=2 N=3 K=48, one row with a block far below the tensor amax
    af = seeded_bf16((2, 48), 41).float()
    af[1, 16:32] *= 1e-5
    a = af.bfloat16()
    w = seeded_bf16((3, 48), 42, 0.02)
    qa, sba, ga = q_nvfp4(to_list(a))
    qw, sbw, gw = q_nvfp4(to_list(w))
    ad = [[e2m1_value(qa[m][k]) * e4m3_value(sba[m][k // 16]) * ga for k in range(48)]
          for m in range(2)]
    wd = [[e2m1_value(qw[n][k]) * e4m3_value(sbw[n][k // 16]) * gw for k in range(48)]
          for n in range(3)]
    kat.update(nv_a=a.view(torch.int16).numpy(), nv_w=w.view(torch.int16).numpy(),
               nv_qa=np.array(pack(qa), np.uint8), nv_sa=np.array(sba, np.uint8),
               nv_ga=np.float32(ga), nv_qw=np.array(pack(qw), np.uint8),
               nv_sw=np.array(sbw, np.uint8), nv_gw=np.float32(gw),
               nv_c=np.array(matmul64(ad, wd)))
    # grouped FP8 (per-row / per-channel), 4 groups with counts [2, 0, 3, 1], N=4, K=32
    counts = [2, 0, 3, 1]
    offs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    x, w = seeded_bf16((6, 32), 51), seeded_bf16((4, 4, 32), 52, 0.02)
    qx, sx = q_fp8_blocks(to_list(x), 1, 32)
    qw, sw = q_fp8_blocks(to_list(w.reshape(16, 32)), 1, 32)
    y = np.zeros((6, 4))
    for e in range(4):
        for r in range(offs[e], offs[e + 1]):
            for n in range(4):
                dot = math.fsum(e4m3_value(qx[r][k]) * e4m3_value(qw[e * 4 + n][k])
                                for k in range(32))
                y[r, n] = dot * sx[r][0] * sw[e * 4 + n][0]
    kat.update(grp_x=x.view(torch.int16).numpy(), grp_w=w.view(torch.int16).numpy(),
               grp_off=offs, grp_qx=np.array(qx, np.uint8), grp_sx=np.array(sx, np.float32)[:, 0],
               grp_qw=np.array(qw, np.uint8).reshape(4, 4, 32),
               grp_sw=np.array(sw, np.float32)[:, 0].reshape(4, 4), grp_y=y)
    np.savez(os.path.join(HERE, "kat_gemm.npz"), **kat)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
