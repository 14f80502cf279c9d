"""Seeded random grouped FP8 GEMMs and LoRA products through the router.

Group counts are drawn at random (empty groups, single rows, groups of
thousands of rows; the average decides between the grouped streaming tiles
and the persistent walk), N any width and K any multiple of 16, so every
grouped kernel meets ragged groups and odd K.  LoRA draws M, N, K (K % 8),
adapter rank and count (L * R % 8) across its one-pass, two-pass and
vector-ALU plans.  Each product is checked against the oracle on the same
codes (grouped) or the fp64 formula (LoRA: 2e-5).
"""
import numpy as np
import pytest
import torch

from oracle import gemm as OG
from oracle import quant as OQ
from dsl_tool_amd import gemm as G
from dsl_tool_amd import quant as Q
from dsl_tool_amd import workloads as W
from tests.util import assert_close, np_f32, np_u8

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _grouped_cases(seed, n_cases):
    rng = np.random.default_rng(seed)
    out = []
    for c in range(n_cases):
        g = int(rng.integers(1, 80))
        kind = c % 3
        if kind == 0:      # decode-like: a few rows per group, many empty
            counts = rng.integers(0, 12, g) * (rng.random(g) < 0.6)
        elif kind == 1:    # skewed: a Zipf-like spread of group sizes
            counts = np.minimum((rng.pareto(1.2, g) * 60).astype(int), 3000)
        else:              # even: a few hundred rows per group
            counts = rng.integers(100, 600, g)
        n = int(rng.integers(1, 2049))
        k = 16 * int(rng.integers(1, 2048 // 16 + 1))
        # keep the oracle's product near 2e10 multiply-adds at most
        cap = max(1, int(2e10 / (n * k)))
        if counts.sum() > cap:
            counts = (counts * cap) // counts.sum()
        out.append((tuple(int(x) for x in counts), n, k))
    return out


GROUPED = _grouped_cases(8101, 12)


@pytest.mark.parametrize("counts,n,k", GROUPED,
                         ids=lambda v: f"{len(v)}g{sum(v)}r" if isinstance(v, tuple) else str(v))
def test_random_grouped(counts, n, k):
    gn, rows = len(counts), int(sum(counts))
    what = f"random grouped G={gn} rows={rows} N={n} K={k}"
    print(what, flush=True)
    offsets = np.zeros(gn + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    x = W.randn_bf16((max(rows, 1), k), 8200 + gn)[:rows]
    w = W.randn_bf16((gn, n, k), 8300 + n % 101, 0.02)
    qx, sx = Q.quant_fp8_blocks(x.to(DEV), 1, k)
    qw, sw = Q.quant_fp8_blocks(w.reshape(gn * n, k).to(DEV), 1, k)
    out_dtype = torch.float32 if k % 32 else torch.bfloat16
    y = G.grouped_fp8_gemm_packed(qx, sx, qw.reshape(gn, n, k), sw.reshape(gn, n),
                                  torch.from_numpy(offsets).to(DEV), out_dtype=out_dtype)
    assert tuple(y.shape) == (rows, n) and y.dtype == out_dtype
    if rows == 0:
        return
    qx_h, sx_h = OQ.quant_fp8_blockwise(x.float().numpy(), 1, k)
    qw_h, sw_h = OQ.quant_fp8_blockwise(w.reshape(gn * n, k).float().numpy(), 1, k)
    assert np.array_equal(np_u8(qx), qx_h) and np.array_equal(np_u8(qw), qw_h)
    if out_dtype == torch.bfloat16:
        ref = OG.ref_grouped_fp8(qx_h, sx_h[:, 0], qw_h.reshape(gn, n, k), sw_h.reshape(gn, n),
                                 offsets)
    else:
        # ref_grouped_fp8 rounds to bf16: the fp32 output against the fp32 sum
        ref = np.zeros((rows, n), np.float32)
        xd = OG.dequant_fp8_blocks(qx_h, sx_h, 1, k)
        wd = OG.dequant_fp8_blocks(qw_h, sw_h, 1, k).reshape(gn, n, k)
        for e in range(gn):
            r0, r1 = offsets[e], offsets[e + 1]
            if r1 > r0:
                ref[r0:r1] = OG._mm(xd[r0:r1], wd[e])
    assert_close(y, ref, what=what)


def _lora_cases(seed, n_cases):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n_cases):
        m = int(np.exp(rng.uniform(0, np.log(3000))))
        n = 8 * int(rng.integers(1, 2048 // 8 + 1))
        k = 8 * int(rng.integers(1, 2048 // 8 + 1))
        r = int(rng.choice([4, 8, 16, 32, 64]))
        l = int(rng.integers(1, 9))
        while (l * r) % 8:
            l += 1
        out.append((max(m, 1), n, k, r, l))
    return out


@pytest.mark.parametrize("m,n,k,r,l", _lora_cases(8401, 10))
def test_random_lora(m, n, k, r, l):
    print(f"random lora {m}x{n}x{k} r={r} l={l}", flush=True)
    x = W.randn_bf16((m, k), 8500 + m % 31)
    w = W.randn_bf16((n, k), 8501, 0.05)
    a = W.randn_bf16((l, k, r), 8502, 0.05)
    b = W.randn_bf16((l, r, n), 8503, 0.05)
    s = [0.75 * (i + 1) * (-1) ** i for i in range(l)]
    y = G.lora_fused_gemm(x.to(DEV), w.to(DEV).t(), a.to(DEV), b.to(DEV), s)
    assert tuple(y.shape) == (m, n) and y.dtype == torch.float32
    ref = OG.ref_lora(x.float().numpy(), w.float().numpy(), a.float().numpy(), b.float().numpy(), s)
    glob, _ = OG.rel_errors(np_f32(y), ref)
    assert glob <= 2e-5, f"lora {m}x{n}x{k} r={r} l={l}: {glob:.3g}"
