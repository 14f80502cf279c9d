"""Seeded random shapes on every mode, through whatever kernel the router picks.

The other GPU tests pin each kernel on shapes chosen for it; these draw
shapes at random (fixed seed, so every run draws the same ones) within the
C ABI's documented limits, from 1 row or column up to several rounds of the
largest tiles, with K any multiple of the mode's unit, so that route edges,
ragged tiles and short or odd K meet every mode.  Each product is checked
against the dequantize -> matmul oracle on the same codes: the north-star
bound, and for block scales the derived elementwise bound of the rescaling
kernels.
"""
import numpy as np
import pytest
import torch

from oracle import formats as OF
from oracle import gemm as OG
from dsl_tool_amd import gemm as G
from dsl_tool_amd import quant as Q
from dsl_tool_amd import workloads as W
from tests.util import (assert_close, assert_close_block_bound, block_fp8_error_bound, np_f32,
                        np_u8)

pytestmark = pytest.mark.gpu
DEV = "cuda"

# K unit per mode: FP8 K % 16, FP4 K % 32, bf16 K % 8 (the C ABI's checks)
UNIT = {"tensor": 16, "block": 16, "group": 16, "mxfp4": 32, "nvfp4": 32, "bf16": 8}


def _shapes(mode, seed):
    rng = np.random.default_rng(seed)
    u = UNIT[mode]
    out = []
    for _ in range(6):     # 1 .. 2500 rows / columns, K up to 3072
        m = int(np.exp(rng.uniform(0, np.log(2500))))
        n = int(np.exp(rng.uniform(0, np.log(2500))))
        k = u * int(rng.integers(1, 3072 // u + 1))
        out.append((max(m, 1), max(n, 1), k))
    for _ in range(3):     # a few rounds of the large tiles, short K
        m = int(rng.integers(1500, 6000))
        n = int(rng.integers(1500, 6000))
        k = u * int(rng.integers(1, 768 // u + 1))
        out.append((m, n, k))
    return out


CASES = [(mode, *s) for i, mode in enumerate(sorted(UNIT)) for s in _shapes(mode, 7001 + i)]


@pytest.mark.parametrize("mode,m,n,k", CASES, ids=lambda v: str(v))
def test_random_shape(mode, m, n, k):
    out_dtype = torch.float32 if (m + n + k) % 2 else torch.bfloat16
    what = f"random {mode} {m}x{n}x{k} {out_dtype}"
    print(what, flush=True)
    a = W.randn_bf16((m, k), 7100 + m % 97)
    w = W.randn_bf16((n, k), 7200 + n % 89, 0.02)
    if mode == "tensor":
        qa, sa = Q.quant_fp8_tensor(a.to(DEV))
        qw, sw = Q.quant_fp8_tensor(w.to(DEV))
        c = G.fp8_gemm_packed(qa, qw, sa, sw, out_dtype=out_dtype)
        ref = OG.ref_fp8_per_tensor(np_u8(qa), np_f32(sa)[0], np_u8(qw), np_f32(sw)[0])
    elif mode == "block":
        qa, sa = Q.quant_fp8_blocks(a.to(DEV), 1, 128)
        qw, sw = Q.quant_fp8_blocks(w.to(DEV), 128, 128)
        c = G.fp8_gemm_packed(qa, qw, sa, sw, block=True, out_dtype=out_dtype)
        qa_h, sa_h, qw_h, sw_h = np_u8(qa), np_f32(sa), np_u8(qw), np_f32(sw)
        ref = OG.ref_fp8_groupwise(qa_h, sa_h, qw_h, sw_h)
        assert c.dtype == out_dtype
        assert_close_block_bound(c, ref, block_fp8_error_bound(qa_h, sa_h, qw_h, sw_h), what=what)
        return
    elif mode == "group":
        qa, sa = Q.quant_fp8_blocks(a.to(DEV), 1, 128)
        qw, swr = Q.quant_fp8_blocks(w.to(DEV), 1, 128)
        sb = swr.t().contiguous()
        c = G.fp8_gemm_packed(qa, qw, sa, sb, group=True, out_dtype=out_dtype)
        ref = OG.ref_fp8_groupwise_cols(np_u8(qa), np_f32(sa), np_u8(qw), np_f32(sb), 128)
    elif mode == "mxfp4":
        qa, ea = Q.quant_mxfp4(a.to(DEV))
        qw, ew = Q.quant_mxfp4(w.to(DEV))
        c = G.fp4_gemm_packed(qa, ea, qw, ew, fmt="mxfp4", out_dtype=out_dtype)
        ref = OG.ref_mxfp4(np_u8(qa), np_u8(ea), np_u8(qw), np_u8(ew))
    elif mode == "nvfp4":
        qa, sa, ga = Q.quant_nvfp4(a.to(DEV))
        qw, sw, gw = Q.quant_nvfp4(w.to(DEV))
        c = G.fp4_gemm_packed(qa, sa, qw, sw, fmt="nvfp4", global_a=ga, global_w=gw,
                              out_dtype=out_dtype)
        ref = OG.ref_nvfp4(np_u8(qa), np_u8(sa), np_f32(ga)[0], np_u8(qw), np_u8(sw),
                           np_f32(gw)[0])
    else:
        c = G.bf16_gemm(a.to(DEV), w.to(DEV).t(), out_dtype=out_dtype)
        ref = OG.ref_bf16(a.float().numpy(), w.float().numpy())
        if out_dtype == torch.bfloat16:
            ref = OF.round_to_bf16(ref)
    assert c.dtype == out_dtype and tuple(c.shape) == (m, n)
    assert_close(c, ref, what=what)


# The smallest K each mode accepts (one MFMA step or less), at row counts that
# take the decode, streaming, 128x128 and persistent routes (or their
# short-K fallbacks).
MIN_K_CASES = [(mode, m, 512, {"bf16": 8, "mxfp4": 32, "nvfp4": 32}.get(mode, 16))
               for mode in sorted(UNIT) for m in (1, 16, 300, 4096)]


@pytest.mark.parametrize("mode,m,n,k", MIN_K_CASES, ids=lambda v: str(v))
def test_minimum_k(mode, m, n, k):
    test_random_shape(mode, m, n, k)
