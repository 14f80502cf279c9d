"""GPU bf16 GEMM (gemm.bf16_gemm) against the exact-sum oracle.

bf16 x bf16 products are exact in fp32, so the oracle (fp64 sum, one
rounding to fp32) is the exact answer; the GPU accumulates in fp32 in its
own order.  fp32 output is bounded by F32_TOL relative to max|R|; bf16
output by the usual north-star bound after rounding the oracle to bf16.
"""
import numpy as np
import pytest
import torch

from oracle import gemm as OG
from oracle import formats as F
from dsl_tool_amd import _native as N
from dsl_tool_amd import gemm as G
from dsl_tool_amd import workloads as W
from tests.util import assert_close, np_f32

pytestmark = pytest.mark.gpu
DEV = "cuda"

# fp32 accumulation over K <= 4096 of unit-variance products: a few ulp of
# max|C| (the MFMA's internal order and alignment included).
F32_TOL = 2e-5

SHAPES = [
    (4096, 4352, 512),    # persistent kernel (272 tiles of 256x256)
    (2048, 2048, 1024),   # register-staged 256x256 tiles
    (300, 520, 264),      # ragged M / N, K % 64 != 0
    (513, 257, 136),
    (16, 2048, 4096),     # 2 <= M <= 16: the decode kernel
    (12, 7168, 1024),
    (32, 7168, 1024),     # 17 <= M <= 256: the streaming kernel
    (16, 512, 1032),      # small M, other K: split K over a workspace
    (1, 256, 64),
    (128, 4096, 2048),
    (72, 1000, 512),
    (48, 4000, 1024),     # 33..64 rows in one round: two 32-row blocks of two W tiles
    (520, 1000, 1024),    # more than 256 rows on the streaming kernel (small N)
    (1536, 1024, 1024),   # pipelined 128x128 tiles (too few 256x256 tiles for a persistent round)
    (1100, 2000, 512),    # the same with ragged M and N
]


def _inputs(m, n, k, seed):
    a = W.randn_bf16((m, k), seed)
    w = W.randn_bf16((n, k), seed + 1)
    return a, w


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_bf16_gemm_matches_exact_oracle(m, n, k, out_dtype):
    a, w = _inputs(m, n, k, 200)
    c = G.bf16_gemm(a.to(DEV), w.to(DEV).t(), out_dtype=out_dtype)
    ref = OG.ref_bf16(a.float().numpy(), w.float().numpy())
    assert c.dtype == out_dtype and tuple(c.shape) == (m, n)
    if out_dtype == torch.float32:
        glob, _ = OG.rel_errors(np_f32(c), ref)
        assert glob <= F32_TOL, f"bf16 {m}x{n}x{k} fp32 out: max|C-R|/max|R| = {glob:.3g}"
    else:
        assert_close(c, F.round_to_bf16(ref), what=f"bf16 {m}x{n}x{k} bf16 out")


def test_bf16_gemm_reference_layout_b_is_copied_to_k_major():
    # the reference's B [K, N] as a contiguous tensor (not a W.t() view)
    a, w = _inputs(200, 300, 192, 210)
    b_kn = w.t().contiguous()
    c = G.bf16_gemm(a.to(DEV), b_kn.to(DEV))
    ref = OG.ref_bf16(a.float().numpy(), w.float().numpy())
    glob, _ = OG.rel_errors(np_f32(c), ref)
    assert glob <= F32_TOL
    # a strided (non-contiguous) A is copied too
    wide = W.randn_bf16((200, 256), 212)
    a2 = wide.to(DEV)[:, :192]
    c2 = G.bf16_gemm(a2, b_kn.to(DEV))
    ref2 = OG.ref_bf16(wide[:, :192].float().numpy(), w.float().numpy())
    assert OG.rel_errors(np_f32(c2), ref2)[0] <= F32_TOL


def test_bf16_gemm_exact_on_small_integers():
    # integer-valued operands with exact fp32 sums: the result is exact
    g = torch.Generator().manual_seed(213)
    a = torch.randint(-8, 9, (256, 512), generator=g).to(torch.bfloat16)
    w = torch.randint(-8, 9, (512, 512), generator=g).to(torch.bfloat16)
    c = G.bf16_gemm(a.to(DEV), w.to(DEV).t())
    ref = a.double() @ w.double().t()
    assert torch.equal(c.cpu().double(), ref)


def test_bf16_gemm_argument_errors():
    a = torch.zeros((16, 24), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(TypeError):
        G.bf16_gemm(a.float(), a.t())
    with pytest.raises(ValueError):
        G.bf16_gemm(a, torch.zeros((16, 8), dtype=torch.bfloat16, device=DEV))
    odd = torch.zeros((16, 12), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(N.DslError):
        G.bf16_gemm(odd, odd.t())
