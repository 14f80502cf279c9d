"""LoRA fused GEMM (gemm.lora_fused_gemm) against the float64 formula of
cuda/gemm/grouped_gemm.cu:106-140 on the same bf16 operands.

The base product accumulates in fp32 and the adapter term is carried as a
bf16 hi + lo pair, so the result sits within LORA_TOL of max|Y| (measured
~1e-6; the bound leaves room for K = 4096 sums)."""
import numpy as np
import pytest
import torch

from oracle import gemm as OG
from dsl_tool_amd import gemm as G
from dsl_tool_amd import workloads as W
from tests.util import np_f32

pytestmark = pytest.mark.gpu
DEV = "cuda"
LORA_TOL = 2e-5


# T = X A^T is computed transposed on the streaming kernel when L*R <= 256
# and K suits it (its epilogue writes the scaled hi | lo pair, transposed
# back); K = 264 and L*R = 320 take the register-staged tiles and a separate
# split pass.  With L*R = 64, 128 or 256 the base GEMM reads B^T twice
# instead of a copied B^T | B^T (1, 2 and 4 pairs per row); L*R = 24, 32, 48
# take the copy (24 and 48 also pad hi | lo to 64 columns).  Up to 256 rows
# the base GEMM runs on its own kernel, T*s comes from the vector-ALU kernel
# (as hi | lo, padded: L*R = 24 at M = 40) and the adapter term is added by a
# second streaming pass into the fp32 result (M = 8..256; N = 2056 leaves a
# ragged column edge for that pass's scalar epilogue); M = 1, 2 add it on
# the vector ALUs in fp32; L*R = 640 at M = 8 takes the register-staged T.
# M = 1536 N = 1024 and M = 2000 N = 1100 run the base GEMM and the add on
# the 128x128 pipelined tiles (one round of them).
@pytest.mark.parametrize("m,n,k,r,l", [(512, 768, 1024, 16, 2), (300, 520, 264, 8, 3),
                                       (4096, 4352, 512, 16, 4), (16, 256, 2048, 64, 1),
                                       (256, 512, 1024, 64, 5), (1024, 1024, 4096, 16, 4),
                                       (512, 640, 4096, 32, 4), (256, 1000, 2048, 64, 4),
                                       (300, 520, 3072, 24, 2), (700, 260, 2048, 8, 3),
                                       (1, 4096, 4096, 16, 4), (64, 2056, 1024, 32, 2),
                                       (40, 520, 1024, 8, 3), (2, 1000, 512, 8, 2),
                                       (8, 512, 1024, 64, 10), (1536, 1024, 1024, 16, 4),
                                       (2000, 1100, 512, 8, 3)])
def test_lora_fused_gemm(m, n, k, r, l):
    x = W.randn_bf16((m, k), 500)
    w = W.randn_bf16((n, k), 501, 0.05)
    a = W.randn_bf16((l, k, r), 502, 0.05)
    b = W.randn_bf16((l, r, n), 503, 0.05)
    s = [1.5 * (i + 1) * (-1) ** i for i in range(l)]
    y = G.lora_fused_gemm(x.to(DEV), w.to(DEV).t(), a.to(DEV), b.to(DEV), s)
    ref = OG.ref_lora(x.float().numpy(), w.float().numpy(), a.float().numpy(), b.float().numpy(), s)
    glob, _ = OG.rel_errors(np_f32(y), ref)
    assert glob <= LORA_TOL, f"lora {m}x{n}x{k} r={r} l={l}: {glob:.3g}"
    # the adapter term is a visible part of the result
    base = OG.ref_lora(x.float().numpy(), w.float().numpy(), a.float().numpy() * 0, b.float().numpy(), s)
    assert OG.rel_errors(base, ref)[0] > 100 * LORA_TOL


def test_lora_reference_layout_w_and_tensor_scales():
    x = W.randn_bf16((128, 256), 510)
    w_kn = W.randn_bf16((256, 384), 511, 0.05)          # contiguous [K, N]
    a = W.randn_bf16((2, 256, 8), 512, 0.05)
    b = W.randn_bf16((2, 8, 384), 513, 0.05)
    s = torch.tensor([0.25, 4.0])
    y = G.lora_fused_gemm(x.to(DEV), w_kn.to(DEV), a.to(DEV), b.to(DEV), s.to(DEV))
    ref = OG.ref_lora(x.float().numpy(), w_kn.float().numpy().T, a.float().numpy(), b.float().numpy(),
                      s.numpy())
    assert OG.rel_errors(np_f32(y), ref)[0] <= LORA_TOL
