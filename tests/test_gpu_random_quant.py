"""Seeded random quantizer inputs, bit for bit against the oracle.

Sizes from one row up to a few thousand, columns any multiple of the
format's unit (FP8 any, NVFP4 16, MXFP4 32), bf16 / fp16 / fp32 sources,
contiguous, row-padded and transposed (the reference's B[K, N] read as its
[N, K] view) layouts, magnitudes spread over several decades with rare
outliers: codes and scales must equal the oracle's exactly.
"""
import numpy as np
import pytest
import torch

from oracle import quant as OQ
from dsl_tool_amd import quant as Q
from tests.util import np_f32, np_u8

pytestmark = pytest.mark.gpu
DEV = "cuda"

FORMATS = ["fp8_tensor", "fp8_rows", "fp8_tiles", "mxfp4", "nvfp4"]
UNIT = {"fp8_tensor": 1, "fp8_rows": 1, "fp8_tiles": 1, "mxfp4": 32, "nvfp4": 16}


def _cases(seed, per_format=5):
    rng = np.random.default_rng(seed)
    out = []
    for f in FORMATS:
        for _ in range(per_format):
            r = max(1, int(np.exp(rng.uniform(0, np.log(3000)))))
            u = UNIT[f]
            c = u * max(1, int(np.exp(rng.uniform(np.log(max(u, 8)), np.log(3000))) // u))
            dt = str(rng.choice(["bf16", "fp16", "fp32"]))
            layout = str(rng.choice(["contiguous", "padded", "transposed"]))
            out.append((f, r, c, dt, layout, int(rng.integers(0, 1 << 30))))
    return out


DT = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


@pytest.mark.parametrize("fmt,r,c,dt,layout,seed", _cases(9001), ids=lambda v: str(v))
def test_random_quant(fmt, r, c, dt, layout, seed):
    print(f"random quant {fmt} {r}x{c} {dt} {layout}", flush=True)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((r, c), generator=g) * torch.exp(torch.empty((r, 1)).uniform_(-4, 4, generator=g))
    spikes = torch.rand((r, c), generator=g) < 1e-3
    x = torch.where(spikes, x * 50, x)
    if dt == "fp16":
        x = x.clamp(-6e4, 6e4)
    x = x.to(DT[dt])
    ref_in = x.float().numpy()                     # the source's own values, exactly
    if layout == "padded":
        buf = torch.zeros((r, c + 24), dtype=x.dtype)
        buf[:, :c] = x
        xd = buf.to(DEV)[:, :c]
    elif layout == "transposed":
        xd = x.t().contiguous().to(DEV).t()
    else:
        xd = x.to(DEV)
    if fmt == "fp8_tensor":
        q, s = Q.quant_fp8_tensor(xd)
        q_ref, s_ref = OQ.quant_fp8_per_tensor(ref_in)
        assert np_f32(s)[0] == s_ref
    elif fmt in ("fp8_rows", "fp8_tiles"):
        gr, gc = (1, 128) if fmt == "fp8_rows" else (128, 128)
        q, s = Q.quant_fp8_blocks(xd, gr, gc)
        q_ref, s_ref = OQ.quant_fp8_blockwise(ref_in, gr, gc)
        assert np.array_equal(np_f32(s), s_ref)
    elif fmt == "mxfp4":
        q, s = Q.quant_mxfp4(xd)
        q_ref, s_ref = OQ.quant_mxfp4(ref_in)
        assert np.array_equal(np_u8(s), s_ref)
    else:
        q, s, sg = Q.quant_nvfp4(xd)
        q_ref, s_ref, sg_ref = OQ.quant_nvfp4(ref_in)
        assert np_f32(sg)[0] == sg_ref
        assert np.array_equal(np_u8(s), s_ref)
    assert np.array_equal(np_u8(q), q_ref)
