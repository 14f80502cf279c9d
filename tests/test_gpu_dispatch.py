"""GPU: the hip entries driven through KernelDispatcher.run_from_spec and the
REST service exactly as a CLI/REST caller drives them (bf16 specs in, bf16
out), checked against the oracle."""
import base64

import numpy as np
import pytest
import torch

from dsl_tool_amd.dispatcher import KernelDispatcher
from oracle import gemm as OG
from oracle import quant as OQ
from tests.util import assert_close

pytestmark = pytest.mark.gpu


def _spec(t: torch.Tensor) -> dict:
    return {"shape": list(t.shape), "dtype": "bfloat16",
            "data": base64.b64encode(t.float().numpy().tobytes()).decode()}


def _seeded(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).bfloat16()


def test_run_from_spec_fp8_and_fp4():
    d = KernelDispatcher()
    a, w = _seeded((32, 256), 901), _seeded((64, 256), 902, 0.02)
    res = d.run_from_spec("gemm.fp8_gemm", "hip", [_spec(a), _spec(w.t().contiguous())],
                          {"scale_a": 1.0, "scale_b": 1.0})
    qa, sa = OQ.quant_fp8_per_tensor(a.float().numpy())
    qw, sw = OQ.quant_fp8_per_tensor(w.float().numpy())
    assert_close(res.output, OG.ref_fp8_per_tensor(qa, sa, qw, sw), what="dispatch fp8")
    res = d.run_from_spec("gemm.fp4_gemm", "hip", [_spec(a), _spec(w.t().contiguous())],
                          {"fmt": "nvfp4"})
    pa, sba, ga = OQ.quant_nvfp4(a.float().numpy())
    pw, sbw, gw = OQ.quant_nvfp4(w.float().numpy())
    assert_close(res.output, OG.ref_nvfp4(pa, sba, ga, pw, sbw, gw), what="dispatch nvfp4")


def test_rest_run_grouped_with_offsets():
    from fastapi.testclient import TestClient

    from dsl_tool_amd.dispatcher.api import app
    x, w = _seeded((40, 128), 903), _seeded((3, 128, 32), 904, 0.02)     # B [G, K, N]
    off = np.array([0, 15, 15, 40], np.int32)
    req = {"kernel_name": "gemm.grouped_gemm", "backend": "hip",
           "inputs": [_spec(x), _spec(w),
                      {"shape": [4], "dtype": "int32",
                       "data": base64.b64encode(off.tobytes()).decode()}]}
    with TestClient(app) as c:
        r = c.post("/api/v1/kernels/run", json=req)
    assert r.status_code == 200, r.text
    out = r.json()["output"]
    y = np.frombuffer(base64.b64decode(out["data"]), np.float32).reshape(out["shape"])
    qx, sx = OQ.quant_fp8_blockwise(x.float().numpy(), 1, 128)
    wt = w.transpose(1, 2).reshape(96, 128).float().numpy()
    qw, sw = OQ.quant_fp8_blockwise(wt, 1, 128)
    ref = OG.ref_grouped_fp8(qx, sx[:, 0], qw.reshape(3, 32, 128), sw.reshape(3, 32), off)
    glob, elem = OG.rel_errors(y, ref)
    assert glob <= 1e-2 and elem <= 1e-2
