"""Caller-provided outputs with padded rows (ldc > N, odd) on every dense route.

The router does not look at ldc, so the same kernel runs for a contiguous
output and for a padded one: the N columns must come out byte for byte the
same, and the padding (NaN sentinels) must stay untouched.  An odd ldc turns
off every vectorized store path (8- and 16-byte C writes need ldc % 4 or
% 8), so the per-element edge stores of each kernel are exercised on whole
tiles too.  One product per shape is checked against the oracle as well.
"""
import numpy as np
import pytest
import torch

from oracle import gemm as OG
from dsl_tool_amd import gemm as G
from dsl_tool_amd import quant as Q
from dsl_tool_amd import workloads as W
from tests.util import assert_close, np_u8, np_f32

pytestmark = pytest.mark.gpu
DEV = "cuda"

# (m, n, k): decode kernel (N/32 workgroups fill the CUs), streaming kernel,
# one round of 128x128 pipelined tiles, persistent 256x256 tiles, and the
# register-staged tiles (K not a multiple of 64)
ROUTES = {
    "decode": (16, 8192, 1024),
    "stream": (128, 4096, 1024),
    "tiles128": (1100, 3000, 1024),
    "persistent": (4096, 4096, 512),
    "staged": (300, 500, 1056),
}
PAD = 3


def _run(mode, a, w, out):
    if mode == "tensor":
        qa, sa = Q.quant_fp8_tensor(a)
        qw, sw = Q.quant_fp8_tensor(w)
        c = G.fp8_gemm_packed(qa, qw, sa, sw, out_dtype=out.dtype, out=out)
        return c, lambda: OG.ref_fp8_per_tensor(np_u8(qa), np_f32(sa)[0], np_u8(qw), np_f32(sw)[0])
    if mode == "mxfp4":
        qa, ea = Q.quant_mxfp4(a)
        qw, ew = Q.quant_mxfp4(w)
        c = G.fp4_gemm_packed(qa, ea, qw, ew, fmt="mxfp4", out_dtype=out.dtype, out=out)
        return c, lambda: OG.ref_mxfp4(np_u8(qa), np_u8(ea), np_u8(qw), np_u8(ew))
    c = G.bf16_gemm(a, w.t(), out_dtype=out.dtype, out=out)
    return c, lambda: OG.ref_bf16(a.float().cpu().numpy(), w.float().cpu().numpy())


@pytest.mark.parametrize("route", sorted(ROUTES))
@pytest.mark.parametrize("mode", ["tensor", "mxfp4", "bf16"])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_padded_output_rows(route, mode, out_dtype):
    m, n, k = ROUTES[route]
    if mode == "mxfp4" and k % 32:
        k += 32 - k % 32
    a = W.randn_bf16((m, k), 971).to(DEV)
    w = W.randn_bf16((n, k), 972, 0.02).to(DEV)
    what = f"padded out {route} {mode} {m}x{n}x{k} {out_dtype}"
    dense = torch.empty((m, n), dtype=out_dtype, device=DEV)
    c0, ref = _run(mode, a, w, dense)
    big = torch.full((m, n + PAD), float("nan"), dtype=out_dtype, device=DEV)
    view = big[:, :n]
    c1, _ = _run(mode, a, w, view)
    torch.cuda.synchronize()
    assert c1.data_ptr() == big.data_ptr() and c1.stride(0) == n + PAD
    assert torch.equal(c1, c0), f"{what}: padded result differs from the contiguous one"
    assert torch.isnan(big[:, n:]).all(), f"{what}: padding columns were written"
    if route in ("stream", "staged") and out_dtype == torch.float32:
        r = ref()
        if mode == "bf16":
            np.testing.assert_allclose(c0.cpu().numpy(), r, rtol=0,
                                       atol=2e-5 * float(np.abs(r).max()), err_msg=what)
        else:
            assert_close(c0, r, what=what)
