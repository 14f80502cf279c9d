"""GPU: dsl_quant_fp8_tensor_noalloc (library-held amax partials, no
workspace, no allocation) against dsl_quant_fp8_tensor (caller workspace),
byte for byte, on two calls in a row with the second input smaller than the
first (the library's array then still holds the first call's partials)."""
import numpy as np
import pytest
import torch

from dsl_tool_amd import _native as N
from dsl_tool_amd import workloads as W
from oracle import quant as OQ

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _with_workspace(x: torch.Tensor, x_dtype: int):
    r, c = x.shape
    q = torch.empty((r, c), dtype=torch.uint8, device=DEV)
    s = torch.empty(1, dtype=torch.float32, device=DEV)
    nb = N.lib().dsl_quant_workspace_bytes(r, c)
    ws = torch.empty(nb // 4, dtype=torch.float32, device=DEV)
    N.call("dsl_quant_fp8_tensor", N.ptr(x), r, c, x.stride(0), x.stride(1), x_dtype, N.ptr(q),
           N.ptr(s), N.ptr(ws), nb, N.stream_of(x.device))
    return q, s


def _no_alloc(x: torch.Tensor, x_dtype: int):
    r, c = x.shape
    q = torch.empty((r, c), dtype=torch.uint8, device=DEV)
    s = torch.empty(1, dtype=torch.float32, device=DEV)
    N.call("dsl_quant_fp8_tensor_noalloc", N.ptr(x), r, c, x.stride(0), x.stride(1), x_dtype,
           N.ptr(q), N.ptr(s), N.stream_of(x.device))
    return q, s


def _same(a, b):
    torch.cuda.synchronize()
    return torch.equal(a[0], b[0]) and torch.equal(a[1].view(torch.int32), b[1].view(torch.int32))


def test_no_alloc_matches_workspace_entry_point_twice():
    big = W.activations(1, 4096, 4096).to(DEV)          # 1024 amax partials
    small = (W.randn_bf16((300, 272), 77) * 3).to(DEV)  # a handful, strided path
    for x in (big, small):
        assert _same(_no_alloc(x, N.IN_BF16), _with_workspace(x, N.IN_BF16))
    # the smaller call's result is its own: a larger amax left behind by the
    # first call must not leak into the scale
    q, s = _no_alloc(small, N.IN_BF16)
    torch.cuda.synchronize()
    q_ref, s_ref = OQ.quant_fp8_per_tensor(small.float().cpu().numpy())
    assert float(s.cpu()[0]) == s_ref
    assert np.array_equal(q.cpu().numpy(), q_ref)


def test_no_alloc_fp32_source_and_strided_view():
    x32 = torch.from_numpy(np.random.default_rng(8).standard_normal((512, 1024)).astype(np.float32) * 7)
    b_kn = x32.to(DEV).t()                                # [1024, 512] view, stride (1, 1024)
    assert _same(_no_alloc(b_kn, N.IN_F32), _with_workspace(b_kn, N.IN_F32))
    x16 = x32[:64, :256].contiguous().bfloat16().to(DEV)
    assert _same(_no_alloc(x16, N.IN_BF16), _with_workspace(x16, N.IN_BF16))


_CAPTURE_CHILD = r"""
import sys, torch
sys.path.insert(0, sys.argv[1])
from dsl_tool_amd import _native as N
dev = torch.device("cuda:0")
torch.cuda.set_device(dev)
g0 = torch.Generator().manual_seed(5)
x = (torch.randn((1024, 2048), generator=g0) * 3).bfloat16().to(dev)
q = torch.empty((1024, 2048), dtype=torch.uint8, device=dev)
s = torch.empty(1, dtype=torch.float32, device=dev)
side = torch.cuda.Stream(device=dev)          # capture stream, default priority
graph = torch.cuda.CUDAGraph()
# the process's first call of the entry point happens inside the capture
with torch.cuda.graph(graph, stream=side):
    N.call("dsl_quant_fp8_tensor_noalloc", N.ptr(x), 1024, 2048, 2048, 1, N.IN_BF16, N.ptr(q),
           N.ptr(s), torch.cuda.current_stream(dev).cuda_stream)
nb = N.lib().dsl_quant_workspace_bytes(1024, 2048)
ws = torch.empty(nb // 4, dtype=torch.float32, device=dev)
for rep in range(3):
    if rep == 2:
        x.mul_(0.25)                            # new input between replays
    graph.replay()
    torch.cuda.synchronize()
    q2 = torch.empty_like(q)
    s2 = torch.empty_like(s)
    N.call("dsl_quant_fp8_tensor", N.ptr(x), 1024, 2048, 2048, 1, N.IN_BF16, N.ptr(q2), N.ptr(s2),
           N.ptr(ws), nb, torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(q, q2) and torch.equal(s.view(torch.int32), s2.view(torch.int32)), rep
print("capture ok")
"""


def test_no_alloc_first_call_inside_graph_capture():
    """In a fresh process, the entry point's first call (which looks up the
    library-held array's device address) is made inside HIP graph capture;
    the captured graph, replayed three times with the input changed before
    the last replay, matches dsl_quant_fp8_tensor byte for byte each time."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD, root], capture_output=True,
                         text=True, timeout=300)
    assert res.returncode == 0 and "capture ok" in res.stdout, res.stdout + res.stderr
