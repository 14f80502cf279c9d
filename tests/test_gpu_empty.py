"""Empty operands through the Python entry points on the GPU: no rows, no
output columns, an all-empty grouped table.  Each call returns a correctly
shaped (empty or unchanged) result without launching work that would read
past the empty operands."""
import pytest
import torch

from dsl_tool_amd import gemm as G
from dsl_tool_amd import quant as Q

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bf16(*shape):
    return torch.randn(shape, device=DEV).to(torch.bfloat16)


@pytest.mark.parametrize("m,n", [(0, 256), (64, 0), (0, 0)])
def test_fp8_and_bf16_gemm_with_empty_sides(m, n):
    k = 256
    a, w = _bf16(m, k), _bf16(n, k)
    c = G.fp8_gemm(a, w.t())
    assert tuple(c.shape) == (m, n)
    c = G.fp8_gemm(a, w.t(), granularity="block")
    assert tuple(c.shape) == (m, n)
    c = G.bf16_gemm(a, w.t())
    assert tuple(c.shape) == (m, n) and c.dtype == torch.float32
    c = G.fp4_gemm(a, w.t(), fmt="mxfp4")
    assert tuple(c.shape) == (m, n)


def test_quantizers_with_no_rows():
    x = _bf16(0, 256)
    q, s = Q.quant_fp8_blocks(x, 1, 128)
    assert tuple(q.shape) == (0, 256) and tuple(s.shape) == (0, 2)
    q, e = Q.quant_mxfp4(x)
    assert tuple(q.shape) == (0, 128) and tuple(e.shape) == (0, 8)
    # the per-tensor and NVFP4 global scales of an empty tensor are those of
    # amax 0: the 1e-12 floor (cuda/gemm/fp8_gemm.cu:133-134), not left unset
    q, s = Q.quant_fp8_tensor(x)
    assert tuple(q.shape) == (0, 256) and s.item() == torch.tensor(1e-12, dtype=torch.float32).item()
    q, sb, sg = Q.quant_nvfp4(x)
    assert tuple(q.shape) == (0, 128) and tuple(sb.shape) == (0, 16)
    assert sg.item() == torch.tensor(1e-12, dtype=torch.float32).item()


def test_grouped_with_every_group_empty():
    k, n, g = 256, 128, 4
    qx, sx = Q.quant_fp8_blocks(_bf16(0, k), 1, k)
    qw, sw = Q.quant_fp8_blocks(_bf16(g * n, k), 1, k)
    off = torch.zeros(g + 1, dtype=torch.int32, device=DEV)
    y = G.grouped_fp8_gemm_packed(qx, sx, qw.reshape(g, n, k), sw.reshape(g, n), off)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (0, n)


def test_lora_with_no_tokens():
    k, n, r, l = 256, 128, 8, 2
    y = G.lora_fused_gemm(_bf16(0, k), _bf16(n, k).t(), _bf16(l, k, r), _bf16(l, r, n), [1.0, 2.0])
    torch.cuda.synchronize()
    assert tuple(y.shape) == (0, n) and y.dtype == torch.float32
