"""Operand views the kernels cannot read in place: a storage offset that is
not a multiple of 16 bytes, or a row stride that is not a multiple of 8
elements.  The C ABI refuses such pointers; the Python entry points copy
them to fresh storage first, so every call must give exactly the bytes the
same values in fresh contiguous tensors give."""
import pytest
import torch

from dsl_tool_amd import fused as F
from dsl_tool_amd import gemm as G
from dsl_tool_amd import moe as M
from dsl_tool_amd import quant as Q

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bf16(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16).to(DEV)


def _offset_view(t, elems):
    """The values of contiguous ``t`` in a view starting ``elems`` elements
    into a larger buffer (so its start is misaligned for elems * size % 16)."""
    buf = torch.zeros(t.numel() + elems + 16, dtype=t.dtype, device=t.device)
    v = buf[elems:elems + t.numel()].view(t.shape)
    v.copy_(t)
    assert v.data_ptr() % 16 != 0
    return v


def _padded_rows(t, pad):
    """``t`` [rows, cols] in a view whose row stride is cols + pad."""
    r, c = t.shape
    buf = torch.zeros((r, c + pad), dtype=t.dtype, device=t.device)
    buf[:, :c] = t
    return buf[:, :c]


@pytest.mark.parametrize("m,n,k", [(1, 256, 512), (300, 500, 1024), (2048, 2048, 512)])
def test_fp8_and_fp4_codes_at_odd_offsets(m, n, k):
    print(f"misaligned fp8/fp4 {m}x{n}x{k}", flush=True)
    a, w = _bf16((m, k), 1), _bf16((n, k), 2, 0.05)
    qa, sa = Q.quant_fp8_tensor(a)
    qw, sw = Q.quant_fp8_tensor(w)
    want = G.fp8_gemm_packed(qa, qw, sa, sw)
    got = G.fp8_gemm_packed(_offset_view(qa, 3), _offset_view(qw, 5), sa, sw)
    assert torch.equal(got, want)
    ba, bsa = Q.quant_fp8_blocks(a, 1, 128)
    bw, bsw = Q.quant_fp8_blocks(w, 128, 128)
    want = G.fp8_gemm_packed(ba, bw, bsa, bsw, block=True)
    got = G.fp8_gemm_packed(_offset_view(ba, 7), bw, bsa, bsw, block=True)
    assert torch.equal(got, want)
    fa, ea = Q.quant_mxfp4(a)
    fw, ew = Q.quant_mxfp4(w)
    want = G.fp4_gemm_packed(fa, ea, fw, ew, fmt="mxfp4")
    got = G.fp4_gemm_packed(_offset_view(fa, 1), _offset_view(ea, 3), _offset_view(fw, 9),
                            _offset_view(ew, 1), fmt="mxfp4")
    assert torch.equal(got, want)


@pytest.mark.parametrize("m,n,k", [(1, 512, 1024), (700, 300, 256)])
def test_bf16_operands_at_odd_offsets(m, n, k):
    print(f"misaligned bf16 {m}x{n}x{k}", flush=True)
    a, w = _bf16((m, k), 3), _bf16((n, k), 4, 0.05)
    want = G.bf16_gemm(a, w.t())
    got = G.bf16_gemm(_offset_view(a, 1), _offset_view(w, 3).t())
    assert torch.equal(got, want)


def test_grouped_and_routed_operands_at_odd_offsets():
    print("misaligned grouped / MoE", flush=True)
    T, k, E, K, Nn = 257, 2, 8, 512, 384
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, E, (T, k), generator=g, dtype=torch.int32).to(DEV)
    x = _bf16((T, K), 6)
    w = _bf16((E * Nn, K), 7, 0.05)
    route = M.moe_route(ids, E)
    qx, sx = M.moe_permute_quant(x, route)
    qx2, sx2 = M.moe_permute_quant(_offset_view(x, 3), route)
    assert torch.equal(qx, qx2) and torch.equal(sx, sx2)
    qx2, sx2 = M.moe_permute_quant(_padded_rows(x, 3), route)
    assert torch.equal(qx, qx2) and torch.equal(sx, sx2)
    qw, sw = Q.quant_fp8_blocks(w, 1, K)
    qw, sw = qw.reshape(E, Nn, K), sw.reshape(E, Nn)
    want = G.grouped_fp8_gemm_packed(qx, sx, qw, sw, route.offsets)
    got = G.grouped_fp8_gemm_packed(_offset_view(qx, 5), sx, _offset_view(qw, 11), sw,
                                    route.offsets)
    assert torch.equal(got, want)
    tq, ts = M.moe_quant_tokens(x, route)
    tq2, ts2 = M.moe_quant_tokens(_offset_view(x, 1), route)
    assert torch.equal(tq, tq2) and torch.equal(ts, ts2)
    want = M.moe_grouped_fp8_gemm(tq, ts, route, qw, sw)
    got = M.moe_grouped_fp8_gemm(_offset_view(tq, 3), ts, route, _offset_view(qw, 1), sw)
    assert torch.equal(got, want)
    r1, q1, s1 = M.moe_route_quant_tokens(ids[:64], x[:64], E)
    r2, q2, s2 = M.moe_route_quant_tokens(ids[:64], _padded_rows(x[:64], 5), E)
    assert torch.equal(q1, q2) and torch.equal(s1, s2) and torch.equal(r1.dest, r2.dest)


def test_fused_producers_and_lora_at_odd_offsets():
    print("misaligned fused producers / LoRA", flush=True)
    rows, cols = 33, 1024
    x = _bf16((rows, cols), 8)
    wt = _bf16((cols,), 9)
    for fmt in ("fp8", "mxfp4"):
        want = F.rmsnorm_quant(x, wt, fmt=fmt)
        for v in (_offset_view(x, 3), _padded_rows(x, 3)):
            got = F.rmsnorm_quant(v, wt, fmt=fmt)
            assert all(torch.equal(p, q) for p, q in zip(got, want))
        gu = _bf16((rows, 2 * cols), 10)
        want = F.swiglu_quant(gu, fmt=fmt)
        for v in (_offset_view(gu, 1), _padded_rows(gu, 5)):
            got = F.swiglu_quant(v, fmt=fmt)
            assert all(torch.equal(p, q) for p, q in zip(got, want))
    M_, K, Nn, L, R = 40, 512, 256, 2, 16
    X, Wt = _bf16((M_, K), 11), _bf16((Nn, K), 12, 0.05)
    A, B = _bf16((L, K, R), 13, 0.05), _bf16((L, R, Nn), 14, 0.05)
    want = G.lora_fused_gemm(X, Wt.t(), A, B, [0.5, 2.0])
    got = G.lora_fused_gemm(_offset_view(X, 1), _offset_view(Wt, 3).t(), _offset_view(A, 5),
                            _offset_view(B, 7), [0.5, 2.0])
    assert torch.equal(got, want)
