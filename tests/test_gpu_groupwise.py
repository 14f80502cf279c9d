"""GPU: FP8 GEMM with the reference's own groupwise scale layout
(cuda/gemm/fp8_gemm.cu:67-99): sa [M, ceil(K/G)] per activation row and
K group, sb [ceil(K/G), N] per K group and output column,
C = sum_g (sum_{k in g} a*b) * sa[m, g] * sb[g, n].

The operands are quantized on the GPU (1 x G groups along K, the weight
per output column) and checked byte for byte against the oracle quantizer;
the GEMM output is then held to the dequantize -> matmul oracle
(oracle.gemm.ref_fp8_groupwise_cols) on the same codes.  Shapes are chosen
to take every kernel that serves the mode: the decode kernel (9 <= M <= 16
where its 32-row grid fills the CUs), the streaming kernel (M <= 1024 while
ceil(M/64) N stays small, the other skinny sizes), the pipelined
128x128 and 256x256 per-stage partial kernels, and the register-staged tiles
(K % 128 != 0, with and without split-K).  Every kernel here starts each
group's MFMA sum from zero, so the elementwise bound is the plain 1e-2.
"""
import numpy as np
import pytest
import torch

from dsl_tool_amd import gemm as G
from dsl_tool_amd import quant as Q
from dsl_tool_amd import workloads as W
from oracle import gemm as OG
from oracle import quant as OQ
from tests.test_gpu_fullsize import _cols, _freivalds, _sample
from tests.util import assert_close, np_f32, np_u8

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _quant_cols(a, w, gsize):
    """A in 1 x G groups, W [N, K] in 1 x G groups per row (= per output
    column of B = W^T), on the GPU; codes and scales checked against the
    oracle.  Returns device codes, sa [M, ceil(K/G)], sb [ceil(K/G), N]."""
    qa, sa = Q.quant_fp8_blocks(a.to(DEV), 1, gsize)
    qw, swr = Q.quant_fp8_blocks(w.to(DEV), 1, gsize)
    qa_r, sa_r = OQ.quant_fp8_blockwise(a.float().numpy(), 1, gsize)
    qw_r, sw_r = OQ.quant_fp8_blockwise(w.float().numpy(), 1, gsize)
    assert np.array_equal(np_u8(qa), qa_r) and np.array_equal(np_f32(sa), sa_r)
    assert np.array_equal(np_u8(qw), qw_r) and np.array_equal(np_f32(swr), sw_r)
    return qa, qw, sa, swr.t().contiguous()


# (m, n, k): kernel the default route takes
GROUP_SHAPES = [
    (16, 7168, 4096),     # decode kernel, config 2's decode shape
    (1, 1000, 2048),      # streaming, one row, ragged N
    (128, 4096, 4096),    # streaming, 64-row blocks
    (33, 4100, 1536),     # streaming, ragged N (column scales clamped at the edge)
    (1500, 1000, 1024),   # pipelined 128x128 per-stage partials
    (2048, 2048, 1024),   # pipelined 256x256 per-stage partials
    (5, 200, 272),        # register-staged tiles, partial last group
    (70, 300, 1040),      # register-staged tiles with split-K, partial last group
    (300, 384, 400),      # register-staged tiles
]


@pytest.mark.parametrize("m,n,k", GROUP_SHAPES)
def test_fp8_groupwise_cols(m, n, k):
    a = W.activations(2, m, k, outliers=True)
    w = W.randn_bf16((n, k), 2202, 0.02)
    qa, qw, sa, sb = _quant_cols(a, w, 128)
    c = G.fp8_gemm_packed(qa, qw, sa, sb, group=True)
    ref = OG.ref_fp8_groupwise_cols(np_u8(qa), np_f32(sa), np_u8(qw), np_f32(sb), 128)
    assert_close(c, ref, what=f"fp8 groupwise cols {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(16, 7168, 4096), (1500, 1000, 1024), (70, 300, 1040)])
def test_fp8_groupwise_cols_fp32_out(m, n, k):
    a = W.activations(2, m, k, outliers=True)
    w = W.randn_bf16((n, k), 2203, 0.02)
    qa, qw, sa, sb = _quant_cols(a, w, 128)
    c = G.fp8_gemm_packed(qa, qw, sa, sb, group=True, out_dtype=torch.float32)
    assert c.dtype == torch.float32
    ref = OG._mm(OG.dequant_fp8_blocks(np_u8(qa), np_f32(sa), 1, 128),
                 OG.dequant_fp8_blocks(np_u8(qw), np_f32(sb).T, 1, 128))
    assert_close(c, ref, what=f"fp8 groupwise cols fp32 {m}x{n}x{k}")


def test_fp8_groupwise_cols_distinct_column_scales_matter():
    """Columns of one 128-column block with very different weight scales:
    a kernel that read one scale per 128 columns (the block layout) would be
    off by the ratio on all but one column."""
    m, n, k = 48, 256, 1024
    a = W.randn_bf16((m, k), 2204)
    w = W.randn_bf16((n, k), 2205, 0.02)
    w = (w.float() * torch.logspace(-3, 3, n).reshape(n, 1)).bfloat16()
    qa, qw, sa, sb = _quant_cols(a, w, 128)
    assert float(np_f32(sb).max() / np_f32(sb).min()) > 1e4
    c = G.fp8_gemm_packed(qa, qw, sa, sb, group=True, out_dtype=torch.float32)
    ref = OG._mm(OG.dequant_fp8_blocks(np_u8(qa), np_f32(sa), 1, 128),
                 OG.dequant_fp8_blocks(np_u8(qw), np_f32(sb).T, 1, 128))
    # columnwise: each column against its own magnitude
    got = np_f32(c)
    err = np.abs(got - ref).max(axis=0) / np.abs(ref).max(axis=0)
    assert err.max() < 1e-2, err.max()


@pytest.mark.parametrize("gsize", [128, 256, 512])
def test_fp8_groupwise_registered_callable(gsize):
    """gemm.fp8_gemm(A, B, granularity='group', group_size=G) from bf16
    inputs, and from pre-quantized float8 codes with the reference's scale
    layout (scale tensors positional, as run_from_spec passes them)."""
    m, n, k = 96, 640, 1408            # K = 11 x 128: the last G group is partial for G > 128
    a = W.activations(2, m, k, outliers=True)
    w = W.randn_bf16((n, k), 2206, 0.02)
    c = G.fp8_gemm(a.to(DEV), w.to(DEV).t(), granularity="group", group_size=gsize)
    qa, sa = OQ.quant_fp8_blockwise(a.float().numpy(), 1, gsize)
    qw, swr = OQ.quant_fp8_blockwise(w.float().numpy(), 1, gsize)
    ref = OG.ref_fp8_groupwise_cols(qa, sa, qw, swr.T, gsize)
    assert_close(c, ref, what=f"fp8_gemm group G={gsize}")
    A8 = torch.from_numpy(qa).view(torch.float8_e4m3fn).to(DEV)
    B8 = torch.from_numpy(qw).view(torch.float8_e4m3fn).to(DEV).t()      # [K, N] view
    sa_t, sb_t = torch.from_numpy(sa).to(DEV), torch.from_numpy(np.ascontiguousarray(swr.T)).to(DEV)
    c2 = G.fp8_gemm(A8, B8, sa_t, sb_t, group_size=gsize)                # layout inferred
    assert torch.equal(c2, c)
    c3 = G.fp8_gemm(A8, B8, sa_t, sb_t, granularity="group", group_size=gsize,
                    out_dtype="float32")
    assert c3.dtype == torch.float32
    assert_close(c3, ref, what=f"fp8_gemm group G={gsize} fp32 out")


def test_fp8_groupwise_rejects_bad_group_size():
    a = torch.zeros((4, 256), dtype=torch.bfloat16, device=DEV)
    w = torch.zeros((256, 8), dtype=torch.bfloat16, device=DEV)
    for bad in (64, 100, 0, 192):
        with pytest.raises(ValueError, match="multiple of 128"):
            G.fp8_gemm(a, w, granularity="group", group_size=bad)


@pytest.mark.parametrize("m", [16, 4096])
def test_fp8_groupwise_config2_shapes(m):
    """BASELINE config 2's shapes (N=7168, K=4096, 0.1% x50 activation
    outliers) with per-column weight scales: sampled entries against the
    oracle and every entry by Freivalds' check (M=4096), or the whole output
    (M=16)."""
    n, k = 7168, 4096
    a = W.activations(2, m, k, outliers=True)
    w = W.weights(2, n, k)
    qa, qw, sa, sb = _quant_cols(a, w, 128)
    c = G.fp8_gemm_packed(qa, qw, sa, sb, group=True)
    qa_h, qw_h, sa_h, sb_h = np_u8(qa), np_u8(qw), np_f32(sa), np_f32(sb)
    if m == 16:
        ref = OG.ref_fp8_groupwise_cols(qa_h, sa_h, qw_h, sb_h, 128)
        assert_close(c, ref, what="fp8 groupwise cols config 2 M=16")
        return
    rows, blks = _sample(m, n, 2207)
    cols = _cols(blks, n)
    ref = OG.ref_fp8_groupwise_cols(qa_h[rows], sa_h[rows], qw_h[cols], sb_h[:, cols], 128)
    assert_close(c[torch.from_numpy(rows).to(DEV)][:, torch.from_numpy(cols).to(DEV)], ref,
                 what="fp8 groupwise cols config 2 M=4096 sampled")
    _freivalds(c, OG.dequant_fp8_blocks(qa_h, sa_h, 1, 128),
               OG.dequant_fp8_blocks(qw_h, sb_h.T, 1, 128), 2208, "fp8 groupwise cols config 2")
