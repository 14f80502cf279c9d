"""The 128x128 pipelined tiles (one round of tiles: more rows than the
streaming kernel takes, too few 256x256 tiles for the persistent kernel),
every mode, bf16 and fp32 output, against the dequantize -> fp32 matmul
oracle on the same codes.

These tiles hold the output with the W fragment in the MFMA's first operand
slot and stage it through LDS in packed 8-byte (bf16) or 16-byte (fp32)
writes; M = 1100 and N = 3000 leave ragged edge tiles in both dimensions, and
1024 x 4096 is whole tiles.  Block-scaled FP8 takes the per-stage partial
kernel there (a fresh 128-K partial per group, folded with sa * sb).
"""
import pytest
import torch

from oracle import formats as OF
from oracle import gemm as OG
from dsl_tool_amd import gemm as G
from dsl_tool_amd import quant as Q
from dsl_tool_amd import workloads as W
from tests.util import assert_close, assert_close_block_bound, block_fp8_error_bound, np_f32, np_u8

pytestmark = pytest.mark.gpu
DEV = "cuda"

SHAPES = [(1100, 3000, 1024), (1024, 4096, 512)]


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("mode", ["tensor", "block", "mxfp4", "nvfp4", "bf16"])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_pipelined_128_tiles(m, n, k, mode, out_dtype):
    a = W.activations(3, m, k, outliers=True) if mode == "block" else W.randn_bf16((m, k), 951)
    w = W.randn_bf16((n, k), 952, 0.02)
    what = f"128x128 pipelined {mode} {m}x{n}x{k} {out_dtype}"
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
    assert c.dtype == out_dtype
    assert_close(c, ref, what=what)


# The shortest K each mode's tiles take: two 64-byte stages (the prefetch
# schedule's least, and an even count), or one 128-byte stage for block
# scales.
MIN_K = {"tensor": 128, "block": 128, "mxfp4": 256, "nvfp4": 256, "bf16": 64}


@pytest.mark.parametrize("mode", sorted(MIN_K))
def test_pipelined_128_tiles_shortest_k(mode):
    test_pipelined_128_tiles(1100, 3000, MIN_K[mode], mode, torch.bfloat16)


def test_pipelined_128_tiles_bf16_repeatable():
    # the packed staging writes leave no lane-order dependence: two runs give
    # the same bytes
    a = W.randn_bf16((1100, 1024), 953).to(DEV)
    w = W.randn_bf16((3000, 1024), 954, 0.02).to(DEV)
    c1 = G.bf16_gemm(a, w.t(), out_dtype=torch.float32)
    c2 = G.bf16_gemm(a, w.t(), out_dtype=torch.float32)
    assert torch.equal(c1, c2)
