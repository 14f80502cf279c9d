"""Quantize/pack outputs at the benchmark configurations' full sizes, byte for
byte against the oracle (codes and scales), for every operand of every
BASELINE configuration:

- config 1: A [128, 4096] and W [4096, 4096], per-tensor E4M3
  (quantize_to_fp8_kernel, cuda/gemm/fp8_gemm.cu:118-144);
- config 2: A [4096, 4096] (and the decode A [16, 4096]) in 1x128 groups with
  0.1% x50 outliers, W [7168, 4096] in 128x128 blocks (the scale layout of
  fp8_gemm_groupwise_kernel, cuda/gemm/fp8_gemm.cu:67-99);
- config 3: A and W [8192, 8192] MXFP4;
- config 4: W [14336, 4096] and A [2048, 4096] NVFP4, whose global scale
  comes from a two-pass amax over the whole tensor;
- config 5: X [32768, 2048] per row and W [64 * 1536, 2048] per channel.

The smaller parity tests check the same kernels on shapes the oracle handles
in milliseconds; these run the very launches the benchmark configurations
run (grid sizes, amax partial counts, packed-path chunk indices near 2^31
bytes), so an indexing slip that only shows at full size fails here.
"""
import numpy as np
import pytest
import torch

from dsl_tool_amd import quant as Q
from dsl_tool_amd import workloads as W
from oracle import quant as OQ
from tests.util import np_f32, np_u8

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _same(got: torch.Tensor, want: np.ndarray, what: str):
    g = np_u8(got) if want.dtype == np.uint8 else np_f32(got)
    assert g.shape == want.shape, (what, g.shape, want.shape)
    if not np.array_equal(g.view(np.uint8), want.view(np.uint8)):
        bad = np.argwhere(g.view(np.uint8).reshape(g.shape[0], -1)
                          != want.view(np.uint8).reshape(want.shape[0], -1))
        raise AssertionError(f"{what}: {len(bad)} bytes differ, first at {bad[0].tolist()}")


def _fp8_tensor(x: torch.Tensor, what: str):
    q, s = Q.quant_fp8_tensor(x.to(DEV))
    q_ref, s_ref = OQ.quant_fp8_per_tensor(x.float().numpy())
    assert np_f32(s)[0] == s_ref, f"{what}: scale {np_f32(s)[0]!r} != {s_ref!r}"
    _same(q, q_ref, f"{what} codes")


def _fp8_blocks(x: torch.Tensor, gr: int, gc: int, what: str):
    q, s = Q.quant_fp8_blocks(x.to(DEV), gr, gc)
    q_ref, s_ref = OQ.quant_fp8_blockwise(x.float().numpy(), gr, gc)
    _same(s, s_ref, f"{what} scales")
    _same(q, q_ref, f"{what} codes")


def test_config1_per_tensor():
    _fp8_tensor(W.activations(1, 128, 4096), "config 1 A [128, 4096]")
    _fp8_tensor(W.weights(1, 4096, 4096), "config 1 W [4096, 4096]")


def test_config2_groupwise():
    _fp8_blocks(W.activations(2, 4096, 4096, outliers=True), 1, 128, "config 2 A [4096, 4096] 1x128")
    _fp8_blocks(W.activations(2, 16, 4096, outliers=True), 1, 128, "config 2 A [16, 4096] 1x128")
    _fp8_blocks(W.weights(2, 7168, 4096), 128, 128, "config 2 W [7168, 4096] 128x128")


@pytest.mark.parametrize("operand", ["A", "W"])
def test_config3_mxfp4(operand):
    x = W.activations(3, 8192, 8192) if operand == "A" else W.weights(3, 8192, 8192)
    q, e = Q.quant_mxfp4(x.to(DEV))
    q_ref, e_ref = OQ.quant_mxfp4(x.float().numpy())
    _same(e, e_ref, f"config 3 {operand} E8M0")
    _same(q, q_ref, f"config 3 {operand} E2M1")


@pytest.mark.parametrize("operand", ["A", "W"])
def test_config4_nvfp4(operand):
    x = W.activations(4, 2048, 4096) if operand == "A" else W.weights(4, 14336, 4096)
    q, sb, sg = Q.quant_nvfp4(x.to(DEV))
    q_ref, sb_ref, sg_ref = OQ.quant_nvfp4(x.float().numpy())
    assert np_f32(sg)[0] == sg_ref, f"config 4 {operand}: global scale differs"
    _same(sb, sb_ref, f"config 4 {operand} E4M3 block scales")
    _same(q, q_ref, f"config 4 {operand} E2M1")


def test_config5_per_row_and_channel():
    x, w, _, _ = W.moe_problem(5)
    e, n, k = w.shape
    _fp8_blocks(x, 1, k, f"config 5 X [{x.shape[0]}, {k}] per row")
    _fp8_blocks(w.reshape(e * n, k), 1, k, f"config 5 W [{e * n}, {k}] per channel")
