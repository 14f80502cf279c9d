"""Grouped FP8 GEMM with group-offset tables outside the contract.

Every grouped kernel clamps the device offset table into [0, rows] and
makes each group's end no smaller than its start, so a malformed table can
never address outside X or Y.  These tables hold negative entries, entries
past the row count, a first offset above 0 and a last one below the row
count, without groups overlapping after the clamp.  The rows a clamped group
covers must match the oracle on the clamped table, and the rows no group
covers must keep the caller's sentinel.  One case per grouped kernel: the
persistent walk (K % 128 == 0, 48 or more rows per group on average), the
streaming tiles (fewer rows per group, K % 256 == 0), the pipelined grouped
tiles (K % 128 != 0) and the register-staged grouped kernel (K % 64 != 0).
"""
import numpy as np
import pytest
import torch

from oracle import gemm as OG
from oracle import quant as OQ
from dsl_tool_amd import gemm as G
from dsl_tool_amd import quant as Q
from dsl_tool_amd import workloads as W
from tests.util import assert_close, np_u8

pytestmark = pytest.mark.gpu
DEV = "cuda"

# name: (rows, N, K, offsets as passed)
CASES = {
    "persistent": (300, 384, 512, [16, 40, 40, 260, 1000]),
    "stream": (100, 384, 512, [-3, 10, 10, 40, 75, 5000, 5000, 5000, 5000]),
    "pipelined": (300, 384, 192, [-1, 100, 100, 250, 301]),
    "register_staged": (200, 256, 80, [0, 60, 60, 150, 150]),
}


def _clamped(offsets, rows):
    c = np.clip(np.asarray(offsets, np.int64), 0, rows)
    out = c.copy()
    for g in range(len(c) - 1):
        out[g + 1] = max(c[g + 1], c[g])      # a group's end never below its start
    return c, out


@pytest.mark.parametrize("name", sorted(CASES))
def test_malformed_offsets_are_clamped(name):
    T, n, k, offs = CASES[name]
    Gn = len(offs) - 1
    x = W.randn_bf16((T, k), 611)
    w = W.randn_bf16((Gn, n, k), 612, 0.02)
    qx, sx = Q.quant_fp8_blocks(x.to(DEV), 1, k)
    qw, sw = Q.quant_fp8_blocks(w.reshape(Gn * n, k).to(DEV), 1, k)
    off_d = torch.tensor(offs, dtype=torch.int32, device=DEV)
    y = torch.full((T, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    print(f"grouped malformed table {name}: rows {T} N {n} K {k} offsets {offs}", flush=True)
    G.grouped_fp8_gemm_packed(qx, sx, qw.reshape(Gn, n, k), sw.reshape(Gn, n), off_d, out=y)
    torch.cuda.synchronize()
    starts, ends = _clamped(offs, T)
    assert np.all(np.diff(starts) >= 0), "test tables are non-decreasing once clamped"
    covered = np.zeros(T, bool)
    for g in range(Gn):
        assert not covered[starts[g]:ends[g + 1]].any(), "test tables must not overlap"
        covered[starts[g]:ends[g + 1]] = True
    qx_h, sx_h = OQ.quant_fp8_blockwise(x.float().numpy(), 1, k)
    qw_h, sw_h = OQ.quant_fp8_blockwise(w.reshape(Gn * n, k).float().numpy(), 1, k)
    assert np.array_equal(np_u8(qx), qx_h) and np.array_equal(np_u8(qw), qw_h)
    # the oracle on a non-decreasing table with the same group row ranges
    table = np.concatenate([[starts[0]], ends[1:]]).astype(np.int64)
    ref = OG.ref_grouped_fp8(qx_h, sx_h[:, 0], qw_h.reshape(Gn, n, k), sw_h.reshape(Gn, n), table)
    yc = y.float().cpu().numpy()
    rows = np.nonzero(covered)[0]
    assert_close(torch.from_numpy(yc[rows]), ref[rows], what=f"grouped malformed {name}")
    assert np.isnan(yc[~covered]).all(), f"{name}: rows outside every group were written"
