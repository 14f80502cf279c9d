"""Helpers shared by the tests (not part of the product)."""
import numpy as np
import torch

from oracle import gemm as OG

# Output tolerance against the dequantize -> fp32 matmul -> bf16 oracle.
# TOL is the north-star bound on max|C-R| / max|R|.  ELEM_TOL bounds the
# elementwise relative error on entries with |R| >= 0.1 rms(R) at the same
# 1e-2: the two sides rounded to bf16 may sit one bf16 ulp apart (2^-7, 0.78%)
# where a value lies near a rounding boundary, and the gfx950
# FP8 MFMA sums the products of one instruction after aligning them to the
# largest (measured: error <= 1e-4 of max|C| for codes spanning the whole
# E4M3 range, exact for narrow ranges;
# tests/test_gpu_gemm.py::test_fp8_mfma_accumulation_bound).
TOL = 1e-2
ELEM_TOL = 1e-2

# (what, max-rel, elementwise) of every assert_close in this session; the
# terminal summary (tests/conftest.py) prints the largest measured errors.
MEASURED: list = []


def np_u8(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def np_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().float().numpy()


def f32_of_bf16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().float().numpy()


def assert_close(c: torch.Tensor, ref: np.ndarray, tol: float = TOL, what: str = "",
                 elem_tol: float | None = ELEM_TOL):
    elem_tol = ELEM_TOL if elem_tol is None else elem_tol
    got = np_f32(c)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    glob, elem = OG.rel_errors(got, ref)
    MEASURED.append((what, glob, elem))
    if not (glob <= tol and elem <= elem_tol):
        err = np.abs(got.astype(np.float64) - ref)
        r, c = np.unravel_index(int(err.argmax()), err.shape)
        bad = err > tol * np.abs(ref).max()
        rows, cols = np.nonzero(bad)
        where = (f"worst at [{r}, {c}] got {got[r, c]:.6g} want {ref[r, c]:.6g}; "
                 f"{int(bad.sum())} entries over the global bound"
                 + (f", rows {rows.min()}..{rows.max()}, cols {cols.min()}..{cols.max()}"
                    if bad.any() else ""))
        raise AssertionError(f"{what}: max-rel {glob:.3e} (bound {tol}), elementwise {elem:.3e} "
                             f"(bound {elem_tol}); {where}")
    return glob, elem
