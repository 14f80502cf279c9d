"""Helpers shared by the tests (not part of the product)."""
import numpy as np
import torch

from oracle import gemm as OG

TOL = 1e-2   # max|C-R|/max|R| and elementwise rel. on |R| >= 0.1 rms(R)


def np_u8(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def np_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().float().numpy()


def f32_of_bf16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().float().numpy()


def assert_close(c: torch.Tensor, ref: np.ndarray, tol: float = TOL, what: str = ""):
    got = np_f32(c)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    glob, elem = OG.rel_errors(got, ref)
    assert glob <= tol and elem <= tol, f"{what}: max-rel {glob:.3e}, elementwise {elem:.3e} > {tol}"
    return glob, elem
