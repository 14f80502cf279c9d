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


# ------------------------------------------------------------------------
# Block-scaled FP8 with 50x activation outliers.  The FP8 MFMA aligns the
# addends of one instruction to the largest before summing, so its error is
# relative to its largest addend: pinned per element by
# test_fp8_mfma_accumulation_bound as at most MFMA_STEP_REL times the largest
# product per 64 K of the sum (measured 5.9e-4 for K = 128, 6.8e-4 for
# K = 512 and 1.2e-3 for K = 4096: the per-step errors largely cancel, so
# the linear bound is loose).  In a block-scaled kernel the largest addend of
# a step is a product of group g's codes, at most 448 sa[m,g] x 448
# sb[n/128,g] in output units (the group's amax codes), and, where the
# accumulator is kept in units of the current group's scale and fed back
# into the MFMA (persistent and per-tile prefetch pipelined kernels,
#     acc_g = acc_{g-1} * (s_{g-1} / s_g) + sum of group g's products,
#     C = acc_G * s_G;
# the ratio multiplies add ~2^-22 relative per group, negligible), the
# running sum itself.  With P the largest of those, the partial sums over
# groups 1..g and the group terms of an entry,
#     |C - R| <= 2^-7 |R|  (bf16 rounding of C and of R, 2^-8 each)
#                + (K / 64) * MFMA_STEP_REL * P.
# An entry whose terms cancel to a small value after a large outlier term
# can exceed the plain 1e-2 elementwise bound within this one.
MFMA_STEP_REL = 5e-4


def block_fp8_error_bound(qa, sa, qw, sw) -> np.ndarray:
    """(K/64) * MFMA_STEP_REL * P per output entry, P from the oracle's
    float64 group terms s_a[m,g] s_b[n/128,g] sum_{k in g} a w, their
    running sums and the groups' largest products (1x128 activation groups,
    128x128 weight blocks; cuda/gemm/fp8_gemm.cu:84-97)."""
    from oracle import formats as OF

    da = OF.e4m3_decode(qa).astype(np.float64)
    dw = OF.e4m3_decode(qw).astype(np.float64)
    K = da.shape[1]
    G = -(-K // 128)
    sa = np.asarray(sa, np.float64)
    sw = np.asarray(sw, np.float64)
    colblk = np.arange(dw.shape[0]) // 128
    S = np.zeros((da.shape[0], dw.shape[0]))
    P = np.zeros_like(S)
    for g in range(G):
        k0, k1 = 128 * g, min(K, 128 * g + 128)
        sag, sbg = sa[:, g:g + 1], sw[colblk, g][None, :]
        term = (da[:, k0:k1] @ dw[:, k0:k1].T) * sag * sbg
        np.maximum(P, np.abs(term), out=P)
        np.maximum(P, (448.0 * sag) * (448.0 * sbg), out=P)   # the group's largest product
        S += term
        np.maximum(P, np.abs(S), out=P)
        del term
    return (-(-K // 64)) * MFMA_STEP_REL * P


def assert_close_block_bound(c: torch.Tensor, ref: np.ndarray, bound: np.ndarray,
                             what: str = ""):
    """The north-star max-relative bound, and per entry with |R| >= 0.1
    rms(R) the elementwise 1e-2 bound or the derived bound above (whichever
    is larger)."""
    got = np_f32(c)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    glob, elem = OG.rel_errors(got, ref)
    r = ref.astype(np.float64)
    err = np.abs(got.astype(np.float64) - r)
    big = np.abs(r) >= 0.1 * np.sqrt(np.mean(r * r))
    allowed = np.maximum(ELEM_TOL * np.abs(r), 2.0 ** -7 * np.abs(r) + bound)
    over = big & (err > allowed)
    used = big & (err > ELEM_TOL * np.abs(r))       # entries that needed the derived bound
    worst = float((err[used] / allowed[used]).max()) if used.any() else 0.0
    MEASURED.append((what + f" [{int(used.sum())} entries within the derived bound, "
                            f"worst {worst:.2f} of it]", glob, elem))
    if glob > TOL or over.any():
        i = np.unravel_index(int(np.argmax(np.where(big, err / allowed, 0))), err.shape)
        raise AssertionError(
            f"{what}: max-rel {glob:.3e} (bound {TOL}); {int(over.sum())} entries over the "
            f"derived elementwise bound, worst at {i}: got {got[i]:.6g} want {ref[i]:.6g} "
            f"allowed {allowed[i]:.3g}")
    return glob, elem
