"""CPU: the oracle against the golden fixtures (tests/golden/, written by
independent scalar code and torch casts) and against closed forms.

Each check is chosen so that a plausible slip in the oracle (a tie rule, an
off-by-one exponent, a swapped operand, a dropped scale) fails it; the
``test_*_discriminates`` cases plant such slips in copies of the oracle
functions and assert the same fixture rejects them.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import gemm as OG
from oracle import quant as OQ

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
BITS = np.arange(65536, dtype=np.uint16)
VALS = F.bf16_bits_to_f32(BITS)
FINITE = np.isfinite(VALS)


def gold(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


@pytest.fixture(scope="module")
def kat():
    with np.load(os.path.join(GOLD, "kat_gemm.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bf16_from_bits(a):
    return F.bf16_bits_to_f32(np.asarray(a).view(np.uint16))


# ------------------------------------------------------------------ formats --
def test_e4m3_encode_matches_torch_cast_for_every_bf16():
    assert np.array_equal(F.e4m3_encode(VALS), gold("e4m3_bf16.npy"))


def test_e4m3_encode_matches_torch_on_dense_fp32_sweep():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-500, 500, 200_000),
                        rng.uniform(-2 ** -6, 2 ** -6, 100_000),
                        np.array([448, 464, 464.0001, 480, -464, 2 ** -10, 3 * 2 ** -10,
                                  1.0625, 1.1875, 0.0, -0.0])]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(F.e4m3_encode(x), want)


def test_e4m3_spec_special_values():
    # OCP FP8 E4M3FN: max 448 = S.1111.110, NaN = S.1111.111, min subnormal 2^-9
    assert F.e4m3_encode(np.float32([448.0, -448.0]))[0] == 0x7E
    assert F.e4m3_encode(np.float32([-448.0]))[0] == 0xFE
    assert F.e4m3_decode(np.uint8([0x7E]))[0] == 448.0
    assert F.e4m3_decode(np.uint8([0x01]))[0] == 2.0 ** -9
    assert np.isnan(F.e4m3_decode(np.uint8([0x7F, 0xFF]))).all()
    codes = np.arange(256, dtype=np.uint8)
    dec = F.e4m3_decode(codes)
    ok = ~np.isnan(dec)
    assert np.array_equal(F.e4m3_encode(dec[ok]), codes[ok])     # decode is an exact inverse


def test_e2m1_encode_matches_brute_force_for_every_bf16():
    want = gold("e2m1_bf16.npy")
    assert np.array_equal(F.e2m1_encode(VALS[FINITE]), want[FINITE])


def test_e2m1_decode_is_the_reference_table():
    # cuda/gemm/fp4_gemm.cu:30-33: {0,.5,1,1.5,2,3,4,6}, bit 3 = sign
    assert list(F.e2m1_decode(np.arange(8))) == [0, .5, 1, 1.5, 2, 3, 4, 6]
    assert list(F.e2m1_decode(np.arange(8, 16))) == [-0.0, -.5, -1, -1.5, -2, -3, -4, -6]
    assert np.array_equal(F.e2m1_encode(F.e2m1_decode(np.arange(16))), np.arange(16))


def test_e2m1_reference_tie_rule_differs_only_on_ties():
    v = VALS[FINITE & (np.abs(VALS) <= 6)]
    rne, ref = F.e2m1_encode(v), F.e2m1_encode_reference_ties(v)
    diff = F.e2m1_decode(rne) != F.e2m1_decode(ref)
    ties = np.isin(np.abs(v), [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])
    assert not (diff & ~ties).any()
    assert diff[ties].any()


def test_nibble_packing_low_nibble_is_even_index():
    # cuda/gemm/fp4_gemm.cu:45-47, :88: byte = (q1 << 4) | q0
    p = F.pack_nibbles(np.array([[1, 2, 15, 0]], np.uint8))
    assert p.tolist() == [[0x21, 0x0F]]
    assert np.array_equal(F.unpack_nibbles(p), [[1, 2, 15, 0]])


def test_e8m0_exponent_matches_frexp_for_every_positive_bf16():
    want = gold("e8m0_bf16.npy")
    sel = FINITE & (VALS >= 0)
    e = np.clip(F.floor_log2(VALS[sel]) - 2, -127, 127) + 127
    e = np.where(VALS[sel] == 0, 0, e)
    assert np.array_equal(e.astype(np.uint8), want[sel])


def test_e8m0_decode_matches_torch():
    codes = np.arange(255, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e8m0fnu).float().numpy()
    assert np.array_equal(F.e8m0_decode(codes), want)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(100_000) * 10.0 ** rng.integers(-30, 30, 100_000)).astype(np.float32)
    want = torch.from_numpy(x).bfloat16().float().numpy()
    assert np.array_equal(F.round_to_bf16(x), want)


# --------------------------------------------------------------- quantizers --
def test_fp8_tensor_kat(kat):
    q, s = OQ.quant_fp8_per_tensor(bf16_from_bits(kat["fp8t_a"]))
    assert s == kat["fp8t_sa"] and np.array_equal(q, kat["fp8t_qa"])
    q, s = OQ.quant_fp8_per_tensor(bf16_from_bits(kat["fp8t_w"]))
    assert s == kat["fp8t_sw"] and np.array_equal(q, kat["fp8t_qw"])


def test_fp8_block_kat(kat):
    q, s = OQ.quant_fp8_blockwise(bf16_from_bits(kat["fp8b_a"]), 1, 128)
    assert np.array_equal(s, kat["fp8b_sa"]) and np.array_equal(q, kat["fp8b_qa"])
    q, s = OQ.quant_fp8_blockwise(bf16_from_bits(kat["fp8b_w"]), 128, 128)
    assert np.array_equal(s, kat["fp8b_sw"]) and np.array_equal(q, kat["fp8b_qw"])


def test_mxfp4_kat(kat):
    q, e = OQ.quant_mxfp4(bf16_from_bits(kat["mx_a"]))
    assert np.array_equal(e, kat["mx_ea"]) and np.array_equal(q, kat["mx_qa"])
    q, e = OQ.quant_mxfp4(bf16_from_bits(kat["mx_w"]))
    assert np.array_equal(e, kat["mx_ew"]) and np.array_equal(q, kat["mx_qw"])


def test_nvfp4_kat(kat):
    q, sb, sg = OQ.quant_nvfp4(bf16_from_bits(kat["nv_a"]))
    assert sg == kat["nv_ga"] and np.array_equal(sb, kat["nv_sa"]) and np.array_equal(q, kat["nv_qa"])
    q, sb, sg = OQ.quant_nvfp4(bf16_from_bits(kat["nv_w"]))
    assert sg == kat["nv_gw"] and np.array_equal(sb, kat["nv_sw"]) and np.array_equal(q, kat["nv_qw"])


def test_fp8_amax_element_maps_to_448_and_zero_tensor_uses_floor():
    x = np.float32([[0.1, -3.0, 2.0], [1.5, 0.0, -0.25]])
    q, s = OQ.quant_fp8_per_tensor(x)
    assert s == np.float32(3.0) / np.float32(448.0)
    assert q[0, 1] == 0xFE                       # -amax -> -448
    q0, s0 = OQ.quant_fp8_per_tensor(np.zeros((2, 4), np.float32))
    assert s0 == np.float32(1e-12) and not q0.any()


def test_mxfp4_power_of_two_invariance():
    rng = np.random.default_rng(2)
    x = F.round_to_bf16(rng.standard_normal((4, 64)).astype(np.float32))
    q, e = OQ.quant_mxfp4(x)
    for k in (-40, -3, 5, 60):
        q2, e2 = OQ.quant_mxfp4((x * np.float32(2.0 ** k)).astype(np.float32))
        assert np.array_equal(q2, q) and np.array_equal(e2.astype(int), e.astype(int) + k)


def test_mxfp4_block_max_lands_in_top_binade():
    # amax in [2^(e+2), 2^(e+3)) -> amax * 2^-e in [4, 8) -> code 6 (4.0) or 7 (6.0)
    rng = np.random.default_rng(3)
    x = F.round_to_bf16(rng.standard_normal((8, 128)).astype(np.float32))
    q, _ = OQ.quant_mxfp4(x)
    codes = F.unpack_nibbles(q).reshape(8, 4, 32)
    arg = np.abs(x).reshape(8, 4, 32).argmax(-1)
    top = np.take_along_axis(codes & 7, arg[..., None], -1)
    assert np.isin(top, [6, 7]).all()


def test_nvfp4_block_holding_tensor_amax_gets_scale_448():
    rng = np.random.default_rng(4)
    x = F.round_to_bf16(rng.standard_normal((2, 32)).astype(np.float32))
    q, sb, sg = OQ.quant_nvfp4(x)
    r, c = np.unravel_index(np.abs(x).argmax(), x.shape)
    assert sb[r, c // 16] == 0x7E                 # e4m3(448)
    assert (F.unpack_nibbles(q)[r, c] & 7) == 7   # x / (448 * amax/2688) = +-6


# -------------------------------------------------------------------- GEMMs --
def test_ref_fp8_tensor_kat(kat):
    c = OG.ref_fp8_per_tensor(kat["fp8t_qa"], kat["fp8t_sa"], kat["fp8t_qw"], kat["fp8t_sw"],
                              f64=True)
    assert np.array_equal(c, F.round_to_bf16(kat["fp8t_c"].astype(np.float32)))


def test_ref_fp8_groupwise_kat(kat):
    c = OG.ref_fp8_groupwise(kat["fp8b_qa"], kat["fp8b_sa"], kat["fp8b_qw"], kat["fp8b_sw"],
                             f64=True)
    g, e = OG.rel_errors(c, kat["fp8b_c"])
    assert g < 4e-3 and e < 8e-3          # bf16 rounding of the output only


@pytest.mark.parametrize("G", [128, 256])
def test_fp8_groupwise_cols_kat(kat, G):
    """The reference's own groupwise layout (cuda/gemm/fp8_gemm.cu:67-99),
    K = 320 so the last group is partial: the 1 x G quantizer gives the
    fixture's codes and scales (the weight's per-row scales are sb
    transposed), and the dequantize -> matmul oracle equals the float64
    group-partial triple loop of that kernel."""
    a, w = bf16_from_bits(kat["fp8g_a"]), bf16_from_bits(kat["fp8g_w"])
    qa, sa = OQ.quant_fp8_blockwise(a, 1, G)
    qw, sw = OQ.quant_fp8_blockwise(w, 1, G)
    assert np.array_equal(qa, kat[f"fp8g{G}_qa"]) and np.array_equal(sa, kat[f"fp8g{G}_sa"])
    assert np.array_equal(qw, kat[f"fp8g{G}_qw"]) and np.array_equal(sw.T, kat[f"fp8g{G}_sb"])
    c = OG.ref_fp8_groupwise_cols(kat[f"fp8g{G}_qa"], kat[f"fp8g{G}_sa"], kat[f"fp8g{G}_qw"],
                                  kat[f"fp8g{G}_sb"], G, f64=True)
    assert np.array_equal(c, F.round_to_bf16(kat[f"fp8g{G}_c"].astype(np.float32)))


def test_fp8_groupwise_cols_kat_discriminates_slips(kat):
    """Plausible slips in the groupwise oracle fail the fixture: the column
    scales read as 128-column blocks (the block layout), scales transposed
    onto the wrong axis, the partial last group dropped, and G = 256 scales
    applied per 128."""
    qa, sa, qw, sb = (kat[f"fp8g256_{k}"] for k in ("qa", "sa", "qw", "sb"))
    want = kat["fp8g256_c"]

    def far(c):
        return OG.rel_errors(c, want)[0] > 1e-2

    da = OG.dequant_fp8_blocks(qa, sa, 1, 256)
    # one weight scale per 128-column block (column 0's), not per column
    blockish = OG.dequant_fp8_blocks(qw, np.repeat(sb.T[:1], qw.shape[0], axis=0), 1, 256)
    assert far(OG.ref_gemm_dequant(da, blockish, True))
    # sb indexed [n][g] read as [g][n] (same values, wrong axis): swap via reshape
    swapped = np.ascontiguousarray(sb).reshape(sb.shape[1], sb.shape[0])
    assert far(OG.ref_gemm_dequant(da, OG.dequant_fp8_blocks(qw, swapped, 1, 256), True))
    # partial last group (k = 256..319) dropped
    qa0 = qa.copy()
    qa0[:, 256:] = 0
    assert far(OG.ref_fp8_groupwise_cols(qa0, sa, qw, sb, 256, f64=True))
    # G = 256 scales expanded to 128-element groups: repeated twice each (what
    # the GPU path does) passes, read once per 128 (the last padded) fails
    sa2, sb2 = np.repeat(sa, 2, axis=1)[:, :3], np.repeat(sb, 2, axis=0)[:3]
    assert not far(OG.ref_fp8_groupwise_cols(qa, sa2, qw, sb2, 128, f64=True))
    sa1, sb1 = np.pad(sa, ((0, 0), (0, 1)), mode="edge"), np.pad(sb, ((0, 1), (0, 0)), mode="edge")
    assert far(OG.ref_fp8_groupwise_cols(qa, sa1, qw, sb1, 128, f64=True))


def test_ref_mxfp4_kat(kat):
    c = OG.ref_mxfp4(kat["mx_qa"], kat["mx_ea"], kat["mx_qw"], kat["mx_ew"], f64=True)
    want = kat["mx_c"]
    assert np.allclose(c, want, rtol=2 ** -8, atol=0)


def test_ref_nvfp4_kat(kat):
    c = OG.ref_nvfp4(kat["nv_qa"], kat["nv_sa"], kat["nv_ga"], kat["nv_qw"], kat["nv_sw"],
                     kat["nv_gw"], f64=True)
    assert np.allclose(c, kat["nv_c"], rtol=2 ** -8, atol=1e-30)


def test_ref_grouped_kat(kat):
    y = OG.ref_grouped_fp8(kat["grp_qx"], kat["grp_sx"], kat["grp_qw"], kat["grp_sw"],
                           kat["grp_off"], f64=True)
    assert np.allclose(y, kat["grp_y"], rtol=2 ** -8, atol=1e-30)


def test_tiled_grouped_reference_cpu_path(kat):
    """The grouped tiled restatement (64x64x32 tiles per group,
    tilelang/gemm/gemm_kernels.py:116-133) against the float64 triple-loop
    known answer, and against the dense grouped oracle on groups that span
    several 64-row tiles, a ragged N and an empty group; restricting it to
    some groups leaves the other rows at zero."""
    y = OG.tiled_grouped_fp8_gemm(kat["grp_qx"], kat["grp_sx"], kat["grp_qw"], kat["grp_sw"],
                                  kat["grp_off"])
    assert np.allclose(y, kat["grp_y"], rtol=2 ** -8, atol=1e-30)
    rng = np.random.default_rng(17)
    counts = [70, 0, 130, 5]
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    qx = F.e4m3_encode(rng.standard_normal((205, 96)).astype(np.float32))
    qw = F.e4m3_encode(rng.standard_normal((4, 72, 96)).astype(np.float32))
    sx = np.float32(rng.uniform(0.5, 2, 205))
    sw = np.float32(rng.uniform(0.5, 2, (4, 72)))
    tiled = OG.tiled_grouped_fp8_gemm(qx, sx, qw, sw, off)
    dense = np.concatenate([
        (F.e4m3_decode(qx[off[g]:off[g + 1]]).astype(np.float64)
         @ F.e4m3_decode(qw[g]).astype(np.float64).T) * sx[off[g]:off[g + 1], None] * sw[g][None, :]
        for g in range(4)])
    assert np.allclose(tiled, dense, rtol=1e-5, atol=1e-6)
    part = OG.tiled_grouped_fp8_gemm(qx, sx, qw, sw, off, groups=[2])
    assert np.array_equal(part[70:200], tiled[70:200]) and not part[:70].any() and not part[200:].any()


def test_groupwise_partial_form_equals_dequant_form():
    # sum_g sa[m,g] sb[n/128,g] sum_{k in g} a w  (cuda/gemm/fp8_gemm.cu:84-97)
    rng = np.random.default_rng(5)
    a = F.round_to_bf16(rng.standard_normal((3, 384)).astype(np.float32))
    w = F.round_to_bf16((rng.standard_normal((200, 384)) * 0.02).astype(np.float32))
    qa, sa = OQ.quant_fp8_blockwise(a, 1, 128)
    qw, sw = OQ.quant_fp8_blockwise(w, 128, 128)
    da, dw = F.e4m3_decode(qa).astype(np.float64), F.e4m3_decode(qw).astype(np.float64)
    part = np.zeros((3, 200))
    for g in range(3):
        blk = da[:, g * 128:(g + 1) * 128] @ dw[:, g * 128:(g + 1) * 128].T
        part += blk * sa[:, g:g + 1] * sw[np.arange(200) // 128, g][None, :]
    ref = OG.ref_fp8_groupwise(qa, sa, qw, sw, f64=True)
    g_, e_ = OG.rel_errors(ref, part)
    assert g_ < 4e-3 and e_ < 8e-3


def test_tiled_reference_cpu_path_matches_dense_oracle():
    rng = np.random.default_rng(6)
    a = F.round_to_bf16(rng.standard_normal((70, 100)).astype(np.float32))
    w = F.round_to_bf16((rng.standard_normal((90, 100)) * 0.02).astype(np.float32))
    qa, sa = OQ.quant_fp8_per_tensor(a)
    qw, sw = OQ.quant_fp8_per_tensor(w)
    tiled = OG.tiled_fp8_gemm(qa, qw, sa, sw)
    dense = OG._mm(F.e4m3_decode(qa), F.e4m3_decode(qw), f64=True) * float(sa) * float(sw)
    assert np.allclose(tiled, dense, rtol=1e-5, atol=1e-6)


def test_ref_bf16_matches_exact_rational_brute_force():
    # bf16 operands: every product is exact, so the exact sum (Fractions) rounded
    # once to fp32 is the answer; a transposed operand or a dropped K term fails.
    from fractions import Fraction
    rng = np.random.default_rng(8)
    a = F.round_to_bf16((rng.standard_normal((5, 24)) * 3).astype(np.float32))
    w = F.round_to_bf16(rng.standard_normal((7, 24)).astype(np.float32))
    got = OG.ref_bf16(a, w)
    want = np.empty((5, 7), np.float32)
    for i in range(5):
        for j in range(7):
            want[i, j] = np.float32(float(sum(Fraction(float(a[i, k])) * Fraction(float(w[j, k]))
                                              for k in range(24))))
    assert np.array_equal(got, want)
    assert not np.array_equal(OG.ref_bf16(a[:, :23], w[:, :23]), want)
    sq = F.round_to_bf16(rng.standard_normal((24, 24)).astype(np.float32))
    assert not np.allclose(OG.ref_bf16(sq, sq), OG.ref_bf16(sq, sq.T.copy()), rtol=1e-3)


def test_ref_lora_matches_elementwise_loops():
    rng = np.random.default_rng(14)
    M, N, K, R, L = 3, 4, 6, 2, 2
    x, w = rng.standard_normal((M, K)), rng.standard_normal((N, K))
    a, b = rng.standard_normal((L, K, R)), rng.standard_normal((L, R, N))
    s = [0.5, -2.0]
    y = OG.ref_lora(x, w, a, b, s)
    for i in range(M):
        for j in range(N):
            v = sum(x[i, k] * w[j, k] for k in range(K))
            for l in range(L):
                v += s[l] * sum(sum(x[i, k] * a[l, k, r] for k in range(K)) * b[l, r, j] for r in range(R))
            assert abs(y[i, j] - v) <= 1e-5 * (1 + abs(v))
    assert not np.allclose(OG.ref_lora(x, w, a, b, [0.5, 2.0]), y)        # a dropped sign fails


def test_tiled_bf16_reference_cpu_path_matches_dense_oracle():
    rng = np.random.default_rng(9)
    a = F.round_to_bf16(rng.standard_normal((150, 100)).astype(np.float32))
    w = F.round_to_bf16(rng.standard_normal((140, 100)).astype(np.float32))
    assert np.allclose(OG.tiled_bf16_gemm(a, w), OG.ref_bf16(a, w), rtol=1e-5, atol=1e-5)


def test_rmsnorm_oracle_against_float64_and_closed_form():
    from oracle import fused as OF
    rng = np.random.default_rng(10)
    x = F.round_to_bf16((rng.standard_normal((20, 384)) * 2).astype(np.float32))
    w = F.round_to_bf16((1 + 0.1 * rng.standard_normal(384)).astype(np.float32))
    y = OF.rmsnorm_bf16(x, w, 1e-6)
    x64 = x.astype(np.float64)
    y64 = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    d = np.abs(F.f32_to_bf16_bits(y).astype(np.int32) -
               F.f32_to_bf16_bits(y64.astype(np.float32)).astype(np.int32))
    assert d.max() <= 1 and (d > 0).mean() < 0.01
    # a constant row c normalises to sign(c) * w (up to eps)
    c = np.full((1, 64), -3.0, np.float32)
    assert np.array_equal(OF.rmsnorm_bf16(c, np.ones(64, np.float32), 0.0), -np.ones((1, 64), np.float32))
    # dropping the weight or squaring the wrong thing is caught by the fp64 check
    assert not np.allclose(OF.rmsnorm_bf16(x, np.ones(384, np.float32)), y64, rtol=1e-2)


def test_swiglu_oracle_against_float64_and_limits():
    from oracle import fused as OF
    rng = np.random.default_rng(11)
    x = F.round_to_bf16((rng.standard_normal((16, 256)) * 4).astype(np.float32))
    y = OF.swiglu_bf16(x)
    g, u = x[:, :128].astype(np.float64), x[:, 128:].astype(np.float64)
    y64 = g / (1 + np.exp(-g)) * u
    d = np.abs(F.f32_to_bf16_bits(y).astype(np.int32) -
               F.f32_to_bf16_bits(y64.astype(np.float32)).astype(np.int32))
    assert d.max() <= 1
    lim = np.array([[0.0, 30.0, -30.0, 1.0, 2.0, 2.0, 2.0, 0.5]], np.float32)
    out = OF.swiglu_bf16(lim)
    assert out[0, 0] == 0 and out[0, 1] == 60.0 and -1e-10 < out[0, 2] < 0   # silu(-30) = -30 e^-30
    # gate and up swapped is a different function
    assert not np.allclose(OF.swiglu_bf16(np.concatenate([x[:, 128:], x[:, :128]], 1)), y)


def test_moe_route_matches_brute_force_stable_sort():
    from oracle import moe as OM
    rng = np.random.default_rng(12)
    T, k, E = 23, 3, 5
    ids = rng.integers(-1, E + 1, (T, k)).astype(np.int32)      # includes dropped ids -1 and E
    offsets, dest, src = OM.route(ids, E)
    rows = []                                                    # brute force: expert by expert
    for e in range(E):
        for a in range(T * k):
            if ids.reshape(-1)[a] == e:
                rows.append(a)
    assert list(src) == [a // k for a in rows]
    for r, a in enumerate(rows):
        assert dest[a] == r
    assert (dest[~np.isin(ids.reshape(-1), range(E))] == -1).all()
    assert list(offsets) == [0] + list(np.cumsum([np.sum(ids == e) for e in range(E)]))


def test_moe_combine_closed_forms():
    from oracle import moe as OM
    rng = np.random.default_rng(13)
    y = F.round_to_bf16(rng.standard_normal((12, 16)).astype(np.float32))
    dest = np.array([3, 7, -1, 0, 11, 5], np.int32)               # 3 tokens x top-2
    onehot = np.array([[1, 0], [0, 1], [1, 0]], np.float32)
    out = OM.combine(y, dest, onehot, 3, 2)
    assert np.array_equal(out, np.stack([y[3], y[0], y[11]]))
    half = np.full((3, 2), 0.5, np.float32)
    out2 = OM.combine(y, dest, half, 3, 2)
    assert np.array_equal(out2[0], F.round_to_bf16(0.5 * y[3] + 0.5 * y[7]))
    assert np.array_equal(out2[1], F.round_to_bf16(0.5 * y[0]))  # dropped slot skipped


def test_grouped_empty_groups_and_permutation():
    rng = np.random.default_rng(7)
    counts = [3, 0, 2, 0]
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    qx = F.e4m3_encode(rng.standard_normal((5, 32)).astype(np.float32))
    qw = F.e4m3_encode(rng.standard_normal((4, 6, 32)).astype(np.float32))
    sx = np.float32(rng.uniform(0.5, 2, 5))
    sw = np.float32(rng.uniform(0.5, 2, (4, 6)))
    y = OG.ref_grouped_fp8(qx, sx, qw, sw, off)
    # swapping groups 0 and 2 permutes output rows accordingly
    perm = np.array([3, 4, 0, 1, 2])
    off2 = np.array([0, 2, 2, 5, 5], np.int32)
    qw2 = qw[[2, 1, 0, 3]]
    sw2 = sw[[2, 1, 0, 3]]
    y2 = OG.ref_grouped_fp8(qx[perm], sx[perm], qw2, sw2, off2)
    assert np.array_equal(y2, y[perm])


def test_rel_errors_definition():
    r = np.array([[1.0, -2.0], [0.001, 4.0]])
    c = r.copy()
    c[1, 0] += 0.001        # tiny entry (below 0.1 rms) does not count elementwise
    g, e = OG.rel_errors(c, r)
    assert math.isclose(g, 0.001 / 4.0) and e == 0.0
    c[0, 0] = 1.02
    g, e = OG.rel_errors(c, r)
    assert math.isclose(e, 0.02, rel_tol=1e-9)


# ------------------------------------------- the fixtures reject planted slips --
def test_e2m1_fixture_discriminates_tie_and_saturation_slips():
    want = gold("e2m1_bf16.npy")[FINITE]
    v = VALS[FINITE]
    ties_away = np.where(np.isin(np.abs(v), [0.25, 1.25, 2.5, 5.0]),
                         F.e2m1_encode(v * np.float32(1.0001)), F.e2m1_encode(v))
    assert not np.array_equal(ties_away, want)
    assert not np.array_equal(F.e2m1_encode_reference_ties(v) & 7, want & 7)


def test_e8m0_fixture_discriminates_off_by_one():
    want = gold("e8m0_bf16.npy")
    sel = FINITE & (VALS > 0)
    slip = (np.clip(F.floor_log2(VALS[sel]) - 1, -127, 127) + 127).astype(np.uint8)
    assert not np.array_equal(slip, want[sel])
    # log2-based rounding (torch's e8m0 cast rounds up) would also be caught
    up = (np.clip(np.ceil(np.log2(VALS[sel].astype(np.float64))) - 2, -127, 127) + 127).astype(np.uint8)
    assert not np.array_equal(up, want[sel])


def test_gemm_kat_discriminates_transposed_operand_and_dropped_scale(kat):
    qa, sa, qw, sw = kat["fp8b_qa"], kat["fp8b_sa"], kat["fp8b_qw"], kat["fp8b_sw"]
    # weight block scales indexed by k-block for n-block (transposed scale grid)
    bad = OG.ref_gemm_dequant(OG.dequant_fp8_blocks(qa, sa, 1, 128),
                              OG.dequant_fp8_blocks(qw, np.ones_like(sw), 128, 128), True)
    g, _ = OG.rel_errors(bad, kat["fp8b_c"])
    assert g > 1e-2


def test_freivalds_check_catches_misplaced_and_misscaled_tiles():
    """The whole-output check of the full-size GPU tests (C v against
    A' (W'^T v), row by row) passes a correct bf16 product and fails one
    with a tile copied from elsewhere, a tile left at zero or a tile off by
    a 10% scale."""
    import torch

    from tests.test_gpu_fullsize import _freivalds

    rng = np.random.default_rng(5)
    a = rng.standard_normal((512, 256)).astype(np.float32)
    w = (0.02 * rng.standard_normal((384, 256))).astype(np.float32)
    c = torch.from_numpy(OG.round_to_bf16(a @ w.T))
    _freivalds(c, a, w, 1, "correct")
    bad = [c.clone() for _ in range(3)]
    bad[0][256:512, 128:256] = c[0:256, 128:256]
    bad[1][0:256, 256:384] = 0
    bad[2][256:512, 0:128] *= 1.1
    for i, b in enumerate(bad):
        with pytest.raises(AssertionError):
            _freivalds(b, a, w, 1, f"planted {i}")
