"""GPU quantize/pack kernels vs the CPU oracle: bit-exact codes and scales."""
import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import quant as OQ
from dsl_tool_amd import quant as Q
from dsl_tool_amd import workloads as W
from tests.util import np_u8, np_f32

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _f32(x: torch.Tensor) -> np.ndarray:
    return x.float().numpy()


def _all_bf16_upto(limit: float) -> np.ndarray:
    """Every finite bf16 value with |v| <= limit (both signs, zeros, subnormals)."""
    v = F.bf16_bits_to_f32(np.arange(65536, dtype=np.uint16))
    return v[np.isfinite(v) & (np.abs(v) <= limit)]


def _rows_with_pin(values: np.ndarray, group: int, pin: float) -> np.ndarray:
    """Lay values out in rows of `group` elements whose first element is `pin`
    (which fixes the group's scale); pads with zeros."""
    per = group - 1
    n = -(-len(values) // per)
    body = np.zeros(n * per, np.float32)
    body[:len(values)] = values
    rows = np.concatenate([np.full((n, 1), pin, np.float32), body.reshape(n, per)], axis=1)
    return rows


def _to_gpu_bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).bfloat16().to(DEV)


@pytest.mark.parametrize("shape", [(128, 4096), (37, 272), (1, 16)])
def test_fp8_tensor_matches_oracle(shape):
    x = W.randn_bf16(shape, 11)
    q, s = Q.quant_fp8_tensor(x.to(DEV))
    q_ref, s_ref = OQ.quant_fp8_per_tensor(_f32(x))
    assert np_f32(s)[0] == s_ref
    assert np.array_equal(np_u8(q), q_ref)


def test_fp8_tensor_strided_input_matches():
    # the reference's B[K, N] passed as a contiguous [K, N] tensor: its [N, K]
    # view has stride (1, N) and takes the strided path
    b_kn = W.randn_bf16((256, 96), 12, 0.02)
    q, s = Q.quant_fp8_tensor(b_kn.to(DEV).t())
    q_ref, s_ref = OQ.quant_fp8_per_tensor(_f32(b_kn.t()))
    assert np_f32(s)[0] == s_ref
    assert np.array_equal(np_u8(q), q_ref)


def test_fp8_tensor_zero_input_uses_scale_floor():
    x = torch.zeros((8, 64), dtype=torch.bfloat16, device=DEV)
    q, s = Q.quant_fp8_tensor(x)
    assert np_f32(s)[0] == np.float32(1e-12)
    assert not np_u8(q).any()


def test_e4m3_encoder_exhaustive_at_unit_scale():
    # every bf16 value in [-448, 448], grouped 1x128 with a pinned 448 -> scale 1.0
    rows = _rows_with_pin(_all_bf16_upto(448.0), 128, 448.0)
    q, s = Q.quant_fp8_blocks(_to_gpu_bf16(rows), 1, 128)
    assert (np_f32(s) == 1.0).all()
    want = torch.from_numpy(rows).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(np_u8(q), want)


# The vector quantizers divide through the reciprocal of the scale and fall
# back to the exact quotient only where it lies within a few ulp of an E4M3 /
# E2M1 rounding boundary.  Every bf16 value under a pinned group amax with a
# non-power-of-two scale puts many quotients at or next to those boundaries.
@pytest.mark.parametrize("amax", [1.7, 3.3, 100.1, 0.013, 447.0, 5.9e-3, 2.0e4])
def test_fp8_division_near_rounding_boundaries(amax):
    amax = float(np.float32(torch.tensor(amax).bfloat16().float()))
    rows = _rows_with_pin(_all_bf16_upto(amax), 128, amax)
    for layout in ("row", "tile", "tensor"):
        if layout == "tensor":
            q, s = Q.quant_fp8_tensor(_to_gpu_bf16(rows))
            q_ref, s_ref = OQ.quant_fp8_per_tensor(rows)
            assert np_f32(s)[0] == np.float32(s_ref)
        else:
            gr, gc = (1, 128) if layout == "row" else (128, 128)
            q, s = Q.quant_fp8_blocks(_to_gpu_bf16(rows), gr, gc)
            q_ref, s_ref = OQ.quant_fp8_blockwise(rows, gr, gc)
            assert np.array_equal(np_f32(s), s_ref)
        assert np.array_equal(np_u8(q), q_ref), layout


@pytest.mark.parametrize("amax,boost", [(1.7, 1.0), (5.3, 1.37), (100.1, 1.0),
                                        (0.013, 2.9), (3.0e3, 1.11)])
def test_nvfp4_division_near_rounding_boundaries(amax, boost):
    # `boost` adds one block whose amax sets the global scale above the pinned
    # blocks', so their E4M3 block scales land between powers of two.
    amax = float(np.float32(torch.tensor(amax).bfloat16().float()))
    flat = _rows_with_pin(_all_bf16_upto(amax), 16, amax).reshape(-1)
    top = np.zeros(16, np.float32)
    top[0] = float(np.float32(torch.tensor(amax * boost).bfloat16().float()))
    flat = np.concatenate([top, flat, np.zeros(-(flat.size + 16) % 64, np.float32)])
    rows = flat.reshape(-1, 64)
    q, sb, sg = Q.quant_nvfp4(_to_gpu_bf16(rows))
    q_ref, sb_ref, sg_ref = OQ.quant_nvfp4(rows)
    assert np_f32(sg)[0] == sg_ref
    assert np.array_equal(np_u8(sb), sb_ref)
    assert np.array_equal(np_u8(q), q_ref)


@pytest.mark.parametrize("gr,gc", [(1, 128), (128, 128), (1, 4096), (1, 64), (16, 48), (1, 200), (1, 2048),
                                   (1, 16384), (1, 32), (1, 512), (1, 1024), (1, 264), (1, 1000)])
def test_fp8_blocks_match_oracle(gr, gc):
    x = W.activations(2, 300, 4096, outliers=True)
    q, s = Q.quant_fp8_blocks(x.to(DEV), gr, gc)
    q_ref, s_ref = OQ.quant_fp8_blockwise(_f32(x), gr, gc)
    assert np.array_equal(np_f32(s), s_ref)
    assert np.array_equal(np_u8(q), q_ref)


def test_fp8_blocks_strided_input_matches():
    b_kn = W.randn_bf16((384, 200), 13, 0.02)
    q, s = Q.quant_fp8_blocks(b_kn.to(DEV).t(), 128, 128)
    q_ref, s_ref = OQ.quant_fp8_blockwise(_f32(b_kn.t()), 128, 128)
    assert np.array_equal(np_f32(s), s_ref)
    assert np.array_equal(np_u8(q), q_ref)


# Row-padded views (row stride > C, still 16-byte aligned rows) and row
# lengths that are not a multiple of the group take the team / non-packed
# kernels instead of the packed ones.
def _padded(shape, seed, pad=64):
    wide = W.randn_bf16((shape[0], shape[1] + pad), seed)
    return wide.to(DEV)[:, :shape[1]], _f32(wide[:, :shape[1]])


@pytest.mark.parametrize("fmt", ["fp8_tensor", "fp8_row128", "fp8_row32", "fp8_tile", "mxfp4", "nvfp4"])
def test_padded_rows_match_oracle(fmt):
    xd, xr = _padded((40, 512), 41)
    assert xd.stride(0) == 576
    if fmt == "fp8_tensor":
        q, s = Q.quant_fp8_tensor(xd)
        q_ref, s_ref = OQ.quant_fp8_per_tensor(xr)
        assert np_f32(s)[0] == s_ref
    elif fmt.startswith("fp8"):
        gr, gc = {"fp8_row128": (1, 128), "fp8_row32": (1, 32), "fp8_tile": (128, 128)}[fmt]
        q, s = Q.quant_fp8_blocks(xd, gr, gc)
        q_ref, s_ref = OQ.quant_fp8_blockwise(xr, gr, gc)
        assert np.array_equal(np_f32(s), s_ref)
    elif fmt == "mxfp4":
        q, s = Q.quant_mxfp4(xd)
        q_ref, s_ref = OQ.quant_mxfp4(xr)
        assert np.array_equal(np_u8(s), s_ref)
    else:
        q, s, g = Q.quant_nvfp4(xd)
        q_ref, s_ref, g_ref = OQ.quant_nvfp4(xr)
        assert np_f32(g)[0] == g_ref
        assert np.array_equal(np_u8(s), s_ref)
    assert np.array_equal(np_u8(q), q_ref)


@pytest.mark.parametrize("cols,gc", [(200, 128), (72, 64), (520, 256)])
def test_fp8_row_groups_ragged_cols(cols, gc):
    x = W.randn_bf16((9, cols), 42)
    q, s = Q.quant_fp8_blocks(x.to(DEV), 1, gc)
    q_ref, s_ref = OQ.quant_fp8_blockwise(_f32(x), 1, gc)
    assert np.array_equal(np_f32(s), s_ref)
    assert np.array_equal(np_u8(q), q_ref)


def test_e2m1_encoder_exhaustive_at_unit_scale():
    # every bf16 value with |v| < 8 in 32-blocks pinned by 4.0 -> E8M0 127 (2^0)
    vals = _all_bf16_upto(7.96875)
    rows = _rows_with_pin(vals, 32, 4.0)
    q, e = Q.quant_mxfp4(_to_gpu_bf16(rows))
    assert (np_u8(e) == 127).all()
    want = F.pack_nibbles(F.e2m1_encode(rows))
    assert np.array_equal(np_u8(q), want)


@pytest.mark.parametrize("shape,seed", [((64, 8192), 21), ((33, 96), 22), ((16, 32), 23)])
def test_mxfp4_matches_oracle(shape, seed):
    x = W.randn_bf16(shape, seed)
    q, e = Q.quant_mxfp4(x.to(DEV))
    q_ref, e_ref = OQ.quant_mxfp4(_f32(x))
    assert np.array_equal(np_u8(e), e_ref)
    assert np.array_equal(np_u8(q), q_ref)


def test_mxfp4_wide_dynamic_range_and_zero_blocks():
    x = W.randn_bf16((32, 256), 24).float()
    scale = torch.exp2(torch.arange(-60, 68, 4, dtype=torch.float32))[:, None]
    x = x * scale
    x[3] = 0.0
    x[5, :32] = 1e-40      # fp32-subnormal magnitudes (bf16 subnormals)
    x = x.bfloat16()
    q, e = Q.quant_mxfp4(x.to(DEV))
    q_ref, e_ref = OQ.quant_mxfp4(_f32(x))
    assert np.array_equal(np_u8(e), e_ref)
    assert np.array_equal(np_u8(q), q_ref)


def test_mxfp4_strided_input_matches():
    b_kn = W.randn_bf16((256, 40), 25, 0.02)
    q, e = Q.quant_mxfp4(b_kn.to(DEV).t())
    q_ref, e_ref = OQ.quant_mxfp4(_f32(b_kn.t()))
    assert np.array_equal(np_u8(e), e_ref)
    assert np.array_equal(np_u8(q), q_ref)


@pytest.mark.parametrize("shape,seed", [((64, 4096), 31), ((3, 48), 32), ((1, 16), 33)])
def test_nvfp4_matches_oracle(shape, seed):
    x = W.randn_bf16(shape, seed)
    q, sb, sg = Q.quant_nvfp4(x.to(DEV))
    q_ref, sb_ref, sg_ref = OQ.quant_nvfp4(_f32(x))
    assert np_f32(sg)[0] == sg_ref
    assert np.array_equal(np_u8(sb), sb_ref)
    assert np.array_equal(np_u8(q), q_ref)


def test_nvfp4_underflowing_blocks_and_zero_tensor():
    x = W.randn_bf16((8, 64), 34).float()
    x[0, 0] = 3.0e4          # large amax: tiny blocks' E4M3 scales underflow to 0
    x[2, 16:32] *= 1e-6
    x[4] = 0.0
    x = x.bfloat16()
    q, sb, sg = Q.quant_nvfp4(x.to(DEV))
    q_ref, sb_ref, sg_ref = OQ.quant_nvfp4(_f32(x))
    assert np_f32(sg)[0] == sg_ref
    assert np.array_equal(np_u8(sb), sb_ref)
    assert np.array_equal(np_u8(q), q_ref)
    z = torch.zeros((2, 32), dtype=torch.bfloat16, device=DEV)
    qz, sbz, sgz = Q.quant_nvfp4(z)
    assert np_f32(sgz)[0] == np.float32(1e-12) and not np_u8(qz).any() and not np_u8(sbz).any()


def test_nvfp4_strided_input_matches():
    b_kn = W.randn_bf16((128, 24), 35, 0.02)
    q, sb, sg = Q.quant_nvfp4(b_kn.to(DEV).t())
    q_ref, sb_ref, sg_ref = OQ.quant_nvfp4(_f32(b_kn.t()))
    assert np_f32(sg)[0] == sg_ref
    assert np.array_equal(np_u8(sb), sb_ref)
    assert np.array_equal(np_u8(q), q_ref)


# ------------------------------------------------------- fp32 / fp16 sources --
# The reference quantizers read fp32 (cuda/gemm/fp8_gemm.cu:118-144,
# cuda/gemm/fp4_gemm.cu:49-90).  fp32 sources are quantized from their own
# values: codes of the IEEE quotient of the fp32 element by the fp32 scale.
# The inputs sit one ulp either side of the E4M3 / E2M1 rounding midpoints,
# and the amax is not a bf16 value, so rounding the source to bf16 first (or
# dividing by a reciprocal) changes codes; each test checks that it would.

def _near(vals: np.ndarray) -> np.ndarray:
    """vals and their fp32 neighbours one ulp below and above."""
    v = vals.astype(np.float32)
    return np.concatenate([np.nextafter(v, np.float32(-np.inf)), v,
                           np.nextafter(v, np.float32(np.inf))]).astype(np.float32)


E4M3_MIDS = np.array([0.5 * (a + b) for a, b in
                      zip(F.e4m3_decode(np.arange(0, 0x7E, dtype=np.uint8)),
                          F.e4m3_decode(np.arange(1, 0x7F, dtype=np.uint8)))], np.float32)
E2M1_MIDS = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32)


def _fp32_rows(body: np.ndarray, cols: int, pin: float) -> np.ndarray:
    """body laid out in rows of `cols` (zero padded), every row led by `pin`."""
    per = cols - 1
    n = -(-len(body) // per)
    flat = np.zeros(n * per, np.float32)
    flat[:len(body)] = body
    return np.concatenate([np.full((n, 1), pin, np.float32), flat.reshape(n, per)], axis=1)


def _signed(v: np.ndarray) -> np.ndarray:
    return np.concatenate([v, -v]).astype(np.float32)


def test_fp8_tensor_fp32_source_near_midpoints():
    amax = np.float32(1.2345678)                 # not a bf16 value
    s = np.float32(amax / np.float32(448.0))
    x = _fp32_rows(_signed(_near((E4M3_MIDS[E4M3_MIDS < 448] * s).astype(np.float32))), 128, amax)
    q, sc = Q.quant_fp8_tensor(torch.from_numpy(x).to(DEV))
    q_ref, s_ref = OQ.quant_fp8_per_tensor(x)
    assert np_f32(sc)[0] == s_ref
    assert np.array_equal(np_u8(q), q_ref)
    # the bf16-rounded source would encode differently
    q_bf, _ = OQ.quant_fp8_per_tensor(torch.from_numpy(x).bfloat16().float().numpy())
    assert not np.array_equal(q_bf, q_ref)


@pytest.mark.parametrize("gr,gc", [(1, 128), (128, 128)])
def test_fp8_blocks_fp32_source(gr, gc):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((256, 384)) * 3).astype(np.float32)
    x[::7, ::5] *= np.float32(1.0009765)        # mantissa bits bf16 does not hold
    q, s = Q.quant_fp8_blocks(torch.from_numpy(x).to(DEV), gr, gc)
    q_ref, s_ref = OQ.quant_fp8_blockwise(x, gr, gc)
    assert np.array_equal(np_f32(s), s_ref)
    assert np.array_equal(np_u8(q), q_ref)
    # strided fp32 view (the reference's B[K, N] orientation)
    xt = torch.from_numpy(np.ascontiguousarray(x.T)).to(DEV).t()
    q2, s2 = Q.quant_fp8_blocks(xt, gr, gc)
    assert np.array_equal(np_f32(s2), s_ref) and np.array_equal(np_u8(q2), q_ref)


def _f32_rows_dev(x: np.ndarray, pad: int) -> torch.Tensor:
    """x on the GPU as a view with row stride cols + pad."""
    t = torch.from_numpy(np.ascontiguousarray(x)).to(DEV)
    return torch.nn.functional.pad(t, (0, pad))[:, :x.shape[1]] if pad else t


# fp32 rows with unit column stride take the vector fp32 kernels (a team of
# lanes per group, IEEE quotients); other layouts the strided kernels
@pytest.mark.parametrize("gc", [32, 64, 128, 256])
@pytest.mark.parametrize("cols,pad", [(384, 0), (200, 0), (520, 12)])
def test_fp8_row_groups_fp32_source(gc, cols, pad):
    rng = np.random.default_rng(gc + cols)
    x = (rng.standard_normal((97, cols)) * 3).astype(np.float32)
    x[::5, ::3] *= np.float32(1.0009765)       # mantissa bits bf16 does not hold
    x[7] = 0.0                                  # an all-zero row: the 1e-12 floor
    q, s = Q.quant_fp8_blocks(_f32_rows_dev(x, pad), 1, gc)
    q_ref, s_ref = OQ.quant_fp8_blockwise(x, 1, gc)
    assert np.array_equal(np_f32(s), s_ref)
    assert np.array_equal(np_u8(q), q_ref)


@pytest.mark.parametrize("pad", [0, 4])
def test_fp32_source_padded_rows_all_formats(pad):
    rng = np.random.default_rng(pad + 3)
    x = (rng.standard_normal((65, 256)) * 2).astype(np.float32)
    x[3, :32] *= np.float32(1e-30)              # tiny block
    x[9, 16:32] = 0.0                           # zero NVFP4 block
    xd = _f32_rows_dev(x, pad)
    q, sc = Q.quant_fp8_tensor(xd)
    q_ref, s_ref = OQ.quant_fp8_per_tensor(x)
    assert np_f32(sc)[0] == s_ref and np.array_equal(np_u8(q), q_ref)
    q, e = Q.quant_mxfp4(xd)
    q_ref, e_ref = OQ.quant_mxfp4(x)
    assert np.array_equal(np_u8(e), e_ref) and np.array_equal(np_u8(q), q_ref)
    q, sb, g = Q.quant_nvfp4(xd)
    q_ref, sb_ref, g_ref = OQ.quant_nvfp4(x)
    assert np_f32(g)[0] == g_ref
    assert np.array_equal(np_u8(sb), sb_ref) and np.array_equal(np_u8(q), q_ref)


def test_mxfp4_fp32_source_near_midpoints():
    # blocks of 32 whose amax 5.5 * 2^k fixes the shared exponent k, the other
    # 31 elements one ulp around the E2M1 midpoints of that exponent
    rows = []
    for k in (-3, 0, 4):
        body = _signed(_near(E2M1_MIDS * np.float32(2.0 ** k)))
        rows.append(_fp32_rows(body, 32, np.float32(5.5 * 2.0 ** k)))
    x = np.concatenate(rows, axis=0)
    x = np.concatenate([x, np.zeros((x.shape[0], 32), np.float32)], axis=1)   # zero blocks
    q, e = Q.quant_mxfp4(torch.from_numpy(x).to(DEV))
    q_ref, e_ref = OQ.quant_mxfp4(x)
    assert np.array_equal(np_u8(e), e_ref)
    assert np.array_equal(np_u8(q), q_ref)
    q_bf, _ = OQ.quant_mxfp4(torch.from_numpy(x).bfloat16().float().numpy())
    assert not np.array_equal(q_bf, q_ref)


def test_nvfp4_fp32_source_near_midpoints():
    amax_t = np.float32(7.654321)                # global scale amax / 2688 from an fp32 amax
    sg = np.float32(amax_t / np.float32(2688.0))
    rows = []
    for bmax in (np.float32(7.654321), np.float32(0.3141593), np.float32(2.7182817)):
        sb = F.e4m3_decode(F.e4m3_encode(np.float32(np.float32(bmax / np.float32(6.0)) / sg)))
        d = np.float32(np.float32(sb) * sg)
        body = _signed(_near((E2M1_MIDS * d).astype(np.float32)))
        body = body[np.abs(body) <= bmax]
        rows.append(_fp32_rows(body, 16, bmax))
    x = np.concatenate(rows, axis=0)
    q, sbc, g = Q.quant_nvfp4(torch.from_numpy(x).to(DEV))
    q_ref, sb_ref, g_ref = OQ.quant_nvfp4(x)
    assert np_f32(g)[0] == g_ref
    assert np.array_equal(np_u8(sbc), sb_ref)
    assert np.array_equal(np_u8(q), q_ref)
    q_bf, _, _ = OQ.quant_nvfp4(torch.from_numpy(x).bfloat16().float().numpy())
    assert not np.array_equal(q_bf, q_ref)


def test_fp16_source_is_widened_exactly():
    rng = np.random.default_rng(6)
    x16 = torch.from_numpy((rng.standard_normal((64, 256)) * 5).astype(np.float16))
    x32 = x16.float().numpy()
    q, s = Q.quant_fp8_tensor(x16.to(DEV))
    q_ref, s_ref = OQ.quant_fp8_per_tensor(x32)
    assert np_f32(s)[0] == s_ref and np.array_equal(np_u8(q), q_ref)
    q, e = Q.quant_mxfp4(x16.to(DEV))
    q_ref, e_ref = OQ.quant_mxfp4(x32)
    assert np.array_equal(np_u8(e), e_ref) and np.array_equal(np_u8(q), q_ref)
