"""MoE glue on the GPU: routing tables, permute + quantize and combine bit
for bit against the oracle; the routed grouped GEMM end to end within the
GEMM tolerance."""
import numpy as np
import pytest
import torch

from oracle import gemm as OG
from oracle import moe as OM
from dsl_tool_amd import moe as M
from dsl_tool_amd import workloads as W
from tests.util import assert_close, np_f32, np_u8

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ids(T, k, E, seed, drop=False):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, E, (T, k), generator=g, dtype=torch.int32)
    if drop:
        m = torch.rand((T, k), generator=g) < 0.05
        ids[m] = -1
        ids[0, 0] = E          # out of range: dropped too
    return ids


# Route paths: one wave (<= 1024 assignments: 1 x 1, 37 x 3 over 5, 128 x 8
# and 32 x 8 over 64, 100 x 6 over 300 (five 64-expert runs of the scan),
# 256 x 4 over 2000), one workgroup (<= 4096 assignments, <= 1024 experts), and
# count + scatter for the rest, the scatter blocks forming their own bases
# from a small histogram (4096 x 8 over 64 experts, 2100 x 3 over 100: two
# 64-expert runs, ragged last chunk; 5000 x 2 over 3; 200 x 8 over 1100) or
# after a separate scan of a large one (3000 x 6 over 2048; 40000 x 8 over
# 256: more blocks than the scan's 16 ranges cover evenly); no assignments
# over 1500 experts still writes the zero offsets.
ROUTE_CASES = [(4096, 8, 64, False), (37, 3, 5, True), (1, 1, 1, False), (3000, 6, 2048, True),
               (513, 4, 7, False), (512, 8, 64, True), (1024, 4, 1000, False),
               (2100, 3, 100, True), (5000, 2, 3, False), (40000, 8, 256, True),
               (0, 4, 1500, False), (200, 8, 1100, True), (128, 8, 64, True), (100, 6, 300, True),
               (32, 8, 64, False), (256, 4, 2000, True)]


@pytest.mark.parametrize("T,k,E,drop", ROUTE_CASES)
def test_route_matches_oracle(T, k, E, drop):
    ids = _ids(T, k, E, 400 + T, drop)
    r = M.moe_route(ids.to(DEV), E)
    off, dest, src = OM.route(ids.numpy(), E)
    assert np.array_equal(r.offsets.cpu().numpy(), off)
    assert np.array_equal(r.dest.cpu().numpy(), dest)
    n = int(off[-1])
    assert np.array_equal(r.src_token.cpu().numpy()[:n], src)


def test_route_config5_routing():
    ids, _ = W.moe_routing()
    r = M.moe_route(ids.to(DEV), 64)
    counts = W.moe_counts()
    assert np.array_equal(np.diff(r.offsets.cpu().numpy()), counts.numpy())
    assert (np.diff(r.offsets.cpu().numpy()) == 0).sum() >= 4        # forced-empty experts


@pytest.mark.parametrize("T,k,E,K,pad", [(300, 4, 9, 2048, 0), (64, 2, 3, 136, 8), (5, 3, 4, 7168, 0),
                                         (1000, 8, 64, 2048, 0), (3, 8, 5, 32768, 16), (1, 1, 1, 8, 0)])
def test_permute_quant_matches_oracle(T, k, E, K, pad):
    ids = _ids(T, k, E, 410 + T, drop=True)
    x = W.randn_bf16((T, K), 411) * 3
    r = M.moe_route(ids.to(DEV), E)
    xd = x.to(DEV)
    if pad:      # row stride K + pad: the kernel reads rows at ldx
        xd = torch.nn.functional.pad(xd, (0, pad))[:, :K]
    qx, sx = M.moe_permute_quant(xd, r)
    off, dest, src = OM.route(ids.numpy(), E)
    q_ref, s_ref = OM.permute_quant(x.float().numpy(), src)
    n = int(off[-1])
    assert np.array_equal(np_u8(qx)[:n], q_ref)
    assert np.array_equal(np_f32(sx)[:n], s_ref)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_combine_matches_oracle(out_dtype):
    T, k, E, Nn = 257, 8, 16, 1536
    ids = _ids(T, k, E, 420, drop=True)
    wts = torch.softmax(torch.randn((T, k), generator=torch.Generator().manual_seed(421)), 1)
    r = M.moe_route(ids.to(DEV), E)
    y = W.randn_bf16((T * k, Nn), 422)
    out = M.moe_combine(y.to(DEV), r, wts.to(DEV), out_dtype=out_dtype)
    ref = OM.combine(y.float().numpy(), r.dest.cpu().numpy(), wts.numpy(), T, k,
                     out_bf16=out_dtype == torch.bfloat16)
    assert np.array_equal(np_f32(out), ref)


def test_routed_grouped_gemm_end_to_end():
    """The routed chain stage by stage, each to its own bar: routing tables
    and token codes bit-exact, the grouped GEMM's rows y against the grouped
    oracle (max-relative and elementwise 1e-2), the combine of that y
    bit-exact against the oracle combine of the same y, and the one-call
    routed_grouped_gemm equal to the chain bit for bit; end to end against
    the all-oracle chain the north-star max-relative bound (the combine sums
    topk bf16-rounded GEMM rows, and one bf16 ulp of a large row lands whole
    on a sum that cancels, so elementwise the end-to-end error is the
    GEMM's, carried through the exact combine)."""
    T, k, E, K, Nn = 512, 4, 16, 1024, 768
    ids = _ids(T, k, E, 430)
    wts = torch.softmax(torch.randn((T, k), generator=torch.Generator().manual_seed(431)), 1)
    x = W.randn_bf16((T, K), 432)
    w = W.randn_bf16((E, K, Nn), 433, 0.02)
    out = M.routed_grouped_gemm(x.to(DEV), ids.to(DEV), wts.to(DEV), w.to(DEV),
                                out_dtype=torch.float32)
    # oracle chain: route -> permute_quant -> grouped reference -> combine
    off, dest, src = OM.route(ids.numpy(), E)
    qx, sx = OM.permute_quant(x.float().numpy(), src)
    from oracle import quant as OQ
    wt = w.float().numpy().transpose(0, 2, 1).reshape(E * Nn, K)
    qw, sw = OQ.quant_fp8_blockwise(wt, 1, K)
    y_ref = OG.ref_grouped_fp8(qx, sx, qw.reshape(E, Nn, K), sw.reshape(E, Nn), off)
    ref = OM.combine(y_ref, dest, wts.numpy(), T, k, out_bf16=False)
    # the same chain on the GPU, stage by stage
    from dsl_tool_amd import quant as Q
    r = M.moe_route(ids.to(DEV), E)
    assert np.array_equal(r.offsets.cpu().numpy(), off)
    assert np.array_equal(r.dest.cpu().numpy(), dest)
    qwd, swd = Q.quant_fp8_blocks(w.to(DEV).transpose(1, 2).reshape(E * Nn, K), 1, K)
    assert np.array_equal(np_u8(qwd), qw) and np.array_equal(np_f32(swd), sw)
    qt, sxt = M.moe_quant_tokens(x.to(DEV), r)
    n = int(off[-1])
    assert np.array_equal(np_u8(qt)[src[:n]], qx) and np.array_equal(np_f32(sxt)[:n], sx)
    y = M.moe_grouped_fp8_gemm(qt, sxt, r, qwd.reshape(E, Nn, K), swd.reshape(E, Nn))
    assert_close(y[:n], y_ref, what="routed grouped gemm: grouped rows")
    comb = M.moe_combine(y, r, wts.to(DEV), out_dtype=torch.float32)
    assert np.array_equal(np_f32(comb), OM.combine(np_f32(y), dest, wts.numpy(), T, k,
                                                   out_bf16=False))
    assert torch.equal(comb, out)
    # end to end: the north-star max-relative bound, and per entry the error
    # is the grouped rows' error carried through the (positive) combine
    # weights, sum_j w_tj |y - y_ref|[dest], up to the combine's fp32 rounding
    glob, _ = OG.rel_errors(np_f32(out), ref)
    assert glob <= 1e-2, glob
    yerr = np.zeros((T * k, Nn), np.float32)
    yerr[:n] = np.abs(np_f32(y)[:n].astype(np.float64) - y_ref)
    carried = OM.combine(yerr, dest, wts.numpy(), T, k, out_bf16=False).astype(np.float64)
    # fp32 rounding of the two combines: a few ulps of sum_j w_tj |y_ref|
    mag = OM.combine(np.abs(y_ref).astype(np.float32), dest, wts.numpy(), T, k,
                     out_bf16=False).astype(np.float64)
    err = np.abs(np_f32(out).astype(np.float64) - ref)
    assert (err <= carried * (1 + 1e-5) + 1e-6 * mag + 1e-30).all()


@pytest.mark.parametrize("T,k,E,K,pad", [(300, 4, 9, 2048, 0), (64, 2, 3, 136, 8), (1000, 8, 64, 2048, 0),
                                         (3, 8, 5, 32768, 16), (1, 1, 1, 8, 0)])
def test_quant_tokens_matches_oracle(T, k, E, K, pad):
    # token-major codes; the scales at every sorted row of the token
    ids = _ids(T, k, E, 440 + T, drop=True)
    x = W.randn_bf16((T, K), 441) * 3
    r = M.moe_route(ids.to(DEV), E)
    xd = x.to(DEV)
    if pad:
        xd = torch.nn.functional.pad(xd, (0, pad))[:, :K]
    qt, sx = M.moe_quant_tokens(xd, r)
    off, dest, src = OM.route(ids.numpy(), E)
    q_ref, s_ref = OM.permute_quant(x.float().numpy(), src)
    n = int(off[-1])
    assert np.array_equal(np_u8(qt)[src], q_ref)
    assert np.array_equal(np_f32(sx)[:n], s_ref)


# Route + per-token quantize in one launch (decode sizes, tokens * topk <=
# 1024, K <= 2048): every table, code and scale equal to the two launches
# it replaces and to the oracle.  Dropped ids; one token; 1024 assignments
# (the most one wave ranks); 2000 experts (the scan in 32 runs of 64);
# padded rows; K of one 8-element chunk and of four chunks per lane; and
# sizes past the limits, which take the two calls.
ROUTE_QUANT_CASES = [(32, 8, 64, 2048, 0, True), (1, 8, 64, 2048, 0, False),
                     (128, 8, 64, 1024, 8, True), (37, 3, 5, 136, 0, True),
                     (256, 4, 2000, 512, 16, True), (5, 1, 1, 8, 0, False),
                     (200, 8, 64, 2048, 0, False), (4, 2, 3, 4096, 0, False)]


@pytest.mark.parametrize("T,k,E,K,pad,drop", ROUTE_QUANT_CASES)
def test_route_quant_tokens_matches_two_launches(T, k, E, K, pad, drop):
    ids = _ids(T, k, E, 470 + T, drop)
    x = W.randn_bf16((T, K), 471) * 3
    xd = x.to(DEV)
    if pad:
        xd = torch.nn.functional.pad(xd, (0, pad))[:, :K]
    fused = M.route_quant_applies(T, k, E, K)
    assert fused == (T * k <= 1024 and K <= 2048)
    r, qt, sx = M.moe_route_quant_tokens(ids.to(DEV), xd, E)
    r2 = M.moe_route(ids.to(DEV), E)
    qt2, sx2 = M.moe_quant_tokens(xd, r2)
    off, dest, src = OM.route(ids.numpy(), E)
    n = int(off[-1])
    assert np.array_equal(r.offsets.cpu().numpy(), off)
    assert np.array_equal(r.dest.cpu().numpy(), dest)
    assert np.array_equal(r.src_token.cpu().numpy()[:n], src)
    assert torch.equal(r.offsets, r2.offsets) and torch.equal(r.dest, r2.dest)
    assert torch.equal(r.src_token[:n], r2.src_token[:n])
    assert torch.equal(qt, qt2)
    assert torch.equal(sx[:n], sx2[:n])
    q_ref, s_ref = OM.permute_quant(x.float().numpy(), src)
    assert np.array_equal(np_u8(qt)[src], q_ref)
    assert np.array_equal(np_f32(sx)[:n], s_ref)


def test_route_quant_tokens_unsupported_sizes_report():
    from dsl_tool_amd import _native as N
    ids = torch.zeros((300, 4), dtype=torch.int32, device=DEV)
    x = torch.zeros((300, 256), dtype=torch.bfloat16, device=DEV)
    off = torch.empty(9, dtype=torch.int32, device=DEV)
    dest = torch.empty(1200, dtype=torch.int32, device=DEV)
    src = torch.empty(1200, dtype=torch.int32, device=DEV)
    qx = torch.empty((300, 256), dtype=torch.uint8, device=DEV)
    sx = torch.empty(1200, dtype=torch.float32, device=DEV)
    rc = N.lib().dsl_moe_route_quant_tokens(ids.data_ptr(), 300, 4, 8, x.data_ptr(), 256, 256,
                                            off.data_ptr(), dest.data_ptr(), src.data_ptr(),
                                            qx.data_ptr(), sx.data_ptr(), N.stream_of(x.device))
    assert rc == N.DSL_ERR_UNSUPPORTED


def _expert_weights(E, Nn, K, seed):
    from dsl_tool_amd import quant as Q
    w = W.randn_bf16((E * Nn, K), seed, 0.02).to(DEV)
    qw, sw = Q.quant_fp8_blocks(w, 1, K)
    return qw.reshape(E, Nn, K), sw.reshape(E, Nn)


# The gather kernel against the persistent kernel over the permuted copy:
# the same codes, scales and MFMA order, so the same bits.  K = 128 is one
# pair per tile (the next tile's row table is waited for before the first
# copies); ragged N; one expert; config 5's routing and sizes.  Below 48
# rows per group on average the gather streams (the streaming grouped tiles
# over the permuted copy are the reference): decode sizes with 16- and
# 32-row blocks, K of an odd number of 256-byte chunks, ragged N, and
# K % 256 != 0 (the persistent kernel again).
GATHER_CASES = [(512, 4, 16, 1024, 768), (300, 3, 2, 128, 520), (1000, 2, 5, 256, 256),
                (2000, 1, 1, 384, 300), (4096, 8, 64, 2048, 1536),
                (32, 8, 64, 2048, 1536), (1, 8, 64, 2048, 1536), (200, 8, 64, 2048, 1536),
                (7, 2, 3, 256, 520), (40, 4, 8, 768, 300), (30, 2, 4, 384, 256)]


@pytest.mark.parametrize("T,k,E,K,Nn", GATHER_CASES)
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_gather_gemm_equals_permuted(T, k, E, K, Nn, out_dtype):
    from dsl_tool_amd import gemm as G
    if (T, E) == (4096, 64):
        ids = W.moe_routing()[0]
    else:
        ids = _ids(T, k, E, 450 + T, drop=True)
    assert M.gather_applies(T, k, E, K)
    x = (W.randn_bf16((T, K), 451) * 2).to(DEV)
    qw, sw = _expert_weights(E, Nn, K, 452)
    r = M.moe_route(ids.to(DEV), E)
    qt, st = M.moe_quant_tokens(x, r)
    qp, sp = M.moe_permute_quant(x, r)
    yg = M.moe_grouped_fp8_gemm(qt, st, r, qw, sw, out_dtype=out_dtype)
    yp = G.grouped_fp8_gemm_packed(qp, sp, qw, sw, r.offsets, out_dtype=out_dtype)
    torch.cuda.synchronize()
    n = int(r.offsets[-1].item())
    assert torch.equal(yg[:n].view(torch.int16 if out_dtype == torch.bfloat16 else torch.int32),
                       yp[:n].view(torch.int16 if out_dtype == torch.bfloat16 else torch.int32))


@pytest.mark.parametrize("T,k,E", [(700, 2, 3), (40, 4, 8)])   # persistent, streaming
def test_gather_gemm_clamps_bad_row_map(T, k, E):
    # row-map entries outside [0, tokens) read the last token's row
    from dsl_tool_amd import gemm as G
    K, Nn = 256, 384
    ids = _ids(T, k, E, 460)
    x = W.randn_bf16((T, K), 461).to(DEV)
    qw, sw = _expert_weights(E, Nn, K, 462)
    r = M.moe_route(ids.to(DEV), E)
    qt, st = M.moe_quant_tokens(x, r)
    bad = r.src_token.clone()
    bad[5], bad[(T * k) // 2], bad[T * k - 1] = -7, T, 1 << 30   # first tile, later tiles
    rb = r._replace(src_token=bad)
    yg = M.moe_grouped_fp8_gemm(qt, st, rb, qw, sw)
    qp = qt[bad.clamp(0, T - 1).long()]                    # -7 -> 2^32 - 7 -> last token too
    qp[5] = qt[T - 1]
    yp = G.grouped_fp8_gemm_packed(qp, st, qw, sw, r.offsets)
    torch.cuda.synchronize()
    assert torch.equal(yg.view(torch.int16), yp.view(torch.int16))
