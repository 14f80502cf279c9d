#!/usr/bin/env python3
"""Benchmark of the quantized GEMM path on one MI355X.

``python bench.py [--gpus 1] [--steps K] [--warmup W] [--cases LIST] [--no-cpu]``

A "step" is one GEMM on operands that are already quantized/packed and
resident in HBM (the quantize pass is timed separately as its own case).
The headline workload is BASELINE config 2 at its compute-bound size: FP8
E4M3 with 1x128 activation groups and 128x128 weight blocks, M=4096,
N=7168, K=4096.  ``value`` is its throughput in TFLOP/s over exactly K timed
steps, bracketed by ``torch.cuda.synchronize()``; the step time comes from
HIP events recorded on the stream the kernels are launched on.

The other BASELINE workloads are reported in ``cases`` (TFLOP/s, fraction of
the MFMA peak, algorithmic GB/s and fraction of HBM peak).  HBM-bound cases
rotate through enough weight copies (> 256 MB) that the 256 MB Infinity
Cache cannot serve them, and are timed as a captured HIP graph of K launches
so host launch latency does not enter the kernel time.

``cpu_baseline`` times the CPU oracle (dequantize -> fp32 torch matmul) on
the headline workload, on the host's cores, and in ``legs`` the reference's
own tiled CPU path (restated) on BASELINE config 1 and config 5; it states
the threads used, ``os.cpu_count()`` and the CPU model.

``roofline.traffic`` is the headline kernel's HBM bytes per launch from two
``rocprofv3 --pmc`` runs (FETCH_SIZE, then WRITE_SIZE) of
``python3 bench.py --profile-traffic``, each scaled by the same counter's
reading for a plain 256 MiB device copy in that run; the summary lives in
``profiles/fp8_block_m4096_traffic.txt`` and is read from there (null when
the file is absent).

Only one GPU: ``--gpus N`` with N > 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import shutil
import subprocess
import sys
import threading
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_FP8_TFLOPS = 5000.0      # MI355X dense fp8 MFMA
PEAK_FP4_TFLOPS = 10100.0     # MI355X dense fp4 MFMA
PEAK_FP16_TFLOPS = 2500.0     # MI355X dense fp16 MFMA (the NVFP4 kernels dequantize to fp16)
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
HEADLINE = "fp8_block_m4096"
MALL_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "fp8_block_m4096_traffic.txt")
# algorithmic bytes of one headline GEMM: A and W codes, fp32 1x128 / 128x128
# scales and the bf16 C, each once
HEADLINE_BYTES = 4096 * 4096 + 7168 * 4096 + 4096 * 32 * 4 + 56 * 32 * 4 + 4096 * 7168 * 2
COPY_BYTES = 256 << 20          # calibration copy for the HBM byte counters
WARM_MS = 50.0                  # per-case warm-up time on the GPU before timing


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# --------------------------------------------------------------------------
# Case construction: each case returns (launch(i, stream), flops, bytes, peak,
# n_rot) with every buffer preallocated; launch() calls the C ABI directly.
# --------------------------------------------------------------------------

def _rotations(bytes_per_copy: int) -> int:
    """Copies of the weight operand needed to exceed the Infinity Cache."""
    return max(1, min(16, -(-2 * MALL_BYTES // max(bytes_per_copy, 1))))


class Case:
    def __init__(self, name, flops, nbytes, peak_tflops, bound, launch, rot, note="",
                 format_peak=None):
        self.name, self.flops, self.nbytes = name, flops, nbytes
        self.peak_tflops, self.bound, self.launch, self.rot = peak_tflops, bound, launch, rot
        self.note = note
        # the peak of the data format itself where the kernel runs on a
        # wider MFMA (NVFP4 dequantized to fp16): reported beside frac_mfma
        self.format_peak = format_peak


def build_cases(names, dev):
    import torch

    from dsl_tool_amd import _native as N
    from dsl_tool_amd import moe as MOE
    from dsl_tool_amd import quant as Q
    from dsl_tool_amd import workloads as W

    L = N.lib()
    cases = {}
    gdev = torch.Generator(device=dev)

    def rnd(shape, seed, std=1.0):
        gdev.manual_seed(seed)
        return (torch.randn(shape, generator=gdev, device=dev) * std).to(torch.bfloat16)

    def ws_for(op, m, n, k):
        nb = L.dsl_gemm_workspace_bytes(op, m, n, k)
        return torch.empty(max(nb, 16) // 4, dtype=torch.float32, device=dev), nb

    def fp8_case(name, m, n, k, block, a_bf16=None, w_bf16=None, group=False):
        a = a_bf16.to(dev) if a_bf16 is not None else rnd((m, k), 1)
        w = w_bf16.to(dev) if w_bf16 is not None else rnd((n, k), 2, 0.02)
        if group:      # the reference groupwise layout: sb [K/128][N] per output column
            qa, sa = Q.quant_fp8_blocks(a, 1, 128)
            qw, swr = Q.quant_fp8_blocks(w, 1, 128)
            sw = swr.t().contiguous()
        elif block:
            qa, sa = Q.quant_fp8_blocks(a, 1, 128)
            qw, sw = Q.quant_fp8_blocks(w, 128, 128)
        else:
            qa, sa = Q.quant_fp8_tensor(a)
            qw, sw = Q.quant_fp8_tensor(w)
        del a, w
        wbytes = qw.numel() + sw.numel() * 4
        rot = _rotations(wbytes) if m <= 256 else 1
        qws = [qw] + [qw.clone() for _ in range(rot - 1)]
        c = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        ws, nb = ws_for(N.OP_FP8, m, n, k)
        mode = N.SCALE_GROUP128 if group else (N.SCALE_BLOCK128 if block else N.SCALE_TENSOR)

        def launch(i, stream):
            return L.dsl_fp8_gemm(qa.data_ptr(), qws[i % rot].data_ptr(), c.data_ptr(), m, n, k,
                                  n, N.OUT_BF16, mode, sa.data_ptr(), sw.data_ptr(),
                                  ws.data_ptr(), nb, stream)
        nbytes = qa.numel() + wbytes + sa.numel() * 4 + 2 * m * n
        bound = "hbm" if 2 * m * n * k / nbytes < PEAK_FP8_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9) else "mfma"
        kind = ("1x128 / per-column 128x1 groupwise (scale_b [K/128][N])" if group
                else ("1x128/128x128 block" if block else "per-tensor"))
        return Case(name, 2.0 * m * n * k, nbytes, PEAK_FP8_TFLOPS, bound, launch, rot,
                    f"fp8 {kind} M={m} N={n} K={k}")

    def fp4_case(name, m, n, k, fmt):
        a, w = rnd((m, k), 3), rnd((n, k), 4, 0.02)
        if fmt == "mxfp4":
            qa, sa = Q.quant_mxfp4(a)
            qw, sw = Q.quant_mxfp4(w)
            ga = gw = None
            code = N.FMT_MXFP4
        else:
            qa, sa, ga = Q.quant_nvfp4(a)
            qw, sw, gw = Q.quant_nvfp4(w)
            code = N.FMT_NVFP4
        del a, w
        wbytes = qw.numel() + sw.numel()
        rot = _rotations(wbytes) if m <= 256 else 1
        pairs = [(qw, sw)] + [(qw.clone(), sw.clone()) for _ in range(rot - 1)]
        c = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        ws, nb = ws_for(N.OP_FP4, m, n, k)
        gap = ga.data_ptr() if ga is not None else None
        gwp = gw.data_ptr() if gw is not None else None

        def launch(i, stream):
            w_, s_ = pairs[i % rot]
            return L.dsl_fp4_gemm(qa.data_ptr(), w_.data_ptr(), c.data_ptr(), m, n, k, n,
                                  N.OUT_BF16, code, sa.data_ptr(), s_.data_ptr(), gap, gwp,
                                  ws.data_ptr(), nb, stream)
        nbytes = qa.numel() + sa.numel() + wbytes + 2 * m * n
        peak = PEAK_FP4_TFLOPS if fmt == "mxfp4" else PEAK_FP16_TFLOPS
        ridge = peak * 1e12 / (PEAK_HBM_GBS * 1e9)
        bound = "hbm" if 2 * m * n * k / nbytes < ridge else "mfma"
        return Case(name, 2.0 * m * n * k, nbytes, peak, bound, launch, rot,
                    f"{fmt} M={m} N={n} K={k}" + ("" if fmt == "mxfp4" else
                                                   " (frac_mfma of the fp16 MFMA peak it runs on, "
                                                   "frac_fp4 of the FP4 peak)"),
                    format_peak=None if fmt == "mxfp4" else PEAK_FP4_TFLOPS)

    def bf16_case(name, m, n, k):
        a, w = rnd((m, k), 6), rnd((n, k), 7, 0.02)
        wbytes = 2 * n * k
        rot = _rotations(wbytes) if m <= 256 else 1
        ws_ = [w] + [w.clone() for _ in range(rot - 1)]
        c = torch.empty((m, n), dtype=torch.float32, device=dev)
        ws, nb = ws_for(N.OP_BF16, m, n, k)

        def launch(i, stream):
            return L.dsl_bf16_gemm(a.data_ptr(), ws_[i % rot].data_ptr(), c.data_ptr(), m, n, k, n,
                                   N.OUT_F32, ws.data_ptr(), nb, stream)
        nbytes = 2 * m * k + wbytes + 4 * m * n
        ridge = PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
        bound = "hbm" if 2 * m * n * k / nbytes < ridge else "mfma"
        return Case(name, 2.0 * m * n * k, nbytes, PEAK_BF16_TFLOPS, bound, launch, rot,
                    f"bf16 M={m} N={n} K={k}, fp32 out (bf16 MFMA peak)")

    def grouped_case(name, tokens=4096):
        """Config 5's grouped GEMM; with few tokens (MoE decode) it streams the
        non-empty experts' weights and is HBM-bound."""
        x, w, offsets, counts = W.moe_problem(tokens=tokens)
        T, K = x.shape
        E, Nn, _ = w.shape
        qx, sx = Q.quant_fp8_blocks(x.to(dev), 1, K)
        qw, sw = Q.quant_fp8_blocks(w.reshape(E * Nn, K).to(dev), 1, K)
        off = offsets.to(dev)
        y = torch.empty((T, Nn), dtype=torch.bfloat16, device=dev)
        # the experts' weights (~190 MB) fit the 256 MB Infinity Cache: rotate
        # copies (> 2 x 256 MB in all) so every launch reads them from HBM
        rot = _rotations(qw.numel())
        qws = [qw] + [qw.clone() for _ in range(rot - 1)]

        def launch(i, stream):
            return L.dsl_grouped_fp8_gemm(qx.data_ptr(), qws[i % rot].data_ptr(), y.data_ptr(),
                                          off.data_ptr(), E, T, Nn, K, Nn, N.OUT_BF16,
                                          sx.data_ptr(), sw.data_ptr(), stream)
        nonempty = int((counts > 0).sum())
        flops = 2.0 * T * Nn * K
        nbytes = T * K + nonempty * Nn * K + 4 * T + 4 * nonempty * Nn + 2 * T * Nn
        return Case(name, flops, nbytes, PEAK_FP8_TFLOPS, "mfma" if tokens >= 1024 else "hbm", launch,
                    rot, f"grouped fp8 MoE E={E} T={T}"
                    + (f" ({tokens} tokens x top-8, decode)" if tokens < 1024 else "")
                    + f" N={Nn} K={K} ({E - nonempty} empty), {rot} weight copies rotated")

    def quant_case(name, kind, r, k, f32=False):
        """One quantize/pack pass over a bf16 (or fp32, the reference's own
        input type) [r, k] operand resident in HBM."""
        x = rnd((r, k), 5, 0.02)
        if f32:
            x = x.float()
        xin, esz = (N.IN_F32, 4) if f32 else (N.IN_BF16, 2)
        ws = torch.empty(L.dsl_quant_workspace_bytes(r, k) // 4, dtype=torch.float32, device=dev)
        if kind == "fp8_block128":
            q = torch.empty((r, k), dtype=torch.uint8, device=dev)
            sc = torch.empty((-(-r // 128), -(-k // 128)), dtype=torch.float32, device=dev)
            out_b, passes = r * k + sc.numel() * 4, 1

            def launch(i, stream):
                return L.dsl_quant_fp8_blocks(x.data_ptr(), r, k, k, 1, xin, 128, 128, q.data_ptr(),
                                              sc.data_ptr(), stream)
        elif kind == "fp8_row128":
            q = torch.empty((r, k), dtype=torch.uint8, device=dev)
            sc = torch.empty((r, -(-k // 128)), dtype=torch.float32, device=dev)
            out_b, passes = r * k + sc.numel() * 4, 1

            def launch(i, stream):
                return L.dsl_quant_fp8_blocks(x.data_ptr(), r, k, k, 1, xin, 1, 128, q.data_ptr(),
                                              sc.data_ptr(), stream)
        elif kind == "fp8_tensor":
            q = torch.empty((r, k), dtype=torch.uint8, device=dev)
            sc = torch.empty(1, dtype=torch.float32, device=dev)
            out_b, passes = r * k + 4, 2

            def launch(i, stream):
                return L.dsl_quant_fp8_tensor(x.data_ptr(), r, k, k, 1, xin, q.data_ptr(), sc.data_ptr(),
                                              ws.data_ptr(), ws.numel() * 4, stream)
        elif kind == "mxfp4":
            q = torch.empty((r, k // 2), dtype=torch.uint8, device=dev)
            sc = torch.empty((r, k // 32), dtype=torch.uint8, device=dev)
            out_b, passes = r * k // 2 + r * k // 32, 1

            def launch(i, stream):
                return L.dsl_quant_mxfp4(x.data_ptr(), r, k, k, 1, xin, q.data_ptr(), sc.data_ptr(),
                                         stream)
        else:
            q = torch.empty((r, k // 2), dtype=torch.uint8, device=dev)
            sc = torch.empty((r, k // 16), dtype=torch.uint8, device=dev)
            g = torch.empty(1, dtype=torch.float32, device=dev)
            out_b, passes = r * k // 2 + r * k // 16 + 4, 2

            def launch(i, stream):
                return L.dsl_quant_nvfp4(x.data_ptr(), r, k, k, 1, xin, q.data_ptr(), sc.data_ptr(),
                                         g.data_ptr(), ws.data_ptr(), ws.numel() * 4, stream)
        nbytes = passes * esz * r * k + out_b
        return Case(name, 0.0, nbytes, PEAK_FP8_TFLOPS, "hbm", launch, 1,
                    f"quantize {kind} [{r}, {k}] {'fp32' if f32 else 'bf16'} "
                    f"({passes} read pass{'es' if passes > 1 else ''})")

    def lora_case(name, m, n, k, r, l):
        x, w = rnd((m, k), 11), rnd((n, k), 12, 0.05)
        a_t, b_t = rnd((l * r, k), 13, 0.05), rnd((n, l * r), 14, 0.05)
        s = torch.linspace(0.5, 2.0, l, device=dev)
        y = torch.empty((m, n), dtype=torch.float32, device=dev)
        nb = L.dsl_lora_gemm_workspace_bytes(m, n, k, r, l)
        ws = torch.empty(max(nb, 256) // 4, dtype=torch.float32, device=dev)

        def launch(i, stream):
            return L.dsl_lora_gemm(x.data_ptr(), w.data_ptr(), a_t.data_ptr(), b_t.data_ptr(),
                                   s.data_ptr(), y.data_ptr(), m, n, k, r, l, n, ws.data_ptr(), nb,
                                   stream)
        flops = 2.0 * m * n * k + 2.0 * m * k * l * r + 2 * 2.0 * m * l * r * n
        nbytes = 2 * m * k + 2 * n * k + 2 * l * r * (k + n) + 4 * m * n
        return Case(name, flops, nbytes, PEAK_BF16_TFLOPS, "mfma", launch, 1,
                    f"LoRA fused GEMM M={m} N={n} K={k}, {l} adapters of rank {r}, fp32 out")

    def moe_case(name, stage, tokens=4096):
        """BASELINE config 5 routing (4096 tokens, top-8 of 64 experts,
        K=2048, N=1536) through the MoE glue: one stage, or the whole
        projection route -> permute + quantize -> grouped GEMM -> combine.
        With few tokens (decode) the experts' weights rotate over copies past
        the Infinity Cache and the step is timed as a captured graph."""
        ids, wts = W.moe_routing(tokens=tokens)
        T, k = ids.shape
        E, Nn, K = 64, 1536, 2048
        ids, wts = ids.to(dev), wts.to(dev)
        x = rnd((T, K), 9)
        w = rnd((E * Nn, K), 10, 0.02)
        qw, sw = Q.quant_fp8_blocks(w, 1, K)
        del w
        decode = tokens < 1024
        # every stage that runs the grouped GEMM reads its weights from
        # copies rotated past the Infinity Cache (the layer as well as the
        # grouped stage alone, so the two are timed on the same footing)
        rot = _rotations(qw.numel()) if stage.startswith(("grouped", "layer")) else 1
        qws = [qw] + [qw.clone() for _ in range(rot - 1)]
        rows = T * k
        off = torch.empty(E + 1, dtype=torch.int32, device=dev)
        dest = torch.empty(rows, dtype=torch.int32, device=dev)
        src = torch.empty(rows, dtype=torch.int32, device=dev)
        nbw = L.dsl_moe_route_workspace_bytes(T, k, E)
        rws = torch.empty(max(nbw, 4) // 4, dtype=torch.int32, device=dev)
        # the permuted copy, or (gather form) token-major codes read through
        # the row map
        gather = MOE.gather_applies(T, k, E, K)
        qx = torch.empty((rows, K), dtype=torch.uint8, device=dev)
        qt = torch.empty((T, K), dtype=torch.uint8, device=dev)
        sx = torch.empty(rows, dtype=torch.float32, device=dev)
        y = torch.empty((rows, Nn), dtype=torch.bfloat16, device=dev)
        out = torch.empty((T, Nn), dtype=torch.bfloat16, device=dev)

        def route(st):
            return L.dsl_moe_route(ids.data_ptr(), T, k, E, off.data_ptr(), dest.data_ptr(),
                                   src.data_ptr(), rws.data_ptr(), nbw, st)

        def permute(st):
            return L.dsl_moe_permute_quant(x.data_ptr(), T, K, K, dest.data_ptr(), k, rows,
                                           qx.data_ptr(), sx.data_ptr(), st)

        def quant_tokens(st):
            return L.dsl_moe_quant_tokens(x.data_ptr(), T, K, K, dest.data_ptr(), k, rows,
                                          qt.data_ptr(), sx.data_ptr(), st)

        # decode sizes: route and per-token quantize in one launch
        fused = gather and MOE.route_quant_applies(T, k, E, K)

        def route_quant(st):
            return L.dsl_moe_route_quant_tokens(ids.data_ptr(), T, k, E, x.data_ptr(), K, K,
                                                off.data_ptr(), dest.data_ptr(), src.data_ptr(),
                                                qt.data_ptr(), sx.data_ptr(), st)

        it = [0]

        def grouped(st):
            it[0] += 1
            return L.dsl_grouped_fp8_gemm(qx.data_ptr(), qws[it[0] % rot].data_ptr(), y.data_ptr(),
                                          off.data_ptr(), E, rows, Nn, K, Nn, N.OUT_BF16, sx.data_ptr(),
                                          sw.data_ptr(), st)

        def grouped_gather(st):
            it[0] += 1
            return L.dsl_moe_grouped_fp8_gemm(qt.data_ptr(), T, src.data_ptr(), qws[it[0] % rot].data_ptr(),
                                              y.data_ptr(), off.data_ptr(), E, rows, Nn, K, Nn,
                                              N.OUT_BF16, sx.data_ptr(), sw.data_ptr(), st)

        def combine(st):
            return L.dsl_moe_combine(y.data_ptr(), rows, Nn, Nn, dest.data_ptr(), wts.data_ptr(), T, k,
                                     out.data_ptr(), Nn, N.OUT_BF16, st)
        s0 = torch.cuda.current_stream().cuda_stream
        # tables and buffers valid before timing
        for f in ((route, permute, grouped, quant_tokens) + ((grouped_gather,) if gather else ())
                  + ((route_quant,) if fused else ()) + (combine,)):
            assert f(s0) == 0
        stages = {"route": [route], "permute": [permute], "quant_tokens": [quant_tokens],
                  "combine": [combine], "grouped": [grouped], "grouped_gather": [grouped_gather],
                  "layer": ([route_quant, grouped_gather, combine] if fused
                            else [route, quant_tokens, grouped_gather, combine]) if gather
                  else [route, permute, grouped, combine],
                  "layer_permuted": [route, permute, grouped, combine]}[stage]

        def launch(i, stream):
            for f in stages:
                rc = f(stream)
                if rc:
                    return rc
            return 0
        counts = W.moe_counts(tokens=tokens)
        nonempty = int((counts > 0).sum())
        flops = 2.0 * rows * Nn * K if stage in ("layer", "layer_permuted", "grouped",
                                                 "grouped_gather") else 0.0
        nbytes = {"route": 4 * rows * 3 + 4 * (E + 1),
                  "permute": 2 * T * K + rows * K + 4 * rows * 2,
                  "quant_tokens": 2 * T * K + T * K + 4 * rows * 2,
                  "grouped": rows * K + nonempty * Nn * K + 4 * rows + 4 * nonempty * Nn + 2 * rows * Nn,
                  "grouped_gather": T * K + 4 * rows + nonempty * Nn * K + 4 * rows
                                    + 4 * nonempty * Nn + 2 * rows * Nn,
                  "combine": 2 * rows * Nn + 4 * rows * 2 + 2 * T * Nn,
                  "layer": 2 * T * K + nonempty * Nn * K + 2 * T * Nn,
                  "layer_permuted": 2 * T * K + nonempty * Nn * K + 2 * T * Nn}[stage]
        what = {"route": "MoE route (stable counting sort) of 4096x8 ids over 64 experts",
                "permute": "MoE permute + per-row E4M3: 4096 tokens quantized once, K=2048, "
                           "scattered to their 32768 routed rows",
                "quant_tokens": "MoE per-row E4M3 of 4096 tokens in token order, K=2048, scales "
                                "to their 32768 routed rows",
                "combine": "MoE weighted combine of 32768 rows, N=1536 -> 4096 tokens",
                "layer": "MoE projection cfg5: route + per-token E4M3 + grouped FP8 GEMM reading A "
                         f"through the row map + combine, {rot} weight copies rotated",
                "layer_permuted": "MoE projection cfg5 over the permuted copy: route + permute/quant + "
                                  f"grouped FP8 GEMM + combine, {rot} weight copies rotated",
                "grouped": f"grouped FP8 GEMM of the routed rows (permuted copy), {rot} weight copies "
                           "rotated",
                "grouped_gather": f"grouped FP8 GEMM of the routed rows, A read through the row map "
                                  f"from 4096 token-major rows, {rot} weight copies rotated"}[stage]
        if decode:
            glue = ("route + per-token E4M3 in one launch + grouped FP8 GEMM reading A through "
                    "the row map" if stage == "layer" and fused else
                    "route + per-token E4M3 + grouped FP8 GEMM reading A through the row map"
                    if stage == "layer" and gather else "route + permute/quant + grouped FP8 GEMM")
            what = (f"MoE projection at decode size ({tokens} tokens x top-8 over 64 experts, N=1536 "
                    f"K=2048): {glue} + combine, {rot} weight copies rotated"
                    ) if stage.startswith("layer") else what.replace("4096", str(tokens)).replace(
                        "32768", str(rows))
        return Case(name, flops, nbytes, PEAK_FP8_TFLOPS,
                    "mfma" if flops and not decode else "hbm", launch, rot, what)

    def producer_case(name, kind, r, c, fused=True):
        """RMSNorm / SwiGLU with the output quantized to FP8 1x128 groups:
        fused (one launch, x read once, codes written) or unfused (the
        operator writes bf16 y, then the activation quantizer reads it)."""
        ncol_in = 2 * c if kind == "swiglu" else c
        x = rnd((r, ncol_in), 8)
        w = torch.ones(c, dtype=torch.bfloat16, device=dev)
        q = torch.empty((r, c), dtype=torch.uint8, device=dev)
        sc = torch.empty((r, -(-c // 128)), dtype=torch.float32, device=dev)
        y = torch.empty((r, c), dtype=torch.bfloat16, device=dev)
        yp = 0 if fused else y.data_ptr()

        def produce(stream):
            if kind == "rmsnorm":
                return L.dsl_rmsnorm_quant(x.data_ptr(), r, c, ncol_in, w.data_ptr(), N.W_BF16,
                                           1e-6, N.QFMT_FP8_G128, q.data_ptr(), sc.data_ptr(),
                                           yp or None, c, stream)
            return L.dsl_swiglu_quant(x.data_ptr(), r, c, ncol_in, N.QFMT_FP8_G128, q.data_ptr(),
                                      sc.data_ptr(), yp or None, c, stream)

        def launch(i, stream):
            rc = produce(stream)
            if rc or fused:
                return rc
            return L.dsl_quant_fp8_blocks(y.data_ptr(), r, c, c, 1, 0, 1, 128, q.data_ptr(),
                                          sc.data_ptr(), stream)
        out_b = r * c + sc.numel() * 4
        nbytes = 2 * r * ncol_in + 2 * c + out_b if fused else 2 * r * ncol_in + 2 * c + 4 * r * c + out_b
        return Case(name, 0.0, nbytes, PEAK_FP8_TFLOPS, "hbm", launch, 1,
                    f"{kind} [{r}, {ncol_in}] -> FP8 1x128, {'fused' if fused else 'unfused (bf16 y, then quantize)'}")

    builders = {
        "fp8_block_m4096": lambda: fp8_case("fp8_block_m4096", 4096, 7168, 4096, True,
                                            W.activations(2, 4096, 4096, outliers=True),
                                            W.weights(2, 7168, 4096)),
        "fp8_block_m16": lambda: fp8_case("fp8_block_m16", 16, 7168, 4096, True),
        "fp8_group_m4096": lambda: fp8_case("fp8_group_m4096", 4096, 7168, 4096, False,
                                            W.activations(2, 4096, 4096, outliers=True),
                                            W.weights(2, 7168, 4096), group=True),
        "fp8_group_m16": lambda: fp8_case("fp8_group_m16", 16, 7168, 4096, False, group=True),
        "fp8_tensor_m4096": lambda: fp8_case("fp8_tensor_m4096", 4096, 7168, 4096, False),
        "fp8_tensor_cfg1": lambda: fp8_case("fp8_tensor_cfg1", 128, 4096, 4096, False),
        # mid-size shapes on the 128x128 pipelined tiles (one round of tiles)
        "fp8_tensor_m1024": lambda: fp8_case("fp8_tensor_m1024", 1024, 4096, 4096, False),
        "fp8_block_m1024": lambda: fp8_case("fp8_block_m1024", 1024, 4096, 4096, True),
        "fp8_tensor_8192": lambda: fp8_case("fp8_tensor_8192", 8192, 8192, 8192, False),
        "mxfp4_8192": lambda: fp4_case("mxfp4_8192", 8192, 8192, 8192, "mxfp4"),
        "mxfp4_m16": lambda: fp4_case("mxfp4_m16", 16, 8192, 8192, "mxfp4"),
        "nvfp4_m1": lambda: fp4_case("nvfp4_m1", 1, 14336, 4096, "nvfp4"),
        "nvfp4_m2048": lambda: fp4_case("nvfp4_m2048", 2048, 14336, 4096, "nvfp4"),
        "grouped_moe": lambda: grouped_case("grouped_moe"),
        "grouped_moe_decode": lambda: grouped_case("grouped_moe_decode", tokens=32),
        "bf16_8192": lambda: bf16_case("bf16_8192", 8192, 8192, 8192),
        "bf16_m4096": lambda: bf16_case("bf16_m4096", 4096, 7168, 4096),
        "bf16_m16": lambda: bf16_case("bf16_m16", 16, 7168, 4096),
        "bf16_m1536": lambda: bf16_case("bf16_m1536", 1536, 2048, 4096),
        "rmsnorm_quant_fp8": lambda: producer_case("rmsnorm_quant_fp8", "rmsnorm", 4096, 7168),
        "rmsnorm_then_quant_fp8": lambda: producer_case("rmsnorm_then_quant_fp8", "rmsnorm", 4096, 7168,
                                                        fused=False),
        "swiglu_quant_fp8": lambda: producer_case("swiglu_quant_fp8", "swiglu", 4096, 14336),
        "swiglu_then_quant_fp8": lambda: producer_case("swiglu_then_quant_fp8", "swiglu", 4096, 14336,
                                                       fused=False),
        "lora_m4096": lambda: lora_case("lora_m4096", 4096, 4096, 4096, 16, 4),
        "bf16_4096": lambda: bf16_case("bf16_4096", 4096, 4096, 4096),
        "moe_route": lambda: moe_case("moe_route", "route"),
        "moe_permute_quant": lambda: moe_case("moe_permute_quant", "permute"),
        "moe_quant_tokens": lambda: moe_case("moe_quant_tokens", "quant_tokens"),
        "moe_grouped_permuted": lambda: moe_case("moe_grouped_permuted", "grouped"),
        "moe_grouped_gather": lambda: moe_case("moe_grouped_gather", "grouped_gather"),
        "moe_layer_decode": lambda: moe_case("moe_layer_decode", "layer", tokens=32),
        "moe_layer_decode_permuted": lambda: moe_case("moe_layer_decode_permuted", "layer_permuted",
                                                      tokens=32),
        "moe_combine": lambda: moe_case("moe_combine", "combine"),
        "moe_layer_cfg5": lambda: moe_case("moe_layer_cfg5", "layer"),
        "quant_fp8_block128_w": lambda: quant_case("quant_fp8_block128_w", "fp8_block128", 7168, 4096),
        "quant_fp8_row128_a": lambda: quant_case("quant_fp8_row128_a", "fp8_row128", 4096, 4096),
        "quant_fp8_tensor_w": lambda: quant_case("quant_fp8_tensor_w", "fp8_tensor", 4096, 4096),
        "quant_mxfp4_w": lambda: quant_case("quant_mxfp4_w", "mxfp4", 8192, 8192),
        "quant_nvfp4_w": lambda: quant_case("quant_nvfp4_w", "nvfp4", 14336, 4096),
        "quant_fp8_row128_a_f32": lambda: quant_case("quant_fp8_row128_a_f32", "fp8_row128", 4096,
                                                     4096, f32=True),
        "quant_fp8_tensor_w_f32": lambda: quant_case("quant_fp8_tensor_w_f32", "fp8_tensor", 4096,
                                                     4096, f32=True),
        "quant_mxfp4_w_f32": lambda: quant_case("quant_mxfp4_w_f32", "mxfp4", 8192, 8192, f32=True),
        "quant_nvfp4_w_f32": lambda: quant_case("quant_nvfp4_w_f32", "nvfp4", 8192, 8192, f32=True),
    }
    for nm in names:
        cases[nm] = builders[nm]()
    return cases


ALL_CASES = ["fp8_block_m4096", "fp8_block_m16", "fp8_group_m4096", "fp8_group_m16",
             "fp8_tensor_m4096", "fp8_tensor_cfg1", "fp8_tensor_m1024", "fp8_block_m1024",
             "fp8_tensor_8192",
             "mxfp4_8192", "mxfp4_m16", "nvfp4_m1", "nvfp4_m2048", "grouped_moe", "grouped_moe_decode",
             "bf16_8192", "bf16_m4096", "bf16_m16", "bf16_m1536",
             "rmsnorm_quant_fp8", "rmsnorm_then_quant_fp8", "swiglu_quant_fp8", "swiglu_then_quant_fp8",
             "moe_route", "moe_permute_quant", "moe_quant_tokens", "moe_combine", "moe_grouped_permuted",
             "moe_grouped_gather", "moe_layer_cfg5", "moe_layer_decode", "moe_layer_decode_permuted", "lora_m4096", "bf16_4096",
             "quant_fp8_block128_w", "quant_fp8_row128_a", "quant_fp8_tensor_w", "quant_mxfp4_w",
             "quant_nvfp4_w", "quant_fp8_row128_a_f32", "quant_fp8_tensor_w_f32", "quant_mxfp4_w_f32",
             "quant_nvfp4_w_f32"]


def _host_ns():
    """Host timestamps bracketing a timed region, in both clocks a kernel
    trace may use (CLOCK_MONOTONIC and CLOCK_BOOTTIME)."""
    return {"monotonic": time.clock_gettime_ns(time.CLOCK_MONOTONIC),
            "boottime": time.clock_gettime_ns(time.CLOCK_BOOTTIME)}


TRACE_WINDOWS: list = []       # (case, steps, start clocks, end clocks) of each timed region


def time_case(case, steps, warmup, dev, graph):
    """Average step time (ms) over `steps` launches, HIP events on the launch stream."""
    import torch

    from dsl_tool_amd import _native as N

    def run(i, stream):
        rc = case.launch(i, stream)
        if rc != 0:
            raise N.DslError(case.name, rc, N.lib().dsl_last_error().decode())

    stream = torch.cuda.Stream(device=dev)          # default priority
    sp = stream.cuda_stream
    with torch.cuda.stream(stream):
        for i in range(warmup):
            run(i, sp)
    torch.cuda.synchronize(dev)
    # then keep the GPU busy with this case for WARM_MS: the shader clock
    # settles under the power limit within tens of milliseconds, and a case
    # timed right after a different one otherwise measures the transition
    w0 = torch.cuda.Event(enable_timing=True)
    w1 = torch.cuda.Event(enable_timing=True)
    busy = 0.0
    for _ in range(200):
        if busy >= WARM_MS:
            break
        with torch.cuda.stream(stream):
            w0.record(stream)
            for i in range(max(warmup, 1)):
                run(i, sp)
            w1.record(stream)
        torch.cuda.synchronize(dev)
        busy += w0.elapsed_time(w1)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    if graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            cap = torch.cuda.current_stream(dev).cuda_stream
            for i in range(steps):
                run(i, cap)
        torch.cuda.synchronize(dev)
        g.replay()                                    # warm replay
        torch.cuda.synchronize(dev)
        t0 = _host_ns()
        with torch.cuda.stream(stream):
            start.record(stream)
            g.replay()
            end.record(stream)
    else:
        torch.cuda.synchronize(dev)
        t0 = _host_ns()
        with torch.cuda.stream(stream):
            start.record(stream)
            for i in range(steps):
                run(i, sp)
            end.record(stream)
    torch.cuda.synchronize(dev)
    TRACE_WINDOWS.append((case.name, steps, t0, _host_ns()))
    return start.elapsed_time(end) / steps


def _smi_sample(exe: str) -> list:
    """One amd-smi reading per GPU: socket power (W), mean GFX clock over the
    XCDs and the memory clock (MHz)."""
    r = subprocess.run([exe, "metric", "-p", "-c", "--json"], capture_output=True, text=True,
                       timeout=20)
    d = json.loads(r.stdout[r.stdout.index("{"):])

    def num(v):
        v = v.get("value") if isinstance(v, dict) else None
        return float(v) if isinstance(v, (int, float)) else None

    out = []
    for g in d.get("gpu_data", []):
        clk = g.get("clock", {}) or {}
        gfx = [num(v.get("clk")) for k, v in clk.items() if k.startswith("gfx_") and isinstance(v, dict)]
        gfx = [x for x in gfx if x is not None]
        mem = clk.get("mem_0")
        out.append({"power_w": num((g.get("power", {}) or {}).get("socket_power")),
                    "gfx_mhz": sum(gfx) / len(gfx) if gfx else None,
                    "mem_mhz": num(mem.get("clk")) if isinstance(mem, dict) else None})
    return out


def telemetry(case, dev, seconds: float = 3.0):
    """Socket power and clocks while `case` runs back to back (amd-smi sampled
    from a second thread), or None where amd-smi is missing or unreadable.
    Taken after every timed region, so it changes no timing.  With several
    GPUs in the node, the one drawing the most power is reported."""
    import torch

    exe = shutil.which("amd-smi") or "/opt/rocm/bin/amd-smi"
    if not os.path.exists(exe):
        return None
    stream = torch.cuda.Stream(device=dev)          # default priority
    sp = stream.cuda_stream

    def burst(i0, n):
        with torch.cuda.stream(stream):
            for i in range(i0, i0 + n):
                if case.launch(i, sp) != 0:
                    raise RuntimeError(f"telemetry: {case.name} launch failed")
        torch.cuda.synchronize(dev)

    t_warm = time.time() + WARM_MS / 1000.0
    i = 0
    while time.time() < t_warm:                       # settle the clock first
        burst(i, 20)
        i += 20
    samples, stop = [], threading.Event()

    def sampler():
        while not stop.is_set():
            try:
                samples.append(_smi_sample(exe))
            except Exception:                         # unreadable: report what was read
                return

    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    t_end = time.time() + seconds
    while th.is_alive() and (time.time() < t_end or len(samples) < 3) and time.time() < t_end + 20:
        burst(i, 20)
        i += 20
    stop.set()
    th.join(timeout=30)
    samples = [s_ for s_ in samples if s_]
    if not samples:
        return None
    ng = min(len(s_) for s_ in samples)

    def mean(vals):
        vals = [v for v in vals if v is not None]
        return round(sum(vals) / len(vals), 1) if vals else None

    per_gpu = [{k: mean([s_[g][k] for s_ in samples]) for k in ("power_w", "gfx_mhz", "mem_mhz")}
               for g in range(ng)]
    busy = max(per_gpu, key=lambda x: x["power_w"] or 0.0)
    return {"case": case.name, "samples": len(samples), "socket_power_w": busy["power_w"],
            "gfx_clock_mhz": busy["gfx_mhz"], "mem_clock_mhz": busy["mem_mhz"],
            "source": "amd-smi metric -p -c --json, sampled while the case runs back to back "
                      "after the timed regions"}


TRACE_FILE = os.path.join(ROOT, "profiles", "bench_default_kernel_trace.txt")


def read_trace_medians(path: str = TRACE_FILE) -> dict:
    """case -> (kernel, median us) of the case's main kernel in the committed
    kernel-trace summary (an earlier profiled run of this bench), or {}."""
    import re
    out, case = {}, None
    try:
        lines = open(path).read().splitlines()
    except OSError:
        return out
    for line in lines:
        m = re.match(r"case (\S+): ", line)
        if m:
            case = m.group(1)
            continue
        m = re.match(r"\s+(\S.*?)\s+n=\s*\d+ median\s+([\d.]+)", line)
        if m and case and case not in out:          # kernels are listed by total time
            out[case] = (m.group(1), float(m.group(2)))
    return out


def read_traffic(path: str = TRAFFIC_FILE):
    """HBM bytes per headline launch recorded by the counter runs, or None."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        return None
    return None


def profile_traffic(steps: int) -> int:
    """Workload for the FETCH_SIZE / WRITE_SIZE counter runs: a plain device
    copy of COPY_BYTES (the calibration), then `steps` headline launches."""
    import torch

    dev = torch.device("cuda:0")
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).random_(0, 255)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize(dev)
    case = build_cases([HEADLINE], dev)[HEADLINE]
    s = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(s):
        for i in range(steps):
            rc = case.launch(i, s.cuda_stream)
            if rc != 0:
                raise RuntimeError(f"headline launch failed with status {rc}")
    torch.cuda.synchronize(dev)
    log(f"profile-traffic: 3 copies of {COPY_BYTES} bytes, {steps} headline launches")
    return 0


# Kernels profiled with hardware counters: the headline, the north-star
# targets (FP8 and MXFP4 8192^3, decode M=16), the grouped MoE GEMM and
# BASELINE config 1.
PROFILE_CASES = ["fp8_block_m4096", "fp8_tensor_8192", "mxfp4_8192", "grouped_moe",
                 "fp8_block_m16", "mxfp4_m16", "fp8_tensor_cfg1", "fp8_group_m4096",
                 "nvfp4_m2048"]
PROFILE_PASSES = [
    ["MfmaUtil", "GRBM_GUI_ACTIVE", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_LDS",
     "SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_INSTS_VALU_MFMA_MOPS_F8",
     "SQ_INSTS_VALU_MFMA_MOPS_F6F4"],
    ["FETCH_SIZE"],
    ["WRITE_SIZE", "TCC_HIT_sum", "TCC_MISS_sum"],
    ["TCP_TCC_READ_REQ_sum", "TCP_TCC_READ_REQ_LATENCY_sum"],
]


def profile_counters(steps: int) -> int:
    """Workload for the ``rocprofv3 --pmc`` passes: the calibration copy,
    then for each PROFILE_CASES entry `steps` launches bracketed by two
    one-element fill kernels that mark where the case's dispatches begin and
    end in the counter CSV."""
    import torch

    dev = torch.device("cuda:0")
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).random_(0, 255)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    del src, dst
    marker = torch.empty(1, dtype=torch.int64, device=dev)   # FillFunctor<long> dispatches
    torch.cuda.synchronize(dev)
    for i, nm in enumerate(PROFILE_CASES):
        case = build_cases([nm], dev)[nm]
        torch.cuda.synchronize(dev)
        marker.fill_(i + 1)
        s = torch.cuda.Stream(device=dev)
        with torch.cuda.stream(s):
            for j in range(steps):
                rc = case.launch(j, s.cuda_stream)
                if rc != 0:
                    raise RuntimeError(f"{nm}: launch failed with status {rc}")
        torch.cuda.synchronize(dev)
        marker.fill_(-(i + 1))
        torch.cuda.synchronize(dev)
        log(f"profile-counters: {nm}, {steps} launches")
        del case
        torch.cuda.empty_cache()
    return 0


def _counter_rows(csv_dir: str):
    """{dispatch id: (kernel name, {counter: value})} from a rocprofv3 csv dir."""
    import csv
    import glob

    files = glob.glob(os.path.join(csv_dir, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise FileNotFoundError(f"no counter_collection.csv under {csv_dir}")
    out = {}
    for row in csv.DictReader(open(files[0])):
        d = int(row["Dispatch_Id"])
        name, vals = out.setdefault(d, (row["Kernel_Name"], {}))
        vals[row["Counter_Name"]] = vals.get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
    return out


def summarize_counters(dirs, commands) -> int:
    """Write profiles/<case>_counters.txt from the PROFILE_PASSES csv dirs:
    per case, the mean over its launches (the first one dropped) of every
    counter, with FETCH_SIZE / WRITE_SIZE scaled by what they read for the
    256 MiB calibration copy."""
    import statistics

    per_case = {nm: {} for nm in PROFILE_CASES}
    kname = {}
    calib = {}
    for d in dirs:
        rows = _counter_rows(d)
        ids = sorted(rows)
        marks = [i for i in ids if "FillFunctor<long" in rows[i][0]]
        # calibration: the three copies before the first marker
        first = marks[0] if marks else ids[-1]
        copies = [i for i in ids if i < first and "copy" in rows[i][0].lower()][:3]
        for cn in ("FETCH_SIZE", "WRITE_SIZE"):
            vals = [rows[i][1][cn] for i in copies if cn in rows[i][1]]
            if vals:
                calib[cn] = (COPY_BYTES / 1024.0) / statistics.mean(vals[1:] or vals)
        for c, nm in enumerate(PROFILE_CASES):
            if 2 * c + 1 >= len(marks):
                break
            lo, hi = marks[2 * c], marks[2 * c + 1]
            disp = [i for i in ids if lo < i < hi]
            if not disp:
                continue
            main = max(set(rows[i][0] for i in disp), key=lambda k: sum(rows[i][0] == k for i in disp))
            kname[nm] = main
            use = [i for i in disp if rows[i][0] == main]
            use = use[1:] or use
            for cn in rows[use[0]][1]:
                per_case[nm][cn] = statistics.mean(rows[i][1][cn] for i in use)
    os.makedirs(os.path.join(ROOT, "profiles"), exist_ok=True)
    for nm, vals in per_case.items():
        if not vals:
            continue
        lines = [f"# {nm}: hardware counters of its main kernel, mean per launch",
                 f"# kernel: {kname.get(nm, '?')}",
                 "# commands (run from the repository root on one MI355X):"]
        lines += [f"#   {c}" for c in commands]
        lines.append("")
        for cn in sorted(vals):
            lines.append(f"{cn}: {vals[cn]:.6g}")
        fs, ws = vals.get("FETCH_SIZE"), vals.get("WRITE_SIZE")
        if fs is not None and "FETCH_SIZE" in calib:
            lines.append(f"hbm_read_bytes (FETCH_SIZE x {calib['FETCH_SIZE']:.4f}, the factor that "
                         f"maps a {COPY_BYTES >> 20} MiB device copy to its true bytes): "
                         f"{fs * 1024 * calib['FETCH_SIZE']:.4g}")
        if ws is not None and "WRITE_SIZE" in calib:
            lines.append(f"hbm_write_bytes (WRITE_SIZE x {calib['WRITE_SIZE']:.4f}): "
                         f"{ws * 1024 * calib['WRITE_SIZE']:.4g}")
        if "TCC_HIT_sum" in vals and "TCC_MISS_sum" in vals:
            tot = vals["TCC_HIT_sum"] + vals["TCC_MISS_sum"]
            lines.append(f"l2_hit_rate: {vals['TCC_HIT_sum'] / tot:.4f}" if tot else "l2_hit_rate: -")
        if vals.get("TCP_TCC_READ_REQ_sum"):
            lines.append(f"l1_to_l2_read_latency_cycles (LATENCY_sum / READ_REQ_sum): "
                         f"{vals.get('TCP_TCC_READ_REQ_LATENCY_sum', 0) / vals['TCP_TCC_READ_REQ_sum']:.1f}")
        if vals.get("SQ_LDS_IDX_ACTIVE"):
            lines.append(f"lds_bank_conflict_ratio (SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE): "
                         f"{vals.get('SQ_LDS_BANK_CONFLICT', 0) / vals['SQ_LDS_IDX_ACTIVE']:.4f}")
        with open(os.path.join(ROOT, "profiles", f"{nm}_counters.txt"), "w") as f:
            f.write("\n".join(lines) + "\n")
        log(f"wrote profiles/{nm}_counters.txt")
        if nm == HEADLINE and fs is not None and ws is not None and "FETCH_SIZE" in calib \
                and "WRITE_SIZE" in calib:
            rd = fs * 1024 * calib["FETCH_SIZE"]
            wr = ws * 1024 * calib["WRITE_SIZE"]
            t = ["# HBM traffic of the headline kernel (fp8 block-scaled M=4096 N=7168 K=4096)",
                 f"# kernel: {kname.get(nm, '?')}",
                 f"# from the FETCH_SIZE / WRITE_SIZE passes of profiles/{nm}_counters.txt "
                 "(commands there)",
                 f"hbm_read_bytes: {rd:.0f}", f"hbm_write_bytes: {wr:.0f}",
                 f"algorithmic_bytes: {HEADLINE_BYTES}",
                 f"measured_over_algorithmic: {(rd + wr) / HEADLINE_BYTES:.3f}",
                 f"traffic_bytes_per_launch: {int(round(rd + wr))}"]
            with open(TRAFFIC_FILE, "w") as f:
                f.write("\n".join(t) + "\n")
            log(f"wrote {os.path.relpath(TRAFFIC_FILE, ROOT)}")
    return 0


def summarize_trace(trace_dir: str, bench_log: str, windows: str, command: str) -> int:
    """Write profiles/bench_default_kernel_trace.txt from a rocprofv3
    --kernel-trace --stats csv dir of a bench run, that run's stderr and its
    --trace-windows file: per case, the dispatches that ran inside the
    case's timed region (host clock bounds; warm-up launches excluded), their
    count and median duration per kernel, and for the headline the roofline
    fraction recomputed from that median beside the one the bench line
    reported from HIP events."""
    import csv
    import glob
    import re
    import statistics

    trace = glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True)
    rows = list(csv.DictReader(open(trace[0])))
    disp = []
    for r in rows:
        n = r.get("Kernel_Name") or r.get("Name") or ""
        if "dsl::" not in n:
            continue
        n = re.sub(r"\(.*\)$", "", n.replace("void ", ""))
        disp.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), n))
    wins = [json.loads(line) for line in open(windows) if line.strip()]
    # the clock the trace uses: the one under which the most dispatches fall
    # inside some window
    def inside(clock):
        return sum(1 for s0, e0, _ in disp
                   for w in wins if w["t0"][clock] <= s0 and e0 <= w["t1"][clock])
    clock = max(("monotonic", "boottime"), key=inside)
    text = open(bench_log).read()
    bench_us = {c[0]: float(c[1]) for c in
                re.findall(r"\[bench\] case (\S+): \{'us': ([\d.]+)", text)}
    whats = dict(re.findall(r"\[bench\] case (\S+): \{.*?'what': '([^']*)'", text))
    out = ["# rocprofv3 kernel-trace summary: default bench run (all cases)",
           f"# command (run from the repository root on one MI355X): {command}",
           f"# dispatches inside each case's timed region ({clock} clock), warm-up excluded;",
           "# median / mean kernel duration in microseconds; bench_us = the case's HIP-event",
           "# time per step in the same run (kernel time plus any launch gaps)", ""]
    head = None
    for w in wins:
        sel = [(e0 - s0) / 1e3 for s0, e0, _ in disp
               if w["t0"][clock] <= s0 and e0 <= w["t1"][clock]]
        per = {}
        for s0, e0, n in disp:
            if w["t0"][clock] <= s0 and e0 <= w["t1"][clock]:
                per.setdefault(n, []).append((e0 - s0) / 1e3)
        out.append(f"case {w['case']}: {w['steps']} timed steps, bench_us "
                   f"{bench_us.get(w['case'], float('nan')):.2f}   ({whats.get(w['case'], '')})")
        for n, d in sorted(per.items(), key=lambda kv: -sum(kv[1])):
            out.append(f"    {n[:110]:110s} n={len(d):4d} median {statistics.median(d):9.2f} "
                       f"mean {statistics.fmean(d):9.2f}")
        if w["case"] == HEADLINE and per:
            main = max(per.items(), key=lambda kv: sum(kv[1]))
            head = (main[0], statistics.median(main[1]), len(sel))
    if head:
        flops = 2.0 * 4096 * 7168 * 4096
        frac_trace = flops / (head[1] * 1e-6) / 1e12 / PEAK_FP8_TFLOPS
        frac_bench = flops / (bench_us[HEADLINE] * 1e-6) / 1e12 / PEAK_FP8_TFLOPS
        out += ["", f"headline kernel {head[0]}: median {head[1]:.2f} us over its timed launches "
                f"-> roofline frac {frac_trace:.4f}; the bench line's frac from HIP events "
                f"{frac_bench:.4f} (ratio {frac_bench / frac_trace:.4f})"]
    with open(os.path.join(ROOT, "profiles", "bench_default_kernel_trace.txt"), "w") as f:
        f.write("\n".join(out) + "\n")
    log("wrote profiles/bench_default_kernel_trace.txt")
    return 0


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def _repeat(fn, min_seconds: float):
    """Run fn until at least min_seconds of it have been timed: (out, runs, seconds)."""
    reps, dt, out = 0, 0.0, None
    while reps == 0 or dt < min_seconds:
        t0 = time.perf_counter()
        out = fn()
        dt += time.perf_counter() - t0
        reps += 1
    return out, reps, dt


def cpu_baseline(sample_rows: int, min_seconds: float = 10.0, leg_seconds: float = 5.0):
    """CPU paths timed on the host's cores, each repeated until enough CPU
    work is timed (mean rate):

    * the headline: the oracle (dequantize -> fp32 CPU matmul -> bf16) on
      the M=4096 block-scaled workload restricted to its first `sample_rows`
      activation rows (``value``);
    * ``legs``: the reference's own CPU path restated tile for tile
      (64x64x32 tiles, fp32 accumulation, tilelang/gemm/gemm_kernels.py:
      96-113 and :116-133), on BASELINE config 1 in full and on a sample of
      config 5's expert groups.

    The tiled legs' operand codes come from the GPU quantizers (bit-exact
    with the oracle's, tests/test_gpu_quant_fullsize.py) to keep the setup
    short; only the CPU GEMMs are timed."""
    import numpy as np
    import torch

    from dsl_tool_amd import quant as Q
    from dsl_tool_amd import workloads as W
    from oracle import gemm as OG
    from oracle import quant as OQ

    m, n, k = sample_rows, 7168, 4096
    a = W.activations(2, 4096, 4096, outliers=True)[:m].float().numpy()
    w = W.weights(2, n, k).float().numpy()
    qa, sa = OQ.quant_fp8_blockwise(a, 1, 128)
    qw, sw = OQ.quant_fp8_blockwise(w, 128, 128)
    out, reps, dt = _repeat(lambda: OG.ref_fp8_groupwise(qa, sa, qw, sw), min_seconds)
    assert np.isfinite(out).all()
    head = {"value": round(reps * 2.0 * m * n * k / dt / 1e12, 5), "unit": "TFLOP/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"oracle ref_fp8_groupwise (numpy dequant + torch fp32 matmul) on rows "
                      f"0..{m - 1} of the M=4096 headline, full N={n} K={k}; {reps} runs, "
                      f"{dt:.1f} s in total",
            "threads": torch.get_num_threads(), "cpu_count": os.cpu_count(),
            "cpu_model": _cpu_model()}
    del a, w, qa, qw, out

    dev = torch.device("cuda:0")
    legs = []
    # config 1 in full: FP8 per-tensor, A [128, 4096], W [4096, 4096]
    a1 = W.activations(1, 128, 4096).to(dev)
    w1 = W.weights(1, 4096, 4096).to(dev)
    qa1, sa1 = Q.quant_fp8_tensor(a1)
    qw1, sw1 = Q.quant_fp8_tensor(w1)
    qa1, qw1 = qa1.cpu().numpy(), qw1.cpu().numpy()
    sa1, sw1 = float(sa1.cpu()[0]), float(sw1.cpu()[0])
    _, reps, dt = _repeat(lambda: OG.tiled_fp8_gemm(qa1, qw1, sa1, sw1), leg_seconds)
    legs.append({"value": round(reps * 2.0 * 128 * 4096 * 4096 / dt / 1e12, 6), "unit": "TFLOP/s",
                 "ms_per_gemm": round(dt / reps * 1e3, 2), "kind": "port",
                 "sample": f"tiled_fp8_gemm (64x64x32 tiles, the reference's fp8_gemm_tiled "
                           f"restated) on BASELINE config 1 in full, M=128 N=4096 K=4096; "
                           f"{reps} runs, {dt:.1f} s"})
    del a1, w1
    # config 5: grouped MoE, per-row / per-channel E4M3, a sample of the groups
    x5, w5, off5, _ = W.moe_problem(5)
    e5, n5, k5 = w5.shape
    qx, sx = Q.quant_fp8_blocks(x5.to(dev), 1, k5)
    qw5, sw5 = Q.quant_fp8_blocks(w5.reshape(e5 * n5, k5).to(dev), 1, k5)
    qx, sx = qx.cpu().numpy(), sx.cpu().numpy()[:, 0]
    qw5, sw5 = qw5.cpu().numpy().reshape(e5, n5, k5), sw5.cpu().numpy().reshape(e5, n5)
    off = off5.numpy()
    groups, rows = [], 0
    for g in reversed(range(e5)):          # the smallest (last Zipf-rank) non-empty groups, >= 512 rows
        cnt = int(off[g + 1] - off[g])
        if cnt and rows < 512:
            groups.append(g)
            rows += cnt
    groups.sort()
    _, reps, dt = _repeat(lambda: OG.tiled_grouped_fp8_gemm(qx, sx, qw5, sw5, off, groups=groups),
                          leg_seconds)
    legs.append({"value": round(reps * 2.0 * rows * n5 * k5 / dt / 1e12, 6), "unit": "TFLOP/s",
                 "ms_per_gemm": round(dt / reps * 1e3, 2), "kind": "port",
                 "sample": f"tiled_grouped_fp8_gemm (64x64x32 tiles per group, the reference's "
                           f"grouped_gemm_tiled restated) on config 5 groups {groups} "
                           f"({rows} of {int(off[-1])} routed rows), N={n5} K={k5}; "
                           f"{reps} runs, {dt:.1f} s"})
    head["legs"] = legs
    return head


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cases", default="all",
                    help="comma list of extra cases, 'all' or 'none' (headline always runs)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-telemetry", action="store_true",
                    help="skip the amd-smi power / clock samples of the headline case")
    ap.add_argument("--cpu-rows", type=int, default=4096)
    ap.add_argument("--profile-traffic", action="store_true",
                    help="run only the copy calibration and headline launches for rocprofv3 --pmc")
    ap.add_argument("--profile-counters", action="store_true",
                    help="run the copy calibration and launches of each counter-profiled case")
    ap.add_argument("--summarize-counters", nargs="+", metavar="CSV_DIR",
                    help="write profiles/<case>_counters.txt from rocprofv3 --pmc output dirs")
    ap.add_argument("--commands", nargs="*", default=[],
                    help="with --summarize-counters: the commands to record in the summaries")
    ap.add_argument("--summarize-trace", nargs=3, metavar=("TRACE_DIR", "BENCH_LOG", "WINDOWS"),
                    help="write profiles/bench_default_kernel_trace.txt from a kernel-trace run, "
                         "its stderr and its --trace-windows file")
    ap.add_argument("--trace-windows", metavar="FILE",
                    help="write each case's timed region (host clock bounds) to FILE as JSON lines")
    args = ap.parse_args(argv)
    if args.summarize_counters:
        return summarize_counters(args.summarize_counters, args.commands)
    if args.summarize_trace:
        return summarize_trace(*args.summarize_trace, " ".join(args.commands))
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the quantized GEMM "
              "path has no multi-GPU component in this build", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    from dsl_tool_amd import _native as N
    N.lib()
    if args.profile_traffic:
        return profile_traffic(args.steps)
    if args.profile_counters:
        return profile_counters(args.steps)

    extra = ALL_CASES[1:] if args.cases == "all" else (
        [] if args.cases == "none" else [c for c in args.cases.split(",") if c and c != HEADLINE])
    names = [HEADLINE] + extra
    props = torch.cuda.get_device_properties(dev)
    log(f"device {props.name} CUs={props.multi_processor_count} cases={names}")

    results = {}
    traced = read_trace_medians()
    head_ms, head = None, None
    for nm in names:
        log(f"case {nm}: build")
        case = build_cases([nm], dev)[nm]
        graph = case.bound == "hbm"
        ms = time_case(case, args.steps, args.warmup, dev, graph=graph)
        tflops = case.flops / (ms * 1e-3) / 1e12 if case.flops else 0.0
        gbs = case.nbytes / (ms * 1e-3) / 1e9
        results[nm] = {"us": round(ms * 1e3, 2), "tflops": round(tflops, 1),
                       "frac_mfma": round(tflops / case.peak_tflops, 4),
                       "gbs": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
                       "bound": case.bound, "rot": case.rot, "timing": "graph" if graph else "eager",
                       "what": case.note}
        if case.format_peak:
            results[nm]["frac_fp4"] = round(tflops / case.format_peak, 4)
        if nm in traced:
            # the case's main kernel as the committed rocprofv3 summary
            # timed it (median of its timed launches in that run)
            results[nm]["rocprof_kernel_us"] = traced[nm][1]
        log(f"case {nm}: {results[nm]}")
        if nm == HEADLINE:
            head_ms, head = ms, case
        del case
        torch.cuda.empty_cache()

    tele = None
    if not args.no_telemetry and not args.trace_windows and head_ms is not None:
        log("telemetry")
        try:
            tele = telemetry(head, dev)
        except Exception as e:                        # the measurement stands without it
            log(f"telemetry unavailable: {e}")
        log(f"telemetry: {tele}")
    del head
    torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline(args.cpu_rows)
        log(f"cpu baseline: {cpu}")

    h = results[HEADLINE]
    line = {
        "metric": "TFLOPS & % of MFMA peak (fp8/MXFP4 GEMM); HBM GB/s at decode M=16",
        "value": h["tflops"], "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(head_ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp8_e4m3",
        "data": "synthetic (seeded CPU randn, BASELINE config 2 distributions incl. 0.1% x50 "
                "outliers), quantized on the GPU before timing",
        "config": {"workload": "gemm.fp8_gemm block-scaled (1x128 act, 128x128 weight) "
                               "M=4096 N=7168 K=4096, bf16 out (BASELINE config 2)",
                   "M": 4096, "N": 7168, "K": 4096, "device": props.name,
                   "cus": props.multi_processor_count},
        "roofline": {"bound": "mfma", "achieved": h["tflops"], "peak": PEAK_FP8_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(h["tflops"] / PEAK_FP8_TFLOPS, 4),
                     "traffic": read_traffic()},
        "cpu_baseline": cpu,
        "telemetry": tele,
        "cases": results,
    }
    print(json.dumps(line), flush=True)
    if args.trace_windows:
        with open(args.trace_windows, "w") as f:
            for nm, steps, t0, t1 in TRACE_WINDOWS:
                f.write(json.dumps({"case": nm, "steps": steps, "t0": t0, "t1": t1}) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
