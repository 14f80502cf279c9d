"""Seeded synthetic inputs for the quantized GEMM workloads.

Every tensor is generated on the CPU with ``torch.Generator().manual_seed``
(fp32 ``randn`` -> scaled -> ``.bfloat16()``), so the CPU oracle and the GPU
see identical bytes (CPU and GPU RNG streams differ).  Seeds per config n:
A = 1000n+1, W = 1000n+2, outlier mask = 1000n+3, MoE routing = 1000n+4.

Configs (BASELINE configs[n-1]):
  1  FP8 per-tensor      A [128, 4096] ~N(0,1), W [4096, 4096] ~N(0, .02)
  2  FP8 block-scaled    A [M, 4096] ~N(0,1) with 0.1% of entries x50,
                         W [7168, 4096] ~N(0, .02), M in {16, 4096}
  3  MXFP4               A [M, 8192] ~N(0,1), W [8192, 8192] ~N(0, .02)
  4  NVFP4               A [M, 4096] ~N(0,1), W [14336, 4096] ~N(0, .02)
  5  grouped FP8 MoE     64 experts, 4096 tokens top-8 (Gumbel top-k without
                         replacement over a Zipf(1.2) pmf with 4 seeded
                         experts forced to zero), X [sum n_e, 2048] ~N(0,1),
                         W [64, 1536, 2048] ~N(0, .02)
"""
from __future__ import annotations

import torch

W_STD = 0.02


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(int(seed))


def randn_bf16(shape, seed: int, std: float = 1.0) -> torch.Tensor:
    x = torch.randn(tuple(shape), generator=_gen(seed), dtype=torch.float32)
    if std != 1.0:
        x = x * std
    return x.bfloat16()


def activations(cfg: int, m: int, k: int, outliers: bool = False) -> torch.Tensor:
    x = torch.randn((m, k), generator=_gen(1000 * cfg + 1), dtype=torch.float32)
    if outliers:
        n_out = int(round(0.001 * m * k))
        idx = torch.randperm(m * k, generator=_gen(1000 * cfg + 3))[:n_out]
        x.view(-1)[idx] *= 50.0
    return x.bfloat16()


def weights(cfg: int, n: int, k: int) -> torch.Tensor:
    return randn_bf16((n, k), 1000 * cfg + 2, W_STD)


def moe_routing(num_experts: int = 64, tokens: int = 4096, top_k: int = 8, zipf_s: float = 1.2,
                n_empty: int = 4, seed: int = 5004):
    """Seeded top-k routing (Gumbel-top-k over a Zipf pmf with n_empty experts
    never chosen): ``(topk_ids int32 [T, k], topk_weights float32 [T, k])``,
    the weights a softmax over each token's chosen scores."""
    g = _gen(seed)
    pmf = torch.arange(1, num_experts + 1, dtype=torch.float64) ** (-zipf_s)
    empty = torch.randperm(num_experts, generator=g)[:n_empty]
    pmf[empty] = 0.0
    pmf = pmf / pmf.sum()
    u = torch.rand((tokens, num_experts), generator=g, dtype=torch.float64).clamp_min(1e-300)
    scores = pmf.log() - (-u.log()).log()
    top = scores.topk(top_k, dim=1)
    w = torch.softmax(top.values, dim=1).to(torch.float32)
    return top.indices.to(torch.int32), w


def moe_counts(num_experts: int = 64, tokens: int = 4096, top_k: int = 8, zipf_s: float = 1.2,
               n_empty: int = 4, seed: int = 5004) -> torch.Tensor:
    g = _gen(seed)
    pmf = torch.arange(1, num_experts + 1, dtype=torch.float64) ** (-zipf_s)
    empty = torch.randperm(num_experts, generator=g)[:n_empty]
    pmf[empty] = 0.0
    pmf = pmf / pmf.sum()
    u = torch.rand((tokens, num_experts), generator=g, dtype=torch.float64).clamp_min(1e-300)
    scores = pmf.log() - (-u.log()).log()
    top = scores.topk(top_k, dim=1).indices
    return torch.bincount(top.reshape(-1), minlength=num_experts)


def moe_problem(cfg: int = 5, num_experts: int = 64, tokens: int = 4096, top_k: int = 8,
                n: int = 1536, k: int = 2048):
    """(X [T, K] bf16, W [E, N, K] bf16, offsets int32 [E+1], counts [E])."""
    counts = moe_counts(num_experts, tokens, top_k, seed=1000 * cfg + 4)
    offsets = torch.zeros(num_experts + 1, dtype=torch.int32)
    offsets[1:] = torch.cumsum(counts, 0).to(torch.int32)
    total = int(offsets[-1])
    x = randn_bf16((total, k), 1000 * cfg + 1)
    w = randn_bf16((num_experts, n, k), 1000 * cfg + 2, W_STD)
    return x, w, offsets, counts
