"""Seeded synthetic inputs for the benchmark configurations (CPU generation, so the same
seed gives the same tensors on every host; callers move them to the GPU).

Shapes and distributions follow the workload definitions: activations ~N(0,1) bf16,
weights ~N(0, 0.02) fp32 before 128x128 block quantisation, indexer keys ~N(0,1) before
per-key quantisation, head weights ~N(0, 1/64), MoE routing = 8 distinct experts per
token drawn uniformly from 256 with softmax weights over N(0,1) logits.
"""
from __future__ import annotations

import torch


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def activations(M: int, K: int, g: torch.Generator) -> torch.Tensor:
    return torch.randn(M, K, generator=g, dtype=torch.float32).to(torch.bfloat16)


def weight_fp32(N: int, K: int, g: torch.Generator, std: float = 0.02) -> torch.Tensor:
    return torch.randn(N, K, generator=g, dtype=torch.float32) * std


def routing(M: int, n_experts: int, topk: int, g: torch.Generator) -> tuple[torch.Tensor, torch.Tensor]:
    """topk_idx int32 [M, topk] (distinct per token), topk_w fp32 [M, topk] (softmax)."""
    idx = torch.stack([torch.randperm(n_experts, generator=g)[:topk] for _ in range(M)]).to(torch.int32)
    logits = torch.randn(M, topk, generator=g, dtype=torch.float32)
    return idx, torch.softmax(logits, dim=-1)


def per_row_quant_e4m3(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row e4m3fn quantisation with scale amax/448 (key-cache and query format).
    CPU helper for input generation: x fp32 [R, D] -> (fp8 [R, D], fp32 [R])."""
    amax = x.abs().amax(dim=-1).clamp_min(1e-4)
    s = amax / 448.0
    q = torch.clamp(x / s[:, None], -448.0, 448.0).to(torch.float8_e4m3fn)
    return q, s.float()


def indexer_inputs(M: int, H: int, L: int, g: torch.Generator, dim: int = 128):
    """q fp8 [M,H,dim] + per-token scale [M]; k fp8 [L,dim] + per-key scale [L]; w bf16 [M,H]."""
    q32 = torch.randn(M, H, dim, generator=g, dtype=torch.float32)
    qq, qs = per_row_quant_e4m3(q32.reshape(M, H * dim))
    k32 = torch.randn(L, dim, generator=g, dtype=torch.float32)
    kq, ks = per_row_quant_e4m3(k32)
    w = (torch.randn(M, H, generator=g, dtype=torch.float32) * (1.0 / 8.0)).to(torch.bfloat16)
    return qq.reshape(M, H, dim), qs, kq, ks, w
