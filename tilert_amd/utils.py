"""Comparison metrics with the semantics of tilert/utils.py:65-90."""
from __future__ import annotations

import torch


def cosine_similarity(gt: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """Cosine similarity of the flattened fp32 tensors (tilert/utils.py:65-77)."""
    return torch.nn.functional.cosine_similarity(gt.flatten().float(), out.flatten().float(), dim=-1)


def relative_l2_error(gt: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """``||gt - out|| / ||gt||`` (tilert/utils.py:80-90), computed in fp32."""
    gt = gt.float()
    return torch.norm(gt - out.float()) / torch.norm(gt)
