"""GLM-5's indexer + top-k with the reference's signature
(tilert/models/glm_5/ops/sparse_index_v3.py:10-51): 32 index heads, bf16 q / key cache /
head weights, fp32 logits, int32 indices -- ``tilert_amd.sparse_index.sparse_index_topk``'s
kernel at H = 32."""
from __future__ import annotations

import torch

from .sparse_index import _bf16_topk

__all__ = ["sparse_index_topk_v3"]


def sparse_index_topk_v3(q: torch.Tensor, kv: torch.Tensor, weights: torch.Tensor, logits: torch.Tensor,
                         indices: torch.Tensor, cur_pos: int, profile_logs: torch.Tensor | None = None) -> None:
    """GLM5 sparse index + top-k selection (32 heads, head dim 128)."""
    head = q.shape[-2]
    if head != 32:
        raise ValueError(f"Unsupported head size: {head}. SparseIndexV3 fused op "
                         "supports head number of 32 (GLM5).")
    _bf16_topk(q, kv, weights, logits, indices, cur_pos, profile_logs)
