"""Exact top-k over indexer logits with the reference's ``topk_accurate`` contract
(ops/topk.py:62-109): sample i of n considers its first ``seq_len - n + 1 + i`` columns."""
from __future__ import annotations

import torch

from . import _lib
from .kernel import _Workspace, _require_cuda, _stream

_WS = _Workspace()


def topk_rows(logits: torch.Tensor, valid_base: int, k: int,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """Rows of ``logits`` [rows, ld]; row i considers columns [0, valid_base + 1 + i).
    Returns int32 [rows, k]: the selected columns in ascending order, -1 padding."""
    if logits.dtype != torch.float32 or logits.dim() != 2 or not logits.is_contiguous():
        raise ValueError("logits must be a contiguous 2-D float32 tensor")
    _require_cuda("topk", logits)
    rows, ld = logits.shape
    if out is None:
        out = torch.empty(rows, k, dtype=torch.int32, device=logits.device)
    st = _stream(logits)
    nbytes = _lib.query("tl_topk_workspace_bytes", rows, ld, k)
    ws = _WS.get(logits.device, st, nbytes)
    _lib.call("tl_topk_rows", logits.data_ptr(), rows, ld, int(valid_base), k, out.data_ptr(),
              ws.data_ptr(), ws.numel(), st)
    return out


def topk_accurate(logits: torch.Tensor, seq_len: int, topk: int,
                  profile_logs: torch.Tensor | None = None, model_arch: str = "deepseek_v3_2",
                  compute_kernel_type: str = "general", ratio: int = 1) -> torch.Tensor:
    """Exact top-``topk`` of ``logits`` [1, n, L] (fp32).  For the n samples the valid
    lengths are seq_len-n+1, ..., seq_len.  Returns int32 [n, topk] (ascending column
    indices; the selected set equals torch.topk's on each valid prefix)."""
    if logits.dtype != torch.float32:
        raise ValueError("logits must be a float32 tensor.")
    if topk not in (512, 1024, 2048):
        raise ValueError("topk must be 512, 1024, or 2048.")
    assert logits.shape[0] == 1, "batch must be 1 in this version"
    if ratio != 1:
        raise ValueError("ratio != 1 (compressed token domain) is not supported")
    num_samples = logits.shape[1]
    return topk_rows(logits.reshape(num_samples, -1).contiguous(), seq_len - num_samples, topk)
