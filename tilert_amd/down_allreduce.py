"""``down_allreduce`` with the reference operator's signature
(tilert/models/deepseek_v3_2/ops/down_allreduce.py:24-59) on the gfx950 HIP library: the
dense MLP's down projection over the device's chunks, each chunk's term rounded to bf16
and summed in fp32 (golden :293-320), plus the residual ``x_in`` (the single-GPU form of
the allreduce-add epilogue, padded_allreduce_add.py:100-114; ``flag`` is unused)."""
from __future__ import annotations

import torch

from . import _lib
from .expert_down_allreduce import DownExperts, _check_out
from .kernel import _require_cuda, _stream


def down_allreduce(vec_in: torch.Tensor, mat_in: DownExperts, mat_scale: torch.Tensor | None,
                   x_in: torch.Tensor | None, flag: int, vec_out: torch.Tensor,
                   profile_logs: torch.Tensor | None = None, model_arch: str = "deepseek_v3_2",
                   compute_kernel_type: str = "bf16") -> None:
    """vec_in bf16 [1, s, n_chunks, I] (``rmsnorm_up_gate_silu``'s hidden_out); mat_in =
    ``DownExperts`` of the chunks (``mat_scale`` may be None: the scales ride along);
    x_in bf16 [1, s, D] or None; vec_out bf16 [1, s, D]."""
    if model_arch not in ("deepseek_v3_2", "glm_5"):
        raise ValueError(f"Unsupported architecture: {model_arch}")
    if compute_kernel_type not in ("bf16", "bf16mma", "general"):
        raise ValueError(f"Unsupported compute_kernel_type: {compute_kernel_type}")
    w = mat_in
    if vec_in.dtype != torch.bfloat16 or vec_in.shape[-1] != w.I or vec_in.shape[-2] != w.n_local \
            or not vec_in.is_contiguous():
        raise ValueError(f"vec_in must be a contiguous bfloat16 [1, s, {w.n_local}, {w.I}] tensor")
    s = vec_in.numel() // (w.n_local * w.I)
    _check_out(vec_out, x_in, s, w.D, "down_allreduce")
    _require_cuda("down_allreduce", vec_in, x_in, vec_out, w.w2, w.s2)
    _lib.call("tl_down_allreduce", vec_in.data_ptr(), w.w2.data_ptr(), w.s2.data_ptr(),
              x_in.data_ptr() if x_in is not None else None, s, w.n_local, w.D, w.I, vec_out.data_ptr(),
              _stream(vec_in))
