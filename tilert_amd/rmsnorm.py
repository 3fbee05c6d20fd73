"""RMSNorm with optional fused activation quantisation, with the reference operator's
signature (ops/rmsnorm_quant.py:19-63): ``rmsnorm_quant`` writes the normalised bf16 rows
and, when the quantised outputs are given, their per-1x128 e4m3fn quantisation -- one
launch instead of RMSNorm then act_quant (the norm of tilert/models/common.py:92-133)."""
from __future__ import annotations

import torch

from . import _lib
from .kernel import SCALE_MODES, _require_cuda, _stream

BLOCK_SIZE = 128
DIM_DEEPSEEK_V3_2 = 7168
DIM_GLM_5 = 6144
EPS = 1e-6  # RMSNorm's default (tilert/models/common.py:101)


def rmsnorm_quant(hidden_in: torch.Tensor, gamma_in: torch.Tensor, hidden_out: torch.Tensor,
                  quant_hidden_out: torch.Tensor | None = None,
                  quant_hidden_scale_out: torch.Tensor | None = None,
                  profile_logs: torch.Tensor | None = None, compute_kernel_type: str = "general", *,
                  model_arch: str, scale_fmt: str | None = None, eps: float = EPS) -> None:
    """hidden_in bf16 (..., dim); gamma_in (dim,) fp32 (or bf16, widened); hidden_out bf16
    (..., dim); quant_hidden_out e4m3fn (..., dim) and quant_hidden_scale_out fp32
    (..., dim // 128), both or neither.  ``scale_fmt`` selects the act_quant scale rule."""
    if profile_logs is None:
        raise ValueError("profile_logs is required when calling rmsnorm_quant.")
    if hidden_in.dtype != torch.bfloat16 or hidden_out.dtype != torch.bfloat16:
        raise ValueError("hidden_in and hidden_out must be bfloat16 tensors")
    dim = hidden_in.shape[-1]
    if gamma_in.numel() != dim:
        raise ValueError("gamma_in must be (dim,)")
    if hidden_out.shape != hidden_in.shape:
        raise ValueError("hidden_out must have hidden_in's shape")
    if (quant_hidden_out is None) != (quant_hidden_scale_out is None):
        raise ValueError("quant_hidden_out and quant_hidden_scale_out go together")
    if quant_hidden_out is not None:
        if quant_hidden_out.dtype != torch.float8_e4m3fn or quant_hidden_out.shape != hidden_in.shape:
            raise ValueError("quant_hidden_out must be float8_e4m3fn with hidden_in's shape")
        if quant_hidden_scale_out.dtype != torch.float32 or \
                quant_hidden_scale_out.numel() != hidden_in.numel() // BLOCK_SIZE:
            raise ValueError("quant_hidden_scale_out must be float32 (..., dim // 128)")
    for t in (hidden_in, hidden_out, quant_hidden_out, quant_hidden_scale_out):
        if t is not None and not t.is_contiguous():
            raise ValueError("rmsnorm_quant tensors must be contiguous")
    gamma = gamma_in.reshape(dim).to(torch.float32).contiguous()
    _require_cuda("rmsnorm_quant", hidden_in, gamma, hidden_out, quant_hidden_out, quant_hidden_scale_out)
    rows = hidden_in.numel() // dim if dim else 0
    _lib.call("tl_rmsnorm_quant", hidden_in.data_ptr(), gamma.data_ptr(), float(eps), rows, dim,
              hidden_out.data_ptr(),
              quant_hidden_out.data_ptr() if quant_hidden_out is not None else None,
              quant_hidden_scale_out.data_ptr() if quant_hidden_scale_out is not None else None,
              SCALE_MODES.get(scale_fmt, 1), _stream(hidden_in))
