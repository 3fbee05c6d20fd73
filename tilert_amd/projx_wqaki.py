"""The indexer's input projections with the reference operators' signatures:

* ``projx_wqaki`` (tilert/models/deepseek_v3_2/ops/projx_wqaki.py:11-44): x_quant . [wq_a;
  wk]^T in one FP8 GEMV launch, routed to q (q_lora_rank) and ki (the indexer key, 128);
* ``projx_wis`` (ops/projx_wis.py:18-37): the bf16 head-weight projection weights_proj
  (64 rows) of the bf16 normalised rows;
* ``rmsnorm_projx_wqakis``: the DECOUPLED ``RMSNormProjxWqakis`` module
  (ops/rmsnorm_projx_wqakis.py:301-335): rmsnorm_quant, then the two projections.

``pack_wqaki`` is the weight converter (the role of ``ProjxWqakiWeightsConverter``,
projx_wqaki.py:47-243): it stacks the two block-quantised weights and packs them into
MFMA fragments once, keeping their 128x128 block scales.
"""
from __future__ import annotations

import torch

from . import _lib
from .kernel import BLOCK, _WS, PackedFP8Weight, _require_cuda, _stream, pack_weight

EPS = {"deepseek_v3_2": 1e-6, "glm_5": 1e-5}


class PackedWqaki(PackedFP8Weight):
    """[wq_a; wk] stacked and fragment-packed, with the widths of the two outputs."""

    def __init__(self, packed: PackedFP8Weight, q_rank: int, ki_dim: int) -> None:
        super().__init__(packed.data, packed.scale, packed.N, packed.K)
        self.q_rank, self.ki_dim = q_rank, ki_dim


def pack_wqaki(wq_a: torch.Tensor, wq_a_scale: torch.Tensor, wk: torch.Tensor, wk_scale: torch.Tensor) -> PackedWqaki:
    """wq_a [q_rank, dim] (q_rank % 128 == 0) over the indexer's wk [ki_dim, dim], both
    e4m3fn with fp32/bf16 block scales."""
    q_rank, dim = wq_a.shape
    ki = wk.shape[0]
    if wk.shape[1] != dim:
        raise ValueError("pack_wqaki: wq_a and wk must have the same input dim")
    if q_rank % BLOCK:
        raise ValueError(f"pack_wqaki: q_lora_rank={q_rank} must be a multiple of {BLOCK}")
    if wq_a_scale.shape != (q_rank // BLOCK, dim // BLOCK) or wk_scale.shape != ((ki + BLOCK - 1) // BLOCK, dim // BLOCK):
        raise ValueError("pack_wqaki: scale shapes do not match the weights")
    w = torch.cat([wq_a, wk], 0).contiguous()
    s = torch.cat([wq_a_scale.float(), wk_scale.float()], 0).contiguous()
    return PackedWqaki(pack_weight(w, s), q_rank, ki)


def projx_wqaki(x_quant: torch.Tensor, x_scale: torch.Tensor, wqaki: PackedWqaki, out_q: torch.Tensor,
                out_ki: torch.Tensor, profile_logs: torch.Tensor | None = None, compute_kernel_type: str = "fp8mma",
                *, model_arch: str) -> None:
    """x_quant e4m3fn [1, s, dim] + x_scale fp32 [1, s, dim/128]; out_q bf16 [1, s, q_rank];
    out_ki bf16 [1, s, ki_dim].  ``compute_kernel_type`` "fp8mma" (and the reference's
    "fp8mma_68cta" / "fp8mma_136cta" grid variants) all run the FP8 GEMV."""
    if compute_kernel_type not in ("fp8mma", "fp8mma_68cta", "fp8mma_136cta"):
        raise ValueError(f"projx_wqaki: unsupported compute_kernel_type {compute_kernel_type!r}")
    if model_arch not in EPS:
        raise ValueError(f"projx_wqaki: unknown model_arch {model_arch!r}")
    if not isinstance(wqaki, PackedWqaki):
        raise ValueError("projx_wqaki: wqaki must come from pack_wqaki")
    if x_quant.dtype != torch.float8_e4m3fn or x_quant.shape[-1] != wqaki.K:
        raise ValueError(f"projx_wqaki: x_quant must be float8_e4m3fn [1, s, {wqaki.K}]")
    dim = wqaki.K
    M = x_quant.numel() // dim
    if x_scale.dtype != torch.float32 or x_scale.numel() != M * (dim // BLOCK):
        raise ValueError("projx_wqaki: x_scale must be float32 [1, s, dim/128]")
    if out_q.dtype != torch.bfloat16 or out_q.numel() != M * wqaki.q_rank:
        raise ValueError(f"projx_wqaki: out_q must be bfloat16 [1, s, {wqaki.q_rank}]")
    if out_ki.dtype != torch.bfloat16 or out_ki.numel() != M * wqaki.ki_dim:
        raise ValueError(f"projx_wqaki: out_ki must be bfloat16 [1, s, {wqaki.ki_dim}]")
    for t in (x_quant, x_scale, out_q, out_ki):
        if not t.is_contiguous():
            raise ValueError("projx_wqaki: tensors must be contiguous")
    _require_cuda("projx_wqaki", x_quant, x_scale, wqaki.data, wqaki.scale, out_q, out_ki)
    st = _stream(x_quant)
    nbytes = _lib.query("tl_fp8_gemm_workspace_bytes", M, wqaki.N, dim)
    ws_ptr, ws_len = None, 0
    if nbytes:
        ws = _WS.get(x_quant.device, st, nbytes)
        ws_ptr, ws_len = ws.data_ptr(), ws.numel()
    _lib.call("tl_projx_wqaki", x_quant.data_ptr(), x_scale.data_ptr(), wqaki.data.data_ptr(), wqaki.scale.data_ptr(),
              out_q.data_ptr(), out_ki.data_ptr(), M, dim, wqaki.q_rank, wqaki.ki_dim, ws_ptr, ws_len, st)


def projx_wis(x_in: torch.Tensor, w: torch.Tensor, output: torch.Tensor, compute_kernel_type: str = "bf16",
              profile_logs: torch.Tensor | None = None, model_arch: str = "deepseek_v3_2") -> None:
    """x_in bf16 [1, s, dim]; w bf16 [n_heads, dim] (weights_proj); output bf16 [1, s, n_heads]."""
    if compute_kernel_type not in ("bf16", "bf16mma"):
        raise ValueError(f"projx_wis: unsupported compute_kernel_type {compute_kernel_type!r}")
    if model_arch not in EPS:
        raise ValueError(f"projx_wis: unknown model_arch {model_arch!r}")
    if w.dtype != torch.bfloat16 or w.dim() != 2 or not w.is_contiguous():
        raise ValueError("projx_wis: w must be a contiguous bfloat16 [n_heads, dim] tensor")
    N, dim = w.shape
    if x_in.dtype != torch.bfloat16 or x_in.shape[-1] != dim or not x_in.is_contiguous():
        raise ValueError(f"projx_wis: x_in must be a contiguous bfloat16 [1, s, {dim}] tensor")
    M = x_in.numel() // dim
    if output.dtype != torch.bfloat16 or output.numel() != M * N or not output.is_contiguous():
        raise ValueError(f"projx_wis: output must be a contiguous bfloat16 [1, s, {N}] tensor")
    _require_cuda("projx_wis", x_in, w, output)
    st = _stream(x_in)
    nbytes = _lib.query("tl_bf16_gemv_workspace_bytes", M, N, dim)
    ws_ptr, ws_len = None, 0
    if nbytes:
        ws = _WS.get(x_in.device, st, nbytes)
        ws_ptr, ws_len = ws.data_ptr(), ws.numel()
    _lib.call("tl_bf16_gemv", x_in.data_ptr(), w.data_ptr(), M, N, dim, output.data_ptr(), ws_ptr, ws_len, st)


_NO_LOGS: dict = {}


def rmsnorm_projx_wqakis(x: torch.Tensor, gamma: torch.Tensor, wqaki: PackedWqaki, wis: torch.Tensor,
                         q_out: torch.Tensor, ki_out: torch.Tensor, idx_scores_out: torch.Tensor,
                         x_rmsnorm_out: torch.Tensor | None = None, profile_logs: torch.Tensor | None = None, *,
                         model_arch: str, scale_fmt: str | None = None) -> None:
    """The DECOUPLED ``RMSNormProjxWqakis`` (rmsnorm_projx_wqakis.py:301-335): the bf16
    normalised rows and their act_quant (``rmsnorm_quant``, one launch), then ``projx_wqaki``
    on the quantised rows and ``projx_wis`` on the bf16 rows.  x bf16 [1, s, dim]; gamma
    [dim]; q_out / ki_out / idx_scores_out bf16 [1, s, q_rank / ki_dim / n_heads]."""
    from .rmsnorm import rmsnorm_quant
    if x.dtype != torch.bfloat16 or x.shape[-1] != wqaki.K:
        raise ValueError(f"rmsnorm_projx_wqakis: x must be bfloat16 [1, s, {wqaki.K}]")
    dim = wqaki.K
    y = torch.empty_like(x) if x_rmsnorm_out is None else x_rmsnorm_out
    xq = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
    xs = torch.empty(*x.shape[:-1], dim // BLOCK, dtype=torch.float32, device=x.device)
    logs = profile_logs
    if logs is None:  # rmsnorm_quant requires the tensor; it is never written
        logs = _NO_LOGS.get(x.device)
        if logs is None:
            logs = _NO_LOGS[x.device] = torch.zeros(1, device=x.device)
    rmsnorm_quant(x, gamma, y, xq, xs, logs, model_arch=model_arch, scale_fmt=scale_fmt, eps=EPS[model_arch])
    projx_wqaki(xq, xs, wqaki, q_out, ki_out, profile_logs, model_arch=model_arch)
    projx_wis(y, wis, idx_scores_out, "bf16", profile_logs, model_arch)
