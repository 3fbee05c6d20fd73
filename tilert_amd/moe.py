"""MoE expert layer at one expert-parallel shard (EP = 8: 32 local experts of 256, whole
experts per GPU), on the gfx950 HIP kernels:
  * ``ep_gate_up_swiglu``: grouped gate/up GEMM + SwiGLU for the shard's hit experts (the
    grouped GEMM of expert_select_up_gate_silu_op, deepseek_v3_2/ops/
    expert_sel_up_gate_silu.py:23-48, golden :670-692);
  * ``ep_down_combine``: grouped down GEMM + routing-weighted sum (expert_down_allreduce_op,
    deepseek_v3_2/ops/expert_down_allreduce.py:23-63, golden :455-468) without the
    cross-GPU sum: the output is the shard's partial.
Routing is an input here (``expert_indices`` [M, topk] int32, ``expert_probs`` [M, topk]
fp32).  The reference's own operators -- routing on the device, the shared expert, the
tensor-parallel expert layout -- are ``tilert_amd.expert_sel_up_gate_silu`` and
``tilert_amd.expert_down_allreduce``.
"""
from __future__ import annotations

import torch

from . import _lib
from .kernel import _require_cuda, _stream

BLOCK = 128


def pack_moe_weight(w: torch.Tensor) -> torch.Tensor:
    """Tile-major fragment packing of stacked per-expert weights [rows, K] (tl_moe_pack_weight)."""
    rows, K = w.shape
    out = torch.empty(rows * K, dtype=torch.uint8, device=w.device)
    _lib.call("tl_moe_pack_weight", w.data_ptr(), out.data_ptr(), rows, K, _stream(w))
    return out


class LocalExperts:
    """The fp8 weights of the ``n_local`` experts this shard owns, packed for the kernels.

    gate/up [E, I, D] and down [E, D, I] are e4m3fn with 128x128 block scales
    [E, I/128, D/128] / [E, D/128, I/128].  Built once (the reference's
    ``ExpertSelectUpGateSiLUWeightsConverter`` / ``ExpertDownAllReduce`` converters play
    this role); the canonical tensors are not kept.
    """

    def __init__(self, gate, gate_s, up, up_s, down, down_s, expert_begin: int = 0) -> None:
        for t in (gate, up, down):
            if t.dtype != torch.float8_e4m3fn or t.dim() != 3:
                raise ValueError("LocalExperts: weights must be 3-D float8_e4m3fn")
        _require_cuda("LocalExperts", gate, gate_s, up, up_s, down, down_s)
        E, I, D = gate.shape
        if up.shape != (E, I, D) or down.shape != (E, D, I):
            raise ValueError("LocalExperts: inconsistent gate/up/down shapes")
        self.n_local, self.I, self.D, self.expert_begin = E, I, D, expert_begin
        w13 = torch.cat([gate, up], dim=1).reshape(E * 2 * I, D).contiguous()
        self.s13 = torch.cat([gate_s, up_s], dim=1).float().contiguous()
        self.w13 = pack_moe_weight(w13)
        self.w2 = pack_moe_weight(down.reshape(E * D, I).contiguous())
        self.s2 = down_s.float().contiguous()

    @property
    def device(self) -> torch.device:
        return self.w13.device


def _tokens(x: torch.Tensor, D: int) -> torch.Tensor:
    if x.dtype != torch.bfloat16:
        raise ValueError("MoE activations must be bfloat16")
    if x.shape[-1] != D:
        raise ValueError(f"hidden size {x.shape[-1]} != experts' {D}")
    return x.reshape(-1, D).contiguous()


def _routing(idx: torch.Tensor, M: int) -> torch.Tensor:
    if idx.dtype != torch.int32:
        raise ValueError("expert indices must be int32")
    idx = idx.reshape(M, -1).contiguous()
    return idx


def ep_gate_up_swiglu(hidden_in: torch.Tensor, expert_indices: torch.Tensor,
                               experts: LocalExperts, hidden_out: torch.Tensor | None = None,
                               profile_logs: torch.Tensor | None = None,
                               algorithm: str = "bf16mma", *, model_arch: str = "deepseek_v3_2"
                               ) -> torch.Tensor:
    """Gate/up GEMM + SwiGLU for this shard's hit experts.

    hidden_in bf16 [..., D] (M <= 16 tokens); expert_indices int32 [M, topk] global ids.
    Returns hidden_out bf16 [n_local, M, I]: slot s (the s-th hit local expert, ascending)
    holds ``bf16(silu(x G^T) * (x U^T))`` for every token.  ``profile_logs`` is accepted
    and left untouched; ``algorithm`` must be "bf16mma" (the reference MoE's numerics).
    """
    if algorithm not in ("bf16mma", "bf16"):
        raise ValueError(f"unsupported algorithm {algorithm!r} (the MoE kernels run bf16 MMA)")
    x = _tokens(hidden_in, experts.D)
    M = x.shape[0]
    idx = _routing(expert_indices, M)
    if hidden_out is None:
        hidden_out = torch.empty(experts.n_local, M, experts.I, dtype=torch.bfloat16, device=x.device)
    elif hidden_out.dtype != torch.bfloat16 or hidden_out.numel() < experts.n_local * M * experts.I \
            or not hidden_out.is_contiguous():
        raise ValueError("hidden_out must be a contiguous bf16 tensor of n_local*M*I elements")
    _require_cuda("ep_gate_up_swiglu", x, idx, experts.w13, experts.s13, hidden_out)
    _lib.call("tl_moe_gate_up_swiglu", x.data_ptr(), experts.w13.data_ptr(), experts.s13.data_ptr(),
              idx.data_ptr(), M, idx.shape[1], experts.expert_begin, experts.n_local, experts.D,
              experts.I, hidden_out.data_ptr(), _stream(x))
    return hidden_out


def ep_down_combine(vec_in: torch.Tensor, experts: LocalExperts, indices: torch.Tensor,
                          scores: torch.Tensor, x_in: torch.Tensor | None = None, flag: int = 0,
                          vec_out: torch.Tensor | None = None,
                          profile_logs: torch.Tensor | None = None,
                          model_arch: str = "deepseek_v3_2",
                          compute_kernel_type: str = "bf16") -> torch.Tensor:
    """Down GEMM + routing-weighted combine for this shard (argument order of the reference
    op; ``mat_in``/``mat_scale`` are carried by ``experts``).

    vec_in bf16 [n_local, M, I] from ``ep_gate_up_swiglu``; indices int32 and
    scores fp32 [M, topk].  Returns vec_out bf16 [M, D].  ``x_in``/``flag`` belong to the
    cross-GPU allreduce epilogue, which one shard does not run (the reference's
    single-GPU golden, padded_allreduce_add.py:100-114, is the identity); they are
    accepted and ignored.
    """
    if compute_kernel_type not in ("bf16", "bf16mma"):
        raise ValueError(f"unsupported compute_kernel_type {compute_kernel_type!r}")
    M = indices.reshape(-1, indices.shape[-1]).shape[0]
    idx = _routing(indices, M)
    if scores.dtype != torch.float32:
        raise ValueError("scores must be float32")
    w = scores.reshape(M, -1).contiguous()
    if w.shape != idx.shape:
        raise ValueError("scores and indices shapes differ")
    if vec_in.dtype != torch.bfloat16 or not vec_in.is_contiguous() \
            or vec_in.numel() < experts.n_local * M * experts.I:
        raise ValueError("vec_in must be the contiguous bf16 [n_local, M, I] gate/up output")
    if vec_out is None:
        vec_out = torch.empty(M, experts.D, dtype=torch.bfloat16, device=vec_in.device)
    elif vec_out.dtype != torch.bfloat16 or vec_out.numel() != M * experts.D or not vec_out.is_contiguous():
        raise ValueError("vec_out must be a contiguous bf16 tensor of M*D elements")
    _require_cuda("ep_down_combine", vec_in, idx, w, experts.w2, experts.s2, vec_out)
    _lib.call("tl_moe_down_combine", vec_in.data_ptr(), experts.w2.data_ptr(), experts.s2.data_ptr(),
              idx.data_ptr(), w.data_ptr(), M, idx.shape[1], experts.expert_begin, experts.n_local,
              experts.D, experts.I, vec_out.data_ptr(), _stream(vec_in))
    return vec_out


def moe_forward(x: torch.Tensor, experts: LocalExperts, expert_indices: torch.Tensor,
                expert_probs: torch.Tensor, h_buf: torch.Tensor | None = None,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """The shard's routed-expert layer: gate/up + SwiGLU, down, weighted combine."""
    h = ep_gate_up_swiglu(x, expert_indices, experts, h_buf)
    return ep_down_combine(h, experts, expert_indices, expert_probs, vec_out=out)
