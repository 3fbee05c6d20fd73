"""The fused FP8 attention down-projection, with the reference operator's signature
(tilert/models/deepseek_v3_2/ops/projx_wqkva.py:22-48): one GEMV launch computes
``x . [wq_a; wkv_a]^T`` and routes its columns to q (q_lora_rank), kv (kv_lora_rank) and
the rope part, which lands in ``pe_cache_out`` at ``cur_pos``.

The weight converter (the role of ``RMSNormProjQKVAFP8MMAWeightsConverter``,
rmsnorm_projx_wqkva.py:18-119) is ``pack_wqkva``: it stacks the two block-quantised
weights and packs them into MFMA fragments once, at load time.  Unlike the reference
converter it keeps the checkpoint's 128x128 block scales (no re-quantisation), so results
equal ``fp8_gemm`` on each weight.
"""
from __future__ import annotations

import torch

from . import _lib
from .kernel import BLOCK, _WS, PackedFP8Weight, _require_cuda, _stream, pack_weight

# (dim, q_lora_rank, kv_lora_rank, qk_rope_head_dim) per model_arch
ARCH_DIMS = {
    "deepseek_v3_2": (7168, 1536, 512, 64),
    "glm_5": (6144, 2048, 512, 64),
}


class PackedWqkva(PackedFP8Weight):
    """[wq_a; wkv_a] stacked and fragment-packed, with the widths of the three outputs."""

    def __init__(self, packed: PackedFP8Weight, q_rank: int, kv_rank: int, rope_dim: int) -> None:
        super().__init__(packed.data, packed.scale, packed.N, packed.K)
        self.q_rank, self.kv_rank, self.rope_dim = q_rank, kv_rank, rope_dim


def pack_wqkva(wq_a: torch.Tensor, wq_a_scale: torch.Tensor, wkv_a: torch.Tensor,
               wkv_a_scale: torch.Tensor, kv_lora_rank: int) -> PackedWqkva:
    """Stack wq_a [q_rank, dim] (scales [q_rank/128, dim/128]) over wkv_a
    (kv_a_proj_with_mqa, [kv_rank + rope, dim], scales [ceil((kv_rank + rope)/128), dim/128])
    and pack them.  q_rank must be a multiple of 128 so the scale rows stack unchanged."""
    q_rank, dim = wq_a.shape
    rows_kv = wkv_a.shape[0]
    if wkv_a.shape[1] != dim:
        raise ValueError("pack_wqkva: wq_a and wkv_a must have the same input dim")
    if q_rank % BLOCK:
        raise ValueError(f"pack_wqkva: q_lora_rank={q_rank} must be a multiple of {BLOCK}")
    if not 0 < kv_lora_rank < rows_kv:
        raise ValueError("pack_wqkva: kv_lora_rank must split wkv_a into latent and rope rows")
    if wq_a_scale.shape != (q_rank // BLOCK, dim // BLOCK) or \
            wkv_a_scale.shape != ((rows_kv + BLOCK - 1) // BLOCK, dim // BLOCK):
        raise ValueError("pack_wqkva: scale shapes do not match the weights")
    w = torch.cat([wq_a, wkv_a], 0).contiguous()
    s = torch.cat([wq_a_scale.float(), wkv_a_scale.float()], 0).contiguous()
    return PackedWqkva(pack_weight(w, s), q_rank, kv_lora_rank, rows_kv - kv_lora_rank)


def projx_wqkva(x_quant: torch.Tensor, x_scale: torch.Tensor, wqkva: PackedWqkva,
                cur_pos: torch.Tensor, q_out: torch.Tensor, kv_out: torch.Tensor,
                pe_cache_out: torch.Tensor, profile_logs: torch.Tensor | None = None,
                compute_kernel_type: str = "fp8mma", *, model_arch: str) -> None:
    """x_quant e4m3fn [batch, seq, dim] + x_scale fp32 [batch, seq, dim/128];
    cur_pos int32 (1,) on the device; q_out bf16 [batch, seq, q_rank]; kv_out bf16
    [batch, seq, kv_rank]; pe_cache_out bf16 [batch, max_len, rope_dim], written at rows
    cur_pos .. cur_pos + seq - 1 (rows past max_len are dropped).  profile_logs is accepted
    and left untouched."""
    if compute_kernel_type != "fp8mma":
        raise ValueError(f"projx_wqkva: compute_kernel_type {compute_kernel_type!r} is not supported "
                         "(only 'fp8mma')")
    if model_arch not in ARCH_DIMS:
        raise ValueError(f"projx_wqkva: unknown model_arch {model_arch!r}")
    if not isinstance(wqkva, PackedWqkva):
        raise ValueError("projx_wqkva: wqkva must come from pack_wqkva")
    if x_quant.dim() != 3 or x_quant.dtype != torch.float8_e4m3fn:
        raise ValueError("projx_wqkva: x_quant must be float8_e4m3fn [batch, seq, dim]")
    batch, seq, dim = x_quant.shape
    if dim != wqkva.K:
        raise ValueError(f"projx_wqkva: x dim {dim} does not match the weight's {wqkva.K}")
    if x_scale.dtype != torch.float32 or x_scale.numel() != batch * seq * (dim // BLOCK):
        raise ValueError("projx_wqkva: x_scale must be float32 [batch, seq, dim/128]")
    q_rank, kv_rank, rope = wqkva.q_rank, wqkva.kv_rank, wqkva.rope_dim
    for name, t, shape in (("q_out", q_out, (batch, seq, q_rank)), ("kv_out", kv_out, (batch, seq, kv_rank))):
        if t.dtype != torch.bfloat16 or tuple(t.shape) != shape:
            raise ValueError(f"projx_wqkva: {name} must be bfloat16 {shape}")
    if pe_cache_out.dtype != torch.bfloat16 or pe_cache_out.dim() != 3 or \
            pe_cache_out.shape[0] != batch or pe_cache_out.shape[2] != rope:
        raise ValueError(f"projx_wqkva: pe_cache_out must be bfloat16 [{batch}, max_len, {rope}]")
    if cur_pos.dtype != torch.int32 or cur_pos.numel() < 1:
        raise ValueError("projx_wqkva: cur_pos must be an int32 tensor")
    for t in (x_quant, x_scale, q_out, kv_out, pe_cache_out, cur_pos):
        if not t.is_contiguous():
            raise ValueError("projx_wqkva: tensors must be contiguous")
    _require_cuda("projx_wqkva", x_quant, x_scale, wqkva.data, wqkva.scale, q_out, kv_out, pe_cache_out, cur_pos)
    M, N = batch * seq, wqkva.N
    st = _stream(x_quant)
    nbytes = _lib.query("tl_fp8_gemm_workspace_bytes", M, N, dim)
    ws_ptr, ws_len = None, 0
    if nbytes:
        ws = _WS.get(x_quant.device, st, nbytes)
        ws_ptr, ws_len = ws.data_ptr(), ws.numel()
    _lib.call("tl_projx_wqkva", x_quant.data_ptr(), x_scale.data_ptr(), wqkva.data.data_ptr(),
              wqkva.scale.data_ptr(), cur_pos.data_ptr(), q_out.data_ptr(), kv_out.data_ptr(),
              pe_cache_out.data_ptr(), batch, seq, pe_cache_out.shape[1], dim, q_rank, kv_rank, rope,
              ws_ptr, ws_len, st)



_NO_LOGS: dict = {}


def rmsnorm_projx_wqkva(x: torch.Tensor, gamma: torch.Tensor, wqkva: PackedWqkva, cur_pos: torch.Tensor,
                        q_out: torch.Tensor, kv_out: torch.Tensor, pe_cache_out: torch.Tensor,
                        x_rmsnorm_out: torch.Tensor | None = None, profile_logs: torch.Tensor | None = None, *,
                        model_arch: str, scale_fmt: str | None = None, eps: float = 1e-6) -> None:
    """The DECOUPLED ``RMSNormProjxWqkva`` (rmsnorm_projx_wqkva.py:473-509): ``rmsnorm_quant``
    (RMSNorm + act_quant, one launch) into scratch tensors, then ``projx_wqkva``.  x bf16
    [batch, seq, dim]; gamma [dim]; outputs as for ``projx_wqkva``; ``x_rmsnorm_out`` (bf16,
    x's shape), when given, receives the normalised rows.  A single launch that recomputes
    the norm in every GEMV workgroup measured slower on MI355X (15.4-20.8 vs 11.0 us at M = 4,
    7168 -> 2112): each of its 132 workgroups quantises all M x 7168 values."""
    from .rmsnorm import rmsnorm_quant
    if x.dim() != 3 or x.dtype != torch.bfloat16:
        raise ValueError("rmsnorm_projx_wqkva: x must be bfloat16 [batch, seq, dim]")
    if not isinstance(wqkva, PackedWqkva):
        raise ValueError("rmsnorm_projx_wqkva: wqkva must come from pack_wqkva")
    batch, seq, dim = x.shape
    if dim != wqkva.K:
        raise ValueError(f"rmsnorm_projx_wqkva: x dim {dim} does not match the weight's {wqkva.K}")
    y = torch.empty_like(x) if x_rmsnorm_out is None else x_rmsnorm_out
    xq = torch.empty(batch, seq, dim, dtype=torch.float8_e4m3fn, device=x.device)
    xs = torch.empty(batch, seq, dim // BLOCK, dtype=torch.float32, device=x.device)
    logs = profile_logs
    if logs is None:  # rmsnorm_quant requires the tensor; it is never written
        logs = _NO_LOGS.get(x.device)
        if logs is None:
            logs = _NO_LOGS[x.device] = torch.zeros(1, device=x.device)
    rmsnorm_quant(x, gamma, y, xq, xs, logs, model_arch=model_arch, scale_fmt=scale_fmt, eps=eps)
    projx_wqkva(xq, xs, wqkva, cur_pos, q_out, kv_out, pe_cache_out, profile_logs, model_arch=model_arch)
