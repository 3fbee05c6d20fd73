"""``projq_wqb`` with the reference operator's signature
(tilert/models/deepseek_v3_2/ops/projq_wqb.py:24-54) on the gfx950 HIP library: the absorbed
query projection of MLA, q_lat[t, h, :] = q_nope[t, h, :] . wkv_b[h, :nope, :] (golden
``einsum("bshd,hdc->bshc")``, :448-450), for the device's local heads.

``HeadWeights`` is the per-head weight form the per-head GEMV (``tl_head_gemm_bf16``)
consumes: H weights [N, K] packed once (the role of ``ProjqWqbWeightsConverter``).  Here the
contraction runs over wkv_b's rows, so ``convert_projq_wqb`` stores each head's nope block
transposed (N = kv_lora_rank, K = qk_nope_head_dim); 128x128 block scales transpose with
it.  Numerics: bf16 activations times bf16-rounded dequantised weights, fp32 accumulation.
"""
from __future__ import annotations

import torch

from . import _lib
from .kernel import _require_cuda, _stream
from .moe import pack_moe_weight

BLOCK = 128


class HeadWeights:
    """H fp8 weights W_h [N, K] (e4m3fn [H, N, K], fp32 scales [H, ceil(N/128), K/128]),
    packed for ``tl_head_gemm_bf16``."""

    def __init__(self, w: torch.Tensor, s: torch.Tensor) -> None:
        if w.dtype != torch.float8_e4m3fn or w.dim() != 3:
            raise ValueError("head weights must be 3-D float8_e4m3fn [H, N, K]")
        H, N, K = w.shape
        if N % 16 or K % BLOCK:
            raise ValueError("N must be a multiple of 16 and K of 128")
        if s.shape != (H, (N + BLOCK - 1) // BLOCK, K // BLOCK):
            raise ValueError("scales must be [H, ceil(N/128), K/128]")
        _require_cuda("HeadWeights", w, s)
        self.H, self.N, self.K = H, N, K
        self.w = pack_moe_weight(w.reshape(H * N, K).contiguous())
        self.s = s.float().contiguous()

    @property
    def device(self) -> torch.device:
        return self.w.device


def head_gemm(x: torch.Tensor, weights: HeadWeights, out: torch.Tensor, x_in: torch.Tensor | None = None) -> None:
    """out[t, h, :] = bf16(x[t, h, :] . W_h^T) (+ x_in, rounded again); x bf16 [..., H, K],
    out bf16 [..., H, N]."""
    H, N, K = weights.H, weights.N, weights.K
    if x.dtype != torch.bfloat16 or not x.is_contiguous() or x.numel() % (H * K):
        raise ValueError(f"x must be a contiguous bfloat16 [..., {H}, {K}] tensor")
    M = x.numel() // (H * K)
    if out.dtype != torch.bfloat16 or not out.is_contiguous() or out.numel() != M * H * N:
        raise ValueError(f"output must be a contiguous bfloat16 [..., {H}, {N}] tensor")
    if x_in is not None and (x_in.dtype != torch.bfloat16 or not x_in.is_contiguous() or x_in.numel() != M * H * N):
        raise ValueError(f"x_in must be a contiguous bfloat16 [..., {H * N}] tensor")
    _require_cuda("head_gemm", x, out, x_in, weights.w, weights.s)
    _lib.call("tl_head_gemm_bf16", x.data_ptr(), weights.w.data_ptr(), weights.s.data_ptr(),
              x_in.data_ptr() if x_in is not None else None, M, H, N, K, out.data_ptr(), _stream(x))


def convert_projq_wqb(wkv_b: torch.Tensor, wkv_b_scales: torch.Tensor, n_heads: int, nope_dim: int = 128,
                      v_dim: int = 128) -> HeadWeights:
    """The device's kv_b_proj shard [n_heads * (nope + v), kv_lora] (+ fp32 block scales)
    -> each head's nope block [nope, kv_lora] transposed to [kv_lora, nope]."""
    hd = nope_dim + v_dim
    kv = wkv_b.shape[1]
    if wkv_b.shape[0] != n_heads * hd or nope_dim % BLOCK or hd % BLOCK:
        raise ValueError("wkv_b must be [n_heads * (nope + v), kv_lora] with 128-aligned head blocks")
    w = wkv_b.view(torch.uint8).reshape(n_heads, hd, kv)[:, :nope_dim].transpose(1, 2).contiguous()
    s = wkv_b_scales.float().reshape(n_heads, hd // BLOCK, kv // BLOCK)[:, :nope_dim // BLOCK].transpose(1, 2)
    return HeadWeights(w.view(torch.float8_e4m3fn), s.contiguous())


def projq_wqb(q_nope_in: torch.Tensor, wkv_b_a: HeadWeights, wkv_b_a_scales: torch.Tensor | None,
              output: torch.Tensor, profile_logs: torch.Tensor | None = None,
              compute_kernel_type: str = "fp16mma", *, model_arch: str) -> None:
    """q_nope_in bf16 [b, s, heads, nope]; wkv_b_a = ``convert_projq_wqb(...)`` (its scales
    ride along, so ``wkv_b_a_scales`` may be None); output bf16 [b, s, heads, kv_lora].
    ``compute_kernel_type`` ("fp16mma", "bf16mma") is accepted; the kernel runs bf16 MMA."""
    if model_arch not in ("deepseek_v3_2", "glm_5"):
        raise ValueError(f"Unsupported architecture: {model_arch}")
    if compute_kernel_type not in ("fp16mma", "bf16mma"):
        raise ValueError(f"Unsupported compute_kernel_type: {compute_kernel_type}")
    if q_nope_in.shape[-2:] != (wkv_b_a.H, wkv_b_a.K):
        raise ValueError(f"q_nope_in must be [b, s, {wkv_b_a.H}, {wkv_b_a.K}]")
    head_gemm(q_nope_in, wkv_b_a, output)
