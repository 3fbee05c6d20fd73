"""One GPU's share of a DeepSeek-V3.2-style FP8 checkpoint (Hugging Face safetensors
layout: e4m3fn ``*.weight`` with fp32 ``*.weight_scale_inv`` per 128x128 block), loaded
into the layouts the kernels here run on -- the role of the reference's WeightConverter
(tilert/models/preprocess/weight_converter.py:243-403), which shards each layer's tensors
per device before its per-op converters pack them.

The share is the plain TP / EP layout: attention at tensor-parallel rank ``tp_rank`` of ``tp``
(q_b / kv_b rows and o_proj columns of ``n_heads / tp`` heads, q_a / kv_a replicated) and
experts at expert-parallel rank ``ep_rank`` of ``ep`` (experts ``n_experts / ep * ep_rank``
onwards, whole).  (The reference instead shards each expert's inter dim across devices,
expert_down_allreduce.py:354-377; one GPU's kernels here run the EP=8 share.)  Tensors
are read lazily, slice by slice, so a shard never loads the whole checkpoint.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass

import torch
from safetensors import safe_open

from .kernel import PackedFP8Weight, pack_weight
from .moe import LocalExperts
from .projx import PackedWqkva, pack_wqkva

BLOCK = 128


class Checkpoint:
    """A safetensors checkpoint: one file, or a directory with
    ``model.safetensors.index.json`` (its ``weight_map``) or a single ``*.safetensors``."""

    def __init__(self, path: str) -> None:
        if os.path.isdir(path):
            index = os.path.join(path, "model.safetensors.index.json")
            if os.path.exists(index):
                with open(index) as f:
                    wmap = json.load(f)["weight_map"]
                self._file = {k: os.path.join(path, v) for k, v in wmap.items()}
            else:
                files = sorted(p for p in os.listdir(path) if p.endswith(".safetensors"))
                if not files:
                    raise FileNotFoundError(f"no safetensors files in {path}")
                self._file = {}
                for name in files:
                    with safe_open(os.path.join(path, name), framework="pt") as f:
                        for k in f.keys():
                            self._file[k] = os.path.join(path, name)
        else:
            with safe_open(path, framework="pt") as f:
                self._file = {k: path for k in f.keys()}

    def __contains__(self, name: str) -> bool:
        return name in self._file

    def get(self, name: str, rows: tuple[int, int] | None = None,
            cols: tuple[int, int] | None = None) -> torch.Tensor:
        """The tensor, or its [rows, cols] slice (half-open ranges), read from disk."""
        if name not in self._file:
            raise KeyError(f"{name} is not in the checkpoint")
        with safe_open(self._file[name], framework="pt") as f:
            sl = f.get_slice(name)
            if rows is None and cols is None:
                return sl[:]
            r0, r1 = rows if rows is not None else (0, sl.get_shape()[0])
            if cols is None:
                return sl[r0:r1]
            return sl[r0:r1, cols[0]:cols[1]]

    def fp8(self, name: str, rows: tuple[int, int] | None = None,
            cols: tuple[int, int] | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """An e4m3fn weight slice and the matching rows/columns of its block scales; the
        slice must start on a 128 boundary (block scales are per 128 x 128)."""
        for rng in (rows, cols):
            if rng is not None and rng[0] % BLOCK:
                raise ValueError(f"{name}: slice {rng} does not start on a {BLOCK} boundary")
        w = self.get(name + ".weight", rows, cols)
        if w.dtype != torch.float8_e4m3fn:
            raise ValueError(f"{name}.weight is {w.dtype}, expected float8_e4m3fn")
        srows = None if rows is None else (rows[0] // BLOCK, (rows[1] + BLOCK - 1) // BLOCK)
        scols = None if cols is None else (cols[0] // BLOCK, (cols[1] + BLOCK - 1) // BLOCK)
        s = self.get(name + ".weight_scale_inv", srows, scols).float()
        return w.contiguous(), s.contiguous()


@dataclass
class MlaShard:
    """The attention weights of one layer at one tensor-parallel rank, packed."""
    wqkva: PackedWqkva        # q_a_proj stacked over kv_a_proj_with_mqa (projx_wqkva)
    wq_b: PackedFP8Weight     # q_b_proj rows of this rank's heads
    wkv_b: PackedFP8Weight    # kv_b_proj rows of this rank's heads
    wo: PackedFP8Weight       # o_proj columns of this rank's heads
    q_norm: torch.Tensor      # q_a_layernorm weight, fp32
    kv_norm: torch.Tensor     # kv_a_layernorm weight, fp32


def load_mla_shard(ckpt: Checkpoint, layer: int, tp_rank: int, tp: int, device: torch.device, *,
                   n_heads: int = 128, qk_nope: int = 128, qk_rope: int = 64, v_head: int = 128,
                   kv_lora_rank: int = 512) -> MlaShard:
    """Attention of ``model.layers.{layer}`` at rank ``tp_rank`` of ``tp`` (DeepSeek-V3.2
    defaults, deepseek_v3_2/model_args.py:64-80)."""
    if n_heads % tp:
        raise ValueError(f"n_heads={n_heads} does not split over tp={tp}")
    hl = n_heads // tp
    p = f"model.layers.{layer}.self_attn."
    qa, qa_s = ckpt.fp8(p + "q_a_proj")
    kva, kva_s = ckpt.fp8(p + "kv_a_proj_with_mqa")
    qb_rows = hl * (qk_nope + qk_rope)
    qb, qb_s = ckpt.fp8(p + "q_b_proj", rows=(tp_rank * qb_rows, (tp_rank + 1) * qb_rows))
    kvb_rows = hl * (qk_nope + v_head)
    kvb, kvb_s = ckpt.fp8(p + "kv_b_proj", rows=(tp_rank * kvb_rows, (tp_rank + 1) * kvb_rows))
    o_cols = hl * v_head
    wo, wo_s = ckpt.fp8(p + "o_proj", cols=(tp_rank * o_cols, (tp_rank + 1) * o_cols))

    def dev(t):
        return t.to(device)
    return MlaShard(
        wqkva=pack_wqkva(dev(qa), dev(qa_s), dev(kva), dev(kva_s), kv_lora_rank),
        wq_b=pack_weight(dev(qb), dev(qb_s)),
        wkv_b=pack_weight(dev(kvb), dev(kvb_s)),
        wo=pack_weight(dev(wo), dev(wo_s)),
        q_norm=dev(ckpt.get(p + "q_a_layernorm.weight").float()),
        kv_norm=dev(ckpt.get(p + "kv_a_layernorm.weight").float()),
    )


def load_expert_shard(ckpt: Checkpoint, layer: int, ep_rank: int, ep: int, device: torch.device, *,
                      n_experts: int = 256) -> LocalExperts:
    """The routed experts of ``model.layers.{layer}.mlp`` at rank ``ep_rank`` of ``ep``:
    experts ``n_experts / ep * ep_rank`` .. (whole gate / up / down), packed for the MoE
    kernels; ``expert_begin`` is the first global expert id."""
    if n_experts % ep:
        raise ValueError(f"n_experts={n_experts} does not split over ep={ep}")
    nl = n_experts // ep
    e0 = ep_rank * nl
    parts = {k: ([], []) for k in ("gate_proj", "up_proj", "down_proj")}
    for e in range(e0, e0 + nl):
        for k, (ws, ss) in parts.items():
            w, s = ckpt.fp8(f"model.layers.{layer}.mlp.experts.{e}.{k}")
            ws.append(w)
            ss.append(s)
    t = {k: (torch.stack(ws).to(device), torch.stack(ss).to(device)) for k, (ws, ss) in parts.items()}
    return LocalExperts(*t["gate_proj"], *t["up_proj"], *t["down_proj"], expert_begin=e0)


def load_dense_mlp(ckpt: Checkpoint, layer: int, device: torch.device) -> dict[str, PackedFP8Weight]:
    """The dense MLP of ``model.layers.{layer}`` (gate / up / down, unsharded: the
    7168 <-> 18432 layers of the dense-MLP workload), packed."""
    out = {}
    for k in ("gate_proj", "up_proj", "down_proj"):
        w, s = ckpt.fp8(f"model.layers.{layer}.mlp.{k}")
        out[k] = pack_weight(w.to(device), s.to(device))
    return out
