"""A small DeepSeek-V3.2-style FP8 checkpoint (HF names, two safetensors shards + index)
for the loader tests: 32 heads (4 per rank at tp=8), q_lora 512, kv_lora 512 + 64 rope,
hidden 1024, 16 experts (2 per rank at ep=8) of inter 512, a dense MLP of inter 2048."""
import json
import os

import torch
from safetensors.torch import save_file

from oracle import reference as ref
from tilert_amd import synth

CFG = dict(n_heads=32, qk_nope=128, qk_rope=64, v_head=128, kv_lora_rank=512)
DIM, Q_LORA, N_EXPERTS, MOE_INTER, INTER = 1024, 512, 16, 512, 2048


def write(path: str, layer: int = 3) -> dict:
    g = synth.gen(7)
    t = {}

    def fp8(name, n, k):
        q, s = ref.weight_quant(synth.weight_fp32(n, k, g))
        t[name + ".weight"], t[name + ".weight_scale_inv"] = q, s

    p = f"model.layers.{layer}."
    h = CFG["n_heads"]
    fp8(p + "self_attn.q_a_proj", Q_LORA, DIM)
    fp8(p + "self_attn.kv_a_proj_with_mqa", CFG["kv_lora_rank"] + CFG["qk_rope"], DIM)
    fp8(p + "self_attn.q_b_proj", h * (CFG["qk_nope"] + CFG["qk_rope"]), Q_LORA)
    fp8(p + "self_attn.kv_b_proj", h * (CFG["qk_nope"] + CFG["v_head"]), CFG["kv_lora_rank"])
    fp8(p + "self_attn.o_proj", DIM, h * CFG["v_head"])
    t[p + "self_attn.q_a_layernorm.weight"] = torch.rand(Q_LORA, generator=g).to(torch.bfloat16)
    t[p + "self_attn.kv_a_layernorm.weight"] = torch.rand(CFG["kv_lora_rank"], generator=g).to(torch.bfloat16)
    for e in range(N_EXPERTS):
        fp8(p + f"mlp.experts.{e}.gate_proj", MOE_INTER, DIM)
        fp8(p + f"mlp.experts.{e}.up_proj", MOE_INTER, DIM)
        fp8(p + f"mlp.experts.{e}.down_proj", DIM, MOE_INTER)
    q = f"model.layers.{layer + 1}.mlp."
    fp8(q + "gate_proj", INTER, DIM)
    fp8(q + "up_proj", INTER, DIM)
    fp8(q + "down_proj", DIM, INTER)
    names = sorted(t)
    half = len(names) // 2
    shards = {"model-00001-of-00002.safetensors": names[:half], "model-00002-of-00002.safetensors": names[half:]}
    wmap = {}
    for fname, ks in shards.items():
        save_file({k: t[k].contiguous() for k in ks}, os.path.join(path, fname))
        wmap.update({k: fname for k in ks})
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wmap}, f)
    return t
