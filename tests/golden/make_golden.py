"""Write the small seeded fixtures under tests/golden/ from the CPU oracle.

The reference ships no golden vectors for this path (no tests directory; its random
weights come from unseeded torch.randn), so these fixtures are this build's own: inputs
and expected outputs of the oracle restatement, pinned by the oracle's tests.  They are
regression anchors for both the oracle (tests/test_golden.py) and the HIP path
(tests/test_gpu_golden.py).  Regenerate with  python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import reference as ref  # noqa: E402
from tilert_amd import synth  # noqa: E402


def u8(t):
    return t.contiguous().view(torch.uint8).numpy()


def bf(t):
    return t.contiguous().view(torch.int16).numpy()


def main() -> None:
    g = synth.gen(2024)
    # act_quant, three scale modes
    x = synth.activations(4, 1024, g) * 3
    d = {"x_bf16": bf(x)}
    for m in (0, 1, 2):
        y, s = ref.act_quant(x, 128, m)
        d[f"y{m}_fp8"], d[f"s{m}"] = u8(y), s.numpy()
    np.savez_compressed(HERE / "act_quant.npz", **d)

    # block-scaled GEMM, M = 4, wkv_a-like partial scale row (N = 192)
    xq, xs = ref.act_quant(synth.activations(4, 512, g))
    wq, ws = ref.weight_quant(synth.weight_fp32(192, 512, g))
    np.savez_compressed(HERE / "fp8_gemm.npz", a_fp8=u8(xq), a_s=xs.numpy(), b_fp8=u8(wq), b_s=ws.numpy(),
                        c_bf16=bf(ref.fp8_gemm(xq, xs, wq, ws)))

    # MoE: 4 local experts (global ids 4..7), D = 256, I = 128, M = 3, top-3
    E, D, I, M = 4, 256, 128, 3
    parts = []
    for (n, k) in ((I, D), (I, D), (D, I)):
        q, s = zip(*[ref.weight_quant(synth.weight_fp32(n, k, g)) for _ in range(E)])
        parts += [torch.stack(q), torch.stack(s)]
    xm = synth.activations(M, D, g)
    idx = torch.tensor([[4, 9, 6], [1, 2, 3], [7, 6, 12]], dtype=torch.int32)
    w = torch.tensor([[0.5, 0.25, 0.25], [0.2, 0.3, 0.5], [0.6, 0.3, 0.1]])
    y = ref.moe_forward(xm, *parts, idx, w, 4)
    np.savez_compressed(HERE / "moe.npz", x_bf16=bf(xm), gate_fp8=u8(parts[0]), gate_s=parts[1].numpy(),
                        up_fp8=u8(parts[2]), up_s=parts[3].numpy(), down_fp8=u8(parts[4]), down_s=parts[5].numpy(),
                        topk_idx=idx.numpy(), topk_w=w.numpy(), expert_begin=np.array(4), y_bf16=bf(y))

    # indexer + top-k: M = 2, H = 64, L = 512, tokens at 509, 510
    q, qs, k, ks, wi = synth.indexer_inputs(2, 64, 512, g)
    logits = ref.indexer_scores(q, qs, k, ks, wi, 509)
    top = ref.topk_rows(logits, [510, 511], 64)
    np.savez_compressed(HERE / "indexer.npz", q_fp8=u8(q), q_s=qs.numpy(), k_fp8=u8(k), k_s=ks.numpy(),
                        w_bf16=bf(wi), cur_pos=np.array(509), logits=logits.numpy(), top64=top.numpy())
    ki_producer()
    sparse_mla()
    print("fixtures written to", HERE)


def ki_producer() -> None:
    """Indexer key producer (LayerNorm -> RoPE -> Hadamard): 9 keys, non-trivial norm
    weight / bias and random RoPE angles."""
    g = synth.gen(2025)
    x = (torch.randn(9, 128, generator=g) * 2 + 0.3).to(torch.bfloat16)
    w = torch.rand(128, generator=g) * 0.2 + 0.9
    b = torch.randn(128, generator=g) * 0.1
    theta = torch.rand(9, 32, generator=g, dtype=torch.float64) * 6.28
    fr = torch.stack([theta.cos(), theta.sin()], dim=-1).reshape(9, 64).float()
    k = ref.layernorm_rope_rotate(x, w, b, fr)
    np.savez_compressed(HERE / "ki_producer.npz", x_bf16=bf(x), weight=w.numpy(), bias=b.numpy(), freqs=fr.numpy(),
                        k_bf16=bf(k))


def sparse_mla() -> None:
    """Sparse MLA attention: 2 tokens, 8 heads, 100 of 160 positions selected per token
    (two splits, the second partial), glm_5's softmax scale."""
    g = synth.gen(2026)
    q = (torch.randn(2, 8, 512, generator=g) * 0.5).to(torch.bfloat16)
    qp = (torch.randn(2, 8, 64, generator=g) * 0.5).to(torch.bfloat16)
    kv = torch.randn(160, 512, generator=g).to(torch.bfloat16)
    pe = torch.randn(160, 64, generator=g).to(torch.bfloat16)
    idx = torch.stack([torch.randperm(159, generator=g)[:100] for _ in range(2)]).to(torch.int32)
    out = ref.flash_sparse_mla(q, qp, kv, pe, idx, 158, ref.mla_softmax_scale("glm_5"))
    np.savez_compressed(HERE / "sparse_mla.npz", q_bf16=bf(q), qpe_bf16=bf(qp), kv_bf16=bf(kv), pe_bf16=bf(pe),
                        indices=idx.numpy(), cur_pos=np.array(158), out_bf16=bf(out))


if __name__ == "__main__":
    main()
