"""The oracle reproduces the committed fixtures bit for bit (CPU)."""
import torch

from oracle import reference as ref
from tests._golden import bf16, f32, fp8, load


def test_act_quant_fixture():
    d = load("act_quant")
    x = bf16(d["x_bf16"])
    for m in (0, 1, 2):
        y, s = ref.act_quant(x, 128, m)
        assert torch.equal(y.view(torch.uint8), fp8(d[f"y{m}_fp8"]).view(torch.uint8))
        assert torch.equal(s, f32(d[f"s{m}"]))


def test_fp8_gemm_fixture():
    d = load("fp8_gemm")
    c = ref.fp8_gemm(fp8(d["a_fp8"]), f32(d["a_s"]), fp8(d["b_fp8"]), f32(d["b_s"]))
    assert torch.equal(c, bf16(d["c_bf16"]))


def test_moe_fixture():
    d = load("moe")
    y = ref.moe_forward(bf16(d["x_bf16"]), fp8(d["gate_fp8"]), f32(d["gate_s"]), fp8(d["up_fp8"]),
                        f32(d["up_s"]), fp8(d["down_fp8"]), f32(d["down_s"]), torch.from_numpy(d["topk_idx"]),
                        f32(d["topk_w"]), int(d["expert_begin"]))
    assert torch.equal(y, bf16(d["y_bf16"]))


def test_indexer_fixture():
    d = load("indexer")
    lg = ref.indexer_scores(fp8(d["q_fp8"]), f32(d["q_s"]), fp8(d["k_fp8"]), f32(d["k_s"]),
                            bf16(d["w_bf16"]), int(d["cur_pos"]))
    assert torch.equal(lg, f32(d["logits"]))
    assert torch.equal(ref.topk_rows(lg, [510, 511], 64), torch.from_numpy(d["top64"]))


def test_ki_producer_fixture():
    d = load("ki_producer")
    k = ref.layernorm_rope_rotate(bf16(d["x_bf16"]), f32(d["weight"]), f32(d["bias"]), f32(d["freqs"]))
    assert torch.equal(k, bf16(d["k_bf16"]))


def test_sparse_mla_fixture():
    d = load("sparse_mla")
    out = ref.flash_sparse_mla(bf16(d["q_bf16"]), bf16(d["qpe_bf16"]), bf16(d["kv_bf16"]), bf16(d["pe_bf16"]),
                               torch.from_numpy(d["indices"]), int(d["cur_pos"]), ref.mla_softmax_scale("glm_5"))
    assert torch.equal(out, bf16(d["out_bf16"]))
