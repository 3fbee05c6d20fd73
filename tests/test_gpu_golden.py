"""The HIP path against the committed fixtures (GPU)."""
import pytest
import torch

from tests._golden import bf16, f32, fp8, load
from tests._tol import assert_gemm_close
from tilert_amd import kernel as K
from tilert_amd import moe
from tilert_amd import sparse_index as si
from tilert_amd.topk import topk_rows

pytestmark = pytest.mark.gpu


def test_act_quant_fixture_gpu(cuda):
    d = load("act_quant")
    x = bf16(d["x_bf16"]).to(cuda)
    for m, fmt in ((0, None), (1, "ue8m0"), (2, "div")):
        y, s = K.act_quant(x, 128, fmt)
        assert torch.equal(y.cpu().view(torch.uint8), fp8(d[f"y{m}_fp8"]).view(torch.uint8))
        assert torch.equal(s.cpu(), f32(d[f"s{m}"]))


def test_fp8_gemm_fixture_gpu(cuda):
    d = load("fp8_gemm")
    a, a_s, b, b_s = (fp8(d["a_fp8"]).to(cuda), f32(d["a_s"]).to(cuda), fp8(d["b_fp8"]).to(cuda), f32(d["b_s"]).to(cuda))
    assert_gemm_close(K.fp8_gemm(a, a_s, b, b_s), bf16(d["c_bf16"]), "fixture gemm")
    assert_gemm_close(K.fp8_gemm(a, a_s, K.pack_weight(b, b_s)), bf16(d["c_bf16"]), "fixture gemm packed")


def test_moe_fixture_gpu(cuda):
    d = load("moe")
    ex = moe.LocalExperts(fp8(d["gate_fp8"]).to(cuda), f32(d["gate_s"]).to(cuda), fp8(d["up_fp8"]).to(cuda),
                          f32(d["up_s"]).to(cuda), fp8(d["down_fp8"]).to(cuda), f32(d["down_s"]).to(cuda),
                          expert_begin=int(d["expert_begin"]))
    y = moe.moe_forward(bf16(d["x_bf16"]).to(cuda), ex, torch.from_numpy(d["topk_idx"]).to(cuda),
                        f32(d["topk_w"]).to(cuda))
    assert_gemm_close(y, bf16(d["y_bf16"]), "fixture moe")


def test_indexer_fixture_gpu(cuda):
    d = load("indexer")
    logits = torch.empty(2, 512, device=cuda)
    si.sparse_index_fp8(fp8(d["q_fp8"]).to(cuda), f32(d["q_s"]).to(cuda), fp8(d["k_fp8"]).to(cuda),
                    f32(d["k_s"]).to(cuda), bf16(d["w_bf16"]).to(cuda), logits, int(d["cur_pos"]))
    want = f32(d["logits"])
    got = logits.cpu()
    assert torch.equal(torch.isinf(got), torch.isinf(want))
    fin = torch.isfinite(want)
    assert ((got[fin] - want[fin]).abs().max() / want[fin].abs().max()) < 1e-4
    idx = topk_rows(f32(d["logits"]).to(cuda), 509, 64).cpu()
    for i in range(2):  # fixture order is by score; ours is ascending column
        assert torch.equal(idx[i].sort().values, torch.from_numpy(d["top64"][i]).sort().values)


def test_ki_producer_fixture_gpu(cuda):
    from tilert_amd.layernorm_rope_rotate import layernorm_rope_rotate
    d = load("ki_producer")
    x = bf16(d["x_bf16"])
    n = x.shape[0]
    cache = torch.zeros(1, n, 128, dtype=torch.bfloat16, device=cuda)
    layernorm_rope_rotate(x[None].to(cuda), torch.zeros(1, dtype=torch.int32, device=cuda), cache,
                          f32(d["weight"]).to(cuda), f32(d["bias"]).to(cuda), f32(d["freqs"]).reshape(n, 1, 64).to(cuda),
                          None, "deepseek_v3_2")
    got, want = cache[0].cpu().float(), bf16(d["k_bf16"]).float()
    e = torch.floor(torch.log2(torch.maximum(got.abs(), want.abs()).clamp_min(2.0 ** -126)))
    assert torch.all((got - want).abs() <= torch.pow(2.0, e - 7))  # within one bf16 step
    assert (got == want).float().mean().item() > 0.99


def test_sparse_mla_fixture_gpu(cuda):
    from tilert_amd.flash_sparse_mla import flash_sparse_mla
    d = load("sparse_mla")
    q = bf16(d["q_bf16"])
    out = torch.zeros(1, *q.shape, dtype=torch.bfloat16, device=cuda)
    flash_sparse_mla(q[None].to(cuda), bf16(d["qpe_bf16"])[None].to(cuda), bf16(d["kv_bf16"])[None].to(cuda),
                     bf16(d["pe_bf16"])[None].to(cuda), torch.from_numpy(d["indices"])[None].to(cuda),
                     torch.tensor([int(d["cur_pos"])], dtype=torch.int32, device=cuda), out, None, model_arch="glm_5")
    assert_gemm_close(out[0], bf16(d["out_bf16"]), "sparse_mla fixture")
