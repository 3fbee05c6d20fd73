"""One GPU's share loaded from a checkpoint, checked against the oracle run on the
UNSLICED checkpoint tensors (the loader's rank slicing is pinned by the oracle, not by a
second slicing of the same tensors):

* column-parallel layers (q_b, kv_b): the shard's output equals the oracle's full-layer
  output restricted to the rank's rows;
* the row-parallel o_proj: the fp32 sum of the 8 ranks' partial outputs equals the oracle's
  full-layer output (what the allreduce would produce);
* experts: each EP rank equals the oracle MoE over its own experts, and the sum of the 8
  ranks equals the oracle over all experts;
* the dense MLP and the stacked wq_a + wkv_a projection equal the oracle on the tensors.

The loader reads the reference's HF checkpoint layout (`preprocess/weight_converter.py:243-403`
reads the same names).
"""
import pytest
import torch

from oracle import reference as ref
from tests import _mini_ckpt as mini
from tests._tol import assert_gemm_close
from tilert_amd import kernel as K
from tilert_amd import moe, synth
from tilert_amd.checkpoint import Checkpoint, load_dense_mlp, load_expert_shard, load_mla_shard
from tilert_amd.projx import projx_wqkva

pytestmark = pytest.mark.gpu

TP = 8


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt")
    t = mini.write(str(d))
    return Checkpoint(str(d)), t


def _xq(M, K_, seed):
    return ref.act_quant(synth.activations(M, K_, synth.gen(seed)))


def _rel_l2(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return (torch.norm(a - b) / torch.norm(b)).item()


@pytest.mark.parametrize("rank", [0, 5, 7])
def test_mla_column_parallel_shard_vs_oracle(cuda, ckpt, rank):
    c, t = ckpt
    sh = load_mla_shard(c, 3, rank, TP, cuda, **mini.CFG)
    p = "model.layers.3.self_attn."
    hl = mini.CFG["n_heads"] // TP
    for packed, name, rows in ((sh.wq_b, "q_b_proj", hl * 192), (sh.wkv_b, "kv_b_proj", hl * 256)):
        w, s = t[p + name + ".weight"], t[p + name + ".weight_scale_inv"]
        xq, xs = _xq(4, w.shape[1], 1 + rank)
        want = ref.fp8_gemm(xq, xs, w, s)[:, rank * rows:(rank + 1) * rows]
        assert_gemm_close(K.fp8_gemm(xq.to(cuda), xs.to(cuda), packed), want, f"{name} rank {rank}")
    assert torch.equal(sh.q_norm.cpu(), t[p + "q_a_layernorm.weight"].float())
    assert torch.equal(sh.kv_norm.cpu(), t[p + "kv_a_layernorm.weight"].float())


def test_mla_wqkva_vs_oracle(cuda, ckpt):
    c, t = ckpt
    sh = load_mla_shard(c, 3, 2, TP, cuda, **mini.CFG)
    p = "model.layers.3.self_attn."
    xq, xs = _xq(4, mini.DIM, 9)
    rq, rkv, rpe = ref.projx_wqkva(xq, xs, t[p + "q_a_proj.weight"], t[p + "q_a_proj.weight_scale_inv"],
                                   t[p + "kv_a_proj_with_mqa.weight"], t[p + "kv_a_proj_with_mqa.weight_scale_inv"],
                                   mini.CFG["kv_lora_rank"])
    q = torch.empty(1, 4, mini.Q_LORA, dtype=torch.bfloat16, device=cuda)
    kv = torch.empty(1, 4, mini.CFG["kv_lora_rank"], dtype=torch.bfloat16, device=cuda)
    pe = torch.zeros(1, 8, mini.CFG["qk_rope"], dtype=torch.bfloat16, device=cuda)
    cur = torch.tensor([2], dtype=torch.int32, device=cuda)
    projx_wqkva(xq.reshape(1, 4, -1).to(cuda), xs.reshape(1, 4, -1).to(cuda), sh.wqkva, cur, q, kv, pe, None,
                model_arch="deepseek_v3_2")
    assert_gemm_close(q.reshape(4, -1), rq, "q")
    assert_gemm_close(kv.reshape(4, -1), rkv, "kv")
    assert_gemm_close(pe[0, 2:6], rpe, "pe")


def test_mla_row_parallel_o_proj_sums_to_oracle(cuda, ckpt):
    c, t = ckpt
    p = "model.layers.3.self_attn.o_proj"
    w, s = t[p + ".weight"], t[p + ".weight_scale_inv"]
    xq, xs = _xq(4, w.shape[1], 11)
    want = ref.fp8_gemm(xq, xs, w, s)
    cols = mini.CFG["n_heads"] // TP * mini.CFG["v_head"]
    total = torch.zeros(4, w.shape[0])
    for r in range(TP):
        sh = load_mla_shard(c, 3, r, TP, cuda, **mini.CFG)
        xr = xq[:, r * cols:(r + 1) * cols].contiguous().to(cuda)
        xsr = xs[:, r * cols // 128:(r + 1) * cols // 128].contiguous().to(cuda)
        total += K.fp8_gemm(xr, xsr, sh.wo).float().cpu()
    # 8 bf16-rounded partials summed in fp32: the GEMM's relative bar on the whole output
    assert _rel_l2(total, want) <= 5e-3


def _expert_stacks(t, e0, n):
    out = []
    for k in ("gate_proj", "up_proj", "down_proj"):
        out.append(torch.stack([t[f"model.layers.3.mlp.experts.{e}.{k}.weight"] for e in range(e0, e0 + n)]))
        out.append(torch.stack([t[f"model.layers.3.mlp.experts.{e}.{k}.weight_scale_inv"] for e in range(e0, e0 + n)]))
    return out


def test_expert_shards_vs_oracle(cuda, ckpt):
    c, t = ckpt
    nl = mini.N_EXPERTS // TP
    x = synth.activations(4, mini.DIM, synth.gen(2))
    idx = torch.tensor([[6, 7, 1, 9], [7, 0, 2, 3], [6, 5, 11, 12], [15, 14, 7, 6]], dtype=torch.int32)
    w = torch.softmax(torch.randn(4, 4, generator=synth.gen(3)), -1)
    total = torch.zeros(4, mini.DIM)
    for r in range(TP):
        ex = load_expert_shard(c, 3, r, TP, cuda, n_experts=mini.N_EXPERTS)
        assert ex.expert_begin == r * nl
        y = moe.moe_forward(x.to(cuda), ex, idx.to(cuda), w.to(cuda)).cpu()
        want = ref.moe_forward(x, *_expert_stacks(t, r * nl, nl), idx, w, r * nl)
        if torch.count_nonzero(want):
            assert_gemm_close(y, want, f"expert shard {r}")
        else:
            assert torch.equal(y, want)
        total += y.float()
    full = ref.moe_forward(x, *_expert_stacks(t, 0, mini.N_EXPERTS), idx, w, 0)
    assert _rel_l2(total, full) <= 5e-3


def test_dense_mlp_vs_oracle(cuda, ckpt):
    c, t = ckpt
    mlp = load_dense_mlp(c, 4, cuda)
    for k, packed in mlp.items():
        w, s = t[f"model.layers.4.mlp.{k}.weight"], t[f"model.layers.4.mlp.{k}.weight_scale_inv"]
        xq, xs = _xq(4, w.shape[1], 4)
        assert_gemm_close(K.fp8_gemm(xq.to(cuda), xs.to(cuda), packed), ref.fp8_gemm(xq, xs, w, s), k)
