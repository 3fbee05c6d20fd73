"""One GPU's share loaded from a checkpoint gives bit-identical results to the same
weights sliced and packed by hand."""
import pytest
import torch

from tests import _mini_ckpt as mini
from tilert_amd import kernel as K
from tilert_amd import moe, synth
from tilert_amd.projx import pack_wqkva
from tilert_amd.checkpoint import Checkpoint, load_dense_mlp, load_expert_shard, load_mla_shard

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt")
    t = mini.write(str(d))
    return Checkpoint(str(d)), t


def _x(M, K_, seed, dev):
    return K.act_quant(synth.activations(M, K_, synth.gen(seed)).to(dev))


def test_mla_shard_matches_hand_slices(cuda, ckpt):
    c, t = ckpt
    rank, tp = 5, 8
    sh = load_mla_shard(c, 3, rank, tp, cuda, **mini.CFG)
    p = "model.layers.3.self_attn."
    hl = mini.CFG["n_heads"] // tp
    cases = [(sh.wq_b, p + "q_b_proj", slice(rank * hl * 192, (rank + 1) * hl * 192), None),
             (sh.wkv_b, p + "kv_b_proj", slice(rank * hl * 256, (rank + 1) * hl * 256), None),
             (sh.wo, p + "o_proj", None, slice(rank * hl * 128, (rank + 1) * hl * 128))]
    for packed, name, rs, cs in cases:
        w, s = t[name + ".weight"], t[name + ".weight_scale_inv"]
        if rs is not None:
            w, s = w[rs], s[rs.start // 128:rs.stop // 128]
        else:
            w, s = w[:, cs], s[:, cs.start // 128:cs.stop // 128]
        xq, xs = _x(4, w.shape[1], 1, cuda)
        want = K.fp8_gemm(xq, xs, K.pack_weight(w.contiguous().to(cuda), s.contiguous().to(cuda)))
        assert torch.equal(K.fp8_gemm(xq, xs, packed), want), name
    def d(name):
        return t[p + name + ".weight"].to(cuda), t[p + name + ".weight_scale_inv"].to(cuda)
    want = pack_wqkva(*d("q_a_proj"), *d("kv_a_proj_with_mqa"), mini.CFG["kv_lora_rank"])
    assert torch.equal(sh.wqkva.data, want.data) and torch.equal(sh.wqkva.scale, want.scale)
    assert torch.equal(sh.q_norm.cpu(), t[p + "q_a_layernorm.weight"].float())


def test_expert_shard_matches_hand_slices(cuda, ckpt):
    c, t = ckpt
    rank, ep = 3, 8
    ex = load_expert_shard(c, 3, rank, ep, cuda, n_experts=mini.N_EXPERTS)
    nl = mini.N_EXPERTS // ep
    e0 = rank * nl
    parts = []
    for k in ("gate_proj", "up_proj", "down_proj"):
        parts.append(torch.stack([t[f"model.layers.3.mlp.experts.{e}.{k}.weight"] for e in range(e0, e0 + nl)]).to(cuda))
        parts.append(torch.stack([t[f"model.layers.3.mlp.experts.{e}.{k}.weight_scale_inv"]
                                  for e in range(e0, e0 + nl)]).to(cuda))
    ref_ex = moe.LocalExperts(*parts, expert_begin=e0)
    assert ex.expert_begin == e0
    x = synth.activations(4, mini.DIM, synth.gen(2)).to(cuda)
    idx = torch.tensor([[6, 7, 1, 9], [7, 0, 2, 3], [6, 5, 11, 12], [15, 14, 7, 6]], dtype=torch.int32, device=cuda)
    w = torch.softmax(torch.randn(4, 4, generator=synth.gen(3)), -1).to(cuda)
    assert torch.equal(moe.moe_forward(x, ex, idx, w), moe.moe_forward(x, ref_ex, idx, w))


def test_dense_mlp_matches_hand_packing(cuda, ckpt):
    c, t = ckpt
    mlp = load_dense_mlp(c, 4, cuda)
    for k, packed in mlp.items():
        w, s = t[f"model.layers.4.mlp.{k}.weight"], t[f"model.layers.4.mlp.{k}.weight_scale_inv"]
        xq, xs = _x(4, w.shape[1], 4, cuda)
        assert torch.equal(K.fp8_gemm(xq, xs, packed), K.fp8_gemm(xq, xs, K.pack_weight(w.to(cuda), s.to(cuda)))), k
