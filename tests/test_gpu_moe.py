"""GPU parity of the MoE expert layer against the CPU oracle (the reference's BF16MMA
goldens): gate/up + SwiGLU per hit expert, down + routing-weighted combine."""
import functools

import pytest
import torch

from oracle import reference as ref
from tests._tol import assert_gemm_close
from tilert_amd import moe, synth

pytestmark = pytest.mark.gpu


@functools.lru_cache(maxsize=2)
def _experts(E, D, I, seed):
    g = synth.gen(seed)
    qs = {}
    for name, (n, k) in (("gate", (I, D)), ("up", (I, D)), ("down", (D, I))):
        q, s = zip(*[ref.weight_quant(synth.weight_fp32(n, k, g)) for _ in range(E)])
        qs[name] = (torch.stack(q), torch.stack(s))
    return qs


def _run(M, E, D, I, topk, n_experts, e0, seed, idx=None, w=None):
    cuda = torch.device("cuda:0")
    W = _experts(E, D, I, E + D + I)  # shared by the cases of one shape
    g = synth.gen(seed + 1)
    x = synth.activations(M, D, g)
    if idx is None:
        idx, w = synth.routing(M, n_experts, topk, g)
    ex = moe.LocalExperts(*(t.to(cuda) for t in (W["gate"][0], W["gate"][1], W["up"][0], W["up"][1],
                                                   W["down"][0], W["down"][1])), expert_begin=e0)
    h = moe.ep_gate_up_swiglu(x.to(cuda), idx.to(cuda), ex)
    y = moe.ep_down_combine(h, ex, idx.to(cuda), w.to(cuda))
    rh, hits = ref.moe_gate_up(x, W["gate"][0], W["gate"][1], W["up"][0], W["up"][1], idx, e0)
    ry = ref.moe_down(rh, hits, W["down"][0], W["down"][1], idx, w, e0)
    torch.cuda.synchronize()
    if hits:
        assert_gemm_close(h[: len(hits)], rh, "gate/up+SwiGLU")
    return y.cpu(), ry, hits


@pytest.mark.parametrize("M,E,D,I,topk,n_exp,e0", [
    (4, 8, 512, 256, 8, 32, 0),
    (4, 8, 512, 256, 8, 32, 8),
    (1, 4, 1024, 512, 8, 16, 4),
    (16, 8, 256, 384, 4, 16, 8),
    (3, 32, 7168, 2048, 8, 256, 32),  # config 2 shapes (shard 1 of 8), odd M
    (4, 32, 7168, 2048, 8, 256, 32),  # config 2: M = 4, shard 1 of 8
    (4, 32, 7168, 2048, 8, 256, 224),  # config 2: M = 4, shard 7 of 8
    (4, 32, 7168, 2048, 8, 32, 0),  # every expert local: ~20 hits, several down batches,
                                    # more gate/up items than gate/up workgroups
    (16, 8, 512, 256, 8, 32, 0),  # 128 routed pairs: the kernels without LDS activations
    (8, 4, 7168, 256, 2, 16, 0),  # x [8, 7168] exceeds 64 KB: gate/up without LDS, down with
])
def test_moe_vs_oracle(cuda, M, E, D, I, topk, n_exp, e0):
    y, ry, hits = _run(M, E, D, I, topk, n_exp, e0, seed=M * 1000 + E + D + e0)
    if hits:
        assert_gemm_close(y, ry, "moe output")
    else:
        assert torch.equal(y, torch.zeros_like(y))


def test_moe_no_local_hits_gives_zero(cuda):
    idx = torch.tensor([[20, 21], [22, 23]], dtype=torch.int32)
    w = torch.full((2, 2), 0.5)
    y, ry, hits = _run(2, 8, 256, 256, 2, 32, 0, seed=5, idx=idx, w=w)
    assert hits == [] and torch.equal(y, torch.zeros_like(y))


def test_moe_unrouted_token_zero_and_shared_expert(cuda):
    """token 0 hits local experts 1 and 3, token 1 none, token 2 only expert 1."""
    idx = torch.tensor([[1, 3, 20], [17, 18, 19], [30, 1, 25]], dtype=torch.int32)
    w = torch.tensor([[0.5, 0.25, 0.25], [0.3, 0.3, 0.4], [0.2, 0.7, 0.1]])
    y, ry, hits = _run(3, 8, 512, 256, 3, 32, 0, seed=6, idx=idx, w=w)
    assert hits == [1, 3]
    assert torch.equal(y[1], torch.zeros_like(y[1]))
    assert_gemm_close(y, ry, "moe output")
