"""GPU parity of the fused attention down-projection ``projx_wqkva`` (one launch for
x . [wq_a; wkv_a]^T, routed to q, kv and the rope cache) against the CPU oracle of its
golden (projx_wqkva.py:268-294), plus bit-identity with plain fp8_gemm calls."""
import pytest
import torch

from oracle import reference as ref
from tests._tol import assert_gemm_close
from tilert_amd import kernel as K
from tilert_amd import synth
from tilert_amd.projx import ARCH_DIMS, pack_wqkva, projx_wqkva

pytestmark = pytest.mark.gpu

SENTINEL = -12352.0  # bf16-exact (193 * 2^6); marks pe cache rows the call must not touch


def _weights(dim, q_rank, kv_rank, rope, g):
    wq, wqs = ref.weight_quant(synth.weight_fp32(q_rank, dim, g))
    wkv, wkvs = ref.weight_quant(synth.weight_fp32(kv_rank + rope, dim, g))
    return wq, wqs, wkv, wkvs


def _run(cuda, batch, seq, dims, max_len, pos, seed, arch="deepseek_v3_2"):
    dim, q_rank, kv_rank, rope = dims
    g = synth.gen(seed)
    wq, wqs, wkv, wkvs = _weights(dim, q_rank, kv_rank, rope, g)
    xq, xs = ref.act_quant(synth.activations(batch * seq, dim, g))
    xq, xs = xq.reshape(batch, seq, dim), xs.reshape(batch, seq, dim // 128)
    w = pack_wqkva(wq.to(cuda), wqs.to(cuda), wkv.to(cuda), wkvs.to(cuda), kv_rank)
    q = torch.empty(batch, seq, q_rank, dtype=torch.bfloat16, device=cuda)
    kv = torch.empty(batch, seq, kv_rank, dtype=torch.bfloat16, device=cuda)
    cache = torch.full((batch, max_len, rope), SENTINEL, dtype=torch.bfloat16, device=cuda)
    cur = torch.tensor([pos], dtype=torch.int32, device=cuda)
    projx_wqkva(xq.to(cuda), xs.to(cuda), w, cur, q, kv, cache, torch.zeros(1, device=cuda), model_arch=arch)
    torch.cuda.synchronize()
    want = ref.projx_wqkva(xq, xs, wq, wqs, wkv, wkvs, kv_rank)
    return (q, kv, cache), want, (xq, xs, wq, wqs, wkv, wkvs)


@pytest.mark.parametrize("batch,seq,max_len,pos", [(1, 4, 128, 0), (2, 2, 64, 17), (4, 1, 32, 31), (1, 16, 40, 30)])
def test_projx_wqkva_vs_oracle_dsv32(cuda, batch, seq, max_len, pos):
    """DeepSeek-V3.2 widths (7168 -> 1536 | 512 | 64).  The last case puts 6 of 16 tokens
    past the cache end: those rows are dropped and every other cache row keeps its
    sentinel."""
    (q, kv, cache), (wq_, wkv_, wpe_), _ = _run(cuda, batch, seq, ARCH_DIMS["deepseek_v3_2"], max_len, pos, 300 + pos)
    assert_gemm_close(q, wq_, "q")
    assert_gemm_close(kv, wkv_, "kv")
    c = cache.cpu().float()
    for b in range(batch):
        for r in range(max_len):
            s = r - pos
            if 0 <= s < seq:
                assert_gemm_close(c[b, r], wpe_[b, s], f"pe b={b} s={s}")
            else:
                assert torch.all(c[b, r] == SENTINEL), f"cache row b={b} r={r} was written"


def test_projx_wqkva_glm5_widths_and_split_k(cuda):
    """GLM-5 widths (6144 -> 2048 | 512 | 64) at 32 tokens: a narrow layer at M > 16 takes
    the split-K path, whose reduction must route the same way."""
    (q, kv, cache), (wq_, wkv_, wpe_), _ = _run(cuda, 2, 16, ARCH_DIMS["glm_5"], 16, 0, 9, arch="glm_5")
    assert_gemm_close(q, wq_, "q")
    assert_gemm_close(kv, wkv_, "kv")
    assert_gemm_close(cache.cpu(), wpe_, "pe")


def test_projx_wqkva_equals_fp8_gemm_on_stacked_weight(cuda):
    """Same kernel, same plan: the routed outputs are bit-identical to fp8_gemm on the
    stacked weight, column range by column range."""
    dims = ARCH_DIMS["deepseek_v3_2"]
    (q, kv, cache), _, (xq, xs, wq, wqs, wkv, wkvs) = _run(cuda, 1, 4, dims, 8, 2, 5)
    full = K.fp8_gemm(xq.reshape(4, -1).to(cuda), xs.reshape(4, -1).to(cuda),
                      torch.cat([wq, wkv]).to(cuda), torch.cat([wqs, wkvs]).to(cuda))
    torch.cuda.synchronize()
    assert torch.equal(q.reshape(4, -1), full[:, :1536])
    assert torch.equal(kv.reshape(4, -1), full[:, 1536:2048])
    assert torch.equal(cache[0, 2:6], full[:, 2048:])


def test_projx_wqkva_rejects_bad_args(cuda):
    dim, q_rank, kv_rank, rope = 512, 128, 48, 16
    g = synth.gen(1)
    wq, wqs, wkv, wkvs = (t.to(cuda) for t in _weights(dim, q_rank, kv_rank, rope, g))
    w = pack_wqkva(wq, wqs, wkv, wkvs, kv_rank)
    xq = torch.zeros(1, 2, dim, dtype=torch.float8_e4m3fn, device=cuda)
    xs = torch.ones(1, 2, dim // 128, device=cuda)
    q = torch.empty(1, 2, q_rank, dtype=torch.bfloat16, device=cuda)
    kv = torch.empty(1, 2, kv_rank, dtype=torch.bfloat16, device=cuda)
    cache = torch.zeros(1, 8, rope, dtype=torch.bfloat16, device=cuda)
    cur = torch.zeros(1, dtype=torch.int32, device=cuda)
    with pytest.raises(ValueError):
        projx_wqkva(xq, xs, w, cur, q, kv, cache, None, "fp16mma", model_arch="deepseek_v3_2")
    with pytest.raises(ValueError):
        projx_wqkva(xq, xs, w, cur, q[:, :1], kv, cache, None, model_arch="deepseek_v3_2")
    with pytest.raises(ValueError):
        projx_wqkva(xq, xs, w, cur.long(), q, kv, cache, None, model_arch="deepseek_v3_2")
    with pytest.raises(ValueError):
        pack_wqkva(wkv[:, :], wkvs, wkv, wkvs, kv_rank)  # q rows not a multiple of 128
    projx_wqkva(xq, xs, w, cur, q, kv, cache, None, model_arch="deepseek_v3_2")
    torch.cuda.synchronize()
    assert torch.all(q == 0) and torch.all(kv == 0) and torch.all(cache[0, :2] == 0)
