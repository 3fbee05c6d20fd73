"""GPU parity of the indexer + exact top-k as one call (sparse_index_topk,
ops/sparse_index.py:72-128) and of the reference's bf16 indexer operators (sparse_index, sparse_index_topk and GLM-5's
sparse_index_topk_v3, glm_5/ops/sparse_index_v3.py:10-51).

Two checks per call:
* the logits against the CPU oracle (fp8: ``indexer_scores``; bf16: ``indexer_scores_bf16``);
* the indices against the oracle's exact top-k (``topk_rows``: descending score, ties to the
  lowest column) applied to the kernel's OWN logits -- the selection contract is exact
  whatever the scoring rounding, so the sets must be identical, ties included.
Each case prints its name first, so a failure names its shape."""
import pytest
import torch

from oracle import reference as ref
from tilert_amd import sparse_index as si
from tilert_amd import synth
from tilert_amd.sparse_index_v3 import sparse_index_topk_v3

pytestmark = pytest.mark.gpu


def _scores_close(out, want, tol):
    out, want = out.cpu(), want.cpu()
    assert torch.equal(torch.isinf(out), torch.isinf(want))
    fin = torch.isfinite(want)
    scale = want[fin].abs().max().clamp_min(1e-30)
    err = ((out[fin] - want[fin]).abs().max() / scale).item()
    assert err < tol, f"max error {err:.3e} of the score scale"


def _assert_exact_selection(idx, logits, cur_pos, k, L):
    """indices == the exact top-k (as a set, ascending, -1 padded) of each row's visible
    logits as the kernel computed them."""
    idx, logits = idx.cpu(), logits.cpu()
    M = idx.shape[0]
    valid = [min(L, cur_pos + 1 + t) for t in range(M)]
    want = ref.topk_rows(logits[:, :L], valid, k)
    for t in range(M):
        n = min(k, valid[t])
        got = idx[t]
        assert torch.all(got[n:] == -1), f"row {t}: padding"
        sel = got[:n].long()
        assert torch.all(sel[1:] > sel[:-1]), f"row {t}: indices must be strictly ascending"
        assert torch.equal(sel, want[t, :n].long().sort().values), f"row {t}: selection differs"


def _fp8_case(M, H, L, seed, per_head=False):
    g = synth.gen(seed)
    q, qs, k, ks, w = synth.indexer_inputs(M, H, L, g)
    if per_head:
        qs = (torch.rand(M, H, generator=g) + 0.5) * qs[:, None]
    return q, qs.contiguous(), k, ks, w


@pytest.mark.parametrize("M,L,cur_pos,k,per_head", [
    (4, 131072, 131068, 2048, False),  # the indexer workload (config 4)
    (4, 5000, 4996, 2048, False),      # two chunks, the second partial
    (1, 1500, 1499, 2048, False),      # fewer visible keys than k: all of them, then -1
    (3, 9000, 3000, 2048, True),       # masked tail: keys past cur_pos + 2 are never read
    (2, 70000, 69990, 512, False),
    (4, 12305, 12301, 1024, True),     # 4 chunks, last holds 17 keys
    (2, 262136, 262134, 2048, False),  # the widest logits rows the top-k takes (ld = 262144)
])
def test_fp8_sparse_index_topk(cuda, M, L, cur_pos, k, per_head):
    print(f"fp8 topk M={M} L={L} cur_pos={cur_pos} k={k}", flush=True)
    q, qs, kk, ks, w = _fp8_case(M, 64, L, M * 1000 + L, per_head)
    ld = (L + 8 + 3) // 4 * 4  # the top-k reads 16-byte rows
    logits = torch.full((M, ld), 7.0, device=cuda)
    idx = torch.full((M, k), -7, dtype=torch.int32, device=cuda)
    si.sparse_index_topk_fp8(q.to(cuda), qs.to(cuda), kk.to(cuda), ks.to(cuda), w.to(cuda), logits, idx, cur_pos)
    want = ref.indexer_scores(q, qs, kk, ks, w, cur_pos)
    _scores_close(logits[:, :L], want, 1e-4)
    assert torch.all(logits[:, L:].cpu() == 7.0), "columns past L must be untouched"
    _assert_exact_selection(idx, logits, cur_pos, k, L)


def _clustered_fp8(M, L, hot, seed):
    """Keys whose top scores crowd into one region (keys in `hot` are aligned with every
    query head): the selection's per-chunk candidate sets are far from uniform."""
    g = synth.gen(seed)
    u = torch.randn(128, generator=g)
    q32 = u[None, None, :] + 0.3 * torch.randn(M, 64, 128, generator=g)
    qq, qs = synth.per_row_quant_e4m3(q32.reshape(M, -1))
    k32 = torch.randn(L, 128, generator=g)
    k32[hot] += 3.0 * u
    kq, ks = synth.per_row_quant_e4m3(k32)
    w = (torch.rand(M, 64, generator=g) / 8).to(torch.bfloat16)  # positive: aligned keys score high
    return qq.reshape(M, 64, 128), qs, kq, ks, w


@pytest.mark.parametrize("L,hot", [
    (131072, slice(131072 - 3000, 131072)),  # recency: the top 2048 all in the last chunk
    (131072, slice(40000, 46000)),            # one band across two chunks
    (20000, slice(0, 20000, 7)),              # spread: nothing deficient
])
def test_topk_clustered_scores_stay_exact(cuda, L, hot):
    print(f"fp8 clustered L={L} hot={hot}", flush=True)
    M, k = 4, 2048
    q, qs, kk, ks, w = _clustered_fp8(M, L, hot, L)
    logits = torch.empty(M, L, device=cuda)
    idx = torch.empty(M, k, dtype=torch.int32, device=cuda)
    si.sparse_index_topk_fp8(q.to(cuda), qs.to(cuda), kk.to(cuda), ks.to(cuda), w.to(cuda), logits, idx, L - M)
    _scores_close(logits, ref.indexer_scores(q, qs, kk, ks, w, L - M), 1e-4)
    _assert_exact_selection(idx, logits, L - M, k, L)


def test_topk_ties_take_lowest_columns(cuda):
    """Duplicated keys give exactly tied scores across chunks: the tie at the threshold goes
    to the lowest columns."""
    print("fp8 ties", flush=True)
    M, L, k = 2, 30000, 2048
    q, qs, kk, ks, w = _fp8_case(M, 64, L, 5)
    kk[1::2] = kk[0::2][: kk[1::2].shape[0]]  # every odd key repeats the key before it
    ks[1::2] = ks[0::2][: ks[1::2].shape[0]]
    logits = torch.empty(M, L, device=cuda)
    idx = torch.empty(M, k, dtype=torch.int32, device=cuda)
    si.sparse_index_topk_fp8(q.to(cuda), qs.to(cuda), kk.to(cuda), ks.to(cuda), w.to(cuda), logits, idx, L - M)
    lg = logits.cpu()
    assert torch.equal(lg[:, 1:L - 2:2], lg[:, 0:L - 3:2]), "duplicated keys must score identically"
    _assert_exact_selection(idx, logits, L - M, k, L)


def test_topk_repeatable_and_shares_its_workspace(cuda):
    """The workspace is left reusable: repeated calls and calls of other shapes in between
    (one workspace) give identical results."""
    print("fp8 repeat", flush=True)
    cases = []
    for M, L, k in ((4, 131072, 2048), (2, 9000, 512), (3, 40000, 1024)):
        q, qs, kk, ks, w = (t.to(cuda) for t in _fp8_case(M, 64, L, 11 * L))
        cases.append((q, qs, kk, ks, w, L, M, k))
    outs = {}
    for rep in range(6):
        for j, (q, qs, kk, ks, w, L, M, k) in enumerate(cases):
            logits = torch.empty(M, L, device=cuda)
            idx = torch.empty(M, k, dtype=torch.int32, device=cuda)
            si.sparse_index_topk_fp8(q, qs, kk, ks, w, logits, idx, L - M)
            if rep == 0:
                outs[j] = idx
                _assert_exact_selection(idx, logits, L - M, k, L)
            else:
                assert torch.equal(idx, outs[j]), (rep, j)


def test_topk_graph_replays_match_eager(cuda):
    print("fp8 graph", flush=True)
    M, L, k = 4, 65536, 2048
    caches = [tuple(t.to(cuda) for t in _fp8_case(M, 64, L, 300 + i)) for i in range(3)]
    logits = torch.empty(M, L, device=cuda)
    idx = torch.empty(3, M, k, dtype=torch.int32, device=cuda)

    def run():
        for i, (q, qs, kk, ks, w) in enumerate(caches):
            si.sparse_index_topk_fp8(q, qs, kk, ks, w, logits, idx[i], L - M)
    run()
    torch.cuda.synchronize()
    eager = idx.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    for _ in range(4):
        idx.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(idx, eager)


# ------------------------------------------------------------ the bf16 operators
def _bf16_case(M, H, L, seed):
    g = synth.gen(seed)
    q = torch.randn(1, M, H, 128, generator=g).to(torch.bfloat16)
    kv = torch.randn(1, L, 128, generator=g).to(torch.bfloat16)
    w = (torch.randn(1, M, H, generator=g) / 8).to(torch.bfloat16)
    return q, kv, w


@pytest.mark.parametrize("M,H,L,cur_pos", [
    (4, 64, 4096, 4092), (1, 64, 1000, 999), (3, 64, 20000, 9000), (2, 32, 3000, 100), (8, 32, 1536, 1530),
    (4, 32, 70000, 69996), (4, 64, 131072, 131068),
])
def test_bf16_sparse_index_vs_oracle(cuda, M, H, L, cur_pos):
    print(f"bf16 scores M={M} H={H} L={L}", flush=True)
    q, kv, w = _bf16_case(M, H, L, M + H + L)
    logits = torch.full((1, M, L + 8), 7.0, device=cuda)
    si.sparse_index(q.to(cuda), kv.to(cuda), w.to(cuda), logits, cur_pos, None, model_arch="deepseek_v3_2")
    want = ref.indexer_scores_bf16(q[0], kv[0], w[0], cur_pos, si.score_scale(H))
    _scores_close(logits[0, :, :L], want, 2e-5)
    assert torch.all(logits[0, :, L:].cpu() == 7.0)


@pytest.mark.parametrize("M,L,cur_pos,k", [(4, 131072, 131068, 2048), (4, 20000, 19996, 2048), (2, 3000, 1000, 2048),
                                           (1, 65536, 65535, 2048)])
def test_bf16_sparse_index_topk_dsv32(cuda, M, L, cur_pos, k):
    print(f"bf16 topk dsv32 M={M} L={L}", flush=True)
    q, kv, w = _bf16_case(M, 64, L, 7 * L + M)
    logits = torch.empty(1, M, L + 8, device=cuda)
    idx = torch.empty(1, M, k, dtype=torch.int32, device=cuda)
    si.sparse_index_topk(q.to(cuda), kv.to(cuda), w.to(cuda), logits, idx, cur_pos, None)
    _scores_close(logits[0, :, :L], ref.indexer_scores_bf16(q[0], kv[0], w[0], cur_pos, si.score_scale(64)), 2e-5)
    _assert_exact_selection(idx[0], logits[0], cur_pos, k, L)


@pytest.mark.parametrize("M,L,cur_pos,k", [(4, 131072, 131068, 2048), (2, 8000, 7998, 2048), (3, 50000, 20000, 1024)])
def test_bf16_sparse_index_topk_v3_glm5(cuda, M, L, cur_pos, k):
    print(f"bf16 topk v3 M={M} L={L}", flush=True)
    q, kv, w = _bf16_case(M, 32, L, 11 * L + M)
    logits = torch.empty(1, M, L + 8, device=cuda)
    idx = torch.empty(1, M, k, dtype=torch.int32, device=cuda)
    sparse_index_topk_v3(q.to(cuda), kv.to(cuda), w.to(cuda), logits, idx, cur_pos, None)
    _scores_close(logits[0, :, :L], ref.indexer_scores_bf16(q[0], kv[0], w[0], cur_pos, si.score_scale(32)), 2e-5)
    _assert_exact_selection(idx[0], logits[0], cur_pos, k, L)


def test_bf16_operators_keep_the_reference_checks(cuda):
    q, kv, w = (t.to(cuda) for t in _bf16_case(4, 64, 1024, 1))
    logits = torch.empty(1, 4, 1024, device=cuda)
    idx = torch.empty(1, 4, 2048, dtype=torch.int32, device=cuda)
    with pytest.raises(ValueError, match="input must be a bfloat16 tensor"):
        si.sparse_index(q.float(), kv, w, logits, 1000, None, model_arch="deepseek_v3_2")
    with pytest.raises(ValueError, match="kv must be a bfloat16 tensor"):
        si.sparse_index_topk(q, kv.float(), w, logits, idx, 1000, None)
    with pytest.raises(ValueError, match="logits must be a float32 tensor"):
        si.sparse_index_topk(q, kv, w, logits.half(), idx, 1000, None)
    with pytest.raises(ValueError, match="supports head number of 64"):
        si.sparse_index_topk(q[:, :, :32].contiguous(), kv, w[:, :, :32].contiguous(), logits, idx, 1000, None)
    with pytest.raises(ValueError, match="supports head number of 32"):
        sparse_index_topk_v3(q, kv, w, logits, idx, 1000, None)
    with pytest.raises(ValueError, match="dim must be 128"):
        si.sparse_index(q[..., :64].contiguous(), kv, w, logits, 1000, None, model_arch="deepseek_v3_2")
    with pytest.raises(ValueError, match="same device"):
        si.sparse_index(q, kv.cpu(), w, logits, 1000, None, model_arch="deepseek_v3_2")
