"""Pins of the torch-CPU oracle (oracle/reference.py) against closed forms, invariants
and fp64 brute force -- CPU only, each check chosen so a plausible slip (dropped scale,
transposed operand, wrong index, sign error) fails it."""
import math

import numpy as np
import pytest
import torch

from oracle import brute, fp8
from oracle import reference as ref
from tilert_amd import synth


# --------------------------------------------------------------------------- act_quant
def test_act_quant_zero_group_scale_and_codes():
    y, s = ref.act_quant(torch.zeros(2, 256, dtype=torch.bfloat16))
    assert torch.all(s == torch.tensor(1e-4, dtype=torch.float32) * torch.tensor(1 / 448, dtype=torch.float32))
    assert torch.all(y.view(torch.uint8) == 0)


def test_act_quant_group_max_maps_to_448_and_scale_formula():
    g = synth.gen(1)
    x = synth.activations(8, 512, g)
    y, s = ref.act_quant(x)
    yf = y.float().reshape(8, 4, 128)
    assert torch.all(yf.abs().amax(-1) == 448.0)
    amax = x.float().reshape(8, 4, 128).abs().amax(-1)
    assert torch.equal(s, amax * torch.tensor(1 / 448, dtype=torch.float32))


def test_act_quant_matches_independent_numpy_codec():
    g = synth.gen(2)
    x = synth.activations(16, 1024, g) * 3
    for mode in (0, 1, 2):
        y, s = ref.act_quant(x, 128, mode)
        xf = x.float().numpy().reshape(16, 8, 128)
        q = fp8.encode(np.clip(xf / s.numpy()[..., None], -448, 448)).reshape(16, 1024)
        assert np.array_equal(q, y.view(torch.uint8).numpy())


def test_act_quant_ue8m0_is_smallest_power_of_two_covering_amax():
    g = synth.gen(3)
    x = synth.activations(4, 1024, g) * 10
    _, s = ref.act_quant(x, 128, ref.SCALE_MODE_UE8M0)
    amax = x.float().reshape(4, 8, 128).abs().amax(-1)
    target = amax * torch.tensor(1 / 448, dtype=torch.float32)
    e = torch.log2(s)
    assert torch.all(e == torch.round(e))          # power of two
    assert torch.all(s >= target) and torch.all(s / 2 < target)


# ----------------------------------------------------------------- weights and GEMM
def test_weight_quant_dequant_error_bound_and_partial_blocks():
    w = synth.weight_fp32(300, 520, synth.gen(4))
    q, s = ref.weight_quant(w)
    assert s.shape == (3, 5)
    d = ref.weight_dequant(q, s)
    # e4m3 has 3 mantissa bits: relative rounding error <= 2^-4 for normals
    blk = s.repeat_interleave(128, 0)[:300].repeat_interleave(128, 1)[:, :520]
    assert torch.all((d - w).abs() <= blk * 448 * 2.0 ** -4 + blk * 2.0 ** -9)
    zq, zs = ref.weight_quant(torch.zeros(128, 128))
    assert zs.item() == 1.0 and torch.all(ref.weight_dequant(zq, zs) == 0)


@pytest.mark.parametrize("M,N,K", [(1, 16, 128), (3, 32, 256), (2, 130, 384)])
def test_fp8_gemm_vs_fp64_brute_force(M, N, K):
    g = synth.gen(M * N + K)
    xq, xs = ref.act_quant(synth.activations(M, K, g))
    wq, ws = ref.weight_quant(synth.weight_fp32(N, K, g))
    want = brute.gemm_fp64(xq.view(torch.uint8).numpy(), xs.numpy(), wq.view(torch.uint8).numpy(), ws.numpy())
    got = ref.fp8_gemm(xq, xs, wq, ws).double().numpy()
    # the oracle rounds to bf16 once: within half a bf16 ulp (+ fp32 accumulation)
    ulp = 2.0 ** (np.floor(np.log2(np.abs(want) + 1e-30)) - 7)
    assert np.all(np.abs(got - want) <= 0.5 * ulp + 1e-6 * np.abs(want) + 1e-30)


def test_fp8_gemm_scale_linearity_and_transpose_sensitivity():
    g = synth.gen(5)
    xq, xs = ref.act_quant(synth.activations(4, 512, g))
    wq, ws = ref.weight_quant(synth.weight_fp32(256, 512, g))
    base = ref.fp8_gemm(xq, xs, wq, ws)
    assert torch.equal(ref.fp8_gemm(xq, xs, wq, ws * 2), base * 2)   # exact: power of two
    assert torch.equal(ref.fp8_gemm(xq, xs * 4, wq, ws), base * 4)
    ws2 = ws.clone()
    ws2[1, 0] *= 2  # scale of rows 128..255, K block 0 only
    out = ref.fp8_gemm(xq, xs, wq, ws2)
    assert torch.equal(out[:, :128], base[:, :128]) and not torch.equal(out[:, 128:], base[:, 128:])


def test_projx_wqkva_parts_vs_fp64_brute_force():
    """q, kv and pe are the three column ranges of x . [wq_a; wkv_a]^T: each is checked
    against fp64 brute force over the whole of its weight (so a wrong latent/rope split
    row or a shifted scale row fails)."""
    g = synth.gen(77)
    xq, xs = ref.act_quant(synth.activations(3, 256, g))
    wq, wqs = ref.weight_quant(synth.weight_fp32(128, 256, g))
    wkv, wkvs = ref.weight_quant(synth.weight_fp32(160, 256, g) * 3)  # 2 scale rows, the second partial
    q, kv, pe = ref.projx_wqkva(xq, xs, wq, wqs, wkv, wkvs, kv_lora_rank=144)
    assert q.shape == (3, 128) and kv.shape == (3, 144) and pe.shape == (3, 16)
    xc, xsn = xq.view(torch.uint8).numpy(), xs.numpy()
    want_q = brute.gemm_fp64(xc, xsn, wq.view(torch.uint8).numpy(), wqs.numpy())
    want_kv = brute.gemm_fp64(xc, xsn, wkv.view(torch.uint8).numpy(), wkvs.numpy())
    for got, want in ((q, want_q), (kv, want_kv[:, :144]), (pe, want_kv[:, 144:])):
        got = got.double().numpy()
        ulp = 2.0 ** (np.floor(np.log2(np.abs(want) + 1e-30)) - 7)
        assert np.all(np.abs(got - want) <= 0.5 * ulp + 1e-6 * np.abs(want) + 1e-30)


# ----------------------------------------------------------------------------- MoE
def _tiny_experts(E, D, I, g):
    out = []
    for (n, k) in ((I, D), (I, D), (D, I)):
        q, s = zip(*[ref.weight_quant(synth.weight_fp32(n, k, g)) for _ in range(E)])
        out += [torch.stack(q), torch.stack(s)]
    return out


def test_moe_vs_fp64_per_pair():
    E, D, I, M = 4, 256, 128, 3
    g = synth.gen(6)
    gq, gs, uq, us, dq, ds = _tiny_experts(E, D, I, g)
    x = synth.activations(M, D, g)
    idx = torch.tensor([[0, 9, 2], [7, 8, 9], [2, 3, 11]], dtype=torch.int32)
    w = torch.tensor([[0.5, 0.3, 0.2], [0.4, 0.4, 0.2], [0.1, 0.6, 0.3]])
    y = ref.moe_forward(x, gq, gs, uq, us, dq, ds, idx, w, 0)
    xd = x.double()
    want = torch.zeros(M, D, dtype=torch.float64)
    for t in range(M):
        for j in range(3):
            e = int(idx[t, j])
            if e >= E:
                continue
            G = ref.weight_dequant(gq[e], gs[e]).to(torch.bfloat16).double()
            U = ref.weight_dequant(uq[e], us[e]).to(torch.bfloat16).double()
            Dw = ref.weight_dequant(dq[e], ds[e]).to(torch.bfloat16).double()
            gg, uu = xd[t] @ G.T, xd[t] @ U.T
            h = (gg / (1 + torch.exp(-gg)) * uu).to(torch.bfloat16).double()
            want[t] += float(w[t, j]) * (h @ Dw.T)
    assert torch.all(y[1] == 0)  # token 1 routes to no local expert
    rel = (y.double() - want).norm() / want.norm()
    assert rel < 3e-3


# ------------------------------------------------------------------------- indexer
@pytest.mark.parametrize("per_head", [False, True])
def test_indexer_vs_fp64_brute_force(per_head):
    M, H, L, cur = 2, 32, 40, 35
    g = synth.gen(7)
    q, qs, k, ks, w = synth.indexer_inputs(M, H, L, g)
    if per_head:
        qs = (torch.rand(M, H, generator=g) + 0.5) * qs[:, None]
    got = ref.indexer_scores(q, qs, k, ks, w, cur).double().numpy()
    want = brute.indexer_fp64(q.view(torch.uint8).numpy(), qs.numpy(), k.view(torch.uint8).numpy(),
                              ks.numpy(), w.float().numpy(), cur)
    assert np.array_equal(np.isinf(got), np.isinf(want))
    fin = np.isfinite(want)
    assert np.abs(got[fin] - want[fin]).max() <= 1e-5 * np.abs(want[fin]).max()
    assert np.isinf(got[0, cur + 1:]).all() and np.isfinite(got[1, : cur + 2]).all()


def test_indexer_scale_factoring_identity():
    """s_k scales scores linearly (positive scales commute with ReLU)."""
    g = synth.gen(8)
    q, qs, k, ks, w = synth.indexer_inputs(2, 64, 64, g)
    a = ref.indexer_scores(q, qs, k, ks, w, 63)
    b = ref.indexer_scores(q, qs, k, ks * 4, w, 63)
    assert torch.allclose(b, a * 4, rtol=1e-6, atol=0)


def test_bf16_indexer_vs_fp64_brute_force_and_one_hot():
    """The bf16 indexer against fp64 loops over (token, key, head), the causal -inf
    pattern, the score scale as a plain factor, and a one-hot query/weight that must read
    one key element back (a transposed contraction or a wrong head index fails it)."""
    M, H, L, cur, sc = 3, 32, 50, 44, 0.0625
    g = synth.gen(10)
    q = torch.randn(M, H, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(L, 128, generator=g).to(torch.bfloat16)
    w = (torch.randn(M, H, generator=g) / 8).to(torch.bfloat16)
    got = ref.indexer_scores_bf16(q, k, w, cur, sc).double()
    qd, kd, wd = q.double(), k.double(), w.double()
    for t in range(M):
        for l in range(L):
            if l > cur + t:
                assert got[t, l] == float("-inf")
                continue
            want = sc * sum(float(wd[t, h]) * max(0.0, float(qd[t, h] @ kd[l])) for h in range(H))
            assert abs(float(got[t, l]) - want) <= 1e-5 * (1 + abs(want))
    # one-hot: token 0 has head 3 = e_17 with weight 1, all other heads zero
    q1 = torch.zeros(1, H, 128, dtype=torch.bfloat16)
    q1[0, 3, 17] = 1.0
    w1 = torch.zeros(1, H, dtype=torch.bfloat16)
    w1[0, 3] = 1.0
    one = ref.indexer_scores_bf16(q1, k, w1, L - 1, 1.0)[0]
    assert torch.equal(one, torch.relu(k[:, 17].float()))


# --------------------------------------------------------------------------- top-k
def test_topk_vs_selection_brute_force_with_ties():
    g = synth.gen(9)
    x = torch.round(torch.randn(3, 300, generator=g) * 4) / 4  # many exact ties
    valid = [300, 150, 10]
    want = brute.topk_fp64(x.numpy(), valid, 32)
    got = ref.topk_rows(x, valid, 32)
    assert np.array_equal(got.numpy().astype(np.int64), want)
    assert torch.all(got[2, 10:] == -1)


# --------------------------------------------------------------------------- rmsnorm
def _bf16_ulp(v: torch.Tensor) -> torch.Tensor:
    e = torch.floor(torch.log2(v.abs().clamp_min(1e-30)))
    return torch.pow(2.0, e - 7)


def test_rmsnorm_vs_fp64_and_one_hot_divisor():
    g = synth.gen(21)
    x = (torch.randn(6, 7168, generator=g) * 3).to(torch.bfloat16)
    w = 1 + 0.1 * torch.randn(7168, generator=g)
    out = ref.rmsnorm(x, w).double()
    xd = x.double()
    want = w.double() * xd / torch.sqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-6)
    assert torch.all((out - want).abs() <= _bf16_ulp(want))  # within one bf16 step of fp64
    # one-hot row: mean(x^2) = a^2 / dim, so out_i = w_i * a / sqrt(a^2/dim + eps) ~ w_i * sqrt(dim)
    oh = torch.zeros(1, 7168, dtype=torch.bfloat16)
    oh[0, 5] = 2.0
    o = ref.rmsnorm(oh, w).double()[0]
    exp = w[5].double() * 2.0 / math.sqrt(4.0 / 7168 + 1e-6)
    assert abs(o[5].item() - exp) <= _bf16_ulp(torch.tensor(exp)).item()
    assert torch.all(o[torch.arange(7168) != 5] == 0)


def test_rmsnorm_power_of_two_invariance_and_constant_rows():
    g = synth.gen(22)
    x = torch.randn(3, 1024, generator=g).to(torch.bfloat16)
    w = torch.rand(1024, generator=g) + 0.5
    # with eps = 0, scaling x by 2^k scales mean(x^2) by 4^k exactly and rsqrt by 2^-k
    assert torch.equal(ref.rmsnorm(x, w, eps=0.0), ref.rmsnorm(x * 8, w, eps=0.0))
    # a constant row c normalises to w * c / sqrt(c^2 + eps)
    c = torch.full((1, 1024), -0.75, dtype=torch.bfloat16)
    o = ref.rmsnorm(c, w).double()[0]
    want = w.double() * -0.75 / math.sqrt(0.5625 + 1e-6)
    assert torch.all((o - want).abs() <= _bf16_ulp(want))


def test_rmsnorm_quant_is_act_quant_of_the_bf16_norm():
    g = synth.gen(23)
    x = torch.randn(4, 512, generator=g).to(torch.bfloat16)
    w = torch.ones(512)
    y, q, s = ref.rmsnorm_quant(x, w)
    q2, s2 = ref.act_quant(y)
    assert torch.equal(q.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(s, s2)


# ------------------------------------------------- indexer key producer (LN, RoPE, Hadamard)
def _bf16_ulp_of(t: torch.Tensor) -> torch.Tensor:
    e = torch.floor(torch.log2(t.abs().clamp_min(2.0 ** -126)))
    return torch.pow(2.0, e - 7)


def test_hadamard_matrix_is_scipy_sylvester_and_orthogonal():
    import scipy.linalg
    h = ref.hadamard_matrix(128)
    assert np.array_equal(h.numpy(), scipy.linalg.hadamard(128).astype(np.float32))
    assert torch.equal(h @ h.T, 128 * torch.eye(128))


def test_rotate_activation_vs_fp64_and_involution():
    import scipy.linalg
    g = synth.gen(31)
    x = (torch.randn(64, 128, generator=g) * 3).to(torch.bfloat16)
    y = ref.rotate_activation(x)
    h64 = torch.tensor(scipy.linalg.hadamard(128), dtype=torch.float64)
    want = ((x.double() @ h64.T) * 128 ** -0.5)
    diff = (y.double() - want).abs()
    assert torch.all(diff <= _bf16_ulp_of(want.float()).double())  # at most one bf16 rounding
    assert (y.double() == want.to(torch.bfloat16).double()).float().mean() > 0.99
    back = ref.rotate_activation(y)  # H / sqrt(128) is its own inverse
    assert ((back.float() - x.float()).norm() / x.float().norm()).item() < 1e-2


def test_rope_half_special_angles_and_fp64():
    g = synth.gen(32)
    pe = torch.randn(8, 64, generator=g).to(torch.bfloat16)
    one = torch.zeros(8, 64)
    one[:, 0::2] = 1.0
    assert torch.equal(ref.rope_half(pe, one), pe)                     # angle 0: identity
    quarter = torch.zeros(8, 64)
    quarter[:, 1::2] = 1.0                                              # angle pi/2: (a, b) -> (-b, a)
    assert torch.equal(ref.rope_half(pe, quarter), torch.cat([-pe[:, 32:], pe[:, :32]], dim=-1))
    theta = torch.rand(8, 32, generator=g, dtype=torch.float64) * 6.28
    fr = torch.stack([theta.cos(), theta.sin()], dim=-1).reshape(8, 64).float()
    out = ref.rope_half(pe, fr).double()
    a, b = pe[:, :32].double(), pe[:, 32:].double()
    c, s = fr[:, 0::2].double(), fr[:, 1::2].double()
    want = torch.cat([a * c - b * s, a * s + b * c], dim=-1)
    assert torch.all((out - want).abs() <= _bf16_ulp_of(want.float()).double())


def test_layernorm_rope_rotate_vs_fp64_brute_force():
    import scipy.linalg
    g = synth.gen(33)
    s = 16
    x = (torch.randn(s, 128, generator=g) * 2 + 0.5).to(torch.bfloat16)
    w = torch.rand(128, generator=g) * 0.2 + 0.9
    b = torch.randn(128, generator=g) * 0.1
    theta = torch.rand(s, 32, generator=g, dtype=torch.float64) * 6.28
    fr = torch.stack([theta.cos(), theta.sin()], dim=-1).reshape(s, 64).float()
    got = ref.layernorm_rope_rotate(x, w, b, fr)
    # fp64 restatement of golden_forward, with its two bf16 roundings (after the norm and
    # after the RoPE) and the last one after the transform
    xd = x.double()
    mu = xd.mean(-1, keepdim=True)
    var = ((xd - mu) ** 2).mean(-1, keepdim=True)
    k = ((xd - mu) / torch.sqrt(var + 1e-6) * w.double() + b.double()).to(torch.bfloat16).double()
    a, bb = k[:, :32], k[:, 32:64]
    c, sn = fr[:, 0::2].double(), fr[:, 1::2].double()
    pe = torch.cat([a * c - bb * sn, a * sn + bb * c], dim=-1).to(torch.bfloat16).double()
    kk = torch.cat([pe, k[:, 64:]], dim=-1)
    want = (kk @ torch.tensor(scipy.linalg.hadamard(128), dtype=torch.float64).T) * 128 ** -0.5
    rel = ((got.double() - want).norm() / want.norm()).item()
    assert rel < 4e-3, rel
    # a dropped scale, a sign slip in the rotation or interleaved pairing would fail these
    assert (got.double() - want).abs().max().item() < 0.05 * want.abs().max().item()


# --------------------------------------------------------------- sparse MLA attention
def _mla_inputs(s, h, T, g):
    q = (torch.randn(s, h, 512, generator=g) * 0.5).to(torch.bfloat16)
    qp = (torch.randn(s, h, 64, generator=g) * 0.5).to(torch.bfloat16)
    kv = torch.randn(T, 512, generator=g).to(torch.bfloat16)
    pe = torch.randn(T, 64, generator=g).to(torch.bfloat16)
    return q, qp, kv, pe


def test_mla_softmax_scale_closed_form():
    assert ref.mla_softmax_scale("glm_5") == 1 / 16
    ms = 0.1 * math.log(40) + 1
    assert abs(ref.mla_softmax_scale("deepseek_v3_2") - ms * ms / math.sqrt(192)) < 1e-15


def test_flash_sparse_mla_vs_fp64_brute_force():
    g = synth.gen(41)
    s, h, T, k = 3, 16, 200, 48
    q, qp, kv, pe = _mla_inputs(s, h, T, g)
    idx = torch.stack([torch.randperm(T, generator=g)[:k] for _ in range(s)])
    cur = T - s
    sc = 0.1352
    got = ref.flash_sparse_mla(q, qp, kv, pe, idx, cur, sc).double()
    want = torch.zeros(s, h, 512, dtype=torch.float64)
    for t in range(s):
        sel = [int(i) for i in idx[t] if int(i) <= cur + t]  # s > 1: the triu mask
        kd, pd = kv[sel].double(), pe[sel].double()
        for hh in range(h):
            z = (kd @ q[t, hh].double() + pd @ qp[t, hh].double()) * sc
            p = torch.softmax(z, 0).to(torch.bfloat16).double()
            want[t, hh] = p @ kd
    assert ((got - want).norm() / want.norm()).item() < 2e-3
    assert (got - want).abs().max().item() < 2 * 2.0 ** -7 * want.abs().max().item()


def test_flash_sparse_mla_special_cases():
    g = synth.gen(42)
    q, qp, kv, pe = _mla_inputs(1, 8, 64, g)
    # one selected position: its probability is exactly 1, the output is that kv row
    out = ref.flash_sparse_mla(q, qp, kv, pe, torch.tensor([[17]]), 63, 0.1)
    assert torch.equal(out[0], kv[17].expand(8, 512))
    # zero queries: uniform weights 1/4 (exact in bf16) over 4 positions -> their mean
    z = torch.zeros_like(q), torch.zeros_like(qp)
    sel = [3, 9, 40, 41]
    out = ref.flash_sparse_mla(*z, kv, pe, torch.tensor([sel]), 63, 0.1)
    assert torch.equal(out[0, 0], (kv[sel].double().sum(0) / 4).to(torch.bfloat16))
    # the order of the indices does not matter
    idx = torch.randperm(64, generator=g)[:20][None]
    a = ref.flash_sparse_mla(q, qp, kv, pe, idx, 63, 0.1)
    b = ref.flash_sparse_mla(q, qp, kv, pe, idx.flip(-1), 63, 0.1)
    assert torch.equal(a, b)
    # two tokens: position cur_pos + 1 is visible to token 1 only
    q2, qp2, _, _ = _mla_inputs(2, 8, 64, g)
    two = ref.flash_sparse_mla(q2, qp2, kv, pe, torch.tensor([[5, 31], [5, 31]]), 30, 0.1)
    only5 = ref.flash_sparse_mla(q2[:1], qp2[:1], kv, pe, torch.tensor([[5]]), 30, 0.1)
    assert torch.equal(two[0], only5[0])
    assert not torch.equal(two[1], ref.flash_sparse_mla(q2[1:], qp2[1:], kv, pe, torch.tensor([[5]]), 30, 0.1)[0])


# ------------------------------------------------------- q RMSNorm + wq_b (BF16MMA)
def test_rmsnorm_projq_wqb_vs_fp64_and_head_split():
    g = synth.gen(51)
    s, heads, rank = 4, 4, 256
    q = (torch.randn(s, rank, generator=g) * 2).to(torch.bfloat16)
    gamma = torch.rand(rank, generator=g) + 0.5
    wq, ws = ref.weight_quant(synth.weight_fp32(heads * 192, rank, g))
    nope, pe = ref.rmsnorm_projq_wqb(q, gamma, wq, ws, heads)
    assert nope.shape == (s, heads, 128) and pe.shape == (s, heads, 64)
    # fp64: the norm (rounded to bf16, as the golden), the weight's bf16 dequantisation
    qd = q.double()
    qr = (qd * torch.rsqrt(qd.pow(2).mean(-1, keepdim=True) + 1e-6) * gamma.double()).to(torch.bfloat16).double()
    wd = (wq.float() * ws.repeat_interleave(128, 0).repeat_interleave(128, 1)).to(torch.bfloat16).double()
    want = (qr @ wd.T).view(s, heads, 192)
    got = torch.cat([nope, pe], -1).double()
    assert ((got - want).norm() / want.norm()).item() < 4e-3
    # head h's rows 192 h .. 192 h + 127 are its nope part, the next 64 its rope part
    assert torch.equal(torch.cat([nope, pe], -1).reshape(s, heads * 192), torch.cat(
        [torch.cat([nope[:, h], pe[:, h]], -1) for h in range(heads)], -1))
    # a one-hot weight row picks one normalised input element
    wq1 = torch.zeros(heads * 192, rank)
    wq1[5, 17] = 1.0
    q1, s1 = ref.weight_quant(wq1)
    n1, _ = ref.rmsnorm_projq_wqb(q, gamma, q1, s1, heads)
    assert torch.equal(n1[:, 0, 5].float(), (qr[:, 17].float() * wd.new_tensor(1.0).float()).to(torch.bfloat16).float())


# ------------------------------------------------------------- routing (expert select)
@pytest.mark.parametrize("n_groups,topk_groups,with_bias", [(8, 4, True), (8, 4, False), (1, 1, True)])
def test_expert_select_vs_python_sort(n_groups, topk_groups, with_bias):
    g = synth.gen(40 + n_groups)
    logits = torch.randn(6, 256, generator=g)
    bias = torch.randn(256, generator=g) * 0.1 if with_bias else None
    w, idx = ref.expert_select(logits, bias, 8, n_groups, topk_groups, 2.5)
    bw, bi = brute.expert_select_py(logits.tolist(), bias.tolist() if bias is not None else None, 8, n_groups,
                                    topk_groups, 2.5)
    assert idx.tolist() == bi
    assert torch.allclose(w.double(), torch.tensor(bw, dtype=torch.float64), rtol=1e-6, atol=0)


def test_expert_select_invariants():
    g = synth.gen(44)
    logits = torch.randn(16, 256, generator=g) * 3
    bias = torch.randn(256, generator=g)
    w, idx = ref.expert_select(logits, bias, 8, 8, 4, 2.5)
    assert torch.allclose(w.sum(-1), torch.full((16,), 2.5), rtol=1e-6)
    for t in range(16):
        assert len(set(idx[t].tolist())) == 8
        assert len({int(e) // 32 for e in idx[t]}) <= 4  # group-limited to 4 of 8 groups
        b = logits[t].sigmoid() + bias
        assert torch.all(b[idx[t]][:-1] >= b[idx[t]][1:])  # descending by biased score
        # the bias steers the choice only: weights are the unbiased sigmoid scores
        sel = logits[t].sigmoid()[idx[t]]
        assert torch.allclose(w[t], sel / sel.sum() * 2.5, rtol=1e-6)


def test_expert_select_bias_changes_choice_not_weights():
    logits = torch.zeros(1, 256)
    logits[0, :8] = 1.0  # the unbiased top-8
    bias = torch.zeros(256)
    bias[100:108] = 5.0  # a large bias moves the choice to 100..107 (one group-pair)
    w, idx = ref.expert_select(logits, bias, 8, 8, 4, 2.5)
    assert sorted(idx[0].tolist()) == list(range(100, 108))
    assert torch.allclose(w, torch.full((1, 8), 2.5 / 8))


# ----------------------------------------------------------- reference-layout MoE goldens
def _tp_experts(E, D, I, g):
    out = {}
    for name, (n, k) in (("gate", (I, D)), ("up", (I, D)), ("down", (D, I))):
        q, s = zip(*[ref.weight_quant(synth.weight_fp32(n, k, g)) for _ in range(E)])
        out[name] = (torch.stack(q), torch.stack(s))
    return out


def test_expert_select_up_gate_silu_and_down_vs_fp64():
    """The per-position goldens against fp64 recomputation with explicit loops over
    (token, position): the shared expert at position 0, routed expert j at 1 + idx."""
    g = synth.gen(45)
    E, D, I, T, k = 6, 256, 128, 2, 3
    W = _tp_experts(E, D, I, g)
    x = synth.activations(T, D, g)
    idx = torch.tensor([[4, 0, 2], [1, 4, 3]])
    probs = torch.tensor([[0.5, 0.3, 0.2], [0.1, 0.6, 0.3]])
    h = ref.expert_select_up_gate_silu(x, idx, *W["gate"], *W["up"])
    assert h.shape == (T, 1 + k, I)
    xd = x.double()
    for t in range(T):
        for p, e in enumerate([0] + [1 + int(j) for j in idx[t]]):
            gw = ref.weight_dequant(*[a[e] for a in W["gate"]]).to(torch.bfloat16).double()
            uw = ref.weight_dequant(*[a[e] for a in W["up"]]).to(torch.bfloat16).double()
            a, b = xd[t] @ gw.T, xd[t] @ uw.T
            want = (a / (1 + torch.exp(-a)) * b)
            assert torch.allclose(h[t, p].double(), want, rtol=1e-2, atol=1e-3)
    xin = synth.activations(T, D, g)
    y = ref.expert_down_allreduce(h, idx, probs, *W["down"], x_in=xin)
    for t in range(T):
        acc = torch.zeros(D, dtype=torch.float64)
        for p, e in enumerate([0] + [1 + int(j) for j in idx[t]]):
            dw = ref.weight_dequant(*[a[e] for a in W["down"]]).to(torch.bfloat16).double()
            wt = 1.0 if p == 0 else float(probs[t, p - 1])
            acc += wt * (h[t, p].double() @ dw.T)
        assert torch.allclose(y[t].double(), acc + xin[t].double(), rtol=2e-2, atol=2e-2)


def test_dense_mlp_goldens_vs_fp64_and_variants():
    g = synth.gen(46)
    C, D, I, T = 3, 256, 128, 2
    W = _tp_experts(C, D, I, g)
    x = synth.activations(T, D, g)
    gamma = torch.rand(D, generator=g) + 0.5
    h32 = ref.rmsnorm_up_gate_silu(x, gamma, 1e-6, *W["gate"], *W["up"], bf16_operands=False)
    h16 = ref.rmsnorm_up_gate_silu(x, gamma, 1e-6, *W["gate"], *W["up"], bf16_operands=True)
    xd = x.double()
    xn = xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + 1e-6) * gamma.double()
    for i in range(C):
        a = xn @ ref.weight_dequant(*[w[i] for w in W["gate"]]).double().T
        b = xn @ ref.weight_dequant(*[w[i] for w in W["up"]]).double().T
        want = a / (1 + torch.exp(-a)) * b
        assert torch.allclose(h32[:, i].double(), want, rtol=1e-2, atol=1e-4)
    # rounding the operands to bf16 moves the result by about a bf16 step, no more
    rel = (torch.norm(h16.float() - h32.float()) / torch.norm(h32.float())).item()
    assert 0 < rel < 1e-2
    y = ref.down_allreduce(h16, *W["down"], bf16_weights=False)
    acc = sum(h16[:, i].double() @ ref.weight_dequant(*[w[i] for w in W["down"]]).double().T for i in range(C))
    assert torch.allclose(y.double(), acc, rtol=2e-2, atol=2e-2)


# -------------------------------------------------------- absorbed MLA projections
def test_absorbed_mla_goldens_vs_fp64_loops():
    g = synth.gen(47)
    H, nope, v, kv, T = 3, 128, 128, 256, 2
    wq, ws = ref.weight_quant(synth.weight_fp32(H * (nope + v), kv, g))
    wd = ref.weight_dequant(wq, ws).double()
    q = synth.activations(T, H * nope, g).reshape(1, T, H, nope)
    o = synth.activations(T, H * kv, g).reshape(1, T, H, kv)
    ql = ref.projq_wqb(q, wq, ws, H, nope, bf16_weights=False)
    ov = ref.projo_wkvb(o, wq, ws, H, v, bf16_weights=False)
    for t in range(T):
        for h in range(H):
            blk = wd[h * (nope + v):(h + 1) * (nope + v)]
            want_q = sum(q[0, t, h, d].double() * blk[d] for d in range(nope))  # rows contracted
            assert torch.allclose(ql[0, t, h].double(), want_q, rtol=1e-2, atol=1e-3)
            want_o = blk[nope:] @ o[0, t, h].double()  # columns contracted
            assert torch.allclose(ov[0, t, h].double(), want_o, rtol=1e-2, atol=1e-3)
    wo, wos = ref.weight_quant(synth.weight_fp32(256, H * v, g))
    xin = synth.activations(T, 256, g).reshape(1, T, 256)
    x = synth.activations(T, H * v, g).reshape(1, T, H, v)
    y = ref.unproj_o_allreduce(x, wo, wos, bf16_weights=False, x_in=xin)
    want = x.reshape(T, -1).double() @ ref.weight_dequant(wo, wos).double().T + xin[0].double()
    assert torch.allclose(y[0].double(), want, rtol=2e-2, atol=2e-2)


# ------------------------------------------------------- the indexer's projections
def test_projx_wis_vs_fp64_and_one_hot_rows():
    """projx_wis is x . W^T with bf16 operands: fp64 loops over (token, head), one-hot weight
    rows that must pick one input column each (a transposed weight or swapped output axis
    picks the wrong one), and a non-square shape so a transpose cannot type-check."""
    g = synth.gen(48)
    T, H, D = 3, 5, 384
    x = synth.activations(T, D, g)
    w = (torch.randn(H, D, generator=g) * 0.05).to(torch.bfloat16)
    got = ref.projx_wis(x, w)
    assert got.shape == (T, H) and got.dtype == torch.bfloat16
    xd, wd = x.double(), w.double()
    for t in range(T):
        for h in range(H):
            want = sum(float(xd[t, k]) * float(wd[h, k]) for k in range(D))
            assert abs(float(got[t, h]) - want) <= 2.0 ** -8 * abs(want) + 1e-6
    cols = [7, 0, 383, 200, 129]
    one = torch.zeros(H, D, dtype=torch.bfloat16)
    for h, c in enumerate(cols):
        one[h, c] = 1.0
    assert torch.equal(ref.projx_wis(x, one), x[:, cols])


def test_rmsnorm_projx_wqakis_vs_fp64_brute_force():
    """The golden's three outputs against fp64 brute force: fp64 RMSNorm (gamma applied per
    column), then the fp64 block-scaled dot products with wq_a and wk (decoded e4m3 codes
    times their block scales) and the bf16 weights_proj.  A one-hot gamma row and a one-hot
    weights_proj row pin which column each output reads."""
    g = synth.gen(49)
    T, D, QR = 2, 256, 256
    x = synth.activations(T, D, g)
    gamma = torch.rand(D, generator=g) + 0.5
    wq, wqs = ref.weight_quant(synth.weight_fp32(QR, D, g))
    wk, wks = ref.weight_quant(synth.weight_fp32(128, D, g) * 3)
    wis = (torch.randn(4, D, generator=g) * 0.05).to(torch.bfloat16)
    eps = 1e-6
    q, ki, sc = ref.rmsnorm_projx_wqakis(x, gamma, wq, wqs, wk, wks, wis, eps)
    assert q.shape == (T, QR) and ki.shape == (T, 128) and sc.shape == (T, 4)
    xd = x.double().numpy()
    xn = xd / np.sqrt((xd * xd).mean(-1, keepdims=True) + eps) * gamma.double().numpy()

    def dense(codes, s):
        w = fp8.decode(codes.view(torch.uint8).numpy()).astype(np.float64)
        sn = s.double().numpy()
        for r in range(w.shape[0]):
            for kb in range(w.shape[1] // 128):
                w[r, kb * 128:(kb + 1) * 128] *= sn[r // 128, kb]
        return w

    for got, want in ((q, xn @ dense(wq, wqs).T), (ki, xn @ dense(wk, wks).T),
                      (sc, xn @ wis.double().numpy().T)):
        got = got.double().numpy()
        ulp = 2.0 ** (np.floor(np.log2(np.abs(want) + 1e-30)) - 7)
        assert np.all(np.abs(got - want) <= 0.5 * ulp + 1e-5 * np.abs(want) + 1e-30)
    # weights_proj row h = e_c reads the normalised column c
    one = torch.zeros(4, D, dtype=torch.bfloat16)
    for h, c in enumerate((3, 100, 255, 128)):
        one[h, c] = 1.0
    _, _, sc1 = ref.rmsnorm_projx_wqakis(x, gamma, wq, wqs, wk, wks, one, eps)
    want1 = torch.from_numpy(xn[:, [3, 100, 255, 128]]).to(torch.bfloat16)
    assert (sc1.double() - want1.double()).abs().max() <= 2.0 ** -7 * want1.double().abs().max()
