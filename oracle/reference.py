"""torch-CPU restatement of the reference goldens for the FP8 decode hot path.

Test infrastructure only (see ``oracle/__init__.py``).  All citations are relative to the
reference tree (tile-ai/TileRT).  Tensors are CPU tensors; fp8 data is carried as
``torch.float8_e4m3fn`` (or uint8 codes where noted).

Conventions shared with the HIP library:
  * block size 128 everywhere (``tilert/models/deepseek_config.py`` ``block_size = 128``);
  * activation scales are one fp32 per (row, 128-column group);
  * weight scales are one fp32 per (128-row, 128-column) block, shape
    [ceil(N/128), ceil(K/128)];
  * outputs of linears are bf16 (``torch.get_default_dtype()`` in DeepSeek inference).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

BLOCK = 128
E4M3_MAX = 448.0
# tilelang folds ``1 / fp8_max`` into an fp32 immediate (refs/kernel.py:160)
INV_448_F32 = torch.tensor(1.0 / 448.0, dtype=torch.float32)
AMAX_FLOOR_F32 = torch.tensor(1e-4, dtype=torch.float32)

SCALE_MODE_REFERENCE = 0  # s = amax * fp32(1/448)             refs/kernel.py:191
SCALE_MODE_UE8M0 = 1  # s = 2^ceil(log2(amax * fp32(1/448)))  refs/kernel.py:140-151,189
SCALE_MODE_DIV = 2  # s = amax / 448 (IEEE division), the workload's stated convention


def _group_scale(amax: torch.Tensor, scale_mode: int) -> torch.Tensor:
    """Per-group scale from the fp32 amax (refs/kernel.py:186-191)."""
    amax = torch.maximum(amax, AMAX_FLOOR_F32)
    if scale_mode == SCALE_MODE_REFERENCE:
        return amax * INV_448_F32
    if scale_mode == SCALE_MODE_DIV:
        return amax / torch.tensor(448.0, dtype=torch.float32)
    if scale_mode == SCALE_MODE_UE8M0:
        # _fast_round_scale: pow2(ceil(log2(amax * inv))) with exponent/mantissa bit ops
        v = (amax * INV_448_F32).contiguous()
        bits = v.view(torch.int32).to(torch.int64)
        exp = (bits >> 23) & 0xFF
        man = bits & ((1 << 23) - 1)
        e = exp - 127 + (man != 0).to(torch.int64)
        return ((e + 127) << 23).to(torch.int32).view(torch.float32)
    raise ValueError(f"unknown scale_mode {scale_mode}")


def act_quant(
    x: torch.Tensor, block_size: int = BLOCK, scale_mode: int = SCALE_MODE_REFERENCE
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-(row, 128-group) e4m3fn quantisation.

    Follows ``act_quant_kernel`` (refs/kernel.py:154-199) and its wrapper ``act_quant``
    (refs/kernel.py:252-279): amax over the group in fp32, floored at 1e-4, scale per
    ``scale_mode``, then ``e4m3fn(clamp(x / s, -448, 448))`` with IEEE fp32 division and
    round-to-nearest-even.  Returns (y float8_e4m3fn, s float32 [..., K/128]).
    """
    assert x.shape[-1] % block_size == 0
    K = x.shape[-1]
    xf = x.float().reshape(-1, K // block_size, block_size)
    amax = xf.abs().amax(dim=-1)
    s = _group_scale(amax, scale_mode)
    y = torch.clamp(xf / s[..., None], -E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return y.reshape(x.shape), s.reshape(*x.shape[:-1], K // block_size)


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``RMSNorm.forward`` without residual (tilert/models/common.py:110-128): fp32 math,
    x * rsqrt(mean(x^2) + eps), times the fp32 weight, cast to bf16."""
    xf = x.float()
    var = xf.pow(2).mean(-1, keepdim=True)
    xf = xf * torch.rsqrt(var + eps)
    return (weight.float() * xf).to(torch.bfloat16)


def rmsnorm_quant(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
                  scale_mode: int = SCALE_MODE_REFERENCE):
    """``rmsnorm_quant_op`` (ops/rmsnorm_quant.py:19-63): the bf16 norm, then act_quant of
    those bf16 values per 1x128 group."""
    y = rmsnorm(x, weight, eps)
    q, s = act_quant(y, BLOCK, scale_mode)
    return y, q, s


def act_dequant(y: torch.Tensor, s: torch.Tensor, block_size: int = BLOCK) -> torch.Tensor:
    """fp32 x = fp8 * group scale, as the goldens do (projx_wqkva.py:280-285)."""
    K = y.shape[-1]
    yf = y.float().reshape(-1, K // block_size, block_size)
    return (yf * s.reshape(-1, K // block_size, 1)).reshape(y.shape)


def weight_quant(w: torch.Tensor, block_size: int = BLOCK) -> tuple[torch.Tensor, torch.Tensor]:
    """128x128 block quantisation of a weight (synthetic-weight preparation).

    The workload's convention: ``s = block_amax / 448`` (IEEE division), ``q = e4m3fn(w / s)``.
    Rows/columns that do not fill a block (e.g. N=576) form a partial block.  All-zero
    blocks get s = 1 (so that dequantisation returns exact zeros).
    """
    N, K = w.shape
    nb, kb = math.ceil(N / block_size), math.ceil(K / block_size)
    wp = torch.zeros(nb * block_size, kb * block_size, dtype=torch.float32)
    wp[:N, :K] = w.float()
    blocks = wp.reshape(nb, block_size, kb, block_size)
    amax = blocks.abs().amax(dim=(1, 3))
    s = torch.where(amax > 0, amax / torch.tensor(448.0), torch.ones_like(amax))
    q = torch.clamp(blocks / s[:, None, :, None], -E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    q = q.reshape(nb * block_size, kb * block_size)[:N, :K].contiguous()
    return q, s.contiguous()


def weight_dequant(q: torch.Tensor, s: torch.Tensor, block_size: int = BLOCK) -> torch.Tensor:
    """fp32 ``W[n,k] = fp32(Wq[n,k]) * S[n//128, k//128]``.

    ``_weight_dequant_torch`` (refs/kernel.py:82-94), extended to partial edge blocks.
    """
    N, K = q.shape
    s_full = s.repeat_interleave(block_size, 0)[:N].repeat_interleave(block_size, 1)[:, :K]
    return q.float() * s_full


def fp8_gemm(a: torch.Tensor, a_s: torch.Tensor, b: torch.Tensor, b_s: torch.Tensor) -> torch.Tensor:
    """``C = dequant(A) . dequant(B)^T`` in fp32, output bf16.

    The golden of every FP8 projection (projx_wqkva.py:280-294: dequantise x per 1x128,
    matmul with the fp32 dequantised weight, ``.to(torch.bfloat16)``), which is what
    ``fp8_gemm`` (refs/kernel.py:282-306) computes with per-128-K-block scaling.
    """
    K = a.shape[-1]
    xa = act_dequant(a.reshape(-1, K), a_s.reshape(-1, K // BLOCK))
    wb = weight_dequant(b, b_s)
    c = xa @ wb.T
    return c.to(torch.bfloat16).reshape(*a.shape[:-1], b.shape[0])


def linear(x: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor, scale_mode: int = 0) -> torch.Tensor:
    """``common.linear`` FP8 branch (tilert/models/common.py:83-89): act_quant -> fp8_gemm."""
    xq, xs = act_quant(x, BLOCK, scale_mode)
    return fp8_gemm(xq, xs, wq, ws)


def projx_wqkva(x_q: torch.Tensor, x_s: torch.Tensor, wq_a: torch.Tensor, wq_a_s: torch.Tensor,
                wkv_a: torch.Tensor, wkv_a_s: torch.Tensor, kv_lora_rank: int
                ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Golden of projx_wqkva (projx_wqkva.py:268-294): dequantise x per 1x128, dequantise
    wq_a and kv_a_proj_with_mqa (whose first kv_lora_rank rows are the latent projection and
    the rest w_pe, :195-196), three fp32 matmuls, each rounded to bf16 -> (q, kv, pe)."""
    K = x_q.shape[-1]
    xa = act_dequant(x_q.reshape(-1, K), x_s.reshape(-1, K // BLOCK))
    wq = weight_dequant(wq_a, wq_a_s)
    wkv = weight_dequant(wkv_a, wkv_a_s)
    lead = x_q.shape[:-1]
    q = (xa @ wq.T).to(torch.bfloat16).reshape(*lead, -1)
    kv = (xa @ wkv[:kv_lora_rank].T).to(torch.bfloat16).reshape(*lead, -1)
    pe = (xa @ wkv[kv_lora_rank:].T).to(torch.bfloat16).reshape(*lead, -1)
    return q, kv, pe


def swiglu(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """``silu(g) * u`` in fp32 (expert_sel_up_gate_silu.py:687)."""
    return F.silu(g.float()) * u.float()


def local_pairs(topk_idx: torch.Tensor, expert_begin: int, n_local: int) -> list[tuple[int, int, int]]:
    """(token, k-slot, local expert) for every routed pair that lands on this shard."""
    out = []
    M, topk = topk_idx.shape
    for t in range(M):
        for j in range(topk):
            e = int(topk_idx[t, j]) - expert_begin
            if 0 <= e < n_local:
                out.append((t, j, e))
    return out


def hit_experts(topk_idx: torch.Tensor, expert_begin: int, n_local: int) -> list[int]:
    """Local experts hit by at least one token, ascending (the slot order)."""
    return sorted({e for (_, _, e) in local_pairs(topk_idx, expert_begin, n_local)})


def moe_gate_up(
    x: torch.Tensor,
    gq: torch.Tensor, gs: torch.Tensor, uq: torch.Tensor, us: torch.Tensor,
    topk_idx: torch.Tensor, expert_begin: int,
) -> tuple[torch.Tensor, list[int]]:
    """Grouped gate/up + SwiGLU for every hit local expert and every token.

    ``ExpertSelectUpGateSiLU.golden_forward`` (deepseek_v3_2/ops/expert_sel_up_gate_silu.py:
    670-692) with its reference weights (``init_reference_weights`` :545-552: each expert's
    fp8 weight dequantised per 128x128 block, then rounded to bf16): per (token, expert)
    ``h = bf16(silu(x.float() @ G.float().T) * (x.float() @ U.float().T))``.  x is bf16 and
    NOT quantised (the reference MoE runs BF16MMA, deepseek_v3_2/modules/moe.py:32-45).
    Returns h [n_hit, M, I] bf16 (slot order = ascending local expert id) and the hit list.
    """
    E = gq.shape[0]
    xf = x.float()
    hits = hit_experts(topk_idx, expert_begin, E)
    hs = []
    for e in hits:
        g = xf @ weight_dequant(gq[e], gs[e]).to(torch.bfloat16).float().T
        u = xf @ weight_dequant(uq[e], us[e]).to(torch.bfloat16).float().T
        hs.append(swiglu(g, u).to(torch.bfloat16))
    I = gq.shape[1]
    h = torch.stack(hs) if hs else torch.zeros(0, x.shape[0], I, dtype=torch.bfloat16)
    return h, hits


def moe_down(
    h: torch.Tensor, hits: list[int],
    dq: torch.Tensor, ds: torch.Tensor,
    topk_idx: torch.Tensor, topk_w: torch.Tensor, expert_begin: int,
) -> torch.Tensor:
    """Down projection + routing-weighted sum over the local experts.

    ``ExpertDownAllReduce.golden_forward`` (deepseek_v3_2/ops/expert_down_allreduce.py:
    455-468, weights rounded to bf16 after dequantisation as in :389-393): each term
    ``bf16(w[t,e] * (h[t,e].float() @ D_e.float().T))``, summed over the token's local
    experts in fp32 (ascending expert order) and rounded once to bf16.  Tokens with no
    local expert get 0 (the shard's share; the cross-shard sum is the allreduce).
    """
    M = topk_idx.shape[0]
    D = dq.shape[1]
    acc = torch.zeros(M, D, dtype=torch.float32)
    pairs = local_pairs(topk_idx, expert_begin, dq.shape[0])
    slot = {e: i for i, e in enumerate(hits)}
    for e in hits:
        wd = weight_dequant(dq[e], ds[e]).to(torch.bfloat16).float()
        for (t, j, ee) in pairs:
            if ee != e:
                continue
            term = h[slot[e], t].float() @ wd.T
            acc[t] += (term * topk_w[t, j].float()).to(torch.bfloat16).float()
    return acc.to(torch.bfloat16)


def moe_forward(x, gq, gs, uq, us, dq, ds, topk_idx, topk_w, expert_begin):
    """Whole local-expert MoE layer (config 2): gate/up + SwiGLU, down, weighted sum."""
    h, hits = moe_gate_up(x, gq, gs, uq, us, topk_idx, expert_begin)
    return moe_down(h, hits, dq, ds, topk_idx, topk_w, expert_begin)


def indexer_scores(
    q: torch.Tensor, q_s: torch.Tensor, k: torch.Tensor, k_s: torch.Tensor,
    w: torch.Tensor, cur_pos: int,
) -> torch.Tensor:
    """DSA lightning-indexer logits, fp32 [M, L].

    ``score[t,l] = sum_h w[t,h] * ReLU(q[t,h] . k[l])`` on dequantised fp8 inputs
    (q: [M,H,128] e4m3fn with scale per token [M] or per (token, head) [M,H];
    k: [L,128] e4m3fn with per-key scale [L]; w: bf16 [M,H]).  Token t sits at position
    ``cur_pos + t`` and sees keys ``l <= cur_pos + t``; masked positions are -inf.
    The reference ships no golden for this (ops/sparse_index.py:11-69 describes it as
    "q * kv * weights"); the formula is the one the indexer workload (config 4) states.
    """
    M, H, Dh = q.shape
    L = k.shape[0]
    qs = q_s.float().reshape(M, -1)
    qd = q.float() * (qs[:, :, None] if qs.shape[1] == H else qs[:, :1, None])
    kd = k.float() * k_s.float().reshape(L, 1)
    logits = torch.einsum("thd,ld->thl", qd, kd)
    logits = torch.relu(logits)
    score = torch.einsum("thl,th->tl", logits, w.float())
    pos = torch.arange(L)[None, :]
    lim = (cur_pos + torch.arange(M))[:, None]
    return torch.where(pos <= lim, score, torch.tensor(float("-inf")))


def indexer_scores_bf16(q: torch.Tensor, k: torch.Tensor, w: torch.Tensor, cur_pos: int,
                        score_scale: float) -> torch.Tensor:
    """The reference's bf16 indexer (``sparse_index``, ops/sparse_index.py:11-69: "q * kv *
    weights"; bf16 q [M,H,128], bf16 key cache [L,128], bf16 head weights [M,H]), fp32 [M, L]:
    ``score_scale * sum_h w[t,h] * ReLU(q[t,h] . k[l])`` in fp32, -inf for l > cur_pos + t.
    ``score_scale`` is the constant the operator applies inside the kernel ("we precompute
    scale inner kernel", :58-59); this build uses (128 H)^-1/2."""
    M, H, _ = q.shape
    L = k.shape[0]
    logits = torch.relu(torch.einsum("thd,ld->thl", q.float(), k.float()))
    score = torch.einsum("thl,th->tl", logits, w.float()) * score_scale
    pos = torch.arange(L)[None, :]
    lim = (cur_pos + torch.arange(M))[:, None]
    return torch.where(pos <= lim, score, torch.tensor(float("-inf")))


def topk_rows(logits: torch.Tensor, valid: list[int], k: int) -> torch.Tensor:
    """Per-row top-k indices among the first ``valid[i]`` columns, int32 [rows, k].

    ``TopK.golden_forward`` is ``logits.topk(min(k, L))[1]`` (ops/topk.py:128-143); sample i
    of ``topk_accurate`` only considers its valid prefix (ops/topk.py:77-80,101).  Order:
    descending score, ties by ascending index; slots beyond the valid length are -1.
    """
    rows = logits.shape[0]
    out = torch.full((rows, k), -1, dtype=torch.int32)
    for i in range(rows):
        v = logits[i, : valid[i]].double()
        n = min(k, v.numel())
        if n == 0:
            continue
        order = sorted(range(v.numel()), key=lambda j: (-float(v[j]), j)) if v.numel() < 4096 \
            else _sort_desc_stable(v)
        out[i, :n] = torch.tensor(order[:n], dtype=torch.int32)
    return out


def _sort_desc_stable(v: torch.Tensor) -> list[int]:
    # stable sort on -v keeps ascending index among equal scores
    return torch.sort(-v, stable=True).indices.tolist()


# ----------------------------------------------------------------- indexer key producer
HADAMARD_SCALE_128 = torch.tensor(128 ** -0.5, dtype=torch.float32)


def hadamard_matrix(n: int) -> torch.Tensor:
    """Sylvester-ordered Hadamard matrix, H[i, j] = (-1)^popcount(i & j) (the ordering of
    scipy.linalg.hadamard and of fast_hadamard_transform), fp32 +-1 entries."""
    i = torch.arange(n)
    bits = torch.bitwise_and(i[:, None], i[None, :])
    parity = torch.zeros_like(bits)
    while torch.any(bits):
        parity ^= bits & 1
        bits = bits >> 1
    return (1 - 2 * parity).to(torch.float32)


def rotate_activation(k: torch.Tensor) -> torch.Tensor:
    """``rotate_activation`` (ops/rotate.py:17-21): fast_hadamard_transform(x, scale=d^-0.5)
    on a bf16 [..., 128] tensor.  fast_hadamard_transform (an unpinned third-party package,
    absent here) computes the transform in fp32 and returns the input dtype, so this is
    bf16(fp32(H x) * fp32(128^-0.5)).  Its scipy fallback (ops/rotate.py:22-49) would run the
    matmul in bf16 and round twice; the production path is the one restated."""
    d = k.shape[-1]
    h = hadamard_matrix(d)
    y = k.float().reshape(-1, d) @ h.T
    return (y * HADAMARD_SCALE_128).to(torch.bfloat16).reshape(k.shape)


def rope_half(pe: torch.Tensor, freqs: torch.Tensor) -> torch.Tensor:
    """``apply_rotary_emb(..., interleaved=False)`` (tilert/models/utils.py:121-145) on bf16
    [s, 64]: element i pairs with element i + 32 as the complex number (x_i, x_{i+32}),
    which is multiplied by freqs_cis[s, i] in complex64; the result is bf16 with real parts
    in 0..31 and imaginary parts in 32..63.  ``freqs`` is the op's fp32 [s, 64] operand
    (view_as_real of freqs_cis: cos, sin interleaved, layernorm_rope_rotate.py:224-226)."""
    s, d = pe.shape
    x = pe.view(s, 2, d // 2).transpose(-1, -2).contiguous()
    xc = torch.view_as_complex(x.float().reshape(s, d // 2, 2))
    fc = torch.view_as_complex(freqs.float().reshape(s, d // 2, 2).contiguous())
    y = torch.view_as_real(xc * fc).flatten(1)
    y = torch.cat([y[..., 0::2], y[..., 1::2]], dim=-1)
    return y.to(torch.bfloat16)


def layernorm_rope_rotate(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                          freqs: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``LayerNormRoPERotate.golden_forward`` (ops/layernorm_rope_rotate.py:206-220) on bf16
    [s, 128]: k = bf16(LayerNorm(x) * weight + bias); the first 64 dims take the
    non-interleaved RoPE; then rotate_activation (the 128-point Hadamard, scale 128^-0.5)."""
    k = F.layer_norm(x.float(), (x.shape[-1],), weight.float(), bias.float(), eps).to(torch.bfloat16)
    pe = rope_half(k[:, :64], freqs)
    return rotate_activation(torch.cat([pe, k[:, 64:]], dim=-1))


# ------------------------------------------------------------------ sparse MLA attention
def mla_softmax_scale(model_arch: str) -> float:
    """FlashSparseMLACombine.softmax_scale (ops/flash_sparse_mla.py:125-130):
    (qk_nope_head_dim + qk_rope_head_dim)^-1/2 * mscale^2, mscale = 0.1 ln(rope_factor) + 1
    (1 without a rope factor).  deepseek_v3_2: 128 + 64, rope_factor 40
    (deepseek_v3_2/model_args.py:76-82); glm_5: 192 + 64, no rope factor
    (glm_5/model_args.py:42-48)."""
    nope, rope, factor = {"deepseek_v3_2": (128, 64, 40.0), "glm_5": (192, 64, None)}[model_arch]
    mscale = 1.0 if factor is None else 0.1 * math.log(factor) + 1.0
    return (nope + rope) ** -0.5 * mscale * mscale


def flash_sparse_mla(q_nope: torch.Tensor, q_pe: torch.Tensor, kv: torch.Tensor, pe: torch.Tensor,
                     indices: torch.Tensor, cur_pos: int, softmax_scale: float) -> torch.Tensor:
    """``FlashSparseMLACombine.golden_forward`` (ops/flash_sparse_mla.py:152-196) for batch 1:
    q_nope bf16 [s, h, 512], q_pe bf16 [s, h, 64], kv bf16 [T, 512], pe bf16 [T, 64], indices
    int [s, topk] (distinct positions).  scores = (q_nope . kv + q_pe . pe) * scale in fp32;
    every position not in the token's indices is -inf, and for s > 1 also every position
    after cur_pos + token (the triu mask); softmax in fp32, probabilities rounded to bf16,
    times kv -> bf16 [s, h, 512]."""
    s, h, _ = q_nope.shape
    T = kv.shape[0]
    scores = (torch.einsum("shc,tc->sht", q_nope.float(), kv.float())
              + torch.einsum("shr,tr->sht", q_pe.float(), pe.float())) * softmax_scale
    index_mask = torch.full((s, T), float("-inf")).scatter_(-1, indices.long(), 0)
    if s > 1:
        index_mask += torch.full((s, T), float("-inf")).triu_(cur_pos + 1)
    scores = (scores + index_mask[:, None, :]).softmax(dim=-1, dtype=torch.float32)
    return torch.einsum("sht,tc->shc", scores.to(torch.bfloat16), kv)


# ------------------------------------------------------- q RMSNorm + wq_b (BF16MMA)
def rmsnorm_projq_wqb(q: torch.Tensor, q_norm_weight: torch.Tensor, wq_b: torch.Tensor, wq_b_s: torch.Tensor,
                      n_heads: int, nope_dim: int = 128, rope_dim: int = 64, eps: float = 1e-6):
    """``RmsnormProjqWqb.golden_forward`` (ops/rmsnorm_projq_wqb.py:496-512): qr =
    bf16(rms_norm(q fp32, weight, eps)); out = qr @ weight_dequant(wq_b)^T with the weight
    dequantised to bf16 (``init_random_weights`` :463-474 builds ``ref_wq_b`` that way) and
    the product in bf16 (fp32 accumulation, bf16 result); split per head into q_nope
    [..., n_heads, nope_dim] and q_pe [..., n_heads, rope_dim].  q bf16 [s, q_lora_rank]."""
    qr = F.rms_norm(q.float(), [q.shape[-1]], q_norm_weight.float(), eps).to(torch.bfloat16)
    w = weight_dequant(wq_b, wq_b_s).to(torch.bfloat16)
    out = torch.matmul(qr, w.T).view(*q.shape[:-1], n_heads, nope_dim + rope_dim)
    return out[..., :nope_dim], out[..., nope_dim:]


# ------------------------------------------------ reference-layout MoE and dense MLP ops
def expert_select(scores: torch.Tensor, bias: torch.Tensor | None, topk: int, n_groups: int,
                  topk_groups: int, route_scale: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Routing of ``expert_select_up_gate_silu`` for logits [T, n_routed] (fp32):
    ``_ref_expert_select_ds`` (glm_5/_dsa_v32/ops/expert_sel_up_gate_silu.py:714-737; DeepSeek
    V3.2 uses 8 groups, top-4 groups) and ``_ref_expert_select_glm5`` (deepseek_v3_2/ops/
    expert_sel_up_gate_silu.py:641-652, = one group).  sigmoid, + bias for the choice only,
    group-limited (group score = sum of the group's top-2 biased scores, or its max without
    bias), top-k in descending order, weights = the chosen UNBIASED sigmoid scores
    normalised to sum 1, times route_scale.  Returns (weights fp32 [T, topk], indices int64
    [T, topk])."""
    s = scores.float().sigmoid()
    orig = s
    if bias is not None:
        s = s + bias.float()
    T, n = s.shape
    if n_groups > 1:
        g = s.view(T, n_groups, -1)
        gs = g.amax(dim=-1) if bias is None else g.topk(2, dim=-1)[0].sum(dim=-1)
        keep = gs.topk(topk_groups, dim=-1)[1]
        mask = s.new_ones(T, n_groups, dtype=torch.bool).scatter_(1, keep, False)
        s = g.masked_fill(mask.unsqueeze(-1), float("-inf")).flatten(1)
    idx = torch.topk(s, topk, dim=-1)[1]
    w = orig.gather(-1, idx)
    w = w / w.sum(dim=-1, keepdim=True)
    w = w * route_scale
    return w, idx


def expert_select_up_gate_silu(x: torch.Tensor, idx: torch.Tensor, gq: torch.Tensor, gs: torch.Tensor,
                               uq: torch.Tensor, us: torch.Tensor) -> torch.Tensor:
    """``ExpertSelectUpGateSiLU.golden_forward`` (deepseek_v3_2/ops/expert_sel_up_gate_silu.py:
    654-692) at one device's share: x bf16 [T, D]; idx [T, topk] routed ids; gq/uq e4m3fn
    [1 + n_routed, I, D] with block scales (expert 0 = the shared expert, routed expert j at
    1 + j), dequantised then rounded to bf16 (:545-552).  Per token: the shared expert, then
    the selected experts in idx order: h = bf16(silu(x G^T) * (x U^T)) in fp32 ->
    [T, 1 + topk, I] bf16."""
    T = x.shape[0]
    xf = x.float()
    cache: dict[int, tuple[torch.Tensor, torch.Tensor]] = {}

    def w(e):
        if e not in cache:
            cache[e] = (weight_dequant(gq[e], gs[e]).to(torch.bfloat16).float(),
                        weight_dequant(uq[e], us[e]).to(torch.bfloat16).float())
        return cache[e]
    out = []
    for t in range(T):
        rows = []
        for e in [0] + [1 + int(j) for j in idx[t]]:
            g, u = w(e)
            rows.append(swiglu(xf[t] @ g.T, xf[t] @ u.T))
        out.append(torch.stack(rows))
    return torch.stack(out).to(torch.bfloat16)


def expert_down_allreduce(h: torch.Tensor, idx: torch.Tensor, probs: torch.Tensor, dq: torch.Tensor,
                          ds: torch.Tensor, x_in: torch.Tensor | None = None) -> torch.Tensor:
    """``ExpertDownAllReduce.golden_forward`` (deepseek_v3_2/ops/expert_down_allreduce.py:
    445-468) at one device's share: h bf16 [T, 1 + topk, I]; dq e4m3fn [1 + n_routed, D, I]
    + block scales, dequantised then rounded to bf16 (:389-393).  Per token the shared term
    h[t,0] D_0^T and the routed terms probs[t,j] * (h[t,1+j] D_{1+idx}^T), each rounded to
    bf16, summed in fp32 and rounded once -> [T, D] bf16.  ``x_in`` (the residual the op's
    allreduce epilogue adds; single-GPU golden of padded_allreduce_add.py:100-114 is
    x_in + allreduce(partial)) is added to the bf16 sum when given."""
    T = h.shape[0]
    cache: dict[int, torch.Tensor] = {}

    def w(e):
        if e not in cache:
            cache[e] = weight_dequant(dq[e], ds[e]).to(torch.bfloat16).float()
        return cache[e]
    out = []
    for t in range(T):
        acc = (h[t, 0].float() @ w(0).T).to(torch.bfloat16).float()
        for j in range(idx.shape[1]):
            term = (h[t, 1 + j].float() @ w(1 + int(idx[t, j])).T) * probs[t, j].float()
            acc = acc + term.to(torch.bfloat16).float()
        out.append(acc)
    y = torch.stack(out).to(torch.bfloat16)
    if x_in is not None:
        y = (y.float() + x_in.float()).to(torch.bfloat16)
    return y


def rms_norm_f32(x: torch.Tensor, gamma: torch.Tensor, eps: float) -> torch.Tensor:
    """``torch.nn.functional.rms_norm(x.float(), [dim], gamma, eps)`` as the dense-MLP golden
    calls it (rmsnorm_up_gate_silu.py:333-335), fp32 out."""
    xf = x.float()
    return xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * gamma.float()


def rmsnorm_up_gate_silu(x: torch.Tensor, gamma: torch.Tensor, eps: float, gq: torch.Tensor, gs: torch.Tensor,
                         uq: torch.Tensor, us: torch.Tensor, bf16_operands: bool) -> torch.Tensor:
    """``RMSNormUpGateSiLU.golden_forward`` (deepseek_v3_2/ops/rmsnorm_up_gate_silu.py:323-347):
    x bf16 [T, D] -> fp32 RMSNorm -> for each of the device's chunks i (gq/uq e4m3fn
    [n_chunks, I, D] + block scales): h[t,i] = bf16(silu(xn G_i^T) * (xn U_i^T)) ->
    [T, n_chunks, I] bf16.  ``bf16_operands=False`` is the golden (fp32 normalised x, fp32
    dequantised weights); ``True`` rounds both operands to bf16 first, the numerics of the
    reference's FP16MMA/BF16MMA kernels (modules/mlp.py:24-29 selects FP16MMA) that the HIP
    kernel follows."""
    xn = rms_norm_f32(x, gamma, eps)
    if bf16_operands:
        xn = xn.to(torch.bfloat16).float()
    out = []
    for i in range(gq.shape[0]):
        g = weight_dequant(gq[i], gs[i])
        u = weight_dequant(uq[i], us[i])
        if bf16_operands:
            g, u = g.to(torch.bfloat16).float(), u.to(torch.bfloat16).float()
        out.append(swiglu(xn @ g.T, xn @ u.T))
    return torch.stack(out, dim=1).to(torch.bfloat16)


def down_allreduce(h: torch.Tensor, dq: torch.Tensor, ds: torch.Tensor, bf16_weights: bool,
                   x_in: torch.Tensor | None = None) -> torch.Tensor:
    """``DownAllReduce.golden_forward`` (deepseek_v3_2/ops/down_allreduce.py:293-320): h bf16
    [T, n_chunks, I], dq e4m3fn [n_chunks, D, I] + block scales; per token the chunk terms
    h[t,i] D_i^T, each rounded to bf16, summed in fp32, rounded once -> [T, D] bf16 (+ x_in
    as in ``expert_down_allreduce``).  ``bf16_weights`` rounds the dequantised weights to bf16
    (the kernel's numerics); the golden keeps them fp32."""
    terms = []
    for i in range(dq.shape[0]):
        w = weight_dequant(dq[i], ds[i])
        if bf16_weights:
            w = w.to(torch.bfloat16).float()
        terms.append((h[:, i].float() @ w.T).to(torch.bfloat16).float())
    y = torch.stack(terms).sum(0).to(torch.bfloat16)
    if x_in is not None:
        y = (y.float() + x_in.float()).to(torch.bfloat16)
    return y


# ------------------------------------------------------ absorbed MLA projections
def _kv_b_heads(wkv_b: torch.Tensor, s: torch.Tensor, n_heads: int, bf16_weights: bool) -> torch.Tensor:
    w = weight_dequant(wkv_b, s)
    if bf16_weights:
        w = w.to(torch.bfloat16).float()
    return w.view(n_heads, -1, w.shape[-1])


def projq_wqb(q_nope: torch.Tensor, wkv_b: torch.Tensor, s: torch.Tensor, n_heads: int, nope_dim: int,
              bf16_weights: bool) -> torch.Tensor:
    """``ProjqWqb.golden_forward`` (deepseek_v3_2/ops/projq_wqb.py:448-450, weights from
    ``init_reference_weights`` :374-385): the device's kv_b_proj shard dequantised, viewed
    [heads, nope + v, kv_lora], its first nope rows per head; ``einsum("bshd,hdc->bshc")`` in
    fp32 -> bf16.  ``bf16_weights`` rounds the dequantised weights to bf16 (bf16 inference's
    default dtype, the kernel's numerics)."""
    w = _kv_b_heads(wkv_b, s, n_heads, bf16_weights)[:, :nope_dim]
    return torch.einsum("bshd,hdc->bshc", q_nope.float(), w).to(torch.bfloat16)


def projo_wkvb(o_lat: torch.Tensor, wkv_b: torch.Tensor, s: torch.Tensor, n_heads: int, v_dim: int,
               bf16_weights: bool) -> torch.Tensor:
    """``ProjoWKVb.golden_forward`` (deepseek_v3_2/ops/projo_wkvb.py:465-467, weights :390-400):
    each head's last v_dim rows; ``einsum("bshc,hdc->bshd")`` in fp32 -> bf16."""
    w = _kv_b_heads(wkv_b, s, n_heads, bf16_weights)[:, -v_dim:]
    return torch.einsum("bshc,hdc->bshd", o_lat.float(), w).to(torch.bfloat16)


def unproj_o_allreduce(vec_in: torch.Tensor, wo: torch.Tensor, s: torch.Tensor, bf16_weights: bool,
                       x_in: torch.Tensor | None = None) -> torch.Tensor:
    """``UnProjOAllReduce.golden_forward`` (deepseek_v3_2/ops/unproj_o_allreduce.py:480-498):
    vec_in [1, s, ...] flattened per token, fp32 @ the dequantised o_proj shard^T -> bf16;
    + x_in as in ``expert_down_allreduce``."""
    w = weight_dequant(wo, s)
    if bf16_weights:
        w = w.to(torch.bfloat16).float()
    y = (vec_in.reshape(vec_in.shape[0], vec_in.shape[1], -1).float() @ w.T).to(torch.bfloat16)
    if x_in is not None:
        y = (y.float() + x_in.float()).to(torch.bfloat16)
    return y


# ------------------------------------------------------ the indexer's projections
def rmsnorm_projq_wqi(q: torch.Tensor, gamma: torch.Tensor, wqi: torch.Tensor, wqi_s: torch.Tensor, n_heads: int,
                      head_dim: int = 128, eps: float = 1e-6) -> torch.Tensor:
    """``RmsnormProjqWqi.golden_forward`` (deepseek_v3_2/ops/rmsnorm_projq_wqi.py:301-314):
    qr = bf16(rms_norm(q fp32, gamma, eps)); iq = qr @ bf16(dequant(wqi))^T viewed
    [..., n_heads, head_dim] -- ``rmsnorm_projq_wqb`` with no rope split."""
    iq, _ = rmsnorm_projq_wqb(q, gamma, wqi, wqi_s, n_heads, head_dim, 0, eps)
    return iq


def projx_wis(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``proj_w_op`` as the decoupled module runs it (rmsnorm_projx_wqakis.py:325-333): the
    bf16 normalised rows times the bf16 weights_proj^T, fp32 accumulation -> bf16."""
    return (x.float() @ w.float().T).to(torch.bfloat16)


def rmsnorm_projx_wqakis(x: torch.Tensor, gamma: torch.Tensor, wq_a: torch.Tensor, wq_a_s: torch.Tensor,
                         wk: torch.Tensor, wk_s: torch.Tensor, wis: torch.Tensor, eps: float = 1e-6):
    """``RMSNormProjxWqakis.golden_forward`` (deepseek_v3_2/ops/rmsnorm_projx_wqakis.py:279-299):
    fp32 rms_norm, then fp32 matmuls with the dequantised wq_a and wk and the bf16 weights_proj
    -> (q, ki, idx_scores) bf16."""
    xn = rms_norm_f32(x, gamma, eps)
    q = (xn @ weight_dequant(wq_a, wq_a_s).T).to(torch.bfloat16)
    ki = (xn @ weight_dequant(wk, wk_s).T).to(torch.bfloat16)
    sc = (xn @ wis.float().T).to(torch.bfloat16)
    return q, ki, sc
