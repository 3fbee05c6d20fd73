"""fp64 brute-force evaluations on tiny inputs, built directly on the e4m3fn codec.

Test infrastructure only (see ``oracle/__init__.py``).  These use explicit Python/numpy
loops and the format-definition decoder in ``oracle.fp8`` -- no torch matmul, no torch
fp8 cast -- so that they pin ``oracle.reference`` independently of its own formulas.
"""
from __future__ import annotations

import numpy as np

from . import fp8


def gemm_fp64(a_codes, a_s, b_codes, b_s, block=128):
    """C[m,n] = sum_k dec(A)[m,k]*a_s[m,k//128] * dec(B)[n,k]*b_s[n//128,k//128], fp64 loops."""
    A = fp8.decode(a_codes).astype(np.float64)
    B = fp8.decode(b_codes).astype(np.float64)
    M, K = A.shape
    N = B.shape[0]
    C = np.zeros((M, N), dtype=np.float64)
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for kb in range(K // block):
                sl = slice(kb * block, (kb + 1) * block)
                acc += float(np.dot(A[m, sl], B[n, sl])) * float(a_s[m, kb]) * float(b_s[n // block, kb])
            C[m, n] = acc
    return C


def indexer_fp64(q_codes, q_s, k_codes, k_s, w, cur_pos):
    """score[t,l] = sum_h w[t,h] * max(0, sum_d qd[t,h,d] kd[l,d]) in fp64; -inf past the causal limit."""
    Q = fp8.decode(q_codes).astype(np.float64)
    Kc = fp8.decode(k_codes).astype(np.float64)
    M, H, D = Q.shape
    L = Kc.shape[0]
    qs = np.asarray(q_s, dtype=np.float64).reshape(M, -1)
    out = np.full((M, L), -np.inf)
    for t in range(M):
        for l in range(min(L, cur_pos + t + 1)):
            kd = Kc[l] * float(k_s[l])
            acc = 0.0
            for h in range(H):
                sq = qs[t, h] if qs.shape[1] == H else qs[t, 0]
                dot = float(np.dot(Q[t, h] * sq, kd))
                acc += float(w[t, h]) * max(dot, 0.0)
            out[t, l] = acc
    return out


def topk_fp64(scores, valid, k):
    """Top-k by selection: repeatedly take the max (lowest index on ties) -- O(k*L)."""
    rows = scores.shape[0]
    out = np.full((rows, k), -1, dtype=np.int64)
    for i in range(rows):
        v = np.array(scores[i, : valid[i]], dtype=np.float64)
        taken = np.zeros(v.shape[0], dtype=bool)
        for j in range(min(k, v.shape[0])):
            cand = np.where(taken, -np.inf, v)
            best = int(np.argmax(cand))  # argmax returns the first maximal index
            if taken[best]:
                break
            out[i, j] = best
            taken[best] = True
    return out


def expert_select_py(logits, bias, topk, n_groups, topk_groups, route_scale):
    """Routing by plain Python sorting, one token at a time (fp64 sigmoid): per group the
    sum of its two largest biased scores (its max without bias), keep the topk_groups best
    groups, then the topk best biased scores among their experts (descending), weights =
    unbiased sigmoid / their sum * route_scale."""
    import math
    T, n = len(logits), len(logits[0])
    gsz = n // n_groups
    W, I = [], []
    for t in range(T):
        s = [1.0 / (1.0 + math.exp(-float(v))) for v in logits[t]]
        b = [s[e] + (float(bias[e]) if bias is not None else 0.0) for e in range(n)]
        groups = list(range(n_groups))
        if n_groups > 1:
            def gscore(g):
                vals = sorted(b[g * gsz:(g + 1) * gsz], reverse=True)
                return vals[0] if bias is None else vals[0] + vals[1]
            groups = sorted(groups, key=lambda g: -gscore(g))[:topk_groups]
        allowed = [e for g in groups for e in range(g * gsz, (g + 1) * gsz)]
        chosen = sorted(allowed, key=lambda e: -b[e])[:topk]
        tot = sum(s[e] for e in chosen)
        I.append(chosen)
        W.append([s[e] / tot * route_scale for e in chosen])
    return W, I
