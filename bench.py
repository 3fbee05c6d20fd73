#!/usr/bin/env python3
"""MI355X benchmark of the FP8 decode hot path -- prints ONE JSON line.

Headline (the workload's stated metric): the block-scaled FP8 linear 7168 -> 18432 at M = 4
tokens (config 0's layer at decode + MTP=3 width): activations already quantised per
1x128 (the rmsnorm_quant output the projection ops consume), weights e4m3fn with one
fp32 scale per 128x128 block, output bf16.  One step = one GEMM call; K steps are
captured in a HIP graph and replayed, so the timed region is GPU work only.  Five
distinct weight copies (660 MB) rotate so the 256 MB Infinity Cache cannot serve
repeat reads.

  python bench.py [--steps K] [--warmup W] [--extras] [--no-cpu-baseline] [--only A,B]

The same line carries, under "configs", every other configuration of the workload, each
with µs per call, algorithmic bytes, its HBM fraction and a CPU baseline: the MLA
projections (config 1), the MoE layer at the EP=8 share (config 2), the M sweep with MFMA
utilisation (config 3), the indexer + exact top-2048 at 128K (config 4), and the
reference-layout operators (tensor-parallel MoE, dense-MLP share, absorbed MLA
projections).  Each configuration's graph holds a fixed 20 calls (20 routings for the
MoE), whatever --steps is, so its committed rocprof summary covers the same workload.
``--extras`` adds the launch-sized ops (RMSNorm + act_quant, paged indexer, key producer,
sparse MLA).  All inputs come from seeded CPU generators.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0
WARMUP_MIN_S = 0.2
CALLS = 20          # calls per captured graph for every configuration but the headline
MOE_ROUTINGS = CALLS  # config 2's routings: fixed, whatever --steps is
SECTIONS = ("headline", "moe_ep8_M4", "indexer_topk_128k_M4", "mla_projections_M4", "m_sweep", "ref_layout",
            "indexer_bf16", "extras")
METRIC = "µs/call + achieved HBM GB/s (% of peak) for FP8 block-scaled GEMM at M=4"


def _graph_time_us(torch, fn, steps: int, warmup: int) -> float:
    """Capture ``steps`` calls of fn(i) in a HIP graph; return mean GPU time per call."""
    for i in range(min(3, steps)):
        fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            fn(i)
    # Untimed warm-up: at least `warmup` calls and at least WARMUP_MIN_S of replays, so the
    # GPU clocks have ramped before the timed replay (one replay alone left per-call times
    # varying by +-0.5 us between otherwise identical runs).
    t_end = time.perf_counter() + WARMUP_MIN_S
    done = 0
    while done < max(1, warmup) or time.perf_counter() < t_end:
        g.replay()
        torch.cuda.synchronize()
        done += steps
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1000.0 / steps


def randn(torch, shape, gen, dev, scale=1.0):
    """N(0, scale^2) drawn on the CPU generator ``gen`` (so every host draws the same tensor
    for a seed), then copied to ``dev`` as fp32."""
    t = torch.randn(*shape, generator=gen)
    if scale != 1.0:
        t.mul_(scale)
    return t.to(dev)


def gemm_bytes(M: int, N: int, K: int) -> int:
    """Algorithmic HBM bytes of one block-scaled FP8 GEMM call: fp8 weight, fp32 block
    scales, fp8 activations + fp32 group scales, bf16 output."""
    return N * K + ((N + 127) // 128) * (K // 128) * 4 + M * K + M * (K // 128) * 4 + M * N * 2


def make_linear(torch, K, N, M, copies, seed, dev):
    """``copies`` weights W ~ N(0, 0.02) [N, K] block-quantised 128x128, and x ~ N(0, 1)
    [M, K] bf16 quantised per 1x128, all drawn on the CPU generator seeded ``seed`` (x first,
    then the weight copies; copy 0 is the configuration's seeded weight)."""
    g = torch.Generator().manual_seed(seed)
    x = randn(torch, (M, K), g, dev).to(torch.bfloat16)
    ws = []
    for _ in range(copies):
        q, s = K_.weight_quant(randn(torch, (N, K), g, dev, 0.02))
        ws.append((q, s, K_.pack_weight(q, s)))
    xq, xs = K_.act_quant(x)
    return ws, x, xq, xs


def bench_gemm(torch, M, N, K, steps, warmup, copies, dev, seed=0):
    ws, x, xq, xs = make_linear(torch, K, N, M, copies, seed, dev)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    us = _graph_time_us(torch, lambda i: K_.fp8_gemm(xq, xs, ws[i % copies][2], out=out), steps, warmup)
    return us, ws, x, xq, xs, out


def cpu_baseline_linear(torch, q, s, xq, xs, M, N, K):
    """Reference torch CPU path (oracle restatement of the projx goldens): fp32
    pre-dequantised weight, x_deq @ W^T -> bf16, timed on the host cores."""
    from oracle import reference as ref  # the checker/baseline only
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    qc, sc = q.cpu(), s.cpu()
    xqc, xsc = xq.cpu(), xs.cpu()
    wd = ref.weight_dequant(qc, sc)
    xd = ref.act_dequant(xqc, xsc)

    def fwd():
        return (xd @ wd.T).to(torch.bfloat16)

    for _ in range(3):
        fwd()
    ts = []
    for _ in range(10):
        t0 = time.perf_counter_ns()
        fwd()
        ts.append((time.perf_counter_ns() - t0) / 1e3)
    us = statistics.median(ts)
    t0 = time.perf_counter_ns()
    (ref.act_dequant(xqc, xsc) @ ref.weight_dequant(qc, sc).T).to(torch.bfloat16)
    us_deq = (time.perf_counter_ns() - t0) / 1e3
    return us, us_deq, cores


def measured_traffic(name: str, key: str = "traffic_bytes_per_launch"):
    """HBM bytes per launch from the committed rocprofv3 PMC summary (FETCH_SIZE +
    WRITE_SIZE, each scaled by a plain copy's reading), or None when absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(key + ":"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ----------------------------------------------------------------- configs 2 and 4
def moe_routes(torch, n, M=4, seed=3):
    """Config 2's routing: per token 8 distinct experts of 256, softmax weights over N(0,1)
    logits (CPU generator, so every host draws the same routes)."""
    gc = torch.Generator().manual_seed(seed)
    routes = []
    for _ in range(n):
        idx = torch.stack([torch.randperm(256, generator=gc)[:8] for _ in range(M)]).to(torch.int32)
        w = torch.softmax(torch.randn(M, 8, generator=gc), -1)
        routes.append((idx, w))
    return routes


def bench_moe(torch, dev, cpu=True):
    """Config 2: the MoE layer at the EP=8 share (32 local experts of 256, here experts
    32..63), M = 4, top-8.  One step = gate/up + SwiGLU and down + weighted combine for one
    routing; the MOE_ROUTINGS routings (fixed, whatever --steps is) rotate one per captured
    call over two weight copies (> MALL).  Weights and x are drawn on the CPU generator."""
    from tilert_amd import moe
    E, D, I, M, e0 = 32, 7168, 2048, 4, 32
    st = MOE_ROUTINGS
    g = torch.Generator().manual_seed(2)
    x = randn(torch, (M, D), g, dev).to(torch.bfloat16)
    copies, parts0 = [], None
    for _ in range(2):
        parts = []
        for (n, k) in ((I, D), (I, D), (D, I)):
            qs_, ss_ = [], []
            for _e in range(E):
                q, s = K_.weight_quant(randn(torch, (n, k), g, dev, 0.02))
                qs_.append(q)
                ss_.append(s)
            parts += [torch.stack(qs_), torch.stack(ss_)]
        copies.append(moe.LocalExperts(*parts, expert_begin=e0))
        if parts0 is None:
            parts0 = parts
        del parts, qs_, ss_
    routes = moe_routes(torch, st, M)
    routes_d = [(i.to(dev), w.to(dev)) for i, w in routes]
    hits = [len({int(e) for e in i.flatten() if e0 <= int(e) < e0 + E}) for i, _ in routes]
    h = torch.empty(E, M, I, dtype=torch.bfloat16, device=dev)
    y = torch.empty(M, D, dtype=torch.bfloat16, device=dev)
    us = _graph_time_us(torch, lambda i: moe.moe_forward(x, copies[i % 2], routes_d[i][0], routes_d[i][1], h, y),
                        st, 5)
    mean_hits = sum(hits) / len(hits)
    per_expert = 3 * I * D + 3 * (I // 128) * (D // 128) * 4
    # weights of the hit experts + x read + y written + h written and read back
    b = mean_hits * per_expert + M * D * 2 * 2 + mean_hits * M * I * 2 * 2
    res = {"us": round(us, 2), "mean_hit_experts": round(mean_hits, 3), "bytes_per_call": round(b),
           "GBs": round(b / us / 1e3, 1), "hbm_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
           "routings": len(routes), "weight_copies_rotated": 2,
           "roofline": {"bound": "hbm", "achieved": round(b / us / 1e3, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                        "traffic": measured_traffic("moe_ep8_M4.md"),
                        "traffic_source": "profiles/moe_ep8_M4.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; "
                                          f"gate/up + down per call over the same {MOE_ROUTINGS} routings)",
                        "kernel": "tl::moe_gate_up_lds_kernel + tl::moe_down_lds_kernel<2>",
                        "bytes_per_call": round(b)}}
    del copies
    if cpu:
        # the reference torch path on the host cores over the SAME routings the GPU ran (a
        # bounded sample of them): the goldens' per-pair fp32 products with bf16-rounded
        # dequantised weights (expert_sel_up_gate_silu.py:670-692, expert_down_allreduce.py:
        # 455-468), the bf16 weights of every hit expert dequantised beforehand (as
        # init_reference_weights does) and widened per use, as the goldens do
        from oracle import reference as ref  # the checker/baseline only
        sample = routes  # every routing the GPU ran
        need = sorted({e for i, _ in sample for e in ref.hit_experts(i, e0, E)})
        deq = {e: [ref.weight_dequant(parts0[2 * j][e].cpu(), parts0[2 * j + 1][e].cpu()).to(torch.bfloat16)
                   for j in range(3)] for e in need}
        xc = x.cpu()

        def moe_cpu(idx, w):
            xf = xc.float()
            y_ = torch.zeros(M, D)
            for (t, kk, e) in ref.local_pairs(idx, e0, E):
                g_, u_, d_ = deq[e]
                hh = (torch.nn.functional.silu(xf[t] @ g_.float().T) * (xf[t] @ u_.float().T)).to(torch.bfloat16)
                y_[t] += (w[t, kk] * (hh.float() @ d_.float().T)).to(torch.bfloat16).float()
            return y_.to(torch.bfloat16)
        torch.set_num_threads(len(os.sched_getaffinity(0)))
        moe_cpu(*sample[0])
        t0 = time.perf_counter_ns()
        for idx, w in sample:
            moe_cpu(idx, w)
        cus = (time.perf_counter_ns() - t0) / 1e3 / len(sample)
        s_hits = sum(hits[:len(sample)]) / len(sample)
        res["cpu_baseline"] = {"value": round(b / cus / 1e3, 2), "unit": "GB/s", "us": round(cus, 1),
                               "cores": len(os.sched_getaffinity(0)), "kind": "port",
                               "sample": f"the first {len(sample)} of the GPU's {len(routes)} routings "
                                         f"({s_hits:.2f} mean hit experts), one call each after a warm-up"}
        del deq
    del parts0
    torch.cuda.empty_cache()
    return res


def indexer_caches(torch, dev, n, L=131072, seed=4):
    """n fp8 key caches [L, 128]: keys ~N(0,1) (CPU generator) with per-key scale amax/448."""
    gk = torch.Generator().manual_seed(seed)
    caches = []
    for _ in range(n):
        k32 = randn(torch, (L, 128), gk, dev)
        ks = (k32.abs().amax(-1).clamp_min(1e-4) / 448.0).float()
        caches.append(((k32 / ks[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn), ks))
        del k32
    return caches, gk


def indexer_queries(torch, dev, gk, M, H):
    """q e4m3fn [M, H, 128] with a per-token scale (N(0,1) before act_quant-style scaling) and
    head weights bf16 [M, H] ~ N(0, 1/64), from the CPU generator gk."""
    q32 = randn(torch, (M, H * 128), gk, dev)
    qsc = (q32.abs().amax(-1).clamp_min(1e-4) / 448.0).float()
    q = (q32 / qsc[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn).reshape(M, H, 128)
    w = randn(torch, (M, H), gk, dev, 1 / 8).to(torch.bfloat16)
    return q, qsc, w


def bench_indexer(torch, dev, cpu=True, keep=False):
    """Config 4: DSA lightning-indexer scores over an fp8 key cache of 128K keys, M = 4
    tokens x 64 heads, then the exact top-2048 per token.  20 rotating caches (> MALL)."""
    from tilert_amd import sparse_index as si
    from tilert_amd.topk import topk_rows
    M, H, L, k = 4, 64, 131072, 2048
    st = CALLS
    caches, gk = indexer_caches(torch, dev, 20, L)
    q, qsc, w = indexer_queries(torch, dev, gk, M, H)
    logits = torch.empty(M, L, device=dev)
    idx = torch.empty(M, k, dtype=torch.int32, device=dev)
    us_s = _graph_time_us(torch, lambda i: si.sparse_index_fp8(q, qsc, caches[i % 20][0], caches[i % 20][1], w, logits,
                                                           L - 4), st, 5)
    us_k = _graph_time_us(torch, lambda i: topk_rows(logits, L - 4, k, out=idx), st, 5)
    us_b = _graph_time_us(torch, lambda i: si.sparse_index_topk_fp8(q, qsc, caches[i % 20][0], caches[i % 20][1], w,
                                                                logits, idx, L - 4), st, 5)
    b_s = L * 128 + L * 4 + M * H * 128 + M * 4 + M * H * 2 + M * L * 4
    b_all = b_s + M * L * 4 + M * k * 4  # + logits read back by the selection, indices written
    flops = 2 * M * H * 128 * L
    res = {"us": round(us_b, 2), "launches": 2, "scores_us": round(us_s, 2), "topk_us": round(us_k, 2),
           "bytes_per_call": b_all, "GBs": round(b_all / us_b / 1e3, 1),
           "hbm_frac": round(b_all / us_b / 1e3 / HBM_PEAK_GBS, 4),
           "scores_hbm_frac": round(b_s / us_s / 1e3 / HBM_PEAK_GBS, 4),
           "scores_mfma_util": round(flops / us_s / 1e6 / FP8_PEAK_TFLOPS, 4), "caches_rotated": 20,
           "roofline": {"bound": "hbm", "achieved": round(b_all / us_b / 1e3, 1), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(b_all / us_b / 1e3 / HBM_PEAK_GBS, 4),
                        "traffic": measured_traffic("indexer_topk_128k_M4.md"),
                        "traffic_source": "profiles/indexer_topk_128k_M4.md (rocprofv3 --pmc FETCH_SIZE, "
                                          "WRITE_SIZE; indexer + top-k per call)",
                        "kernel": "tl::indexer_kernel<4, 64, 16, 0> + tl::topk_kernel<4>", "bytes_per_call": b_all}}
    if cpu:
        # the reference torch path on the host cores: fp32 einsum of the dequantised q and
        # keys, ReLU, head-weighted sum, causal mask, torch.topk (ops/topk.py:128-143)
        qd_c = (q.float() * qsc[:, None, None]).cpu()
        kd_c = (caches[0][0].float() * caches[0][1][:, None]).cpu()
        w_c = w.float().cpu()

        def idx_cpu():
            sc_ = torch.einsum("thd,ld->thl", qd_c, kd_c).relu_()
            lg = torch.einsum("thl,th->tl", sc_, w_c)
            lim = (L - 4 + torch.arange(M))[:, None]
            lg = torch.where(torch.arange(L)[None, :] <= lim, lg, torch.tensor(float("-inf")))
            return lg.topk(k, dim=-1).indices
        cus = _cpu_time_us(torch, idx_cpu)
        res["cpu_baseline"] = {"value": round(b_all / cus / 1e3, 3), "unit": "GB/s", "us": cus,
                               "cores": len(os.sched_getaffinity(0)),
                               "kind": "port", "sample": "the full workload on one of the 20 caches, median of 3 "
                                                         "after a warm-up"}
        del qd_c, kd_c
    if keep:
        return res, caches, q, qsc, w, logits
    del caches
    torch.cuda.empty_cache()
    return res


def bench_indexer_bf16(torch, dev):
    """The reference's own bf16 indexer operators at 128K keys, M = 4, top-2048:
    sparse_index_topk (DeepSeek-V3.2, 64 heads) and sparse_index_topk_v3 (GLM-5, 32 heads),
    each one call (scores, then the exact top-k); 10 rotating bf16 caches (335 MB)."""
    from tilert_amd import sparse_index as si
    from tilert_amd.sparse_index_v3 import sparse_index_topk_v3
    M, L, k = 4, 131072, 2048
    g = torch.Generator().manual_seed(31)
    caches = [randn(torch, (1, L, 128), g, dev).to(torch.bfloat16) for _ in range(10)]
    logits = torch.empty(1, M, L, device=dev)
    idx = torch.empty(1, M, k, dtype=torch.int32, device=dev)
    out = {}
    for name, H, op in (("indexer_bf16_topk_dsv32_128k_M4", 64, si.sparse_index_topk),
                        ("indexer_bf16_topk_v3_glm5_128k_M4", 32, sparse_index_topk_v3)):
        q = randn(torch, (1, M, H, 128), g, dev).to(torch.bfloat16)
        w = randn(torch, (1, M, H), g, dev, 1 / 8).to(torch.bfloat16)
        us = _graph_time_us(torch, lambda i: op(q, caches[i % 10], w, logits, idx, L - 4, None), CALLS, 5)
        b = L * 256 + M * H * 256 + M * H * 2 + 2 * M * L * 4 + M * k * 4
        flops = 2 * M * H * 128 * L
        tkey = "traffic_bytes_per_launch_" + ("dsv32" if H == 64 else "glm5")
        out[name] = {"us": round(us, 2), "launches": 2, "bytes_per_call": b, "GBs": round(b / us / 1e3, 1),
                     "hbm_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                     "mfma_util_bf16": round(flops / us / 1e6 / BF16_PEAK_TFLOPS, 4),
                     "roofline": {"bound": "hbm", "achieved": round(b / us / 1e3, 1), "peak": HBM_PEAK_GBS,
                                  "unit": "GB/s", "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                                  "traffic": measured_traffic("indexer_bf16_128k_M4.md", tkey),
                                  "traffic_source": "profiles/indexer_bf16_128k_M4.md (rocprofv3 --pmc FETCH_SIZE, "
                                                    "WRITE_SIZE; scores + top-k per call)",
                                  "kernel": f"tl::indexer_kernel<4, {H}, {H // 4}, 2> + tl::topk_kernel<4>",
                                  "bytes_per_call": b}}
    del caches
    return out


def _stack_quant(torch, n, k, cnt, g, dev):
    """cnt weights N(0, 0.02) [n, k] (CPU generator g), block-quantised and stacked."""
    qs, ss = [], []
    for _ in range(cnt):
        q, s_ = K_.weight_quant(randn(torch, (n, k), g, dev, 0.02))
        qs.append(q)
        ss.append(s_)
    return torch.stack(qs), torch.stack(ss)


def bench_ref_layout(torch, dev):
    """The reference's own operator layouts at one device's share (DeepSeek-V3.2, M = 4):
    the tensor-parallel MoE (257 experts x 256 rows, routing on the device, residual), the
    dense MLP's 9 chunks x 256, and the absorbed MLA projections (16 heads)."""
    from tilert_amd.down_allreduce import down_allreduce
    from tilert_amd.expert_down_allreduce import DownExperts, expert_down_allreduce
    from tilert_amd.expert_sel_up_gate_silu import UpGateExperts, expert_select, expert_select_up_gate_silu
    from tilert_amd.projo_wkvb import convert_projo_wkvb, projo_wkvb
    from tilert_amd.projq_wqb import convert_projq_wqb, projq_wqb
    from tilert_amd.rmsnorm_up_gate_silu import rmsnorm_up_gate_silu
    from tilert_amd.unproj_o_allreduce import convert_unproj_o, unproj_o_allreduce
    out = {}
    st = CALLS
    M, D, I, E = 4, 7168, 256, 257
    g = torch.Generator().manual_seed(11)
    x = randn(torch, (1, M, D), g, dev).to(torch.bfloat16)
    xin = randn(torch, (1, M, D), g, dev).to(torch.bfloat16)
    copies = []
    for _ in range(2):  # 2 x 1.4 GB of expert weights: the MALL cannot hold a copy
        copies.append((UpGateExperts(*_stack_quant(torch, I, D, E, g, dev), *_stack_quant(torch, I, D, E, g, dev)),
                       DownExperts(*_stack_quant(torch, D, I, E, g, dev))))
    gc = torch.Generator().manual_seed(12)
    scores = [torch.randn(1, M, 256, generator=gc).to(dev) for _ in range(st)]
    bias = (torch.randn(256, generator=gc) * 0.1).to(dev)
    h = torch.empty(1, M, 9, I, dtype=torch.bfloat16, device=dev)
    probs = torch.empty(1, M, 8, device=dev)
    idx = torch.empty(1, M, 8, dtype=torch.int32, device=dev)
    y = torch.empty(1, M, D, dtype=torch.bfloat16, device=dev)

    def moe_step(i):
        up, dn = copies[i % 2]
        expert_select_up_gate_silu(x, scores[i], bias, up, h, probs, idx, None, model_arch="deepseek_v3_2")
        expert_down_allreduce(h, dn, None, idx, probs, xin, 0, y)
    us = _graph_time_us(torch, moe_step, st, 5)
    hits = []
    for sc in scores:
        pr = torch.empty(1, M, 8, device=dev)
        ix = torch.empty(1, M, 8, dtype=torch.int32, device=dev)
        expert_select(sc, bias, pr, ix, model_arch="deepseek_v3_2")
        hits.append(1 + len(set(ix.flatten().tolist())))
    mh = sum(hits) / len(hits)
    b = mh * (3 * I * D + 3 * (I // 128) * (D // 128) * 4) + M * D * 2 * 3 + M * 9 * I * 2 * 2
    out["moe_ref_layout_M4"] = {"us": round(us, 2), "mean_hit_experts": round(mh, 2), "bytes_per_call": round(b),
                                "GBs": round(b / us / 1e3, 1), "hbm_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                                "routings": st,
                                "roofline": {"bound": "hbm", "achieved": round(b / us / 1e3, 1), "peak": HBM_PEAK_GBS,
                                             "unit": "GB/s", "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                                             "traffic": measured_traffic("moe_ref_layout_M4.md"),
                                             "traffic_source": "profiles/moe_ref_layout_M4.md (rocprofv3 --pmc FETCH_SIZE, "
                                                               "WRITE_SIZE; gate/up + down per call)",
                                             "kernel": "tl::ref_gate_up_kernel<false> + tl::ref_down_kernel<false>",
                                             "bytes_per_call": round(b)}}
    del copies
    torch.cuda.empty_cache()

    # dense MLP share: 9 chunks x 256 rows, eight weight copies rotated
    dense = [(UpGateExperts(*_stack_quant(torch, I, D, 9, g, dev), *_stack_quant(torch, I, D, 9, g, dev)),
              DownExperts(*_stack_quant(torch, D, I, 9, g, dev))) for _ in range(8)]
    gam = (torch.rand(D, generator=g) + 0.5).to(dev)
    hd = torch.empty(1, M, 9, I, dtype=torch.bfloat16, device=dev)

    def dense_step(i):
        up, dn = dense[i % 8]
        rmsnorm_up_gate_silu(x, gam, up, hd, None, "deepseek_v3_2")
        down_allreduce(hd, dn, None, xin, 0, y, None, "deepseek_v3_2")
    us = _graph_time_us(torch, dense_step, st, 5)
    b = 9 * 3 * I * D + M * D * 2 * 3 + M * 9 * I * 2 * 2
    out["dense_mlp_share_M4"] = {"us": round(us, 2), "bytes_per_call": b, "GBs": round(b / us / 1e3, 1),
                                 "hbm_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                                 "roofline": {"bound": "hbm", "achieved": round(b / us / 1e3, 1), "peak": HBM_PEAK_GBS,
                                              "unit": "GB/s", "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                                              "traffic": measured_traffic("moe_ref_layout_M4.md",
                                                                          "traffic_bytes_per_launch_dense"),
                                              "traffic_source": "profiles/moe_ref_layout_M4.md (rocprofv3 --pmc "
                                                                "FETCH_SIZE, WRITE_SIZE; gate/up + down per call)",
                                              "kernel": "tl::ref_gate_up_kernel<true> + tl::ref_down_kernel<true>",
                                              "bytes_per_call": b}}
    del dense

    # absorbed MLA projections at the 16-head share
    H = 16
    wkv = [K_.weight_quant(randn(torch, (H * 256, 512), g, dev, 0.02)) for _ in range(8)]
    pq = [convert_projq_wqb(q, s_, H) for q, s_ in wkv]
    po = [convert_projo_wkvb(q, s_, H) for q, s_ in wkv]
    wo = [convert_unproj_o(*K_.weight_quant(randn(torch, (D, H * 128), g, dev, 0.02))) for _ in range(4)]
    qn = randn(torch, (1, M, H, 128), g, dev).to(torch.bfloat16)
    ol = randn(torch, (1, M, H, 512), g, dev).to(torch.bfloat16)
    ql = torch.empty(1, M, H, 512, dtype=torch.bfloat16, device=dev)
    ov = torch.empty(1, M, H, 128, dtype=torch.bfloat16, device=dev)
    res = {}
    us = _graph_time_us(torch, lambda i: projq_wqb(qn, pq[i % 8], None, ql, None, model_arch="deepseek_v3_2"), st, 5)
    res["projq_wqb"] = {"us": round(us, 2), "GBs": round((H * 128 * 512) / us / 1e3, 1)}
    us = _graph_time_us(torch, lambda i: projo_wkvb(ol, po[i % 8], None, ov, None, "deepseek_v3_2"), st, 5)
    res["projo_wkvb"] = {"us": round(us, 2), "GBs": round((H * 128 * 512) / us / 1e3, 1)}
    us = _graph_time_us(torch, lambda i: unproj_o_allreduce(ov, wo[i % 4], None, xin, 0, y, None, "deepseek_v3_2"),
                        st, 5)
    res["unproj_o_allreduce"] = {"us": round(us, 2), "GBs": round((D * H * 128) / us / 1e3, 1)}
    out["mla_absorbed_M4"] = res
    return out


def _cpu_time_us(torch, fn, reps=3):
    """Median wall time of fn() on the host cores (after one warm-up call)."""
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter_ns()
        fn()
        ts.append((time.perf_counter_ns() - t0) / 1e3)
    return round(statistics.median(ts), 1)


def bench_mla(torch, dev, cpu=True):
    """Config 1: the MLA attention projections of one decoder layer at the TP=8 share (16
    heads), M = 4: the five block-scaled FP8 linears one at a time, then the reference's own
    fusions -- projx_wqkva (wq_a + wkv_a in one launch), the DECOUPLED RMSNormProjxWqkva, and
    RmsnormProjqWqb (q RMSNorm + wq_b, BF16MMA) against RMSNorm + act_quant + the FP8 GEMV."""
    from tilert_amd.projx import pack_wqkva, projx_wqkva, rmsnorm_projx_wqkva
    from tilert_amd.rmsnorm import rmsnorm_quant
    from tilert_amd.rmsnorm_projq_wqb import rmsnorm_projq_wqb_op
    st = CALLS
    logs = torch.zeros(1, device=dev)
    mla = {"wq_a": (7168, 1536), "wq_b": (1536, 3072), "wkv_a": (7168, 576), "wkv_b": (512, 4096), "wo": (2048, 7168)}
    tot_us, tot_b = 0.0, 0
    per = {}
    cpu_layers = []
    for j, (name, (K, N)) in enumerate(mla.items()):
        us, ws_, _x, xq_, xs_q, _o = bench_gemm(torch, 4, N, K, st, 5, 8, dev, seed=10 + j)
        if cpu:
            from oracle import reference as ref  # the checker/baseline only
            cpu_layers.append((ref.act_dequant(xq_.cpu(), xs_q.cpu()),
                               ref.weight_dequant(ws_[0][0].cpu(), ws_[0][1].cpu())))
        del ws_
        b = gemm_bytes(4, N, K)
        per[name] = {"us": round(us, 2), "GBs": round(b / us / 1e3, 1), "hbm_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 3),
                     "bytes_per_call": b}
        tot_us += us
        tot_b += b
    # the fused wq_a + wkv_a launch (projx_wqkva, the reference's own fusion of the two)
    pw = []
    g = torch.Generator().manual_seed(100)
    for c in range(8):
        wq_, wqs_ = K_.weight_quant(randn(torch, (1536, 7168), g, dev, 0.02))
        wkv_, wkvs_ = K_.weight_quant(randn(torch, (576, 7168), g, dev, 0.02))
        pw.append(pack_wqkva(wq_, wqs_, wkv_, wkvs_, 512))
    xq4, xs4 = K_.act_quant(randn(torch, (1, 4, 7168), g, dev).to(torch.bfloat16))
    q4 = torch.empty(1, 4, 1536, dtype=torch.bfloat16, device=dev)
    kv4 = torch.empty(1, 4, 512, dtype=torch.bfloat16, device=dev)
    pe4 = torch.empty(1, 128, 64, dtype=torch.bfloat16, device=dev)
    cur4 = torch.tensor([7], dtype=torch.int32, device=dev)
    us = _graph_time_us(torch, lambda i: projx_wqkva(xq4, xs4, pw[i % 8], cur4, q4, kv4, pe4, None,
                                                     model_arch="deepseek_v3_2"), st, 5)
    b = gemm_bytes(4, 2112, 7168)
    fused_us = tot_us - per["wq_a"]["us"] - per["wkv_a"]["us"] + us
    xb4 = [randn(torch, (1, 4, 7168), g, dev).to(torch.bfloat16) for _ in range(4)]
    gx = (torch.rand(7168, generator=g) * 0.2 + 0.9).to(dev)  # RMSNorm scale ~U(0.9, 1.1)
    us_rx = _graph_time_us(torch, lambda i: rmsnorm_projx_wqkva(xb4[i % 4], gx, pw[i % 8], cur4, q4, kv4, pe4,
                                                                model_arch="deepseek_v3_2"), st, 5)
    b_rx = gemm_bytes(4, 2112, 7168) - 4 * 7168 - 4 * 56 * 4 + 4 * 7168 * 2 + 7168 * 4
    rx = {"us": round(us_rx, 2), "GBs": round(b_rx / us_rx / 1e3, 1), "launches": 2}
    qb_w = [K_.pack_weight(*K_.weight_quant(randn(torch, (3072, 1536), g, dev, 0.02))) for _ in range(8)]
    qa = randn(torch, (1, 4, 1536), g, dev).to(torch.bfloat16)
    qn_w = (torch.rand(1536, generator=g) * 0.2 + 0.9).to(dev)
    q_nope = torch.empty(1, 4, 16, 128, dtype=torch.bfloat16, device=dev)
    q_pe = torch.empty(1, 4, 16, 64, dtype=torch.bfloat16, device=dev)
    us_pq = _graph_time_us(torch, lambda i: rmsnorm_projq_wqb_op(qa, qb_w[i % 8], None, qn_w, q_nope, q_pe, None,
                                                                 "bf16mma", "deepseek_v3_2"), st, 5)
    qn_b = torch.empty(1, 4, 1536, dtype=torch.bfloat16, device=dev)
    qn_q = torch.empty(1, 4, 1536, dtype=torch.float8_e4m3fn, device=dev)
    qn_s = torch.empty(1, 4, 12, dtype=torch.float32, device=dev)
    qb_out = torch.empty(4, 3072, dtype=torch.bfloat16, device=dev)

    def two_launch(i):
        rmsnorm_quant(qa, qn_w, qn_b, qn_q, qn_s, logs, model_arch="deepseek_v3_2")
        K_.fp8_gemm(qn_q.view(4, 1536), qn_s.view(4, 12), qb_w[i % 8], out=qb_out)
    us_pq2 = _graph_time_us(torch, two_launch, st, 5)
    b_pq = 3072 * 1536 + 24 * 12 * 4 + 4 * 1536 * 2 + 1536 * 4 + 4 * 3072 * 2
    pq = {"us": round(us_pq, 2), "GBs": round(b_pq / us_pq / 1e3, 1),
          "rmsnorm_quant_then_fp8_gemv_us": round(us_pq2, 2)}
    res = {"layers": per, "us_total": round(tot_us, 2), "bytes_per_call": tot_b,
           "GBs": round(tot_b / tot_us / 1e3, 1), "hbm_frac": round(tot_b / tot_us / 1e3 / HBM_PEAK_GBS, 3),
           "projx_wqkva": {"us": round(us, 2), "GBs": round(b / us / 1e3, 1)},
           "rmsnorm_projq_wqb": pq, "rmsnorm_projx_wqkva": rx,
           "us_total_with_projx": round(fused_us, 2),
           "hbm_frac_with_projx": round(tot_b / fused_us / 1e3 / HBM_PEAK_GBS, 3),
           "weight_copies_rotated": 8}
    if cpu:
        # the reference torch path on the host cores: the goldens' fp32 x_deq @ W_deq^T -> bf16
        # per layer, weights dequantised beforehand (as init_reference_weights does)
        cus = _cpu_time_us(torch, lambda: [(xd @ wd.T).to(torch.bfloat16) for xd, wd in cpu_layers])
        res["cpu_baseline"] = {"value": round(tot_b / cus / 1e3, 2), "unit": "GB/s", "us": cus,
                               "cores": len(os.sched_getaffinity(0)), "kind": "port",
                               "sample": "the five layers once each, median of 3 after a warm-up"}
    return res


def bench_m_sweep(torch, dev, cpu=True):
    """Config 3: the dense MLP's up 7168 -> 18432 and down 18432 -> 7168 at M in {1, 4, 16,
    64, 256} (x for the i-th M drawn with seed i, i = 1..5; four weight copies rotated),
    with MFMA utilisation against the fp8 dense peak for M >= 64."""
    st = CALLS
    sweep = {}
    for tag, (K, N) in {"up_7168x18432": (7168, 18432), "down_18432x7168": (18432, 7168)}.items():
        ws, *_ = make_linear(torch, K, N, 1, 4, 7, dev)
        wd = None
        if cpu:
            from oracle import reference as ref  # the checker/baseline only
            wd = ref.weight_dequant(ws[0][0].cpu(), ws[0][1].cpu())
        for seed, M in enumerate((1, 4, 16, 64, 256), start=1):
            g = torch.Generator().manual_seed(seed)
            xq, xs = K_.act_quant(randn(torch, (M, K), g, dev).to(torch.bfloat16))
            o = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
            us = _graph_time_us(torch, lambda i: K_.fp8_gemm(xq, xs, ws[i % 4][2], out=o), st, 5)
            b = gemm_bytes(M, N, K)
            e = {"us": round(us, 2), "GBs": round(b / us / 1e3, 1), "hbm_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 3),
                 "bytes_per_call": b}
            if M >= 64:
                e["mfma_util"] = round(2.0 * M * N * K / us / 1e6 / FP8_PEAK_TFLOPS, 4)
            if cpu:
                xd = ref.act_dequant(xq.cpu(), xs.cpu())
                e["cpu_us"] = _cpu_time_us(torch, lambda: (xd @ wd.T).to(torch.bfloat16))
            sweep[f"{tag}_M{M}"] = e
        del ws, wd
        torch.cuda.empty_cache()
    if cpu:
        sweep["cpu_baseline"] = {"kind": "port", "cores": len(os.sched_getaffinity(0)),
                                 "sample": "cpu_us per entry: torch CPU fp32 x_deq @ W_deq^T -> bf16, weight "
                                           "pre-dequantised, median of 3 after a warm-up"}
    return sweep


def extras(torch, dev):
    """Launch-latency-sized ops of the path, beyond the configurations: RMSNorm + act_quant,
    the paged indexer, the indexer key producer, the indexer's input projections and sparse
    MLA attention."""
    from tilert_amd import sparse_index as si
    from tilert_amd.rmsnorm import rmsnorm_quant
    out = {}
    st = CALLS
    g = torch.Generator().manual_seed(21)
    xs_ = [randn(torch, (4, 7168), g, dev).to(torch.bfloat16) for _ in range(4)]
    gam = torch.ones(7168, device=dev)
    yb = torch.empty(4, 7168, dtype=torch.bfloat16, device=dev)
    yq = torch.empty(4, 7168, dtype=torch.float8_e4m3fn, device=dev)
    ysc = torch.empty(4, 56, dtype=torch.float32, device=dev)
    logs = torch.zeros(1, device=dev)
    us = _graph_time_us(torch, lambda i: rmsnorm_quant(xs_[i % 4], gam, yb, yq, ysc, logs, model_arch="deepseek_v3_2"),
                        st, 5)
    b = 4 * 7168 * 2 + 7168 * 4 + 4 * 7168 * 2 + 4 * 7168 + 4 * 56 * 4
    out["rmsnorm_quant_M4"] = {"us": round(us, 2), "bytes": b}

    # the paged form of config 4 (64-key pages of 8448 B), 20 rotating page sets
    M, H, L = 4, 64, 131072
    caches, gk = indexer_caches(torch, dev, 20, L)
    q, qsc, w = indexer_queries(torch, dev, gk, M, H)
    logits = torch.empty(M, L, device=dev)
    b_s = L * 128 + L * 4 + M * H * 128 + M * 4 + M * H * 2 + M * L * 4
    pages = [si.ki_pages_from_flat(kc, ksc) for kc, ksc in caches]
    del caches
    us_p = _graph_time_us(torch, lambda i: si.sparse_index_paged(q, qsc, pages[i % 20], w, logits, L - 4, L), st, 5)
    out["indexer_paged_128k_M4"] = {"scores_us": round(us_p, 2), "scores_GBs": round(b_s / us_p / 1e3, 1),
                                    "scores_hbm_frac": round(b_s / us_p / 1e3 / HBM_PEAK_GBS, 3)}
    del pages

    # the indexer key producer at decode (M = 4 new keys): LayerNorm -> RoPE -> Hadamard into
    # the KI pages in one launch, against the bf16 cache write followed by the page writer
    from tilert_amd.layernorm_rope_rotate import layernorm_rope_rotate, layernorm_rope_rotate_ki
    kx = randn(torch, (1, M, 128), g, dev).to(torch.bfloat16)
    kw, kb = torch.ones(128, device=dev), torch.zeros(128, device=dev)
    th = (torch.rand(M, 32, generator=g) * 6.28).to(dev)
    kf = torch.stack([th.cos(), th.sin()], -1).reshape(M, 1, 64).contiguous()
    kpos = torch.tensor([L - 4], dtype=torch.int32, device=dev)
    kpages = torch.zeros(L // 64, si.KI_PAGE_BYTES, dtype=torch.uint8, device=dev)
    kcache = torch.zeros(1, L, 128, dtype=torch.bfloat16, device=dev)
    us_f = _graph_time_us(torch, lambda i: layernorm_rope_rotate_ki(kx, kpos, kpages, kw, kb, kf), st, 5)

    def two_step(i):
        layernorm_rope_rotate(kx, kpos, kcache, kw, kb, kf, None, "deepseek_v3_2")
        si.ki_cache_write(kcache[0, L - 4:], kpages, L - 4)
    us_2 = _graph_time_us(torch, two_step, st, 5)
    out["ki_producer_M4"] = {"fused_us": round(us_f, 2), "bf16_cache_then_page_write_us": round(us_2, 2)}
    del kpages, kcache

    # the indexer's input projections at decode (M = 4, DeepSeek-V3.2): projx_wqaki (wq_a
    # and the indexer's wk in one FP8 GEMV, 1536 + 128 rows), projx_wis (the bf16 64 x 7168
    # weights_proj GEMV) and the DECOUPLED RMSNormProjxWqakis (rmsnorm_quant + the two),
    # 8 rotating weight sets
    from tilert_amd.projx_wqaki import pack_wqaki, projx_wis, projx_wqaki, rmsnorm_projx_wqakis
    gi = torch.Generator().manual_seed(31)
    pk, wis = [], []
    for _ in range(8):
        wq_, wqs_ = K_.weight_quant(randn(torch, (1536, 7168), gi, dev, 0.02))
        wk_, wks_ = K_.weight_quant(randn(torch, (128, 7168), gi, dev, 0.02))
        pk.append(pack_wqaki(wq_, wqs_, wk_, wks_))
        wis.append(randn(torch, (64, 7168), gi, dev, 0.02).to(torch.bfloat16))
    xi = [randn(torch, (1, M, 7168), gi, dev).to(torch.bfloat16) for _ in range(4)]
    xiq, xis = K_.act_quant(xi[0])
    gi_ = (torch.rand(7168, generator=gi) * 0.2 + 0.9).to(dev)
    qi = torch.empty(1, M, 1536, dtype=torch.bfloat16, device=dev)
    kii = torch.empty(1, M, 128, dtype=torch.bfloat16, device=dev)
    sci = torch.empty(1, M, 64, dtype=torch.bfloat16, device=dev)
    us_a = _graph_time_us(torch, lambda i: projx_wqaki(xiq, xis, pk[i % 8], qi, kii, None,
                                                       model_arch="deepseek_v3_2"), st, 5)
    us_w = _graph_time_us(torch, lambda i: projx_wis(xi[i % 4], wis[i % 8], sci), st, 5)
    us_r = _graph_time_us(torch, lambda i: rmsnorm_projx_wqakis(xi[i % 4], gi_, pk[i % 8], wis[i % 8], qi, kii, sci,
                                                                model_arch="deepseek_v3_2"), st, 5)
    b_a = gemm_bytes(M, 1664, 7168)
    b_w = 64 * 7168 * 2 + M * 7168 * 2 + M * 64 * 2
    out["indexer_projections_M4"] = {
        "projx_wqaki": {"us": round(us_a, 2), "GBs": round(b_a / us_a / 1e3, 1)},
        "projx_wis": {"us": round(us_w, 2), "GBs": round(b_w / us_w / 1e3, 1)},
        "rmsnorm_projx_wqakis": {"us": round(us_r, 2), "launches": 3}}
    del pk, wis

    # sparse MLA decode attention over the top-2048 of a 128K latent cache: 4 tokens x 16
    # heads (TP=8 share), independent selections per token, 3 rotating caches (> MALL)
    from tilert_amd.flash_sparse_mla import flash_sparse_mla
    T, Hm, km = L, 16, 2048
    gm = torch.Generator().manual_seed(5)
    kvs = [(randn(torch, (1, T, 512), gm, dev).to(torch.bfloat16),
            randn(torch, (1, T, 64), gm, dev).to(torch.bfloat16)) for _ in range(3)]
    qm = randn(torch, (1, M, Hm, 512), gm, dev, 0.5).to(torch.bfloat16)
    qpm = randn(torch, (1, M, Hm, 64), gm, dev, 0.5).to(torch.bfloat16)
    im = torch.stack([torch.randperm(T - 4, generator=gm)[:km] for _ in range(M)]).to(torch.int32)[None].to(dev)
    om = torch.empty(1, M, Hm, 512, dtype=torch.bfloat16, device=dev)
    pm = torch.tensor([T - 4], dtype=torch.int32, device=dev)
    us_m = _graph_time_us(torch, lambda i: flash_sparse_mla(qm, qpm, kvs[i % 3][0], kvs[i % 3][1], im, pm, om, None,
                                                            model_arch="deepseek_v3_2"), st, 5)
    gathered = M * km * (512 + 64) * 2
    acc = 2 * M * Hm * 32 * 512 * 4  # output_acc written by the split kernel, read by the combine
    out["sparse_mla_128k_M4"] = {"us": round(us_m, 2), "gathered_bytes": gathered,
                                 "gathered_GBs": round(gathered / us_m / 1e3, 1),
                                 "all_bytes_GBs": round((gathered + acc + qm.numel() * 2 * 2) / us_m / 1e3, 1),
                                 "hbm_frac_gathered": round(gathered / us_m / 1e3 / HBM_PEAK_GBS, 3)}
    del kvs
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--extras", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", default="", help=f"comma-separated subset of {list(SECTIONS)} (profiling runs)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 256 MiB device copy 10 times (scales rocprof FETCH/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU's share of the layout (TP/EP shard shapes); "
              f"--gpus {args.gpus} is not supported -- run with --gpus 1.", file=sys.stderr)
        return 2

    import torch
    global K_
    from tilert_amd import kernel as K_  # noqa: N811
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    if args.copy_calibration:
        n = 256 << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "calls": 10}))
        return 0
    only = set(args.only.split(",")) if args.only else None
    unknown = (only or set()) - set(SECTIONS)
    if unknown:
        print(f"bench.py: unknown --only names {sorted(unknown)}; choose from {list(SECTIONS)}", file=sys.stderr)
        return 2

    def want(name):
        return name in only if only else (name != "extras" or args.extras)

    def progress(msg):
        print(f"bench.py: {msg} ({time.perf_counter() - t_start:.0f} s)", file=sys.stderr, flush=True)
    t_start = time.perf_counter()
    cpu = not args.no_cpu_baseline
    res = {}
    M, N, Kd = 4, 18432, 7168
    if want("headline"):
        us, ws, x, xq, xs, out = bench_gemm(torch, M, N, Kd, args.steps, args.warmup, 5, dev)
        nbytes = gemm_bytes(M, N, Kd)
        gbs = nbytes / us / 1e3
        res = {
            "metric": METRIC,
            "value": round(gbs, 1),
            "unit": "GB/s",
            "us_per_call": round(us, 3),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": round(us / 1000.0, 6),
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "fp8e4m3 x fp8e4m3 -> fp32 acc -> bf16",
            "data": "synthetic (weights N(0,0.02) block-quantised 128x128, x N(0,1) act_quant 1x128; "
                    "drawn from seeded CPU generators)",
            "config": {"workload": "fp8_block_scaled_linear_7168x18432_M4", "M": M, "K": Kd, "N": N,
                       "weight_layout": "mfma-fragment-packed", "weight_copies_rotated": 5,
                       "timing": "HIP graph of K calls, HIP events around the replay",
                       "warmup_policy": f"max(W calls, {WARMUP_MIN_S} s of untimed replays)"},
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "traffic": measured_traffic("fp8_gemm_M4_7168x18432.md"),
                         "traffic_source": "profiles/fp8_gemm_M4_7168x18432.md (rocprofv3 --pmc FETCH_SIZE, "
                                           "WRITE_SIZE)",
                         "kernel": "tl::fp8_gemm_kernel<1, 8, true, 4, 1, false>", "bytes_per_call": nbytes},
        }
        if cpu:
            q, s, _ = ws[0]
            cus, cus_deq, cores = cpu_baseline_linear(torch, q, s, xq, xs, M, N, Kd)
            res["cpu_baseline"] = {"value": round(nbytes / cus / 1e3, 2), "unit": "GB/s", "cores": cores,
                                   "kind": "port", "us_per_call": round(cus, 1),
                                   "us_per_call_incl_dequant": round(cus_deq, 1),
                                   "sample": f"full workload, 1 call: torch CPU fp32 x_deq @ W_deq^T -> bf16 with "
                                             f"the weight pre-dequantised (oracle.reference), median of 10 after 3 "
                                             f"warm-up, {cores} threads on {cpu_model()}"}
        del ws
        torch.cuda.empty_cache()
        progress(f"headline {us:.2f} us")
    # every configuration of the workload on the default line, plus the reference-layout ops
    configs = {}
    runners = {"moe_ep8_M4": lambda: bench_moe(torch, dev, cpu=cpu),
               "indexer_topk_128k_M4": lambda: bench_indexer(torch, dev, cpu=cpu),
               "mla_projections_M4": lambda: bench_mla(torch, dev, cpu=cpu),
               "m_sweep": lambda: bench_m_sweep(torch, dev, cpu=cpu)}
    for name, run in runners.items():
        if want(name):
            configs[name] = run()
            torch.cuda.empty_cache()
            progress(name)
    if want("ref_layout"):
        configs.update(bench_ref_layout(torch, dev))
        torch.cuda.empty_cache()
        progress("ref_layout")
    if want("indexer_bf16"):
        configs.update(bench_indexer_bf16(torch, dev))
        progress("indexer_bf16")
    if configs:
        res["configs"] = configs
    if want("extras"):
        res["extras"] = extras(torch, dev)
        progress("extras")
    print(json.dumps(res))
    return 0


if __name__ == "__main__":
    sys.exit(main())
