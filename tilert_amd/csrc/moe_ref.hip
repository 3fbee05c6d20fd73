// The reference's MoE and dense-MLP operators in their own tensor layout: one device's share
// of the tensor-parallel split of every expert's intermediate dim (I = moe_inter_dim / 8 =
// 256 rows of gate, up and down per expert and device).
//
//  * expert_select_up_gate_silu_op (deepseek_v3_2/ops/expert_sel_up_gate_silu.py:23-48):
//    routing on the device -- sigmoid, + e_score_correction_bias for the choice only,
//    group-limited top-k, the chosen unbiased scores normalised and scaled by route_scale
//    (golden _ref_expert_select_ds, glm_5/_dsa_v32/ops/expert_sel_up_gate_silu.py:714-737;
//    one group = _ref_expert_select_glm5) -- then gate/up + SwiGLU of the shared expert and
//    the token's selected experts into hidden_out [T, 1 + topk, I] (golden :654-692).
//  * expert_down_allreduce_op (.../expert_down_allreduce.py:23-63, golden :445-468):
//    y[t] = bf16( sum over positions p of bf16(w[t,p] * (h[t,p] . D_{e(t,p)}^T)) ), the
//    shared position weighing 1, plus the residual x_in when given (the single-GPU form of
//    the allreduce epilogue, padded_allreduce_add.py:100-114).
//  * rmsnorm_up_gate_silu_op / down_allreduce_op (.../rmsnorm_up_gate_silu.py:26-44, golden
//    :318-347; .../down_allreduce.py:24-59, golden :293-320): the dense MLP's device share as
//    n_chunks pseudo-experts of I rows that every token uses, the RMSNorm fused into the
//    gate/up kernel.
//
// Local expert numbering: 0 = the shared expert, 1 + j = routed expert j (the reference's
// stacking, expert_sel_up_gate_silu.py:478-499); for the dense MLP, chunk i.  Weights use
// the MoE kernels' tile-major fragment packing (tl_moe_pack_weight) of the stacked
// [n_local * 2I, D] gate/up and [n_local * D, I] down matrices.
//
// Numerics: bf16 activations times fp8 weights dequantised in registers to
// bf16(fp32(q) * scale), v_mfma_f32_16x16x32_bf16, fp32 accumulation -- the goldens' own
// bf16 weights (expert_sel_up_gate_silu.py:545-552, expert_down_allreduce.py:389-393).
//
// Each token's (position -> local expert, weight) pairs are held one per lane (pair p =
// token p / P, position p % P; M * P <= 64), so hit sets are wave reductions and output
// positions and routing weights small LDS tables, with no host synchronisation and no
// dependent loads.
#include <math.h>

#include <algorithm>

#include "common.h"
#include "moe_common.h"
#include "../../include/tilert_amd.h"

namespace tl {

constexpr int kRefWaves = 8;
constexpr int kRefMaskWords = 5;            // local experts < 320 (shared + 256 routed)
constexpr int kRefMaxLocal = 64 * kRefMaskWords;
constexpr int kRefMaxRouted = 256;          // 4 per lane in the routing wave
constexpr int kRefLdsX = 64 * 1024;         // staged activations (x or gathered h)
constexpr int kRefGuDepth = 2;              // gate/up weight blocks (2 fragments each) in flight per wave
// down weight fragments in flight per wave (measured at M = 4: the MoE's ~7 items per wave
// are fastest at 3 (15.0 us vs 16.6 at 6), the dense share's 2-4 at 4 (8.4 vs 9.0 us))
__host__ __device__ constexpr int ref_down_depth(bool dense) { return dense ? 4 : 3; }

// Hit set over local experts, wave-uniform (scalar registers).
struct ExpertMask {
  uint64_t w[kRefMaskWords];
  int n;
};

// The set of local experts the lanes name (e < 0: none).
__device__ inline ExpertMask lanes_mask(int e) {
  ExpertMask m;
  m.n = 0;
#pragma unroll
  for (int k = 0; k < kRefMaskWords; ++k) {
    const uint64_t b = (e >= 64 * k && e < 64 * k + 64) ? (1ull << (e - 64 * k)) : 0ull;
    m.w[k] = wave_or_u64(b);
    m.n += __builtin_popcountll(m.w[k]);
  }
  return m;
}

// The n-th hit local expert in ascending order.
__device__ inline int mask_nth(const ExpertMask& m, int n) {
#pragma unroll
  for (int k = 0; k < kRefMaskWords; ++k) {
    const int c = __builtin_popcountll(m.w[k]);
    if (n < c) return 64 * k + nth_set_bit(m.w[k], n);
    n -= c;
  }
  return 0;
}

// This lane's pair: local expert (-1 past the M * P pairs, and for a routed id outside
// [0, n_local - 1), which is ignored) and weight.  The loads are unconditional (clamped),
// so wait counts of later loads stay exact.
template <bool DENSE>
__device__ inline void pair_lane(const int32_t* __restrict__ idx, const float* __restrict__ probs, int M, int P,
                                 int topk, int n_local, int& e, float& w) {
  const int lane = threadIdx.x & 63;
  const int t = lane / P, pos = lane - t * P;
  const bool live = lane < M * P;
  if (DENSE) {
    e = live ? pos : -1;
    w = 1.f;
    return;
  }
  const int q = min(t * topk + max(pos - 1, 0), M * topk - 1);
  const int ie = idx[q];
  const float pw = probs ? probs[q] : 0.f;
  e = !live ? -1 : (pos == 0 ? 0 : (ie >= 0 && ie < n_local - 1 ? 1 + ie : -1));
  w = pos == 0 ? 1.f : pw;
}

// ------------------------------------------------------------------------ routing
// One wave per token: lane l holds routed experts l, l + 64, l + 128, l + 192.  The wave
// is latency-bound (one wave, dependent steps), so every reduction is a register-level one:
// groups of 32 experts (DeepSeek-V3.2's 8 groups of 256) are the two 32-lane halves of one
// expert column, reduced with xor shuffles; each top-k round is one 64-bit DPP max over
// (order-preserving key, expert) pairs.
__device__ inline bool better(float v, int e, float bv, int be) { return v > bv || (v == bv && e < be); }

__device__ inline uint32_t route_key(float f) {  // larger float, larger key; 0 = unavailable
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}


// Top-2 (m1 >= m2) of this lane's pair and the pair a DPP move brings from another lane
// (-inf where the move has no source or the row is masked off).
template <int CTRL, int RMASK>
__device__ inline void top2_dpp(float& m1, float& m2) {
  const int ninf = __builtin_bit_cast(int, -INFINITY);
  const float o1 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(ninf, __builtin_bit_cast(int, m1), CTRL, RMASK, 0xf, false));
  const float o2 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(ninf, __builtin_bit_cast(int, m2), CTRL, RMASK, 0xf, false));
  const float lo = fminf(m1, o1);
  m1 = fmaxf(m1, o1);
  m2 = fmaxf(lo, fmaxf(m2, o2));
}

// Routing of one token by one wave (scores row `srow` [n]): on return lanes r < topk hold
// the token's r-th expert and its normalised, scaled probability.  bl [kRefMaxRouted],
// gscore [64] and gkeep [64] are this wave's LDS scratch (the general group path only); the
// wave's own LDS writes are ordered before its reads (wave-scope fences), so several waves
// of a workgroup can route tokens side by side.
__device__ inline void route_one(const float* __restrict__ srow, const float* __restrict__ bias, int n, int topk,
                                 int n_groups, int topk_groups, float route_scale, float* bl, float* gscore, int* gkeep,
                                 int& out_e, float& out_p) {
  const int lane = threadIdx.x & 63;
  auto wave_sync = [] {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  float s[4], b[4];
  bool live[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + 64 * i;
    live[i] = e < n;
    const float x = srow[min(e, n - 1)];
    s[i] = 1.0f / (1.0f + expf(-x));  // sigmoid
    b[i] = live[i] ? s[i] + (bias ? bias[min(e, n - 1)] : 0.f) : -INFINITY;
  }
  if (n_groups > 1) {  // keep the topk_groups best groups (score: top-2 sum with bias, else max)
    const int gsz = n / n_groups;
    if (gsz == 32 && n == 256) {
      // group 2 i + (lane >= 32) is held by one 32-lane half of column i: its top-2 by an
      // inclusive DPP scan (row shifts, then row 0 into row 1 and row 2 into row 3), which
      // leaves the half's top-2 in lanes 31 and 63
      float gs[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float m1 = b[i], m2 = -INFINITY;
        top2_dpp<0x111, 0xf>(m1, m2);  // row_shr:1
        top2_dpp<0x112, 0xf>(m1, m2);  // row_shr:2
        top2_dpp<0x114, 0xf>(m1, m2);  // row_shr:4
        top2_dpp<0x118, 0xf>(m1, m2);  // row_shr:8
        top2_dpp<0x142, 0xa>(m1, m2);  // row_bcast:15
        gs[i] = bias ? m1 + m2 : m1;
      }
      // group g's score: column g / 2, half g % 2
      float gv[8];
#pragma unroll
      for (int g = 0; g < 8; ++g)
        gv[g] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gs[g >> 1]), (g & 1) ? 63 : 31));
      // lane g < 8 ranks group g against the other seven; the kept groups are a ballot
      float mine = gv[0];
#pragma unroll
      for (int g = 1; g < 8; ++g) mine = lane == g ? gv[g] : mine;
      int rank = 0;
#pragma unroll
      for (int h = 0; h < 8; ++h) rank += better(gv[h], h, mine, lane) ? 1 : 0;
      const uint32_t keep_bits = static_cast<uint32_t>(__ballot(lane < 8 && rank < topk_groups));
      bool keep[8];
#pragma unroll
      for (int g = 0; g < 8; ++g) keep[g] = (keep_bits >> g) & 1u;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool k0 = keep[2 * i], k1 = keep[2 * i + 1];
        if (!(lane < 32 ? k0 : k1)) b[i] = -INFINITY;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (live[i]) bl[lane + 64 * i] = b[i];
      wave_sync();
      if (lane < n_groups) {
        float m1 = -INFINITY, m2 = -INFINITY;
        for (int j = 0; j < gsz; ++j) {
          const float v = bl[lane * gsz + j];
          if (v > m1) {
            m2 = m1;
            m1 = v;
          } else if (v > m2) {
            m2 = v;
          }
        }
        gscore[lane] = bias ? m1 + m2 : m1;
      }
      wave_sync();
      if (lane < n_groups) {
        int rank = 0;
        for (int g = 0; g < n_groups; ++g) rank += better(gscore[g], g, gscore[lane], lane) ? 1 : 0;
        gkeep[lane] = rank < topk_groups;
      }
      wave_sync();
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (live[i] && !gkeep[(lane + 64 * i) / gsz]) b[i] = -INFINITY;
    }
  }
  // top-k by repeated wave arg-max, descending, lowest expert first on ties: per round one
  // 32-bit DPP max of the order-preserving keys, then the lowest expert holding that key from
  // four ballots (expert lane + 64 i, so column order then lane order is expert order).
  // Taken and absent experts hold key 0, below every candidate.
  uint32_t ck[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) ck[i] = live[i] ? route_key(b[i]) : 0u;
  int my_e = 0;
  auto round = [&](int r) __attribute__((always_inline)) {
    const uint32_t best = wave_max_u32(max(max(ck[0], ck[1]), max(ck[2], ck[3])));
    const uint64_t b0 = __ballot(ck[0] == best), b1 = __ballot(ck[1] == best), b2 = __ballot(ck[2] == best),
                   b3 = __ballot(ck[3] == best);
    const int col = b0 ? 0 : (b1 ? 1 : (b2 ? 2 : 3));
    const int owner = __builtin_ctzll(b0 ? b0 : (b1 ? b1 : (b2 ? b2 : b3)));
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (i == col && lane == owner) ck[i] = 0u;
    if (lane == r) my_e = 64 * col + owner;
  };
  if (topk == 8) {  // both models' k: the rounds unrolled
#pragma unroll
    for (int r = 0; r < 8; ++r) round(r);
  } else {
    for (int r = 0; r < topk; ++r) round(r);
  }
  // lane r < topk: the unbiased score of its expert, from the lane that holds it; their sum
  // in round order
  const int own = my_e & 63, colr = my_e >> 6;
  const float s0 = __shfl(s[0], own), s1 = __shfl(s[1], own), s2 = __shfl(s[2], own), s3 = __shfl(s[3], own);
  const float my_s = colr == 0 ? s0 : (colr == 1 ? s1 : (colr == 2 ? s2 : s3));
  float sum = 0.f;
  for (int r = 0; r < topk; ++r) sum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_s), r));
  out_e = my_e;
  out_p = my_s / sum * route_scale;
}

__global__ __launch_bounds__(64) void moe_route_kernel(const float* __restrict__ scores, const float* __restrict__ bias,
                                                       int n, int topk, int n_groups, int topk_groups, float route_scale,
                                                       float* __restrict__ probs, int32_t* __restrict__ idx) {
  __shared__ float bl[kRefMaxRouted];
  __shared__ float gscore[64];
  __shared__ int gkeep[64];
  const int t = blockIdx.x, lane = threadIdx.x;
  int e;
  float p;
  route_one(scores + static_cast<size_t>(t) * n, bias, n, topk, n_groups, topk_groups, route_scale, bl, gscore, gkeep, e, p);
  if (lane < topk) {
    idx[t * topk + lane] = e;
    probs[t * topk + lane] = p;
  }
}

// ------------------------------------------------------------------------ gate/up
// Work item = (hit local expert, 16-row tile); a persistent grid strides over the items.
// Routing inputs and outputs of the fused expert selection (MoE gate/up only).
struct RouteArgs {
  const float* scores;  // [M, n_routed]
  const float* bias;    // [n_routed] or null
  int n_routed, n_groups, topk_groups;
  float route_scale;
  float* probs_out;     // [M, topk], written by workgroup 0
  int32_t* idx_out;     // [M, topk], written by workgroup 0
};

// x [M, D] bf16 is staged in LDS once per workgroup (DENSE: RMS-normalised there, in fp32,
// rounded to bf16, each wave normalising its own K blocks in its first pass); the waves
// stream weight fragments kRefGuDepth blocks ahead and read their activation operands from
// LDS.  The epilogue writes token r's row to every position p at which r uses the expert:
// h [M, P, I].
template <bool DENSE>
__global__ __launch_bounds__(kRefWaves * 64, 2) void ref_gate_up_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ gamma, float eps, const uint8_t* __restrict__ w13,
    const float* __restrict__ s13, const RouteArgs ra, int M, int P, int topk, int n_local, int D, int I,
    uint16_t* __restrict__ h) {
  extern __shared__ __align__(16) uint16_t xl[];  // [M][D]
  __shared__ v4f red[kRefWaves - 1][2][64];  // [wave][gate, up][lane]; before the items: the waves' routing scratch
  __shared__ float ssq[16][kRefWaves];
  __shared__ int8_t ptab[64 * 16];  // [slot][token]: the position where the token uses the slot's expert, -1 none
  __shared__ int16_t rpe[64];       // MoE: local expert of pair q (token q / P, position q % P)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int pe;
  float pw;
  if (DENSE) {
    pair_lane<true>(nullptr, nullptr, M, P, topk, n_local, pe, pw);
  } else {
    // The routing, fused: wave w selects the experts of tokens w, w + 8 (every workgroup
    // does so; workgroup 0 also writes them out for the down kernel).  Position 0 is the
    // shared expert (local 0), position 1 + r the token's r-th routed expert (local 1 + id).
    static_assert(sizeof(red) >= sizeof(float) * kRefWaves * (kRefMaxRouted + 128), "routing scratch");
    if (M <= kRefWaves / 2 && wave >= kRefWaves / 2) {
      // waves that route no token copy x straight into LDS meanwhile (no registers)
      const int x16 = M * D / 8, t0 = threadIdx.x - kRefWaves * 32;
      for (int cw = t0 - lane; cw < x16; cw += kRefWaves * 32)  // cw: this wave's first chunk (uniform)
        if (cw + lane < x16)
          __builtin_amdgcn_global_load_lds(reinterpret_cast<const u32x4*>(x) + cw + lane,
                                           (lds_ptr)(xl + static_cast<size_t>(cw) * 8), 16, 0, 0);
      __builtin_amdgcn_s_waitcnt(0);  // landed before the barrier below
    }
    float* scratch = reinterpret_cast<float*>(&red[0][0][0]) + wave * (kRefMaxRouted + 128);
    for (int t = wave; t < M; t += kRefWaves) {
      int e;
      float p;
      route_one(ra.scores + static_cast<size_t>(t) * ra.n_routed, ra.bias, ra.n_routed, topk, ra.n_groups,
                ra.topk_groups, ra.route_scale, scratch, scratch + kRefMaxRouted,
                reinterpret_cast<int*>(scratch + kRefMaxRouted + 64), e, p);
      if (lane < topk) {
        rpe[t * P + 1 + lane] = static_cast<int16_t>(1 + e);
        if (blockIdx.x == 0) {
          ra.idx_out[t * topk + lane] = e;
          ra.probs_out[t * topk + lane] = p;
        }
      }
      if (lane == 0) rpe[t * P] = 0;
    }
    __syncthreads();
    pe = lane < M * P ? rpe[lane] : -1;
    pw = 0.f;
  }
  const ExpertMask mask = lanes_mask(pe);
  // x straight into LDS (no registers), unless the routing's idle waves did so: waited for
  // in the first item's ring start, after the first weight fetches have been requested
  // (DENSE: before them, see below)
  const bool x_staged = !DENSE && M <= kRefWaves / 2;
  const int x16 = M * D / 8;
  if (!x_staged) {  // every chunk once (the copies are waited for explicitly, so their count may vary)
    const int c0 = threadIdx.x - lane;
    for (int cw = c0; cw < x16; cw += kRefWaves * 64)  // cw: this wave's first chunk (uniform)
      if (cw + lane < x16)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const u32x4*>(x) + cw + lane,
                                         (lds_ptr)(xl + static_cast<size_t>(cw) * 8), 16, 0, 0);
  }
  // DENSE: gamma [D] fp32 into LDS behind x (gl); x and gamma are waited for before any
  // weight fetch is issued, so the row statistics (in the first item's ring start) are
  // computed while the first weight fetches are in flight
  constexpr int kNormChunks = 2;  // D / 8 <= 1024 chunks of 8 per row
  float* gl = reinterpret_cast<float*>(xl + static_cast<size_t>(M) * D);
  if (DENSE) {
    const int g16 = D / 4, c0 = threadIdx.x - lane;
    for (int cw = c0; cw < g16; cw += kRefWaves * 64)
      if (cw + lane < g16)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const u32x4*>(gamma) + cw + lane,
                                         (lds_ptr)(gl + static_cast<size_t>(cw) * 4), 16, 0, 0);
    __builtin_amdgcn_s_waitcnt(0);
  }
  if (!DENSE && wave == 0) {  // position table from the lane-held pairs
    for (int i = lane; i < 64 * 16; i += 64) ptab[i] = -1;
    if (pe >= 0) {
      int slot = 0;
#pragma unroll
      for (int k = 0; k < kRefMaskWords; ++k) {
        const int base = 64 * k;
        slot += __builtin_popcountll(pe >= base + 64 ? mask.w[k]
                                                     : (pe > base ? mask.w[k] & ((1ull << (pe - base)) - 1ull) : 0ull));
      }
      const int t = lane / P;
      ptab[slot * 16 + t] = static_cast<int8_t>(lane - t * P);
    }
  }
  bool prepared = false;
  float rsv[4] = {0.f, 0.f, 0.f, 0.f};  // DENSE: 1 / rms of rows (lane >> 4) + 4 p
  bool norm_pending = DENSE;            // DENSE: this wave's K blocks not yet normalised
  // first item's ring start: x has landed and is visible to every wave; DENSE: the rows'
  // RMS statistics
  auto prepare = [&]() {
    if (prepared) return;
    prepared = true;
    if (x_staged) return;  // landed before the routing's barrier
    if (!DENSE) __builtin_amdgcn_s_waitcnt(0);  // DENSE: x and gamma were waited for before the fetches
    __syncthreads();
    if (DENSE) {
      // Row sums of squares, rows one at a time in rolled loops (this runs once per
      // workgroup between the first fetches and the first MFMA, where every wave
      // instruction costs its issue time): one DPP wave sum per row, the 8 wave partials
      // through LDS.  Each lane then holds 1 / rms of rows (lane >> 4) + 4 p, the rows it
      // normalises in the blocks of its wave.
      const int c16 = D / 8;
#pragma unroll 1
      for (int m = 0; m < M; ++m) {
        float a = 0.f;
#pragma unroll
        for (int u = 0; u < kNormChunks; ++u) {
          const int c = threadIdx.x + u * kRefWaves * 64;
          if (c < c16) {
            const u32x4 v = reinterpret_cast<const u32x4*>(xl + m * D)[c];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const float lo = bf16_to_f32(v[j] & 0xffffu), hi = bf16_to_f32(v[j] >> 16);
              a += lo * lo + hi * hi;
            }
          }
        }
        a = wave_sum_f32(a);
        if (lane == 0) ssq[m][wave] = a;
      }
      __syncthreads();
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int m = min((lane >> 4) + 4 * p, M - 1);
        float ss = 0.f;
#pragma unroll
        for (int w = 0; w < kRefWaves; ++w) ss += ssq[m][w];
        rsv[p] = 1.0f / sqrtf(ss / static_cast<float>(D) + eps);
      }
    }
  };
  const int KB = D >> 7, tiles = I >> 4, rows_e = 2 * I;
  const int r = lane & 15, g = lane >> 4;
  const uint16_t* xrow = xl + min(r, M - 1) * D;
  const int n = wave < KB ? (KB - wave + kRefWaves - 1) / kRefWaves : 0;  // K blocks wave + i * 8

  for (int item = blockIdx.x; item < mask.n * tiles; item += gridDim.x) {
    const int slot = item / tiles, rt = item - slot * tiles;
    const int e = mask_nth(mask, slot);
    const uint8_t* gate = w13 + (static_cast<size_t>(e) * (rows_e >> 4) + rt) * KB * 2048;
    const uint8_t* up = gate + static_cast<size_t>(tiles) * KB * 2048;
    const float* gs = s13 + (static_cast<size_t>(e) * (rows_e >> 7) + ((rt * 16) >> 7)) * KB;
    const float* us = s13 + (static_cast<size_t>(e) * (rows_e >> 7) + ((I + rt * 16) >> 7)) * KB;
    v4f ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
    struct Ops {
      v8i wg, wu;
      float gs, us;
    };
    Ops buf[kRefGuDepth];
    ring_pipeline(
        n, buf,
        [&](int i, Ops& o) {
          const int kb = wave + i * kRefWaves;
          o.wg = load_fragment(gate + static_cast<size_t>(kb) * 2048, lane);
          o.wu = load_fragment(up + static_cast<size_t>(kb) * 2048, lane);
          o.gs = load_f32_vector(gs + kb);
          o.us = load_f32_vector(us + kb);
        },
        [&](int i, const Ops& o) {
          const int kb = wave + i * kRefWaves;
          if (DENSE && norm_pending) {
            // RMSNorm of K block kb (this wave's own: no other wave reads it), in place:
            // x * (1 / rms) * gamma in fp32, rounded to bf16; lane (row m, 16-byte chunk c)
            const int c = lane & 15;
            const v4f g0 = *reinterpret_cast<const v4f*>(gl + kb * kBlock + 8 * c);
            const v4f g1 = *reinterpret_cast<const v4f*>(gl + kb * kBlock + 8 * c + 4);
            const float gv[8] = {g0[0], g0[1], g0[2], g0[3], g1[0], g1[1], g1[2], g1[3]};
#pragma unroll
            for (int p = 0; p < 4; ++p) {
              const int m = (lane >> 4) + 4 * p;
              if (4 * p < M && m < M) {
                u32x4* px = reinterpret_cast<u32x4*>(xl + m * D + kb * kBlock) + c;
                u32x4 v = *px;
#pragma unroll
                for (int j = 0; j < 4; ++j) {  // RNE to bf16 two at a time (v_cvt_pk_bf16_f32)
                  const v2f pr = {bf16_to_f32(v[j] & 0xffffu) * rsv[p] * gv[2 * j],
                                  bf16_to_f32(v[j] >> 16) * rsv[p] * gv[2 * j + 1]};
                  v[j] = bf16x2_bits(pr);
                }
                *px = v;
              }
            }
            // the wave's own LDS writes before its operand reads
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
          }
          const uint16_t* xk = xrow + kb * kBlock;
          const int off[4] = {16 * g, 16 * g + 8, 64 + 16 * g, 64 + 16 * g + 8};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const v8bf xa = *reinterpret_cast<const v8bf*>(xk + off[j]);
            ag = __builtin_amdgcn_mfma_f32_16x16x32_bf16(dequant8_bf16(o.wg[2 * j], o.wg[2 * j + 1], o.gs), xa, ag, 0, 0, 0);
            au = __builtin_amdgcn_mfma_f32_16x16x32_bf16(dequant8_bf16(o.wu[2 * j], o.wu[2 * j + 1], o.us), xa, au, 0, 0, 0);
          }
        },
        prepare);
    norm_pending = false;
    if (wave > 0) {
      red[wave - 1][0][lane] = ag;
      red[wave - 1][1][lane] = au;
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int w = 0; w < kRefWaves - 1; ++w) {
        ag += red[w][0][lane];
        au += red[w][1][lane];
      }
      const int pos = DENSE ? e : ptab[slot * 16 + min(r, M - 1)];
      if (r < M && pos >= 0) {
        uint16_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = f32_to_bf16(silu(ag[j]) * au[j]);
        uint16_t* dst = h + (static_cast<size_t>(r) * P + pos) * I + rt * 16 + 4 * g;
        *reinterpret_cast<uint2*>(dst) = make_uint2(o[0] | (static_cast<uint32_t>(o[1]) << 16),
                                                    o[2] | (static_cast<uint32_t>(o[3]) << 16));
      }
    }
    __syncthreads();
  }
  if (!prepared) __builtin_amdgcn_s_waitcnt(0);  // no item: the LDS copies land before the workgroup ends
}

// -------------------------------------------------------------------- down + combine
// One workgroup per 16-row output tile.  The rows each hit expert multiplies -- token r's
// h row at the position where r uses it, zero where r does not -- are gathered into LDS as
// [slot][M][I]; wave w takes slots w, w + 8, ... with all their K blocks (kRefGuDepth weight
// blocks in flight), so each slot's product is complete in one wave, which then adds the
// per-token terms bf16(weight * product) (the goldens' per-term rounding) to its fp32
// partial.  The 8 wave partials are summed in wave order (deterministic), rounded to bf16,
// and the residual x_in, when given, is added and rounded again.
template <bool DENSE>
__global__ __launch_bounds__(kRefWaves * 64, 2) void ref_down_kernel(
    const uint16_t* __restrict__ h, const uint8_t* __restrict__ w2, const float* __restrict__ s2,
    const int32_t* __restrict__ idx, const float* __restrict__ probs, const uint16_t* __restrict__ x_in, int M,
    int P, int topk, int n_local, int D, int I, uint16_t* __restrict__ y) {
  extern __shared__ __align__(16) uint16_t hl[];  // [M * P + 1][I]: h, then a zero row
  __shared__ v4f red[kRefWaves][64];
  __shared__ float wtab[64 * 16];    // [slot][token]: the token's routing weight for the slot's expert (0: unused)
  __shared__ uint8_t rtab[64 * 16];  // [slot][token]: the row of hl the product reads (MoE)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int pe;
  float pw;
  pair_lane<DENSE>(idx, probs, M, P, topk, n_local, pe, pw);
  const int KB = I >> 7;
  const int r = lane & 15, g = lane >> 4;
  const int row = min(r, M - 1);
  const int rt = blockIdx.x;
  // the residual this lane adds at the end, requested now (after the routing loads, so
  // waiting for those does not wait for it)
  uint2 xres = make_uint2(0u, 0u);
  if (x_in) xres = *reinterpret_cast<const uint2*>(x_in + static_cast<size_t>(row) * D + rt * 16 + 4 * g);
  const ExpertMask mask = lanes_mask(pe);
  // The slot of this lane's pair's expert: the rank of pe in the hit set.  h ([M * P][I], pair
  // q = token q / P, position q % P) is copied whole into LDS, followed by one zero row; the
  // product of slot j for token t reads row rtab[j][t]: its pair's row, or the zero row when
  // the token does not use the slot's expert.  The copy runs once the first weight fetches are
  // in flight (ring_pipeline's start).
  int pslot = -1;
  if (pe >= 0) {
    pslot = 0;
#pragma unroll
    for (int k = 0; k < kRefMaskWords; ++k) {
      const int base = 64 * k;
      const uint64_t below = pe >= base + 64 ? mask.w[k] : (pe > base ? mask.w[k] & ((1ull << (pe - base)) - 1ull) : 0ull);
      pslot += __builtin_popcountll(below);
    }
  }
  const int pairs = M * P;
  auto gather = [&]() {
    const int h16 = pairs * I / 8;  // 16-byte chunks of h
    const int c0 = threadIdx.x - lane;
    for (int cw = c0; cw < h16; cw += kRefWaves * 64)  // cw: this wave's first chunk (uniform)
      if (cw + lane < h16)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const u32x4*>(h) + cw + lane,
                                         (lds_ptr)(hl + static_cast<size_t>(cw) * 8), 16, 0, 0);
    for (int c = threadIdx.x; c < I / 8; c += blockDim.x)  // the zero row
      reinterpret_cast<u32x4*>(hl + static_cast<size_t>(pairs) * I)[c] = u32x4{0u, 0u, 0u, 0u};
    if (!DENSE) {
      for (int c = threadIdx.x; c < mask.n * 16; c += blockDim.x) {
        wtab[c] = 0.f;
        rtab[c] = static_cast<uint8_t>(pairs);
      }
      __syncthreads();
      if (wave == 0 && pslot >= 0) {  // the pair's weight (shared: 1) and row
        wtab[pslot * 16 + lane / P] = pw;
        rtab[pslot * 16 + lane / P] = static_cast<uint8_t>(lane);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  };
  v4f yacc = {0.f, 0.f, 0.f, 0.f};
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  const int my_slots = wave < mask.n ? (mask.n - wave + kRefWaves - 1) / kRefWaves : 0;
  const int n = my_slots * KB;  // item i: slot wave + (i / KB) * 8, K block i % KB
  struct Ops {
    v8i w;
    float sc;
  };
  Ops buf[ref_down_depth(DENSE)];
  ring_pipeline(
      n, buf,
      [&](int i, Ops& o) {
        const int j = wave + (i / KB) * kRefWaves, kb = i % KB;
        const int e = mask_nth(mask, j);
        o.w = load_fragment(w2 + ((static_cast<size_t>(e) * (D >> 4) + rt) * KB + kb) * 2048, lane);
        o.sc = load_f32_vector(s2 + (static_cast<size_t>(e) * (D >> 7) + ((rt * 16) >> 7)) * KB + kb);
      },
      [&](int i, const Ops& o) {
        const int j = wave + (i / KB) * kRefWaves, kb = i % KB;
        const int hr = DENSE ? row * P + j : rtab[j * 16 + row];  // dense: token row's chunk j
        const ActOperand xa = lds_act(hl + static_cast<size_t>(hr) * I + kb * kBlock, g);
        acc = mfma_block_bf16(o.w, o.sc, xa, acc);
        if (kb == KB - 1) {  // the slot's product is complete: add its weighted term
          const float wt = DENSE ? 1.f : wtab[j * 16 + row];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            yacc[q] += bf16_to_f32(f32_to_bf16(acc[q] * wt));
            acc[q] = 0.f;
          }
        }
      },
      gather);  // (ring_pipeline runs the gather even for a wave with no items: every wave meets its barriers)
  red[wave][lane] = yacc;
  __syncthreads();
  if (wave == 0 && r < M) {
    v4f s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kRefWaves; ++w) s += red[w][lane];
    uint16_t o[4];
    const size_t off = static_cast<size_t>(r) * D + rt * 16 + 4 * g;
    const uint16_t xr[4] = {static_cast<uint16_t>(xres.x & 0xffffu), static_cast<uint16_t>(xres.x >> 16),
                            static_cast<uint16_t>(xres.y & 0xffffu), static_cast<uint16_t>(xres.y >> 16)};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      o[q] = f32_to_bf16(s[q]);
      if (x_in) o[q] = f32_to_bf16(bf16_to_f32(o[q]) + bf16_to_f32(xr[q]));
    }
    *reinterpret_cast<uint2*>(y + off) = make_uint2(o[0] | (static_cast<uint32_t>(o[1]) << 16),
                                                    o[2] | (static_cast<uint32_t>(o[3]) << 16));
  }
}

static int check_common(const char* who, int64_t M, int64_t P, int64_t D, int64_t I) {
  if (M < 1 || M * P > 64) { set_error("%s: M=%lld with %lld positions per token: at most 64 pairs", who, (long long)M, (long long)P); return kErrUnsupported; }
  // The gate/up and down kernels compute one 16-token MFMA row tile (token r = lane & 15).
  if (M > 16) { set_error("%s: M=%lld > 16 tokens (one 16-row MFMA tile per call)", who, (long long)M); return kErrUnsupported; }
  if (D <= 0 || I <= 0 || D % kBlock || I % kBlock) { set_error("%s: D=%lld and I=%lld must be positive multiples of 128", who, (long long)D, (long long)I); return kErrArg; }
  if (D > (1 << 16) || I > (1 << 16)) { set_error("%s: D or I too large", who); return kErrArg; }
  return kOk;
}

static int launch_gate_up(bool dense, const void* x, const float* gamma, float eps, const void* w13, const float* s13,
                          const RouteArgs& ra, int64_t M, int64_t P, int64_t topk, int64_t n_local, int64_t D, int64_t I,
                          void* h, hipStream_t st) {
  const int64_t x_bytes = M * D * 2;
  if (x_bytes > kRefLdsX) { set_error("gate/up: M * D * 2 = %lld bytes of activations exceed %d", (long long)x_bytes, kRefLdsX); return kErrUnsupported; }
  const int64_t max_items = std::min<int64_t>(n_local, M * P) * (I / 16);
  const int grid = static_cast<int>(std::min<int64_t>(max_items, 512));
  const void* fn = dense ? reinterpret_cast<const void*>(ref_gate_up_kernel<true>) : reinterpret_cast<const void*>(ref_gate_up_kernel<false>);
  // DENSE: gamma [D] fp32 (D <= 8192) lies in LDS behind x
  const int64_t lds = x_bytes + (dense ? D * 4 : 0);
  if (int rc = allow_dynamic_lds(fn, dense ? kRefLdsX + 8192 * 4 : kRefLdsX, "gate/up")) return rc;
  if (dense)
    hipLaunchKernelGGL(ref_gate_up_kernel<true>, dim3(grid), dim3(kRefWaves * 64), static_cast<size_t>(lds), st,
                       (const uint16_t*)x, gamma, eps, (const uint8_t*)w13, s13, ra, (int)M, (int)P, (int)topk, (int)n_local, (int)D,
                       (int)I, (uint16_t*)h);
  else
    hipLaunchKernelGGL(ref_gate_up_kernel<false>, dim3(grid), dim3(kRefWaves * 64), static_cast<size_t>(x_bytes), st,
                       (const uint16_t*)x, gamma, eps, (const uint8_t*)w13, s13, ra, (int)M, (int)P, (int)topk, (int)n_local, (int)D,
                       (int)I, (uint16_t*)h);
  return check_launch("gate/up");
}

static int launch_down(bool dense, const void* h, const void* w2, const float* s2, const int32_t* idx, const float* probs,
                       const void* x_in, int64_t M, int64_t P, int64_t topk, int64_t n_local, int64_t D, int64_t I, void* y,
                       hipStream_t st) {
  const int64_t lds = (M * P + 1) * I * 2;  // h and one zero row
  if (lds > 96 * 1024) { set_error("down: %lld bytes of h rows exceed 96 KB (M=%lld, P=%lld, I=%lld)", (long long)lds, (long long)M, (long long)P, (long long)I); return kErrUnsupported; }
  const void* fn = dense ? reinterpret_cast<const void*>(ref_down_kernel<true>) : reinterpret_cast<const void*>(ref_down_kernel<false>);
  if (int rc = allow_dynamic_lds(fn, 96 * 1024, "down")) return rc;
  if (dense)
    hipLaunchKernelGGL(ref_down_kernel<true>, dim3(D / 16), dim3(kRefWaves * 64), static_cast<size_t>(lds), st,
                       (const uint16_t*)h, (const uint8_t*)w2, s2, idx, probs, (const uint16_t*)x_in, (int)M, (int)P,
                       (int)topk, (int)n_local, (int)D, (int)I, (uint16_t*)y);
  else
    hipLaunchKernelGGL(ref_down_kernel<false>, dim3(D / 16), dim3(kRefWaves * 64), static_cast<size_t>(lds), st,
                       (const uint16_t*)h, (const uint8_t*)w2, s2, idx, probs, (const uint16_t*)x_in, (int)M, (int)P,
                       (int)topk, (int)n_local, (int)D, (int)I, (uint16_t*)y);
  return check_launch("down");
}

static int check_routing(const char* who, int64_t M, int64_t n_routed, int64_t topk, int64_t n_groups, int64_t topk_groups,
                         bool has_bias) {
  if (M < 1 || M > 65535) { set_error("%s: M=%lld out of range", who, (long long)M); return kErrArg; }
  if (n_routed < 1 || n_routed > kRefMaxRouted) { set_error("%s: n_routed=%lld must be in [1, %d]", who, (long long)n_routed, kRefMaxRouted); return kErrUnsupported; }
  if (n_groups < 1 || n_groups > 64 || n_routed % n_groups) { set_error("%s: n_groups=%lld must divide n_routed=%lld (<= 64 groups)", who, (long long)n_groups, (long long)n_routed); return kErrArg; }
  if (topk_groups < 1 || topk_groups > n_groups) { set_error("%s: topk_groups=%lld must be in [1, n_groups]", who, (long long)topk_groups); return kErrArg; }
  if (topk < 1 || topk > 64 || topk > topk_groups * (n_routed / n_groups)) { set_error("%s: topk=%lld exceeds the experts of the kept groups", who, (long long)topk); return kErrArg; }
  // With a bias a group scores as the sum of its two best experts: groups need two experts.
  if (has_bias && n_groups > 1 && n_routed / n_groups < 2) { set_error("%s: with a bias each of the n_groups=%lld groups needs >= 2 experts", who, (long long)n_groups); return kErrArg; }
  return kOk;
}

}  // namespace tl

using namespace tl;


extern "C" int tl_moe_route(const float* scores, const float* bias, int64_t M, int64_t n_routed, int64_t topk,
                            int64_t n_groups, int64_t topk_groups, float route_scale, float* probs_out, int32_t* idx_out,
                            void* stream) {
  if (int rc = check_routing("moe_route", M, n_routed, topk, n_groups, topk_groups, bias != nullptr)) return rc;
  if (!scores || !probs_out || !idx_out) { set_error("moe_route: null pointer"); return kErrArg; }
  hipLaunchKernelGGL(moe_route_kernel, dim3(static_cast<unsigned>(M)), dim3(64), 0, (hipStream_t)stream, scores, bias,
                     (int)n_routed, (int)topk, (int)n_groups, (int)topk_groups, route_scale, probs_out, idx_out);
  return check_launch("moe_route");
}

extern "C" int tl_expert_select_up_gate_silu(const void* x_bf16, const float* scores, const float* bias,
                                             const void* w13_packed, const float* s13, int64_t M, int64_t n_routed,
                                             int64_t topk, int64_t n_groups, int64_t topk_groups, float route_scale,
                                             int64_t D, int64_t I, void* h_bf16, float* probs_out, int32_t* idx_out,
                                             void* stream) {
  const char* who = "expert_select_up_gate_silu";
  if (int rc = check_routing(who, M, n_routed, topk, n_groups, topk_groups, bias != nullptr)) return rc;
  if (int rc = check_common(who, M, 1 + topk, D, I)) return rc;
  if (!x_bf16 || !scores || !w13_packed || !s13 || !h_bf16 || !probs_out || !idx_out) { set_error("%s: null pointer", who); return kErrArg; }
  if ((reinterpret_cast<uintptr_t>(x_bf16) | reinterpret_cast<uintptr_t>(w13_packed) | reinterpret_cast<uintptr_t>(h_bf16)) & 15) {
    set_error("%s: x, weights and hidden_out must be 16-byte aligned", who);
    return kErrArg;
  }
  const RouteArgs ra{scores, bias, (int)n_routed, (int)n_groups, (int)topk_groups, route_scale, probs_out, idx_out};
  return launch_gate_up(false, x_bf16, nullptr, 0.f, w13_packed, s13, ra, M, 1 + topk, topk, 1 + n_routed, D, I,
                        h_bf16, (hipStream_t)stream);
}

extern "C" int tl_expert_down_allreduce(const void* h_bf16, const void* w2_packed, const float* s2, const int32_t* idx,
                                        const float* probs, const void* x_in_bf16, int64_t M, int64_t n_routed,
                                        int64_t topk, int64_t D, int64_t I, void* y_bf16, void* stream) {
  const char* who = "expert_down_allreduce";
  if (n_routed < 1 || n_routed + 1 > kRefMaxLocal) { set_error("%s: n_routed=%lld out of range", who, (long long)n_routed); return kErrUnsupported; }
  if (topk < 1) { set_error("%s: topk must be positive", who); return kErrArg; }
  if (int rc = check_common(who, M, 1 + topk, D, I)) return rc;
  if (!h_bf16 || !w2_packed || !s2 || !idx || !probs || !y_bf16) { set_error("%s: null pointer", who); return kErrArg; }
  if ((reinterpret_cast<uintptr_t>(h_bf16) | reinterpret_cast<uintptr_t>(w2_packed)) & 15 || reinterpret_cast<uintptr_t>(y_bf16) & 7 ||
      reinterpret_cast<uintptr_t>(x_in_bf16) & 7) {
    set_error("%s: h and weights must be 16-byte aligned, y and x_in 8-byte aligned", who);
    return kErrArg;
  }
  return launch_down(false, h_bf16, w2_packed, s2, idx, probs, x_in_bf16, M, 1 + topk, topk, 1 + n_routed, D, I, y_bf16,
                     (hipStream_t)stream);
}

extern "C" int tl_rmsnorm_up_gate_silu(const void* x_bf16, const float* gamma, float eps, const void* w13_packed,
                                       const float* s13, int64_t M, int64_t n_chunks, int64_t D, int64_t I, void* h_bf16,
                                       void* stream) {
  const char* who = "rmsnorm_up_gate_silu";
  if (D > 8192) { set_error("%s: D=%lld > 8192 (the norm takes two 8-element chunks per thread)", who, (long long)D); return kErrUnsupported; }
  if (n_chunks < 1 || n_chunks > kRefMaxLocal) { set_error("%s: n_chunks=%lld out of range", who, (long long)n_chunks); return kErrArg; }
  if (int rc = check_common(who, M, n_chunks, D, I)) return rc;
  if (!x_bf16 || !gamma || !w13_packed || !s13 || !h_bf16) { set_error("%s: null pointer", who); return kErrArg; }
  if ((reinterpret_cast<uintptr_t>(x_bf16) | reinterpret_cast<uintptr_t>(w13_packed) | reinterpret_cast<uintptr_t>(gamma) |
       reinterpret_cast<uintptr_t>(h_bf16)) & 15) {
    set_error("%s: x, gamma, weights and hidden_out must be 16-byte aligned", who);
    return kErrArg;
  }
  return launch_gate_up(true, x_bf16, gamma, eps, w13_packed, s13, RouteArgs{}, M, n_chunks, 0, n_chunks, D, I, h_bf16,
                        (hipStream_t)stream);
}

extern "C" int tl_down_allreduce(const void* h_bf16, const void* w2_packed, const float* s2, const void* x_in_bf16, int64_t M,
                                 int64_t n_chunks, int64_t D, int64_t I, void* y_bf16, void* stream) {
  const char* who = "down_allreduce";
  if (n_chunks < 1 || n_chunks > kRefMaxLocal) { set_error("%s: n_chunks=%lld out of range", who, (long long)n_chunks); return kErrArg; }
  if (int rc = check_common(who, M, n_chunks, D, I)) return rc;
  if (!h_bf16 || !w2_packed || !s2 || !y_bf16) { set_error("%s: null pointer", who); return kErrArg; }
  if ((reinterpret_cast<uintptr_t>(h_bf16) | reinterpret_cast<uintptr_t>(w2_packed)) & 15 || reinterpret_cast<uintptr_t>(y_bf16) & 7 ||
      reinterpret_cast<uintptr_t>(x_in_bf16) & 7) {
    set_error("%s: h and weights must be 16-byte aligned, y and x_in 8-byte aligned", who);
    return kErrArg;
  }
  return launch_down(true, h_bf16, w2_packed, s2, nullptr, nullptr, x_in_bf16, M, n_chunks, 0, n_chunks, D, I, y_bf16,
                     (hipStream_t)stream);
}
