// MoE expert layer at one expert-parallel shard: grouped gate/up GEMM with fused SwiGLU,
// then the down GEMM with the routing-weighted combine.
//
// Numerics follow the reference MoE (BF16MMA: bf16 activations, fp8 weights dequantised
// per 128x128 block; expert_sel_up_gate_silu.py:670-692, expert_down_allreduce.py:455-468).
// Each fp8 weight is dequantised in registers exactly as the reference's golden weights
// are built (init_reference_weights, expert_sel_up_gate_silu.py:545-552:
// bf16(fp32(q) * block_scale), round-to-nearest-even) and multiplied on the bf16 MFMA
// v_mfma_f32_16x16x32_bf16 with fp32 accumulation over the whole K -- so the products
// are the reference's products and only the fp32 summation order differs.
// (v_cvt_scalef32_pk_bf16_fp8 cannot do this: it applies only the scale's exponent.)
//
// Routing is an input (token -> 8 global expert ids).  Every kernel derives the shard's
// hit-expert set on the device from topk_idx, so no host synchronisation is needed: a
// local expert hit by any token gets a "slot" (ascending expert order); only hit experts'
// weights are read.  With M <= 16 tokens the MFMA's 16 columns cover every token, so
// each hit expert is evaluated for all tokens (unrouted rows are ignored by the combine).
//
// Weight layout: the fragment-packed layout of tl_fp8_pack_weight applied to the stacked
// per-expert matrices: gate/up as w13 [E][2I rows (gate then up)][D], down as
// w2 [E][D rows][I]; scales [E][2I/128][D/128] and [E][D/128][I/128].
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "moe_common.h"
#include "../../include/tilert_amd.h"

namespace tl {

constexpr int kMoeWaves = 8;        // gate/up waves per workgroup (2 workgroups per CU)
constexpr int kDownWaves = 8;       // down waves per workgroup
constexpr int kDownSlots = 4;  // hit experts reduced together by the down kernel
constexpr int kDnSlots = 8;    // hit experts per batch of the LDS down kernel
constexpr int kDownRedBytes = sizeof(float) * kDownWaves * kDnSlots * 4 * 64;  // cross-wave partials
constexpr int kDownTermBytes = sizeof(float) * kDnSlots * 4 * 64;              // per-slot terms
constexpr int kDnHBytes = 128 * 1024;  // staged h limit of the LDS down kernel (one workgroup per CU)
constexpr int kMaxLocalExperts = 64;

// Hit-expert bitmask of this shard, computed by each wave on its own (no LDS, no
// barrier): lanes test the routed ids and the 64-bit masks are OR-reduced across the
// wave's lanes.
__device__ inline uint64_t routing_mask(const int32_t* __restrict__ topk_idx, int pairs, int e0, int n_local) {
  const int lane = threadIdx.x & 63;
  uint64_t m = 0;
  for (int i = lane; i < pairs; i += 64) {
    const int e = topk_idx[i] - e0;
    if (e >= 0 && e < n_local) m |= 1ull << e;
  }
  // wave-uniform result (read from one lane), so the hit count, expert ids and weight
  // addresses derived from it live in scalar registers
  return wave_or_u64(m);
}


// One routed (expert, weight) pair per lane, loaded at kernel start and read back with
// lane shuffles by routing_weight: no dependent loads after the weight stream.
// The loads are unconditional (lanes past `pairs` reread the last pair), so wait counts
// for loads issued after them stay exact.
__device__ inline int lane_pair_expert(const int32_t* __restrict__ topk_idx, int pairs, int e0) {
  const int lane = threadIdx.x & 63;
  const int v = topk_idx[min(lane, pairs - 1)];
  return lane < pairs ? v - e0 : -1;
}
__device__ inline float lane_pair_weight(const float* __restrict__ topk_w, int pairs) {
  const int lane = threadIdx.x & 63;
  const float v = topk_w[min(lane, pairs - 1)];
  return lane < pairs ? v : 0.f;
}

// Hit-expert bitmask from the lane-held pairs (pairs <= 64), wave-uniform.
__device__ inline uint64_t lane_pairs_mask(int my_e, int n_local) {
  return wave_or_u64((my_e >= 0 && my_e < n_local) ? (1ull << my_e) : 0ull);
}

// Routing weight of (token r, local expert e); 0 when the token does not use it.  Pairs
// beyond the 64 held by the lanes are read from memory.
__device__ inline float routing_weight(const int32_t* __restrict__ topk_idx, const float* __restrict__ topk_w,
                                       int my_e, float my_w, int pairs, int topk, int e0, int r, bool tok, int e) {
  float wj = 0.f;
  for (int k = 0; k < topk; ++k) {
    const int src = r * topk + k;
    int ee;
    float v;
    if (pairs <= 64) {
      ee = __shfl(my_e, src & 63);
      v = __shfl(my_w, src & 63);
    } else {
      ee = tok ? topk_idx[src] - e0 : -1;
      v = tok ? topk_w[src] : 0.f;
    }
    if (tok && ee == e) wj = v;
  }
  return wj;
}

constexpr int kGuDepth = 2;  // weight blocks in flight per wave (gate/up, LDS activations)
constexpr int kDnDepth = 2;  // down items in flight per wave (LDS activations)
constexpr int kLdsActBytes = 64 * 1024;  // activation staging limit (2 workgroups per CU)

// ------------------------------------------------------ gate/up, LDS activations
// Used when x [M, D] bf16 fits in 64 KB (M <= 4 at D = 7168).  The workgroup stages x in
// LDS once; the waves then stream only weight fragments, kGuDepth blocks ahead through
// ring_pipeline, and read their activation operands from LDS, so nothing but the weight
// stream is waited on.  Work items, reduction and output as in moe_gate_up_kernel.
__global__ __launch_bounds__(kMoeWaves * 64, 4) void moe_gate_up_lds_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ w13, const float* __restrict__ s13,
    const int32_t* __restrict__ topk_idx, int M, int topk, int e0, int n_local, int D, int I,
    uint16_t* __restrict__ h) {
  extern __shared__ __align__(16) uint16_t xl[];  // [M][D]
  __shared__ v4f red[kMoeWaves - 1][2][64];
  // the routing and the x staging loads are in flight together (one round trip)
  const int pairs = M * topk;
  const int lane = threadIdx.x & 63;
  const int raw_e = topk_idx[min(lane, pairs - 1)];
  // x is copied straight into LDS (global_load_lds: no registers) once the hit set is
  // known, and the first weight fetches are requested right after it, before it has
  // landed; it is waited for just before the first compute.  (Issued before the routing
  // load is consumed, the copies would be waited for there: the compiler does not count
  // direct-to-LDS loads, so its wait for the routing load is a full vmcnt(0).)  Every
  // thread issues the same kStageChunks copies; sources past x repeat its last chunk and
  // their LDS destinations lie in the unused tail of the 64 KB allocation.
  const uint64_t mask = lane_pairs_mask(lane < pairs ? raw_e - e0 : -1, n_local);
  const int x16 = M * D / 8;
  copy_to_lds_fixed<kStageChunks>(x, x16, xl);
  const int n_hit = __builtin_popcountll(mask);
  const int KB = D >> 7;
  const int tiles = I >> 4;
  const int rows_e = 2 * I;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int r = lane & 15, g = lane >> 4;
  const uint16_t* xrow = xl + min(r, M - 1) * D;
  const int n = wave < KB ? (KB - wave + kMoeWaves - 1) / kMoeWaves : 0;  // K blocks wave + i*8
  bool staged = false;

  for (int item = blockIdx.x; item < n_hit * tiles; item += gridDim.x) {
    const int slot = item / tiles, rt = item - slot * tiles;
    const int e = nth_set_bit(mask, slot);
    const uint8_t* gate = w13 + (static_cast<size_t>(e) * (rows_e >> 4) + rt) * KB * 2048;
    const uint8_t* up = gate + static_cast<size_t>(tiles) * KB * 2048;
    const float* gs = s13 + (static_cast<size_t>(e) * (rows_e >> 7) + ((rt * 16) >> 7)) * KB;
    const float* us = s13 + (static_cast<size_t>(e) * (rows_e >> 7) + ((I + rt * 16) >> 7)) * KB;
    v4f ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
    struct Ops {
      v8i wg, wu;
      float gs, us;
    };
    Ops buf[kGuDepth];
    ring_pipeline(
        n, buf,
        [&](int i, Ops& o) {
          const int kb = wave + i * kMoeWaves;
          o.wg = load_fragment(gate + static_cast<size_t>(kb) * 2048, lane);
          o.wu = load_fragment(up + static_cast<size_t>(kb) * 2048, lane);
          o.gs = load_f32_vector(gs + kb);
          o.us = load_f32_vector(us + kb);
        },
        [&](int i, const Ops& o) {
          const int kb = wave + i * kMoeWaves;
          const uint16_t* xk = xrow + kb * kBlock;
          const int off[4] = {16 * g, 16 * g + 8, 64 + 16 * g, 64 + 16 * g + 8};
#pragma unroll
          for (int j = 0; j < 4; ++j) {  // one 32-wide K step at a time: few live registers
            const v8bf xa = *reinterpret_cast<const v8bf*>(xk + off[j]);
            ag = __builtin_amdgcn_mfma_f32_16x16x32_bf16(dequant8_bf16(o.wg[2 * j], o.wg[2 * j + 1], o.gs), xa, ag, 0, 0, 0);
            au = __builtin_amdgcn_mfma_f32_16x16x32_bf16(dequant8_bf16(o.wu[2 * j], o.wu[2 * j + 1], o.us), xa, au, 0, 0, 0);
          }
        },
        [&] {  // first item: x has landed (this wave's copies) and is visible (barrier)
          if (!staged) {
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            staged = true;
          }
        });
    if (wave > 0) {
      red[wave - 1][0][lane] = ag;
      red[wave - 1][1][lane] = au;
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int w = 0; w < kMoeWaves - 1; ++w) {
        ag += red[w][0][lane];
        au += red[w][1][lane];
      }
      if (r < M) {
        uint16_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = f32_to_bf16(silu(ag[j]) * au[j]);
        uint16_t* dst = h + (static_cast<size_t>(slot) * M + r) * I + rt * 16 + 4 * g;
        *reinterpret_cast<uint2*>(dst) = make_uint2(o[0] | (static_cast<uint32_t>(o[1]) << 16),
                                                    o[2] | (static_cast<uint32_t>(o[3]) << 16));
      }
    }
    __syncthreads();
  }
  if (!staged) __builtin_amdgcn_s_waitcnt(0);  // no item: the LDS copies land before the workgroup ends
}

// ------------------------------------------------------ down, LDS activations
// Used when one hit expert's h rows [M, I] fit in 64 KB.  A workgroup covers TPW 16-row
// output tiles with 8 waves each, so the staged h rows serve TPW tiles.  Hit experts are
// taken `sb` at a time (sb * M * I * 2 <= 64 KB); the batch's h rows are staged in LDS and
// each tile's (slot, K block) items, dealt round-robin to its 8 waves, are streamed
// kDnDepth ahead through ring_pipeline, one fp32 accumulator per slot.  After the stream
// the same LDS holds the cross-wave partials: local wave j of a tile reduces slot j over
// the tile's waves in order and rounds its weighted term to bf16 (the golden's per-term
// rounding, as moe_down_kernel does); local wave 0 adds the terms in slot order.
template <int TPW>
__global__ __launch_bounds__(kDownWaves * 64 * TPW, 4) void moe_down_lds_kernel(
    const uint16_t* __restrict__ h, const uint8_t* __restrict__ w2, const float* __restrict__ s2,
    const int32_t* __restrict__ topk_idx, const float* __restrict__ topk_w, int M, int topk, int e0,
    int n_local, int D, int I, int sb, uint16_t* __restrict__ y) {
  extern __shared__ __align__(16) uint8_t smem[];
  uint16_t* hl = reinterpret_cast<uint16_t*>(smem);  // [sb][M][I] during the stream
  v4f(*red)[kDnSlots][64] = reinterpret_cast<v4f(*)[kDnSlots][64]>(smem);  // after it
  v4f(*term)[kDnSlots][64] = reinterpret_cast<v4f(*)[kDnSlots][64]>(smem + TPW * kDownRedBytes);
  const int pairs = M * topk;
  const int my_e = lane_pair_expert(topk_idx, pairs, e0);
  const float my_w = lane_pair_weight(topk_w, pairs);
  // The hit set first (the routing loads are waited for here), then the first batch's h
  // rows are copied straight into LDS (global_load_lds, no registers) and the first weight
  // fetches requested behind them; the copy is waited for just before the first compute.
  // (Issued before the routing loads are consumed, the copies would be waited for there:
  // the compiler does not count direct-to-LDS loads, so its wait for them is a vmcnt(0).)
  const uint64_t mask = lane_pairs_mask(my_e, n_local);
  const int n_hit = __builtin_popcountll(mask);
  {
    const int ln = threadIdx.x & 63;
    const int c_end = min(n_hit, sb) * M * I / 8;
    for (int c0 = threadIdx.x - ln; c0 < c_end; c0 += blockDim.x)  // c0: this wave's first chunk
      if (c0 + ln < c_end)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const u32x4*>(h) + c0 + ln,
                                         (lds_ptr)(smem + static_cast<size_t>(c0) * 16), 16, 0, 0);
  }
  const int KB = I >> 7;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int tt = wave / kDownWaves, wl = wave % kDownWaves;           // tile in group, local wave
  const int r = lane & 15, g = lane >> 4;
  const bool tok = r < M;
  const int row = min(r, M - 1);
  const int rt = blockIdx.x * TPW + tt;
  v4f yacc = {0.f, 0.f, 0.f, 0.f};

  for (int s0 = 0; s0 < n_hit; s0 += sb) {
    const int ns = min(sb, n_hit - s0);
    const int h16 = ns * M * I / 8;
    v4f acc[kDnSlots];
#pragma unroll
    for (int j = 0; j < kDnSlots; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
    const int items = ns * KB;  // item = (slot it / KB, K block it % KB)
    const int n = wl < items ? (items - wl + kDownWaves - 1) / kDownWaves : 0;
    struct Ops {
      v8i w;
      float sc;
    };
    Ops buf[kDnDepth];
    float wj = 0.f;  // routing weight of (token r, slot s0 + wl): local wave j reduces slot j
    ring_pipeline(
        n, buf,
        [&](int i, Ops& o) {
          const int it = wl + i * kDownWaves;
          const int j = it / KB, kb = it - j * KB;
          const int e = nth_set_bit(mask, s0 + j);  // scalar bit arithmetic (no indexed array)
          const uint8_t* f = w2 + (static_cast<size_t>(e) * (D >> 4) + rt) * KB * 2048;
          const float* sp = s2 + (static_cast<size_t>(e) * (D >> 7) + ((rt * 16) >> 7)) * KB;
          o.w = load_fragment(f + static_cast<size_t>(kb) * 2048, lane);
          o.sc = load_f32_vector(sp + kb);
        },
        [&](int i, const Ops& o) {
          const int it = wl + i * kDownWaves;
          const int j = it / KB, kb = it - j * KB;
          const ActOperand xa = lds_act(hl + (j * M + row) * I + kb * kBlock, g);
#pragma unroll
          for (int jj = 0; jj < kDnSlots; ++jj)
            if (jj == j) acc[jj] = mfma_block_bf16(o.w, o.sc, xa, acc[jj]);
        },
        [&] {  // the batch's h rows into LDS while the first weight fetches are in flight
          if (s0 > 0) stage_commit(hl, stage_issue(h + static_cast<size_t>(s0) * M * I, h16), h16);
          if (wl < ns)
            wj = routing_weight(topk_idx, topk_w, my_e, my_w, pairs, topk, e0, r, tok, nth_set_bit(mask, s0 + wl));
          if (s0 == 0) __builtin_amdgcn_s_waitcnt(0);  // this wave's part of the direct copy has landed
          __syncthreads();
        });
    __syncthreads();  // every wave is done with hl before it becomes the partials
#pragma unroll
    for (int j = 0; j < kDnSlots; ++j)
      if (j < ns) red[wave][j][lane] = acc[j];  // (slots past the batch hold nothing)
    __syncthreads();
    if (wl < ns) {
      v4f t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < kDownWaves; ++w) t += red[tt * kDownWaves + w][wl][lane];
      v4f tw;
#pragma unroll
      for (int q = 0; q < 4; ++q) tw[q] = bf16_to_f32(f32_to_bf16(t[q] * wj));
      term[tt][wl][lane] = tw;
    }
    __syncthreads();
    if (wl == 0) {
      for (int j = 0; j < ns; ++j) yacc += term[tt][j][lane];
    }
    __syncthreads();
  }
  if (wl == 0 && tok) {
    uint16_t* dst = y + static_cast<size_t>(r) * D + rt * 16 + 4 * g;
    *reinterpret_cast<uint2*>(dst) =
        make_uint2(f32_to_bf16(yacc[0]) | (static_cast<uint32_t>(f32_to_bf16(yacc[1])) << 16),
                   f32_to_bf16(yacc[2]) | (static_cast<uint32_t>(f32_to_bf16(yacc[3])) << 16));
  }
}

// ---------------------------------------------------------------------- gate/up
// Work item = (slot, 16-channel tile); a persistent grid strides over n_hit * I/16 items.
// <= 128 VGPRs (4 waves per SIMD): two 8-wave workgroups per CU, so a 4-expert call's
// 512 work items run in one generation
__global__ __launch_bounds__(kMoeWaves * 64, 4) void moe_gate_up_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ w13, const float* __restrict__ s13,
    const int32_t* __restrict__ topk_idx, int M, int topk, int e0, int n_local, int D, int I,
    uint16_t* __restrict__ h) {
  __shared__ v4f red[kMoeWaves - 1][2][64];
  const uint64_t mask = routing_mask(topk_idx, M * topk, e0, n_local);
  const int n_hit = __builtin_popcountll(mask);
  const int KB = D >> 7;
  const int tiles = I >> 4;
  const int rows_e = 2 * I;  // gate rows then up rows
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const bool tok = r < M;
  const uint16_t* xrow = x + static_cast<size_t>(tok ? r : 0) * D;

  for (int item = blockIdx.x; item < n_hit * tiles; item += gridDim.x) {
    const int slot = item / tiles, rt = item - slot * tiles;
    const int e = nth_set_bit(mask, slot);
    const uint8_t* gate = w13 + (static_cast<size_t>(e) * (rows_e >> 4) + rt) * KB * 2048;
    const uint8_t* up = gate + static_cast<size_t>(tiles) * KB * 2048;
    const float* gs = s13 + (static_cast<size_t>(e) * (rows_e >> 7) + ((rt * 16) >> 7)) * KB;
    const float* us = s13 + (static_cast<size_t>(e) * (rows_e >> 7) + ((I + rt * 16) >> 7)) * KB;
    // Every operand of the next K block (both fragments, the activation block, both
    // scales) is requested one iteration ahead.  Vector loads retire in issue order, so a
    // current-iteration load issued after a prefetch would make the wait cover the
    // prefetch too; here the loop body only consumes registers loaded earlier.
    v4f ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
    int kb = wave;
    v8i wg_n = zero_v8i(), wu_n = zero_v8i();
    ActOperand xa_n = {};
    float gs_n = 0.f, us_n = 0.f;
    if (kb < KB) {
      wg_n = load_fragment(gate + static_cast<size_t>(kb) * 2048, lane);
      wu_n = load_fragment(up + static_cast<size_t>(kb) * 2048, lane);
      xa_n = load_act(xrow + kb * kBlock, g, tok);
      gs_n = gs[kb];
      us_n = us[kb];
    }
    for (; kb < KB; kb += kMoeWaves) {
      const v8i wg = wg_n, wu = wu_n;
      const ActOperand xa = xa_n;
      const float gsc = gs_n, usc = us_n;
      const int kn = kb + kMoeWaves;
      if (kn < KB) {
        wg_n = load_fragment(gate + static_cast<size_t>(kn) * 2048, lane);
        wu_n = load_fragment(up + static_cast<size_t>(kn) * 2048, lane);
        xa_n = load_act(xrow + kn * kBlock, g, tok);
        gs_n = gs[kn];
        us_n = us[kn];
      }
      ag = mfma_block_bf16(wg, gsc, xa, ag);
      au = mfma_block_bf16(wu, usc, xa, au);
    }
    if (wave > 0) {
      red[wave - 1][0][lane] = ag;
      red[wave - 1][1][lane] = au;
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int w = 0; w < kMoeWaves - 1; ++w) {
        ag += red[w][0][lane];
        au += red[w][1][lane];
      }
      if (tok) {
        uint16_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = f32_to_bf16(silu(ag[j]) * au[j]);
        uint16_t* dst = h + (static_cast<size_t>(slot) * M + r) * I + rt * 16 + 4 * g;
        *reinterpret_cast<uint2*>(dst) = make_uint2(o[0] | (static_cast<uint32_t>(o[1]) << 16),
                                                    o[2] | (static_cast<uint32_t>(o[3]) << 16));
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------- down + combine
// One workgroup per 16-row output tile.  Hit experts are taken kDownSlots at a time; the
// (slot, K block) items of a batch are dealt round-robin to the waves, each wave keeping
// one fp32 accumulator per slot, so every wave has a weight fragment in flight for the
// whole batch.  The per-slot partials are then reduced across waves in wave order and
// wave 0 applies, slot by slot in ascending order, the routing weight and the per-term
// bf16 rounding before the fp32 sum -- a fixed order, so the result is deterministic.
__global__ __launch_bounds__(kDownWaves * 64, 4) void moe_down_kernel(
    const uint16_t* __restrict__ h, const uint8_t* __restrict__ w2, const float* __restrict__ s2,
    const int32_t* __restrict__ topk_idx, const float* __restrict__ topk_w, int M, int topk, int e0,
    int n_local, int D, int I, uint16_t* __restrict__ y) {
  __shared__ float red[kDownWaves][kDownSlots][4][64];
  const uint64_t mask = routing_mask(topk_idx, M * topk, e0, n_local);
  const int n_hit = __builtin_popcountll(mask);
  const int KB = I >> 7;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const bool tok = r < M;
  const int rt = blockIdx.x;
  v4f yacc = {0.f, 0.f, 0.f, 0.f};
  // one routed (expert, weight) pair per lane, loaded now and consumed by the combine:
  // no dependent loads after the weight stream (M * topk <= 64 here; larger is looped)
  const int pairs = M * topk;
  const int my_e = lane_pair_expert(topk_idx, pairs, e0);
  const float my_w = lane_pair_weight(topk_w, pairs);

  for (int s0 = 0; s0 < n_hit; s0 += kDownSlots) {
    const int ns = min(kDownSlots, n_hit - s0);
    int ex[kDownSlots];
#pragma unroll
    for (int j = 0; j < kDownSlots; ++j) ex[j] = j < ns ? nth_set_bit(mask, s0 + j) : 0;
    v4f acc[kDownSlots];
#pragma unroll
    for (int j = 0; j < kDownSlots; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
    const int items = ns * KB;  // item i = (slot i / KB, K block i % KB)
    auto frag_of = [&](int it, int j) -> const uint8_t* {
      return w2 + ((static_cast<size_t>(ex[j]) * (D >> 4) + rt) * KB + (it - j * KB)) * 2048;
    };
    // next item's fragment, activation block and scale are requested one iteration
    // ahead (see the gate/up kernel for why all of them)
    auto scale_of = [&](int it, int j) -> float {
      return s2[(static_cast<size_t>(ex[j]) * (D >> 7) + ((rt * 16) >> 7)) * KB + (it - j * KB)];
    };
    auto act_of = [&](int it, int j) -> ActOperand {
      const uint16_t* hrow = h + (static_cast<size_t>(s0 + j) * M + (tok ? r : 0)) * I;
      return load_act(hrow + (it - j * KB) * kBlock, g, tok);
    };
    // Ping-pong over two operand buffers (the loop is unrolled by two) so the next item's
    // loads are in flight during this one's MFMAs. A plain `cur = next` rotation makes the
    // compiler copy registers at the end of each iteration, waiting for those loads.
    struct Ops {
      v8i w;
      ActOperand xa;
      float sc;
      int j;
    };
    auto fetch = [&](int it, Ops& o) {
      o.j = it / KB;
      o.w = load_fragment(frag_of(it, o.j), lane);
      o.xa = act_of(it, o.j);
      o.sc = scale_of(it, o.j);
    };
    auto compute = [&](const Ops& o) {
#pragma unroll
      for (int jj = 0; jj < kDownSlots; ++jj)
        if (jj == o.j) acc[jj] = mfma_block_bf16(o.w, o.sc, o.xa, acc[jj]);
    };
    constexpr int W = kDownWaves;
    Ops b0, b1;
    if (wave < items) fetch(wave, b0);
    for (int it = wave; it < items; it += 2 * W) {
      if (it + W < items) fetch(it + W, b1);
      compute(b0);
      if (it + W >= items) break;
      if (it + 2 * W < items) fetch(it + 2 * W, b0);
      compute(b1);
    }
#pragma unroll
    for (int j = 0; j < kDownSlots; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) red[wave][j][q][lane] = acc[j][q];
    __syncthreads();
    if (wave == 0) {
      for (int j = 0; j < ns; ++j) {
        v4f t = {0.f, 0.f, 0.f, 0.f};
        for (int w = 0; w < kDownWaves; ++w)
#pragma unroll
          for (int q = 0; q < 4; ++q) t[q] += red[w][j][q][lane];
        const float wj = routing_weight(topk_idx, topk_w, my_e, my_w, pairs, topk, e0, r, tok, ex[j]);
#pragma unroll
        for (int q = 0; q < 4; ++q) yacc[q] += bf16_to_f32(f32_to_bf16(t[q] * wj));
      }
    }
    __syncthreads();
  }
  if (wave == 0 && tok) {
    uint16_t* dst = y + static_cast<size_t>(r) * D + rt * 16 + 4 * g;
    *reinterpret_cast<uint2*>(dst) =
        make_uint2(f32_to_bf16(yacc[0]) | (static_cast<uint32_t>(f32_to_bf16(yacc[1])) << 16),
                   f32_to_bf16(yacc[2]) | (static_cast<uint32_t>(f32_to_bf16(yacc[3])) << 16));
  }
}

static int check_moe(const char* who, int64_t M, int64_t topk, int64_t n_local, int64_t D, int64_t I) {
  if (M < 1 || M > 16) { set_error("%s: M=%lld must be in [1, 16]", who, (long long)M); return kErrUnsupported; }
  if (topk < 1 || topk > 64) { set_error("%s: topk=%lld must be in [1, 64]", who, (long long)topk); return kErrArg; }
  if (n_local < 1 || n_local > kMaxLocalExperts) { set_error("%s: n_local=%lld must be in [1, %d]", who, (long long)n_local, kMaxLocalExperts); return kErrUnsupported; }
  if (D <= 0 || I <= 0 || D % kBlock || I % kBlock) { set_error("%s: D=%lld and I=%lld must be positive multiples of 128", who, (long long)D, (long long)I); return kErrArg; }
  if (D > (1 << 20) || I > (1 << 20)) { set_error("%s: D or I too large", who); return kErrArg; }
  return kOk;
}

}  // namespace tl

using namespace tl;

extern "C" int tl_moe_gate_up_swiglu(const void* x_bf16, const void* w13_packed, const float* s13,
                                     const int32_t* topk_idx, int64_t M, int64_t topk,
                                     int64_t expert_begin, int64_t n_local, int64_t D, int64_t I,
                                     void* h_bf16, void* stream) {
  int rc = check_moe("moe_gate_up_swiglu", M, topk, n_local, D, I);
  if (rc) return rc;
  if (!x_bf16 || !w13_packed || !s13 || !topk_idx || !h_bf16) { set_error("moe_gate_up_swiglu: null pointer"); return kErrArg; }
  if ((reinterpret_cast<uintptr_t>(x_bf16) | reinterpret_cast<uintptr_t>(w13_packed)) & 15) { set_error("moe_gate_up_swiglu: x and weights must be 16-byte aligned"); return kErrArg; }
  // enough workgroups for the largest possible hit set, capped at 4 per CU
  const int64_t max_items = n_local * (I / 16);
  const int grid = static_cast<int>(max_items < 512 ? max_items : 512);  // 2 x 8 waves per CU
  const int64_t x_bytes = M * D * 2;
  if (x_bytes <= kLdsActBytes && M * topk <= 64) {  // activations staged in LDS, routing in lanes
    rc = allow_dynamic_lds(reinterpret_cast<const void*>(moe_gate_up_lds_kernel), kLdsActBytes, "moe_gate_up_swiglu");
    if (rc) return rc;
    hipLaunchKernelGGL(moe_gate_up_lds_kernel, dim3(grid), dim3(kMoeWaves * 64), static_cast<size_t>(kLdsActBytes),
                       (hipStream_t)stream, (const uint16_t*)x_bf16, (const uint8_t*)w13_packed, s13, topk_idx,
                       (int)M, (int)topk, (int)expert_begin, (int)n_local, (int)D, (int)I, (uint16_t*)h_bf16);
  } else {
    hipLaunchKernelGGL(moe_gate_up_kernel, dim3(grid), dim3(kMoeWaves * 64), 0, (hipStream_t)stream,
                       (const uint16_t*)x_bf16, (const uint8_t*)w13_packed, s13, topk_idx, (int)M, (int)topk,
                       (int)expert_begin, (int)n_local, (int)D, (int)I, (uint16_t*)h_bf16);
  }
  return check_launch("moe_gate_up_swiglu");
}

extern "C" int tl_moe_down_combine(const void* h_bf16, const void* w2_packed, const float* s2,
                                   const int32_t* topk_idx, const float* topk_w, int64_t M,
                                   int64_t topk, int64_t expert_begin, int64_t n_local, int64_t D,
                                   int64_t I, void* y_bf16, void* stream) {
  int rc = check_moe("moe_down_combine", M, topk, n_local, D, I);
  if (rc) return rc;
  if (!h_bf16 || !w2_packed || !s2 || !topk_idx || !topk_w || !y_bf16) { set_error("moe_down_combine: null pointer"); return kErrArg; }
  if ((reinterpret_cast<uintptr_t>(h_bf16) | reinterpret_cast<uintptr_t>(w2_packed)) & 15) { set_error("moe_down_combine: h and weights must be 16-byte aligned"); return kErrArg; }
  const int64_t h_bytes = M * I * 2;  // one hit expert's h rows
  if (h_bytes <= kDnHBytes && M * topk <= 64) {  // activations staged in LDS, sb hit experts per batch
    // (the later batches are staged through registers: kStageChunks x 16 B per thread)
    const int64_t stage_cap = (D / 16) % 2 == 0 ? 2 * kLdsActBytes : kLdsActBytes;
    const int sb = static_cast<int>(std::min<int64_t>(kDnSlots, stage_cap / h_bytes));
    // two output tiles per workgroup when the tile count is even: the staged h serves both
    auto launch = [&](auto tpw_tag) -> int {
      constexpr int TPW = decltype(tpw_tag)::value;
      const size_t lds = std::max<size_t>(static_cast<size_t>(sb) * h_bytes, TPW * (kDownRedBytes + kDownTermBytes));
      const void* fn = reinterpret_cast<const void*>(moe_down_lds_kernel<TPW>);
      const int rc2 = allow_dynamic_lds(fn, static_cast<int>(lds), "moe_down_combine");
      if (rc2) return rc2;
      hipLaunchKernelGGL((moe_down_lds_kernel<TPW>), dim3(D / 16 / TPW), dim3(kDownWaves * 64 * TPW), lds,
                         (hipStream_t)stream, (const uint16_t*)h_bf16, (const uint8_t*)w2_packed, s2, topk_idx, topk_w,
                         (int)M, (int)topk, (int)expert_begin, (int)n_local, (int)D, (int)I, sb, (uint16_t*)y_bf16);
      return 0;
    };
    rc = (D / 16) % 2 == 0 ? launch(std::integral_constant<int, 2>{}) : launch(std::integral_constant<int, 1>{});
    if (rc) return rc;
  } else {
    hipLaunchKernelGGL(moe_down_kernel, dim3(D / 16), dim3(kDownWaves * 64), 0, (hipStream_t)stream,
                       (const uint16_t*)h_bf16, (const uint8_t*)w2_packed, s2, topk_idx, topk_w, (int)M, (int)topk,
                       (int)expert_begin, (int)n_local, (int)D, (int)I, (uint16_t*)y_bf16);
  }
  return check_launch("moe_down_combine");
}
