// Device helpers shared by the MoE kernels (moe.hip: the expert-parallel shard;
// moe_ref.hip: the reference's tensor-parallel expert layout and the dense MLP).
#pragma once

#include "common.h"

namespace tl {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));


__device__ inline v8i load_fragment(const uint8_t* frag, int lane) {
  const u32x4* p = reinterpret_cast<const u32x4*>(frag);
  const u32x4 lo = __builtin_nontemporal_load(p + lane);
  const u32x4 hi = __builtin_nontemporal_load(p + 64 + lane);
  v8i r;
  r[0] = lo.x; r[1] = lo.y; r[2] = lo.z; r[3] = lo.w;
  r[4] = hi.x; r[5] = hi.y; r[6] = hi.z; r[7] = hi.w;
  return r;
}

// The bf16 activation operand matching a packed weight fragment: lane group g holds
// K offsets {16g..16g+15} and {64+16g..64+16g+15} of the block, as 4 groups of 8.
struct ActOperand {
  v8bf v[4];
};

__device__ inline ActOperand load_act(const uint16_t* row_kblock, int g, bool live) {
  ActOperand o;
  const int off[4] = {16 * g, 16 * g + 8, 64 + 16 * g, 64 + 16 * g + 8};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    u32x4 d = {0u, 0u, 0u, 0u};
    if (live) d = *reinterpret_cast<const u32x4*>(row_kblock + off[j]);
    o.v[j] = __builtin_bit_cast(v8bf, d);
  }
  return o;
}

// acc[16 rows x 16 tokens] += dequant(W block) . x over one 128-wide K block: 4 chained
// bf16 MFMAs on the block's bf16-rounded dequantised weights.
__device__ inline v4f mfma_block_bf16(const v8i& w, float scale, const ActOperand& x, v4f acc) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(dequant8_bf16(w[2 * j], w[2 * j + 1], scale), x.v[j], acc, 0, 0, 0);
  return acc;
}

__device__ inline int nth_set_bit(uint64_t m, int n) {
  for (int i = 0; i < n; ++i) m &= m - 1;
  return __builtin_ctzll(m);
}

__device__ inline float silu(float g) { return g / (1.0f + __expf(-g)); }

// The activation operand read from LDS: lane (r, g) takes row `row` (token r, clamped
// to a valid row: columns past M are never stored) at the lane group's K offsets.
__device__ inline ActOperand lds_act(const uint16_t* row_kblock, int g) {
  ActOperand o;
  const int off[4] = {16 * g, 16 * g + 8, 64 + 16 * g, 64 + 16 * g + 8};
#pragma unroll
  for (int j = 0; j < 4; ++j) o.v[j] = *reinterpret_cast<const v8bf*>(row_kblock + off[j]);
  return o;
}

// Workgroup-wide copy of n16 16-byte chunks (n16 <= kStageChunks * blockDim.x) from global
// memory into LDS, split in two so other loads can be issued in between: stage_issue
// issues a FIXED number of loads per thread (surplus threads reload the last chunk), so
// the compiler's wait counts for the loads issued before it stay exact; stage_commit
// writes the chunks to LDS once they have arrived.
typedef __attribute__((address_space(3))) void* lds_ptr;
constexpr int kStageChunks = 8;  // 64 KB with 512 threads
struct Staged {
  u32x4 v[kStageChunks];
};
__device__ inline Staged stage_issue(const void* src, int n16) {
  const u32x4* s = reinterpret_cast<const u32x4*>(src);
  Staged st;
#pragma unroll
  for (int u = 0; u < kStageChunks; ++u) st.v[u] = s[min(static_cast<int>(threadIdx.x + u * blockDim.x), n16 - 1)];
  return st;
}
__device__ inline void stage_commit(void* lds, const Staged& st, int n16) {
  u32x4* d = reinterpret_cast<u32x4*>(lds);
#pragma unroll
  for (int u = 0; u < kStageChunks; ++u) {
    const int c = threadIdx.x + u * blockDim.x;
    if (c < n16) d[c] = st.v[u];
  }
}

// Workgroup-wide direct copy of chunks [0, n16) of 16 bytes from global memory to LDS
// (global_load_lds): every thread issues exactly F copies, chunk c = wave's first chunk +
// lane + i * blockDim (sources past n16 repeat the last chunk), so the compiler's wait
// counts for loads issued before the copies stay exact.  LDS destinations run up to
// F * blockDim * 16 bytes: the caller's allocation must cover them.
template <int F>
__device__ inline void copy_to_lds_fixed(const void* src, int n16, void* lds) {
  const int lane = threadIdx.x & 63;
  const int c0 = threadIdx.x - lane;
#pragma unroll
  for (int i = 0; i < F; ++i) {
    const int cw = c0 + i * static_cast<int>(blockDim.x);  // this wave's first chunk (uniform)
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const u32x4*>(src) + min(cw + lane, n16 - 1),
                                     (lds_ptr)(static_cast<uint8_t*>(lds) + static_cast<size_t>(cw) * 16), 16, 0, 0);
  }
}

}  // namespace tl
