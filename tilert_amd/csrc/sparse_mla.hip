// Sparse MLA decode attention over the indexer's top-k selection: the contract of
// flash_sparse_mla_op (ops/flash_sparse_mla.py:18-93; golden FlashSparseMLACombine.
// golden_forward :152-196).  For token s and head h,
//   score[t] = (q_nope[s,h] . kv[t] + q_pe[s,h] . pe[t]) * softmax_scale   over the selected t
//   out[s,h] = softmax(score) . kv[selected]        (bf16 probabilities, fp32 accumulation)
// with positions outside the selection masked, and for s > 1 also positions past
// cur_pos + s (the golden's triu mask).
//
// Split-K decoding in two launches, the split the reference op exposes (split_size 64, at
// most 32 splits, lse_acc / output_acc per split):
//   split kernel   one 256-thread workgroup per (split j, token s).  The split's 64 selected
//                  kv rows (1 KB) and pe rows (128 B) are gathered into LDS together with
//                  the token's queries; wave w scores key tile w (16 keys) for every head
//                  tile on v_mfma_f32_16x16x32_bf16 (18 K steps over 512 + 64), the
//                  split's softmax statistics are reduced across lanes and waves, the
//                  probabilities exp(score - max) go to LDS as bf16, and the waves multiply
//                  them with the split's kv rows (each wave 8 of the 32 16-wide value
//                  tiles).  Stores output_acc[s,h,j] = O_j / l_j and lse_acc[s,h,j] =
//                  max_j + ln l_j (-inf for a split with no visible position).
//   combine kernel one workgroup per (head, token, 128 dims): lse = ln sum_j e^lse_j, out = sum_j
//                  e^(lse_j - lse) output_acc_j, rounded to bf16.
// Reading the gathered rows once from LDS serves both products, so every selected row is
// read from memory once.
#include <math.h>

#include "common.h"
#include "../../include/tilert_amd.h"

namespace tl {

typedef __bf16 v8bf_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4s __attribute__((ext_vector_type(4)));

constexpr int kMlaDim = 512;       // kv_lora_rank
constexpr int kMlaPe = 64;         // qk_rope_head_dim
constexpr int kMlaSplit = 64;      // selected positions per split (split_size)
constexpr int kMlaMaxSplits = 32;  // at most 2048 selected positions
constexpr int kMlaKvStride = kMlaDim * 2 + 16;  // padded LDS row: rows 4 banks apart
constexpr int kMlaThreads = 256;

// LDS layout of the split kernel, for HT 16-row head tiles
template <int HT>
struct MlaLds {
  static constexpr int KV_OFF = 0;
  static constexpr int PE_OFF = KV_OFF + kMlaSplit * kMlaKvStride;
  static constexpr int Q_OFF = PE_OFF + kMlaSplit * kMlaPe * 2;          // [HT*16][576] bf16
  static constexpr int P_OFF = Q_OFF + HT * 16 * (kMlaDim + kMlaPe) * 2;  // [HT*16][64] bf16
  static constexpr int RED_OFF = P_OFF + HT * 16 * kMlaSplit * 2;         // [4 waves][HT*16] f32 maxima
  static constexpr int SUM_OFF = RED_OFF + 4 * HT * 16 * 4;               // [4 waves][HT*16] f32 sums
  static constexpr int IDX_OFF = SUM_OFF + 4 * HT * 16 * 4;               // [64] i32
  static constexpr int BYTES = IDX_OFF + kMlaSplit * 4;
};

__device__ inline v8bf_t lds_v8bf(const uint8_t* p) { return *reinterpret_cast<const v8bf_t*>(p); }

template <int HT>
__global__ __launch_bounds__(kMlaThreads) void sparse_mla_split_kernel(
    const uint16_t* __restrict__ q_nope, const uint16_t* __restrict__ q_pe, const uint16_t* __restrict__ kv,
    const uint16_t* __restrict__ pe, const int32_t* __restrict__ indices, const int32_t* __restrict__ cur_pos,
    int seqlen, int heads, int topk, int64_t T, float scale, float* __restrict__ out_acc, float* __restrict__ lse_acc) {
  using S = MlaLds<HT>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int split = blockIdx.x, s = blockIdx.y;
  const int n_splits = gridDim.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  int32_t* idx_l = reinterpret_cast<int32_t*>(smem + S::IDX_OFF);

  // the split's positions and the token's queries, loaded together: a masked position
  // (past topk, outside [0, T), or after the token's position when seqlen > 1) is stored
  // as -1; query rows h < heads, 576 bf16 each (rows past them zero), as 16-byte chunks
  constexpr int QCH = HT * 16 * 72;  // 64 chunks of q_nope + 8 of q_pe per head
  constexpr int QPT = (QCH + kMlaThreads - 1) / kMlaThreads;
  // every wave loads all 64 positions (lane l: row l) and hands them out by readlane / lane
  // shuffle, so the gather needs no barrier
  int t_idx = -1;
  {
    const int j = split * kMlaSplit + lane;
    t_idx = indices[static_cast<int64_t>(s) * topk + min(j, topk - 1)];
    if (j >= topk || t_idx < 0 || t_idx >= T || (seqlen > 1 && t_idx > *cur_pos + s)) t_idx = -1;
  }
  u32x4s qv[QPT];
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    const int c = min(tid + u * kMlaThreads, QCH - 1);
    const int h = min(c / 72, heads - 1), k = c % 72;
    qv[u] = k < 64 ? reinterpret_cast<const u32x4s*>(q_nope + (static_cast<int64_t>(s) * heads + h) * kMlaDim)[k]
                   : reinterpret_cast<const u32x4s*>(q_pe + (static_cast<int64_t>(s) * heads + h) * kMlaPe)[k - 64];
  }
  if (tid < kMlaSplit) idx_l[tid] = t_idx;  // read after the gather's barrier
  // gather: kv row of position idx_l[row] into LDS row `row` (64 chunks of 16 B), pe row
  // (8 chunks); a masked row is loaded from row 0 (unconditional loads) and stored as
  // zeros, so whatever row 0 holds cannot reach the products
  {
    // kv: chunk tid + 256 u is row wave + 4 u (wave-uniform), chunk lane; pe: row
    // (tid >> 3) + 32 u, chunk tid & 7
    u32x4s v[16], w[2];
    int tv[16], tw[2];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      tv[u] = __builtin_amdgcn_readlane(t_idx, wave + 4 * u);
      v[u] = reinterpret_cast<const u32x4s*>(kv + static_cast<int64_t>(max(tv[u], 0)) * kMlaDim)[lane];
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      tw[u] = __shfl(t_idx, ((tid >> 3) + 32 * u) & 63);
      w[u] = reinterpret_cast<const u32x4s*>(pe + static_cast<int64_t>(max(tw[u], 0)) * kMlaPe)[tid & 7];
    }
    const u32x4s zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
      const int c = tid + u * kMlaThreads;
      if (c < QCH) {
        const int h = c / 72, k = c % 72;
        *reinterpret_cast<u32x4s*>(smem + S::Q_OFF + h * (kMlaDim + kMlaPe) * 2 + k * 16) = h < heads ? qv[u] : zero;
      }
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int row = wave + 4 * u;
      *reinterpret_cast<u32x4s*>(smem + S::KV_OFF + row * kMlaKvStride + lane * 16) = tv[u] >= 0 ? v[u] : zero;
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int row = (tid >> 3) + 32 * u;
      *reinterpret_cast<u32x4s*>(smem + S::PE_OFF + row * kMlaPe * 2 + (tid & 7) * 16) = tw[u] >= 0 ? w[u] : zero;
    }
  }
  __syncthreads();

  // ---- scores: wave w, key tile w (keys 16w .. 16w+15), every head tile
  const int key = wave * 16 + r;  // the B-operand row (key) of this lane
  v4f sc[HT];
#pragma unroll
  for (int ht = 0; ht < HT; ++ht) sc[ht] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < 18; ++ks) {
    const v8bf_t b = ks < 16 ? lds_v8bf(smem + S::KV_OFF + key * kMlaKvStride + (ks * 32 + g * 8) * 2)
                             : lds_v8bf(smem + S::PE_OFF + key * kMlaPe * 2 + ((ks - 16) * 32 + g * 8) * 2);
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
      const v8bf_t a = lds_v8bf(smem + S::Q_OFF + (ht * 16 + r) * (kMlaDim + kMlaPe) * 2 + (ks * 32 + g * 8) * 2);
      sc[ht] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, sc[ht], 0, 0, 0);
    }
  }
  // lane holds score[head 16 ht + 4 g + i][key 16 wave + r]
  const bool live = idx_l[wave * 16 + r] >= 0;
  float* red = reinterpret_cast<float*>(smem + S::RED_OFF);  // [wave][head]
  float mx[HT][4];
#pragma unroll
  for (int ht = 0; ht < HT; ++ht)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = live ? sc[ht][i] * scale : -INFINITY;
      sc[ht][i] = v;
      mx[ht][i] = row16_reduce<true>(v);
    }
  if (r == 0) {
#pragma unroll
    for (int ht = 0; ht < HT; ++ht)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave * HT * 16 + ht * 16 + 4 * g + i] = mx[ht][i];
  }
  __syncthreads();
  float m[HT][4];
#pragma unroll
  for (int ht = 0; ht < HT; ++ht)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = ht * 16 + 4 * g + i;
      m[ht][i] = fmaxf(fmaxf(red[h], red[HT * 16 + h]), fmaxf(red[2 * HT * 16 + h], red[3 * HT * 16 + h]));
    }
  red = reinterpret_cast<float*>(smem + S::SUM_OFF);  // the sums go to their own slots: no barrier here
  // probabilities relative to the split's max (0 where masked, and for a split with no
  // visible position), stored as bf16 P[head][key]; their fp32 sums per head
  uint16_t* P = reinterpret_cast<uint16_t*>(smem + S::P_OFF);
  float sm[HT][4];
#pragma unroll
  for (int ht = 0; ht < HT; ++ht)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = (m[ht][i] == -INFINITY || sc[ht][i] == -INFINITY) ? 0.f : expf(sc[ht][i] - m[ht][i]);
      P[(ht * 16 + 4 * g + i) * kMlaSplit + wave * 16 + r] = f32_to_bf16(p);
      sm[ht][i] = row16_reduce<false>(p);
    }
  if (r == 0) {
#pragma unroll
    for (int ht = 0; ht < HT; ++ht)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave * HT * 16 + ht * 16 + 4 * g + i] = sm[ht][i];
  }
  __syncthreads();
  float l[HT][4];
#pragma unroll
  for (int ht = 0; ht < HT; ++ht)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = ht * 16 + 4 * g + i;
      l[ht][i] = (red[h] + red[HT * 16 + h]) + (red[2 * HT * 16 + h] + red[3 * HT * 16 + h]);
    }

  // ---- O = P . V: wave w takes value tiles 8w .. 8w+7 (16 dims each), 2 K steps of 32 keys
  v4f o[HT][8];
#pragma unroll
  for (int ht = 0; ht < HT; ++ht)
#pragma unroll
    for (int d = 0; d < 8; ++d) o[ht][d] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    v8bf_t a[HT];
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) a[ht] = lds_v8bf(smem + S::P_OFF + ((ht * 16 + r) * kMlaSplit + ks * 32 + g * 8) * 2);
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      // The operand lane (column r, key group g) needs keys ks*32 + 8g .. +7 of value column
      // 16 (8 wave + d) + r: a column of the key-major rows.  ds_read_b64_tr_b16 transposes
      // within each 16-lane group: result element j of lane i is element i % 4 of the 4
      // contiguous values addressed by lane 4 j + i / 4 of the group.  So lane r of group g
      // addresses row (key) ks*32 + 8g + r / 4 (+ 4 for the upper half), values
      // 16 (8 wave + d) + 4 (r % 4) .. +3, and receives its column's 4 (8) keys.
      const uint8_t* src = smem + S::KV_OFF + (ks * 32 + g * 8 + (r >> 2)) * kMlaKvStride +
                           ((wave * 8 + d) * 16 + 4 * (r & 3)) * 2;
      typedef short v4s_t __attribute__((ext_vector_type(4)));
      const v4s_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s_t*)(src));
      const v4s_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) v4s_t*)(src + 4 * kMlaKvStride));
      const v8bf_t b = __builtin_bit_cast(v8bf_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) o[ht][d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[ht], b, o[ht][d], 0, 0, 0);
    }
  }
  // lane holds O[head 16 ht + 4 g + i][dim 16 (8 wave + d) + r]
#pragma unroll
  for (int ht = 0; ht < HT; ++ht)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = ht * 16 + 4 * g + i;
      if (h >= heads) continue;
      const float inv = l[ht][i] > 0.f ? 1.0f / l[ht][i] : 0.f;
      float* dst = out_acc + ((static_cast<int64_t>(s) * heads + h) * kMlaMaxSplits + split) * kMlaDim;
#pragma unroll
      for (int d = 0; d < 8; ++d) dst[(wave * 8 + d) * 16 + r] = o[ht][d][i] * inv;
      if (wave == 0 && r == 0)
        lse_acc[(static_cast<int64_t>(s) * heads + h) * kMlaMaxSplits + split] =
            l[ht][i] > 0.f ? m[ht][i] + logf(l[ht][i]) : -INFINITY;
    }
  (void)n_splits;
}

// One 64-thread workgroup per (head, token, quarter of the 512 dims).  Lane l takes dims
// 4 (l % 32) .. +3 of the quarter and the splits of parity l / 32 (16-byte loads, 16 per
// lane, unconditional and clamped; splits past n_splits weigh 0); the two half-waves' sums
// meet through a lane shuffle and each half stores two of the four dims.  The split lse is
// requested first (memory operations complete in order, so the weights are computed while
// the split rows arrive); the weights are computed lane-parallel (lane j: split j's lse,
// its exponentials; max and sum by DPP) and read back per split with readlane.
__global__ __launch_bounds__(64) void sparse_mla_combine_kernel(const float* __restrict__ out_acc,
                                                                const float* __restrict__ lse_acc, int heads,
                                                                int n_splits, uint16_t* __restrict__ out,
                                                                float* __restrict__ lse) {
  const int h = blockIdx.x, s = blockIdx.y, quarter = blockIdx.z, tid = threadIdx.x;
  const int64_t row = static_cast<int64_t>(s) * heads + h;
  const int d0 = quarter * 128 + 4 * (tid & 31), par = tid >> 5;
  constexpr int kHalf = kMlaMaxSplits / 2;
  const float lj = tid < n_splits ? lse_acc[row * kMlaMaxSplits + min(tid, kMlaMaxSplits - 1)] : -INFINITY;
  __builtin_amdgcn_sched_barrier(0);
  v4f v[kHalf];
#pragma unroll
  for (int i = 0; i < kHalf; ++i)
    v[i] = *reinterpret_cast<const v4f*>(out_acc + (row * kMlaMaxSplits + min(2 * i + par, n_splits - 1)) * kMlaDim + d0);
  __builtin_amdgcn_sched_barrier(0);
  const float mx = wave_max_f32(lj);
  const float sum = wave_sum_f32(lj == -INFINITY ? 0.f : expf(lj - mx));
  const float L = mx == -INFINITY ? -INFINITY : mx + logf(sum);
  const int wl = __builtin_bit_cast(int, lj == -INFINITY ? 0.f : expf(lj - L));  // lane j: split j's weight
  v4f a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kHalf; ++i) {
    const float we = __builtin_bit_cast(float, __builtin_amdgcn_readlane(wl, 2 * i));
    const float wo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(wl, 2 * i + 1));
    a += v[i] * (par ? wo : we);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) a[k] += __shfl_xor(a[k], 32);  // even + odd splits (the same sum in both halves)
  const float lo = par ? a[2] : a[0], hi = par ? a[3] : a[1];
  reinterpret_cast<uint32_t*>(out + row * kMlaDim + d0)[par] =
      f32_to_bf16(lo) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
  if (quarter == 0 && tid == 0) lse[row] = L;
}

}  // namespace tl

using namespace tl;

extern "C" int tl_flash_sparse_mla(const void* q_nope_bf16, const void* q_pe_bf16, const void* kv_bf16,
                                   const void* pe_bf16, const int32_t* indices, const int32_t* cur_pos,
                                   int64_t seqlen, int64_t heads, int64_t topk, int64_t kv_rows,
                                   float softmax_scale, void* out_bf16, float* out_acc, float* lse,
                                   float* lse_acc, void* stream) {
  if (seqlen < 1 || seqlen > 16) { set_error("flash_sparse_mla: seqlen=%lld must be in [1, 16]", (long long)seqlen); return kErrUnsupported; }
  if (heads < 1 || heads > 32) { set_error("flash_sparse_mla: heads=%lld must be in [1, 32]", (long long)heads); return kErrUnsupported; }
  if (topk < 1 || topk > kMlaSplit * kMlaMaxSplits) { set_error("flash_sparse_mla: topk=%lld must be in [1, %d]", (long long)topk, kMlaSplit * kMlaMaxSplits); return kErrUnsupported; }
  if (kv_rows < 1 || kv_rows > (1ll << 31) - 1) { set_error("flash_sparse_mla: kv_rows=%lld out of range", (long long)kv_rows); return kErrArg; }
  if (!q_nope_bf16 || !q_pe_bf16 || !kv_bf16 || !pe_bf16 || !indices || !cur_pos || !out_bf16 || !out_acc || !lse || !lse_acc) {
    set_error("flash_sparse_mla: null pointer");
    return kErrArg;
  }
  if ((reinterpret_cast<uintptr_t>(q_nope_bf16) | reinterpret_cast<uintptr_t>(q_pe_bf16) | reinterpret_cast<uintptr_t>(kv_bf16) |
       reinterpret_cast<uintptr_t>(pe_bf16) | reinterpret_cast<uintptr_t>(out_acc)) & 15) {
    set_error("flash_sparse_mla: q, kv, pe and output_acc must be 16-byte aligned");
    return kErrArg;
  }
  hipStream_t st = (hipStream_t)stream;
  const int n_splits = static_cast<int>(cdiv(topk, kMlaSplit));
  const dim3 grid(static_cast<unsigned>(n_splits), static_cast<unsigned>(seqlen));
  auto launch = [&](auto ht_tag) -> int {
    constexpr int HT = decltype(ht_tag)::value;
    const void* fn = reinterpret_cast<const void*>(sparse_mla_split_kernel<HT>);
    if (int rc = allow_dynamic_lds(fn, MlaLds<HT>::BYTES, "flash_sparse_mla")) return rc;
    hipLaunchKernelGGL((sparse_mla_split_kernel<HT>), grid, dim3(kMlaThreads), MlaLds<HT>::BYTES, st,
                       (const uint16_t*)q_nope_bf16, (const uint16_t*)q_pe_bf16, (const uint16_t*)kv_bf16,
                       (const uint16_t*)pe_bf16, indices, cur_pos, (int)seqlen, (int)heads, (int)topk, kv_rows,
                       softmax_scale, out_acc, lse_acc);
    return check_launch("flash_sparse_mla");
  };
  if (int rc = heads <= 16 ? launch(std::integral_constant<int, 1>{}) : launch(std::integral_constant<int, 2>{})) return rc;
  hipLaunchKernelGGL(sparse_mla_combine_kernel, dim3(static_cast<unsigned>(heads), static_cast<unsigned>(seqlen), 4), dim3(64),
                     0, st, out_acc, lse_acc, (int)heads, n_splits, (uint16_t*)out_bf16, lse);
  return check_launch("flash_sparse_mla");
}
