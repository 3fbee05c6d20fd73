// DSA lightning-indexer scores over an fp8 key cache:
//   logits[t, l] = k_s[l] * sum_h (w[t,h] * q_s[t(,h)]) * ReLU(q8[t,h] . k8[l])
// which equals sum_h w[t,h] * ReLU(qd[t,h] . kd[l]) on the dequantised inputs because
// every scale is positive (the form of sparse_index_op, ops/sparse_index.py:11-69, on the
// fp8 cache layout of pd_vllm/profiles/mla_nsa.py:211-228).
//
// gfx950 mapping: the M*H query rows form M*H/16 tiles of 16 rows x 128 dims, staged
// once per workgroup through LDS and held in registers for the whole kernel (A operand);
// each wave streams its own range of 16-key tiles (B operand, 2 KB contiguous each, one
// tile prefetched ahead) through the native fp8 MFMA v_mfma_f32_16x16x128_f8f6f4 -- one
// MFMA is a whole 128-long dot product for 16 heads x 16 keys.  Epilogue per MFMA: ReLU
// and the head weight (2 VALU ops per element, weights read from LDS); the head sum over
// a lane's 4 heads and a token's tiles stays in registers, and the 4 lane groups are
// combined with v_permlane32_swap / v_permlane16_swap.
#include "common.h"
#include "../../include/tilert_amd.h"

namespace tl {

constexpr int kIdxWaves = 8;

template <int M, int H>
__global__ __launch_bounds__(kIdxWaves * 64) void indexer_kernel(
    const uint8_t* __restrict__ q, const float* __restrict__ q_s, int q_s_per_head,
    const uint8_t* __restrict__ k, const float* __restrict__ k_s, const uint16_t* __restrict__ w,
    float* __restrict__ logits, int L, int64_t ld, int64_t cur_pos, int n_tiles, int tiles_per_wave) {
  constexpr int TPT = H / 16;   // query tiles per token
  constexpr int QT = M * TPT;   // query tiles
  const int lane = threadIdx.x & 63;
  const int wave_global = blockIdx.x * kIdxWaves + (threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int t_begin = wave_global * tiles_per_wave;

  auto load_keys = [&](int tile) -> v8i {
    const int key = tile * 16 + r;
    return key < L ? load_kblock_stream(k + static_cast<size_t>(key) * kBlock, g) : zero_v8i();
  };
  // the first key tile is in flight while the workgroup stages the queries
  v8i kb_next = t_begin < n_tiles ? load_keys(t_begin) : zero_v8i();

  // stage the queries and the folded head weights w[t,h] * q_s once per workgroup
  __shared__ __attribute__((aligned(16))) uint8_t q_lds[QT * 16 * kBlock];
  __shared__ __attribute__((aligned(16))) float wq_lds[QT * 16];
  for (int i = threadIdx.x; i < QT * 16 * kBlock / 16; i += kIdxWaves * 64)
    reinterpret_cast<uint4*>(q_lds)[i] = reinterpret_cast<const uint4*>(q)[i];
  for (int row = threadIdx.x; row < QT * 16; row += kIdxWaves * 64)
    wq_lds[row] = bf16_to_f32(w[row]) * (q_s_per_head ? q_s[row] : q_s[row / H]);
  __syncthreads();
  if (t_begin >= n_tiles) return;
  const int t_end = min(n_tiles, t_begin + tiles_per_wave);

  v8i qa[QT];  // query tiles (A operands), resident for the whole kernel
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) qa[qt] = load_kblock(q_lds + (qt * 16 + r) * kBlock, g);

  for (int tile = t_begin; tile < t_end; ++tile) {
    const v8i kbv = kb_next;
    if (tile + 1 < t_end) kb_next = load_keys(tile + 1);
    const int key = tile * 16 + r;
    const float ks = key < L ? k_s[key] : 0.f;
    float part[M];
#pragma unroll
    for (int t = 0; t < M; ++t) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < TPT; ++i) {
        const int qt = t * TPT + i;
        const v4f c = mfma_16x16x128_fp8(qa[qt], kbv);
        const float4 wq = *reinterpret_cast<const float4*>(wq_lds + qt * 16 + 4 * g);
        acc = __builtin_fmaf(fmaxf(c[0], 0.f), wq.x, acc);
        acc = __builtin_fmaf(fmaxf(c[1], 0.f), wq.y, acc);
        acc = __builtin_fmaf(fmaxf(c[2], 0.f), wq.z, acc);
        acc = __builtin_fmaf(fmaxf(c[3], 0.f), wq.w, acc);
      }
      part[t] = acc;
    }
    // lanes r, r+16, r+32, r+48 hold the 4 partial head sums of key r: sum them with
    // the gfx950 lane-swap instructions (VALU, no LDS round trip)
    float score[M];
#pragma unroll
    for (int t = 0; t < M; ++t) {
      const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(part[t]), __float_as_uint(part[t]), false, false);
      const float y = __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
      const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
      score[t] = (__uint_as_float(s16[0]) + __uint_as_float(s16[1])) * ks;
    }
    // lane group g stores tokens g, g+4, ...: a 64-byte row segment per token
#pragma unroll
    for (int t0 = 0; t0 < M; t0 += 4) {
      const int t = t0 + g;
      if (t < M && key < L) {
        float v = score[0];
#pragma unroll
        for (int tt = 1; tt < M; ++tt)
          if (tt == t) v = score[tt];
        if (static_cast<int64_t>(key) > cur_pos + t) v = -__builtin_inff();
        logits[static_cast<int64_t>(t) * ld + key] = v;
      }
    }
  }
}

// Columns no token can see (key > cur_pos + M - 1) are -inf for every row.
__global__ void fill_masked_kernel(float* __restrict__ logits, int M, int64_t ld, int64_t begin, int64_t end) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t n = end - begin;
  if (i >= n * M) return;
  const int64_t t = i / n, c = begin + (i - t * n);
  logits[t * ld + c] = -__builtin_inff();
}

template <int M, int H>
static void launch_indexer(dim3 grid, hipStream_t st, const uint8_t* q, const float* q_s, int per_head,
                           const uint8_t* k, const float* k_s, const uint16_t* w, float* logits,
                           int L, int64_t ld, int64_t cur_pos, int n_tiles, int tpw) {
  hipLaunchKernelGGL((indexer_kernel<M, H>), grid, dim3(kIdxWaves * 64), 0, st, q, q_s, per_head, k, k_s, w,
                     logits, L, ld, cur_pos, n_tiles, tpw);
}

}  // namespace tl

using namespace tl;

extern "C" int tl_indexer_fp8_scores(const void* q_fp8, const float* q_s, int q_s_per_head,
                                     const void* k_fp8, const float* k_s, const void* w_bf16,
                                     float* logits, int64_t M, int64_t H, int64_t L, int64_t ld,
                                     int64_t cur_pos, void* stream) {
  if (H != 32 && H != 64) { set_error("indexer: H=%lld must be 32 or 64", (long long)H); return kErrUnsupported; }
  if (M < 1 || M * H > 256) { set_error("indexer: need 1 <= M and M*H <= 256 (M=%lld H=%lld)", (long long)M, (long long)H); return kErrUnsupported; }
  if (L < 0 || L > (1ll << 30) || ld < L) { set_error("indexer: bad L=%lld / ld=%lld", (long long)L, (long long)ld); return kErrArg; }
  if (cur_pos < 0) { set_error("indexer: cur_pos=%lld must be >= 0", (long long)cur_pos); return kErrArg; }
  if (!q_fp8 || !q_s || !k_fp8 || !k_s || !w_bf16 || !logits) { set_error("indexer: null pointer"); return kErrArg; }
  if ((reinterpret_cast<uintptr_t>(q_fp8) | reinterpret_cast<uintptr_t>(k_fp8)) & 15) { set_error("indexer: q and k must be 16-byte aligned"); return kErrArg; }
  if (L == 0) return kOk;
  hipStream_t st = (hipStream_t)stream;
  // keys past the last token's position are masked for every token: no need to read them
  const int64_t visible = cur_pos + M < L ? cur_pos + M : L;
  const int n_tiles = static_cast<int>(cdiv(visible, 16));
  if (visible < L) {
    const int64_t n = (L - visible) * M;
    hipLaunchKernelGGL(fill_masked_kernel, dim3(cdiv(n, 256)), dim3(256), 0, st, logits, (int)M, ld, visible, L);
  }
  // 4 key tiles (64 keys, 8 KB) per wave at 128K keys: 2048 waves = 2 per SIMD, one
  // 8-wave workgroup per CU (the kernel uses ~244 VGPRs at M*H = 256)
  const int tpw = static_cast<int>(cdiv(n_tiles, 2048) < 2 ? 2 : cdiv(n_tiles, 2048));
  const int waves = static_cast<int>(cdiv(n_tiles, tpw));
  const dim3 grid(static_cast<unsigned>(cdiv(waves, kIdxWaves)));
  const uint8_t* q = (const uint8_t*)q_fp8;
  const uint8_t* k = (const uint8_t*)k_fp8;
  const uint16_t* w = (const uint16_t*)w_bf16;
  const int Li = static_cast<int>(L);
#define TL_IDX(MM, HH) \
  if (M == MM && H == HH) { launch_indexer<MM, HH>(grid, st, q, q_s, q_s_per_head, k, k_s, w, logits, Li, ld, cur_pos, n_tiles, tpw); return check_launch("indexer"); }
  TL_IDX(1, 64) TL_IDX(2, 64) TL_IDX(3, 64) TL_IDX(4, 64)
  TL_IDX(1, 32) TL_IDX(2, 32) TL_IDX(3, 32) TL_IDX(4, 32) TL_IDX(5, 32) TL_IDX(6, 32) TL_IDX(7, 32) TL_IDX(8, 32)
#undef TL_IDX
  set_error("indexer: unsupported M=%lld H=%lld", (long long)M, (long long)H);
  return kErrUnsupported;
}
