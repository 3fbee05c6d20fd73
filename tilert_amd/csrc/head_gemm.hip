// Per-head bf16 x fp8 GEMV: y[t, h, :] = x[t, h, :] . W_h^T for H independent weights
// W_h [N, K] (fp8 e4m3fn, 128x128 block scales), with an optional residual.  It carries
// three operators of the absorbed MLA attention at one device's share (DeepSeek-V3.2 /
// GLM-5, 16 local heads):
//  * projq_wqb (deepseek_v3_2/ops/projq_wqb.py:24-54, golden :448-450): q_lat[t,h,:] =
//    q_nope[t,h,:] . wkv_b[h, :128, :] -- the weight's ROWS are contracted, so the converter
//    stores each head's nope block transposed (N = kv_lora_rank 512, K = 128);
//  * projo_wkvb (.../projo_wkvb.py:24-54, golden :465-467): o[t,h,:] = o_lat[t,h,:] .
//    wkv_b[h, 128:, :]^T (N = v_head_dim 128, K = 512);
//  * unproj_o_allreduce (.../unproj_o_allreduce.py:23-58, golden :480-498): H = 1,
//    y = o_flat . wo_shard^T (N = dim, K = local heads * 128) + the residual x_in.
// Numerics: bf16 activations times the block-dequantised weights rounded to bf16 (the
// goldens' weights in bf16 inference), v_mfma_f32_16x16x32_bf16, fp32 accumulation, bf16
// output; with a residual, bf16(bf16(y) + x_in).
//
// Layout: W is the tile-major fragment packing of tl_moe_pack_weight applied to the
// stacked [H * N, K] matrix; scales fp32 [H][N/128][K/128].  Work item = (head, 16-row
// tile) over a persistent grid; per item the workgroup loads the head's x rows [M, K] into
// registers first, then requests its first weight fragments, and only then writes x to LDS
// (so the x round trip overlaps the weight one, and a workgroup reads 1/H of x, not all of
// it; with one head x is staged once, before the items); its waves take the K blocks
// round-robin (two in flight each) and are reduced through LDS in wave order.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "moe_common.h"
#include "../../include/tilert_amd.h"

namespace tl {

constexpr int kHgMaxWaves = 8;
constexpr int kHgXChunks = 4;  // 16-byte x chunks per thread and item (M * K * 2 <= 4 * 16 * 64 * waves)

template <bool ONCE>
__global__ __launch_bounds__(kHgMaxWaves * 64, 2) void head_gemm_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ w, const float* __restrict__ s,
    const uint16_t* __restrict__ x_in, int M, int H, int N, int K, uint16_t* __restrict__ y) {
  extern __shared__ __align__(16) uint16_t xl[];  // [M][K]: the current item's head rows
  __shared__ v4f red[kHgMaxWaves - 1][64];
  const int lane = threadIdx.x & 63;
  const int nw = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int KB = K >> 7, tiles = N >> 4, SB = (N + 127) >> 7;
  const int r = lane & 15, g = lane >> 4;
  const int row = min(r, M - 1);
  const int n = wave < KB ? (KB - wave + nw - 1) / nw : 0;  // K blocks wave + i * nw
  const int k16 = K / 8, xk16 = M * k16;                      // 16-byte chunks of a head's rows
  // ONCE (one head): x is staged once, before the items (measured faster there)
  if (ONCE) {
    for (int c = threadIdx.x; c < xk16; c += blockDim.x) reinterpret_cast<u32x4*>(xl)[c] = reinterpret_cast<const u32x4*>(x)[c];
    __syncthreads();
  }
  for (int item = blockIdx.x; item < H * tiles; item += gridDim.x) {
    const int h = item / tiles, rt = item - h * tiles;
    const uint8_t* wt = w + (static_cast<size_t>(h) * tiles + rt) * KB * 2048;
    const float* st = s + (static_cast<size_t>(h) * SB + ((rt * 16) >> 7)) * KB;
    u32x4 xs[ONCE ? 1 : kHgXChunks];  // this thread's chunks c = tid + u * blockDim of x[:, h, :]
#pragma unroll
    for (int u = 0; u < (ONCE ? 0 : kHgXChunks); ++u) {
      const int c = static_cast<int>(threadIdx.x) + u * static_cast<int>(blockDim.x);
      if (c < xk16) {
        const int t = c / k16, kc = c - t * k16;
        xs[u] = reinterpret_cast<const u32x4*>(x + (static_cast<size_t>(t) * H + h) * K)[kc];
      }
    }
    // the residual this lane adds, requested now rather than after the reduction
    const size_t off = (static_cast<size_t>(row) * H + h) * N + rt * 16 + 4 * g;
    uint2 xres = make_uint2(0u, 0u);
    if (x_in) xres = *reinterpret_cast<const uint2*>(x_in + off);
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    struct Ops {
      v8i w;
      float sc;
    };
    Ops buf[2];
    ring_pipeline(
        n, buf,
        [&](int i, Ops& o) {
          const int kb = wave + i * nw;
          o.w = load_fragment(wt + static_cast<size_t>(kb) * 2048, lane);
          o.sc = load_f32_vector(st + kb);
        },
        [&](int i, const Ops& o) {
          const int kb = wave + i * nw;
          acc = mfma_block_bf16(o.w, o.sc, lds_act(xl + row * K + kb * kBlock, g), acc);
        },
        [&] {  // behind the first weight fetches: x to LDS (the previous item's reads are done)
          if (ONCE) return;
#pragma unroll
          for (int u = 0; u < (ONCE ? 0 : kHgXChunks); ++u) {
            const int c = static_cast<int>(threadIdx.x) + u * static_cast<int>(blockDim.x);
            if (c < xk16) reinterpret_cast<u32x4*>(xl)[c] = xs[u];
          }
          __syncthreads();
        });
    if (wave > 0) {
      red[wave - 1][lane] = acc;
    }
    __syncthreads();
    if (wave == 0 && r < M) {
      for (int ww = 0; ww < nw - 1; ++ww)
        acc += red[ww][lane];
      const uint16_t xr[4] = {static_cast<uint16_t>(xres.x & 0xffffu), static_cast<uint16_t>(xres.x >> 16),
                              static_cast<uint16_t>(xres.y & 0xffffu), static_cast<uint16_t>(xres.y >> 16)};
      uint16_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        o[q] = f32_to_bf16(acc[q]);
        if (x_in) o[q] = f32_to_bf16(bf16_to_f32(o[q]) + bf16_to_f32(xr[q]));
      }
      *reinterpret_cast<uint2*>(y + off) = make_uint2(o[0] | (static_cast<uint32_t>(o[1]) << 16),
                                                      o[2] | (static_cast<uint32_t>(o[3]) << 16));
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------ bf16-weight GEMV
// y[t, n] = bf16( sum_k x[t, k] * w[n, k] ), x and w bf16 row-major (no scales), fp32
// accumulation on v_mfma_f32_16x16x32_bf16: proj_w_op, the indexer's head-weight projection
// (deepseek_v3_2/ops/projx_wis.py:18-37; its weights_proj stays bf16, rmsnorm_projx_wqakis.py:38-41).
// The weight is narrow (64 x 7168: four 16-row tiles), so K is split: workgroup (tile, s)
// of 8 waves takes K blocks 8 s .. 8 s + 7 (one per wave, all loads issued before the
// MFMAs), its waves are reduced through LDS in wave order, and with more than one slice
// the fp32 tile partials go to the workspace; the tile's last slice to arrive (an
// agent-scope counter, left zero again) adds them in slice order and writes y, so the
// result is deterministic.  At 64 x 7168, M = 4: 6.9 us (slices of 4 / 16 blocks: 8.1 /
// 7.2 us), against 12.2 us for one 16-wave workgroup per tile (four CUs streaming it all).
constexpr int kBgWaves = 8;  // K blocks per slice, one per wave

__global__ __launch_bounds__(kBgWaves * 64) void bf16_gemv_kernel(const uint16_t* __restrict__ x,
                                                                  const uint16_t* __restrict__ w, int M, int N, int K,
                                                                  uint16_t* __restrict__ y, uint32_t* __restrict__ counters,
                                                                  float* __restrict__ partial) {
  __shared__ v4f red[kBgWaves - 1][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int KB = K >> 7, S = gridDim.y, sl = blockIdx.y;
  const int rt = blockIdx.x;
  const int kb = min(sl * kBgWaves + wave, KB - 1);  // unconditional loads (clamped)
  const uint16_t* wr = w + static_cast<size_t>(16 * rt + r) * K + kb * kBlock;
  const uint16_t* xr = x + static_cast<size_t>(min(r, M - 1)) * K + kb * kBlock;
  const int off[4] = {16 * g, 16 * g + 8, 64 + 16 * g, 64 + 16 * g + 8};
  v8bf wa[4], xa[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    wa[j] = *reinterpret_cast<const v8bf*>(wr + off[j]);
    xa[j] = *reinterpret_cast<const v8bf*>(xr + off[j]);
  }
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  if (sl * kBgWaves + wave < KB) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa[j], xa[j], acc, 0, 0, 0);
  }
  if (wave > 0) red[wave - 1][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int ww = 0; ww < kBgWaves - 1; ++ww) acc += red[ww][lane];
  const int ncol = 16 * rt + 4 * g;
  auto store_y = [&](const v4f& v) {
    if (r < M)
      *reinterpret_cast<uint2*>(y + static_cast<size_t>(r) * N + ncol) =
          make_uint2(f32_to_bf16(v[0]) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16),
                     f32_to_bf16(v[2]) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16));
  };
  if (S == 1) {
    store_y(acc);
    return;
  }
  // partials as agent-scope stores (written through past this XCD's L2), complete before
  // the counter bump; the last arrival reads them with agent-scope loads
  if (r < M) {
    float* dst = partial + (static_cast<size_t>(sl) * M + r) * N + ncol;
#pragma unroll
    for (int j = 0; j < 4; ++j) __hip_atomic_store(dst + j, acc[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);
  uint32_t prev = 0;
  if (lane == 0) prev = __hip_atomic_fetch_add(&counters[rt], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  prev = __shfl(prev, 0);
  if (prev != static_cast<uint32_t>(S - 1)) return;
  v4f sum = {0.f, 0.f, 0.f, 0.f};
  if (r < M) {
    for (int q = 0; q < S; ++q) {
      const float* src = partial + (static_cast<size_t>(q) * M + r) * N + ncol;
#pragma unroll
      for (int j = 0; j < 4; ++j) sum[j] += __hip_atomic_load(src + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  store_y(sum);
  if (lane == 0) __hip_atomic_store(&counters[rt], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace tl

using namespace tl;

// Slices of the bf16 GEMV's K (1 when K <= 512: no workspace).
static int bf16_gemv_slices(int64_t K) { return static_cast<int>(cdiv(K / kBlock, kBgWaves)); }

extern "C" size_t tl_bf16_gemv_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || M > 16 || N <= 0 || N % 16 || K <= 0 || K % kBlock) return 0;
  const int S = bf16_gemv_slices(K);
  return S > 1 ? kWsCounterBytes + static_cast<size_t>(S) * M * N * sizeof(float) : 0;
}

extern "C" int tl_bf16_gemv(const void* x_bf16, const void* w_bf16, int64_t M, int64_t N, int64_t K, void* y_bf16,
                            void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "bf16_gemv";
  if (M < 1 || M > 16) { set_error("%s: M=%lld must be in [1, 16]", who, (long long)M); return kErrUnsupported; }
  if (N <= 0 || N % 16 || K <= 0 || K % kBlock || N > 16ll * kWsCounterTiles) { set_error("%s: N=%lld must be a positive multiple of 16 (at most %d) and K=%lld of 128", who, (long long)N, 16 * kWsCounterTiles, (long long)K); return kErrArg; }
  if (K > (1 << 16)) { set_error("%s: K=%lld > %d", who, (long long)K, 1 << 16); return kErrUnsupported; }
  if (!x_bf16 || !w_bf16 || !y_bf16) { set_error("%s: null pointer", who); return kErrArg; }
  if ((reinterpret_cast<uintptr_t>(x_bf16) | reinterpret_cast<uintptr_t>(w_bf16)) & 15 || reinterpret_cast<uintptr_t>(y_bf16) & 7) {
    set_error("%s: x and w must be 16-byte aligned, y 8-byte aligned", who);
    return kErrArg;
  }
  const int S = bf16_gemv_slices(K);
  const size_t need = tl_bf16_gemv_workspace_bytes(M, N, K);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 15))) {
    set_error("%s: a 16-byte aligned workspace of %zu bytes is required (got %zu)", who, need, workspace_bytes);
    return kErrArg;
  }
  uint32_t* counters = need ? static_cast<uint32_t*>(workspace) : nullptr;
  float* partial = need ? reinterpret_cast<float*>(static_cast<char*>(workspace) + kWsCounterBytes) : nullptr;
  hipLaunchKernelGGL(bf16_gemv_kernel, dim3(static_cast<unsigned>(N / 16), static_cast<unsigned>(S)), dim3(kBgWaves * 64), 0,
                     (hipStream_t)stream, (const uint16_t*)x_bf16, (const uint16_t*)w_bf16, (int)M, (int)N, (int)K,
                     (uint16_t*)y_bf16, counters, partial);
  return check_launch(who);
}

extern "C" int tl_head_gemm_bf16(const void* x_bf16, const void* w_packed, const float* w_s, const void* x_in_bf16,
                                 int64_t M, int64_t H, int64_t N, int64_t K, void* y_bf16, void* stream) {
  const char* who = "head_gemm_bf16";
  if (M < 1 || M > 16 || H < 1 || H > 1024) { set_error("%s: M=%lld must be in [1, 16], H=%lld in [1, 1024]", who, (long long)M, (long long)H); return kErrUnsupported; }
  if (N <= 0 || K <= 0 || N % 16 || K % kBlock || N > (1 << 20) || K > (1 << 16)) {
    set_error("%s: N=%lld must be a positive multiple of 16 and K=%lld of 128", who, (long long)N, (long long)K);
    return kErrArg;
  }
  const int waves = static_cast<int>(std::min<int64_t>(kHgMaxWaves, std::max<int64_t>(K / kBlock, 1)));
  const int64_t x_bytes = M * K * 2;  // one head's rows, staged per item
  if (x_bytes > static_cast<int64_t>(kHgXChunks) * 16 * 64 * waves) {
    set_error("%s: one head's x rows (M * K * 2 = %lld bytes) exceed %d", who, (long long)x_bytes, kHgXChunks * 16 * 64 * waves);
    return kErrUnsupported;
  }
  if (!x_bf16 || !w_packed || !w_s || !y_bf16) { set_error("%s: null pointer", who); return kErrArg; }
  if ((reinterpret_cast<uintptr_t>(x_bf16) | reinterpret_cast<uintptr_t>(w_packed)) & 15 ||
      (reinterpret_cast<uintptr_t>(y_bf16) | reinterpret_cast<uintptr_t>(x_in_bf16)) & 7) {
    set_error("%s: x and weights must be 16-byte aligned, y and x_in 8-byte aligned", who);
    return kErrArg;
  }
  const int64_t items = H * (N / 16);
  const int grid = static_cast<int>(std::min<int64_t>(items, 512));
  auto launch = [&](auto once_tag) -> int {
    constexpr bool ONCE = decltype(once_tag)::value;
    if (int rc = allow_dynamic_lds(reinterpret_cast<const void*>(head_gemm_kernel<ONCE>), kHgXChunks * 16 * 64 * kHgMaxWaves, who))
      return rc;
    hipLaunchKernelGGL(head_gemm_kernel<ONCE>, dim3(grid), dim3(waves * 64), static_cast<size_t>(x_bytes),
                       (hipStream_t)stream, (const uint16_t*)x_bf16, (const uint8_t*)w_packed, w_s,
                       (const uint16_t*)x_in_bf16, (int)M, (int)H, (int)N, (int)K, (uint16_t*)y_bf16);
    return 0;
  };
  if (int rc = H == 1 ? launch(std::true_type{}) : launch(std::false_type{})) return rc;
  return check_launch(who);
}
