// Block-scaled FP8 GEMM for decode shapes: C[M,N] (bf16) = A[M,K] . B[N,K]^T with
// A e4m3fn + fp32 scales per (row, 128 cols) and B e4m3fn + fp32 scales per 128x128
// block -- the contract of fp8_gemm (refs/kernel.py:282-306, kernel :202-249).
//
// Design (gfx950):
//   * The weight B is the only large operand (132 MB at 18432x7168); every byte of it
//     is read exactly once, with 16-byte non-temporal loads, so the kernel is an HBM
//     stream.  The tiny activation A (<= 256 rows) stays L1/L2 resident.
//   * Math runs on the native OCP-fp8 MFMA v_mfma_f32_16x16x128_f8f6f4: one MFMA covers
//     16 weight rows x 16 tokens x one whole 128-wide K block, i.e. exactly one scale
//     block, so the per-block scale product (b_s * a_s) is applied once per MFMA to the
//     fp32 partial -- the same per-K-block scaling as the reference kernel
//     (refs/kernel.py:238-244).  For M <= 16 the unused token columns are free: the
//     kernel is bandwidth-bound by >20x margin on the matrix cores.
//   * Work split: a 256-thread workgroup (4 wave64s) owns 16 output rows and a slice of
//     K blocks; the 4 waves interleave over the slice and are summed through LDS in a
//     fixed order.  Narrow layers (few 16-row tiles) add a split over K across
//     workgroups; the last workgroup to finish a row tile (agent-scope counter) sums the
//     fp32 partials in split order, so results are deterministic.
#include "common.h"
#include "../../include/tilert_amd.h"

namespace tl {

constexpr int kWaves = 4;

template <int MT, int U>
__global__ __launch_bounds__(256) void fp8_gemm_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ B,
    const float* __restrict__ Bs, uint16_t* __restrict__ C, float* __restrict__ partial,
    uint32_t* __restrict__ counters, int M, int N, int K, int kb_per_split) {
  __shared__ float red[kWaves - 1][MT][4][64];
  const int KB = K >> 7;
  const int ksplit = gridDim.y;
  const int ks = blockIdx.y;
  const int kb_begin = ks * kb_per_split;
  const int kb_end = min(KB, kb_begin + kb_per_split);
  const int n0 = blockIdx.x * 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;

  const uint8_t* brow = B + static_cast<size_t>(n0 + r) * K;
  const float* bs_row = Bs + static_cast<size_t>(n0 >> 7) * KB;

  v4f acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int kb0 = kb_begin + wave; kb0 < kb_end; kb0 += kWaves * U) {
    v8i a[U];
    v8i x0[U];
    float xs0[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kb = kb0 + kWaves * u;
      a[u] = kb < kb_end ? load_kblock_stream(brow + static_cast<size_t>(kb) * kBlock, g) : zero_v8i();
      const bool tok = (kb < kb_end) && (r < M);
      x0[u] = tok ? load_kblock(A + static_cast<size_t>(r) * K + kb * kBlock, g) : zero_v8i();
      xs0[u] = tok ? As[static_cast<size_t>(r) * KB + kb] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kb = kb0 + kWaves * u;
      if (kb < kb_end) {
        const float bsc = bs_row[kb];
        {
          const v4f c = mfma_16x16x128_fp8(a[u], x0[u]);
          const float sc = bsc * xs0[u];
          acc[0] += c * sc;
        }
#pragma unroll
        for (int mt = 1; mt < MT; ++mt) {
          const int t = mt * 16 + r;
          const bool tok = t < M;
          const v8i x = tok ? load_kblock(A + static_cast<size_t>(t) * K + kb * kBlock, g) : zero_v8i();
          const float xs = tok ? As[static_cast<size_t>(t) * KB + kb] : 0.f;
          const v4f c = mfma_16x16x128_fp8(a[u], x);
          acc[mt] += c * (bsc * xs);
        }
      }
    }
  }

  // ---- cross-wave reduction (fixed order w0 + w1 + w2 + w3)
  if (wave > 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) red[wave - 1][mt][j][lane] = acc[mt][j];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[mt][j] = ((acc[mt][j] + red[0][mt][j][lane]) + red[1][mt][j][lane]) + red[2][mt][j][lane];

  // lane holds rows n0 + 4g + j (j = 0..3) of token mt*16 + r
  const int ncol = n0 + 4 * g;
  if (ksplit == 1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int t = mt * 16 + r;
      if (t < M) {
        const uint32_t lo = f32_to_bf16(acc[mt][0]) | (static_cast<uint32_t>(f32_to_bf16(acc[mt][1])) << 16);
        const uint32_t hi = f32_to_bf16(acc[mt][2]) | (static_cast<uint32_t>(f32_to_bf16(acc[mt][3])) << 16);
        *reinterpret_cast<uint2*>(C + static_cast<size_t>(t) * N + ncol) = make_uint2(lo, hi);
      }
    }
    return;
  }

  // ---- split-K: publish fp32 partials, the last arriving slice reduces in order
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int t = mt * 16 + r;
    if (t < M)
      *reinterpret_cast<v4f*>(partial + (static_cast<size_t>(ks) * M + t) * N + ncol) = acc[mt];
  }
  __threadfence();
  uint32_t prev = 0;
  if (lane == 0) prev = atomicAdd(&counters[blockIdx.x], 1u);
  prev = __shfl(prev, 0);
  if (prev != static_cast<uint32_t>(ksplit - 1)) return;
  __threadfence();
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int t = mt * 16 + r;
    if (t < M) {
      v4f s = {0.f, 0.f, 0.f, 0.f};
      for (int q = 0; q < ksplit; ++q)
        s += __builtin_nontemporal_load(
            reinterpret_cast<const v4f*>(partial + (static_cast<size_t>(q) * M + t) * N + ncol));
      const uint32_t lo = f32_to_bf16(s[0]) | (static_cast<uint32_t>(f32_to_bf16(s[1])) << 16);
      const uint32_t hi = f32_to_bf16(s[2]) | (static_cast<uint32_t>(f32_to_bf16(s[3])) << 16);
      *reinterpret_cast<uint2*>(C + static_cast<size_t>(t) * N + ncol) = make_uint2(lo, hi);
    }
  }
  if (lane == 0) atomicExch(&counters[blockIdx.x], 0u);  // ready for the next call
}

struct GemmPlan {
  int ksplit;
  int kb_per_split;
  int row_tiles;
};

// Pick the K split: keep >= ~768 workgroups (3 per CU) in flight and give every wave
// of a slice at least one K block.
static GemmPlan plan_gemm(int64_t M, int64_t N, int64_t K) {
  GemmPlan p;
  const int KB = static_cast<int>(K / kBlock);
  p.row_tiles = static_cast<int>(N / 16);
  int want = 1;
  if (p.row_tiles < 768) want = static_cast<int>(cdiv(768, p.row_tiles));
  int per = static_cast<int>(cdiv(KB, want));
  per = static_cast<int>(cdiv(per, kWaves) * kWaves);  // whole waves per slice
  if (per > KB) per = KB;
  p.kb_per_split = per;
  p.ksplit = static_cast<int>(cdiv(KB, per));
  (void)M;
  return p;
}

// The workspace starts with a fixed counter region (one uint32 per 16-row tile, for
// every problem size) that stays all-zero between calls; fp32 partials follow it.  A
// fixed region keeps one problem's partials from ever landing on another's counters.
constexpr int kMaxRowTiles = 16384;  // N <= 262144
constexpr size_t kCounterBytes = kMaxRowTiles * sizeof(uint32_t);

}  // namespace tl

using namespace tl;

extern "C" size_t tl_fp8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || N % 16 || K % kBlock) return 0;
  GemmPlan p = plan_gemm(M, N, K);
  if (p.ksplit == 1) return 0;
  return kCounterBytes + static_cast<size_t>(p.ksplit) * M * N * sizeof(float);
}

extern "C" int tl_fp8_gemm(const void* a, const float* a_s, const void* b, const float* b_s,
                           void* c_bf16, int64_t M, int64_t N, int64_t K, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (M <= 0 || N <= 0 || K <= 0) { set_error("fp8_gemm: empty problem M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K); return kErrArg; }
  if (K % kBlock) { set_error("fp8_gemm: K=%lld must be a multiple of 128", (long long)K); return kErrArg; }
  if (N % 16) { set_error("fp8_gemm: N=%lld must be a multiple of 16", (long long)N); return kErrArg; }
  if (M > 256) { set_error("fp8_gemm: M=%lld > 256 is not supported by the decode kernel", (long long)M); return kErrUnsupported; }
  if (N > 16ll * kMaxRowTiles || K > (1ll << 30)) { set_error("fp8_gemm: N or K too large"); return kErrArg; }
  if (!a || !a_s || !b || !b_s || !c_bf16) { set_error("fp8_gemm: null pointer"); return kErrArg; }
  if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) { set_error("fp8_gemm: a and b must be 16-byte aligned"); return kErrArg; }
  if (reinterpret_cast<uintptr_t>(c_bf16) & 7) { set_error("fp8_gemm: c must be 8-byte aligned"); return kErrArg; }
  GemmPlan p = plan_gemm(M, N, K);
  const size_t need = tl_fp8_gemm_workspace_bytes(M, N, K);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    set_error("fp8_gemm: workspace of %zu bytes required (got %zu)", need, workspace_bytes);
    return kErrArg;
  }
  uint32_t* counters = need ? static_cast<uint32_t*>(workspace) : nullptr;
  float* partial = need ? reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes) : nullptr;
  dim3 grid(p.row_tiles, p.ksplit);
  hipStream_t st = (hipStream_t)stream;
  const uint8_t* A = (const uint8_t*)a;
  const uint8_t* B = (const uint8_t*)b;
  uint16_t* C = (uint16_t*)c_bf16;
  const int m = (int)M, n = (int)N, k = (int)K, per = p.kb_per_split;
  if (M <= 16) hipLaunchKernelGGL((fp8_gemm_kernel<1, 4>), grid, dim3(256), 0, st, A, a_s, B, b_s, C, partial, counters, m, n, k, per);
  else if (M <= 32) hipLaunchKernelGGL((fp8_gemm_kernel<2, 4>), grid, dim3(256), 0, st, A, a_s, B, b_s, C, partial, counters, m, n, k, per);
  else if (M <= 64) hipLaunchKernelGGL((fp8_gemm_kernel<4, 2>), grid, dim3(256), 0, st, A, a_s, B, b_s, C, partial, counters, m, n, k, per);
  else if (M <= 128) hipLaunchKernelGGL((fp8_gemm_kernel<8, 2>), grid, dim3(256), 0, st, A, a_s, B, b_s, C, partial, counters, m, n, k, per);
  else hipLaunchKernelGGL((fp8_gemm_kernel<16, 1>), grid, dim3(256), 0, st, A, a_s, B, b_s, C, partial, counters, m, n, k, per);
  return check_launch("fp8_gemm");
}
