// Block-scaled FP8 GEMM for decode shapes: C[M,N] (bf16) = A[M,K] . B[N,K]^T with
// A e4m3fn + fp32 scales per (row, 128 cols) and B e4m3fn + fp32 scales per 128x128
// block -- the contract of fp8_gemm (refs/kernel.py:282-306, kernel :202-249).
//
// Design (gfx950):
//   * The weight B is the only large operand (132 MB at 18432x7168) and every byte is
//     read exactly once with 16-byte non-temporal loads: the kernel is an HBM stream.
//     The activation A (<= 256 rows) stays L1/L2 resident.
//   * Math is the native OCP-fp8 MFMA v_mfma_f32_16x16x128_f8f6f4: one MFMA covers 16
//     weight rows x 16 tokens x one whole 128-wide K block = exactly one scale block, so
//     the scale product b_s * a_s is applied once per MFMA to the fp32 partial (the
//     per-K-block scaling of refs/kernel.py:238-244).  For M <= 16 the unused token
//     columns are free: the matrix cores have >20x headroom over the weight stream.
//   * Weight layouts.  Canonical row-major [N,K] (the drop-in fp8_gemm operand), or
//     "fragment-packed": for every (16-row tile, 128-col block) the 2 KB MFMA operand
//     fragment is stored contiguously in lane order ([2 pieces][64 lanes][16 B]), so
//     each wave-wide load reads 1 KB of consecutive memory.  Packing is done once at
//     weight-load time (tl_fp8_pack_weight), like the reference's per-op weight
//     converters.  Measured on MI355X: packed fragments stream ~25% faster.
//   * One weight fragment in flight per wave (U = 1) and 4-8 waves per workgroup: on
//     this memory system deeper per-wave prefetch lowers achieved bandwidth.
//   * Work split: a workgroup owns one 16-row tile and a slice of K blocks; its waves
//     interleave over the slice and are summed through LDS in a fixed order.  The K split
//     is chosen so the grid covers the 256 CUs evenly; the last workgroup of a row tile
//     (agent-scope counter and agent-scope atomic partials) sums the fp32 partials in slice
//     order, so results are deterministic.
#include "common.h"
#include "../../include/tilert_amd.h"

namespace tl {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ inline v8i load_packed_fragment(const uint8_t* frag, int lane) {
  const u32x4* p = reinterpret_cast<const u32x4*>(frag);
  const u32x4 lo = __builtin_nontemporal_load(p + lane);
  const u32x4 hi = __builtin_nontemporal_load(p + 64 + lane);
  v8i r;
  r[0] = lo.x; r[1] = lo.y; r[2] = lo.z; r[3] = lo.w;
  r[4] = hi.x; r[5] = hi.y; r[6] = hi.z; r[7] = hi.w;
  return r;
}

__device__ inline uint2 pack_bf16x4(v4f v) {
  return make_uint2(f32_to_bf16(v[0]) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16),
                    f32_to_bf16(v[2]) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16));
}

// Fragment-packed layout ("K-group-major"): fragment (t, kb) -- 16 rows x 128 columns,
// 2048 bytes in MFMA lane order -- lives at fragment index
//   ((kb / 4) * NT + t) * 4 + kb % 4,      NT = N / 16,
// so the 4 K blocks a 4-wave workgroup reads in one step are 8 KB of consecutive memory
// and neighbouring row tiles' steps are neighbours: the whole grid sweeps the weight as
// one moving window, the access pattern this memory system streams best.
constexpr int kGroup = 4;

__device__ inline size_t packed_fragment(int t, int kb, int NT) {
  return ((static_cast<size_t>(kb / kGroup) * NT + t) * kGroup + (kb % kGroup)) * 2048;
}

// MT: 16-token tiles (M <= 16*MT); WAVES: waves per workgroup; PACKED: weight layout.
// Every operand of the next K block -- weight fragment, activation block, both scales --
// is requested one block ahead, so L2 latency of the activations hides behind the
// current MFMA.  Staging activations in LDS instead was measured slower: its prologue
// costs what it saves.
template <int MT, int WAVES, bool PACKED>
__global__ __launch_bounds__(WAVES * 64) void fp8_gemm_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ B,
    const float* __restrict__ Bs, uint16_t* __restrict__ C, float* __restrict__ partial,
    uint32_t* __restrict__ counters, int M, int N, int K, int kb_per_split) {
  __shared__ float red[WAVES - 1][MT][4][64];
  const int KB = K >> 7;
  const int NT = N >> 4;
  const int ksplit = gridDim.y;
  const int ks = blockIdx.y;
  const int kb_begin = ks * kb_per_split;
  const int kb_end = min(KB, kb_begin + kb_per_split);
  const int rt = blockIdx.x;
  const int n0 = rt * 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;

  const uint8_t* brow = B + static_cast<size_t>(n0 + r) * K;  // canonical layout
  const float* bs_row = Bs + static_cast<size_t>(n0 >> 7) * KB;
  auto load_w = [&](int kb) -> v8i {
    return PACKED ? load_packed_fragment(B + packed_fragment(rt, kb, NT), lane)
                  : load_kblock_stream(brow + static_cast<size_t>(kb) * kBlock, g);
  };
  // Activation rows past M are read from row M-1 and zeroed afterwards, so every load
  // in the loop below is unconditional: the compiler's wait-count pass can then wait for
  // exactly the operands an MFMA needs instead of for everything in flight.
  const int wv = __builtin_amdgcn_readfirstlane(wave);

  v4f acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};

  // Ping-pong over two operand buffers (the loop is unrolled by two) so the next K
  // block's loads are in flight during this block's MFMAs.  A `cur = next` rotation
  // would make the compiler copy registers at the end of each iteration -- and wait for
  // the loads in flight to do so, serialising the stream.
  struct Ops {
    v8i a, x[MT];
    float xs[MT], bs;
  };
  auto fetch = [&](int kb, Ops& o) {
    o.a = load_w(kb);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int t = min(mt * 16 + r, M - 1);
      o.x[mt] = load_kblock(A + static_cast<size_t>(t) * K + kb * kBlock, g);
      o.xs[mt] = As[static_cast<size_t>(t) * KB + kb];
    }
    o.bs = bs_row[kb];
    __builtin_amdgcn_sched_barrier(0);  // keep the loads issued ahead of the MFMAs after them
  };
  auto compute = [&](const Ops& o) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const float xs = mt * 16 + r < M ? o.xs[mt] : 0.f;  // zero rows past M
      acc[mt] += mfma_16x16x128_fp8(o.a, o.x[mt]) * (o.bs * xs);
    }
  };
  // this wave's K blocks: kb_begin + wv + i*WAVES, i < n
  const int kb0 = kb_begin + wv;
  const int n = kb0 < kb_end ? (kb_end - kb0 + WAVES - 1) / WAVES : 0;
  Ops b0, b1;
  if (n > 0) {
    fetch(kb0, b0);
    int i = 0;
    for (; i + 2 < n; i += 2) {
      fetch(kb0 + (i + 1) * WAVES, b1);
      compute(b0);
      fetch(kb0 + (i + 2) * WAVES, b0);
      compute(b1);
    }
    if (i + 1 < n) {
      fetch(kb0 + (i + 1) * WAVES, b1);
      compute(b0);
      compute(b1);
    } else {
      compute(b0);
    }
  }

  // ---- cross-wave reduction in fixed order w0 + w1 + ... + w(WAVES-1)
  if (wave > 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) red[wave - 1][mt][j][lane] = acc[mt][j];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < WAVES - 1; ++w)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[mt][j] += red[w][mt][j][lane];

  // lane holds output columns n0 + 4g + j (j = 0..3) of token mt*16 + r
  const int ncol = n0 + 4 * g;
  if (ksplit == 1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int t = mt * 16 + r;
      if (t < M) *reinterpret_cast<uint2*>(C + static_cast<size_t>(t) * N + ncol) = pack_bf16x4(acc[mt]);
    }
    return;
  }

  // ---- split-K: publish fp32 partials; the last slice to arrive reduces them in order.
  // Partials are agent-scope atomic stores/loads (written through to the device
  // coherence point, read past this XCD's L2), so no cache-wide writeback or
  // invalidate is needed; s_waitcnt makes the stores complete before the counter bump.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int t = mt * 16 + r;
    if (t < M) {
      float* dst = partial + (static_cast<size_t>(ks) * M + t) * N + ncol;
#pragma unroll
      for (int j = 0; j < 4; ++j) __hip_atomic_store(dst + j, acc[mt][j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  uint32_t prev = 0;
  if (lane == 0) prev = __hip_atomic_fetch_add(&counters[rt], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  prev = __shfl(prev, 0);
  if (prev != static_cast<uint32_t>(ksplit - 1)) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int t = mt * 16 + r;
    if (t < M) {
      // issue the loads of 8 slices at a time, then add them in slice order
      v4f s = {0.f, 0.f, 0.f, 0.f};
      for (int q0 = 0; q0 < ksplit; q0 += 8) {
        v4f v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int q = q0 + u < ksplit ? q0 + u : ksplit - 1;
          const float* src = partial + (static_cast<size_t>(q) * M + t) * N + ncol;
#pragma unroll
          for (int j = 0; j < 4; ++j) v[u][j] = __hip_atomic_load(src + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (q0 + u < ksplit) s += v[u];
      }
      *reinterpret_cast<uint2*>(C + static_cast<size_t>(t) * N + ncol) = pack_bf16x4(s);
    }
  }
  if (lane == 0) __hip_atomic_store(&counters[rt], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Pack a canonical [N, K] fp8 weight into K-group-major MFMA fragments (see
// packed_fragment): within fragment (t, kb), piece p, lane l = r + 16 g holds the 16
// bytes of row 16 t + r, columns 128 kb + 64 p + 16 g ... +15, at offset p*1024 + l*16.
__global__ __launch_bounds__(256) void pack_weight_kernel(const uint8_t* __restrict__ W,
                                                          uint8_t* __restrict__ P, int N, int K) {
  const int KB = K >> 7;
  const int NT = N >> 4;
  const int64_t chunk = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // 16-byte chunk id
  const int64_t total = static_cast<int64_t>(N) * K / 16;
  if (chunk >= total) return;
  const int64_t frag = chunk >> 7;  // 128 chunks per fragment, tile-major source order
  const int within = static_cast<int>(chunk & 127);
  const int p = within >> 6, l = within & 63;
  const int t = static_cast<int>(frag / KB), kb = static_cast<int>(frag % KB);
  const int row = t * 16 + (l & 15);
  const int col = kb * 128 + 64 * p + 16 * (l >> 4);
  *reinterpret_cast<uint4*>(P + packed_fragment(t, kb, NT) + within * 16) =
      *reinterpret_cast<const uint4*>(W + static_cast<size_t>(row) * K + col);
}

// Tile-major fragment packing used by the MoE kernels: fragment (t, kb) at
// (t * KB + kb) * 2048, same in-fragment order as above.
__global__ __launch_bounds__(256) void pack_tile_major_kernel(const uint8_t* __restrict__ W,
                                                              uint8_t* __restrict__ P, int N, int K) {
  const int KB = K >> 7;
  const int64_t chunk = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (chunk >= static_cast<int64_t>(N) * K / 16) return;
  const int64_t frag = chunk >> 7;
  const int within = static_cast<int>(chunk & 127);
  const int p = within >> 6, l = within & 63;
  const int t = static_cast<int>(frag / KB), kb = static_cast<int>(frag % KB);
  const int row = t * 16 + (l & 15);
  const int col = kb * 128 + 64 * p + 16 * (l >> 4);
  reinterpret_cast<uint4*>(P)[chunk] = *reinterpret_cast<const uint4*>(W + static_cast<size_t>(row) * K + col);
}

struct GemmPlan {
  int ksplit;
  int kb_per_split;
  int row_tiles;
  int waves;
};

// K split.  Wide layers (>= 512 row tiles, i.e. >= 2 workgroups per CU) run unsplit:
// measured on MI355X, the split's extra round trips (partial store, counter, reload)
// cost more than the better CU balance buys.  Narrow layers take the smallest split
// giving >= 1024 workgroups (4 per CU), preferring a grid that is a whole multiple of
// the 256 CUs, with slices of whole K groups, never leaving a slice empty.
static GemmPlan plan_gemm(int64_t N, int64_t K) {
  GemmPlan p;
  const int KB = static_cast<int>(K / kBlock);
  const int groups = static_cast<int>(cdiv(KB, kGroup));
  p.row_tiles = static_cast<int>(N / 16);
  int s = 1;
  if (p.row_tiles < 512) {
    int smin = static_cast<int>(cdiv(1024, p.row_tiles));
    if (smin > groups) smin = groups;
    if (smin < 1) smin = 1;
    s = smin;
    for (int c = smin; c <= 2 * smin && c <= groups; ++c) {
      if ((static_cast<int64_t>(p.row_tiles) * c) % 256 == 0) { s = c; break; }
    }
  }
  p.kb_per_split = static_cast<int>(cdiv(groups, s)) * kGroup;
  p.ksplit = static_cast<int>(cdiv(KB, p.kb_per_split));
  // wide layers: 8 waves (two K groups per step); split slices: 4 (one group)
  p.waves = (p.ksplit == 1 && KB >= 32) ? 8 : kGroup;
  return p;
}

// The workspace starts with a fixed counter region (one uint32 per 16-row tile, for
// every problem size) that stays all-zero between calls; fp32 partials follow it.  A
// fixed region keeps one problem's partials from ever landing on another's counters.
constexpr int kMaxRowTiles = 16384;  // N <= 262144
constexpr size_t kCounterBytes = kMaxRowTiles * sizeof(uint32_t);

template <bool PACKED>
static int launch_gemm(const uint8_t* A, const float* As, const uint8_t* B, const float* Bs,
                       uint16_t* C, int M, int N, int K, void* workspace, hipStream_t st) {
  const GemmPlan p = plan_gemm(N, K);
  uint32_t* counters = p.ksplit > 1 ? static_cast<uint32_t*>(workspace) : nullptr;
  float* partial = p.ksplit > 1 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes) : nullptr;
  const dim3 grid(p.row_tiles, p.ksplit);
  const int per = p.kb_per_split;
#define TL_GEMM_LAUNCH(MT, W) \
  hipLaunchKernelGGL((fp8_gemm_kernel<MT, W, PACKED>), grid, dim3(W * 64), 0, st, A, As, B, Bs, C, partial, counters, M, N, K, per)
  if (p.waves == 8) {
    if (M <= 16) TL_GEMM_LAUNCH(1, 8);
    else if (M <= 32) TL_GEMM_LAUNCH(2, 8);
    else if (M <= 64) TL_GEMM_LAUNCH(4, 8);
    else if (M <= 128) TL_GEMM_LAUNCH(8, 4);
    else TL_GEMM_LAUNCH(16, 4);
  } else {
    if (M <= 16) TL_GEMM_LAUNCH(1, 4);
    else if (M <= 32) TL_GEMM_LAUNCH(2, 4);
    else if (M <= 64) TL_GEMM_LAUNCH(4, 4);
    else if (M <= 128) TL_GEMM_LAUNCH(8, 4);
    else TL_GEMM_LAUNCH(16, 4);
  }
#undef TL_GEMM_LAUNCH
  return check_launch("fp8_gemm");
}

static int validate(const char* who, const void* a, const float* a_s, const void* b,
                    const float* b_s, void* c, int64_t M, int64_t N, int64_t K, void* workspace,
                    size_t workspace_bytes, size_t need) {
  if (M <= 0 || N <= 0 || K <= 0) { set_error("%s: empty problem M=%lld N=%lld K=%lld", who, (long long)M, (long long)N, (long long)K); return kErrArg; }
  if (K % kBlock) { set_error("%s: K=%lld must be a multiple of 128", who, (long long)K); return kErrArg; }
  if (N % 16) { set_error("%s: N=%lld must be a multiple of 16", who, (long long)N); return kErrArg; }
  if (M > 256) { set_error("%s: M=%lld > 256 is not supported by the decode kernel", who, (long long)M); return kErrUnsupported; }
  if (N > 16ll * kMaxRowTiles || K > (1ll << 30)) { set_error("%s: N or K too large", who); return kErrArg; }
  if (!a || !a_s || !b || !b_s || !c) { set_error("%s: null pointer", who); return kErrArg; }
  if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) { set_error("%s: a and b must be 16-byte aligned", who); return kErrArg; }
  if (reinterpret_cast<uintptr_t>(c) & 7) { set_error("%s: c must be 8-byte aligned", who); return kErrArg; }
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    set_error("%s: workspace of %zu bytes required (got %zu)", who, need, workspace_bytes);
    return kErrArg;
  }
  return kOk;
}

}  // namespace tl

using namespace tl;

extern "C" size_t tl_fp8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || N % 16 || K % kBlock || M > 256) return 0;
  const GemmPlan p = plan_gemm(N, K);
  if (p.ksplit == 1) return 0;
  return kCounterBytes + static_cast<size_t>(p.ksplit) * M * N * sizeof(float);
}

extern "C" int tl_fp8_gemm(const void* a, const float* a_s, const void* b, const float* b_s,
                           void* c_bf16, int64_t M, int64_t N, int64_t K, void* workspace,
                           size_t workspace_bytes, void* stream) {
  const size_t need = tl_fp8_gemm_workspace_bytes(M, N, K);
  int rc = validate("fp8_gemm", a, a_s, b, b_s, c_bf16, M, N, K, workspace, workspace_bytes, need);
  if (rc) return rc;
  return launch_gemm<false>((const uint8_t*)a, a_s, (const uint8_t*)b, b_s, (uint16_t*)c_bf16,
                            (int)M, (int)N, (int)K, workspace, (hipStream_t)stream);
}

extern "C" int tl_fp8_pack_weight(const void* b, void* packed, int64_t N, int64_t K, void* stream) {
  if (N <= 0 || K <= 0 || N % 16 || K % (kBlock * kGroup)) { set_error("pack_weight: need N %% 16 == 0 and K %% 512 == 0 (N=%lld K=%lld)", (long long)N, (long long)K); return kErrArg; }
  if (!b || !packed) { set_error("pack_weight: null pointer"); return kErrArg; }
  if ((reinterpret_cast<uintptr_t>(b) | reinterpret_cast<uintptr_t>(packed)) & 15) { set_error("pack_weight: pointers must be 16-byte aligned"); return kErrArg; }
  if (b == packed) { set_error("pack_weight: in-place packing is not supported"); return kErrArg; }
  const int64_t chunks = N * K / 16;
  hipLaunchKernelGGL(pack_weight_kernel, dim3(cdiv(chunks, 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)b, (uint8_t*)packed, (int)N, (int)K);
  return check_launch("pack_weight");
}

extern "C" int tl_moe_pack_weight(const void* b, void* packed, int64_t rows, int64_t K, void* stream) {
  if (rows <= 0 || K <= 0 || rows % 16 || K % kBlock) { set_error("moe_pack_weight: need rows %% 16 == 0 and K %% 128 == 0 (rows=%lld K=%lld)", (long long)rows, (long long)K); return kErrArg; }
  if (!b || !packed) { set_error("moe_pack_weight: null pointer"); return kErrArg; }
  if ((reinterpret_cast<uintptr_t>(b) | reinterpret_cast<uintptr_t>(packed)) & 15) { set_error("moe_pack_weight: pointers must be 16-byte aligned"); return kErrArg; }
  if (b == packed) { set_error("moe_pack_weight: in-place packing is not supported"); return kErrArg; }
  hipLaunchKernelGGL(pack_tile_major_kernel, dim3(cdiv(rows * K / 16, 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)b, (uint8_t*)packed, (int)rows, (int)K);
  return check_launch("moe_pack_weight");
}

extern "C" int tl_fp8_gemm_packed(const void* a, const float* a_s, const void* b_packed,
                                  const float* b_s, void* c_bf16, int64_t M, int64_t N, int64_t K,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  if (K % (kBlock * kGroup)) { set_error("fp8_gemm_packed: K=%lld must be a multiple of 512", (long long)K); return kErrArg; }
  const size_t need = tl_fp8_gemm_workspace_bytes(M, N, K);
  int rc = validate("fp8_gemm_packed", a, a_s, b_packed, b_s, c_bf16, M, N, K, workspace, workspace_bytes, need);
  if (rc) return rc;
  return launch_gemm<true>((const uint8_t*)a, a_s, (const uint8_t*)b_packed, b_s, (uint16_t*)c_bf16,
                           (int)M, (int)N, (int)K, workspace, (hipStream_t)stream);
}
