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
//   * M <= 64 (fp8_gemm_kernel; on packed weights with N % 128 = 0 only up to M = 16, and
//     at M = 17..32 where the wide kernel below would split K in more than 4): a workgroup
//     owns one 16-row tile and a slice of K blocks;
//     its 4-8 waves interleave over the slice, each with the next block's operands in
//     flight (two buffers in ping-pong; deeper rings measured no faster), and are summed
//     through LDS in a fixed order.  The K split is chosen so the grid covers the 256 CUs
//     evenly; the last workgroup of a row tile (agent-scope counter and agent-scope atomic
//     partials) sums the fp32 partials in slice order, so results are deterministic.
//   * from M = 17 (K split in <= 4) or 33 on packed weights with N % 128 = 0
//     (fp8_gemm_wide_kernel): F row
//     tiles x 64 or 128 tokens per workgroup, one balanced round of 256 workgroups,
//     operands staged in LDS.
//   * M > 64 otherwise (fp8_gemm_tiled_kernel): 128-row workgroups share activation chunks
//     staged in LDS (see below).
#include <algorithm>
#include <cstdint>
#include <type_traits>
#include <mutex>
#include <utility>

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

// The same fragment through the caches (activation images are re-read by every workgroup).
__device__ inline v8i load_fragment(const uint8_t* frag, int lane) {
  const uint4 lo = reinterpret_cast<const uint4*>(frag)[lane];
  const uint4 hi = reinterpret_cast<const uint4*>(frag)[64 + lane];
  return v8i{static_cast<int>(lo.x), static_cast<int>(lo.y), static_cast<int>(lo.z), static_cast<int>(lo.w),
             static_cast<int>(hi.x), static_cast<int>(hi.y), static_cast<int>(hi.z), static_cast<int>(hi.w)};
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
// Where the output lands.  Column n of row t goes to segment 0 (n < end0), 1
// (n < end1) or 2, at column n - (segment start) of row t with the segment's leading
// dimension; segment 2 may instead be a cache indexed by position: row
// (t / seq) * cache_rows + *cur_pos + t % seq, skipped when that position is outside
// [0, cache_rows).  A plain GEMM is one segment: C [M, N].  The 4 columns a lane stores
// lie in one 16-column tile, so in one segment (segment bounds are multiples of 16).
struct OutRoute {
  uint16_t* p0;
  uint16_t* p1;
  uint16_t* p2;
  int end0, end1;
  int ld0, ld1, ld2;
  const int32_t* cur_pos;  // null: segment 2 is a plain [M, ld2] matrix
  int seq, cache_rows;
};

__host__ inline OutRoute plain_out(uint16_t* C, int N) {
  return OutRoute{C, nullptr, nullptr, N, N, N, 0, 0, nullptr, 1, 0};
}

__device__ inline void store_out(const OutRoute& o, int t, int n, uint2 v) {
  uint16_t* dst;
  if (n < o.end0) {
    dst = o.p0 + static_cast<size_t>(t) * o.ld0 + n;
  } else if (n < o.end1) {
    dst = o.p1 + static_cast<size_t>(t) * o.ld1 + (n - o.end0);
  } else {
    int row = t;
    if (o.cur_pos) {
      const int pos = *o.cur_pos + t % o.seq;
      if (pos < 0 || pos >= o.cache_rows) return;
      row = (t / o.seq) * o.cache_rows + pos;
    }
    dst = o.p2 + static_cast<size_t>(row) * o.ld2 + (n - o.end1);
  }
  *reinterpret_cast<uint2*>(dst) = v;
}

// D: operand buffers per wave.  D = 2 is the ping-pong below; narrow layers (few row
// tiles, so few waves on the chip) take a deeper ring so that enough weight bytes are in
// flight to cover HBM latency without splitting K.
// RT: 16-row tiles per workgroup (1, 2 or 4; within one 128-row scale block).  Each
// activation fragment a wave loads then serves RT weight fragments, which divides the
// activation traffic (as large as the weight traffic itself from M = 16 on) by RT.
// XF: A / As are the activation image of act_image_kernel (fragment order, transposed
// scales) instead of x [M, K] / [M, K/128].
template <int MT, int WAVES, bool PACKED, int D = 2, int RT = 1, bool XF = false>
__global__ __launch_bounds__(WAVES * 64) void fp8_gemm_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ B,
    const float* __restrict__ Bs, const OutRoute out, float* __restrict__ partial,
    uint32_t* __restrict__ counters, int M, int N, int K, int kb_per_split) {
  constexpr int NA = RT * MT;  // accumulators per lane: (row tile j, token tile mt) at j * MT + mt
  __shared__ v4f red[WAVES - 1][NA][64];
  const int KB = K >> 7;
  const int NT = N >> 4;
  const int ksplit = gridDim.y;
  const int ks = blockIdx.y;
  const int kb_begin = ks * kb_per_split;
  const int kb_end = min(KB, kb_begin + kb_per_split);
  const int rt = blockIdx.x * RT;  // first row tile
  const int n0 = rt * 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;

  const uint8_t* brow = B + static_cast<size_t>(n0 + r) * K;  // canonical layout
  const float* bs_row = Bs + static_cast<size_t>(n0 >> 7) * KB;
  auto load_w = [&](int kb, int j) -> v8i {
    return PACKED ? load_packed_fragment(B + packed_fragment(rt + j, kb, NT), lane)
                  : load_kblock_stream(brow + static_cast<size_t>(16 * j) * K + static_cast<size_t>(kb) * kBlock, g);
  };
  // Activation rows past M are read from row M-1 and zeroed afterwards, so every load
  // in the loop below is unconditional: the compiler's wait-count pass can then wait for
  // exactly the operands an MFMA needs instead of for everything in flight.
  const int wv = __builtin_amdgcn_readfirstlane(wave);

  v4f acc[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};

  // Ping-pong over two operand buffers (the loop is unrolled by two) so the next K
  // block's loads are in flight during this block's MFMAs.  A `cur = next` rotation
  // would make the compiler copy registers at the end of each iteration -- and wait for
  // the loads in flight to do so, serialising the stream.
  struct Ops {
    v8i a[RT], x[MT];
    float xs[MT], bs;
  };
  auto fetch = [&](int kb, Ops& o) {
#pragma unroll
    for (int j = 0; j < RT; ++j) o.a[j] = load_w(kb, j);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if constexpr (XF) {
        const int mtt = (M + 15) >> 4;
        o.x[mt] = load_fragment(A + (static_cast<size_t>(kb) * mtt + mt) * 2048, lane);
        o.xs[mt] = As[static_cast<size_t>(kb) * mtt * 16 + mt * 16 + r];
      } else {
        const int t = min(mt * 16 + r, M - 1);
        o.x[mt] = load_kblock(A + static_cast<size_t>(t) * K + kb * kBlock, g);
        o.xs[mt] = As[static_cast<size_t>(t) * KB + kb];
      }
    }
    o.bs = bs_row[kb];
    __builtin_amdgcn_sched_barrier(0);  // keep the loads issued ahead of the MFMAs after them
  };
  auto compute = [&](const Ops& o) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const float xs = mt * 16 + r < M ? o.xs[mt] : 0.f;  // zero rows past M
#pragma unroll
      for (int j = 0; j < RT; ++j) acc[j * MT + mt] += mfma_16x16x128_fp8(o.a[j], o.x[mt]) * (o.bs * xs);
    }
  };
  // this wave's K blocks: kb_begin + wv + i*WAVES, i < n
  const int kb0 = kb_begin + wv;
  const int n = kb0 < kb_end ? (kb_end - kb0 + WAVES - 1) / WAVES : 0;
  if constexpr (D > 2) {
    Ops ring[D];
    ring_pipeline<D>(n, ring, [&](int i, Ops& o) { fetch(kb0 + i * WAVES, o); },
                     [&](int, const Ops& o) { compute(o); });
  } else {
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
  }

  // ---- cross-wave reduction in fixed order w0 + w1 + ... + w(WAVES-1)
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < NA; ++i) red[wave - 1][i][lane] = acc[i];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < WAVES - 1; ++w)
#pragma unroll
    for (int i = 0; i < NA; ++i) acc[i] += red[w][i][lane];

  // lane holds output columns n0 + 16 jt + 4g + j (j = 0..3) of token mt*16 + r
  if (ksplit == 1) {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int t = (i % MT) * 16 + r;
      if (t < M) store_out(out, t, n0 + 16 * (i / MT) + 4 * g, pack_bf16x4(acc[i]));
    }
    return;
  }

  // ---- split-K: publish fp32 partials; the last slice to arrive reduces them in order.
  // Partials are agent-scope atomic stores/loads (written through to the device
  // coherence point, read past this XCD's L2), so no cache-wide writeback or
  // invalidate is needed; s_waitcnt makes the stores complete before the counter bump.
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int t = (i % MT) * 16 + r;
    if (t < M) {
      float* dst = partial + (static_cast<size_t>(ks) * M + t) * N + n0 + 16 * (i / MT) + 4 * g;
#pragma unroll
      for (int j = 0; j < 4; ++j) __hip_atomic_store(dst + j, acc[i][j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  uint32_t prev = 0;
  if (lane == 0) prev = __hip_atomic_fetch_add(&counters[rt], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  prev = __shfl(prev, 0);
  if (prev != static_cast<uint32_t>(ksplit - 1)) return;
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int t = (i % MT) * 16 + r;
    const int ncol = n0 + 16 * (i / MT) + 4 * g;
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
      store_out(out, t, ncol, pack_bf16x4(s));
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

// Activation image for the GEMVs at M > 16: x [M, K] rearranged so that the MFMA operand
// of token tile tt and K block kb is 2 KB of consecutive memory at (kb * MTT + tt) * 2048
// (MTT = ceil(M / 16); in-fragment order as in the weight packing; tokens past M repeat
// token M-1), and the scales transposed to [K/128, 16 MTT] (0 past M).  The GEMV's
// activation loads then become contiguous 1 KB reads.  The gather they replace (16 rows x
// 64 B per instruction) was measured at ~9 TB/s of L2-resident reads across the chip,
// against ~33 TB/s for contiguous ones.
__global__ __launch_bounds__(256) void act_image_kernel(const uint8_t* __restrict__ A, const float* __restrict__ As,
                                                        uint8_t* __restrict__ X, float* __restrict__ Xs, int M, int K) {
  const int KB = K >> 7;
  const int mtt = (M + 15) >> 4;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < static_cast<int64_t>(KB) * mtt * 128) {  // one 16-byte chunk per thread
    const int64_t frag = i >> 7;
    const int within = static_cast<int>(i & 127);
    const int p = within >> 6, l = within & 63;
    const int kb = static_cast<int>(frag / mtt), tt = static_cast<int>(frag % mtt);
    const int row = min(tt * 16 + (l & 15), M - 1);
    *reinterpret_cast<uint4*>(X + i * 16) =
        *reinterpret_cast<const uint4*>(A + static_cast<size_t>(row) * K + kb * 128 + 64 * p + 16 * (l >> 4));
  }
  if (i < static_cast<int64_t>(KB) * mtt * 16) {  // one scale per thread
    const int kb = static_cast<int>(i / (mtt * 16)), t = static_cast<int>(i % (mtt * 16));
    Xs[i] = t < M ? As[static_cast<size_t>(t) * KB + kb] : 0.f;
  }
}

__host__ inline size_t act_image_bytes(int64_t M, int64_t K) {
  const int64_t mtt = cdiv(M, 16), KB = K / kBlock;
  return static_cast<size_t>(KB * mtt * 2048 + KB * mtt * 16 * 4);
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

// ---------------------------------------------------------------- M > 64: tiled
// For M > 64 tokens the activation blocks are no longer small next to the weights: a
// wave that reads them from L1/L2 for each of its token tiles moves up to 4x the weight
// bytes through the texture path.  Here a workgroup of 8 waves covers 128 rows (one
// 16-row tile per wave) x all TT token tiles over a slice of K blocks:
//   * activations (MFMA fragment order) and their scales are staged in LDS by the whole
//     workgroup in chunks of KC = 16 / TT K blocks (32 KB), double-buffered and loaded
//     one chunk ahead -- one barrier per chunk;
//   * each wave streams its weight fragments through a ring of kTiledDepth buffers that
//     runs on across chunk boundaries, so a barrier never drains the weight stream;
//   * full chunks issue unconditional loads only (exact wait counts); the last chunks of
//     a slice guard the weight fetches, so no fragment is read twice.
// Split-K slices are reduced as in fp8_gemm_kernel (partials + last-arriver, in slice
// order, deterministic).
// static_for<N>(f): f(std::integral_constant<int, 0>{}) ... f(<N-1>) -- compile-time loop
template <int... I, class F>
__device__ __attribute__((always_inline)) inline void static_for_impl(std::integer_sequence<int, I...>, F&& f) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __attribute__((always_inline)) inline void static_for(F&& f) {
  static_for_impl(std::make_integer_sequence<int, N>{}, f);
}

constexpr int kTiledWaves = 8;
constexpr int kTiledDepth = 4;

template <int TT>
struct TiledShape {
  static constexpr int THREADS = kTiledWaves * 64;
  static constexpr int KC = 16 / TT >= 1 ? 16 / TT : 1;   // K blocks per chunk
  static_assert(KC % kTiledDepth == 0 || kTiledDepth % KC == 0, "ring slots must be static");
  static constexpr int XCH = KC * TT * 128;                // 16-byte chunks per chunk
  static constexpr int XPT = (XCH + THREADS - 1) / THREADS;
  static constexpr int XBUF = XPT * THREADS * 16;          // bytes per buffer (padded)
  static constexpr int SCN = KC * TT * 16;                 // activation scales per chunk
  static constexpr int SPT = (SCN + THREADS - 1) / THREADS;
  static constexpr int SBUF = SPT * THREADS;               // floats per buffer (padded)
  static constexpr int LDS = 2 * XBUF + 2 * SBUF * 4;
};

// dynamic LDS of fp8_gemm_tiled_kernel<TT>
template <int TT>
constexpr int tiled_lds_bytes() { return TiledShape<TT>::LDS; }

template <int TT, bool PACKED>
__global__ __launch_bounds__(kTiledWaves * 64) void fp8_gemm_tiled_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ B,
    const float* __restrict__ Bs, const OutRoute out, float* __restrict__ partial,
    uint32_t* __restrict__ counters, int M, int N, int K, int kb_per_split) {
  using S = TiledShape<TT>;
  constexpr int KC = S::KC, D = kTiledDepth, THREADS = S::THREADS;
  extern __shared__ __attribute__((aligned(16))) uint8_t tiled_smem[];
  __shared__ uint32_t last_flag;
  const int KB = K >> 7;
  const int NT = N >> 4;
  const int ksplit = gridDim.y, ks = blockIdx.y;
  const int kb_begin = ks * kb_per_split;
  const int n = max(0, min(KB, kb_begin + kb_per_split) - kb_begin);  // K blocks in this slice
  const int nch = (n + KC - 1) / KC;                                  // chunks
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int rt = min(static_cast<int>(blockIdx.x) * kTiledWaves + wave, NT - 1);  // rows past N: not stored
  const bool row_ok = static_cast<int>(blockIdx.x) * kTiledWaves + wave < NT;
  const uint8_t* brow = B + static_cast<size_t>(rt * 16 + r) * K;
  const float* bs_row = Bs + static_cast<size_t>(rt >> 3) * KB;

  // ---- activation chunks: chunk c covers K blocks kb_begin + c*KC + j, j < KC.  LDS
  // image chunk d: block j = d / (TT*128), token tile tt = (d / 128) % TT, piece
  // (d / 64) % 2, lane d % 64 -> token 16 tt + l % 16 (clamped), 16-byte piece 4 p + l / 16
  u32x4 xr[S::XPT];  // ext-vector type: a HIP uint4 struct copy would stay in scratch
  float sr[S::SPT];
  auto x_issue = [&](int c) __attribute__((always_inline)) {  // unconditional, indices clamped
    static_for<S::XPT>([&](auto ut) __attribute__((always_inline)) {
      constexpr int u = decltype(ut)::value;
      const int d = min(tid + u * THREADS, S::XCH - 1);
      const int j = d / (TT * 128), tt = (d >> 7) % TT, pp = (d >> 6) & 1, l = d & 63;
      const int kb = kb_begin + min(c * KC + j, n - 1);
      const int tok = min(tt * 16 + (l & 15), M - 1);
      xr[u] = *reinterpret_cast<const u32x4*>(A + static_cast<size_t>(tok) * K + kb * kBlock + pp * 64 + (l >> 4) * 16);
    });
    static_for<S::SPT>([&](auto ut) __attribute__((always_inline)) {
      constexpr int u = decltype(ut)::value;
      const int e = min(tid + u * THREADS, S::SCN - 1);  // scale e: block e / (TT*16), token e % (TT*16)
      const int kb = kb_begin + min(c * KC + e / (TT * 16), n - 1);
      sr[u] = As[static_cast<size_t>(min(e % (TT * 16), M - 1)) * KB + kb];
    });
  };
  auto x_put = [&](int buf) __attribute__((always_inline)) {  // unconditional writes (padding absorbs the surplus)
    u32x4* xl = reinterpret_cast<u32x4*>(tiled_smem + buf * S::XBUF);
    float* sl = reinterpret_cast<float*>(tiled_smem + 2 * S::XBUF) + buf * S::SBUF;
    static_for<S::XPT>([&](auto ut) __attribute__((always_inline)) { xl[tid + decltype(ut)::value * THREADS] = xr[decltype(ut)::value]; });
    static_for<S::SPT>([&](auto ut) __attribute__((always_inline)) {
      constexpr int u = decltype(ut)::value;
      const int e = tid + u * THREADS;
      sl[e] = (e % (TT * 16)) < M ? sr[u] : 0.f;  // tokens past M contribute 0
    });
  };

  // ---- weight ring: item i = K block kb_begin + i
  v8i wr[D];
  float bsr[D];
  // slot = i % D, always passed as a compile-time value (a runtime index would put the
  // ring in scratch memory)
  auto w_fetch = [&](int i, auto slot_tag) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_tag)::value;
    const int kb = kb_begin + min(i, n - 1);
    wr[slot] = PACKED ? load_packed_fragment(B + packed_fragment(rt, kb, NT), lane)
                      : load_kblock_stream(brow + static_cast<size_t>(kb) * kBlock, g);
    bsr[slot] = bs_row[kb];
  };

  v4f acc[TT];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) acc[tt] = v4f{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](auto slot_tag, int buf, int j) __attribute__((always_inline)) {  // chunk block j of buffer buf
    constexpr int slot = decltype(slot_tag)::value;
    const u32x4* xl = reinterpret_cast<const u32x4*>(tiled_smem + buf * S::XBUF) + j * TT * 128;
    const float* sl = reinterpret_cast<const float*>(tiled_smem + 2 * S::XBUF) + buf * S::SBUF + j * TT * 16;
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      const u32x4 lo = xl[tt * 128 + lane];
      const u32x4 hi = xl[tt * 128 + 64 + lane];
      const v8i xb = {static_cast<int>(lo.x), static_cast<int>(lo.y), static_cast<int>(lo.z), static_cast<int>(lo.w),
                      static_cast<int>(hi.x), static_cast<int>(hi.y), static_cast<int>(hi.z), static_cast<int>(hi.w)};
      acc[tt] += mfma_16x16x128_fp8(wr[slot], xb) * (bsr[slot] * sl[tt * 16 + r]);
      if ((tt & 3) == 3) __builtin_amdgcn_sched_barrier(0);  // bound the operand reads in flight
    }
  };

  if (n > 0) {
    // prologue: chunk 0 into LDS buffer 0, chunk 1 into registers, the first D-1 weights
    x_issue(0);
    x_put(0);
    x_issue(1);
    static_for<D - 1>([&](auto i) __attribute__((always_inline)) { w_fetch(decltype(i)::value, i); });
    // one chunk: stage chunk c+1 (registers -> LDS), request chunk c+2, then its KC
    // items.  CC = c % CPI is compile-time, so every ring slot is.  SAFE: every weight
    // fetch of the chunk is inside the slice (no guard needed).
    auto chunk = [&](int c, auto cc_tag, auto safe_tag) __attribute__((always_inline)) {
      constexpr int CC = decltype(cc_tag)::value;
      constexpr bool SAFE = decltype(safe_tag)::value;
      __syncthreads();   // chunk c-1 is done everywhere: its buffer may be refilled
      x_put((c + 1) & 1);
      x_issue(c + 2);
      static_for<KC>([&](auto jt) __attribute__((always_inline)) {
        constexpr int j = decltype(jt)::value;
        const int i = c * KC + j;
        const auto cur = std::integral_constant<int, (CC * KC + j) % D>{};
        const auto nxt = std::integral_constant<int, (CC * KC + j + D - 1) % D>{};
        if (SAFE) {
          w_fetch(i + D - 1, nxt);
          compute(cur, c & 1, j);
        } else if (i < n) {
          if (i + D - 1 < n) w_fetch(i + D - 1, nxt);
          compute(cur, c & 1, j);
        }
      });
    };
    __syncthreads();  // chunk 0 visible
    // CPI chunks per loop step, unrolled, so that item i's ring slot i % D is a
    // compile-time index (CPI * KC is a multiple of D)
    constexpr int CPI = KC >= D ? 1 : D / KC;
    int c = 0;
    // a step is safe when its last fetch, item (c+CPI)*KC + D - 2, is inside the slice
    for (; (c + CPI) * KC + D - 2 < n; c += CPI)
      static_for<CPI>([&](auto cc) __attribute__((always_inline)) { chunk(c + decltype(cc)::value, cc, std::true_type{}); });
    for (; c < nch; c += CPI)
      static_for<CPI>([&](auto cc) __attribute__((always_inline)) {
        if (c + decltype(cc)::value < nch) chunk(c + decltype(cc)::value, cc, std::false_type{});
      });
  }

  // lane holds output rows rt*16 + 4g + j (j = 0..3) of token tt*16 + r
  const int ncol = rt * 16 + 4 * g;
  if (ksplit == 1) {
    if (row_ok) {
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        const int t = tt * 16 + r;
        if (t < M) store_out(out, t, ncol, pack_bf16x4(acc[tt]));
      }
    }
    return;
  }
  // split-K: agent-scope partials, then the last slice of this row group sums them
  if (row_ok) {
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      const int t = tt * 16 + r;
      if (t < M) {
        float* dst = partial + (static_cast<size_t>(ks) * M + t) * N + ncol;
#pragma unroll
        for (int j = 0; j < 4; ++j) __hip_atomic_store(dst + j, acc[tt][j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();  // every wave's partials are complete before the counter moves
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&counters[blockIdx.x], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_flag = prev == static_cast<uint32_t>(ksplit - 1);
  }
  __syncthreads();
  if (!last_flag) return;
  if (row_ok) {
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      const int t = tt * 16 + r;
      if (t < M) {
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
        store_out(out, t, ncol, pack_bf16x4(s));
      }
    }
  }
  if (tid == 0) __hip_atomic_store(&counters[blockIdx.x], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- M > 32: MFMA GEMM
// Wide-tile MFMA GEMM for 16 < M <= 256 on packed weights (fp8_gemm_wide_kernel<F, TJ>).
// A workgroup (8 waves, one workgroup per CU) owns F consecutive 16-row weight tiles x one
// group of 4 TJ token fragments (64 or 128 tokens; TJ = 1 up to M = 64) over one of S K
// ranges.  The host picks F (4..9) and S so that tiles x token groups x S <= 256
// workgroups give every CU the same work in one round (up 7168 -> 18432 at M = 256: F = 9,
// 128 row tiles x 2 token groups; down 18432 -> 7168: F = 7, 64 x 2 x 2 K ranges).  Waves
// w and w + 4 (one SIMD) share token fragments w % 4 and split the F rows, so every
// fragment a wave reads from LDS feeds several MFMAs and each SIMD has two waves to hide
// the other's latencies.
// Per K block the weight fragments, the activation rows (read from x [M, K] itself) and
// their scales are copied global -> LDS (global_load_lds, no registers) into a 4-stage
// ring; each wave reads block i + 1's operands into a second register set while
// block i's MFMAs run.  The 2F weight pieces are dealt to the waves round robin, wave 2
// copies the weight scales and the token scales come in 16-block windows, so per-wave copy
// counts differ, but each wave issues the same count every block (plus the window copies
// at a window's first block, which only make the next waits stricter) and waits for its
// own copies with a fixed s_waitcnt before the block's s_barrier.
// Workgroup ids: the token groups of one weight slice (row tile, K range) are 8 ids apart,
// so that, with consecutive ids dealt to the 8 XCDs round robin, both run on one XCD and
// the second read of each weight fragment hits its L2 (FETCH_SIZE at M = 256 up: 148 MB
// per call for 132 MB of weights).
// With S > 1 the S partial sums of a tile are fp32 partials in the workspace, written and
// read with 16-byte sc1 accesses (past this XCD's L2, like agent-scope atomics); the
// workgroup that completes a tile (agent-scope counter) sums them in range order, so
// results are deterministic.
// When the wide kernel replaces the GEMV on packed weights (measured, us, wide vs GEMV):
// from M = 33 on always (up 7168 -> 18432 at M = 33 / 48 / 64: 28.1 / 28.7 / 29.5 vs
// 48.9 / 49.1 / 51.2; down 18432 -> 7168 at M = 64: 29.8 vs 41.3; 7168 -> 1536 at M = 64:
// 12.7 vs 22.5); at M = 17..32 only when its plan splits K at most in 4 (up at M = 17 / 32:
// 28.5 / 27.9 vs 35.7 / 35.8; down at M = 17 / 24 / 32: 29.4 / 29.1 / 29.4 vs 30.2 / 30.3 /
// 30.3; small layers that split K 8 ways or more lose: 7168 -> 1024 at M = 32 14.3 vs
// 10.5, 2048 -> 4096 at M = 24 9.5 vs 6.5); at M <= 16 never (up at M = 16: GEMV 27.2).
constexpr int kWideMinM = 32;      // from M = 33 on always
constexpr int kWideMinM2 = 16;     // from M = 17 on when the K split is small:
constexpr int kWideMaxSplit2 = 4;  // at most this many K ranges
constexpr int kWideGrid = 256;
constexpr int kCpolSc1 = 16;            // buffer access cache policy: sc1
constexpr int kRsrcWord3 = 0x00020000;  // buffer resource word 3: 32-bit data format

// 8 waves: waves w and w + 4 (same SIMD) share token fragments w % 4 and split the F rows
// (FH and F - FH), so each SIMD has two waves to hide the other's LDS and MFMA latencies.
constexpr int kWideWaves = 8;

// TJ: token fragments per wave (1 up to M = 64, else 2); a workgroup covers TT = 4 TJ
// token fragments (16 TT tokens).
template <int F, int TJ>
struct WideShape {
  static constexpr int TT = 4 * TJ;
  static constexpr int STAGES = 4;                      // ring depth (5 measured no faster at TJ = 1)
  static constexpr int FH = (F + 1) / 2;                // rows of the first split
  static constexpr int W = F * 2048;                    // weight fragments of one K block
  static constexpr int A = TT * 2048;                   // activation fragments
  static constexpr int WS = W + A;                      // weight scales (F floats)
  static constexpr int STAGE = WS + 256;
  static constexpr int WIN = STAGES * STAGE;            // token-scale windows: [2][128][16] fp32
  static constexpr int LDS = WIN + 2 * 128 * 16 * 4;
  static constexpr int SLOT = F * TT * 256;             // floats of one partial
  static_assert(16 * TT <= 128, "the token-scale windows hold 128 tokens");
};

// Copy instructions wave w issues per K block: its weight pieces (the 2F 1 KB pieces dealt
// round robin), TJ activation pieces, and the weight scales (wave 2).  At the first block
// of each 16-block window (and of the range) waves 0 .. TT - 1 also copy their 16 tokens'
// scales of the window (4 more copies); those blocks' waits then cover a few copies of the
// next block too, which is conservative.
__host__ __device__ constexpr int wide_ops(int F, int TJ, int w) {
  return (2 * F - w + kWideWaves - 1) / kWideWaves + TJ + (w == 2 ? 1 : 0);
}

// Load-to-LDS copies as in copy_to_lds16 / copy_to_lds4 (common.h), but taking the LDS
// address as a wave-uniform 32-bit value already computed, with no generic-to-LDS pointer
// conversion per copy (m0, a reserved register, is saved and restored as there): the wide
// kernel issues 4-8 of these per K block.
__device__ inline void dma_lds16(const void* src, uint32_t lds) {
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(saved) : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}
__device__ inline void dma_lds4(const void* src, uint32_t lds) {
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(saved) : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}

template <int F, int TJ>
__global__ __launch_bounds__(kWideWaves * 64) void fp8_gemm_wide_kernel(
    const uint8_t* __restrict__ X, const float* __restrict__ Xs, const uint8_t* __restrict__ B,
    const float* __restrict__ Bs, const OutRoute out, float* __restrict__ partial,
    uint32_t* __restrict__ counters, int M, int N, int K, int TG, int S, int per) {
  // X [M, K] e4m3fn and Xs [M, K / 128] fp32: the activations and their scales
  using Sh = WideShape<F, TJ>;
  constexpr int TT = Sh::TT, FH = Sh::FH;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ uint32_t last_flag;
  const int KB = K >> 7, NT = N >> 4;
  // id -> (weight slice q, token group tg): the groups of one slice are 8 ids apart
  const int id = static_cast<int>(blockIdx.x);
  const int q = (id / (8 * TG)) * 8 + id % 8, tg = (id / 8) % TG;
  if (q >= (NT / F) * S) return;  // padding ids of the last group of 8 slices
  const int tile = q / S, seg = q % S;
  const int kb0 = seg * per;
  const int n = KB - kb0 < per ? KB - kb0 : per;  // >= 1 (host plan)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tp = wave & 3, rh = wave >> 2;  // token fragments group, row split
  const int r = lane & 15, g = lane >> 4;
  const int t0 = 16 * TT * tg;        // first token of the group
  const int tf0 = TT * tg + TJ * tp;  // this wave's first token fragment
  const int f0 = rh * FH;             // this wave's first row fragment
  const int ops = wide_ops(F, TJ, wave);
  // Activations straight from x [M, K] (no image pass).  Piece p of the group (wave w copies
  // p = w + 8 u, u < TJ) is rows 8 (p % 2) .. +7 of token fragment p / 2: lane l copies
  // the 16-byte chunk c = (l % 8) ^ (l / 8) of row l / 8 of the K block, so each row's
  // 128 bytes are read by 8 lanes (coalesced) and land in LDS with chunk c of fragment row
  // q at 16 (c ^ (q % 8)) -- the swizzle keeps the fragment reads below free of bank
  // conflicts.  Rows past M repeat row M - 1; their tokens are never stored.
  const int arow = 8 * (wave & 1) + (lane >> 3);
  const int achunk = (lane & 7) ^ (lane >> 3);
  const uint8_t* xa[TJ];
#pragma unroll
  for (int u = 0; u < TJ; ++u)
    xa[u] = X + static_cast<size_t>(min(t0 + 16 * (4 * u + (wave >> 1)) + arow, M - 1)) * K + achunk * 16;
  // Token scales come in 16-block windows, double-buffered in LDS as [token][16] fp32:
  // copy u of wave w brings tokens 16 w + 4 u .. +3 of the group, 16 lanes (64 contiguous
  // bytes of x_s) per token; blocks past K repeat the row's last one.
  const int srow[4] = {min(t0 + 16 * wave + (lane >> 4), M - 1), min(t0 + 16 * wave + 4 + (lane >> 4), M - 1),
                       min(t0 + 16 * wave + 8 + (lane >> 4), M - 1), min(t0 + 16 * wave + 12 + (lane >> 4), M - 1)};
  const int sblk = lane & 15;
  const int fr = lane < F - 1 ? lane : F - 1;
  const float* ws_src = Bs + static_cast<size_t>((16 * (F * tile + fr)) >> 7) * KB;  // weight scales (wave 2)

  // this lane's weight pieces at K block 0 (a block's fragments lie a fixed offset further)
  constexpr int WPW = (2 * F + kWideWaves - 1) / kWideWaves;
  const uint8_t* wsrc[WPW];
#pragma unroll
  for (int u = 0; u < WPW; ++u) {
    const int p = wave + kWideWaves * u < 2 * F - 1 ? wave + kWideWaves * u : 2 * F - 1;
    wsrc[u] = B + packed_fragment(F * tile + (p >> 1), 0, NT) + (p & 1) * 1024 + lane * 16;
  }
  const uint32_t lds0 =
      __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_u8_ptr)smem)));

  // copies of K block kb into stage sidx
  auto issue = [&](int kb, int sidx) {
    const uint32_t ls = lds0 + sidx * Sh::STAGE;
    const size_t koff = (static_cast<size_t>(kb >> 2) * NT * kGroup + (kb & 3)) * 2048;
#pragma unroll
    for (int u = 0; u < WPW; ++u) {
      const int p = wave + kWideWaves * u;  // fragment p / 2, half p % 2
      if (p < 2 * F) dma_lds16(wsrc[u] + koff, ls + p * 1024);
    }
#pragma unroll
    for (int u = 0; u < TJ; ++u) dma_lds16(xa[u] + kb * 128, ls + Sh::W + (wave + 8 * u) * 1024);
    if (wave == 2) dma_lds4(ws_src + kb, ls + Sh::WS);
    if (wave < TT && ((kb & 15) == 0 || kb == kb0)) {  // the window of kb: a buffer last used 16 blocks ago
      const int b = (kb & ~15) + sblk < KB ? (kb & ~15) + sblk : KB - 1;
      const uint32_t win = lds0 + Sh::WIN + ((kb >> 4) & 1) * 8192 + wave * 1024;
#pragma unroll
      for (int u = 0; u < 4; ++u) dma_lds4(Xs + static_cast<size_t>(srow[u]) * KB + b, win + u * 256);
    }
  };
  // MFMA operand of a token fragment in the swizzled layout: lane (r, g) reads chunks g
  // and 4 + g of row r
  const int ao0 = r * 128 + ((g ^ (r & 7)) << 4), ao1 = r * 128 + (((4 + g) ^ (r & 7)) << 4);
  auto load_act = [&](const uint8_t* frag) {
    const uint4 lo = *reinterpret_cast<const uint4*>(frag + ao0);
    const uint4 hi = *reinterpret_cast<const uint4*>(frag + ao1);
    return v8i{static_cast<int>(lo.x), static_cast<int>(lo.y), static_cast<int>(lo.z), static_cast<int>(lo.w),
               static_cast<int>(hi.x), static_cast<int>(hi.y), static_cast<int>(hi.z), static_cast<int>(hi.w)};
  };

  v4f acc[FH][TJ];
#pragma unroll
  for (int f = 0; f < FH; ++f)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[f][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // Operands of one K block for rows f0 .. f0 + NR - 1, read from LDS into registers.
  // The loop is software-pipelined over two such sets: block i + 1's fragments are read
  // while block i's MFMAs run, so LDS reads and matrix work overlap.
  // OPS: this wave's copies per block, a compile-time constant in each specialisation so
  // that every wait is a single immediate s_waitcnt
  auto run = [&](auto nr_tag, auto ops_tag) {
    constexpr int NR = decltype(nr_tag)::value;
    constexpr int OPS = decltype(ops_tag)::value;
    struct Ops {
      v8i a[TJ], w[NR];
      float ts[TJ], ws[NR];
    };
    auto stage = [&](int i) { return smem + (i % Sh::STAGES) * Sh::STAGE; };
    auto last = [&](int i) { return kb0 + (i < n - 1 ? i : n - 1); };  // past the range: re-copy the last block
    auto load = [&](int i, Ops& o) {  // block kb0 + i (past the range: unused values)
      const uint8_t* st = stage(i);
      const int kb = kb0 + i;
#pragma unroll
      for (int j = 0; j < TJ; ++j) o.a[j] = load_act(st + Sh::W + (TJ * tp + j) * 2048);
#pragma unroll
      for (int f = 0; f < NR; ++f) o.w[f] = load_fragment(st + (f0 + f) * 2048, lane);
      const float* tsr = reinterpret_cast<const float*>(smem + Sh::WIN + ((kb >> 4) & 1) * 8192) +
                         (16 * TJ * tp + r) * 16 + (kb & 15);
      const float* wsr = reinterpret_cast<const float*>(st + Sh::WS) + f0;
#pragma unroll
      for (int j = 0; j < TJ; ++j) o.ts[j] = tsr[256 * j];
#pragma unroll
      for (int f = 0; f < NR; ++f) o.ws[f] = wsr[f];
    };
    // all MFMAs first, then the scaled accumulation (independent products issue back to back)
    auto mma = [&](const Ops& o) {
      v4f pr[NR][TJ];
#pragma unroll
      for (int f = 0; f < NR; ++f)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          pr[f][j] = mfma_16x16x128_fp8(o.w[f], o.a[j]);
#pragma unroll
      for (int f = 0; f < NR; ++f)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[f][j] += pr[f][j] * (o.ts[j] * o.ws[f]);
    };
    // Ring of SN stages.  Iteration i: wait for block i + 1's copies (this wave's; the
    // barrier then covers every wave's), read them into the other register set, copy
    // block i + SN - 1 into the stage block i - 1 used (its reads finished in iteration
    // i - 2), and multiply block i.  Each wave always has the same number of its copies in
    // flight, so the wait counts are fixed.
    constexpr int SN = Sh::STAGES;
    static_for<SN - 1>([&](auto j) { issue(last(decltype(j)::value), decltype(j)::value); });
    __builtin_amdgcn_s_waitcnt(vmcnt_imm((SN - 2) * OPS));  // block 0 landed
    asm volatile("s_barrier" ::: "memory");
    Ops o0, o1;
    load(0, o0);
    auto step = [&](int i, const Ops& cur, Ops& nxt) {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm((SN - 3) * OPS));  // block i + 1 landed (not i + 2 .. i + SN - 2)
      asm volatile("s_barrier" ::: "memory");
      issue(last(i + SN - 1), (i + SN - 1) % SN);
      load(i + 1, nxt);  // unconditional (past the range it reads a stage unused): no
      mma(cur);          // branch, so the wait for cur's reads stays partial
    };
    for (int i = 0; i < n; i += 2) {
      step(i, o0, o1);
      if (i + 1 < n) step(i + 1, o1, o0);
    }
  };
  // the wave's copy count takes one of at most three consecutive values (weight pieces
  // differ by one between waves, wave 2 adds the weight scales)
  constexpr int OPS_LO = wide_ops(F, TJ, kWideWaves - 1);
  static_assert(wide_ops(F, TJ, 0) <= OPS_LO + 1 && wide_ops(F, TJ, 2) <= OPS_LO + 2, "copy counts");
  auto by_ops = [&](auto nr_tag) {
    if (ops == OPS_LO) run(nr_tag, std::integral_constant<int, OPS_LO>{});
    else if (ops == OPS_LO + 1) run(nr_tag, std::integral_constant<int, OPS_LO + 1>{});
    else run(nr_tag, std::integral_constant<int, OPS_LO + 2>{});
  };
  if (rh == 0) by_ops(std::integral_constant<int, FH>{});
  else by_ops(std::integral_constant<int, F - FH>{});
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // no copy may land after the workgroup ends

  // lane holds rows 16 (F tile + f0 + f) + 4 g + (0..3) of token 16 (tf0 + j) + r
  const int nrows = rh == 0 ? FH : F - FH;
  auto token = [&](int j) { return 16 * (tf0 + j) + r; };
  auto column = [&](int f) { return 16 * (F * tile + f0 + f) + 4 * g; };
  auto store_all = [&]() {
#pragma unroll
    for (int f = 0; f < FH; ++f)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
        if (f < nrows && token(j) < M) store_out(out, token(j), column(f), pack_bf16x4(acc[f][j]));
  };
  if (S == 1) {
    store_all();
    return;
  }
  // partial of (tile, tg, seg): [row fragment][token fragment of the group][lane][4] fp32
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  const int slot_bytes = Sh::SLOT * 4;
  const size_t tile_slots = (static_cast<size_t>(tile) * TG + tg) * S;
  auto off = [&](int f, int j) { return (((f0 + f) * TT + TJ * tp + j) * 64 + lane) * 16; };
  {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(partial + (tile_slots + seg) * Sh::SLOT, 0, slot_bytes, kRsrcWord3);
#pragma unroll
    for (int f = 0; f < FH; ++f)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
        if (f < nrows)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4v, acc[f][j]), rs, off(f, j), 0, kCpolSc1);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0)
    last_flag = __hip_atomic_fetch_add(&counters[tile * TG + tg], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                static_cast<uint32_t>(S - 1);
  __syncthreads();
  if (!last_flag) return;
#pragma unroll
  for (int f = 0; f < FH; ++f)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[f][j] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int sq = 0; sq < S; ++sq) {  // ranges in K order
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(partial + (tile_slots + sq) * Sh::SLOT, 0, slot_bytes, kRsrcWord3);
#pragma unroll
    for (int f = 0; f < FH; ++f)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
        if (f < nrows)
          acc[f][j] += __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rs, off(f, j), 0, kCpolSc1));
  }
  store_all();
  if (tid == 0) __hip_atomic_store(&counters[tile * TG + tg], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Plan of the wide kernel: F (row tiles per workgroup, 4..9, dividing N / 16) and the K
// split S minimising rounds x F x (K blocks per range) -- the MFMA work of the busiest CU
// -- with at most 256 workgroups per round (token groups x tiles x S); ties go to fewer
// K ranges.  F = 0: no F divides N / 16.
struct WidePlan {
  int F, TJ, TG, S, per, tiles;
  int grid() const { return static_cast<int>(cdiv(static_cast<int64_t>(tiles) * S, 8)) * 8 * TG; }
};

__host__ inline WidePlan plan_wide(int64_t M, int64_t N, int64_t K) {
  const int NT = static_cast<int>(N / 16), KB = static_cast<int>(K / kBlock);
  const int TJ = cdiv(M, 16) <= 4 ? 1 : 2;
  const int TG = static_cast<int>(cdiv(cdiv(M, 16), 4 * TJ));
  WidePlan best{0, TJ, TG, 1, KB, 0};
  int64_t best_cost = INT64_MAX;
  for (int F = 9; F >= 4; --F) {
    if (NT % F) continue;
    const int tiles = NT / F;
    int S = std::max(1, std::min(KB, kWideGrid / (tiles * TG)));
    const int per = static_cast<int>(cdiv(KB, S));
    S = static_cast<int>(cdiv(KB, per));
    const int64_t cost = cdiv(static_cast<int64_t>(tiles) * TG * S, kWideGrid) * F * per * 16 + (S - 1);
    if (cost < best_cost) { best_cost = cost; best = WidePlan{F, TJ, TG, S, per, tiles}; }
  }
  return best;
}

__host__ inline size_t wide_partial_bytes(int64_t M, int64_t N, int64_t K) {
  const WidePlan w = plan_wide(M, N, K);
  if (w.S == 1) return 0;
  return static_cast<size_t>(w.tiles) * w.TG * w.S * w.F * 4 * w.TJ * 256 * sizeof(float);
}


struct GemmPlan {
  bool mm;     // packed weight, N % 128 = 0, M > 32 (or > 16, K split <= 4): fp8_gemm_wide_kernel
  bool tiled;  // M > 64, canonical weight: fp8_gemm_tiled_kernel
  int ksplit;
  int kb_per_split;
  int row_groups;  // grid.x: 16-row tiles (GEMV) or 128-row groups (tiled)
  int waves;
  int depth;  // GEMV operand buffers per wave
  int rt;     // GEMV row tiles per workgroup
  bool xf;    // GEMV reads the activation image (act_image_kernel) from the workspace
};

// K split.  GEMV (M <= 16): never split.  Measured on MI355X at every MLA, MLP and
// MoE-sized layer, the split's extra round trips (partial store, counter, reload: ~2 us)
// cost more than the extra CUs buy -- even a 36-tile layer, whose workgroups each stream
// 114 KB, is faster unsplit (5.6 vs 7.7 us).  M = 17..64: a layer of fewer than 192 row
// tiles splits K into cdiv(256, tiles) <= 4 slices of whole K groups (there the activation
// reads make a workgroup's work long enough for the split to pay); wider layers do not.
// Tiled (M > 64; measured faster than the per-row-tile kernel from M = 128 on, slower at
// M = 32 and 64): the smallest split giving >= 512 workgroups (2 per CU) with slices of
// at least 8 K blocks.
static GemmPlan plan_gemm(int64_t M, int64_t N, int64_t K, bool packed) {
  GemmPlan p;
  const int KB = static_cast<int>(K / kBlock);
  p.mm = packed && N % 128 == 0 && K % (kBlock * kGroup) == 0 &&
         (M > kWideMinM || (M > kWideMinM2 && plan_wide(M, N, K).S <= kWideMaxSplit2));
  p.tiled = M > 64 && !p.mm;
  p.depth = 2;
  p.rt = 1;
  p.xf = false;
  if (p.mm) {  // the wide kernel (N % 128 = 0: F = 8 always divides N / 16)
    p.row_groups = 0;
    p.ksplit = 1;
    p.kb_per_split = KB;
    p.waves = kWideWaves;
    p.xf = false;  // reads x [M, K] itself
    return p;
  }
  if (p.tiled) {
    p.row_groups = static_cast<int>(cdiv(N / 16, kTiledWaves));
    int s = static_cast<int>(cdiv(512, p.row_groups));
    s = std::max(1, std::min(s, KB / 8));
    p.kb_per_split = static_cast<int>(cdiv(KB, s));
    p.ksplit = static_cast<int>(cdiv(KB, p.kb_per_split));
    p.waves = kTiledWaves;
    return p;
  }
  const int groups = static_cast<int>(cdiv(KB, kGroup));
  p.row_groups = static_cast<int>(N / 16);
  int s = 1;
  if (M > 16 && p.row_groups < 192) s = std::max(1, std::min({4, groups, static_cast<int>(cdiv(256, p.row_groups))}));
  p.kb_per_split = static_cast<int>(cdiv(groups, s)) * kGroup;
  p.ksplit = static_cast<int>(cdiv(KB, p.kb_per_split));
  // unsplit layers: 8 waves (4 for K < 1024, where 8 would leave waves idle); split: 4
  p.waves = (p.ksplit == 1 && KB >= 8) ? 8 : kGroup;
  // long, wide GEMVs keep 4 K blocks in flight per wave (measured ~1% faster on the
  // 7168 x 18432 and 18432 x 7168 layers; no gain on narrow ones)
  if (M <= 16 && p.waves == 8 && KB >= 48 && p.row_groups >= 448) p.depth = 4;
  // From M = 5 on, each activation fragment serves 2 or 4 row tiles (measured: up
  // 7168 -> 18432 at M = 16 / 32 / 64: 33.2 -> 28.7 / 53.7 -> 40.8 / 103.7 -> 68.3 us; down
  // 18432 -> 7168 at M = 16 / 64: 35.2 -> 26.8 / 103.1 -> 59.8 us; at M = 4 it is 1 us
  // slower), keeping >= 192 workgroups; 4 row tiles only from M = 17 on (slower at 16).
  if (M > 4 && p.ksplit == 1 && p.waves == 8) {
    const int want = M > 16 ? 4 : 2;
    for (int rt = want; rt > 1; rt /= 2) {
      if (p.row_groups % rt == 0 && p.row_groups / rt >= 192) { p.rt = rt; break; }
    }
    if (p.rt > 1) p.depth = 2;
  }
  // The activation image costs a launch: measured worth it from M = 16 on (M = 16 up /
  // down: 28.7 -> 27.2 / 26.7 -> 25.9 us; M = 64: 68.4 -> 51.9 / 59.9 -> 43.0 us), not at
  // M = 8 (25.3 -> 27.7 us).
  p.xf = M > 16 || (M == 16 && p.rt == 2);
  return p;
}

// The workspace starts with a fixed counter region (one uint32 per 16-row tile, for
// every problem size) that stays all-zero between calls; fp32 partials follow it.  A
// fixed region keeps one problem's partials from ever landing on another's counters.
constexpr int kMaxRowTiles = kWsCounterTiles;  // N <= 262144
constexpr size_t kCounterBytes = kWsCounterBytes;

// Workspace: counters, then the split-K partials, then the activation image (256-aligned).

static size_t image_offset(const GemmPlan& p, int64_t M, int64_t N, int64_t K) {
  const size_t partial = p.mm ? wide_partial_bytes(M, N, K)
                              : (p.ksplit > 1 ? static_cast<size_t>(p.ksplit) * M * N * sizeof(float) : 0);
  return kCounterBytes + (partial + 255) / 256 * 256;
}

template <bool PACKED>
static int launch_gemm(const uint8_t* A, const float* As, const uint8_t* B, const float* Bs,
                       const OutRoute& out, int M, int N, int K, void* workspace, hipStream_t st) {
  const GemmPlan p = plan_gemm(M, N, K, PACKED);
  uint32_t* counters = p.ksplit > 1 ? static_cast<uint32_t*>(workspace) : nullptr;
  float* partial = p.ksplit > 1 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes) : nullptr;
  const dim3 grid(p.row_groups / p.rt, p.ksplit);
  const int per = p.kb_per_split;
  // From M = 16 on the activations are first rearranged into the workspace (act_image_kernel).
  const uint8_t* xa = A;
  const float* xsa = As;
  if (p.xf) {
    uint8_t* img = static_cast<uint8_t*>(workspace) + image_offset(p, M, N, K);
    const int64_t KB = K / kBlock, mtt = cdiv(M, 16);
    float* img_s = reinterpret_cast<float*>(img + KB * mtt * 2048);
    hipLaunchKernelGGL(act_image_kernel, dim3(static_cast<unsigned>(cdiv(KB * mtt * 128, 256))), dim3(256), 0, st,
                       A, As, img, img_s, M, K);
    xa = img;
    xsa = img_s;
  }
  if (p.mm) {
    uint32_t* cnt = static_cast<uint32_t*>(workspace);
    float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
    const WidePlan w = plan_wide(M, N, K);
    auto go = [&](auto f_tag, auto tj_tag) -> int {
      constexpr int F_ = decltype(f_tag)::value, TJ_ = decltype(tj_tag)::value;
      constexpr int lds = WideShape<F_, TJ_>::LDS;
      const void* fn = reinterpret_cast<const void*>(fp8_gemm_wide_kernel<F_, TJ_>);
      if (const int rc = allow_dynamic_lds(fn, lds, "fp8_gemm")) return rc;
      hipLaunchKernelGGL((fp8_gemm_wide_kernel<F_, TJ_>), dim3(w.grid()), dim3(kWideWaves * 64), lds, st, A, As, B,
                         Bs, out, part, cnt, M, N, K, w.TG, w.S, w.per);
      return check_launch("fp8_gemm");
    };
    auto go_f = [&](auto tj_tag) -> int {
      switch (w.F) {
        case 9: return go(std::integral_constant<int, 9>{}, tj_tag);
        case 8: return go(std::integral_constant<int, 8>{}, tj_tag);
        case 7: return go(std::integral_constant<int, 7>{}, tj_tag);
        case 6: return go(std::integral_constant<int, 6>{}, tj_tag);
        case 5: return go(std::integral_constant<int, 5>{}, tj_tag);
        default: return go(std::integral_constant<int, 4>{}, tj_tag);
      }
    };
    if (w.TJ == 1) return go_f(std::integral_constant<int, 1>{});
    return go_f(std::integral_constant<int, 2>{});
  }
  if (p.tiled) {
    auto launch = [&](auto tt_tag) -> int {
      constexpr int TT = decltype(tt_tag)::value;
      const void* fn = reinterpret_cast<const void*>(fp8_gemm_tiled_kernel<TT, PACKED>);
      if (tiled_lds_bytes<TT>() > 60 * 1024) {
        const int rc = allow_dynamic_lds(fn, tiled_lds_bytes<TT>(), "fp8_gemm");
        if (rc) return rc;
      }
      hipLaunchKernelGGL((fp8_gemm_tiled_kernel<TT, PACKED>), grid, dim3(kTiledWaves * 64), tiled_lds_bytes<TT>(), st,
                         A, As, B, Bs, out, partial, counters, M, N, K, per);
      return check_launch("fp8_gemm");
    };
    if (M <= 128) return launch(std::integral_constant<int, 8>{});
    return launch(std::integral_constant<int, 16>{});
  }
  auto gemv = [&](auto mt, auto w, auto d, auto rt, auto xf) {
    hipLaunchKernelGGL((fp8_gemm_kernel<decltype(mt)::value, decltype(w)::value, PACKED, decltype(d)::value,
                                        decltype(rt)::value, decltype(xf)::value>),
                       grid, dim3(decltype(w)::value * 64), 0, st, xa, xsa, B, Bs, out, partial, counters, M, N, K, per);
  };
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I4 = std::integral_constant<int, 4>;
  using I8 = std::integral_constant<int, 8>;
  using F = std::false_type;
  using T = std::true_type;
  // token tiles 2 or 4 (M > 16), with or without the activation image
  auto gemv_mt = [&](auto w, auto rt) {
    if (M <= 32) {
      if (p.xf) gemv(I2{}, w, I2{}, rt, T{}); else gemv(I2{}, w, I2{}, rt, F{});
    } else {
      if (p.xf) gemv(I4{}, w, I2{}, rt, T{}); else gemv(I4{}, w, I2{}, rt, F{});
    }
  };
  if (M <= 16) {
    if (p.rt == 2 && p.xf) gemv(I1{}, I8{}, I2{}, I2{}, T{});
    else if (p.rt == 2) gemv(I1{}, I8{}, I2{}, I2{}, F{});
    else if (p.depth == 4) gemv(I1{}, I8{}, I4{}, I1{}, F{});
    else if (p.waves == 8) gemv(I1{}, I8{}, I2{}, I1{}, F{});
    else gemv(I1{}, I4{}, I2{}, I1{}, F{});
  } else if (p.rt == 4) {
    gemv_mt(I8{}, I4{});
  } else if (p.rt == 2) {
    gemv_mt(I8{}, I2{});
  } else if (p.waves == 8) {
    gemv_mt(I8{}, I1{});
  } else {
    gemv_mt(I4{}, I1{});
  }
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

// ------------------------------------------------ q RMSNorm + wq_b on bf16 MFMA
// RmsnormProjqWqb (rmsnorm_projq_wqb.py:20-44, golden :496-512): qr = bf16(rms_norm(q) *
// weight) in fp32, then qr . dequant(wq_b)^T with the weight dequantised to bf16(fp32(w8) *
// scale) (the golden's bf16 ref_wq_b) on v_mfma_f32_16x16x32_bf16 with fp32 accumulation,
// written per head as q_nope [M, heads, nope] and q_pe [M, heads, rope].  One launch: every
// workgroup recomputes the M <= 16 normalised rows (wave w normalises rows w, w+4, ...)
// into LDS as bf16 -- a few KB from L2 -- then its 4 waves stream the packed weight
// fragments of one 16-row tile (K blocks w, w+4, ...), all loads issued up front.
constexpr int kPqWaves = 4;
constexpr int kPqMaxKb = 16;  // K <= 2048: at most 4 K blocks per wave

__global__ __launch_bounds__(kPqWaves * 64) void rmsnorm_projq_kernel(
    const uint16_t* __restrict__ q, const float* __restrict__ gamma, float eps, const uint8_t* __restrict__ B,
    const float* __restrict__ Bs, uint16_t* __restrict__ q_nope, uint16_t* __restrict__ q_pe, int M, int N, int K,
    int nope, int rope) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xl[];  // [M][K] normalised bf16 rows
  __shared__ v4f red[kPqWaves - 1][64];
  constexpr int KPW = kPqMaxKb / kPqWaves;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int KB = K >> 7, NT = N >> 4, t = blockIdx.x;
  // gamma and this wave's first row first (L2-resident: they land while the weight
  // fragments are in flight, so the norm below waits for them alone -- memory operations
  // complete in order); lane l holds elements 8 l + 512 i .. +7 (16-byte loads; chunks
  // past K reload chunk 0 and are not used)
  constexpr int CPL = kPqMaxKb * kBlock / 512;  // chunks per lane
  typedef uint32_t u32x4q __attribute__((ext_vector_type(4)));
  const int nch = K >> 9;
  auto chunk0 = [&](int i) { return i < nch ? 512 * i + 8 * lane : 8 * lane; };
  auto load_row = [&](int m, u32x4q (&xv)[CPL]) {
    const uint16_t* row = q + static_cast<size_t>(m) * K;
#pragma unroll
    for (int i = 0; i < CPL; ++i) xv[i] = *reinterpret_cast<const u32x4q*>(row + chunk0(i));
  };
  v4f g0[CPL], g1[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    g0[i] = *reinterpret_cast<const v4f*>(gamma + chunk0(i));
    g1[i] = *reinterpret_cast<const v4f*>(gamma + chunk0(i) + 4);
  }
  u32x4q xv[CPL];
  load_row(min(wave, M - 1), xv);
  __builtin_amdgcn_sched_barrier(0);  // issued ahead of the weight loads
  // this wave's weight fragments and scales (unconditional; blocks past K weigh 0)
  v8i wf[KPW];
  float ws[KPW];
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    const int kb = min(wave + i * kPqWaves, KB - 1);
    wf[i] = load_packed_fragment(B + packed_fragment(t, kb, NT), lane);
    ws[i] = wave + i * kPqWaves < KB ? Bs[static_cast<size_t>((16 * t) >> 7) * KB + kb] : 0.f;
  }
  __builtin_amdgcn_sched_barrier(0);
  // normalised rows: x * rsqrt(mean(x^2) + eps) * gamma in fp32, rounded to bf16
  for (int m = wave; m < M; m += kPqWaves) {
    if (m != wave) load_row(m, xv);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      if (i < nch) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = bf16_to_f32(xv[i][e] & 0xffffu), hi = bf16_to_f32(xv[i][e] >> 16);
          ss += lo * lo + hi * hi;
        }
      }
    }
    ss = wave_sum_f32(ss);
    const float rs = 1.0f / sqrtf(ss / static_cast<float>(K) + eps);
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      if (i < nch) {
        u32x4q o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float ga = e < 2 ? g0[i][2 * e] : g1[i][2 * e - 4], gb = e < 2 ? g0[i][2 * e + 1] : g1[i][2 * e - 3];
          o[e] = f32_to_bf16(bf16_to_f32(xv[i][e] & 0xffffu) * rs * ga) |
                 (static_cast<uint32_t>(f32_to_bf16(bf16_to_f32(xv[i][e] >> 16) * rs * gb)) << 16);
        }
        *reinterpret_cast<u32x4q*>(xl + m * K + 512 * i + 8 * lane) = o;
      }
    }
  }
  __syncthreads();
  // 16 weight rows x 16 tokens (rows past M repeat row M-1 and are not stored)
  const uint16_t* xrow = xl + min(r, M - 1) * K;
  v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    const int kb = min(wave + i * kPqWaves, KB - 1);
    const uint16_t* xk = xrow + kb * kBlock;
    const int off[4] = {16 * g, 16 * g + 8, 64 + 16 * g, 64 + 16 * g + 8};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const v8bf xa = *reinterpret_cast<const v8bf*>(xk + off[j]);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(dequant8_bf16(wf[i][2 * j], wf[i][2 * j + 1], ws[i]), xa, acc, 0, 0, 0);
    }
  }
  if (wave > 0) {
    red[wave - 1][lane] = acc;
  }
  __syncthreads();
  if (wave != 0 || r >= M) return;
#pragma unroll
  for (int w = 0; w < kPqWaves - 1; ++w)
    acc += red[w][lane];
  // features f .. f+3 of token r: head f / (nope + rope), inside one 16-wide tile
  const int f = 16 * t + 4 * g, hd = nope + rope;
  const int head = f / hd, d = f % hd;
  const int heads = N / hd;
  uint16_t* dst = d < nope ? q_nope + (static_cast<size_t>(r) * heads + head) * nope + d
                           : q_pe + (static_cast<size_t>(r) * heads + head) * rope + (d - nope);
  *reinterpret_cast<uint2*>(dst) = pack_bf16x4(acc);
}

}  // namespace tl

using namespace tl;

// Workspace bytes of one weight layout's plan (0 = none).
static size_t plan_workspace_bytes(int64_t M, int64_t N, int64_t K, bool packed) {
  const GemmPlan p = plan_gemm(M, N, K, packed);
  if (p.ksplit > 1 || p.xf || p.mm) return image_offset(p, M, N, K) + (p.xf ? act_image_bytes(M, K) : 0);
  return 0;
}

extern "C" size_t tl_fp8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || N % 16 || K % kBlock || M > 256) return 0;
  // one size serves both weight layouts
  return std::max(plan_workspace_bytes(M, N, K, false), plan_workspace_bytes(M, N, K, true));
}

extern "C" int tl_fp8_gemm(const void* a, const float* a_s, const void* b, const float* b_s,
                           void* c_bf16, int64_t M, int64_t N, int64_t K, void* workspace,
                           size_t workspace_bytes, void* stream) {
  const size_t need = tl_fp8_gemm_workspace_bytes(M, N, K);
  int rc = validate("fp8_gemm", a, a_s, b, b_s, c_bf16, M, N, K, workspace, workspace_bytes, need);
  if (rc) return rc;
  return launch_gemm<false>((const uint8_t*)a, a_s, (const uint8_t*)b, b_s, plain_out((uint16_t*)c_bf16, (int)N),
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
  return launch_gemm<true>((const uint8_t*)a, a_s, (const uint8_t*)b_packed, b_s, plain_out((uint16_t*)c_bf16, (int)N),
                           (int)M, (int)N, (int)K, workspace, (hipStream_t)stream);
}

extern "C" int tl_projx_wqkva(const void* x_q, const float* x_s, const void* w_packed,
                              const float* w_s, const int32_t* cur_pos, void* q_out, void* kv_out,
                              void* pe_cache, int64_t batch, int64_t seq, int64_t cache_rows,
                              int64_t dim, int64_t q_rank, int64_t kv_rank, int64_t rope_dim,
                              void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "projx_wqkva";
  if (batch <= 0 || seq <= 0 || cache_rows <= 0 || q_rank <= 0 || kv_rank <= 0 || rope_dim <= 0) {
    set_error("%s: batch, seq, cache rows and the three output widths must be positive", who);
    return kErrArg;
  }
  if (q_rank % kBlock || kv_rank % 16 || rope_dim % 16) {
    set_error("%s: q_rank must be a multiple of 128 and kv_rank, rope_dim of 16 (got %lld, %lld, %lld)", who,
              (long long)q_rank, (long long)kv_rank, (long long)rope_dim);
    return kErrArg;
  }
  if (dim % (kBlock * kGroup)) { set_error("%s: dim=%lld must be a multiple of 512", who, (long long)dim); return kErrArg; }
  const int64_t M = batch * seq, N = q_rank + kv_rank + rope_dim;
  if (M > 64) { set_error("%s: batch*seq=%lld > 64 is not supported (decode GEMV)", who, (long long)M); return kErrUnsupported; }
  if (!cur_pos || !kv_out || !pe_cache) { set_error("%s: null pointer", who); return kErrArg; }
  if ((reinterpret_cast<uintptr_t>(kv_out) | reinterpret_cast<uintptr_t>(pe_cache)) & 7) {
    set_error("%s: outputs must be 8-byte aligned", who);
    return kErrArg;
  }
  if (cache_rows > (1ll << 30) / rope_dim) { set_error("%s: cache too large", who); return kErrArg; }
  const size_t need = tl_fp8_gemm_workspace_bytes(M, N, dim);
  int rc = validate(who, x_q, x_s, w_packed, w_s, q_out, M, N, dim, workspace, workspace_bytes, need);
  if (rc) return rc;
  OutRoute out{(uint16_t*)q_out, (uint16_t*)kv_out, (uint16_t*)pe_cache, (int)q_rank, (int)(q_rank + kv_rank),
               (int)q_rank, (int)kv_rank, (int)rope_dim, cur_pos, (int)seq, (int)cache_rows};
  return launch_gemm<true>((const uint8_t*)x_q, x_s, (const uint8_t*)w_packed, w_s, out, (int)M, (int)N,
                           (int)dim, workspace, (hipStream_t)stream);
}

extern "C" int tl_rmsnorm_projq_wqb(const void* q_bf16, const float* q_norm_weight, float eps, const void* wq_b_packed,
                                    const float* wq_b_s, void* q_nope_bf16, void* q_pe_bf16, int64_t M, int64_t heads,
                                    int64_t q_rank, int64_t nope_dim, int64_t rope_dim, void* stream) {
  const int64_t N = heads * (nope_dim + rope_dim), K = q_rank;
  if (M < 1 || M > 16) { set_error("rmsnorm_projq_wqb: M=%lld must be in [1, 16]", (long long)M); return kErrUnsupported; }
  // rope_dim = 0: every feature goes to q_nope (rmsnorm_proj_qi_op's single output)
  if (heads < 1 || nope_dim <= 0 || rope_dim < 0 || nope_dim % 16 || rope_dim % 16) {
    set_error("rmsnorm_projq_wqb: heads=%lld, nope=%lld, rope=%lld (dims must be positive multiples of 16)",
              (long long)heads, (long long)nope_dim, (long long)rope_dim);
    return kErrArg;
  }
  if (K % (kBlock * kGroup) || K > kPqMaxKb * kBlock) { set_error("rmsnorm_projq_wqb: q_rank=%lld must be a multiple of 512 and <= %d", (long long)K, kPqMaxKb * kBlock); return kErrUnsupported; }
  if (!q_bf16 || !q_norm_weight || !wq_b_packed || !wq_b_s || !q_nope_bf16 || (rope_dim > 0 && !q_pe_bf16)) { set_error("rmsnorm_projq_wqb: null pointer"); return kErrArg; }
  if ((reinterpret_cast<uintptr_t>(q_bf16) | reinterpret_cast<uintptr_t>(wq_b_packed)) & 15 ||
      (reinterpret_cast<uintptr_t>(q_nope_bf16) | reinterpret_cast<uintptr_t>(q_pe_bf16)) & 7) {
    set_error("rmsnorm_projq_wqb: q and the weight must be 16-byte aligned, outputs 8-byte aligned");
    return kErrArg;
  }
  const size_t lds = static_cast<size_t>(M) * K * 2;
  if (lds > 48 * 1024) {
    if (int rc = allow_dynamic_lds(reinterpret_cast<const void*>(rmsnorm_projq_kernel), static_cast<int>(lds), "rmsnorm_projq_wqb"))
      return rc;
  }
  hipLaunchKernelGGL(rmsnorm_projq_kernel, dim3(static_cast<unsigned>(N / 16)), dim3(kPqWaves * 64), lds, (hipStream_t)stream,
                     (const uint16_t*)q_bf16, q_norm_weight, eps, (const uint8_t*)wq_b_packed, wq_b_s, (uint16_t*)q_nope_bf16,
                     (uint16_t*)q_pe_bf16, (int)M, (int)N, (int)K, (int)nope_dim, (int)rope_dim);
  return check_launch("rmsnorm_projq_wqb");
}

// ------------------------------------------ allocation-free entry point (static scratch)
// tl_fp8_gemm_packed_static runs tl_fp8_gemm_packed's kernels with their scratch (the
// split-K counters, fp32 partials and the activation image) in a file-scope device array
// instead of a caller-passed workspace, for callers that cannot allocate device memory.
// Each GPU holds its own copy of the array for the life of the process.  In host code
// `scratch` names a host-side stand-in, never the device memory: its per-device address
// comes from hipGetSymbolAddress (with that device current) and only that address is
// passed to kernels.
static_assert(TL_FP8_GEMM_STATIC_SCRATCH_BYTES % 256 == 0, "scratch size");
static __device__ __align__(256) uint8_t scratch[TL_FP8_GEMM_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};  // device address of each device's `scratch`

// The current device's scratch address, looked up on the device's first call.  The array
// is zero-initialised when the code object is loaded (device globals have static storage),
// and every call leaves its counter region zero again, so no call needs to clear it: two
// threads making their first calls on different streams cannot see an uncleared array, and
// a first call made under graph capture records nothing extra.
int scratch_for_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) { set_error("fp8_gemm_packed_static: hipGetDevice failed: %s", hipGetErrorString(e)); return kErrHip; }
  if (dev < 0 || dev >= kMaxDevices) { set_error("fp8_gemm_packed_static: device %d out of range", dev); return kErrUnsupported; }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      set_error("fp8_gemm_packed_static: hipGetSymbolAddress failed on device %d: %s", dev, hipGetErrorString(e));
      return kErrHip;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return kOk;
}

}  // namespace

extern "C" int tl_fp8_gemm_packed_static(const void* a, const float* a_s, const void* b_packed, const float* b_s,
                                         void* c_bf16, int64_t M, int64_t N, int64_t K, void* stream) {
  const char* who = "fp8_gemm_packed_static";
  if (K % (kBlock * kGroup)) { set_error("%s: K=%lld must be a multiple of 512", who, (long long)K); return kErrArg; }
  int rc = validate(who, a, a_s, b_packed, b_s, c_bf16, M, N, K, nullptr, 0, 0);
  if (rc) return rc;
  const size_t need = plan_workspace_bytes(M, N, K, true);
  if (need > TL_FP8_GEMM_STATIC_SCRATCH_BYTES) {
    set_error("%s: M=%lld N=%lld K=%lld needs %zu bytes of scratch, above the static maximum of %zu", who,
              (long long)M, (long long)N, (long long)K, need, static_cast<size_t>(TL_FP8_GEMM_STATIC_SCRATCH_BYTES));
    return kErrUnsupported;
  }
  void* ws = nullptr;
  if (need) {
    rc = scratch_for_current_device(&ws);
    if (rc) return rc;
  }
  return launch_gemm<true>((const uint8_t*)a, a_s, (const uint8_t*)b_packed, b_s, plain_out((uint16_t*)c_bf16, (int)N),
                           (int)M, (int)N, (int)K, ws, (hipStream_t)stream);
}

extern "C" int tl_projx_wqaki(const void* x_q, const float* x_s, const void* w_packed, const float* w_s, void* q_out,
                              void* ki_out, int64_t M, int64_t dim, int64_t q_rank, int64_t ki_dim, void* workspace,
                              size_t workspace_bytes, void* stream) {
  const char* who = "projx_wqaki";
  if (M <= 0 || q_rank <= 0 || ki_dim <= 0) { set_error("%s: M and the output widths must be positive", who); return kErrArg; }
  if (q_rank % kBlock || ki_dim % 16) {
    set_error("%s: q_rank must be a multiple of 128 and ki_dim of 16 (got %lld, %lld)", who, (long long)q_rank, (long long)ki_dim);
    return kErrArg;
  }
  if (dim % (kBlock * kGroup)) { set_error("%s: dim=%lld must be a multiple of 512", who, (long long)dim); return kErrArg; }
  if (M > 64) { set_error("%s: M=%lld > 64 is not supported (decode GEMV)", who, (long long)M); return kErrUnsupported; }
  if (!ki_out) { set_error("%s: null pointer", who); return kErrArg; }
  if (reinterpret_cast<uintptr_t>(ki_out) & 7) { set_error("%s: outputs must be 8-byte aligned", who); return kErrArg; }
  const int64_t N = q_rank + ki_dim;
  const size_t need = tl_fp8_gemm_workspace_bytes(M, N, dim);
  int rc = validate(who, x_q, x_s, w_packed, w_s, q_out, M, N, dim, workspace, workspace_bytes, need);
  if (rc) return rc;
  // two output segments: columns [0, q_rank) -> q_out, the rest -> ki_out
  OutRoute out{(uint16_t*)q_out, (uint16_t*)ki_out, nullptr, (int)q_rank, (int)N, (int)q_rank, (int)ki_dim, 0, nullptr, 1, 0};
  return launch_gemm<true>((const uint8_t*)x_q, x_s, (const uint8_t*)w_packed, w_s, out, (int)M, (int)N, (int)dim,
                           workspace, (hipStream_t)stream);
}
