// Exact per-row top-k by radix select (the contract of topk_accurate_op, ops/topk.py:62-109;
// its golden is torch.topk, :128-143), as ONE kernel.
//
// Scores map to order-preserving 32-bit keys (larger score = larger key).  A row is cut
// into 16K-column chunks, one 1024-thread workgroup each, which load their keys once and
// keep them in registers.  Three passes find the k-th largest key T digit by digit (11,
// 11, 10 bits): each workgroup histograms its chunk's keys that match the prefix found
// so far in LDS and publishes the histogram (agent-scope stores); the row's workgroups
// meet at a per-row barrier; then EVERY workgroup merges all partials (so no second
// barrier is needed), picks the same digit, and accumulates how many elements of the
// chunks before its own are now known to be > T (and, after the last pass, == T).  It
// then writes its selected columns -- every key > T plus the lowest-column keys == T
// until k are taken -- in ascending column order at their global rank.  The set is exact
// and deterministic, ties included.
//
// The per-row barrier needs the row's workgroups co-resident: the launch is at most one
// workgroup per CU (<= 256 workgroups, checked on the host) and the kernel is the only
// work on its stream; the wait is bounded (about a second) so a wave can never hang.
//
// Rows are the topk_accurate samples: row i considers columns [0, valid_base + 1 + i).

#include "common.h"
#include "../../include/tilert_amd.h"

namespace tl {

constexpr int kTkThreads = 1024;
constexpr int kTkPerThread = 16;                      // 4 float4 loads in flight per thread
constexpr int kTkChunk = kTkThreads * kTkPerThread;   // 16384 columns per workgroup
constexpr int kBins = 2048;                           // widest digit: 11 bits
constexpr int kMaxK = 8192;
// every workgroup keeps all chunks' partial histograms of a pass in LDS: 16 x 8 KB
constexpr int kMaxChunks = 16;
constexpr int kMaxCols = kMaxChunks * kTkChunk;  // 262144
constexpr int kMaxGroups = 256;                  // one workgroup per CU at most
constexpr uint32_t kSpinLimit = 1u << 22;        // x s_sleep(8): ~1 s

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct TopkWs {
  uint32_t* part;     // [rows][3 passes][chunks][kBins] partial histograms
  uint32_t* arrive;   // [rows] barrier arrivals, zero between calls
  uint32_t* leave;    // [rows] finished workgroups, zero between calls
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

__host__ __device__ inline TopkWs carve(void* base, int64_t rows) {
  char* p = static_cast<char*>(base);
  TopkWs w;
  w.arrive = reinterpret_cast<uint32_t*>(p);
  p += align256(rows * sizeof(uint32_t));
  w.leave = reinterpret_cast<uint32_t*>(p);
  p += align256(rows * sizeof(uint32_t));
  w.part = reinterpret_cast<uint32_t*>(p);
  return w;
}

__device__ inline uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ inline int row_valid(int row, int64_t valid_base, int64_t ld) {
  int64_t n = valid_base + 1 + row;
  if (n < 0) n = 0;
  if (n > ld) n = ld;
  return static_cast<int>(n);
}

// The 16 keys of this thread's contiguous columns [c0, c0 + 16); invalid ones flagged.
__device__ inline void load_keys(const float* __restrict__ src, int64_t c0, int n, uint32_t (&key)[kTkPerThread],
                                 uint32_t& valid_mask) {
  valid_mask = 0;
  if (c0 + kTkPerThread <= n) {
    f32x4 v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = *reinterpret_cast<const f32x4*>(src + c0 + 4 * i);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) key[4 * i + j] = order_key(v[i][j]);
    valid_mask = 0xffffu;
  } else {
#pragma unroll
    for (int i = 0; i < kTkPerThread; ++i) {
      const bool ok = c0 + i < n;
      key[i] = ok ? order_key(src[c0 + i]) : 0u;
      valid_mask |= ok ? (1u << i) : 0u;
    }
  }
}

// Block-wide exclusive prefix sum over the 1024 threads (returns the block total too).
__device__ inline uint32_t block_excl_scan(uint32_t v, uint32_t* s_waves, uint32_t& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) s_waves[wave] = x;
  __syncthreads();
  uint32_t before = 0;
  total = 0;
#pragma unroll
  for (int w = 0; w < kTkThreads / 64; ++w) {
    const uint32_t s = s_waves[w];
    before += w < wave ? s : 0u;
    total += s;
  }
  __syncthreads();
  return before + x - v;
}

__device__ inline uint32_t block_sum(uint32_t v, uint32_t* s_waves) {
  uint32_t total;
  block_excl_scan(v, s_waves, total);
  return total;
}

__global__ __launch_bounds__(kTkThreads) void topk_kernel(const float* __restrict__ logits, int64_t ld,
                                                          int64_t valid_base, int k, TopkWs ws,
                                                          int32_t* __restrict__ out) {
  extern __shared__ uint32_t plds[];  // [chunks][nb]: every chunk's partial of this pass
  __shared__ uint32_t h[kBins];
  __shared__ uint32_t s_waves[kTkThreads / 64];
  __shared__ uint32_t s_digit, s_above;
  const int row = blockIdx.y;
  const int chunks = gridDim.x, chunk = blockIdx.x;
  const int n = row_valid(row, valid_base, ld);
  int32_t* o = out + static_cast<int64_t>(row) * k;
  if (n <= k) {  // every valid column, then -1 padding (no barrier: the whole row exits)
    const int64_t base = static_cast<int64_t>(chunk) * kTkChunk;
    for (int64_t c = base + threadIdx.x; c < base + kTkChunk && c < k; c += kTkThreads)
      o[c] = c < n ? static_cast<int32_t>(c) : -1;
    return;
  }

  const float* src = logits + static_cast<int64_t>(row) * ld;
  const int64_t c0 = static_cast<int64_t>(chunk) * kTkChunk + static_cast<int64_t>(threadIdx.x) * kTkPerThread;
  uint32_t key[kTkPerThread], vm;
  load_keys(src, c0, n, key, vm);

  uint32_t prefix = 0;
  int k_rem = k;
  uint32_t gt_before = 0, eq_before = 0;  // over the chunks preceding this one
  for (int pass = 0; pass < 3; ++pass) {
    const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
    const int width = pass == 2 ? 10 : 11;
    const uint32_t nb = 1u << width;
    for (uint32_t b = threadIdx.x; b < nb; b += kTkThreads) h[b] = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kTkPerThread; ++i) {
      const bool match = ((vm >> i) & 1u) && (pass == 0 || (key[i] >> (shift + width)) == prefix);
      if (match) atomicAdd(&h[(key[i] >> shift) & (nb - 1)], 1u);
    }
    __syncthreads();
    uint32_t* part = ws.part + (static_cast<size_t>(row) * 3 + pass) * chunks * kBins;
    for (uint32_t b = threadIdx.x; b < nb; b += kTkThreads)
      __hip_atomic_store(&part[static_cast<size_t>(chunk) * kBins + b], h[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // ---- per-row barrier (bounded wait)
    if (threadIdx.x == 0) {
      __hip_atomic_fetch_add(&ws.arrive[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t target = static_cast<uint32_t>(chunks) * (pass + 1);
      for (uint32_t it = 0; it < kSpinLimit; ++it) {
        if (__hip_atomic_load(&ws.arrive[row], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target) break;
        __builtin_amdgcn_s_sleep(8);
      }
    }
    __syncthreads();
    // ---- merge every chunk's partial (batched agent-scope loads) into LDS
    for (uint32_t b = threadIdx.x; b < nb; b += kTkThreads) {
      uint32_t s = 0;
      for (int cg = 0; cg < chunks; cg += 16) {
        uint32_t v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int c = cg + u < chunks ? cg + u : chunks - 1;
          v[u] = __hip_atomic_load(&part[static_cast<size_t>(c) * kBins + b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int u = 0; u < 16; ++u)
          if (cg + u < chunks) {
            plds[(cg + u) * nb + b] = v[u];
            s += v[u];
          }
      }
      h[b] = s;
    }
    __syncthreads();
    // ---- the digit holding the k_rem-th largest: thread j owns digits
    // [nb - (j+1)*per, nb - j*per), i.e. descending order across threads
    const uint32_t per = nb / kTkThreads;  // 2 or 1
    const uint32_t hi = nb - threadIdx.x * per;
    uint32_t own = 0;
    for (uint32_t b = hi - per; b < hi; ++b) own += h[b];
    uint32_t total;
    const uint32_t above_me = block_excl_scan(own, s_waves, total);
    if (above_me < static_cast<uint32_t>(k_rem) && above_me + own >= static_cast<uint32_t>(k_rem)) {
      uint32_t above = above_me;
      uint32_t d = hi - 1;
      for (;; --d) {
        if (above + h[d] >= static_cast<uint32_t>(k_rem)) break;
        above += h[d];
      }
      s_digit = d;
      s_above = above;
    }
    __syncthreads();
    const uint32_t d = s_digit;
    // elements of the preceding chunks now known to be > T (digit above d)
    uint32_t g = 0;
    for (int i = threadIdx.x; i < chunk * static_cast<int>(nb); i += kTkThreads) {
      const uint32_t b = static_cast<uint32_t>(i) & (nb - 1);
      g += b > d ? plds[i] : 0u;
    }
    gt_before += block_sum(g, s_waves);
    if (pass == 2) {
      uint32_t e = 0;
      for (int c = threadIdx.x; c < chunk; c += kTkThreads) e += plds[c * nb + d];
      eq_before = block_sum(e, s_waves);
    }
    prefix = (prefix << width) | d;
    k_rem -= static_cast<int>(s_above);
    __syncthreads();
  }

  // ---- emit this chunk's selected columns in ascending order at their global rank
  const uint32_t T = prefix;
  const uint32_t need_eq = static_cast<uint32_t>(k_rem);
  uint32_t n_eq = 0;
#pragma unroll
  for (int i = 0; i < kTkPerThread; ++i) n_eq += ((vm >> i) & 1u) && key[i] == T;
  uint32_t tot;
  uint32_t eq_rank = eq_before + block_excl_scan(n_eq, s_waves, tot);
  uint32_t sel_bits = 0;
#pragma unroll
  for (int i = 0; i < kTkPerThread; ++i) {
    const bool valid = (vm >> i) & 1u;
    const bool eq = valid && key[i] == T;
    const bool sel = (valid && key[i] > T) || (eq && eq_rank < need_eq);
    eq_rank += eq;
    sel_bits |= sel ? (1u << i) : 0u;
  }
  const uint32_t sel_base = gt_before + (eq_before < need_eq ? eq_before : need_eq);
  uint32_t pos = sel_base + block_excl_scan(__builtin_popcount(sel_bits), s_waves, tot);
#pragma unroll
  for (int i = 0; i < kTkPerThread; ++i)
    if ((sel_bits >> i) & 1u) o[pos++] = static_cast<int32_t>(c0 + i);

  // ---- the last workgroup of the row out re-arms the barrier counters
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&ws.leave[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == static_cast<uint32_t>(chunks - 1)) {
      __hip_atomic_store(&ws.arrive[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&ws.leave[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace tl

using namespace tl;

static int64_t topk_chunks(int64_t ld) { return cdiv(ld, kTkChunk); }

extern "C" size_t tl_topk_workspace_bytes(int64_t rows, int64_t ld, int64_t k) {
  (void)k;
  if (rows <= 0 || ld <= 0) return 0;
  const int64_t chunks = topk_chunks(ld);
  return 2 * align256(rows * 4) + align256(static_cast<size_t>(rows) * 3 * chunks * kBins * 4);
}

extern "C" int tl_topk_rows(const float* logits, int64_t rows, int64_t ld, int64_t valid_base, int64_t k,
                            int32_t* out, void* workspace, size_t workspace_bytes, void* stream) {
  if (rows <= 0 || ld <= 0) { set_error("topk: empty input (rows=%lld ld=%lld)", (long long)rows, (long long)ld); return kErrArg; }
  if (k < 1 || k > kMaxK) { set_error("topk: k=%lld must be in [1, %d]", (long long)k, kMaxK); return kErrUnsupported; }
  if (ld > kMaxCols) { set_error("topk: ld=%lld > %d columns is not supported", (long long)ld, kMaxCols); return kErrUnsupported; }
  if (ld % 4) { set_error("topk: ld=%lld must be a multiple of 4 (16-byte rows)", (long long)ld); return kErrArg; }
  const int64_t chunks = topk_chunks(ld);
  if (rows * chunks > kMaxGroups) { set_error("topk: rows * ceil(ld/16384) = %lld exceeds %d co-resident workgroups", (long long)(rows * chunks), kMaxGroups); return kErrUnsupported; }
  if (!logits || !out) { set_error("topk: null pointer"); return kErrArg; }
  if (reinterpret_cast<uintptr_t>(logits) & 15) { set_error("topk: logits must be 16-byte aligned"); return kErrArg; }
  const size_t need = tl_topk_workspace_bytes(rows, ld, k);
  if (!workspace || workspace_bytes < need) { set_error("topk: workspace of %zu bytes required (got %zu)", need, workspace_bytes); return kErrArg; }
  const TopkWs ws = carve(workspace, rows);
  const size_t lds = static_cast<size_t>(chunks) * kBins * sizeof(uint32_t);
  const int rc = allow_dynamic_lds(reinterpret_cast<const void*>(topk_kernel), kMaxChunks * kBins * static_cast<int>(sizeof(uint32_t)), "topk");
  if (rc) return rc;
  hipLaunchKernelGGL(topk_kernel, dim3(static_cast<unsigned>(chunks), static_cast<unsigned>(rows)), dim3(kTkThreads),
                     lds, (hipStream_t)stream, logits, ld, valid_base, (int)k, ws, out);
  return check_launch("topk");
}
