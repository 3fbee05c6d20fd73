// Exact per-row top-k (the contract of topk_accurate_op, ops/topk.py:62-109; its golden
// is torch.topk, :128-143), as ONE kernel with one cross-workgroup barrier and one handoff.
//
// Scores map to order-preserving 32-bit keys (larger score = larger key).  A row is cut
// into 16K-column chunks, one 1024-thread workgroup each, which load their keys once and
// keep them in registers (16 contiguous columns per thread).
//   Stage 1 (every chunk): a histogram of the keys' top 11 bits in LDS, published with
//     agent-scope stores; the row's chunks meet at a barrier (bounded spin), every chunk
//     sums all partials and finds the digit d0 holding the row's k-th largest key and how
//     many keys lie above it.  Each chunk then publishes its keys with digit >= d0 -- the
//     only ones that can be selected -- as (key, column) pairs in ascending column order
//     (typically ~2k per row in all).
//   Stage 2 (the row's last chunk to finish, found with an agent-scope counter): two more
//     radix passes (11 and 10 bits) over the candidates of digit d0 give the k-th largest
//     key T; every candidate > T plus the lowest-column candidates == T until k are taken
//     are written in ascending column order.  Candidates stay in registers when they fit
//     (<= 8 per thread); otherwise they are streamed in batches, so any input is exact.
// The set is exact and deterministic, ties included.  Two radix rounds that needed a
// cross-workgroup exchange each are replaced by workgroup-local passes over the few
// candidates: measured on MI355X, each exchange round costs several microseconds.
//
// The barrier needs the row's workgroups co-resident: the launch is at most one workgroup
// per CU (<= 256 workgroups, checked on the host) and the kernel is the only work on its
// stream; the wait is bounded (about a second) so a wave can never hang.
//
// Rows are the topk_accurate samples: row i considers columns [0, valid_base + 1 + i).

#include "common.h"
#include "../../include/tilert_amd.h"

namespace tl {

constexpr int kTkThreads = 1024;
constexpr int kTkPerThread = 16;                      // 4 float4 loads per thread
constexpr int kTkChunk = kTkThreads * kTkPerThread;   // 16384 columns per workgroup
constexpr int kBins = 2048;                           // widest digit: 11 bits
constexpr int kMaxK = 8192;
constexpr int kMaxChunks = 16;
constexpr int kMaxCols = kMaxChunks * kTkChunk;       // 262144
constexpr int kMaxGroups = 256;                       // one workgroup per CU at most
constexpr int kCandPerThread = 8;                     // stage-2 register batch per thread
constexpr int kCandBatch = kTkThreads * kCandPerThread;
constexpr uint32_t kSpinLimit = 1u << 22;             // x s_sleep(8): ~1 s

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct TopkWs {
  uint32_t* arrive;  // [rows] barrier arrivals, zero between calls
  uint32_t* done;    // [rows] chunks finished with stage 1, zero between calls
  uint32_t* count;   // [rows][chunks] candidates published per chunk
  uint32_t* part;    // [rows][chunks][kBins] pass-0 partial histograms
  uint64_t* cand;    // [rows][chunks][kTkChunk] (key << 32 | column)
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

__host__ __device__ inline TopkWs carve(void* base, int64_t rows, int64_t chunks) {
  char* p = static_cast<char*>(base);
  TopkWs w;
  w.arrive = reinterpret_cast<uint32_t*>(p);
  p += align256(rows * sizeof(uint32_t));
  w.done = reinterpret_cast<uint32_t*>(p);
  p += align256(rows * sizeof(uint32_t));
  w.count = reinterpret_cast<uint32_t*>(p);
  p += align256(rows * chunks * sizeof(uint32_t));
  w.part = reinterpret_cast<uint32_t*>(p);
  p += align256(rows * chunks * kBins * sizeof(uint32_t));
  w.cand = reinterpret_cast<uint64_t*>(p);
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

struct TopkShared {
  uint32_t h[kBins];
  uint32_t waves[kTkThreads / 64];
  uint32_t digit, above, flag;
  uint32_t offs[kMaxChunks + 1];
};

// The digit (of nb bins, histogram in sh.h) holding the k_rem-th largest key, and how
// many keys lie in the digits above it.  Thread j owns digits [nb - (j+1)*per, nb - j*per),
// i.e. descending order across threads; one block scan finds the owner.
__device__ inline void find_digit(uint32_t nb, uint32_t k_rem, TopkShared& sh, uint32_t& digit, uint32_t& above) {
  const uint32_t per = nb / kTkThreads;  // 2 or 1
  const uint32_t hi = nb - threadIdx.x * per;
  uint32_t own = 0;
  for (uint32_t b = hi - per; b < hi; ++b) own += sh.h[b];
  uint32_t total;
  const uint32_t above_me = block_excl_scan(own, sh.waves, total);
  if (above_me < k_rem && above_me + own >= k_rem) {
    uint32_t a = above_me;
    uint32_t d = hi - 1;
    for (;; --d) {
      if (a + sh.h[d] >= k_rem) break;
      a += sh.h[d];
    }
    sh.digit = d;
    sh.above = a;
  }
  __syncthreads();
  digit = sh.digit;
  above = sh.above;
  __syncthreads();
}

__global__ __launch_bounds__(kTkThreads) void topk_kernel(const float* __restrict__ logits, int64_t ld,
                                                          int64_t valid_base, int k, TopkWs ws,
                                                          int32_t* __restrict__ out) {
  __shared__ TopkShared sh;
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

  // ---- stage 1: this chunk's keys (16 contiguous columns per thread)
  const float* src = logits + static_cast<int64_t>(row) * ld;
  const int64_t c0 = static_cast<int64_t>(chunk) * kTkChunk + static_cast<int64_t>(threadIdx.x) * kTkPerThread;
  uint32_t key[kTkPerThread], vm = 0;
  if (c0 + kTkPerThread <= n) {
    f32x4 v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = *reinterpret_cast<const f32x4*>(src + c0 + 4 * i);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) key[4 * i + j] = order_key(v[i][j]);
    vm = 0xffffu;
  } else {
#pragma unroll
    for (int i = 0; i < kTkPerThread; ++i) {
      const bool ok = c0 + i < n;
      key[i] = ok ? order_key(src[c0 + i]) : 0u;
      vm |= ok ? (1u << i) : 0u;
    }
  }
  for (uint32_t b = threadIdx.x; b < kBins; b += kTkThreads) sh.h[b] = 0;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kTkPerThread; ++i)
    if ((vm >> i) & 1u) atomicAdd(&sh.h[key[i] >> 21], 1u);
  __syncthreads();
  uint32_t* part = ws.part + static_cast<size_t>(row) * chunks * kBins;
  for (uint32_t b = threadIdx.x; b < kBins; b += kTkThreads)
    __hip_atomic_store(&part[static_cast<size_t>(chunk) * kBins + b], sh.h[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // per-row barrier (bounded wait)
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(&ws.arrive[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (uint32_t it = 0; it < kSpinLimit; ++it) {
      if (__hip_atomic_load(&ws.arrive[row], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= static_cast<uint32_t>(chunks)) break;
      __builtin_amdgcn_s_sleep(8);
    }
  }
  __syncthreads();
  // every chunk's partial summed (batched agent-scope loads)
  for (uint32_t b = threadIdx.x; b < kBins; b += kTkThreads) {
    uint32_t v[kMaxChunks];
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c)
      v[c] = __hip_atomic_load(&part[static_cast<size_t>(c < chunks ? c : chunks - 1) * kBins + b], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    uint32_t s = 0;
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) s += c < chunks ? v[c] : 0u;
    sh.h[b] = s;
  }
  __syncthreads();
  uint32_t d0, above0;
  find_digit(kBins, static_cast<uint32_t>(k), sh, d0, above0);

  // candidates: keys with digit >= d0, compacted in ascending column order
  uint32_t cbits = 0;
#pragma unroll
  for (int i = 0; i < kTkPerThread; ++i) cbits |= (((vm >> i) & 1u) && (key[i] >> 21) >= d0) ? (1u << i) : 0u;
  uint32_t n_cand;
  uint32_t pos = block_excl_scan(__builtin_popcount(cbits), sh.waves, n_cand);
  uint64_t* cand = ws.cand + (static_cast<size_t>(row) * chunks + chunk) * kTkChunk;
#pragma unroll
  for (int i = 0; i < kTkPerThread; ++i)
    if ((cbits >> i) & 1u) {
      const uint64_t v = (static_cast<uint64_t>(key[i]) << 32) | static_cast<uint32_t>(c0 + i);
      __hip_atomic_store(cand + pos++, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  if (threadIdx.x == 0)
    __hip_atomic_store(&ws.count[row * chunks + chunk], n_cand, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);  // this chunk's candidates are complete before it reports
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&ws.done[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sh.flag = prev == static_cast<uint32_t>(chunks - 1);
  }
  __syncthreads();
  if (!sh.flag) return;

  // ---- stage 2 (the row's last chunk): the candidates, in ascending column order
  if (threadIdx.x == 0) {
    uint32_t acc = 0;
    for (int c = 0; c < chunks; ++c) {
      sh.offs[c] = acc;
      acc += __hip_atomic_load(&ws.count[row * chunks + c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    for (int c = chunks; c <= kMaxChunks; ++c) sh.offs[c] = acc;
    // every chunk of the row is past the barrier and has reported: re-arm both counters
    __hip_atomic_store(&ws.arrive[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&ws.done[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  const uint32_t C = sh.offs[chunks];
  uint32_t offs[kMaxChunks + 1];  // in registers: the load addresses need no LDS round trips
#pragma unroll
  for (int c = 0; c <= kMaxChunks; ++c) offs[c] = sh.offs[c];
  const uint64_t* rc = ws.cand + static_cast<size_t>(row) * chunks * kTkChunk;
  // candidate j of batch b0: thread t holds j = b0 + t*32 + i (contiguous, in order)
  uint64_t cv[kCandPerThread];
  auto load_batch = [&](uint32_t b0) {
#pragma unroll
    for (int i = 0; i < kCandPerThread; ++i) {  // all loads issued before any is used
      const uint32_t j = min(b0 + threadIdx.x * kCandPerThread + i, C - 1);
      int c = 0;
#pragma unroll
      for (int cc = 1; cc < kMaxChunks; ++cc) c += (offs[cc] <= j && cc < chunks) ? 1 : 0;
      cv[i] = __hip_atomic_load(rc + static_cast<size_t>(c) * kTkChunk + (j - offs[c]), __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
    }
  };
  auto batch_mask = [&](uint32_t b0) {
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < kCandPerThread; ++i) m |= (b0 + threadIdx.x * kCandPerThread + i < C) ? (1u << i) : 0u;
    return m;
  };
  const bool resident = C <= static_cast<uint32_t>(kCandBatch);
  if (resident) load_batch(0);

  // two radix passes over the candidates of digit d0 (the rest are above it)
  uint32_t prefix = d0;
  uint32_t k_rem = static_cast<uint32_t>(k) - above0;
  for (int pass = 1; pass < 3; ++pass) {
    const int shift = pass == 1 ? 10 : 0;
    const int width = pass == 1 ? 11 : 10;
    const uint32_t nb = 1u << width;
    for (uint32_t b = threadIdx.x; b < kBins; b += kTkThreads) sh.h[b] = 0;
    __syncthreads();
    for (uint32_t b0 = 0; b0 < C; b0 += kCandBatch) {
      if (!resident) load_batch(b0);
      const uint32_t m = batch_mask(b0);
#pragma unroll
      for (int i = 0; i < kCandPerThread; ++i) {
        const uint32_t kk = static_cast<uint32_t>(cv[i] >> 32);
        if (((m >> i) & 1u) && (kk >> (shift + width)) == prefix) atomicAdd(&sh.h[(kk >> shift) & (nb - 1)], 1u);
      }
    }
    __syncthreads();
    uint32_t d, above;
    find_digit(nb, k_rem, sh, d, above);
    prefix = (prefix << width) | d;
    k_rem -= above;
  }
  const uint32_t T = prefix;
  const uint32_t need_eq = k_rem;

  // emit: candidates > T, then == T in order until need_eq, in ascending column order
  uint32_t base = 0, eq_base = 0;
  for (uint32_t b0 = 0; b0 < C; b0 += kCandBatch) {
    if (!resident) load_batch(b0);
    const uint32_t m = batch_mask(b0);
    uint32_t n_eq = 0;
#pragma unroll
    for (int i = 0; i < kCandPerThread; ++i) n_eq += ((m >> i) & 1u) && static_cast<uint32_t>(cv[i] >> 32) == T;
    uint32_t eq_tot;
    uint32_t eq_rank = eq_base + block_excl_scan(n_eq, sh.waves, eq_tot);
    uint32_t sel = 0;
#pragma unroll
    for (int i = 0; i < kCandPerThread; ++i) {
      const uint32_t kk = static_cast<uint32_t>(cv[i] >> 32);
      const bool valid = (m >> i) & 1u;
      const bool eq = valid && kk == T;
      sel |= ((valid && kk > T) || (eq && eq_rank < need_eq)) ? (1u << i) : 0u;
      eq_rank += eq;
    }
    uint32_t sel_tot;
    uint32_t p = base + block_excl_scan(__builtin_popcount(sel), sh.waves, sel_tot);
#pragma unroll
    for (int i = 0; i < kCandPerThread; ++i)
      if ((sel >> i) & 1u) o[p++] = static_cast<int32_t>(static_cast<uint32_t>(cv[i]));
    base += sel_tot;
    eq_base += eq_tot;
  }
}

}  // namespace tl

using namespace tl;

static int64_t topk_chunks(int64_t ld) { return cdiv(ld, kTkChunk); }

extern "C" size_t tl_topk_workspace_bytes(int64_t rows, int64_t ld, int64_t k) {
  (void)k;
  if (rows <= 0 || ld <= 0) return 0;
  const int64_t chunks = topk_chunks(ld);
  return 2 * align256(rows * 4) + align256(rows * chunks * 4) + align256(static_cast<size_t>(rows) * chunks * kBins * 4) +
         static_cast<size_t>(rows) * chunks * kTkChunk * 8;
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
  const TopkWs ws = carve(workspace, rows, chunks);
  hipLaunchKernelGGL(topk_kernel, dim3(static_cast<unsigned>(chunks), static_cast<unsigned>(rows)), dim3(kTkThreads),
                     0, (hipStream_t)stream, logits, ld, valid_base, (int)k, ws, out);
  return check_launch("topk");
}
