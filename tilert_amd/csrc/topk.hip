// Exact per-row top-k (the contract of topk_accurate_op, ops/topk.py:62-109; its golden
// is torch.topk, :128-143) in ONE kernel with a single hand-off and no waiting.
//
// Scores map to order-preserving 32-bit keys (larger score = larger key).  A row is cut
// into chunks of 1024 * PT columns, one 1024-thread workgroup each (PT contiguous columns
// per thread, kept in registers).
//   Stage 1 (every chunk, independently): the chunk's keys and a fixed sample of the row
//     (S = min(4096, n) columns: 1024 runs of 4 spread evenly over it) are loaded together.  From the
//     sample every chunk computes the same conservative threshold theta: a lower bound of
//     the sample's r-th largest key, r = lambda + 4 sqrt(lambda) + 16 with lambda = k S / n
//     the expected number of sampled keys among the row's top k (three 6-bit radix passes
//     over the sample: theta keeps the top 18 bits of that key).  It publishes its keys >= theta as (key, column) pairs in
//     ascending column order and counts itself in (two-level arrival counter).
//   Stage 2 (the row's last chunk to arrive): with C >= k candidates, every key of the
//     row's top k is among them (C >= k keys are >= theta, so the k-th largest key T is
//     >= theta), and 6-bit radix passes below the bits every candidate shares (stopping as
//     soon as the threshold digit's whole bin is needed) find T; every candidate above T plus the lowest-column
//     candidates equal to T are written in ascending column order.  If the sample fell
//     short (C < k: a badly unrepresentative sample), the same selection runs over the
//     whole row instead, so every input is exact.
// Candidates are read in batches and stay in registers when one batch holds them;
// otherwise every pass streams the batches again.  Scans are DPP row shifts and
// broadcasts inside a wave and one LDS exchange across the sixteen waves.
// Histograms: scores bunch into few digits (a score's sign and exponent fill the top bits),
// and LDS atomics that hit one address in one instruction serialise (measured: 2-4 us per
// 11-bit pass over 4096 keys with one shared histogram).  Bulk LDS traffic is slow too
// (measured: ~1 us to clear 64 KB per workgroup), and each 16-wave barrier costs ~0.13 us.
// So digits are 6 bits wide, lane l counts into row l % 16 of a [16][65] histogram (4 KB;
// at most 4 lanes share an address), and one wave sums, clears and picks: a pass is the
// atomics and two barriers.
//
// No workgroup waits for another (the last arrival does the final work), so nothing
// depends on workgroups being co-resident and no wait can time out.  The set is exact
// and deterministic, ties included.
//
// Rows are the topk_accurate samples: row i considers columns [0, valid_base + 1 + i).

#include <math.h>

#include <algorithm>
#include <type_traits>

#include "common.h"
#include "../../include/tilert_amd.h"

namespace tl {

constexpr int kTkThreads = 1024;
constexpr int kTkWaves = kTkThreads / 64;
constexpr int kDigitBits = 6;
constexpr int kBins = 1 << kDigitBits;                // 64 digits per pass
constexpr int kHistRows = 16;                         // lane l counts into row l % 16
static_assert(kBins * kHistRows == kTkThreads, "one thread per (digit, row)");
constexpr int kHistPad = kBins + 1;                   // row stride (words)
constexpr int kMaxK = 8192;
constexpr int kMaxCols = 262144;
constexpr int kMaxChunks = 256;                       // per row
constexpr int kSamplePerThread = 4;
constexpr int kSample = kTkThreads * kSamplePerThread;  // 4096
constexpr int kMaxRowsPerLaunch = 1024;               // arrival-counter slots

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2t __attribute__((ext_vector_type(2)));

// The workspace starts with a fixed region of arrival counters -- per launch row slot
// (blockIdx.y, at most kMaxRowsPerLaunch rows per launch) -- that must be zero when a call
// starts and is left zero by every call.  Its offsets do not depend on the problem shape,
// so calls of any shapes can share one workspace.  Same-address device-scope atomics
// serialise (tens of ns each), so a row's chunks count in per group of G = min(8, chunks)
// first (chunk % G), and the last of a group bumps the row counter.
constexpr int kGroups = 8;
constexpr int kBufferRsrcWord3 = 0x00020000;  // buffer resource word 3: 32-bit data format
constexpr int kCachePolicySc1 = 16;           // buffer access cache policy: sc1
constexpr size_t kCounterBytes = static_cast<size_t>(kMaxRowsPerLaunch) * (kGroups + 1) * sizeof(uint32_t);

struct TopkWs {
  uint32_t* arrive1;  // [kMaxRowsPerLaunch][kGroups] chunks of a group that have published
  uint32_t* arrive2;  // [kMaxRowsPerLaunch] groups that have published
  uint32_t* count;    // [rows][chunks] candidates published per chunk
  uint64_t* cand;     // [rows][chunks][chunk columns] (key << 32 | column)
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

__host__ __device__ inline TopkWs carve(void* base, int64_t rows, int64_t chunks) {
  char* p = static_cast<char*>(base);
  TopkWs w;
  w.arrive1 = reinterpret_cast<uint32_t*>(p);
  w.arrive2 = w.arrive1 + kMaxRowsPerLaunch * kGroups;
  p += align256(kCounterBytes);
  w.count = reinterpret_cast<uint32_t*>(p);
  p += align256(rows * chunks * sizeof(uint32_t));
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

__device__ inline uint32_t ld_agent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_agent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Inclusive prefix sum over a wave's 64 lanes: Hillis-Steele inside each 16-lane row
// (row_shr 1, 2, 4, 8; lanes shifted in from outside the row read 0), then the last lane
// of rows 0 / 2 is added to rows 1 / 3 (row_bcast:15) and the last lane of row 1 to rows
// 2 and 3 (row_bcast:31).
__device__ inline uint32_t wave_incl_scan(uint32_t x) {
  x += __builtin_amdgcn_update_dpp(0u, x, 0x111, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0u, x, 0x112, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0u, x, 0x114, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0u, x, 0x118, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0u, x, 0x142, 0xa, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0u, x, 0x143, 0xc, 0xf, false);
  return x;
}

struct TopkShared {
  uint32_t hist[kHistRows * kHistPad];
  uint32_t waves[2][kTkWaves];
  uint32_t wmax[kTkWaves], wmin[kTkWaves];
  uint32_t digit, above, dcount, flag;
  uint32_t offs[kMaxChunks + 1];
};

// Block-wide exclusive prefix sum over the 1024 threads (and the block total).  The two
// wave-total slots alternate between calls, so one barrier per scan suffices: a slot is
// rewritten only after the next scan's barrier, which every reader of it has passed.
__device__ inline uint32_t block_excl_scan(uint32_t v, TopkShared& sh, int& slot, uint32_t& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t x = wave_incl_scan(v);
  if (lane == 63) sh.waves[slot][wave] = x;
  __syncthreads();
  uint32_t before = 0;
  total = 0;
#pragma unroll
  for (int w = 0; w < kTkWaves; ++w) {
    const uint32_t s = sh.waves[slot][w];
    before += w < wave ? s : 0u;
    total += s;
  }
  slot ^= 1;
  return before + x - v;
}

// Two-level arrival (thread 0): true for the row's last chunk.  Group g = chunk % G holds
// chunks g, g+G, ...; its last arrival bumps the row counter.
__device__ inline bool arrive_last(uint32_t* level1, uint32_t* level2, int chunk, int chunks, int groups) {
  const int g = chunk % groups;
  const uint32_t gsize = static_cast<uint32_t>((chunks - 1 - g) / groups + 1);
  const uint32_t p1 = __hip_atomic_fetch_add(&level1[g], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (p1 != gsize - 1) return false;
  if (groups == 1) return true;
  const uint32_t p2 = __hip_atomic_fetch_add(level2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return p2 == static_cast<uint32_t>(groups - 1);
}

// ---- 6-bit radix passes over the [16][65] histogram (kept all-zero between passes)
// Count the digit (key >> shift) & (2^w - 1) of every valid key whose bits above
// shift + w equal `prefix`, into row lane % 16.
template <int N>
__device__ inline void hist_add(TopkShared& sh, const uint32_t (&keys)[N], uint32_t valid, int shift, int w,
                                uint32_t prefix) {
  uint32_t* row = sh.hist + (threadIdx.x & (kHistRows - 1)) * kHistPad;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const uint32_t kk = keys[i];
    if (((valid >> i) & 1u) && (static_cast<uint64_t>(kk) >> (shift + w)) == prefix)
      atomicAdd(&row[(kk >> shift) & ((1u << w) - 1u)], 1u);
  }
}

// The digit holding the k_rem-th largest counted key, how many counted keys lie in the
// digits above it, and its own count.  One wave does it (a block-wide scan costs two more
// barriers): lane l sums digit 63 - l over the 16 rows and clears them, so lane order is
// descending digit order and one wave scan finds the owner.
__device__ inline void pick_digit(TopkShared& sh, uint32_t k_rem, uint32_t& digit, uint32_t& above,
                                  uint32_t& dcount) {
  if (threadIdx.x < 64) {
    const int b = kBins - 1 - static_cast<int>(threadIdx.x);
    uint32_t c = 0;
#pragma unroll
    for (int r = 0; r < kHistRows; ++r) c += sh.hist[r * kHistPad + b];
#pragma unroll
    for (int r = 0; r < kHistRows; ++r) sh.hist[r * kHistPad + b] = 0u;
    const uint32_t incl = wave_incl_scan(c);
    const uint32_t before = incl - c;
    if (before < k_rem && incl >= k_rem) {
      sh.digit = static_cast<uint32_t>(b);
      sh.above = before;
      sh.dcount = c;
    }
  }
  __syncthreads();
  digit = sh.digit;
  above = sh.above;
  dcount = sh.dcount;
}

// Wave min by the DPP max (common.h) of the complements.
__device__ inline uint32_t wave_min_u32(uint32_t x) { return ~wave_max_u32(~x); }

// Block-wide max and min of the valid keys (one LDS exchange).
__device__ inline void block_max_min(uint32_t vmax, uint32_t vmin, TopkShared& sh, uint32_t& kmax, uint32_t& kmin) {
  vmax = wave_max_u32(vmax);
  vmin = wave_min_u32(vmin);
  if ((threadIdx.x & 63) == 0) {
    sh.wmax[threadIdx.x >> 6] = vmax;
    sh.wmin[threadIdx.x >> 6] = vmin;
  }
  __syncthreads();
  kmax = 0u;
  kmin = 0xffffffffu;
#pragma unroll
  for (int w = 0; w < kTkWaves; ++w) {
    kmax = max(kmax, sh.wmax[w]);
    kmin = min(kmin, sh.wmin[w]);
  }
}

// The exact selection over a column-ordered stream of E entries ((key << 32 | column),
// some of which may be invalid) holding C valid candidates, read in batches by
// load_batch(b0, cv) (returns the validity mask of this thread's CPT contiguous entries
// b0 + CPT t + i).  Writes the k selected columns in ascending order to o.
template <int CPT, class LoadBatch>
__device__ inline void select_topk(uint32_t E, uint32_t C, int k, TopkShared& sh, int& slot, int32_t* __restrict__ o,
                                   LoadBatch&& load_batch) {
  constexpr int CB = kTkThreads * CPT;
  uint64_t cv[CPT];
  const uint32_t n_batches = (E + CB - 1) / CB;
  const uint32_t m_res = load_batch(0u, cv);
  // body(mask) over every candidate batch (the first one stays loaded)
  auto for_batches = [&](auto&& body) __attribute__((always_inline)) {
    for (uint32_t bi = 0; bi < n_batches; ++bi) {
      uint32_t m = m_res;
      if (n_batches > 1) m = load_batch(bi * CB, cv);
      body(m);
    }
  };
  uint32_t prefix = 0, k_rem = static_cast<uint32_t>(k);
  int tshift = 32;
  bool resolved = C == static_cast<uint32_t>(k);  // every candidate is needed
  if (!resolved) {
    // the bits every candidate shares (those of the largest and smallest key) need no pass
    uint32_t vmax = 0u, vmin = 0xffffffffu;
    for_batches([&](uint32_t m) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const uint32_t kk = static_cast<uint32_t>(cv[i] >> 32);
        vmax = ((m >> i) & 1u) ? max(vmax, kk) : vmax;
        vmin = ((m >> i) & 1u) ? min(vmin, kk) : vmin;
      }
    });
    uint32_t kmax, kmin;
    block_max_min(vmax, vmin, sh, kmax, kmin);
    const int lead = kmax == kmin ? 32 : __builtin_clz(kmax ^ kmin);
    tshift = 32 - lead;
    prefix = lead == 32 ? kmax : (lead == 0 ? 0u : kmax >> tshift);
    // (all candidates equal, lead = 32: no pass; the lowest-column k of them are taken)
    // 6-bit passes below the shared bits until the threshold digit's whole bin is needed
    while (!resolved && tshift > 0) {
      const int w = min(kDigitBits, tshift), shift = tshift - w;
      for_batches([&](uint32_t m) __attribute__((always_inline)) {
        uint32_t keys[CPT];
#pragma unroll
        for (int i = 0; i < CPT; ++i) keys[i] = static_cast<uint32_t>(cv[i] >> 32);
        hist_add(sh, keys, m, shift, w, prefix);
      });
      __syncthreads();
      uint32_t d, above, dc;
      pick_digit(sh, k_rem, d, above, dc);
      prefix = (prefix << w) | d;
      k_rem -= above;
      tshift = shift;
      resolved = dc == k_rem;
    }
  }
  const uint64_t T = prefix;
  const uint32_t need_eq = k_rem;

  // emit: candidates above T, then those equal to T (compared on bits >= tshift) in column
  // order until need_eq, all in ascending column order
  uint32_t base = 0, eq_base = 0;
  if (resolved) {  // every key of the threshold bin is taken: one scan per batch
    for_batches([&](uint32_t m) __attribute__((always_inline)) {
      uint32_t sel = 0;
#pragma unroll
      for (int i = 0; i < CPT; ++i)
        sel |= (((m >> i) & 1u) && ((cv[i] >> 32) >> tshift) >= T) ? (1u << i) : 0u;
      uint32_t sel_tot;
      uint32_t p = base + block_excl_scan(__builtin_popcount(sel), sh, slot, sel_tot);
#pragma unroll
      for (int i = 0; i < CPT; ++i)
        if ((sel >> i) & 1u) {
          if (p < static_cast<uint32_t>(k)) o[p] = static_cast<int32_t>(static_cast<uint32_t>(cv[i]));
          ++p;
        }
      base += sel_tot;
    });
    return;
  }
  for_batches([&](uint32_t m) __attribute__((always_inline)) {
    uint32_t n_eq = 0;
#pragma unroll
    for (int i = 0; i < CPT; ++i) n_eq += ((m >> i) & 1u) && ((cv[i] >> 32) >> tshift) == T;
    uint32_t eq_tot;
    uint32_t eq_rank = eq_base + block_excl_scan(n_eq, sh, slot, eq_tot);
    uint32_t sel = 0;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const uint64_t kk = (cv[i] >> 32) >> tshift;
      const bool valid = (m >> i) & 1u;
      const bool eq = valid && kk == T;
      sel |= ((valid && kk > T) || (eq && eq_rank < need_eq)) ? (1u << i) : 0u;
      eq_rank += eq;
    }
    uint32_t sel_tot;
    uint32_t p = base + block_excl_scan(__builtin_popcount(sel), sh, slot, sel_tot);
#pragma unroll
    for (int i = 0; i < CPT; ++i)
      if ((sel >> i) & 1u) {
        if (p < static_cast<uint32_t>(k)) o[p] = static_cast<int32_t>(static_cast<uint32_t>(cv[i]));
        ++p;
      }
    base += sel_tot;
    eq_base += eq_tot;
  });
}

template <int PT>
__global__ __launch_bounds__(kTkThreads) void topk_kernel(const float* __restrict__ logits, int64_t ld,
                                                          int64_t valid_base, int k, int row0, TopkWs ws,
                                                          int32_t* __restrict__ out) {
  constexpr int kChunk = kTkThreads * PT;
  static_assert(PT % 4 == 0 && PT <= 32, "float4 loads, one mask bit per key");
  __shared__ TopkShared sh;
  int slot = 0;
  const int row = row0 + static_cast<int>(blockIdx.y), y = blockIdx.y;
  const int chunks = gridDim.x, chunk = blockIdx.x;
  const int n = row_valid(row, valid_base, ld);
  int32_t* o = out + static_cast<int64_t>(row) * k;
  if (n <= k) {  // every valid column, then -1 padding (the whole row exits: no counters)
    // chunk c writes columns [c kChunk, (c+1) kChunk); the last chunk also pads up to k
    // when k exceeds the row's chunk span
    const int base = chunk * kChunk;
    const int end = chunk == chunks - 1 ? k : min(base + kChunk, k);
    for (int c = base + static_cast<int>(threadIdx.x); c < end; c += kTkThreads) o[c] = c < n ? c : -1;
    return;
  }

  // ---- stage 1: this chunk's keys (PT contiguous columns per thread) and the row sample
  // (the histogram is cleared first: the barrier would otherwise wait for the loads)
  for (int i = threadIdx.x; i < kHistRows * kHistPad; i += kTkThreads) sh.hist[i] = 0u;
  __syncthreads();
  const float* src = logits + static_cast<int64_t>(row) * ld;
  const int c0 = chunk * kChunk + static_cast<int>(threadIdx.x) * PT;
  const int S = min(kSample, n);
  uint32_t skey[kSamplePerThread];
  uint32_t svalid = 0;
  if (n >= kSample) {  // 1024 runs of 4 columns (one 16-byte load each) spread over [0, n)
    const int p0 = static_cast<int>((static_cast<int64_t>(threadIdx.x) * n / kTkThreads) & ~int64_t{3});
    const f32x4 sv = *reinterpret_cast<const f32x4*>(src + p0);
#pragma unroll
    for (int i = 0; i < kSamplePerThread; ++i) skey[i] = order_key(sv[i]);
    svalid = (1u << kSamplePerThread) - 1u;
  } else {  // short row: every column
    float sv[kSamplePerThread];
#pragma unroll
    for (int i = 0; i < kSamplePerThread; ++i) {
      const int j = static_cast<int>(threadIdx.x) * kSamplePerThread + i;
      sv[i] = src[min(j, n - 1)];
      svalid |= j < n ? (1u << i) : 0u;
    }
#pragma unroll
    for (int i = 0; i < kSamplePerThread; ++i) skey[i] = order_key(sv[i]);
  }
  uint32_t key[PT], vm = 0;
  if (c0 + PT <= n) {
    f32x4 v[PT / 4];
#pragma unroll
    for (int i = 0; i < PT / 4; ++i) v[i] = *reinterpret_cast<const f32x4*>(src + c0 + 4 * i);
#pragma unroll
    for (int i = 0; i < PT / 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) key[4 * i + j] = order_key(v[i][j]);
    vm = PT == 32 ? 0xffffffffu : ((1u << PT) - 1u);
  } else {
#pragma unroll
    for (int i = 0; i < PT; ++i) {
      const bool ok = c0 + i < n;
      key[i] = ok ? order_key(src[ok ? c0 + i : 0]) : 0u;
      vm |= ok ? (1u << i) : 0u;
    }
  }
  // theta: a lower bound of the sample's r-th largest key (its top 18 bits)
  uint32_t theta = 0;
  {
    const float lam = static_cast<float>(k) * static_cast<float>(S) / static_cast<float>(n);
    const uint32_t r = static_cast<uint32_t>(ceilf(lam + 4.0f * sqrtf(lam) + 16.0f));
    if (r < static_cast<uint32_t>(S)) {
      uint32_t prefix = 0, k_rem = r;
#pragma unroll
      for (int pass = 0; pass < 3; ++pass) {
        const int shift = 26 - kDigitBits * pass;
        hist_add(sh, skey, svalid, shift, kDigitBits, prefix);
        __syncthreads();
        uint32_t d, above, dc;
        pick_digit(sh, k_rem, d, above, dc);
        prefix = (prefix << kDigitBits) | d;
        k_rem -= above;
      }
      theta = prefix << 14;
    }
  }

  // candidates: keys >= theta, compacted in ascending column order
  uint32_t cbits = 0;
#pragma unroll
  for (int i = 0; i < PT; ++i) cbits |= (((vm >> i) & 1u) && key[i] >= theta) ? (1u << i) : 0u;
  uint32_t n_cand;
  uint32_t pos = block_excl_scan(__builtin_popcount(cbits), sh, slot, n_cand);
  uint64_t* cand = ws.cand + (static_cast<int64_t>(row) * chunks + chunk) * kChunk;
#pragma unroll
  for (int i = 0; i < PT; ++i)
    if ((cbits >> i) & 1u) {
      const uint64_t v = (static_cast<uint64_t>(key[i]) << 32) | static_cast<uint32_t>(c0 + i);
      __hip_atomic_store(cand + pos++, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  if (threadIdx.x == 0) st_agent(&ws.count[static_cast<int64_t>(row) * chunks + chunk], n_cand);
  __builtin_amdgcn_s_waitcnt(0);  // this chunk's candidates are complete before it reports
  __syncthreads();
  const int groups = min(kGroups, chunks);
  if (threadIdx.x == 0) sh.flag = arrive_last(ws.arrive1 + y * kGroups, ws.arrive2 + y, chunk, chunks, groups);
  __syncthreads();
  if (!sh.flag) return;

  // ---- stage 2 (the row's last chunk): every chunk has published; re-arm the counters
  if (threadIdx.x < static_cast<unsigned>(groups)) st_agent(&ws.arrive1[y * kGroups + threadIdx.x], 0u);
  if (threadIdx.x == 0) st_agent(&ws.arrive2[y], 0u);
  const uint64_t* rc = ws.cand + static_cast<int64_t>(row) * chunks * kChunk;
  const __amdgpu_buffer_rsrc_t crs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t*>(rc), 0,
                                                                       chunks * kChunk * 8, kBufferRsrcWord3);
  auto load_cand = [&](uint32_t e) -> uint64_t {  // plain sc1 buffer loads (past this XCD's L2, like the
    return __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(crs, static_cast<int>(e * 8u), 0, kCachePolicySc1));
  };                                              // agent-scope atomic loads), kept in flight together
  // counts -> per-chunk offsets (entries past the last chunk hold C)
  uint32_t C;
  {
    const uint32_t cn = threadIdx.x < static_cast<unsigned>(chunks)
                            ? ld_agent(&ws.count[static_cast<int64_t>(row) * chunks + threadIdx.x]) : 0u;
    const uint32_t before = block_excl_scan(cn, sh, slot, C);
    if (threadIdx.x < static_cast<unsigned>(kMaxChunks)) sh.offs[threadIdx.x] = before;
    if (threadIdx.x == 0) sh.offs[kMaxChunks] = C;
    __syncthreads();
  }
  int lg = 0;  // binary-search depth: smallest power of two >= chunks
  while ((1 << lg) < chunks) ++lg;

  // Candidate batches of CB = 1024 * CPT in column order: thread t takes the CPT contiguous
  // entries b0 + CPT t + i (so thread order is column order), each located by a binary
  // search over the chunk offsets; a wave's loads cover contiguous stretches of the chunks'
  // regions.  RAW: the entries are the row's own columns (the fallback when the sample
  // fell short).
  auto make_loader = [&](auto cpt_tag, auto raw_tag) {
    constexpr int CPT = decltype(cpt_tag)::value;
    constexpr bool RAW = decltype(raw_tag)::value;
    const uint32_t total = RAW ? static_cast<uint32_t>(n) : C;
    return [&, total](uint32_t b0, uint64_t (&cv)[CPT]) __attribute__((always_inline)) -> uint32_t {
      uint32_t j[CPT];
#pragma unroll
      for (int i = 0; i < CPT; ++i) j[i] = min(b0 + threadIdx.x * CPT + i, total - 1);
      if (RAW) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) cv[i] = (static_cast<uint64_t>(order_key(src[j[i]])) << 32) | j[i];
      } else {
        int c[CPT];
#pragma unroll
        for (int i = 0; i < CPT; ++i) c[i] = 0;
        // the largest chunk c with offs[c] <= j: chunks without candidates share their
        // successor's offset, so they are stepped over
        for (int sstep = lg - 1; sstep >= 0; --sstep) {
#pragma unroll
          for (int i = 0; i < CPT; ++i) {
            const int nc = c[i] + (1 << sstep);  // <= 255: offs[] past the last chunk hold C > j
            c[i] = sh.offs[nc] <= j[i] ? nc : c[i];
          }
        }
        uint32_t off[CPT];
#pragma unroll
        for (int i = 0; i < CPT; ++i) off[i] = sh.offs[c[i]];
#pragma unroll
        for (int i = 0; i < CPT; ++i) cv[i] = load_cand(static_cast<uint32_t>(c[i]) * kChunk + (j[i] - off[i]));
      }
      uint32_t m = 0;
#pragma unroll
      for (int i = 0; i < CPT; ++i) m |= (b0 + threadIdx.x * CPT + i < total) ? (1u << i) : 0u;
      return m;
    };
  };
  using I4 = std::integral_constant<int, 4>;
  using I8 = std::integral_constant<int, 8>;
  if (C >= static_cast<uint32_t>(k)) {
    if (C <= static_cast<uint32_t>(kTkThreads * 4))
      select_topk<4>(C, C, k, sh, slot, o, make_loader(I4{}, std::false_type{}));
    else
      select_topk<8>(C, C, k, sh, slot, o, make_loader(I8{}, std::false_type{}));
  } else {
    select_topk<8>(static_cast<uint32_t>(n), static_cast<uint32_t>(n), k, sh, slot, o,
                   make_loader(I8{}, std::true_type{}));
  }
}

}  // namespace tl

using namespace tl;

namespace {

// Columns per thread: 4 (chunks of 4096 columns) when a row spans at most 64 such chunks,
// otherwise 8 (rows up to 262144 columns in at most 32 chunks of 8192).
struct TopkPlan {
  int pt, chunks, rows_per_launch;
};

TopkPlan plan_topk(int64_t rows, int64_t ld) {
  TopkPlan p{8, 0, 0};
  const int64_t ch4 = cdiv(ld, static_cast<int64_t>(kTkThreads) * 4);
  if (ch4 <= 64) {
    p.pt = 4;
    p.chunks = static_cast<int>(ch4);
  } else {
    p.pt = 8;
    p.chunks = static_cast<int>(cdiv(ld, static_cast<int64_t>(kTkThreads) * 8));
  }
  p.rows_per_launch = static_cast<int>(std::min<int64_t>(rows, kMaxRowsPerLaunch));
  return p;
}

}  // namespace

extern "C" size_t tl_topk_workspace_bytes(int64_t rows, int64_t ld, int64_t k) {
  (void)k;
  if (rows <= 0 || ld <= 0 || ld > kMaxCols) return 0;
  const TopkPlan p = plan_topk(rows, ld);
  const size_t chunk_cols = static_cast<size_t>(kTkThreads) * p.pt;
  return align256(kCounterBytes) + align256(static_cast<size_t>(rows) * p.chunks * 4) +
         static_cast<size_t>(rows) * p.chunks * chunk_cols * 8;
}

extern "C" int tl_topk_rows(const float* logits, int64_t rows, int64_t ld, int64_t valid_base, int64_t k,
                            int32_t* out, void* workspace, size_t workspace_bytes, void* stream) {
  if (rows <= 0 || ld <= 0) { set_error("topk: empty input (rows=%lld ld=%lld)", (long long)rows, (long long)ld); return kErrArg; }
  if (k < 1 || k > kMaxK) { set_error("topk: k=%lld must be in [1, %d]", (long long)k, kMaxK); return kErrUnsupported; }
  if (ld > kMaxCols) { set_error("topk: ld=%lld > %d columns is not supported", (long long)ld, kMaxCols); return kErrUnsupported; }
  if (ld % 4) { set_error("topk: ld=%lld must be a multiple of 4 (16-byte rows)", (long long)ld); return kErrArg; }
  if (rows > (1 << 20)) { set_error("topk: rows=%lld exceeds %d", (long long)rows, 1 << 20); return kErrUnsupported; }
  if (!logits || !out) { set_error("topk: null pointer"); return kErrArg; }
  if (reinterpret_cast<uintptr_t>(logits) & 15) { set_error("topk: logits must be 16-byte aligned"); return kErrArg; }
  const size_t need = tl_topk_workspace_bytes(rows, ld, k);
  if (!workspace || workspace_bytes < need) { set_error("topk: workspace of %zu bytes required (got %zu)", need, workspace_bytes); return kErrArg; }
  const TopkPlan p = plan_topk(rows, ld);
  if (p.chunks < 1 || p.chunks > kMaxChunks || p.rows_per_launch < 1) {
    set_error("topk: internal plan error (chunks=%d)", p.chunks);
    return kErrUnsupported;
  }
  const TopkWs ws = carve(workspace, rows, p.chunks);
  auto kern = p.pt == 4 ? topk_kernel<4> : topk_kernel<8>;
  for (int64_t r0 = 0; r0 < rows; r0 += p.rows_per_launch) {
    const int nr = static_cast<int>(std::min<int64_t>(p.rows_per_launch, rows - r0));
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(p.chunks), static_cast<unsigned>(nr)), dim3(kTkThreads), 0,
                       (hipStream_t)stream, logits, ld, valid_base, (int)k, static_cast<int>(r0), ws, out);
    if (int rc = check_launch("topk")) return rc;
  }
  return kOk;
}
