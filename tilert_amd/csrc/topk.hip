// Exact per-row top-k (the contract of topk_accurate_op, ops/topk.py:62-109; its golden
// is torch.topk, :128-143), as ONE kernel with one cross-workgroup barrier and one handoff.
//
// Scores map to order-preserving 32-bit keys (larger score = larger key).  A row is cut
// into chunks of 1024 * PT columns, one 1024-thread workgroup each (PT contiguous columns
// per thread, kept in registers).  Sixteen waves per workgroup hide the LDS and memory
// latencies that dominate the one-workgroup final stage (measured: a 256-thread
// workgroup with 32 candidates per thread spent ~1.5 us on each radix pass and on the
// emission, nearly all of it waiting).
//   Stage 1 (every chunk): a histogram of the keys' top 11 bits in LDS; its non-zero bins
//     are added into its group's copy of the row histogram with agent-scope atomics.  The
//     row's last chunk to arrive (two-level counter) sums the copies, finds the digit d0
//     holding the row's k-th largest key and how many keys lie above it, and broadcasts
//     both; the other chunks wait for the word (bounded spin).  Each chunk then publishes
//     its keys with digit >= d0 -- the only ones that can be selected -- as (key, column)
//     pairs in ascending column order.
//   Stage 2 (the row's last chunk to publish, found with a second two-level counter):
//     radix passes (11, then 10 bits) over the candidates of digit d0 give the k-th
//     largest key T, stopping early when the threshold digit's whole bin is needed; every
//     candidate above T plus the lowest-column candidates equal to it until k are taken
//     are written in ascending column order.  Candidates are read coalesced in batches of
//     8192 and stay in registers when one batch holds them; otherwise every pass streams
//     the batches again, so any input is exact.  The last chunk re-arms the counters.
// Scans use DPP row shifts and row broadcasts inside a wave (no LDS round trips) and one
// LDS exchange across the sixteen waves.
// The set is exact and deterministic, ties included.  Measured on MI355X, the cost is a
// chain of device-scope round trips (~0.25 us each when uncontended; same-address atomics
// serialise at tens of ns each, hence the groups), not bandwidth.
//
// The barrier needs a launch's workgroups co-resident: a launch holds at most 128
// workgroups (larger inputs are launched in groups of rows), and the wait is bounded
// (about a second) so a wave can never hang.
//
// Rows are the topk_accurate samples: row i considers columns [0, valid_base + 1 + i).

#include <algorithm>
#include <type_traits>

#include "common.h"
#include "../../include/tilert_amd.h"

namespace tl {

constexpr int kTkThreads = 1024;
constexpr int kTkWaves = kTkThreads / 64;
constexpr int kBins = 2048;                           // widest digit: 11 bits
constexpr int kBinsPerThread = kBins / kTkThreads;    // 2
static_assert(kBinsPerThread == 2, "the histogram code below moves 2 bins per thread");
constexpr int kMaxK = 8192;
constexpr int kMaxCols = 262144;
constexpr int kMaxGroups = 128;                       // workgroups per launch (one per CU, half the chip)
constexpr int kMaxChunks = 256;                       // per row
constexpr int kCandPerThread = 8;                     // stage-2 register batch per thread
constexpr int kCandBatch = kTkThreads * kCandPerThread;
constexpr uint32_t kSpinLimit = 1u << 22;             // x s_sleep(8): ~1 s

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2t __attribute__((ext_vector_type(2)));

// The workspace starts with a fixed state region -- per launch slot (blockIdx.y, at most
// 128 rows per launch): arrival counters, the broadcast word and the row histograms --
// that must be zero when a call starts and is left zero by every call.  Its offsets do
// not depend on the problem shape, so calls of any shapes can share one workspace without
// one call's candidates landing on another call's state.
//
// Same-address device-scope atomics serialise (tens of ns each), so a row's chunks are
// split into G = min(8, chunks) groups (chunk % G): arrivals count per group first and the
// last of a group bumps the row counter; the histogram has one copy per group; the
// broadcast word one replica per group.
constexpr int kSlots = kMaxGroups;
constexpr int kGroups = 8;
constexpr int kBufferRsrcWord3 = 0x00020000;  // buffer resource word 3: 32-bit data format
constexpr int kCachePolicySc1 = 16;           // buffer access cache policy: sc1
constexpr size_t kCounterBytes = 32768;
constexpr size_t kStateBytes = kCounterBytes + static_cast<size_t>(kSlots) * kBins * sizeof(uint32_t);

struct TopkWs {
  uint32_t* arrive1;  // [kSlots][kGroups] chunks of a group past the histogram
  uint32_t* arrive2;  // [kSlots] groups past the histogram
  uint32_t* done1;    // [kSlots][kGroups] chunks of a group past the candidate publication
  uint32_t* done2;    // [kSlots] groups past the candidate publication
  uint32_t* bcast;    // [kSlots][kGroups] (1 << 31) | d0 << 13 | above0
  uint32_t* hist;     // [kSlots][kBins] histograms of the top 11 bits: launch row y uses
                      // slots y*chunks .. y*chunks + G - 1 (one per group)
  uint32_t* count;    // [rows][chunks] candidates published per chunk
  uint64_t* cand;     // [rows][chunks][chunk columns] (key << 32 | column)
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

__host__ __device__ inline TopkWs carve(void* base, int64_t rows, int64_t chunks) {
  char* p = static_cast<char*>(base);
  TopkWs w;
  w.arrive1 = reinterpret_cast<uint32_t*>(p);
  w.arrive2 = w.arrive1 + kSlots * kGroups;
  w.done1 = w.arrive2 + kSlots;
  w.done2 = w.done1 + kSlots * kGroups;
  w.bcast = w.done2 + kSlots;
  w.hist = reinterpret_cast<uint32_t*>(p + kCounterBytes);
  p += kStateBytes;
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
  uint32_t h[kBins + 64];  // + one spare bin per lane (branch-free histogram adds)
  uint32_t waves[2][kTkWaves];
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

// The digit holding the k_rem-th largest key, and how many keys lie in the digits above
// it.  Thread t holds the counts of digits hi-1, hi-2, ..., hi-PER (hi = nb - t*PER), so
// thread order is descending digit order and one block scan finds the owner.
template <int PER>
__device__ inline void pick_digit(const uint32_t (&cnt)[PER], uint32_t hi, uint32_t k_rem, TopkShared& sh,
                                  int& slot, uint32_t& digit, uint32_t& above, uint32_t& dcount) {
  uint32_t own = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) own += cnt[i];
  uint32_t total;
  const uint32_t before = block_excl_scan(own, sh, slot, total);
  if (before < k_rem && before + own >= k_rem) {
    uint32_t a = before, d = hi - PER, dc = 0;
    bool found = false;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if (!found && a + cnt[i] >= k_rem) {
        d = hi - 1 - i;
        dc = cnt[i];
        found = true;
      }
      if (!found) a += cnt[i];
    }
    sh.digit = d;
    sh.above = a;
    sh.dcount = dc;
  }
  __syncthreads();
  digit = sh.digit;
  above = sh.above;
  dcount = sh.dcount;
}

// Two-level arrival (thread 0): true for the row's last chunk.  Group g = chunk % G holds
// chunks g, g+G, ...; its last arrival bumps the row counter.
__device__ inline bool arrive_last(uint32_t* level1, uint32_t* level2, int chunk, int chunks, int groups) {
  const int g = chunk % groups;
  const uint32_t gsize = static_cast<uint32_t>((chunks - 1 - g) / groups + 1);
  const uint32_t p1 = __hip_atomic_fetch_add(&level1[g], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (p1 != gsize - 1) return false;
  const uint32_t p2 = __hip_atomic_fetch_add(level2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return p2 == static_cast<uint32_t>(groups - 1);
}

__device__ inline void zero_bins(TopkShared& sh) {  // thread t clears bins 2t, 2t+1
  reinterpret_cast<u32x2t*>(sh.h)[threadIdx.x] = u32x2t{0u, 0u};
}

template <int PT>
__global__ __launch_bounds__(kTkThreads) void topk_kernel(const float* __restrict__ logits, int64_t ld,
                                                          int64_t valid_base, int k, int row0, TopkWs ws,
                                                          int32_t* __restrict__ out) {
  constexpr int kChunk = kTkThreads * PT;
  static_assert(PT % 4 == 0 && PT <= 32, "float4 loads, one mask bit per key");
  __shared__ TopkShared sh;
  extern __shared__ uint64_t stage[];  // [kCandBatch / kCandPerThread * (kCandPerThread + 1)]: stage-2 staging
  int slot = 0;
  const int row = row0 + static_cast<int>(blockIdx.y), y = blockIdx.y;
  const int chunks = gridDim.x, chunk = blockIdx.x;
  const int n = row_valid(row, valid_base, ld);
  int32_t* o = out + static_cast<int64_t>(row) * k;
  if (n <= k) {  // every valid column, then -1 padding (no barrier: the whole row exits)
    // chunk c writes columns [c kChunk, (c+1) kChunk); the last chunk also pads up to k
    // when k exceeds the row's chunk span
    const int base = chunk * kChunk;
    const int end = chunk == chunks - 1 ? k : min(base + kChunk, k);
    for (int c = base + static_cast<int>(threadIdx.x); c < end; c += kTkThreads)
      o[c] = c < n ? c : -1;
    return;
  }

  // ---- stage 1: this chunk's keys (PT contiguous columns per thread)
  const float* src = logits + static_cast<int64_t>(row) * ld;
  const int c0 = chunk * kChunk + static_cast<int>(threadIdx.x) * PT;
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
  zero_bins(sh);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < PT; ++i)
    if ((vm >> i) & 1u) atomicAdd(&sh.h[key[i] >> 21], 1u);
  __syncthreads();
  // this chunk's non-zero bins into its group's histogram (thread t: bins 2t, 2t+1)
  const int groups = min(kGroups, chunks), grp = chunk % groups;
  uint32_t* rh = ws.hist + static_cast<int64_t>(y) * chunks * kBins;  // group g's at rh + g*kBins
  {
    const u32x2t a = reinterpret_cast<const u32x2t*>(sh.h)[threadIdx.x];
    const uint32_t hv[2] = {a.x, a.y};
#pragma unroll
    for (int i = 0; i < 2; ++i)
      if (hv[i])
        __hip_atomic_fetch_add(&rh[grp * kBins + threadIdx.x * 2 + i], hv[i], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) sh.flag = arrive_last(ws.arrive1 + y * kGroups, ws.arrive2 + y, chunk, chunks, groups);
  __syncthreads();
  // The row's last chunk to arrive sums the group histograms (thread t: digits hi-1,
  // hi-2, hi = 2048 - 2t), finds d0, broadcasts (valid bit, d0, above0) and re-zeroes the
  // histograms; the others wait for their group's replica of that word (bounded spin).
  if (sh.flag) {
    const uint32_t hi = kBins - threadIdx.x * kBinsPerThread;
    // 8-byte loads that bypass the non-coherent cache level (sc1), as the agent-scope
    // atomic loads do; every sub-histogram's atomics completed before its chunk arrived
    const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc(rh, 0, kGroups * kBins * 4, kBufferRsrcWord3);
    u32x2t a[kGroups];
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
      const int off = (g < groups ? g : 0) * kBins * 4 + static_cast<int>(hi - 2) * 4;
      a[g] = __builtin_bit_cast(u32x2t, __builtin_amdgcn_raw_buffer_load_b64(hr, off, 0, kCachePolicySc1));
    }
    uint32_t cnt[kBinsPerThread] = {};
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
      if (g < groups) {
        cnt[0] += a[g].y;
        cnt[1] += a[g].x;
      }
    }
    uint32_t d, above, dc;
    pick_digit(cnt, hi, static_cast<uint32_t>(k), sh, slot, d, above, dc);
    if (threadIdx.x < static_cast<unsigned>(groups)) st_agent(&ws.bcast[y * kGroups + threadIdx.x], 0x80000000u | (d << 13) | above);
    // re-zeroed after the broadcast: nothing reads them again before this kernel ends
    for (int g = 0; g < groups; ++g) *reinterpret_cast<u32x2t*>(rh + g * kBins + hi - 2) = u32x2t{0u, 0u};
  } else if (threadIdx.x == 0) {
    uint32_t w = 0;
    for (uint32_t it = 0; it < kSpinLimit; ++it) {
      w = ld_agent(&ws.bcast[y * kGroups + grp]);
      if (w >> 31) break;
      __builtin_amdgcn_s_sleep(4);
    }
    sh.digit = (w >> 13) & (kBins - 1);
    sh.above = w & 0x1fffu;
  }
  __syncthreads();
  const uint32_t d0 = sh.digit, above0 = sh.above;

  // candidates: keys with digit >= d0, compacted in ascending column order
  uint32_t cbits = 0;
#pragma unroll
  for (int i = 0; i < PT; ++i) cbits |= (((vm >> i) & 1u) && (key[i] >> 21) >= d0) ? (1u << i) : 0u;
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
  if (threadIdx.x == 0) sh.flag = arrive_last(ws.done1 + y * kGroups, ws.done2 + y, chunk, chunks, groups);
  __syncthreads();
  if (!sh.flag) return;

  // ---- stage 2 (the row's last chunk)
  const uint64_t* rc = ws.cand + static_cast<int64_t>(row) * chunks * kChunk;
  const __amdgpu_buffer_rsrc_t crs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t*>(rc), 0,
                                                                       chunks * kChunk * 8, kBufferRsrcWord3);
  // offsets of every chunk's candidates (entries past the last chunk hold C)
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
  // CPT candidates per thread: 4 when the candidates fit one batch of 4096 (the common
  // case, fewer registers and instructions), else 8 (batches of 8192).
  auto select = [&](auto cpt_tag) __attribute__((always_inline)) {
    constexpr int CPT = decltype(cpt_tag)::value;
    constexpr int CB = kTkThreads * CPT;
    // Candidate batches of CB = 1024 * CPT in column order.  A batch is read coalesced
    // (thread t loads j = b0 + 1024 i + t), staged in LDS, and taken back as CPT contiguous
    // candidates per thread (j = b0 + CPT t + i), so thread order is column order.  Rows
    // padded to CPT + 1 entries keep both LDS access patterns free of bank conflicts.
    uint64_t cv[CPT];
    auto load_batch = [&](uint32_t b0) __attribute__((always_inline)) {
      uint32_t j[CPT];
      int c[CPT];
  #pragma unroll
      for (int i = 0; i < CPT; ++i) {
        j[i] = min(b0 + i * kTkThreads + threadIdx.x, C - 1);
        c[i] = 0;
      }
      // the largest chunk c with offs[c] <= j: chunks without candidates share their
      // successor's offset, so they are stepped over
      for (int sstep = lg - 1; sstep >= 0; --sstep) {
  #pragma unroll
        for (int i = 0; i < CPT; ++i) {
          const int nc = c[i] + (1 << sstep);  // <= 255: offs[] past the last chunk hold C > j
          c[i] = sh.offs[nc] <= j[i] ? nc : c[i];
        }
      }
      // all offsets first, then the candidate loads: plain sc1 buffer loads (past this
      // XCD's L2, like the agent-scope atomic loads) that the compiler can keep in flight
      // together -- atomic loads interleaved with the LDS reads waited on each read
      uint32_t off[CPT];
  #pragma unroll
      for (int i = 0; i < CPT; ++i) off[i] = sh.offs[c[i]];
      uint64_t v[CPT];
  #pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const uint32_t e = static_cast<uint32_t>(c[i]) * kChunk + (j[i] - off[i]);
        v[i] = __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(crs, static_cast<int>(e * 8u), 0, kCachePolicySc1));
      }
      __syncthreads();  // the previous batch's staging reads are complete
  #pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const int e = i * kTkThreads + threadIdx.x;
        stage[(e / CPT) * (CPT + 1) + (e % CPT)] = v[i];
      }
      __syncthreads();
  #pragma unroll
      for (int i = 0; i < CPT; ++i) cv[i] = stage[threadIdx.x * (CPT + 1) + i];
      uint32_t m = 0;
  #pragma unroll
      for (int i = 0; i < CPT; ++i) m |= (b0 + threadIdx.x * CPT + i < C) ? (1u << i) : 0u;
      return m;
    };
    const uint32_t n_batches = (C + CB - 1) / CB;
    const uint32_t m_res = load_batch(0);
    // body(mask) over every candidate batch (the first one stays loaded)
    auto for_batches = [&](auto&& body) __attribute__((always_inline)) {
      for (uint32_t bi = 0; bi < n_batches; ++bi) {
        uint32_t m = m_res;
        if (n_batches > 1) m = load_batch(bi * CB);
        body(m);
      }
    };

    // radix passes over the candidates of digit d0 (the rest are above it) until the
    // threshold digit's whole bin is needed: then every key of that bin is taken
    uint32_t prefix = d0, tshift = 21;
    uint32_t k_rem = static_cast<uint32_t>(k) - above0;
    bool resolved = C == static_cast<uint32_t>(k);  // digit d0's whole bin is needed
  #pragma unroll
    for (int pass = 1; pass < 3; ++pass) {
      if (resolved) break;
      const int shift = pass == 1 ? 10 : 0;
      const int width = pass == 1 ? 11 : 10;
      zero_bins(sh);
      __syncthreads();
      for_batches([&](uint32_t m) __attribute__((always_inline)) {
        // a slot is skipped when no lane of the wave has a match (wave-uniform test);
        // otherwise lanes without one add into their own spare bin (no branch, no
        // same-address conflict)
        const uint32_t spare = kBins + (threadIdx.x & 63);
  #pragma unroll
        for (int i = 0; i < CPT; ++i) {
          const uint32_t kk = static_cast<uint32_t>(cv[i] >> 32);
          const bool hit = ((m >> i) & 1u) && (kk >> (shift + width)) == prefix;
          if (__builtin_amdgcn_ballot_w64(hit))
            atomicAdd(&sh.h[hit ? (kk >> shift) & ((1u << width) - 1u) : spare], 1u);
        }
      });
      __syncthreads();
      uint32_t d, above, dc;
      if (pass == 1) {  // 2048 digits, 2 per thread
        const uint32_t hi = kBins - threadIdx.x * 2;
        const u32x2t a = *reinterpret_cast<const u32x2t*>(sh.h + hi - 2);
        const uint32_t cnt[2] = {a.y, a.x};
        pick_digit(cnt, hi, k_rem, sh, slot, d, above, dc);
      } else {  // 1024 digits, 1 per thread
        const uint32_t hi = (kBins / 2) - threadIdx.x;
        const uint32_t cnt[1] = {sh.h[hi - 1]};
        pick_digit(cnt, hi, k_rem, sh, slot, d, above, dc);
      }
      prefix = (prefix << width) | d;
      k_rem -= above;
      tshift = shift;
      resolved = dc == k_rem;
    }
    const uint32_t T = prefix;
    const uint32_t need_eq = k_rem;

    // emit: candidates above T, then those equal to T (compared on bits >= tshift) in
    // column order until need_eq, all in ascending column order
    uint32_t base = 0, eq_base = 0;
    if (resolved) {  // every key of the threshold bin is taken: one scan per batch
      for_batches([&](uint32_t m) __attribute__((always_inline)) {
        uint32_t sel = 0;
  #pragma unroll
        for (int i = 0; i < CPT; ++i)
          sel |= (((m >> i) & 1u) && (static_cast<uint32_t>(cv[i] >> 32) >> tshift) >= T) ? (1u << i) : 0u;
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
      for (int i = 0; i < CPT; ++i)
        n_eq += ((m >> i) & 1u) && (static_cast<uint32_t>(cv[i] >> 32) >> tshift) == T;
      uint32_t eq_tot;
      uint32_t eq_rank = eq_base + block_excl_scan(n_eq, sh, slot, eq_tot);
      uint32_t sel = 0;
  #pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const uint32_t kk = static_cast<uint32_t>(cv[i] >> 32) >> tshift;
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
  };
  if (C <= static_cast<uint32_t>(kTkThreads * 4))
    select(std::integral_constant<int, 4>{});
  else
    select(std::integral_constant<int, 8>{});

  // every chunk is past the broadcast and has published its candidates: re-arm the row's
  // counters (last, so that no wait on these stores delays the selection)
  if (threadIdx.x < static_cast<unsigned>(groups)) {
    st_agent(&ws.arrive1[y * kGroups + threadIdx.x], 0u);
    st_agent(&ws.done1[y * kGroups + threadIdx.x], 0u);
    st_agent(&ws.bcast[y * kGroups + threadIdx.x], 0u);
  }
  if (threadIdx.x == 0) {
    st_agent(&ws.arrive2[y], 0u);
    st_agent(&ws.done2[y], 0u);
  }
}

}  // namespace tl

using namespace tl;

namespace {

// Columns per thread: 4 (chunks of 4096) when every row of the call fits one launch that
// way (rows * chunks <= 256), otherwise 8, and rows are launched in groups.
struct TopkPlan {
  int pt, chunks, rows_per_launch;
};

TopkPlan plan_topk(int64_t rows, int64_t ld) {
  TopkPlan p{8, 0, 0};
  for (int pt : {4, 8}) {
    const int64_t ch = cdiv(ld, static_cast<int64_t>(kTkThreads) * pt);
    if (rows * ch <= kMaxGroups || pt == 8) {
      p.pt = pt;
      p.chunks = static_cast<int>(ch);
      break;
    }
  }
  p.rows_per_launch = static_cast<int>(std::min<int64_t>(rows, kMaxGroups / std::max(p.chunks, 1)));
  return p;
}

}  // namespace

extern "C" size_t tl_topk_workspace_bytes(int64_t rows, int64_t ld, int64_t k) {
  (void)k;
  if (rows <= 0 || ld <= 0 || ld > kMaxCols) return 0;
  const TopkPlan p = plan_topk(rows, ld);
  const size_t chunk_cols = static_cast<size_t>(kTkThreads) * p.pt;
  return kStateBytes + align256(static_cast<size_t>(rows) * p.chunks * 4) +
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
  const int stage_bytes = kCandBatch / kCandPerThread * (kCandPerThread + 1) * static_cast<int>(sizeof(uint64_t));
  if (int rc = allow_dynamic_lds(reinterpret_cast<const void*>(kern), stage_bytes, "topk"))
    return rc;
  for (int64_t r0 = 0; r0 < rows; r0 += p.rows_per_launch) {
    const int nr = static_cast<int>(std::min<int64_t>(p.rows_per_launch, rows - r0));
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(p.chunks), static_cast<unsigned>(nr)), dim3(kTkThreads), stage_bytes,
                       (hipStream_t)stream, logits, ld, valid_base, (int)k, static_cast<int>(r0), ws, out);
    if (int rc = check_launch("topk")) return rc;
  }
  return kOk;
}
