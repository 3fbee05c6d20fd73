// Exact per-row top-k by radix select (the contract of topk_accurate_op, ops/topk.py:62-109;
// its golden is torch.topk, :128-143).
//
// Scores are mapped to order-preserving 32-bit keys (larger score = larger key).  Three
// passes over the row find the k-th largest key T digit by digit (11, 11, 10 bits): each
// pass builds per-workgroup LDS histograms of the next digit among the elements that
// match the prefix found so far, merges them into a per-row global histogram with
// agent-scope atomics, and the last workgroup of the row to finish picks the digit.  A
// count pass and a write pass then emit, in ascending index order, every element with
// key > T plus the lowest-index elements with key == T until k are taken -- so the output
// set is exact and deterministic, ties included.
//
// Rows are the topk_accurate samples: row i considers columns [0, valid_base + 1 + i).
#include "common.h"
#include "../../include/tilert_amd.h"

namespace tl {

constexpr int kTopkThreads = 256;
constexpr int kChunk = 4096;     // elements per workgroup per row
constexpr int kBins = 2048;      // max digit width 11 bits
constexpr int kMaxK = 8192;

struct RowState {
  uint32_t prefix;  // key bits decided so far (right-aligned)
  int32_t k_rem;    // still to take among elements matching the prefix
  uint32_t pad[2];
};

// Workspace layout (bytes): [hist rows*kBins u32][counter rows u32][state rows RowState]
// [counts rows*chunks*2 u32]
struct TopkWs {
  uint32_t* hist;
  uint32_t* counter;
  RowState* state;
  uint32_t* counts;
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

__host__ __device__ inline TopkWs carve(void* base, int64_t rows, int64_t chunks) {
  char* p = static_cast<char*>(base);
  TopkWs w;
  w.hist = reinterpret_cast<uint32_t*>(p);
  p += align256(rows * kBins * sizeof(uint32_t));
  w.counter = reinterpret_cast<uint32_t*>(p);
  p += align256(rows * sizeof(uint32_t));
  w.state = reinterpret_cast<RowState*>(p);
  p += align256(rows * sizeof(RowState));
  w.counts = reinterpret_cast<uint32_t*>(p);
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

// pass 0: bits 31..21, pass 1: 20..10, pass 2: 9..0
__device__ inline int pass_shift(int p) { return p == 0 ? 21 : (p == 1 ? 10 : 0); }
__device__ inline int pass_width(int p) { return p == 2 ? 10 : 11; }

__global__ __launch_bounds__(kTopkThreads) void radix_pass_kernel(const float* __restrict__ logits, int64_t ld,
                                                                  int64_t valid_base, int k, TopkWs ws, int pass) {
  __shared__ uint32_t h[kBins];
  __shared__ uint32_t part[kTopkThreads];
  __shared__ int last;
  const int row = blockIdx.y;
  const int n = row_valid(row, valid_base, ld);
  if (n <= k) return;  // the whole row is selected
  const int shift = pass_shift(pass), width = pass_width(pass);
  const uint32_t nb = 1u << width;
  uint32_t prefix = 0;
  int k_rem = k;
  if (pass > 0) {
    prefix = ws.state[row].prefix;
    k_rem = ws.state[row].k_rem;
  }
  for (uint32_t b = threadIdx.x; b < nb; b += kTopkThreads) h[b] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kChunk;
  const float* src = logits + static_cast<int64_t>(row) * ld;
  for (int i = threadIdx.x; i < kChunk; i += kTopkThreads) {
    const int64_t c = base + i;
    if (c < n) {
      const uint32_t key = order_key(src[c]);
      const bool match = pass == 0 || (key >> (shift + width)) == prefix;
      if (match) atomicAdd(&h[(key >> shift) & (nb - 1)], 1u);
    }
  }
  __syncthreads();
  uint32_t* gh = ws.hist + static_cast<size_t>(row) * kBins;
  for (uint32_t b = threadIdx.x; b < nb; b += kTopkThreads)
    if (h[b]) __hip_atomic_fetch_add(&gh[b], h[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t chunks = gridDim.x;
    const uint32_t prev = __hip_atomic_fetch_add(&ws.counter[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = prev == chunks - 1;
  }
  __syncthreads();
  if (!last) return;

  // ---- last workgroup of the row: pick the digit holding the k_rem-th largest key
  for (uint32_t b = threadIdx.x; b < nb; b += kTopkThreads) {
    h[b] = __hip_atomic_load(&gh[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&gh[b], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  // thread j owns the bins [nb - (j+1)*per, nb - j*per) (descending digit order)
  const uint32_t per = nb / kTopkThreads;
  const uint32_t hi = nb - threadIdx.x * per;
  uint32_t s = 0;
  for (uint32_t b = hi - per; b < hi; ++b) s += h[b];
  part[threadIdx.x] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t above = 0;  // elements with a larger digit
    int j = 0;
    for (; j < kTopkThreads; ++j) {
      if (above + part[j] >= static_cast<uint32_t>(k_rem)) break;
      above += part[j];
    }
    const uint32_t top = nb - j * per;
    uint32_t d = top - 1;
    for (;; --d) {
      if (above + h[d] >= static_cast<uint32_t>(k_rem)) break;
      above += h[d];
    }
    ws.state[row].prefix = (prefix << width) | d;
    ws.state[row].k_rem = k_rem - static_cast<int>(above);
    __hip_atomic_store(&ws.counter[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// per chunk: number of keys > T and == T
__global__ __launch_bounds__(kTopkThreads) void count_kernel(const float* __restrict__ logits, int64_t ld,
                                                             int64_t valid_base, int k, TopkWs ws) {
  __shared__ uint32_t sgt, seq;
  const int row = blockIdx.y;
  const int n = row_valid(row, valid_base, ld);
  if (n <= k) return;
  if (threadIdx.x == 0) { sgt = 0; seq = 0; }
  __syncthreads();
  const uint32_t T = ws.state[row].prefix;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kChunk;
  const float* src = logits + static_cast<int64_t>(row) * ld;
  uint32_t gt = 0, eq = 0;
  for (int i = threadIdx.x; i < kChunk; i += kTopkThreads) {
    const int64_t c = base + i;
    if (c < n) {
      const uint32_t key = order_key(src[c]);
      gt += key > T;
      eq += key == T;
    }
  }
  atomicAdd(&sgt, gt);
  atomicAdd(&seq, eq);
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t* cnt = ws.counts + (static_cast<size_t>(row) * gridDim.x + blockIdx.x) * 2;
    cnt[0] = sgt;
    cnt[1] = seq;
  }
}

// Emit the selected indices of this chunk in ascending order at their global rank.
__global__ __launch_bounds__(kTopkThreads) void write_kernel(const float* __restrict__ logits, int64_t ld,
                                                             int64_t valid_base, int k, TopkWs ws,
                                                             int32_t* __restrict__ out) {
  __shared__ uint32_t wsel[kTopkThreads / 64], weq[kTopkThreads / 64];
  __shared__ uint32_t s_sel_base, s_eq_base;
  const int row = blockIdx.y;
  const int n = row_valid(row, valid_base, ld);
  int32_t* o = out + static_cast<int64_t>(row) * k;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kChunk;
  if (n <= k) {  // everything valid is selected; pad with -1
    for (int i = threadIdx.x; i < kChunk; i += kTopkThreads) {
      const int64_t c = base + i;
      if (c < k) o[c] = c < n ? static_cast<int32_t>(c) : -1;
    }
    if (blockIdx.x == 0)  // k may exceed the chunked range
      for (int64_t c = static_cast<int64_t>(gridDim.x) * kChunk + threadIdx.x; c < k; c += kTopkThreads)
        o[c] = c < n ? static_cast<int32_t>(c) : -1;
    return;
  }
  const uint32_t T = ws.state[row].prefix;
  const uint32_t need_eq = static_cast<uint32_t>(ws.state[row].k_rem);
  if (threadIdx.x == 0) {
    uint32_t gt = 0, eq = 0;
    const uint32_t* cnt = ws.counts + static_cast<size_t>(row) * gridDim.x * 2;
    for (uint32_t c = 0; c < blockIdx.x; ++c) {
      gt += cnt[2 * c];
      eq += cnt[2 * c + 1];
    }
    s_sel_base = gt + (eq < need_eq ? eq : need_eq);
    s_eq_base = eq;
  }
  __syncthreads();
  const float* src = logits + static_cast<int64_t>(row) * ld;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int i0 = 0; i0 < kChunk; i0 += kTopkThreads) {
    const int64_t c = base + i0 + threadIdx.x;
    uint32_t key = 0;
    bool valid = c < n;
    if (valid) key = order_key(src[c]);
    const bool is_eq = valid && key == T;
    const bool is_gt = valid && key > T;
    // rank of this element among the chunk's equals so far (ascending index)
    const uint64_t eq_mask = __ballot(is_eq);
    const uint32_t eq_lane = __builtin_popcountll(eq_mask & ((1ull << lane) - 1));
    if (lane == 0) weq[wave] = __builtin_popcountll(eq_mask);
    __syncthreads();
    uint32_t eq_before_wave = 0;
    for (int w = 0; w < wave; ++w) eq_before_wave += weq[w];
    const uint32_t eq_rank = s_eq_base + eq_before_wave + eq_lane;
    const bool sel = is_gt || (is_eq && eq_rank < need_eq);
    const uint64_t sel_mask = __ballot(sel);
    const uint32_t sel_lane = __builtin_popcountll(sel_mask & ((1ull << lane) - 1));
    if (lane == 0) wsel[wave] = __builtin_popcountll(sel_mask);
    __syncthreads();
    uint32_t sel_before_wave = 0, sel_total = 0, eq_total = 0;
    for (int w = 0; w < kTopkThreads / 64; ++w) {
      if (w < wave) sel_before_wave += wsel[w];
      sel_total += wsel[w];
      eq_total += weq[w];
    }
    if (sel) o[s_sel_base + sel_before_wave + sel_lane] = static_cast<int32_t>(c);
    __syncthreads();
    if (threadIdx.x == 0) {
      s_sel_base += sel_total;
      s_eq_base += eq_total;
    }
    __syncthreads();
  }
}

}  // namespace tl

using namespace tl;

static int64_t topk_chunks(int64_t ld) { return cdiv(ld, kChunk); }

extern "C" size_t tl_topk_workspace_bytes(int64_t rows, int64_t ld, int64_t k) {
  (void)k;
  if (rows <= 0 || ld <= 0) return 0;
  const int64_t chunks = topk_chunks(ld);
  return align256(rows * kBins * 4) + align256(rows * 4) + align256(rows * sizeof(RowState)) +
         align256(rows * chunks * 2 * 4);
}

extern "C" int tl_topk_rows(const float* logits, int64_t rows, int64_t ld, int64_t valid_base, int64_t k,
                            int32_t* out, void* workspace, size_t workspace_bytes, void* stream) {
  if (rows <= 0 || ld <= 0) { set_error("topk: empty input (rows=%lld ld=%lld)", (long long)rows, (long long)ld); return kErrArg; }
  if (k < 1 || k > kMaxK) { set_error("topk: k=%lld must be in [1, %d]", (long long)k, kMaxK); return kErrUnsupported; }
  if (rows > 65535 || ld > (1ll << 30)) { set_error("topk: too many rows or columns"); return kErrArg; }
  if (!logits || !out) { set_error("topk: null pointer"); return kErrArg; }
  const size_t need = tl_topk_workspace_bytes(rows, ld, k);
  if (!workspace || workspace_bytes < need) { set_error("topk: workspace of %zu bytes required (got %zu)", need, workspace_bytes); return kErrArg; }
  const int64_t chunks = topk_chunks(ld);
  const TopkWs ws = carve(workspace, rows, chunks);
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(rows));
  for (int p = 0; p < 3; ++p)
    hipLaunchKernelGGL(radix_pass_kernel, grid, dim3(kTopkThreads), 0, st, logits, ld, valid_base, (int)k, ws, p);
  hipLaunchKernelGGL(count_kernel, grid, dim3(kTopkThreads), 0, st, logits, ld, valid_base, (int)k, ws);
  hipLaunchKernelGGL(write_kernel, grid, dim3(kTopkThreads), 0, st, logits, ld, valid_base, (int)k, ws, out);
  return check_launch("topk");
}
