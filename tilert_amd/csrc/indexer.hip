// DSA lightning-indexer scores over an fp8 key cache:
//   logits[t, l] = k_s[l] * sum_h (w[t,h] * q_s[t(,h)]) * ReLU(q8[t,h] . k8[l])
// which equals sum_h w[t,h] * ReLU(qd[t,h] . kd[l]) on the dequantised inputs because
// every scale is positive (the form of sparse_index_op, ops/sparse_index.py:11-69, on the
// fp8 cache layout of pd_vllm/profiles/mla_nsa.py:211-228).
//
// gfx950 mapping: the M*H query rows form M*H/16 tiles of 16 rows x 128 dims, staged
// once per workgroup through LDS (in MFMA fragment order); each wave holds the tiles of
// its tokens in registers (A operand) and takes its own range of 16-key tiles (B operand,
// 2 KB contiguous each) through the native fp8 MFMA v_mfma_f32_16x16x128_f8f6f4 -- one
// MFMA is a whole 128-long dot product for 16 heads x 16 keys.  Epilogue per MFMA: ReLU
// (one integer max) and the head weight (one FMA); the head sum over a lane's 4 heads
// and a token's tiles stays in registers, and the 4 lane groups are combined with
// v_permlane32_swap / v_permlane16_swap.
#include "common.h"
#include "../../include/tilert_amd.h"

namespace tl {

// ReLU as one integer max on the bit pattern (negative floats are negative integers):
// fmaxf(x, 0) costs two instructions under IEEE mode (a NaN-quieting max first).
__device__ inline float relu(float x) { return __int_as_float(max(__float_as_int(x), 0)); }

constexpr int kIdxWaves = 8;  // waves per workgroup
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// Work split.  A wave scores TW tokens (at most 4 query tiles, held in registers) against
// TPW key tiles; the SPLIT = ceil(M / TW) waves that share a key range sit in the same
// workgroup, KW = 8 / SPLIT ranges per workgroup, KW * TPW contiguous key tiles in all.
//
// Key path: the key cache is row-major [L, 128], but the MFMA wants lane (r, g) to hold
// 32 bytes of key r -- a strided read (16 rows per instruction) that measured ~2 us
// slower over 16 MB than contiguous 1 KB reads.  So the workgroup reads its key tiles
// contiguously into LDS (16-byte chunk c of row r stored at chunk position c ^ (r & 7):
// the MFMA-layout reads are then free of bank conflicts), in PH phases that are all
// requested at kernel start; phase p is computed while the later phases still arrive.
// Query tiles (in MFMA fragment order), folded head weights and key scales are staged
// in LDS by the same loads.  Every loop is unrolled with compile-time trip counts, all
// loads are unconditional (indices clamped), and scores stay in registers until the
// end, so no wait covers a later load or a store.
template <int M, int H, int TW, int TPW>
struct IdxShape {
  static constexpr int TPT = H / 16;              // query tiles per token
  static constexpr int QT = M * TPT;              // query tiles
  static constexpr int QTW = TW * TPT;            // query tiles per wave
  static constexpr int SPLIT = (M + TW - 1) / TW; // waves per key range
  static constexpr int KW = kIdxWaves / SPLIT;    // key ranges per workgroup
  static constexpr int PH = TPW >= 2 ? 2 : 1;     // key phases
  static constexpr int TPP = TPW / PH;            // tiles per range per phase
  static constexpr int PT = KW * TPP;             // tiles per phase (workgroup)
  static constexpr int NT = KW * TPW;             // key tiles per workgroup
  static constexpr int THREADS = kIdxWaves * 64;
  static constexpr int QCH = QT * 128;            // 16-byte query chunks
  static constexpr int QPT = (QCH + THREADS - 1) / THREADS;
  static constexpr int KPT = (PT * 128 + THREADS - 1) / THREADS;  // key chunks per thread per phase
  static constexpr int KSPT = (NT * 16 + THREADS - 1) / THREADS;  // key scales per thread
  // LDS carve-up (bytes)
  static constexpr int Q_OFF = 0;
  static constexpr int WQ_OFF = Q_OFF + QPT * THREADS * 16;
  static constexpr int KS_OFF = WQ_OFF + THREADS * 4;
  static constexpr int K_OFF = KS_OFF + KSPT * THREADS * 4;
  static constexpr int K_BYTES = KPT * THREADS * 16;  // one phase buffer
  static constexpr int LDS = K_OFF + PH * K_BYTES;
  static_assert(kIdxWaves % SPLIT == 0 && TW <= 4 && QT * 16 <= THREADS, "work split");
};

// Key cache layouts.  Flat: fp8 [L, 128] plus fp32 scales [L].  Paged (PAGED): the
// 64-token pages of pd_vllm/profiles/mla_nsa.py:38-41,211-228 -- page p is 64 x 128 fp8
// (8192 B) followed by the 64 tokens' fp32 scales (256 B), 8448 B in all; key l sits in
// page l / 64, row l % 64.  A 16-key tile is still 2 KB contiguous either way.
constexpr int kKiPageKeys = 64;
constexpr int kKiPageBytes = kKiPageKeys * 128 + kKiPageKeys * 4;  // 8448

template <bool PAGED>
__device__ inline int64_t key_tile_byte(int tile) {
  return PAGED ? static_cast<int64_t>(tile >> 2) * kKiPageBytes + (tile & 3) * 2048 : static_cast<int64_t>(tile) * 2048;
}

template <int M, int H, int TW, int TPW, bool PAGED>
__global__ __launch_bounds__(kIdxWaves * 64) void indexer_kernel(
    const uint8_t* __restrict__ q, const float* __restrict__ q_s, int q_s_per_head,
    const uint8_t* __restrict__ k, const float* __restrict__ k_s, const uint16_t* __restrict__ w,
    float* __restrict__ logits, int L, int64_t ld, int64_t cur_pos, int n_tiles) {
  using S = IdxShape<M, H, TW, TPW>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int t0 = (wave % S::SPLIT) * TW;  // first token of this wave
  const int rr = wave / S::SPLIT;         // key range of this wave
  const int wg_tile = blockIdx.x * S::NT; // first key tile of the workgroup

  // ---- all global loads, issued together
  // query chunk d of the LDS image (fragment order): tile d / 128, piece (d / 64) % 2,
  // lane d % 64 -> row 16 qt + l % 16, 16-byte piece 4 p + l / 16 of that row
  uint4 qv[S::QPT];
#pragma unroll
  for (int u = 0; u < S::QPT; ++u) {
    const int d = min(tid + u * S::THREADS, S::QCH - 1);
    const int qt = d >> 7, pp = (d >> 6) & 1, l = d & 63;
    qv[u] = reinterpret_cast<const uint4*>(q)[((qt * 16 + (l & 15)) << 3) + pp * 4 + (l >> 4)];
  }
  const int wrow = min(tid, S::QT * 16 - 1);
  const float wqv = bf16_to_f32(w[wrow]) * q_s[q_s_per_head ? wrow : wrow / H];
  float ksv[S::KSPT];
#pragma unroll
  for (int u = 0; u < S::KSPT; ++u) {
    const int e = tid + u * S::THREADS;  // key e % 16 of workgroup tile e / 16
    const int key = min(min(wg_tile + e / 16, n_tiles - 1) * 16 + (e & 15), L - 1);
    ksv[u] = PAGED ? *reinterpret_cast<const float*>(k + static_cast<int64_t>(key / kKiPageKeys) * kKiPageBytes +
                                                     kKiPageKeys * 128 + (key % kKiPageKeys) * 4)
                   : k_s[key];
  }
  // key chunk c of phase p: phase tile pt = c / 128 (range pt / TPP, its tile
  // p * TPP + pt % TPP), row (c / 8) % 16, 16-byte chunk c % 8 -- contiguous 1 KB reads
  auto key_src = [&](int p, int c) {
    const int pt = min(c >> 7, S::PT - 1);
    const int tile = min(wg_tile + (pt / S::TPP) * TPW + p * S::TPP + pt % S::TPP, n_tiles - 1);
    const int64_t byte = key_tile_byte<PAGED>(tile) + (c & 127) * 16;
    // flat: a short last tile stops at the cache end; paged: pages are whole
    return reinterpret_cast<const u32x4v*>(k + (PAGED ? byte : min(byte, static_cast<int64_t>(L) * kBlock - 16)));
  };
  u32x4v kv[S::PH][S::KPT];
#pragma unroll
  for (int p = 0; p < S::PH; ++p)
#pragma unroll
    for (int u = 0; u < S::KPT; ++u) kv[p][u] = __builtin_nontemporal_load(key_src(p, tid + u * S::THREADS));

  // ---- stage queries, weights, key scales and key phase 0
  uint4* q_lds = reinterpret_cast<uint4*>(smem + S::Q_OFF);
  float* wq_lds = reinterpret_cast<float*>(smem + S::WQ_OFF);
  float* ks_lds = reinterpret_cast<float*>(smem + S::KS_OFF);
  auto key_lds = [&](int p) { return smem + S::K_OFF + p * S::K_BYTES; };
  auto put_keys = [&](int p) {
#pragma unroll
    for (int u = 0; u < S::KPT; ++u) {
      const int c = tid + u * S::THREADS;  // chunks past the phase land in the padding
      const int row = (c >> 3) & 15, ch = c & 7;
      *reinterpret_cast<u32x4v*>(key_lds(p) + (c >> 7) * 2048 + row * 128 + ((ch ^ (row & 7)) << 4)) = kv[p][u];
    }
  };
#pragma unroll
  for (int u = 0; u < S::QPT; ++u) q_lds[tid + u * S::THREADS] = qv[u];
  wq_lds[tid] = wqv;
#pragma unroll
  for (int u = 0; u < S::KSPT; ++u) ks_lds[tid + u * S::THREADS] = ksv[u];
  put_keys(0);
  __syncthreads();

  // ---- this wave's query tiles (A operands) and head weights; tokens past M (a short
  //      last group) repeat token M-1 and are not stored
  v8i qa[S::QTW];
  float4 wq[S::QTW];
#pragma unroll
  for (int j = 0; j < S::QTW; ++j) {
    const int qt = min(t0 + j / S::TPT, M - 1) * S::TPT + j % S::TPT;
    const uint4 lo = q_lds[qt * 128 + lane];
    const uint4 hi = q_lds[qt * 128 + 64 + lane];
    qa[j] = v8i{static_cast<int>(lo.x), static_cast<int>(lo.y), static_cast<int>(lo.z), static_cast<int>(lo.w),
                static_cast<int>(hi.x), static_cast<int>(hi.y), static_cast<int>(hi.z), static_cast<int>(hi.w)};
    wq[j] = *reinterpret_cast<const float4*>(wq_lds + qt * 16 + 4 * g);
  }

  float out[TPW];  // lane group g < TW: token t0 + g of key r
#pragma unroll
  for (int p = 0; p < S::PH; ++p) {
    if (p > 0) {  // the next phase's keys have (mostly) arrived while this one computed
      put_keys(p);
      __syncthreads();
    }
#pragma unroll
    for (int ii = 0; ii < S::TPP; ++ii) {
      const int i = p * S::TPP + ii;
      const uint8_t* tile = key_lds(p) + (rr * S::TPP + ii) * 2048 + r * 128;
      const uint4 lo = *reinterpret_cast<const uint4*>(tile + ((g ^ (r & 7)) << 4));
      const uint4 hi = *reinterpret_cast<const uint4*>(tile + (((g + 4) ^ (r & 7)) << 4));
      const v8i kt = {static_cast<int>(lo.x), static_cast<int>(lo.y), static_cast<int>(lo.z), static_cast<int>(lo.w),
                      static_cast<int>(hi.x), static_cast<int>(hi.y), static_cast<int>(hi.z), static_cast<int>(hi.w)};
      // all MFMAs of the tile first, into separate results, then the epilogue
      v4f c[S::QTW];
#pragma unroll
      for (int j = 0; j < S::QTW; ++j) c[j] = mfma_16x16x128_fp8(qa[j], kt);
      const float ksc = ks_lds[(rr * TPW + i) * 16 + r];
      float score[TW];
#pragma unroll
      for (int t = 0; t < TW; ++t) {
        float acc = 0.f;
#pragma unroll
        for (int jj = 0; jj < S::TPT; ++jj) {
          const int j = t * S::TPT + jj;
          acc = __builtin_fmaf(relu(c[j][0]), wq[j].x, acc);
          acc = __builtin_fmaf(relu(c[j][1]), wq[j].y, acc);
          acc = __builtin_fmaf(relu(c[j][2]), wq[j].z, acc);
          acc = __builtin_fmaf(relu(c[j][3]), wq[j].w, acc);
        }
        // lanes r, r+16, r+32, r+48 hold the 4 partial head sums of key r: sum them with
        // the gfx950 lane-swap instructions (VALU, no LDS round trip)
        const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc), __float_as_uint(acc), false, false);
        const float y = __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
        const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
        score[t] = (__uint_as_float(s16[0]) + __uint_as_float(s16[1])) * ksc;
      }
      float v = score[0];
#pragma unroll
      for (int tt = 1; tt < TW; ++tt)
        if (tt == g) v = score[tt];
      out[i] = v;
    }
  }

  // lane group g stores token t0 + g: a 64-byte row segment per tile
  const int tok = t0 + g;
  const int t_begin = wg_tile + rr * TPW;
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int key = (t_begin + i) * 16 + r;
    if (g < TW && tok < M && t_begin + i < n_tiles && key < L)
      logits[static_cast<int64_t>(tok) * ld + key] = static_cast<int64_t>(key) > cur_pos + tok ? -__builtin_inff() : out[i];
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

constexpr int kIdxMaxWaves = 4096;  // 16 per CU: beyond that a wave takes more key tiles

template <int M, int H, int TW, int TPW, bool PAGED>
static int launch_indexer_t(hipStream_t st, const uint8_t* q, const float* q_s, int per_head,
                            const uint8_t* k, const float* k_s, const uint16_t* w, float* logits,
                            int L, int64_t ld, int64_t cur_pos, int n_tiles) {
  using S = IdxShape<M, H, TW, TPW>;
  const void* fn = reinterpret_cast<const void*>(indexer_kernel<M, H, TW, TPW, PAGED>);
  if (S::LDS > 64 * 1024) {
    const int rc = allow_dynamic_lds(fn, S::LDS, "indexer");
    if (rc) return rc;
  }
  const dim3 grid(static_cast<unsigned>(cdiv(n_tiles, static_cast<int64_t>(S::NT))));
  hipLaunchKernelGGL((indexer_kernel<M, H, TW, TPW, PAGED>), grid, dim3(kIdxWaves * 64), S::LDS, st, q, q_s, per_head, k,
                     k_s, w, logits, L, ld, cur_pos, n_tiles);
  return check_launch("indexer");
}

// Tokens per wave: at most 4 query tiles (one token at H = 64), so a wave stays near 100
// VGPRs and 4 waves share each SIMD (measured 5% faster than 8 query tiles at 2 waves per
// SIMD); raised where needed so that the waves sharing a key range divide the workgroup.
constexpr int pick_tw(int M, int TPT) {
  int tw = (4 / TPT < M) ? 4 / TPT : M;
  while (tw < M && (kIdxWaves % ((M + tw - 1) / tw) != 0)) ++tw;
  return tw;
}

template <int M, int H, bool PAGED>
static int launch_indexer(hipStream_t st, const uint8_t* q, const float* q_s, int per_head,
                          const uint8_t* k, const float* k_s, const uint16_t* w, float* logits,
                          int L, int64_t ld, int64_t cur_pos, int n_tiles) {
  constexpr int TPT = H / 16;
  constexpr int TW = pick_tw(M, TPT);
  constexpr int SPLIT = (M + TW - 1) / TW;
  // smallest tiles-per-wave that keeps the grid within 8 waves per CU
  int tpw = 1;
  while (tpw < 8 && static_cast<int64_t>(n_tiles) * SPLIT > static_cast<int64_t>(kIdxMaxWaves) * tpw) tpw *= 2;
  switch (tpw) {
    case 1: return launch_indexer_t<M, H, TW, 1, PAGED>(st, q, q_s, per_head, k, k_s, w, logits, L, ld, cur_pos, n_tiles);
    case 2: return launch_indexer_t<M, H, TW, 2, PAGED>(st, q, q_s, per_head, k, k_s, w, logits, L, ld, cur_pos, n_tiles);
    case 4: return launch_indexer_t<M, H, TW, 4, PAGED>(st, q, q_s, per_head, k, k_s, w, logits, L, ld, cur_pos, n_tiles);
    default: return launch_indexer_t<M, H, TW, 8, PAGED>(st, q, q_s, per_head, k, k_s, w, logits, L, ld, cur_pos, n_tiles);
  }
}

template <bool PAGED>
static int indexer_scores(const char* who, const void* q_fp8, const float* q_s, int q_s_per_head, const void* k_fp8,
                          const float* k_s, const void* w_bf16, float* logits, int64_t M, int64_t H, int64_t L,
                          int64_t ld, int64_t cur_pos, void* stream) {
  if (H != 32 && H != 64) { set_error("%s: H=%lld must be 32 or 64", who, (long long)H); return kErrUnsupported; }
  if (M < 1 || M * H > 256) { set_error("%s: need 1 <= M and M*H <= 256 (M=%lld H=%lld)", who, (long long)M, (long long)H); return kErrUnsupported; }
  if (L < 0 || L > (1ll << 30) || ld < L) { set_error("%s: bad L=%lld / ld=%lld", who, (long long)L, (long long)ld); return kErrArg; }
  if (cur_pos < 0) { set_error("%s: cur_pos=%lld must be >= 0", who, (long long)cur_pos); return kErrArg; }
  if (!q_fp8 || !q_s || !k_fp8 || (!PAGED && !k_s) || !w_bf16 || !logits) { set_error("%s: null pointer", who); return kErrArg; }
  if ((reinterpret_cast<uintptr_t>(q_fp8) | reinterpret_cast<uintptr_t>(k_fp8)) & 15) { set_error("%s: q and k must be 16-byte aligned", who); return kErrArg; }
  if (L == 0) return kOk;
  hipStream_t st = (hipStream_t)stream;
  // keys past the last token's position are masked for every token: no need to read them
  const int64_t visible = cur_pos + M < L ? cur_pos + M : L;
  const int n_tiles = static_cast<int>(cdiv(visible, 16));
  if (visible < L) {
    const int64_t n = (L - visible) * M;
    hipLaunchKernelGGL(fill_masked_kernel, dim3(cdiv(n, 256)), dim3(256), 0, st, logits, (int)M, ld, visible, L);
  }
  const uint8_t* q = (const uint8_t*)q_fp8;
  const uint8_t* k = (const uint8_t*)k_fp8;
  const uint16_t* w = (const uint16_t*)w_bf16;
  const int Li = static_cast<int>(L);
#define TL_IDX(MM, HH) \
  if (M == MM && H == HH) return launch_indexer<MM, HH, PAGED>(st, q, q_s, q_s_per_head, k, k_s, w, logits, Li, ld, cur_pos, n_tiles);
  TL_IDX(1, 64) TL_IDX(2, 64) TL_IDX(3, 64) TL_IDX(4, 64)
  TL_IDX(1, 32) TL_IDX(2, 32) TL_IDX(3, 32) TL_IDX(4, 32) TL_IDX(5, 32) TL_IDX(6, 32) TL_IDX(7, 32) TL_IDX(8, 32)
#undef TL_IDX
  set_error("%s: unsupported M=%lld H=%lld", who, (long long)M, (long long)H);
  return kErrUnsupported;
}

// One thread per 8 key elements, 16 threads per key: quantise the key like act_quant
// (amax, scale by scale_mode, e4m3fn of the clamped quotient) and write it into its page.
__global__ __launch_bounds__(256) void ki_write_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ pages,
                                                       int64_t rows, int64_t pos, int scale_mode) {
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t row = tid >> 4;
  const bool live = row < rows;
  uint4 raw = make_uint4(0, 0, 0, 0);
  if (live) raw = reinterpret_cast<const uint4*>(x)[tid];
  float v[8];
  v[0] = bf16_to_f32(raw.x & 0xffff); v[1] = bf16_to_f32(raw.x >> 16);
  v[2] = bf16_to_f32(raw.y & 0xffff); v[3] = bf16_to_f32(raw.y >> 16);
  v[4] = bf16_to_f32(raw.z & 0xffff); v[5] = bf16_to_f32(raw.z >> 16);
  v[6] = bf16_to_f32(raw.w & 0xffff); v[7] = bf16_to_f32(raw.w >> 16);
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, __builtin_fabsf(v[i]));
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 16));
  const float sc = group_scale(amax, scale_mode);
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lo |= f32_to_e4m3(fminf(fmaxf(v[i] / sc, -kE4m3Max), kE4m3Max)) << (8 * i);
    hi |= f32_to_e4m3(fminf(fmaxf(v[i + 4] / sc, -kE4m3Max), kE4m3Max)) << (8 * i);
  }
  if (live) {
    const int64_t key = pos + row;
    uint8_t* page = pages + (key / kKiPageKeys) * kKiPageBytes;
    const int r = static_cast<int>(key % kKiPageKeys);
    *reinterpret_cast<uint2*>(page + r * 128 + (tid & 15) * 8) = make_uint2(lo, hi);
    if ((tid & 15) == 0) *reinterpret_cast<float*>(page + kKiPageKeys * 128 + r * 4) = sc;
  }
}


// ------------------------------------------------------------- indexer key producer
// LayerNormRoPERotate (ops/layernorm_rope_rotate.py:23-82, golden :206-220) for 128-wide
// indexer keys: k = bf16(LayerNorm(x) * weight + bias) (eps as given, biased variance);
// dims 0..63 take the non-interleaved RoPE (element i pairs with i + 32 as a complex
// number times freqs[i] = (cos, sin), tilert/models/utils.py:121-145), rounded to bf16;
// then the 128-point Hadamard transform with scale 128^-1/2 (rotate_activation,
// ops/rotate.py:17-21), rounded to bf16.  One wave per token: lane l holds elements l and
// l + 64, so the norm's sums are wave reductions, the RoPE partner of element l < 32 is
// lane l + 32 (and back), and the transform is the within-lane butterfly (bit 6) plus six
// cross-lane butterflies (bits 0..5).  Token t lands at row *cur_pos + t: of the bf16 key
// cache (KI = false, the reference op's output), or quantised per token into its KI page
// (KI = true, the format tl_ki_cache_write writes).  Rows outside the cache are dropped.
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ inline float bf16_round(float v) { return bf16_to_f32(f32_to_bf16(v)); }

template <bool KI>
__global__ __launch_bounds__(256) void ln_rope_rotate_kernel(
    const uint16_t* __restrict__ x, int64_t seq, const int32_t* __restrict__ cur_pos, uint16_t* __restrict__ cache,
    int64_t cache_rows, uint8_t* __restrict__ pages, const float* __restrict__ weight, const float* __restrict__ bias,
    const float* __restrict__ freqs, float eps, int scale_mode) {
  const int64_t tok = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (tok >= seq) return;  // wave-uniform
  const uint16_t* xr = x + tok * 128;
  const float x0 = bf16_to_f32(xr[lane]), x1 = bf16_to_f32(xr[lane + 64]);
  const float w0 = weight[lane], w1 = weight[lane + 64], b0 = bias[lane], b1 = bias[lane + 64];
  const int i = lane & 31;
  const float fc = freqs[tok * 64 + 2 * i], fs = freqs[tok * 64 + 2 * i + 1];
  const int64_t row = static_cast<int64_t>(*cur_pos) + tok;

  // LayerNorm in fp32: mean, biased variance, 1 / sqrt(var + eps)
  const float mean = wave_sum(x0 + x1) * (1.0f / 128.0f);
  const float d0 = x0 - mean, d1 = x1 - mean;
  const float var = wave_sum(d0 * d0 + d1 * d1) * (1.0f / 128.0f);
  const float rstd = 1.0f / sqrtf(var + eps);
  float v0 = bf16_round(d0 * rstd * w0 + b0);
  float v1 = bf16_round(d1 * rstd * w1 + b1);
  // RoPE on elements 0..63 (v0 of every lane): (re, im) = (x_i, x_{i+32}) times (c, s)
  const float p = __shfl_xor(v0, 32);
  v0 = bf16_round(lane < 32 ? v0 * fc - p * fs : p * fs + v0 * fc);
  // Hadamard: bit 6 inside the lane, bits 5..0 across lanes
  {
    const float a = v0, b = v1;
    v0 = a + b;
    v1 = a - b;
  }
#pragma unroll
  for (int bit = 32; bit >= 1; bit >>= 1) {
    const float q0 = __shfl_xor(v0, bit), q1 = __shfl_xor(v1, bit);
    const bool hi = lane & bit;
    v0 = hi ? q0 - v0 : v0 + q0;
    v1 = hi ? q1 - v1 : v1 + q1;
  }
  constexpr float kScale = 0.08838834764831845f;  // fp32(128^-1/2)
  const uint16_t o0 = f32_to_bf16(v0 * kScale), o1 = f32_to_bf16(v1 * kScale);
  if (row < 0 || row >= cache_rows) return;  // wave-uniform: outside the cache
  if constexpr (!KI) {
    uint16_t* dst = cache + row * 128;
    dst[lane] = o0;
    dst[lane + 64] = o1;
  } else {
    // the key's act_quant over its 128 bf16 values (as ki_write_kernel)
    const float f0 = bf16_to_f32(o0), f1 = bf16_to_f32(o1);
    float amax = fmaxf(__builtin_fabsf(f0), __builtin_fabsf(f1));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    const float sc = group_scale(amax, scale_mode);
    uint8_t* page = pages + (row / kKiPageKeys) * kKiPageBytes;
    const int r = static_cast<int>(row % kKiPageKeys);
    page[r * 128 + lane] = static_cast<uint8_t>(f32_to_e4m3(fminf(fmaxf(f0 / sc, -kE4m3Max), kE4m3Max)));
    page[r * 128 + lane + 64] = static_cast<uint8_t>(f32_to_e4m3(fminf(fmaxf(f1 / sc, -kE4m3Max), kE4m3Max)));
    if (lane == 0) *reinterpret_cast<float*>(page + kKiPageKeys * 128 + r * 4) = sc;
  }
}

}  // namespace tl

using namespace tl;

extern "C" int tl_indexer_fp8_scores(const void* q_fp8, const float* q_s, int q_s_per_head,
                                     const void* k_fp8, const float* k_s, const void* w_bf16,
                                     float* logits, int64_t M, int64_t H, int64_t L, int64_t ld,
                                     int64_t cur_pos, void* stream) {
  return indexer_scores<false>("indexer", q_fp8, q_s, q_s_per_head, k_fp8, k_s, w_bf16, logits, M, H, L, ld, cur_pos,
                               stream);
}

extern "C" int tl_indexer_fp8_scores_paged(const void* q_fp8, const float* q_s, int q_s_per_head,
                                           const void* ki_pages, int64_t n_pages, const void* w_bf16,
                                           float* logits, int64_t M, int64_t H, int64_t L, int64_t ld,
                                           int64_t cur_pos, void* stream) {
  if (n_pages < 0 || L > n_pages * kKiPageKeys) {
    set_error("indexer_paged: L=%lld keys need %lld pages (got %lld)", (long long)L, (long long)cdiv(L, kKiPageKeys), (long long)n_pages);
    return kErrArg;
  }
  return indexer_scores<true>("indexer_paged", q_fp8, q_s, q_s_per_head, ki_pages, nullptr, w_bf16, logits, M, H, L, ld,
                              cur_pos, stream);
}

extern "C" int tl_ki_cache_write(const void* k_bf16, int64_t rows, void* ki_pages, int64_t n_pages, int64_t pos,
                                 int scale_mode, void* stream) {
  if (rows < 0 || pos < 0 || pos + rows > n_pages * kKiPageKeys) {
    set_error("ki_cache_write: keys [%lld, %lld) exceed %lld pages", (long long)pos, (long long)(pos + rows), (long long)n_pages);
    return kErrArg;
  }
  if (scale_mode < 0 || scale_mode > 2) { set_error("ki_cache_write: bad scale_mode %d", scale_mode); return kErrArg; }
  if (!k_bf16 || !ki_pages) { set_error("ki_cache_write: null pointer"); return kErrArg; }
  if ((reinterpret_cast<uintptr_t>(k_bf16) | reinterpret_cast<uintptr_t>(ki_pages)) & 15) { set_error("ki_cache_write: pointers must be 16-byte aligned"); return kErrArg; }
  if (rows == 0) return kOk;
  hipLaunchKernelGGL(ki_write_kernel, dim3(cdiv(rows * 16, 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)k_bf16, (uint8_t*)ki_pages, rows, pos, scale_mode);
  return check_launch("ki_cache_write");
}

static int ln_rope_rotate_check(const char* who, const void* x, int64_t seq, const int32_t* cur_pos, const void* out,
                                const float* weight, const float* bias, const float* freqs) {
  if (seq < 0 || seq > (1ll << 24)) { set_error("%s: seq=%lld out of range", who, (long long)seq); return kErrArg; }
  if (!x || !cur_pos || !out || !weight || !bias || !freqs) { set_error("%s: null pointer", who); return kErrArg; }
  return kOk;
}

extern "C" int tl_layernorm_rope_rotate(const void* x_bf16, int64_t seq, const int32_t* cur_pos, void* k_cache_bf16,
                                        int64_t cache_rows, const float* weight, const float* bias, const float* freqs,
                                        float eps, void* stream) {
  if (int rc = ln_rope_rotate_check("layernorm_rope_rotate", x_bf16, seq, cur_pos, k_cache_bf16, weight, bias, freqs))
    return rc;
  if (cache_rows < 0) { set_error("layernorm_rope_rotate: cache_rows=%lld", (long long)cache_rows); return kErrArg; }
  if (seq == 0) return kOk;
  hipLaunchKernelGGL(ln_rope_rotate_kernel<false>, dim3(static_cast<unsigned>(cdiv(seq, 4))), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)x_bf16, seq, cur_pos, (uint16_t*)k_cache_bf16, cache_rows,
                     nullptr, weight, bias, freqs, eps, 0);
  return check_launch("layernorm_rope_rotate");
}

extern "C" int tl_layernorm_rope_rotate_ki(const void* x_bf16, int64_t seq, const int32_t* cur_pos, void* ki_pages,
                                           int64_t n_pages, const float* weight, const float* bias, const float* freqs,
                                           float eps, int scale_mode, void* stream) {
  if (int rc = ln_rope_rotate_check("layernorm_rope_rotate_ki", x_bf16, seq, cur_pos, ki_pages, weight, bias, freqs))
    return rc;
  if (n_pages < 0) { set_error("layernorm_rope_rotate_ki: n_pages=%lld", (long long)n_pages); return kErrArg; }
  if (scale_mode < 0 || scale_mode > 2) { set_error("layernorm_rope_rotate_ki: bad scale_mode %d", scale_mode); return kErrArg; }
  if (seq == 0) return kOk;
  hipLaunchKernelGGL(ln_rope_rotate_kernel<true>, dim3(static_cast<unsigned>(cdiv(seq, 4))), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)x_bf16, seq, cur_pos, nullptr, n_pages * kKiPageKeys,
                     (uint8_t*)ki_pages, weight, bias, freqs, eps, scale_mode);
  return check_launch("layernorm_rope_rotate_ki");
}
