// DSA lightning-indexer scores over an fp8 key cache:
//   logits[t, l] = k_s[l] * sum_h (w[t,h] * q_s[t(,h)]) * ReLU(q8[t,h] . k8[l])
// which equals sum_h w[t,h] * ReLU(qd[t,h] . kd[l]) on the dequantised inputs because
// every scale is positive (the form of sparse_index_op, ops/sparse_index.py:11-69, on the
// fp8 cache layout of pd_vllm/profiles/mla_nsa.py:211-228).
//
// gfx950 mapping: the M*H query rows form M*H/16 tiles of 16 rows x 128 dims; a wave holds
// 4 of them in registers (A operands: one token at H = 64, two at H = 32) and scores 16-key
// tiles (B operands, 2 KB contiguous each) through the native fp8 MFMA
// v_mfma_f32_16x16x128_f8f6f4 -- one MFMA is a whole 128-long dot product for 16 heads x
// 16 keys.  Epilogue per MFMA: ReLU (one integer max) and the head weight (one FMA) into a
// per-lane partial over the lane's 4 heads of each query tile.
#include <type_traits>

#include "common.h"
#include "../../include/tilert_amd.h"

namespace tl {

// ReLU as one integer max on the bit pattern (negative floats are negative integers):
// fmaxf(x, 0) costs two instructions under IEEE mode (a NaN-quieting max first).
__device__ inline float relu(float x) { return __int_as_float(max(__float_as_int(x), 0)); }

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
constexpr int kBufWord3 = 0x00020000;     // buffer resource word 3: 32-bit data format
constexpr int kBufNonTemporal = 2;        // buffer access cache policy: nt (streamed once)

// A buffer's record count from a byte count (an int64 ternary, so it stays scalar: HIP's
// int64 min() goes through f64 VALU ops, which makes the resource divergent).
__device__ inline int clamp_records(int64_t bytes) { return bytes < 0x7fffffff ? static_cast<int>(bytes) : 0x7fffffff; }

// Key cache layouts.  Flat: fp8 [L, 128] plus fp32 scales [L].  Paged (PAGED): the
// 64-token pages of pd_vllm/profiles/mla_nsa.py:38-41,211-228 -- page p is 64 x 128 fp8
// (8192 B) followed by the 64 tokens' fp32 scales (256 B), 8448 B in all; key l sits in
// page l / 64, row l % 64.  A 16-key tile is still 2 KB contiguous either way.
constexpr int kKiPageKeys = 64;
constexpr int kKiPageBytes = kKiPageKeys * 128 + kKiPageKeys * 4;  // 8448


// Key formats: fp8 e4m3fn keys with a per-key fp32 scale, flat ([L, 128] + [L]) or in KI
// pages; or bf16 keys [L, 128] with no scale (the reference op's own index cache).
enum KeyFmt { kKeyFp8 = 0, kKeyFp8Paged = 1, kKeyBf16 = 2 };

// Work split.  A workgroup owns KW key ranges of NTR contiguous key tiles; SPLIT waves
// share each range (wave sp of a range holds query tiles 4 sp .. 4 sp + 3), so the
// range's key tiles go through LDS once for all of them.  All global loads are requested
// at kernel start -- queries, head weights and key scales straight into registers in the
// layouts they are used in (one coalesced load per lane for the weights and scales, spread
// by lane shuffles), then the key tiles quad by quad (4 tiles = 64 keys) as contiguous
// 1 KB reads -- and quad s is put into LDS and scored as soon as it has landed while the
// later quads still arrive; quad s + 1's MFMAs are issued before quad s's epilogue.  The
// head sum over the 4 lane groups is done for a whole quad at once: two v_permlane32_swap
// and one v_permlane16_swap leave lane l with the total of key 16 (l / 16) + l % 16 of
// the quad (3 swaps and 3 adds per quad instead of 2 + 2 per tile), so each lane scales,
// masks and stores one score: one 256-byte contiguous store per wave, token and quad.
// bf16 keys: a 16-key tile is 4 KB (rows of 256 B) and a (query tile, key tile) product
// is four v_mfma_f32_16x16x32_bf16 (lane group g holds dims 32 g .. 32 g + 31 of its row,
// step u the 8 dims 32 g + 8 u ..; queries and keys use the same assignment, so each dim
// meets its partner exactly once).
template <int M, int H, int NTR, int KF>
struct IdxShape {
  static constexpr bool BF16 = KF == kKeyBf16;
  static constexpr int TB = BF16 ? 4096 : 2048;        // bytes of a 16-row tile (keys or queries)
  static constexpr int ROWB = TB / 16;                  // bytes of one row
  static constexpr int PIECES = ROWB / 16;              // 16-byte pieces per row
  static constexpr int CPTILE = TB / 16;                // 16-byte pieces per tile
  static constexpr int TPT = H / 16;                    // query tiles per token
  static constexpr int QT = M * TPT;                    // query tiles
  static constexpr int TW = 4 / TPT;                    // tokens per wave (4 tile slots)
  static constexpr int SPLIT = (QT + 3) / 4;            // waves per key range
  static constexpr int KW = SPLIT >= 4 ? 1 : 4 / SPLIT;  // key ranges per workgroup
  static constexpr int WAVES = SPLIT * KW;
  static constexpr int THREADS = WAVES * 64;
  static constexpr int NQ = NTR / 4;                    // quads per range
  static constexpr int NT = KW * NTR;                   // key tiles per workgroup
  static constexpr int QCH = KW * 4 * CPTILE;           // 16-byte key pieces per quad step
  static constexpr int CPT = (QCH + THREADS - 1) / THREADS;
  static constexpr int LDS = NT * TB + 2048;            // + a dump row for padding pieces
  static_assert(NTR % 4 == 0 && TPT * TW == 4 && WAVES <= 4, "shape");
};

// The indexer's scoring for one workgroup: every (token, key) of its key tiles gets
// logits[tok, key] = ksv * sum_h wq[tok, h] * ReLU(q[tok, h] . k[key]) (ksv the key's scale
// for fp8 keys, `kscale` for bf16 ones; wq = w * q_s), -inf past the token's position.
template <int M, int H, int NTR, int KF>
__device__ __forceinline__ void indexer_body(const uint8_t* __restrict__ q, const float* __restrict__ q_s,
                                             int q_s_per_head, const uint8_t* __restrict__ k,
                                             const float* __restrict__ k_s, const uint16_t* __restrict__ w,
                                             float kscale, float* __restrict__ logits, int L, int64_t ld,
                                             int64_t cur_pos, int n_tiles, uint8_t* smem) {
  using S = IdxShape<M, H, NTR, KF>;
  constexpr bool PAGED = KF == kKeyFp8Paged;
  constexpr bool BF16 = S::BF16;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int sp = wave % S::SPLIT;          // which 4 query tiles
  const int rr = wave / S::SPLIT;          // which key range
  const int wg_tile = blockIdx.x * S::NT;  // first key tile of the workgroup
  const int r_tile = wg_tile + rr * NTR;   // first key tile of this wave's range

  // ---- every load is a buffer load from a workgroup-uniform base with a 32-bit lane
  //      offset; records past the end read as zero, so no lane clamps its address.
  //      All are unconditional and issued before any result is used, so the only waits
  //      are the compiler's in-order counts for the operands of each step.
  const __amdgpu_buffer_rsrc_t qrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(q), 0, S::QT * S::TB, kBufWord3);
  v8i qa[4];      // fp8: a query tile's 128 dims in one MFMA operand
  v8bf qb[4][4];  // bf16: four 32-dim steps
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int qt = min(4 * sp + j, S::QT - 1);
    if constexpr (BF16) {
      const int qo = (qt * 16 + r) * 256 + g * 64;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        qb[j][u] = __builtin_bit_cast(v8bf, __builtin_amdgcn_raw_buffer_load_b128(qrs, qo + 16 * u, 0, 0));
    } else {
      const int qo = (qt * 16 + r) * 128 + g * 16;
      const u32x4v lo = __builtin_amdgcn_raw_buffer_load_b128(qrs, qo, 0, 0);
      const u32x4v hi = __builtin_amdgcn_raw_buffer_load_b128(qrs, qo + 64, 0, 0);
      qa[j] = v8i{static_cast<int>(lo.x), static_cast<int>(lo.y), static_cast<int>(lo.z), static_cast<int>(lo.w),
                  static_cast<int>(hi.x), static_cast<int>(hi.y), static_cast<int>(hi.z), static_cast<int>(hi.w)};
    }
  }
  // head weights and query scales of the wave's 64 (token, head) rows: one load each per
  // lane (lane l holds row 64 sp + l), spread to the MFMA layout by lane shuffles later
  const int hrow = min(64 * sp + lane, S::QT * 16 - 1);
  const uint16_t wraw = w[hrow];
  const float qsraw = BF16 ? 1.0f : q_s[q_s_per_head ? hrow : hrow / H];
  // key bytes of this workgroup: flat from tile wg_tile, paged from page wg_tile / 4
  // (NTR % 4 == 0, so a workgroup starts on a page); a quad of 4 tiles is one page
  const int64_t kbase = PAGED ? static_cast<int64_t>(wg_tile / 4) * kKiPageBytes : static_cast<int64_t>(wg_tile) * S::TB;
  const int64_t kend = PAGED ? cdiv(n_tiles, 4) * kKiPageBytes : static_cast<int64_t>(L) * S::ROWB;
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(k) + kbase, 0, clamp_records(kend - kbase), kBufWord3);
  auto tile_off = [](int lt) { return PAGED ? (lt >> 2) * kKiPageBytes + (lt & 3) * 2048 : lt * S::TB; };
  float ksv[S::NQ];  // key r_tile * 16 + 64 s + lane
  if constexpr (BF16) {
#pragma unroll
    for (int s = 0; s < S::NQ; ++s) ksv[s] = kscale;
  } else {
    const __amdgpu_buffer_rsrc_t srs = PAGED ? krs
        : __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(k_s) + wg_tile * 16, 0,
                                            clamp_records((static_cast<int64_t>(L) - wg_tile * 16) * 4), kBufWord3);
#pragma unroll
    for (int s = 0; s < S::NQ; ++s) {
      const int lt = rr * NTR + 4 * s;  // workgroup-local first tile of the quad
      ksv[s] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
          srs, PAGED ? (lt >> 2) * kKiPageBytes + kKiPageKeys * 128 + lane * 4 : (lt * 16 + lane) * 4, 0, 0));
    }
  }
  // ---- key quads: piece c of step s -> range c / (4 CPTILE), tile 4 s + (c / CPTILE) % 4,
  //      byte (c % CPTILE) * 16 of the tile (contiguous reads)
  u32x4v kv[S::NQ][S::CPT];
#pragma unroll
  for (int s = 0; s < S::NQ; ++s)
#pragma unroll
    for (int u = 0; u < S::CPT; ++u) {
      const int c = min(tid + u * S::THREADS, S::QCH - 1);
      const int lt = (c / (4 * S::CPTILE)) * NTR + 4 * s + ((c / S::CPTILE) & 3);
      kv[s][u] = __builtin_amdgcn_raw_buffer_load_b128(krs, tile_off(lt) + (c % S::CPTILE) * 16, 0, kBufNonTemporal);
    }
  // scheduling boundary: nothing below (which waits for loads) moves above the requests
  asm volatile("" ::: "memory");
  // lane (r, g) needs heads 4 g .. 4 g + 3 of each of its 4 query tiles: rows 16 j + 4 g + e
  const float wqv = bf16_to_f32(wraw) * qsraw;
  float4 wq[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    wq[j] = make_float4(__shfl(wqv, 16 * j + 4 * g), __shfl(wqv, 16 * j + 4 * g + 1), __shfl(wqv, 16 * j + 4 * g + 2),
                        __shfl(wqv, 16 * j + 4 * g + 3));
  if constexpr (!BF16) {
#pragma unroll
    for (int s = 0; s < S::NQ; ++s) asm volatile("" : "+v"(ksv[s]));  // keep the scale loads up front
  }

  const int tok0 = (4 * sp) / S::TPT;  // first token of this wave
  // put quad s into LDS (piece c of row r stored at piece c ^ (r % PIECES): conflict-free
  // MFMA-layout reads)
  auto put = [&](int s) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < S::CPT; ++u) {
      const int c = tid + u * S::THREADS;
      const int row = (c / S::PIECES) & 15, ch = c % S::PIECES;
      const int lt = (c / (4 * S::CPTILE)) * NTR + 4 * s + ((c / S::CPTILE) & 3);  // workgroup-local tile
      uint8_t* dst = c < S::QCH ? smem + lt * S::TB + row * S::ROWB + ((ch ^ (row & (S::PIECES - 1))) << 4)
                                : smem + S::NT * S::TB;
      *reinterpret_cast<u32x4v*>(dst) = kv[s][u];
    }
  };
  auto products = [&](int s, v4f (&c)[4][4]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint8_t* tile = smem + (rr * NTR + 4 * s + i) * S::TB + r * S::ROWB;
      if constexpr (BF16) {
        v8bf kt[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) kt[u] = *reinterpret_cast<const v8bf*>(tile + (((4 * g + u) ^ r) << 4));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qb[j][u], kt[u], acc, 0, 0, 0);
          c[i][j] = acc;
        }
      } else {
        const uint4 lo = *reinterpret_cast<const uint4*>(tile + ((g ^ (r & 7)) << 4));
        const uint4 hi = *reinterpret_cast<const uint4*>(tile + (((g + 4) ^ (r & 7)) << 4));
        const v8i kt = {static_cast<int>(lo.x), static_cast<int>(lo.y), static_cast<int>(lo.z), static_cast<int>(lo.w),
                        static_cast<int>(hi.x), static_cast<int>(hi.y), static_cast<int>(hi.z), static_cast<int>(hi.w)};
#pragma unroll
        for (int j = 0; j < 4; ++j) c[i][j] = mfma_16x16x128_fp8(qa[j], kt);
      }
    }
  };
  auto epilogue = [&](int s, const v4f (&c)[4][4]) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < S::TW; ++t) {
      // lane partial (its 4 heads of each of the token's query tiles) per tile of the quad
      float a[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float acc = 0.f;
#pragma unroll
        for (int jj = 0; jj < S::TPT; ++jj) {
          const int j = t * S::TPT + jj;
          acc = __builtin_fmaf(relu(c[i][j][0]), wq[j].x, acc);
          acc = __builtin_fmaf(relu(c[i][j][1]), wq[j].y, acc);
          acc = __builtin_fmaf(relu(c[i][j][2]), wq[j].z, acc);
          acc = __builtin_fmaf(relu(c[i][j][3]), wq[j].w, acc);
        }
        a[i] = acc;
      }
      // rows (16-lane groups) hold partial sums over disjoint heads: pair tiles (0, 2)
      // and (1, 3) across the 32-lane halves, then the two results across odd/even rows;
      // lane group g ends with the total of tile g
      const auto p02 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[0]), __float_as_uint(a[2]), false, false);
      const auto p13 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[1]), __float_as_uint(a[3]), false, false);
      const float x = __uint_as_float(p02[0]) + __uint_as_float(p02[1]);
      const float y = __uint_as_float(p13[0]) + __uint_as_float(p13[1]);
      const auto pxy = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
      const float score = (__uint_as_float(pxy[0]) + __uint_as_float(pxy[1])) * ksv[s];
      const int tok = tok0 + t;  // wave-uniform
      if (tok < M) {
        // keys past L are dropped by the buffer's bound; keys past the token's position
        // (cur_pos + tok, at most L - 1 here) are masked
        const int key = (r_tile + 4 * s) * 16 + lane;
        const int lim = cur_pos + tok < L ? static_cast<int>(cur_pos + tok) : L - 1;
        const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(logits + tok * ld, 0, L * 4, kBufWord3);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, key > lim ? -__builtin_inff() : score), ors,
                                              key * 4, 0, 0);
      }
    }
  };
  if constexpr (BF16) {
    // one accumulator set (the bf16 operands take the registers of the second): each
    // quad's epilogue overlaps the other wave of the SIMD instead
    v4f cb[4][4];
#pragma unroll
    for (int s = 0; s < S::NQ; ++s) {
      put(s);
      __syncthreads();
      products(s, cb);
      epilogue(s, cb);
    }
  } else {
    // software pipeline: quad s + 1's MFMAs are issued before quad s's epilogue, so the
    // matrix core works while the VALU finishes the previous quad
    v4f cb[2][4][4];
    put(0);
    __syncthreads();
    products(0, cb[0]);
#pragma unroll
    for (int s = 0; s < S::NQ; ++s) {
      if (s + 1 < S::NQ) {
        put(s + 1);
        __syncthreads();
        products(s + 1, cb[(s + 1) & 1]);
      }
      epilogue(s, cb[s & 1]);
    }
  }
}

template <int M, int H, int NTR, int KF>
__global__ __launch_bounds__(256) void indexer_kernel(
    const uint8_t* __restrict__ q, const float* __restrict__ q_s, int q_s_per_head,
    const uint8_t* __restrict__ k, const float* __restrict__ k_s, const uint16_t* __restrict__ w, float kscale,
    float* __restrict__ logits, int L, int64_t ld, int64_t cur_pos, int n_tiles) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  indexer_body<M, H, NTR, KF>(q, q_s, q_s_per_head, k, k_s, w, kscale, logits, L, ld, cur_pos, n_tiles, smem);
}

// Columns no token can see (key > cur_pos + M - 1) are -inf for every row.
__global__ void fill_masked_kernel(float* __restrict__ logits, int M, int64_t ld, int64_t begin, int64_t end) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t n = end - begin;
  if (i >= n * M) return;
  const int64_t t = i / n, c = begin + (i - t * n);
  logits[t * ld + c] = -__builtin_inff();
}

template <int M, int H, int NTR, int KF>
static int launch_indexer_t(hipStream_t st, const uint8_t* q, const float* q_s, int per_head, const uint8_t* k,
                            const float* k_s, const uint16_t* w, float kscale, float* logits, int L, int64_t ld,
                            int64_t cur_pos, int n_tiles) {
  using S = IdxShape<M, H, NTR, KF>;
  const dim3 grid(static_cast<unsigned>(cdiv(n_tiles, static_cast<int64_t>(S::NT))));
  const void* fn = reinterpret_cast<const void*>(indexer_kernel<M, H, NTR, KF>);
  if (S::LDS > 64 * 1024) {
    if (int rc = allow_dynamic_lds(fn, S::LDS, "indexer")) return rc;
  }
  hipLaunchKernelGGL((indexer_kernel<M, H, NTR, KF>), grid, dim3(S::THREADS), S::LDS, st, q, q_s, per_head, k, k_s, w,
                     kscale, logits, L, ld, cur_pos, n_tiles);
  return check_launch("indexer");
}

// Key tiles per range: 16 (4 quads; two 4-wave workgroups per CU at M = 4, H = 64 --
// measured against 8 and 32 at 128K keys: 8.0 vs 8.4 / 8.4 us) while that still gives
// >= 512 workgroups, fewer for short caches so the grid keeps filling the chip.
template <int M, int H, int KF>
static int launch_indexer(hipStream_t st, const uint8_t* q, const float* q_s, int per_head, const uint8_t* k,
                          const float* k_s, const uint16_t* w, float kscale, float* logits, int L, int64_t ld,
                          int64_t cur_pos, int n_tiles) {
  constexpr int KW = IdxShape<M, H, 4, KF>::KW;
  // bf16 keys: at most 16 tiles per workgroup (66 KB of LDS, 64 prefetch registers)
  constexpr int kMaxNtr = KF == kKeyBf16 ? (16 / KW < 4 ? 4 : 16 / KW) : 16;
  int ntr = kMaxNtr;
  while (ntr > 4 && cdiv(n_tiles, static_cast<int64_t>(KW) * ntr) < 512) ntr /= 2;
  auto run = [&](auto ntr_tag) {
    constexpr int NTR = decltype(ntr_tag)::value;
    return launch_indexer_t<M, H, NTR, KF>(st, q, q_s, per_head, k, k_s, w, kscale, logits, L, ld, cur_pos, n_tiles);
  };
  if constexpr (kMaxNtr >= 16) {
    if (ntr == 16) return run(std::integral_constant<int, 16>{});
  }
  if constexpr (kMaxNtr >= 8) {
    if (ntr == 8) return run(std::integral_constant<int, 8>{});
  }
  return run(std::integral_constant<int, 4>{});
}

// Shared argument checks and dispatch of every indexer entry point.  topk > 0 adds the
// exact top-k (indices int32 [M, topk] into `out`): tl_topk_rows on the logits just written,
// on the same stream, with the caller's workspace (tl_indexer_topk_workspace_bytes).
// Measured and not kept: the selection fused into the scoring launch (see the top-k notes of
// the package documentation) -- every variant was slower than the two launches.
template <int KF>
static int indexer_run(const char* who, const void* q, const float* q_s, int q_s_per_head, const void* kp,
                       const float* k_s, const void* w_bf16, float kscale, float* logits, int64_t M, int64_t H,
                       int64_t L, int64_t ld, int64_t cur_pos, int64_t topk, int32_t* out, void* workspace,
                       size_t workspace_bytes, void* stream) {
  constexpr bool BF16 = KF == kKeyBf16;
  if (H != 32 && H != 64) { set_error("%s: H=%lld must be 32 or 64", who, (long long)H); return kErrUnsupported; }
  if (M < 1 || M * H > 256) { set_error("%s: need 1 <= M and M*H <= 256 (M=%lld H=%lld)", who, (long long)M, (long long)H); return kErrUnsupported; }
  if (L < 0 || L > (1ll << 28) || ld < L) { set_error("%s: bad L=%lld / ld=%lld", who, (long long)L, (long long)ld); return kErrArg; }
  if (cur_pos < 0) { set_error("%s: cur_pos=%lld must be >= 0", who, (long long)cur_pos); return kErrArg; }
  if (!q || (!BF16 && !q_s) || !kp || (KF == kKeyFp8 && !k_s) || !w_bf16 || !logits) { set_error("%s: null pointer", who); return kErrArg; }
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kp)) & 15) { set_error("%s: q and k must be 16-byte aligned", who); return kErrArg; }
  if (topk > 0) {
    // validated before anything is launched (tl_topk_rows repeats these checks)
    if (L == 0) { set_error("%s: top-k over an empty cache", who); return kErrArg; }
    const size_t need = tl_topk_workspace_bytes(M, ld, topk);
    if (need == 0 || topk > 8192 || ld % 4 || (reinterpret_cast<uintptr_t>(logits) & 15)) {
      set_error("%s: top-k needs topk <= 8192, ld %% 4 == 0, 16-byte aligned logits and ld <= 262144", who);
      return kErrUnsupported;
    }
    if (!out) { set_error("%s: null indices", who); return kErrArg; }
    if (!workspace || workspace_bytes < need) { set_error("%s: workspace of %zu bytes required (got %zu)", who, need, workspace_bytes); return kErrArg; }
  }
  hipStream_t st = (hipStream_t)stream;
  // keys past the last token's position are masked for every token: no need to read them
  const int64_t visible = cur_pos + M < L ? cur_pos + M : L;
  if (visible < L) {
    const int64_t n = (L - visible) * M;
    hipLaunchKernelGGL(fill_masked_kernel, dim3(cdiv(n, 256)), dim3(256), 0, st, logits, (int)M, ld, visible, L);
  }
  int rc = kOk;
  if (visible > 0) {
    const int n_tiles = static_cast<int>(cdiv(visible, 16));
    const uint8_t* qq = (const uint8_t*)q;
    const uint8_t* k = (const uint8_t*)kp;
    const uint16_t* w = (const uint16_t*)w_bf16;
    const int Li = static_cast<int>(L);
    rc = kErrUnsupported;
#define TL_IDX(MM, HH) \
    if (M == MM && H == HH) rc = launch_indexer<MM, HH, KF>(st, qq, q_s, q_s_per_head, k, k_s, w, kscale, logits, Li, ld, cur_pos, n_tiles);
    TL_IDX(1, 64) TL_IDX(2, 64) TL_IDX(3, 64) TL_IDX(4, 64)
    TL_IDX(1, 32) TL_IDX(2, 32) TL_IDX(3, 32) TL_IDX(4, 32) TL_IDX(5, 32) TL_IDX(6, 32) TL_IDX(7, 32) TL_IDX(8, 32)
#undef TL_IDX
    if (rc == kErrUnsupported) set_error("%s: unsupported M=%lld H=%lld", who, (long long)M, (long long)H);
  }
  if (rc != kOk || topk <= 0) return rc;
  return tl_topk_rows(logits, M, ld, cur_pos, topk, out, workspace, workspace_bytes, stream);
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
  amax = row16_reduce<true>(amax);  // the group's 16 lanes
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
__device__ inline float bf16_round(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// The value of lane (lane ^ B), without an LDS round trip: DPP quad permutes for 1 and 2,
// row shifts for 4, a row rotation for 8, and gfx950's row / half-wave swaps for 16 and 32
// (v_permlane16_swap / v_permlane32_swap of a register with itself: the lanes a swap
// replaces in either copy are the partners).
template <int B>
__device__ inline float lane_xor(float v) {
  const int x = __builtin_bit_cast(int, v);
  const int lane = threadIdx.x & 63;
  if constexpr (B == 1) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0xb1, 0xf, 0xf, false));
  if constexpr (B == 2) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x4e, 0xf, 0xf, false));
  if constexpr (B == 4) {
    const int up = __builtin_amdgcn_mov_dpp(x, 0x104, 0xf, 0xf, false);  // row_shl:4: lane + 4
    const int dn = __builtin_amdgcn_mov_dpp(x, 0x114, 0xf, 0xf, false);  // row_shr:4: lane - 4
    return __builtin_bit_cast(float, (lane & 4) ? dn : up);
  }
  if constexpr (B == 8) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x128, 0xf, 0xf, false));  // row_ror:8
  if constexpr (B == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(static_cast<unsigned>(x), static_cast<unsigned>(x), false, false);
    return __builtin_bit_cast(float, (lane & 16) ? p[0] : p[1]);
  }
  const auto p = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(x), static_cast<unsigned>(x), false, false);
  return __builtin_bit_cast(float, (lane & 32) ? p[0] : p[1]);
}

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
  const float mean = wave_sum_f32(x0 + x1) * (1.0f / 128.0f);
  const float d0 = x0 - mean, d1 = x1 - mean;
  const float var = wave_sum_f32(d0 * d0 + d1 * d1) * (1.0f / 128.0f);
  const float rstd = 1.0f / sqrtf(var + eps);
  float v0 = bf16_round(d0 * rstd * w0 + b0);
  float v1 = bf16_round(d1 * rstd * w1 + b1);
  // RoPE on elements 0..63 (v0 of every lane): (re, im) = (x_i, x_{i+32}) times (c, s)
  const float p = lane_xor<32>(v0);
  v0 = bf16_round(lane < 32 ? v0 * fc - p * fs : p * fs + v0 * fc);
  // Hadamard: bit 6 inside the lane, bits 5..0 across lanes
  {
    const float a = v0, b = v1;
    v0 = a + b;
    v1 = a - b;
  }
  auto butterfly = [&](auto bit_tag) {
    constexpr int bit = decltype(bit_tag)::value;
    const float q0 = lane_xor<bit>(v0), q1 = lane_xor<bit>(v1);
    const bool hi = lane & bit;
    v0 = hi ? q0 - v0 : v0 + q0;
    v1 = hi ? q1 - v1 : v1 + q1;
  };
  butterfly(std::integral_constant<int, 32>{});
  butterfly(std::integral_constant<int, 16>{});
  butterfly(std::integral_constant<int, 8>{});
  butterfly(std::integral_constant<int, 4>{});
  butterfly(std::integral_constant<int, 2>{});
  butterfly(std::integral_constant<int, 1>{});
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
    amax = wave_max_f32(amax);
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
  return indexer_run<kKeyFp8>("indexer", q_fp8, q_s, q_s_per_head, k_fp8, k_s, w_bf16, 1.0f, logits, M, H, L, ld,
                              cur_pos, 0, nullptr, nullptr, 0, stream);
}

extern "C" int tl_indexer_fp8_scores_paged(const void* q_fp8, const float* q_s, int q_s_per_head,
                                           const void* ki_pages, int64_t n_pages, const void* w_bf16,
                                           float* logits, int64_t M, int64_t H, int64_t L, int64_t ld,
                                           int64_t cur_pos, void* stream) {
  if (n_pages < 0 || L > n_pages * kKiPageKeys) {
    set_error("indexer_paged: L=%lld keys need %lld pages (got %lld)", (long long)L, (long long)cdiv(L, kKiPageKeys), (long long)n_pages);
    return kErrArg;
  }
  return indexer_run<kKeyFp8Paged>("indexer_paged", q_fp8, q_s, q_s_per_head, ki_pages, nullptr, w_bf16, 1.0f, logits,
                                   M, H, L, ld, cur_pos, 0, nullptr, nullptr, 0, stream);
}

extern "C" size_t tl_indexer_topk_workspace_bytes(int64_t M, int64_t ld, int64_t topk) {
  return tl_topk_workspace_bytes(M, ld, topk);
}

extern "C" int tl_indexer_fp8_topk(const void* q_fp8, const float* q_s, int q_s_per_head, const void* k_fp8,
                                   const float* k_s, const void* w_bf16, float* logits, int64_t M, int64_t H,
                                   int64_t L, int64_t ld, int64_t cur_pos, int64_t topk, int32_t* indices,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  if (topk < 1) { set_error("indexer_topk: topk=%lld must be positive", (long long)topk); return kErrArg; }
  return indexer_run<kKeyFp8>("indexer_topk", q_fp8, q_s, q_s_per_head, k_fp8, k_s, w_bf16, 1.0f, logits, M, H, L, ld,
                              cur_pos, topk, indices, workspace, workspace_bytes, stream);
}

extern "C" int tl_indexer_bf16_scores(const void* q_bf16, const void* k_bf16, const void* w_bf16, float score_scale,
                                      float* logits, int64_t M, int64_t H, int64_t L, int64_t ld, int64_t cur_pos,
                                      void* stream) {
  return indexer_run<kKeyBf16>("indexer_bf16", q_bf16, nullptr, 0, k_bf16, nullptr, w_bf16, score_scale, logits, M, H,
                               L, ld, cur_pos, 0, nullptr, nullptr, 0, stream);
}

extern "C" int tl_indexer_bf16_topk(const void* q_bf16, const void* k_bf16, const void* w_bf16, float score_scale,
                                    float* logits, int64_t M, int64_t H, int64_t L, int64_t ld, int64_t cur_pos,
                                    int64_t topk, int32_t* indices, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  if (topk < 1) { set_error("indexer_bf16_topk: topk=%lld must be positive", (long long)topk); return kErrArg; }
  return indexer_run<kKeyBf16>("indexer_bf16_topk", q_bf16, nullptr, 0, k_bf16, nullptr, w_bf16, score_scale, logits, M,
                               H, L, ld, cur_pos, topk, indices, workspace, workspace_bytes, stream);
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
