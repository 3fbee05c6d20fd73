// Shared device helpers for the gfx950 FP8 decode kernels.
//
// Conventions (all kernels):
//   * fp8 is OCP e4m3fn (bias 7, max 448, NaN 0x7f/0xff) -- gfx950's native FP8 format,
//     used directly by v_mfma_*_f8f6f4 with cbsz/blgp = 0.  No fnuz conversion anywhere.
//   * block size 128: activation scales per (row, 128 columns), weight scales per
//     (128 rows, 128 columns), stored row-major [ceil(N/128), K/128].
//   * bf16 is carried as uint16_t bit patterns; fp32 -> bf16 is round-to-nearest-even.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tilert_amd.h"

namespace tl {

constexpr int kBlock = 128;
constexpr float kE4m3Max = 448.0f;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- error reporting
void set_error(const char* fmt, ...);
int check_launch(const char* what);
// Raise a kernel's dynamic-LDS limit to `bytes` (gfx950 has 160 KB per CU; launches
// above 64 KB need it), once per (device, kernel); thread-safe.
int allow_dynamic_lds(const void* kernel, int bytes, const char* who);

enum Status { kOk = 0, kErrArg = 1, kErrHip = 2, kErrUnsupported = 3 };

// ---------------------------------------------------------------- scalar codecs
__host__ __device__ inline float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

__host__ __device__ inline uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest, ties to even
  return static_cast<uint16_t>(u >> 16);
}

// e4m3fn encode, round-to-nearest-even.  Callers clamp to [-448, 448] first (the
// reference does, refs/kernel.py:193), so the result is always finite.
__device__ inline uint32_t f32_to_e4m3(float v) {
  uint32_t u = __float_as_uint(v);
  uint32_t sign = (u >> 24) & 0x80u;
  float a = __builtin_fabsf(v);
  if (a != a) return 0x7fu | sign;
  uint32_t code;
  if (a < 0.015625f) {  // below 2^-6: subnormal grid m * 2^-9, m in [0, 8]
    code = static_cast<uint32_t>(__builtin_rintf(a * 512.0f));  // exact scaling, RNE
  } else {
    uint32_t au = __float_as_uint(a);
    uint32_t e = (au >> 23) - 127u + 7u;  // biased e4m3 exponent, 1..15
    uint32_t m = au & 0x7fffffu;
    uint32_t r = (m + 0x7ffffu + ((m >> 20) & 1u)) >> 20;  // RNE to 3 mantissa bits (0..8)
    code = (e << 3) + r;  // r == 8 carries into the exponent
    if (code > 0x7eu) code = 0x7eu;  // only reachable for |v| > 448 (clamped by callers)
  }
  return code | sign;
}

// Quantisation scale of a 128-element group from its fp32 amax; mirrors
// refs/kernel.py:186-191 (amax floor 1e-4, s = amax * fp32(1/448)) and the power-of-two
// round-scale form :140-151; TL_SCALE_DIV is the plain amax / 448 (IEEE division) of the
// workload's statement.
__device__ inline float group_scale(float amax, int scale_mode) {
  amax = fmaxf(amax, 1e-4f);
  if (scale_mode == TL_SCALE_UE8M0) {
    uint32_t bits = __float_as_uint(amax * (1.0f / 448.0f));
    int e = static_cast<int>((bits >> 23) & 0xffu) - 127 + ((bits & 0x7fffffu) != 0 ? 1 : 0);
    return __uint_as_float(static_cast<uint32_t>(e + 127) << 23);
  }
  if (scale_mode == TL_SCALE_DIV) return amax / 448.0f;
  return amax * (1.0f / 448.0f);
}

// ------------------------------------------------------------- wave reductions
// OR of a 32-bit value over the wave's 64 lanes, wave-uniform.  An inclusive OR scan on
// DPP (row shifts by 1, 2, 4, 8 within each 16-lane row, then the row broadcasts of lanes
// 15 and 31), read from lane 63: six VALU steps, where the same reduction through lane
// shuffles is six dependent LDS-permute round trips.
__device__ inline uint32_t wave_or_u32(uint32_t v) {
  v |= static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x111, 0xf, 0xf, false));  // row_shr:1
  v |= static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x112, 0xf, 0xf, false));  // row_shr:2
  v |= static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x114, 0xf, 0xf, false));  // row_shr:4
  v |= static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x118, 0xf, 0xf, false));  // row_shr:8
  v |= static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x142, 0xa, 0xf, false));  // row_bcast:15
  v |= static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x143, 0xc, 0xf, false));  // row_bcast:31
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}
// Sum / max of an fp32 value over the wave, wave-uniform: the same DPP scan (row shifts,
// then row broadcasts; lane 63 ends with the result).
template <bool MAX>
__device__ inline float wave_reduce_f32(float v) {
  auto step = [&](float o) { v = MAX ? fmaxf(v, o) : v + o; };
  const int id = MAX ? __builtin_bit_cast(int, -INFINITY) : 0;
  step(__builtin_bit_cast(float, __builtin_amdgcn_update_dpp(id, __builtin_bit_cast(int, v), 0x111, 0xf, 0xf, false)));
  step(__builtin_bit_cast(float, __builtin_amdgcn_update_dpp(id, __builtin_bit_cast(int, v), 0x112, 0xf, 0xf, false)));
  step(__builtin_bit_cast(float, __builtin_amdgcn_update_dpp(id, __builtin_bit_cast(int, v), 0x114, 0xf, 0xf, false)));
  step(__builtin_bit_cast(float, __builtin_amdgcn_update_dpp(id, __builtin_bit_cast(int, v), 0x118, 0xf, 0xf, false)));
  step(__builtin_bit_cast(float, __builtin_amdgcn_update_dpp(id, __builtin_bit_cast(int, v), 0x142, 0xa, 0xf, false)));
  step(__builtin_bit_cast(float, __builtin_amdgcn_update_dpp(id, __builtin_bit_cast(int, v), 0x143, 0xc, 0xf, false)));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ inline float wave_sum_f32(float v) { return wave_reduce_f32<false>(v); }
__device__ inline float wave_max_f32(float v) { return wave_reduce_f32<true>(v); }

// Max / sum over each 16-lane row with DPP, the result in every lane of the row: swaps
// within quads, then the half-row mirror (lane i <-> 7 - i) and the row mirror
// (i <-> 15 - i) pair every lane with one holding the other half's partial.
template <int CTRL, bool MAX>
__device__ inline float dpp_combine(float x) {
  const float y = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
  return MAX ? fmaxf(x, y) : x + y;
}
template <bool MAX>
__device__ inline float row16_reduce(float v) {
  v = dpp_combine<0xb1, MAX>(v);      // quad_perm [1, 0, 3, 2]
  v = dpp_combine<0x4e, MAX>(v);      // quad_perm [2, 3, 0, 1]
  v = dpp_combine<0x141, MAX>(v);     // row_half_mirror
  return dpp_combine<0x140, MAX>(v);  // row_mirror
}

// Max of a 32-bit unsigned value over the wave, wave-uniform (the same DPP scan).
__device__ inline uint32_t wave_max_u32(uint32_t v) {
#define TL_DPP_MAXU(ctrl, rmask) \
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), ctrl, rmask, 0xf, false)))
  TL_DPP_MAXU(0x111, 0xf);
  TL_DPP_MAXU(0x112, 0xf);
  TL_DPP_MAXU(0x114, 0xf);
  TL_DPP_MAXU(0x118, 0xf);
  TL_DPP_MAXU(0x142, 0xa);
  TL_DPP_MAXU(0x143, 0xc);
#undef TL_DPP_MAXU
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}
__device__ inline uint64_t wave_or_u64(uint64_t m) {
  const uint32_t lo = wave_or_u32(static_cast<uint32_t>(m)), hi = wave_or_u32(static_cast<uint32_t>(m >> 32));
  return static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32);
}

// ---------------------------------------------------------- bf16 dequantisation
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

__device__ inline uint32_t bf16x2_bits(v2f f) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, v2bf));  // v_cvt_pk_bf16_f32, RNE
}

// fp8 dwords d0, d1 (8 weights, k order = byte order) -> bf16(fp32(q) * s) MFMA operand.
__device__ inline v8bf dequant8_bf16(uint32_t d0, uint32_t d1, float s) {
  uint32_t __attribute__((ext_vector_type(4))) r;
  r.x = bf16x2_bits(__builtin_amdgcn_cvt_pk_f32_fp8(d0, false) * s);
  r.y = bf16x2_bits(__builtin_amdgcn_cvt_pk_f32_fp8(d0, true) * s);
  r.z = bf16x2_bits(__builtin_amdgcn_cvt_pk_f32_fp8(d1, false) * s);
  r.w = bf16x2_bits(__builtin_amdgcn_cvt_pk_f32_fp8(d1, true) * s);
  return __builtin_bit_cast(v8bf, r);
}

// --------------------------------------------------------------- MFMA tile helper
// One wave: C[16x16] = A[16x128] * B[128x16] in fp8 with fp32 accumulation.
//
// Lane l holds A row (l & 15) and B column (l & 15); both operands carry the same
// 32 K-positions per lane (loaded by the same addressing), so the product sums every
// K position exactly once whatever the hardware's in-register K order is.  The result
// layout is the CDNA 16x16 accumulator layout: lane l holds C[4*(l>>4) + j][l & 15].
__device__ inline v4f mfma_16x16x128_fp8(const v8i& a, const v8i& b) {
  v4f z = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 0, 0, 0);
}

// Byte offsets (within a 128-byte K block) of the two 16-byte pieces lane group g owns.
__device__ inline int kpiece0(int g) { return g * 16; }
__device__ inline int kpiece1(int g) { return 64 + g * 16; }

__device__ inline v8i load_kblock(const uint8_t* row_kblock, int g) {
  const uint4 lo = *reinterpret_cast<const uint4*>(row_kblock + kpiece0(g));
  const uint4 hi = *reinterpret_cast<const uint4*>(row_kblock + kpiece1(g));
  v8i r;
  r[0] = lo.x; r[1] = lo.y; r[2] = lo.z; r[3] = lo.w;
  r[4] = hi.x; r[5] = hi.y; r[6] = hi.z; r[7] = hi.w;
  return r;
}

// Non-temporal variant for weights that are streamed exactly once.
__device__ inline v8i load_kblock_stream(const uint8_t* row_kblock, int g) {
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  const u4 lo = __builtin_nontemporal_load(reinterpret_cast<const u4*>(row_kblock + kpiece0(g)));
  const u4 hi = __builtin_nontemporal_load(reinterpret_cast<const u4*>(row_kblock + kpiece1(g)));
  v8i r;
  r[0] = lo.x; r[1] = lo.y; r[2] = lo.z; r[3] = lo.w;
  r[4] = hi.x; r[5] = hi.y; r[6] = hi.z; r[7] = hi.w;
  return r;
}

__device__ inline v8i zero_v8i() {
  v8i r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = 0;
  return r;
}

// A wave-uniform float read through the vector memory path.  Scalar loads share their
// wait counter with LDS reads, and SMEM returns out of order, so every wait on an LDS
// read would also wait for a scalar prefetch; a vector load is counted in issue order
// with the other prefetched operands instead.
__device__ inline float load_f32_vector(const float* p) {
  int zero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(zero));  // hides the uniform address
  return p[zero];
}

// s_waitcnt immediate: vmcnt(n), no wait on the other counters
__host__ __device__ constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

typedef __attribute__((address_space(3))) uint8_t* lds_u8_ptr;

// Load-to-LDS copies written as inline assembly: lane l copies SIZE bytes from its own
// global address to LDS at (wave-uniform) lds + l * SIZE.  Through the builtin, the
// compiler cannot tell these LDS writes from the operand reads of another ring stage and
// puts a wait for every copy in flight before each LDS read; as assembly they are
// invisible to it, and the kernel's own s_waitcnt + s_barrier order them.
// m0 is saved into a scratch SGPR and restored inside the statement: it is a reserved
// register that the compiler may keep live, so the assembly leaves it as it found it.
__device__ inline void copy_to_lds16(const void* src, uint8_t* lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_u8_ptr)lds)));
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(saved) : "v"(src), "s"(m0) : "memory");
}
__device__ inline void copy_to_lds4(const void* src, uint8_t* lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_u8_ptr)lds)));
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(saved) : "v"(src), "s"(m0) : "memory");
}

// Software pipeline over n items with D operand buffers: item i's loads are issued D-1
// items ahead of its compute.  fetch(i, buf) must issue the same, unconditional loads for
// every i, so the steady-state loop has a fixed number of loads in flight and the
// compiler's wait counts cover only the operands being consumed.  Buffer indices are
// compile-time constants (the loop is unrolled by D), so no register copies -- which
// would wait for the loads -- are needed.  The last 2D-2 items run in a guarded tail; a
// stream of fewer than D-1 items issues all its loads, runs start(), then computes them
// (no round trip per item).
// start() runs once, after the first fetches are issued and before the first compute
// (for work that should overlap them, e.g. filling LDS); it runs even when n == 0, so it
// may contain a workgroup barrier as long as every wave calls ring_pipeline.
template <int D, class Buf, class Fetch, class Compute, class Start>
__device__ inline void ring_pipeline(int n, Buf (&buf)[D], Fetch&& fetch, Compute&& compute, Start&& start) {
  if (n < D - 1) {  // too short to fill the ring: every item's loads are issued up front
#pragma unroll
    for (int j = 0; j < D - 1; ++j)
      if (j < n) fetch(j, buf[j]);
    start();
#pragma unroll
    for (int j = 0; j < D - 1; ++j)
      if (j < n) compute(j, buf[j]);
    return;
  }
#pragma unroll
  for (int j = 0; j < D - 1; ++j) fetch(j, buf[j]);
  start();
  int i = 0;
  for (; i + 2 * D - 2 < n; i += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      fetch(i + j + D - 1, buf[(j + D - 1) % D]);
      compute(i + j, buf[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < 2 * D - 2; ++j) {
    if (i + j < n) {
      if (i + j + D - 1 < n) fetch(i + j + D - 1, buf[(j + D - 1) % D]);
      compute(i + j, buf[j % D]);
    }
  }
}

template <int D, class Buf, class Fetch, class Compute>
__device__ inline void ring_pipeline(int n, Buf (&buf)[D], Fetch&& fetch, Compute&& compute) {
  ring_pipeline(n, buf, fetch, compute, [] {});
}

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// The split-K workspace that the FP8 GEMM and the bf16 GEMV share (one per stream): per-row-
// tile arrival counters first, which every call leaves zero, then the fp32 partials.
constexpr int kWsCounterTiles = 16384;  // N <= 262144
constexpr size_t kWsCounterBytes = kWsCounterTiles * sizeof(uint32_t);

}  // namespace tl
