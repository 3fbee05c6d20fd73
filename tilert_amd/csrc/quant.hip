// act_quant (per 1x128 group, e4m3fn + fp32 scale), 128x128 block weight quantisation
// and weight dequantisation.
#include "common.h"
#include "../../include/tilert_amd.h"

namespace tl {

// One thread = 8 consecutive elements; 16 threads = one 128-element group.
__global__ __launch_bounds__(256) void act_quant_kernel(const uint16_t* __restrict__ x,
                                                        uint8_t* __restrict__ y,
                                                        float* __restrict__ s, int64_t n_groups,
                                                        int scale_mode) {
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t grp = tid >> 4;
  const bool live = grp < n_groups;
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
    reinterpret_cast<uint2*>(y)[tid] = make_uint2(lo, hi);
    if ((tid & 15) == 0) s[grp] = sc;
  }
}

// One 256-thread workgroup per 128x128 block: amax, s = amax/448 (1 for all-zero
// blocks), q = e4m3(clamp(w/s)).
template <typename T>
__device__ inline float load_w(const T* p);
template <>
__device__ inline float load_w<float>(const float* p) { return *p; }
template <>
__device__ inline float load_w<uint16_t>(const uint16_t* p) { return bf16_to_f32(*p); }

template <typename T>
__global__ __launch_bounds__(256) void weight_quant_kernel(const T* __restrict__ w,
                                                           uint8_t* __restrict__ q,
                                                           float* __restrict__ s, int64_t N,
                                                           int64_t K) {
  __shared__ float red[256];
  const int64_t nb = blockIdx.y, kb = blockIdx.x;
  const int64_t KB = cdiv(K, kBlock);
  const int col = threadIdx.x & 127;
  const int r0 = threadIdx.x >> 7;  // 0..1
  const int64_t c = kb * kBlock + col;
  float amax = 0.f;
  for (int r = r0; r < kBlock; r += 2) {
    const int64_t n = nb * kBlock + r;
    if (n < N && c < K) amax = fmaxf(amax, __builtin_fabsf(load_w(w + n * K + c)));
  }
  red[threadIdx.x] = amax;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (static_cast<int>(threadIdx.x) < o) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + o]);
    __syncthreads();
  }
  amax = red[0];
  const float sc = amax > 0.f ? amax / 448.0f : 1.0f;
  if (threadIdx.x == 0) s[nb * KB + kb] = sc;
  for (int r = r0; r < kBlock; r += 2) {
    const int64_t n = nb * kBlock + r;
    if (n < N && c < K) {
      float v = load_w(w + n * K + c) / sc;
      q[n * K + c] = static_cast<uint8_t>(f32_to_e4m3(fminf(fmaxf(v, -kE4m3Max), kE4m3Max)));
    }
  }
}

__device__ inline float e4m3_to_f32(uint32_t code) {
  const uint32_t sign = (code & 0x80u) << 24;
  const uint32_t e = (code >> 3) & 0xfu, m = code & 7u;
  float mag;
  if (e == 0xfu && m == 7u) return __uint_as_float(0x7fc00000u);
  if (e == 0) mag = static_cast<float>(m) * 0.001953125f;  // m * 2^-9
  else mag = __uint_as_float(((e + 120u) << 23) | (m << 20));
  return __uint_as_float(__float_as_uint(mag) | sign);
}

__global__ __launch_bounds__(256) void weight_dequant_kernel(const uint8_t* __restrict__ q,
                                                             const float* __restrict__ s,
                                                             void* __restrict__ out, int64_t N,
                                                             int64_t K, int out_bf16) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= N * K) return;
  const int64_t n = i / K, k = i - n * K;
  const float v = e4m3_to_f32(q[i]) * s[(n / kBlock) * cdiv(K, kBlock) + k / kBlock];
  if (out_bf16) static_cast<uint16_t*>(out)[i] = f32_to_bf16(v);
  else static_cast<float*>(out)[i] = v;
}

// RMSNorm (tilert/models/common.py:92-133, no residual): y = bf16(gamma * x * rsqrt(mean(x^2)
// + eps)) in fp32, then -- when y8/ys are given -- act_quant of those bf16 values per
// 1x128 group (rmsnorm_quant_op, ops/rmsnorm_quant.py:19-63).  rsqrt is 1 / sqrt with IEEE
// sqrt and division, as torch's.
// A row's sum of squares is taken over a fixed tree of kNormVirt virtual threads: virtual
// thread v adds the squares of chunks (8 elements) v, v + kNormVirt, ... in order, each
// 64 virtual threads are one DPP wave reduction, and the kNormVirt / 64 wave partials are
// added in order -- the same float result whatever the launch shape.  The row is then cut
// into slices of kNormSlice chunks, one 256-thread workgroup each (thread = one chunk, 16
// threads = one 128-element group): every workgroup of a row recomputes the row's sum
// (the row is 8-32 KB, read from L2 after the first) and normalises and quantises only
// its slice.  One 1024-thread workgroup per row left a decode step's 4 rows on 4 CUs,
// issue-bound on the quantisation (5.2 us at 4 x 7168).
constexpr int kNormThreads = 256;
constexpr int kNormVirt = 1024;
constexpr int kNormPerThread = kNormVirt / kNormThreads;  // virtual threads per thread
constexpr int kNormMaxChunks = 2;                           // chunks per virtual thread
constexpr int kNormSlice = kNormThreads;                    // chunks per workgroup
constexpr int kNormMaxDim = kNormMaxChunks * kNormVirt * 8;  // 16384

__global__ __launch_bounds__(kNormThreads) void rmsnorm_quant_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ gamma, float eps, int dim,
    uint16_t* __restrict__ y, uint8_t* __restrict__ y8, float* __restrict__ ys, int scale_mode) {
  __shared__ float part[kNormVirt / 64];
  const int row = blockIdx.x, tid = threadIdx.x;
  const int nch = dim / 8;
  const int c = blockIdx.y * kNormSlice + tid;  // this thread's chunk
  const bool live = c < nch;
  const uint4* xr = reinterpret_cast<const uint4*>(x + static_cast<int64_t>(row) * dim);
  // every load up front (clamped, unconditional): the row for the sum, this chunk, gamma
  uint4 raw[kNormPerThread][kNormMaxChunks];
#pragma unroll
  for (int u = 0; u < kNormPerThread; ++u)
#pragma unroll
    for (int i = 0; i < kNormMaxChunks; ++i) raw[u][i] = xr[min(tid + u * kNormThreads + i * kNormVirt, nch - 1)];
  const int cc = min(c, nch - 1);
  const uint4 mine = xr[cc];
  const float4 g0 = reinterpret_cast<const float4*>(gamma)[2 * cc];
  const float4 g1 = reinterpret_cast<const float4*>(gamma)[2 * cc + 1];
#pragma unroll
  for (int u = 0; u < kNormPerThread; ++u) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kNormMaxChunks; ++i) {
      const bool in = tid + u * kNormThreads + i * kNormVirt < nch;
      const uint32_t w4[4] = {raw[u][i].x, raw[u][i].y, raw[u][i].z, raw[u][i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = in ? bf16_to_f32(w4[j] & 0xffff) : 0.f;
        const float hi = in ? bf16_to_f32(w4[j] >> 16) : 0.f;
        ss = __builtin_fmaf(lo, lo, ss);
        ss = __builtin_fmaf(hi, hi, ss);
      }
    }
    ss = wave_sum_f32(ss);
    if ((tid & 63) == 0) part[(tid >> 6) + u * (kNormThreads / 64)] = ss;
  }
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kNormVirt / 64; ++w) tot += part[w];
  const float r = 1.0f / __builtin_sqrtf(tot / static_cast<float>(dim) + eps);
  const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
  const uint32_t w4[4] = {mine.x, mine.y, mine.z, mine.w};
  uint16_t b[8];
  float q[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    b[2 * j] = f32_to_bf16(gv[2 * j] * (bf16_to_f32(w4[j] & 0xffff) * r));
    b[2 * j + 1] = f32_to_bf16(gv[2 * j + 1] * (bf16_to_f32(w4[j] >> 16) * r));
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) q[j] = bf16_to_f32(b[j]);
  if (live)
    reinterpret_cast<uint4*>(y + static_cast<int64_t>(row) * dim)[c] =
        make_uint4(b[0] | (static_cast<uint32_t>(b[1]) << 16), b[2] | (static_cast<uint32_t>(b[3]) << 16),
                   b[4] | (static_cast<uint32_t>(b[5]) << 16), b[6] | (static_cast<uint32_t>(b[7]) << 16));
  if (!y8) return;  // kernel-uniform
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) amax = fmaxf(amax, __builtin_fabsf(q[j]));
  amax = row16_reduce<true>(amax);  // the group's 16 lanes
  const float sc = group_scale(amax, scale_mode);
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    lo |= f32_to_e4m3(fminf(fmaxf(q[j] / sc, -kE4m3Max), kE4m3Max)) << (8 * j);
    hi |= f32_to_e4m3(fminf(fmaxf(q[j + 4] / sc, -kE4m3Max), kE4m3Max)) << (8 * j);
  }
  if (live) {
    reinterpret_cast<uint2*>(y8 + static_cast<int64_t>(row) * dim)[c] = make_uint2(lo, hi);
    if ((c & 15) == 0) ys[static_cast<int64_t>(row) * (dim / kBlock) + (c >> 4)] = sc;
  }
}

}  // namespace tl

using namespace tl;

extern "C" int tl_rmsnorm_quant(const void* x_bf16, const float* gamma, float eps, int64_t rows, int64_t dim,
                                void* y_bf16, void* y_fp8, float* y_scale, int scale_mode, void* stream) {
  if (rows < 0 || dim <= 0 || dim % kBlock || dim > kNormMaxDim) {
    set_error("rmsnorm_quant: dim=%lld must be a positive multiple of 128, at most %d", (long long)dim,
              kNormMaxDim);
    return kErrArg;
  }
  if (scale_mode < 0 || scale_mode > 2) { set_error("rmsnorm_quant: bad scale_mode %d", scale_mode); return kErrArg; }
  if (!x_bf16 || !gamma || !y_bf16 || (!y_fp8) != (!y_scale)) {
    set_error("rmsnorm_quant: null pointer (y_fp8 and y_scale are given together or not at all)");
    return kErrArg;
  }
  if ((reinterpret_cast<uintptr_t>(x_bf16) | reinterpret_cast<uintptr_t>(gamma) | reinterpret_cast<uintptr_t>(y_bf16) |
       reinterpret_cast<uintptr_t>(y_fp8)) & 15) {
    set_error("rmsnorm_quant: pointers must be 16-byte aligned");
    return kErrArg;
  }
  if (rows == 0) return kOk;
  if (rows > 0x7fffffff) { set_error("rmsnorm_quant: too many rows (%lld)", (long long)rows); return kErrArg; }
  const unsigned slices = static_cast<unsigned>(cdiv(dim / 8, kNormSlice));
  hipLaunchKernelGGL(rmsnorm_quant_kernel, dim3(static_cast<unsigned>(rows), slices), dim3(kNormThreads), 0,
                     (hipStream_t)stream, (const uint16_t*)x_bf16, gamma, eps, (int)dim, (uint16_t*)y_bf16,
                     (uint8_t*)y_fp8, y_scale, scale_mode);
  return check_launch("rmsnorm_quant");
}

extern "C" int tl_act_quant(const void* x_bf16, void* y_fp8, float* s, int64_t rows, int64_t K,
                            int64_t group, int scale_mode, void* stream) {
  if (group != kBlock) { set_error("act_quant: only group size 128 is supported (got %lld)", (long long)group); return kErrUnsupported; }
  if (rows < 0 || K <= 0 || K % kBlock != 0) { set_error("act_quant: K=%lld must be a positive multiple of 128", (long long)K); return kErrArg; }
  if (scale_mode < 0 || scale_mode > 2) { set_error("act_quant: bad scale_mode %d", scale_mode); return kErrArg; }
  if (!x_bf16 || !y_fp8 || !s) { set_error("act_quant: null pointer"); return kErrArg; }
  if (rows == 0) return kOk;
  const int64_t n_groups = rows * (K / kBlock);
  const int64_t threads = n_groups * 16;
  hipLaunchKernelGGL(act_quant_kernel, dim3(cdiv(threads, 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x_bf16, (uint8_t*)y_fp8, s, n_groups, scale_mode);
  return check_launch("act_quant");
}

extern "C" int tl_weight_quant(const void* w, int w_is_bf16, void* q_fp8, float* s, int64_t N,
                               int64_t K, void* stream) {
  if (N <= 0 || K <= 0) { set_error("weight_quant: empty weight"); return kErrArg; }
  if (!w || !q_fp8 || !s) { set_error("weight_quant: null pointer"); return kErrArg; }
  dim3 grid(cdiv(K, kBlock), cdiv(N, kBlock));
  if (w_is_bf16)
    hipLaunchKernelGGL(weight_quant_kernel<uint16_t>, grid, dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)w, (uint8_t*)q_fp8, s, N, K);
  else
    hipLaunchKernelGGL(weight_quant_kernel<float>, grid, dim3(256), 0, (hipStream_t)stream,
                       (const float*)w, (uint8_t*)q_fp8, s, N, K);
  return check_launch("weight_quant");
}

extern "C" int tl_weight_dequant(const void* q_fp8, const float* s, void* out, int out_bf16,
                                 int64_t N, int64_t K, void* stream) {
  if (N <= 0 || K <= 0) { set_error("weight_dequant: empty weight"); return kErrArg; }
  if (!q_fp8 || !s || !out) { set_error("weight_dequant: null pointer"); return kErrArg; }
  hipLaunchKernelGGL(weight_dequant_kernel, dim3(cdiv(N * K, 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)q_fp8, s, out, N, K, out_bf16);
  return check_launch("weight_dequant");
}
