// Shared device/host helpers for the gfx950 FP8 path: bf16 and OCP-e4m3 conversions,
// the per-tensor scale rule, MFMA wrappers and launch plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dpa_fp8.h"

namespace dpa {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned short us2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr float kFp8Max = 448.0f;  // torch.finfo(torch.float8_e4m3fn).max

// ---------------------------------------------------------------------------------------
// bf16 <-> fp32
// ---------------------------------------------------------------------------------------
__host__ __device__ inline float bf16_bits_to_f32(uint32_t b16) {
  uint32_t u = b16 << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

// fp32 -> bf16 bits, round to nearest even; NaN -> canonical quiet NaN of the same sign.
__host__ __device__ inline uint32_t f32_to_bf16_bits(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) & 0x8000u) | 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// ---------------------------------------------------------------------------------------
// Per-tensor scale: amax > 0 ? RN32(amax / 448) : 1  (fp8_kernels.py:100-101).
// amax is carried as the bf16 bit pattern of |x| (max over integer patterns equals the max
// over values for non-negative bf16, so the reduction is exact and order-free).
// ---------------------------------------------------------------------------------------
__host__ __device__ inline float scale_from_amax_bits(uint32_t amax_bf16_bits) {
  float amax = bf16_bits_to_f32(amax_bf16_bits);
  return amax > 0.0f ? amax / kFp8Max : 1.0f;
}

// ---------------------------------------------------------------------------------------
// fp32 -> OCP e4m3 (float8_e4m3fn) with round-to-nearest-even, software version.
// |v| > 464 and NaN -> 0x7f (NaN), like torch's CPU conversion; 448 < |v| <= 464 -> 448.
// Used as the in-kernel reference of the GPU self-test and for documentation of the rule.
// ---------------------------------------------------------------------------------------
__host__ __device__ inline uint32_t e4m3_rne_soft(float v) {
  uint32_t b;
  __builtin_memcpy(&b, &v, 4);
  const uint32_t sign = (b >> 24) & 0x80u;
  const uint32_t a = b & 0x7fffffffu;
  if (a > 0x43e80000u) return sign | 0x7fu;  // > 464 (incl. inf/NaN)
  if (a >= 0x3c800000u) {                    // normal e4m3: |v| >= 2^-6
    const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
    return sign | ((r >> 20) - 0x3c0u);
  }
  // subnormal e4m3: multiples of 2^-9
  const int e = (int)(a >> 23) - 127;
  if (e < -127 + 1) return sign;  // fp32 zero / denormal rounds to 0
  const uint32_t mant = (a & 0x7fffffu) | 0x800000u;
  const int s = 14 - e;  // >= 21 here
  if (s >= 25) return sign;
  uint32_t m = mant >> s;
  const uint32_t rem = mant & ((1u << s) - 1u);
  const uint32_t half = 1u << (s - 1);
  if (rem > half || (rem == half && (m & 1u))) ++m;
  return sign | m;
}

// Clamp in the reference kernel's order: max(-448, min(v, 448))  (fp8_kernels.py:119).
// fminf/fmaxf follow IEEE minNum/maxNum, so a NaN quotient becomes +448.
__device__ __forceinline__ float clamp_fp8(float v) {
  return fmaxf(-kFp8Max, fminf(v, kFp8Max));
}

// Four clamped fp32 values -> four e4m3 bytes (RNE) with gfx950's v_cvt_pk_fp8_f32.
__device__ __forceinline__ uint32_t pack4_e4m3(float a, float b, float c, float d) {
  int r = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  r = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, r, true);
  return (uint32_t)r;
}

// q = e4m3(clamp(RN32(x / scale))) for the 2 bf16 halves of w -> 2 result floats.
__device__ __forceinline__ float quant_div(float x, float scale) {
  return clamp_fp8(x / scale);
}

// The same quotient without a division per element: with r = RN32(1 / scale) a normal float,
// q0 = RN(x r), e = x - scale q0 (exact through the FMA) and q1 = RN(q0 + e r) is the
// correctly rounded x / scale (Markstein's correction; the test of every bf16 input against
// every reachable scale checks it bit for bit). Where q0 is +-inf (x / scale overflows) q1 is
// NaN, and where q1 is 0 its sign may differ from x / scale: q0 is kept in both cases.
__device__ __forceinline__ float quant_rcp(float x, float scale, float r) {
  const float q0 = x * r;
  const float e = __builtin_fmaf(-q0, scale, x);
  const float q1 = __builtin_fmaf(e, r, q0);
  return clamp_fp8((q1 != q1 || q1 == 0.0f) ? q0 : q1);
}

// r = RN32(1 / scale) when the fast quotient is valid for this scale, else 0. The residual
// x - scale q0 is ~2^-23 x; for every quotient that can round to a nonzero e4m3 value
// (x / scale >= 2^-10) it stays a normal float when scale >= 2^-64. Smaller scales (tensors
// whose amax is below ~2^-55) take the division.
__device__ __forceinline__ float quant_recip(float scale) {
  return (scale >= 0x1p-64f && scale <= 0x1p+120f) ? 1.0f / scale : 0.0f;
}

// 8 bf16 (one uint4) -> 8 e4m3 bytes (one uint2), fast quotient (r from quant_recip != 0).
__device__ __forceinline__ uint2 quant8_rcp(uint4 v, float scale, float r) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  float f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = quant_rcp(__uint_as_float(w[i] << 16), scale, r);
    f[2 * i + 1] = quant_rcp(__uint_as_float(w[i] & 0xffff0000u), scale, r);
  }
  uint2 o;
  o.x = pack4_e4m3(f[0], f[1], f[2], f[3]);
  o.y = pack4_e4m3(f[4], f[5], f[6], f[7]);
  return o;
}

// 8 bf16 (one uint4) -> 8 e4m3 bytes (one uint2).
__device__ __forceinline__ uint2 quant8(uint4 v, float scale) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  float f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = quant_div(__uint_as_float(w[i] << 16), scale);
    f[2 * i + 1] = quant_div(__uint_as_float(w[i] & 0xffff0000u), scale);
  }
  uint2 o;
  o.x = pack4_e4m3(f[0], f[1], f[2], f[3]);
  o.y = pack4_e4m3(f[4], f[5], f[6], f[7]);
  return o;
}

// |bf16| magnitude max over the 8 bf16 of a uint4, as packed u16 pairs.
__device__ __forceinline__ us2 absmax8(us2 acc, uint4 v) {
  const uint32_t m = 0x7fff7fffu;
  us2 a = __builtin_bit_cast(us2, v.x & m);
  us2 b = __builtin_bit_cast(us2, v.y & m);
  us2 c = __builtin_bit_cast(us2, v.z & m);
  us2 d = __builtin_bit_cast(us2, v.w & m);
  acc = __builtin_elementwise_max(acc, a);
  acc = __builtin_elementwise_max(acc, b);
  acc = __builtin_elementwise_max(acc, c);
  acc = __builtin_elementwise_max(acc, d);
  return acc;
}

// The delayed-scaling cast of 8 bf16 with a window scale (r = quant_recip(scale)): the same
// bytes as the standalone cast kernel writes for them.
__device__ __forceinline__ uint2 quant8_delayed(uint4 v, float scale, float r) {
  return r != 0.0f ? quant8_rcp(v, scale, r) : quant8(v, scale);
}

// Amax-window state of a delayed-scaling module (diffusion/unet.py:82-91 and
// diffusion/fp8_kernels.py:888-889): window[pos] = scale and, for the last tensor of the
// forward, pos = (pos + 1) % len. A pos outside [0, len) (never produced by this update)
// leaves both untouched. Called by one thread.
__device__ __forceinline__ void window_record(float scale, float* window, int64_t* pos,
                                              int64_t len, int advance) {
  if (!window) return;
  const int64_t p = *pos;
  if (p < 0 || p >= len) return;
  window[p] = scale;
  if (advance) *pos = p + 1 == len ? 0 : p + 1;
}

// Wave-level max of a u32 (64 lanes).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    uint32_t o = __shfl_xor(v, off, 64);
    v = v > o ? v : o;
  }
  return v;
}

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// One u32 amax partial per workgroup for a producer kernel that casts its output: the
// workgroup max of acc (packed bf16 magnitudes) goes to partials[blk]; workgroup 0 also stores
// the partial count nblk. Call from every thread (uniform); red holds one u32 per wave.
__device__ __forceinline__ void store_amax_partial(us2 acc, uint32_t* red, uint32_t* partials,
                                                   uint32_t* count, uint32_t blk,
                                                   uint32_t nblk) {
  uint32_t m = acc.x > acc.y ? acc.x : acc.y;
  m = wave_max_u32(m);
  const int nw = (int)(blockDim.x >> 6);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = red[0];
    for (int i = 1; i < nw; ++i) r = r > red[i] ? r : red[i];
    partials[blk] = r;
    if (blk == 0 && count) *count = nblk;
  }
}

// ---------------------------------------------------------------------------------------
// MFMA: D(16x16 f32) += A(16x128 e4m3) * B(128x16 e4m3).
// Lane l supplies row (l & 15) of A and column (l & 15) of B, 32 K-bytes each at K offset
// 32 * (l >> 4); lane l receives D[4*(l>>4) + t][l & 15], t = 0..3.
// The E8M0 block scales are fixed at 127 (2^0), which makes the scaled form a plain GEMM.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ v4f mfma16x16x128_e4m3(const v8i& a, const v8i& b, const v4f& c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// 16-byte streaming (non-temporal) global load/store.
__device__ __forceinline__ uint4 ld_nt16(const void* p) {
  u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return uint4{v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ void st_nt16(void* p, uint4 v) {
  u32x4 w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
}
__device__ __forceinline__ void st_nt8(void* p, uint2 v) {
  u32x2 w = {v.x, v.y};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x2*>(p));
}

// Two fp32 -> packed bf16 pair (round to nearest even) with gfx950's v_cvt_pk_bf16_f32.
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const v2bf r = __builtin_convertvector((v2f){a, b}, v2bf);
  return __builtin_bit_cast(uint32_t, r);
}

// Bytes of {hi:lo} selected by sel (v_perm_b32).
__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// ---------------------------------------------------------------------------------------
// Global -> LDS DMA and the explicit waits that pipeline it.
// ---------------------------------------------------------------------------------------
#define LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

// 16-B-per-lane global -> LDS DMA (lane i lands at lds + 16 i). Issued through inline asm so
// the compiler does not guard later LDS reads with conservative vmcnt(0) waits: all waits for
// these DMAs are explicit in-order vmcnt counts in the kernels that issue them (in-order counting
// keeps every compiler-inserted wait conservative, hence correct). The asm sets m0 itself and
// lists it as clobbered; clang warns that m0 is a reserved register whose value it may not
// preserve around the statement. In the kernels built here nothing else uses m0 (in the
// compiled igemm / hwgrad / wgrad code every m0 access is one of these s_mov / DMA pairs), so
// no compiler-held value is live across it.
__device__ __forceinline__ void dma16(const void* src, const void* lds) {
  const uint32_t l = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)LDS_PTR(lds));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(l) : "m0");
}

// Same DMA with the LDS destination given as a 32-bit LDS address (wave-uniform).
__device__ __forceinline__ void dma16_lds(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "m0");
}

// 32-bit LDS address of a __shared__ object (no generic-pointer null check).
#define LDS_ADDR(obj) ((uint32_t)(uintptr_t)((__attribute__((address_space(3))) uint8_t*)(obj)))

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] | expcnt | lgkmcnt | vmcnt[5:4]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xc07f); }
// LDS (and scalar-memory) operations complete in order, so lgkmcnt(N) waits for all but the
// N most recently issued LDS operations.
template <int N>
__device__ __forceinline__ void wait_lgkmcnt() {
  static_assert(N >= 0 && N < 16, "lgkmcnt");
  __builtin_amdgcn_s_waitcnt(0xc07f | (N << 8));
}

// Workgroup barrier that the compiler may not move memory operations across (the DMA
// writes above are invisible to it), nor any other instruction: the scheduler would
// otherwise hoist the next step's MFMAs (register-only) above it, next to the fragment reads
// they consume, and undo the read-ahead of the pipelined loops.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// ---------------------------------------------------------------------------------------
// Integer division by a launch-time constant without the ~40-instruction runtime divide.
// ---------------------------------------------------------------------------------------
// x / d for 0 <= x < 2^31 via a precomputed (magic, shift) pair (Granlund-Montgomery).
struct FastDiv {
  uint32_t magic, shift, d;
};
__host__ __device__ inline uint32_t fdiv(uint32_t x, const FastDiv& f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return (__umulhi(x, f.magic) + x) >> f.shift;
#else
  return (uint32_t)((((uint64_t)x * f.magic) >> 32) + x) >> f.shift;
#endif
}
inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  f.shift = s;
  f.magic = (uint32_t)(((1ull << 32) * ((1ull << s) - d)) / d + 1);
  return f;
}

// ---------------------------------------------------------------------------------------
// Host helpers
// ---------------------------------------------------------------------------------------
inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? DPA_OK : (int)e;
}

inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace dpa
