// Per-tensor absmax scaling and OCP-e4m3 cast (current and delayed scaling).
//
// Reference: diffusion/fp8_kernels.py
//   partial_amax_kernel          :54-64    -> amax_partials_kernel (first pass, current)
//   finalize_amax_kernel         :90-102   -> folded into cast_current_kernel / finalize_kernel
//   quantize_fp8_kernel          :105-120  -> cast_current_kernel
//   partial_amax_kernel_delayed  :69-87    -> cast_delayed_kernel
//   quantize_fp8 / _delayed      :518-601  -> dpa_quantize_fp8_bf16 / _delayed_bf16
//
// Design: the amax is reduced as bf16 magnitude bit patterns with packed u16 max (exact and
// order-free). Partials are one u32 per block; every block of the cast kernel re-reduces
// the (<= kMaxPartials) partials from L2 and derives the scale itself, so current scaling
// needs two launches, no atomics and no zero-initialised state (safe under graph capture).
#include "dpa_common.hpp"

namespace dpa {

constexpr int kQThreads = 256;
constexpr int kMaxPartials = 1024;
constexpr int kElemsPerIter = 16;  // per thread and iteration: two uint4 of bf16

__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, uint32_t* red) {
  v = wave_max_u32(v);
  const int wid = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wid] = v;
  __syncthreads();
  uint32_t r = red[0];
#pragma unroll
  for (int i = 1; i < kQThreads / 64; ++i) r = r > red[i] ? r : red[i];
  return r;
}

// Max over the partials written by the first pass, recomputed by every block.
__device__ __forceinline__ uint32_t reduce_partials(const uint32_t* partials, int np,
                                                    uint32_t* red) {
  uint32_t m = 0;
  for (int i = threadIdx.x; i < np; i += kQThreads) {
    uint32_t p = partials[i];
    m = m > p ? m : p;
  }
  return block_max_u32(m, red);
}

// Pass 1 (current scaling): per-block amax of |x| as bf16 bits.
template <bool kVec>
__global__ __launch_bounds__(kQThreads) void amax_partials_kernel(const uint16_t* __restrict__ x,
                                                                  int64_t n,
                                                                  uint32_t* __restrict__ partials) {
  __shared__ uint32_t red[kQThreads / 64];
  us2 acc = {0, 0};
  uint32_t accs = 0;
  const int64_t stride = (int64_t)gridDim.x * kQThreads * kElemsPerIter;
  int64_t i = ((int64_t)blockIdx.x * kQThreads + threadIdx.x) * kElemsPerIter;
  if (kVec) {
    for (; i + kElemsPerIter <= n; i += stride) {
      uint4 v0 = ld_nt16(x + i);
      uint4 v1 = ld_nt16(x + i + 8);
      acc = absmax8(acc, v0);
      acc = absmax8(acc, v1);
    }
    // ragged tail: at most one partial group, handled by whichever thread reached it
    if (i < n) {
      for (int64_t j = i; j < n; ++j) {
        uint32_t a = x[j] & 0x7fffu;
        accs = accs > a ? accs : a;
      }
    }
  } else {
    for (; i < n; i += stride) {
      for (int64_t j = i; j < i + kElemsPerIter && j < n; ++j) {
        uint32_t a = x[j] & 0x7fffu;
        accs = accs > a ? accs : a;
      }
    }
  }
  uint32_t m = acc.x > acc.y ? acc.x : acc.y;
  m = m > accs ? m : accs;
  m = block_max_u32(m, red);
  if (threadIdx.x == 0) partials[blockIdx.x] = m;
}

// Pass 2 (current scaling): scale from the partials, then q = e4m3(clamp(x / scale)).
template <bool kVec>
__global__ __launch_bounds__(kQThreads) void cast_current_kernel(
    const uint16_t* __restrict__ x, int64_t n, const uint32_t* __restrict__ partials, int np,
    uint8_t* __restrict__ q, float* __restrict__ scale_out) {
  __shared__ uint32_t red[kQThreads / 64];
  const uint32_t amax_bits = reduce_partials(partials, np, red);
  const float scale = scale_from_amax_bits(amax_bits);
  if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;

  const int64_t stride = (int64_t)gridDim.x * kQThreads * kElemsPerIter;
  int64_t i = ((int64_t)blockIdx.x * kQThreads + threadIdx.x) * kElemsPerIter;
  if (kVec) {
    for (; i + kElemsPerIter <= n; i += stride) {
      uint4 v0 = ld_nt16(x + i);
      uint4 v1 = ld_nt16(x + i + 8);
      uint2 a = quant8(v0, scale);
      uint2 b = quant8(v1, scale);
      uint4 o = {a.x, a.y, b.x, b.y};
      st_nt16(q + i, o);
    }
    if (i < n) {
      for (int64_t j = i; j < n; ++j) {
        float f = quant_div(bf16_bits_to_f32(x[j]), scale);
        q[j] = (uint8_t)(pack4_e4m3(f, 0.f, 0.f, 0.f) & 0xffu);
      }
    }
  } else {
    for (; i < n; i += stride) {
      for (int64_t j = i; j < i + kElemsPerIter && j < n; ++j) {
        float f = quant_div(bf16_bits_to_f32(x[j]), scale);
        q[j] = (uint8_t)(pack4_e4m3(f, 0.f, 0.f, 0.f) & 0xffu);
      }
    }
  }
}

// Delayed scaling, one pass: q = cast(x, *prev_scale) and per-block amax of x.
template <bool kVec>
__global__ __launch_bounds__(kQThreads) void cast_delayed_kernel(
    const uint16_t* __restrict__ x, int64_t n, const float* __restrict__ prev_scale,
    uint8_t* __restrict__ q, uint32_t* __restrict__ partials) {
  __shared__ uint32_t red[kQThreads / 64];
  const float scale = *prev_scale;
  us2 acc = {0, 0};
  uint32_t accs = 0;
  const int64_t stride = (int64_t)gridDim.x * kQThreads * kElemsPerIter;
  int64_t i = ((int64_t)blockIdx.x * kQThreads + threadIdx.x) * kElemsPerIter;
  if (kVec) {
    for (; i + kElemsPerIter <= n; i += stride) {
      uint4 v0 = ld_nt16(x + i);
      uint4 v1 = ld_nt16(x + i + 8);
      acc = absmax8(acc, v0);
      acc = absmax8(acc, v1);
      uint2 a = quant8(v0, scale);
      uint2 b = quant8(v1, scale);
      uint4 o = {a.x, a.y, b.x, b.y};
      st_nt16(q + i, o);
    }
    if (i < n) {
      for (int64_t j = i; j < n; ++j) {
        uint32_t a = x[j] & 0x7fffu;
        accs = accs > a ? accs : a;
        float f = quant_div(bf16_bits_to_f32(x[j]), scale);
        q[j] = (uint8_t)(pack4_e4m3(f, 0.f, 0.f, 0.f) & 0xffu);
      }
    }
  } else {
    for (; i < n; i += stride) {
      for (int64_t j = i; j < i + kElemsPerIter && j < n; ++j) {
        uint32_t a = x[j] & 0x7fffu;
        accs = accs > a ? accs : a;
        float f = quant_div(bf16_bits_to_f32(x[j]), scale);
        q[j] = (uint8_t)(pack4_e4m3(f, 0.f, 0.f, 0.f) & 0xffu);
      }
    }
  }
  uint32_t m = acc.x > acc.y ? acc.x : acc.y;
  m = m > accs ? m : accs;
  m = block_max_u32(m, red);
  if (threadIdx.x == 0) partials[blockIdx.x] = m;
}

// Delayed scaling, finalize: cur_scale = scale(max(partials))  (finalize_amax_kernel).
__global__ __launch_bounds__(kQThreads) void finalize_scale_kernel(
    const uint32_t* __restrict__ partials, int np, float* __restrict__ scale_out) {
  __shared__ uint32_t red[kQThreads / 64];
  const uint32_t amax_bits = reduce_partials(partials, np, red);
  if (threadIdx.x == 0) *scale_out = scale_from_amax_bits(amax_bits);
}

static int grid_for(int64_t n, int cap) {
  int64_t g = ceil_div(n, (int64_t)kQThreads * kElemsPerIter);
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (int)g;
}

}  // namespace dpa

using namespace dpa;

extern "C" int64_t dpa_quant_workspace_bytes(int64_t n) {
  (void)n;
  return (int64_t)kMaxPartials * 4;
}

extern "C" int dpa_quantize_fp8_bf16(const void* x, int64_t n, void* q, float* scale_out,
                                     void* workspace, int64_t workspace_bytes, void* stream) {
  if (!x || !q || !scale_out) return DPA_ERR_NULL;
  if (n <= 0) return DPA_ERR_SIZE;
  if (!workspace || workspace_bytes < dpa_quant_workspace_bytes(n)) return DPA_ERR_WORKSPACE;
  if (!aligned(workspace, 4) || !aligned(scale_out, 4) || !aligned(x, 2)) return DPA_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  const bool vec = aligned(x, 16) && aligned(q, 16);
  const int np = grid_for(n, kMaxPartials);
  const int gc = grid_for(n, 4096);
  auto* xp = (const uint16_t*)x;
  auto* part = (uint32_t*)workspace;
  if (vec) {
    amax_partials_kernel<true><<<np, kQThreads, 0, s>>>(xp, n, part);
    cast_current_kernel<true><<<gc, kQThreads, 0, s>>>(xp, n, part, np, (uint8_t*)q, scale_out);
  } else {
    amax_partials_kernel<false><<<np, kQThreads, 0, s>>>(xp, n, part);
    cast_current_kernel<false><<<gc, kQThreads, 0, s>>>(xp, n, part, np, (uint8_t*)q,
                                                        scale_out);
  }
  return launch_status();
}

extern "C" int dpa_quantize_fp8_delayed_bf16(const void* x, int64_t n, const float* prev_scale,
                                             void* q, float* cur_scale_out, void* workspace,
                                             int64_t workspace_bytes, void* stream) {
  if (!x || !q || !prev_scale || !cur_scale_out) return DPA_ERR_NULL;
  if (n <= 0) return DPA_ERR_SIZE;
  if (!workspace || workspace_bytes < dpa_quant_workspace_bytes(n)) return DPA_ERR_WORKSPACE;
  if (!aligned(workspace, 4) || !aligned(cur_scale_out, 4) || !aligned(prev_scale, 4) ||
      !aligned(x, 2))
    return DPA_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  const bool vec = aligned(x, 16) && aligned(q, 16);
  const int np = grid_for(n, kMaxPartials);
  auto* xp = (const uint16_t*)x;
  auto* part = (uint32_t*)workspace;
  if (vec)
    cast_delayed_kernel<true><<<np, kQThreads, 0, s>>>(xp, n, prev_scale, (uint8_t*)q, part);
  else
    cast_delayed_kernel<false><<<np, kQThreads, 0, s>>>(xp, n, prev_scale, (uint8_t*)q, part);
  finalize_scale_kernel<<<1, kQThreads, 0, s>>>(part, np, cur_scale_out);
  return launch_status();
}
