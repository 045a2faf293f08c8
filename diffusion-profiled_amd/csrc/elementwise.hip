// Residual join of the U-Net blocks: y = (a + b) / sqrt(2) on bf16 tensors
// (diffusion/unet.py:161 ResidualBlock and :203 the attention block), in one pass with torch's
// two roundings: t = bf16(f32(a) + f32(b)), y = bf16(f32(t) * inv) with inv = RN32(1 / s) (torch
// divides a tensor by a CPU scalar as a product with the fp32 reciprocal). Its backward is
// the same scaling of the incoming gradient. The fp32 form (an fp32 skip path plus a bf16
// branch) does torch's fp32 add and scaling in one pass, and its backward writes both
// operands' gradients in one pass.
#include "dpa_common.hpp"

namespace dpa {

constexpr int kEwThreads = 256;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_round(float v) {
  return __uint_as_float(f32_to_bf16_bits(v) << 16);
}

// 8 elements per thread (one uint4 of each operand); b == nullptr: y = bf16(a * inv).
__global__ __launch_bounds__(kEwThreads) void residual_scale_kernel(
    const uint4* __restrict__ a, const uint4* __restrict__ b, uint4* __restrict__ y,
    int64_t n8, float inv) {
  const int64_t i = (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
  if (i >= n8) return;
  const uint4 va = a[i];
  const uint32_t wa[4] = {va.x, va.y, va.z, va.w};
  uint32_t wb[4] = {0u, 0u, 0u, 0u};
  if (b) {
    const uint4 vb = b[i];
    wb[0] = vb.x; wb[1] = vb.y; wb[2] = vb.z; wb[3] = vb.w;
  }
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float lo = bf16_lo(wa[k]), hi = bf16_hi(wa[k]);
    if (b) {
      lo = bf16_round(lo + bf16_lo(wb[k]));
      hi = bf16_round(hi + bf16_hi(wb[k]));
    }
    o[k] = pack_bf16x2(lo * inv, hi * inv);
  }
  y[i] = uint4{o[0], o[1], o[2], o[3]};
}

// fp32 residual stream (below the first level the skip path is fp32 under autocast): a fp32,
// b bf16, y = RN32(RN32(a + f32(b)) * inv), torch's fp32 add and scalar division; 4 elements
// per thread.
__global__ __launch_bounds__(kEwThreads) void residual_f32_kernel(const float4* __restrict__ a,
                                                                   const uint2* __restrict__ b,
                                                                   float4* __restrict__ y,
                                                                   int64_t n4, float inv) {
  const int64_t i = (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
  if (i >= n4) return;
  const float4 va = a[i];
  const uint2 vb = b[i];
  y[i] = float4{(va.x + bf16_lo(vb.x)) * inv, (va.y + bf16_hi(vb.x)) * inv,
                (va.z + bf16_lo(vb.y)) * inv, (va.w + bf16_hi(vb.y)) * inv};
}

// Its backward: both operands get g * inv, the fp32 one as it is, the bf16 one rounded to bf16
// (autograd's cast of the gradient to the operand's dtype).
__global__ __launch_bounds__(kEwThreads) void residual_f32_bwd_kernel(
    const float4* __restrict__ g, float4* __restrict__ ga, uint2* __restrict__ gb, int64_t n4,
    float inv) {
  const int64_t i = (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
  if (i >= n4) return;
  const float4 v = g[i];
  const float4 s = float4{v.x * inv, v.y * inv, v.z * inv, v.w * inv};
  ga[i] = s;
  gb[i] = uint2{pack_bf16x2(s.x, s.y), pack_bf16x2(s.z, s.w)};
}

}  // namespace dpa

using namespace dpa;

extern "C" int dpa_residual_scale_f32(const float* a, const void* b, float* y, int64_t n,
                                      float inv, void* stream) {
  if (!a || !b || !y) return DPA_ERR_NULL;
  if (n <= 0 || n % 4 != 0) return DPA_ERR_SIZE;
  if (!aligned(a, 16) || !aligned(b, 8) || !aligned(y, 16)) return DPA_ERR_ALIGN;
  const int64_t n4 = n / 4;
  residual_f32_kernel<<<(unsigned)ceil_div(n4, (int64_t)kEwThreads), kEwThreads, 0,
                        (hipStream_t)stream>>>((const float4*)a, (const uint2*)b, (float4*)y, n4,
                                               inv);
  return launch_status();
}

extern "C" int dpa_residual_scale_bwd_f32(const float* g, float* ga, void* gb, int64_t n,
                                          float inv, void* stream) {
  if (!g || !ga || !gb) return DPA_ERR_NULL;
  if (n <= 0 || n % 4 != 0) return DPA_ERR_SIZE;
  if (!aligned(g, 16) || !aligned(ga, 16) || !aligned(gb, 8)) return DPA_ERR_ALIGN;
  const int64_t n4 = n / 4;
  residual_f32_bwd_kernel<<<(unsigned)ceil_div(n4, (int64_t)kEwThreads), kEwThreads, 0,
                            (hipStream_t)stream>>>((const float4*)g, (float4*)ga, (uint2*)gb, n4,
                                                   inv);
  return launch_status();
}

extern "C" int dpa_residual_scale_bf16(const void* a, const void* b, void* y, int64_t n,
                                       float inv, void* stream) {
  if (!a || !y) return DPA_ERR_NULL;
  if (n <= 0 || n % 8 != 0) return DPA_ERR_SIZE;
  if (!aligned(a, 16) || !aligned(b, 16) || !aligned(y, 16)) return DPA_ERR_ALIGN;
  const int64_t n8 = n / 8;
  residual_scale_kernel<<<(unsigned)ceil_div(n8, (int64_t)kEwThreads), kEwThreads, 0,
                          (hipStream_t)stream>>>((const uint4*)a, (const uint4*)b, (uint4*)y, n8,
                                                 inv);
  return launch_status();
}
