// Residual join of the U-Net blocks: y = (a + b) / sqrt(2) on bf16 tensors
// (diffusion/unet.py:161 ResidualBlock and :203 the attention block), in one pass with torch's
// two roundings: t = bf16(f32(a) + f32(b)), y = bf16(f32(t) * inv) with inv = RN32(1 / s) (torch
// divides a tensor by a CPU scalar as a product with the fp32 reciprocal). Its backward is
// the same scaling of the incoming gradient. The fp32 form (an fp32 skip path plus a bf16
// branch) does torch's fp32 add and scaling in one pass, and its backward writes both
// operands' gradients in one pass. The decoder's upsample + concatenation is one pass each way
// as well (below).
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

// The join's backward when the bf16 operand b is the output of a delayed-scaling FP8 conv:
// b's gradient bf16(g * inv) is not stored but cast for that conv's weight and input
// gradients, e4m3(gb / *scale) (the standalone cast's bytes), with one amax partial of gb per
// workgroup; a's gradient is stored as in the plain backward (fp32 g * inv for the fp32 form,
// the same bf16 values for the bf16 form). Grid-strided over groups of 8 elements.
constexpr int kResQBlocks = 1024;

template <bool kF32>
__global__ __launch_bounds__(kEwThreads) void residual_bwd_q_kernel(
    const void* __restrict__ g, void* __restrict__ ga, uint8_t* __restrict__ q,
    const float* __restrict__ scale_p, uint32_t* __restrict__ part, uint32_t* __restrict__ count,
    int64_t n8, float inv) {
  __shared__ uint32_t red[kEwThreads / 64];
  const float scale = *scale_p;
  const float r = quant_recip(scale);
  us2 acc = {0, 0};
  for (int64_t i = (int64_t)blockIdx.x * kEwThreads + threadIdx.x; i < n8;
       i += (int64_t)gridDim.x * kEwThreads) {
    uint4 gb;
    if constexpr (kF32) {
      const float4* gp = static_cast<const float4*>(g) + 2 * i;
      const float4 v0 = gp[0], v1 = gp[1];
      const float4 s0 = float4{v0.x * inv, v0.y * inv, v0.z * inv, v0.w * inv};
      const float4 s1 = float4{v1.x * inv, v1.y * inv, v1.z * inv, v1.w * inv};
      float4* ap = static_cast<float4*>(ga) + 2 * i;
      ap[0] = s0;
      ap[1] = s1;
      gb = uint4{pack_bf16x2(s0.x, s0.y), pack_bf16x2(s0.z, s0.w), pack_bf16x2(s1.x, s1.y),
                 pack_bf16x2(s1.z, s1.w)};
    } else {
      const uint4 v = static_cast<const uint4*>(g)[i];
      gb = uint4{pack_bf16x2(bf16_lo(v.x) * inv, bf16_hi(v.x) * inv),
                 pack_bf16x2(bf16_lo(v.y) * inv, bf16_hi(v.y) * inv),
                 pack_bf16x2(bf16_lo(v.z) * inv, bf16_hi(v.z) * inv),
                 pack_bf16x2(bf16_lo(v.w) * inv, bf16_hi(v.w) * inv)};
      static_cast<uint4*>(ga)[i] = gb;
    }
    st_nt8(q + 8 * i, quant8_delayed(gb, scale, r));
    acc = absmax8(acc, gb);
  }
  store_amax_partial(acc, red, part, count, blockIdx.x, gridDim.x);
}

// Decoder input of the U-Net (diffusion/unet.py:379-382): y = cat([up(a), h], channels) in
// NHWC, fp32 (autocast runs F.interpolate in fp32 and the concatenation promotes), where
// up(a) is a 2x nearest upsampling of a (or a itself). One pass reads a and h once and writes
// y; the upsampled tensor is never formed. 4 channels per thread.
template <typename T>
__device__ __forceinline__ float4 load4f(const T* p);
template <>
__device__ __forceinline__ float4 load4f<float>(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}
template <>
__device__ __forceinline__ float4 load4f<uint16_t>(const uint16_t* p) {
  const uint2 v = *reinterpret_cast<const uint2*>(p);
  return float4{bf16_lo(v.x), bf16_hi(v.x), bf16_lo(v.y), bf16_hi(v.y)};
}
template <typename T>
__device__ __forceinline__ void store4(T* p, float4 v);
template <>
__device__ __forceinline__ void store4<float>(float* p, float4 v) {
  *reinterpret_cast<float4*>(p) = v;
}
template <>
__device__ __forceinline__ void store4<uint16_t>(uint16_t* p, float4 v) {
  *reinterpret_cast<uint2*>(p) = uint2{pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)};
}

struct UpcatArgs {
  int N, H, W, C1, C2, up;  // output H x W; a is (H >> up) x (W >> up) x C1, h is H x W x C2
};

template <typename TA, typename TH>
__global__ __launch_bounds__(kEwThreads) void upcat_fwd_kernel(const TA* __restrict__ a,
                                                                const TH* __restrict__ h,
                                                                float* __restrict__ y,
                                                                UpcatArgs g, int64_t total4) {
  const int64_t i = (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
  if (i >= total4) return;
  const int ct4 = (g.C1 + g.C2) >> 2;
  const int64_t pix = i / ct4;
  const int c = (int)(i - pix * ct4) * 4;
  float4 v;
  if (c < g.C1) {
    const int64_t hw = (int64_t)g.H * g.W;
    const int64_t n = pix / hw;
    const int r = (int)(pix - n * hw);
    const int yy = r / g.W, xx = r - yy * g.W;
    const int64_t q = (n * (g.H >> g.up) + (yy >> g.up)) * (g.W >> g.up) + (xx >> g.up);
    v = load4f<TA>(a + q * g.C1 + c);
  } else {
    v = load4f<TH>(h + pix * g.C2 + (c - g.C1));
  }
  *reinterpret_cast<float4*>(y + pix * (g.C1 + g.C2) + c) = v;
}

// Backward: ga = sum of gy over each 2x2 window (channels < C1), accumulated from zero in
// row-major order as torch's upsample_nearest2d_backward does, in a's dtype; gh = gy's
// channels >= C1 in h's dtype. Items [0, na4) are ga's, the rest gh's.
template <typename TA, typename TH>
__global__ __launch_bounds__(kEwThreads) void upcat_bwd_kernel(const float* __restrict__ gy,
                                                                TA* __restrict__ ga,
                                                                TH* __restrict__ gh, UpcatArgs g,
                                                                int64_t na4, int64_t total4) {
  const int64_t i = (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
  if (i >= total4) return;
  const int ct = g.C1 + g.C2;
  if (i < na4) {
    const int c14 = g.C1 >> 2;
    const int64_t q = i / c14;
    const int c = (int)(i - q * c14) * 4;
    const int hl = g.H >> g.up, wl = g.W >> g.up;
    const int64_t hwl = (int64_t)hl * wl;
    const int64_t n = q / hwl;
    const int r = (int)(q - n * hwl);
    const int yl = r / wl, xl = r - yl * wl;
    const int s = 1 << g.up;
    float4 acc = float4{0.f, 0.f, 0.f, 0.f};
    for (int dy = 0; dy < s; ++dy)
      for (int dx = 0; dx < s; ++dx) {
        const int64_t p = (n * g.H + (yl * s + dy)) * g.W + (xl * s + dx);
        const float4 v = *reinterpret_cast<const float4*>(gy + p * ct + c);
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
      }
    store4<TA>(ga + q * g.C1 + c, acc);
  } else {
    const int64_t j = i - na4;
    const int c24 = g.C2 >> 2;
    const int64_t p = j / c24;
    const int c = (int)(j - p * c24) * 4;
    store4<TH>(gh + p * g.C2 + c, *reinterpret_cast<const float4*>(gy + p * ct + g.C1 + c));
  }
}

// Encoder downsampling F.interpolate(a, scale_factor=0.5, mode="nearest") (diffusion/unet.py:
// 370-373) under autocast: y[i][j] = f32(a[2i][2j]) in NHWC, fp32 out; backward ga[2i][2j] =
// gy[i][j] and 0 elsewhere, in a's dtype. 4 channels per thread.
template <typename TA>
__global__ __launch_bounds__(kEwThreads) void down2_fwd_kernel(const TA* __restrict__ a,
                                                                float* __restrict__ y, int H,
                                                                int W, int C, int64_t total4) {
  const int64_t i = (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
  if (i >= total4) return;
  const int c4 = C >> 2, ho = H >> 1, wo = W >> 1;
  const int64_t q = i / c4;
  const int c = (int)(i - q * c4) * 4;
  const int64_t hwo = (int64_t)ho * wo;
  const int64_t n = q / hwo;
  const int r = (int)(q - n * hwo);
  const int yo = r / wo, xo = r - yo * wo;
  const int64_t p = (n * H + 2 * yo) * W + 2 * xo;
  *reinterpret_cast<float4*>(y + q * C + c) = load4f<TA>(a + p * C + c);
}

template <typename TA>
__global__ __launch_bounds__(kEwThreads) void down2_bwd_kernel(const float* __restrict__ gy,
                                                                TA* __restrict__ ga, int H, int W,
                                                                int C, int64_t total4) {
  const int64_t i = (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
  if (i >= total4) return;
  const int c4 = C >> 2;
  const int64_t p = i / c4;
  const int c = (int)(i - p * c4) * 4;
  const int64_t hw = (int64_t)H * W;
  const int64_t n = p / hw;
  const int r = (int)(p - n * hw);
  const int yy = r / W, xx = r - yy * W;
  float4 v = float4{0.f, 0.f, 0.f, 0.f};
  if (((yy | xx) & 1) == 0) {
    const int64_t q = (n * (H >> 1) + (yy >> 1)) * (W >> 1) + (xx >> 1);
    v = *reinterpret_cast<const float4*>(gy + q * C + c);
  }
  store4<TA>(ga + p * C + c, v);
}

// The same backward with the gradient that a's other reader (the decoder's concatenation)
// sent added in: ga = a_dtype(gy or 0) + gskip, rounded as autograd's sum of the two
// gradients (the downsampling's in a's dtype, then one add in a's dtype; every pixel gets the
// add, so a -0 skip gradient beside a 0 becomes +0 as there). ga may alias gskip.
template <typename TA>
__global__ __launch_bounds__(kEwThreads) void down2_bwd_add_kernel(
    const float* __restrict__ gy, const TA* gskip, TA* ga, int H, int W, int C, int64_t total4) {
  const int64_t i = (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
  if (i >= total4) return;
  const int c4 = C >> 2;
  const int64_t p = i / c4;
  const int c = (int)(i - p * c4) * 4;
  const int64_t hw = (int64_t)H * W;
  const int64_t n = p / hw;
  const int r = (int)(p - n * hw);
  const int yy = r / W, xx = r - yy * W;
  float4 v = float4{0.f, 0.f, 0.f, 0.f};
  if (((yy | xx) & 1) == 0) {
    const int64_t q = (n * (H >> 1) + (yy >> 1)) * (W >> 1) + (xx >> 1);
    v = *reinterpret_cast<const float4*>(gy + q * C + c);
  }
  const float4 s = load4f<TA>(gskip + p * C + c);
  float4 o;
  if constexpr (sizeof(TA) == 2) {  // bf16(bf16(v) + s)
    o = float4{bf16_round(v.x) + s.x, bf16_round(v.y) + s.y, bf16_round(v.z) + s.z,
               bf16_round(v.w) + s.w};
  } else {
    o = float4{v.x + s.x, v.y + s.y, v.z + s.z, v.w + s.w};
  }
  store4<TA>(ga + p * C + c, o);
}

}  // namespace dpa

using namespace dpa;

extern "C" int dpa_downsample2_f32(const void* a, int a_dtype, float* y, int N, int H, int W,
                                   int C, void* stream) {
  const int af = a_dtype == DPA_DTYPE_F32;
  if (!af && a_dtype != DPA_DTYPE_BF16) return DPA_ERR_SHAPE;
  if (!a || !y) return DPA_ERR_NULL;
  if (N <= 0 || H <= 0 || W <= 0 || C <= 0 || C % 4) return DPA_ERR_SIZE;
  if (H % 2 || W % 2) return DPA_ERR_SHAPE;
  if (!aligned(a, af ? 16 : 8) || !aligned(y, 16)) return DPA_ERR_ALIGN;
  const int64_t total4 = (int64_t)N * (H / 2) * (W / 2) * (C / 4);
  const unsigned grid = (unsigned)ceil_div(total4, (int64_t)kEwThreads);
  if (af)
    down2_fwd_kernel<float><<<grid, kEwThreads, 0, (hipStream_t)stream>>>((const float*)a, y, H, W, C, total4);
  else
    down2_fwd_kernel<uint16_t><<<grid, kEwThreads, 0, (hipStream_t)stream>>>((const uint16_t*)a, y, H, W, C, total4);
  return launch_status();
}

extern "C" int dpa_downsample2_bwd_f32(const float* gy, void* ga, int a_dtype, int N, int H,
                                       int W, int C, void* stream) {
  const int af = a_dtype == DPA_DTYPE_F32;
  if (!af && a_dtype != DPA_DTYPE_BF16) return DPA_ERR_SHAPE;
  if (!gy || !ga) return DPA_ERR_NULL;
  if (N <= 0 || H <= 0 || W <= 0 || C <= 0 || C % 4) return DPA_ERR_SIZE;
  if (H % 2 || W % 2) return DPA_ERR_SHAPE;
  if (!aligned(ga, af ? 16 : 8) || !aligned(gy, 16)) return DPA_ERR_ALIGN;
  const int64_t total4 = (int64_t)N * H * W * (C / 4);
  const unsigned grid = (unsigned)ceil_div(total4, (int64_t)kEwThreads);
  if (af)
    down2_bwd_kernel<float><<<grid, kEwThreads, 0, (hipStream_t)stream>>>(gy, (float*)ga, H, W, C, total4);
  else
    down2_bwd_kernel<uint16_t><<<grid, kEwThreads, 0, (hipStream_t)stream>>>(gy, (uint16_t*)ga, H, W, C, total4);
  return launch_status();
}

static int upcat_check(const void* a, const void* h, const void* y, int a_f32, int h_f32, int N,
                       int H, int W, int C1, int C2, int up) {
  if (!a || !h || !y) return DPA_ERR_NULL;
  if (N <= 0 || H <= 0 || W <= 0 || C1 <= 0 || C2 <= 0 || C1 % 4 || C2 % 4) return DPA_ERR_SIZE;
  if ((up != 0 && up != 1) || (up && (H % 2 || W % 2))) return DPA_ERR_SHAPE;
  if ((int64_t)N * H * W * (C1 + C2) > ((int64_t)1 << 40)) return DPA_ERR_SIZE;
  if (!aligned(a, a_f32 ? 16 : 8) || !aligned(h, h_f32 ? 16 : 8) || !aligned(y, 16))
    return DPA_ERR_ALIGN;
  return DPA_OK;
}

extern "C" int dpa_upsample_concat_f32(const void* a, int a_dtype, const void* h, int h_dtype,
                                       float* y, int N, int H, int W, int C1, int C2, int up,
                                       void* stream) {
  const int af = a_dtype == DPA_DTYPE_F32, hf = h_dtype == DPA_DTYPE_F32;
  if ((!af && a_dtype != DPA_DTYPE_BF16) || (!hf && h_dtype != DPA_DTYPE_BF16)) return DPA_ERR_SHAPE;
  const int st = upcat_check(a, h, y, af, hf, N, H, W, C1, C2, up);
  if (st != DPA_OK) return st;
  UpcatArgs g{N, H, W, C1, C2, up};
  const int64_t total4 = (int64_t)N * H * W * ((C1 + C2) / 4);
  const unsigned grid = (unsigned)ceil_div(total4, (int64_t)kEwThreads);
  hipStream_t s = (hipStream_t)stream;
  if (af && hf)
    upcat_fwd_kernel<float, float><<<grid, kEwThreads, 0, s>>>((const float*)a, (const float*)h, y, g, total4);
  else if (af)
    upcat_fwd_kernel<float, uint16_t><<<grid, kEwThreads, 0, s>>>((const float*)a, (const uint16_t*)h, y, g, total4);
  else if (hf)
    upcat_fwd_kernel<uint16_t, float><<<grid, kEwThreads, 0, s>>>((const uint16_t*)a, (const float*)h, y, g, total4);
  else
    upcat_fwd_kernel<uint16_t, uint16_t><<<grid, kEwThreads, 0, s>>>((const uint16_t*)a, (const uint16_t*)h, y, g, total4);
  return launch_status();
}

extern "C" int dpa_upsample_concat_bwd_f32(const float* gy, void* ga, int a_dtype, void* gh,
                                           int h_dtype, int N, int H, int W, int C1, int C2,
                                           int up, void* stream) {
  const int af = a_dtype == DPA_DTYPE_F32, hf = h_dtype == DPA_DTYPE_F32;
  if ((!af && a_dtype != DPA_DTYPE_BF16) || (!hf && h_dtype != DPA_DTYPE_BF16)) return DPA_ERR_SHAPE;
  const int st = upcat_check(ga, gh, gy, af, hf, N, H, W, C1, C2, up);
  if (st != DPA_OK) return st;
  UpcatArgs g{N, H, W, C1, C2, up};
  const int64_t na4 = (int64_t)N * (H >> up) * (W >> up) * (C1 / 4);
  const int64_t total4 = na4 + (int64_t)N * H * W * (C2 / 4);
  const unsigned grid = (unsigned)ceil_div(total4, (int64_t)kEwThreads);
  hipStream_t s = (hipStream_t)stream;
  if (af && hf)
    upcat_bwd_kernel<float, float><<<grid, kEwThreads, 0, s>>>(gy, (float*)ga, (float*)gh, g, na4, total4);
  else if (af)
    upcat_bwd_kernel<float, uint16_t><<<grid, kEwThreads, 0, s>>>(gy, (float*)ga, (uint16_t*)gh, g, na4, total4);
  else if (hf)
    upcat_bwd_kernel<uint16_t, float><<<grid, kEwThreads, 0, s>>>(gy, (uint16_t*)ga, (float*)gh, g, na4, total4);
  else
    upcat_bwd_kernel<uint16_t, uint16_t><<<grid, kEwThreads, 0, s>>>(gy, (uint16_t*)ga, (uint16_t*)gh, g, na4, total4);
  return launch_status();
}

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

// The join's backward for a gradient an FP8 GEMM quantizes next with current scaling (the
// attention out-projection's dy, a 1x1 skip conv's or a current-scaling conv's dy): the bf16
// gradient bf16(g * inv) is stored (kF32: ga = g * inv in fp32 and gb = its bf16 rounding;
// otherwise the one bf16 tensor both operands receive, written to gb) with one amax partial of
// those bf16 values per workgroup, so the GEMM's cast runs without its amax pass. Grid-strided
// over groups of 8 elements, as residual_bwd_q_kernel.
template <bool kF32>
__global__ __launch_bounds__(kEwThreads) void residual_bwd_amax_kernel(
    const void* __restrict__ g, float* __restrict__ ga, uint4* __restrict__ gb,
    uint32_t* __restrict__ part, int64_t n8, float inv) {
  __shared__ uint32_t red[kEwThreads / 64];
  us2 acc = {0, 0};
  for (int64_t i = (int64_t)blockIdx.x * kEwThreads + threadIdx.x; i < n8;
       i += (int64_t)gridDim.x * kEwThreads) {
    uint4 o;
    if constexpr (kF32) {
      const float4* gp = static_cast<const float4*>(g) + 2 * i;
      const float4 v0 = gp[0], v1 = gp[1];
      const float4 s0 = float4{v0.x * inv, v0.y * inv, v0.z * inv, v0.w * inv};
      const float4 s1 = float4{v1.x * inv, v1.y * inv, v1.z * inv, v1.w * inv};
      float4* ap = reinterpret_cast<float4*>(ga) + 2 * i;
      ap[0] = s0;
      ap[1] = s1;
      o = uint4{pack_bf16x2(s0.x, s0.y), pack_bf16x2(s0.z, s0.w), pack_bf16x2(s1.x, s1.y),
                pack_bf16x2(s1.z, s1.w)};
    } else {
      const uint4 v = static_cast<const uint4*>(g)[i];
      o = uint4{pack_bf16x2(bf16_lo(v.x) * inv, bf16_hi(v.x) * inv),
                pack_bf16x2(bf16_lo(v.y) * inv, bf16_hi(v.y) * inv),
                pack_bf16x2(bf16_lo(v.z) * inv, bf16_hi(v.z) * inv),
                pack_bf16x2(bf16_lo(v.w) * inv, bf16_hi(v.w) * inv)};
    }
    gb[i] = o;
    acc = absmax8(acc, o);
  }
  store_amax_partial(acc, red, part, nullptr, blockIdx.x, gridDim.x);
}

static int64_t residual_q_blocks(int64_t n) {
  const int64_t b = ceil_div(n / 8, (int64_t)kEwThreads);
  return b < kResQBlocks ? b : kResQBlocks;
}

extern "C" int dpa_residual_scale_fp8_partials(int64_t n) {
  return n > 0 && n % 8 == 0 ? (int)residual_q_blocks(n) : 0;
}

extern "C" int dpa_residual_scale_bwd_amax(const void* g, int g_dtype, float* ga, void* gb,
                                           uint32_t* gb_partials, int gb_partials_cap,
                                           int64_t n, float inv, void* stream) {
  if (!g || !gb || !gb_partials) return DPA_ERR_NULL;
  if (g_dtype != DPA_DTYPE_BF16 && g_dtype != DPA_DTYPE_F32) return DPA_ERR_SHAPE;
  if ((g_dtype == DPA_DTYPE_F32) != (ga != nullptr)) return DPA_ERR_NULL;
  if (n <= 0 || n % 8 != 0) return DPA_ERR_SIZE;
  const int64_t nb = residual_q_blocks(n);
  if (gb_partials_cap < nb) return DPA_ERR_WORKSPACE;
  if (!aligned(g, 16) || !aligned(ga, 16) || !aligned(gb, 16) || !aligned(gb_partials, 4))
    return DPA_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  if (g_dtype == DPA_DTYPE_F32)
    residual_bwd_amax_kernel<true><<<(unsigned)nb, kEwThreads, 0, s>>>(
        g, ga, (uint4*)gb, gb_partials, n / 8, inv);
  else
    residual_bwd_amax_kernel<false><<<(unsigned)nb, kEwThreads, 0, s>>>(
        g, nullptr, (uint4*)gb, gb_partials, n / 8, inv);
  return launch_status();
}

extern "C" int dpa_residual_scale_bwd_fp8(const void* g, int g_dtype, void* ga, void* gbq,
                                          const float* gb_scale, uint32_t* gb_partials,
                                          int gb_partials_cap, uint32_t* gb_count, int64_t n,
                                          float inv, void* stream) {
  if (!g || !ga || !gbq || !gb_scale || !gb_partials || !gb_count) return DPA_ERR_NULL;
  if (g_dtype != DPA_DTYPE_BF16 && g_dtype != DPA_DTYPE_F32) return DPA_ERR_SHAPE;
  if (n <= 0 || n % 8 != 0) return DPA_ERR_SIZE;
  const int64_t nb = residual_q_blocks(n);
  if (gb_partials_cap < nb) return DPA_ERR_WORKSPACE;
  if (!aligned(g, 16) || !aligned(ga, 16) || !aligned(gbq, 8) || !aligned(gb_scale, 4) ||
      !aligned(gb_partials, 4) || !aligned(gb_count, 4))
    return DPA_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  if (g_dtype == DPA_DTYPE_F32)
    residual_bwd_q_kernel<true><<<(unsigned)nb, kEwThreads, 0, s>>>(
        g, ga, (uint8_t*)gbq, gb_scale, gb_partials, gb_count, n / 8, inv);
  else
    residual_bwd_q_kernel<false><<<(unsigned)nb, kEwThreads, 0, s>>>(
        g, ga, (uint8_t*)gbq, gb_scale, gb_partials, gb_count, n / 8, inv);
  return launch_status();
}

extern "C" int dpa_downsample2_bwd_add_f32(const float* gy, const void* gskip, void* ga,
                                           int a_dtype, int N, int H, int W, int C,
                                           void* stream) {
  const int af = a_dtype == DPA_DTYPE_F32;
  if (!af && a_dtype != DPA_DTYPE_BF16) return DPA_ERR_SHAPE;
  if (!gy || !gskip || !ga) return DPA_ERR_NULL;
  if (N <= 0 || H <= 0 || W <= 0 || C <= 0 || C % 4) return DPA_ERR_SIZE;
  if (H % 2 || W % 2) return DPA_ERR_SHAPE;
  if (!aligned(ga, af ? 16 : 8) || !aligned(gskip, af ? 16 : 8) || !aligned(gy, 16))
    return DPA_ERR_ALIGN;
  const int64_t total4 = (int64_t)N * H * W * (C / 4);
  const unsigned grid = (unsigned)ceil_div(total4, (int64_t)kEwThreads);
  if (af)
    down2_bwd_add_kernel<float><<<grid, kEwThreads, 0, (hipStream_t)stream>>>(
        gy, (const float*)gskip, (float*)ga, H, W, C, total4);
  else
    down2_bwd_add_kernel<uint16_t><<<grid, kEwThreads, 0, (hipStream_t)stream>>>(
        gy, (const uint16_t*)gskip, (uint16_t*)ga, H, W, C, total4);
  return launch_status();
}
