// LayerNorm over the channel axis of token rows, bf16 in and out, fp32 statistics: the
// attention block's norm (diffusion/unet.py:174, nn.LayerNorm(hidden) on the [B, H*W, C]
// token view of the channels-last activation, run by autocast in fp32 and rounded to bf16 by
// the qkv projection's cast). Reading the bf16 tokens and writing the bf16 result directly
// replaces torch's fp32 upcast copy, fp32 LayerNorm and the bf16 downcast copy (and the same
// three in the backward).
//
//   forward:  y = bf16( (x - mean) * rstd * gamma + beta ),  var biased, rstd = 1/sqrt(var+eps)
//   backward: g = dy * gamma; dx = rstd * (g - mean(g) - xhat * mean(g * xhat))
//             dgamma = sum_rows dy * xhat, dbeta = sum_rows dy
//
// One wave per row (C / 64 channels per lane, held in registers; mean and variance in two
// passes over the registers); a wave loads all of its 2-8 rows before using any, so each wave
// makes one memory round trip. The backward's column sums go to per-workgroup partials (a
// fixed row range each), reduced over workgroups in a fixed order by a second kernel
// (deterministic).
#include <type_traits>

#include "dpa_common.hpp"

namespace dpa {

constexpr int kLnThreads = 256;
constexpr int kLnWaves = kLnThreads / 64;
constexpr int kLnMaxPerLane = 16;  // C <= 1024
constexpr int kLnRedSlices = 32;   // parameter reduce: block partials per column in 32 slices

// Rows per wave: all of a wave's rows are loaded before any is used (one memory round trip).
template <int V>
constexpr int ln_rows() { return V <= 4 ? 8 : (V == 8 ? 4 : 2); }
template <int V>
constexpr int ln_rows_per_block() { return kLnWaves * ln_rows<V>(); }

struct LnArgs {
  const void* x;  // bf16 or fp32 rows
  const uint16_t* dout;
  const float* gamma;
  const float* beta;
  void* out;  // forward: bf16 y; backward: dx in x's type
  float* mean;
  float* rstd;
  float* part;  // bwd: [blocks][2][C]
  uint32_t* amax_part;  // fwd, optional: per-workgroup max of |y| (bf16 magnitude bits)
  const void* dx_add;   // bwd, optional: added to dx as it is stored (x's type)
  int64_t rows;
  int C;
  float eps;
};

// Lane l holds channels l*V .. l*V+V-1 (V = C / 64) of a row, as V/2 packed bf16 pairs (V = 1:
// one bf16 in the low half).
template <int V>
struct LnRaw {
  uint32_t w[(V + 1) / 2];
};

template <int V>
__device__ __forceinline__ void ln_load(const uint16_t* row, int lane, LnRaw<V>& r) {
  const uint16_t* p = row + lane * V;
  if constexpr (V % 8 == 0) {
#pragma unroll
    for (int k = 0; k < V; k += 8) {
      const uint4 u = *reinterpret_cast<const uint4*>(p + k);
      r.w[k / 2] = u.x;
      r.w[k / 2 + 1] = u.y;
      r.w[k / 2 + 2] = u.z;
      r.w[k / 2 + 3] = u.w;
    }
  } else if constexpr (V == 4) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    r.w[0] = u.x;
    r.w[1] = u.y;
  } else if constexpr (V == 2) {
    r.w[0] = *reinterpret_cast<const uint32_t*>(p);
  } else {
    r.w[0] = p[0];
  }
}

template <int V>
__device__ __forceinline__ void ln_unpack(const LnRaw<V>& r, float (&f)[V]) {
  if constexpr (V == 1) {
    f[0] = __uint_as_float(r.w[0] << 16);
  } else {
#pragma unroll
    for (int k = 0; k < V / 2; ++k) {
      f[2 * k] = __uint_as_float(r.w[k] << 16);
      f[2 * k + 1] = __uint_as_float(r.w[k] & 0xffff0000u);
    }
  }
}

// Returns the packed magnitudes of what it wrote folded into am (u16 max per half).
template <int V>
__device__ __forceinline__ void ln_store(uint16_t* row, int lane, const float (&f)[V], us2& am) {
  uint16_t* p = row + lane * V;
  if constexpr (V % 2 == 0) {
#pragma unroll
    for (int k = 0; k < V; k += 2) {
      const uint32_t w = pack_bf16x2(f[k], f[k + 1]);
      *reinterpret_cast<uint32_t*>(p + k) = w;
      am = __builtin_elementwise_max(am, __builtin_bit_cast(us2, w & 0x7fff7fffu));
    }
  } else {
    const uint32_t b = f32_to_bf16_bits(f[0]);
    p[0] = (uint16_t)b;
    am = __builtin_elementwise_max(am, us2{(unsigned short)(b & 0x7fffu), 0});
  }
}

// fp32 rows (the fp32 residual stream, which autocast's float32 LayerNorm reads as it is)
template <int V>
struct LnRawF {
  float f[V];
};

template <int V>
__device__ __forceinline__ void ln_load(const float* row, int lane, LnRawF<V>& r) {
  const float* p = row + lane * V;
  if constexpr (V % 4 == 0) {
#pragma unroll
    for (int k = 0; k < V; k += 4) {
      const float4 u = *reinterpret_cast<const float4*>(p + k);
      r.f[k] = u.x;
      r.f[k + 1] = u.y;
      r.f[k + 2] = u.z;
      r.f[k + 3] = u.w;
    }
  } else if constexpr (V == 2) {
    const float2 u = *reinterpret_cast<const float2*>(p);
    r.f[0] = u.x;
    r.f[1] = u.y;
  } else {
    r.f[0] = p[0];
  }
}

template <int V>
__device__ __forceinline__ void ln_unpack(const LnRawF<V>& r, float (&f)[V]) {
#pragma unroll
  for (int k = 0; k < V; ++k) f[k] = r.f[k];
}

template <int V>
__device__ __forceinline__ void ln_store(float* row, int lane, const float (&f)[V]) {
  float* p = row + lane * V;
  if constexpr (V % 4 == 0) {
#pragma unroll
    for (int k = 0; k < V; k += 4)
      *reinterpret_cast<float4*>(p + k) = float4{f[k], f[k + 1], f[k + 2], f[k + 3]};
  } else {
#pragma unroll
    for (int k = 0; k < V; ++k) p[k] = f[k];
  }
}
template <int V>
__device__ __forceinline__ void ln_store(float* row, int lane, const float (&f)[V], us2&) {
  ln_store<V>(row, lane, f);
}

template <bool kF32>
using LnXT = typename std::conditional<kF32, float, uint16_t>::type;
template <int V, bool kF32>
using LnXRaw = typename std::conditional<kF32, LnRawF<V>, LnRaw<V>>::type;

template <int V, bool kF32>
__global__ __launch_bounds__(kLnThreads) void ln_fwd_kernel(const LnArgs p) {
  using XT = LnXT<kF32>;
  const XT* px = static_cast<const XT*>(p.x);
  constexpr int R = ln_rows<V>();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r0 = (int64_t)blockIdx.x * ln_rows_per_block<V>() + wave * R;
  LnXRaw<V, kF32> raw[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int64_t r = r0 + i < p.rows ? r0 + i : p.rows - 1;  // past the end: a valid row
    ln_load<V>(px + r * p.C, lane, raw[i]);
  }
  float g[V], b[V];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    g[k] = p.gamma[lane * V + k];
    b[k] = p.beta[lane * V + k];
  }
  const float inv_c = 1.0f / (float)p.C;
  us2 am = {0, 0};
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int64_t r = r0 + i;
    float f[V];
    ln_unpack<V>(raw[i], f);
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) s += f[k];
    const float mu = wave_sum_f32(s) * inv_c;
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const float d = f[k] - mu;
      q += d * d;
    }
    const float rs = 1.0f / sqrtf(wave_sum_f32(q) * inv_c + p.eps);
#pragma unroll
    for (int k = 0; k < V; ++k) f[k] = (f[k] - mu) * rs * g[k] + b[k];
    if (r < p.rows) {
      ln_store<V>(static_cast<uint16_t*>(p.out) + r * p.C, lane, f, am);
      if (lane == 0) {
        p.mean[r] = mu;
        p.rstd[r] = rs;
      }
    }
  }
  if (p.amax_part) {  // the workgroup's max |y| for the consumer's current-scaling cast
    __shared__ uint32_t red[kLnWaves];
    uint32_t m = am.x > am.y ? am.x : am.y;
    m = wave_max_u32(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t b = red[0];
#pragma unroll
      for (int w = 1; w < kLnWaves; ++w) b = b > red[w] ? b : red[w];
      p.amax_part[blockIdx.x] = b;
    }
  }
}

template <int V, bool kF32>
__global__ __launch_bounds__(kLnThreads) void ln_bwd_kernel(const LnArgs p) {
  using XT = LnXT<kF32>;
  const XT* px = static_cast<const XT*>(p.x);
  constexpr int R = ln_rows<V>();
  __shared__ float red[kLnWaves][2][64 * V];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r0 = (int64_t)blockIdx.x * ln_rows_per_block<V>() + wave * R;
  LnXRaw<V, kF32> rx[R], ra[R];
  LnRaw<V> rd[R];
  float mus[R], rss[R];
  const XT* padd = static_cast<const XT*>(p.dx_add);
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int64_t r = r0 + i < p.rows ? r0 + i : p.rows - 1;
    ln_load<V>(px + r * p.C, lane, rx[i]);
    ln_load<V>(p.dout + r * p.C, lane, rd[i]);
    if (padd) ln_load<V>(padd + r * p.C, lane, ra[i]);
    mus[i] = p.mean[r];
    rss[i] = p.rstd[r];
  }
  float g[V], dg[V], db[V];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    g[k] = p.gamma[lane * V + k];
    dg[k] = 0.f;
    db[k] = 0.f;
  }
  const float inv_c = 1.0f / (float)p.C;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int64_t r = r0 + i;
    const bool live = r < p.rows;
    float f[V], d[V];
    ln_unpack<V>(rx[i], f);
    ln_unpack<V>(rd[i], d);
    const float mu = mus[i], rs = rss[i];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const float xh = (f[k] - mu) * rs;
      const float gx = d[k] * g[k];
      s1 += gx;
      s2 += gx * xh;
      if (live) {
        dg[k] += d[k] * xh;
        db[k] += d[k];
      }
      f[k] = xh;
      d[k] = gx;
    }
    const float m1 = wave_sum_f32(s1) * inv_c, m2 = wave_sum_f32(s2) * inv_c;
#pragma unroll
    for (int k = 0; k < V; ++k) f[k] = rs * (d[k] - m1 - f[k] * m2);
    if (padd) {
      // the skip path's gradient of the same tensor, added as autograd adds two gradients in
      // x's type: fp32 + fp32, or bf16(dx) + bf16 computed in fp32 and rounded once more
      float ad[V];
      ln_unpack<V>(ra[i], ad);
#pragma unroll
      for (int k = 0; k < V; ++k) {
        if (!kF32) f[k] = bf16_bits_to_f32(f32_to_bf16_bits(f[k]));
        f[k] = f[k] + ad[k];
      }
    }
    if (live) {
      us2 unused = {0, 0};
      ln_store<V>(static_cast<XT*>(p.out) + r * p.C, lane, f, unused);
    }
  }
  // this block's column sums: the waves in order
#pragma unroll
  for (int k = 0; k < V; ++k) {
    red[wave][0][lane * V + k] = dg[k];
    red[wave][1][lane * V + k] = db[k];
  }
  __syncthreads();
  float* out = p.part + (int64_t)blockIdx.x * 2 * p.C;
  for (int c = threadIdx.x; c < p.C; c += kLnThreads) {
    float a = red[0][0][c], bb = red[0][1][c];
#pragma unroll
    for (int w = 1; w < kLnWaves; ++w) {
      a += red[w][0][c];
      bb += red[w][1][c];
    }
    out[c] = a;
    out[p.C + c] = bb;
  }
}

// dgamma[c] = sum over blocks of part[b][0][c], dbeta from part[b][1][c]: 32 interleaved slices
// of blocks per column (8 loads in flight per thread), then the slices in order
// (deterministic). Block: 8 columns x 32 slices.
__global__ __launch_bounds__(kLnThreads) void ln_param_reduce_kernel(const float* __restrict__ part,
                                                                     int blocks, int C,
                                                                     float* __restrict__ dgamma,
                                                                     float* __restrict__ dbeta) {
  __shared__ float red[kLnRedSlices][8];
  const int cl = threadIdx.x & 7, sl = threadIdx.x >> 3;
  const int c = blockIdx.x * 8 + cl;  // 0 .. 2C-1 over [dgamma | dbeta]
  float s = 0.f;
  if (c < 2 * C) {
    const float* q = part + c;
#pragma unroll 8
    for (int b = sl; b < blocks; b += kLnRedSlices) s += q[(int64_t)b * 2 * C];
  }
  red[sl][cl] = s;
  __syncthreads();
  if (sl == 0 && c < 2 * C) {
    float t = red[0][cl];
    for (int k = 1; k < kLnRedSlices; ++k) t += red[k][cl];
    if (c < C) dgamma[c] = t;
    else dbeta[c - C] = t;
  }
}

static_assert(kLnThreads == 8 * kLnRedSlices, "reduce block: 8 columns x 32 slices");

template <int V>
static int ln_blocks_v(int64_t rows) { return (int)ceil_div(rows, (int64_t)ln_rows_per_block<V>()); }

static int ln_blocks(int64_t rows, int C) {
  switch (C / 64) {
    case 1: return ln_blocks_v<1>(rows);
    case 2: return ln_blocks_v<2>(rows);
    case 4: return ln_blocks_v<4>(rows);
    case 8: return ln_blocks_v<8>(rows);
    case 16: return ln_blocks_v<16>(rows);
    default: return 0;
  }
}

static bool ln_shape_ok(int64_t rows, int C) {
  const int v = C / 64;
  return rows > 0 && rows < ((int64_t)1 << 30) && C > 0 && C % 64 == 0 &&
         (v == 1 || v == 2 || v == 4 || v == 8 || v == 16);
}

template <template <int, bool> class Launch, bool kF32>
static int ln_dispatch_t(int C, hipStream_t s, const LnArgs& a, int blocks) {
  switch (C / 64) {
    case 1: Launch<1, kF32>::go(a, blocks, s); break;
    case 2: Launch<2, kF32>::go(a, blocks, s); break;
    case 4: Launch<4, kF32>::go(a, blocks, s); break;
    case 8: Launch<8, kF32>::go(a, blocks, s); break;
    case 16: Launch<16, kF32>::go(a, blocks, s); break;
    default: return DPA_ERR_SHAPE;
  }
  return launch_status();
}
template <template <int, bool> class Launch>
static int ln_dispatch(int C, hipStream_t s, const LnArgs& a, int blocks, bool f32 = false) {
  return f32 ? ln_dispatch_t<Launch, true>(C, s, a, blocks)
             : ln_dispatch_t<Launch, false>(C, s, a, blocks);
}

template <int V, bool kF32>
struct LnFwdLaunch {
  static void go(const LnArgs& a, int blocks, hipStream_t s) {
    ln_fwd_kernel<V, kF32><<<(unsigned)blocks, kLnThreads, 0, s>>>(a);
  }
};
template <int V, bool kF32>
struct LnBwdLaunch {
  static void go(const LnArgs& a, int blocks, hipStream_t s) {
    ln_bwd_kernel<V, kF32><<<(unsigned)blocks, kLnThreads, 0, s>>>(a);
  }
};

}  // namespace dpa

using namespace dpa;

static int ln_fwd(const void* x, bool f32, const float* gamma, const float* beta, void* out,
                  float* mean, float* rstd, int64_t rows, int C, float eps, void* stream,
                  uint32_t* amax_part = nullptr) {
  if (!x || !gamma || !beta || !out || !mean || !rstd) return DPA_ERR_NULL;
  if (!ln_shape_ok(rows, C)) return DPA_ERR_SHAPE;
  if (!aligned(x, 16) || !aligned(out, 16)) return DPA_ERR_ALIGN;
  LnArgs a{};
  a.x = x;
  a.gamma = gamma;
  a.beta = beta;
  a.out = out;
  a.mean = mean;
  a.rstd = rstd;
  a.rows = rows;
  a.C = C;
  a.eps = eps;
  a.amax_part = amax_part;
  return ln_dispatch<LnFwdLaunch>(C, (hipStream_t)stream, a, ln_blocks(rows, C), f32);
}

extern "C" int dpa_layernorm_fwd_bf16(const void* x, const float* gamma, const float* beta,
                                      void* out, float* mean, float* rstd, int64_t rows, int C,
                                      float eps, void* stream) {
  return ln_fwd(x, false, gamma, beta, out, mean, rstd, rows, C, eps, stream);
}

extern "C" int dpa_layernorm_fwd_ex(const void* x, int x_dtype, const float* gamma,
                                    const float* beta, void* out, float* mean, float* rstd,
                                    int64_t rows, int C, float eps, void* stream) {
  if (x_dtype != DPA_DTYPE_BF16 && x_dtype != DPA_DTYPE_F32) return DPA_ERR_SHAPE;
  return ln_fwd(x, x_dtype == DPA_DTYPE_F32, gamma, beta, out, mean, rstd, rows, C, eps, stream);
}

// The forward's workgroups, one amax partial each (0 for an unsupported shape).
extern "C" int dpa_layernorm_fwd_partials(int64_t rows, int C) {
  return ln_shape_ok(rows, C) ? ln_blocks(rows, C) : 0;
}

// dpa_layernorm_fwd_ex that also leaves the per-workgroup maxima of |out| (bf16 magnitude
// bits, dpa_layernorm_fwd_partials(rows, C) of them) in amax_partials, for the consumer's
// current-scaling cast (dpa_quantize_fp8_bf16_from_partials) in place of its amax pass.
extern "C" int dpa_layernorm_fwd_amax(const void* x, int x_dtype, const float* gamma,
                                      const float* beta, void* out, float* mean, float* rstd,
                                      int64_t rows, int C, float eps, void* amax_partials,
                                      void* stream) {
  if (x_dtype != DPA_DTYPE_BF16 && x_dtype != DPA_DTYPE_F32) return DPA_ERR_SHAPE;
  if (!amax_partials) return DPA_ERR_NULL;
  if (!aligned(amax_partials, 4)) return DPA_ERR_ALIGN;
  return ln_fwd(x, x_dtype == DPA_DTYPE_F32, gamma, beta, out, mean, rstd, rows, C, eps, stream,
                (uint32_t*)amax_partials);
}

extern "C" int64_t dpa_layernorm_bwd_workspace_bytes(int64_t rows, int C) {
  if (!ln_shape_ok(rows, C)) return 0;
  return (int64_t)ln_blocks(rows, C) * 2 * C * 4;
}

static int ln_bwd(const void* x, bool f32, const void* dout, const float* gamma,
                  const float* mean, const float* rstd, void* dx, float* dgamma, float* dbeta,
                  void* workspace, int64_t workspace_bytes, int64_t rows, int C, void* stream,
                  const void* dx_add = nullptr) {
  if (!x || !dout || !gamma || !mean || !rstd || !dx || !dgamma || !dbeta) return DPA_ERR_NULL;
  if (!ln_shape_ok(rows, C)) return DPA_ERR_SHAPE;
  if (!workspace || workspace_bytes < dpa_layernorm_bwd_workspace_bytes(rows, C))
    return DPA_ERR_WORKSPACE;
  if (!aligned(x, 16) || !aligned(dout, 16) || !aligned(dx, 16) || !aligned(workspace, 4) ||
      !aligned(dx_add, 16))
    return DPA_ERR_ALIGN;
  LnArgs a{};
  a.dx_add = dx_add;
  a.x = x;
  a.dout = (const uint16_t*)dout;
  a.gamma = gamma;
  a.out = dx;
  a.mean = const_cast<float*>(mean);
  a.rstd = const_cast<float*>(rstd);
  a.part = (float*)workspace;
  a.rows = rows;
  a.C = C;
  hipStream_t s = (hipStream_t)stream;
  const int blocks = ln_blocks(rows, C);
  int st = ln_dispatch<LnBwdLaunch>(C, s, a, blocks, f32);
  if (st != DPA_OK) return st;
  ln_param_reduce_kernel<<<(unsigned)ceil_div(2 * C, 8), kLnThreads, 0, s>>>(
      (const float*)workspace, blocks, C, dgamma, dbeta);
  return launch_status();
}

extern "C" int dpa_layernorm_bwd_bf16(const void* x, const void* dout, const float* gamma,
                                      const float* mean, const float* rstd, void* dx,
                                      float* dgamma, float* dbeta, void* workspace,
                                      int64_t workspace_bytes, int64_t rows, int C,
                                      void* stream) {
  return ln_bwd(x, false, dout, gamma, mean, rstd, dx, dgamma, dbeta, workspace,
                workspace_bytes, rows, C, stream);
}

extern "C" int dpa_layernorm_bwd_ex(const void* x, int x_dtype, const void* dout,
                                    const float* gamma, const float* mean, const float* rstd,
                                    void* dx, float* dgamma, float* dbeta, void* workspace,
                                    int64_t workspace_bytes, int64_t rows, int C, void* stream) {
  if (x_dtype != DPA_DTYPE_BF16 && x_dtype != DPA_DTYPE_F32) return DPA_ERR_SHAPE;
  return ln_bwd(x, x_dtype == DPA_DTYPE_F32, dout, gamma, mean, rstd, dx, dgamma, dbeta,
                workspace, workspace_bytes, rows, C, stream);
}

extern "C" int dpa_layernorm_bwd_ex_add(const void* x, int x_dtype, const void* dout,
                                        const float* gamma, const float* mean,
                                        const float* rstd, const void* dx_add, void* dx,
                                        float* dgamma, float* dbeta, void* workspace,
                                        int64_t workspace_bytes, int64_t rows, int C,
                                        void* stream) {
  if (x_dtype != DPA_DTYPE_BF16 && x_dtype != DPA_DTYPE_F32) return DPA_ERR_SHAPE;
  if (!dx_add) return DPA_ERR_NULL;
  return ln_bwd(x, x_dtype == DPA_DTYPE_F32, dout, gamma, mean, rstd, dx, dgamma, dbeta,
                workspace, workspace_bytes, rows, C, stream, dx_add);
}
