// Fused GroupNorm (+FiLM) + SiLU, forward and backward, NHWC bf16 with fp32 statistics.
//
// Reference sites (diffusion/unet.py): F.silu(self.norm1(x)) at :151 and
// self.dropout(F.silu((w + 1) * self.norm2(x) + b)) at :157-159, with nn.GroupNorm(32, C)
// (:132-133, eps 1e-5, affine). Under autocast GroupNorm runs in fp32; the FP8 conv then
// rounds its input to bf16 (diffusion/fp8_kernels.py:835), which is what `out` stores.
//
// Layout: one workgroup per (image n, 64-channel slab): PLN pixel lanes (32, 64 or 128 by
// image size) x 8 granules of 8 channels (16 B of bf16). Every group of the slab lies inside
// the slab (64 % (C/G) == 0), so the statistics reduce inside the workgroup: 4-channel
// half-granule partials -> wave shuffles over the 8 pixel lanes of a wave -> LDS over the
// waves. Each lane keeps four 16-B loads in flight. The kernels make several passes over
// their inputs (after the first mostly from L2).
//
// Images of 256+ pixels use a chunked form instead, which spreads each (image, slab) over
// workgroups of 128 pixels (2048 workgroups at 32x32 x 128 channels, batch 128, against 256
// for one workgroup per slab, whose passes were latency-bound): every workgroup holds its
// chunk in registers, and the per-group statistics cross workgroups through a workspace
// between two launches.
//   forward:  stats (chunk mean and sum of squared deviations per group) ->
//             apply (merge the chunks in order, Chan et al.'s pairwise update; normalise)
//   backward: sums (per-channel chunk sums of the four backward terms) ->
//             apply (chunk sums in order -> group means -> dx; chunk 0 also writes the
//             per-image dgamma/dbeta partials and the FiLM gradients)
#include "dpa_common.hpp"

namespace dpa {

constexpr int kSlab = 64;  // channels per workgroup
constexpr int kGnUnrollFwd = 4;  // pixels per lane per loop iteration (loads in flight)
constexpr int kGnUnrollBwd = 2;  // (two sources per pixel)

struct GnArgs {
  const void* x;  // [N][HW][C] bf16, or fp32 for the chunked and small-image forms
  const uint16_t* dout;
  const float* gamma;
  const float* beta;
  const float* fs;  // film scale [N][C] or null
  const float* fb;  // film shift [N][C]
  void* out;  // forward: bf16 output; backward: dx in x's type
  float* mean;
  float* rstd;
  float* part;  // bwd: [2][N][C] per-image channel sums of dgamma / dbeta
  float* dfs;   // bwd: FiLM gradients [N][C] or null
  float* dfb;
  const uint16_t* wb;  // or FiLM from the bf16 time projection [N][2C]: scale bf16(w + 1), shift b
  uint16_t* dwb;       // bwd: its gradient [N][2C] bf16, or null
  const uint64_t* drop_seed;  // dropout after the SiLU: seed in device memory, or null
  uint32_t drop_keep;         // keep an element when its 16-bit hash is >= this (p * 2^16)
  float drop_scale;           // RN32(1 / (1 - p))
  const void* dx_add;  // bwd: a gradient added to dx (chunked and small forms), or null
  int dx_add_bf16;     // bwd: dx_add is bf16 while x and dx are fp32
  uint16_t* x_bf16;    // fwd: fp32 x also written as bf16 here (chunked and small forms), or null
  uint32_t* xb_part;   // fwd: with x_bf16, one amax partial of its bf16 values per workgroup
  // Two-source x (a decoder stage's first GroupNorm with the upsample-and-concatenate before
  // it, diffusion/unet.py:379-382): channels [0, cat_ca) are the 2x nearest upsampling of
  // cat_a ([N][H/2][W/2][cat_ca], bf16), the others cat_h ([N][H][W][C - cat_ca], bf16 or
  // fp32); the concatenation they replace is fp32 and holds exactly these values. Images of
  // cat_w columns.
  const uint16_t* cat_a;
  const uint16_t* cat_h;
  int cat_ca, cat_w;
  int cat_hf;        // cat_h (and its gradient) fp32 instead of bf16 (forms with an fp32 x)
  uint16_t* cat_ga;  // bwd: gradient of cat_a (each 2x2 window of dx summed), bf16
  void* cat_gh;      // bwd: gradient of cat_h, in cat_h's type
  // Producer-fused cast for a delayed-scaling consumer (chunked and small forms): instead of
  // the bf16 output (fwd) or bf16 dx (bwd), e4m3(bf16 value / *q_scale) goes to q, and each
  // workgroup leaves the amax of its bf16 values in q_part[workgroup] (count in *q_count)
  uint8_t* q;
  const float* q_scale;
  uint32_t* q_part;
  uint32_t* q_count;
  int N, HW, C, G, cpg;
  float eps;
};

// Dropout of the GroupNorm+SiLU output (diffusion/unet.py:160, nn.Dropout before conv_2): the
// keep decision of element idx (NHWC index) is a counter hash of (seed, idx), so the backward
// recomputes the mask instead of storing it; kept values are scaled by 1 / (1 - p) in fp32
// before the bf16 rounding, as the reference drops its fp32 SiLU output before the conv's
// bf16 cast. The hash: splitmix64 of seed + (idx / 4) * golden ratio, one output per four
// elements: element idx is kept when bits [16 (idx % 4), 16 (idx % 4) + 16) of its hash, as
// a 16-bit number, are >= floor(p * 2^16). Four elements per 64-bit hash halve the hash's vector
// instructions against one per pair (its multiplies are done in 32-bit halves); 16 bits
// still give a drop rate within 2^-16 of p.
// Returns the keep bits of the 8 elements idx0 .. idx0 + 7 (idx0 a multiple of 8).
__device__ __forceinline__ uint32_t drop_keep8(uint64_t seed, int64_t idx0, uint32_t keep_from) {
  constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;
  const uint64_t z0 = seed + (uint64_t)(idx0 >> 2) * kGolden;
  uint32_t bits = 0;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    uint64_t z = z0 + (uint64_t)i * kGolden;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t r = (uint32_t)(z >> (16 * j)) & 0xffffu;
      bits |= (uint32_t)(r >= keep_from) << (4 * i + j);
    }
  }
  return bits;
}

// v * scale if bit e of the keep bits is set, else +0: the selection as a mask of the bit
// (v_bfe_i32 gives 0 or all ones) and'ed into the product, so no per-element lane mask is
// formed (in the backward, which keeps each pixel's keep bits for both passes, those masks
// took 2 scalar registers per element and were spilled to vector lanes: ~700 v_readlane /
// v_writelane per thread in the 1024-pixel form)
__device__ __forceinline__ float drop_sel(float v, uint32_t keep, int e, float scale) {
  uint32_t m;
  // (as an instruction of its own: the compiler would turn the and back into a select)
  asm("v_bfe_i32 %0, %1, %2, 1" : "=v"(m) : "v"(keep), "i"(e));
  return __uint_as_float(__float_as_uint(v * scale) & m);
}

// sigmoid(v) = 1 / (1 + e^-v) from the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32,
// about 1 ulp each), e^-v = 2^(-v log2 e). The SiLU and its derivative are rounded to bf16
// (2^16 fp32 ulps), so this changes an output bit only at rounding ties; the IEEE-exact
// exponential and division cost about a third of the forward kernels' time. Saturates as the
// exact form does: e^-v overflows to inf below v = -88.7 and the result is 0.
__device__ __forceinline__ float sigmoid_hw(float v) {
  const float e = __builtin_amdgcn_exp2f(v * -1.44269504f);
  return __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ void unpack8(uint4 v, float (&f)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

// Sum v over the PLN pixel lanes that share this thread's granule (8 per wave by shuffles,
// then the waves in order through LDS); result valid in every lane. red holds
// (PLN / 8) waves x 8 granules x NV floats.
template <int NV, int PLN>
__device__ __forceinline__ void slab_reduce(float (&v)[NV], float* red) {
  constexpr int kWaves = PLN / 8;
  const int gq = threadIdx.x & 7;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    float s = v[k];
    s += __shfl_xor(s, 8, 64);
    s += __shfl_xor(s, 16, 64);
    s += __shfl_xor(s, 32, 64);
    v[k] = s;
  }
  if ((threadIdx.x & 63) < 8) {
#pragma unroll
    for (int k = 0; k < NV; ++k) red[(wave * 8 + gq) * NV + k] = v[k];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < NV; ++k) v[k] = red[gq * NV + k];
#pragma unroll 1
  for (int w = 1; w < kWaves; ++w) {
#pragma unroll
    for (int k = 0; k < NV; ++k) v[k] += red[(w * 8 + gq) * NV + k];
  }
  __syncthreads();
}

// Per-group value from half-granule (4-channel) sums hs[16] of the slab: group of this
// thread's channel half h (0/1) = consecutive cpg/4 half-granules.
__device__ __forceinline__ float group_sum(const float* hs, int half_idx, int cpg) {
  const int hpg = cpg / 4;  // half-granules per group (1, 2, 4, ... 16)
  const int g0 = (half_idx / hpg) * hpg;
  float s = 0.f;
  for (int i = 0; i < hpg; ++i) s += hs[g0 + i];
  return s;
}

// 8 consecutive floats (two 16-B loads when the address allows, as it does for torch's tensors)
__device__ __forceinline__ void load8f(const float* src, float (&v)[8]) {
  if ((reinterpret_cast<uintptr_t>(src) & 15) == 0) {
    const float4 a = reinterpret_cast<const float4*>(src)[0];
    const float4 b = reinterpret_cast<const float4*>(src)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = src[e];
  }
}

// FiLM scale/shift of channels ch..ch+7 of image n: fp32 [N][C] pairs, or the bf16 time
// projection [N][2C] with scale bf16(w + 1) (the reference adds 1 in bf16) and shift b; no FiLM
// gives 1 and 0.
__device__ __forceinline__ bool load_film(const GnArgs& p, int n, int ch, float (&fsc)[8],
                                          float (&fsh)[8]) {
  if (p.fs) {
    load8f(p.fs + (int64_t)n * p.C + ch, fsc);
    load8f(p.fb + (int64_t)n * p.C + ch, fsh);
    return true;
  }
  if (p.wb) {
    const uint16_t* w = p.wb + (int64_t)n * 2 * p.C + ch;
    float wf[8];
    if ((reinterpret_cast<uintptr_t>(w) & 15) == 0) {  // (uniform: base alignment)
      unpack8(*reinterpret_cast<const uint4*>(w), wf);
      unpack8(*reinterpret_cast<const uint4*>(w + p.C), fsh);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        wf[e] = bf16_bits_to_f32(w[e]);
        fsh[e] = bf16_bits_to_f32(w[p.C + e]);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const uint32_t pk = pack_bf16x2(wf[e] + 1.0f, wf[e + 1] + 1.0f);
      fsc[e] = __uint_as_float(pk << 16);
      fsc[e + 1] = __uint_as_float(pk & 0xffff0000u);
    }
    return true;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    fsc[e] = 1.0f;
    fsh[e] = 0.0f;
  }
  return false;
}

// Pixel loop of a pass: lane pl visits pixels pl, pl + PLN, ... in groups of U whose 16-B
// loads (from each of the NL sources) are all issued before any is used; pixels past HW load
// pixel HW - 1 (a valid address) and reach body(px, ok, v0, v1) with ok false.
template <int PLN, int NL, int U, typename F>
__device__ __forceinline__ void gn_pixels(const uint16_t* const (&src)[NL], int C, int pl, int HW,
                                          F body) {
  for (int px0 = pl; px0 < HW; px0 += U * PLN) {
    int pxs[U];
    bool oks[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int px = px0 + u * PLN;
      oks[u] = px < HW;
      pxs[u] = oks[u] ? px : HW - 1;
    }
    uint4 v[NL][U];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int l = 0; l < NL; ++l)
        v[l][u] = *reinterpret_cast<const uint4*>(src[l] + (int64_t)pxs[u] * C);
#pragma unroll
    for (int u = 0; u < U; ++u) body(pxs[u], oks[u], v[0][u], v[NL - 1][u]);
  }
}

// Layout: one workgroup per (image n, 64-channel slab): 8 x PLN threads = PLN pixel lanes x
// 8 granules of 8 channels (16 B of bf16).
template <int PLN>
__global__ __launch_bounds__(8 * PLN) void gn_silu_fwd_kernel(const GnArgs p) {
  __shared__ float red[(PLN / 8) * 8 * 2];
  __shared__ float hs[16];
  const int n = blockIdx.y;
  const int c0 = blockIdx.x * kSlab;
  const int gq = threadIdx.x & 7;
  const int pl = threadIdx.x >> 3;
  const int ch = c0 + gq * 8;
  const int HW = p.HW;
  const uint16_t* xb = static_cast<const uint16_t*>(p.x) + (int64_t)n * HW * p.C + ch;

  // pass 1: mean
  float s[2] = {0.f, 0.f};
  const uint16_t* const xsrc[1] = {xb};
  gn_pixels<PLN, 1, kGnUnrollFwd>(xsrc, p.C, pl, HW, [&](int, bool ok, uint4 xv, uint4) {
    float f[8];
    unpack8(xv, f);
    if (ok) {
      s[0] += (f[0] + f[1]) + (f[2] + f[3]);
      s[1] += (f[4] + f[5]) + (f[6] + f[7]);
    }
  });
  slab_reduce<2, PLN>(s, red);
  if ((threadIdx.x >> 3) == 0) {
    hs[2 * gq] = s[0];
    hs[2 * gq + 1] = s[1];
  }
  __syncthreads();
  const float inv_cnt = 1.0f / (float)((int64_t)HW * p.cpg);
  const float mu[2] = {group_sum(hs, 2 * gq, p.cpg) * inv_cnt,
                       group_sum(hs, 2 * gq + 1, p.cpg) * inv_cnt};
  __syncthreads();

  // pass 2: biased variance around the mean
  float q[2] = {0.f, 0.f};
  gn_pixels<PLN, 1, kGnUnrollFwd>(xsrc, p.C, pl, HW, [&](int, bool ok, uint4 xv, uint4) {
    float f[8];
    unpack8(xv, f);
    if (ok) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = f[e] - mu[e >> 2];
        q[e >> 2] += d * d;
      }
    }
  });
  slab_reduce<2, PLN>(q, red);
  if ((threadIdx.x >> 3) == 0) {
    hs[2 * gq] = q[0];
    hs[2 * gq + 1] = q[1];
  }
  __syncthreads();
  float rs[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float var = group_sum(hs, 2 * gq + h, p.cpg) * inv_cnt;
    rs[h] = 1.0f / sqrtf(var + p.eps);
  }
  // statistics out: one writer per group
  if (pl == 0) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int cc = ch + 4 * h;
      if (cc % p.cpg == 0) {
        const int g = cc / p.cpg;
        p.mean[n * p.G + g] = mu[h];
        p.rstd[n * p.G + g] = rs[h];
      }
    }
  }

  // pass 3: normalise, affine, FiLM, SiLU, bf16
  float a[8], b[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = p.gamma[ch + e];
    b[e] = p.beta[ch + e];
  }
  float fsc[8], fsh[8];
  const bool film = load_film(p, n, ch, fsc, fsh);
  uint16_t* ob = static_cast<uint16_t*>(p.out) + (int64_t)n * HW * p.C + ch;
  gn_pixels<PLN, 1, kGnUnrollFwd>(xsrc, p.C, pl, HW, [&](int px, bool ok, uint4 xv, uint4) {
    float f[8];
    unpack8(xv, f);
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      float z[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int ee = e + k;
        float v = (f[ee] - mu[ee >> 2]) * rs[ee >> 2] * a[ee] + b[ee];
        if (film) v = fsc[ee] * v + fsh[ee];
        z[k] = v * sigmoid_hw(v);
      }
      o[e >> 1] = f32_to_bf16_bits(z[0]) | (f32_to_bf16_bits(z[1]) << 16);
    }
    if (ok) st_nt16(ob + (int64_t)px * p.C, uint4{o[0], o[1], o[2], o[3]});
  });
}

// Backward. With zp = film? fs*z + fb : z (z = GN output), u = silu(zp):
//   g   = dout * sig(zp) * (1 + zp * (1 - sig(zp)))        (d u / d zp)
//   dfs = sum_hw g * z,  dfb = sum_hw g;   gz = film? g * fs : g
//   dgamma += sum gz * xhat, dbeta += sum gz;   gxh = gz * gamma
//   dx = rstd * (gxh - mean_grp(gxh) - xhat * mean_grp(gxh * xhat))
template <int PLN>
__global__ __launch_bounds__(8 * PLN) void gn_silu_bwd_kernel(const GnArgs p) {
  __shared__ float red[(PLN / 8) * 8 * 32];
  __shared__ float hs[2][16];
  const int n = blockIdx.y;
  const int c0 = blockIdx.x * kSlab;
  const int gq = threadIdx.x & 7;
  const int pl = threadIdx.x >> 3;
  const int ch = c0 + gq * 8;
  const int HW = p.HW;
  const int64_t base = (int64_t)n * HW * p.C + ch;

  float mu[2], rs[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int g = (ch + 4 * h) / p.cpg;
    mu[h] = p.mean[n * p.G + g];
    rs[h] = p.rstd[n * p.G + g];
  }
  float gm[8], bt[8], fsc[8], fsh[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    gm[e] = p.gamma[ch + e];
    bt[e] = p.beta[ch + e];
  }
  load_film(p, n, ch, fsc, fsh);

  // pass 1: per-channel sums of gz, gz*xhat, g*z, g
  float acc[4][8];
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[k][e] = 0.f;
  const uint16_t* const srcs[2] = {static_cast<const uint16_t*>(p.x) + base, p.dout + base};
  gn_pixels<PLN, 2, kGnUnrollBwd>(srcs, p.C, pl, HW, [&](int, bool ok, uint4 xv, uint4 dv) {
    float f[8], d[8];
    unpack8(xv, f);
    unpack8(dv, d);
    if (ok) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xh = (f[e] - mu[e >> 2]) * rs[e >> 2];
        const float z = xh * gm[e] + bt[e];
        const float zp = fsc[e] * z + fsh[e];
        const float sg = sigmoid_hw(zp);
        const float g = d[e] * (sg * (1.0f + zp * (1.0f - sg)));
        const float gz = g * fsc[e];
        acc[0][e] += gz;
        acc[1][e] += gz * xh;
        acc[2][e] += g * z;
        acc[3][e] += g;
      }
    }
  });
  // reduce the 32 per-channel sums over pixel lanes
  {
    float* v = &acc[0][0];
    float tmp[32];
#pragma unroll
    for (int k = 0; k < 32; ++k) tmp[k] = v[k];
    slab_reduce<32, PLN>(tmp, red);
#pragma unroll
    for (int k = 0; k < 32; ++k) v[k] = tmp[k];
  }
  // per-image channel partials for dgamma/dbeta and the FiLM gradients
  if (pl == 0) {
    const int64_t nc = (int64_t)p.N * p.C;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t o = (int64_t)n * p.C + ch + e;
      p.part[0 * nc + o] = acc[1][e];  // dgamma partial
      p.part[1 * nc + o] = acc[0][e];  // dbeta partial
      if (p.dfs) {                      // FiLM gradients are per image: final here
        p.dfs[o] = acc[2][e];
        p.dfb[o] = acc[3][e];
      } else if (p.dwb) {
        const int64_t ob = (int64_t)n * 2 * p.C + ch + e;
        p.dwb[ob] = (uint16_t)f32_to_bf16_bits(acc[2][e]);
        p.dwb[ob + p.C] = (uint16_t)f32_to_bf16_bits(acc[3][e]);
      }
    }
    // group sums of gxh = gz*gamma and gxh*xhat, per 4-channel half
    float h1[2] = {0.f, 0.f}, h2[2] = {0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      h1[e >> 2] += acc[0][e] * gm[e];
      h2[e >> 2] += acc[1][e] * gm[e];
    }
    hs[0][2 * gq] = h1[0];
    hs[0][2 * gq + 1] = h1[1];
    hs[1][2 * gq] = h2[0];
    hs[1][2 * gq + 1] = h2[1];
  }
  __syncthreads();
  const float inv_cnt = 1.0f / (float)((int64_t)HW * p.cpg);
  float m1[2], m2[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    m1[h] = group_sum(hs[0], 2 * gq + h, p.cpg) * inv_cnt;
    m2[h] = group_sum(hs[1], 2 * gq + h, p.cpg) * inv_cnt;
  }

  // pass 2: dx
  gn_pixels<PLN, 2, kGnUnrollBwd>(srcs, p.C, pl, HW, [&](int px, bool ok, uint4 xv, uint4 dv) {
    float f[8], d[8];
    unpack8(xv, f);
    unpack8(dv, d);
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      float r2[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int ee = e + k;
        const int h = ee >> 2;
        const float xh = (f[ee] - mu[h]) * rs[h];
        const float z = xh * gm[ee] + bt[ee];
        const float zp = fsc[ee] * z + fsh[ee];
        const float sg = sigmoid_hw(zp);
        const float g = d[ee] * (sg * (1.0f + zp * (1.0f - sg)));
        const float gxh = g * fsc[ee] * gm[ee];
        r2[k] = rs[h] * (gxh - m1[h] - xh * m2[h]);
      }
      o[e >> 1] = f32_to_bf16_bits(r2[0]) | (f32_to_bf16_bits(r2[1]) << 16);
    }
    if (ok) st_nt16(static_cast<uint16_t*>(p.out) + base + (int64_t)px * p.C, uint4{o[0], o[1], o[2], o[3]});
  });
}

// dgamma[c] = sum_n part[0][n][c], dbeta[c] = sum_n part[1][n][c]: 16 interleaved image
// slices (slice s sums images s, s + 16, ... in order, all its loads in flight at once), then
// a fixed pairwise tree over the slices (deterministic). One workgroup per 64 channels:
// 64 channel lanes x 16 image slices.
constexpr int kPrSlices = 16;
__global__ __launch_bounds__(64 * kPrSlices) void gn_param_reduce_kernel(
    const float* __restrict__ part, float* __restrict__ dgamma, float* __restrict__ dbeta, int N,
    int C) {
  __shared__ float red[2][kPrSlices][64];
  const int lane = threadIdx.x & 63;
  const int slice = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  const int64_t nc = (int64_t)N * C;
  float sg = 0.f, sb = 0.f;
  if (c < C) {
#pragma unroll 8
    for (int n = slice; n < N; n += kPrSlices) {
      sg += part[(int64_t)n * C + c];
      sb += part[nc + (int64_t)n * C + c];
    }
  }
  red[0][slice][lane] = sg;
  red[1][slice][lane] = sb;
  __syncthreads();
  if (slice < 2 && c < C) {
    float v[kPrSlices];
#pragma unroll
    for (int i = 0; i < kPrSlices; ++i) v[i] = red[slice][i][lane];
#pragma unroll
    for (int w = kPrSlices / 2; w >= 1; w /= 2)
#pragma unroll
      for (int i = 0; i < w; ++i) v[i] = v[i] + v[i + w];
    (slice == 0 ? dgamma : dbeta)[c] = v[0];
  }
}

// ---- chunked form (HW >= kChunkMinHW) ----
constexpr int kChPLN = 32;                 // pixel lanes per workgroup (256 threads)
constexpr int kChU = 4;                    // pixels per lane, all loads in flight
constexpr int kChunkPx = kChPLN * kChU;    // 128 pixels per workgroup
constexpr int kChunkMinHW = 256;
constexpr int kMaxChunks = 64;             // larger images run the one-launch form
static_assert(8 * kChPLN == 4 * kSlab, "backward apply: four chunk slices of 64 channels");

// Lane pl's pixels of the chunk starting at px0: px0 + pl + 32 u; pixels past HW load pixel
// HW - 1 (a valid address) with ok false.
template <int NL>
__device__ __forceinline__ void chunk_load(const uint8_t* const (&src)[NL],
                                           const int (&stride)[NL], int px0, int pl, int HW,
                                           uint4 (&v)[NL][kChU], bool (&ok)[kChU],
                                           int (&pxs)[kChU]) {
#pragma unroll
  for (int u = 0; u < kChU; ++u) {
    const int px = px0 + pl + u * kChPLN;
    ok[u] = px < HW;
    pxs[u] = ok[u] ? px : HW - 1;
  }
#pragma unroll
  for (int u = 0; u < kChU; ++u)
#pragma unroll
    for (int l = 0; l < NL; ++l)
      v[l][u] = *reinterpret_cast<const uint4*>(src[l] + (int64_t)pxs[u] * stride[l]);
}

// Sources of the chunk loop: the 8 channels of x at element offset off (one 16-B part in
// bf16, two in fp32), then, with kDout, the bf16 gradient of the output.
template <bool kF32, bool kDout>
struct GnSrc {
  static constexpr int kX = kF32 ? 2 : 1;
  static constexpr int kN = kX + (kDout ? 1 : 0);
  const uint8_t* src[kN];
  int stride[kN];  // bytes per pixel
  __device__ __forceinline__ GnSrc(const GnArgs& p, int64_t off) {
    constexpr int eb = kF32 ? 4 : 2;
    const uint8_t* xp = static_cast<const uint8_t*>(p.x) + off * eb;
#pragma unroll
    for (int k = 0; k < kX; ++k) {
      src[k] = xp + 16 * k;
      stride[k] = p.C * eb;
    }
    if (kDout) {
      src[kN - 1] = reinterpret_cast<const uint8_t*>(p.dout + off);
      stride[kN - 1] = p.C * 2;
    }
  }
};

// x of pixel u from the loaded parts
template <bool kF32, int NL, int U>
__device__ __forceinline__ void unpack_x(const uint4 (&v)[NL][U], int u, float (&f)[8]) {
  if constexpr (kF32) {
    const uint4 a = v[0][u], b = v[1][u];
    f[0] = __uint_as_float(a.x);
    f[1] = __uint_as_float(a.y);
    f[2] = __uint_as_float(a.z);
    f[3] = __uint_as_float(a.w);
    f[4] = __uint_as_float(b.x);
    f[5] = __uint_as_float(b.y);
    f[6] = __uint_as_float(b.z);
    f[7] = __uint_as_float(b.w);
  } else {
    unpack8(v[0][u], f);
  }
}

// The producer-fused cast in one thread (GnArgs::q): the window scale, its reciprocal for the
// fast quotient, and the running amax of the bf16 values cast.
struct GnQ {
  float s = 1.0f, r = 0.0f;
  us2 acc = {0, 0};
  __device__ __forceinline__ explicit GnQ(const GnArgs& p) {
    if (p.q) {
      s = *p.q_scale;
      r = quant_recip(s);
    }
  }
  // the 8 bf16 values v of element offset off
  __device__ __forceinline__ void put(const GnArgs& p, int64_t off, uint4 v) {
    st_nt8(p.q + off, quant8_delayed(v, s, r));
    acc = absmax8(acc, v);
  }
  // the workgroup's amax partial (every thread; red: one u32 per wave)
  __device__ __forceinline__ void finish(const GnArgs& p, uint32_t* red) const {
    const uint32_t blk = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
    store_amax_partial(acc, red, p.q_part, p.q_count, blk, gridDim.x * gridDim.y * gridDim.z);
  }
};

// dx of 8 channels at element offset off, in x's type; dx(e) gives channel e's value
template <bool kF32, typename F>
__device__ __forceinline__ void store_dx(const GnArgs& p, int64_t off, F dx, GnQ& qo) {
  // with dx_add: dx + add as torch's gradient accumulation forms it (one fp32 add; in bf16 the
  // sum of the two bf16 gradients, rounded once more)
  const bool add = p.dx_add != nullptr;
  if constexpr (kF32) {
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = dx(e);
    if (add && p.dx_add_bf16) {
      float a[8];
      unpack8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.dx_add) + off), a);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] += a[e];
    } else if (add) {
      const float* a = static_cast<const float*>(p.dx_add) + off;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint4 w = *reinterpret_cast<const uint4*>(a + 4 * h);
        v[4 * h] += __uint_as_float(w.x);
        v[4 * h + 1] += __uint_as_float(w.y);
        v[4 * h + 2] += __uint_as_float(w.z);
        v[4 * h + 3] += __uint_as_float(w.w);
      }
    }
    float* d = static_cast<float*>(p.out) + off;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      st_nt16(d + 4 * h, uint4{__float_as_uint(v[4 * h]), __float_as_uint(v[4 * h + 1]),
                               __float_as_uint(v[4 * h + 2]), __float_as_uint(v[4 * h + 3])});
  } else {
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = dx(e);
    if (add) {
      float a[8];
      unpack8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.dx_add) + off), a);
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const uint32_t w = pack_bf16x2(v[e], v[e + 1]);
        v[e] = __uint_as_float(w << 16) + a[e];
        v[e + 1] = __uint_as_float(w & 0xffff0000u) + a[e + 1];
      }
    }
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) o[e >> 1] = pack_bf16x2(v[e], v[e + 1]);
    if (p.q)
      qo.put(p, off, uint4{o[0], o[1], o[2], o[3]});
    else
      st_nt16(static_cast<uint16_t*>(p.out) + off, uint4{o[0], o[1], o[2], o[3]});
  }
}

// fp32 x also stored rounded to bf16 (RNE), for a consumer that rounds it anyway (the residual
// block's 1x1 skip conv), so no separate cast pass reads x again
__device__ __forceinline__ uint4 store_x_bf16(const GnArgs& p, int64_t off, const float (&f)[8]) {
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 8; e += 2) o[e >> 1] = pack_bf16x2(f[e], f[e + 1]);
  const uint4 w = uint4{o[0], o[1], o[2], o[3]};
  st_nt16(p.x_bf16 + off, w);
  return w;
}

// The workgroup's amax partial of the bf16 copy of x (every thread; red: one u32 per wave), for
// the current-scaling FP8 conv that quantizes that copy next
__device__ __forceinline__ void finish_xb_amax(const GnArgs& p, us2 acc, uint32_t* red) {
  const uint32_t blk = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
  store_amax_partial(acc, red, p.xb_part, nullptr, blk, gridDim.x * gridDim.y * gridDim.z);
}

// The forward's per-channel affine of this thread's 8 channels: out = silu(x A + B) with
// A = rstd gamma and B = beta - mean A, both times the FiLM scale (plus its shift in B) --
// normalise, affine and FiLM in one fma per element.
template <bool kFilm>
__device__ __forceinline__ void fwd_affine(const GnArgs& p, int n, int ch, const float (&mu)[2],
                                           const float (&rs)[2], float (&A)[8], float (&B)[8]) {
  float fsc[8], fsh[8], gm[8], bt[8];
  if (kFilm) load_film(p, n, ch, fsc, fsh);
  load8f(p.gamma + ch, gm);
  load8f(p.beta + ch, bt);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float a = rs[e >> 2] * gm[e];
    const float b = __builtin_fmaf(-mu[e >> 2], a, bt[e]);
    A[e] = kFilm ? fsc[e] * a : a;
    B[e] = kFilm ? __builtin_fmaf(fsc[e], b, fsh[e]) : b;
  }
}

// 8 outputs silu(f A + B) (dropout: kept ones times drop_scale, the rest 0), packed bf16
template <bool kDrop>
__device__ __forceinline__ uint4 fwd_out8(const float (&f)[8], const float (&A)[8],
                                          const float (&B)[8], uint32_t keep, float drop_scale) {
  float z[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float t = __builtin_fmaf(f[e], A[e], B[e]);
    float o = t * sigmoid_hw(t);
    if (kDrop) o = (keep >> e) & 1u ? o * drop_scale : 0.0f;
    z[e] = o;
  }
  return uint4{pack_bf16x2(z[0], z[1]), pack_bf16x2(z[2], z[3]), pack_bf16x2(z[4], z[5]),
               pack_bf16x2(z[6], z[7])};
}

__device__ __forceinline__ int chunk_pixels(int HW, int chunk) {
  const int r = HW - chunk * kChunkPx;
  return r < kChunkPx ? r : kChunkPx;
}

// Forward, launch 1: grid (C / 64, N, chunks). cs[n][chunk][g] = (chunk mean, chunk sum of
// squared deviations from it) of group g.
template <bool kF32>
__global__ __launch_bounds__(8 * kChPLN) void gn_chunk_stats_kernel(const GnArgs p,
                                                                   float2* __restrict__ cs,
                                                                   int nchunk) {
  __shared__ float red[(kChPLN / 8) * 8 * 2];
  __shared__ float hs[16];
  const int n = blockIdx.y, chunk = blockIdx.z;
  const int c0 = blockIdx.x * kSlab;
  const int gq = threadIdx.x & 7;
  const int pl = threadIdx.x >> 3;
  const int ch = c0 + gq * 8;
  const GnSrc<kF32, false> in(p, (int64_t)n * p.HW * p.C + ch);
  uint4 v[in.kN][kChU];
  bool ok[kChU];
  int pxs[kChU];
  chunk_load(in.src, in.stride, chunk * kChunkPx, pl, p.HW, v, ok, pxs);
  float f[kChU][8];
#pragma unroll
  for (int u = 0; u < kChU; ++u) unpack_x<kF32>(v, u, f[u]);

  float sm[2] = {0.f, 0.f};
#pragma unroll
  for (int u = 0; u < kChU; ++u)
    if (ok[u]) {
      sm[0] += (f[u][0] + f[u][1]) + (f[u][2] + f[u][3]);
      sm[1] += (f[u][4] + f[u][5]) + (f[u][6] + f[u][7]);
    }
  slab_reduce<2, kChPLN>(sm, red);
  if (pl == 0) {
    hs[2 * gq] = sm[0];
    hs[2 * gq + 1] = sm[1];
  }
  __syncthreads();
  const float inv_cnt = 1.0f / (float)(chunk_pixels(p.HW, chunk) * p.cpg);
  const float mu[2] = {group_sum(hs, 2 * gq, p.cpg) * inv_cnt,
                       group_sum(hs, 2 * gq + 1, p.cpg) * inv_cnt};
  __syncthreads();
  float q[2] = {0.f, 0.f};
#pragma unroll
  for (int u = 0; u < kChU; ++u)
    if (ok[u]) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = f[u][e] - mu[e >> 2];
        q[e >> 2] += d * d;
      }
    }
  slab_reduce<2, kChPLN>(q, red);
  if (pl == 0) {
    hs[2 * gq] = q[0];
    hs[2 * gq + 1] = q[1];
  }
  __syncthreads();
  if (pl == 0) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int cc = ch + 4 * h;
      if (cc % p.cpg == 0)
        cs[((int64_t)n * nchunk + chunk) * p.G + cc / p.cpg] =
            float2{mu[h], group_sum(hs, 2 * gq + h, p.cpg)};
    }
  }
}

// Forward, launch 2: merge the chunk statistics of the slab's groups in chunk order, then
// normalise, affine, FiLM, SiLU, bf16 for this workgroup's chunk. Chunk 0 writes mean/rstd.
template <bool kF32, bool kFilm, bool kDrop>
__global__ __launch_bounds__(8 * kChPLN) void gn_chunk_apply_kernel(const GnArgs p,
                                                                   const float2* __restrict__ cs,
                                                                   int nchunk) {
  __shared__ uint32_t qred[8 * kChPLN / 64];
  __shared__ float2 gstat[kSlab / 4];
  __shared__ float2 lcs[kMaxChunks * (kSlab / 4)];
  const int n = blockIdx.y, chunk = blockIdx.z;
  const int c0 = blockIdx.x * kSlab;
  const int gq = threadIdx.x & 7;
  const int pl = threadIdx.x >> 3;
  const int ch = c0 + gq * 8;
  const GnSrc<kF32, false> in(p, (int64_t)n * p.HW * p.C + ch);
  uint4 v[in.kN][kChU];
  bool ok[kChU];
  int pxs[kChU];
  chunk_load(in.src, in.stride, chunk * kChunkPx, pl, p.HW, v, ok, pxs);

  // the slab's chunk statistics, all loads in flight at once, then merged from LDS
  const int ngs = kSlab / p.cpg;
  const int g0 = c0 / p.cpg;
  for (int i = threadIdx.x; i < ngs * nchunk; i += 8 * kChPLN) {
    const int k = i / ngs;
    lcs[i] = cs[((int64_t)n * nchunk + k) * p.G + g0 + (i - k * ngs)];
  }
  __syncthreads();
  if ((int)threadIdx.x < ngs) {
    const int g = g0 + threadIdx.x;
    float na = 0.f, mean = 0.f, m2 = 0.f;
    for (int k = 0; k < nchunk; ++k) {
      const float2 b = lcs[k * ngs + threadIdx.x];
      const float nb = (float)(chunk_pixels(p.HW, k) * p.cpg);
      const float nt = na + nb;
      const float d = b.x - mean;
      const float wgt = nb / nt;
      mean += d * wgt;
      m2 += b.y + d * d * (na * wgt);
      na = nt;
    }
    const float rs = 1.0f / sqrtf(m2 / na + p.eps);
    gstat[threadIdx.x] = float2{mean, rs};
    if (chunk == 0) {
      p.mean[n * p.G + g] = mean;
      p.rstd[n * p.G + g] = rs;
    }
  }
  __syncthreads();
  float mu[2], rs[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float2 st = gstat[(ch + 4 * h - c0) / p.cpg];
    mu[h] = st.x;
    rs[h] = st.y;
  }
  float A[8], B[8];
  fwd_affine<kFilm>(p, n, ch, mu, rs, A, B);
  uint16_t* ob = static_cast<uint16_t*>(p.out) + (int64_t)n * p.HW * p.C + ch;
  const uint64_t seed = kDrop ? *p.drop_seed : 0;
  GnQ qo(p);
  us2 xacc = {0, 0};
#pragma unroll
  for (int u = 0; u < kChU; ++u) {
    float f[8];
    unpack_x<kF32>(v, u, f);
    const int64_t off = ((int64_t)n * p.HW + pxs[u]) * p.C + ch;
    if constexpr (kF32) {
      if (p.x_bf16 && ok[u]) xacc = absmax8(xacc, store_x_bf16(p, off, f));
    }
    const uint32_t kb = kDrop ? drop_keep8(seed, off, p.drop_keep) : 0u;
    const uint4 o = fwd_out8<kDrop>(f, A, B, kb, p.drop_scale);
    if (ok[u]) {
      if (p.q)
        qo.put(p, off, o);
      else
        st_nt16(ob + (int64_t)pxs[u] * p.C, o);
    }
  }
  if (p.q) qo.finish(p, qred);
  if constexpr (kF32) {
    if (p.x_bf16 && p.xb_part) {
      __syncthreads();  // qred is reused
      finish_xb_amax(p, xacc, qred);
    }
  }
}

struct GnBwdSetup {
  float mu[2], rs[2], nmr[2], gm[8], bt[8], fsc[8], fsh[8], gC[8];  // nmr = -mu rs, gC = fs gm
};

// The backward terms of one pixel's 8 channels (see gn_silu_bwd_kernel): xhat, and g = dout
// times d silu(zp) / d zp at zp = fs (xhat gamma + beta) + fb (no FiLM: fs = 1, fb = 0).
template <bool kFilm>
__device__ __forceinline__ void bwd_terms(const float (&f)[8], const float (&d)[8],
                                          const GnBwdSetup& st, float (&xh)[8], float (&g)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    xh[e] = __builtin_fmaf(f[e], st.rs[e >> 2], st.nmr[e >> 2]);
    const float z = __builtin_fmaf(xh[e], st.gm[e], st.bt[e]);
    const float zp = kFilm ? __builtin_fmaf(st.fsc[e], z, st.fsh[e]) : z;
    const float sg = sigmoid_hw(zp);
    g[e] = d[e] * (sg * __builtin_fmaf(zp, 1.0f - sg, 1.0f));
  }
}

// dout of 8 channels, masked and scaled by the forward's dropout
template <bool kDrop>
__device__ __forceinline__ void bwd_dout(uint4 v, uint64_t seed, int64_t off, const GnArgs& p,
                                         float (&d)[8]) {
  unpack8(v, d);
  if (kDrop) {
    const uint32_t kb = drop_keep8(seed, off, p.drop_keep);
#pragma unroll
    for (int e = 0; e < 8; ++e) d[e] = (kb >> e) & 1u ? d[e] * p.drop_scale : 0.0f;
  }
}

// the same with the keep bits already formed (the resident backward hashes once per pixel)
template <bool kDrop>
__device__ __forceinline__ void bwd_dout_kb(uint4 v, uint32_t kb, float drop_scale,
                                            float (&d)[8]) {
  unpack8(v, d);
  if (kDrop) {
#pragma unroll
    for (int e = 0; e < 8; ++e) d[e] = drop_sel(d[e], kb, e, drop_scale);
  }
}

template <bool kFilm>
__device__ __forceinline__ void gn_bwd_setup(const GnArgs& p, int n, int ch, GnBwdSetup& st) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int g = (ch + 4 * h) / p.cpg;
    st.mu[h] = p.mean[n * p.G + g];
    st.rs[h] = p.rstd[n * p.G + g];
  }
  load8f(p.gamma + ch, st.gm);
  load8f(p.beta + ch, st.bt);
  if (kFilm) {
    load_film(p, n, ch, st.fsc, st.fsh);
  } else {  // compile-time identity: the FiLM terms fold away
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      st.fsc[e] = 1.0f;
      st.fsh[e] = 0.0f;
    }
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) st.nmr[h] = -st.mu[h] * st.rs[h];
#pragma unroll
  for (int e = 0; e < 8; ++e) st.gC[e] = kFilm ? st.fsc[e] * st.gm[e] : st.gm[e];
}

// Backward, launch 1: grid (C / 64, N, chunks). cp[chunk][n][c] = chunk sums of
// (gz, gz * xhat, g * z, g) of channel c. FiLM scale/shift, gamma and beta are constant per
// (image, channel), so all four follow from S1 = sum g and S2 = sum g * xhat:
// (fs S1, fs S2, gamma S2 + beta S1, S1); only those two sums are accumulated.
template <bool kFilm, bool kF32, bool kDrop>
__global__ __launch_bounds__(8 * kChPLN) void gn_chunk_bwd_sums_kernel(const GnArgs p,
                                                                      float4* __restrict__ cp) {
  constexpr int NS = 16;
  __shared__ float red[(kChPLN / 8) * 8 * NS];
  const int n = blockIdx.y, chunk = blockIdx.z;
  const int c0 = blockIdx.x * kSlab;
  const int gq = threadIdx.x & 7;
  const int pl = threadIdx.x >> 3;
  const int ch = c0 + gq * 8;
  const int64_t base = (int64_t)n * p.HW * p.C + ch;
  const uint64_t seed = kDrop ? *p.drop_seed : 0;
  const GnSrc<kF32, true> in(p, base);
  uint4 v[in.kN][kChU];
  bool ok[kChU];
  int pxs[kChU];
  chunk_load(in.src, in.stride, chunk * kChunkPx, pl, p.HW, v, ok, pxs);
  GnBwdSetup st;
  gn_bwd_setup<kFilm>(p, n, ch, st);
  float acc[NS];
#pragma unroll
  for (int k = 0; k < NS; ++k) acc[k] = 0.f;
#pragma unroll
  for (int u = 0; u < kChU; ++u) {
    float f[8], d[8], xh[8], g[8];
    unpack_x<kF32>(v, u, f);
    bwd_dout<kDrop>(v[in.kN - 1][u], seed, base + (int64_t)pxs[u] * p.C, p, d);
    bwd_terms<kFilm>(f, d, st, xh, g);
    if (ok[u]) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        acc[e] += g[e];
        acc[8 + e] += g[e] * xh[e];
      }
    }
  }
  slab_reduce<NS, kChPLN>(acc, red);
  if (pl == 0) {
    float4* o = cp + ((int64_t)chunk * p.N + n) * p.C + ch;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float s1 = acc[e], s2 = acc[8 + e];
      o[e] = kFilm ? float4{st.fsc[e] * s1, st.fsc[e] * s2, st.gm[e] * s2 + st.bt[e] * s1, s1}
                   : float4{s1, s2, 0.f, 0.f};
    }
  }
}

// Backward, launch 2: per-channel totals over the chunks in order, group means of
// gxh = gz * gamma and gxh * xhat, then dx for this chunk. Chunk 0 writes the per-image
// channel partials of dgamma/dbeta and the FiLM gradients.
template <bool kFilm, bool kF32, bool kDrop>
__global__ __launch_bounds__(8 * kChPLN) void gn_chunk_bwd_apply_kernel(const GnArgs p,
                                                                       const float4* __restrict__ cp,
                                                                       int nchunk) {
  __shared__ uint32_t qred[8 * kChPLN / 64];
  __shared__ float4 tot[kSlab];
  __shared__ float4 slice[4][kSlab];
  __shared__ float hs[2][16];
  const int n = blockIdx.y, chunk = blockIdx.z;
  const int c0 = blockIdx.x * kSlab;
  const int gq = threadIdx.x & 7;
  const int pl = threadIdx.x >> 3;
  const int ch = c0 + gq * 8;
  const int64_t base = (int64_t)n * p.HW * p.C + ch;
  const uint64_t seed = kDrop ? *p.drop_seed : 0;
  const GnSrc<kF32, true> in(p, base);
  uint4 v[in.kN][kChU];
  bool ok[kChU];
  int pxs[kChU];
  chunk_load(in.src, in.stride, chunk * kChunkPx, pl, p.HW, v, ok, pxs);
  GnBwdSetup st;
  gn_bwd_setup<kFilm>(p, n, ch, st);
  GnQ qo(p);

  // channel totals over the chunks: four interleaved slices of chunks per channel (loads
  // in flight together), then the slices in order (deterministic)
  {
    const int cl = threadIdx.x & (kSlab - 1), sl = threadIdx.x >> 6;
    const float4* q = cp + (int64_t)n * p.C + c0 + cl;
    const int64_t stride = (int64_t)p.N * p.C;
    float4 t = float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int k = sl; k < nchunk; k += 4) {
      const float4 b = q[k * stride];
      t.x += b.x;
      t.y += b.y;
      t.z += b.z;
      t.w += b.w;
    }
    slice[sl][cl] = t;
  }
  __syncthreads();
  if (threadIdx.x < kSlab) {
    const int c = c0 + threadIdx.x;
    float4 t = slice[0][threadIdx.x];
#pragma unroll
    for (int sl = 1; sl < 4; ++sl) {
      const float4 b = slice[sl][threadIdx.x];
      t.x += b.x;
      t.y += b.y;
      t.z += b.z;
      t.w += b.w;
    }
    tot[threadIdx.x] = t;
    if (chunk == 0) {
      const int64_t nc = (int64_t)p.N * p.C;
      const int64_t o = (int64_t)n * p.C + c;
      p.part[o] = t.y;       // dgamma partial
      p.part[nc + o] = t.x;  // dbeta partial
      if (p.dfs) {
        p.dfs[o] = t.z;
        p.dfb[o] = t.w;
      } else if (p.dwb) {
        const int64_t ob = (int64_t)n * 2 * p.C + c;
        p.dwb[ob] = (uint16_t)f32_to_bf16_bits(t.z);
        p.dwb[ob + p.C] = (uint16_t)f32_to_bf16_bits(t.w);
      }
    }
  }
  __syncthreads();
  if (pl == 0) {
    float h1[2] = {0.f, 0.f}, h2[2] = {0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float4 t = tot[gq * 8 + e];
      h1[e >> 2] += t.x * st.gm[e];
      h2[e >> 2] += t.y * st.gm[e];
    }
    hs[0][2 * gq] = h1[0];
    hs[0][2 * gq + 1] = h1[1];
    hs[1][2 * gq] = h2[0];
    hs[1][2 * gq + 1] = h2[1];
  }
  __syncthreads();
  const float inv_cnt = 1.0f / (float)((int64_t)p.HW * p.cpg);
  float m1[2], m2[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    m1[h] = group_sum(hs[0], 2 * gq + h, p.cpg) * inv_cnt;
    m2[h] = group_sum(hs[1], 2 * gq + h, p.cpg) * inv_cnt;
  }
#pragma unroll
  for (int u = 0; u < kChU; ++u) {
    float f[8], d[8], xh[8], g[8];
    unpack_x<kF32>(v, u, f);
    bwd_dout<kDrop>(v[in.kN - 1][u], seed, base + (int64_t)pxs[u] * p.C, p, d);
    bwd_terms<kFilm>(f, d, st, xh, g);
    auto dx = [&](int e) __attribute__((always_inline)) {
      const int h = e >> 2;
      return st.rs[h] * __builtin_fmaf(-xh[e], m2[h], g[e] * st.gC[e] - m1[h]);
    };
    if (ok[u]) store_dx<kF32>(p, base + (int64_t)pxs[u] * p.C, dx, qo);
  }
  if (p.q) qo.finish(p, qred);
}

// ---- resident form (HW <= kResMaxHW: the 32x32, 16x16, 8x8 and 4x4 levels): one workgroup
// per (image, slab) of PLN pixel lanes x 8 granules holds all of the slab's pixels in
// registers (U per lane, packed as loaded), so the forward and the backward each read their
// inputs once and write their outputs once; every pass unpacks from those registers ----
constexpr int kResMaxHW = 1024;

// v unchanged, but opaque to the optimiser (no value numbering across this point)
__device__ __forceinline__ void opaque_u4(uint4& v) {
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
}

// Lane pl's pixels pl + PLN u; pixels past HW load pixel HW - 1 (a valid address) with ok false.
template <int NL, int PLN, int U>
__device__ __forceinline__ void res_load(const uint8_t* const (&src)[NL], const int (&stride)[NL],
                                         int pl, int HW, uint4 (&v)[NL][U], bool (&ok)[U],
                                         int (&pxs)[U]) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int px = pl + u * PLN;
    ok[u] = px < HW;
    pxs[u] = ok[u] ? px : HW - 1;
  }
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int l = 0; l < NL; ++l)
      v[l][u] = *reinterpret_cast<const uint4*>(src[l] + (int64_t)pxs[u] * stride[l]);
}

// Two-source x (GnArgs::cat_a / cat_h) of channels ch .. ch + 7 (all of them from one source:
// cat_ca is a multiple of the slab), lane pl's pixels pl + PLN u as res_load's. kF32: x as
// fp32 bits in v[0] (channels 0-3) and v[1] (4-7), bf16 sources widened; else bf16 in v[0]
// (cat_h bf16). kDout: dout of the pixel in v[NL - 1].
template <int NL, int PLN, int U, bool kF32, bool kDout>
__device__ __forceinline__ void cat_load(const GnArgs& p, int n, int ch, int pl, uint4 (&v)[NL][U],
                                         bool (&ok)[U], int (&pxs)[U]) {
  static_assert(NL == (kF32 ? 2 : 1) + (kDout ? 1 : 0), "x parts and dout");
  const int W = p.cat_w, wl = W >> 1, ca = p.cat_ca;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int px = pl + PLN * u;
    ok[u] = px < p.HW;
    pxs[u] = ok[u] ? px : p.HW - 1;
  }
  auto widen = [&](int u) __attribute__((always_inline)) {
    if constexpr (kF32) {
      const uint4 b = v[0][u];
      v[0][u] = uint4{b.x << 16, b.x & 0xffff0000u, b.y << 16, b.y & 0xffff0000u};
      v[1][u] = uint4{b.z << 16, b.z & 0xffff0000u, b.w << 16, b.w & 0xffff0000u};
    }
  };
  if (ch < ca) {
    const uint16_t* a = p.cat_a + (int64_t)n * (p.HW >> 2) * ca + ch;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int y = pxs[u] / W, x = pxs[u] - y * W;
      v[0][u] = *reinterpret_cast<const uint4*>(a + ((y >> 1) * wl + (x >> 1)) * ca);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) widen(u);
  } else {
    const int chh = p.C - ca;
    const int64_t off = (int64_t)n * p.HW * chh + (ch - ca);
    bool f32 = false;
    if constexpr (kF32) f32 = p.cat_hf != 0;
    if (f32) {
      const float* h = static_cast<const float*>(static_cast<const void*>(p.cat_h)) + off;
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int k = 0; k < (kF32 ? 2 : 1); ++k)
          v[k][u] = *reinterpret_cast<const uint4*>(h + (int64_t)pxs[u] * chh + 4 * k);
    } else {
      const uint16_t* h = p.cat_h + off;
#pragma unroll
      for (int u = 0; u < U; ++u) v[0][u] = *reinterpret_cast<const uint4*>(h + (int64_t)pxs[u] * chh);
#pragma unroll
      for (int u = 0; u < U; ++u) widen(u);
    }
  }
  if constexpr (kDout) {
    const uint16_t* d = p.dout + (int64_t)n * p.HW * p.C + ch;
#pragma unroll
    for (int u = 0; u < U; ++u)
      v[NL - 1][u] = *reinterpret_cast<const uint4*>(d + (int64_t)pxs[u] * p.C);
  }
}

template <int PLN, int U, bool kFilm, bool kF32, bool kDrop, bool kCat = false>
__global__ __launch_bounds__(8 * PLN) void gn_res_fwd_kernel(const GnArgs p) {
  static_assert(!kCat || PLN * U == 1024 || (kF32 && PLN * U == 256), "32x32 or 16x16 images");
  __shared__ uint32_t qred[PLN / 8];
  __shared__ float red[(PLN / 8) * 8 * 2];
  __shared__ float hs[16];
  const int n = blockIdx.y;
  const int c0 = blockIdx.x * kSlab;
  const int gq = threadIdx.x & 7;
  const int pl = threadIdx.x >> 3;
  const int ch = c0 + gq * 8;
  const GnSrc<kF32, false> in(p, (int64_t)n * p.HW * p.C + ch);
  uint4 v[in.kN][U];
  bool ok[U];
  int pxs[U];
  if constexpr (kCat)
    cat_load<in.kN, PLN, U, kF32, false>(p, n, ch, pl, v, ok, pxs);
  else
    res_load<in.kN, PLN, U>(in.src, in.stride, pl, p.HW, v, ok, pxs);
  if constexpr (kCat && !kF32) {
    // the bf16 copy of the concatenation is the loaded values themselves
    if (p.x_bf16) {
      us2 xacc = {0, 0};
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (ok[u]) {
          st_nt16(p.x_bf16 + ((int64_t)n * p.HW + pxs[u]) * p.C + ch, v[0][u]);
          xacc = absmax8(xacc, v[0][u]);
        }
      if (p.xb_part) finish_xb_amax(p, xacc, qred);
    }
  } else if constexpr (kF32) {
    if (p.x_bf16) {
      us2 xacc = {0, 0};
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (ok[u]) {
          float f[8];
          unpack_x<kF32>(v, u, f);
          xacc = absmax8(xacc, store_x_bf16(p, ((int64_t)n * p.HW + pxs[u]) * p.C + ch, f));
        }
      if (p.xb_part) finish_xb_amax(p, xacc, qred);
    }
  }
  float sm[2] = {0.f, 0.f};
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (ok[u]) {
      float f[8];
      unpack_x<kF32>(v, u, f);
      sm[0] += (f[0] + f[1]) + (f[2] + f[3]);
      sm[1] += (f[4] + f[5]) + (f[6] + f[7]);
    }
  slab_reduce<2, PLN>(sm, red);
  if (pl == 0) {
    hs[2 * gq] = sm[0];
    hs[2 * gq + 1] = sm[1];
  }
  __syncthreads();
  const float inv_cnt = 1.0f / (float)(p.HW * p.cpg);
  const float mu[2] = {group_sum(hs, 2 * gq, p.cpg) * inv_cnt,
                       group_sum(hs, 2 * gq + 1, p.cpg) * inv_cnt};
  __syncthreads();
  float q[2] = {0.f, 0.f};
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (ok[u]) {
      float f[8];
      unpack_x<kF32>(v, u, f);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = f[e] - mu[e >> 2];
        q[e >> 2] += d * d;
      }
    }
  slab_reduce<2, PLN>(q, red);
  if (pl == 0) {
    hs[2 * gq] = q[0];
    hs[2 * gq + 1] = q[1];
  }
  __syncthreads();
  float rs[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) rs[h] = 1.0f / sqrtf(group_sum(hs, 2 * gq + h, p.cpg) * inv_cnt + p.eps);
  if (pl == 0) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int cc = ch + 4 * h;
      if (cc % p.cpg == 0) {
        p.mean[n * p.G + cc / p.cpg] = mu[h];
        p.rstd[n * p.G + cc / p.cpg] = rs[h];
      }
    }
  }
  float A[8], B[8];
  fwd_affine<kFilm>(p, n, ch, mu, rs, A, B);
  uint16_t* ob = static_cast<uint16_t*>(p.out) + (int64_t)n * p.HW * p.C + ch;
  const uint64_t seed = kDrop ? *p.drop_seed : 0;
  GnQ qo(p);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float f[8];
    unpack_x<kF32>(v, u, f);
    const int64_t off = ((int64_t)n * p.HW + pxs[u]) * p.C + ch;
    const uint32_t kb = kDrop ? drop_keep8(seed, off, p.drop_keep) : 0u;
    const uint4 o = fwd_out8<kDrop>(f, A, B, kb, p.drop_scale);
    if (ok[u]) {
      if (p.q)
        qo.put(p, off, o);
      else
        st_nt16(ob + (int64_t)pxs[u] * p.C, o);
    }
  }
  if (p.q) qo.finish(p, qred);
}

// The backward keeps x in registers and, at 16 pixels per lane (where x and dout together
// would exceed the register file), dout in LDS: DMA'd there at the start (lane i of a wave's
// u-th transfer at 16-B slot u * 8 PLN + thread), read back by the same thread in both passes.
template <int PLN, int U>
struct GnResDout {
  static constexpr bool kLds = U >= 16;
  static constexpr int kBytes = kLds ? U * 8 * PLN * 16 : 16;
};

template <int PLN, int U, bool kFilm, bool kF32, bool kDrop, bool kCat = false>
__global__ __launch_bounds__(8 * PLN) void gn_res_bwd_kernel(const GnArgs p) {
  static_assert(!kCat || (!kF32 && PLN == 64 && U == 16) || (kF32 && PLN == 32 && U == 8),
                "32x32 images (bf16 sources) or 16x16 (cat_h bf16 or fp32)");
  using DL = GnResDout<PLN, U>;
  __shared__ __attribute__((aligned(16))) uint8_t dls[DL::kBytes];
  __shared__ uint32_t qred[PLN / 8];
  __shared__ float red[(PLN / 8) * 8 * 16];
  __shared__ float hs[2][16];
  // kCat without the dout copy in LDS: four pixel rows of the 2x2 window exchange
  __shared__ __attribute__((aligned(16))) float xch[kCat && !DL::kLds ? 4 * (PLN / 4) * 8 * 16 : 4];
  const int n = blockIdx.y;
  const int c0 = blockIdx.x * kSlab;
  const int gq = threadIdx.x & 7;
  const int pl = threadIdx.x >> 3;
  const int ch = c0 + gq * 8;
  const int64_t base = (int64_t)n * p.HW * p.C + ch;
  const uint64_t seed = kDrop ? *p.drop_seed : 0;
  // x (and, without the LDS copy, dout) in registers
  const GnSrc<kF32, !DL::kLds> in(p, base);
  uint4 v[in.kN][U];
  bool ok[U];
  int pxs[U];
  if constexpr (kCat) {
    cat_load<in.kN, PLN, U, kF32, !DL::kLds>(p, n, ch, pl, v, ok, pxs);
  } else {
    res_load<in.kN, PLN, U>(in.src, in.stride, pl, p.HW, v, ok, pxs);
  }
  if constexpr (DL::kLds) {
    const uint32_t lbase =
        __builtin_amdgcn_readfirstlane(LDS_ADDR(dls) + (uint32_t)(threadIdx.x & ~63) * 16);
#pragma unroll
    for (int u = 0; u < U; ++u)
      dma16_lds(p.dout + base + (int64_t)pxs[u] * p.C, lbase + (uint32_t)(u * 8 * PLN * 16));
    wait_vmcnt<0>();
    asm volatile("" ::: "memory");  // the DMA writes are invisible to the compiler
  }
  // dout of pixel u
  auto dout_u = [&](int u) __attribute__((always_inline)) {
    if constexpr (DL::kLds)
      return *reinterpret_cast<const uint4*>(dls + (u * 8 * PLN + threadIdx.x) * 16);
    else
      return v[in.kN - 1][u];
  };
  GnBwdSetup st;
  gn_bwd_setup<kFilm>(p, n, ch, st);
  GnQ qo(p);
  // per-channel S1 = sum g, S2 = sum g * xhat over the image (every lane gets the totals)
  float acc[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) acc[k] = 0.f;
  uint32_t keep[U];  // the dropout keep bits of each pixel, hashed once for both passes
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float f[8], d[8], xh[8], g[8];
    unpack_x<kF32>(v, u, f);
    keep[u] = kDrop ? drop_keep8(seed, base + (int64_t)pxs[u] * p.C, p.drop_keep) : 0u;
    bwd_dout_kb<kDrop>(dout_u(u), keep[u], p.drop_scale, d);
    bwd_terms<kFilm>(f, d, st, xh, g);
    if (ok[u]) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        acc[e] += g[e];
        acc[8 + e] += g[e] * xh[e];
      }
    }
    // one pixel at a time: the packed inputs stay resident, each pixel's unpacked terms die
    // before the next pixel's are formed (else the interleaved pixels exceed the registers)
    __builtin_amdgcn_sched_barrier(0);
  }
  slab_reduce<16, PLN>(acc, red);
  if (pl == 0) {
    const int64_t nc = (int64_t)p.N * p.C;
    float h1[2] = {0.f, 0.f}, h2[2] = {0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float s1 = acc[e], s2 = acc[8 + e];
      const float gz = st.fsc[e] * s1, gzx = st.fsc[e] * s2;  // sums of gz and gz * xhat
      const int64_t o = (int64_t)n * p.C + ch + e;
      p.part[o] = gzx;       // dgamma partial
      p.part[nc + o] = gz;   // dbeta partial
      if (kFilm) {
        const float gzs = st.gm[e] * s2 + st.bt[e] * s1;  // sum g * z
        if (p.dfs) {
          p.dfs[o] = gzs;
          p.dfb[o] = s1;
        } else if (p.dwb) {
          const int64_t ob = (int64_t)n * 2 * p.C + ch + e;
          p.dwb[ob] = (uint16_t)f32_to_bf16_bits(gzs);
          p.dwb[ob + p.C] = (uint16_t)f32_to_bf16_bits(s1);
        }
      }
      h1[e >> 2] += gz * st.gm[e];
      h2[e >> 2] += gzx * st.gm[e];
    }
    hs[0][2 * gq] = h1[0];
    hs[0][2 * gq + 1] = h1[1];
    hs[1][2 * gq] = h2[0];
    hs[1][2 * gq + 1] = h2[1];
  }
  __syncthreads();
  const float inv_cnt = 1.0f / (float)(p.HW * p.cpg);
  float m1[2], m2[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    m1[h] = group_sum(hs[0], 2 * gq + h, p.cpg) * inv_cnt;
    m2[h] = group_sum(hs[1], 2 * gq + h, p.cpg) * inv_cnt;
  }
  // pixel u's dx (the fused concatenation's form; the loop below is the same per pixel)
  auto pixel_dx = [&](int u, float (&t)[8]) __attribute__((always_inline)) {
#pragma unroll
    for (int l = 0; l < in.kN; ++l) opaque_u4(v[l][u]);
    float f[8], d[8], xh[8], g[8];
    unpack_x<kF32>(v, u, f);
    bwd_dout_kb<kDrop>(dout_u(u), keep[u], p.drop_scale, d);
    bwd_terms<kFilm>(f, d, st, xh, g);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int h = e >> 2;
      t[e] = st.rs[h] * __builtin_fmaf(-xh[e], m2[h], g[e] * st.gC[e] - m1[h]);
    }
  };
  if constexpr (kCat) {
    // The concatenation's fp32 gradient (plus the bf16 skip-path gradient, as autograd adds
    // it), split as the upsample-and-concatenate's backward does: cat_h's channels in
    // cat_h's type (bf16: rounded); cat_a's summed over each 2x2 window from zero in
    // row-major order, then rounded to bf16 (torch's upsample_nearest2d_backward). The
    // images are PLN / 2 wide, so pixel pl + PLN u is row 2u + pl / kW, column pl mod kW:
    // window (u, j) holds lanes 2j, 2j + 1 (row 2u) and 2j + kW, 2j + kW + 1 (row 2u + 1). The
    // odd lane's value comes by a shuffle (8 threads on), the lower row's two through LDS
    // (the dout slots already read, or an exchange buffer), four pixels per exchange.
    constexpr int kW = PLN / 2;
    constexpr int kEnt = (kW / 2) * 8 * 16;  // floats per pixel row pair: (window, granule) x 16
    const bool in_a = ch < p.cat_ca;  // workgroup-uniform
    const bool even = (pl & 1) == 0;
    float* xs = DL::kLds ? reinterpret_cast<float*>(dls) : xch;
    constexpr int kSlot = DL::kLds ? 8 * PLN * 4 : kEnt;  // floats between pixel rows u
    static_assert(kEnt <= kSlot, "an exchange fits a dout slot");
    bool hf = false;
    if constexpr (kF32) hf = p.cat_hf != 0;
#pragma unroll
    for (int u0 = 0; u0 < U; u0 += 4) {
      float t[4][8];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int u = u0 + k;
        pixel_dx(u, t[k]);
        if (p.dx_add) {
          float a[8];
          unpack8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.dx_add) +
                                                  base + (int64_t)pxs[u] * p.C), a);
#pragma unroll
          for (int e = 0; e < 8; ++e) t[k][e] += a[e];
        }
        if (!in_a) {
          const int64_t o = ((int64_t)n * p.HW + pxs[u]) * (p.C - p.cat_ca) + (ch - p.cat_ca);
          if (hf) {
            float* gh = static_cast<float*>(p.cat_gh) + o;
#pragma unroll
            for (int q4 = 0; q4 < 2; ++q4)
              st_nt16(gh + 4 * q4, uint4{__float_as_uint(t[k][4 * q4]), __float_as_uint(t[k][4 * q4 + 1]),
                                         __float_as_uint(t[k][4 * q4 + 2]), __float_as_uint(t[k][4 * q4 + 3])});
          } else {
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 8; e += 2) w[e >> 1] = pack_bf16x2(t[k][e], t[k][e + 1]);
            st_nt16(static_cast<uint16_t*>(p.cat_gh) + o, uint4{w[0], w[1], w[2], w[3]});
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (in_a) {
        __syncthreads();  // every thread has read the dout slots u0 .. u0 + 3 (or the buffer)
        float r[4][8];  // the odd neighbour's values (lane + 8: pixel lane pl + 1)
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int e = 0; e < 8; ++e) r[k][e] = __shfl_down(t[k][e], 8, 64);
        // row u0 + k, entry (window column j, granule gq): row 2u + 1's pair, 16 floats
        const int ent = (((pl % kW) >> 1) * 8 + gq) * 16;
        if (pl >= kW && even) {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            float* e0 = xs + (DL::kLds ? u0 + k : k) * kSlot + ent;
#pragma unroll
            for (int q4 = 0; q4 < 2; ++q4) {
              *reinterpret_cast<v4f*>(e0 + 4 * q4) =
                  v4f{t[k][4 * q4], t[k][4 * q4 + 1], t[k][4 * q4 + 2], t[k][4 * q4 + 3]};
              *reinterpret_cast<v4f*>(e0 + 8 + 4 * q4) =
                  v4f{r[k][4 * q4], r[k][4 * q4 + 1], r[k][4 * q4 + 2], r[k][4 * q4 + 3]};
            }
          }
        }
        __syncthreads();
        if (pl < kW && even) {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const float* e0 = xs + (DL::kLds ? u0 + k : k) * kSlot + ent;
            float acc[8];
#pragma unroll
            for (int q4 = 0; q4 < 2; ++q4) {
              const v4f lo = *reinterpret_cast<const v4f*>(e0 + 4 * q4);
              const v4f hi = *reinterpret_cast<const v4f*>(e0 + 8 + 4 * q4);
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int c = 4 * q4 + e;
                acc[c] = 0.0f;
                acc[c] += t[k][c];  // (2u, 2j)
                acc[c] += r[k][c];  // (2u, 2j + 1)
                acc[c] += lo[e];    // (2u + 1, 2j)
                acc[c] += hi[e];    // (2u + 1, 2j + 1)
              }
            }
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 8; e += 2) w[e >> 1] = pack_bf16x2(acc[e], acc[e + 1]);
            const int wi = (u0 + k) * (kW / 2) + (pl >> 1);  // window row u0 + k, column pl / 2
            st_nt16(p.cat_ga + ((int64_t)n * (p.HW >> 2) + wi) * p.cat_ca + ch,
                    uint4{w[0], w[1], w[2], w[3]});
          }
        }
        // (the buffer's next writes come after the next four pixels' first barrier)
      }
    }
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // the second pass forms the per-pixel terms again from the packed registers: hidden
      // from the compiler, which would otherwise keep the first pass's unpacked terms of
      // every pixel alive across the reduction (8-16 registers per pixel more)
#pragma unroll
      for (int l = 0; l < in.kN; ++l) opaque_u4(v[l][u]);
      float f[8], d[8], xh[8], g[8];
      unpack_x<kF32>(v, u, f);
      bwd_dout_kb<kDrop>(dout_u(u), keep[u], p.drop_scale, d);
      bwd_terms<kFilm>(f, d, st, xh, g);
      auto dx = [&](int e) __attribute__((always_inline)) {
        const int h = e >> 2;
        return st.rs[h] * __builtin_fmaf(-xh[e], m2[h], g[e] * st.gC[e] - m1[h]);
      };
      if (ok[u]) store_dx<kF32>(p, base + (int64_t)pxs[u] * p.C, dx, qo);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (p.q) qo.finish(p, qred);
}

// Resident-form geometry for an image of HW pixels: (pixel lanes, pixels per lane), or
// (0, 0) when HW exceeds kResMaxHW.
struct GnRes {
  int pln, u;
};
static GnRes gn_res_shape(int HW) {
  if (HW <= 128) return {32, 4};
  if (HW <= 256) return {32, 8};
  if (HW <= kResMaxHW) return {64, 16};
  return {0, 0};
}
// The backward with an fp32 x holds 2 x 16 B of x per pixel in registers (dout goes to LDS at
// 16 pixels per lane): that fits at 16 pixels per lane without FiLM and dropout (their
// per-channel terms and keep bits are the registers that do not fit); with them, images
// above 256 pixels take the chunked form.
static bool gn_res_bwd_ok(int HW, bool x_f32, bool film, bool drop) {
  return HW <= kResMaxHW && (!x_f32 || HW <= 256 || (!film && !drop));
}

static int gn_chunks(int HW) {
  const int k = (int)ceil_div(HW, kChunkPx);
  return HW >= kChunkMinHW && k <= kMaxChunks ? k : 0;
}

// Pixel lanes per workgroup: enough that every lane has a few pixels to stream.
static int gn_pixel_lanes(int HW) { return HW >= 1024 ? 128 : (HW >= 256 ? 64 : 32); }

static bool gn_shape_ok(int N, int HW, int C, int G) {
  if (N <= 0 || HW <= 0 || C <= 0 || G <= 0) return false;
  if (C % G != 0 || C % kSlab != 0) return false;
  const int cpg = C / G;
  return cpg >= 4 && kSlab % cpg == 0;
}

}  // namespace dpa

using namespace dpa;

#include <type_traits>

// Calls f(bool_constant<a>, bool_constant<b>, bool_constant<c>): one launch site for the
// eight compile-time variants of a kernel.
template <typename F>
static void dispatch3(bool a, bool b, bool c, F f) {
  auto lc = [&](auto A, auto B) {
    if (c)
      f(A, B, std::true_type{});
    else
      f(A, B, std::false_type{});
  };
  auto lb = [&](auto A) {
    if (b)
      lc(A, std::true_type{});
    else
      lc(A, std::false_type{});
  };
  if (a)
    lb(std::true_type{});
  else
    lb(std::false_type{});
}

// The producer-fused e4m3 output of the fp8 entry points (GnArgs::q).
struct GnQOut {
  void* q;
  const float* scale;
  uint32_t* part;
  int cap;
  uint32_t* count;
};

// Workgroups of the launch that writes the output (one amax partial each), 0 for the form
// without the fused cast (HW > 8192 pixels).
static int64_t gn_q_blocks(int N, int HW, int C) {
  if (HW <= kResMaxHW) return (int64_t)(C / kSlab) * N;
  const int nchunk = gn_chunks(HW);
  return nchunk > 0 ? (int64_t)(C / kSlab) * N * nchunk : 0;
}

static int gn_set_q(GnArgs& a, const GnQOut* qo, int64_t nblk) {
  if (!qo) return DPA_OK;
  if (!qo->q || !qo->scale || !qo->part || !qo->count) return DPA_ERR_NULL;
  if (nblk <= 0) return DPA_ERR_SHAPE;
  if (qo->cap < nblk) return DPA_ERR_WORKSPACE;
  if (!aligned(qo->q, 8) || !aligned(qo->scale, 4) || !aligned(qo->part, 4) ||
      !aligned(qo->count, 4))
    return DPA_ERR_ALIGN;
  a.q = (uint8_t*)qo->q;
  a.q_scale = qo->scale;
  a.q_part = qo->part;
  a.q_count = qo->count;
  return DPA_OK;
}

static int64_t gn_fwd_workspace(int N, int HW, int G) {
  return (int64_t)N * gn_chunks(HW) * G * (int64_t)sizeof(float2);
}

// Dropout arguments: keep when the 16-bit hash is >= floor(p * 2^16) (p < 1: at most 65535);
// scale 1 / (1 - p) rounded as torch's dropout forms it (1 - p in double, rounded to fp32, its
// reciprocal rounded to fp32).
static int gn_set_dropout(GnArgs& a, const void* seed, float p) {
  if (!seed) return DPA_OK;
  if (!(p >= 0.0f && p < 1.0f)) return DPA_ERR_SIZE;
  if (!aligned(seed, 8)) return DPA_ERR_ALIGN;
  a.drop_seed = (const uint64_t*)seed;
  a.drop_keep = (uint32_t)((double)p * 65536.0);
  const float pa = (float)(1.0 - (double)p);
  a.drop_scale = (float)(1.0 / (double)pa);
  return DPA_OK;
}

static int gn_fwd(const void* x, const float* gamma, const float* beta, const float* film_scale,
                  const float* film_shift, const void* film_wb, void* out, float* mean,
                  float* rstd, int N, int HW, int C, int G, float eps, void* stream,
                  void* workspace = nullptr, int64_t workspace_bytes = 0, bool x_f32 = false,
                  const void* drop_seed = nullptr, float drop_p = 0.0f, void* x_bf16 = nullptr,
                  const GnQOut* qo = nullptr, uint32_t* xb_part = nullptr,
                  int xb_part_cap = 0) {
  if (!x || !gamma || !beta || (!out && !qo) || !mean || !rstd) return DPA_ERR_NULL;
  if (qo && out) return DPA_ERR_SHAPE;  // one output: bf16 or e4m3
  if ((film_scale == nullptr) != (film_shift == nullptr)) return DPA_ERR_NULL;
  if (!gn_shape_ok(N, HW, C, G)) return DPA_ERR_SHAPE;
  if (!aligned(x, 16) || !aligned(out, 16) || !aligned(film_wb, 2)) return DPA_ERR_ALIGN;
  GnArgs a{};
  a.x = x;
  a.gamma = gamma;
  a.beta = beta;
  a.fs = film_scale;
  a.fb = film_shift;
  a.wb = (const uint16_t*)film_wb;
  a.out = out;
  a.mean = mean;
  a.rstd = rstd;
  a.N = N; a.HW = HW; a.C = C; a.G = G; a.cpg = C / G; a.eps = eps;
  const int nchunk = gn_chunks(HW);
  const GnRes rs = gn_res_shape(HW);
  const bool resident = rs.pln > 0;
  const bool chunked = !resident && nchunk > 0 && workspace &&
                       workspace_bytes >= gn_fwd_workspace(N, HW, G) && aligned(workspace, 8);
  // fp32 x and dropout: the resident form or the chunked form (workspace)
  if ((x_f32 || drop_seed) && !chunked && !resident)
    return nchunk > 0 ? DPA_ERR_WORKSPACE : DPA_ERR_SHAPE;
  if (x_bf16 && !x_f32) return DPA_ERR_SHAPE;  // the bf16 copy is of an fp32 x
  if (!aligned(x_bf16, 16)) return DPA_ERR_ALIGN;
  a.x_bf16 = (uint16_t*)x_bf16;
  if (xb_part) {
    // one partial per workgroup of the launch that writes the copy (the resident form, or
    // the chunked form's apply launch)
    if (!x_bf16) return DPA_ERR_NULL;
    if (!chunked && !resident) return nchunk > 0 ? DPA_ERR_WORKSPACE : DPA_ERR_SHAPE;
    if (xb_part_cap < gn_q_blocks(N, HW, C)) return DPA_ERR_WORKSPACE;
    if (!aligned(xb_part, 4)) return DPA_ERR_ALIGN;
    a.xb_part = xb_part;
  }
  const int dst = gn_set_dropout(a, drop_seed, drop_p);
  if (dst != DPA_OK) return dst;
  if (qo) {
    if (!chunked && !resident) return nchunk > 0 ? DPA_ERR_WORKSPACE : DPA_ERR_SHAPE;
    const int qst = gn_set_q(a, qo, gn_q_blocks(N, HW, C));
    if (qst != DPA_OK) return qst;
    a.out = qo->q;  // not written: the kernels store through a.q
  }
  hipStream_t s = (hipStream_t)stream;
  if (chunked) {
    dim3 cgrid((unsigned)(C / kSlab), (unsigned)N, (unsigned)nchunk);
    float2* cs = (float2*)workspace;
    if (x_f32)
      gn_chunk_stats_kernel<true><<<cgrid, 8 * kChPLN, 0, s>>>(a, cs, nchunk);
    else
      gn_chunk_stats_kernel<false><<<cgrid, 8 * kChPLN, 0, s>>>(a, cs, nchunk);
    int st = launch_status();
    if (st != DPA_OK) return st;
    dispatch3(x_f32, a.fs || a.wb, a.drop_seed != nullptr, [&](auto F32, auto FILM, auto DROP) {
      gn_chunk_apply_kernel<decltype(F32)::value, decltype(FILM)::value, decltype(DROP)::value>
          <<<cgrid, 8 * kChPLN, 0, s>>>(a, cs, nchunk);
    });
    return launch_status();
  }
  dim3 grid((unsigned)(C / kSlab), (unsigned)N);
  if (resident) {
    dispatch3(a.fs || a.wb, x_f32, a.drop_seed != nullptr, [&](auto FILM, auto F32, auto DROP) {
      constexpr bool kF = decltype(FILM)::value, k3 = decltype(F32)::value,
                     kD = decltype(DROP)::value;
      if (rs.u == 4)
        gn_res_fwd_kernel<32, 4, kF, k3, kD><<<grid, 8 * 32, 0, s>>>(a);
      else if (rs.u == 8)
        gn_res_fwd_kernel<32, 8, kF, k3, kD><<<grid, 8 * 32, 0, s>>>(a);
      else
        gn_res_fwd_kernel<64, 16, kF, k3, kD><<<grid, 8 * 64, 0, s>>>(a);
    });
    return launch_status();
  }
  const int pln = gn_pixel_lanes(HW);
  if (pln == 128)
    gn_silu_fwd_kernel<128><<<grid, 8 * 128, 0, (hipStream_t)stream>>>(a);
  else if (pln == 64)
    gn_silu_fwd_kernel<64><<<grid, 8 * 64, 0, (hipStream_t)stream>>>(a);
  else
    gn_silu_fwd_kernel<32><<<grid, 8 * 32, 0, (hipStream_t)stream>>>(a);
  return launch_status();
}

extern "C" int dpa_gn_silu_fwd_bf16(const void* x, const float* gamma, const float* beta,
                                    const float* film_scale, const float* film_shift, void* out,
                                    float* mean, float* rstd, int N, int HW, int C, int G,
                                    float eps, void* stream) {
  return gn_fwd(x, gamma, beta, film_scale, film_shift, nullptr, out, mean, rstd, N, HW, C, G,
                eps, stream);
}

extern "C" int dpa_gn_silu_film_fwd_bf16(const void* x, const float* gamma, const float* beta,
                                         const void* film_wb, void* out, float* mean, float* rstd,
                                         int N, int HW, int C, int G, float eps, void* stream) {
  if (!film_wb) return DPA_ERR_NULL;
  return gn_fwd(x, gamma, beta, nullptr, nullptr, film_wb, out, mean, rstd, N, HW, C, G, eps,
                stream);
}

extern "C" int64_t dpa_gn_silu_fwd_workspace_bytes(int N, int HW, int C, int G) {
  if (!gn_shape_ok(N, HW, C, G)) return 0;
  return gn_fwd_workspace(N, HW, G);
}

extern "C" int dpa_gn_silu_fwd_ws_bf16(const void* x, const float* gamma, const float* beta,
                                       const float* film_scale, const float* film_shift,
                                       const void* film_wb, void* out, float* mean, float* rstd,
                                       void* workspace, int64_t workspace_bytes, int N, int HW,
                                       int C, int G, float eps, void* stream) {
  if (film_wb && film_scale) return DPA_ERR_SHAPE;  // one FiLM form at a time
  if (gn_shape_ok(N, HW, C, G) && workspace_bytes < gn_fwd_workspace(N, HW, G))
    return DPA_ERR_WORKSPACE;
  if (workspace_bytes > 0 && !workspace) return DPA_ERR_WORKSPACE;
  if (!aligned(workspace, 8)) return DPA_ERR_ALIGN;
  return gn_fwd(x, gamma, beta, film_scale, film_shift, film_wb, out, mean, rstd, N, HW, C, G,
                eps, stream, workspace, workspace_bytes);
}

extern "C" int dpa_gn_silu_fwd_ex(const void* x, int x_dtype, const float* gamma,
                                  const float* beta, const float* film_scale,
                                  const float* film_shift, const void* film_wb, void* out,
                                  float* mean, float* rstd, void* workspace,
                                  int64_t workspace_bytes, int N, int HW, int C, int G, float eps,
                                  const void* drop_seed, float drop_p, void* x_bf16,
                                  void* stream) {
  if (x_dtype != DPA_DTYPE_BF16 && x_dtype != DPA_DTYPE_F32) return DPA_ERR_SHAPE;
  if (film_wb && film_scale) return DPA_ERR_SHAPE;
  if (gn_shape_ok(N, HW, C, G) && workspace_bytes < gn_fwd_workspace(N, HW, G))
    return DPA_ERR_WORKSPACE;
  if (workspace_bytes > 0 && !workspace) return DPA_ERR_WORKSPACE;
  if (!aligned(workspace, 8)) return DPA_ERR_ALIGN;
  return gn_fwd(x, gamma, beta, film_scale, film_shift, film_wb, out, mean, rstd, N, HW, C, G,
                eps, stream, workspace, workspace_bytes, x_dtype == DPA_DTYPE_F32, drop_seed,
                drop_p, x_bf16);
}

extern "C" int dpa_gn_silu_fwd_ex_amax(const void* x, int x_dtype, const float* gamma,
                                       const float* beta, const float* film_scale,
                                       const float* film_shift, const void* film_wb, void* out,
                                       float* mean, float* rstd, void* workspace,
                                       int64_t workspace_bytes, int N, int HW, int C, int G,
                                       float eps, const void* drop_seed, float drop_p,
                                       void* x_bf16, uint32_t* xb_partials, int xb_partials_cap,
                                       void* stream) {
  if (x_dtype != DPA_DTYPE_BF16 && x_dtype != DPA_DTYPE_F32) return DPA_ERR_SHAPE;
  if (film_wb && film_scale) return DPA_ERR_SHAPE;
  if (!xb_partials) return DPA_ERR_NULL;
  if (gn_shape_ok(N, HW, C, G) && workspace_bytes < gn_fwd_workspace(N, HW, G))
    return DPA_ERR_WORKSPACE;
  if (workspace_bytes > 0 && !workspace) return DPA_ERR_WORKSPACE;
  if (!aligned(workspace, 8)) return DPA_ERR_ALIGN;
  return gn_fwd(x, gamma, beta, film_scale, film_shift, film_wb, out, mean, rstd, N, HW, C, G,
                eps, stream, workspace, workspace_bytes, x_dtype == DPA_DTYPE_F32, drop_seed,
                drop_p, x_bf16, nullptr, xb_partials, xb_partials_cap);
}

// per-image channel partials of dgamma/dbeta, then (chunked form) the chunk sums
static int64_t gn_bwd_workspace(int N, int HW, int C) {
  return (int64_t)2 * N * C * 4 + (int64_t)gn_chunks(HW) * N * C * (int64_t)sizeof(float4);
}

extern "C" int64_t dpa_gn_silu_bwd_workspace_bytes(int N, int HW, int C, int G) {
  (void)G;
  if (N <= 0 || HW <= 0 || C <= 0) return 0;
  return gn_bwd_workspace(N, HW, C);
}

static int gn_bwd(const void* x, const void* dout, const float* gamma, const float* beta,
                  const float* film_scale, const float* film_shift, const void* film_wb,
                  const float* mean, const float* rstd, void* dx, float* dgamma, float* dbeta,
                  float* dfilm_scale, float* dfilm_shift, void* dfilm_wb, void* workspace,
                  int64_t workspace_bytes, int N, int HW, int C, int G, void* stream,
                  bool x_f32 = false, const void* drop_seed = nullptr, float drop_p = 0.0f,
                  const void* dx_add = nullptr, bool dx_add_bf16 = false,
                  const GnQOut* qo = nullptr) {
  if (qo) dx = qo->q;  // the e4m3 dx replaces the bf16 one
  if (!x || !dout || !gamma || !beta || !mean || !rstd || !dx || !dgamma || !dbeta)
    return DPA_ERR_NULL;
  if ((film_scale == nullptr) != (film_shift == nullptr)) return DPA_ERR_NULL;
  if (film_scale && (!dfilm_scale || !dfilm_shift)) return DPA_ERR_NULL;
  if (film_wb && !dfilm_wb) return DPA_ERR_NULL;
  if (!gn_shape_ok(N, HW, C, G)) return DPA_ERR_SHAPE;
  if (!workspace || workspace_bytes < (int64_t)2 * N * C * 4) return DPA_ERR_WORKSPACE;
  if (!aligned(x, 16) || !aligned(dout, 16) || !aligned(dx, 16) || !aligned(workspace, 4) ||
      !aligned(film_wb, 2) || !aligned(dfilm_wb, 2))
    return DPA_ERR_ALIGN;
  GnArgs a{};
  a.x = x;
  a.dout = (const uint16_t*)dout;
  a.gamma = gamma;
  a.beta = beta;
  a.fs = film_scale;
  a.fb = film_shift;
  a.wb = (const uint16_t*)film_wb;
  a.out = dx;
  a.mean = const_cast<float*>(mean);
  a.rstd = const_cast<float*>(rstd);
  a.part = (float*)workspace;
  a.dfs = film_scale ? dfilm_scale : nullptr;
  a.dfb = film_scale ? dfilm_shift : nullptr;
  a.dwb = film_wb ? (uint16_t*)dfilm_wb : nullptr;
  a.N = N; a.HW = HW; a.C = C; a.G = G; a.cpg = C / G; a.eps = 0.f;
  hipStream_t s = (hipStream_t)stream;
  const int nchunk = gn_chunks(HW);
  const GnRes rs = gn_res_shape(HW);
  const bool resident =
      gn_res_bwd_ok(HW, x_f32, film_scale || film_wb, drop_seed != nullptr);
  const bool chunked = !resident && nchunk > 0 && workspace_bytes >= gn_bwd_workspace(N, HW, C) &&
                       aligned(workspace, 16);
  if ((x_f32 || drop_seed || dx_add) && !chunked && !resident)
    return nchunk > 0 ? DPA_ERR_WORKSPACE : DPA_ERR_SHAPE;
  if (!aligned(dx_add, 16)) return DPA_ERR_ALIGN;
  a.dx_add = dx_add;
  a.dx_add_bf16 = x_f32 && dx_add_bf16;
  const int dst = gn_set_dropout(a, drop_seed, drop_p);
  if (dst != DPA_OK) return dst;
  if (qo) {
    if (x_f32 || dx_add) return DPA_ERR_SHAPE;  // e4m3 of a bf16 dx, nothing added
    if (!chunked && !resident) return nchunk > 0 ? DPA_ERR_WORKSPACE : DPA_ERR_SHAPE;
    const int qst = gn_set_q(a, qo, gn_q_blocks(N, HW, C));
    if (qst != DPA_OK) return qst;
  }
  const bool film = a.fs || a.wb;
  int st = DPA_OK;
  if (chunked) {
    // chunk sums after the 2*N*C per-image partials (16-B aligned: 8*N*C bytes, C % 64 == 0)
    float4* cp = (float4*)((float*)workspace + (int64_t)2 * N * C);
    dim3 cgrid((unsigned)(C / kSlab), (unsigned)N, (unsigned)nchunk);
    const bool drop = a.drop_seed != nullptr;
    dispatch3(film, x_f32, drop, [&](auto FILM, auto F32, auto DROP) {
      gn_chunk_bwd_sums_kernel<decltype(FILM)::value, decltype(F32)::value, decltype(DROP)::value>
          <<<cgrid, 8 * kChPLN, 0, s>>>(a, cp);
    });
    st = launch_status();
    if (st != DPA_OK) return st;
    dispatch3(film, x_f32, drop, [&](auto FILM, auto F32, auto DROP) {
      gn_chunk_bwd_apply_kernel<decltype(FILM)::value, decltype(F32)::value, decltype(DROP)::value>
          <<<cgrid, 8 * kChPLN, 0, s>>>(a, cp, nchunk);
    });
  } else if (resident) {
    dim3 grid((unsigned)(C / kSlab), (unsigned)N);
    dispatch3(film, x_f32, a.drop_seed != nullptr, [&](auto FILM, auto F32, auto DROP) {
      constexpr bool kF = decltype(FILM)::value, k3 = decltype(F32)::value,
                     kD = decltype(DROP)::value;
      if (rs.u == 4)
        gn_res_bwd_kernel<32, 4, kF, k3, kD><<<grid, 8 * 32, 0, s>>>(a);
      else if (rs.u == 8)
        gn_res_bwd_kernel<32, 8, kF, k3, kD><<<grid, 8 * 32, 0, s>>>(a);
      else if constexpr (!k3 || (!kF && !kD))  // (gn_res_bwd_ok)
        gn_res_bwd_kernel<64, 16, kF, k3, kD><<<grid, 8 * 64, 0, s>>>(a);
    });
  } else {
    dim3 grid((unsigned)(C / kSlab), (unsigned)N);
    const int pln = gn_pixel_lanes(HW);
    if (pln == 128)
      gn_silu_bwd_kernel<128><<<grid, 8 * 128, 0, s>>>(a);
    else if (pln == 64)
      gn_silu_bwd_kernel<64><<<grid, 8 * 64, 0, s>>>(a);
    else
      gn_silu_bwd_kernel<32><<<grid, 8 * 32, 0, s>>>(a);
  }
  st = launch_status();
  if (st != DPA_OK) return st;
  gn_param_reduce_kernel<<<(unsigned)ceil_div(C, 64), 64 * kPrSlices, 0, s>>>(
      (const float*)workspace, dgamma, dbeta, N, C);
  return launch_status();
}

extern "C" int dpa_gn_silu_bwd_bf16(const void* x, const void* dout, const float* gamma,
                                    const float* beta, const float* film_scale,
                                    const float* film_shift, const float* mean,
                                    const float* rstd, void* dx, float* dgamma, float* dbeta,
                                    float* dfilm_scale, float* dfilm_shift, void* workspace,
                                    int64_t workspace_bytes, int N, int HW, int C, int G,
                                    void* stream) {
  return gn_bwd(x, dout, gamma, beta, film_scale, film_shift, nullptr, mean, rstd, dx, dgamma,
                dbeta, dfilm_scale, dfilm_shift, nullptr, workspace, workspace_bytes, N, HW, C, G,
                stream);
}

extern "C" int dpa_gn_silu_film_bwd_bf16(const void* x, const void* dout, const float* gamma,
                                         const float* beta, const void* film_wb,
                                         const float* mean, const float* rstd, void* dx,
                                         float* dgamma, float* dbeta, void* dfilm_wb,
                                         void* workspace, int64_t workspace_bytes, int N, int HW,
                                         int C, int G, void* stream) {
  if (!film_wb || !dfilm_wb) return DPA_ERR_NULL;
  return gn_bwd(x, dout, gamma, beta, nullptr, nullptr, film_wb, mean, rstd, dx, dgamma, dbeta,
                nullptr, nullptr, dfilm_wb, workspace, workspace_bytes, N, HW, C, G, stream);
}

extern "C" int dpa_gn_silu_bwd_ex(const void* x, int x_dtype, const void* dout, const float* gamma,
                                  const float* beta, const float* film_scale,
                                  const float* film_shift, const void* film_wb, const float* mean,
                                  const float* rstd, void* dx, const void* dx_add,
                                  int dx_add_dtype, float* dgamma,
                                  float* dbeta, float* dfilm_scale, float* dfilm_shift,
                                  void* dfilm_wb, void* workspace, int64_t workspace_bytes, int N,
                                  int HW, int C, int G, const void* drop_seed, float drop_p,
                                  void* stream) {
  if (x_dtype != DPA_DTYPE_BF16 && x_dtype != DPA_DTYPE_F32) return DPA_ERR_SHAPE;
  if (film_wb && film_scale) return DPA_ERR_SHAPE;
  // the added gradient is x's dtype, or bf16 beside an fp32 x; nothing else is read
  if (dx_add && dx_add_dtype != DPA_DTYPE_BF16 && dx_add_dtype != DPA_DTYPE_F32)
    return DPA_ERR_SHAPE;
  if (dx_add && x_dtype == DPA_DTYPE_BF16 && dx_add_dtype != DPA_DTYPE_BF16)
    return DPA_ERR_SHAPE;
  return gn_bwd(x, dout, gamma, beta, film_scale, film_shift, film_wb, mean, rstd, dx, dgamma,
                dbeta, dfilm_scale, dfilm_shift, dfilm_wb, workspace, workspace_bytes, N, HW, C, G,
                stream, x_dtype == DPA_DTYPE_F32, drop_seed, drop_p, dx_add,
                dx_add_dtype == DPA_DTYPE_BF16);
}

extern "C" int dpa_gn_silu_fp8_partials(int N, int HW, int C, int G) {
  if (!gn_shape_ok(N, HW, C, G)) return 0;
  const int64_t nb = gn_q_blocks(N, HW, C);
  return nb <= INT32_MAX ? (int)nb : 0;
}

extern "C" int dpa_gn_silu_fwd_fp8(const void* x, int x_dtype, const float* gamma,
                                   const float* beta, const float* film_scale,
                                   const float* film_shift, const void* film_wb, void* q,
                                   const float* q_scale, uint32_t* q_partials,
                                   int q_partials_cap, uint32_t* q_count, float* mean,
                                   float* rstd, void* workspace, int64_t workspace_bytes, int N,
                                   int HW, int C, int G, float eps, const void* drop_seed,
                                   float drop_p, void* x_bf16, void* stream) {
  if (x_dtype != DPA_DTYPE_BF16 && x_dtype != DPA_DTYPE_F32) return DPA_ERR_SHAPE;
  if (film_wb && film_scale) return DPA_ERR_SHAPE;
  if (!q) return DPA_ERR_NULL;
  if (gn_shape_ok(N, HW, C, G) && workspace_bytes < gn_fwd_workspace(N, HW, G))
    return DPA_ERR_WORKSPACE;
  if (workspace_bytes > 0 && !workspace) return DPA_ERR_WORKSPACE;
  if (!aligned(workspace, 8)) return DPA_ERR_ALIGN;
  const GnQOut qo{q, q_scale, q_partials, q_partials_cap, q_count};
  return gn_fwd(x, gamma, beta, film_scale, film_shift, film_wb, nullptr, mean, rstd, N, HW, C,
                G, eps, stream, workspace, workspace_bytes, x_dtype == DPA_DTYPE_F32, drop_seed,
                drop_p, x_bf16, &qo);
}

extern "C" int dpa_gn_silu_fwd_fp8_amax(const void* x, int x_dtype, const float* gamma,
                                        const float* beta, const float* film_scale,
                                        const float* film_shift, const void* film_wb, void* q,
                                        const float* q_scale, uint32_t* q_partials,
                                        int q_partials_cap, uint32_t* q_count, float* mean,
                                        float* rstd, void* workspace, int64_t workspace_bytes,
                                        int N, int HW, int C, int G, float eps,
                                        const void* drop_seed, float drop_p, void* x_bf16,
                                        uint32_t* xb_partials, int xb_partials_cap,
                                        void* stream) {
  if (x_dtype != DPA_DTYPE_BF16 && x_dtype != DPA_DTYPE_F32) return DPA_ERR_SHAPE;
  if (film_wb && film_scale) return DPA_ERR_SHAPE;
  if (!q || !xb_partials) return DPA_ERR_NULL;
  if (gn_shape_ok(N, HW, C, G) && workspace_bytes < gn_fwd_workspace(N, HW, G))
    return DPA_ERR_WORKSPACE;
  if (workspace_bytes > 0 && !workspace) return DPA_ERR_WORKSPACE;
  if (!aligned(workspace, 8)) return DPA_ERR_ALIGN;
  const GnQOut qo{q, q_scale, q_partials, q_partials_cap, q_count};
  return gn_fwd(x, gamma, beta, film_scale, film_shift, film_wb, nullptr, mean, rstd, N, HW, C,
                G, eps, stream, workspace, workspace_bytes, x_dtype == DPA_DTYPE_F32, drop_seed,
                drop_p, x_bf16, &qo, xb_partials, xb_partials_cap);
}

extern "C" int dpa_gn_silu_bwd_fp8(const void* x, const void* dout, const float* gamma,
                                   const float* beta, const float* film_scale,
                                   const float* film_shift, const void* film_wb,
                                   const float* mean, const float* rstd, void* dxq,
                                   const float* dx_scale, uint32_t* dx_partials,
                                   int dx_partials_cap, uint32_t* dx_count, float* dgamma,
                                   float* dbeta, float* dfilm_scale, float* dfilm_shift,
                                   void* dfilm_wb, void* workspace, int64_t workspace_bytes,
                                   int N, int HW, int C, int G, const void* drop_seed,
                                   float drop_p, void* stream) {
  if (film_wb && film_scale) return DPA_ERR_SHAPE;
  if (!dxq) return DPA_ERR_NULL;
  const GnQOut qo{dxq, dx_scale, dx_partials, dx_partials_cap, dx_count};
  return gn_bwd(x, dout, gamma, beta, film_scale, film_shift, film_wb, mean, rstd, dxq, dgamma,
                dbeta, dfilm_scale, dfilm_shift, dfilm_wb, workspace, workspace_bytes, N, HW, C, G,
                stream, false, drop_seed, drop_p, nullptr, false, &qo);
}

// ---- a decoder stage's first GroupNorm+SiLU fused with the upsample-and-concatenate before
// it (diffusion/unet.py:379-382 and :151): x = cat([up2(a), h], channels), read from a (bf16)
// and h (bf16, or fp32 at 16x16), NHWC, instead of the fp32 concatenation; the backward
// writes the gradients of a and h instead of the concatenation's. The resident forms of
// 32x32 images (64 pixel lanes x 16 pixels, h bf16) and 16x16 images (32 x 8). ----

static int upcat_gn_check(const void* a, const void* h, int h_dtype, int N, int H, int W,
                          int Ca, int Ch, int G) {
  if (!a || !h) return DPA_ERR_NULL;
  if (N <= 0 || H <= 0 || W <= 0 || Ca <= 0 || Ch <= 0) return DPA_ERR_SIZE;
  if (h_dtype != DPA_DTYPE_BF16 && h_dtype != DPA_DTYPE_F32) return DPA_ERR_SHAPE;
  const bool s32 = H == 32 && W == 32 && h_dtype == DPA_DTYPE_BF16;
  const bool s16 = H == 16 && W == 16;
  if (!(s32 || s16) || Ca % kSlab != 0 || Ch % kSlab != 0 ||
      !gn_shape_ok(N, H * W, Ca + Ch, G))
    return DPA_ERR_SHAPE;
  if ((int64_t)N * H * W * (Ca + Ch) > 0x7fffffffLL) return DPA_ERR_SIZE;
  if (!aligned(a, 16) || !aligned(h, 16)) return DPA_ERR_ALIGN;
  return DPA_OK;
}

extern "C" int dpa_upcat_gn_silu_fwd(const void* a, const void* h, int h_dtype, int N, int H,
                                     int W, int Ca, int Ch, const float* gamma,
                                     const float* beta, void* out, void* q,
                                     const float* q_scale, uint32_t* q_partials,
                                     int q_partials_cap, uint32_t* q_count, float* mean,
                                     float* rstd, void* x_bf16, uint32_t* xb_partials,
                                     int xb_partials_cap, int G, float eps, void* stream) {
  const int st0 = upcat_gn_check(a, h, h_dtype, N, H, W, Ca, Ch, G);
  if (st0 != DPA_OK) return st0;
  if (!gamma || !beta || !mean || !rstd || (!out && !q)) return DPA_ERR_NULL;
  if (out && q) return DPA_ERR_SHAPE;  // one output: bf16 or e4m3
  if (xb_partials && !x_bf16) return DPA_ERR_NULL;
  if (!aligned(out, 16) || !aligned(x_bf16, 16) || !aligned(xb_partials, 4)) return DPA_ERR_ALIGN;
  const int C = Ca + Ch, HW = H * W;
  GnArgs g{};
  g.x = h;  // (not read: the kernel reads cat_a and cat_h)
  g.cat_a = (const uint16_t*)a;
  g.cat_h = (const uint16_t*)h;
  g.cat_ca = Ca;
  g.cat_w = W;
  g.cat_hf = h_dtype == DPA_DTYPE_F32;
  g.gamma = gamma;
  g.beta = beta;
  g.out = out;
  g.mean = mean;
  g.rstd = rstd;
  g.x_bf16 = (uint16_t*)x_bf16;
  g.N = N; g.HW = HW; g.C = C; g.G = G; g.cpg = C / G; g.eps = eps;
  const int64_t nblk = gn_q_blocks(N, HW, C);
  if (xb_partials) {
    if (xb_partials_cap < nblk) return DPA_ERR_WORKSPACE;
    g.xb_part = xb_partials;
  }
  if (q) {
    const GnQOut qo{q, q_scale, q_partials, q_partials_cap, q_count};
    const int qst = gn_set_q(g, &qo, nblk);
    if (qst != DPA_OK) return qst;
    g.out = q;  // not written: the kernel stores through g.q
  }
  dim3 grid((unsigned)(C / kSlab), (unsigned)N);
  hipStream_t s = (hipStream_t)stream;
  if (H == 32)
    gn_res_fwd_kernel<64, 16, false, false, false, true><<<grid, 8 * 64, 0, s>>>(g);
  else
    gn_res_fwd_kernel<32, 8, false, true, false, true><<<grid, 8 * 32, 0, s>>>(g);
  return launch_status();
}

extern "C" int dpa_upcat_gn_silu_bwd(const void* a, const void* h, int h_dtype, int N, int H,
                                     int W, int Ca, int Ch, const void* dout, const float* gamma,
                                     const float* beta, const float* mean, const float* rstd,
                                     const void* dx_add, void* ga, void* gh, float* dgamma,
                                     float* dbeta, void* workspace, int64_t workspace_bytes,
                                     int G, void* stream) {
  const int st0 = upcat_gn_check(a, h, h_dtype, N, H, W, Ca, Ch, G);
  if (st0 != DPA_OK) return st0;
  if (!dout || !gamma || !beta || !mean || !rstd || !ga || !gh || !dgamma || !dbeta)
    return DPA_ERR_NULL;
  const int C = Ca + Ch, HW = H * W;
  if (!workspace || workspace_bytes < (int64_t)2 * N * C * 4) return DPA_ERR_WORKSPACE;
  if (!aligned(dout, 16) || !aligned(dx_add, 16) || !aligned(ga, 16) || !aligned(gh, 16) ||
      !aligned(workspace, 4))
    return DPA_ERR_ALIGN;
  GnArgs g{};
  g.x = h;  // (not read: the kernel reads cat_a and cat_h)
  g.cat_a = (const uint16_t*)a;
  g.cat_h = (const uint16_t*)h;
  g.cat_ca = Ca;
  g.cat_w = W;
  g.cat_hf = h_dtype == DPA_DTYPE_F32;
  g.cat_ga = (uint16_t*)ga;
  g.cat_gh = gh;
  g.dout = (const uint16_t*)dout;
  g.gamma = gamma;
  g.beta = beta;
  g.mean = const_cast<float*>(mean);
  g.rstd = const_cast<float*>(rstd);
  g.part = (float*)workspace;
  g.dx_add = dx_add;
  g.dx_add_bf16 = 1;
  g.N = N; g.HW = HW; g.C = C; g.G = G; g.cpg = C / G; g.eps = 0.f;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid((unsigned)(C / kSlab), (unsigned)N);
  if (H == 32)
    gn_res_bwd_kernel<64, 16, false, false, false, true><<<grid, 8 * 64, 0, s>>>(g);
  else
    gn_res_bwd_kernel<32, 8, false, true, false, true><<<grid, 8 * 32, 0, s>>>(g);
  int st = launch_status();
  if (st != DPA_OK) return st;
  gn_param_reduce_kernel<<<(unsigned)ceil_div(C, 64), 64 * kPrSlices, 0, s>>>(
      (const float*)workspace, dgamma, dbeta, N, C);
  return launch_status();
}
