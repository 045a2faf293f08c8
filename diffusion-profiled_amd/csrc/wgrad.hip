// FP8 convolution weight gradient on gfx950 MFMA.
//
// Reference: diffusion/fp8_kernels.py
//   transpose_fp8_2d_kernel     :321-337  (dy pre-transpose; not needed here)
//   conv2d_dw_fp8_kernel        :340-443  -> wgrad_partial_kernel
//   conv2d_dw_reduce_fp8_kernel :446-468  -> wgrad_reduce_kernel
//   conv2d_bwd_weight_fp8_prequantized :723-808 -> dpa_conv2d_wgrad_fp8
//
// GEMM view, per tap: D[ci][co] = sum over output pixels of x[shifted pix][ci] * dy[pix][co].
// The reduction runs over pixels, the strided dimension of both NHWC operands. Each K-step
// DMAs a 128-pixel x 128-channel block of each operand into LDS in its natural layout
// (global_load_lds, 16 B per lane; padding taps read a zero page), and the MFMA fragments are
// formed with ds_read_b64_tr_b8: a 16-lane group pointing at an 8-pixel x 16-channel block
// receives, in lane j, the 8 pixels of channel j. No transposed copy touches HBM or VALU.
//
// Workgroup tile: 128 input channels x 128 output channels of one tap; 4 waves (2 x 2) of
// 64 x 64. Pixels are split over workgroups (split-K), ordered so the workgroups that read
// one pixel range (all taps and channel tiles) share an XCD and its L2. Every split writes
// an fp32 partial tile (through LDS, as contiguous 512-B rows); the reduce kernel sums the
// splits in index order, scales by RN32(sx * sdy) and rounds to bf16.
#include "dpa_common.hpp"

namespace dpa {

constexpr int kWgThreads = 256;
constexpr int kWgTile = 128;                       // channels per tile side, pixels per K-step
constexpr int kWgOperandBytes = kWgTile * kWgTile;  // 16 KB
constexpr int kWgStageBytes = 2 * kWgOperandBytes;  // x block then dy block
constexpr int kWgLoads = kWgOperandBytes / 16 / kWgThreads;  // 4 DMA per operand per thread
constexpr int kWgPPitch = kWgTile * 4 + 16;  // fp32 partial-tile row pitch in LDS (bytes)

__shared__ __attribute__((aligned(1024))) uint8_t wg_smem[3 * kWgStageBytes];
static_assert(kWgTile * kWgPPitch <= 3 * kWgStageBytes, "partial tile must fit in LDS");

__device__ __attribute__((aligned(64))) uint8_t wg_zero16[64];

// Row r (a pixel, 128 B) keeps its 16-B granule g at g ^ wswz(r): conflict-free for the
// transpose reads (8 rows per 16-lane group, 4 groups at row offsets of 32).
__device__ __forceinline__ int wswz(int row) { return ((row >> 1) ^ (row >> 4)) & 7; }

#define WG_LDS(p) ((__attribute__((address_space(3))) void*)(p))

struct WgradArgs {
  const uint8_t* x;   // [N][H][W][Cin]
  const uint8_t* dy;  // [N][P][Q][Cout]
  float* partial;     // [splits][Cout][T*Cin]
  int N, H, W, Cin, Cout, R, S, stride, pad, P, Q;
  int npix, nchunks, splits;
  int ci_tiles, co_tiles, taps;
  int total, per_xcd;
  FastDiv divQ, divP;
};

template <int ST>
__device__ __forceinline__ void wg_issue(const WgradArgs& p, int chunk, int ci0, int co0, int kr,
                                         int ks, int wave, int lane) {
  uint8_t* st = wg_smem + ST * kWgStageBytes;
#pragma unroll
  for (int j = 0; j < kWgLoads; ++j) {
    const int row = wave * 32 + 8 * j + (lane >> 3);
    const int g = (lane & 7) ^ wswz(row);
    const int pix = chunk * kWgTile + row;
    const uint8_t* xs = wg_zero16;
    const uint8_t* ds = wg_zero16;
    if (pix < p.npix) {
      ds = p.dy + (uint32_t)(pix * p.Cout + co0 + g * 16);
      const uint32_t t = fdiv((uint32_t)pix, p.divQ);
      const int q = pix - (int)t * p.Q;
      const uint32_t n = fdiv(t, p.divP);
      const int pp = (int)t - (int)n * p.P;
      const int ih = pp * p.stride + kr - p.pad;
      const int iw = q * p.stride + ks - p.pad;
      if ((unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W)
        xs = p.x + (uint32_t)((((int)n * p.H + ih) * p.W + iw) * p.Cin + ci0 + g * 16);
    }
    __builtin_amdgcn_global_load_lds(xs, WG_LDS(st + (wave * 32 + 8 * j) * kWgTile), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(ds, WG_LDS(st + kWgOperandBytes + (wave * 32 + 8 * j) * kWgTile),
                                     16, 0, 0);
  }
}

typedef int v2i __attribute__((ext_vector_type(2)));

// 32 pixels (K) x 1 channel per lane: lane l -> channel row (l & 15) of the 16-channel
// group starting at granule G, pixels [32*(l>>4), +32), via four 8-pixel transpose reads.
__device__ __forceinline__ v8i ld_frag_tr(const uint8_t* base, int G, int lane) {
  const int k = lane & 15, q = lane >> 4;
  v8i f;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int row = 32 * q + 8 * s + (k >> 1);
    const uint8_t* a = base + row * kWgTile + ((G ^ wswz(row)) * 16) + 8 * (k & 1);
    const v2i v = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
        (v2i __attribute__((address_space(3)))*)(a));
    f[2 * s] = v.x;
    f[2 * s + 1] = v.y;
  }
  return f;
}

template <int ST>
__device__ __forceinline__ void wg_step(const WgradArgs& p, int c, int c_end, int ci0, int co0,
                                        int kr, int ks, int wave, int lane, int wc, int wo,
                                        v4f (&acc)[4][4]) {
  __syncthreads();  // this stage's DMA landed (the fence waits for it) and is visible to all
  const uint8_t* sx = wg_smem + ST * kWgStageBytes;
  const uint8_t* sd = sx + kWgOperandBytes;
  v8i xf[4], df[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) xf[i] = ld_frag_tr(sx, wc * 4 + i, lane);
#pragma unroll
  for (int i = 0; i < 4; ++i) df[i] = ld_frag_tr(sd, wo * 4 + i, lane);
  if (c + 2 < c_end) wg_issue<(ST + 2) % 3>(p, c + 2, ci0, co0, kr, ks, wave, lane);
  // D rows = input channels, D cols = output channels
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = mfma16x16x128_e4m3(xf[i], df[j], acc[i][j]);
}

__global__ __launch_bounds__(kWgThreads, 1) void wgrad_partial_kernel(const WgradArgs p) {
  // XCD-aware order: logical workgroup index = split-major, so the workgroups reading one
  // pixel range are consecutive and land on the same XCD (hardware deals round-robin).
  const int logical = (blockIdx.x & 7) * p.per_xcd + (blockIdx.x >> 3);
  if (logical >= p.total) return;
  const int per_split = p.ci_tiles * p.co_tiles * p.taps;
  const int split = logical / per_split;
  int rem = logical - split * per_split;
  const int tap = rem / (p.ci_tiles * p.co_tiles);
  rem -= tap * (p.ci_tiles * p.co_tiles);
  const int ci0 = (rem % p.ci_tiles) * kWgTile;
  const int co0 = (rem / p.ci_tiles) * kWgTile;
  const int kr = tap / p.S, ks = tap - (tap / p.S) * p.S;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wc = wave & 1;   // input-channel half (D rows)
  const int wo = wave >> 1;  // output-channel half (D cols)

  const int c_begin = (int)(((int64_t)p.nchunks * split) / p.splits);
  const int c_end = (int)(((int64_t)p.nchunks * (split + 1)) / p.splits);

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  if (c_begin < c_end) wg_issue<0>(p, c_begin, ci0, co0, kr, ks, wave, lane);
  if (c_begin + 1 < c_end) wg_issue<1>(p, c_begin + 1, ci0, co0, kr, ks, wave, lane);
  for (int c = c_begin; c < c_end; c += 3) {
    wg_step<0>(p, c, c_end, ci0, co0, kr, ks, wave, lane, wc, wo, acc);
    if (c + 1 < c_end) wg_step<1>(p, c + 1, c_end, ci0, co0, kr, ks, wave, lane, wc, wo, acc);
    if (c + 2 < c_end) wg_step<2>(p, c + 2, c_end, ci0, co0, kr, ks, wave, lane, wc, wo, acc);
  }

  // partial[split][co][tap*Cin + ci]: stage [co][ci] fp32 in LDS, then 512-B row stores
  __syncthreads();
  const int frow = lane & 15, fq = lane >> 4;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int co = wo * 64 + j * 16 + frow;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ci = wc * 64 + i * 16 + 4 * fq;
      *reinterpret_cast<v4f*>(wg_smem + co * kWgPPitch + ci * 4) = acc[i][j];
    }
  }
  __syncthreads();
  const int64_t kk = (int64_t)p.taps * p.Cin;
  float* base = p.partial + (int64_t)split * p.Cout * kk + (int64_t)tap * p.Cin + ci0;
  constexpr int kChunks = kWgTile * 4 / 16;            // 32 x 16 B per co row
  constexpr int kRowsPerPass = kWgThreads / kChunks;  // 8
  const int ch = threadIdx.x % kChunks;
#pragma unroll 4
  for (int r0 = 0; r0 < kWgTile; r0 += kRowsPerPass) {
    const int co = r0 + threadIdx.x / kChunks;
    *reinterpret_cast<v4f*>(base + (int64_t)(co0 + co) * kk + ch * 4) =
        *reinterpret_cast<const v4f*>(wg_smem + co * kWgPPitch + ch * 16);
  }
}

// dw[e] = bf16( RN32(sum_{s in order} partial[s][e]) * RN32(sx * sdy) ), 4 elements/thread.
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(const float* __restrict__ partial,
                                                           uint16_t* __restrict__ dw,
                                                           const float* __restrict__ sx,
                                                           const float* __restrict__ sdy,
                                                           int64_t total, int splits) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= total) return;
  const float scale = sx[0] * sdy[0];
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < splits; ++s) {
    const v4f v = *reinterpret_cast<const v4f*>(partial + (int64_t)s * total + i);
    acc = acc + v;
  }
  uint2 o;
  o.x = f32_to_bf16_bits(acc[0] * scale) | (f32_to_bf16_bits(acc[1] * scale) << 16);
  o.y = f32_to_bf16_bits(acc[2] * scale) | (f32_to_bf16_bits(acc[3] * scale) << 16);
  *reinterpret_cast<uint2*>(dw + i) = o;
}

static bool wgrad_shape_ok(int N, int H, int W, int Cin, int Cout, int R, int S, int stride,
                           int pad) {
  if (N <= 0 || H <= 0 || W <= 0 || Cin <= 0 || Cout <= 0) return false;
  if (Cin % kWgTile != 0 || Cout % kWgTile != 0) return false;
  const bool k3 = (R == 3 && S == 3 && pad == 1 && (stride == 1 || stride == 2));
  const bool k1 = (R == 1 && S == 1 && pad == 0 && stride == 1);
  return k3 || k1;
}

struct WgradPlan {
  int P, Q, npix, nchunks, tiles, splits;
};

static WgradPlan plan_wgrad(int N, int H, int W, int Cin, int Cout, int R, int S, int stride,
                            int pad, int split_k) {
  WgradPlan pl;
  pl.P = (H + 2 * pad - R) / stride + 1;
  pl.Q = (W + 2 * pad - S) / stride + 1;
  pl.npix = N * pl.P * pl.Q;
  pl.nchunks = (int)ceil_div(pl.npix, kWgTile);
  pl.tiles = (Cin / kWgTile) * (Cout / kWgTile) * R * S;
  if (split_k > 0) {
    pl.splits = split_k;
  } else {
    // one round of workgroups over the 256 CUs, at least 4 K-steps per split
    int s = 256 / pl.tiles;
    if (s < 1) s = 1;
    int maxs = pl.nchunks / 4;
    if (maxs < 1) maxs = 1;
    pl.splits = s < maxs ? s : maxs;
  }
  if (pl.splits > pl.nchunks) pl.splits = pl.nchunks;
  return pl;
}

}  // namespace dpa

using namespace dpa;

extern "C" int64_t dpa_conv2d_wgrad_workspace_bytes(int N, int H, int W, int Cin, int Cout,
                                                    int R, int S, int stride, int pad,
                                                    int split_k) {
  if (!wgrad_shape_ok(N, H, W, Cin, Cout, R, S, stride, pad)) return 0;
  WgradPlan pl = plan_wgrad(N, H, W, Cin, Cout, R, S, stride, pad, split_k);
  return (int64_t)pl.splits * Cout * R * S * Cin * 4;
}

extern "C" int dpa_conv2d_wgrad_fp8(const void* xq, const void* dyq, const float* x_scale,
                                    const float* dy_scale, void* dw, void* workspace,
                                    int64_t workspace_bytes, int N, int H, int W, int Cin,
                                    int Cout, int R, int S, int stride, int pad, int split_k,
                                    void* stream) {
  if (!xq || !dyq || !x_scale || !dy_scale || !dw) return DPA_ERR_NULL;
  if (!wgrad_shape_ok(N, H, W, Cin, Cout, R, S, stride, pad)) return DPA_ERR_SHAPE;
  if (split_k < 0) return DPA_ERR_SIZE;
  WgradPlan pl = plan_wgrad(N, H, W, Cin, Cout, R, S, stride, pad, split_k);
  const int64_t need = (int64_t)pl.splits * Cout * R * S * Cin * 4;
  if (!workspace || workspace_bytes < need) return DPA_ERR_WORKSPACE;
  if (!aligned(xq, 16) || !aligned(dyq, 16) || !aligned(workspace, 16) || !aligned(dw, 8))
    return DPA_ERR_ALIGN;
  // 32-bit byte offsets inside the kernel
  if ((int64_t)N * H * W * Cin > 0x7fffffff || (int64_t)pl.npix * Cout > 0x7fffffff)
    return DPA_ERR_SIZE;
  hipStream_t s = (hipStream_t)stream;
  WgradArgs a{};
  a.x = (const uint8_t*)xq;
  a.dy = (const uint8_t*)dyq;
  a.partial = (float*)workspace;
  a.N = N; a.H = H; a.W = W; a.Cin = Cin; a.Cout = Cout; a.R = R; a.S = S;
  a.stride = stride; a.pad = pad; a.P = pl.P; a.Q = pl.Q;
  a.npix = pl.npix; a.nchunks = pl.nchunks; a.splits = pl.splits;
  a.ci_tiles = Cin / kWgTile;
  a.co_tiles = Cout / kWgTile;
  a.taps = R * S;
  a.total = pl.tiles * pl.splits;
  a.per_xcd = (int)ceil_div(a.total, 8);
  a.divQ = make_fastdiv((uint32_t)pl.Q);
  a.divP = make_fastdiv((uint32_t)pl.P);
  wgrad_partial_kernel<<<(unsigned)(a.per_xcd * 8), kWgThreads, 0, s>>>(a);
  int st = launch_status();
  if (st != DPA_OK) return st;
  const int64_t total = (int64_t)Cout * R * S * Cin;
  wgrad_reduce_kernel<<<(unsigned)ceil_div(total, 1024), 256, 0, s>>>(
      (const float*)workspace, (uint16_t*)dw, x_scale, dy_scale, total, pl.splits);
  return launch_status();
}
