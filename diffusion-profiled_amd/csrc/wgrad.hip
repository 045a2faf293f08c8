// FP8 convolution weight gradient on gfx950 MFMA.
//
// Reference: diffusion/fp8_kernels.py
//   transpose_fp8_2d_kernel     :321-337  (dy pre-transpose; not needed here)
//   conv2d_dw_fp8_kernel        :340-443  -> wgrad_partial_kernel
//   conv2d_dw_reduce_fp8_kernel :446-468  -> wgrad_reduce_kernel
//   conv2d_bwd_weight_fp8_prequantized :723-808 -> dpa_conv2d_wgrad_fp8
//
// GEMM view: D[ci][co] (per tap) = sum over output pixels of x[shifted pix][ci] * dy[pix][co].
// The reduction runs over pixels, which is the strided dimension of both NHWC operands, so
// each K-step loads a 128-pixel x 128-channel block of each operand with 16-B row loads and
// transposes it in registers (4x4 byte blocks, v_perm_b32) while writing it to LDS as
// [channel][pixel]; the MFMA then reads 32 contiguous pixels per lane. No transposed copy
// of dy or x ever touches HBM.
//
// Workgroup tile: 128 input channels x 128 output channels of one tap; 4 waves (2 x 2) of
// 64 x 64. The pixel range is split over gridDim.z (split-K); every split writes an fp32
// partial tile, and the reduce kernel sums splits in index order, scales and casts to bf16.
#include "dpa_common.hpp"

namespace dpa {

constexpr int kWgThreads = 256;
constexpr int kWgTile = 128;  // channels per tile side and pixels per K-step

// LDS row swizzle: rows are 128 B = 8 granules of 16 B.
__device__ __forceinline__ int wswz(int row) { return (row ^ (row >> 4)) & 7; }

struct WgradArgs {
  const uint8_t* x;   // [N][H][W][Cin]
  const uint8_t* dy;  // [N][P][Q][Cout]
  float* partial;     // [splits][Cout][T*Cin]
  int N, H, W, Cin, Cout, R, S, stride, pad, P, Q;
  int npix;           // N*P*Q
  int nchunks;        // ceil(npix / 128)
  int splits;
};

// 4 rows (pixels) x 16 bytes (channels) -> 16 dwords, dword j = bytes j of the 4 rows.
__device__ __forceinline__ void transpose4x16(const uint4 (&r)[4], uint32_t (&o)[16]) {
  const uint32_t a[4] = {r[0].x, r[0].y, r[0].z, r[0].w};
  const uint32_t b[4] = {r[1].x, r[1].y, r[1].z, r[1].w};
  const uint32_t c[4] = {r[2].x, r[2].y, r[2].z, r[2].w};
  const uint32_t d[4] = {r[3].x, r[3].y, r[3].z, r[3].w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t lo01 = perm_b32(b[k], a[k], 0x05010400u);  // a0 b0 a1 b1
    const uint32_t hi01 = perm_b32(b[k], a[k], 0x07030602u);  // a2 b2 a3 b3
    const uint32_t lo23 = perm_b32(d[k], c[k], 0x05010400u);  // c0 d0 c1 d1
    const uint32_t hi23 = perm_b32(d[k], c[k], 0x07030602u);  // c2 d2 c3 d3
    o[4 * k + 0] = perm_b32(lo23, lo01, 0x05040100u);         // a0 b0 c0 d0
    o[4 * k + 1] = perm_b32(lo23, lo01, 0x07060302u);         // a1 b1 c1 d1
    o[4 * k + 2] = perm_b32(hi23, hi01, 0x05040100u);         // a2 b2 c2 d2
    o[4 * k + 3] = perm_b32(hi23, hi01, 0x07060302u);         // a3 b3 c3 d3
  }
}

__global__ __launch_bounds__(kWgThreads) void wgrad_partial_kernel(const WgradArgs p) {
  // [buf][operand x|dy][128 rows (channels)][128 B (pixels)]
  __shared__ __attribute__((aligned(16))) uint8_t smem[2][2][kWgTile * kWgTile];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wc = wave & 1;   // input-channel half (D rows)
  const int wo = wave >> 1;  // output-channel half (D cols)

  const int ci_tiles = p.Cin / kWgTile;
  const int ci0 = (blockIdx.x % ci_tiles) * kWgTile;
  const int co0 = (blockIdx.x / ci_tiles) * kWgTile;
  const int tap = blockIdx.y;
  const int kr = tap / p.S, ks = tap % p.S;
  const int split = blockIdx.z;

  // pixel chunks [c_begin, c_end) of this split
  const int c_begin = (int)(((int64_t)p.nchunks * split) / p.splits);
  const int c_end = (int)(((int64_t)p.nchunks * (split + 1)) / p.splits);

  // load assignment: pixel quad pq (4 pixels), channel granule cg (16 channels)
  const int pq = tid >> 3;  // 0..31
  const int cg = tid & 7;   // 0..7

  uint4 rx[4], rd[4];
  auto load_step = [&](int chunk) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int pix = chunk * kWgTile + pq * 4 + e;
      uint4 vx = {0u, 0u, 0u, 0u}, vd = {0u, 0u, 0u, 0u};
      if (pix < p.npix) {
        vd = *reinterpret_cast<const uint4*>(p.dy + (int64_t)pix * p.Cout + co0 + cg * 16);
        const int q = pix % p.Q;
        const int t = pix / p.Q;
        const int pp = t % p.P;
        const int n = t / p.P;
        const int ih = pp * p.stride + kr - p.pad;
        const int iw = q * p.stride + ks - p.pad;
        if (ih >= 0 && ih < p.H && iw >= 0 && iw < p.W)
          vx = *reinterpret_cast<const uint4*>(
              p.x + (((int64_t)n * p.H + ih) * p.W + iw) * p.Cin + ci0 + cg * 16);
      }
      rx[e] = vx;
      rd[e] = vd;
    }
  };
  auto store_step = [&](int buf) {
    uint32_t tx[16], td[16];
    transpose4x16(rx, tx);
    transpose4x16(rd, td);
    uint8_t* sx = smem[buf][0];
    uint8_t* sd = smem[buf][1];
    const int gr = pq >> 2;        // granule within the 128-pixel row
    const int wi = (pq & 3) * 4;   // byte within granule
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int row = cg * 16 + j;
      const int off = row * kWgTile + ((gr ^ wswz(row)) * 16) + wi;
      *reinterpret_cast<uint32_t*>(sx + off) = tx[j];
      *reinterpret_cast<uint32_t*>(sd + off) = td[j];
    }
  };

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  const int frow = lane & 15;
  const int fq = lane >> 4;

  if (c_begin < c_end) {
    load_step(c_begin);
    store_step(0);
  }
  __syncthreads();

  for (int c = c_begin; c < c_end; ++c) {
    const int buf = (c - c_begin) & 1;
    if (c + 1 < c_end) load_step(c + 1);

    const uint8_t* sx = smem[buf][0];
    const uint8_t* sd = smem[buf][1];
    v8i xf[4], df[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = wc * 64 + i * 16 + frow;
      const int sw = wswz(row);
      const uint4 lo = *reinterpret_cast<const uint4*>(sx + row * kWgTile + ((2 * fq) ^ sw) * 16);
      const uint4 hi =
          *reinterpret_cast<const uint4*>(sx + row * kWgTile + ((2 * fq + 1) ^ sw) * 16);
      xf[i] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                  (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = wo * 64 + i * 16 + frow;
      const int sw = wswz(row);
      const uint4 lo = *reinterpret_cast<const uint4*>(sd + row * kWgTile + ((2 * fq) ^ sw) * 16);
      const uint4 hi =
          *reinterpret_cast<const uint4*>(sd + row * kWgTile + ((2 * fq + 1) ^ sw) * 16);
      df[i] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                  (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    }
    // D rows = input channels, D cols = output channels
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = mfma16x16x128_e4m3(xf[i], df[j], acc[i][j]);

    if (c + 1 < c_end) store_step(buf ^ 1);
    __syncthreads();
  }

  // partial[split][co][tap*Cin + ci]: lane holds 4 consecutive ci for one co -> float4
  const int64_t kk = (int64_t)p.R * p.S * p.Cin;
  float* base = p.partial + (int64_t)split * p.Cout * kk + (int64_t)tap * p.Cin;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int co = co0 + wo * 64 + j * 16 + frow;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ci = ci0 + wc * 64 + i * 16 + 4 * fq;
      *reinterpret_cast<v4f*>(base + (int64_t)co * kk + ci) = acc[i][j];
    }
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

static int default_splits(int tiles, int nchunks) {
  // one round of workgroups over the 256 CUs, at least 4 K-steps per split
  int s = 256 / (tiles > 0 ? tiles : 1);
  if (s < 1) s = 1;
  int maxs = nchunks / 4;
  if (maxs < 1) maxs = 1;
  if (s > maxs) s = maxs;
  return s;
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
  pl.splits = split_k > 0 ? split_k : default_splits(pl.tiles, pl.nchunks);
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
  hipStream_t s = (hipStream_t)stream;
  WgradArgs a{};
  a.x = (const uint8_t*)xq;
  a.dy = (const uint8_t*)dyq;
  a.partial = (float*)workspace;
  a.N = N; a.H = H; a.W = W; a.Cin = Cin; a.Cout = Cout; a.R = R; a.S = S;
  a.stride = stride; a.pad = pad; a.P = pl.P; a.Q = pl.Q;
  a.npix = pl.npix; a.nchunks = pl.nchunks; a.splits = pl.splits;
  dim3 grid((unsigned)((Cin / kWgTile) * (Cout / kWgTile)), (unsigned)(R * S),
            (unsigned)pl.splits);
  wgrad_partial_kernel<<<grid, kWgThreads, 0, s>>>(a);
  int st = launch_status();
  if (st != DPA_OK) return st;
  const int64_t total = (int64_t)Cout * R * S * Cin;
  wgrad_reduce_kernel<<<(unsigned)ceil_div(total, 1024), 256, 0, s>>>(
      (const float*)workspace, (uint16_t*)dw, x_scale, dy_scale, total, pl.splits);
  return launch_status();
}
