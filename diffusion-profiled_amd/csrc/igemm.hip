// FP8 implicit-GEMM convolution (forward and data-gradient) and FP8 GEMM on gfx950 MFMA.
//
// Reference: diffusion/fp8_kernels.py
//   conv2d_fwd_fp8_kernel  :142-247 (+ launcher :604-639)  -> dpa_conv2d_fwd_fp8
//   conv2d_dx_fp8_kernel   :250-318 (+ launcher :671-709)  -> dpa_conv2d_dgrad_fp8
//
// One kernel serves every case. The GEMM is
//   out[pix, co] = sum_{tap, c} act[pix shifted by tap, c] * wgt[co, tap, c]
// where the tap list (<= 9 entries) says, per tap, the input-pixel offset and which weight
// tap to use. Forward convs (stride 1 or 2, 3x3 or 1x1) use the natural tap list; the data
// gradient is the same kernel on dy with the weight transposed to [Cin][R][S][Cout] and
// mirrored offsets; stride-2 dgrad runs once per output parity class with only the taps
// that class touches; the linear is the 1x1 case with H = W = 1.
//
// Tile: 128 output pixels x 128 output channels per workgroup of 4 waves (2 x 2), each
// wave 64 x 64 = 4 x 4 MFMA 16x16x128 tiles. K advances 128 channels (one tap) per step.
// Operands are staged global -> registers -> LDS (double-buffered, one barrier per step);
// LDS rows are 128 B with the 16-B granules XOR-swizzled by (row & 7).
// Epilogue: out = bf16(RN32(acc * RN32(sa * sb)) [+ bias]) with 8-byte stores.
#include "dpa_common.hpp"

namespace dpa {

constexpr int kIgThreads = 256;
constexpr int kBM = 128;  // output pixels per workgroup
constexpr int kBN = 128;  // output channels per workgroup
constexpr int kBK = 128;  // K bytes per step (MFMA depth)
constexpr int kMaxTaps = 9;

struct IgemmArgs {
  const uint8_t* act;  // [N][Hi][Wi][C]
  const uint8_t* wgt;  // [Cout][T][C]
  uint16_t* out;       // bf16 [N][Ho][Wo][Cout]
  const float* sa;
  const float* sb;
  const float* bias;  // [Cout] or null
  int N, Hi, Wi, C, Cout, T;
  int Pg, Qg;  // output grid enumerated by this launch
  int Ho, Wo;
  int oy_step, oy_off, ox_step, ox_off;  // out pixel = (i*oy_step + oy_off, j*ox_step + ox_off)
  int iy_step, ix_step;                  // in pixel  = (i*iy_step + tap_dy, j*ix_step + tap_dx)
  int M;                                 // N * Pg * Qg
  int ntaps;
  int tap_dy[kMaxTaps], tap_dx[kMaxTaps], tap_w[kMaxTaps];
};

__device__ __forceinline__ int swz(int row, int granule) { return granule ^ (row & 7); }

__global__ __launch_bounds__(kIgThreads) void igemm_fp8_kernel(const IgemmArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2][(kBM + kBN) * kBK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave & 1;   // pixel half
  const int wn = wave >> 1;  // channel half

  const int m0 = blockIdx.x * kBM;
  const int n0 = blockIdx.y * kBN;

  // ---- per-thread load assignment: granule g of rows r0 + 32*i ----
  const int g = tid & 7;
  const int r0 = tid >> 3;
  constexpr int kRowsPerThread = kBM / 32;  // A and B both 128 rows
  int a_base[kRowsPerThread];               // n * Hi (or -1 if pixel out of range)
  int a_iy[kRowsPerThread], a_ix[kRowsPerThread];
#pragma unroll
  for (int i = 0; i < kRowsPerThread; ++i) {
    const int m = m0 + r0 + 32 * i;
    if (m < p.M) {
      const int j = m % p.Qg;
      const int t = m / p.Qg;
      const int ii = t % p.Pg;
      const int n = t / p.Pg;
      a_base[i] = n * p.Hi;
      a_iy[i] = ii * p.iy_step;
      a_ix[i] = j * p.ix_step;
    } else {
      a_base[i] = -1;
      a_iy[i] = 0;
      a_ix[i] = 0;
    }
  }

  const int kc_per_tap = p.C / kBK;
  const int nk = p.ntaps * kc_per_tap;
  const int64_t wrow = (int64_t)p.T * p.C;

  uint4 ra[kRowsPerThread], rb[kRowsPerThread];

  auto load_step = [&](int k) {
    const int t = k / kc_per_tap;
    const int c0 = (k - t * kc_per_tap) * kBK + g * 16;
    const int dy = p.tap_dy[t], dx = p.tap_dx[t];
#pragma unroll
    for (int i = 0; i < kRowsPerThread; ++i) {
      const int iy = a_iy[i] + dy, ix = a_ix[i] + dx;
      uint4 v = {0u, 0u, 0u, 0u};
      if (a_base[i] >= 0 && iy >= 0 && iy < p.Hi && ix >= 0 && ix < p.Wi) {
        const int64_t off = ((int64_t)(a_base[i] + iy) * p.Wi + ix) * p.C + c0;
        v = *reinterpret_cast<const uint4*>(p.act + off);
      }
      ra[i] = v;
    }
    const int64_t woff = (int64_t)p.tap_w[t] * p.C + c0;
#pragma unroll
    for (int i = 0; i < kRowsPerThread; ++i) {
      const int co = n0 + r0 + 32 * i;
      rb[i] = *reinterpret_cast<const uint4*>(p.wgt + (int64_t)co * wrow + woff);
    }
  };

  auto store_step = [&](int buf) {
    uint8_t* sa = smem[buf];
    uint8_t* sb = smem[buf] + kBM * kBK;
#pragma unroll
    for (int i = 0; i < kRowsPerThread; ++i) {
      const int row = r0 + 32 * i;
      *reinterpret_cast<uint4*>(sa + row * kBK + swz(row, g) * 16) = ra[i];
      *reinterpret_cast<uint4*>(sb + row * kBK + swz(row, g) * 16) = rb[i];
    }
  };

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  const int frow = lane & 15;
  const int fq = lane >> 4;

  load_step(0);
  store_step(0);
  __syncthreads();

  for (int k = 0; k < nk; ++k) {
    const int buf = k & 1;
    if (k + 1 < nk) load_step(k + 1);

    const uint8_t* sa = smem[buf];
    const uint8_t* sb = smem[buf] + kBM * kBK;
    v8i af[4], bf[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = wm * 64 + i * 16 + frow;
      const uint4 lo = *reinterpret_cast<const uint4*>(sa + row * kBK + swz(row, 2 * fq) * 16);
      const uint4 hi =
          *reinterpret_cast<const uint4*>(sa + row * kBK + swz(row, 2 * fq + 1) * 16);
      af[i] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                  (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = wn * 64 + i * 16 + frow;
      const uint4 lo = *reinterpret_cast<const uint4*>(sb + row * kBK + swz(row, 2 * fq) * 16);
      const uint4 hi =
          *reinterpret_cast<const uint4*>(sb + row * kBK + swz(row, 2 * fq + 1) * 16);
      bf[i] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                  (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    }
    // D rows = output channels (weight operand), D cols = pixels (activation operand)
#pragma unroll
    for (int ci = 0; ci < 4; ++ci)
#pragma unroll
      for (int pj = 0; pj < 4; ++pj) acc[ci][pj] = mfma16x16x128_e4m3(bf[ci], af[pj], acc[ci][pj]);

    if (k + 1 < nk) store_step(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue ----
  const float scale = p.sa[0] * p.sb[0];
#pragma unroll
  for (int pj = 0; pj < 4; ++pj) {
    const int m = m0 + wm * 64 + pj * 16 + frow;
    if (m >= p.M) continue;
    const int j = m % p.Qg;
    const int t = m / p.Qg;
    const int ii = t % p.Pg;
    const int n = t / p.Pg;
    const int oy = ii * p.oy_step + p.oy_off;
    const int ox = j * p.ox_step + p.ox_off;
    uint16_t* orow = p.out + (((int64_t)n * p.Ho + oy) * p.Wo + ox) * p.Cout;
#pragma unroll
    for (int ci = 0; ci < 4; ++ci) {
      const int co = n0 + wn * 64 + ci * 16 + 4 * fq;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = acc[ci][pj][e] * scale;
        if (p.bias) v[e] = v[e] + p.bias[co + e];
      }
      uint2 o;
      o.x = f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16);
      o.y = f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16);
      *reinterpret_cast<uint2*>(orow + co) = o;
    }
  }
}

// wt[ci][r][s][co] = w[co][r][s][ci] (e4m3 bytes): 32x32 byte tiles through LDS.
__global__ __launch_bounds__(256) void weight_transpose_kernel(const uint8_t* __restrict__ w,
                                                               uint8_t* __restrict__ wt,
                                                               int Cout, int T, int Cin) {
  __shared__ uint8_t tile[32][33];
  const int t = blockIdx.z;
  const int co0 = blockIdx.y * 32, ci0 = blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int r = ty; r < 32; r += 8) {
    const int co = co0 + r, ci = ci0 + tx;
    tile[r][tx] = (co < Cout && ci < Cin) ? w[((int64_t)co * T + t) * Cin + ci] : 0;
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const int ci = ci0 + r, co = co0 + tx;
    if (ci < Cin && co < Cout) wt[((int64_t)ci * T + t) * Cout + co] = tile[tx][r];
  }
}

static int launch_igemm(IgemmArgs& a, hipStream_t s) {
  if (a.M <= 0) return DPA_OK;
  dim3 grid((unsigned)ceil_div(a.M, kBM), (unsigned)(a.Cout / kBN));
  igemm_fp8_kernel<<<grid, kIgThreads, 0, s>>>(a);
  return launch_status();
}

static bool conv_shape_ok(int N, int H, int W, int Cin, int Cout, int R, int S, int stride,
                          int pad) {
  if (N <= 0 || H <= 0 || W <= 0 || Cin <= 0 || Cout <= 0) return false;
  if (Cin % kBK != 0 || Cout % kBN != 0) return false;
  const bool k3 = (R == 3 && S == 3 && pad == 1 && (stride == 1 || stride == 2));
  const bool k1 = (R == 1 && S == 1 && pad == 0 && stride == 1);
  return k3 || k1;
}

static void fill_common(IgemmArgs& a, const void* act, const void* wgt, void* out,
                        const float* sa, const float* sb, const float* bias) {
  a.act = (const uint8_t*)act;
  a.wgt = (const uint8_t*)wgt;
  a.out = (uint16_t*)out;
  a.sa = sa;
  a.sb = sb;
  a.bias = bias;
}

static int conv_fwd(const void* xq, const void* wq, const float* xs, const float* ws,
                    const float* bias, void* y, int N, int H, int W, int Cin, int Cout, int R,
                    int S, int stride, int pad, hipStream_t s) {
  IgemmArgs a{};
  fill_common(a, xq, wq, y, xs, ws, bias);
  const int P = (H + 2 * pad - R) / stride + 1;
  const int Q = (W + 2 * pad - S) / stride + 1;
  a.N = N; a.Hi = H; a.Wi = W; a.C = Cin; a.Cout = Cout; a.T = R * S;
  a.Pg = P; a.Qg = Q; a.Ho = P; a.Wo = Q;
  a.oy_step = 1; a.oy_off = 0; a.ox_step = 1; a.ox_off = 0;
  a.iy_step = stride; a.ix_step = stride;
  a.M = N * P * Q;
  a.ntaps = R * S;
  for (int r = 0; r < R; ++r)
    for (int c = 0; c < S; ++c) {
      const int t = r * S + c;
      a.tap_dy[t] = r - pad;
      a.tap_dx[t] = c - pad;
      a.tap_w[t] = t;
    }
  return launch_igemm(a, s);
}

// dx[n, h, w, ci] = sum_{r,s,co} dy[n, (h+pad-r)/st, (w+pad-s)/st, co] * w[co, r, s, ci]
// over the (r, s) for which the division is exact and in range.
static int conv_dgrad(const void* dyq, const void* wt, const float* dys, const float* ws,
                      void* dx, int N, int H, int W, int Cin, int Cout, int R, int S,
                      int stride, int pad, hipStream_t s) {
  const int P = (H + 2 * pad - R) / stride + 1;
  const int Q = (W + 2 * pad - S) / stride + 1;
  for (int ay = 0; ay < stride; ++ay)
    for (int ax = 0; ax < stride; ++ax) {
      IgemmArgs a{};
      fill_common(a, dyq, wt, dx, dys, ws, nullptr);
      a.N = N; a.Hi = P; a.Wi = Q; a.C = Cout; a.Cout = Cin; a.T = R * S;
      a.Pg = (H - ay + stride - 1) / stride;
      a.Qg = (W - ax + stride - 1) / stride;
      a.Ho = H; a.Wo = W;
      a.oy_step = stride; a.oy_off = ay; a.ox_step = stride; a.ox_off = ax;
      a.iy_step = 1; a.ix_step = 1;
      a.M = N * a.Pg * a.Qg;
      int nt = 0;
      for (int r = 0; r < R; ++r) {
        const int ey = ay + pad - r;
        if (((ey % stride) + stride) % stride != 0) continue;
        for (int c = 0; c < S; ++c) {
          const int ex = ax + pad - c;
          if (((ex % stride) + stride) % stride != 0) continue;
          // floor division of the exact multiples
          a.tap_dy[nt] = ey >= 0 ? ey / stride : -((-ey) / stride);
          a.tap_dx[nt] = ex >= 0 ? ex / stride : -((-ex) / stride);
          a.tap_w[nt] = r * S + c;
          ++nt;
        }
      }
      a.ntaps = nt;
      if (nt == 0 || a.M == 0) {
        // no tap reaches this class (cannot happen for the supported shapes)
        return DPA_ERR_SHAPE;
      }
      int st = launch_igemm(a, s);
      if (st != DPA_OK) return st;
    }
  return DPA_OK;
}

}  // namespace dpa

using namespace dpa;

extern "C" int dpa_conv2d_fwd_fp8(const void* xq, const void* wq, const float* x_scale,
                                  const float* w_scale, const float* bias, void* y, int N,
                                  int H, int W, int Cin, int Cout, int R, int S, int stride,
                                  int pad, void* stream) {
  if (!xq || !wq || !x_scale || !w_scale || !y) return DPA_ERR_NULL;
  if (!conv_shape_ok(N, H, W, Cin, Cout, R, S, stride, pad)) return DPA_ERR_SHAPE;
  if (!aligned(xq, 16) || !aligned(wq, 16) || !aligned(y, 8)) return DPA_ERR_ALIGN;
  return conv_fwd(xq, wq, x_scale, w_scale, bias, y, N, H, W, Cin, Cout, R, S, stride, pad,
                  (hipStream_t)stream);
}

extern "C" int64_t dpa_conv2d_dgrad_workspace_bytes(int Cin, int Cout, int R, int S) {
  return (int64_t)Cin * Cout * R * S;
}

extern "C" int dpa_weight_transpose_fp8(const void* wq, void* wq_t, int Cout, int R, int S,
                                        int Cin, void* stream) {
  if (!wq || !wq_t) return DPA_ERR_NULL;
  if (Cout <= 0 || Cin <= 0 || R <= 0 || S <= 0) return DPA_ERR_SIZE;
  dim3 grid((unsigned)ceil_div(Cin, 32), (unsigned)ceil_div(Cout, 32), (unsigned)(R * S));
  weight_transpose_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(
      (const uint8_t*)wq, (uint8_t*)wq_t, Cout, R * S, Cin);
  return launch_status();
}

extern "C" int dpa_conv2d_dgrad_fp8_wt(const void* dyq, const void* wq_t, const float* dy_scale,
                                       const float* w_scale, void* dx, int N, int H, int W,
                                       int Cin, int Cout, int R, int S, int stride, int pad,
                                       void* stream) {
  if (!dyq || !wq_t || !dy_scale || !w_scale || !dx) return DPA_ERR_NULL;
  // the dgrad GEMM reduces over Cout and produces Cin channels
  if (!conv_shape_ok(N, H, W, Cout, Cin, R, S, stride, pad)) return DPA_ERR_SHAPE;
  if (!aligned(dyq, 16) || !aligned(wq_t, 16) || !aligned(dx, 8)) return DPA_ERR_ALIGN;
  return conv_dgrad(dyq, wq_t, dy_scale, w_scale, dx, N, H, W, Cin, Cout, R, S, stride, pad,
                    (hipStream_t)stream);
}

extern "C" int dpa_conv2d_dgrad_fp8(const void* dyq, const void* wq, const float* dy_scale,
                                    const float* w_scale, void* dx, void* workspace,
                                    int64_t workspace_bytes, int N, int H, int W, int Cin,
                                    int Cout, int R, int S, int stride, int pad, void* stream) {
  if (!dyq || !wq || !dy_scale || !w_scale || !dx) return DPA_ERR_NULL;
  if (!conv_shape_ok(N, H, W, Cout, Cin, R, S, stride, pad)) return DPA_ERR_SHAPE;
  if (!workspace || workspace_bytes < dpa_conv2d_dgrad_workspace_bytes(Cin, Cout, R, S))
    return DPA_ERR_WORKSPACE;
  if (!aligned(dyq, 16) || !aligned(workspace, 16) || !aligned(dx, 8)) return DPA_ERR_ALIGN;
  int st = dpa_weight_transpose_fp8(wq, workspace, Cout, R, S, Cin, stream);
  if (st != DPA_OK) return st;
  return conv_dgrad(dyq, workspace, dy_scale, w_scale, dx, N, H, W, Cin, Cout, R, S, stride,
                    pad, (hipStream_t)stream);
}

extern "C" int dpa_gemm_fp8(const void* a, const void* b, const float* a_scale,
                            const float* b_scale, const float* bias, void* c, int M, int N,
                            int K, void* stream) {
  if (!a || !b || !a_scale || !b_scale || !c) return DPA_ERR_NULL;
  if (M <= 0 || N <= 0 || K <= 0) return DPA_ERR_SIZE;
  if (K % kBK != 0 || N % kBN != 0) return DPA_ERR_SHAPE;
  if (!aligned(a, 16) || !aligned(b, 16) || !aligned(c, 8)) return DPA_ERR_ALIGN;
  // a linear is a 1x1 convolution over M "pixels" of K channels
  return conv_fwd(a, b, a_scale, b_scale, bias, c, M, 1, 1, K, N, 1, 1, 1, 0,
                  (hipStream_t)stream);
}
