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
// Workgroup tile: 128 input channels x 128 output channels of one tap. Four consumer waves
// (2 x 2 of 64 x 64) run the MFMAs; four producer waves compute the DMA addresses and issue
// the DMAs into a 4-deep LDS ring, so address arithmetic overlaps the matrix pipe on every
// SIMD. Pixels are split over workgroups (split-K), ordered so the workgroups that read
// one pixel range (all taps and channel tiles) share an XCD and its L2. Every split writes
// an fp32 partial tile (through LDS, as contiguous 512-B rows); the reduce kernel sums the
// splits in index order, scales by RN32(sx * sdy) and rounds to bf16.
#include "dpa_common.hpp"

namespace dpa {

constexpr int kWgConsumers = 256;                  // 4 MFMA waves (2 x 2 of 64 x 64)
constexpr int kWgProducers = 256;                  // 4 DMA waves
constexpr int kWgThreads = kWgConsumers + kWgProducers;
constexpr int kWgTile = 128;                       // channels per tile side, pixels per K-step
constexpr int kWgOperandBytes = kWgTile * kWgTile;  // 16 KB
constexpr int kWgStageBytes = 2 * kWgOperandBytes;  // x block then dy block
constexpr int kWgLoads = kWgOperandBytes / 16 / kWgProducers;  // 4 DMA per operand per producer
constexpr int kWgPPitch = kWgTile * 4 + 16;  // fp32 partial-tile row pitch in LDS (bytes)

constexpr int kWgStages = 4;                         // LDS ring depth (DMA latency budget)

__shared__ __attribute__((aligned(1024))) uint8_t wg_smem[kWgStages * kWgStageBytes];
static_assert(kWgTile * kWgPPitch <= kWgStages * kWgStageBytes, "partial tile must fit in LDS");

__device__ __attribute__((aligned(64))) uint8_t wg_zero16[64];

// Row r (a pixel, 128 B) keeps its 16-B granule g at g ^ wswz(r): conflict-free for the
// transpose reads (8 rows per 16-lane group, 4 groups at row offsets of 32).
__device__ __forceinline__ int wswz(int row) { return ((row >> 1) ^ (row >> 4)) & 7; }

struct WgradArgs {
  const uint8_t* x;   // [N][H][W][Cin]
  const uint8_t* dy;  // [N][P][Q][Cout]
  float* partial;     // [splits][Cout][T*Cin]
  int N, H, W, Cin, Cout, R, S, stride, pad, P, Q;
  int npix, nchunks, splits;
  int ci_tiles, co_tiles, taps;
  int total, per_xcd;
  int dq, dpp;              // one chunk (kWgTile pixels) as a (p, q) increment (+ images)
  int x_step, x_cq, x_cp;   // x byte-offset change per chunk, and on a q / p wrap
  FastDiv divQ, divP;
};

constexpr int kWgLoadsPerStage = 2 * kWgLoads;  // x and dy DMAs per producer thread per stage

typedef int v2i __attribute__((ext_vector_type(2)));

// Transpose-read address tables. With k = lane & 15, q = lane >> 4, m = k >> 1, h = k & 1,
// fragment read s of granule G touches LDS row r = 32q + 8s + m at granule position
// G ^ wswz(r), and wswz(r) = L ^ C(s) with L = (m >> 1) ^ 2q (lane) and
// C(s) = ((s & 1) << 2) ^ (s >> 1). So the byte offset is T[G ^ C(s)] + 1024 s with
// T[v] = (32q + m) * 128 + 8h + 16 (v ^ L): eight per-lane values, and every read of the
// loop is one of them plus an immediate.
__device__ __forceinline__ constexpr int wg_c(int s) { return ((s & 1) << 2) ^ (s >> 1); }

__device__ __forceinline__ v8i ld_frag_tbl(const uint8_t* stage_op, const uint32_t (&T)[8], int i) {
  v8i f;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint8_t* a = stage_op + T[i ^ wg_c(s)] + 1024 * s;
    const v2i v = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
        (v2i __attribute__((address_space(3)))*)(a));
    f[2 * s] = v.x;
    f[2 * s + 1] = v.y;
  }
  return f;
}

// Per-thread DMA state: 4 LDS rows (pixels) of the current chunk, advanced one chunk per issue.
struct WgRows {
  int pix[kWgLoads], rp[kWgLoads], rq[kWgLoads], xo[kWgLoads];
  uint32_t dyo[kWgLoads];
};

template <int ST>
__device__ __forceinline__ void wg_issue(const WgradArgs& p, WgRows& r, bool live_step, int kr,
                                         int ks, uint32_t lds_wave, uint32_t dy_step) {
  const uint32_t st = LDS_ADDR(wg_smem) + ST * kWgStageBytes + lds_wave;
#pragma unroll
  for (int j = 0; j < kWgLoads; ++j) {
    // bitwise & (not &&): no short-circuit branches, only selects
    const bool live = live_step & (r.pix[j] < p.npix);
    const int ih = r.rp[j] * p.stride + kr - p.pad;
    const int iw = r.rq[j] * p.stride + ks - p.pad;
    const bool ok = live & ((unsigned)ih < (unsigned)p.H) & ((unsigned)iw < (unsigned)p.W);
    const uint8_t* xs = ok ? p.x + r.xo[j] : wg_zero16;
    const uint8_t* ds = live ? p.dy + r.dyo[j] : wg_zero16;
    dma16_lds(xs, st + 8 * j * kWgTile);
    dma16_lds(ds, st + kWgOperandBytes + 8 * j * kWgTile);
    // next chunk: (p, q) += (dpp, dq) with carries; x offset follows
    int q = r.rq[j] + p.dq;
    const bool cq = q >= p.Q;
    q = cq ? q - p.Q : q;
    int pp = r.rp[j] + p.dpp + (cq ? 1 : 0);
    const bool cp = pp >= p.P;
    pp = cp ? pp - p.P : pp;
    r.rq[j] = q;
    r.rp[j] = pp;
    r.xo[j] += p.x_step + (cq ? p.x_cq : 0) + (cp ? p.x_cp : 0);
    r.dyo[j] += dy_step;
    r.pix[j] += kWgTile;
  }
}

// Consumer step s (stage ST = s % kWgStages): barrier (the producers have waited for stage
// s+1's DMAs, and every consumer wave holds stage s's fragments in registers), then 16 MFMAs
// per wave on stage s (fragments xc, dc) with the 32 transpose reads of stage s+1 (into xn,
// dn) spread between them, two per MFMA, so the LDS reads overlap the matrix pipe and have
// all landed by the next barrier.
template <int ST>
__device__ __forceinline__ void wg_consume(const uint32_t (&Tx)[8], const uint32_t (&Td)[8],
                                           const v8i (&xc)[4], const v8i (&dc)[4], v8i (&xn)[4],
                                           v8i (&dn)[4], v4f (&acc)[4][4]) {
  constexpr int NX = (ST + 1) % kWgStages;
  wait_lgkmcnt0();
  lds_barrier();
  const uint8_t* nx = wg_smem + NX * kWgStageBytes;
  // D rows = input channels, D cols = output channels
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = mfma16x16x128_e4m3(xc[i], dc[j], acc[i][j]);
    xn[i] = ld_frag_tbl(nx, Tx, i);
    dn[i] = ld_frag_tbl(nx + kWgOperandBytes, Td, i);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // then 2 DS reads
    }
  }
}

// Producer step s: wait until stage s+1 has landed (stages s+2 .. s+kWgStages-1 may still be
// in flight), barrier, then queue stage s+kWgStages into buffer ST, which every consumer
// finished reading before this barrier.
template <int ST>
__device__ __forceinline__ void wg_produce(const WgradArgs& p, WgRows& r, int s, int nsteps,
                                           int kr, int ks, uint32_t lds_wave, uint32_t dy_step) {
  wait_vmcnt<(kWgStages - 2) * kWgLoadsPerStage>();
  lds_barrier();
  wg_issue<ST>(p, r, s + kWgStages < nsteps, kr, ks, lds_wave, dy_step);
}

// One workgroup: one (split, tap, ci tile, co tile); K-steps walk the split's chunks of
// kWgTile pixels through a kWgStages-deep LDS ring. Waves 0-3 run the MFMAs, waves 4-7 the
// address arithmetic and DMAs, so the two overlap on every SIMD.
__global__ __launch_bounds__(kWgThreads, 1) void wgrad_partial_kernel(const WgradArgs p) {
  // XCD-aware order: logical workgroup index = split-major, so the workgroups reading one
  // pixel range (all taps and channel tiles) are consecutive and land on the same XCD.
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
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  const int c_begin = (int)(((int64_t)p.nchunks * split) / p.splits);
  const int c_end = (int)(((int64_t)p.nchunks * (split + 1)) / p.splits);
  const int nsteps = c_end - c_begin;
  static_assert(kWgStages == 4, "prologue and loops below are written for 4 stages");

  v4f acc[4][4];
  const int wc = wave & 1;         // consumers: input-channel half (D rows)
  const int wo = (wave >> 1) & 1;  // consumers: output-channel half (D cols)

  if (wave >= 4) {
    // ---------------- producers ----------------
    const int pw = wave - 4;
    WgRows r;
#pragma unroll
    for (int j = 0; j < kWgLoads; ++j) {
      const int row = pw * 32 + 8 * j + (lane >> 3);
      const int g = (lane & 7) ^ wswz(row);  // pre-swizzled granule for this LDS row
      const uint32_t pix = (uint32_t)(c_begin * kWgTile + row);
      const uint32_t t = fdiv(pix, p.divQ);
      const int q = (int)(pix - t * (uint32_t)p.Q);
      const uint32_t n = fdiv(t, p.divP);
      const int pp = (int)(t - n * (uint32_t)p.P);
      r.pix[j] = (int)pix;
      r.rq[j] = q;
      r.rp[j] = pp;
      r.xo[j] = ((((int)n * p.H + pp * p.stride + kr - p.pad) * p.W + q * p.stride + ks - p.pad) *
                 p.Cin) + ci0 + g * 16;
      r.dyo[j] = pix * (uint32_t)p.Cout + (uint32_t)(co0 + g * 16);
    }
    const uint32_t dy_step = (uint32_t)kWgTile * (uint32_t)p.Cout;
    const uint32_t lds_wave = (uint32_t)(pw * 32 * kWgTile);
    wg_issue<0>(p, r, 0 < nsteps, kr, ks, lds_wave, dy_step);
    wg_issue<1>(p, r, 1 < nsteps, kr, ks, lds_wave, dy_step);
    wg_issue<2>(p, r, 2 < nsteps, kr, ks, lds_wave, dy_step);
    wg_issue<3>(p, r, 3 < nsteps, kr, ks, lds_wave, dy_step);
    wait_vmcnt<(kWgStages - 1) * kWgLoadsPerStage>();  // stage 0 landed
    lds_barrier();
    for (int s = 0; s < nsteps; s += 4) {
      wg_produce<0>(p, r, s, nsteps, kr, ks, lds_wave, dy_step);
      if (s + 1 < nsteps) wg_produce<1>(p, r, s + 1, nsteps, kr, ks, lds_wave, dy_step);
      if (s + 2 < nsteps) wg_produce<2>(p, r, s + 2, nsteps, kr, ks, lds_wave, dy_step);
      if (s + 3 < nsteps) wg_produce<3>(p, r, s + 3, nsteps, kr, ks, lds_wave, dy_step);
    }
    wait_vmcnt<0>();  // trailing DMAs land before LDS is reused
    lds_barrier();
  } else {
    // ---------------- consumers ----------------
    uint32_t Tx[8], Td[8];
    {
      const int k = lane & 15, q = lane >> 4, m = k >> 1;
      const int L = (m >> 1) ^ (2 * q);
      const uint32_t lb = (uint32_t)((32 * q + m) * kWgTile + 8 * (k & 1));
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        Tx[u] = lb + 16u * (uint32_t)((u ^ (4 * wc)) ^ L);
        Td[u] = lb + 16u * (uint32_t)((u ^ (4 * wo)) ^ L);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
    lds_barrier();  // stage 0 landed
    // two fragment sets (a, b) alternate between "current" and "next" from step to step
    v8i xa[4], da[4], xb[4], db[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) xa[i] = ld_frag_tbl(wg_smem, Tx, i);
#pragma unroll
    for (int j = 0; j < 4; ++j) da[j] = ld_frag_tbl(wg_smem + kWgOperandBytes, Td, j);
    for (int s = 0; s < nsteps; s += 4) {
      wg_consume<0>(Tx, Td, xa, da, xb, db, acc);
      if (s + 1 < nsteps) wg_consume<1>(Tx, Td, xb, db, xa, da, acc);
      if (s + 2 < nsteps) wg_consume<2>(Tx, Td, xa, da, xb, db, acc);
      if (s + 3 < nsteps) wg_consume<3>(Tx, Td, xb, db, xa, da, acc);
    }
    wait_lgkmcnt0();
    lds_barrier();  // pairs with the producers' final barrier
  }

  // partial[split][co][tap*Cin + ci]: consumers stage [co][ci] fp32 in LDS, then all eight
  // waves store contiguous 512-B rows (nontemporal: read once, by the reduce)
  if (wave < 4) {
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
  }
  __syncthreads();
  const int64_t kk = (int64_t)p.taps * p.Cin;
  float* base = p.partial + (int64_t)split * p.Cout * kk + (int64_t)tap * p.Cin + ci0;
  constexpr int kChunks = kWgTile * 4 / 16;            // 32 x 16 B per co row
  constexpr int kRowsPerPass = kWgThreads / kChunks;  // 16
  const int ch = threadIdx.x % kChunks;
#pragma unroll 4
  for (int r0 = 0; r0 < kWgTile; r0 += kRowsPerPass) {
    const int co = r0 + threadIdx.x / kChunks;
    __builtin_nontemporal_store(*reinterpret_cast<const v4f*>(wg_smem + co * kWgPPitch + ch * 16),
                                reinterpret_cast<v4f*>(base + (int64_t)(co0 + co) * kk + ch * 4));
  }
}

// dw[e] = bf16( RN32(sum over splits of partial[s][e]) * RN32(sx * sdy) ).
// A workgroup owns 64 x 4 consecutive elements; its four 64-thread groups each sum one
// contiguous quarter of the splits (all of a thread's loads are issued before the adds), and
// group 0 adds the four quarter sums in order. The association is fixed, so results do not
// depend on timing.
constexpr int kRedLanes = 64;
constexpr int kRedGroups = 4;
constexpr int kRedThreads = kRedLanes * kRedGroups;
// kF32: dw is fp32 holding the bf16-rounded values.
template <bool kF32>
__global__ __launch_bounds__(kRedThreads) void wgrad_reduce_kernel(const float* __restrict__ partial,
                                                                  void* __restrict__ dw,
                                                                  const float* __restrict__ sx,
                                                                  const float* __restrict__ sdy,
                                                                  int64_t total, int splits) {
  __shared__ v4f part[kRedGroups - 1][kRedLanes];
  const int lane = threadIdx.x % kRedLanes, grp = threadIdx.x / kRedLanes;
  const int64_t i = ((int64_t)blockIdx.x * kRedLanes + lane) * 4;
  const bool live = i < total;
  const int s0 = splits * grp / kRedGroups, s1 = splits * (grp + 1) / kRedGroups;
  const float* src = partial + (live ? i : 0);
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  int s = s0;
  for (; s + 8 <= s1; s += 8) {
    v4f v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = *reinterpret_cast<const v4f*>(src + (int64_t)(s + k) * total);
#pragma unroll
    for (int k = 0; k < 8; ++k) acc = acc + v[k];
  }
  for (; s < s1; ++s) acc = acc + *reinterpret_cast<const v4f*>(src + (int64_t)s * total);
  if (grp > 0) part[grp - 1][lane] = acc;
  __syncthreads();
  if (grp != 0 || !live) return;
#pragma unroll
  for (int g = 0; g < kRedGroups - 1; ++g) acc = acc + part[g][lane];
  const float scale = sx[0] * sdy[0];
  uint32_t b[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) b[k] = f32_to_bf16_bits(acc[k] * scale);
  if (kF32) {
    *reinterpret_cast<uint4*>((float*)dw + i) = uint4{b[0] << 16, b[1] << 16, b[2] << 16, b[3] << 16};
  } else {
    *reinterpret_cast<uint2*>((uint16_t*)dw + i) = uint2{b[0] | (b[1] << 16), b[2] | (b[3] << 16)};
  }
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

// Three-tap kernel for 3x3 / stride-1 / pad-1 convolutions of 16- and 32-pixel-wide images
// (hwgrad.hip); its partial tiles have the layout wgrad_reduce_kernel sums.
bool hwgrad_supported(int N, int H, int W, int Cin, int Cout);
int hwgrad_splits(int N, int H, int W, int Cin, int Cout, int split_k);
int hwgrad_partial_run(const void* xq, const void* dyq, float* partial, int N, int H, int W,
                       int Cin, int Cout, int splits, hipStream_t s);

static bool use_hwgrad(int N, int H, int W, int Cin, int Cout, int R, int S, int stride,
                       int pad) {
  return R == 3 && S == 3 && stride == 1 && pad == 1 && hwgrad_supported(N, H, W, Cin, Cout);
}

static int wgrad_splits(int N, int H, int W, int Cin, int Cout, int R, int S, int stride,
                        int pad, int split_k) {
  if (use_hwgrad(N, H, W, Cin, Cout, R, S, stride, pad))
    return hwgrad_splits(N, H, W, Cin, Cout, split_k);
  return plan_wgrad(N, H, W, Cin, Cout, R, S, stride, pad, split_k).splits;
}

}  // namespace dpa

using namespace dpa;

extern "C" int64_t dpa_conv2d_wgrad_workspace_bytes(int N, int H, int W, int Cin, int Cout,
                                                    int R, int S, int stride, int pad,
                                                    int split_k) {
  if (!wgrad_shape_ok(N, H, W, Cin, Cout, R, S, stride, pad) || split_k < 0) return 0;
  const int splits = wgrad_splits(N, H, W, Cin, Cout, R, S, stride, pad, split_k);
  return (int64_t)splits * Cout * R * S * Cin * 4;
}

static int wgrad_run(const void* xq, const void* dyq, const float* x_scale,
                     const float* dy_scale, void* dw, bool f32out, void* workspace,
                     int64_t workspace_bytes, int N, int H, int W, int Cin, int Cout, int R,
                     int S, int stride, int pad, int split_k, void* stream) {
  if (!xq || !dyq || !x_scale || !dy_scale || !dw) return DPA_ERR_NULL;
  if (!wgrad_shape_ok(N, H, W, Cin, Cout, R, S, stride, pad)) return DPA_ERR_SHAPE;
  if (split_k < 0) return DPA_ERR_SIZE;
  const int splits = wgrad_splits(N, H, W, Cin, Cout, R, S, stride, pad, split_k);
  const int64_t need = (int64_t)splits * Cout * R * S * Cin * 4;
  if (!workspace || workspace_bytes < need) return DPA_ERR_WORKSPACE;
  if (!aligned(xq, 16) || !aligned(dyq, 16) || !aligned(workspace, 16) ||
      !aligned(dw, f32out ? 16 : 8))
    return DPA_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  const int64_t total = (int64_t)Cout * R * S * Cin;
  if (use_hwgrad(N, H, W, Cin, Cout, R, S, stride, pad)) {
    int st = hwgrad_partial_run(xq, dyq, (float*)workspace, N, H, W, Cin, Cout, splits, s);
    if (st != DPA_OK) return st;
    if (f32out)
      wgrad_reduce_kernel<true><<<(unsigned)ceil_div(total, 4 * kRedLanes), kRedThreads, 0, s>>>(
          (const float*)workspace, dw, x_scale, dy_scale, total, splits);
    else
      wgrad_reduce_kernel<false><<<(unsigned)ceil_div(total, 4 * kRedLanes), kRedThreads, 0, s>>>(
          (const float*)workspace, dw, x_scale, dy_scale, total, splits);
    return launch_status();
  }
  WgradPlan pl = plan_wgrad(N, H, W, Cin, Cout, R, S, stride, pad, split_k);
  // 32-bit byte offsets inside the kernel
  if ((int64_t)N * H * W * Cin > 0x7fffffff || (int64_t)pl.npix * Cout > 0x7fffffff)
    return DPA_ERR_SIZE;
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
  {
    // one chunk of kWgTile pixels = dn images + dpp rows + dq columns
    const int dq = kWgTile % pl.Q, dpp = (kWgTile / pl.Q) % pl.P, dn = kWgTile / (pl.Q * pl.P);
    a.dq = dq;
    a.dpp = dpp;
    a.x_step = ((dn * H + dpp * stride) * W + dq * stride) * Cin;
    a.x_cq = (stride * W - pl.Q * stride) * Cin;       // q wraps: next output row
    a.x_cp = (H - pl.P * stride) * W * Cin;            // p wraps: next image
  }
  wgrad_partial_kernel<<<(unsigned)(a.per_xcd * 8), kWgThreads, 0, s>>>(a);
  int st = launch_status();
  if (st != DPA_OK) return st;
  if (f32out)
    wgrad_reduce_kernel<true><<<(unsigned)ceil_div(total, 4 * kRedLanes), kRedThreads, 0, s>>>(
        (const float*)workspace, dw, x_scale, dy_scale, total, pl.splits);
  else
    wgrad_reduce_kernel<false><<<(unsigned)ceil_div(total, 4 * kRedLanes), kRedThreads, 0, s>>>(
        (const float*)workspace, dw, x_scale, dy_scale, total, pl.splits);
  return launch_status();
}

extern "C" int dpa_conv2d_wgrad_fp8(const void* xq, const void* dyq, const float* x_scale,
                                    const float* dy_scale, void* dw, void* workspace,
                                    int64_t workspace_bytes, int N, int H, int W, int Cin,
                                    int Cout, int R, int S, int stride, int pad, int split_k,
                                    void* stream) {
  return wgrad_run(xq, dyq, x_scale, dy_scale, dw, false, workspace, workspace_bytes, N, H, W,
                   Cin, Cout, R, S, stride, pad, split_k, stream);
}

extern "C" int dpa_conv2d_wgrad_fp8_f32(const void* xq, const void* dyq, const float* x_scale,
                                        const float* dy_scale, float* dw, void* workspace,
                                        int64_t workspace_bytes, int N, int H, int W, int Cin,
                                        int Cout, int R, int S, int stride, int pad, int split_k,
                                        void* stream) {
  return wgrad_run(xq, dyq, x_scale, dy_scale, dw, true, workspace, workspace_bytes, N, H, W,
                   Cin, Cout, R, S, stride, pad, split_k, stream);
}
