// FP8 weight gradient of a 3x3 / stride-1 / pad-1 convolution for images W = 16 or 32 pixels
// wide: one workgroup computes the three taps of one kernel row, so each K-step's operand
// blocks feed three times the MFMAs of a one-tap tile.
//
// Reference: diffusion/fp8_kernels.py conv2d_dw_fp8_kernel :340-443 (partials over pixel
// blocks) and conv2d_dw_reduce_fp8_kernel :446-468 (split sum, scale, bf16); the split sum is
// wgrad.hip's wgrad_reduce_kernel, unchanged.
//
// dW[r][s][ci][co] = sum over output pixels (p, q) of x[p + r - 1][q + s - 1][ci] * dy[p][q][co].
// A K-step is 128 output pixels = 128 / W whole image rows. For kernel row r the three taps
// read the same x rows (p + r - 1) shifted by one column each, so a stage holds the dy block
// (128 px x 128 co) and one x block (those rows, 64 input channels, laid out as rows of W + 2
// pixels whose first and last pixel stay zero: the column padding). Tap s reads its A
// fragments at a one-pixel offset s. Per K-step that is 24 KB from L2 for 3 x 64 x 128 x 128
// MACs, against 32 KB for 128 x 128 x 128 in the one-tap kernel of wgrad.hip.
//
// Workgroup: 4 consumer waves (2 x 2: 32 input channels x 64 output channels each, three
// taps) and 4 producer waves that compute DMA addresses and keep a 6-deep LDS ring full.
// Operands are pixel-major in LDS and the MFMA fragments (K = pixels) are formed with
// ds_read_b64_tr_b8. Splits of the pixel range write fp32 partial tiles that
// wgrad_reduce_kernel sums in split order.
#include "dpa_common.hpp"

namespace dpa {

constexpr int kHwConsumers = 256;
constexpr int kHwThreads = 512;
constexpr int kHwCi = 64;                              // input channels per tile
constexpr int kHwCo = 128;                             // output channels per tile
constexpr int kHwPix = 128;                            // output pixels per K-step
constexpr int kHwXBytes = 9216;                        // x block: max over W of (128/W)(W+2) x 64 B
constexpr int kHwDyBytes = kHwPix * kHwCo;             // 16 KB
constexpr int kHwStageBytes = kHwXBytes + kHwDyBytes;  // 25 KB
constexpr int kHwStages = 6;
constexpr int kHwDyLoads = kHwDyBytes / 16 / 256;      // 4 dy DMAs per producer thread
constexpr int kHwXLoads = kHwPix * kHwCi / 16 / 256;   // 2 x DMAs per producer thread
constexpr int kHwLoadsPerStage = kHwDyLoads + kHwXLoads;
constexpr int kHwPPitch = 3 * kHwCi * 4 + 16;          // partial staging: [co][tap][ci] fp32

__shared__ __attribute__((aligned(1024))) uint8_t hw_smem[kHwStages * kHwStageBytes];
static_assert(kHwCo * kHwPPitch <= kHwStages * kHwStageBytes, "partial tile must fit in LDS");

__device__ __attribute__((aligned(64))) uint8_t hw_zero16[64];

struct HwgradArgs {
  const uint8_t* x;   // [N][H][W][Cin]
  const uint8_t* dy;  // [N][H][W][Cout]
  float* partial;     // [splits][Cout][9 * Cin]
  int N, H, Cin, Cout;
  int nchunks, splits, tiles, ci_tiles, total, per_xcd;
};

// dy rows (pixels, 128 B): granule g at g ^ hw_dyswz(r). A fragment read (r = 32 q + 8 s + m,
// q = lane >> 4, m = (lane & 15) >> 1) is served per half-wave on gfx950, lanes 0-31 then
// 32-63, over 32 8-B bank slots: the granule must take 8 values across (m >> 1, q & 1) of a
// half-wave, so bit 2 follows q & 1 (row bit 5) and bit 1 follows q >> 1 (row bit 6), each
// XOR a bit of s: bit 0 = r1 ^ r4, bit 1 = r2 ^ r6, bit 2 = r5 ^ r3.
__device__ __forceinline__ int hw_dyswz(int row) {
  return (((row >> 1) ^ (row >> 4)) & 1) | ((((row >> 2) ^ (row >> 6)) & 1) << 1) |
         ((((row >> 5) ^ (row >> 3)) & 1) << 2);
}
__device__ __forceinline__ constexpr int hw_c(int s) { return ((s & 1) << 2) ^ (s >> 1); }

// x pixels (64 B = 4 granules): granule g at g ^ bit 2 of the pixel index. A transpose read
// covers 8 consecutive pixels at one granule; pixels e and e + 4 share banks and differ in
// bit 2, so any 8 consecutive pixels fall in 8 distinct bank groups.
__device__ __forceinline__ int hw_xswz(int e) { return (e >> 2) & 1; }

typedef int v2i_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ v2i_t hw_tr8(const uint8_t* a) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((v2i_t __attribute__((address_space(3)))*)(a));
}

// dy fragment j (16 output channels) of a stage, as wgrad.hip's ld_frag_tbl.
__device__ __forceinline__ v8i hw_ld_dy(const uint8_t* dyt, const uint32_t (&T)[8], int j) {
  v8i f;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const v2i_t v = hw_tr8(dyt + T[j ^ hw_c(s)] + 1024 * s);
    f[2 * s] = v.x;
    f[2 * s + 1] = v.y;
  }
  return f;
}

// x fragment of tap S for one 16-channel granule. Read kb covers output pixels 32q + 8kb + m
// (q = lane >> 4, m = (lane & 15) >> 1), i.e. x pixel e = Eq + Ec + m with Eq the lane
// group's row offset and Ec = row(8kb) (W + 2) + col(8kb) + S a constant; the per-lane table
// holds 64 (Eq + m) + 16 (g ^ bit2(Eq + m + v)) + 8h for v = Ec mod 8.
template <int W, int S>
__device__ __forceinline__ v8i hw_ld_x(const uint8_t* xt, const uint32_t (&T)[8]) {
  v8i f;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const int ec = ((8 * kb) / W) * (W + 2) + (8 * kb) % W + S;
    const v2i_t v = hw_tr8(xt + T[ec & 7] + 64 * ec);
    f[2 * kb] = v.x;
    f[2 * kb + 1] = v.y;
  }
  return f;
}

template <int W, int P>
__device__ __forceinline__ v8i hw_ld_xp(const uint8_t* xt, const uint32_t (&T0)[8],
                                        const uint32_t (&T1)[8]) {
  // pair P = 2 * tap + granule
  return (P & 1) ? hw_ld_x<W, (P >> 1)>(xt, T1) : hw_ld_x<W, (P >> 1)>(xt, T0);
}

// Consumer step on stage ST: the barrier (producers have seen stage ST+1 land; every consumer
// has finished reading stage ST-1), then 24 MFMAs = 6 (tap, granule) pairs x 4 dy fragments.
// x fragments stream through 3 registers sets, two pairs ahead: pairs 2..5 of this stage
// and, at the end, pairs 0 and 1 of the next stage; the next stage's dy fragments are read
// between the MFMAs. Pairs 0 and 1 of this stage are in X[0], X[1] on entry.
template <int W, int ST>
__device__ __forceinline__ void hw_consume(const uint32_t (&T0)[8], const uint32_t (&T1)[8],
                                           const uint32_t (&Td)[8], v8i (&X)[3],
                                           const v8i (&dc)[4], v8i (&dn)[4], v4f (&acc)[6][4]) {
  constexpr int NX = (ST + 1) % kHwStages;
  const uint8_t* cur = hw_smem + ST * kHwStageBytes;
  const uint8_t* nxt = hw_smem + NX * kHwStageBytes;
  wait_lgkmcnt<8>();  // only the two prefetched pairs (stage ST) may still be in flight
  lds_barrier();
#pragma unroll
  for (int pr = 0; pr < 6; ++pr) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[pr][j] = mfma16x16x128_e4m3(X[pr % 3], dc[j], acc[pr][j]);
    if (pr < 4) {
      dn[pr] = hw_ld_dy(nxt + kHwXBytes, Td, pr);
    }
    // pair pr + 2 of this stage, or pair pr - 4 of the next one
    switch (pr) {
      case 0: X[2] = hw_ld_xp<W, 2>(cur, T0, T1); break;
      case 1: X[0] = hw_ld_xp<W, 3>(cur, T0, T1); break;
      case 2: X[1] = hw_ld_xp<W, 4>(cur, T0, T1); break;
      case 3: X[2] = hw_ld_xp<W, 5>(cur, T0, T1); break;
      case 4: X[0] = hw_ld_xp<W, 0>(nxt, T0, T1); break;
      default: X[1] = hw_ld_xp<W, 1>(nxt, T0, T1); break;
    }
    // pin the interleave: each MFMA is followed by this pair's share of the reads, so the
    // reads are issued a pair (4 MFMAs) or more before their data is needed
    if (pr < 4) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // 2 DS reads
      }
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 DS read
      }
    }
  }
}

// Producer DMA state: dy rows advance by 128 pixels per step; x rows by 128 / W image rows,
// with ih (the x row this thread's block reads) wrapping at the image height.
struct HwRows {
  uint32_t dyo[kHwDyLoads];
  int xo[kHwXLoads];
  int ih[kHwXLoads];
};

template <int W, int ST>
__device__ __forceinline__ void hw_issue(const HwgradArgs& p, HwRows& r, bool live, int pw,
                                         uint32_t x_step, uint32_t dy_step) {
  constexpr int RO = kHwPix / W;
  const uint32_t st = LDS_ADDR(hw_smem) + ST * kHwStageBytes;
#pragma unroll
  for (int j = 0; j < kHwDyLoads; ++j) {
    const uint8_t* src = live ? p.dy + r.dyo[j] : hw_zero16;
    dma16_lds(src, st + kHwXBytes + (uint32_t)(pw * 32 + 8 * j) * 128);
    r.dyo[j] += dy_step;
  }
#pragma unroll
  for (int j = 0; j < kHwXLoads; ++j) {
    const int b = 2 * pw + j;  // 16-pixel block of the step
    const int row = (16 * b) / W, col0 = (16 * b) % W;
    const bool ok = live & ((unsigned)r.ih[j] < (unsigned)p.H);
    const uint8_t* src = ok ? p.x + r.xo[j] : hw_zero16;
    dma16_lds(src, st + (uint32_t)(row * (W + 2) + 1 + col0) * 64);
    r.xo[j] += (int)x_step;
    const int ih = r.ih[j] + RO;
    r.ih[j] = ih;
  }
}

template <int W>
__global__ __launch_bounds__(kHwThreads, 1) void hwgrad_partial_kernel(const HwgradArgs p) {
  constexpr int RO = kHwPix / W;  // image rows per K-step
  const int logical = (blockIdx.x & 7) * p.per_xcd + (blockIdx.x >> 3);
  if (logical >= p.total) return;
  const int split = logical / p.tiles;
  int rem = logical - split * p.tiles;
  const int kr = rem % 3;  // kernel row
  rem /= 3;
  const int ci0 = (rem % p.ci_tiles) * kHwCi;
  const int co0 = (rem / p.ci_tiles) * kHwCo;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c_begin = (int)(((int64_t)p.nchunks * split) / p.splits);
  const int c_end = (int)(((int64_t)p.nchunks * (split + 1)) / p.splits);
  const int nsteps = c_end - c_begin;
  const int chunks_per_img = p.H / RO;
  static_assert(kHwStages == 6, "prologue and loops below are written for 6 stages");

  v4f acc[6][4];
  const int wc = wave & 1;         // consumers: 32-channel half of the 64 input channels
  const int wo = (wave >> 1) & 1;  // consumers: 64-channel half of the 128 output channels

  if (wave >= 4) {
    // ---------------- producers ----------------
    const int pw = wave - 4;
    HwRows r;
    const int n0 = c_begin / chunks_per_img;
    const int p0 = (c_begin - n0 * chunks_per_img) * RO;  // first output row of the split
#pragma unroll
    for (int j = 0; j < kHwDyLoads; ++j) {
      const int row = pw * 32 + 8 * j + (lane >> 3);
      const int g = (lane & 7) ^ hw_dyswz(row);
      const uint32_t pix = (uint32_t)c_begin * kHwPix + (uint32_t)row;
      r.dyo[j] = pix * (uint32_t)p.Cout + (uint32_t)(co0 + g * 16);
    }
#pragma unroll
    for (int j = 0; j < kHwXLoads; ++j) {
      const int b = 2 * pw + j;
      const int row = (16 * b) / W, col = (16 * b) % W + (lane >> 2);
      const int e = row * (W + 2) + 1 + col;
      const int g = (lane & 3) ^ hw_xswz(e);
      const int ih = p0 + row + kr - 1;
      r.ih[j] = ih;
      // the offset may point outside x while ih is out of range; it is only used when valid
      r.xo[j] = ((n0 * p.H + ih) * W + col) * p.Cin + ci0 + 16 * g;
    }
    const uint32_t x_step = (uint32_t)(RO * W * p.Cin);
    const uint32_t dy_step = (uint32_t)kHwPix * (uint32_t)p.Cout;
    // ih wraps at the image height: rows p0 + row + kr - 1 for p0 = 0, RO, ..., H - RO.
    // Subtract H whenever the output row block passes the end of an image.
    int prow = p0;
    auto advance_rows = [&]() {
      prow += RO;
      if (prow == p.H) {
        prow = 0;
#pragma unroll
        for (int j = 0; j < kHwXLoads; ++j) r.ih[j] -= p.H;
      }
    };
#define HW_ISSUE(ST, LIVE)                                                 \
  do {                                                                     \
    hw_issue<W, ST>(p, r, (LIVE), pw, x_step, dy_step);              \
    advance_rows();                                                        \
  } while (0)
    HW_ISSUE(0, 0 < nsteps);
    HW_ISSUE(1, 1 < nsteps);
    HW_ISSUE(2, 2 < nsteps);
    HW_ISSUE(3, 3 < nsteps);
    HW_ISSUE(4, 4 < nsteps);
    wait_vmcnt<4 * kHwLoadsPerStage>();  // stage 0 landed
    lds_barrier();                        // B0
    // step s: wait for stage s + 1, barrier, refill the buffer of stage s - 1 with s + 5
#define HW_PRODUCE(ST, S)                                  \
  do {                                                     \
    wait_vmcnt<3 * kHwLoadsPerStage>();                    \
    lds_barrier();                                         \
    HW_ISSUE((ST + 5) % kHwStages, (S) + 5 < nsteps);      \
  } while (0)
    for (int s = 0; s < nsteps; s += 6) {
      HW_PRODUCE(0, s);
      if (s + 1 < nsteps) HW_PRODUCE(1, s + 1);
      if (s + 2 < nsteps) HW_PRODUCE(2, s + 2);
      if (s + 3 < nsteps) HW_PRODUCE(3, s + 3);
      if (s + 4 < nsteps) HW_PRODUCE(4, s + 4);
      if (s + 5 < nsteps) HW_PRODUCE(5, s + 5);
    }
#undef HW_PRODUCE
#undef HW_ISSUE
    wait_vmcnt<0>();  // trailing DMAs land before LDS is reused
    lds_barrier();
  } else {
    // ---------------- consumers ----------------
    const int k = lane & 15, q = lane >> 4, m = k >> 1, h = k & 1;
    uint32_t Td[8], T0[8], T1[8];
    {
      const int L = (m >> 1) ^ (2 * (q >> 1)) ^ (4 * (q & 1));  // hw_dyswz(32 q + m)
      const uint32_t lb = (uint32_t)((32 * q + m) * 128 + 8 * h);
#pragma unroll
      for (int u = 0; u < 8; ++u) Td[u] = lb + 16u * (uint32_t)((u ^ (4 * wo)) ^ L);
      const int eq = q * (32 / W) * (W + 2) + m;  // x pixel of kb = 0 without the tap shift
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const int b2 = hw_xswz(eq + v);
        T0[v] = (uint32_t)(64 * eq + 16 * ((2 * wc + 0) ^ b2) + 8 * h);
        T1[v] = (uint32_t)(64 * eq + 16 * ((2 * wc + 1) ^ b2) + 8 * h);
      }
    }
    // zero the padding pixels (x columns -1 and W) of every stage; no DMA writes them
    for (int i = threadIdx.x; i < kHwStages * RO * 2 * 4; i += kHwConsumers) {
      const int g = i & 3, side = (i >> 2) & 1, rs = i >> 3;
      const int row = rs % RO, stg = rs / RO;
      const int e = row * (W + 2) + (side ? W + 1 : 0);
      *reinterpret_cast<uint4*>(hw_smem + stg * kHwStageBytes + e * 64 + g * 16) =
          uint4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < 6; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
    wait_lgkmcnt0();
    lds_barrier();  // B0: stage 0 landed, padding zeroed
    v8i X[3], da[4], db[4];
    X[0] = hw_ld_xp<W, 0>(hw_smem, T0, T1);
    X[1] = hw_ld_xp<W, 1>(hw_smem, T0, T1);
#pragma unroll
    for (int j = 0; j < 4; ++j) da[j] = hw_ld_dy(hw_smem + kHwXBytes, Td, j);
    for (int s = 0; s < nsteps; s += 6) {
      hw_consume<W, 0>(T0, T1, Td, X, da, db, acc);
      if (s + 1 < nsteps) hw_consume<W, 1>(T0, T1, Td, X, db, da, acc);
      if (s + 2 < nsteps) hw_consume<W, 2>(T0, T1, Td, X, da, db, acc);
      if (s + 3 < nsteps) hw_consume<W, 3>(T0, T1, Td, X, db, da, acc);
      if (s + 4 < nsteps) hw_consume<W, 4>(T0, T1, Td, X, da, db, acc);
      if (s + 5 < nsteps) hw_consume<W, 5>(T0, T1, Td, X, db, da, acc);
    }
    wait_lgkmcnt0();
    lds_barrier();  // pairs with the producers' final barrier
  }

  // partial[split][co][(3 kr + s) Cin + ci]: consumers stage [co][s][ci] fp32 in LDS, then all
  // eight waves store 256-B row segments
  if (wave < 4) {
    const int frow = lane & 15, fq = lane >> 4;
#pragma unroll
    for (int pr = 0; pr < 6; ++pr) {
      const int s = pr >> 1, i = pr & 1;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int co = wo * 64 + j * 16 + frow;
        const int ci = wc * 32 + i * 16 + 4 * fq;
        *reinterpret_cast<v4f*>(hw_smem + co * kHwPPitch + (s * kHwCi + ci) * 4) = acc[pr][j];
      }
    }
  }
  __syncthreads();
  const int64_t kk = (int64_t)9 * p.Cin;
  float* base = p.partial + (int64_t)split * p.Cout * kk + (int64_t)(3 * kr) * p.Cin + ci0;
  constexpr int kSegChunks = kHwCi * 4 / 16;                 // 16 x 16 B per 256-B segment
  constexpr int kSegsPerPass = kHwThreads / kSegChunks;      // 32
  const int ch = threadIdx.x % kSegChunks;
#pragma unroll 4
  for (int sg0 = 0; sg0 < kHwCo * 3; sg0 += kSegsPerPass) {
    const int sg = sg0 + threadIdx.x / kSegChunks;
    const int co = sg / 3, s = sg - (sg / 3) * 3;
    *reinterpret_cast<v4f*>(base + (int64_t)(co0 + co) * kk + (int64_t)s * p.Cin + ch * 4) =
        *reinterpret_cast<const v4f*>(hw_smem + co * kHwPPitch + (s * kHwCi) * 4 + ch * 16);
  }
}

bool hwgrad_supported(int N, int H, int W, int Cin, int Cout) {
  if (N <= 0 || H <= 0) return false;
  if (W != 16 && W != 32) return false;
  if (H % (kHwPix / W) != 0) return false;
  if (Cin % kHwCi != 0 || Cout % kHwCo != 0) return false;
  if ((int64_t)N * H * W * Cin > 0x7fffffff || (int64_t)N * H * W * Cout > 0x7fffffff)
    return false;
  return true;
}

int hwgrad_splits(int N, int H, int W, int Cin, int Cout, int split_k) {
  const int nchunks = (int)((int64_t)N * H * W / kHwPix);
  const int tiles = 3 * (Cin / kHwCi) * (Cout / kHwCo);
  int s = split_k;
  if (s <= 0) {
    // one round of workgroups over the 256 CUs, at least 4 K-steps per split
    s = 256 / tiles;
    if (s < 1) s = 1;
    int maxs = nchunks / 4;
    if (maxs < 1) maxs = 1;
    if (s > maxs) s = maxs;
  }
  if (s > nchunks) s = nchunks;
  return s;
}

// Launches the partial kernel; the caller has checked hwgrad_supported and the workspace
// (splits x Cout x 9 x Cin fp32).
int hwgrad_partial_run(const void* xq, const void* dyq, float* partial, int N, int H, int W,
                       int Cin, int Cout, int splits, hipStream_t s) {
  HwgradArgs a{};
  a.x = (const uint8_t*)xq;
  a.dy = (const uint8_t*)dyq;
  a.partial = partial;
  a.N = N; a.H = H; a.Cin = Cin; a.Cout = Cout;
  a.nchunks = (int)((int64_t)N * H * W / kHwPix);
  a.splits = splits;
  a.ci_tiles = Cin / kHwCi;
  a.tiles = 3 * a.ci_tiles * (Cout / kHwCo);
  a.total = a.tiles * splits;
  a.per_xcd = (int)ceil_div(a.total, 8);
  const unsigned grid = (unsigned)(a.per_xcd * 8);
  if (W == 32)
    hwgrad_partial_kernel<32><<<grid, kHwThreads, 0, s>>>(a);
  else
    hwgrad_partial_kernel<16><<<grid, kHwThreads, 0, s>>>(a);
  return launch_status();
}

}  // namespace dpa
