// FP8 implicit-GEMM convolution (forward and data-gradient) and FP8 GEMM on gfx950 MFMA.
//
// Reference: diffusion/fp8_kernels.py
//   conv2d_fwd_fp8_kernel  :142-247 (+ launcher :604-639)  -> dpa_conv2d_fwd_fp8
//   conv2d_dx_fp8_kernel   :250-318 (+ launcher :671-709)  -> dpa_conv2d_dgrad_fp8
//
// One kernel serves every case. The GEMM is
//   out[pix, co] = sum_{tap, c} act[pix shifted by tap, c] * wgt[co, tap, c]
// over a tap grid (ty, tx) in [0, ny) x [0, nx) whose input offset and weight tap are linear
// in (ty, tx). Forward convs (stride 1 or 2, 3x3 or 1x1) use the natural grid; the data
// gradient is the same kernel on dy with the weight transposed to [Cin][R][S][Cout] and a
// mirrored grid; stride-2 dgrad runs once per output parity class with only the taps that
// class touches; the linear is the 1x1 case with H = W = 1.
//
// Schedule: persistent. One workgroup of 8 waves (4 x 2, two per SIMD) per CU walks its
// output tiles of 256 pixels x 128 channels (128 or 64 pixels for launches with few output
// pixels, IgCfg; a contiguous run per XCD, so neighbouring
// tiles share halo rows in that XCD's L2) as one continuous stream of K-steps (128 input
// channels of one tap per step). Operands reach LDS by DMA (global_load_lds, 16 B per lane)
// through a 3-stage ring, issued three steps ahead, also across tile boundaries. Each wave
// owns a 64 x 64 output tile (4 x 4 MFMA 16x16x128); step k runs its 16 MFMAs on fragments
// read during step k-1 while it reads step k+1's fragments, so LDS reads, DMA and MFMA of
// neighbouring steps overlap. LDS rows are 128 B with 16-B granules XOR-swizzled by
// ((row ^ (row >> 3)) & 7), conflict-free for the 16-row fragment reads.
// Epilogue per finished tile, per wave, while the next tile's DMA is in flight:
//   out = bf16(RN32(acc * RN32(sa * sb)) [+ bias]), staged through the wave's private 2 KB
// LDS slot so every pixel's 64 channels leave as one 128-B run, with nontemporal stores (the
// output is not read again by this kernel; plain stores left the next launch's first loads
// queued behind write-backs).
#include "dpa_common.hpp"

namespace dpa {

constexpr int kIgThreads = 512;  // 8 waves: 2 per SIMD
constexpr int kWaves = kIgThreads / 64;
constexpr int kWavesM = 4;
constexpr int kWTM = 64, kWTN = 64;  // wave tile
constexpr int kBM = 256;             // output pixels per tile
constexpr int kBN = 128;             // output channels per tile
constexpr int kBK = 128;             // K bytes per step (MFMA depth)
constexpr int kStageBytes = (kBM + kBN) * kBK;         // 48 KB: A tile then B tile
constexpr int kALoads = kBM * kBK / 16 / kIgThreads;  // 16-B DMA per thread per stage: 4
constexpr int kBLoads = kBN * kBK / 16 / kIgThreads;  // 2
constexpr int kLoadsPerStage = kALoads + kBLoads;     // per wave (one per instruction)
constexpr int kARowsPerWave = kBM / kWaves;           // 32
constexpr int kBRowsPerWave = kBN / kWaves;           // 16
constexpr int kSlotBytes = 16 * kWTN * 2;             // 16 pixels x 64 channels of bf16
constexpr int kMaxTapDim = 3;

// Tile shape of an igemm_fp8_kernel instance: BM output pixels x BN channels, the 8 waves as
// kWavesM x kWavesN wave tiles of kWTM pixels x kWTN channels. 256 x 128 is the default;
// 128 x 128 (64 x 32 wave tiles, 32 KB stages) and 64 x 128 (64 x 16, 24 KB stages) give
// launches with few output pixels two or four times the tiles, so they fill the CUs without
// splitting K; 64 x 32 (4 x 2 waves of 16 x 16, 12 KB stages) four times the 64 x 128 ones.
// Its B tile is 256 DMAs of 16 B, so waves 0-3 load it (kBLoadWaves) and waves 4-7 wait for
// their A loads only.
template <int BM, int BN = kBN>
struct IgCfg {
  static constexpr int kWavesM = BN == dpa::kBN ? BM / dpa::kWTM : BM / 16;
  static constexpr int kBM = BM, kBN = BN;
  static constexpr int kWavesN = kWaves / kWavesM;
  static constexpr int kWTM = BM / kWavesM;
  static constexpr int kWTN = BN / kWavesN;
  static constexpr int kFA = kWTM / 16;  // 16-pixel MFMA blocks per wave
  static constexpr int kCB = kWTN / 16;  // 16-channel MFMA blocks per wave
  static constexpr int kStageBytes = (BM + BN) * kBK;
  static constexpr int kALoads = BM * kBK / 16 / kIgThreads;
  static constexpr int kBLoadWaves = BN * kBK / 16 / 64 < kWaves ? BN * kBK / 16 / 64 : kWaves;
  static constexpr int kBLoads = BN * kBK / 16 / (64 * kBLoadWaves);  // per B-loading wave
  static constexpr int kLoadsPerStage = kALoads + kBLoads;          // of a B-loading wave
  static constexpr int kARowsPerWave = BM / kWaves;
  static constexpr int kBRowsPerWave = BN / kBLoadWaves;
  static constexpr int kSlotG = kWTN / 8;                 // 16-B granules per slot row
  static constexpr int kSlotBytes = 16 * kSlotG * 16;      // 16 pixels x kWTN channels, bf16
  static_assert(kWavesM * kWavesN == kWaves && kFA >= 1 && kCB >= 1 && kALoads >= 1 &&
                    kBLoads >= 1 && kWTM % 16 == 0 && kWTN % 16 == 0,
                "wave tiles of whole MFMA blocks, whole DMAs per wave");
};
static_assert(IgCfg<256>::kWTN == kWTN && IgCfg<256>::kLoadsPerStage == kLoadsPerStage &&
                  IgCfg<256>::kSlotBytes == kSlotBytes && IgCfg<256>::kFA == 4 &&
                  IgCfg<256>::kBLoadWaves == kWaves && IgCfg<128>::kFA == 4 &&
                  IgCfg<64>::kFA == 4 && IgCfg<64, 32>::kFA == 1 && IgCfg<64, 32>::kCB == 1,
              "the tiles");

struct IgemmArgs {
  const uint8_t* act;  // [N][Hi][Wi][C]
  const uint8_t* wgt;  // [Cout][T][C]
  uint16_t* out;       // bf16 [N][Ho][Wo][Cout]
  const float* sa;
  const float* sb;
  const float* bias;  // [Cout] or null
  int Hi, Wi, C, Cout, T;
  int Pg, Qg;  // output grid enumerated by this launch
  int Ho, Wo;
  int oy_step, oy_off, ox_step, ox_off;  // out pixel = (i*oy_step + oy_off, j*ox_step + ox_off)
  int iy_step, ix_step;                  // in pixel  = (i*iy_step + dy, j*ix_step + dx)
  int M;                                 // N * Pg * Qg
  int tiles_n, tiles, tiles_per_xcd, wg_per_xcd;  // tiles: work items (tiles x splits)
  // tap grid: tap (ty, tx), ty < ny, tx < nx: input offset (dy0 + ty*dys, dx0 + tx*dxs),
  // weight tap w0 + ty*wys + tx*wxs
  int ny, nx, dy0, dys, dx0, dxs, w0, wys, wxs;
  int kc_per_tap, nk;  // K-steps per tap (C / 128) and per work item (a tile's K range)
  int splits;          // K ranges per tile: work item = (tile, split), item / splits = tile
  float* partial;      // splits > 1: fp32 partial sums per work item, in accumulator order
  // Output parity classes of a strided data gradient in one launch. Tiles are class-major,
  // tiles_pc per class; class c offsets its output pixels by (oy, ox) and its taps by input
  // (dy0, dx0) and weight tap w0, and only ny x nx of the launch's ny x nx taps are real (the
  // others read zero rows, so their MFMAs add zeros). cls[c] packs them as 4-bit fields
  // (cls_field). nclass = 1: the scalar fields above.
  int nclass, tiles_pc;
  uint32_t cls[4];
  FastDiv divQ, divP, divKC, divNX, divNK, divTN, divSP, divPC;
};

// 16 zero bytes: the DMA source for padding taps and rows past M.
__device__ __attribute__((aligned(64))) uint8_t g_zero16[64];
constexpr int64_t kMaxOperandBytes = 0x7fffffff;  // 32-bit offsets


// LDS rows are 128 B = 8 granules of 16 B; granule g of row r lives at (g ^ swz(r)). Measured
// on gfx950 (SQ_LDS_BANK_CONFLICT): this swizzle makes the 16-row, one-granule fragment
// reads of ds_read_b128 conflict-free, where (r & 7) or ((r >> 1) & 7) cost 2 passes.
__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }

// m -> (n, i, j) of the launch grid [N, Pg, Qg]
__device__ __forceinline__ void decode_pixel(const IgemmArgs& p, int m, int& n, int& i, int& j) {
  const uint32_t t = fdiv((uint32_t)m, p.divQ);
  j = m - (int)t * p.Qg;
  const uint32_t nn = fdiv(t, p.divP);
  i = (int)t - (int)nn * p.Pg;
  n = (int)nn;
}

__device__ __forceinline__ int out_offset(const IgemmArgs& p, int m, int oy_off, int ox_off) {
  int n, ii, jj;
  decode_pixel(p, m, n, ii, jj);
  return ((n * p.Ho + ii * p.oy_step + oy_off) * p.Wo + jj * p.ox_step + ox_off) * p.Cout;
}

// output tile -> (class, tile within the class)
__device__ __forceinline__ int tile_class(const IgemmArgs& p, int tile, int& tic) {
  const int c = p.nclass > 1 ? (int)fdiv((uint32_t)tile, p.divPC) : 0;
  tic = tile - c * p.tiles_pc;
  return c;
}

// fields of a packed class word, 4 bits each
enum ClsField { kClsOy = 0, kClsOx = 4, kClsDy0 = 8, kClsDx0 = 12, kClsW0 = 16, kClsNy = 20,
                kClsNx = 24 };
__host__ __device__ __forceinline__ int cls_field(uint32_t w, ClsField f) {
  return (int)((w >> f) & 15u);
}

// p.cls[c] by constant indices: the kernel arguments are then all read at the start, in one
// batch, instead of by a load whose address waits for c
__device__ __forceinline__ uint32_t cls_word(const IgemmArgs& p, int c) {
  uint32_t v = p.cls[0];
  v = c == 1 ? p.cls[1] : v;
  v = c == 2 ? p.cls[2] : v;
  v = c == 3 ? p.cls[3] : v;
  return v;
}

__device__ __forceinline__ v8i ld_frag(const uint8_t* base, int row, int q) {
  const int s = swz(row);
  const uint4 lo = *reinterpret_cast<const uint4*>(base + row * kBK + (((2 * q) ^ s) * 16));
  const uint4 hi = *reinterpret_cast<const uint4*>(base + row * kBK + (((2 * q + 1) ^ s) * 16));
  return v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}

// kClasses: the launch holds several output parity classes (p.nclass > 1). The one-class
// instance reads the scalar tap grid only: the class tables would take SGPRs the main loop
// needs (with them it reloads kernel arguments inside the loop, ~1 us per launch).
template <bool kClasses, int BM = 256, int BN = kBN>
__global__ __launch_bounds__(kIgThreads, 1) void igemm_fp8_kernel(const IgemmArgs p) {
  // this instance's tile (IgCfg); the names shadow the default tile's constants
  using Cfg = IgCfg<BM, BN>;
  constexpr int kBM = Cfg::kBM, kBN = Cfg::kBN, kWavesM = Cfg::kWavesM, kWTM = Cfg::kWTM;
  constexpr int kWTN = Cfg::kWTN, kFA = Cfg::kFA, kCB = Cfg::kCB;
  constexpr int kALoads = Cfg::kALoads, kBLoads = Cfg::kBLoads, kBLoadWaves = Cfg::kBLoadWaves;
  constexpr int kLoadsPerStage = Cfg::kLoadsPerStage;
  constexpr int kARowsPerWave = Cfg::kARowsPerWave, kBRowsPerWave = Cfg::kBRowsPerWave;
  constexpr int kSlotG = Cfg::kSlotG;
  // three pipeline stages and the per-wave epilogue slots: 3 x 48 KB + 8 x 2 KB = 160 KB
  // (BM = 256), 3 x 32 KB + 8 x 1 KB (BM = 128)
  __shared__ __attribute__((aligned(1024))) uint8_t ig_st[3][Cfg::kStageBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t ig_slot[kWaves][Cfg::kSlotBytes];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % kWavesM;  // pixel block (kWTM rows)
  const int wn = wave / kWavesM;  // channel block (kWTN cols)
  const int frow = lane & 15, fq = lane >> 4;
  // this wave loads B rows (all waves but with the 64 x 32 tile); wave-uniform
  const bool b_wave =
      kBLoadWaves == kWaves || __builtin_amdgcn_readfirstlane(wave) < kBLoadWaves;

  // this workgroup's work items (tile, K range): XCD x owns items [x*tiles_per_xcd,
  // +tiles_per_xcd); its wg_per_xcd workgroups take them round-robin
  const int xcd = blockIdx.x & 7;
  const int wi = blockIdx.x >> 3;
  const int t_begin = xcd * p.tiles_per_xcd + wi;
  int t_end = (xcd + 1) * p.tiles_per_xcd;
  if (t_end > p.tiles) t_end = p.tiles;
  if (t_begin >= t_end) return;
  const int nt = (t_end - t_begin + p.wg_per_xcd - 1) / p.wg_per_xcd;
  const int nk = p.nk;
  const int total = nt * nk;
  const float scale = p.sa[0] * p.sb[0];

  // ---- DMA side: row metadata of the tile being loaded ----
  int a_off[kALoads], a_mask[kALoads], b_off[kBLoads];
  int dma_tile = -1;
  int dma_k0 = 0;  // first global K-step of the item being loaded
  int dma_dy0 = 0, dma_dx0 = 0, dma_w0 = 0, dma_ny = 0, dma_nx = 0;  // its class's taps
  auto set_dma_tile = [&](int j) __attribute__((always_inline)) {
    const int item = t_begin + j * p.wg_per_xcd;
    const int tile = (int)fdiv((uint32_t)item, p.divSP);
    dma_k0 = (item - tile * p.splits) * nk;
    int tic = tile;
    if constexpr (kClasses) {
      const uint32_t cw = cls_word(p, tile_class(p, tile, tic));
      dma_dy0 = cls_field(cw, kClsDy0);
      dma_dx0 = cls_field(cw, kClsDx0);
      dma_w0 = cls_field(cw, kClsW0);
      dma_ny = cls_field(cw, kClsNy);
      dma_nx = cls_field(cw, kClsNx);
    } else {
      dma_dy0 = p.dy0;
      dma_dx0 = p.dx0;
      dma_w0 = p.w0;
      dma_ny = p.ny;
      dma_nx = p.nx;
    }
    const int tm = (int)fdiv((uint32_t)tic, p.divTN);
    const int tn = tic - tm * p.tiles_n;
    const int m0 = tm * kBM, n0 = tn * kBN;
#pragma unroll
    for (int r = 0; r < kALoads; ++r) {
      const int row = wave * kARowsPerWave + 8 * r + (lane >> 3);
      const int g = (lane & 7) ^ swz(row);
      const int m = m0 + row;
      int off = 0, mask = 0;
      if (m < p.M) {
        int n, ii, jj;
        decode_pixel(p, m, n, ii, jj);
        const int iy0 = ii * p.iy_step, ix0 = jj * p.ix_step;
        off = ((n * p.Hi + iy0) * p.Wi + ix0) * p.C + g * 16;
#pragma unroll
        for (int ty = 0; ty < kMaxTapDim; ++ty) {
#pragma unroll
          for (int tx = 0; tx < kMaxTapDim; ++tx) {
            const int iy = iy0 + dma_dy0 + ty * p.dys, ix = ix0 + dma_dx0 + tx * p.dxs;
            const bool in = (ty < dma_ny) & (tx < dma_nx) & ((unsigned)iy < (unsigned)p.Hi) &
                            ((unsigned)ix < (unsigned)p.Wi);
            mask |= (int)in << (ty * p.nx + tx);
          }
        }
      }
      a_off[r] = off;
      a_mask[r] = mask;
    }
#pragma unroll
    for (int r = 0; r < kBLoads; ++r) {
      const int row = wave * kBRowsPerWave + 8 * r + (lane >> 3);
      b_off[r] = (n0 + row) * p.T * p.C + ((lane & 7) ^ swz(row)) * 16;
    }
  };
  // DMA of global step s (tile s / nk, K-step s % nk) into stage buffer st. Steps past the
  // end load the zero page, so every step issues the same number of DMAs and the wait
  // counts stay compile-time constants.
  auto issue = [&](uint8_t* st, int s) __attribute__((always_inline)) {
    const bool live = s < total;
    const int ss = live ? s : 0;
    const int j = (int)fdiv((uint32_t)ss, p.divNK);
    if (live && j != dma_tile) {
      set_dma_tile(j);
      dma_tile = j;
    }
    const int k = ss - j * nk + dma_k0;
    const int t = (int)fdiv((uint32_t)k, p.divKC);
    const int c0 = (k - t * p.kc_per_tap) * kBK;
    const int ty = (int)fdiv((uint32_t)t, p.divNX);
    const int tx = t - ty * p.nx;
    const int ad = ((dma_dy0 + ty * p.dys) * p.Wi + dma_dx0 + tx * p.dxs) * p.C + c0;
    // a tap past the class's own grid has only zero A rows; its B rows come from the class's
    // first tap (a valid address; the products are zero)
    const bool tap_ok = !kClasses || ((ty < dma_ny) & (tx < dma_nx));
    const int wd = (tap_ok ? dma_w0 + ty * p.wys + tx * p.wxs : dma_w0) * p.C + c0;
#pragma unroll
    for (int r = 0; r < kALoads; ++r) {
      const bool ok = live & ((a_mask[r] >> t) & 1);
      const uint8_t* real = p.act + (uint32_t)(a_off[r] + ad);
      // 8 rows of the A tile: 1 KB, lane i -> row +i/8, granule slot i%8
      dma16(ok ? real : (const uint8_t*)g_zero16, st + (wave * kARowsPerWave + 8 * r) * kBK);
    }
    if (b_wave) {
#pragma unroll
      for (int r = 0; r < kBLoads; ++r) {
        const uint8_t* real = p.wgt + (uint32_t)(b_off[r] + wd);
        dma16(live ? real : (const uint8_t*)g_zero16,
              st + kBM * kBK + (wave * kBRowsPerWave + 8 * r) * kBK);
      }
    }
  };
  // until at most n stages of this wave's DMAs are in flight
  auto wait_stages = [&](auto n) __attribute__((always_inline)) {
    if (b_wave)
      wait_vmcnt<decltype(n)::value * kLoadsPerStage>();
    else
      wait_vmcnt<decltype(n)::value * kALoads>();
  };

  // ---- compute side ----
  v4f acc[kCB][kFA];
#pragma unroll
  for (int i = 0; i < kCB; ++i)
#pragma unroll
    for (int j = 0; j < kFA; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
  v8i fa[kFA], fb[kCB];

  // finished item j: scale, bias, bf16 -> wave slot -> 128-B runs per pixel; or, with
  // split K, the raw fp32 sums of its K range as the accumulators hold them: item i's
  // kBM x kBN block at partial + i * kBM * kBN, wave-major, then (pj, ci, lane), 16 B per
  // lane, so every store instruction writes 1 KB contiguously
  auto epilogue = [&](int j) __attribute__((always_inline)) {
    const int item = t_begin + j * p.wg_per_xcd;
    const int tile = (int)fdiv((uint32_t)item, p.divSP);
    int tic = tile, oy_off = p.oy_off, ox_off = p.ox_off;
    if constexpr (kClasses) {
      const uint32_t cw = cls_word(p, tile_class(p, tile, tic));
      oy_off = cls_field(cw, kClsOy);
      ox_off = cls_field(cw, kClsOx);
    }
    const int tm = (int)fdiv((uint32_t)tic, p.divTN);
    const int tn = tic - tm * p.tiles_n;
    const int m0 = tm * kBM, n0 = tn * kBN;
    const int c0 = n0 + wn * kWTN;
    if constexpr (BM == 256 && BN == dpa::kBN) {  // (launch_igemm splits the default tile only)
      if (p.splits > 1) {
        float* part = p.partial + (int64_t)item * (kBM * kBN) + wave * (16 * 256) + lane * 4;
#pragma unroll
        for (int pj = 0; pj < 4; ++pj) {
#pragma unroll
          for (int ci = 0; ci < 4; ++ci) {
            __builtin_nontemporal_store(acc[ci][pj],
                                        reinterpret_cast<v4f*>(part + (pj * 4 + ci) * 256));
            acc[ci][pj] = v4f{0.f, 0.f, 0.f, 0.f};
          }
        }
        return;
      }
    }
    uint8_t* slot = ig_slot[wave];
#pragma unroll
    for (int pj = 0; pj < kFA; ++pj) {
#pragma unroll
      for (int ci = 0; ci < kCB; ++ci) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[ci][pj][e] * scale;
        if (p.bias) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = v[e] + p.bias[c0 + ci * 16 + 4 * fq + e];
        }
        const int g = 2 * ci + (fq >> 1);  // 16-B granule of channels ci*16 + 4*fq
        uint2 o;
        o.x = pack_bf16x2(v[0], v[1]);
        o.y = pack_bf16x2(v[2], v[3]);
        *reinterpret_cast<uint2*>(slot + frow * (16 * kSlotG) +
                                  ((g ^ (frow & (kSlotG - 1))) * 16) + (fq & 1) * 8) = o;
      }
      // the slot's 16 x kSlotG 16-B chunks, one per lane and pass
#pragma unroll
      for (int rr = 0; rr < (16 * kSlotG + 63) / 64; ++rr) {
        const int c = lane + 64 * rr;
        const int r = c / kSlotG, g = c % kSlotG;
        if (16 * kSlotG >= 64 || c < 16 * kSlotG) {
          const uint4 v = *reinterpret_cast<const uint4*>(slot + r * (16 * kSlotG) +
                                                          ((g ^ (r & (kSlotG - 1))) * 16));
          const int m = m0 + wm * kWTM + pj * 16 + r;
          if (m < p.M) st_nt16(p.out + out_offset(p, m, oy_off, ox_off) + c0 + g * 8, v);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < kCB; ++i)
#pragma unroll
      for (int jj = 0; jj < kFA; ++jj) acc[i][jj] = v4f{0.f, 0.f, 0.f, 0.f};
  };

  issue(ig_st[0], 0);
  issue(ig_st[1], 1);
  issue(ig_st[2], 2);
  wait_stages(std::integral_constant<int, 2>{});
  lds_barrier();
#pragma unroll
  for (int i = 0; i < kCB; ++i) fb[i] = ld_frag(ig_st[0] + kBM * kBK, wn * kWTN + i * 16 + frow, fq);
#pragma unroll
  for (int i = 0; i < kFA; ++i) fa[i] = ld_frag(ig_st[0], wm * kWTM + i * 16 + frow, fq);

  // Step s on stage buffer cur = s % 3: wait until stage s+1 has landed (its DMA was issued
  // two steps earlier), barrier (every wave finished reading stage s), then the 16 MFMAs on
  // stage s's fragments with stage s+1's fragments read in between, and queue the DMA of
  // stage s+3 into buffer cur.
  int cur = 0, kstep = 0;
  for (int s = 0; s < total; ++s) {
    const int nx = cur == 2 ? 0 : cur + 1;
    wait_stages(std::integral_constant<int, 1>{});
    wait_lgkmcnt0();
    lds_barrier();
    const uint8_t* nxt = ig_st[nx];
#pragma unroll
    for (int pj = 0; pj < kFA; ++pj) {
#pragma unroll
      for (int ci = 0; ci < kCB; ++ci) acc[ci][pj] = mfma16x16x128_e4m3(fb[ci], fa[pj], acc[ci][pj]);
      fa[pj] = ld_frag(nxt, wm * kWTM + pj * 16 + frow, fq);
      __builtin_amdgcn_sched_group_barrier(0x008, kCB, 0);  // kCB MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // then 2 DS reads
    }
    issue(ig_st[cur], s + 3);
#pragma unroll
    for (int i = 0; i < kCB; ++i) fb[i] = ld_frag(nxt + kBM * kBK, wn * kWTN + i * 16 + frow, fq);
    if (++kstep == nk) {
      kstep = 0;
      epilogue((int)fdiv((uint32_t)s, p.divNK));
    }
    cur = nx;
  }
  wait_vmcnt<0>();  // trailing zero-page DMAs land before the workgroup retires
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

// Split-K finish: out = bf16(RN32(RN32(sum over splits, in order) * RN32(sa * sb)) [+ bias]).
// Thread (tile, wave, pj, ci, lane) of the partial layout above sums the splits of one
// accumulator block (1 KB-contiguous loads per wave) and writes pixel
// m0 + 64 wm + 16 pj + frow, channels c0 + 16 ci + 4 fq .. +3. Grid: tiles x 8192 threads.
constexpr int kRedThreadsPerTile = kWaves * 16 * 64;
__global__ __launch_bounds__(256) void igemm_split_reduce_kernel(const IgemmArgs p) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  const int tile = t / kRedThreadsPerTile;
  const int r = t - tile * kRedThreadsPerTile;
  const int wave = r >> 10, pj = (r >> 8) & 3, ci = (r >> 6) & 3, lane = r & 63;
  const int tm = (int)fdiv((uint32_t)tile, p.divTN);
  const int tn = tile - tm * p.tiles_n;
  const int m = tm * kBM + (wave % kWavesM) * kWTM + pj * 16 + (lane & 15);
  if (m >= p.M) return;
  const int c = tn * kBN + (wave / kWavesM) * kWTN + ci * 16 + 4 * (lane >> 4);
  const float* q = p.partial + (int64_t)tile * p.splits * (kBM * kBN) + r * 4;
  v4f acc = *reinterpret_cast<const v4f*>(q);
  for (int sp = 1; sp < p.splits; ++sp)
    acc = acc + *reinterpret_cast<const v4f*>(q + (int64_t)sp * (kBM * kBN));
  const float scale = p.sa[0] * p.sb[0];
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = acc[e] * scale;
    if (p.bias) v[e] = v[e] + p.bias[c + e];
  }
  uint2 o;
  o.x = pack_bf16x2(v[0], v[1]);
  o.y = pack_bf16x2(v[2], v[3]);
  st_nt8(p.out + out_offset(p, m, p.oy_off, p.ox_off) + c, o);
}

static int g_num_cus = 0;

static int num_cus() {
  if (g_num_cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      g_num_cus = n;
    else
      g_num_cus = 256;
  }
  return g_num_cus;
}

// Split-K plan for a launch of `tiles` output tiles and nk K-steps per tile. Each split adds
// a fixed cost per work item (pipeline fill, a 128 KB fp32 partial block written and read
// back), so a split pays only when the tiles leave most CUs idle and each part keeps enough
// K-steps. Measured on MI355X (event time, both kernels, 4x4 and 8x8 U-Net shapes): about six
// K-steps per part is best once there are 16+ tiles, and tiny launches (fewer tiles) gain
// from parts of two steps when the tile has at least eight. Picks the largest divisor d of
// nk with nk / d >= that minimum and tiles * d <= CUs; 1 means no split. *bytes gets the
// partial buffer it needs (one kBM x kBN fp32 block per work item).
static int plan_splits(int tiles, int nk, int cus, int64_t* bytes) {
  int best = 1;
  if (nk >= 8 && tiles * 2 <= cus) {
    const int min_steps = (tiles >= 16 && nk >= 12) ? 6 : 2;
    for (int d = 2; d <= nk / min_steps; ++d)
      if (nk % d == 0 && tiles * d <= cus) best = d;
  }
  *bytes = best > 1 ? (int64_t)best * tiles * kBM * kBN * 4 : 0;
  return best;
}

// Small-tile choice (launch_igemm), measured on the U-Net's 8x8 / 4x4 convs and the stride-2
// conv: 64-pixel tiles win wherever 128-pixel ones would fill at most half the CUs; allowing
// 36 K-steps per unsplit tile (the 512-channel 4x4 convs) instead of 18 changed nothing.
constexpr int kHalfMaxSteps = 18;  // two 128-channel chunks of a 3x3 conv
constexpr int kQuarterFill = 2;

static void finish_geometry(IgemmArgs& a) {
  a.kc_per_tap = a.C / kBK;
  a.nk = a.ny * a.nx * a.kc_per_tap;
  a.tiles_n = a.Cout / kBN;
}

static int64_t igemm_workspace(IgemmArgs& a) {
  if (a.M <= 0) return 0;
  finish_geometry(a);
  const int tiles = (int)ceil_div(a.M, kBM) * a.tiles_n;
  int64_t bytes = 0;
  plan_splits(tiles, a.nk, num_cus(), &bytes);
  return bytes;
}

// act geometry (N, Hi, Wi, C), output geometry, tap grid already in `a`; split K when a
// workspace of the planned size is given
static int launch_igemm(IgemmArgs& a, int N, hipStream_t s, void* workspace,
                        int64_t workspace_bytes) {
  if (a.M <= 0) return DPA_OK;
  const int64_t act_bytes = (int64_t)N * a.Hi * a.Wi * a.C;
  const int64_t wgt_bytes = (int64_t)a.Cout * a.T * a.C;
  const int64_t out_elems = (int64_t)N * a.Ho * a.Wo * a.Cout;
  if (act_bytes > kMaxOperandBytes || wgt_bytes > kMaxOperandBytes || out_elems > kMaxOperandBytes)
    return DPA_ERR_SIZE;
  finish_geometry(a);
  if (a.nclass <= 1) a.nclass = 1;  // one class: the scalar tap grid
  // Launches whose 256-pixel tiles would leave at least half the CUs idle take 128-pixel
  // tiles (twice as many) unsplit, when a tile has at most kHalfMaxSteps K-steps, and
  // 64-pixel tiles when the 128-pixel ones would still leave half the CUs idle.
  int bm = kBM, bn = kBN;
  if (a.nclass == 1 && a.nk <= kHalfMaxSteps) {
    const int cus = num_cus();
    if (ceil_div(a.M, 256) * a.tiles_n * 2 <= cus) bm = 128;
    if (bm == 128 && ceil_div(a.M, 128) * a.tiles_n * kQuarterFill <= cus) bm = 64;
    // 64 x 32 tiles where the 64 x 128 ones fill at most a quarter of the CUs
    if (bm == 64 && ceil_div(a.M, 64) * a.tiles_n * 4 <= cus) bn = 32;
  }
  a.tiles_n = a.Cout / bn;
  const bool half = bm < kBM;
  const int tiles_m = (int)ceil_div(a.M, bm);
  a.tiles_pc = tiles_m * a.tiles_n;
  const int tiles = a.tiles_pc * a.nclass;
  int64_t need = 0;
  int splits = half ? 1 : plan_splits(tiles, a.nk, num_cus(), &need);
  // the split reduce writes class 0's pixels only: several classes run unsplit
  if (splits > 1 && (a.nclass > 1 || !workspace || workspace_bytes < need ||
                     !aligned(workspace, 16)))
    splits = 1;
  a.splits = splits;
  a.partial = (float*)workspace;
  a.nk /= splits;
  a.tiles = tiles * splits;
  a.tiles_per_xcd = (int)ceil_div(a.tiles, 8);
  // one workgroup per CU (160 KB of LDS each), never more than there are work items
  int grid = num_cus();
  grid = (grid / 8) * 8;
  if (grid < 8) grid = 8;
  const int max_grid = a.tiles_per_xcd * 8;
  if (grid > max_grid) grid = max_grid;
  a.wg_per_xcd = grid / 8;
  a.divQ = make_fastdiv((uint32_t)a.Qg);
  a.divP = make_fastdiv((uint32_t)a.Pg);
  a.divKC = make_fastdiv((uint32_t)a.kc_per_tap);
  a.divNX = make_fastdiv((uint32_t)a.nx);
  a.divNK = make_fastdiv((uint32_t)a.nk);
  a.divTN = make_fastdiv((uint32_t)a.tiles_n);
  a.divSP = make_fastdiv((uint32_t)a.splits);
  a.divPC = make_fastdiv((uint32_t)a.tiles_pc);
  if (a.nclass > 1)
    igemm_fp8_kernel<true><<<(unsigned)grid, kIgThreads, 0, s>>>(a);
  else if (bm == 128)
    igemm_fp8_kernel<false, 128><<<(unsigned)grid, kIgThreads, 0, s>>>(a);
  else if (bm == 64 && bn == 32)
    igemm_fp8_kernel<false, 64, 32><<<(unsigned)grid, kIgThreads, 0, s>>>(a);
  else if (bm == 64)
    igemm_fp8_kernel<false, 64><<<(unsigned)grid, kIgThreads, 0, s>>>(a);
  else
    igemm_fp8_kernel<false><<<(unsigned)grid, kIgThreads, 0, s>>>(a);
  int st = launch_status();
  if (st != DPA_OK || splits == 1) return st;
  igemm_split_reduce_kernel<<<(unsigned)(tiles * (kRedThreadsPerTile / 256)), 256, 0, s>>>(a);
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

// halo-patch kernel for 3x3 / stride 1 / pad 1 on 16- and 32-pixel-wide images (hconv.hip)
bool hconv_supported(int N, int H, int W, int C, int Cout);
int hconv_run(const void* act, const void* wgt, const float* sa, const float* sb,
              const float* bias, void* out, int N, int H, int W, int C, int Cout, int flip,
              int wfrag, int num_cus, hipStream_t s);
int weight_frag_run(const void* w, void* out, int rows, int K, int T, int transpose,
                    hipStream_t s);

static bool use_hconv(int N, int H, int W, int C, int Cout, int R, int S, int stride, int pad) {
  return R == 3 && S == 3 && stride == 1 && pad == 1 && hconv_supported(N, H, W, C, Cout);
}

static void fwd_geometry(IgemmArgs& a, int N, int H, int W, int Cin, int Cout, int R, int S,
                         int stride, int pad) {
  const int P = (H + 2 * pad - R) / stride + 1;
  const int Q = (W + 2 * pad - S) / stride + 1;
  a.Hi = H; a.Wi = W; a.C = Cin; a.Cout = Cout; a.T = R * S;
  a.Pg = P; a.Qg = Q; a.Ho = P; a.Wo = Q;
  a.oy_step = 1; a.oy_off = 0; a.ox_step = 1; a.ox_off = 0;
  a.iy_step = stride; a.ix_step = stride;
  a.M = N * P * Q;
  // tap (r, s): input offset (r - pad, s - pad), weight tap r*S + s
  a.ny = R; a.nx = S;
  a.dy0 = -pad; a.dys = 1; a.dx0 = -pad; a.dxs = 1;
  a.w0 = 0; a.wys = S; a.wxs = 1;
}

static int conv_fwd(const void* xq, const void* wq, const float* xs, const float* ws,
                    const float* bias, void* y, int N, int H, int W, int Cin, int Cout, int R,
                    int S, int stride, int pad, hipStream_t s, void* workspace = nullptr,
                    int64_t workspace_bytes = 0) {
  // the halo-patch kernel's epilogue stores 16 B per lane
  if (use_hconv(N, H, W, Cin, Cout, R, S, stride, pad) && aligned(y, 16))
    return hconv_run(xq, wq, xs, ws, bias, y, N, H, W, Cin, Cout, 0, 0, num_cus(), s);
  IgemmArgs a{};
  fill_common(a, xq, wq, y, xs, ws, bias);
  fwd_geometry(a, N, H, W, Cin, Cout, R, S, stride, pad);
  return launch_igemm(a, N, s, workspace, workspace_bytes);
}

static int64_t conv_fwd_workspace(int N, int H, int W, int Cin, int Cout, int R, int S,
                                  int stride, int pad) {
  if (use_hconv(N, H, W, Cin, Cout, R, S, stride, pad)) return 0;
  IgemmArgs a{};
  fwd_geometry(a, N, H, W, Cin, Cout, R, S, stride, pad);
  return igemm_workspace(a);
}

// dx[n, h, w, ci] = sum_{r,s,co} dy[n, (h+pad-r)/st, (w+pad-s)/st, co] * w[co, r, s, ci]
// over the (r, s) for which the division is exact and in range: one launch per output
// parity class (ay, ax); within a class the usable r (and s) form an arithmetic progression
// of step `stride`, so the class's taps are again a linear grid.
// Parity class (ay, ax) of the data gradient: the class's output pixels and taps.
static int dgrad_geometry(IgemmArgs& a, int N, int H, int W, int Cin, int Cout, int R, int S,
                      int stride, int pad, int ay, int ax) {
  const int P = (H + 2 * pad - R) / stride + 1;
  const int Q = (W + 2 * pad - S) / stride + 1;
  a.Hi = P; a.Wi = Q; a.C = Cout; a.Cout = Cin; a.T = R * S;
  a.Pg = (H - ay + stride - 1) / stride;
  a.Qg = (W - ax + stride - 1) / stride;
  a.Ho = H; a.Wo = W;
  a.oy_step = stride; a.oy_off = ay; a.ox_step = stride; a.ox_off = ax;
  a.iy_step = 1; a.ix_step = 1;
  a.M = N * a.Pg * a.Qg;
  // first r with (ay + pad - r) divisible by stride, then every stride-th
  const int r0 = (ay + pad) % stride, s0 = (ax + pad) % stride;
  a.ny = (R - r0 + stride - 1) / stride;
  a.nx = (S - s0 + stride - 1) / stride;
  if (a.ny <= 0 || a.nx <= 0 || a.M == 0) return DPA_ERR_SHAPE;
  a.dy0 = (ay + pad - r0) / stride; a.dys = -1;
  a.dx0 = (ax + pad - s0) / stride; a.dxs = -1;
  a.w0 = r0 * S + s0; a.wys = stride * S; a.wxs = stride;
  return DPA_OK;
}

// A strided data gradient whose parity classes all have the same output grid (H and W
// multiples of the stride) runs as one launch of all classes: every class has its own tap
// grid inside the largest one, padded with zero taps, so the classes share K-step counts.
static bool dgrad_classes_merge(int H, int W, int stride) {
  return stride > 1 && stride * stride <= 4 && H % stride == 0 && W % stride == 0;
}

static int dgrad_merged_geometry(IgemmArgs& a, int N, int H, int W, int Cin, int Cout, int R,
                                 int S, int stride, int pad) {
  int c = 0, ny = 0, nx = 0;
  for (int ay = 0; ay < stride; ++ay)
    for (int ax = 0; ax < stride; ++ax, ++c) {
      IgemmArgs g{};
      const int st = dgrad_geometry(g, N, H, W, Cin, Cout, R, S, stride, pad, ay, ax);
      if (st != DPA_OK) return st;
      if (c == 0) {
        a.Hi = g.Hi; a.Wi = g.Wi; a.C = g.C; a.Cout = g.Cout; a.T = g.T;
        a.Pg = g.Pg; a.Qg = g.Qg; a.Ho = g.Ho; a.Wo = g.Wo;
        a.oy_step = g.oy_step; a.ox_step = g.ox_step; a.iy_step = g.iy_step;
        a.ix_step = g.ix_step; a.M = g.M;
        a.dys = g.dys; a.dxs = g.dxs; a.wys = g.wys; a.wxs = g.wxs;
        a.oy_off = g.oy_off; a.ox_off = g.ox_off; a.dy0 = g.dy0; a.dx0 = g.dx0; a.w0 = g.w0;
      } else if (g.Pg != a.Pg || g.Qg != a.Qg) {
        return DPA_ERR_SHAPE;
      }
      const int f[7] = {g.oy_off, g.ox_off, g.dy0, g.dx0, g.w0, g.ny, g.nx};
      uint32_t w = 0;
      for (int i = 0; i < 7; ++i) {
        if (f[i] < 0 || f[i] > 15) return DPA_ERR_SHAPE;
        w |= (uint32_t)f[i] << (4 * i);
      }
      a.cls[c] = w;
      ny = g.ny > ny ? g.ny : ny;
      nx = g.nx > nx ? g.nx : nx;
    }
  a.nclass = c;
  a.ny = ny;
  a.nx = nx;
  return DPA_OK;
}

static int conv_dgrad(const void* dyq, const void* wt, const float* dys, const float* ws,
                      void* dx, int N, int H, int W, int Cin, int Cout, int R, int S,
                      int stride, int pad, hipStream_t s, void* workspace = nullptr,
                      int64_t workspace_bytes = 0) {
  // the 3x3 / s1 / p1 data gradient is a conv of dy with the mirrored, transposed weight
  if (use_hconv(N, H, W, Cout, Cin, R, S, stride, pad) && aligned(dx, 16))
    return hconv_run(dyq, wt, dys, ws, nullptr, dx, N, H, W, Cout, Cin, 1, 0, num_cus(), s);
  if (dgrad_classes_merge(H, W, stride)) {
    IgemmArgs a{};
    fill_common(a, dyq, wt, dx, dys, ws, nullptr);
    const int st = dgrad_merged_geometry(a, N, H, W, Cin, Cout, R, S, stride, pad);
    if (st != DPA_OK) return st;
    return launch_igemm(a, N, s, nullptr, 0);
  }
  for (int ay = 0; ay < stride; ++ay)
    for (int ax = 0; ax < stride; ++ax) {
      IgemmArgs a{};
      fill_common(a, dyq, wt, dx, dys, ws, nullptr);
      int st = dgrad_geometry(a, N, H, W, Cin, Cout, R, S, stride, pad, ay, ax);
      if (st != DPA_OK) return st;
      st = launch_igemm(a, N, s, workspace, workspace_bytes);  // classes run in stream order
      if (st != DPA_OK) return st;
    }
  return DPA_OK;
}

static int64_t conv_dgrad_workspace(int N, int H, int W, int Cin, int Cout, int R, int S,
                                    int stride, int pad) {
  if (use_hconv(N, H, W, Cout, Cin, R, S, stride, pad)) return 0;
  if (dgrad_classes_merge(H, W, stride)) return 0;  // one launch, never split
  int64_t most = 0;
  for (int ay = 0; ay < stride; ++ay)
    for (int ax = 0; ax < stride; ++ax) {
      IgemmArgs a{};
      if (dgrad_geometry(a, N, H, W, Cin, Cout, R, S, stride, pad, ay, ax) != DPA_OK) continue;
      const int64_t b = igemm_workspace(a);
      if (b > most) most = b;
    }
  return most;
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
  if (use_hconv(N, H, W, Cout, Cin, R, S, stride, pad) && aligned(dx, 16)) {
    // the halo-patch kernel takes the transposed, mirrored weight in its fragment layout
    int st = weight_frag_run(wq, workspace, Cin, Cout, R * S, 1, (hipStream_t)stream);
    if (st != DPA_OK) return st;
    return hconv_run(dyq, workspace, dy_scale, w_scale, nullptr, dx, N, H, W, Cout, Cin, 0, 1,
                     num_cus(), (hipStream_t)stream);
  }
  int st = dpa_weight_transpose_fp8(wq, workspace, Cout, R, S, Cin, stream);
  if (st != DPA_OK) return st;
  return conv_dgrad(dyq, workspace, dy_scale, w_scale, dx, N, H, W, Cin, Cout, R, S, stride,
                    pad, (hipStream_t)stream);
}

// ---- fragment-native weights for the 3x3 / stride-1 / pad-1 halo-patch kernel ----

extern "C" int64_t dpa_weight_frag_bytes(int Cout, int R, int S, int Cin) {
  if (Cout <= 0 || Cin <= 0 || R <= 0 || S <= 0) return 0;
  return (int64_t)Cout * R * S * Cin;
}

extern "C" int dpa_weight_frag_fp8(const void* wq, void* wf, void* wf_dgrad, int Cout, int R,
                                   int S, int Cin, void* stream) {
  if (!wq || (!wf && !wf_dgrad)) return DPA_ERR_NULL;
  if (Cout <= 0 || Cin <= 0 || R <= 0 || S <= 0) return DPA_ERR_SIZE;
  if (Cout % kBN != 0 || Cin % kBK != 0) return DPA_ERR_SHAPE;
  if (!aligned(wq, 16) || !aligned(wf, 16) || !aligned(wf_dgrad, 16)) return DPA_ERR_ALIGN;
  int st = DPA_OK;
  if (wf) st = weight_frag_run(wq, wf, Cout, Cin, R * S, 0, (hipStream_t)stream);
  if (st == DPA_OK && wf_dgrad)
    st = weight_frag_run(wq, wf_dgrad, Cin, Cout, R * S, 1, (hipStream_t)stream);
  return st;
}

extern "C" int dpa_conv2d_fwd_fp8_wf(const void* xq, const void* wf, const float* x_scale,
                                     const float* w_scale, const float* bias, void* y, int N,
                                     int H, int W, int Cin, int Cout, void* stream) {
  if (!xq || !wf || !x_scale || !w_scale || !y) return DPA_ERR_NULL;
  if (!use_hconv(N, H, W, Cin, Cout, 3, 3, 1, 1)) return DPA_ERR_SHAPE;
  if (!aligned(xq, 16) || !aligned(wf, 16) || !aligned(y, 16)) return DPA_ERR_ALIGN;
  return hconv_run(xq, wf, x_scale, w_scale, bias, y, N, H, W, Cin, Cout, 0, 1, num_cus(),
                   (hipStream_t)stream);
}

extern "C" int dpa_conv2d_dgrad_fp8_wf(const void* dyq, const void* wf_dgrad,
                                       const float* dy_scale, const float* w_scale, void* dx,
                                       int N, int H, int W, int Cin, int Cout, void* stream) {
  if (!dyq || !wf_dgrad || !dy_scale || !w_scale || !dx) return DPA_ERR_NULL;
  if (!use_hconv(N, H, W, Cout, Cin, 3, 3, 1, 1)) return DPA_ERR_SHAPE;
  if (!aligned(dyq, 16) || !aligned(wf_dgrad, 16) || !aligned(dx, 16)) return DPA_ERR_ALIGN;
  return hconv_run(dyq, wf_dgrad, dy_scale, w_scale, nullptr, dx, N, H, W, Cout, Cin, 0, 1,
                   num_cus(), (hipStream_t)stream);
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

// ---- split-K variants: same results up to fp32 summation order, for launches whose output
// tiles leave most CUs idle (small images, small batches) ----

extern "C" int64_t dpa_conv2d_fwd_split_workspace_bytes(int N, int H, int W, int Cin, int Cout,
                                                         int R, int S, int stride, int pad) {
  if (!conv_shape_ok(N, H, W, Cin, Cout, R, S, stride, pad)) return 0;
  return conv_fwd_workspace(N, H, W, Cin, Cout, R, S, stride, pad);
}

extern "C" int dpa_conv2d_fwd_fp8_split(const void* xq, const void* wq, const float* x_scale,
                                        const float* w_scale, const float* bias, void* y,
                                        void* workspace, int64_t workspace_bytes, int N, int H,
                                        int W, int Cin, int Cout, int R, int S, int stride,
                                        int pad, void* stream) {
  if (!xq || !wq || !x_scale || !w_scale || !y) return DPA_ERR_NULL;
  if (!conv_shape_ok(N, H, W, Cin, Cout, R, S, stride, pad)) return DPA_ERR_SHAPE;
  if (workspace_bytes < conv_fwd_workspace(N, H, W, Cin, Cout, R, S, stride, pad) ||
      (workspace_bytes > 0 && !workspace))
    return DPA_ERR_WORKSPACE;
  if (!aligned(xq, 16) || !aligned(wq, 16) || !aligned(y, 8) || !aligned(workspace, 16))
    return DPA_ERR_ALIGN;
  return conv_fwd(xq, wq, x_scale, w_scale, bias, y, N, H, W, Cin, Cout, R, S, stride, pad,
                  (hipStream_t)stream, workspace, workspace_bytes);
}

extern "C" int64_t dpa_conv2d_dgrad_split_workspace_bytes(int N, int H, int W, int Cin, int Cout,
                                                           int R, int S, int stride, int pad) {
  if (!conv_shape_ok(N, H, W, Cout, Cin, R, S, stride, pad)) return 0;
  return conv_dgrad_workspace(N, H, W, Cin, Cout, R, S, stride, pad);
}

extern "C" int dpa_conv2d_dgrad_fp8_wt_split(const void* dyq, const void* wq_t,
                                             const float* dy_scale, const float* w_scale,
                                             void* dx, void* workspace, int64_t workspace_bytes,
                                             int N, int H, int W, int Cin, int Cout, int R,
                                             int S, int stride, int pad, void* stream) {
  if (!dyq || !wq_t || !dy_scale || !w_scale || !dx) return DPA_ERR_NULL;
  if (!conv_shape_ok(N, H, W, Cout, Cin, R, S, stride, pad)) return DPA_ERR_SHAPE;
  if (workspace_bytes < conv_dgrad_workspace(N, H, W, Cin, Cout, R, S, stride, pad) ||
      (workspace_bytes > 0 && !workspace))
    return DPA_ERR_WORKSPACE;
  if (!aligned(dyq, 16) || !aligned(wq_t, 16) || !aligned(dx, 8) || !aligned(workspace, 16))
    return DPA_ERR_ALIGN;
  return conv_dgrad(dyq, wq_t, dy_scale, w_scale, dx, N, H, W, Cin, Cout, R, S, stride, pad,
                    (hipStream_t)stream, workspace, workspace_bytes);
}

extern "C" int64_t dpa_gemm_split_workspace_bytes(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % kBK != 0 || N % kBN != 0) return 0;
  return conv_fwd_workspace(M, 1, 1, K, N, 1, 1, 1, 0);
}

extern "C" int dpa_gemm_fp8_split(const void* a, const void* b, const float* a_scale,
                                  const float* b_scale, const float* bias, void* c,
                                  void* workspace, int64_t workspace_bytes, int M, int N, int K,
                                  void* stream) {
  if (!a || !b || !a_scale || !b_scale || !c) return DPA_ERR_NULL;
  if (M <= 0 || N <= 0 || K <= 0) return DPA_ERR_SIZE;
  if (K % kBK != 0 || N % kBN != 0) return DPA_ERR_SHAPE;
  if (workspace_bytes < conv_fwd_workspace(M, 1, 1, K, N, 1, 1, 1, 0) ||
      (workspace_bytes > 0 && !workspace))
    return DPA_ERR_WORKSPACE;
  if (!aligned(a, 16) || !aligned(b, 16) || !aligned(c, 8) || !aligned(workspace, 16))
    return DPA_ERR_ALIGN;
  return conv_fwd(a, b, a_scale, b_scale, bias, c, M, 1, 1, K, N, 1, 1, 1, 0,
                  (hipStream_t)stream, workspace, workspace_bytes);
}
