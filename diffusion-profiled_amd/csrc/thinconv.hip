// bf16 3x3 / stride-1 / pad-1 convolutions with an image-channel side: the U-Net's input conv
// (3 -> C) and output conv (C -> 3).
//
// Reference: diffusion/unet.py:255-257 (conv_in) and :325-329 (the output head's conv), both
// nn.Conv2d(bias=False) run in bf16 under autocast (train.py's torch.autocast region): bf16
// operands (x and the fp32 weight rounded to bf16), fp32 accumulation, bf16 output; the weight
// gradient leaves the conv in bf16 and reaches the fp32 weight through the cast's backward.
//
// One side has Ct <= 3 channels ("thin"), the other Cw in {128, 256} ("wide"); NHWC
// activations. All products run on the bf16 MFMA (v_mfma_f32_16x16x32_bf16, fp32
// accumulate); a thin K (9 taps x Ct <= 27) or a thin output (<= 3 of 16 rows) wastes most
// of each MFMA, which costs nothing here: every kernel is bound by the bytes of its wide
// operand.
//   * thin -> wide (conv_in forward; the output conv's data gradient, a conv of dy with the
//     weight transposed and mirrored): per 16 output pixels one B fragment = the 27-value
//     im2col of each pixel (gathered straight from the small input), times Cw/16 weight
//     fragments held in registers; outputs staged through a per-wave LDS slot and written as
//     16-B runs.
//   * wide -> thin (the output conv's forward): a workgroup tile of 64 pixels (whole image
//     rows) reads its (rows + 2) x (W + 2)-pixel input patch into LDS once; each wave's 16
//     pixels take 9 taps x Cw/32 MFMAs with the pixel fragments read from the patch at a
//     per-tap offset and the weights from LDS.
//   * weight gradient: K = pixels. The wide operand's fragments (16 channels x 8 pixels) come
//     from its NHWC tile in LDS by transpose reads (ds_read_b64_tr_b16); the thin operand sits
//     transposed in LDS ([channel][pixel], for a thin x one copy per column shift so every
//     tap's 8-pixel run is one aligned 16-B read). Each workgroup sums its pixel range into
//     fp32 partials; a second kernel adds the partials in workgroup order (deterministic) and
//     writes fp32(bf16(sum)), the value autograd's bf16 conv gradient has after the cast back.
#include "dpa_common.hpp"

namespace dpa {

namespace {

typedef __bf16 tc_bf16x8 __attribute__((ext_vector_type(8)));
typedef short tc_v4s __attribute__((ext_vector_type(4)));

constexpr int kTcThreads = 256;
constexpr int kTcTilePx = 64;  // wide -> thin and weight-gradient tiles: whole rows, 64 pixels
constexpr int kTcMaxW = 64;
constexpr int kTcMaxCt = 3;

// D(16x16 f32) += A(16x32) B(32x16), bf16 operands: lane l supplies row (l & 15) of A and
// column (l & 15) of B, K elements 8 (l >> 4) .. + 7; lane l receives D[4 (l >> 4) + t][l & 15].
__device__ __forceinline__ v4f tc_mfma(uint4 a, uint4 b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(tc_bf16x8, a),
                                                 __builtin_bit_cast(tc_bf16x8, b), c, 0, 0, 0);
}

// gfx950 transpose read: the 16 lanes of a group address a 4-row x 16-column block of 16-bit
// elements (lane k: row k >> 2, columns 4 (k & 3) .. + 3) and lane j receives column j of the
// 4 rows, in row order.
__device__ __forceinline__ uint2 tc_ld_tr16(const uint8_t* p) {
  const tc_v4s v =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((tc_v4s __attribute__((address_space(3)))*)(p));
  return __builtin_bit_cast(uint2, v);
}

__device__ __forceinline__ uint32_t tc_bf16_of(const void* p, int64_t i, int is_f32) {
  if (is_f32) return f32_to_bf16_bits(reinterpret_cast<const float*>(p)[i]);
  return reinterpret_cast<const uint16_t*>(p)[i];
}

struct TcArgs {
  const void* x;       // thin -> wide: the thin input; wide -> thin / wgrad: x
  const void* dy;      // weight gradient: dy
  const void* w;       // [Cout][Cin][3][3] with element strides ws0..ws3
  void* out;           // bf16 output, or fp32 partials (weight gradient)
  int x_f32, w_f32;    // x / w given as fp32 (rounded to bf16 on load) or bf16
  int ws0, ws1, ws2, ws3;
  int N, H, W, Ct, Cw;
  int wshift, TR;      // log2 W; image rows per 64-pixel tile
  int flip;            // thin -> wide: 1 = data gradient (weight [Ct][Cw], taps mirrored)
  int groups;          // thin -> wide: 16-pixel groups (N H W / 16)
  int tiles, tiles_per_wg;  // 64-pixel tiles; weight gradient: tiles per workgroup
  FastDiv divPC;            // by the patch row pitch W + 2
};

// bf16 bits of the weight element the thin -> wide product uses at row r (wide channel) and
// thin index t, tap (ky, kx) of the im2col
__device__ __forceinline__ uint32_t tw_weight(const TcArgs& p, int r, int t, int ky, int kx) {
  int64_t i;
  if (p.flip)  // data gradient: w[co = t][ci = r][2 - ky][2 - kx]
    i = (int64_t)t * p.ws0 + (int64_t)r * p.ws1 + (2 - ky) * p.ws2 + (2 - kx) * p.ws3;
  else
    i = (int64_t)r * p.ws0 + (int64_t)t * p.ws1 + ky * p.ws2 + kx * p.ws3;
  return tc_bf16_of(p.w, i, p.w_f32);
}

// ---- thin -> wide --------------------------------------------------------------------------
// Each wave takes kTwGroups 16-pixel groups; per group the B fragment (lane: pixel l & 15,
// im2col elements k = 8 (l >> 4) + j, k = tap * Ct + t, zero past 9 Ct) times NB = Cw / 16
// weight fragments, which the workgroup builds once into LDS ([cb][lane] 16 B) and every wave
// copies into registers. Output block cb: lane l holds channels 16 cb + 4 (l >> 4) .. + 3 of
// pixel l & 15; they go into the wave's slot [16 px][Cw] (16-B granule g of pixel row px at
// g ^ (px & 15)), then each lane stores 16 contiguous bytes, 1 KB per instruction.
constexpr int kTwGroups = 4;
constexpr int kTwtGrid = 512;

template <bool kXF32, int NB>
__global__ __launch_bounds__(kTcThreads) void tc_thin_wide_kernel(const TcArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t slot_all[kTcThreads / 64][16 * NB * 16 * 2];
  __shared__ __attribute__((aligned(16))) uint4 wfrag[NB][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15, ks = lane >> 4;
  constexpr int Cw = NB * 16;
  constexpr int kRowBytes = Cw * 2;
  uint8_t* slot = slot_all[wave];

  // im2col coordinates of this lane's 8 K elements (the same for every fragment lane l)
  int kdy[8], kdx[8], kt[8];
  bool kv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int k = 8 * ks + j;
    const int tap = k / p.Ct;
    kv[j] = k < 9 * p.Ct;
    kt[j] = k - tap * p.Ct;
    kdy[j] = tap / 3;
    kdx[j] = tap - 3 * kdy[j];
  }
  // weight fragments: fragment (cb, lane) by thread cb * 64 + lane mod 256
  for (int f = threadIdx.x; f < NB * 64; f += kTcThreads) {
    const int cb = f >> 6;
    uint32_t h[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      h[j] = kv[j] ? tw_weight(p, 16 * cb + col, kt[j], kdy[j], kdx[j]) : 0u;
    wfrag[cb][lane] = uint4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                            h[6] | (h[7] << 16)};
  }
  __syncthreads();
  uint4 a[NB];
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) a[cb] = wfrag[cb][lane];

  const int HW = p.H << p.wshift;
  const int g0 = (blockIdx.x * (kTcThreads / 64) + wave) * kTwGroups;
  // all of the wave's im2col gathers first (8 kTwGroups loads in flight per lane)
  uint4 bq[kTwGroups];
#pragma unroll
  for (int gg = 0; gg < kTwGroups; ++gg) {
    const int g = g0 + gg < p.groups ? g0 + gg : p.groups - 1;
    const int P = 16 * g + col;
    const int n = P / HW;
    const int rem = P - n * HW;
    const int y = rem >> p.wshift, x = rem & (p.W - 1);
    uint32_t h[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int yy = y + kdy[j] - 1, xx = x + kdx[j] - 1;
      const bool ok = kv[j] & ((unsigned)yy < (unsigned)p.H) & ((unsigned)xx < (unsigned)p.W);
      const int64_t i = (((int64_t)n * p.H + yy) * p.W + xx) * p.Ct + kt[j];
      uint32_t v = 0;
      if (ok) {
        if (kXF32)
          v = f32_to_bf16_bits(reinterpret_cast<const float*>(p.x)[i]);
        else
          v = reinterpret_cast<const uint16_t*>(p.x)[i];
      }
      h[j] = v;
    }
    bq[gg] = uint4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                   h[6] | (h[7] << 16)};
  }
#pragma unroll
  for (int gg = 0; gg < kTwGroups; ++gg) {
    const int g = g0 + gg;
    if (g >= p.groups) break;
    const uint4 b = bq[gg];
#pragma unroll
    for (int cb = 0; cb < NB; ++cb) {
      const v4f d = tc_mfma(a[cb], b, v4f{0.f, 0.f, 0.f, 0.f});
      const int gi = 2 * cb + (ks >> 1);  // 16-B granule of channels 16 cb + 4 ks
      *reinterpret_cast<uint2*>(slot + col * kRowBytes + ((gi ^ col) * 16) + (ks & 1) * 8) =
          uint2{pack_bf16x2(d[0], d[1]), pack_bf16x2(d[2], d[3])};
    }
    uint8_t* out = reinterpret_cast<uint8_t*>(p.out) + (int64_t)16 * g * kRowBytes;
#pragma unroll
    for (int i = 0; i < NB / 2; ++i) {  // 16 px x 2 Cw B = NB / 2 stores of 1 KB per wave
      const int c = i * 64 + lane;       // 16-B chunk of the group's output
      const int px = c / (Cw / 8), gi = c - px * (Cw / 8);
      const uint4 v = *reinterpret_cast<const uint4*>(slot + px * kRowBytes + ((gi ^ px) * 16));
      *reinterpret_cast<uint4*>(out + (int64_t)c * 16) = v;
    }
  }
}

// ---- tile staging ---------------------------------------------------------------------------
// A tile's wide operand goes through registers into LDS, so the next tile's loads are in
// flight while the current one is computed: granule e = u * 256 + tid of the tile's region
// (pixel e / (CW / 8), 16-B granule e % (CW / 8)); HALO: the (TR + 2) x (W + 2)-pixel patch
// around the tile's rows (zero outside the image), else the tile's own 64 pixels.
template <int CW, bool HALO>
constexpr int tc_npre() {
  return ((HALO ? 3 * (kTcMaxW + 2) : kTcTilePx) * (CW / 8) + kTcThreads - 1) / kTcThreads;
}

template <int CW, bool HALO>
__device__ __forceinline__ void tc_stage_load(const TcArgs& p, const uint8_t* src, int tile,
                                              uint4 (&v)[tc_npre<CW, HALO>()]) {
  constexpr int kGran = CW / 8;
  const int PC = p.W + 2;
  const int n_gran = (HALO ? (p.TR + 2) * PC : kTcTilePx) * kGran;
  const int rows_per_img = p.H / p.TR;
  const int n = tile / rows_per_img;
  const int y0 = (tile - n * rows_per_img) * p.TR;
#pragma unroll
  for (int u = 0; u < tc_npre<CW, HALO>(); ++u) {
    const int e = u * kTcThreads + (int)threadIdx.x;
    v[u] = uint4{0u, 0u, 0u, 0u};
    if (e < n_gran) {
      const int px = e / kGran, g = e - px * kGran;
      int yy, xx;
      if (HALO) {
        const int pr = (int)fdiv((uint32_t)px, p.divPC);
        yy = y0 + pr - 1;
        xx = px - pr * PC - 1;
      } else {
        yy = y0 + (px >> p.wshift);
        xx = px & (p.W - 1);
      }
      if ((unsigned)yy < (unsigned)p.H && (unsigned)xx < (unsigned)p.W)
        v[u] = *reinterpret_cast<const uint4*>(
            src + ((((int64_t)n * p.H + yy) * p.W + xx) * CW + g * 8) * 2);
    }
  }
}

template <int CW, bool HALO>
__device__ __forceinline__ void tc_stage_store(const TcArgs& p, uint8_t* dst,
                                               const uint4 (&v)[tc_npre<CW, HALO>()]) {
  constexpr int kGran = CW / 8;
  constexpr int kPitch = 2 * CW + 16;
  const int n_gran = (HALO ? (p.TR + 2) * (p.W + 2) : kTcTilePx) * kGran;
#pragma unroll
  for (int u = 0; u < tc_npre<CW, HALO>(); ++u) {
    const int e = u * kTcThreads + (int)threadIdx.x;
    if (e < n_gran) {
      const int px = e / kGran, g = e - px * kGran;
      *reinterpret_cast<uint4*>(dst + px * kPitch + g * 16) = v[u];
    }
  }
}

// ---- wide -> thin --------------------------------------------------------------------------
// Workgroups walk tiles of TR image rows x W = 64 pixels (grid kTwtGrid at most, the weight
// loaded once per workgroup); a tile's input patch (TR + 2) x (W + 2) pixels x Cw channels sits
// in LDS at a (2 Cw + 16)-B pixel pitch (out-of-image pixels zero), the weight as [Ct][9][Cw]
// bf16. Wave w computes pixels 16 w .. + 15 of the tile: D[co][px] over K = tap x channel,
// 9 x Cw / 32 MFMAs, rows co >= Ct zero.
template <int CW>
__global__ __launch_bounds__(kTcThreads) void tc_wide_thin_kernel(const TcArgs p) {
  constexpr int kPitch = 2 * CW + 16;
  extern __shared__ __attribute__((aligned(16))) uint8_t tc_dyn[];
  uint8_t* patch = tc_dyn;
  const int PC = p.W + 2;
  const int patch_px = (p.TR + 2) * PC;
  uint8_t* wl = patch + patch_px * kPitch;  // [Ct][9][CW] bf16
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, ks = lane >> 4;

  // weights into LDS (rounded to bf16)
  for (int e = tid; e < p.Ct * 9 * CW; e += kTcThreads) {
    const int co = e / (9 * CW);
    const int r = e - co * 9 * CW;
    const int tap = r / CW, ci = r - tap * CW;
    const int64_t i = (int64_t)co * p.ws0 + (int64_t)ci * p.ws1 + (tap / 3) * p.ws2 + (tap % 3) * p.ws3;
    reinterpret_cast<uint16_t*>(wl)[e] = (uint16_t)tc_bf16_of(p.w, i, p.w_f32);
  }

  const uint8_t* x = reinterpret_cast<const uint8_t*>(p.x);
  const int q = 16 * wave + col;  // tile pixel of this lane's B column
  const int r = q >> p.wshift, c = q & (p.W - 1);
  const int co = col < p.Ct ? col : 0;
  const bool co_ok = col < p.Ct;
  uint4 v[tc_npre<CW, true>()];
  int tile = blockIdx.x;
  if (tile < p.tiles) tc_stage_load<CW, true>(p, x, tile, v);
  for (; tile < p.tiles; tile += gridDim.x) {
    __syncthreads();  // weights stored; the previous tile's patch reads are done
    tc_stage_store<CW, true>(p, patch, v);
    __syncthreads();
    if (tile + (int)gridDim.x < p.tiles) tc_stage_load<CW, true>(p, x, tile + gridDim.x, v);

    v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
      const int ky = tap / 3, kx = tap % 3;
      const uint8_t* brow = patch + ((r + ky) * PC + c + kx) * kPitch + ks * 16;
      const uint8_t* arow = wl + ((co * 9 + tap) * CW + ks * 8) * 2;
#pragma unroll
      for (int kc = 0; kc < CW / 32; ++kc) {
        uint4 a = *reinterpret_cast<const uint4*>(arow + kc * 64);
        if (!co_ok) a = uint4{0u, 0u, 0u, 0u};
        const uint4 b = *reinterpret_cast<const uint4*>(brow + kc * 64);
        acc = tc_mfma(a, b, acc);
      }
    }
    // lanes 0..15 hold D[t][pixel col], t = 0..3: the Ct output channels of pixel q
    if (ks == 0) {
      uint16_t* out = reinterpret_cast<uint16_t*>(p.out) + ((int64_t)tile * kTcTilePx + q) * p.Ct;
      for (int t = 0; t < p.Ct; ++t) out[t] = (uint16_t)f32_to_bf16_bits(acc[t]);
    }
  }
}

// ---- weight gradient -----------------------------------------------------------------------
// dw[co][ky][kx][ci] = sum_px x[px + (ky - 1, kx - 1)][ci] dy[px][co]. Workgroup wg sums the
// 64-pixel tiles [wg * tiles_per_wg, +tiles_per_wg) into partials[wg][Cout][9][Cin] (fp32),
// the next tile's operands loading while the current one is computed. Per tile and 32-pixel K
// chunk: lane slice ks covers pixels 8 ks .. + 7 of the chunk.
//
// WIDE_X (output conv: x has CW channels, dy Ct): D[ci][co] per tap; A = x^T by transpose
// reads of the x patch (shifted by the tap), B = dy^T[co][px] (rows co >= Ct zero).
// Otherwise (input conv: x has Ct channels, dy CW): D[co][ci] per tap; A = dy^T by transpose
// reads of the dy tile, B = the x plane of the tap's column shift.
// Wave w owns 16-channel blocks w * NBW .. + NBW - 1 of the wide side, all 9 taps.
constexpr int kTcThinPre = (3 * kTcMaxCt * 3 * kTcMaxW + kTcThreads - 1) / kTcThreads;

template <bool WIDE_X, bool kXF32, int CW>
__global__ __launch_bounds__(kTcThreads, CW == 128 ? 2 : 1) void tc_wgrad_kernel(const TcArgs p) {
  constexpr int NBW = CW / 64;                // wide 16-channel blocks per wave
  constexpr int kPitch = 2 * CW + 16;         // wide tile pixel pitch (8-B aligned rows)
  extern __shared__ __attribute__((aligned(16))) uint8_t tc_dyn[];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, ks = lane >> 4;
  const int PC = p.W + 2;
  const int TR = p.TR;
  // LDS: the wide tile (WIDE_X: the x patch (TR + 2) x (W + 2) pixels; else the dy tile
  // 64 pixels), then the thin side (WIDE_X: dy^T [kTcMaxCt][64] bf16; else the x planes
  // [3 column shifts][Ct][TR + 2][W] bf16)
  const int wide_px = WIDE_X ? (TR + 2) * PC : kTcTilePx;
  uint8_t* wide = tc_dyn;
  uint8_t* thin = tc_dyn + wide_px * kPitch;
  const int rows_per_img = p.H / TR;
  const int plane = (TR + 2) * p.W;
  const int n_thin = WIDE_X ? kTcMaxCt * kTcTilePx : 3 * p.Ct * plane;

  v4f acc[9][NBW];
#pragma unroll
  for (int t = 0; t < 9; ++t)
#pragma unroll
    for (int b = 0; b < NBW; ++b) acc[t][b] = v4f{0.f, 0.f, 0.f, 0.f};

  // the thin operand of a tile, as bf16 bits per element of its LDS layout
  auto thin_load = [&](int tile, uint32_t (&tv)[kTcThinPre]) __attribute__((always_inline)) {
    const int n = tile / rows_per_img;
    const int y0 = (tile - n * rows_per_img) * TR;
#pragma unroll
    for (int u = 0; u < kTcThinPre; ++u) {
      const int e = u * kTcThreads + tid;
      uint32_t v = 0;
      if (e < n_thin) {
        if (WIDE_X) {
          const int co = e / kTcTilePx, px = e - co * kTcTilePx;
          if (co < p.Ct)
            v = reinterpret_cast<const uint16_t*>(p.dy)[((int64_t)tile * kTcTilePx + px) * p.Ct + co];
        } else {
          const int sc = e / plane;  // shift * Ct + ci
          const int rr = e - sc * plane;
          const int sh = sc / p.Ct, ci = sc - sh * p.Ct;
          const int pr = rr >> p.wshift, pc = rr & (p.W - 1);
          const int yy = y0 + pr - 1, xx = pc + sh - 1;
          if ((unsigned)yy < (unsigned)p.H && (unsigned)xx < (unsigned)p.W)
            v = tc_bf16_of(p.x, (((int64_t)n * p.H + yy) * p.W + xx) * p.Ct + ci, kXF32);
        }
      }
      tv[u] = v;
    }
  };

  const int t_begin = blockIdx.x * p.tiles_per_wg;
  int t_end = t_begin + p.tiles_per_wg;
  if (t_end > p.tiles) t_end = p.tiles;
  const uint8_t* wsrc = reinterpret_cast<const uint8_t*>(WIDE_X ? p.x : p.dy);
  uint4 wv[tc_npre<CW, WIDE_X>()];
  uint32_t tv[kTcThinPre];
  if (t_begin < t_end) {
    tc_stage_load<CW, WIDE_X>(p, wsrc, t_begin, wv);
    thin_load(t_begin, tv);
  }
  for (int tile = t_begin; tile < t_end; ++tile) {
    __syncthreads();  // the previous tile's reads are done
    tc_stage_store<CW, WIDE_X>(p, wide, wv);
#pragma unroll
    for (int u = 0; u < kTcThinPre; ++u) {
      const int e = u * kTcThreads + tid;
      if (e < n_thin) reinterpret_cast<uint16_t*>(thin)[e] = (uint16_t)tv[u];
    }
    __syncthreads();
    if (tile + 1 < t_end) {
      tc_stage_load<CW, WIDE_X>(p, wsrc, tile + 1, wv);
      thin_load(tile + 1, tv);
    }

#pragma unroll
    for (int h = 0; h < kTcTilePx / 32; ++h) {
      // this lane's transpose-read row: pixel 32 h + 8 ks + (col >> 2) (+ 4), columns
      // 4 (col & 3) .. + 3 of a 16-channel block
      const int q0 = 32 * h + 8 * ks + (col >> 2);
      const int cofs = 8 * (col & 3);  // bytes
      if (WIDE_X) {
        // B: dy^T rows co = col, pixels 32 h + 8 ks .. + 7
        uint4 bf = *reinterpret_cast<const uint4*>(thin + ((col < kTcMaxCt ? col : 0) * kTcTilePx + 32 * h + 8 * ks) * 2);
        if (col >= p.Ct) bf = uint4{0u, 0u, 0u, 0u};
        const int r0 = q0 >> p.wshift, c0 = q0 & (p.W - 1);
        const int r1 = (q0 + 4) >> p.wshift, c1 = (q0 + 4) & (p.W - 1);
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) {
          const int ky = tap / 3, kx = tap % 3;
          const uint8_t* a0 = wide + ((r0 + ky) * PC + c0 + kx) * kPitch + cofs;
          const uint8_t* a1 = wide + ((r1 + ky) * PC + c1 + kx) * kPitch + cofs;
#pragma unroll
          for (int b = 0; b < NBW; ++b) {
            const int boff = (wave * NBW + b) * 32;  // 16 channels x 2 B
            const uint2 lo = tc_ld_tr16(a0 + boff);
            const uint2 hi = tc_ld_tr16(a1 + boff);
            acc[tap][b] = tc_mfma(uint4{lo.x, lo.y, hi.x, hi.y}, bf, acc[tap][b]);
          }
        }
      } else {
        uint4 af[NBW];
#pragma unroll
        for (int b = 0; b < NBW; ++b) {
          const int boff = (wave * NBW + b) * 32;
          const uint2 lo = tc_ld_tr16(wide + q0 * kPitch + cofs + boff);
          const uint2 hi = tc_ld_tr16(wide + (q0 + 4) * kPitch + cofs + boff);
          af[b] = uint4{lo.x, lo.y, hi.x, hi.y};
        }
        // B: x plane (column shift kx, channel col) row r + ky, columns c .. c + 7
        const int qb = 32 * h + 8 * ks;
        const int r = qb >> p.wshift, c = qb & (p.W - 1);
        const int ci = col < p.Ct ? col : 0;
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) {
          const int ky = tap / 3, kx = tap % 3;
          uint4 bf = *reinterpret_cast<const uint4*>(
              thin + ((kx * p.Ct + ci) * plane + (r + ky) * p.W + c) * 2);
          if (col >= p.Ct) bf = uint4{0u, 0u, 0u, 0u};
#pragma unroll
          for (int b = 0; b < NBW; ++b) acc[tap][b] = tc_mfma(af[b], bf, acc[tap][b]);
        }
      }
    }
  }

  // D[row][col]: lane holds rows 4 ks + t of block b, column col (thin channel < Ct)
  if (col < p.Ct) {
    float* part = reinterpret_cast<float*>(p.out) + (int64_t)blockIdx.x * (p.Ct * 9 * CW);
#pragma unroll
    for (int tap = 0; tap < 9; ++tap)
#pragma unroll
      for (int b = 0; b < NBW; ++b)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int wch = (wave * NBW + b) * 16 + 4 * ks + t;  // wide channel
          // partial layout = the weight's OHWI order [Cout][9][Cin]
          const int64_t i = WIDE_X ? ((int64_t)col * 9 + tap) * CW + wch     // co = col, ci = wch
                                   : ((int64_t)wch * 9 + tap) * p.Ct + col;  // co = wch, ci = col
          part[i] = acc[tap][b][t];
        }
  }
}

// dw[i] = fp32(bf16(sum over workgroups)) for the R = Cout * 9 * Cin partial sums. Block:
// 64 outputs x 16 workgroup ranges; thread (range q, output) adds its range's partials in
// order, then the 16 range sums are added in order: a fixed association (deterministic).
constexpr int kTcRedRanges = 16;
__global__ __launch_bounds__(64 * kTcRedRanges) void tc_wgrad_reduce_kernel(
    const float* __restrict__ part, float* __restrict__ dw, int R, int nwg) {
  __shared__ float red[kTcRedRanges][64];
  const int lane = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int i = blockIdx.x * 64 + lane;
  const int per = (nwg + kTcRedRanges - 1) / kTcRedRanges;
  const int w0 = q * per;
  const int w1 = w0 + per < nwg ? w0 + per : nwg;
  float s = 0.f;
  if (i < R)
    for (int w = w0; w < w1; ++w) s += part[(int64_t)w * R + i];
  red[q][lane] = s;
  __syncthreads();
  if (q == 0 && i < R) {
    float t = red[0][lane];
#pragma unroll
    for (int j = 1; j < kTcRedRanges; ++j) t += red[j][lane];
    dw[i] = bf16_bits_to_f32(f32_to_bf16_bits(t));
  }
}

int tc_shape(int N, int H, int W, int Ct, int Cw, TcArgs& a) {
  if (N <= 0 || H <= 0 || W <= 0) return DPA_ERR_SIZE;
  if (Ct < 1 || Ct > kTcMaxCt || (Cw != 128 && Cw != 256)) return DPA_ERR_SHAPE;
  if (W != 16 && W != 32 && W != kTcMaxW) return DPA_ERR_SHAPE;
  const int TR = kTcTilePx / W;
  if (H % TR != 0) return DPA_ERR_SHAPE;
  if ((int64_t)N * H * W * Cw > 0x7fffffff) return DPA_ERR_SIZE;
  a.N = N; a.H = H; a.W = W; a.Ct = Ct; a.Cw = Cw;
  a.wshift = W == 16 ? 4 : (W == 32 ? 5 : 6);
  a.TR = TR;
  a.tiles = N * H / TR;
  a.groups = N * H * W / 16;
  a.divPC = make_fastdiv((uint32_t)(W + 2));
  return DPA_OK;
}

template <int CW>
size_t tc_wide_thin_lds(const TcArgs& a) {
  return (size_t)(a.TR + 2) * (a.W + 2) * (2 * CW + 16) + (size_t)a.Ct * 9 * CW * 2;
}

template <int CW>
size_t tc_wgrad_lds(const TcArgs& a, bool wide_x) {
  const size_t wide = (size_t)(wide_x ? (a.TR + 2) * (a.W + 2) : kTcTilePx) * (2 * CW + 16);
  const size_t thin = wide_x ? (size_t)kTcMaxCt * kTcTilePx * 2 : (size_t)3 * a.Ct * (a.TR + 2) * a.W * 2;
  return wide + thin;
}

constexpr int kTcWgradWgs = 512;

// Dynamic LDS above 64 KB (the Cw = 256 instances) needs the kernel's limit raised once.
template <typename K>
int tc_lds_limit(K kernel, size_t bytes) {
  if (bytes <= 65536) return DPA_OK;
  const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  return e == hipSuccess ? DPA_OK : (int)e;
}

int tc_wgrad_nwg(const TcArgs& a) { return a.tiles < kTcWgradWgs ? a.tiles : kTcWgradWgs; }

}  // namespace
}  // namespace dpa

using namespace dpa;

static void tc_weight(TcArgs& a, const void* w, int w_dtype, int ws0, int ws1, int ws2, int ws3) {
  a.w = w;
  a.w_f32 = w_dtype == DPA_DTYPE_F32;
  a.ws0 = ws0; a.ws1 = ws1; a.ws2 = ws2; a.ws3 = ws3;
}

extern "C" int dpa_conv3x3_thin_fwd(const void* x, int x_dtype, const void* w, int w_dtype,
                                    int ws0, int ws1, int ws2, int ws3, void* y, int N, int H,
                                    int W, int Cin, int Cout, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  if (!x || !w || !y) return DPA_ERR_NULL;
  if (!aligned(y, 16) || !aligned(x, 16)) return DPA_ERR_ALIGN;
  TcArgs a{};
  const bool thin_in = Cin <= kTcMaxCt;
  int st = thin_in ? tc_shape(N, H, W, Cin, Cout, a) : tc_shape(N, H, W, Cout, Cin, a);
  if (st != DPA_OK) return st;
  a.x = x;
  a.x_f32 = x_dtype == DPA_DTYPE_F32;
  tc_weight(a, w, w_dtype, ws0, ws1, ws2, ws3);
  a.out = y;
  if (thin_in) {
    a.flip = 0;
    const int grid = (int)ceil_div(a.groups, (kTcThreads / 64) * kTwGroups);
    if (a.Cw == 128) {
      if (a.x_f32) tc_thin_wide_kernel<true, 8><<<grid, kTcThreads, 0, s>>>(a);
      else tc_thin_wide_kernel<false, 8><<<grid, kTcThreads, 0, s>>>(a);
    } else {
      if (a.x_f32) tc_thin_wide_kernel<true, 16><<<grid, kTcThreads, 0, s>>>(a);
      else tc_thin_wide_kernel<false, 16><<<grid, kTcThreads, 0, s>>>(a);
    }
    return launch_status();
  }
  if (a.x_f32) return DPA_ERR_SHAPE;  // the wide input is bf16
  const int grid = a.tiles < kTwtGrid ? a.tiles : kTwtGrid;
  if (a.Cw == 128) {
    tc_wide_thin_kernel<128><<<grid, kTcThreads, tc_wide_thin_lds<128>(a), s>>>(a);
  } else {
    st = tc_lds_limit(tc_wide_thin_kernel<256>, tc_wide_thin_lds<256>(a));
    if (st != DPA_OK) return st;
    tc_wide_thin_kernel<256><<<grid, kTcThreads, tc_wide_thin_lds<256>(a), s>>>(a);
  }
  return launch_status();
}

extern "C" int dpa_conv3x3_thin_dgrad(const void* dy, const void* w, int w_dtype, int ws0,
                                      int ws1, int ws2, int ws3, void* dx, int N, int H, int W,
                                      int Cin, int Cout, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  if (!dy || !w || !dx) return DPA_ERR_NULL;
  if (!aligned(dx, 16)) return DPA_ERR_ALIGN;
  if (Cout > kTcMaxCt) return DPA_ERR_SHAPE;  // dy must be the thin side
  TcArgs a{};
  const int st = tc_shape(N, H, W, Cout, Cin, a);
  if (st != DPA_OK) return st;
  a.x = dy;
  a.x_f32 = 0;
  tc_weight(a, w, w_dtype, ws0, ws1, ws2, ws3);
  a.out = dx;
  a.flip = 1;
  const int grid = (int)ceil_div(a.groups, (kTcThreads / 64) * kTwGroups);
  if (a.Cw == 128)
    tc_thin_wide_kernel<false, 8><<<grid, kTcThreads, 0, s>>>(a);
  else
    tc_thin_wide_kernel<false, 16><<<grid, kTcThreads, 0, s>>>(a);
  return launch_status();
}

extern "C" int64_t dpa_conv3x3_thin_wgrad_workspace_bytes(int N, int H, int W, int Cin,
                                                          int Cout) {
  TcArgs a{};
  const bool thin_in = Cin <= kTcMaxCt;
  const int st = thin_in ? tc_shape(N, H, W, Cin, Cout, a) : tc_shape(N, H, W, Cout, Cin, a);
  if (st != DPA_OK) return st;
  return (int64_t)tc_wgrad_nwg(a) * a.Ct * 9 * a.Cw * 4;
}

extern "C" int dpa_conv3x3_thin_wgrad(const void* x, int x_dtype, const void* dy, float* dw,
                                      int N, int H, int W, int Cin, int Cout, void* workspace,
                                      int64_t workspace_bytes, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  if (!x || !dy || !dw) return DPA_ERR_NULL;
  if (!aligned(x, 16) || !aligned(dy, 16)) return DPA_ERR_ALIGN;
  TcArgs a{};
  const bool wide_x = Cin > kTcMaxCt;
  int st = wide_x ? tc_shape(N, H, W, Cout, Cin, a) : tc_shape(N, H, W, Cin, Cout, a);
  if (st != DPA_OK) return st;
  if (wide_x && x_dtype != DPA_DTYPE_BF16) return DPA_ERR_SHAPE;
  const int nwg = tc_wgrad_nwg(a);
  const int64_t need = (int64_t)nwg * a.Ct * 9 * a.Cw * 4;
  if (!workspace || workspace_bytes < need || !aligned(workspace, 16)) return DPA_ERR_WORKSPACE;
  a.x = x;
  a.dy = dy;
  a.x_f32 = x_dtype == DPA_DTYPE_F32;
  a.out = workspace;
  a.tiles_per_wg = (int)ceil_div(a.tiles, nwg);
  const int grid = (int)ceil_div(a.tiles, a.tiles_per_wg);
  if (wide_x) {
    if (a.Cw == 128) {
      tc_wgrad_kernel<true, false, 128><<<grid, kTcThreads, tc_wgrad_lds<128>(a, true), s>>>(a);
    } else {
      st = tc_lds_limit(tc_wgrad_kernel<true, false, 256>, tc_wgrad_lds<256>(a, true));
      if (st != DPA_OK) return st;
      tc_wgrad_kernel<true, false, 256><<<grid, kTcThreads, tc_wgrad_lds<256>(a, true), s>>>(a);
    }
  } else if (a.x_f32) {
    if (a.Cw == 128)
      tc_wgrad_kernel<false, true, 128><<<grid, kTcThreads, tc_wgrad_lds<128>(a, false), s>>>(a);
    else
      tc_wgrad_kernel<false, true, 256><<<grid, kTcThreads, tc_wgrad_lds<256>(a, false), s>>>(a);
  } else {
    if (a.Cw == 128)
      tc_wgrad_kernel<false, false, 128><<<grid, kTcThreads, tc_wgrad_lds<128>(a, false), s>>>(a);
    else
      tc_wgrad_kernel<false, false, 256><<<grid, kTcThreads, tc_wgrad_lds<256>(a, false), s>>>(a);
  }
  st = launch_status();
  if (st != DPA_OK) return st;
  const int R = a.Ct * 9 * a.Cw;
  tc_wgrad_reduce_kernel<<<(unsigned)ceil_div(R, 64), 64 * kTcRedRanges, 0, s>>>(
      reinterpret_cast<const float*>(workspace), dw, R, grid);
  return launch_status();
}
