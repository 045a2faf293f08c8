// FP8 3x3 / stride-1 / pad-1 convolution (forward and data gradient) with a halo-patch pixel
// operand, for images W = 16 or 32 pixels wide.
//
// Reference: diffusion/fp8_kernels.py conv2d_fwd_fp8_kernel :142-247 and conv2d_dx_fp8_kernel
// :250-318 (the same arithmetic as igemm.hip, which serves every other shape).
//
// The nine taps of a 3x3 conv read the same input pixels shifted by (dy, dx). An output tile
// of 256 pixels is TR = 256 / W whole image rows, so its input is one (TR + 2) x (W + 2)
// pixel patch. Per 128-channel chunk the patch goes into LDS once and the nine K-steps (one
// per tap) read their pixel fragments from it at offset dy * (W + 2) + dx.
//
// Schedule: persistent, one workgroup of 8 waves per CU, XCD-aware contiguous tile ranges;
// K-steps are (chunk, tap) with taps inner. Workgroup tile 256 pixels x 128 channels; each
// wave owns 128 pixels x 32 channels and keeps its own weight fragments in registers: a
// three-deep ring of per-tap fragments loaded from L2 two taps ahead. No wave reads data
// another wave loads except the patch, so the waves synchronise once per chunk (the patch's
// double buffer), not once per K-step: two waves share each SIMD and while one stalls the
// other issues MFMAs. The next chunk's patch is staged through registers (global loads at
// the chunk start, LDS stores late in the chunk), so every wait is the compiler's own
// precise count. Each fragment's reads are issued two fragments ahead of their MFMAs, and
// scheduling barriers keep the compiler from sinking them (or the weight loads) next to
// their consumers.
//
// Weights: in the fragment-native layout (WFRAG, written by weight_frag_kernel from the
// OHWI e4m3 weight) each per-lane fragment load is one contiguous 1 KB per wave; from the
// OHWI weight itself each load touches 16 half-used cache lines (measured 6 us slower per
// cfg2 launch), which the op-level entry without a weight preparation still accepts.
// Epilogue: the wave's accumulators go through its 8 KB LDS slot and leave as 16-B
// nontemporal stores of 64-B channel runs (8-B stores straight from the accumulators,
// nontemporal or not, were 9-17 us slower per launch; plain 16-B stores 2 us slower). The data gradient is the same kernel
// on dy with the transposed weight and the taps mirrored (baked into its fragment layout).
#include "dpa_common.hpp"

namespace dpa {

constexpr int kHcThreads = 512;
constexpr int kHcWaves = kHcThreads / 64;
constexpr int kHcBM = 256;  // output pixels per tile (TR whole rows)
constexpr int kHcBN = 128;  // output channels per tile
constexpr int kHcBK = 128;  // K bytes per step (MFMA depth)
constexpr int kHcWM = 128;  // pixels per wave
constexpr int kHcWN = 32;   // channels per wave
constexpr int kHcPF = kHcWM / 16;                          // pixel fragments per wave (8)
constexpr int kHcPitch = 144;                              // patch pixel pitch in LDS
constexpr int kHcPatchSlots = 3072;                        // 16-B slots per patch buffer
constexpr int kHcPatchBytes = kHcPatchSlots * 16;          // 48 KB >= 340 pixels x 144 B
constexpr int kHcPatchLoads = kHcPatchSlots / kHcThreads;  // 6 slots per thread per patch
constexpr int kHcSlotBytes = kHcWM * kHcWN * 2;            // epilogue: 128 px x 32 ch bf16
static_assert(kHcWaves == (kHcBM / kHcWM) * (kHcBN / kHcWN), "wave grid");
static_assert(kHcPatchLoads == 6, "six staging registers");

struct HconvArgs {
  const uint8_t* act;  // [N][H][W][C]
  const uint8_t* wgt;  // OHWI [Cout][3][3][C], or the fragment layout (weight_frag_kernel)
  uint16_t* out;       // bf16 [N][H][W][Cout]
  const float* sa;
  const float* sb;
  const float* bias;  // [Cout] or null
  int N, H, W, C, Cout;
  int TR, PC;         // output rows per tile, patch row pitch (W + 2) in pixels
  int wshift;         // log2(W)
  int KC, nk;         // 128-channel chunks, K-steps per tile (9 * KC)
  int tiles_n, tiles, tiles_per_xcd, wg_per_xcd;
  int flip;           // OHWI weight only: 1 = data gradient (weight tap 8 - t)
  FastDiv divTN, divKC, divH;
};

__device__ __attribute__((aligned(64))) uint8_t hc_zero16[64];

// Two patch buffers (the current chunk's and the next one's) and the per-wave epilogue slots:
// 96 + 64 = 160 KB, all of the CU's LDS.
__shared__ __attribute__((aligned(1024))) uint8_t hc_patch[2][kHcPatchBytes];
__shared__ __attribute__((aligned(1024))) uint8_t hc_slot[kHcWaves][kHcSlotBytes];

// Patch pixels sit at a 144-B pitch (128 B of channels + 16 B gap), so consecutive pixels are
// 9 16-B bank slots apart (64 banks = 16 slots), and every tap's address is the pixel's base
// plus a wave-uniform offset. gfx950 serves a ds_read_b128 in four 16-lane cycles: per
// half-wave, the lanes whose bits 2..4 have even parity (0-3, 12-15, 20-27) and the odd ones
// (4-11, 16-19, 28-31). A fragment's lane l reads column l & 15 at K byte 32 (l >> 4), so a
// cycle mixes columns 0-3, 12-15 at one K offset with columns 4-11 at the next (2 slots on);
// with column c on pixel c of the run two columns share a slot in every cycle. Columns 4-11
// take the run's even pixels and the others its odd pixels (hc_col_px): the slots 9 p of even
// and odd pixels p are even and odd, the 2-slot shift keeps parity, and no cycle conflicts.
__device__ __forceinline__ int hc_col_px(int c) {
  return (c >= 4 && c < 12) ? 2 * (c - 4) : 2 * ((c & 3) | ((c >> 1) & 4)) + 1;
}
__device__ __forceinline__ v8i hc_frag2(const uint8_t* base, uint32_t a0) {
  const uint4 lo = *reinterpret_cast<const uint4*>(base + a0);
  const uint4 hi = *reinterpret_cast<const uint4*>(base + a0 + 16);
  return v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}

__device__ __forceinline__ v8i hc_gload2(const uint8_t* lo_src, const uint8_t* hi_src) {
  const uint4 lo = *reinterpret_cast<const uint4*>(lo_src);
  const uint4 hi = *reinterpret_cast<const uint4*>(hi_src);
  return v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}

template <bool WFRAG>
__global__ __launch_bounds__(kHcThreads, 1) void hconv_fp8_kernel(const HconvArgs p) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1;   // pixel half (128 output pixels)
  const int wn = wave >> 1;  // channel quarter (32 output channels)
  const int frow = lane & 15, fq = lane >> 4;

  const int xcd = blockIdx.x & 7;
  const int wi = blockIdx.x >> 3;
  const int t_begin = xcd * p.tiles_per_xcd + wi;
  int t_end = (xcd + 1) * p.tiles_per_xcd;
  if (t_end > p.tiles) t_end = p.tiles;
  if (t_begin >= t_end) return;
  const int nt = (t_end - t_begin + p.wg_per_xcd - 1) / p.wg_per_xcd;
  const int nchunks = nt * p.KC;
  const float scale = p.sa[0] * p.sb[0];

  // ---- patch slots of this thread: slot e = d * 512 + tid covers LDS bytes [16e, +16):
  // pixel e / 9 of the patch, granule e % 9 (granule 8 is the pitch gap). Per slot: patch
  // row | (1 << 8 if the slot holds in-image data), and the source offset from the patch
  // origin (pixel (n, y0 - 1, -1) is row 0, column 0).
  const int patch_px = (p.TR + 2) * p.PC;
  int prw[kHcPatchLoads], pxo[kHcPatchLoads];
#pragma unroll
  for (int d = 0; d < kHcPatchLoads; ++d) {
    const int e = d * kHcThreads + tid;
    const int px = e / 9, g = e - px * 9;
    const int pr = px / p.PC;  // once per kernel: plain divisions are fine
    const int pc = px - pr * p.PC;
    const int ok = (g < 8) & (px < patch_px) & (pc >= 1) & (pc <= p.W);
    prw[d] = pr | (ok << 8);
    pxo[d] = ((pr - 1) * p.W + (pc - 1)) * p.C + g * 16;
  }

  // per-chunk scalars: chunk g -> tile (m0, n0), channel chunk kc; patch origin and first
  // image row; weight base
  struct Chunk {
    int live, m0, n0, y0, pbase, wbase;
  };
  const int cb16 = p.Cout >> 4;  // 16-row weight blocks per tap (fragment layout)
  auto chunk_info = [&](int g) __attribute__((always_inline)) {
    Chunk c;
    c.live = g < nchunks;
    const int gg = c.live ? g : 0;
    const int j = (int)fdiv((uint32_t)gg, p.divKC);
    const int kc = gg - j * p.KC;
    const int tile = t_begin + j * p.wg_per_xcd;
    const int tm = (int)fdiv((uint32_t)tile, p.divTN);
    c.m0 = tm * kHcBM;
    c.n0 = (tile - tm * p.tiles_n) * kHcBN;
    const int row0 = c.m0 >> p.wshift;  // global output row n * H + y0
    c.y0 = row0 - (int)fdiv((uint32_t)row0, p.divH) * p.H;
    c.pbase = row0 * p.W * p.C + kc * kHcBK;
    if (WFRAG)  // 2 KB block of (kc, tap 0, this wave's first 16 rows)
      c.wbase = ((kc * 9) * cb16 + (c.n0 >> 4) + wn * (kHcWN / 16)) * 2048 + lane * 16;
    else
      c.wbase = c.n0 * 9 * p.C + kc * kHcBK;
    return c;
  };

  // The patch of chunk c into registers (out-of-image slots and dead chunks read zeros), and
  // from there into LDS buffer buf. Six named registers with the slot index spelled out: an
  // array here is indexed before the loops unroll and would be promoted to LDS.
  uint4 st0, st1, st2, st3, st4, st5;
#define HC_LD(d, dst, c)                                                                   \
  {                                                                                        \
    const int y_ = (c).y0 + (prw[d] & 0xff) - 1;                                           \
    const bool ok_ = (c).live & ((prw[d] >> 8) != 0) & ((unsigned)y_ < (unsigned)p.H);     \
    const uint8_t* src_ = ok_ ? p.act + (uint32_t)((c).pbase + pxo[d]) : hc_zero16;        \
    dst = *reinterpret_cast<const uint4*>(src_);                                           \
  }
#define HC_LOAD_PATCH(c) \
  HC_LD(0, st0, c) HC_LD(1, st1, c) HC_LD(2, st2, c) HC_LD(3, st3, c) HC_LD(4, st4, c) HC_LD(5, st5, c)
#define HC_ST(d, src, buf) \
  *reinterpret_cast<uint4*>(&hc_patch[(buf)][((d) * kHcThreads + tid) * 16]) = src;
#define HC_STORE_PATCH(buf)                                                                \
  HC_ST(0, st0, buf) HC_ST(1, st1, buf) HC_ST(2, st2, buf) HC_ST(3, st3, buf)              \
  HC_ST(4, st4, buf) HC_ST(5, st5, buf)

  // weight fragments of (chunk c, tap t) for the wave's two 16-channel blocks: lane
  // (frow, fq) holds row 16 cb + frow, K bytes [32 fq, +32) of the chunk (L2-resident; the
  // two pixel halves of a channel quarter read the same lines)
  int wrow[2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) wrow[cb] = (wn * kHcWN + cb * 16 + frow) * 9 * p.C + fq * 32;
  auto load_w = [&](const Chunk& c, int t, v8i (&w)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      if (WFRAG) {
        const uint8_t* src = p.wgt + (uint32_t)(c.wbase + (t * cb16 + cb) * 2048);
        w[cb] = hc_gload2(src, src + 1024);
      } else {
        const int tap = p.flip ? 8 - t : t;
        const uint8_t* src = p.wgt + (uint32_t)(c.wbase + wrow[cb] + tap * p.C);
        w[cb] = hc_gload2(src, src + 16);
      }
    }
  };

  // pixel fragment pf: lane (frow, fq) reads pixel hc_col_px(frow) of the fragment's 16-pixel
  // run (patch centre + tap offset), granules 2 fq and 2 fq + 1; base address per pf, plus
  // (dy * PC + dx) * 144 per tap
  uint32_t abase[kHcPF];
#pragma unroll
  for (int pf = 0; pf < kHcPF; ++pf) {
    const int m = wm * kHcWM + pf * 16 + hc_col_px(frow);
    const int orow = m >> p.wshift, ocol = m & (p.W - 1);
    abase[pf] = (uint32_t)(((orow + 1) * p.PC + ocol + 1) * kHcPitch + 32 * fq);
  }
  auto tap_off = [&](int t) __attribute__((always_inline)) {
    const int ty = t / 3, tx = t - 3 * ty;
    return (uint32_t)(((ty - 1) * p.PC + tx - 1) * kHcPitch);
  };

  v4f acc[2][kHcPF];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < kHcPF; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // Epilogue per finished tile: bf16(RN32(acc * RN32(sa * sb)) [+ bias]). Lane (frow, fq)
  // of block (cb, pf) holds channels 16 cb + 4 fq .. + 3 of pixel 16 pf + hc_col_px(frow):
  // all of them go into the wave's slot [128 px][64 B] first (granule g of row r at
  // g ^ ((r >> 2) & 3): conflict-free both ways), then lane l reads pixel 16 pf + l / 4,
  // granule l % 4 and stores 16 B nontemporally; a store instruction covers 16 pixels x 64 B.
  // All writes before any read, so the LDS latency is paid once per tile, not once per
  // fragment.
  uint8_t* slot = hc_slot[wave];
  auto epilogue = [&](int m0, int n0) __attribute__((always_inline)) {
#pragma unroll
    for (int pf = 0; pf < kHcPF; ++pf) {
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[cb][pf][e] * scale;
        if (p.bias) {
          const int c = n0 + wn * kHcWN + cb * 16 + 4 * fq;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = v[e] + p.bias[c + e];
        }
        const int r = pf * 16 + hc_col_px(frow), g = cb * 2 + (fq >> 1);
        *reinterpret_cast<uint2*>(slot + r * 64 + ((g ^ ((r >> 2) & 3)) * 16) + (fq & 1) * 8) =
            uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        acc[cb][pf] = v4f{0.f, 0.f, 0.f, 0.f};
      }
    }
    const int g_rd = lane & 3;
#pragma unroll
    for (int pf = 0; pf < kHcPF; ++pf) {
      const int r = pf * 16 + (lane >> 2);
      const uint4 o = *reinterpret_cast<const uint4*>(slot + r * 64 + ((g_rd ^ ((r >> 2) & 3)) * 16));
      st_nt16(p.out + (uint32_t)((m0 + wm * kHcWM + r) * p.Cout + n0 + wn * kHcWN + g_rd * 8), o);
    }
  };

  // ---- prologue: patch of chunk 0 and the weights of its first two taps ----
  Chunk cc = chunk_info(0);   // current chunk
  Chunk cn = chunk_info(1);   // next chunk
  v8i w0[2], w1[2], w2[2];    // weight ring: taps with t % 3 == 0, 1, 2
  HC_LOAD_PATCH(cc)
  load_w(cc, 0, w0);
  load_w(cc, 1, w1);
  HC_STORE_PATCH(0)

  for (int gc = 0; gc < nchunks; ++gc) {
    // this chunk's patch is complete (own stores done, then every wave's); every wave is
    // past the previous chunk, so the other buffer is free for the next patch
    wait_lgkmcnt0();
    lds_barrier();
    HC_LOAD_PATCH(cn)
    const uint8_t* pa = hc_patch[gc & 1];
    v8i fa[3];
    fa[0] = hc_frag2(pa, abase[0] + tap_off(0));
    fa[1] = hc_frag2(pa, abase[1] + tap_off(0));
#pragma unroll
    for (int t = 0; t < 9; ++t) {
      v8i(&wc)[2] = t % 3 == 0 ? w0 : (t % 3 == 1 ? w1 : w2);
      v8i(&wp)[2] = t % 3 == 0 ? w2 : (t % 3 == 1 ? w0 : w1);
      // the weights of the step two ahead (this chunk's tap t + 2, or the next chunk's);
      // each stage below is closed by a scheduling barrier, so the loads stay two taps and
      // the fragment reads two stages ahead of their use
      if (t < 7)
        load_w(cc, t + 2, wp);
      else
        load_w(cn, t - 7, wp);
#pragma unroll
      for (int pf = 0; pf < kHcPF; ++pf) {
        const int f = t * kHcPF + pf;
        const int f2 = f + 2;
        if (f2 < 9 * kHcPF)
          fa[f2 % 3] = hc_frag2(pa, abase[f2 % kHcPF] + tap_off(f2 / kHcPF));
        acc[0][pf] = mfma16x16x128_e4m3(wc[0], fa[f % 3], acc[0][pf]);
        acc[1][pf] = mfma16x16x128_e4m3(wc[1], fa[f % 3], acc[1][pf]);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (t == 6) {
        HC_STORE_PATCH((gc + 1) & 1)
      }
    }
    const int j = (int)fdiv((uint32_t)gc, p.divKC);
    if (gc - j * p.KC == p.KC - 1) epilogue(cc.m0, cc.n0);
    cc = cn;
    cn = chunk_info(gc + 2);
  }
#undef HC_LD
#undef HC_LOAD_PATCH
#undef HC_ST
#undef HC_STORE_PATCH
}

// Fragment-native weight layout for hconv_fp8_kernel<true>: 2 KB blocks, block
// (kc * T + t) * (rows / 16) + rb holds, at byte half * 1024 + lane * 16 + b, row
// 16 rb + (lane & 15), K byte 128 kc + 32 (lane >> 4) + 16 half + b of tap t. The forward
// weight is read as [rows = Cout][T][K = Cin] (OHWI); the data gradient's as the transpose
// with the taps mirrored: row ci, K co, tap t <- w[co][T - 1 - t][ci]. One thread per 16 B.
__global__ __launch_bounds__(256) void weight_frag_kernel(const uint8_t* __restrict__ w,
                                                          uint8_t* __restrict__ out, int rows,
                                                          int K, int T, int transpose) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 16-B unit
  const int64_t units = (int64_t)rows * K * T / 16;
  if (i >= units) return;
  const int lane = (int)(i & 63), half = (int)((i >> 6) & 1);
  const int64_t blk = i >> 7;
  const int nrb = rows >> 4;
  const int rb = (int)(blk % nrb);
  const int64_t kt = blk / nrb;
  const int t = (int)(kt % T), kc = (int)(kt / T);
  const int row = rb * 16 + (lane & 15);
  const int k0 = kc * 128 + (lane >> 4) * 32 + half * 16;
  uint4 v;
  if (!transpose) {
    v = *reinterpret_cast<const uint4*>(w + ((int64_t)row * T + t) * K + k0);
  } else {
    const int ts = T - 1 - t;
    uint32_t b[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) b[j] = w[((int64_t)(k0 + j) * T + ts) * rows + row];
    v.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
    v.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
    v.z = b[8] | (b[9] << 8) | (b[10] << 16) | (b[11] << 24);
    v.w = b[12] | (b[13] << 8) | (b[14] << 16) | (b[15] << 24);
  }
  *reinterpret_cast<uint4*>(out + i * 16) = v;
}

static bool hconv_shape_ok(int N, int H, int W, int C, int Cout) {
  if (N <= 0 || C <= 0 || Cout <= 0 || C % kHcBK != 0 || Cout % kHcBN != 0) return false;
  if (W != 16 && W != 32) return false;
  const int TR = kHcBM / W;
  if (H % TR != 0) return false;
  // 32-bit offsets
  if ((int64_t)N * H * W * C > 0x7fffffff || (int64_t)N * H * W * Cout > 0x7fffffff) return false;
  return (TR + 2) * (W + 2) * kHcPitch <= kHcPatchBytes;
}

static int hconv_launch(const void* act, const void* wgt, const float* sa, const float* sb,
                        const float* bias, void* out, int N, int H, int W, int C, int Cout,
                        int flip, int wfrag, int num_cus, hipStream_t s) {
  HconvArgs a{};
  a.act = (const uint8_t*)act;
  a.wgt = (const uint8_t*)wgt;
  a.out = (uint16_t*)out;
  a.sa = sa;
  a.sb = sb;
  a.bias = bias;
  a.N = N; a.H = H; a.W = W; a.C = C; a.Cout = Cout;
  a.TR = kHcBM / W;
  a.PC = W + 2;
  a.wshift = W == 32 ? 5 : 4;
  a.KC = C / kHcBK;
  a.nk = 9 * a.KC;
  a.tiles_n = Cout / kHcBN;
  const int tiles_m = (N * H * W) / kHcBM;
  a.tiles = tiles_m * a.tiles_n;
  a.tiles_per_xcd = (int)ceil_div(a.tiles, 8);
  int grid = (num_cus / 8) * 8;
  if (grid < 8) grid = 8;
  if (grid > a.tiles_per_xcd * 8) grid = a.tiles_per_xcd * 8;
  a.wg_per_xcd = grid / 8;
  a.flip = flip;
  a.divTN = make_fastdiv((uint32_t)a.tiles_n);
  a.divKC = make_fastdiv((uint32_t)a.KC);
  a.divH = make_fastdiv((uint32_t)H);
  if (wfrag)
    hconv_fp8_kernel<true><<<(unsigned)grid, kHcThreads, 0, s>>>(a);
  else
    hconv_fp8_kernel<false><<<(unsigned)grid, kHcThreads, 0, s>>>(a);
  return launch_status();
}

}  // namespace dpa

// Entry points used by igemm.hip's dispatch (same library, C++ linkage).
namespace dpa {
bool hconv_supported(int N, int H, int W, int C, int Cout) {
  return hconv_shape_ok(N, H, W, C, Cout);
}
// wgt: the OHWI weight (flip = 1: the data gradient's transposed weight, taps mirrored), or
// with wfrag = 1 the fragment layout of weight_frag_run (taps already in consumption order).
int hconv_run(const void* act, const void* wgt, const float* sa, const float* sb,
              const float* bias, void* out, int N, int H, int W, int C, int Cout, int flip,
              int wfrag, int num_cus, hipStream_t s) {
  return hconv_launch(act, wgt, sa, sb, bias, out, N, H, W, C, Cout, flip, wfrag, num_cus, s);
}
// Fragment layout of an e4m3 weight w: [rows][T][K] (transpose = 0) or, for the data
// gradient, [K][T][rows] read transposed with the taps mirrored (transpose = 1).
// rows % 16 == 0, K % 128 == 0.
int weight_frag_run(const void* w, void* out, int rows, int K, int T, int transpose,
                    hipStream_t s) {
  if (rows % 16 != 0 || K % 128 != 0 || T <= 0) return DPA_ERR_SHAPE;
  const int64_t units = (int64_t)rows * K * T / 16;
  weight_frag_kernel<<<(unsigned)ceil_div(units, 256), 256, 0, s>>>(
      (const uint8_t*)w, (uint8_t*)out, rows, K, T, transpose);
  return launch_status();
}
}  // namespace dpa
