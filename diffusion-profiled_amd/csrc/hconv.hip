// FP8 3x3 / stride-1 / pad-1 convolution (forward and data gradient) with a halo-patch A
// operand, for images W = 16 or 32 pixels wide.
//
// Reference: diffusion/fp8_kernels.py conv2d_fwd_fp8_kernel :142-247 and conv2d_dx_fp8_kernel
// :250-318 (the same arithmetic as igemm.hip, which serves every other shape).
//
// The nine taps of a 3x3 conv read the same input pixels shifted by (dy, dx). An output tile
// of 256 pixels is TR = 256 / W whole image rows, so its input is one (TR + 2) x (W + 2)
// pixel patch. Per 128-channel chunk the patch is DMA'd into LDS once and the nine K-steps
// (one per tap) read their A fragments from it at offset dy * (W + 2) + dx; only the 16 KB
// weight slice is loaded per step. Against one A tile per tap this moves 2.3x fewer bytes
// from L2 into LDS (cfg2: 21 KB instead of 48 KB per K-step).
//
// Schedule (as igemm.hip): persistent, one workgroup of 8 waves (4 x 2 of 64 x 64) per CU,
// XCD-aware contiguous tile ranges; K-steps are (chunk, tap) with taps inner. The weight
// slices go through a 3-deep LDS ring issued three steps ahead; the patch of the next chunk
// (double-buffered) is issued one 16-B slot per thread over the first steps of the current
// chunk, always ahead of the weight DMA it must precede, so the in-order vmcnt waits that
// guard the ring also guard the patch. The data gradient is the same kernel on dy with the
// weight transposed to [Cin][3][3][Cout] and the taps mirrored.
#include "dpa_common.hpp"

namespace dpa {

constexpr int kHcThreads = 512;
constexpr int kHcWaves = kHcThreads / 64;
constexpr int kHcWavesM = 4;
constexpr int kHcBM = 256;  // output pixels per tile (TR whole rows)
constexpr int kHcBN = 128;  // output channels per tile
constexpr int kHcBK = 128;  // K bytes per step (MFMA depth)
constexpr int kHcPitch = 144;                              // patch pixel pitch in LDS
constexpr int kHcPatchSlots = 3072;                        // 16-B slots per patch buffer
constexpr int kHcPatchBytes = kHcPatchSlots * 16;          // 48 KB >= 340 pixels x 144 B
constexpr int kHcPatchLoads = kHcPatchSlots / kHcThreads;  // 6 DMAs per thread per patch
constexpr int kHcBBytes = kHcBN * kHcBK;                   // 16 KB weight slice
constexpr int kHcBLoads = kHcBBytes / 16 / kHcThreads;     // 2
constexpr int kHcSlotBytes = 16 * 64 * 2;                  // epilogue: 16 px x 64 ch bf16

struct HconvArgs {
  const uint8_t* act;  // [N][H][W][C]
  const uint8_t* wgt;  // [Cout][3][3][C]
  uint16_t* out;       // bf16 [N][H][W][Cout]
  const float* sa;
  const float* sb;
  const float* bias;  // [Cout] or null
  int N, H, W, C, Cout;
  int TR, PC;         // output rows per tile, patch row pitch (W + 2) in pixels
  int wshift;         // log2(W)
  int KC, nk;         // 128-channel chunks, K-steps per tile (9 * KC)
  int tiles_n, tiles, tiles_per_xcd, wg_per_xcd;
  int flip;           // 1: data gradient (weight tap 8 - t)
  FastDiv divTN, divKC, divH;
};

__device__ __attribute__((aligned(64))) uint8_t hc_zero16[64];

// 2 patch buffers + 3 weight stages + per-wave epilogue slots = 96 + 48 + 16 = 160 KB.
__shared__ __attribute__((aligned(1024))) uint8_t hc_patch[2][kHcPatchBytes];
__shared__ __attribute__((aligned(1024))) uint8_t hc_b[3][kHcBBytes];
__shared__ __attribute__((aligned(1024))) uint8_t hc_slot[kHcWaves][kHcSlotBytes];

// Weight rows (aligned 16-row fragments): granule g at g ^ ((r ^ (r >> 3)) & 7).
__device__ __forceinline__ int hc_bswz(int r) { return (r ^ (r >> 3)) & 7; }
// Patch pixels sit at a 144-B pitch (128 B of channels + 16 B gap). A fragment starts at any
// pixel, and measured on gfx950 (SQ_LDS_BANK_CONFLICT) no XOR swizzle is conflict-free at
// arbitrary starts either (the best one saves a pass only at starts that are multiples of
// 4); the pitch makes every tap's address the pixel's base plus a wave-uniform offset.

__device__ __forceinline__ v8i hc_frag2(const uint8_t* base, uint32_t a0, uint32_t a1) {
  const uint4 lo = *reinterpret_cast<const uint4*>(base + a0);
  const uint4 hi = *reinterpret_cast<const uint4*>(base + a1);
  return v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}

__global__ __launch_bounds__(kHcThreads, 1) void hconv_fp8_kernel(const HconvArgs p) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % kHcWavesM;  // pixel quarter (64 output pixels)
  const int wn = wave / kHcWavesM;  // channel half (64 output channels)
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

  // ---- patch DMA slots of this thread: slot e = d * 512 + tid covers LDS bytes [16e, +16):
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
  // weight DMA rows of this thread (relative to the tile's first output channel)
  int b_row[kHcBLoads];
#pragma unroll
  for (int r = 0; r < kHcBLoads; ++r) {
    const int row = wave * (kHcBN / kHcWaves) + 8 * r + (lane >> 3);
    b_row[r] = row * 9 * p.C + ((lane & 7) ^ hc_bswz(row)) * 16;
  }

  // per-chunk scalars: chunk g -> tile (m0, n0), channel chunk kc; patch origin and first
  // image row; weight base
  struct Chunk {
    int live, m0, n0, y0, pbase, wbase;
  };
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
    c.wbase = c.n0 * 9 * p.C + kc * kHcBK;
    return c;
  };

  // patch slot d (wave-uniform, 0..5) of chunk c into buffer `buf`; when the chunk is past
  // the end the slot is filled from the zero page
  auto issue_patch_slot = [&](const Chunk& c, int d, uint32_t buf) __attribute__((always_inline)) {
    int pr = prw[0], po = pxo[0];
#pragma unroll
    for (int q = 1; q < kHcPatchLoads; ++q) {
      pr = d == q ? prw[q] : pr;
      po = d == q ? pxo[q] : po;
    }
    const int y = c.y0 + (pr & 0xff) - 1;
    const bool ok = c.live & ((pr >> 8) != 0) & ((unsigned)y < (unsigned)p.H);
    const uint8_t* src = ok ? p.act + (uint32_t)(c.pbase + po) : hc_zero16;
    dma16_lds(src, buf + (uint32_t)((d * kHcThreads + wave * 64) * 16));
  };
  // weight slice of (chunk c, tap t) into ring stage st
  auto issue_b = [&](const Chunk& c, int t, int st) __attribute__((always_inline)) {
    const int wt = p.flip ? 8 - t : t;
    const int off = c.wbase + wt * p.C;
    const uint32_t base = LDS_ADDR(hc_b) + (uint32_t)(st * kHcBBytes) +
                          (uint32_t)(wave * (kHcBN / kHcWaves) * kHcBK);
#pragma unroll
    for (int r = 0; r < kHcBLoads; ++r) {
      const uint8_t* src = c.live ? p.wgt + (uint32_t)(off + b_row[r]) : hc_zero16;
      dma16_lds(src, base + (uint32_t)(8 * r * kHcBK));
    }
  };

  // ---- compute side ----
  // A fragment: lane (frow, fq) of pixel fragment pj reads patch pixel centre + tap offset,
  // granules 2 fq and 2 fq + 1; base address per pj, plus (dy * PC + dx) * 144 per tap
  uint32_t abase[4];
#pragma unroll
  for (int pj = 0; pj < 4; ++pj) {
    const int m = wm * 64 + pj * 16 + frow;
    const int orow = m >> p.wshift, ocol = m & (p.W - 1);
    abase[pj] = (uint32_t)(((orow + 1) * p.PC + ocol + 1) * kHcPitch + 32 * fq);
  }
  uint32_t b_addr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = wn * 64 + i * 16 + frow;
    b_addr[i] = (uint32_t)(row * kHcBK + (((2 * fq) ^ hc_bswz(row)) * 16));
  }

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
  v8i fa[4], fb[4];

  // Epilogue per finished tile: bf16(RN32(acc * RN32(sa * sb)) [+ bias]) staged through the
  // wave's LDS slot into 128-B rows and written with nontemporal stores (measured 2.3 us
  // faster per cfg2 launch than plain stores, whose write-backs delayed the next loads).
  auto epilogue = [&](int m0, int n0) __attribute__((always_inline)) {
    uint8_t* slot = hc_slot[wave];
    const int c0 = n0 + wn * 64;
#pragma unroll
    for (int pj = 0; pj < 4; ++pj) {
#pragma unroll
      for (int ci = 0; ci < 4; ++ci) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[ci][pj][e] * scale;
        if (p.bias) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = v[e] + p.bias[c0 + ci * 16 + 4 * fq + e];
        }
        const int g = 2 * ci + (fq >> 1);
        uint2 o;
        o.x = pack_bf16x2(v[0], v[1]);
        o.y = pack_bf16x2(v[2], v[3]);
        *reinterpret_cast<uint2*>(slot + frow * 128 + ((g ^ (frow & 7)) * 16) + (fq & 1) * 8) = o;
      }
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int c = lane + 64 * rr;
        const int r = c >> 3, g = c & 7;
        const uint4 v = *reinterpret_cast<const uint4*>(slot + r * 128 + ((g ^ (r & 7)) * 16));
        const int m = m0 + wm * 64 + pj * 16 + r;
        st_nt16(p.out + (uint32_t)(m * p.Cout + c0 + g * 8), v);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) acc[i][jj] = v4f{0.f, 0.f, 0.f, 0.f};
  };

  const uint32_t patch0 = LDS_ADDR(hc_patch);
  auto patch_buf = [&](int g) { return patch0 + (uint32_t)((g & 1) * kHcPatchBytes); };

  // ---- prologue: patch of chunk 0; weight stages 0..2 with one duplicate patch slot
  // before the last, so every step finds three DMAs issued after the stage it waits for ----
  Chunk cc = chunk_info(0);   // current chunk
  Chunk cn = chunk_info(1);   // next chunk
#pragma unroll
  for (int d = 0; d < kHcPatchLoads; ++d) issue_patch_slot(cc, d, patch_buf(0));
  issue_b(cc, 0, 0);
  issue_b(cc, 1, 1);
  issue_patch_slot(cc, 0, patch_buf(0));  // duplicate of a landed-or-landing slot: same bytes
  issue_b(cc, 2, 2);
  wait_vmcnt<2 * kHcBLoads + 1>();  // patch 0 and stage 0 landed
  lds_barrier();
#pragma unroll
  for (int i = 0; i < 4; ++i) fb[i] = hc_frag2(hc_b[0], b_addr[i], b_addr[i] ^ 16u);
  {
    const uint32_t off = (uint32_t)(-(p.PC + 1) * kHcPitch);
#pragma unroll
    for (int i = 0; i < 4; ++i) fa[i] = hc_frag2(hc_patch[0], abase[i] + off, abase[i] + off + 16);
  }

  // Step (chunk gc, tap t), weight stage t % 3 (nine taps per chunk): wait until the next
  // step's stage landed (the last three DMAs may still fly), barrier, the 16 MFMAs of this
  // step interleaved with the next step's fragment reads, then queue patch slot t of chunk
  // gc+1 (a duplicate of slot 0 for t >= 6) and the weight slice three steps ahead.
  for (int gc = 0; gc < nchunks; ++gc) {
    for (int t = 0; t < 9; ++t) {
      // the weight-fragment reads of the previous step (from the stage the DMAs below
      // refill) must be done; the two reads of the last A fragment, issued after them and
      // from a patch buffer no DMA of this step touches, may still be in flight
      wait_vmcnt<kHcBLoads + 1>();
      wait_lgkmcnt<2>();
      lds_barrier();
      const int t1 = t == 8 ? 0 : t + 1;
      const int ty1 = t1 >= 6 ? 2 : (t1 >= 3 ? 1 : 0);
      const uint32_t aoff = (uint32_t)(((ty1 - 1) * p.PC + (t1 - 3 * ty1) - 1) * kHcPitch);
      const uint8_t* pa = hc_patch[(t == 8 ? gc + 1 : gc) & 1];
      const int st = t - (t >= 6 ? 6 : (t >= 3 ? 3 : 0));  // t % 3
      const int st1 = st == 2 ? 0 : st + 1;
      const uint8_t* pb = hc_b[st1];
      // pixel fragments 0..2: 4 MFMAs each, then the next step's A fragment in its place;
      // the DMAs of this step go out after the first group
#pragma unroll
      for (int pj = 0; pj < 3; ++pj) {
#pragma unroll
        for (int ci = 0; ci < 4; ++ci) acc[ci][pj] = mfma16x16x128_e4m3(fb[ci], fa[pj], acc[ci][pj]);
        const uint32_t a0 = abase[pj] + aoff;
        fa[pj] = hc_frag2(pa, a0, a0 + 16);
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  // 4 MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // then 2 DS reads
        if (pj == 0) {
          issue_patch_slot(cn, t < kHcPatchLoads ? t : 0, patch_buf(gc + 1));
          if (t < 6)
            issue_b(cc, t + 3, st);
          else
            issue_b(cn, t - 6, st);
        }
      }
      // pixel fragment 3: each weight fragment's last use, then its next-step reload
#pragma unroll
      for (int ci = 0; ci < 4; ++ci) {
        acc[ci][3] = mfma16x16x128_e4m3(fb[ci], fa[3], acc[ci][3]);
        fb[ci] = hc_frag2(pb, b_addr[ci], b_addr[ci] ^ 16u);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // then 2 DS reads
      }
      {
        const uint32_t a0 = abase[3] + aoff;
        fa[3] = hc_frag2(pa, a0, a0 + 16);
      }
    }
    const int j = (int)fdiv((uint32_t)gc, p.divKC);
    if (gc - j * p.KC == p.KC - 1) epilogue(cc.m0, cc.n0);
    cc = cn;
    cn = chunk_info(gc + 2);
  }
  wait_vmcnt<0>();  // trailing DMAs land before the workgroup retires
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
                        int flip, int num_cus, hipStream_t s) {
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
  hconv_fp8_kernel<<<(unsigned)grid, kHcThreads, 0, s>>>(a);
  return launch_status();
}

}  // namespace dpa

// Entry points used by igemm.hip's dispatch (same library, C++ linkage).
namespace dpa {
bool hconv_supported(int N, int H, int W, int C, int Cout) {
  return hconv_shape_ok(N, H, W, C, Cout);
}
int hconv_run(const void* act, const void* wgt, const float* sa, const float* sb,
              const float* bias, void* out, int N, int H, int W, int C, int Cout, int flip,
              int num_cus, hipStream_t s) {
  return hconv_launch(act, wgt, sa, sb, bias, out, N, H, W, C, Cout, flip, num_cus, s);
}
}  // namespace dpa
