// Per-block device code of the grouped FP8 weight preparation (csrc/wprep.hip), shared with
// csrc/quant.hip, whose combined launches run a weight preparation's blocks beside an
// activation's quantization. Each function does one block's work given its block index b in
// the preparation's own numbering (0 .. total_blocks); blockDim.x must be kWpThreads.
#pragma once
#include "dpa_common.hpp"

namespace dpa {

constexpr int kWpThreads = 256;
constexpr int kWpTile = 64;  // a block's tile: 64 output x 64 input channels of one tap

// Entry of block b: the last entry with blk0 <= b (entries are in blk0 order).
__device__ __forceinline__ int wp_entry_of(const DpaWeightEntry* __restrict__ e, int count,
                                           int b) {
  int lo = 0, hi = count - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (e[mid].blk0 <= b) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// Tile t of an entry: (co tile, tap, ci tile) with ci tiles fastest.
struct WpTile {
  int co0, tap, ci0;
};
__device__ __forceinline__ WpTile wp_tile(const DpaWeightEntry& E, int t) {
  const int nci = (E.cin + kWpTile - 1) / kWpTile;
  WpTile r;
  r.ci0 = (t % nci) * kWpTile;
  t /= nci;
  r.tap = t % E.taps;
  r.co0 = (t / E.taps) * kWpTile;
  return r;
}

// Thread's part of a tile: row co0 + (threadIdx / 8) + 32 h (h = 0, 1), 8 consecutive
// channels ci0 + 8 (threadIdx % 8). Returns false where the row or channels fall outside.
__device__ __forceinline__ bool wp_slot(const DpaWeightEntry& E, const WpTile& T, int h,
                                        int64_t& off, int& row, int& c8) {
  row = (threadIdx.x >> 3) + 32 * h;
  c8 = (threadIdx.x & 7) * 8;
  const int co = T.co0 + row, ci = T.ci0 + c8;
  off = ((int64_t)co * E.taps + T.tap) * E.cin + ci;
  return co < E.cout && ci < E.cin;  // cin % 8 == 0: a group of 8 is all in or all out
}

// Elements off .. off+7 of the weight as 8 bf16 packed in one uint4: fp32 weights rounded
// (RNE), bf16 weights (DPA_WP_BF16) as they are.
__device__ __forceinline__ uint4 wp_bf16x8(const DpaWeightEntry& E, int64_t off) {
  if (E.flags & DPA_WP_BF16)
    return *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(E.w) + off);
  const float* p = E.w + off;
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  uint4 o;
  o.x = f32_to_bf16_bits(a.x) | (f32_to_bf16_bits(a.y) << 16);
  o.y = f32_to_bf16_bits(a.z) | (f32_to_bf16_bits(a.w) << 16);
  o.z = f32_to_bf16_bits(b.x) | (f32_to_bf16_bits(b.y) << 16);
  o.w = f32_to_bf16_bits(b.z) | (f32_to_bf16_bits(b.w) << 16);
  return o;
}

// Byte offset of (row, tap t, K index k) in the fragment-native layout of a [rows][taps][K]
// operand (dpa_weight_frag_fp8): 2 KB blocks (kc * taps + t) * (rows / 16) + row / 16, byte
// (k % 32) / 16 * 1024 + ((k % 128) / 32 * 16 + row % 16) * 16 + k % 16.
__device__ __forceinline__ int64_t wp_frag_off(int rows, int taps, int row, int t, int k) {
  const int64_t blk = ((int64_t)(k >> 7) * taps + t) * (rows >> 4) + (row >> 4);
  return blk * 2048 + ((k >> 4) & 1) * 1024 + ((((k >> 5) & 3) << 4) + (row & 15)) * 16 + (k & 15);
}

__device__ __forceinline__ uint32_t wp_block_max(uint32_t v, uint32_t* red) {
  v = wave_max_u32(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t r = red[0];
#pragma unroll
  for (int i = 1; i < kWpThreads / 64; ++i) r = r > red[i] ? r : red[i];
  return r;
}

// Block b of the amax pass: the maximum of |bf16(w)| over its tile, into partials[b].
__device__ __forceinline__ void wprep_amax_block(const DpaWeightEntry* __restrict__ e, int count,
                                                 uint32_t* __restrict__ partials, int b) {
  __shared__ uint32_t red[kWpThreads / 64];
  __shared__ int s_t;
  if (threadIdx.x == 0) s_t = wp_entry_of(e, count, b);
  __syncthreads();
  const DpaWeightEntry& E = e[s_t];
  const WpTile T = wp_tile(E, b - E.blk0);
  us2 acc = {0, 0};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    int64_t off;
    int row, c8;
    if (wp_slot(E, T, h, off, row, c8)) acc = absmax8(acc, wp_bf16x8(E, off));
  }
  const uint32_t m = wp_block_max(acc.x > acc.y ? acc.x : acc.y, red);
  if (threadIdx.x == 0) partials[b] = m;
}

// Cast of one tile: q rows out directly (64 B per row), the transposed copy through an LDS
// tile so that its rows (64 output channels of one input channel) leave as 64-B runs too.
__device__ __forceinline__ void wprep_cast_block(const DpaWeightEntry* __restrict__ e, int count,
                                                 const uint32_t* __restrict__ partials, int b) {
  __shared__ uint32_t red[kWpThreads / 64];
  __shared__ uint32_t tile[kWpTile][kWpTile / 4 + 1];  // [co row][ci / 4], padded
  __shared__ int s_t;
  if (threadIdx.x == 0) s_t = wp_entry_of(e, count, b);
  __syncthreads();
  const DpaWeightEntry& E = e[s_t];
  const WpTile T = wp_tile(E, b - E.blk0);
  uint4 v[2];
  bool ok[2];
  int64_t off[2];
  int row[2], c8[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    ok[h] = wp_slot(E, T, h, off[h], row[h], c8[h]);
    if (ok[h]) v[h] = wp_bf16x8(E, off[h]);
  }
  // this weight's amax from its blocks' partials (every block re-reduces them)
  uint32_t m = 0;
  for (int i = threadIdx.x; i < E.nblk; i += kWpThreads) {
    const uint32_t pv = partials[E.blk0 + i];
    m = m > pv ? m : pv;
  }
  const uint32_t amax = wp_block_max(m, red);
  const float cur = scale_from_amax_bits(amax);
  const float scale = E.prev_scale ? *E.prev_scale : cur;
  if (b == E.blk0 && threadIdx.x == 0) {
    *E.scale_used = scale;
    if (E.cur_scale) *E.cur_scale = cur;
    window_record(cur, E.window, E.pos, E.window_len, 0);
  }
  const float r = quant_recip(scale);
  uint8_t* q = (uint8_t*)E.q;
  const bool frag = (E.flags & DPA_WP_FRAG) != 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint2 o = uint2{0u, 0u};
    if (ok[h]) {
      o = r != 0.0f ? quant8_rcp(v[h], scale, r) : quant8(v[h], scale);
      // 8 consecutive input channels: 8 contiguous bytes in either layout
      const int64_t dst = frag ? wp_frag_off(E.cout, E.taps, T.co0 + row[h], T.tap, T.ci0 + c8[h])
                               : off[h];
      *reinterpret_cast<uint2*>(q + dst) = o;
    }
    tile[row[h]][c8[h] / 4] = o.x;
    tile[row[h]][c8[h] / 4 + 1] = o.y;
  }
  if (!E.qt) return;
  __syncthreads();
  // qt[(ci * taps + tap) * cout + co]: thread -> input channel ci0 + (tid / 16) + 16 k, output
  // channels co0 + 4 (tid % 16) .. +3 (one u32)
  uint8_t* qt = (uint8_t*)E.qt;
  const int cc = (threadIdx.x & 15) * 4;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int cr = (threadIdx.x >> 4) + 16 * k;  // input channel within the tile
    const int ci = T.ci0 + cr, co = T.co0 + cc;
    if (ci >= E.cin || co >= E.cout) continue;
    uint32_t w = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t word = tile[cc + j][cr >> 2];
      w |= ((word >> (8 * (cr & 3))) & 0xffu) << (8 * j);
    }
    uint8_t* dst = frag ? qt + wp_frag_off(E.cin, E.taps, ci, E.taps - 1 - T.tap, co)
                        : qt + ((int64_t)ci * E.taps + T.tap) * E.cout + co;
    if (frag || (co + 4 <= E.cout && (E.cout & 3) == 0)) {
      *reinterpret_cast<uint32_t*>(dst) = w;
    } else {
      for (int j = 0; j < 4 && co + j < E.cout; ++j) dst[j] = (uint8_t)(w >> (8 * j));
    }
  }
}

}  // namespace dpa
