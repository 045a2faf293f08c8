// Grouped FP8 weight preparation: every FP8 weight of a model quantized in three launches per
// training step, straight from the fp32 master weights.
//
// Reference: per conv/linear call, diffusion/fp8_kernels.py casts the (autocast) bf16 weight
// and quantizes it (quantize_fp8 :518-546 or quantize_fp8_delayed :549-601, kernels :54-120),
// with the delayed-scaling window bookkeeping of diffusion/unet.py:69-91; the data gradient
// reads the weight with its channel axes swapped. Done per layer that is a bf16 cast, one or
// two quantization launches, a window-maximum reduction and, in the backward, a transpose:
// a few microseconds of launch overhead each on tensors of at most a few MB.
//
// Here, once per step for the whole weight set (a table of DpaWeightEntry in device memory):
//   window_max_grouped_kernel   hist[i] = max(window i)            (torch.max of each window)
//   wprep_amax_kernel           per-block |bf16(w)| maxima         (partial_amax_kernel)
//   wprep_cast_kernel           q = e4m3(clamp(bf16(w) / scale)), the transposed copy, the
//                               scale used, this amax's scale and its window record (with
//                               DPA_WP_FRAG both copies in the halo-patch conv's fragment
//                               layouts: forward, and data gradient with the taps mirrored)
// with scale = *prev_scale (delayed scaling: the window maximum) or the scale of this
// weight's own amax (current scaling). bf16(w) is the round-to-nearest-even cast autocast
// performs, so every byte and scale equals the per-layer path's. Each block takes one tile
// of 64 output x 64 input channels of one tap; the transposed copy goes through LDS, so both
// copies are written in 64-B runs.
#include "wprep_body.hpp"

namespace dpa {

// The two passes, one block per 64 x 64 tile (wprep_body.hpp).
__global__ __launch_bounds__(kWpThreads) void wprep_amax_kernel(
    const DpaWeightEntry* __restrict__ e, int count, uint32_t* __restrict__ partials) {
  wprep_amax_block(e, count, partials, blockIdx.x);
}

// Cast of one tile: q rows out directly (64 B per row), the transposed copy through an LDS
// tile so that its rows (64 output channels of one input channel) leave as 64-B runs too.
__global__ __launch_bounds__(kWpThreads) void wprep_cast_kernel(
    const DpaWeightEntry* __restrict__ e, int count, const uint32_t* __restrict__ partials) {
  wprep_cast_block(e, count, partials, blockIdx.x);
}

// hist[i] = torch.max(window i) over len floats; NaN if the window holds a NaN.
__global__ __launch_bounds__(kWpThreads) void window_max_grouped_kernel(
    const float* const* __restrict__ windows, int64_t len, float* __restrict__ hist) {
  __shared__ float redm[kWpThreads / 64];
  __shared__ int redn[kWpThreads / 64];
  const float* w = windows[blockIdx.x];
  float m = -INFINITY;
  int nan = 0;
  for (int64_t i = threadIdx.x; i < len; i += kWpThreads) {
    const float v = w[i];
    nan |= v != v;
    m = fmaxf(m, v);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    m = fmaxf(m, __shfl_xor(m, o, 64));
    nan |= __shfl_xor(nan, o, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    redm[threadIdx.x >> 6] = m;
    redn[threadIdx.x >> 6] = nan;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = redm[0];
    int rn = redn[0];
    for (int k = 1; k < kWpThreads / 64; ++k) {
      r = fmaxf(r, redm[k]);
      rn |= redn[k];
    }
    hist[blockIdx.x] = rn ? __builtin_nanf("") : r;
  }
}

}  // namespace dpa

using namespace dpa;

extern "C" int dpa_weight_prep_plan(DpaWeightEntry* entries, int count) {
  if (!entries) return DPA_ERR_NULL;
  if (count <= 0) return DPA_ERR_SIZE;
  int64_t blocks = 0;
  for (int i = 0; i < count; ++i) {
    DpaWeightEntry& E = entries[i];
    if (!E.w || !E.q || !E.scale_used) return DPA_ERR_NULL;
    if (E.window && !E.pos) return DPA_ERR_NULL;
    if (E.cout <= 0 || E.taps <= 0 || E.cin <= 0 || E.n <= 0) return DPA_ERR_SIZE;
    if (E.n != (int64_t)E.cout * E.taps * E.cin || E.cin % 8 != 0) return DPA_ERR_SHAPE;
    if ((E.flags & DPA_WP_FRAG) && (E.cin % 128 != 0 || E.cout % 128 != 0)) return DPA_ERR_SHAPE;
    if (!aligned(E.w, 16) || !aligned(E.q, 8)) return DPA_ERR_ALIGN;
    E.blk0 = (int32_t)blocks;
    E.nblk = (int32_t)(ceil_div(E.cout, kWpTile) * E.taps * ceil_div(E.cin, kWpTile));
    blocks += E.nblk;
    if (blocks > 0x7fffffff) return DPA_ERR_SIZE;
  }
  return (int)blocks;
}

extern "C" int64_t dpa_weight_prep_workspace_bytes(int total_blocks) {
  return total_blocks > 0 ? (int64_t)total_blocks * 4 : 0;
}

extern "C" int dpa_weight_prep_run(const DpaWeightEntry* entries_dev, int count,
                                   int total_blocks, void* workspace, int64_t workspace_bytes,
                                   void* stream) {
  if (!entries_dev) return DPA_ERR_NULL;
  if (count <= 0 || total_blocks <= 0) return DPA_ERR_SIZE;
  if (!workspace || workspace_bytes < dpa_weight_prep_workspace_bytes(total_blocks))
    return DPA_ERR_WORKSPACE;
  if (!aligned(workspace, 4) || !aligned(entries_dev, 8)) return DPA_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  wprep_amax_kernel<<<(unsigned)total_blocks, kWpThreads, 0, s>>>(entries_dev, count,
                                                                  (uint32_t*)workspace);
  int st = launch_status();
  if (st != DPA_OK) return st;
  wprep_cast_kernel<<<(unsigned)total_blocks, kWpThreads, 0, s>>>(entries_dev, count,
                                                                  (const uint32_t*)workspace);
  return launch_status();
}

extern "C" int dpa_window_max_grouped_f32(const float* const* windows_dev, int count,
                                          int64_t len, float* hist, void* stream) {
  if (!windows_dev || !hist) return DPA_ERR_NULL;
  if (count <= 0 || len <= 0) return DPA_ERR_SIZE;
  window_max_grouped_kernel<<<(unsigned)count, kWpThreads, 0, (hipStream_t)stream>>>(
      windows_dev, len, hist);
  return launch_status();
}
