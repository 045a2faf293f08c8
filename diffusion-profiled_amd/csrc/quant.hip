// Per-tensor absmax scaling and OCP-e4m3 cast (current and delayed scaling).
//
// Reference: diffusion/fp8_kernels.py
//   partial_amax_kernel          :54-64    -> amax_partials_kernel (first pass, current)
//   finalize_amax_kernel         :90-102   -> folded into cast_current_kernel / finalize_kernel
//   quantize_fp8_kernel          :105-120  -> cast_current_kernel
//   partial_amax_kernel_delayed  :69-87    -> cast_delayed_kernel
//   quantize_fp8 / _delayed      :518-601  -> dpa_quantize_fp8_bf16 / _delayed_bf16
//
// Design: the amax is reduced as bf16 magnitude bit patterns with packed u16 max (exact and
// order-free). Partials are one u32 per block; every block of the cast kernel re-reduces
// the (<= kAmaxBlocks) partials from L2 and derives the scale itself, so current scaling
// needs two launches, no atomics and no zero-initialised state (safe under graph capture).
// Tensors of at most kSmallMaxN elements take one single-workgroup launch instead. Both
// passes keep kUnroll 16-B loads in flight per thread over a grid of a few blocks per CU; the
// e4m3 output goes out with nontemporal stores (measured ~2 us faster per 16.8M elements).
#include "dpa_common.hpp"
#include "wprep_body.hpp"

#include <atomic>
#include <mutex>

namespace dpa {

constexpr int kQThreads = 256;
constexpr int kMaxPartials = 1024;
constexpr int kUnroll = 8;          // uint4 loads in flight per thread
constexpr int kAmaxBlocks = 256;    // amax pass grid cap (and partial count cap)
constexpr int kCastBlocks = 1024;   // cast pass grid cap

__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, uint32_t* red) {
  v = wave_max_u32(v);
  const int wid = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wid] = v;
  __syncthreads();
  uint32_t r = red[0];
#pragma unroll
  for (int i = 1; i < kQThreads / 64; ++i) r = r > red[i] ? r : red[i];
  return r;
}

// Max over the partials written by the first pass, recomputed by every block.
__device__ __forceinline__ uint32_t reduce_partials(const uint32_t* partials, int np,
                                                    uint32_t* red) {
  uint32_t m = 0;
  for (int i = threadIdx.x; i < np; i += kQThreads) {
    uint32_t p = partials[i];
    m = m > p ? m : p;
  }
  return block_max_u32(m, red);
}

// Vector loop shared by the passes: every 8-element group v < n / 8 is visited once, kUnroll
// groups (strided over the nb blocks of the pass, this one being block bid) per thread and
// iteration with all their loads issued first; body(v, data) gets the group index and its
// 16 bytes of bf16.
template <typename Body>
__device__ __forceinline__ void for_groups(const uint16_t* __restrict__ x, int64_t nv, int bid,
                                           int nb, Body body) {
  const int64_t gs = (int64_t)nb * kQThreads;
  int64_t v = (int64_t)bid * kQThreads + threadIdx.x;
  for (; v + (kUnroll - 1) * gs < nv; v += kUnroll * gs) {
    uint4 d[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) d[u] = *reinterpret_cast<const uint4*>(x + 8 * (v + u * gs));
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) body(v + u * gs, d[u]);
  }
  for (; v < nv; v += gs) body(v, *reinterpret_cast<const uint4*>(x + 8 * v));
}

// Pass 1 (current scaling): per-block amax of |x| as bf16 bits; block bid of nb.
template <bool kVec>
__device__ __forceinline__ void amax_partials_block(const uint16_t* __restrict__ x, int64_t n,
                                                    uint32_t* __restrict__ partials, int bid,
                                                    int nb) {
  __shared__ uint32_t red[kQThreads / 64];
  us2 acc = {0, 0};
  uint32_t accs = 0;
  int64_t tail = 0;
  if (kVec) {
    const int64_t nv = n >> 3;
    for_groups(x, nv, bid, nb, [&](int64_t, uint4 d) { acc = absmax8(acc, d); });
    tail = nv << 3;
  }
  if (bid == 0) {  // ragged tail (or everything when x is not 16-B aligned)
    for (int64_t j = tail + threadIdx.x; j < n; j += kQThreads) {
      const uint32_t a = x[j] & 0x7fffu;
      accs = accs > a ? accs : a;
    }
  }
  uint32_t m = acc.x > acc.y ? acc.x : acc.y;
  m = m > accs ? m : accs;
  m = block_max_u32(m, red);
  if (threadIdx.x == 0) partials[bid] = m;
}

template <bool kVec>
__global__ __launch_bounds__(kQThreads) void amax_partials_kernel(const uint16_t* __restrict__ x,
                                                                  int64_t n,
                                                                  uint32_t* __restrict__ partials) {
  amax_partials_block<kVec>(x, n, partials, blockIdx.x, gridDim.x);
}

__device__ __forceinline__ void cast_tail(const uint16_t* __restrict__ x, int64_t from, int64_t n,
                                          float scale, uint8_t* __restrict__ q) {
  for (int64_t j = from + threadIdx.x; j < n; j += kQThreads) {
    const float f = quant_div(bf16_bits_to_f32(x[j]), scale);
    q[j] = (uint8_t)(pack4_e4m3(f, 0.f, 0.f, 0.f) & 0xffu);
  }
}

// Pass 2 (current scaling): scale from the partials, then q = e4m3(clamp(x / scale));
// block bid of nb.
template <bool kVec>
__device__ __forceinline__ void cast_current_block(const uint16_t* __restrict__ x, int64_t n,
                                                   const uint32_t* __restrict__ partials, int np,
                                                   uint8_t* __restrict__ q,
                                                   float* __restrict__ scale_out, int bid, int nb) {
  __shared__ uint32_t red[kQThreads / 64];
  const uint32_t amax_bits = reduce_partials(partials, np, red);
  const float scale = scale_from_amax_bits(amax_bits);
  if (bid == 0 && threadIdx.x == 0) *scale_out = scale;
  int64_t tail = 0;
  if (kVec) {
    const int64_t nv = n >> 3;
    const float r = quant_recip(scale);
    if (r != 0.0f)
      for_groups(x, nv, bid, nb, [&](int64_t v, uint4 d) {
        st_nt8(q + 8 * v, quant8_rcp(d, scale, r));
      });
    else
      for_groups(x, nv, bid, nb, [&](int64_t v, uint4 d) {
        st_nt8(q + 8 * v, quant8(d, scale));
      });
    tail = nv << 3;
  }
  if (bid == 0) cast_tail(x, tail, n, scale, q);
}

template <bool kVec>
__global__ __launch_bounds__(kQThreads) void cast_current_kernel(
    const uint16_t* __restrict__ x, int64_t n, const uint32_t* __restrict__ partials, int np,
    uint8_t* __restrict__ q, float* __restrict__ scale_out) {
  cast_current_block<kVec>(x, n, partials, np, q, scale_out, blockIdx.x, gridDim.x);
}

// Current scaling of x and a grouped weight preparation (wprep_body.hpp) in the same two
// launches: blocks [0, wb) are the preparation's, the rest x's pass of nb blocks. The passes
// touch disjoint memory, so each block's work is that of its own launch.
static_assert(kWpThreads == kQThreads, "the combined launches share one block size");

__global__ __launch_bounds__(kQThreads) void amax_with_wprep_kernel(
    const uint16_t* __restrict__ x, int64_t n, uint32_t* __restrict__ partials, int nb,
    const DpaWeightEntry* __restrict__ e, int count, uint32_t* __restrict__ wpart, int wb) {
  if ((int)blockIdx.x < wb) wprep_amax_block(e, count, wpart, blockIdx.x);
  else amax_partials_block<true>(x, n, partials, blockIdx.x - wb, nb);
}

__global__ __launch_bounds__(kQThreads) void cast_with_wprep_kernel(
    const uint16_t* __restrict__ x, int64_t n, const uint32_t* __restrict__ partials, int np,
    uint8_t* __restrict__ q, float* __restrict__ scale_out, int nb,
    const DpaWeightEntry* __restrict__ e, int count, const uint32_t* __restrict__ wpart, int wb) {
  if ((int)blockIdx.x < wb) wprep_cast_block(e, count, wpart, blockIdx.x);
  else cast_current_block<true>(x, n, partials, np, q, scale_out, blockIdx.x - wb, nb);
}

// Delayed scaling, one pass: q = cast(x, *prev_scale) and per-block amax of x. count (if
// given) receives the number of partials, for a finalize in a later launch.
template <bool kVec>
__global__ __launch_bounds__(kQThreads) void cast_delayed_kernel(
    const uint16_t* __restrict__ x, int64_t n, const float* __restrict__ prev_scale,
    uint8_t* __restrict__ q, uint32_t* __restrict__ partials, uint32_t* __restrict__ count) {
  __shared__ uint32_t red[kQThreads / 64];
  const float scale = *prev_scale;
  us2 acc = {0, 0};
  uint32_t accs = 0;
  int64_t tail = 0;
  if (kVec) {
    const int64_t nv = n >> 3;
    const float r = quant_recip(scale);
    if (r != 0.0f)
      for_groups(x, nv, blockIdx.x, gridDim.x, [&](int64_t v, uint4 d) {
        acc = absmax8(acc, d);
        st_nt8(q + 8 * v, quant8_rcp(d, scale, r));
      });
    else
      for_groups(x, nv, blockIdx.x, gridDim.x, [&](int64_t v, uint4 d) {
        acc = absmax8(acc, d);
        st_nt8(q + 8 * v, quant8(d, scale));
      });
    tail = nv << 3;
  }
  if (blockIdx.x == 0) {
    for (int64_t j = tail + threadIdx.x; j < n; j += kQThreads) {
      const uint32_t a = x[j] & 0x7fffu;
      accs = accs > a ? accs : a;
    }
    cast_tail(x, tail, n, scale, q);
  }
  uint32_t m = acc.x > acc.y ? acc.x : acc.y;
  m = m > accs ? m : accs;
  m = block_max_u32(m, red);
  if (threadIdx.x == 0) partials[blockIdx.x] = m;
  if (count && blockIdx.x == 0 && threadIdx.x == 0) *count = gridDim.x;
}

// Deferred window records of delayed-scaling layers (one workgroup per layer), run at the
// start of the next step: the step's x and dy quantizations left their block maxima and
// counts; window_acts[pos] = scale(max x partials), window_dy[pos + 1] = scale(max dy
// partials), pos = pos + 1 (mod len) when x was quantized -- the state the per-call update
// (diffusion/unet.py:82-91, fp8_kernels.py:888-889) leaves after the step. Counts go back to 0.
__global__ __launch_bounds__(kQThreads) void deferred_windows_kernel(
    const DpaDeferredWindow* __restrict__ layers) {
  __shared__ uint32_t red[kQThreads / 64];
  const DpaDeferredWindow& L = layers[blockIdx.x];
  const uint32_t nx = *L.x_count, ndy = *L.dy_count;
  const uint32_t ax = reduce_partials(L.x_partials, (int)nx, red);
  __syncthreads();
  const uint32_t ady = reduce_partials(L.dy_partials, (int)ndy, red);
  if (threadIdx.x == 0) {
    const int64_t p = *L.pos;
    if (p >= 0 && p < L.len) {
      const int64_t p1 = p + 1 == L.len ? 0 : p + 1;
      if (nx > 0) L.window_acts[p] = scale_from_amax_bits(ax);
      if (ndy > 0) L.window_dy[p1] = scale_from_amax_bits(ady);
      if (nx > 0) *L.pos = p1;
    }
    *L.x_count = 0;
    *L.dy_count = 0;
  }
}

// Delayed scaling, finalize: cur_scale = scale(max(partials))  (finalize_amax_kernel), and
// the optional window update.
__global__ __launch_bounds__(kQThreads) void finalize_scale_kernel(
    const uint32_t* __restrict__ partials, int np, float* __restrict__ scale_out,
    float* __restrict__ window, int64_t* __restrict__ pos, int64_t len, int advance) {
  __shared__ uint32_t red[kQThreads / 64];
  const uint32_t amax_bits = reduce_partials(partials, np, red);
  if (threadIdx.x == 0) {
    const float cur = scale_from_amax_bits(amax_bits);
    *scale_out = cur;
    window_record(cur, window, pos, len, advance);
  }
}

// torch.max of each of three fp32 windows (diffusion/unet.py:72-73, fp8_kernels.py:849):
// one workgroup per window; NaN if the window holds a NaN, as torch.max.
__global__ __launch_bounds__(kQThreads) void window_max3_kernel(const float* __restrict__ w0,
                                                                const float* __restrict__ w1,
                                                                const float* __restrict__ w2,
                                                                int64_t n, float* __restrict__ out) {
  __shared__ float redm[kQThreads / 64];
  __shared__ int redn[kQThreads / 64];
  const float* w = blockIdx.x == 0 ? w0 : (blockIdx.x == 1 ? w1 : w2);
  float m = -INFINITY;
  int nan = 0;
  for (int64_t i = threadIdx.x; i < n; i += kQThreads) {
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
    for (int k = 1; k < kQThreads / 64; ++k) {
      m = fmaxf(m, redm[k]);
      nan |= redn[k];
    }
    m = fmaxf(m, redm[0]);
    nan |= redn[0];
    out[blockIdx.x] = nan ? __builtin_nanf("") : m;
  }
}

// Small tensors (weights): one workgroup does amax and cast in a single launch; the second
// pass re-reads x from L2. kDelayed: cast with *prev_scale, scale_out = scale of this amax.
constexpr int kSmallThreads = 1024;
constexpr int64_t kSmallMaxN = 1 << 14;

template <bool kDelayed>
__global__ __launch_bounds__(kSmallThreads) void quant_small_kernel(
    const uint16_t* __restrict__ x, int64_t n, const float* __restrict__ prev_scale,
    uint8_t* __restrict__ q, float* __restrict__ scale_out, float* __restrict__ window,
    int64_t* __restrict__ pos, int64_t len, int advance) {
  __shared__ uint32_t red[kSmallThreads / 64];
  const float prev = kDelayed ? *prev_scale : 0.0f;  // read before scale_out is written
  const int64_t n16 = n & ~(int64_t)15;
  us2 acc = {0, 0};
  uint32_t accs = 0;
  for (int64_t i = (int64_t)threadIdx.x * 16; i < n16; i += kSmallThreads * 16) {
    acc = absmax8(acc, *reinterpret_cast<const uint4*>(x + i));
    acc = absmax8(acc, *reinterpret_cast<const uint4*>(x + i + 8));
  }
  for (int64_t j = n16 + threadIdx.x; j < n; j += kSmallThreads) {
    const uint32_t a = x[j] & 0x7fffu;
    accs = accs > a ? accs : a;
  }
  uint32_t m = acc.x > acc.y ? acc.x : acc.y;
  m = wave_max_u32(m > accs ? m : accs);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  uint32_t amax = red[0];
#pragma unroll
  for (int w = 1; w < kSmallThreads / 64; ++w) amax = amax > red[w] ? amax : red[w];
  const float cur = scale_from_amax_bits(amax);
  const float scale = kDelayed ? prev : cur;
  if (threadIdx.x == 0) {
    *scale_out = cur;
    window_record(cur, window, pos, len, advance);
  }
  const float r = quant_recip(scale);
  for (int64_t i = (int64_t)threadIdx.x * 16; i < n16; i += kSmallThreads * 16) {
    const uint4 v0 = *reinterpret_cast<const uint4*>(x + i);
    const uint4 v1 = *reinterpret_cast<const uint4*>(x + i + 8);
    const uint2 a = r != 0.0f ? quant8_rcp(v0, scale, r) : quant8(v0, scale);
    const uint2 b = r != 0.0f ? quant8_rcp(v1, scale, r) : quant8(v1, scale);
    *reinterpret_cast<uint2*>(q + i) = a;  // q is only required to be 8-B aligned
    *reinterpret_cast<uint2*>(q + i + 8) = b;
  }
  for (int64_t j = n16 + threadIdx.x; j < n; j += kSmallThreads) {
    const float f = quant_div(bf16_bits_to_f32(x[j]), scale);
    q[j] = (uint8_t)(pack4_e4m3(f, 0.f, 0.f, 0.f) & 0xffu);
  }
}

// Blocks for a pass over n elements: one 8-element group per thread up to the cap (large
// tensors then loop, kUnroll groups in flight per thread), so mid-sized tensors such as
// weights still spread over many CUs.
static int grid_for(int64_t n, int cap) {
  int64_t g = ceil_div(n, (int64_t)kQThreads * 8);
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (int)g;
}

}  // namespace dpa

using namespace dpa;

extern "C" int64_t dpa_quant_workspace_bytes(int64_t n) {
  (void)n;
  return (int64_t)kMaxPartials * 4;
}

extern "C" int dpa_quantize_fp8_bf16(const void* x, int64_t n, void* q, float* scale_out,
                                     void* workspace, int64_t workspace_bytes, void* stream) {
  if (!x || !q || !scale_out) return DPA_ERR_NULL;
  if (n <= 0) return DPA_ERR_SIZE;
  if (!workspace || workspace_bytes < dpa_quant_workspace_bytes(n)) return DPA_ERR_WORKSPACE;
  if (!aligned(workspace, 4) || !aligned(scale_out, 4) || !aligned(x, 2)) return DPA_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  const bool vec = aligned(x, 16) && aligned(q, 8);
  const int np = vec ? grid_for(n, kAmaxBlocks) : 1;
  const int gc = vec ? grid_for(n, kCastBlocks) : 1;
  auto* xp = (const uint16_t*)x;
  auto* part = (uint32_t*)workspace;
  if (vec && n <= kSmallMaxN) {
    quant_small_kernel<false><<<1, kSmallThreads, 0, s>>>(xp, n, nullptr, (uint8_t*)q, scale_out,
                                                           nullptr, nullptr, 0, 0);
  } else if (vec) {
    amax_partials_kernel<true><<<np, kQThreads, 0, s>>>(xp, n, part);
    cast_current_kernel<true><<<gc, kQThreads, 0, s>>>(xp, n, part, np, (uint8_t*)q, scale_out);
  } else {
    amax_partials_kernel<false><<<np, kQThreads, 0, s>>>(xp, n, part);
    cast_current_kernel<false><<<gc, kQThreads, 0, s>>>(xp, n, part, np, (uint8_t*)q,
                                                        scale_out);
  }
  return launch_status();
}

// Current scaling of x (dpa_quantize_fp8_bf16) and a planned weight preparation
// (dpa_weight_prep_run) in two launches instead of four: the preparation's blocks run as the
// first blocks of x's amax launch and of x's cast launch. Same bytes and scales as the two
// calls; x below the one-workgroup size or unaligned takes exactly those two calls.
extern "C" int dpa_quantize_fp8_bf16_with_weight_prep(
    const void* x, int64_t n, void* q, float* scale_out, void* workspace, int64_t workspace_bytes,
    const DpaWeightEntry* entries_dev, int count, int total_blocks, void* wp_workspace,
    int64_t wp_workspace_bytes, void* stream) {
  if (!x || !q || !scale_out || !entries_dev) return DPA_ERR_NULL;
  if (n <= 0 || count <= 0 || total_blocks <= 0 || total_blocks > 0x7fffffff - 2 * kCastBlocks)
    return DPA_ERR_SIZE;
  if (!workspace || workspace_bytes < dpa_quant_workspace_bytes(n)) return DPA_ERR_WORKSPACE;
  if (!wp_workspace || wp_workspace_bytes < dpa_weight_prep_workspace_bytes(total_blocks))
    return DPA_ERR_WORKSPACE;
  if (!aligned(workspace, 4) || !aligned(scale_out, 4) || !aligned(x, 2) ||
      !aligned(wp_workspace, 4) || !aligned(entries_dev, 8))
    return DPA_ERR_ALIGN;
  const bool vec = aligned(x, 16) && aligned(q, 8);
  if (!vec || n <= kSmallMaxN) {
    const int st = dpa_quantize_fp8_bf16(x, n, q, scale_out, workspace, workspace_bytes, stream);
    if (st != DPA_OK) return st;
    return dpa_weight_prep_run(entries_dev, count, total_blocks, wp_workspace, wp_workspace_bytes,
                               stream);
  }
  hipStream_t s = (hipStream_t)stream;
  const int np = grid_for(n, kAmaxBlocks), gc = grid_for(n, kCastBlocks);
  auto* xp = (const uint16_t*)x;
  auto* part = (uint32_t*)workspace;
  auto* wpart = (uint32_t*)wp_workspace;
  amax_with_wprep_kernel<<<(unsigned)(total_blocks + np), kQThreads, 0, s>>>(
      xp, n, part, np, entries_dev, count, wpart, total_blocks);
  const int st = launch_status();
  if (st != DPA_OK) return st;
  cast_with_wprep_kernel<<<(unsigned)(total_blocks + gc), kQThreads, 0, s>>>(
      xp, n, part, np, (uint8_t*)q, scale_out, gc, entries_dev, count, wpart, total_blocks);
  return launch_status();
}

// Current scaling whose amax pass ran inside the producer: partials[0..np) are the per-
// workgroup maxima of |x| (bf16 magnitude bits) that the kernel writing x left, so only the
// cast runs here (the same kernel, scale and bytes as dpa_quantize_fp8_bf16).
extern "C" int dpa_quantize_fp8_bf16_from_partials(const void* x, int64_t n, const void* partials,
                                                   int np, void* q, float* scale_out,
                                                   void* stream) {
  if (!x || !q || !scale_out || !partials) return DPA_ERR_NULL;
  if (n <= 0 || np <= 0 || np > (1 << 20)) return DPA_ERR_SIZE;
  if (!aligned(scale_out, 4) || !aligned(x, 2) || !aligned(partials, 4)) return DPA_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  const bool vec = aligned(x, 16) && aligned(q, 8);
  const int gc = vec ? grid_for(n, kCastBlocks) : 1;
  if (vec)
    cast_current_kernel<true><<<gc, kQThreads, 0, s>>>((const uint16_t*)x, n,
                                                       (const uint32_t*)partials, np,
                                                       (uint8_t*)q, scale_out);
  else
    cast_current_kernel<false><<<gc, kQThreads, 0, s>>>((const uint16_t*)x, n,
                                                        (const uint32_t*)partials, np,
                                                        (uint8_t*)q, scale_out);
  return launch_status();
}

// ---------------------------------------------------------------------------------------
// Allocation-free current scaling. The amax partials (one u32 per amax workgroup, at most
// kMaxPartials) live in a file-scope device array, `scratch`, instead of a caller workspace:
// every GPU the library runs on holds its own copy (4 KB) until the process ends. Host code
// never passes the array's name to a kernel (on the host it is only a stand-in symbol); it
// passes the device address hipGetSymbolAddress returns, looked up once per device.
// ---------------------------------------------------------------------------------------
constexpr int kScratchBytes = kMaxPartials * 4;
static __device__ __align__(256) uint32_t scratch[kMaxPartials];

constexpr int kMaxDevices = 64;
static std::atomic<void*> g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// The device address of `scratch` on device dev (looked up with dev current, once).
static int scratch_ptr(int dev, void** out) {
  if (dev < 0 || dev >= kMaxDevices) return DPA_ERR_SIZE;
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      int cur = -1;
      hipError_t e = hipGetDevice(&cur);
      if (e != hipSuccess) return (int)e;
      if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return (int)e;
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (cur != dev) {
        const hipError_t e2 = hipSetDevice(cur);
        if (e == hipSuccess) e = e2;
      }
      if (e != hipSuccess || !p) return e != hipSuccess ? (int)e : DPA_ERR_NULL;
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return DPA_OK;
}

extern "C" int64_t dpa_quantize_fp8_bf16_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" int dpa_quantize_fp8_bf16_noalloc(const void* x, int64_t n, void* q, float* scale_out,
                                             void* stream) {
  if (!x || !q || !scale_out) return DPA_ERR_NULL;
  if (n <= 0) return DPA_ERR_SIZE;
  if (dpa_quant_workspace_bytes(n) > kScratchBytes) return DPA_ERR_WORKSPACE;
  if (!aligned(scale_out, 4) || !aligned(x, 2)) return DPA_ERR_ALIGN;
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice((hipStream_t)stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  void* ws = nullptr;
  const int st = scratch_ptr(dev, &ws);
  if (st != DPA_OK) return st;
  // the same launches as dpa_quantize_fp8_bf16; every partial the cast reads is written first
  return dpa_quantize_fp8_bf16(x, n, q, scale_out, ws, kScratchBytes, stream);
}

static int quantize_delayed(const void* x, int64_t n, const float* prev_scale, void* q,
                            float* cur_scale_out, float* window, int64_t* window_pos,
                            int64_t window_len, int advance, void* workspace,
                            int64_t workspace_bytes, void* stream) {
  if (!x || !q || !prev_scale || !cur_scale_out) return DPA_ERR_NULL;
  if (n <= 0) return DPA_ERR_SIZE;
  if (!workspace || workspace_bytes < dpa_quant_workspace_bytes(n)) return DPA_ERR_WORKSPACE;
  if (!aligned(workspace, 4) || !aligned(cur_scale_out, 4) || !aligned(prev_scale, 4) ||
      !aligned(x, 2))
    return DPA_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  const bool vec = aligned(x, 16) && aligned(q, 8);
  const int np = vec ? grid_for(n, kAmaxBlocks) : 1;
  auto* xp = (const uint16_t*)x;
  auto* part = (uint32_t*)workspace;
  if (vec && n <= kSmallMaxN) {
    quant_small_kernel<true><<<1, kSmallThreads, 0, s>>>(xp, n, prev_scale, (uint8_t*)q,
                                                          cur_scale_out, window, window_pos,
                                                          window_len, advance);
    return launch_status();
  }
  if (vec)
    cast_delayed_kernel<true><<<np, kQThreads, 0, s>>>(xp, n, prev_scale, (uint8_t*)q, part,
                                                       nullptr);
  else
    cast_delayed_kernel<false><<<np, kQThreads, 0, s>>>(xp, n, prev_scale, (uint8_t*)q, part,
                                                        nullptr);
  finalize_scale_kernel<<<1, kQThreads, 0, s>>>(part, np, cur_scale_out, window, window_pos,
                                                 window_len, advance);
  return launch_status();
}

extern "C" int dpa_quantize_fp8_delayed_bf16(const void* x, int64_t n, const float* prev_scale,
                                             void* q, float* cur_scale_out, void* workspace,
                                             int64_t workspace_bytes, void* stream) {
  return quantize_delayed(x, n, prev_scale, q, cur_scale_out, nullptr, nullptr, 0, 0, workspace,
                          workspace_bytes, stream);
}

extern "C" int dpa_quantize_fp8_delayed_window_bf16(const void* x, int64_t n,
                                                    const float* prev_scale, void* q,
                                                    float* cur_scale_out, float* window,
                                                    int64_t* window_pos, int64_t window_len,
                                                    int advance_pos, void* workspace,
                                                    int64_t workspace_bytes, void* stream) {
  if (!window || !window_pos) return DPA_ERR_NULL;
  if (window_len <= 0) return DPA_ERR_SIZE;
  if (!aligned(window, 4) || !aligned(window_pos, 8)) return DPA_ERR_ALIGN;
  return quantize_delayed(x, n, prev_scale, q, cur_scale_out, window, window_pos, window_len,
                          advance_pos ? 1 : 0, workspace, workspace_bytes, stream);
}

extern "C" int dpa_quant_partials_count(int64_t n) {
  return n > 0 ? grid_for(n, kAmaxBlocks) : 0;
}

extern "C" int dpa_quantize_fp8_delayed_deferred_bf16(const void* x, int64_t n,
                                                      const float* prev_scale, void* q,
                                                      uint32_t* partials, int partials_cap,
                                                      uint32_t* count, void* stream) {
  if (!x || !q || !prev_scale || !partials || !count) return DPA_ERR_NULL;
  if (n <= 0) return DPA_ERR_SIZE;
  const int np = grid_for(n, kAmaxBlocks);
  if (partials_cap < np) return DPA_ERR_WORKSPACE;
  if (!aligned(x, 16) || !aligned(q, 8) || !aligned(prev_scale, 4) || !aligned(partials, 4) ||
      !aligned(count, 4))
    return DPA_ERR_ALIGN;
  cast_delayed_kernel<true><<<np, kQThreads, 0, (hipStream_t)stream>>>(
      (const uint16_t*)x, n, prev_scale, (uint8_t*)q, partials, count);
  return launch_status();
}

extern "C" int dpa_delayed_windows_finalize(const DpaDeferredWindow* layers_dev, int count,
                                            void* stream) {
  if (!layers_dev) return DPA_ERR_NULL;
  if (count <= 0) return DPA_ERR_SIZE;
  deferred_windows_kernel<<<(unsigned)count, kQThreads, 0, (hipStream_t)stream>>>(layers_dev);
  return launch_status();
}

extern "C" int dpa_window_max3_f32(const float* w0, const float* w1, const float* w2, int64_t n,
                                   float* out3, void* stream) {
  if (!w0 || !w1 || !w2 || !out3) return DPA_ERR_NULL;
  if (n <= 0) return DPA_ERR_SIZE;
  if (!aligned(w0, 4) || !aligned(w1, 4) || !aligned(w2, 4) || !aligned(out3, 4))
    return DPA_ERR_ALIGN;
  window_max3_kernel<<<3, kQThreads, 0, (hipStream_t)stream>>>(w0, w1, w2, n, out3);
  return launch_status();
}
