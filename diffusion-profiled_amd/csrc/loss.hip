// The training loss of the DDPM step, mean((pred - target)^2) (diffusion/ddpm.py:209-215,
// F.mse_loss under autocast: both operands in fp32), as a deterministic two-launch reduction
// that a captured HIP graph replays correctly: every partial has one writer and a fixed
// summation order, and no memset is recorded (torch's multi-block reductions clear their
// semaphores with one, and a replay of such a graph has returned 0 for this loss).
#include "dpa_common.hpp"

namespace dpa {

constexpr int kMseThreads = 256;
constexpr int kMseBlocks = 256;  // partial sums (one per workgroup)

// Stage 1: workgroup b sums the squared differences of elements b*T + t, stepping by
// blocks*T, each thread in index order, then a fixed tree over the workgroup.
template <bool kBf16>
__global__ __launch_bounds__(kMseThreads) void mse_partial_kernel(const void* __restrict__ pred,
                                                                  const float* __restrict__ tgt,
                                                                  int64_t n,
                                                                  float* __restrict__ part) {
  __shared__ float red[kMseThreads];
  const int64_t stride = (int64_t)gridDim.x * kMseThreads;
  float s = 0.f;
  for (int64_t i = (int64_t)blockIdx.x * kMseThreads + threadIdx.x; i < n; i += stride) {
    const float p = kBf16 ? bf16_bits_to_f32(static_cast<const uint16_t*>(pred)[i])
                          : static_cast<const float*>(pred)[i];
    const float d = p - tgt[i];
    s += d * d;
  }
  red[threadIdx.x] = s;
  __syncthreads();
#pragma unroll
  for (int w = kMseThreads / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

// Stage 2: one workgroup adds the partials in a fixed tree and divides by n (fp32).
__global__ __launch_bounds__(kMseThreads) void mse_final_kernel(const float* __restrict__ part,
                                                                int nparts, float nf,
                                                                float* __restrict__ out) {
  __shared__ float red[kMseThreads];
  float s = 0.f;
  for (int i = threadIdx.x; i < nparts; i += kMseThreads) s += part[i];
  red[threadIdx.x] = s;
  __syncthreads();
#pragma unroll
  for (int w = kMseThreads / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[0] = red[0] / nf;  // the mean as torch forms it: sum / n
}

}  // namespace dpa

using namespace dpa;

extern "C" int64_t dpa_mse_loss_workspace_bytes(void) { return (int64_t)kMseBlocks * 4; }

extern "C" int dpa_mse_loss_f32(const void* pred, int pred_dtype, const float* target, int64_t n,
                                float* out, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  if (!pred || !target || !out) return DPA_ERR_NULL;
  if (n <= 0) return DPA_ERR_SIZE;
  if (pred_dtype != DPA_DTYPE_BF16 && pred_dtype != DPA_DTYPE_F32) return DPA_ERR_SHAPE;
  if (!workspace || workspace_bytes < (int64_t)kMseBlocks * 4) return DPA_ERR_WORKSPACE;
  if (!aligned(pred, pred_dtype == DPA_DTYPE_F32 ? 4 : 2) || !aligned(target, 4) ||
      !aligned(out, 4) || !aligned(workspace, 4))
    return DPA_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  float* part = (float*)workspace;
  int blocks = (int)ceil_div(n, kMseThreads);
  if (blocks > kMseBlocks) blocks = kMseBlocks;
  if (pred_dtype == DPA_DTYPE_BF16)
    mse_partial_kernel<true><<<blocks, kMseThreads, 0, s>>>(pred, target, n, part);
  else
    mse_partial_kernel<false><<<blocks, kMseThreads, 0, s>>>(pred, target, n, part);
  int st = launch_status();
  if (st != DPA_OK) return st;
  mse_final_kernel<<<1, kMseThreads, 0, s>>>(part, blocks, (float)n, out);
  return launch_status();
}
