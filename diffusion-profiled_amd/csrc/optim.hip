// Fused optimizer tail of the training step: gradient-norm clipping, AdamW and the EMA update
// of every parameter in one norm pass and one update pass.
//
// Reference (train.py:104-149 step order, :253 optimizer, :256 EMA):
//   torch.nn.utils.clip_grad_norm_(params, max_norm)      total = ||(||g_t||)_t||, g *= coef
//   torch.optim.AdamW(fused=True, capturable=True).step() (betas, eps, weight_decay)
//   EWMAWrapper.update: ema = beta * ema + (1 - beta) * p  (float parameters and buffers)
// which is a norm pass, a scaling pass, the AdamW pass and two EMA passes over the parameters.
// Here:
//   opt_norm_kernel      per-block sums of g^2 (fixed ranges)
//   opt_finalize_kernel  total = sqrt(sum of the block sums, in order); coef = min(1,
//                        max_norm / (total + 1e-6)); step += 1; bias corrections
//   opt_update_kernel    g *= coef; p *= 1 - lr wd; m = b1 m + (1 - b1) g;
//                        v = b2 v + (1 - b2) g^2; p -= (lr / bc1) m / (sqrt(v) / sqrt(bc2) + eps);
//                        ema = RN(beta ema) + RN((1 - beta) p)   (and ema-only entries)
// Tensor pointers travel in the kernel arguments, kOptMaxT tensors per launch (the updates are
// elementwise, so launches over tensor chunks are independent); the norm is deterministic.
#include "dpa_common.hpp"

namespace dpa {

constexpr int kOptThreads = 256;
constexpr int kOptElems = kOptThreads * 4 * 4;  // per block: 4 float4 per thread
constexpr int kOptMaxT = 36;

struct OptChunk {
  int count;
  int blk0[kOptMaxT + 1];  // first block of each tensor (relative to the launch), + total
  float* p[kOptMaxT];
  const float* g[kOptMaxT];
  float* m[kOptMaxT];
  float* v[kOptMaxT];
  float* e[kOptMaxT];
  int64_t n[kOptMaxT];
  int part0;  // this launch's first block in the partial array
};

// Scalars written by the finalize kernel: [0] coef, [1] step, [2] lr/bc1, [3] sqrt(bc2).
constexpr int kOptScalars = 4;

__device__ __forceinline__ int opt_tensor_of(const OptChunk& c, int b) {
  int t = 0;
  while (t + 1 < c.count && c.blk0[t + 1] <= b) ++t;
  return t;
}

__global__ __launch_bounds__(kOptThreads) void opt_norm_kernel(const OptChunk c,
                                                               float* __restrict__ partials) {
  __shared__ float red[kOptThreads / 64];
  __shared__ int s_t;
  if (threadIdx.x == 0) s_t = opt_tensor_of(c, blockIdx.x);
  __syncthreads();
  const int t = s_t;
  const int64_t i0 = (int64_t)(blockIdx.x - c.blk0[t]) * kOptElems;
  const int64_t n = c.n[t];
  const float* g = c.g[t];
  float s = 0.f;
  if (g) {
    for (int64_t i = i0 + threadIdx.x * 4; i < i0 + kOptElems && i < n; i += kOptThreads * 4) {
      if (i + 4 <= n) {
        const float4 x = *reinterpret_cast<const float4*>(g + i);
        s += (x.x * x.x + x.y * x.y) + (x.z * x.z + x.w * x.w);
      } else {
        for (int64_t j = i; j < n; ++j) s += g[j] * g[j];
      }
    }
  }
  s = wave_sum_f32(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = red[0];
#pragma unroll
    for (int k = 1; k < kOptThreads / 64; ++k) r += red[k];
    partials[c.part0 + blockIdx.x] = r;
  }
}

__global__ __launch_bounds__(kOptThreads) void opt_finalize_kernel(
    const float* __restrict__ partials, int np, float* __restrict__ step,
    float* __restrict__ scalars, float max_norm, float lr, float beta1, float beta2) {
  __shared__ float red[kOptThreads];
  // fixed order: thread k sums partials k, k + 256, ...; then a fixed tree
  float s = 0.f;
  for (int i = threadIdx.x; i < np; i += kOptThreads) s += partials[i];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int w = kOptThreads / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const float total = sqrtf(red[0]);
    float coef = 1.0f;
    if (max_norm > 0.f) {
      coef = max_norm / (total + 1e-6f);
      coef = coef < 1.0f ? coef : 1.0f;
    }
    const float t = *step + 1.0f;
    *step = t;
    const float bc1 = 1.0f - powf(beta1, t);
    const float bc2 = 1.0f - powf(beta2, t);
    scalars[0] = coef;
    scalars[1] = t;
    scalars[2] = lr / bc1;
    scalars[3] = sqrtf(bc2);
  }
}

// One element of the update (all fp32): AdamW on (p, g, m, v) when there is a gradient, then
// the EMA of the new parameter when there is an EMA copy.
__device__ __forceinline__ void opt_elem(float& pv, float gv, float& mv, float& vv, float* ev,
                                         bool has_g, float coef, float decay, float beta1,
                                         float omb1, float beta2, float omb2, float step_size,
                                         float bc2_sqrt, float eps, float ema_beta, float ome) {
  if (has_g) {
    gv = gv * coef;
    pv = pv * decay;
    mv = beta1 * mv + omb1 * gv;
    vv = beta2 * vv + omb2 * (gv * gv);
    const float denom = sqrtf(vv) / bc2_sqrt + eps;
    pv = pv - step_size * (mv / denom);
  }
  if (ev) *ev = ema_beta * *ev + ome * pv;
}

__global__ __launch_bounds__(kOptThreads) void opt_update_kernel(
    const OptChunk c, const float* __restrict__ scalars, float lr, float beta1, float beta2,
    float eps, float weight_decay, float ema_beta) {
  __shared__ int s_t;
  if (threadIdx.x == 0) s_t = opt_tensor_of(c, blockIdx.x);
  __syncthreads();
  const int t = s_t;
  const int64_t i0 = (int64_t)(blockIdx.x - c.blk0[t]) * kOptElems;
  const int64_t n = c.n[t];
  float* p = c.p[t];
  const float* g = c.g[t];
  float* m = c.m[t];
  float* v = c.v[t];
  float* e = c.e[t];
  const bool has_g = g != nullptr;
  const float coef = scalars[0], step_size = scalars[2], bc2_sqrt = scalars[3];
  const float decay = 1.0f - lr * weight_decay;
  const float omb1 = 1.0f - beta1, omb2 = 1.0f - beta2, ome = 1.0f - ema_beta;
  if (i0 + kOptElems <= n) {
    // a full block: every load first (nontemporal: each byte is touched once per step), then
    // the updates, then the stores
    constexpr int kIt = kOptElems / (kOptThreads * 4);
    v4f P[kIt], G[kIt], M[kIt], V[kIt], E[kIt];
    const int64_t b = i0 + threadIdx.x * 4;
#pragma unroll
    for (int k = 0; k < kIt; ++k) {
      const int64_t i = b + k * kOptThreads * 4;
      P[k] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(p + i));
      if (has_g) {
        G[k] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(g + i));
        M[k] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(m + i));
        V[k] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(v + i));
      } else {
        G[k] = M[k] = V[k] = v4f{0.f, 0.f, 0.f, 0.f};
      }
      E[k] = e ? __builtin_nontemporal_load(reinterpret_cast<const v4f*>(e + i))
               : v4f{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int k = 0; k < kIt; ++k) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float pv = P[k][j], mv = M[k][j], vv = V[k][j], ev = E[k][j];
        opt_elem(pv, G[k][j], mv, vv, e ? &ev : nullptr, has_g, coef, decay, beta1, omb1, beta2,
                 omb2, step_size, bc2_sqrt, eps, ema_beta, ome);
        P[k][j] = pv;
        M[k][j] = mv;
        V[k][j] = vv;
        E[k][j] = ev;
      }
    }
#pragma unroll
    for (int k = 0; k < kIt; ++k) {
      const int64_t i = b + k * kOptThreads * 4;
      if (has_g) {
        __builtin_nontemporal_store(P[k], reinterpret_cast<v4f*>(p + i));
        __builtin_nontemporal_store(M[k], reinterpret_cast<v4f*>(m + i));
        __builtin_nontemporal_store(V[k], reinterpret_cast<v4f*>(v + i));
      }
      if (e) __builtin_nontemporal_store(E[k], reinterpret_cast<v4f*>(e + i));
    }
    return;
  }
  for (int64_t i = i0 + threadIdx.x * 4; i < i0 + kOptElems && i < n; i += kOptThreads * 4) {
    if (i + 4 <= n) {
      float4 pv = *reinterpret_cast<float4*>(p + i);
      float4 gv = has_g ? *reinterpret_cast<const float4*>(g + i) : float4{0.f, 0.f, 0.f, 0.f};
      float4 mv = has_g ? *reinterpret_cast<float4*>(m + i) : float4{0.f, 0.f, 0.f, 0.f};
      float4 vv = has_g ? *reinterpret_cast<float4*>(v + i) : float4{0.f, 0.f, 0.f, 0.f};
      float4 ev = e ? *reinterpret_cast<float4*>(e + i) : float4{0.f, 0.f, 0.f, 0.f};
      float* P = &pv.x;
      float* G = &gv.x;
      float* M = &mv.x;
      float* V = &vv.x;
      float* E = &ev.x;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        opt_elem(P[k], G[k], M[k], V[k], e ? E + k : nullptr, has_g, coef, decay, beta1, omb1,
                 beta2, omb2, step_size, bc2_sqrt, eps, ema_beta, ome);
      if (has_g) {
        *reinterpret_cast<float4*>(p + i) = pv;
        *reinterpret_cast<float4*>(m + i) = mv;
        *reinterpret_cast<float4*>(v + i) = vv;
      }
      if (e) *reinterpret_cast<float4*>(e + i) = ev;
    } else {
      for (int64_t j = i; j < n; ++j) {
        float pv = p[j], mv = has_g ? m[j] : 0.f, vv = has_g ? v[j] : 0.f;
        opt_elem(pv, has_g ? g[j] : 0.f, mv, vv, e ? e + j : nullptr, has_g, coef, decay,
                 beta1, omb1, beta2, omb2, step_size, bc2_sqrt, eps, ema_beta, ome);
        if (has_g) {
          p[j] = pv;
          m[j] = mv;
          v[j] = vv;
        }
      }
    }
  }
}

static int opt_blocks(int64_t n) { return (int)ceil_div(n, (int64_t)kOptElems); }

}  // namespace dpa

using namespace dpa;

extern "C" int64_t dpa_adamw_ema_workspace_bytes(const DpaOptTensor* tensors, int count) {
  if (!tensors || count <= 0) return 0;
  int64_t blocks = 0;
  for (int i = 0; i < count; ++i) blocks += opt_blocks(tensors[i].n > 0 ? tensors[i].n : 1);
  return (blocks + kOptScalars) * 4;
}

extern "C" int dpa_adamw_ema_step(const DpaOptTensor* tensors, int count, float* step, float lr,
                                  float beta1, float beta2, float eps, float weight_decay,
                                  float max_norm, float ema_beta, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  if (!tensors || !step || !workspace) return DPA_ERR_NULL;
  if (count <= 0) return DPA_ERR_SIZE;
  if (workspace_bytes < dpa_adamw_ema_workspace_bytes(tensors, count)) return DPA_ERR_WORKSPACE;
  if (!aligned(workspace, 16)) return DPA_ERR_ALIGN;
  for (int i = 0; i < count; ++i) {
    const DpaOptTensor& T = tensors[i];
    if (!T.param || (!T.grad && !T.ema) || (T.grad && (!T.exp_avg || !T.exp_avg_sq)))
      return DPA_ERR_NULL;
    if (T.n <= 0) return DPA_ERR_SIZE;
    if (!aligned(T.param, 16) || !aligned(T.grad, 16) || !aligned(T.exp_avg, 16) ||
        !aligned(T.exp_avg_sq, 16) || !aligned(T.ema, 16))
      return DPA_ERR_ALIGN;
  }
  hipStream_t s = (hipStream_t)stream;
  float* partials = (float*)workspace;
  int64_t total_blocks = 0;
  for (int i = 0; i < count; ++i) total_blocks += opt_blocks(tensors[i].n);
  float* scalars = partials + total_blocks;
  // tensor chunks of at most kOptMaxT, the same chunks for both passes
  auto for_chunks = [&](auto launch) -> int {
    int part0 = 0;
    for (int c0 = 0; c0 < count; c0 += kOptMaxT) {
      OptChunk ch{};
      ch.count = count - c0 < kOptMaxT ? count - c0 : kOptMaxT;
      int b = 0;
      for (int k = 0; k < ch.count; ++k) {
        const DpaOptTensor& T = tensors[c0 + k];
        ch.blk0[k] = b;
        ch.p[k] = T.param;
        ch.g[k] = T.grad;
        ch.m[k] = T.exp_avg;
        ch.v[k] = T.exp_avg_sq;
        ch.e[k] = T.ema;
        ch.n[k] = T.n;
        b += opt_blocks(T.n);
      }
      ch.blk0[ch.count] = b;
      ch.part0 = part0;
      launch(ch, b);
      const int st = launch_status();
      if (st != DPA_OK) return st;
      part0 += b;
    }
    return DPA_OK;
  };
  int st = for_chunks([&](const OptChunk& ch, int b) {
    opt_norm_kernel<<<(unsigned)b, kOptThreads, 0, s>>>(ch, partials);
  });
  if (st != DPA_OK) return st;
  opt_finalize_kernel<<<1, kOptThreads, 0, s>>>(partials, (int)total_blocks, step, scalars,
                                                max_norm, lr, beta1, beta2);
  st = launch_status();
  if (st != DPA_OK) return st;
  return for_chunks([&](const OptChunk& ch, int b) {
    opt_update_kernel<<<(unsigned)b, kOptThreads, 0, s>>>(ch, scalars, lr, beta1, beta2, eps,
                                                           weight_decay, ema_beta);
  });
}
