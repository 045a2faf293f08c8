// Grouped FP8 linear layers that read one shared input: the FiLM projections of the U-Net's
// residual blocks (diffusion/unet.py:101-104 TimeEmbed, used at :135 -- every block projects
// the same time embedding to its (w, b) pair). One launch per direction serves all of them,
// each layer keeping its own per-tensor scales:
//   quantize  q_i   = e4m3(x_i / s_i), s_i = amax(x_i) / 448      (quant.hip's rule, per layer)
//   forward   y_i   = bf16(RN32(x_q w_i^T * RN32(s_x s_wi)))      (igemm.hip's epilogue)
//   wgrad     dw_i  = bf16(dy_i^T x_q * RN32(s_x s_dyi)), as fp32 (wgrad.hip's epilogue)
//   dgrad     dx    = bf16(sum_i RN32(dy_i w_i * RN32(s_dyi s_wi))), the layers summed in fp32
//                     in their order (per-layer dgrads would be rounded to bf16 each and summed
//                     by autograd in bf16).
// The problems are tiny (the batch is M, K = 512, N_i = 2C): the kernels read their MFMA
// fragments straight from global memory (L2-resident) without LDS staging; their cost is the
// launch, which is the point of grouping 22 layers x 4 launches into 5.
#include "dpa_common.hpp"

namespace dpa {

constexpr int kGrMaxSeg = 32;
constexpr int kGrThreads = 256;
constexpr int kGrTile = 64;  // output tile edge of the GEMM kernels (4 waves x 16 rows)

// ---- quantization: one workgroup per layer, over its [R][n_i] bf16 input ----
struct GrQuantArgs {
  const uint16_t* src[kGrMaxSeg];  // [R][n_i] bf16, dense
  int n[kGrMaxSeg];                // n_i (multiple of 8)
  int off[kGrMaxSeg];              // column offset of layer i in the concatenated outputs
  uint8_t* q;                      // [R][ntot] e4m3 (row-major), or null
  uint8_t* qt;                     // [ntot][R] e4m3 (its transpose), or null
  float* scale;                    // [nseg]
  int R, ntot;
};

__global__ __launch_bounds__(kGrThreads) void grouped_quant_kernel(const GrQuantArgs a) {
  __shared__ uint32_t red[kGrThreads / 64];
  const int seg = blockIdx.x;
  const uint16_t* src = a.src[seg];
  const int n = a.n[seg], off = a.off[seg];
  const int nv = a.R * n / 8;  // groups of 8 elements
  us2 acc = {0, 0};
  for (int v = threadIdx.x; v < nv; v += kGrThreads)
    acc = absmax8(acc, *reinterpret_cast<const uint4*>(src + 8 * (int64_t)v));
  uint32_t m = acc.x > acc.y ? acc.x : acc.y;
  m = wave_max_u32(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  uint32_t amax = red[0];
#pragma unroll
  for (int i = 1; i < kGrThreads / 64; ++i) amax = amax > red[i] ? amax : red[i];
  const float scale = scale_from_amax_bits(amax);
  if (threadIdx.x == 0) a.scale[seg] = scale;
  const float r = quant_recip(scale);
  for (int v = threadIdx.x; v < nv; v += kGrThreads) {
    const uint2 q8 = quant8_delayed(*reinterpret_cast<const uint4*>(src + 8 * (int64_t)v), scale, r);
    const int row = (8 * v) / n, col = 8 * v - row * n;
    if (a.q) *reinterpret_cast<uint2*>(a.q + (int64_t)row * a.ntot + off + col) = q8;
    if (a.qt) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        a.qt[(int64_t)(off + col + j) * a.R + row] = (uint8_t)((j < 4 ? q8.x : q8.y) >> (8 * (j & 3)));
    }
  }
}

// ---- GEMM kernels: workgroup tile 64 x 64 of D[row][col] = sum_k A[row][k] B[col][k], A and B
// K-contiguous e4m3 rows; wave w owns rows 16w .. 16w + 15 and all 64 columns. Lane (frow, fq)
// of an MFMA fragment holds row 16 (block) + frow, K bytes [32 fq, +32) of the 128-byte step;
// the result lane holds rows 4 fq .. + 3 of column frow. ----
__device__ __forceinline__ v8i gr_frag(const uint8_t* row_ptr, int k0, int fq) {
  const uint8_t* p = row_ptr + k0 + 32 * fq;
  const uint4 lo = *reinterpret_cast<const uint4*>(p);
  const uint4 hi = *reinterpret_cast<const uint4*>(p + 16);
  return v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}

// acc[j] (column block j) over K bytes: A rows a_row (this lane's row of the wave's block),
// B rows b_rows[j]
__device__ __forceinline__ void gr_mma(const uint8_t* a_row, const uint8_t* const (&b_row)[4],
                                       int K, int fq, v4f (&acc)[4]) {
  for (int k0 = 0; k0 < K; k0 += 128) {
    const v8i fa = gr_frag(a_row, k0, fq);
    v8i fb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) fb[j] = gr_frag(b_row[j], k0, fq);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = mfma16x16x128_e4m3(fa, fb[j], acc[j]);
  }
}

struct GrGemmArgs {
  int nseg;
  int tile0[kGrMaxSeg + 1];   // first column-tile (of 64 features) of each layer; [nseg] = total
  int n[kGrMaxSeg];
  int off[kGrMaxSeg];         // feature offset of the layer in concatenated buffers
  const uint8_t* w[kGrMaxSeg];   // forward: w_i [n_i][K]; dgrad: w_i^T [K][n_i]
  const float* sw[kGrMaxSeg];    // s_wi
  void* out[kGrMaxSeg];          // forward: y_i bf16 [M][n_i]; wgrad: dw_i fp32 [n_i][K]
  const uint8_t* x;   // forward: x_q [M][K]; wgrad: x_q^T [K][M]
  const uint8_t* dy;  // dgrad: dy_q [M][ntot]; wgrad: dy_q^T [ntot][M]
  const float* sx;
  const float* sdy;   // [nseg]
  float* partial;     // dgrad: [nseg][M][K] fp32
  int M, K, ntot;
};

__device__ __forceinline__ int gr_segment(const GrGemmArgs& a, int tile) {
  int s = 0;
  while (s + 1 < a.nseg && a.tile0[s + 1] <= tile) ++s;
  return s;
}

// forward: grid (sum_i n_i / 64, M / 64). D[n][m] = sum_k w_i[n][k] x[m][k]; lane stores
// y_i[m][n .. n + 3] (8 B).
__global__ __launch_bounds__(kGrThreads) void grouped_fwd_kernel(const GrGemmArgs a) {
  const int seg = gr_segment(a, blockIdx.x);
  const int n0 = (blockIdx.x - a.tile0[seg]) * kGrTile, m0 = blockIdx.y * kGrTile;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int frow = lane & 15, fq = lane >> 4;
  const uint8_t* a_row = a.w[seg] + (int64_t)(n0 + 16 * wave + frow) * a.K;
  const uint8_t* b_row[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) b_row[j] = a.x + (int64_t)(m0 + 16 * j + frow) * a.K;
  v4f acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
  gr_mma(a_row, b_row, a.K, fq, acc);
  const float scale = a.sx[0] * a.sw[seg][0];
  uint16_t* y = static_cast<uint16_t*>(a.out[seg]);
  const int n = a.n[seg];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = m0 + 16 * j + frow, f = n0 + 16 * wave + 4 * fq;
    *reinterpret_cast<uint2*>(y + (int64_t)m * n + f) =
        uint2{pack_bf16x2(acc[j][0] * scale, acc[j][1] * scale),
              pack_bf16x2(acc[j][2] * scale, acc[j][3] * scale)};
  }
}

// wgrad: grid (sum_i n_i / 64, K / 64). D[k][n] = sum_m x^T[k][m] dy^T[off_i + n][m]; lane
// stores dw_i[n][k .. k + 3] (16 B of fp32 holding bf16 values).
__global__ __launch_bounds__(kGrThreads) void grouped_wgrad_kernel(const GrGemmArgs a) {
  const int seg = gr_segment(a, blockIdx.x);
  const int n0 = (blockIdx.x - a.tile0[seg]) * kGrTile, k0 = blockIdx.y * kGrTile;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int frow = lane & 15, fq = lane >> 4;
  const uint8_t* a_row = a.x + (int64_t)(k0 + 16 * wave + frow) * a.M;
  const uint8_t* b_row[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    b_row[j] = a.dy + (int64_t)(a.off[seg] + n0 + 16 * j + frow) * a.M;
  v4f acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
  gr_mma(a_row, b_row, a.M, fq, acc);
  const float scale = a.sx[0] * a.sdy[seg];
  float* dw = static_cast<float*>(a.out[seg]);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int nn = n0 + 16 * j + frow, k = k0 + 16 * wave + 4 * fq;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = bf16_bits_to_f32(f32_to_bf16_bits(acc[j][e] * scale));
    *reinterpret_cast<float4*>(dw + (int64_t)nn * a.K + k) = float4{v[0], v[1], v[2], v[3]};
  }
}

// dgrad, per layer: grid (nseg * K / 64, M / 64). D[k][m] = sum_n w_i^T[k][n] dy[m][off_i + n]
// scaled by RN32(s_dyi s_wi) into partial[i][m][k .. k + 3].
__global__ __launch_bounds__(kGrThreads) void grouped_dgrad_kernel(const GrGemmArgs a) {
  const int kt = a.K / kGrTile;
  const int seg = blockIdx.x / kt;
  const int k0 = (blockIdx.x - seg * kt) * kGrTile, m0 = blockIdx.y * kGrTile;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int frow = lane & 15, fq = lane >> 4;
  const int n = a.n[seg];
  const uint8_t* a_row = a.w[seg] + (int64_t)(k0 + 16 * wave + frow) * n;
  const uint8_t* b_row[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    b_row[j] = a.dy + (int64_t)(m0 + 16 * j + frow) * a.ntot + a.off[seg];
  v4f acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
  gr_mma(a_row, b_row, n, fq, acc);
  const float scale = a.sdy[seg] * a.sw[seg][0];
  float* part = a.partial + (int64_t)seg * a.M * a.K;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = m0 + 16 * j + frow, k = k0 + 16 * wave + 4 * fq;
    *reinterpret_cast<float4*>(part + (int64_t)m * a.K + k) =
        float4{acc[j][0] * scale, acc[j][1] * scale, acc[j][2] * scale, acc[j][3] * scale};
  }
}

// dx[m][k] = bf16(sum over layers in order of partial[i][m][k]); 4 elements per thread
__global__ __launch_bounds__(kGrThreads) void grouped_dgrad_reduce_kernel(
    const float* __restrict__ partial, uint16_t* __restrict__ dx, int nseg, int64_t mk) {
  const int64_t i = ((int64_t)blockIdx.x * kGrThreads + threadIdx.x) * 4;
  if (i >= mk) return;
  float4 s = *reinterpret_cast<const float4*>(partial + i);
  for (int g = 1; g < nseg; ++g) {
    const float4 v = *reinterpret_cast<const float4*>(partial + (int64_t)g * mk + i);
    s.x += v.x;
    s.y += v.y;
    s.z += v.z;
    s.w += v.w;
  }
  *reinterpret_cast<uint2*>(dx + i) = uint2{pack_bf16x2(s.x, s.y), pack_bf16x2(s.z, s.w)};
}

}  // namespace dpa

using namespace dpa;

static int gr_check_layers(int nseg, const int* n) {
  if (nseg <= 0 || nseg > kGrMaxSeg || !n) return DPA_ERR_SIZE;
  for (int i = 0; i < nseg; ++i)
    if (n[i] <= 0 || n[i] % kGrTile != 0) return DPA_ERR_SHAPE;
  return DPA_OK;
}

extern "C" int dpa_grouped_quantize_fp8_bf16(const void* const* src, const int* n, int nseg,
                                             int R, void* q, void* qt, float* scale,
                                             void* stream) {
  if (!src || !scale || (!q && !qt)) return DPA_ERR_NULL;
  if (nseg <= 0 || nseg > kGrMaxSeg || R <= 0) return DPA_ERR_SIZE;
  GrQuantArgs a{};
  int off = 0;
  for (int i = 0; i < nseg; ++i) {
    if (!src[i]) return DPA_ERR_NULL;
    if (n[i] <= 0 || n[i] % 8 != 0) return DPA_ERR_SHAPE;
    if (!aligned(src[i], 16)) return DPA_ERR_ALIGN;
    a.src[i] = (const uint16_t*)src[i];
    a.n[i] = n[i];
    a.off[i] = off;
    off += n[i];
  }
  if (!aligned(q, 8) || !aligned(scale, 4)) return DPA_ERR_ALIGN;
  if ((int64_t)R * off > 0x7fffffff) return DPA_ERR_SIZE;
  a.q = (uint8_t*)q;
  a.qt = (uint8_t*)qt;
  a.scale = scale;
  a.R = R;
  a.ntot = off;
  grouped_quant_kernel<<<(unsigned)nseg, kGrThreads, 0, (hipStream_t)stream>>>(a);
  return launch_status();
}

// shared argument setup of the GEMM entries: layers i = 0 .. nseg - 1 with n[i] features
static int gr_gemm_setup(GrGemmArgs& a, int nseg, const int* n, int M, int K) {
  const int st = gr_check_layers(nseg, n);
  if (st != DPA_OK) return st;
  if (M <= 0 || K <= 0 || M % kGrTile != 0 || K % 128 != 0) return DPA_ERR_SHAPE;
  a.nseg = nseg;
  a.M = M;
  a.K = K;
  int off = 0, t = 0;
  for (int i = 0; i < nseg; ++i) {
    a.n[i] = n[i];
    a.off[i] = off;
    a.tile0[i] = t;
    off += n[i];
    t += n[i] / kGrTile;
  }
  a.tile0[nseg] = t;
  a.ntot = off;
  if ((int64_t)M * off > 0x7fffffff || (int64_t)K * off > 0x7fffffff) return DPA_ERR_SIZE;
  return DPA_OK;
}

extern "C" int dpa_grouped_linear_fwd_fp8(const void* xq, const float* x_scale,
                                          const void* const* wq, const float* const* w_scale,
                                          void* const* y, const int* n, int nseg, int M, int K,
                                          void* stream) {
  if (!xq || !x_scale || !wq || !w_scale || !y || !n) return DPA_ERR_NULL;
  GrGemmArgs a{};
  const int st = gr_gemm_setup(a, nseg, n, M, K);
  if (st != DPA_OK) return st;
  for (int i = 0; i < nseg; ++i) {
    if (!wq[i] || !w_scale[i] || !y[i]) return DPA_ERR_NULL;
    if (!aligned(wq[i], 16) || !aligned(y[i], 8)) return DPA_ERR_ALIGN;
    a.w[i] = (const uint8_t*)wq[i];
    a.sw[i] = w_scale[i];
    a.out[i] = y[i];
  }
  if (!aligned(xq, 16)) return DPA_ERR_ALIGN;
  a.x = (const uint8_t*)xq;
  a.sx = x_scale;
  dim3 grid((unsigned)a.tile0[nseg], (unsigned)(M / kGrTile));
  grouped_fwd_kernel<<<grid, kGrThreads, 0, (hipStream_t)stream>>>(a);
  return launch_status();
}

extern "C" int dpa_grouped_linear_wgrad_fp8_f32(const void* xq_t, const float* x_scale,
                                                const void* dyq_t, const float* dy_scale,
                                                float* const* dw, const int* n, int nseg,
                                                int M, int K, void* stream) {
  if (!xq_t || !x_scale || !dyq_t || !dy_scale || !dw || !n) return DPA_ERR_NULL;
  GrGemmArgs a{};
  const int st = gr_gemm_setup(a, nseg, n, M, K);
  if (st != DPA_OK) return st;
  if (M % 128 != 0 || K % kGrTile != 0) return DPA_ERR_SHAPE;  // K of this GEMM is M
  for (int i = 0; i < nseg; ++i) {
    if (!dw[i]) return DPA_ERR_NULL;
    if (!aligned(dw[i], 16)) return DPA_ERR_ALIGN;
    a.out[i] = dw[i];
  }
  if (!aligned(xq_t, 16) || !aligned(dyq_t, 16)) return DPA_ERR_ALIGN;
  a.x = (const uint8_t*)xq_t;
  a.dy = (const uint8_t*)dyq_t;
  a.sx = x_scale;
  a.sdy = dy_scale;
  dim3 grid((unsigned)a.tile0[nseg], (unsigned)(K / kGrTile));
  grouped_wgrad_kernel<<<grid, kGrThreads, 0, (hipStream_t)stream>>>(a);
  return launch_status();
}

extern "C" int64_t dpa_grouped_linear_dgrad_workspace_bytes(int nseg, int M, int K) {
  if (nseg <= 0 || M <= 0 || K <= 0) return 0;
  return (int64_t)nseg * M * K * 4;
}

extern "C" int dpa_grouped_linear_dgrad_fp8(const void* dyq, const float* dy_scale,
                                            const void* const* wq_t, const float* const* w_scale,
                                            void* dx, const int* n, int nseg, int M, int K,
                                            void* workspace, int64_t workspace_bytes,
                                            void* stream) {
  if (!dyq || !dy_scale || !wq_t || !w_scale || !dx || !n) return DPA_ERR_NULL;
  GrGemmArgs a{};
  const int st = gr_gemm_setup(a, nseg, n, M, K);
  if (st != DPA_OK) return st;
  if (K % kGrTile != 0) return DPA_ERR_SHAPE;
  for (int i = 0; i < nseg; ++i) {
    if (n[i] % 128 != 0) return DPA_ERR_SHAPE;  // the K of this GEMM is n_i
    if (!wq_t[i] || !w_scale[i]) return DPA_ERR_NULL;
    if (!aligned(wq_t[i], 16)) return DPA_ERR_ALIGN;
    a.w[i] = (const uint8_t*)wq_t[i];
    a.sw[i] = w_scale[i];
  }
  if (!workspace || workspace_bytes < dpa_grouped_linear_dgrad_workspace_bytes(nseg, M, K))
    return DPA_ERR_WORKSPACE;
  if (!aligned(dyq, 16) || !aligned(dx, 8) || !aligned(workspace, 16)) return DPA_ERR_ALIGN;
  a.dy = (const uint8_t*)dyq;
  a.sdy = dy_scale;
  a.partial = (float*)workspace;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid((unsigned)(nseg * (K / kGrTile)), (unsigned)(M / kGrTile));
  grouped_dgrad_kernel<<<grid, kGrThreads, 0, s>>>(a);
  int r = launch_status();
  if (r != DPA_OK) return r;
  const int64_t mk = (int64_t)M * K;
  grouped_dgrad_reduce_kernel<<<(unsigned)ceil_div(mk / 4, (int64_t)kGrThreads), kGrThreads, 0, s>>>(
      (const float*)workspace, (uint16_t*)dx, nseg, mk);
  return launch_status();
}
