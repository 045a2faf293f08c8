// Self-attention of the U-Net's attention blocks, softmax(q k^T / sqrt(64)) v, forward and
// backward, bf16 operands on the gfx950 bf16 MFMA (v_mfma_f32_16x16x32_bf16), fp32 softmax.
//
// Reference: diffusion/unet.py:181-203 (CHWAttention.forward): q, k, v = chunk(qkv, 3, -1),
// "b l (nh hd) -> b nh l hd", F.scaled_dot_product_attention (:196, no mask, no dropout,
// scale 1 / sqrt(hd)), "b nh l hd -> b l (nh hd)". The kernels read q, k and v in place from
// the qkv projection's output [B][L][3C] (head h at columns h * 64 of each third) and write the
// output as [B][L][C], the out projection's input: no head transposes in HBM. The backward
// writes dq, dk and dv into one [B][L][3C] tensor, the qkv projection's output gradient.
//
// Sequence lengths of the U-Net (16x16, 8x8 and 4x4 tokens: L = 256, 64, 16) fit one
// workgroup per (image, head): the keys and values of a head (L x 64 bf16, 32 KB at L = 256)
// stay in LDS, the scores of a 16-query block (L fp32 per lane-column) in registers, so the
// softmax is exact in one pass (no running rescale) and nothing of size L x L touches HBM.
// L is padded to LP in {32, 64, 128, 256} (L % 16 == 0, LP / 2 < L <= LP); padded keys are
// masked, padded queries skipped.
//
// Numerics (those of the flash-attention kernels torch dispatches to): scores in fp32 from
// bf16 products, p = 2^(s * log2(e) / 8 - m'), row sums of the fp32 p, p rounded to bf16 for
// the p v product, output divided by the row sum in fp32 and rounded to bf16. The backward
// recomputes p from the saved log-sum-exp (base 2), D = rowsum(do * o) from the bf16 output,
// ds = p (dp - D) in fp32, p and ds rounded to bf16 for their products; dq and dk scaled by
// 1/8 (exact) in fp32 before their bf16 rounding. No atomics: every output element has one
// writer and every sum a fixed order, so results are bitwise reproducible.
#include "dpa_common.hpp"

namespace dpa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kAttHD = 64;                            // head dim
constexpr float kAttScale = 0.125f;                   // 1 / sqrt(64), exact
constexpr float kAttC = 0.18033688011112042f;         // log2(e) / 8

// D(16x16 f32) += A(16x32 bf16) * B(32x16 bf16). Lane l supplies row (l & 15) of A and
// column (l & 15) of B, 8 K-elements each (K slice l >> 4); lane l receives
// D[4*(l>>4) + t][l & 15]. Any assignment of logical k to (slice, element) works as long as A
// and B use the same one; the kernels below use that freedom to feed MFMA outputs back in.
__device__ __forceinline__ v4f mfma16x16x32_bf16(uint4 a, uint4 b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint4 ld16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }

__device__ __forceinline__ void unpack8_bf16(uint4 v, float (&f)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    f[2 * t] = __uint_as_float(w[t] << 16);
    f[2 * t + 1] = __uint_as_float(w[t] & 0xffff0000u);
  }
}

typedef short v4s __attribute__((ext_vector_type(4)));

// gfx950 transpose read (ds_read_b64_tr_b16): the 16 lanes of a group address a 4-row x
// 16-column block of 16-bit elements (lane k: row k >> 2, columns 4 (k & 3) .. + 3) and lane j
// receives column j of the 4 rows, in row order.
__device__ __forceinline__ uint2 ld_tr16(const uint16_t* p) {
  const v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((v4s __attribute__((address_space(3)))*)(p));
  return __builtin_bit_cast(uint2, v);
}

// A fragment (rows = dims d0 + frow, k-slice fq) of the transpose of a row-major [rows][72]
// LDS array X, k running over X's rows: elements 0-3 = X[r1 + t][d0 + frow] and 4-7 =
// X[r2 + t][d0 + frow], t = 0..3 (r1, r2: this lane group's first rows).
__device__ __forceinline__ uint4 frag_tr(const uint16_t* x, int r1, int r2, int d0, int frow) {
  const int off = (frow >> 2) * 72 + d0 + 4 * (frow & 3);
  const uint2 lo = ld_tr16(x + r1 * 72 + off);
  const uint2 hi = ld_tr16(x + r2 * 72 + off);
  return uint4{lo.x, lo.y, hi.x, hi.y};
}

struct AttnArgs {
  const uint16_t* qkv;  // [B][L][3C] bf16
  const uint16_t* o;    // [B][L][C] bf16 (forward output; backward input)
  const uint16_t* dout; // [B][L][C] bf16 (backward)
  uint16_t* out;        // forward: o; backward: dqkv [B][L][3C]
  float* lse;           // [B * heads][L]: log2 of sum_k 2^(s * log2(e) / 8)
  uint32_t* amax_part;  // optional: per-workgroup max |out| (bf16 magnitude bits)
  int L, C, heads;
};

// Four fp32 -> two packed bf16 words, their magnitudes folded into am (u16 max per half).
__device__ __forceinline__ uint2 att_pack4(float a, float b, float c, float d, us2& am) {
  const uint2 w = uint2{pack_bf16x2(a, b), pack_bf16x2(c, d)};
  am = __builtin_elementwise_max(am, __builtin_bit_cast(us2, w.x & 0x7fff7fffu));
  am = __builtin_elementwise_max(am, __builtin_bit_cast(us2, w.y & 0x7fff7fffu));
  return w;
}

// The workgroup's max of what it stored, for the consumer's current-scaling cast; every
// thread calls it (uniform), NW waves.
template <int NW>
__device__ __forceinline__ void att_store_partial(us2 am, uint32_t* part) {
  __shared__ uint32_t red[NW];
  uint32_t m = am.x > am.y ? am.x : am.y;
  m = wave_max_u32(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) r = r > red[w] ? r : red[w];
    part[blockIdx.x] = r;
  }
}

// ---------------------------------------------------------------------------------------
// Forward: one workgroup (4 waves) per (image, head); K and V rows of the head in LDS
// (row-major, 144-B rows); wave w takes query blocks w, w + 4, ... of 16 queries. Per block,
// S^T = K Q^T (A = K rows, B = the block's queries from global, loaded one block ahead: lane
// (q = frow, k-slice fq) holds dims 8 fq .. + 7 of each 32-wide half), so lane (frow, fq)
// holds scores of query frow at keys 16 kb + 4 fq + t: the row max and sum need only the
// lane's own values and two shuffles. O^T = V^T P^T: B = P^T straight from those registers
// (k-step kk pairs score blocks 2 kk and 2 kk + 1, i.e. keys 32 kk + 4 fq + t and
// 32 kk + 16 + 4 fq + t in the lane's slice), A = V^T by transpose reads of the V rows at the
// same keys.
// ---------------------------------------------------------------------------------------
template <int LP>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(const AttnArgs p) {
  constexpr int KP = 72;          // K / V row pitch in LDS (144 B: 16 rows on distinct banks)
  constexpr int NKB = LP / 16;    // key blocks
  __shared__ __attribute__((aligned(16))) uint16_t ks[LP * KP];
  __shared__ __attribute__((aligned(16))) uint16_t vs[LP * KP];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int frow = lane & 15, fq = lane >> 4;
  const int bh = blockIdx.x;
  const int b = bh / p.heads, h = bh - b * p.heads;
  const int L = p.L, C = p.C;
  const int64_t S3 = 3 * (int64_t)C;
  const uint16_t* qg = p.qkv + (int64_t)b * L * S3 + h * kAttHD;
  const uint16_t* kg = qg + C;
  const uint16_t* vg = qg + 2 * C;

  // K and V rows into LDS (padded keys zero): every load in flight before the first store
  constexpr int NF = LP * 8 / 256;  // 16-B chunks per thread
  {
    uint4 kv[NF], vv[NF];
#pragma unroll
    for (int r = 0; r < NF; ++r) {
      const int c = tid + 256 * r, j = c >> 3, d0 = (c & 7) * 8;
      kv[r] = vv[r] = uint4{0u, 0u, 0u, 0u};
      if (j < L) {
        kv[r] = ld16(kg + j * S3 + d0);
        vv[r] = ld16(vg + j * S3 + d0);
      }
    }
#pragma unroll
    for (int r = 0; r < NF; ++r) {
      const int c = tid + 256 * r, j = c >> 3, d0 = (c & 7) * 8;
      *reinterpret_cast<uint4*>(ks + j * KP + d0) = kv[r];
      *reinterpret_cast<uint4*>(vs + j * KP + d0) = vv[r];
    }
  }
  // B fragments of the wave's first query block, then always one block ahead
  uint4 qf0 = {0u, 0u, 0u, 0u}, qf1 = {0u, 0u, 0u, 0u};
  if (wave * 16 < L) {
    const uint16_t* qr = qg + (wave * 16 + frow) * S3 + 8 * fq;
    qf0 = ld16(qr);
    qf1 = ld16(qr + 32);
  }
  __syncthreads();

  us2 am = {0, 0};
  for (int q0 = wave * 16; q0 < L; q0 += 64) {
    uint4 nq0 = {0u, 0u, 0u, 0u}, nq1 = {0u, 0u, 0u, 0u};
    if (q0 + 64 < L) {
      const uint16_t* qr = qg + (q0 + 64 + frow) * S3 + 8 * fq;
      nq0 = ld16(qr);
      nq1 = ld16(qr + 32);
    }
    v4f s[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const uint16_t* kr = ks + (16 * kb + frow) * KP + 8 * fq;
      s[kb] = mfma16x16x32_bf16(ld16(kr), qf0, v4f{0.f, 0.f, 0.f, 0.f});
      s[kb] = mfma16x16x32_bf16(ld16(kr + 32), qf1, s[kb]);
    }
    if (L < LP) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if (16 * kb + 4 * fq + t >= L) s[kb][t] = -__builtin_inff();
    }
    // phase boundaries keep the compiler from hoisting the next phase's LDS reads (and
    // their registers) above this one: at LP = 256 the scores alone take 64 registers
    __builtin_amdgcn_sched_barrier(0);
    float m = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int t = 0; t < 4; ++t) m = fmaxf(m, s[kb][t]);
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    const float mc = m * kAttC;
    float l = 0.f;
    uint32_t pk[NKB][2];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      float e[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        e[t] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][t], kAttC, -mc));
        l += e[t];
      }
      pk[kb][0] = pack_bf16x2(e[0], e[1]);
      pk[kb][1] = pack_bf16x2(e[2], e[3]);
    }
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    __builtin_amdgcn_sched_barrier(0);

    v4f o[4];
#pragma unroll
    for (int hb = 0; hb < 4; ++hb) o[hb] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < NKB / 2; ++kk) {
      const uint4 pf = {pk[2 * kk][0], pk[2 * kk][1], pk[2 * kk + 1][0], pk[2 * kk + 1][1]};
#pragma unroll
      for (int hb = 0; hb < 4; ++hb)
        o[hb] = mfma16x16x32_bf16(frag_tr(vs, 32 * kk + 4 * fq, 32 * kk + 16 + 4 * fq, 16 * hb, frow),
                                  pf, o[hb]);
      if (kk % 2 == 1) __builtin_amdgcn_sched_barrier(0);
    }
    const float il = 1.0f / l;
    uint16_t* orow = p.out + ((int64_t)b * L + q0 + frow) * C + h * kAttHD + 4 * fq;
#pragma unroll
    for (int hb = 0; hb < 4; ++hb)
      *reinterpret_cast<uint2*>(orow + 16 * hb) =
          att_pack4(o[hb][0] * il, o[hb][1] * il, o[hb][2] * il, o[hb][3] * il, am);
    if (fq == 0) p.lse[(int64_t)bh * L + q0 + frow] = mc + __builtin_amdgcn_logf(l);
    qf0 = nq0;
    qf1 = nq1;
  }
  if (p.amax_part) att_store_partial<4>(am, p.amax_part);
}

// ---------------------------------------------------------------------------------------
// Backward: one workgroup (8 waves) per (image, head). The head's Q, K and dO rows (row-major,
// 144-B rows), the log-sum-exp and D = rowsum(dO * O) of every query go into LDS once, with
// all their loads in flight together. Wave w owns KB key blocks (keys kw0 = 16 KB w ..) and
// keeps their K and V rows as B fragments and the dK^T, dV^T accumulators in registers;
// query blocks of 32 rows stream through:
//   S = Q K^T and dP = dO V^T (A = Q / dO rows from LDS) in the layout lane (frow, fq) <->
//   (query 16 sub + 4 fq + t, key frow);  P = 2^(S log2(e)/8 - lse), dS = P (dP - D);
//   dV^T += dO^T P and dK^T += Q^T dS: B = P / dS straight from those registers (the k-slice
//   of lane fq is queries 4 fq + t and 16 + 4 fq + t), A = dO^T / Q^T by transpose reads of
//   the rows at those queries;
//   dS (bf16) to one of two LDS buffers, one barrier, then dQ^T = K^T dS^T over all keys, one
//   (16-dim, 16-query) block per wave (A = K^T by transpose reads, B = dS rows). With the dS
//   buffers alternating, a wave can only overwrite one after every wave has passed the next
//   block's barrier, i.e. finished reading it.
// ---------------------------------------------------------------------------------------
template <int LP>
__global__ __launch_bounds__(512, 1) void attn_bwd_kernel(const AttnArgs p) {
  constexpr int KB = LP >= 256 ? 2 : 1;  // key blocks per wave
  constexpr int RP = 72;                 // Q / K / dO row pitch (144 B)
  constexpr int TP = LP + 8;             // dS row pitch
  __shared__ __attribute__((aligned(16))) uint16_t qs[LP * RP];
  __shared__ __attribute__((aligned(16))) uint16_t ks[LP * RP];
  __shared__ __attribute__((aligned(16))) uint16_t gs[LP * RP];
  __shared__ __attribute__((aligned(16))) uint16_t dsb[2][32 * TP];
  __shared__ float lse_s[LP], dd_s[LP];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int frow = lane & 15, fq = lane >> 4;
  const int bh = blockIdx.x;
  const int b = bh / p.heads, h = bh - b * p.heads;
  const int L = p.L, C = p.C;
  const int64_t S3 = 3 * (int64_t)C;
  const int64_t row0 = (int64_t)b * L;
  const uint16_t* qg = p.qkv + row0 * S3 + h * kAttHD;
  const uint16_t* kg = qg + C;
  const uint16_t* vg = qg + 2 * C;
  const uint16_t* og = p.o + row0 * C + h * kAttHD;
  const uint16_t* dg = p.dout + row0 * C + h * kAttHD;
  uint16_t* dqg = p.out + row0 * S3 + h * kAttHD;
  uint16_t* dkg = dqg + C;
  uint16_t* dvg = dqg + 2 * C;

  // Q, K, dO rows, the log-sum-exp and D per query (padded rows: zeros, lse = +inf, so their
  // P is 0); chunk c = row c / 8, dims 8 (c % 8) ..
  constexpr int NCH = LP * 8;
  constexpr int NF = (NCH + 511) / 512;
  // this wave's keys: B fragments of K and V (lane (key frow, k-slice fq): dims 8 fq .. + 7
  // of each 32-wide half), zero for padded keys; issued with the staging loads below
  const int kw0 = wave * 16 * KB;
  const bool kact = kw0 < LP;  // wave-uniform
  uint4 kf[KB][2], vf[KB][2];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int key = kw0 + 16 * kb + frow;
#pragma unroll
    for (int hs = 0; hs < 2; ++hs) {
      kf[kb][hs] = key < L ? ld16(kg + key * S3 + 32 * hs + 8 * fq) : uint4{0u, 0u, 0u, 0u};
      vf[kb][hs] = key < L ? ld16(vg + key * S3 + 32 * hs + 8 * fq) : uint4{0u, 0u, 0u, 0u};
    }
  }
  const float lse_t = tid < L ? p.lse[(int64_t)bh * L + tid] : __builtin_inff();
  {
    uint4 kv[NF], qv[NF], ov[NF], gv[NF];
#pragma unroll
    for (int r = 0; r < NF; ++r) {
      const int c = tid + 512 * r, j = c >> 3, d0 = (c & 7) * 8;
      kv[r] = qv[r] = ov[r] = gv[r] = uint4{0u, 0u, 0u, 0u};
      if (c < NCH && j < L) {
        kv[r] = ld16(kg + j * S3 + d0);
        qv[r] = ld16(qg + j * S3 + d0);
        ov[r] = ld16(og + j * C + d0);
        gv[r] = ld16(dg + j * C + d0);
      }
    }
#pragma unroll
    for (int r = 0; r < NF; ++r) {
      const int c = tid + 512 * r, j = c >> 3, d0 = (c & 7) * 8;
      if (NCH % 512 != 0 && c >= NCH) continue;  // wave-uniform (NCH % 64 == 0)
      *reinterpret_cast<uint4*>(ks + j * RP + d0) = kv[r];
      *reinterpret_cast<uint4*>(qs + j * RP + d0) = qv[r];
      *reinterpret_cast<uint4*>(gs + j * RP + d0) = gv[r];
      float fo[8], fg[8];
      unpack8_bf16(ov[r], fo);
      unpack8_bf16(gv[r], fg);
      float dot8 = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) dot8 += fo[e] * fg[e];
      dot8 += __shfl_xor(dot8, 1, 64);
      dot8 += __shfl_xor(dot8, 2, 64);
      dot8 += __shfl_xor(dot8, 4, 64);
      if ((c & 7) == 0) dd_s[j] = dot8;
    }
  }
  if (tid < LP) lse_s[tid] = lse_t;
  v4f dvt[4][KB], dkt[4][KB];
#pragma unroll
  for (int hb = 0; hb < 4; ++hb)
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) dvt[hb][kb] = dkt[hb][kb] = v4f{0.f, 0.f, 0.f, 0.f};
  __syncthreads();  // Q, K, dO rows, lse and D complete

  // the K^T operand of this wave's dQ block (dims 16 (wave & 3) ..) over all keys: the same
  // for every query block, so read once
  uint4 ktf[LP / 32];
#pragma unroll
  for (int kk = 0; kk < LP / 32; ++kk)
    ktf[kk] = frag_tr(ks, 32 * kk + 8 * fq, 32 * kk + 8 * fq + 4, 16 * (wave & 3), frow);

  // A fragments of a query block: rows q0 + 16 sub + frow of Q and dO (read one block ahead,
  // during the previous block's dQ products)
  uint4 qa[2][2], da[2][2];
  auto load_a = [&](int q0) __attribute__((always_inline)) {
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int hs = 0; hs < 2; ++hs) {
        const int o = (q0 + 16 * sub + frow) * RP + 32 * hs + 8 * fq;
        qa[sub][hs] = ld16(qs + o);
        da[sub][hs] = ld16(gs + o);
      }
  };
  if (kact) load_a(0);

  us2 am = {0, 0};
  // dQ^T block (dims 16 hb .., queries 16 sub ..) of the query block at q0 over all keys, from
  // that block's dS in LDS, in two interleaved accumulators (a shorter dependent chain)
  auto dq_block = [&](int q0, const uint16_t* ds) __attribute__((always_inline)) {
    const int hb = wave & 3, sub = wave >> 2;
    v4f acc2[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int kk = 0; kk < LP / 32; ++kk)
      acc2[kk & 1] = mfma16x16x32_bf16(ktf[kk], ld16(ds + (16 * sub + frow) * TP + 32 * kk + 8 * fq),
                                       acc2[kk & 1]);
    const v4f acc = acc2[0] + acc2[1];
    const int q = q0 + 16 * sub + frow;
    if (q < L)
      *reinterpret_cast<uint2*>(dqg + q * S3 + 16 * hb + 4 * fq) =
          att_pack4(acc[0] * kAttScale, acc[1] * kAttScale, acc[2] * kAttScale,
                    acc[3] * kAttScale, am);
  };
  // Block i's dQ runs in step i + 1, before that step's barrier: every wave has its own
  // products of the next block to issue instead of waiting at the barrier, and dS(i)'s buffer
  // is only rewritten (by block i + 2) after barrier i + 1.
  int q_last = 0;
  for (int q0 = 0, blk = 0; q0 < L; q0 += 32, ++blk) {
    uint16_t* ds = dsb[blk & 1];
    q_last = q0;
    if (kact) {
      uint4 pb[KB], sb[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        uint32_t pw[4], sw[4];
        const bool kin = kw0 + 16 * kb + frow < L;
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
          v4f sc = mfma16x16x32_bf16(qa[sub][0], kf[kb][0], v4f{0.f, 0.f, 0.f, 0.f});
          sc = mfma16x16x32_bf16(qa[sub][1], kf[kb][1], sc);
          v4f dp = mfma16x16x32_bf16(da[sub][0], vf[kb][0], v4f{0.f, 0.f, 0.f, 0.f});
          dp = mfma16x16x32_bf16(da[sub][1], vf[kb][1], dp);
          float pv[4], dsv[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int q = q0 + 16 * sub + 4 * fq + t;
            const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[t], kAttC, -lse_s[q]));
            pv[t] = kin ? e : 0.f;
            dsv[t] = pv[t] * (dp[t] - dd_s[q]);
          }
          pw[2 * sub] = pack_bf16x2(pv[0], pv[1]);
          pw[2 * sub + 1] = pack_bf16x2(pv[2], pv[3]);
          sw[2 * sub] = pack_bf16x2(dsv[0], dsv[1]);
          sw[2 * sub + 1] = pack_bf16x2(dsv[2], dsv[3]);
          // dS rows of the block to LDS for dQ (query 16 sub + 4 fq + t, key column)
          uint16_t* dcol = ds + (16 * sub + 4 * fq) * TP + kw0 + 16 * kb + frow;
          dcol[0] = (uint16_t)(sw[2 * sub] & 0xffffu);
          dcol[TP] = (uint16_t)(sw[2 * sub] >> 16);
          dcol[2 * TP] = (uint16_t)(sw[2 * sub + 1] & 0xffffu);
          dcol[3 * TP] = (uint16_t)(sw[2 * sub + 1] >> 16);
        }
        pb[kb] = uint4{pw[0], pw[1], pw[2], pw[3]};
        sb[kb] = uint4{sw[0], sw[1], sw[2], sw[3]};
      }
      const int r1 = q0 + 4 * fq, r2 = q0 + 16 + 4 * fq;
#pragma unroll
      for (int hb = 0; hb < 4; ++hb) {
        const uint4 da4 = frag_tr(gs, r1, r2, 16 * hb, frow);
        const uint4 qa4 = frag_tr(qs, r1, r2, 16 * hb, frow);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          dvt[hb][kb] = mfma16x16x32_bf16(da4, pb[kb], dvt[hb][kb]);
          dkt[hb][kb] = mfma16x16x32_bf16(qa4, sb[kb], dkt[hb][kb]);
        }
      }
    }
    if (blk > 0) dq_block(q0 - 32, dsb[(blk - 1) & 1]);
    __syncthreads();  // this block's dS complete
    if (kact && q0 + 32 < L) load_a(q0 + 32);
  }
  dq_block(q_last, dsb[((L + 31) / 32 - 1) & 1]);

  // dK, dV of this wave's keys: lane holds dims 16 hb + 4 fq + t of key kw0 + 16 kb + frow
  if (kact) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int key = kw0 + 16 * kb + frow;
      if (key >= L) continue;
#pragma unroll
      for (int hb = 0; hb < 4; ++hb) {
        const v4f k4 = dkt[hb][kb], v4 = dvt[hb][kb];
        *reinterpret_cast<uint2*>(dkg + key * S3 + 16 * hb + 4 * fq) =
            att_pack4(k4[0] * kAttScale, k4[1] * kAttScale, k4[2] * kAttScale,
                      k4[3] * kAttScale, am);
        *reinterpret_cast<uint2*>(dvg + key * S3 + 16 * hb + 4 * fq) =
            att_pack4(v4[0], v4[1], v4[2], v4[3], am);
      }
    }
  }
  if (p.amax_part) att_store_partial<8>(am, p.amax_part);
}

static int attn_lp(int L) {
  if (L <= 0 || L % 16 != 0 || L > 256) return 0;
  return L <= 32 ? 32 : L <= 64 ? 64 : L <= 128 ? 128 : 256;
}

static int attn_check(const void* a, const void* b, const void* c, int B, int L, int C,
                      int heads) {
  if (!a || !b || !c) return DPA_ERR_NULL;
  if (B <= 0 || heads <= 0 || C <= 0) return DPA_ERR_SIZE;
  if (C != heads * kAttHD || !attn_lp(L)) return DPA_ERR_SHAPE;
  if ((int64_t)B * L * 3 * C > 0x7fffffffLL || (int64_t)B * heads > 0x7fffffffLL)
    return DPA_ERR_SIZE;
  return DPA_OK;
}

}  // namespace dpa

using namespace dpa;

static int attn_fwd(const void* qkv, void* out, float* lse, int B, int L, int C, int heads,
                    uint32_t* amax_part, void* stream) {
  int st = attn_check(qkv, out, lse, B, L, C, heads);
  if (st != DPA_OK) return st;
  if (!aligned(qkv, 16) || !aligned(out, 8) || !aligned(lse, 4)) return DPA_ERR_ALIGN;
  AttnArgs a{};
  a.qkv = (const uint16_t*)qkv;
  a.out = (uint16_t*)out;
  a.lse = lse;
  a.amax_part = amax_part;
  a.L = L;
  a.C = C;
  a.heads = heads;
  const unsigned grid = (unsigned)(B * heads);
  hipStream_t s = (hipStream_t)stream;
  switch (attn_lp(L)) {
    case 32: attn_fwd_kernel<32><<<grid, 256, 0, s>>>(a); break;
    case 64: attn_fwd_kernel<64><<<grid, 256, 0, s>>>(a); break;
    case 128: attn_fwd_kernel<128><<<grid, 256, 0, s>>>(a); break;
    default: attn_fwd_kernel<256><<<grid, 256, 0, s>>>(a); break;
  }
  return launch_status();
}

extern "C" int dpa_attention_fwd_bf16(const void* qkv, void* out, float* lse, int B, int L,
                                      int C, int heads, void* stream) {
  return attn_fwd(qkv, out, lse, B, L, C, heads, nullptr, stream);
}

// dpa_attention_fwd_bf16 that also leaves one amax partial per (image, head) workgroup
// (B * heads of them: the max |out| as bf16 magnitude bits) for the out projection's
// current-scaling cast (dpa_quantize_fp8_bf16_from_partials).
extern "C" int dpa_attention_fwd_amax(const void* qkv, void* out, float* lse, int B, int L, int C,
                                      int heads, void* amax_partials, void* stream) {
  if (!amax_partials) return DPA_ERR_NULL;
  if (!aligned(amax_partials, 4)) return DPA_ERR_ALIGN;
  return attn_fwd(qkv, out, lse, B, L, C, heads, (uint32_t*)amax_partials, stream);
}

static int attn_bwd(const void* qkv, const void* out, const void* dout, const float* lse,
                    void* dqkv, int B, int L, int C, int heads, uint32_t* amax_part,
                    void* stream) {
  int st = attn_check(qkv, out, dqkv, B, L, C, heads);
  if (st != DPA_OK) return st;
  if (!dout || !lse) return DPA_ERR_NULL;
  if (!aligned(qkv, 16) || !aligned(out, 16) || !aligned(dout, 16) || !aligned(dqkv, 8) ||
      !aligned(lse, 4))
    return DPA_ERR_ALIGN;
  AttnArgs a{};
  a.qkv = (const uint16_t*)qkv;
  a.o = (const uint16_t*)out;
  a.dout = (const uint16_t*)dout;
  a.out = (uint16_t*)dqkv;
  a.lse = (float*)lse;
  a.amax_part = amax_part;
  a.L = L;
  a.C = C;
  a.heads = heads;
  const unsigned grid = (unsigned)(B * heads);
  hipStream_t s = (hipStream_t)stream;
  switch (attn_lp(L)) {
    case 32: attn_bwd_kernel<32><<<grid, 512, 0, s>>>(a); break;
    case 64: attn_bwd_kernel<64><<<grid, 512, 0, s>>>(a); break;
    case 128: attn_bwd_kernel<128><<<grid, 512, 0, s>>>(a); break;
    default: attn_bwd_kernel<256><<<grid, 512, 0, s>>>(a); break;
  }
  return launch_status();
}

extern "C" int dpa_attention_bwd_bf16(const void* qkv, const void* out, const void* dout,
                                      const float* lse, void* dqkv, int B, int L, int C,
                                      int heads, void* stream) {
  return attn_bwd(qkv, out, dout, lse, dqkv, B, L, C, heads, nullptr, stream);
}

// dpa_attention_bwd_bf16 that also leaves one amax partial per (image, head) workgroup
// (B * heads: the max |dqkv| over the dq, dk, dv it wrote) for the qkv projection's
// current-scaling cast of its output gradient.
extern "C" int dpa_attention_bwd_amax(const void* qkv, const void* out, const void* dout,
                                      const float* lse, void* dqkv, int B, int L, int C,
                                      int heads, void* amax_partials, void* stream) {
  if (!amax_partials) return DPA_ERR_NULL;
  if (!aligned(amax_partials, 4)) return DPA_ERR_ALIGN;
  return attn_bwd(qkv, out, dout, lse, dqkv, B, L, C, heads, (uint32_t*)amax_partials, stream);
}
