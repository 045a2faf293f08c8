/*
 * C restatement of the reference's per-tensor e4m3 cast, for exhaustive checks.
 * TEST INFRASTRUCTURE ONLY (used by tests/ and bench.py's cpu_baseline leg).
 *
 * Reference: diffusion/fp8_kernels.py
 *   finalize_amax_kernel :90-102   scale = amax > 0 ? amax / 448 : 1
 *   quantize_fp8_kernel  :105-120  q = e4m3(max(-448, min(f32(x) / scale, 448)))
 * The fp32 division is IEEE round-to-nearest (x86 SSE, no fast-math); the clamp uses
 * fminf/fmaxf (IEEE minNum/maxNum) in the kernel's order; e4m3 rounding is to nearest even.
 *
 * Digest of one scale: D(s) = sum over all 65536 bf16 bit patterns x of
 *   (q(x, s) + 1) * mix(x)   (mod 2^64), mix = splitmix64 finaliser | 1.
 * Any single changed byte changes D (mix is odd and |dq| < 256).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>

static inline float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint8_t oracle_e4m3_rne(float v) {
  uint32_t b;
  memcpy(&b, &v, 4);
  const uint32_t sign = (b >> 24) & 0x80u;
  const uint32_t a = b & 0x7fffffffu;
  if (a > 0x43e80000u) return (uint8_t)(sign | 0x7fu);
  if (a >= 0x3c800000u) {
    const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
    return (uint8_t)(sign | ((r >> 20) - 0x3c0u));
  }
  const int e = (int)(a >> 23) - 127;
  if (e < -126) return (uint8_t)sign;
  const uint32_t mant = (a & 0x7fffffu) | 0x800000u;
  const int s = 14 - e;
  if (s >= 25) return (uint8_t)sign;
  uint32_t m = mant >> s;
  const uint32_t rem = mant & ((1u << s) - 1u);
  const uint32_t half = 1u << (s - 1);
  if (rem > half || (rem == half && (m & 1u))) ++m;
  return (uint8_t)(sign | m);
}

void oracle_e4m3_rne_array(const float* v, int64_t n, uint8_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_e4m3_rne(v[i]);
}

/* every fp32 bit pattern in [lo, hi) -> e4m3 */
void oracle_e4m3_rne_range(uint32_t lo, uint32_t hi, uint8_t* out) {
  for (uint32_t u = lo; u < hi; ++u) {
    float f;
    memcpy(&f, &u, 4);
    out[u - lo] = oracle_e4m3_rne(f);
  }
}

float oracle_scale_from_amax(float amax) { return amax > 0.0f ? amax / 448.0f : 1.0f; }

static inline uint8_t cast_one(uint16_t x, float scale) {
  float q = bf16_to_f32(x) / scale;
  q = fmaxf(-448.0f, fminf(q, 448.0f));
  return oracle_e4m3_rne(q);
}

void oracle_cast(const uint16_t* x, int64_t n, float scale, uint8_t* q) {
  for (int64_t i = 0; i < n; ++i) q[i] = cast_one(x[i], scale);
}

float oracle_quantize(const uint16_t* x, int64_t n, uint8_t* q) {
  uint16_t m = 0;
  for (int64_t i = 0; i < n; ++i) {
    uint16_t a = x[i] & 0x7fffu;
    if (a > m) m = a;
  }
  float s = oracle_scale_from_amax(bf16_to_f32(m));
  oracle_cast(x, n, s, q);
  return s;
}

static inline uint64_t mix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return (z ^ (z >> 31)) | 1ull;
}

uint64_t oracle_cast_digest(float scale) {
  uint64_t d = 0;
  for (uint32_t x = 0; x < 65536u; ++x) d += (uint64_t)(cast_one((uint16_t)x, scale) + 1u) * mix64(x);
  return d;
}

typedef struct {
  const float* scales;
  int64_t begin, end;
  uint64_t* out;
} digest_job;

static void* digest_worker(void* arg) {
  digest_job* j = (digest_job*)arg;
  for (int64_t i = j->begin; i < j->end; ++i) j->out[i] = oracle_cast_digest(j->scales[i]);
  return 0;
}

void oracle_cast_digests(const float* scales, int64_t ns, uint64_t* out, int nthreads) {
  if (nthreads < 1) nthreads = 1;
  if (nthreads > 64) nthreads = 64;
  pthread_t th[64];
  digest_job jobs[64];
  for (int t = 0; t < nthreads; ++t) {
    jobs[t].scales = scales;
    jobs[t].begin = ns * t / nthreads;
    jobs[t].end = ns * (t + 1) / nthreads;
    jobs[t].out = out;
    pthread_create(&th[t], 0, digest_worker, &jobs[t]);
  }
  for (int t = 0; t < nthreads; ++t) pthread_join(th[t], 0);
}
