/*
 * CPU oracle for the llminfer attention hot path. TEST INFRASTRUCTURE ONLY:
 * loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
 * never by the product library. Declarations and layout notes: oracle.h.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

/* ------------------------------------------------------------------ fp16 */

/* Shift right by `shift` bits, rounding half to even.
 * Same rounding rule as roundShiftEven, lib/ModelFormat/Quantization.cpp:9-15. */
static uint32_t shift_round_even(uint32_t value, unsigned shift) {
  uint32_t kept = value >> shift;
  uint32_t rest = value & ((1u << shift) - 1u);
  uint32_t half = 1u << (shift - 1u);
  if (rest > half || (rest == half && (kept & 1u)))
    kept += 1u;
  return kept;
}

/* lib/ModelFormat/Quantization.cpp:25-41 (floatToHalf). */
uint16_t orc_f32_to_f16(float value) {
  uint32_t bits;
  memcpy(&bits, &value, sizeof bits);
  uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
  int exp = (int)((bits >> 23) & 0xffu) - 127;
  uint32_t man = bits & 0x7fffffu;
  if (exp < -25)
    return sign; /* below half the smallest subnormal: signed zero */
  if (exp < -14) /* subnormal half, implicit bit made explicit */
    return (uint16_t)(sign | shift_round_even(man | 0x800000u,
                                              (unsigned)(-exp - 1)));
  if (exp > 15) /* overflow to inf; NaN keeps a quiet payload bit */
    return (uint16_t)(sign | 0x7c00u | (exp == 128 && man ? 0x200u : 0u));
  /* A mantissa carry propagates into the exponent (and to inf at 65520). */
  return (uint16_t)(sign | ((uint32_t)((exp + 15) << 10) +
                            shift_round_even(man, 13)));
}

/* lib/ModelFormat/Quantization.cpp:43-55 (halfToFloat). */
float orc_f16_to_f32(uint16_t bits) {
  unsigned exp = (bits >> 10) & 0x1fu;
  unsigned man = bits & 0x3ffu;
  if (exp == 0) {
    float mag = ldexpf((float)man, -24);
    return (bits & 0x8000u) ? -mag : mag;
  }
  uint32_t out = ((uint32_t)(bits & 0x8000u) << 16) |
                 ((exp == 31 ? 255u : exp + 112u) << 23) | (man << 13);
  float f;
  memcpy(&f, &out, sizeof f);
  return f;
}

void orc_f32_to_f16_n(const float *in, uint16_t *out, size_t n) {
  for (size_t i = 0; i < n; ++i)
    out[i] = orc_f32_to_f16(in[i]);
}

void orc_f16_to_f32_n(const uint16_t *in, float *out, size_t n) {
  for (size_t i = 0; i < n; ++i)
    out[i] = orc_f16_to_f32(in[i]);
}

/* ------------------------------------------------------------------- RNG */

static const uint64_t kGolden = 0x9E3779B97F4A7C15ull;

static uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static double normal_at(uint64_t key, size_t i) {
  uint64_t a = mix64(key + (2 * (uint64_t)i + 1) * kGolden);
  uint64_t b = mix64(key + (2 * (uint64_t)i + 2) * kGolden);
  double u1 = ((double)(a >> 11) + 1.0) * 0x1p-53; /* (0, 1] */
  double u2 = (double)(b >> 11) * 0x1p-53;         /* [0, 1) */
  return sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925 * u2);
}

static uint64_t stream_key(uint64_t seed, uint64_t stream) {
  return mix64(mix64(seed * kGolden + 0x632BE59BD9B4E019ull) ^
               (stream * 0xD1B54A32D192ED03ull));
}

void orc_fill_normal_f32(uint64_t seed, uint64_t stream, size_t n, double mean,
                         double stddev, float *out) {
  uint64_t key = stream_key(seed, stream);
  for (size_t i = 0; i < n; ++i)
    out[i] = (float)(mean + stddev * normal_at(key, i));
}

void orc_fill_normal_f16(uint64_t seed, uint64_t stream, size_t n, double mean,
                         double stddev, uint16_t *out) {
  uint64_t key = stream_key(seed, stream);
  for (size_t i = 0; i < n; ++i)
    out[i] = orc_f32_to_f16((float)(mean + stddev * normal_at(key, i)));
}

/* tests/FlashAttentionTest.mm:28-36. */
void orc_fill_lcg_f16(uint32_t *state, size_t n, uint16_t *out) {
  uint32_t s = *state;
  for (size_t i = 0; i < n; ++i) {
    s = s * 1664525u + 1013904223u;
    out[i] = orc_f32_to_f16((float)((int)(s >> 24) - 128) / 64.0f);
  }
  *state = s;
}

/* ------------------------------------------------------ parallel helper */

int orc_cpu_count(void) {
  cpu_set_t set;
  if (sched_getaffinity(0, sizeof set, &set) == 0) {
    int n = CPU_COUNT(&set);
    if (n > 0)
      return n;
  }
  return 1;
}

typedef void (*task_fn)(void *ctx, size_t task);
typedef struct {
  task_fn fn;
  void *ctx;
  size_t tasks;
  size_t next; /* shared work counter */
} pool_job;

static void *pool_worker(void *arg) {
  pool_job *job = (pool_job *)arg;
  for (;;) {
    size_t t = __atomic_fetch_add(&job->next, 1, __ATOMIC_RELAXED);
    if (t >= job->tasks)
      break;
    job->fn(job->ctx, t);
  }
  return NULL;
}

static void parallel_for(size_t tasks, int threads, task_fn fn, void *ctx) {
  if (threads <= 0)
    threads = orc_cpu_count();
  if ((size_t)threads > tasks)
    threads = (int)tasks;
  pool_job job = {fn, ctx, tasks, 0};
  if (threads <= 1) {
    pool_worker(&job);
    return;
  }
  pthread_t *ids = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
  int started = 0;
  for (int i = 1; i < threads; ++i)
    if (pthread_create(&ids[started], NULL, pool_worker, &job) == 0)
      ++started;
  pool_worker(&job);
  for (int i = 0; i < started; ++i)
    pthread_join(ids[i], NULL);
  free(ids);
}

/* ------------------------------------------------------------- GQA (f64) */

typedef struct {
  const uint16_t *q, *k, *v;
  double *out;
  uint32_t T, Hq, Hkv, d, P;
} dense_job;

/* One (token, q-head) row of the dense attention; rows are independent, so
 * the result does not depend on how they are spread over threads. */
static void dense_row(void *ctx, size_t row) {
  const dense_job *j = (const dense_job *)ctx;
  uint32_t d = j->d, t = (uint32_t)(row / j->Hq), h = (uint32_t)(row % j->Hq);
  size_t kv_stride = (size_t)j->Hkv * d;
  size_t kv_off = (size_t)(h / (j->Hq / j->Hkv)) * d;
  double scale = 1.0 / sqrt((double)d);
  uint32_t visible = j->P + t + 1;
  double *p = (double *)malloc(sizeof(double) * visible);
  double *qf = (double *)malloc(sizeof(double) * d);
  for (uint32_t x = 0; x < d; ++x)
    qf[x] = orc_f16_to_f32(j->q[row * d + x]);
  double mx = -INFINITY;
  for (uint32_t k = 0; k < visible; ++k) {
    const uint16_t *kr = j->k + (size_t)k * kv_stride + kv_off;
    double dot = 0.0;
    for (uint32_t x = 0; x < d; ++x)
      dot += qf[x] * (double)orc_f16_to_f32(kr[x]);
    p[k] = dot * scale;
    if (p[k] > mx)
      mx = p[k];
  }
  double den = 0.0;
  for (uint32_t k = 0; k < visible; ++k) {
    p[k] = exp(p[k] - mx);
    den += p[k];
  }
  for (uint32_t x = 0; x < d; ++x) {
    double acc = 0.0;
    for (uint32_t k = 0; k < visible; ++k)
      acc += p[k] * (double)orc_f16_to_f32(j->v[(size_t)k * kv_stride + kv_off + x]);
    j->out[row * d + x] = acc / den;
  }
  free(qf);
  free(p);
}

void orc_gqa_dense_f64(const uint16_t *q, const uint16_t *k_cache,
                       const uint16_t *v_cache, double *out, uint32_t T,
                       uint32_t Hq, uint32_t Hkv, uint32_t d, uint32_t P) {
  dense_job job = {q, k_cache, v_cache, out, T, Hq, Hkv, d, P};
  parallel_for((size_t)T * Hq, 0, dense_row, &job);
}

/* --------------------------------------------------- GQA eager fp16 path */

static float round_f16(float x) { return orc_f16_to_f32(orc_f32_to_f16(x)); }

void orc_gqa_eager_f16(const uint16_t *q, const uint16_t *k_cache,
                       const uint16_t *v_cache, uint16_t *out, uint32_t T,
                       uint32_t Hq, uint32_t Hkv, uint32_t d, uint32_t P) {
  size_t kv_stride = (size_t)Hkv * d;
  uint32_t group = Hq / Hkv;
  float rs = 1.0f / sqrtf((float)d);
  float *s = (float *)malloc(sizeof(float) * ((size_t)P + T));
  for (uint32_t t = 0; t < T; ++t) {
    uint32_t count = P + t + 1;
    for (uint32_t h = 0; h < Hq; ++h) {
      size_t row = (size_t)t * Hq + h;
      size_t kv_off = (size_t)(h / group) * d;
      /* gqaScores: fp32 fma dot, rounded to fp16, scaled, rounded again. */
      for (uint32_t j = 0; j < count; ++j) {
        const uint16_t *kr = k_cache + (size_t)j * kv_stride + kv_off;
        float dot = 0.0f;
        for (uint32_t x = 0; x < d; ++x)
          dot = fmaf(orc_f16_to_f32(q[row * d + x]), orc_f16_to_f32(kr[x]),
                     dot);
        s[j] = round_f16(round_f16(dot) * rs);
      }
      /* gqaSoftmax: fp32 max and sum, fp16 probabilities. */
      float mx = -INFINITY;
      for (uint32_t j = 0; j < count; ++j)
        mx = s[j] > mx ? s[j] : mx;
      float sum = 0.0f;
      for (uint32_t j = 0; j < count; ++j)
        sum += expf(s[j] - mx);
      for (uint32_t j = 0; j < count; ++j)
        s[j] = round_f16(expf(s[j] - mx) / sum);
      /* gqaValue: fp32 fma accumulate of fp16 probabilities. */
      for (uint32_t x = 0; x < d; ++x) {
        float acc = 0.0f;
        for (uint32_t j = 0; j < count; ++j)
          acc = fmaf(s[j],
                     orc_f16_to_f32(v_cache[(size_t)j * kv_stride + kv_off + x]),
                     acc);
        out[row * d + x] = orc_f32_to_f16(acc);
      }
    }
  }
  free(s);
}

/* ------------------------------------------------- GQA fp32 (CPU baseline) */

/* Row conversion fp16 -> fp32. F16C when the host has it, else scalar. */
#if defined(__x86_64__)
__attribute__((target("avx2,f16c,fma"))) static void
cvt_row_f16c(const uint16_t *in, float *out, uint32_t n) {
  uint32_t i = 0;
  for (; i + 8 <= n; i += 8)
    _mm256_storeu_ps(out + i,
                     _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(in + i))));
  for (; i < n; ++i)
    out[i] = orc_f16_to_f32(in[i]);
}
#endif

static int g_has_f16c = -1;

static void cvt_row(const uint16_t *in, float *out, uint32_t n) {
#if defined(__x86_64__)
  if (g_has_f16c < 0)
    g_has_f16c = __builtin_cpu_supports("f16c") && __builtin_cpu_supports("avx2") &&
                 __builtin_cpu_supports("fma");
  if (g_has_f16c) {
    cvt_row_f16c(in, out, n);
    return;
  }
#endif
  for (uint32_t i = 0; i < n; ++i)
    out[i] = orc_f16_to_f32(in[i]);
}

typedef struct {
  const uint16_t *q, *k, *v;
  uint16_t *out;
  uint32_t T, Hq, Hkv, d, P;
  uint32_t splits; /* key-range splits per (token, kv head) */
  float *partial;  /* [T*Hkv*splits][group][d + 2] : o (unnormalised), m, l */
} gqa_job;

/* One task = (token, kv head, key split): all q-heads of the group share each
 * converted K/V row, which is how a CPU implementation would use the GQA
 * structure. Online softmax (running max, rescaled sum) in fp32. */
static void gqa_task(void *ctx, size_t task) {
  gqa_job *j = (gqa_job *)ctx;
  uint32_t d = j->d, group = j->Hq / j->Hkv;
  uint32_t split = (uint32_t)(task % j->splits);
  size_t tk = task / j->splits;
  uint32_t kvh = (uint32_t)(tk % j->Hkv), t = (uint32_t)(tk / j->Hkv);
  uint32_t visible = j->P + t + 1;
  uint32_t per = (visible + j->splits - 1) / j->splits;
  uint32_t begin = split * per, end = begin + per;
  if (end > visible)
    end = visible;
  size_t kv_stride = (size_t)j->Hkv * d;
  float scale = 1.0f / sqrtf((float)d);
  float *qf = (float *)malloc(sizeof(float) * (size_t)d * (group + 2));
  float *row = qf + (size_t)d * group;
  float *part = j->partial + task * (size_t)group * (d + 2);
  for (uint32_t g = 0; g < group; ++g) {
    cvt_row(j->q + ((size_t)t * j->Hq + kvh * group + g) * d, qf + (size_t)g * d, d);
    float *o = part + (size_t)g * (d + 2);
    for (uint32_t x = 0; x < d; ++x)
      o[x] = 0.0f;
    o[d] = -INFINITY;
    o[d + 1] = 0.0f;
  }
  float sc[64];
  for (uint32_t key = begin; key < end; ++key) {
    cvt_row(j->k + (size_t)key * kv_stride + (size_t)kvh * d, row, d);
    for (uint32_t g = 0; g < group; ++g) {
      const float *qg = qf + (size_t)g * d;
      float dot = 0.0f;
      for (uint32_t x = 0; x < d; ++x)
        dot += qg[x] * row[x];
      sc[g] = dot * scale;
    }
    cvt_row(j->v + (size_t)key * kv_stride + (size_t)kvh * d, row, d);
    for (uint32_t g = 0; g < group; ++g) {
      float *o = part + (size_t)g * (d + 2);
      float m = o[d], s = sc[g];
      if (s > m) {
        float r = expf(m - s);
        for (uint32_t x = 0; x < d; ++x)
          o[x] = o[x] * r + row[x];
        o[d + 1] = o[d + 1] * r + 1.0f;
        o[d] = s;
      } else {
        float p = expf(s - m);
        for (uint32_t x = 0; x < d; ++x)
          o[x] += p * row[x];
        o[d + 1] += p;
      }
    }
  }
  free(qf);
}

void orc_gqa_f32(const uint16_t *q, const uint16_t *k_cache,
                 const uint16_t *v_cache, uint16_t *out, uint32_t T,
                 uint32_t Hq, uint32_t Hkv, uint32_t d, uint32_t P,
                 int threads) {
  if (threads <= 0)
    threads = orc_cpu_count();
  uint32_t group = Hq / Hkv;
  if (group > 64)
    return;
  size_t rows = (size_t)T * Hkv;
  uint32_t splits = 1;
  while (rows * splits < (size_t)threads * 4 && splits < 64 &&
         (P + 1) / (splits * 2) >= 64)
    splits *= 2;
  gqa_job job = {q, k_cache, v_cache, out, T, Hq, Hkv, d, P, splits, NULL};
  job.partial = (float *)malloc(sizeof(float) * rows * splits * group * (d + 2));
  parallel_for(rows * splits, threads, gqa_task, &job);
  /* Combine the key splits of each (token, kv head, q-head). */
  for (size_t tk = 0; tk < rows; ++tk) {
    uint32_t kvh = (uint32_t)(tk % Hkv), t = (uint32_t)(tk / Hkv);
    for (uint32_t g = 0; g < group; ++g) {
      float m = -INFINITY;
      for (uint32_t s = 0; s < splits; ++s) {
        const float *o = job.partial + ((tk * splits + s) * group + g) * (d + 2);
        if (o[d] > m)
          m = o[d];
      }
      float l = 0.0f;
      for (uint32_t s = 0; s < splits; ++s) {
        const float *o = job.partial + ((tk * splits + s) * group + g) * (d + 2);
        if (o[d] != -INFINITY)
          l += o[d + 1] * expf(o[d] - m);
      }
      uint16_t *dst = out + ((size_t)t * Hq + kvh * group + g) * d;
      for (uint32_t x = 0; x < d; ++x) {
        float acc = 0.0f;
        for (uint32_t s = 0; s < splits; ++s) {
          const float *o = job.partial + ((tk * splits + s) * group + g) * (d + 2);
          if (o[d] == -INFINITY)
            continue;
          acc += o[x] * expf(o[d] - m);
        }
        dst[x] = orc_f32_to_f16(acc / l);
      }
    }
  }
  free(job.partial);
}

void orc_kv_append(const uint16_t *src, uint16_t *cache, uint32_t T,
                   uint32_t Hkv, uint32_t d, uint32_t P) {
  size_t count = (size_t)T * Hkv * d;
  memcpy(cache + (size_t)P * Hkv * d, src, count * sizeof(uint16_t));
}

/* -------------------------------------------------------------- DeltaNet */

void orc_delta_recurrent_f64(const float *q, const float *k, const uint16_t *v,
                             const float *beta, const float *decay,
                             const float *state_in, double *state_out,
                             double *out, uint32_t T, uint32_t Hk, uint32_t dk,
                             uint32_t Hv, uint32_t dv) {
  size_t per_head = (size_t)dk * dv;
  uint32_t ratio = Hv / Hk;
  size_t vwidth = (size_t)Hv * dv;
  double *s = state_out;
  for (size_t i = 0; i < (size_t)Hv * per_head; ++i)
    s[i] = (double)state_in[i];
  for (uint32_t h = 0; h < Hv; ++h) {
    uint32_t kh = h / ratio;
    double *S = s + (size_t)h * per_head;
    for (uint32_t t = 0; t < T; ++t) {
      const float *qt = q + ((size_t)t * Hk + kh) * dk;
      const float *kt = k + ((size_t)t * Hk + kh) * dk;
      double b = beta[(size_t)t * Hv + h], a = decay[(size_t)t * Hv + h];
      for (uint32_t c = 0; c < dv; ++c) {
        double pred = 0.0;
        for (uint32_t i = 0; i < dk; ++i)
          pred += S[(size_t)i * dv + c] * a * (double)kt[i];
        double vj = orc_f16_to_f32(v[(size_t)t * vwidth + (size_t)h * dv + c]);
        double delta = (vj - pred) * b;
        double y = 0.0;
        for (uint32_t i = 0; i < dk; ++i) {
          double next = S[(size_t)i * dv + c] * a + (double)kt[i] * delta;
          S[(size_t)i * dv + c] = next;
          y += next * (double)qt[i];
        }
        if (out)
          out[(size_t)t * vwidth + (size_t)h * dv + c] = y;
      }
    }
  }
}

typedef struct {
  const float *q, *k, *beta, *decay;
  const uint16_t *v;
  float *state;
  uint16_t *out;
  uint32_t T, Hk, dk, Hv, dv, cols_per_task;
} delta_job;

/* updateDeltaColumn (Reference.metal:182-197) per column, fma order kept. */
static void delta_task(void *ctx, size_t task) {
  delta_job *j = (delta_job *)ctx;
  uint32_t dk = j->dk, dv = j->dv;
  size_t vwidth = (size_t)j->Hv * dv;
  size_t first = task * j->cols_per_task;
  for (size_t col = first; col < first + j->cols_per_task && col < vwidth; ++col) {
    uint32_t h = (uint32_t)(col / dv), c = (uint32_t)(col % dv);
    uint32_t kh = h / (j->Hv / j->Hk);
    float *S = j->state + (size_t)h * dk * dv + c;
    for (uint32_t t = 0; t < j->T; ++t) {
      const float *qt = j->q + ((size_t)t * j->Hk + kh) * dk;
      const float *kt = j->k + ((size_t)t * j->Hk + kh) * dk;
      float b = j->beta[(size_t)t * j->Hv + h];
      float a = j->decay[(size_t)t * j->Hv + h];
      float pred = 0.0f;
      for (uint32_t i = 0; i < dk; ++i)
        pred = fmaf(S[(size_t)i * dv] * a, kt[i], pred);
      float vj = orc_f16_to_f32(j->v[(size_t)t * vwidth + col]);
      float delta = (vj - pred) * b;
      float y = 0.0f;
      for (uint32_t i = 0; i < dk; ++i) {
        float next = fmaf(kt[i], delta, S[(size_t)i * dv] * a);
        S[(size_t)i * dv] = next;
        y = fmaf(next, qt[i], y);
      }
      j->out[(size_t)t * vwidth + col] = orc_f32_to_f16(y);
    }
  }
}

void orc_delta_recurrent_f32(const float *q, const float *k, const uint16_t *v,
                             const float *beta, const float *decay,
                             float *state, uint16_t *out, uint32_t T,
                             uint32_t Hk, uint32_t dk, uint32_t Hv, uint32_t dv,
                             int threads) {
  size_t cols = (size_t)Hv * dv;
  delta_job job = {q, k, beta, decay, v, state, out, T, Hk, dk, Hv, dv, 8};
  parallel_for((cols + job.cols_per_task - 1) / job.cols_per_task, threads,
               delta_task, &job);
}

void orc_delta_chunked_f64(const float *q, const float *k, const uint16_t *v,
                           const float *beta, const float *decay,
                           const float *state_in, double *state_out,
                           double *out, uint32_t T, uint32_t Hk, uint32_t dk,
                           uint32_t Hv, uint32_t dv, uint32_t chunk) {
  size_t per_head = (size_t)dk * dv;
  uint32_t ratio = Hv / Hk;
  size_t vwidth = (size_t)Hv * dv;
  uint32_t C = chunk ? chunk : 64;
  for (size_t i = 0; i < (size_t)Hv * per_head; ++i)
    state_out[i] = (double)state_in[i];
  double *g = (double *)malloc(sizeof(double) * C);
  double *A = (double *)malloc(sizeof(double) * C * C);   /* then Tm */
  double *W = (double *)malloc(sizeof(double) * C * dk);
  double *U = (double *)malloc(sizeof(double) * C * dv);
  double *Y = (double *)malloc(sizeof(double) * C * dv);
  for (uint32_t h = 0; h < Hv; ++h) {
    uint32_t kh = h / ratio;
    double *S = state_out + (size_t)h * per_head;
    for (uint32_t t0 = 0; t0 < T; t0 += C) {
      uint32_t n = T - t0 < C ? T - t0 : C;
#define KQ(arr, t, i) ((double)(arr)[((size_t)(t0 + (t)) * Hk + kh) * dk + (i)])
#define BETA(t) ((double)beta[(size_t)(t0 + (t)) * Hv + h])
#define VV(t, c) ((double)orc_f16_to_f32(v[(size_t)(t0 + (t)) * vwidth + (size_t)h * dv + (c)]))
      /* Cumulative log decay. log(0) = -inf is clamped so that differences
       * of equal prefixes stay finite; exp of the clamp is 0 in double. */
      double acc = 0.0;
      for (uint32_t t = 0; t < n; ++t) {
        double a = decay[(size_t)(t0 + t) * Hv + h];
        acc += a > 0.0 ? log(a) : -1.0e4;
        g[t] = acc;
      }
      /* A (strictly lower): beta_t exp(g_t - g_s) k_t.k_s. */
      for (uint32_t t = 0; t < n; ++t)
        for (uint32_t s = 0; s < n; ++s) {
          double val = 0.0;
          if (s < t) {
            double dot = 0.0;
            for (uint32_t i = 0; i < dk; ++i)
              dot += KQ(k, t, i) * KQ(k, s, i);
            val = BETA(t) * exp(g[t] - g[s]) * dot;
          }
          A[(size_t)t * C + s] = val;
        }
      /* Forward substitution: rows of W and U' solve (I + A) X = RHS. */
      for (uint32_t t = 0; t < n; ++t) {
        double bg = BETA(t) * exp(g[t]);
        for (uint32_t i = 0; i < dk; ++i) {
          double x = bg * KQ(k, t, i);
          for (uint32_t s = 0; s < t; ++s)
            x -= A[(size_t)t * C + s] * W[(size_t)s * dk + i];
          W[(size_t)t * dk + i] = x;
        }
        for (uint32_t c = 0; c < dv; ++c) {
          double x = BETA(t) * VV(t, c);
          for (uint32_t s = 0; s < t; ++s)
            x -= A[(size_t)t * C + s] * U[(size_t)s * dv + c];
          U[(size_t)t * dv + c] = x;
        }
      }
      /* U = U' - W S. */
      for (uint32_t t = 0; t < n; ++t)
        for (uint32_t c = 0; c < dv; ++c) {
          double x = 0.0;
          for (uint32_t i = 0; i < dk; ++i)
            x += W[(size_t)t * dk + i] * S[(size_t)i * dv + c];
          U[(size_t)t * dv + c] -= x;
        }
      /* Y = diag(exp g) Q S + M U. */
      for (uint32_t t = 0; t < n; ++t) {
        double eg = exp(g[t]);
        for (uint32_t c = 0; c < dv; ++c) {
          double x = 0.0;
          for (uint32_t i = 0; i < dk; ++i)
            x += KQ(q, t, i) * S[(size_t)i * dv + c];
          Y[(size_t)t * dv + c] = eg * x;
        }
        for (uint32_t s = 0; s <= t; ++s) {
          double dot = 0.0;
          for (uint32_t i = 0; i < dk; ++i)
            dot += KQ(q, t, i) * KQ(k, s, i);
          double m = exp(g[t] - g[s]) * dot;
          for (uint32_t c = 0; c < dv; ++c)
            Y[(size_t)t * dv + c] += m * U[(size_t)s * dv + c];
        }
        if (out)
          for (uint32_t c = 0; c < dv; ++c)
            out[(size_t)(t0 + t) * vwidth + (size_t)h * dv + c] =
                Y[(size_t)t * dv + c];
      }
      /* S = exp(g_C) S + K^T diag(exp(g_C - g)) U. */
      double gl = g[n - 1], el = exp(gl);
      for (uint32_t i = 0; i < dk; ++i)
        for (uint32_t c = 0; c < dv; ++c) {
          double x = el * S[(size_t)i * dv + c];
          for (uint32_t s = 0; s < n; ++s)
            x += KQ(k, s, i) * exp(gl - g[s]) * U[(size_t)s * dv + c];
          S[(size_t)i * dv + c] = x;
        }
#undef KQ
#undef BETA
#undef VV
    }
  }
  free(g);
  free(A);
  free(W);
  free(U);
  free(Y);
}

/* Reference.metal:4-12. */
/* The fp32 pow/cos/sin/exp/log of the reference kernels, taken correctly
 * rounded: evaluated in double and rounded to float once. The device kernels
 * produce the same float (a fast fp32 evaluation with a margin test, else the
 * same double evaluation), so results compare bit for bit. */
static float orc_powf_cr(float x, float y) { return (float)pow((double)x, (double)y); }
static float orc_cosf_cr(float x) { return (float)cos((double)x); }
static float orc_sinf_cr(float x) { return (float)sin((double)x); }
static float orc_expf_cr(float x) { return (float)exp((double)x); }
static float orc_logf_cr(float x) { return (float)log((double)x); }

/* logistic and stableSoftplus, Reference.metal:4, 8-12. */
static float logistic(float x) { return 1.0f / (1.0f + orc_expf_cr(-x)); }
static float stable_softplus(float x) {
  float e = orc_expf_cr(-fabsf(x));
  float tail = e < 1e-4f ? e * (1.0f - 0.5f * e) : orc_logf_cr(1.0f + e);
  return (x > 0.0f ? x : 0.0f) + tail;
}

void orc_delta_gates(const uint16_t *a, const uint16_t *b, const float *a_log,
                     const float *dt_bias, float *beta, float *decay,
                     uint32_t T, uint32_t Hv) {
  for (size_t i = 0; i < (size_t)T * Hv; ++i) {
    uint32_t h = (uint32_t)(i % Hv);
    beta[i] = round_f16(logistic(orc_f16_to_f32(b[i])));
    decay[i] = orc_expf_cr(-orc_expf_cr(a_log[h]) *
                           stable_softplus(orc_f16_to_f32(a[i]) + dt_bias[h]));
  }
}

void orc_l2norm_f32(const uint16_t *in, float *out, uint32_t rows,
                    uint32_t width, float eps, float scale) {
  for (uint32_t r = 0; r < rows; ++r) {
    const uint16_t *x = in + (size_t)r * width;
    float sum = 0.0f;
    for (uint32_t i = 0; i < width; ++i) {
      float f = orc_f16_to_f32(x[i]);
      sum = fmaf(f, f, sum);
    }
    float factor = (1.0f / sqrtf(sum + eps)) * scale;
    for (uint32_t i = 0; i < width; ++i)
      out[(size_t)r * width + i] = orc_f16_to_f32(x[i]) * factor;
  }
}

/* causalConv, Reference.metal:137-161 (ConvParams, ReferenceParams.h:32-34):
 * per channel, acc = x_t * w[k-1] + sum_j history_j * w[j] (fma in j order),
 * output fp16(acc) or fp16(silu(fp16(acc))), then the k-1 history slots shift
 * left and take x_t. Layout: input/output [tokens][channels], weight
 * [channels][k], history [channels][k-1], all fp16; history updated in place. */
void orc_causal_conv(const uint16_t *input, const uint16_t *weight, uint16_t *history,
                     uint16_t *output, uint32_t tokens, uint32_t channels,
                     uint32_t kernel_size, uint32_t apply_silu) {
  uint32_t hs = kernel_size - 1;
  for (uint32_t c = 0; c < channels; ++c) {
    uint16_t *recent = history + (size_t)c * hs;
    const uint16_t *filter = weight + (size_t)c * kernel_size;
    for (uint32_t t = 0; t < tokens; ++t) {
      size_t i = (size_t)t * channels + c;
      uint16_t current = input[i];
      float acc = orc_f16_to_f32(current) * orc_f16_to_f32(filter[hs]);
      for (uint32_t j = 0; j < hs; ++j)
        acc = fmaf(orc_f16_to_f32(recent[j]), orc_f16_to_f32(filter[j]), acc);
      if (apply_silu) {
        float h = round_f16(acc);
        output[i] = orc_f32_to_f16(h * logistic(h));
      } else {
        output[i] = orc_f32_to_f16(acc);
      }
      for (uint32_t j = 1; j < hs; ++j)
        recent[j - 1] = recent[j];
      if (hs)
        recent[hs - 1] = current;
    }
  }
}

/* ---------------------------------------------------- norm, rope, gate */

static float orc_round_f16(float x) { return orc_f16_to_f32(orc_f32_to_f16(x)); }

/* rmsScale, Reference.metal:98-103: fma-accumulated sum of squares in index
 * order, rsqrt(sum / width + eps). */
static float orc_rms_scale(const uint16_t *x, uint32_t width, float eps) {
  float sum = 0.0f;
  for (uint32_t i = 0; i < width; ++i) {
    float f = orc_f16_to_f32(x[i]);
    sum = fmaf(f, f, sum);
  }
  return 1.0f / sqrtf(sum / (float)width + eps);
}


/* rotatePair, Reference.metal:262-269. */
static void orc_rotate_pair(float in_x, float in_y, float position, float theta,
                            uint32_t pair, uint32_t rotary_width, uint16_t *out_x,
                            uint16_t *out_y) {
  float phase = position / orc_powf_cr(theta, 2.0f * (float)pair / (float)rotary_width);
  float cosine = orc_round_f16(orc_cosf_cr(phase));
  float sine = orc_round_f16(orc_sinf_cr(phase));
  *out_x = orc_f32_to_f16(orc_round_f16(in_x * cosine) - orc_round_f16(in_y * sine));
  *out_y = orc_f32_to_f16(orc_round_f16(in_y * cosine) + orc_round_f16(in_x * sine));
}

/* normRope, Reference.metal:271-293. */
void orc_norm_rope(const uint16_t *input, const float *weight, uint16_t *output,
                   uint32_t tokens, uint32_t heads, uint32_t head_dim,
                   uint32_t rotary_dim, uint32_t head_stride, uint32_t past,
                   uint32_t output_start, float epsilon, float theta) {
  uint32_t rows = tokens * heads, half = rotary_dim / 2;
  for (uint32_t row = 0; row < rows; ++row) {
    const uint16_t *head = input + (size_t)row * head_stride;
    uint16_t *out = output + ((size_t)output_start * heads + row) * head_dim;
    float scale = orc_rms_scale(head, head_dim, epsilon);
    float position = (float)(past + row / heads);
    for (uint32_t i = 0; i < half; ++i) {
      uint32_t j = i + half;
      float x = orc_round_f16(orc_f16_to_f32(head[i]) * scale * (1.0f + weight[i]));
      float y = orc_round_f16(orc_f16_to_f32(head[j]) * scale * (1.0f + weight[j]));
      orc_rotate_pair(x, y, position, theta, i, rotary_dim, &out[i], &out[j]);
    }
    for (uint32_t i = rotary_dim; i < head_dim; ++i)
      out[i] = orc_f32_to_f16(orc_f16_to_f32(head[i]) * scale * (1.0f + weight[i]));
  }
}

/* partialRope, Graph.metal:111-129: rotatePair on the raw fp16 halves of
 * the first rotary_dim dims at position past + row / heads, the rest copied. */
void orc_partial_rope(const uint16_t *input, uint16_t *output, uint32_t rows, uint32_t heads,
                      uint32_t width, uint32_t rotary_dim, uint32_t past, float theta) {
  uint32_t half = rotary_dim / 2;
  for (uint32_t row = 0; row < rows; ++row) {
    const uint16_t *in = input + (size_t)row * width;
    uint16_t *out = output + (size_t)row * width;
    float position = (float)(past + row / heads);
    for (uint32_t i = 0; i < half; ++i)
      orc_rotate_pair(orc_f16_to_f32(in[i]), orc_f16_to_f32(in[i + half]), position, theta, i,
                      rotary_dim, &out[i], &out[i + half]);
    for (uint32_t i = rotary_dim; i < width; ++i)
      out[i] = in[i];
  }
}

/* gatedRmsNorm / gatedRmsNormActivated, Reference.metal:228-259:
 * out = fp16(fp16(x * rmsScale) * w[i] * g), g = silu(gate) for an fp16
 * gate, the fp32 gate itself when activated. */
void orc_gated_rms_norm(const uint16_t *input, const uint16_t *gate16, const float *gate32,
                        const float *weight, uint16_t *output, uint32_t rows, uint32_t width,
                        float eps) {
  for (uint32_t r = 0; r < rows; ++r) {
    size_t off = (size_t)r * width;
    float scale = orc_rms_scale(input + off, width, eps);
    for (uint32_t i = 0; i < width; ++i) {
      float norm = orc_round_f16(orc_f16_to_f32(input[off + i]) * scale) * weight[i];
      float value = gate32 ? gate32[off + i] : orc_f16_to_f32(gate16[off + i]);
      float g = gate32 ? value : value * logistic(value);
      output[off + i] = orc_f32_to_f16(norm * g);
    }
  }
}

/* sigmoidMul, Graph.metal:78-85 with logistic, Reference.metal:4. */
void orc_sigmoid_mul(const uint16_t *gate, const uint16_t *input, uint16_t *output,
                     size_t count) {
  for (size_t i = 0; i < count; ++i) {
    float g = orc_round_f16(1.0f / (1.0f + orc_expf_cr(-orc_f16_to_f32(gate[i]))));
    output[i] = orc_f32_to_f16(g * orc_f16_to_f32(input[i]));
  }
}

/* ------------------------------------------------------------- W8A8 path */

/* silu, Reference.metal:6 (x * logistic(x), each step rounded to fp32). */
static float silu(float x) { return x * logistic(x); }

/* quantizeActivation, Graph.metal:33-68: per row and 32-wide group, scale =
 * max|x| / 127 (1 for an all-zero or non-finite group), q = x / scale
 * clamped to [-127, 127] and rounded half to even; a non-finite group sets
 * *invalid and quantizes to zeros. Output rows are groups * 32 wide. */
void orc_quantize_activation(const uint16_t *input, int8_t *quantized, float *scales,
                             uint32_t *invalid, uint32_t rows, uint32_t width,
                             uint32_t groups) {
  for (size_t i = 0; i < (size_t)rows * groups; ++i) {
    uint32_t row = (uint32_t)(i / groups), begin = (uint32_t)(i % groups) * 32u;
    uint32_t length = width - begin < 32u ? width - begin : 32u;
    const uint16_t *group = input + (size_t)row * width + begin;
    float max_abs = 0.0f;
    int finite = 1;
    for (uint32_t j = 0; j < length; ++j) {
      float value = orc_f16_to_f32(group[j]);
      finite = finite && isfinite(value);
      max_abs = fmaxf(max_abs, fabsf(value));
    }
    if (!finite)
      *invalid |= 1u;
    float scale = finite && max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
    scales[i] = scale;
    for (uint32_t j = 0; j < 32; ++j) {
      int rounded = 0;
      if (finite && j < length) {
        float x = orc_f16_to_f32(group[j]) / scale;
        x = x < -127.0f ? -127.0f : (x > 127.0f ? 127.0f : x);
        float lower = floorf(x);
        float fraction = x - lower;
        rounded = (int)lower;
        if (fraction > 0.5f || (fraction == 0.5f && (rounded % 2 != 0)))
          ++rounded;
      }
      quantized[i * 32 + j] = (int8_t)rounded;
    }
  }
}

/* storeLinear, Reference.metal:14-47: the projection rounded to fp16, then
 * the fused epilogue of the consumer. */
static void store_linear(void *output, const void *aux, const float *bias, size_t i,
                         uint32_t col, uint32_t epilogue, uint32_t block,
                         float accumulator) {
  float projected = orc_round_f16(accumulator);
  switch (epilogue) {
  case ORC_LINEAR_SILU:
    projected = orc_round_f16(silu(projected));
    break;
  case ORC_LINEAR_SILU_MUL:
    projected = orc_round_f16(orc_round_f16(silu(projected)) *
                              orc_f16_to_f32(((const uint16_t *)aux)[i]));
    break;
  case ORC_LINEAR_SIGMOID_COLUMNS:
    if ((col / block) % 2 != 0)
      projected = orc_round_f16(logistic(projected));
    break;
  case ORC_LINEAR_SILU_F32:
    ((float *)output)[i] = silu(projected);
    return;
  case ORC_LINEAR_DELTA_BETA:
    ((float *)output)[i] = orc_round_f16(logistic(projected));
    return;
  case ORC_LINEAR_DELTA_DECAY: {
    const float *a_log = (const float *)aux;
    ((float *)output)[i] =
        orc_expf_cr(-orc_expf_cr(a_log[col]) * stable_softplus(projected + bias[col]));
    return;
  }
  default:
    break;
  }
  ((uint16_t *)output)[i] = orc_f32_to_f16(projected);
}

/* linearW8A8Gemv / linearW8A8Gemm, W8A8.metal:28-113 (dispatch by rows,
 * LinearW8Launch.h:14-21): per output (row, column), lane l of the column's
 * `lanes` lanes (16 for one row, else 8, GraphParams.h:17-23) sums in fp32,
 * over groups g = l, l + lanes, ..., the exact int32 dot of the 32 int8
 * activations and weights of group g times the activation scale times the
 * weight scale, in that order; the lanes then combine by the xor butterfly
 * (acc += shuffle_xor(acc, m), m = lanes / 2 ... 1) and lane 0 stores
 * through storeLinear at row * outputWidth + firstRow + column. */
void orc_linear_w8a8(const int8_t *act, const float *act_scales, const int8_t *weight,
                     const uint16_t *weight_scales, void *output, const void *aux,
                     const float *bias, uint32_t output_width, uint32_t first_row,
                     uint32_t groups, uint32_t rows, uint32_t columns, uint32_t epilogue,
                     uint32_t epilogue_block) {
  const uint32_t lanes = rows == 1 ? 16u : 8u;
  float acc[16];
  for (uint32_t row = 0; row < rows; ++row)
    for (uint32_t col = 0; col < columns; ++col) {
      for (uint32_t l = 0; l < lanes; ++l) {
        float a = 0.0f;
        for (uint32_t g = l; g < groups; g += lanes) {
          const int8_t *x = act + ((size_t)row * groups + g) * 32;
          const int8_t *w = weight + ((size_t)col * groups + g) * 32;
          int32_t dot = 0;
          for (int j = 0; j < 32; ++j)
            dot += (int32_t)x[j] * (int32_t)w[j];
          float term = (float)dot * act_scales[(size_t)row * groups + g];
          term = term * orc_f16_to_f32(weight_scales[(size_t)col * groups + g]);
          a = a + term;
        }
        acc[l] = a;
      }
      for (uint32_t m = lanes / 2; m != 0; m >>= 1) {
        float next[16];
        for (uint32_t l = 0; l < lanes; ++l)
          next[l] = acc[l] + acc[l ^ m];
        memcpy(acc, next, sizeof(float) * lanes);
      }
      uint32_t column = first_row + col;
      store_linear(output, aux, bias, (size_t)row * output_width + column, column, epilogue,
                   epilogue_block, acc[0]);
    }
}

/* embeddingW8, Graph.metal:16-31: out[t][c] = fp16(w[row][c] * scale[row][c /
 * 32]) for token ids in [firstRow, firstRow + rowCount), rows `groups * 32`
 * int8 wide; other ids leave the output row untouched. */
void orc_embedding_w8(const uint32_t *ids, const int8_t *weight, const uint16_t *scales,
                      uint16_t *output, uint32_t tokens, uint32_t hidden, uint32_t first_row,
                      uint32_t row_count, uint32_t groups) {
  for (size_t i = 0; i < (size_t)tokens * hidden; ++i) {
    uint32_t id = ids[i / hidden];
    if (id < first_row || id - first_row >= row_count)
      continue;
    size_t row = id - first_row;
    uint32_t col = (uint32_t)(i % hidden);
    output[i] = orc_f32_to_f16((float)weight[row * groups * 32 + col] *
                               orc_f16_to_f32(scales[row * groups + col / 32]));
  }
}

/* embedding, Reference.metal:49-58: fp16 rows copied for ids in range. */
void orc_embedding(const uint32_t *ids, const uint16_t *weight, uint16_t *output,
                   uint32_t tokens, uint32_t hidden, uint32_t first_row, uint32_t row_count) {
  for (size_t i = 0; i < (size_t)tokens * hidden; ++i) {
    uint32_t id = ids[i / hidden];
    if (id >= first_row && id - first_row < row_count)
      output[i] = weight[(size_t)(id - first_row) * hidden + i % hidden];
  }
}

/* ----------------------------------------- elementwise, views, linearF16 */

/* residualAdd, swiGlu, siluF16, multiplyF16 (Reference.metal:119-135,
 * Graph.metal:70-95): kind 0..3 in that order; b is unused by siluF16. */
void orc_elementwise(uint32_t kind, const uint16_t *a, const uint16_t *b, uint16_t *out,
                     size_t count) {
  for (size_t i = 0; i < count; ++i) {
    float x = orc_f16_to_f32(a[i]);
    float r;
    switch (kind) {
    case 0:
      r = x + orc_f16_to_f32(b[i]);
      break;
    case 1:
      r = orc_round_f16(silu(x)) * orc_f16_to_f32(b[i]);
      break;
    case 2:
      r = silu(x);
      break;
    default:
      r = x * orc_f16_to_f32(b[i]);
      break;
    }
    out[i] = orc_f32_to_f16(r);
  }
}

/* copyHalfView, Graph.metal:1-14: out[i] = src[offset + sum_d index_d(i) *
 * strides[d]] over dims (outermost first). */
void orc_copy_half_view(const uint16_t *src, uint16_t *out, uint32_t count, uint32_t offset,
                        const uint32_t *dims, const uint32_t *strides) {
  for (uint32_t i = 0; i < count; ++i) {
    uint32_t rest = i, at = offset;
    for (int d = 2; d >= 0; --d) {
      at += (rest % dims[d]) * strides[d];
      rest /= dims[d];
    }
    out[i] = src[at];
  }
}

/* linearF16, Reference.metal:61-103: per output (row, col), acc = fma(x[k],
 * w[k], acc) over k = 0 .. inputWidth-1 in fp32, then storeLinear. */
void orc_linear_f16(const uint16_t *input, const uint16_t *weight, void *output,
                    const void *aux, const float *bias, uint32_t tokens, uint32_t input_width,
                    uint32_t output_width, uint32_t first_row, uint32_t columns,
                    uint32_t epilogue, uint32_t epilogue_block) {
  for (uint32_t row = 0; row < tokens; ++row)
    for (uint32_t col = 0; col < columns; ++col) {
      float acc = 0.0f;
      for (uint32_t k = 0; k < input_width; ++k)
        acc = fmaf(orc_f16_to_f32(input[(size_t)row * input_width + k]),
                   orc_f16_to_f32(weight[(size_t)col * input_width + k]), acc);
      uint32_t column = first_row + col;
      store_linear(output, aux, bias, (size_t)row * output_width + column, column, epilogue,
                   epilogue_block, acc);
    }
}

/* ------------------------------------------------------------------ cost */

static int mul_ok(uint64_t a, uint64_t b, uint64_t *r) {
  if (a != 0 && b > UINT64_MAX / a)
    return 0;
  *r = a * b;
  return 1;
}
static int add_ok(uint64_t a, uint64_t b, uint64_t *r) {
  if (b > UINT64_MAX - a)
    return 0;
  *r = a + b;
  return 1;
}
static int mul3(uint64_t a, uint64_t b, uint64_t c, uint64_t *r) {
  uint64_t t;
  return mul_ok(a, b, &t) && mul_ok(t, c, r);
}

/* Cost.cpp:56-94 for KvAppend: reads k and v, writes T rows of each cache. */
int orc_cost_kv_append(uint64_t T, uint64_t Hkv, uint64_t d, orc_cost *c) {
  memset(c, 0, sizeof *c);
  uint64_t one;
  if (!mul3(T, Hkv, d, &one) || !mul_ok(one, 2, &one))
    return -1;
  if (!add_ok(one, one, &c->read_bytes) || !add_ok(one, one, &c->write_bytes))
    return -1;
  return 0;
}

/* Cost.cpp:188-201 (math) and :56-94 (traffic) for CausalGqa. */
int orc_cost_causal_gqa(uint64_t T, uint64_t P, uint64_t Hq, uint64_t Hkv,
                        uint64_t d, orc_cost *c) {
  memset(c, 0, sizeof *c);
  uint64_t pairs, tri, scores, macs, qbytes, kv, two;
  if (!mul_ok(T, P, &pairs))
    return -1;
  if (T % 2) {
    if (!mul_ok(T, T / 2 + 1, &tri))
      return -1;
  } else if (!mul_ok(T / 2, T + 1, &tri))
    return -1;
  if (!add_ok(pairs, tri, &pairs) || !mul_ok(Hq, pairs, &scores) ||
      !mul3(2, scores, d, &macs))
    return -1;
  c->fp_macs = macs;
  if (!mul_ok(5, scores, &c->scalar_ops))
    return -1;
  c->exp = scores;
  if (!mul3(T, Hq, d, &qbytes) || !mul_ok(qbytes, 2, &qbytes))
    return -1;
  uint64_t rows;
  if (!add_ok(P, T, &rows) || !mul3(rows, Hkv, d, &kv) ||
      !mul_ok(kv, 2, &kv) || !add_ok(kv, kv, &two))
    return -1;
  if (!add_ok(qbytes, two, &c->read_bytes))
    return -1;
  c->write_bytes = qbytes;
  return 0;
}

/* Cost.cpp:180-187 (math) and :56-94 (traffic) for DeltaUpdate. */
int orc_cost_delta_update(uint64_t T, uint64_t Hk, uint64_t dk, uint64_t Hv,
                          uint64_t dv, orc_cost *c) {
  memset(c, 0, sizeof *c);
  uint64_t state, macs, qk, vbytes, gates, sbytes, tmp, outs;
  if (!mul3(Hv, dk, dv, &state) || !mul3(3, T, state, &macs))
    return -1;
  c->fp_macs = macs;
  if (!mul_ok(T, state, &tmp) || !mul3(T, Hv, dv, &outs) ||
      !mul_ok(outs, 2, &outs) || !add_ok(tmp, outs, &c->scalar_ops))
    return -1;
  if (!mul3(T, Hk, dk, &qk) || !mul_ok(qk, 8, &qk)) /* q and k, fp32 */
    return -1;
  if (!mul3(T, Hv, dv, &vbytes) || !mul_ok(vbytes, 2, &vbytes))
    return -1;
  if (!mul3(T, Hv, 8, &gates)) /* beta and decay, fp32 */
    return -1;
  if (!mul_ok(state, 4, &sbytes))
    return -1;
  if (!add_ok(qk, vbytes, &tmp) || !add_ok(tmp, gates, &tmp) ||
      !add_ok(tmp, sbytes, &c->read_bytes))
    return -1;
  if (!add_ok(vbytes, sbytes, &c->write_bytes))
    return -1;
  return 0;
}
