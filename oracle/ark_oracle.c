/*
 * ark_oracle.c -- TEST INFRASTRUCTURE ONLY: the CPU parity checker for the
 * MI355X optimizer step.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it; the product library never does.
 *
 * Build: -O2 -ffp-contract=off (no implicit fused multiply-add), -mfma so
 * fmaf() is the single-rounding instruction, no -ffast-math.  Every fp32 op
 * below is one IEEE binary32 operation with one rounding, exactly as the NEON
 * instructions of opti.s it restates.
 *
 * Reference paths are relative to proyecto_ark/ark01/.
 */
#include "ark_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#if defined(__F16C__)
#include <immintrin.h>
#endif

static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* ------------------------------------------------------------------------ */
/* fp16 <-> fp32.  The reference converts with fcvtl/fcvt (exact widening,   */
/* opti.s:279, :318) and fcvtn/fcvt (opti.s:307, :345) under the default     */
/* FPCR: round to nearest even, fp16 subnormals kept, overflow to infinity.  */
/* ------------------------------------------------------------------------ */

float ark_ref_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t mant = h & 0x3FFu;
  if (exp == 0x1Fu) {
    if (mant == 0) return u2f(sign | 0x7F800000u);
    return u2f(sign | 0x7FC00000u | (mant << 13)); /* NaN, quieted */
  }
  if (exp != 0) return u2f(sign | ((exp + 112u) << 23) | (mant << 13));
  /* zero or subnormal: mant * 2^-24, exact in fp32 */
  float mag = (float)mant * 5.9604644775390625e-08f;
  return sign ? -mag : mag;
}

uint16_t ark_ref_f32_to_f16(float f) {
  uint32_t x = f2u(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) {
    if (ax == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu)); /* quiet NaN */
  }
  /* 65520 = halfway between 65504 (odd mantissa) and 2^16: ties to even
   * round it, and everything above, to infinity. */
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
  int32_t e = (int32_t)(ax >> 23) - 127;
  if (e >= -14) { /* normal fp16 */
    uint32_t mant = ax & 0x7FFFFFu;
    uint32_t h = ((uint32_t)(e + 15) << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* carry ok */
    return (uint16_t)(sign | h);
  }
  if ((ax >> 23) == 0) return (uint16_t)sign; /* fp32 subnormal: < 2^-126 */
  /* fp16 subnormal range: value = m * 2^(e-23), unit 2^-24 -> shift s */
  int32_t s = -(e + 1);
  if (s >= 25) return (uint16_t)sign; /* below half the smallest subnormal */
  uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
  uint32_t q = m >> s;
  uint32_t rem = m & ((1u << s) - 1u);
  uint32_t half = 1u << (s - 1);
  if (rem > half || (rem == half && (q & 1u))) q += 1u;
  return (uint16_t)(sign | q);
}

void ark_ref_f16_to_f32_array(const uint16_t *in, float *out, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) out[i] = ark_ref_f16_to_f32(in[i]);
}

void ark_ref_f32_to_f16_array(const float *in, uint16_t *out, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) out[i] = ark_ref_f32_to_f16(in[i]);
}

/* ------------------------------------------------------------------------ */
/* Small thread pool helper: run fn(ctx, tid, nthreads) on nthreads threads. */
/* ------------------------------------------------------------------------ */

typedef void (*par_fn)(void *ctx, int tid, int nth);
typedef struct {
  par_fn fn;
  void *ctx;
  int tid, nth;
} par_arg;

static void *par_tramp(void *p) {
  par_arg *a = (par_arg *)p;
  a->fn(a->ctx, a->tid, a->nth);
  return NULL;
}

static void run_parallel(int nth, par_fn fn, void *ctx) {
  if (nth <= 1) {
    fn(ctx, 0, 1);
    return;
  }
  pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nth);
  par_arg *args = (par_arg *)malloc(sizeof(par_arg) * (size_t)nth);
  int started = 0;
  for (int i = 1; i < nth; ++i) {
    args[i].fn = fn;
    args[i].ctx = ctx;
    args[i].tid = i;
    args[i].nth = nth;
    if (pthread_create(&th[i], NULL, par_tramp, &args[i]) != 0) break;
    started = i;
  }
  /* threads that failed to start are run inline, keeping results complete */
  for (int i = started + 1; i < nth; ++i) fn(ctx, i, nth);
  fn(ctx, 0, nth);
  for (int i = 1; i <= started; ++i) pthread_join(th[i], NULL);
  free(th);
  free(args);
}

static void split_range(uint64_t n, int tid, int nth, uint64_t *lo,
                        uint64_t *hi) {
  uint64_t q = n / (uint64_t)nth, r = n % (uint64_t)nth;
  uint64_t t = (uint64_t)tid;
  *lo = t * q + (t < r ? t : r);
  *hi = *lo + q + (t < r ? 1 : 0);
}

/* ------------------------------------------------------------------------ */
/* Exhaustive checks against F16C hardware conversion.                       */
/* ------------------------------------------------------------------------ */


int64_t ark_ref_check_f16_to_f32_f16c(void) {
#if defined(__F16C__)
  int64_t bad = 0;
  for (uint32_t h = 0; h < 65536u; ++h) {
    uint32_t a = f2u(ark_ref_f16_to_f32((uint16_t)h));
    uint32_t b = f2u(_cvtsh_ss((unsigned short)h));
    bad += (a != b); /* NaNs too: F16C quiets and keeps the payload like fcvtl */
  }
  return bad;
#else
  return -1;
#endif
}

typedef struct {
  uint64_t lo, hi;
  int64_t *bad;
} chk32_ctx;

static void chk32_worker(void *p, int tid, int nth) {
#if defined(__F16C__)
  chk32_ctx *c = (chk32_ctx *)p;
  uint64_t lo, hi;
  split_range(c->hi - c->lo, tid, nth, &lo, &hi);
  lo += c->lo;
  hi += c->lo;
  int64_t bad = 0;
  for (uint64_t i = lo; i < hi; ++i) {
    float f = u2f((uint32_t)i);
    uint16_t a = ark_ref_f32_to_f16(f);
    uint16_t b = (uint16_t)_cvtss_sh(f, 0); /* imm 0: round to nearest even */
    bad += (a != b); /* NaNs too: F16C truncates the payload and quiets like fcvtn */
  }
  c->bad[tid] = bad;
#else
  (void)p;
  (void)tid;
  (void)nth;
#endif
}

int64_t ark_ref_check_f32_to_f16_f16c(uint64_t lo, uint64_t hi, int nthreads) {
#if defined(__F16C__)
  if (nthreads < 1) nthreads = 1;
  if (hi > (1ull << 32)) hi = 1ull << 32;
  if (lo >= hi) return 0;
  int64_t *bad = (int64_t *)calloc((size_t)nthreads, sizeof(int64_t));
  chk32_ctx c = {lo, hi, bad};
  run_parallel(nthreads, chk32_worker, &c);
  int64_t tot = 0;
  for (int i = 0; i < nthreads; ++i) tot += bad[i];
  free(bad);
  return tot;
#else
  (void)lo;
  (void)hi;
  (void)nthreads;
  return -1;
#endif
}

/* Compares got[i] with the conversion of the bit pattern lo + i, for the
 * patterns [lo, hi); returns the number of mismatches and the first one. */
typedef struct {
  uint64_t lo, hi;
  const uint16_t *got;
  int64_t *bad;
  uint64_t *first;
} cmp32_ctx;

static void cmp32_worker(void *p, int tid, int nth) {
  cmp32_ctx *c = (cmp32_ctx *)p;
  uint64_t lo, hi;
  split_range(c->hi - c->lo, tid, nth, &lo, &hi);
  int64_t bad = 0;
  uint64_t first = UINT64_MAX;
  for (uint64_t i = lo; i < hi; ++i) {
    uint16_t want = ark_ref_f32_to_f16(u2f((uint32_t)(c->lo + i)));
    if (want != c->got[i]) {
      if (first == UINT64_MAX) first = c->lo + i;
      ++bad;
    }
  }
  c->bad[tid] = bad;
  c->first[tid] = first;
}

int64_t ark_ref_compare_f32_to_f16_range(uint64_t lo, uint64_t hi, const uint16_t *got,
                                         int nthreads, uint64_t *first_bad) {
  if (nthreads < 1) nthreads = 1;
  if (hi > (1ull << 32)) hi = 1ull << 32;
  if (first_bad) *first_bad = UINT64_MAX;
  if (lo >= hi) return 0;
  int64_t *bad = (int64_t *)calloc((size_t)nthreads, sizeof(int64_t));
  uint64_t *first = (uint64_t *)calloc((size_t)nthreads, sizeof(uint64_t));
  cmp32_ctx c = {lo, hi, got, bad, first};
  run_parallel(nthreads, cmp32_worker, &c);
  int64_t tot = 0;
  uint64_t f = UINT64_MAX;
  for (int i = 0; i < nthreads; ++i) {
    tot += bad[i];
    if (first[i] < f) f = first[i];
  }
  free(bad);
  free(first);
  if (first_bad) *first_bad = f;
  return tot;
}

/* ------------------------------------------------------------------------ */
/* Scalar prologue (opti.s:210-271).                                         */
/* ------------------------------------------------------------------------ */

/* opti.s:223-235: res = 1; base = beta; while (k) { if (k & 1) res *= base;
 * base *= base; k >>= 1; }  (each *= is one fmul) */
float ark_ref_pow_binary(float beta, uint32_t t) {
  float res = 1.0f;
  float base = beta;
  uint32_t k = t;
  while (k != 0) {
    if (k & 1u) res = res * base; /* fmul s13, s13, s0   :230 */
    base = base * base;           /* fmul s0, s0, s0     :232 */
    k >>= 1;                      /* lsr w9, w9, #1      :233 */
  }
  return res;
}

void ark_ref_prologue(float lr, float beta1, float beta2, float wd, uint32_t t,
                      ark_ref_scalars *out) {
  if (t == 0) t = 1;                        /* cmp w5,#0; cinc  :211-212 */
  float lw = lr * wd;                       /* fmul s12, s8, s4 :219     */
  out->decay = 1.0f - lw;                   /* fsub s12, s0, s12 :221    */
  out->bc1 = 1.0f - ark_ref_pow_binary(beta1, t); /* :236-237 */
  out->bc2 = 1.0f - ark_ref_pow_binary(beta2, t); /* :252-253 */
  float r = sqrtf(out->bc2);                /* fsqrt s15, s14   :256     */
  r = r / out->bc1;                         /* fdiv s15, s15, s13 :257   */
  out->lr_eff = r * lr;                     /* fmul s15, s15, s8 :258    */
  out->c1 = 1.0f - beta1;                   /* :263-265 */
  out->c2 = 1.0f - beta2;                   /* :266-268 */
}

/* One element of the hot loop (opti.s:278-308; the scalar tail :317-346
 * performs the identical sequence). */
static inline uint16_t adam_elem(uint16_t w16, float g, float *m, float *v,
                                 const ark_ref_scalars *s, float beta1,
                                 float beta2, float eps) {
  float w = ark_ref_f16_to_f32(w16); /* fcvtl v3.4s, v7.4h   :279 */
  float mm = *m * beta1;             /* fmul v1, v1, v16     :286 */
  mm = fmaf(s->c1, g, mm);           /* fmla v1, v18, v0     :287 */
  float vv = *v * beta2;             /* fmul v2, v2, v17     :291 */
  float gg = g * g;                  /* fmul v4, v0, v0      :292 */
  vv = fmaf(s->c2, gg, vv);          /* fmla v2, v19, v4     :293 */
  float d = sqrtf(vv);               /* fsqrt v5, v2         :297 */
  d = d + eps;                       /* fadd v5, v5, v20     :298 */
  float u = mm / d;                  /* fdiv v6, v1, v5      :299 */
  u = u * s->lr_eff;                 /* fmul v6, v6, v21     :300 */
  w = w * s->decay;                  /* fmul v3, v3, v22     :303 */
  w = w - u;                         /* fsub v3, v3, v6      :304 */
  *m = mm;                           /* str q1               :288 */
  *v = vv;                           /* str q2               :294 */
  return ark_ref_f32_to_f16(w);      /* fcvtn v7.4h, v3.4s   :307 */
}

/* One element of _ark_asm_adam_step (opti.s:105-131; the scalar tail
 * :135-160 performs the identical sequence): the fp16 element's operations
 * on fp32 weights, without the two conversions. */
static inline float adam_elem_f32(float w, float g, float *m, float *v,
                                  const ark_ref_scalars *s, float beta1,
                                  float beta2, float eps) {
  float mm = *m * beta1;             /* fmul v1, v1, v16     :114 */
  mm = fmaf(s->c1, g, mm);           /* fmla v1, v18, v0     :115 */
  float vv = *v * beta2;             /* fmul v2, v2, v17     :118 */
  float gg = g * g;                  /* fmul v4, v0, v0      :119 */
  vv = fmaf(s->c2, gg, vv);          /* fmla v2, v19, v4     :120 */
  float d = sqrtf(vv);               /* fsqrt v5, v2         :123 */
  d = d + eps;                       /* fadd v5, v5, v20     :124 */
  float u = mm / d;                  /* fdiv v6, v1, v5      :125 */
  u = u * s->lr_eff;                 /* fmul v6, v6, v21     :126 */
  w = w * s->decay;                  /* fmul v3, v3, v22     :128 */
  w = w - u;                         /* fsub v3, v3, v6      :129 */
  *m = mm;                           /* str q1               :116 */
  *v = vv;                           /* str q2               :121 */
  return w;                          /* str q3               :130 */
}

void ark_ref_adam_step_f32(float *w, const float *g, float *m, float *v, uint64_t n,
                           float lr, float beta1, float beta2, float eps, float wd,
                           uint32_t t) {
  ark_ref_scalars s;
  ark_ref_prologue(lr, beta1, beta2, wd, t, &s); /* opti.s:38-103, as :210-271 */
  for (uint64_t i = 0; i < n; ++i)
    w[i] = adam_elem_f32(w[i], g[i], &m[i], &v[i], &s, beta1, beta2, eps);
}

void ark_ref_adam_step_f16(uint16_t *w, const float *g, float *m, float *v,
                           uint64_t n, float lr, float beta1, float beta2,
                           float eps, float wd, uint32_t t) {
  ark_ref_scalars s;
  ark_ref_prologue(lr, beta1, beta2, wd, t, &s);
  for (uint64_t i = 0; i < n; ++i)
    w[i] = adam_elem(w[i], g[i], &m[i], &v[i], &s, beta1, beta2, eps);
}

/* ------------------------------------------------------------------------ */
/* Global sum of squares (optimizer.rs:127-145 restated with the canonical   */
/* f64 tree instead of the reference's sequential f32 fold) and the finite   */
/* check (training.rs:291, memory.rs:379-395).                               */
/* ------------------------------------------------------------------------ */

#define SEG ARK_OPT_NORM_SEGMENT

double ark_ref_pairwise(const double *x, uint64_t n) {
  if (n == 0) return 0.0;
  uint64_t p = 1;
  while (p < n) p <<= 1;
  double *b = (double *)malloc(sizeof(double) * (size_t)p);
  memcpy(b, x, sizeof(double) * (size_t)n);
  for (uint64_t i = n; i < p; ++i) b[i] = 0.0;
  for (uint64_t w = p >> 1; w >= 1; w >>= 1) {
    for (uint64_t i = 0; i < w; ++i) b[i] = b[2 * i] + b[2 * i + 1];
    if (w == 1) break;
  }
  double r = b[0];
  free(b);
  return r;
}

static inline int grad_nonfinite(const void *g, uint32_t dtype, uint64_t i) {
  if (dtype == ARK_OPT_GRAD_F16)
    return (((const uint16_t *)g)[i] & 0x7C00u) == 0x7C00u;
  return (f2u(((const float *)g)[i]) & 0x7F800000u) == 0x7F800000u;
}

static inline float grad_f32(const void *g, uint32_t dtype, uint64_t i) {
  if (dtype == ARK_OPT_GRAD_F16)
    return ark_ref_f16_to_f32(((const uint16_t *)g)[i]);
  return ((const float *)g)[i];
}

/* ------------------------------------------------------------------------ */
/* Optional 8-wide AVX2/F16C form of the two hot loops, used only to time   */
/* the CPU baseline.  Off by default: the checker runs the scalar           */
/* restatement.  Every operation is the same IEEE binary32 operation (F16C  */
/* conversions equal the software ones bit for bit, NaNs included; vsqrtps  */
/* and vdivps are correctly rounded; vfmadd is one fused rounding like      */
/* fmaf), so both forms give identical bits -- a CPU test checks it.        */
/* ------------------------------------------------------------------------ */

static int g_vector = 0;

int ark_ref_set_vector(int on) {
#if defined(__AVX2__) && defined(__F16C__) && defined(__FMA__)
  g_vector = on ? 1 : 0;
  return g_vector;
#else
  (void)on;
  return 0;
#endif
}

#if defined(__AVX2__) && defined(__F16C__) && defined(__FMA__)
/* Squares of 8 unscaled fp16 gradients into q[0..8) (f64, exact) and the
 * non-finite flag of the 8. */
static inline int sq8_f16(const uint16_t *g, float inv_t, double *q) {
  __m128i h = _mm_loadu_si128((const __m128i *)g);
  __m128i ex = _mm_and_si128(h, _mm_set1_epi16(0x7C00));
  int bad = _mm_movemask_epi8(_mm_cmpeq_epi16(ex, _mm_set1_epi16(0x7C00))) != 0;
  __m256 f = _mm256_mul_ps(_mm256_cvtph_ps(h), _mm256_set1_ps(inv_t));
  __m256d lo = _mm256_cvtps_pd(_mm256_castps256_ps128(f));
  __m256d hi = _mm256_cvtps_pd(_mm256_extractf128_ps(f, 1));
  _mm256_storeu_pd(q, _mm256_mul_pd(lo, lo));
  _mm256_storeu_pd(q + 4, _mm256_mul_pd(hi, hi));
  return bad;
}

/* 8 elements of adam_elem with g already unscaled and clipped. */
static inline void adam8(uint16_t *w16, __m256 g, float *m, float *v, const ark_ref_scalars *s,
                         float beta1, float beta2, float eps) {
  __m256 w = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)w16));
  __m256 mm = _mm256_mul_ps(_mm256_loadu_ps(m), _mm256_set1_ps(beta1));
  mm = _mm256_fmadd_ps(_mm256_set1_ps(s->c1), g, mm);
  __m256 vv = _mm256_mul_ps(_mm256_loadu_ps(v), _mm256_set1_ps(beta2));
  __m256 gg = _mm256_mul_ps(g, g);
  vv = _mm256_fmadd_ps(_mm256_set1_ps(s->c2), gg, vv);
  __m256 d = _mm256_add_ps(_mm256_sqrt_ps(vv), _mm256_set1_ps(eps));
  __m256 u = _mm256_mul_ps(_mm256_div_ps(mm, d), _mm256_set1_ps(s->lr_eff));
  w = _mm256_sub_ps(_mm256_mul_ps(w, _mm256_set1_ps(s->decay)), u);
  _mm256_storeu_ps(m, mm);
  _mm256_storeu_ps(v, vv);
  _mm_storeu_si128((__m128i *)w16,
                   _mm256_cvtps_ph(w, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC));
}
#endif

typedef struct {
  const ark_opt_tensor *tab;
  int32_t nt;
  uint32_t dtype;
  float inv;
  uint64_t nseg;
  const int32_t *seg_tensor;
  const uint64_t *seg_start;
  double *seg_sum;
  int32_t *bad;
} sumsq_ctx;

static void sumsq_worker(void *p, int tid, int nth) {
  sumsq_ctx *c = (sumsq_ctx *)p;
  uint64_t lo, hi;
  split_range(c->nseg, tid, nth, &lo, &hi);
  double buf[SEG];
  int32_t bad = 0;
  for (uint64_t s = lo; s < hi; ++s) {
    const ark_opt_tensor *T = &c->tab[c->seg_tensor[s]];
    float inv_t = (T->flags & ARK_OPT_TENSOR_NO_UNSCALE) ? 1.0f : c->inv;
    uint64_t st = c->seg_start[s];
    uint64_t len = T->n - st < SEG ? T->n - st : SEG;
    uint64_t j0 = 0;
#if defined(__AVX2__) && defined(__F16C__) && defined(__FMA__)
    if (g_vector && c->dtype == ARK_OPT_GRAD_F16)
      for (; j0 + 8 <= len; j0 += 8)
        bad |= sq8_f16((const uint16_t *)T->g + st + j0, inv_t, buf + j0);
#endif
    for (uint64_t j = j0; j < len; ++j) {
      bad |= grad_nonfinite(T->g, c->dtype, st + j);
      float gu = grad_f32(T->g, c->dtype, st + j) * inv_t; /* vDSP_vsmul */
      buf[j] = (double)gu * (double)gu;                     /* exact */
    }
    for (uint64_t j = len; j < SEG; ++j) buf[j] = 0.0;
    for (uint64_t w = SEG / 2; w >= 1; w >>= 1) {
      for (uint64_t i = 0; i < w; ++i) buf[i] = buf[2 * i] + buf[2 * i + 1];
      if (w == 1) break;
    }
    c->seg_sum[s] = buf[0];
  }
  c->bad[tid] = bad;
}

/* Segment list: every tensor's [0, n) cut into SEG-element pieces, tensors
 * in table order. */
static uint64_t build_segments(const ark_opt_tensor *tab, int32_t nt,
                               int32_t **seg_tensor, uint64_t **seg_start) {
  uint64_t nseg = 0;
  for (int32_t i = 0; i < nt; ++i) nseg += (tab[i].n + SEG - 1) / SEG;
  *seg_tensor = (int32_t *)malloc(sizeof(int32_t) * (size_t)(nseg ? nseg : 1));
  *seg_start = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)(nseg ? nseg : 1));
  uint64_t k = 0;
  for (int32_t i = 0; i < nt; ++i)
    for (uint64_t st = 0; st < tab[i].n; st += SEG) {
      (*seg_tensor)[k] = i;
      (*seg_start)[k] = st;
      ++k;
    }
  return nseg;
}

double ark_ref_sumsq(const ark_opt_tensor *tab, int32_t nt, uint32_t grad_dtype,
                     float inv_scale, int nthreads, int32_t *nonfinite) {
  if (nthreads < 1) nthreads = 1;
  int32_t *seg_tensor;
  uint64_t *seg_start;
  uint64_t nseg = build_segments(tab, nt, &seg_tensor, &seg_start);
  double *seg_sum = (double *)malloc(sizeof(double) * (size_t)(nseg ? nseg : 1));
  int32_t *bad = (int32_t *)calloc((size_t)nthreads, sizeof(int32_t));
  sumsq_ctx c = {tab, nt, grad_dtype, inv_scale, nseg, seg_tensor, seg_start,
                 seg_sum, bad};
  if ((uint64_t)nthreads > nseg) nthreads = nseg ? (int)nseg : 1;
  run_parallel(nthreads, sumsq_worker, &c);
  int32_t any = 0;
  for (int i = 0; i < nthreads; ++i) any |= bad[i];
  double r = ark_ref_pairwise(seg_sum, nseg);
  free(seg_tensor);
  free(seg_start);
  free(seg_sum);
  free(bad);
  if (nonfinite) *nonfinite = any;
  return r;
}

/* ------------------------------------------------------------------------ */
/* Fused step.                                                               */
/* ------------------------------------------------------------------------ */

void ark_ref_state_init(const ark_opt_hparams *hp, ark_opt_state *st) {
  memset(st, 0, sizeof(*st));
  st->loss_scale = hp->loss_scale_init; /* training.rs:120 */
}

typedef struct {
  const ark_opt_tensor *tab;
  int32_t nt;
  const ark_opt_hparams *hp;
  uint32_t t;
  float lr, inv, coef;
  int clipped;
  uint64_t total;         /* total elements */
  const uint64_t *prefix; /* prefix[i] = elements before tensor i */
} upd_ctx;

static void upd_worker(void *p, int tid, int nth) {
  upd_ctx *c = (upd_ctx *)p;
  uint64_t lo, hi;
  split_range(c->total, tid, nth, &lo, &hi);
  for (int32_t i = 0; i < c->nt; ++i) {
    const ark_opt_tensor *T = &c->tab[i];
    uint64_t a = c->prefix[i], b = a + T->n;
    uint64_t s0 = a > lo ? a : lo, s1 = b < hi ? b : hi;
    if (s0 >= s1) continue;
    /* per-tensor prologue, as each of the 272 calls of optimizer.rs:185-227
     * runs opti.s:210-271 with its own wd */
    ark_ref_scalars s;
    ark_ref_prologue(c->lr, c->hp->beta1, c->hp->beta2, T->weight_decay, c->t,
                     &s);
    float inv_t = (T->flags & ARK_OPT_TENSOR_NO_UNSCALE) ? 1.0f : c->inv;
    uint64_t e0 = s0 - a;
#if defined(__AVX2__) && defined(__F16C__) && defined(__FMA__)
    if (g_vector) {
      const __m256 vinv = _mm256_set1_ps(inv_t), vcoef = _mm256_set1_ps(c->coef);
      for (; e0 + 8 <= s1 - a; e0 += 8) {
        __m256 g = c->hp->grad_dtype == ARK_OPT_GRAD_F16
                       ? _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)((const uint16_t *)T->g + e0)))
                       : _mm256_loadu_ps((const float *)T->g + e0);
        g = _mm256_mul_ps(g, vinv);
        if (c->clipped) g = _mm256_mul_ps(g, vcoef);
        adam8(T->w + e0, g, T->m + e0, T->v + e0, &s, c->hp->beta1, c->hp->beta2,
              c->hp->eps);
      }
    }
#endif
    for (uint64_t e = e0; e < s1 - a; ++e) {
      float g = grad_f32(T->g, c->hp->grad_dtype, e) * inv_t; /* training.rs:308 */
      if (c->clipped) g = g * c->coef; /* optimizer.rs:151-165 */
      T->w[e] = adam_elem(T->w[e], g, &T->m[e], &T->v[e], &s, c->hp->beta1,
                          c->hp->beta2, c->hp->eps);
    }
  }
}

static void run_update(const ark_opt_tensor *tab, int32_t nt,
                       const ark_opt_hparams *hp, uint32_t t, float lr,
                       float inv, int clipped, float coef, int nthreads) {
  uint64_t *prefix = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)(nt + 1));
  uint64_t tot = 0;
  for (int32_t i = 0; i < nt; ++i) {
    prefix[i] = tot;
    tot += tab[i].n;
  }
  prefix[nt] = tot;
  upd_ctx c = {tab, nt, hp, t, lr, inv, coef, clipped, tot, prefix};
  if (nthreads < 1) nthreads = 1;
  run_parallel(nthreads, upd_worker, &c);
  free(prefix);
}

static void fill_info(ark_opt_step_info *info, const ark_opt_state *st,
                      int applied, int nonfinite, int clipped, int status,
                      double sumsq, float norm, float coef, float inv, float lr,
                      float lr_eff) {
  if (!info) return;
  memset(info, 0, sizeof(*info));
  info->applied = applied;
  info->nonfinite = nonfinite;
  info->clipped = clipped;
  info->status = status;
  info->grad_sumsq = sumsq;
  info->grad_norm = norm;
  info->clip_coef = coef;
  info->inv_scale = inv;
  info->lr = lr;
  info->lr_eff = lr_eff;
  info->state = *st;
}

/* Skip branch shared by the gradient check (training.rs:293-305) and the
 * logits-gradient check (training.rs:230-239). */
static int amp_skip(const ark_opt_hparams *hp, ark_opt_state *st) {
  float s = st->loss_scale * 0.5f;                             /* :294 */
  st->loss_scale = fmaxf(s, hp->loss_scale_min);               /* .max(MIN) */
  st->clean_steps = 0;                                         /* :295 */
  st->skipped_steps += 1;                                      /* :296 */
  st->consecutive_nonfinite += 1;                              /* :297 */
  if (st->consecutive_nonfinite > hp->max_consecutive_nonfinite) { /* :298 */
    st->early_stop = 1;
    return ARK_OPT_EARLY_STOP;
  }
  return ARK_OPT_OK;
}

/* Clean-step bookkeeping after an applied update (training.rs:316-326);
 * `scale` is the scale the step ran with. */
static void amp_clean(const ark_opt_hparams *hp, ark_opt_state *st, float scale) {
  st->clean_steps += 1;                                    /* :317 */
  st->consecutive_nonfinite = 0;                           /* :318 */
  if (st->clean_steps >= hp->scale_up_every) {             /* :319 */
    float nueva = fminf(scale * 2.0f, hp->loss_scale_max); /* :320 */
    if (nueva > scale) st->loss_scale = nueva;             /* :321-324 */
    st->clean_steps = 0;                                   /* :325 */
  }
}

int ark_ref_amp_replay(const ark_opt_hparams *hp, ark_opt_state *st,
                       const uint8_t *events, uint64_t n, float *scale_out) {
  int status = ARK_OPT_OK;
  for (uint64_t i = 0; i < n; ++i) {
    if (st->early_stop) {
      status = ARK_OPT_EARLY_STOP;
    } else if (events[i]) {
      status = amp_skip(hp, st);
    } else {
      float scale = st->loss_scale;
      st->t += 1; /* optimizer.rs:172 */
      amp_clean(hp, st, scale);
      status = ARK_OPT_OK;
    }
    if (scale_out) scale_out[i] = st->loss_scale;
  }
  return status;
}

int ark_ref_finalize(const ark_opt_hparams *hp, ark_opt_state *st,
                     double sumsq, int nonfinite, float lr,
                     ark_opt_step_info *info) {
  if (st->early_stop) {
    fill_info(info, st, 0, 0, 0, ARK_OPT_EARLY_STOP, 0.0, 0.0f, 1.0f,
              1.0f / st->loss_scale, lr, 0.0f);
    return ARK_OPT_EARLY_STOP;
  }
  float scale = st->loss_scale;
  float inv = 1.0f / scale; /* training.rs:244, before any state change */
  if (nonfinite) { /* training.rs:293-305: no update, t unchanged */
    /* the sum of a non-finite step is reported as NaN */
    int status = amp_skip(hp, st);
    fill_info(info, st, 0, 1, 0, status, (double)NAN, NAN, 1.0f, inv, lr, 0.0f);
    return status;
  }
  float norm = sqrtf((float)sumsq);                     /* optimizer.rs:145 */
  int clipped = (norm > hp->grad_clip) && (norm > 0.0f); /* :148 */
  float coef = clipped ? hp->grad_clip / norm : 1.0f;    /* :149 */
  st->t += 1;                                            /* optimizer.rs:172 */
  ark_ref_scalars s0;
  ark_ref_prologue(lr, hp->beta1, hp->beta2, 0.0f, st->t, &s0);
  amp_clean(hp, st, scale); /* training.rs:316-326 */
  fill_info(info, st, 1, 0, clipped, ARK_OPT_OK, sumsq, norm, coef, inv, lr,
            s0.lr_eff);
  return ARK_OPT_OK;
}

int ark_ref_opt_step(const ark_opt_tensor *tab, int32_t nt,
                     const ark_opt_hparams *hp, ark_opt_state *st, float lr,
                     int nthreads, ark_opt_step_info *info) {
  ark_opt_step_info f;
  int32_t nonfinite = 0;
  double sumsq = 0.0;
  if (!st->early_stop) /* the sum is over grads unscaled by the step's scale */
    sumsq = ark_ref_sumsq(tab, nt, hp->grad_dtype, 1.0f / st->loss_scale,
                          nthreads, &nonfinite);
  int status = ark_ref_finalize(hp, st, sumsq, nonfinite, lr, &f);
  /* the update runs with the advanced t (optimizer.rs:172 comes first); the
   * scale bookkeeping inside the finalize does not touch what it reads */
  if (f.applied)
    run_update(tab, nt, hp, st->t, lr, f.inv_scale, f.clipped, f.clip_coef,
               nthreads);
  if (info) *info = f;
  return status;
}

int ark_ref_apply_given(const ark_opt_tensor *tab, int32_t nt,
                        const ark_opt_hparams *hp, uint32_t t, float lr,
                        const ark_opt_step_info *given, int nthreads) {
  if (!given->applied) return ARK_OPT_OK;
  run_update(tab, nt, hp, t, lr, given->inv_scale, given->clipped,
             given->clip_coef, nthreads);
  return ARK_OPT_OK;
}

/* ------------------------------------------------------------------------ */
/* Per-tensor clip (opti.s:369-432).                                         */
/* ------------------------------------------------------------------------ */

/* The clip branch shared by both forms below (opti.s:401-420). */
static void clip_apply(float *g, uint64_t n, float norm, float thr) {
  if (!(norm > thr)) return;   /* fcmp s9, s8; b.le .L_clip_skip  :401-402 */
  const float c = thr / norm;  /* fdiv s17, s8, s9                 :404 */
  for (uint64_t i = 0; i < n; ++i) g[i] = g[i] * c; /* fmul :412, :418 */
}

float ark_ref_grad_clip_literal(float *g, uint64_t n, float thr) {
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}; /* movi v16.4s, #0   :381 */
  uint64_t i = 0;
  for (; i + 4 <= n; i += 4)               /* .L_clip_norm4     :384-389 */
    for (int l = 0; l < 4; ++l)
      acc[l] = fmaf(g[i + l], g[i + l], acc[l]); /* fmla v16.4s, v0.4s, v0.4s */
  /* faddp v16.4s, v16.4s, v16.4s; faddp s16, v16.2s  :391-392 */
  float s = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  for (; i < n; ++i) s = fmaf(g[i], g[i], s); /* fmadd s16, s0, s0, s16 :396 */
  const float norm = sqrtf(s);                 /* fsqrt s9, s16         :399 */
  clip_apply(g, n, norm, thr);
  return norm;                                 /* fmov s0, s9           :423 */
}

float ark_ref_grad_clip(float *g, uint64_t n, float thr, int nthreads) {
  if (n == 0) return 0.0f;
  ark_opt_tensor t;
  memset(&t, 0, sizeof(t));
  t.g = g;
  t.n = n;
  int32_t bad = 0;
  const double sum = ark_ref_sumsq(&t, 1, ARK_OPT_GRAD_F32, 1.0f, nthreads, &bad);
  const float norm = sqrtf((float)sum);
  clip_apply(g, n, norm, thr);
  return norm;
}

int ark_ref_record_overflow(const ark_opt_hparams *hp, ark_opt_state *st,
                            ark_opt_step_info *info) {
  if (st->early_stop) {
    fill_info(info, st, 0, 1, 0, ARK_OPT_EARLY_STOP, 0.0, 0.0f, 1.0f,
              1.0f / st->loss_scale, 0.0f, 0.0f);
    return ARK_OPT_EARLY_STOP;
  }
  float inv = 1.0f / st->loss_scale;
  int status = amp_skip(hp, st);
  fill_info(info, st, 0, 1, 0, status, 0.0, 0.0f, 1.0f, inv, 0.0f, 0.0f);
  return status;
}

/* ------------------------------------------------------------------------ */
/* Synthetic generator (include/ark_synth.h).                                */
/* ------------------------------------------------------------------------ */

#define GOLDEN 0x9E3779B97F4A7C15ull

uint64_t ark_ref_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t ark_ref_splitmix64_next(uint64_t *state) {
  *state += GOLDEN;
  return ark_ref_mix64(*state);
}

uint64_t ark_ref_synth_base(uint64_t seed, uint32_t tensor_id, uint32_t step) {
  uint64_t ctr = ((uint64_t)tensor_id << 32) | (uint64_t)step;
  return ark_ref_mix64(seed + GOLDEN * (ctr + 1));
}

static inline float synth_z(uint64_t base, uint64_t i) {
  uint64_t x = ark_ref_mix64(base + GOLDEN * (i + 1));
  int32_t u = (int32_t)(x & 0xFFFF) + (int32_t)((x >> 16) & 0xFFFF) +
              (int32_t)((x >> 32) & 0xFFFF) + (int32_t)((x >> 48) & 0xFFFF);
  int32_t d = 2 * u - 262140;
  return (float)d * 0x1.bb67aep-17f;
}

void ark_ref_synth_normal_f32(float *out, uint64_t n, uint64_t seed,
                              uint32_t tensor_id, uint32_t step,
                              float sigma_scale) {
  uint64_t base = ark_ref_synth_base(seed, tensor_id, step);
  for (uint64_t i = 0; i < n; ++i) out[i] = synth_z(base, i) * sigma_scale;
}

void ark_ref_synth_normal_f16(uint16_t *out, uint64_t n, uint64_t seed,
                              uint32_t tensor_id, uint32_t step,
                              float sigma_scale) {
  uint64_t base = ark_ref_synth_base(seed, tensor_id, step);
  for (uint64_t i = 0; i < n; ++i)
    out[i] = ark_ref_f32_to_f16(synth_z(base, i) * sigma_scale);
}

/* ------------------------------------------------------------------------ */
/* Gradient hand-off (objc/bridge.m:902-948).                                */
/* ------------------------------------------------------------------------ */

void ark_ref_grad_accumulate(float *dst, const float *src, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) dst[i] += src[i];
}

void ark_ref_embed_scatter(float *embed_grad, uint32_t vocab, uint32_t d,
                           const uint32_t *tokens, const float *dx0, uint32_t batch_seq) {
  for (uint32_t i = 0; i < batch_seq; ++i) {
    uint32_t t = (tokens[i] < vocab) ? tokens[i] : 0;
    for (uint32_t j = 0; j < d; ++j)
      embed_grad[(uint64_t)t * d + j] += dx0[(uint64_t)i * d + j];
  }
}
