/* CPU GQA decode attention for one token: the attention leg of the bench's CPU decode
 * baseline. TEST AND BENCHMARK INFRASTRUCTURE ONLY (tests check it against the float64
 * oracle).
 *
 * The reference runs attention on the NPU only (designs/granite_gemv/granite_attention.h:
 * 80-213; its float64 check granite_attention.py:163-167) and ships no CPU version; this is
 * the CPU counterpart written in the style of its CPU GEMV baseline (cpu_baseline.cpp:43-97,
 * 145-155): AVX2 + FMA, fp32 arithmetic, one thread per core claiming work items (here the
 * query heads) from one atomic counter.
 *
 * out[h] = softmax(scale * K_j q_h) V_j over positions [0, len), q head h reading kv head
 * j = h / (Hq / Hkv); K and V are bf16 [Hkv][l_stride][64] (the decode cache layout), q and
 * out fp32 [Hq][64]. The exponential is e^y = 2^n e^(y - n ln 2) with n the nearest integer
 * to y / ln 2 and e^r on |r| <= ln(2)/2 from its Taylor series to degree 7 (truncation error
 * below 6e-9 relative), assembled with the exponent bits.
 */
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>

#define HD 64

static inline __m256 bf16x8_ld(const uint16_t *p) {
  const __m128i h = _mm_loadu_si128((const __m128i *)p);
  return _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(h), 16));
}

static inline float hsum8(__m256 v) {
  const __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  const __m128 t = _mm_add_ps(s, _mm_movehl_ps(s, s));
  return _mm_cvtss_f32(_mm_add_ss(t, _mm_shuffle_ps(t, t, 1)));
}

/* e^y for y <= 0 (softmax arguments); y below -87 gives 0 */
static inline __m256 exp8(__m256 y) {
  const __m256 ln2 = _mm256_set1_ps(0.6931471805599453f);
  const __m256 n = _mm256_round_ps(_mm256_mul_ps(y, _mm256_set1_ps(1.4426950408889634f)),
                                   _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  const __m256 r = _mm256_fnmadd_ps(n, ln2, y);
  /* 1 + r + r^2/2! + ... + r^7/7!, Horner */
  __m256 p = _mm256_set1_ps(1.0f / 5040.0f);
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 720.0f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 120.0f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 24.0f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 6.0f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(0.5f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f));
  const __m256 keep = _mm256_cmp_ps(y, _mm256_set1_ps(-87.0f), _CMP_GE_OQ);
  const __m256i e = _mm256_slli_epi32(_mm256_add_epi32(_mm256_cvtps_epi32(n),
                                                       _mm256_set1_epi32(127)), 23);
  return _mm256_and_ps(keep, _mm256_mul_ps(p, _mm256_castsi256_ps(e)));
}

typedef struct {
  const float *q;
  const uint16_t *k, *v;
  float *out, *scores;   /* scores: [threads][len] */
  int hq, grp, len, l_stride;
  float scale;
  atomic_int next;
  atomic_int tid;
} attn_job;

static void head(const attn_job *J, int h, float *s) {
  const int j = h / J->grp, len = J->len;
  const float *q = J->q + (size_t)h * HD;
  const uint16_t *kb = J->k + (size_t)j * J->l_stride * HD;
  const uint16_t *vb = J->v + (size_t)j * J->l_stride * HD;
  __m256 qv[8];
  for (int i = 0; i < 8; ++i) qv[i] = _mm256_loadu_ps(q + 8 * i);
  const __m256 sc = _mm256_set1_ps(J->scale);
  __m256 mx = _mm256_set1_ps(-INFINITY);
  int l0 = 0;
  for (; l0 + 8 <= len; l0 += 8) {   /* 8 positions, their dot products summed by hadd */
    __m256 a[8];
    for (int p = 0; p < 8; ++p) {
      const uint16_t *kr = kb + (size_t)(l0 + p) * HD;
      a[p] = _mm256_mul_ps(bf16x8_ld(kr), qv[0]);
      for (int i = 1; i < 8; ++i) a[p] = _mm256_fmadd_ps(bf16x8_ld(kr + 8 * i), qv[i], a[p]);
    }
    const __m256 h01 = _mm256_hadd_ps(a[0], a[1]), h23 = _mm256_hadd_ps(a[2], a[3]);
    const __m256 h45 = _mm256_hadd_ps(a[4], a[5]), h67 = _mm256_hadd_ps(a[6], a[7]);
    const __m256 g0 = _mm256_hadd_ps(h01, h23), g1 = _mm256_hadd_ps(h45, h67);
    /* lanes: [p0 p1 p2 p3 | p0 p1 p2 p3] low/high halves of g0, likewise p4..p7 in g1 */
    const __m256 lo = _mm256_permute2f128_ps(g0, g1, 0x20), hi = _mm256_permute2f128_ps(g0, g1, 0x31);
    const __m256 d = _mm256_mul_ps(_mm256_add_ps(lo, hi), sc);
    _mm256_storeu_ps(s + l0, d);
    mx = _mm256_max_ps(mx, d);
  }
  float m = -INFINITY;
  {
    float t[8];
    _mm256_storeu_ps(t, mx);
    for (int i = 0; i < 8; ++i) m = t[i] > m ? t[i] : m;
  }
  for (int l = l0; l < len; ++l) {
    const uint16_t *kr = kb + (size_t)l * HD;
    __m256 a = _mm256_mul_ps(bf16x8_ld(kr), qv[0]);
    for (int i = 1; i < 8; ++i) a = _mm256_fmadd_ps(bf16x8_ld(kr + 8 * i), qv[i], a);
    s[l] = hsum8(a) * J->scale;
    m = s[l] > m ? s[l] : m;
  }
  const __m256 mv = _mm256_set1_ps(m);
  __m256 tot = _mm256_setzero_ps();
  int l = 0;
  for (; l + 8 <= len; l += 8) {
    const __m256 p = exp8(_mm256_sub_ps(_mm256_loadu_ps(s + l), mv));
    _mm256_storeu_ps(s + l, p);
    tot = _mm256_add_ps(tot, p);
  }
  float sum = hsum8(tot);
  for (; l < len; ++l) {
    s[l] = expf(s[l] - m);
    sum += s[l];
  }
  __m256 acc[8];
  for (int i = 0; i < 8; ++i) acc[i] = _mm256_setzero_ps();
  for (l = 0; l < len; ++l) {
    const uint16_t *vr = vb + (size_t)l * HD;
    const __m256 p = _mm256_set1_ps(s[l]);
    for (int i = 0; i < 8; ++i) acc[i] = _mm256_fmadd_ps(p, bf16x8_ld(vr + 8 * i), acc[i]);
  }
  const __m256 inv = _mm256_set1_ps(1.0f / sum);
  float *o = J->out + (size_t)h * HD;
  for (int i = 0; i < 8; ++i) _mm256_storeu_ps(o + 8 * i, _mm256_mul_ps(acc[i], inv));
}

static void *attn_worker(void *arg) {
  attn_job *J = (attn_job *)arg;
  float *s = J->scores + (size_t)atomic_fetch_add(&J->tid, 1) * J->len;
  for (int h = atomic_fetch_add(&J->next, 1); h < J->hq; h = atomic_fetch_add(&J->next, 1))
    head(J, h, s);
  return 0;
}

/* out fp32 [hq][64] = GQA decode attention of q fp32 [hq][64] over bf16 K/V
 * [hkv][l_stride][64], positions [0, len); `threads` workers (1..256). 0 on success. */
int cpu_gqa_decode(const float *q, const uint16_t *k, const uint16_t *v, float *out, int hq,
                   int hkv, int len, int l_stride, float scale, int threads) {
  if (!q || !k || !v || !out || hq <= 0 || hkv <= 0 || hq % hkv || len <= 0 || l_stride < len)
    return -1;
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  attn_job J;
  J.q = q;
  J.k = k;
  J.v = v;
  J.out = out;
  J.hq = hq;
  J.grp = hq / hkv;
  J.len = len;
  J.l_stride = l_stride;
  J.scale = scale;
  J.scores = (float *)malloc(sizeof(float) * (size_t)threads * len);
  if (!J.scores) return -2;
  atomic_init(&J.next, 0);
  atomic_init(&J.tid, 0);
  pthread_t th[256];
  int started = 0;
  for (int i = 0; i < threads - 1; ++i)
    if (pthread_create(&th[started], 0, attn_worker, &J) == 0) ++started;
  attn_worker(&J);
  for (int i = 0; i < started; ++i) pthread_join(th[i], 0);
  free(J.scores);
  return 0;
}
