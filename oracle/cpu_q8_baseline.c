/* CPU baseline for the q8 lm_head GEMV: y = W x for one token, W in q4nx q8 tiles.
 * TEST AND BENCHMARK INFRASTRUCTURE ONLY (the bench's CPU leg; tests check it against the
 * float64 oracle).
 *
 * The reference ships a CPU baseline for the q4 GEMV only (designs/granite_gemv/
 * cpu_baseline.cpp). This is the same method applied to the q8 tile, so that the q8 CPU
 * figure is like-for-like with it:
 *   - AVX2 + FMA, fp32 accumulation (cpu_baseline.cpp:43-97);
 *   - one thread per core, each claiming the next tile-row from one atomic counter
 *     (cpu_baseline.cpp:145-155);
 *   - the per-(row, 32-K group) scale factored out of the inner sum: for each group the
 *     16 rows of a row block accumulate sum_k code * x over its 32 K, and the group's bf16
 *     scale multiplies that sum once (lm_head.h:21-29 states w = int8 * scale).
 *
 * Tile (tools/q4nx.py:104-111, 140-143): 512 B of bf16 scales indexed g = kb*32 + rb*16 + r
 * (kb the 32-K group, rb the 16-row block, r the row in it), then 8192 int8 codes indexed
 * rb*4096 + k*16 + r: the 16 rows of one row block at one k are 16 consecutive bytes.
 */
#include <immintrin.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>
#include <string.h>

#define Q8_TILE 8704
#define Q8_META 512

/* eight consecutive bf16 values (little-endian bits) widened to fp32 */
static inline __m256 bf16x8(const uint8_t *p) {
  const __m128i h = _mm_loadu_si128((const __m128i *)p);
  return _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(h), 16));
}

/* y[0..31] of one tile-row */
static void q8_row(const uint8_t *row, const float *x, int k_t, float *y) {
  __m256 acc[4];
  for (int i = 0; i < 4; ++i) acc[i] = _mm256_setzero_ps();
  for (int kt = 0; kt < k_t; ++kt) {
    const uint8_t *tile = row + (size_t)kt * Q8_TILE;
    const int8_t *codes = (const int8_t *)(tile + Q8_META);
    const float *xt = x + (size_t)kt * 256;
    for (int kb = 0; kb < 8; ++kb) {
      for (int rb = 0; rb < 2; ++rb) {
        const int8_t *c = codes + rb * 4096 + kb * 32 * 16;
        __m256 s_lo = _mm256_setzero_ps(), s_hi = _mm256_setzero_ps();
        for (int k = 0; k < 32; ++k) {
          const __m128i b = _mm_loadu_si128((const __m128i *)(c + 16 * k));
          const __m256 xv = _mm256_broadcast_ss(xt + kb * 32 + k);
          s_lo = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(b)), xv, s_lo);
          s_hi = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(b, 8))),
                                 xv, s_hi);
        }
        const uint8_t *sc = tile + 2 * (kb * 32 + rb * 16);
        acc[2 * rb] = _mm256_fmadd_ps(bf16x8(sc), s_lo, acc[2 * rb]);
        acc[2 * rb + 1] = _mm256_fmadd_ps(bf16x8(sc + 16), s_hi, acc[2 * rb + 1]);
      }
    }
  }
  for (int i = 0; i < 4; ++i) _mm256_storeu_ps(y + 8 * i, acc[i]);
}

typedef struct {
  const uint8_t *w;
  const float *x;
  float *y;
  int n_t, k_t;
  atomic_int next;   /* the next tile-row to claim */
} q8_job;

static void *q8_worker(void *arg) {
  q8_job *j = (q8_job *)arg;
  const size_t row_bytes = (size_t)j->k_t * Q8_TILE;
  for (int tr = atomic_fetch_add(&j->next, 1); tr < j->n_t; tr = atomic_fetch_add(&j->next, 1))
    q8_row(j->w + (size_t)tr * row_bytes, j->x, j->k_t, j->y + (size_t)tr * 32);
  return 0;
}

/* y fp32 [n_t*32] = W x, x fp32 [k_t*256]; `threads` workers (1..256). 0 on success. */
int cpu_q8_gemv(const uint8_t *w, int n_t, int k_t, const float *x, float *y, int threads) {
  if (!w || !x || !y || n_t <= 0 || k_t <= 0) return -1;
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  q8_job job;
  job.w = w;
  job.x = x;
  job.y = y;
  job.n_t = n_t;
  job.k_t = k_t;
  atomic_init(&job.next, 0);
  pthread_t th[256];
  int started = 0;
  for (int i = 0; i < threads - 1; ++i)
    if (pthread_create(&th[started], 0, q8_worker, &job) == 0) ++started;
  q8_worker(&job);   /* the calling thread works too */
  for (int i = 0; i < started; ++i) pthread_join(th[i], 0);
  return 0;
}
