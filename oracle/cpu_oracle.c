/* C restatement of the q4nx GEMV for large shapes. TEST INFRASTRUCTURE ONLY.
 *
 * y[b][n] = sum_k W[n][k] * x[b][k] with W dequantised exactly as tools/q4nx.py:127-143
 * (w = fp32(code*d + m) for q4, code*s for q8) and accumulated in float64, threads over
 * tile-rows. Same arithmetic as oracle.q4nx_oracle.gemv(acc=float64) up to the float64
 * summation order; checked against it in tests/test_oracle_cpu.py.
 *
 * The tile walk follows the reference CPU GEMV's loop order (designs/granite_gemv/
 * cpu_baseline.cpp:43-97: tile-row -> K tile -> 32-K group -> row block), without its
 * factoring, so that this file checks the factored GPU kernel rather than repeating it.
 */
#include <pthread.h>
#include <stdint.h>
#include <string.h>

static inline float bf16f(const uint8_t *p) {
  uint32_t u = ((uint32_t)p[0] | ((uint32_t)p[1] << 8)) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

typedef struct {
  const uint8_t *w;
  int kind, n_t, k_t, batch;
  const float *x;
  double *y;
  int t0, t1;
} job_t;

static void tile_row(const job_t *j, int tr) {
  const int K = j->k_t * 256, N = j->n_t * 32;
  const size_t tb = j->kind == 4 ? 5120 : 8704;
  double acc[8][32];
  memset(acc, 0, sizeof(acc));
  for (int kt = 0; kt < j->k_t; ++kt) {
    const uint8_t *t = j->w + ((size_t)tr * j->k_t + kt) * tb;
    for (int rb = 0; rb < 2; ++rb)
      for (int k = 0; k < 256; ++k) {
        const int kb = k >> 5;
        float wv[16];
        for (int r = 0; r < 16; ++r) {
          const int g = kb * 32 + rb * 16 + r;
          if (j->kind == 4) {
            const int i = rb * 4096 + k * 16 + r;
            const uint8_t byte = t[1024 + (i >> 1)];
            const int code = (i & 1) ? (byte >> 4) : (byte & 15);
            wv[r] = (float)code * bf16f(t + 2 * g) + bf16f(t + 512 + 2 * g);
          } else {
            const int code = (int8_t)t[512 + rb * 4096 + k * 16 + r];
            wv[r] = (float)code * bf16f(t + 2 * g);
          }
        }
        for (int b = 0; b < j->batch; ++b) {
          const double xk = (double)j->x[(size_t)b * K + kt * 256 + k];
          double *a = acc[b] + rb * 16;
          for (int r = 0; r < 16; ++r) a[r] += (double)wv[r] * xk;
        }
      }
  }
  for (int b = 0; b < j->batch; ++b)
    for (int r = 0; r < 32; ++r) j->y[(size_t)b * N + tr * 32 + r] = acc[b][r];
}

static void *worker(void *arg) {
  const job_t *j = (const job_t *)arg;
  for (int tr = j->t0; tr < j->t1; ++tr) tile_row(j, tr);
  return 0;
}

/* kind 4 or 8; x fp32 [batch][K]; y fp64 [batch][N]; batch <= 8. Returns 0 on success. */
int oracle_gemv(const uint8_t *w, int kind, int n_t, int k_t, const float *x, int batch,
                double *y, int threads) {
  if (!w || !x || !y || (kind != 4 && kind != 8) || n_t <= 0 || k_t <= 0 || batch < 1 ||
      batch > 8)
    return -1;
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  if (threads > n_t) threads = n_t;
  pthread_t th[256];
  job_t jobs[256];
  for (int i = 0; i < threads; ++i) {
    jobs[i] = (job_t){w, kind, n_t, k_t, batch, x, y, (int)((long)n_t * i / threads),
                      (int)((long)n_t * (i + 1) / threads)};
    pthread_create(&th[i], 0, worker, &jobs[i]);
  }
  for (int i = 0; i < threads; ++i) pthread_join(th[i], 0);
  return 0;
}
