// Error plumbing, ABI version and host-side tables for libq4nx_hip.so.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include "common.h"
#include "policy.h"

namespace q4nx {

static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return Q4NX_ERR_LAUNCH;
  }
  return Q4NX_OK;
}

static void policy_defaults(q4nx_policy* p) {
  p->mfma_rows_q4 = 2;   // one q4 row is faster on the row-block kernels, two and more on MFMA
  p->mfma_rows_q8 = 2;   // the same for q8 (lm_head 100352 x 2560: 46.5 against 56.9 us)
  p->rowblock = 1;
  p->gemv_ksplit = 0;
  p->gemv_tiles_per_wave = 0;
  p->gemm_ksplit = 0;
  p->attn_mfma = 1;
}

static const char* policy_problem(const q4nx_policy* p) {
  if (p->mfma_rows_q4 < 0 || p->mfma_rows_q8 < 0) return "mfma_rows must be >= 0";
  if (p->rowblock != 0 && p->rowblock != 1) return "rowblock must be 0 or 1";
  if (p->gemv_ksplit < 0 || p->gemv_ksplit > 8) return "gemv_ksplit must be 0..8";
  if (p->gemv_tiles_per_wave != 0 && p->gemv_tiles_per_wave != 1 &&
      p->gemv_tiles_per_wave != 2 && p->gemv_tiles_per_wave != 4)
    return "gemv_tiles_per_wave must be 0, 1, 2 or 4";
  if (p->gemm_ksplit < 0 || p->gemm_ksplit > 8) return "gemm_ksplit must be 0..8";
  if (p->attn_mfma != 0 && p->attn_mfma != 1) return "attn_mfma must be 0 or 1";
  return nullptr;
}

static void policy_copy(const q4nx_policy& p, Policy* out) {
  out->mfma_rows[0] = p.mfma_rows_q4;
  out->mfma_rows[1] = p.mfma_rows_q8;
  out->rowblock = p.rowblock;
  out->gemv_ksplit = p.gemv_ksplit;
  out->gemv_tpw = p.gemv_tiles_per_wave;
  out->gemm_ksplit = p.gemm_ksplit;
  out->attn_mfma = p.attn_mfma;
}

bool resolve_policy_quiet(const q4nx_policy* p, Policy* out) {
  q4nx_policy d;
  policy_defaults(&d);
  if (p == nullptr) p = &d;
  if (policy_problem(p) != nullptr) return false;
  policy_copy(*p, out);
  return true;
}

int resolve_policy(const q4nx_policy* p, Policy* out, const char* what) {
  q4nx_policy d;
  policy_defaults(&d);
  if (p == nullptr) p = &d;
  const char* bad = policy_problem(p);
  Q4NX_REQUIRE(bad == nullptr, Q4NX_ERR_ARG, "%s: invalid policy: %s", what, bad);
  policy_copy(*p, out);
  return Q4NX_OK;
}

}  // namespace q4nx

extern "C" {

void q4nx_policy_init(q4nx_policy* p) {
  if (p != nullptr) q4nx::policy_defaults(p);
}

int q4nx_abi_version(void) { return Q4NX_ABI_VERSION; }

const char* q4nx_last_error(void) { return q4nx::g_err; }

// cos/sin of pos * theta^(-2i/hd) in float64, rounded once to float32.
// The reference builds the same angles in float64 on the host
// (designs/granite_gemv/granite_elementwise.py:135-138) but then rounds cos/sin to bf16.
int q4nx_rope_table_host(float* tab, int max_pos, int head_dim, double theta) {
  Q4NX_REQUIRE(tab != nullptr, Q4NX_ERR_ARG, "q4nx_rope_table_host: null table");
  Q4NX_REQUIRE(max_pos > 0 && head_dim > 0 && head_dim % 2 == 0 && theta > 0.0, Q4NX_ERR_SHAPE,
               "q4nx_rope_table_host: max_pos=%d head_dim=%d theta=%g", max_pos, head_dim, theta);
  const int half = head_dim / 2;
  for (int p = 0; p < max_pos; ++p) {
    for (int i = 0; i < half; ++i) {
      const double inv = 1.0 / pow(theta, (double)(2 * i) / (double)head_dim);
      const double ang = (double)p * inv;
      tab[(size_t)p * head_dim + i] = (float)cos(ang);
      tab[(size_t)p * head_dim + half + i] = (float)sin(ang);
    }
  }
  return Q4NX_OK;
}

}  // extern "C"
