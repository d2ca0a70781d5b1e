// Error plumbing, ABI version and host-side tables for libq4nx_hip.so.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

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

}  // namespace q4nx

extern "C" {

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
