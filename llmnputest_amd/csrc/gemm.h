// Batched q4nx contraction on the matrix cores: the arguments and host entry shared by the
// GEMM entry point and the GEMV / fused entry points that hand their larger batches to it.
#pragma once

#include "common.h"
#include "policy.h"

namespace q4nx {

enum GemmOp : int { GOP_PLAIN = 0, GOP_GATEUP = 1, GOP_QKV = 2 };

struct GemmArgs {
  // weights: PLAIN one tensor (RT consecutive tile-rows per workgroup); GATEUP gate and up
  // (tile-row t of each); QKV q, k and v (the two tile-rows of one head)
  const uint8_t* w[3];
  int n_tr[3];
  int grp_q, grp_k;      // QKV: groups [0, grp_q) are q heads, then k heads, then v heads
  // input: bf16 x, or (norm) fp32 residual h normalised with norm_w and the producer's sums
  // of squares ssq_in [m][K/16]
  const uint16_t* x;
  const float* hres;
  const uint16_t* norm_w;
  const float* ssq_in;
  uint16_t* xn_out;      // optional [m][x_stride] normalised bf16 input (else in the workspace)
  float eps;
  int64_t x_stride;
  int m_rows, k_t;
  // PLAIN
  float* y;
  int64_t y_stride;
  const float* residual;
  float* ssq_out;                    // [m][2 n_tr] sums of y^2 per 16-row block
  unsigned long long* argmax_keys;   // [m][2 n_tr] (max, first row) keys per 16-row block
  // GATEUP / QKV: fp32 values before the epilogue (optional)
  float* raw_out;
  uint16_t* h_out;
  int64_t h_stride;
  uint16_t* q_out;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t kv_b_stride, kv_h_stride;
  const int32_t* pos;
  const float* rope_tab;
  int max_pos, n_q_heads, n_kv_heads;
  // split K
  int ksplit, kpp;       // workgroups along K, K-tiles per part
  float* part;           // [unit][m_block][part][MB][NW] fp32 (NW: outputs per row)
  uint32_t part_bytes;
  unsigned* counters;    // one arrival counter per (group, m-block)
};

// true when `rows` rows of kind `kind` run on the matrix cores under the policy
bool mfma_use(int kind, int rows, const Policy& P);
// workspace bytes of a launch of `n_units` tile-rows (PLAIN) or output groups (fused)
size_t mfma_ws_bytes(int kind, int op, int n_units, int k_t, int m_rows, const Policy& P);
// whether ws_bytes holds the normalised rows an RMSNorm prologue needs on this path
bool mfma_norm_fits(int k_t, int m_rows, size_t ws_bytes);
// The prefill kernel (gemm_pf.hip) takes plain contractions from this many rows.
constexpr int kPrefillRows = 128;
// workspace bytes the prefill kernel keeps its per-group sums of x in (past the counters,
// the split records and the normalised rows), or 0 when the shape does not take that kernel
size_t pf_ws_bytes(int n_tile_rows, int k_t, int m_rows);
// whether a launch of op `op` described by `a` has the prefill kernel's shape
bool pf_use(int op, const GemmArgs& a);
// launches `a` on the prefill kernel (whole K per workgroup, no split): the per-group sums
// of x into `sums` (pf_ws_bytes of them, 256-byte aligned), then the contraction
void pf_launch(int kind, const GemmArgs& a, void* sums, hipStream_t st);
// launches `a` (all but the split-K fields filled in); returns Q4NX_OK or an error code
int mfma_launch(int kind, int op, GemmArgs& a, int n_units, void* ws, size_t ws_bytes,
                const Policy& P, hipStream_t st, const char* what);

}  // namespace q4nx
