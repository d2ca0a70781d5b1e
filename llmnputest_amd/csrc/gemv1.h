// Batch-1 GEMV family (gemv1.hip): one workgroup per (output group, 16-row block); q4
// tiles, and q8 tiles for a plain GEMV.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q4nx {

enum Gemv1Op : int { G1_PLAIN = 0, G1_QKV = 1, G1_GATEUP = 2 };

struct Gemv1Args {
  // read before the weight stream (kept first and contiguous: one round of scalar loads)
  const uint8_t* w0;         // plain: W; gate/up: gate; q/k/v: q
  const uint8_t* w1;         // gate/up: up; q/k/v: k
  const uint8_t* w2;         // q/k/v: v
  // input: bf16 x, or the fp32 residual h normalised in the prologue (norm_w != nullptr,
  // with the producer's sums of squares ssq_in [K/16]), or attention split records
  const uint16_t* x;
  const float* hres;
  const uint16_t* norm_w;
  const float* ssq_in;
  const float* att_rec;
  const float* residual;     // plain: optional fp32 [N] added to the output
  const int32_t* pos;        // q/k/v: the sequence position
  int k_t;                   // K-tiles
  int n_groups;              // output groups (tile-rows; heads for q/k/v); 2 workgroups each
  int grp_q, grp_k;          // q/k/v: groups [0,grp_q) are q heads, then grp_k k heads, then v
  int att_split, att_g;      // records: splits, query heads per kv head
  float eps;
  int max_pos;
  // read in the epilogue
  uint16_t* xn_out;          // optional normalised row (bf16 [K])
  float* y;
  float* ssq_out;            // optional [N/16]
  unsigned long long* keys;  // optional argmax keys [N/16]
  uint16_t* q_out;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t kv_h_stride;
  const float* rope_tab;
  float* raw_out;            // optional fp32 GEMV outputs (q/k/v, gate/up)
  uint16_t* h_out;           // gate/up
  int n_q_heads, n_kv_heads;
};

int gemv1_tpw(int G, int k_t);
bool gemv1_fits(int G, int k_t, bool norm);
// kind 8 (q8 tiles): plain GEMV only. tpw_req: K-tiles per wave (1, 2 or 4), 0 = the fewest
// that fit the group's K into 16 waves.
int gemv1_launch(int op, const Gemv1Args& a, hipStream_t s, const char* what, int kind = 4,
                 int tpw_req = 0);
int gemv1_attn_launch(const Gemv1Args& a, hipStream_t s, const char* what);

}  // namespace q4nx
