// Launch policy as the kernels' host code sees it: the caller's q4nx_policy, or the defaults.
#pragma once

#include "../../include/q4nx_hip.h"

namespace q4nx {

struct Policy {
  int mfma_rows[2];   // [q4, q8]: rows from which the matrix-core kernels take a call; 0 never
  int rowblock;       // one-row q4 calls on the row-block kernels
  int gemv_ksplit;    // general VALU GEMV: K parts per group, 0 automatic
  int gemv_tpw;       // general VALU GEMV: K-tiles per wave, 0 automatic
  int gemm_ksplit;    // matrix-core contraction: K parts, 0 automatic
  int attn_mfma;      // attention on the matrix cores
};

// Copies *p (NULL: the defaults) into *out. Returns Q4NX_OK, or Q4NX_ERR_ARG with the error
// message set when a field is out of range.
int resolve_policy(const q4nx_policy* p, Policy* out, const char* what);
// The same without an error message, for the size queries (false: invalid policy).
bool resolve_policy_quiet(const q4nx_policy* p, Policy* out);

}  // namespace q4nx
