// RMSNorm, RoPE, SwiGLU and the decode-step helpers (embedding row, argmax) for gfx950.
//
// RMSNorm  designs/granite_gemv/granite_rmsnorm.h:45-87   y = x * rsqrt(mean(x^2)+eps) * w
// RoPE     designs/granite_gemv/granite_elementwise.h:40-75  half-split rotate_half
// SwiGLU   designs/granite_gemv/granite_elementwise.h:77-108, granite_swiglu_f32.h:27-58
// All math is fp32; bf16 outputs are rounded once, RNE, and an optional fp32 copy of the
// pre-rounding value is written for parity checks.

#include <math.h>

#include "common.h"

namespace q4nx {

// ------------------------------------------------------------------ RMSNorm
template <bool XF32>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const void* __restrict__ x,
                                                      const uint16_t* __restrict__ w,
                                                      uint16_t* __restrict__ y,
                                                      float* __restrict__ y_f32, int cols,
                                                      float eps) {
  __shared__ float part[4];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const float* xf = XF32 ? (const float*)x + (size_t)b * cols : nullptr;
  const uint16_t* xb = XF32 ? nullptr : (const uint16_t*)x + (size_t)b * cols;
  float ss = 0.f;
  for (int c = tid; c < cols; c += 256) {
    const float v = XF32 ? xf[c] : bf16_to_f32(xb[c]);
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  const float tot = part[0] + part[1] + part[2] + part[3];
  const float inv = rms_inv(tot, cols, eps);
  for (int c = tid; c < cols; c += 256) {
    const float v = XF32 ? xf[c] : bf16_to_f32(xb[c]);
    const float o = (v * inv) * bf16_to_f32(w[c]);
    y[(size_t)b * cols + c] = f32_to_bf16(o);
    if (y_f32) y_f32[(size_t)b * cols + c] = o;
  }
}

// ------------------------------------------------------------------ RoPE
__global__ __launch_bounds__(256) void rope_kernel(const uint16_t* __restrict__ x,
                                                   uint16_t* __restrict__ y,
                                                   float* __restrict__ y_f32, int n_heads,
                                                   int hd, int batch,
                                                   const int32_t* __restrict__ pos,
                                                   const float* __restrict__ tab, int max_pos) {
  const int half = hd >> 1;
  const int i = blockIdx.x * 256 + threadIdx.x;  // (b, h, d < half); the host keeps it < 2^31
  if (i >= batch * n_heads * half) return;
  const int bh = i / half;
  const int d = i - bh * half;
  const int b = bh / n_heads;
  const int p = pos[b];
  const int64_t base = (int64_t)bh * hd;
  const float x0 = bf16_to_f32(x[base + d]);
  const float x1 = bf16_to_f32(x[base + half + d]);
  float y0, y1;
  if (p >= 0 && p < max_pos) {
    const float c = tab[(int64_t)p * hd + d];
    const float s = tab[(int64_t)p * hd + half + d];
    y0 = fmaf(x0, c, -(x1 * s));
    y1 = fmaf(x1, c, x0 * s);
  } else {
    y0 = y1 = __builtin_nanf("");
  }
  y[base + d] = f32_to_bf16(y0);
  y[base + half + d] = f32_to_bf16(y1);
  if (y_f32) {
    y_f32[base + d] = y0;
    y_f32[base + half + d] = y1;
  }
}

// ------------------------------------------------------------------ SwiGLU
template <bool INF32>
__global__ __launch_bounds__(256) void swiglu_kernel(const void* __restrict__ g,
                                                     const void* __restrict__ u,
                                                     uint16_t* __restrict__ y,
                                                     float* __restrict__ y_f32, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  float gv, uv;
  if (INF32) {  // fp32 accumulators are narrowed to bf16 first (granite_swiglu_f32.h:38-41)
    gv = round_bf16_op(((const float*)g)[i]);
    uv = round_bf16_op(((const float*)u)[i]);
  } else {
    gv = bf16_to_f32(((const uint16_t*)g)[i]);
    uv = bf16_to_f32(((const uint16_t*)u)[i]);
  }
  const float h = swiglu(gv, uv);
  y[i] = f32_to_bf16(h);
  if (y_f32) y_f32[i] = h;
}

// ------------------------------------------------------------------ fp32 -> bf16 rounding
__global__ __launch_bounds__(256) void round_bf16_kernel(const float* __restrict__ x,
                                                         uint16_t* __restrict__ y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) y[i] = f32_to_bf16(x[i]);
}

// ------------------------------------------------------------------ embedding rows
// h[b][c] = row tokens[b] of a [vocab][hidden] table: bf16 (KIND 16), or q4 / q8 tiles
// dequantised as tools/q4nx.py:127-143 does (q4: code * d + m with one rounding, q8: code * s).
template <int KIND>
__device__ __forceinline__ float embed_value_of(const uint8_t* __restrict__ w, int t, int c,
                                                int hidden) {
  if constexpr (KIND == Q4NX_KIND_BF16) {
    return bf16_to_f32(((const uint16_t*)w)[(size_t)t * hidden + c]);
  } else {
    const int k_t = hidden / 256;
    const int tr = t >> 5, row = t & 31, rb = row >> 4, r = row & 15;
    const int kt = c >> 8, k = c & 255, kb = k >> 5;
    const int g = kb * 32 + rb * 16 + r;
    const int i = rb * 4096 + k * 16 + r;        // weight index inside the tile
    if constexpr (KIND == Q4NX_KIND_Q8) {
      const uint8_t* tile = w + ((size_t)tr * k_t + kt) * kQ8TileBytes;
      const uint16_t s = (uint16_t)tile[2 * g] | ((uint16_t)tile[2 * g + 1] << 8);
      return (float)(int)(int8_t)tile[kMetaBytes + i] * bf16_to_f32(s);
    } else {
      const uint8_t* tile = w + ((size_t)tr * k_t + kt) * kQ4TileBytes;
      const uint16_t d = (uint16_t)tile[2 * g] | ((uint16_t)tile[2 * g + 1] << 8);
      const uint16_t m = (uint16_t)tile[kMetaBytes + 2 * g] |
                         ((uint16_t)tile[kMetaBytes + 2 * g + 1] << 8);
      const uint8_t byte = tile[2 * kMetaBytes + (i >> 1)];
      const int code = (i & 1) ? (byte >> 4) : (byte & 15);   // low nibble = even index
      return __fmul_rn((float)code, bf16_to_f32(d)) + bf16_to_f32(m);
    }
  }
}
template <int KIND>
__device__ __forceinline__ float embed_value(const uint8_t* __restrict__ w, int t, int c,
                                             int vocab, int hidden) {
  // a token out of range gives a NaN row
  return t >= 0 && t < vocab ? embed_value_of<KIND>(w, t, c, hidden) : __builtin_nanf("");
}

template <int KIND>
__global__ __launch_bounds__(256) void embed_kernel(const uint8_t* __restrict__ w,
                                                    const int32_t* __restrict__ tokens,
                                                    float* __restrict__ h,
                                                    float* __restrict__ ssq_out, int vocab,
                                                    int hidden) {
  const int b = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;   // hidden % 256 == 0: every lane is live
  const float v = embed_value<KIND>(w, tokens[b], c, vocab, hidden);
  h[(size_t)b * hidden + c] = v;
  if (ssq_out != nullptr) {   // sum of squares per 16 entries, for a following RMSNorm
    const float s16 = group16_sum(v * v);
    if ((c & 15) == 0) ssq_out[(size_t)b * (hidden / 16) + (c >> 4)] = s16;
  }
}

// ------------------------------------------------------------------ argmax
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  // numpy semantics: the first NaN wins, otherwise the first maximum
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ x, int n,
                                                      int64_t stride, int32_t* __restrict__ idx,
                                                      float* __restrict__ max_val) {
  __shared__ float sv[16];
  __shared__ int si[16];
  const int b = blockIdx.x;
  const float* row = x + (size_t)b * stride;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = threadIdx.x; i < n; i += 1024) {
    const float v = row[i];
    if (better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = bv;
    si[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 16; ++w)
      if (better(sv[w], si[w], bv, bi)) {
        bv = sv[w];
        bi = si[w];
      }
    idx[b] = bi;
    if (max_val) max_val[b] = bv;
  }
}

// ------------------------------------------------------------------ decode bookkeeping
// keys: [batch][n_slots] order-preserving argmax keys (one per lm_head tile-row). With s_tok,
// token b is also left in s_tok[b] (batch <= kAdvanceEmbedMaxBatch) for the whole workgroup.
// Without step (a workgroup of one row of several), the history and the step counter are
// left to decode_step_kernel.
constexpr int kAdvanceEmbedMaxBatch = 64;

// max(k, k of the lane DPP control CTRL names), 64-bit (the two halves move together)
template <int CTRL>
__device__ __forceinline__ unsigned long long key_max_dpp(unsigned long long k) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)k, CTRL, 0xf, 0xf, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(k >> 32), CTRL, 0xf,
                                                            0xf, false);
  const unsigned long long o = ((unsigned long long)hi << 32) | lo;
  return o > k ? o : k;
}
// max of a (lo, hi) pair the permlane swaps returned against the other
__device__ __forceinline__ unsigned long long key_max_pair(uint32_t lo0, uint32_t hi0, uint32_t lo1,
                                                          uint32_t hi1) {
  const unsigned long long a = ((unsigned long long)hi0 << 32) | lo0;
  const unsigned long long b = ((unsigned long long)hi1 << 32) | lo1;
  return a > b ? a : b;
}
// The wave's largest key, in every lane, with no LDS round trip: DPP inside each row of 16
// lanes, then the permlane swaps across rows and halves.
__device__ __forceinline__ unsigned long long wave_key_max(unsigned long long k) {
  k = key_max_dpp<kDppXor1>(k);
  k = key_max_dpp<kDppXor2>(k);
  k = key_max_dpp<kDppHalfMirror>(k);
  k = key_max_dpp<kDppRor8>(k);
  const uint32_t lo = (uint32_t)k, hi = (uint32_t)(k >> 32);
  const auto l16 = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
  const auto h16 = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
  k = key_max_pair(l16[0], h16[0], l16[1], h16[1]);
  const uint32_t lo2 = (uint32_t)k, hi2 = (uint32_t)(k >> 32);
  const auto l32 = __builtin_amdgcn_permlane32_swap(lo2, lo2, false, false);
  const auto h32 = __builtin_amdgcn_permlane32_swap(hi2, hi2, false, false);
  return key_max_pair(l32[0], h32[0], l32[1], h32[1]);
}

__device__ __forceinline__ void decode_advance_body(
    const unsigned long long* __restrict__ keys, int n_slots, int32_t* __restrict__ tokens,
    int32_t* __restrict__ pos, int32_t* __restrict__ lens, int32_t* __restrict__ history,
    int32_t* __restrict__ step, int history_len, int batch, int* s_tok) {
  // Rows are taken `groups` at a time, `wpr` waves per row; each lane keeps up to kKeyLoads
  // key loads in flight (a 100352-row head at batch 8: two round trips per lane, not seven),
  // then the lanes and the row's waves combine (max is order-independent). The row's
  // position is loaded ahead of its keys, so no memory round trip follows the max.
  constexpr int kKeyLoads = 32;
  __shared__ unsigned long long sk[16];
  const int tid = threadIdx.x, l = tid & 63, wave = tid >> 6;
  const int n_waves = (int)(blockDim.x >> 6);
  const int wpr = batch >= n_waves ? 1 : n_waves / batch;
  const int groups = n_waves / wpr;
  const int s = step != nullptr ? step[0] : 0;
  for (int b0 = 0; b0 < batch; b0 += groups) {
    const int b = b0 + wave / wpr, sub = wave % wpr;
    const bool active = wave < groups * wpr && b < batch;
    int32_t p_old = 0;
    if (active && sub == 0 && l == 0) p_old = pos[b];
    unsigned long long k = 0ull;
    if (active) {
      const int T = wpr * 64;
      const unsigned long long* row = keys + (int64_t)b * n_slots;
      for (int i = sub * 64 + l; i < n_slots; i += kKeyLoads * T) {
        unsigned long long v[kKeyLoads];
#pragma unroll
        for (int j = 0; j < kKeyLoads; ++j) v[j] = i + j * T < n_slots ? row[i + j * T] : 0ull;
#pragma unroll
        for (int j = 0; j < kKeyLoads; ++j) k = v[j] > k ? v[j] : k;
      }
      k = wave_key_max(k);
    }
    if (l == 0) sk[wave] = k;
    __syncthreads();
    if (active && sub == 0) {   // the row's first wave combines its waves' maxima
      k = wave_key_max(l < wpr ? sk[wave + l] : 0ull);
      if (l == 0) {
        const int32_t tok = (int32_t)(0xffffffffu - (uint32_t)(k & 0xffffffffull));
        tokens[b] = tok;
        if (s_tok != nullptr) s_tok[b] = tok;
        pos[b] = p_old + 1;
        lens[b] = p_old + 2;
        if (step != nullptr && history != nullptr && s < history_len)
          history[(int64_t)s * batch + b] = tok;
      }
    }
    __syncthreads();
  }
  if (tid == 0 && step != nullptr) step[0] = s + 1;
}

__global__ __launch_bounds__(1024) void decode_advance_kernel(
    const unsigned long long* __restrict__ keys, int n_slots, int32_t* __restrict__ tokens,
    int32_t* __restrict__ pos, int32_t* __restrict__ lens, int32_t* __restrict__ history,
    int32_t* __restrict__ step, int history_len, int batch) {
  decode_advance_body(keys, n_slots, tokens, pos, lens, history, step, history_len, batch,
                      nullptr);
}

// history[step][b] = tokens[b] while step < history_len, then step += 1: the end of a greedy
// step whose rows were advanced by one workgroup each. One wave: every lane loads the
// counter before lane 0 stores it.
__global__ __launch_bounds__(64) void decode_step_kernel(const int32_t* __restrict__ tokens,
                                                         int32_t* __restrict__ history,
                                                         int32_t* __restrict__ step,
                                                         int history_len, int batch) {
  const int s = step[0];
  if (history != nullptr && s < history_len)
    for (int b = (int)threadIdx.x; b < batch; b += 64) history[(int64_t)s * batch + b] = tokens[b];
  if (threadIdx.x == 0) step[0] = s + 1;
}

// The embedding rows of s_tok[0..batch) into h / ssq_out (as embed_kernel), by all 1024
// threads of the workgroup.
template <int KIND>
__device__ __forceinline__ void embed_rows(const int* s_tok, int batch,
                                           const uint8_t* __restrict__ table, int vocab,
                                           int hidden, float* __restrict__ h,
                                           float* __restrict__ ssq_out) {
  // Four 1024-entry chunks of the [batch][hidden] rows at a time, across row boundaries:
  // every load of the chunks is issued before the first value is stored, so a group of
  // chunks costs one memory round trip (eight rows of 2560: five, against one per row and
  // chunk). A token out of range loads row 0 and stores a NaN row.
  constexpr int kChunks = 4;
  const int total = batch * hidden;
  for (int f0 = 0; f0 < total; f0 += 1024 * kChunks) {
    float v[kChunks];
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const int f = f0 + 1024 * j + (int)threadIdx.x;
      const int b = f < total ? f / hidden : 0;
      const int c = f < total ? f - b * hidden : 0;
      const int t = s_tok[b];
      const bool ok = t >= 0 && t < vocab;
      v[j] = embed_value_of<KIND>(table, ok ? t : 0, c, hidden);
      if (!ok) v[j] = __builtin_nanf("");
    }
    // h and ssq_out are [batch][hidden] and [batch][hidden / 16], so entry f is h[f] and its
    // 16-entry group ssq_out[f / 16]; hidden % 256 == 0 keeps a 16-lane group inside a row
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const int f = f0 + 1024 * j + (int)threadIdx.x;
      const bool in = f < total;
      if (in) h[f] = v[j];
      if (ssq_out != nullptr) {
        const float s16 = group16_sum(v[j] * v[j]);
        if (in && (f & 15) == 0) ssq_out[f >> 4] = s16;
      }
    }
  }
}

// The advance, then the embedding rows of the new tokens: the next step's input is ready
// when the launch ends, with no launch of its own. One workgroup for all rows.
template <int KIND>
__global__ __launch_bounds__(1024) void decode_advance_embed_kernel(
    const unsigned long long* __restrict__ keys, int n_slots, int32_t* __restrict__ tokens,
    int32_t* __restrict__ pos, int32_t* __restrict__ lens, int32_t* __restrict__ history,
    int32_t* __restrict__ step, int history_len, int batch, const uint8_t* __restrict__ table,
    int vocab, int hidden, float* __restrict__ h, float* __restrict__ ssq_out) {
  __shared__ int s_tok[kAdvanceEmbedMaxBatch];
  decode_advance_body(keys, n_slots, tokens, pos, lens, history, step, history_len, batch,
                      s_tok);
  __syncthreads();
  embed_rows<KIND>(s_tok, batch, table, vocab, hidden, h, ssq_out);
}

// The same with one workgroup per row (blockIdx.x): the row's token, position, length and
// embedding row; decode_step_kernel then writes the history and advances the step. Eight
// rows of a 6272-key head: 18.3 us from one workgroup, as many rows in parallel here.
template <int KIND>
__global__ __launch_bounds__(1024) void decode_rows_embed_kernel(
    const unsigned long long* __restrict__ keys, int n_slots, int32_t* __restrict__ tokens,
    int32_t* __restrict__ pos, int32_t* __restrict__ lens, const uint8_t* __restrict__ table,
    int vocab, int hidden, float* __restrict__ h, float* __restrict__ ssq_out) {
  __shared__ int s_tok[1];
  const int b = blockIdx.x;
  decode_advance_body(keys + (int64_t)b * n_slots, n_slots, tokens + b, pos + b, lens + b,
                      nullptr, nullptr, 0, 1, s_tok);
  __syncthreads();
  embed_rows<KIND>(s_tok, 1, table, vocab, hidden, h + (int64_t)b * hidden,
                   ssq_out != nullptr ? ssq_out + (int64_t)b * (hidden / 16) : nullptr);
}

}  // namespace q4nx

using namespace q4nx;

extern "C" {

int q4nx_rmsnorm(const void* x, int x_f32, const uint16_t* w, uint16_t* y, float* y_f32,
                 int cols, int batch, float eps, void* stream) {
  Q4NX_REQUIRE(x && w && y, Q4NX_ERR_ARG, "q4nx_rmsnorm: x, w and y are required");
  Q4NX_REQUIRE(cols > 0 && batch > 0, Q4NX_ERR_SHAPE, "q4nx_rmsnorm: cols=%d batch=%d", cols,
               batch);
  hipStream_t s = (hipStream_t)stream;
  if (x_f32)
    hipLaunchKernelGGL(rmsnorm_kernel<true>, dim3(batch), dim3(256), 0, s, x, w, y, y_f32, cols, eps);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<false>, dim3(batch), dim3(256), 0, s, x, w, y, y_f32, cols, eps);
  return check_launch("q4nx_rmsnorm");
}

int q4nx_rope(const uint16_t* x, uint16_t* y, float* y_f32, int n_heads, int head_dim, int batch,
              const int32_t* positions, const float* tab, int max_pos, void* stream) {
  Q4NX_REQUIRE(x && y && positions && tab, Q4NX_ERR_ARG,
               "q4nx_rope: x, y, positions and table are required");
  Q4NX_REQUIRE(n_heads > 0 && batch > 0 && head_dim > 0 && head_dim % 2 == 0 && max_pos > 0,
               Q4NX_ERR_SHAPE, "q4nx_rope: n_heads=%d head_dim=%d batch=%d max_pos=%d", n_heads,
               head_dim, batch, max_pos);
  const int64_t total = (int64_t)batch * n_heads * (head_dim / 2);
  Q4NX_REQUIRE(total < ((int64_t)1 << 31) - 256, Q4NX_ERR_SHAPE,
               "q4nx_rope: %lld rotation pairs exceed one launch", (long long)total);
  hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, x, y, y_f32, n_heads, head_dim, batch, positions, tab,
                     max_pos);
  return check_launch("q4nx_rope");
}

int q4nx_swiglu(const void* g, const void* u, int in_f32, uint16_t* y, float* y_f32, int n,
                int batch, void* stream) {
  Q4NX_REQUIRE(g && u && y, Q4NX_ERR_ARG, "q4nx_swiglu: g, u and y are required");
  Q4NX_REQUIRE(n > 0 && batch > 0, Q4NX_ERR_SHAPE, "q4nx_swiglu: n=%d batch=%d", n, batch);
  const int64_t total = (int64_t)n * batch;
  dim3 grid((unsigned)((total + 255) / 256));
  if (in_f32)
    hipLaunchKernelGGL(swiglu_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, g, u, y, y_f32, total);
  else
    hipLaunchKernelGGL(swiglu_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, g, u, y, y_f32, total);
  return check_launch("q4nx_swiglu");
}

int q4nx_round_bf16(const float* x, uint16_t* y, int64_t n, void* stream) {
  Q4NX_REQUIRE(x && y, Q4NX_ERR_ARG, "q4nx_round_bf16: x and y are required");
  Q4NX_REQUIRE(n >= 0 && n < ((int64_t)1 << 40), Q4NX_ERR_SHAPE, "q4nx_round_bf16: n=%lld",
               (long long)n);
  if (n == 0) return Q4NX_OK;
  hipLaunchKernelGGL(round_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, x, y, n);
  return check_launch("q4nx_round_bf16");
}

int q4nx_embed(int kind, const void* table, const int32_t* tokens, float* h, float* ssq_out,
               int vocab, int hidden, int batch, void* stream) {
  const char* what = "q4nx_embed";
  Q4NX_REQUIRE(kind == Q4NX_KIND_Q4 || kind == Q4NX_KIND_Q8 || kind == Q4NX_KIND_BF16,
               Q4NX_ERR_ARG, "%s: kind must be Q4NX_KIND_Q4, _Q8 or _BF16, got %d", what, kind);
  Q4NX_REQUIRE(table && tokens && h, Q4NX_ERR_ARG, "%s: table, tokens and h are required", what);
  Q4NX_REQUIRE(vocab > 0 && (kind == Q4NX_KIND_BF16 || vocab % 32 == 0) && hidden > 0 &&
                   hidden % 256 == 0 && batch > 0,
               Q4NX_ERR_SHAPE, "%s: vocab=%d hidden=%d batch=%d", what, vocab, hidden, batch);
  const dim3 grid(hidden / 256, batch);
  const uint8_t* w = (const uint8_t*)table;
  hipStream_t s = (hipStream_t)stream;
  if (kind == Q4NX_KIND_BF16)
    hipLaunchKernelGGL(embed_kernel<Q4NX_KIND_BF16>, grid, dim3(256), 0, s, w, tokens, h, ssq_out, vocab, hidden);
  else if (kind == Q4NX_KIND_Q8)
    hipLaunchKernelGGL(embed_kernel<Q4NX_KIND_Q8>, grid, dim3(256), 0, s, w, tokens, h, ssq_out, vocab, hidden);
  else
    hipLaunchKernelGGL(embed_kernel<Q4NX_KIND_Q4>, grid, dim3(256), 0, s, w, tokens, h, ssq_out, vocab, hidden);
  return check_launch(what);
}

int q4nx_argmax(const float* logits, int n, int batch, int64_t stride, int32_t* idx,
                float* max_val, void* stream) {
  Q4NX_REQUIRE(logits && idx, Q4NX_ERR_ARG, "q4nx_argmax: logits and idx are required");
  Q4NX_REQUIRE(n > 0 && batch > 0 && stride >= n, Q4NX_ERR_SHAPE,
               "q4nx_argmax: n=%d batch=%d stride=%lld", n, batch, (long long)stride);
  hipLaunchKernelGGL(argmax_kernel, dim3(batch), dim3(1024), 0, (hipStream_t)stream, logits, n,
                     stride, idx, max_val);
  return check_launch("q4nx_argmax");
}

int q4nx_decode_advance(const uint64_t* keys, int n_slots, int32_t* tokens, int32_t* pos,
                        int32_t* lens, int32_t* history, int32_t* step, int history_len,
                        int batch, void* stream) {
  Q4NX_REQUIRE(keys && tokens && pos && lens && step, Q4NX_ERR_ARG,
               "q4nx_decode_advance: keys, tokens, pos, lens and step are required");
  Q4NX_REQUIRE(batch >= 1 && n_slots >= 1, Q4NX_ERR_SHAPE,
               "q4nx_decode_advance: batch=%d n_slots=%d", batch, n_slots);
  hipLaunchKernelGGL(decode_advance_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream,
                     (const unsigned long long*)keys, n_slots, tokens, pos, lens, history, step,
                     history_len, batch);
  return check_launch("q4nx_decode_advance");
}

int q4nx_decode_advance_embed(const uint64_t* keys, int n_slots, int32_t* tokens, int32_t* pos,
                              int32_t* lens, int32_t* history, int32_t* step, int history_len,
                              int batch, int kind, const void* table, int vocab, int hidden,
                              float* h, float* ssq_out, void* stream) {
  const char* what = "q4nx_decode_advance_embed";
  Q4NX_REQUIRE(keys && tokens && pos && lens && step && table && h, Q4NX_ERR_ARG,
               "%s: keys, tokens, pos, lens, step, table and h are required", what);
  Q4NX_REQUIRE(kind == Q4NX_KIND_Q4 || kind == Q4NX_KIND_Q8 || kind == Q4NX_KIND_BF16,
               Q4NX_ERR_ARG, "%s: kind must be Q4NX_KIND_Q4, _Q8 or _BF16, got %d", what, kind);
  Q4NX_REQUIRE(batch >= 1 && batch <= kAdvanceEmbedMaxBatch && n_slots >= 1, Q4NX_ERR_SHAPE,
               "%s: batch=%d (1..%d) n_slots=%d", what, batch, kAdvanceEmbedMaxBatch, n_slots);
  Q4NX_REQUIRE(vocab > 0 && (kind == Q4NX_KIND_BF16 || vocab % 32 == 0) && hidden > 0 &&
                   hidden % 256 == 0 && (int64_t)batch * hidden < ((int64_t)1 << 30),
               Q4NX_ERR_SHAPE, "%s: vocab=%d hidden=%d", what, vocab, hidden);
  const auto* k = (const unsigned long long*)keys;
  const uint8_t* w = (const uint8_t*)table;
  hipStream_t s = (hipStream_t)stream;
  if (batch > 1) {   // a workgroup per row, then the history and the step counter
    if (kind == Q4NX_KIND_BF16)
      hipLaunchKernelGGL(decode_rows_embed_kernel<Q4NX_KIND_BF16>, dim3(batch), dim3(1024), 0,
                         s, k, n_slots, tokens, pos, lens, w, vocab, hidden, h, ssq_out);
    else if (kind == Q4NX_KIND_Q8)
      hipLaunchKernelGGL(decode_rows_embed_kernel<Q4NX_KIND_Q8>, dim3(batch), dim3(1024), 0, s,
                         k, n_slots, tokens, pos, lens, w, vocab, hidden, h, ssq_out);
    else
      hipLaunchKernelGGL(decode_rows_embed_kernel<Q4NX_KIND_Q4>, dim3(batch), dim3(1024), 0, s,
                         k, n_slots, tokens, pos, lens, w, vocab, hidden, h, ssq_out);
    hipLaunchKernelGGL(decode_step_kernel, dim3(1), dim3(64), 0, s, tokens, history, step,
                       history_len, batch);
    return check_launch(what);
  }
  if (kind == Q4NX_KIND_BF16)
    hipLaunchKernelGGL(decode_advance_embed_kernel<Q4NX_KIND_BF16>, dim3(1), dim3(1024), 0, s, k,
                       n_slots, tokens, pos, lens, history, step, history_len, batch, w, vocab,
                       hidden, h, ssq_out);
  else if (kind == Q4NX_KIND_Q8)
    hipLaunchKernelGGL(decode_advance_embed_kernel<Q4NX_KIND_Q8>, dim3(1), dim3(1024), 0, s, k,
                       n_slots, tokens, pos, lens, history, step, history_len, batch, w, vocab,
                       hidden, h, ssq_out);
  else
    hipLaunchKernelGGL(decode_advance_embed_kernel<Q4NX_KIND_Q4>, dim3(1), dim3(1024), 0, s, k,
                       n_slots, tokens, pos, lens, history, step, history_len, batch, w, vocab,
                       hidden, h, ssq_out);
  return check_launch(what);
}

}  // extern "C"
