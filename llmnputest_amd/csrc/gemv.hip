// q4nx GEMV for gfx950: y = W x with W read directly in the q4nx tile layout.
//
// Replaces the per-core AIE kernels designs/granite_gemv/granite_gemv.h:109-300 (q4,
// Q4_1) and designs/lm_head/lm_head.h:53-113 (q8) with one launch over the whole tensor,
// plus the fused epilogues of granite_qkv_rope.h:30-71 and granite_swiglu_f32.h:27-51.
//
// Work decomposition
//   One workgroup owns one output *group*: the tile-rows an epilogue needs together --
//   one tile-row for a plain GEMV, the two tile-rows of an attention head for
//   [q,k,v,RoPE] (RoPE pairs dim i with i+32), or the same tile-row of gate and up for
//   SwiGLU. Each wave of the workgroup owns TPW consecutive K-tiles of one tile-row and
//   the waves combine through LDS once, in a fixed order. When a launch has too few
//   groups to fill the GPU (the 2560-row projections, the attention heads), K is also
//   split over `ksplit` workgroups per group: each publishes its partial sums with
//   system-scope stores, and the last to arrive adds the parts in part order and runs the
//   epilogue, so results stay bit-reproducible.
//
// Data path (decode is HBM-bound: every byte is read once, straight into registers)
//   Four lanes own one (row-block, 32-K group) "unit" of a tile: lane l reads the 64
//   (q4) or 128 (q8) contiguous bytes at unit l/4, quarter l%4, i.e. 8 K x 16 rows. All
//   of a wave's tile loads are issued before any arithmetic; each tile is consumed as
//   soon as its registers arrive. The 4-lane partial sums are reduced with two xor
//   shuffles, then the per-group scale and minimum are applied to the lane's 4 rows.
//
// Arithmetic (exact inputs, fp32 accumulate)
//   x is converted to fp16 with one power-of-two scale per wave, chosen from max|x| over
//   the wave's K range (bf16 values convert exactly in fp16's normal range). A 4-bit code
//   c placed in bits 4-7 of an fp16 is the subnormal c * 2^-20, exactly, and
//   v_dot2_f32_f16 multiplies two of them by two x values with exact products. The low
//   nibbles of a weight dword are shifted up and the high ones masked in place (two ops
//   per dword, shared by its four bytes), then a v_perm_b32 builds [c(k0), 0, c(k1), 0]
//   for one row and two k: one permute and one dot2 per 2 weights. (v_dot2's adder keeps
//   fewer bits when a subnormal operand has leading zeros; codes in bits 0-3 cost about
//   six bits against the largest term on heavy-tailed activations, bits 4-7 two at most.)
//   q8 codes are biased by 128 (xor 0x80) into 1..255 and the bias is removed with
//   128 * sum(x). The Q4_1 minimum factors out of the K sum (granite_gemv.h:19-29):
//   y_r += d_r * sum(c x) + m_r * sum(x) per 32-K group.

#include <atomic>
#include "common.h"
#include "gemm.h"
#include "gemv1.h"
#include "policy.h"

#include <climits>

namespace q4nx {

enum GemvOp : int { OP_PLAIN = 0, OP_QKV = 1, OP_GATEUP = 2 };

struct GemvArgs {
  const uint8_t* w[3];
  int n_tr[3];
  int op;
  int G;             // tile-rows per group (1 or 2)
  int grp_q, grp_k;  // QKV: groups [0,grp_q) are q heads, [grp_q,grp_q+grp_k) k heads, rest v
  int k_t, batch;
  // input: bf16 x, or fp32 residual h normalised with norm_w in the prologue
  const uint16_t* x;
  const float* hres;
  int64_t x_stride;
  const uint16_t* norm_w;
  float eps;
  const float* ssq_in;   // optional [batch][K/16] sums of squares of x, per 16 entries
  uint16_t* xn_out;
  // plain
  float* y;
  int64_t y_stride;
  const float* residual;
  float* ssq_out;        // optional [batch][N/16] sums of squares of y per 16-row block
  // qkv
  uint16_t* q_out;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t kv_b_stride, kv_h_stride;
  const int32_t* pos;
  const float* rope_tab;
  int max_pos;
  int n_q_heads, n_kv_heads;
  float* raw_out;
  // gate/up
  uint16_t* h_out;
  int64_t h_stride;
  // plain: optional argmax keys, uint64 [batch][N/16] (order-preserving (value, -row) per
  // 16-row block)
  unsigned long long* argmax_keys;
  // split K: partial sums [group][part][batch][G*32] fp32 and one arrival counter per group
  int ksplit;
  float* part;
  uint32_t part_bytes;
  unsigned* counters;
};

constexpr int kMaxWaves = 16;

// v_perm selector for result bytes [s1.b_i, 0, s0.b_i, 0]
__device__ __forceinline__ constexpr uint32_t sel_byte(int i) {
  return 0x0c040c00u + (uint32_t)i * 0x00010001u;
}

// 16 values summed over lane bits 1 and 0 (xor 2, then xor 1); lane q keeps 4q..4q+3.
__device__ __forceinline__ void transpose_reduce4(const float (&v)[16], float (&o)[4], int lane) {
  float t8[8];
  const bool up1 = (lane & 2) != 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float keep = up1 ? v[i + 8] : v[i];
    const float send = up1 ? v[i] : v[i + 8];
    t8[i] = keep + dpp<kDppXor2>(send);
  }
  const bool up0 = (lane & 1) != 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float keep = up0 ? t8[i + 4] : t8[i];
    const float send = up0 ? t8[i] : t8[i + 4];
    o[i] = keep + dpp<kDppXor1>(send);
  }
}

// One work item (an output group, or one K part of it) of a GEMV launch. Returns true when
// this workgroup ran the epilogue (for a split group, only the last part to arrive does).
template <int KIND, int B, int TPW>
__device__ __forceinline__ bool gemv_body(const GemvArgs& a, const int blk) {
  constexpr int TB = KIND == 4 ? kQ4TileBytes : kQ8TileBytes;
  constexpr int NCH = KIND == 4 ? 4 : 8;              // 16-byte chunks per lane per tile
  constexpr int CODE_OFF = KIND == 4 ? 1024 : 512;    // start of the codes in a tile
  __shared__ float sred[kMaxWaves][B][32];
  __shared__ float sgrp[B][64];
  __shared__ float snorm[kMaxWaves][B];
  __shared__ unsigned long long skey[B][2];
  __shared__ int s_last;

  // wave-uniform values live in scalar registers: the weight pointer below must be known
  // without a memory round trip, or every wave waits for it before streaming its tiles
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int W = blockDim.x >> 6;
  const int WM = W / a.G;             // waves per member tile-row
  const int member = wave / WM, chunk = wave % WM;
  const int ks = a.ksplit;
  const int group = blk / ks, kpart = blk - group * ks;
  const int kt_lo = kpart * a.k_t / ks, kt_hi = (kpart + 1) * a.k_t / ks;

  int seg, tr;
  if (a.op == OP_PLAIN) {
    seg = 0;
    tr = group;
  } else if (a.op == OP_GATEUP) {
    seg = member;
    tr = group;
  } else {
    int hg;
    if (group < a.grp_q) {
      seg = 0;
      hg = group;
    } else if (group < a.grp_q + a.grp_k) {
      seg = 1;
      hg = group - a.grp_q;
    } else {
      seg = 2;
      hg = group - a.grp_q - a.grp_k;
    }
    tr = 2 * hg + member;
  }
  const int K = a.k_t * kTileK;
  const int kt0 = kt_lo + chunk * TPW;
  const int ntw = max(0, min(TPW, kt_hi - kt0));    // tiles this wave really owns

  // lane roles: q = lane bits 0-1 (8-K quarter), kb = bits 2-4, rb = bit 5
  const int q = lane & 3, kb = (lane >> 2) & 7, rb = lane >> 5;
  const int kx = kb * kGroup + q * 8;                // first K of this lane inside a tile
  const bool norm = a.norm_w != nullptr;

  // ---- 1. activations. Every load is unconditional, from a valid address (clamped row,
  //         or the weights as a stand-in), so nothing waits before the weight stream is
  //         issued; rows past the batch are masked where the values are used.
  uint4 ar[B][TPW][2];    // raw activation bytes: 8 bf16 x (first 16 B) or 8 fp32 h (32 B)
  uint4 nw[TPW];
  const bool pre_ssq = norm && a.ssq_in != nullptr;
  const int n_ss = K / kSsqRows;
  constexpr int kSsqLoads = 2;   // float4s per lane: K / 16 <= 512 partial sums per row
  float4 sq[B][kSsqLoads];
  constexpr int kSsqIt = 3;
  float4 hs[B][kSsqIt];
  const bool split_norm = norm && ks > 1 && !pre_ssq;
  float ep_res = 0.f;   // epilogue prefetches (see the end of this block)
  int ep_pos = 0;
  {
    const void* xbase = norm ? (const void*)a.hres : (const void*)a.x;
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int kt = min(kt0 + t, kt_hi - 1);
      const int k = kt * kTileK + kx;
      nw[t] = *(const uint4*)(norm ? (const void*)(a.norm_w + k) : (const void*)a.w[0]);
#pragma unroll
      for (int b = 0; b < B; ++b) {
        const int bb = min(b, a.batch - 1);
        const size_t off = ((size_t)bb * a.x_stride + k) * (norm ? 4 : 2);
        const uint4* src = (const uint4*)((const uint8_t*)xbase + off);
        ar[b][t][0] = src[0];
        ar[b][t][1] = src[norm ? 1 : 0];
      }
    }
    // RMSNorm sums of squares handed over by the producer of x: K/16 partials per row,
    // every wave sums them itself (the order of ssq_lane_sum) and needs no other wave
    if (pre_ssq) {
#pragma unroll
      for (int b = 0; b < B; ++b)
        ssq_load<kSsqLoads>(a.ssq_in + (size_t)min(b, a.batch - 1) * n_ss, lane, n_ss, sq[b]);
    }
    // with K split and no partials given, this workgroup's tiles see only part of the row:
    // the sum of squares reads the whole row (strided over all threads; three float4 per
    // thread cover K <= 12 * blockDim, a remainder loop the rest)
    if (split_norm) {
#pragma unroll
      for (int it = 0; it < kSsqIt; ++it) {
        const int i = min(tid + it * (int)blockDim.x, K / 4 - 1);
#pragma unroll
        for (int b = 0; b < B; ++b)
          hs[b][it] = *(const float4*)(a.hres + (size_t)min(b, a.batch - 1) * a.x_stride + 4 * i);
      }
    }
    // the epilogue's own inputs for this thread's first output (batch row tid / 32, row
    // tid % 32 of the group): the residual (plain) or the sequence position (q/k/v), in
    // flight with the activations instead of a memory round trip after the reduction.
    // Unconditional loads, from the weights when the launch has no such input.
    const int eb = min(tid >> 5, a.batch - 1), er = tid & 31;
    const bool res = a.op == OP_PLAIN && a.residual != nullptr;
    const float* rp = res ? a.residual + (int64_t)eb * a.y_stride + (int64_t)tr * 32 + er
                          : (const float*)a.w[0];
    ep_res = *rp;
    ep_pos = *(a.op == OP_QKV ? a.pos + eb : (const int32_t*)a.w[0]);
  }

  // ---- 2. weights and per-group metadata of every tile of this wave
  uint4 wq[TPW][NCH];
  uint2 md[TPW], mm[TPW];
  {
    const uint8_t* wseg = seg == 0 ? a.w[0] : seg == 1 ? a.w[1] : a.w[2];
    const uint8_t* rowp = wseg + (size_t)tr * a.k_t * TB;
    const int g = kb * 32 + rb * 16 + q * 4;          // meta index of this lane's 4 rows
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const uint8_t* tile = rowp + (size_t)min(kt0 + t, kt_hi - 1) * TB;
      const uint4* src = (const uint4*)(tile + CODE_OFF + lane * (NCH * 16));
#pragma unroll
      for (int c = 0; c < NCH; ++c) wq[t][c] = src[c];
      md[t] = *(const uint2*)(tile + 2 * g);
      mm[t] = make_uint2(0, 0);
      if (KIND == 4) mm[t] = *(const uint2*)(tile + kMetaBytes + 2 * g);
    }
  }

  // the activations are used from here on (their waits come after the weight stream)
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    pin(nw[t]);
#pragma unroll
    for (int b = 0; b < B; ++b) {
      pin(ar[b][t][0]);
      pin(ar[b][t][1]);
    }
  }
  if (split_norm) {
#pragma unroll
    for (int it = 0; it < kSsqIt; ++it)
#pragma unroll
      for (int b = 0; b < B; ++b) pin(hs[b][it]);
  }
  // RoPE cos/sin of the first epilogue output, now that its position is here (the wait for
  // it is the activations' wait); they arrive while the tiles are reduced
  float ep_c, ep_s;
  {
    const bool rope = a.op == OP_QKV && ep_pos >= 0 && ep_pos < a.max_pos;
    const float* tb = rope ? a.rope_tab + (int64_t)ep_pos * 64 + (tid & 31) : (const float*)a.w[0];
    ep_c = tb[0];
    ep_s = tb[32];
  }
  if (pre_ssq) {
#pragma unroll
    for (int b = 0; b < B; ++b)
#pragma unroll
      for (int j = 0; j < kSsqLoads; ++j) pin(sq[b][j]);
  }

  uint4 xr[B][TPW];       // 8 bf16 per lane per tile
  float hx[B][TPW][8];    // fp32 residual values (RMSNorm prologue only)
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const bool live = b < a.batch;
      const uint32_t r[8] = {ar[b][t][0].x, ar[b][t][0].y, ar[b][t][0].z, ar[b][t][0].w,
                             ar[b][t][1].x, ar[b][t][1].y, ar[b][t][1].z, ar[b][t][1].w};
#pragma unroll
      for (int i = 0; i < 8; ++i) hx[b][t][i] = (norm && live) ? __uint_as_float(r[i]) : 0.f;
      xr[b][t] = (!norm && live) ? ar[b][t][0] : make_uint4(0, 0, 0, 0);
    }

  // ---- 3. RMSNorm prologue: sum of squares over K from member-0 waves, row-block-0 lanes
  //         (or from the whole-row pass above when K is split)
  float ssq[B];
#pragma unroll
  for (int b = 0; b < B; ++b) {
    ssq[b] = 0.f;
    if (split_norm) {
#pragma unroll
      for (int it = 0; it < kSsqIt; ++it) {
        const float4 h = hs[b][it];
        const bool live = b < a.batch && tid + it * (int)blockDim.x < K / 4;
        if (live)
          ssq[b] = fmaf(h.x, h.x, fmaf(h.y, h.y, fmaf(h.z, h.z, fmaf(h.w, h.w, ssq[b]))));
      }
      if (b < a.batch)
        for (int i = tid + kSsqIt * (int)blockDim.x; i < K / 4; i += blockDim.x) {
          const float* hp = a.hres + b * a.x_stride + 4 * i;
          const float4 h = *(const float4*)hp;
          ssq[b] = fmaf(h.x, h.x, fmaf(h.y, h.y, fmaf(h.z, h.z, fmaf(h.w, h.w, ssq[b]))));
        }
    }
  }
  float inv_rms[B];
  if (pre_ssq) {
#pragma unroll
    for (int b = 0; b < B; ++b)
      inv_rms[b] = rms_inv(wave_sum(ssq_lane_sum<kSsqLoads>(sq[b], lane, n_ss)), K, a.eps);
  } else if (norm) {
#pragma unroll
    for (int b = 0; b < B; ++b) {
      float s = ssq[b];
      if (ks == 1) {
#pragma unroll
        for (int t = 0; t < TPW; ++t)
          if (t < ntw && rb == 0 && member == 0) {
#pragma unroll
            for (int i = 0; i < 8; ++i) s = fmaf(hx[b][t][i], hx[b][t][i], s);
          }
      }
      s = wave_sum(s);
      if (lane == 0) snorm[wave][b] = s;
    }
    __syncthreads();
    const int n_sum_waves = ks == 1 ? WM : W;
#pragma unroll
    for (int b = 0; b < B; ++b) {
      float v[kMaxWaves];   // all loads first, then the sum in wave order
#pragma unroll
      for (int w = 0; w < kMaxWaves; ++w) v[w] = snorm[w][b];
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < kMaxWaves; ++w)
        if (w < n_sum_waves) s += v[w];
      inv_rms[b] = rms_inv(s, K, a.eps);
    }
  }
  if (norm) {
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const float inv = inv_rms[b];
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const uint32_t wv[4] = {nw[t].x, nw[t].y, nw[t].z, nw[t].w};
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          o[i] = pack_bf16x2((hx[b][t][2 * i] * inv) * bf16lo(wv[i]),
                             (hx[b][t][2 * i + 1] * inv) * bf16hi(wv[i]));
        xr[b][t] = b < a.batch ? make_uint4(o[0], o[1], o[2], o[3]) : make_uint4(0, 0, 0, 0);
        if (a.xn_out != nullptr && group == 0 && member == 0 && rb == 0 && t < ntw &&
            b < a.batch)
          *(uint4*)(a.xn_out + b * a.x_stride + (kt0 + t) * kTileK + kx) = xr[b][t];
      }
    }
  }

  // ---- 4. fp16 conversion with one power-of-two scale per wave and batch row
  uint32_t xp[B][TPW][4];
  int xexp[B];
#pragma unroll
  for (int b = 0; b < B; ++b) {
    float m = 0.f;
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      if (t < ntw) {
        const uint32_t v[4] = {xr[b][t].x, xr[b][t].y, xr[b][t].z, xr[b][t].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) m = fmaxf(m, fmaxf(fabsf(bf16lo(v[i])), fabsf(bf16hi(v[i]))));
      }
    }
    m = wave_max(m);
    int e = 0;
    if (m > 0.f && m <= 3.0e38f) {
      (void)frexpf(m, &e);  // m < 2^e
      e -= 15;              // scaled max < 2^15 < fp16 max
      e = e < -120 ? -120 : e;
    }
    xexp[b] = e;
    const float s = ldexpf(1.0f, -e);
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const uint32_t v[4] = {xr[b][t].x, xr[b][t].y, xr[b][t].z, xr[b][t].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        half2_t h;
        h.x = (_Float16)(bf16lo(v[i]) * s);
        h.y = (_Float16)(bf16hi(v[i]) * s);
        xp[b][t][i] = h2_bits(h);
      }
    }
  }

  // ---- 5. tiles, in arrival order
  constexpr uint32_t kOne2 = 0x3C003C00u;  // fp16 (1, 1)
  float acc[B][4];
#pragma unroll
  for (int b = 0; b < B; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[b][i] = 0.f;

#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    if (t >= ntw) continue;
    if (KIND == 4) {
      // Both nibbles of a byte are moved to its top half (bits 4-7) before the byte
      // permutes, so each code enters v_dot2 as the fp16 subnormal c * 2^-20. The dot2
      // adder keeps fewer bits the more leading zeros a subnormal operand has (measured on
      // gfx950: codes in bits 0-3 lose about 6 bits against the largest term), so the codes
      // sit as high in the mantissa as the byte permutes allow.
      float pv[B][16], X[B];   // pv[b][r]: row r of the lane's 16, over its 8 K
#pragma unroll
      for (int b = 0; b < B; ++b) {
        X[b] = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) pv[b][i] = 0.f;
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint4 w = wq[t][c];
        const uint32_t Lx = (w.x << 4) & 0xF0F0F0F0u, Ly = (w.y << 4) & 0xF0F0F0F0u;
        const uint32_t Lz = (w.z << 4) & 0xF0F0F0F0u, Lw = (w.w << 4) & 0xF0F0F0F0u;
        const uint32_t Hx = w.x & 0xF0F0F0F0u, Hy = w.y & 0xF0F0F0F0u;
        const uint32_t Hz = w.z & 0xF0F0F0F0u, Hw = w.w & 0xF0F0F0F0u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t o0 = perm(Lz, Lx, sel_byte(i));        // row 2i     (low nibbles)
          const uint32_t o1 = perm(Hz, Hx, sel_byte(i));        // row 2i + 1 (high nibbles)
          const uint32_t o2 = perm(Lw, Ly, sel_byte(i));        // rows 8..15
          const uint32_t o3 = perm(Hw, Hy, sel_byte(i));
#pragma unroll
          for (int b = 0; b < B; ++b) {
            const uint32_t xpc = xp[b][t][c];
            pv[b][2 * i] = dot2(o0, xpc, pv[b][2 * i]);
            pv[b][2 * i + 1] = dot2(o1, xpc, pv[b][2 * i + 1]);
            pv[b][8 + 2 * i] = dot2(o2, xpc, pv[b][8 + 2 * i]);
            pv[b][8 + 2 * i + 1] = dot2(o3, xpc, pv[b][8 + 2 * i + 1]);
          }
        }
#pragma unroll
        for (int b = 0; b < B; ++b) X[b] = dot2(xp[b][t][c], kOne2, X[b]);
      }
#pragma unroll
      for (int b = 0; b < B; ++b) {
        float r4[4];   // rows 4q .. 4q+3, summed over the 32 K of the group
        transpose_reduce4(pv[b], r4, lane);
        float Xs = X[b];
        Xs += dpp<kDppXor1>(Xs);
        Xs += dpp<kDppXor2>(Xs);
        constexpr float kC = 1048576.0f;   // undo the 2^-20 of the codes
        acc[b][0] += fmaf(bf16lo(md[t].x), r4[0] * kC, bf16lo(mm[t].x) * Xs);
        acc[b][1] += fmaf(bf16hi(md[t].x), r4[1] * kC, bf16hi(mm[t].x) * Xs);
        acc[b][2] += fmaf(bf16lo(md[t].y), r4[2] * kC, bf16lo(mm[t].y) * Xs);
        acc[b][3] += fmaf(bf16hi(md[t].y), r4[3] * kC, bf16hi(mm[t].y) * Xs);
      }
    } else {
#pragma unroll
      for (int b = 0; b < B; ++b) {
        float v[16], X = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = 0.f;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const uint4 A = wq[t][2 * p], Bv = wq[t][2 * p + 1];
          const uint32_t av[4] = {A.x ^ 0x80808080u, A.y ^ 0x80808080u, A.z ^ 0x80808080u,
                                  A.w ^ 0x80808080u};
          const uint32_t bv[4] = {Bv.x ^ 0x80808080u, Bv.y ^ 0x80808080u, Bv.z ^ 0x80808080u,
                                  Bv.w ^ 0x80808080u};
          const uint32_t xpc = xp[b][t][p];
#pragma unroll
          for (int qd = 0; qd < 4; ++qd)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              v[4 * qd + i] = dot2(perm(bv[qd], av[qd], sel_byte(i)), xpc, v[4 * qd + i]);
          X = dot2(xpc, kOne2, X);
        }
        float r4[4];
        transpose_reduce4(v, r4, lane);
        X += dpp<kDppXor1>(X);
        X += dpp<kDppXor2>(X);
        const float bias = 128.0f * X;
        acc[b][0] += bf16lo(md[t].x) * fmaf(r4[0], 16777216.0f, -bias);
        acc[b][1] += bf16hi(md[t].x) * fmaf(r4[1], 16777216.0f, -bias);
        acc[b][2] += bf16lo(md[t].y) * fmaf(r4[2], 16777216.0f, -bias);
        acc[b][3] += bf16hi(md[t].y) * fmaf(r4[3], 16777216.0f, -bias);
      }
    }
  }

  // ---- 6. sum over the 8 groups of K (lane bits 2..4), undo the activation scale
#pragma unroll
  for (int b = 0; b < B; ++b) {
    const float sc = ldexpf(1.0f, xexp[b]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = acc[b][i];
      v += dpp<kDppRor4>(v);      // kb 0..3 of the row of 16 (lane bits 2-3)
      v += dpp<kDppRor8>(v);
      v = xor16_sum(v);           // kb 4..7
      if ((lane & 28) == 0) sred[wave][b][rb * 16 + q * 4 + i] = v * sc;
    }
  }
  __syncthreads();

  // ---- 7. waves of one member tile-row, in order
  for (int e = tid; e < a.G * B * 32; e += blockDim.x) {
    const int m = e / (B * 32), rest = e % (B * 32);
    const int b = rest >> 5, r = rest & 31;
    // every wave's value read at once (not one LDS round trip per wave), then added in
    // wave order
    float v[kMaxWaves];
#pragma unroll
    for (int c = 0; c < kMaxWaves; ++c) v[c] = sred[min(m * WM + c, kMaxWaves - 1)][b][r];
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < kMaxWaves; ++c)
      if (c < WM) s += v[c];
    sgrp[b][m * 32 + r] = s;
  }
  // a plain launch of one tile-row per group, K unsplit, reads each group sum back in the
  // thread that wrote it (the same e = tid + i * blockDim mapping below): no barrier
  if (!(a.op == OP_PLAIN && a.G == 1 && ks == 1)) __syncthreads();

  // ---- 7b. split K: publish this part, the last workgroup of the group adds all parts
  if (ks > 1) {
    const int gw = a.G * 32;                     // outputs per batch row of a group
    const int nrec = a.batch * gw;               // floats per part record
    const __amdgpu_buffer_rsrc_t pr = make_rsrc(a.part, a.part_bytes);
    const uint32_t rec = (uint32_t)((group * ks + kpart) * nrec) * 4u;
    for (int e = tid; e < nrec / 4; e += blockDim.x) {
      const int b = (4 * e) / gw, r = (4 * e) % gw;
      st16_sys(pr, rec + 16u * e,
               make_uint4(__float_as_uint(sgrp[b][r]), __float_as_uint(sgrp[b][r + 1]),
                          __float_as_uint(sgrp[b][r + 2]), __float_as_uint(sgrp[b][r + 3])));
    }
    wait_vm();
    __syncthreads();
    if (tid == 0) s_last = ticket(&a.counters[group], ks) ? 1 : 0;
    __syncthreads();
    if (!s_last) return false;
    const uint32_t rec0 = (uint32_t)(group * ks * nrec) * 4u;
    for (int e = tid; e < nrec / 4; e += blockDim.x) {
      uint4 v[8];
#pragma unroll
      for (int p = 0; p < 8; ++p)
        if (p < ks) v[p] = ld16_sys(pr, rec0 + (uint32_t)(p * nrec) * 4u + 16u * e);
      float4 acc4 = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int p = 0; p < 8; ++p)
        if (p < ks) {
          acc4.x += __uint_as_float(v[p].x);
          acc4.y += __uint_as_float(v[p].y);
          acc4.z += __uint_as_float(v[p].z);
          acc4.w += __uint_as_float(v[p].w);
        }
      const int b = (4 * e) / gw, r = (4 * e) % gw;
      sgrp[b][r] = acc4.x;
      sgrp[b][r + 1] = acc4.y;
      sgrp[b][r + 2] = acc4.z;
      sgrp[b][r + 3] = acc4.w;
    }
    __syncthreads();
  }

  // ---- 8. epilogue on the whole group
  if (a.op == OP_PLAIN) {
    if (a.argmax_keys != nullptr && tid < 2 * B) skey[tid >> 1][tid & 1] = 0ull;
    if (a.argmax_keys != nullptr) __syncthreads();
    for (int e0 = 0; e0 < B * 32; e0 += blockDim.x) {   // uniform trip count: 32-lane sums
      const int e = e0 + tid;
      const int b = e >> 5, r = e & 31;
      const bool live = e < B * 32 && b < a.batch;
      float v = 0.f;
      if (live) {
        const int64_t n = (int64_t)tr * 32 + r;
        v = sgrp[b][r];
        if (a.residual != nullptr) v += e0 == 0 ? ep_res : a.residual[b * a.y_stride + n];
        if (a.y != nullptr) a.y[b * a.y_stride + n] = v;
        if (a.argmax_keys != nullptr) atomicMax(&skey[b][r >> 4], argmax_key(v, (uint32_t)n));
      }
      if (a.ssq_out != nullptr) {   // sum of squares of each 16-row block's outputs
        const float sq16 = group16_sum(v * v);
        if (live && (r & 15) == 0) a.ssq_out[(int64_t)b * a.n_tr[0] * 2 + tr * 2 + (r >> 4)] = sq16;
      }
    }
    if (a.argmax_keys != nullptr) {   // one slot per (batch row, tile-row): no contention
      __syncthreads();
      if (tid < 2 * a.batch)
        a.argmax_keys[(int64_t)(tid >> 1) * a.n_tr[0] * 2 + tr * 2 + (tid & 1)] = skey[tid >> 1][tid & 1];
    }
  } else if (a.op == OP_GATEUP) {
    for (int e = tid; e < B * 32; e += blockDim.x) {
      const int b = e >> 5, r = e & 31;
      if (b < a.batch) {
        const int64_t n = (int64_t)group * 32 + r;
        const float gr = sgrp[b][r], ur = sgrp[b][32 + r];
        const float h = swiglu(round_bf16_op(gr), round_bf16_op(ur));
        a.h_out[b * a.h_stride + n] = f32_to_bf16(h);
        if (a.raw_out != nullptr) {
          const int64_t N = (int64_t)a.n_tr[0] * 32;
          a.raw_out[b * 2 * N + n] = gr;
          a.raw_out[b * 2 * N + N + n] = ur;
        }
      }
    }
  } else {  // OP_QKV: one head of q, k or v (64 rows)
    for (int e = tid; e < B * 32; e += blockDim.x) {
      const int b = e >> 5, d = e & 31;
      if (b < a.batch) {
        int hg = group, seg_off = 0;
        if (seg == 1) {
          hg = group - a.grp_q;
          seg_off = a.n_q_heads * 64;
        } else if (seg == 2) {
          hg = group - a.grp_q - a.grp_k;
          seg_off = (a.n_q_heads + a.n_kv_heads) * 64;
        }
        const float r0 = sgrp[b][d], r1 = sgrp[b][32 + d];
        if (a.raw_out != nullptr) {
          const int64_t Wd = (int64_t)(a.n_q_heads + 2 * a.n_kv_heads) * 64;
          a.raw_out[b * Wd + seg_off + hg * 64 + d] = r0;
          a.raw_out[b * Wd + seg_off + hg * 64 + 32 + d] = r1;
        }
        const float x0 = bf16_to_f32(f32_to_bf16(r0));
        const float x1 = bf16_to_f32(f32_to_bf16(r1));
        const bool first = e == tid;   // prefetched position and RoPE row
        const int p = first ? ep_pos : a.pos[b];
        const bool pos_ok = p >= 0 && p < a.max_pos;
        if (seg == 2) {
          if (pos_ok) {
            uint16_t* dst = a.v_cache + b * a.kv_b_stride + hg * a.kv_h_stride + (int64_t)p * 64;
            dst[d] = f32_to_bf16(x0);
            dst[32 + d] = f32_to_bf16(x1);
          }
        } else if (pos_ok) {
          const float c = first ? ep_c : a.rope_tab[(int64_t)p * 64 + d];
          const float sn = first ? ep_s : a.rope_tab[(int64_t)p * 64 + 32 + d];
          const float y0 = fmaf(x0, c, -(x1 * sn));
          const float y1 = fmaf(x1, c, x0 * sn);
          uint16_t* dst = (seg == 0)
                              ? a.q_out + b * (int64_t)a.n_q_heads * 64 + hg * 64
                              : a.k_cache + b * a.kv_b_stride + hg * a.kv_h_stride + (int64_t)p * 64;
          dst[d] = f32_to_bf16(y0);
          dst[32 + d] = f32_to_bf16(y1);
        }
      }
    }
  }
  return true;
}

template <int KIND, int B, int TPW>
__global__ __launch_bounds__(B <= 2 ? 1024 : 512) void gemv_kernel(GemvArgs a) {
  (void)gemv_body<KIND, B, TPW>(a, blockIdx.x);
}

// ------------------------------------------------------------------ host side

static int round_batch(int batch) { return batch <= 1 ? 1 : batch <= 2 ? 2 : batch <= 4 ? 4 : 8; }

// K-tiles per wave: the fewest that fit the group's K into the workgroup's wave budget
// (16 waves for batch <= 2, 8 above); 1, 2 or 4.
// The most K-tiles per wave the automatic plan gives a wave at this batch, raising the K split
// instead. More K-tiles per wave spill registers to scratch in the gfx950 build (four K-tiles
// at any batch; two at 2 and 8 rows, up to 1.2 KB per lane), and the spill traffic costs more
// than a K split's merge: gate/up 2560->8192 at 8 rows 202 us with four K-tiles per wave,
// 113 with two, 47 with one; at 2 rows one K-tile 17.2 us against 19.9. At 4 rows two K-tiles
// spill 12 B (q4) and measured faster than one (26.8 against 28.5 us).
static int spill_free_tpw(int batch) {
  const int b = round_batch(batch);
  return b == 1 || b == 4 ? 2 : 1;
}

// K-tiles per wave for a group of G tile-rows over k_t K-tiles, at most `cap` unless the
// policy forces a count; 0 when that does not fit one workgroup.
static int plan_tpw(int G, int k_t, int batch, const Policy& P, int cap = 4) {
  const int max_waves = round_batch(batch) <= 2 ? kMaxWaves : kMaxWaves / 2;
  const int forced = P.gemv_tpw;
  int tpw = forced > 0 ? forced : (G * k_t + max_waves - 1) / max_waves;
  tpw = tpw <= 1 ? 1 : tpw <= 2 ? 2 : tpw <= 4 ? 4 : 0;
  if (forced <= 0 && tpw > cap) tpw = 0;
  if (tpw && G * ((k_t + tpw - 1) / tpw) > max_waves) tpw = 0;
  return tpw;  // 0: K too long for one workgroup
}

// plan_tpw with the spill-free cap, else (K too long for it) any count that fits
static int plan_tpw_any(int G, int k_t, int batch, const Policy& P) {
  const int t = plan_tpw(G, k_t, batch, P, spill_free_tpw(batch));
  return t > 0 ? t : plan_tpw(G, k_t, batch, P);
}

template <int KIND, int B, int TPW>
static void launch_t(const GemvArgs& a, int blocks, int threads, hipStream_t s) {
  hipLaunchKernelGGL((gemv_kernel<KIND, B, TPW>), dim3(blocks), dim3(threads), 0, s, a);
}

template <int KIND, int B>
static void launch_b(const GemvArgs& a, int tpw, int blocks, int threads, hipStream_t s) {
  switch (tpw) {
    case 1: launch_t<KIND, B, 1>(a, blocks, threads, s); break;
    case 2: launch_t<KIND, B, 2>(a, blocks, threads, s); break;
    default: launch_t<KIND, B, 4>(a, blocks, threads, s); break;
  }
}

// Workgroups per group along K: enough groups x parts to fill the GPU (about 240
// workgroups) when a launch has few output groups of many tiles (a group of 10 tiles
// finishes sooner whole than split, the merge costs more than it saves), at least 2
// K-tiles per part, at most 8.
static int plan_ksplit(int n_groups, int G, int k_t, const Policy& P) {
  int ks;
  const int forced_ks = P.gemv_ksplit;
  if (forced_ks > 0) {
    ks = forced_ks;
  } else {
    if (n_groups >= 192 || G * k_t < 20) return 1;
    ks = (240 + n_groups - 1) / n_groups;
    ks = ks < k_t / 2 ? ks : k_t / 2;
  }
  ks = ks > 8 ? 8 : ks;
  ks = ks > k_t ? k_t : ks;
  return ks < 1 ? 1 : ks;
}

static size_t split_bytes(int n_groups, int G, int ks, int batch) {
  if (ks <= 1 || n_groups > Q4NX_WS_COUNTER_BYTES / 4) return 0;
  return (size_t)Q4NX_WS_COUNTER_BYTES + (size_t)n_groups * ks * batch * G * 32 * 4;
}

// K parts per group: plan_ksplit's choice, raised (up to 8) until one part fits in a
// workgroup at this batch's wave budget (long K with more than two rows).
static int plan_ksplit_fit(int n_groups, int G, int k_t, int batch, const Policy& P) {
  const int ks0 = plan_ksplit(n_groups, G, k_t, P);
  int ks = ks0;
  for (int cap : {spill_free_tpw(batch), 4}) {   // spill-free K-tiles per wave first
    ks = ks0;
    while (ks < 8 && ks < k_t && plan_tpw(G, (k_t + ks - 1) / ks, batch, P, cap) == 0) ++ks;
    if (plan_tpw(G, (k_t + ks - 1) / ks, batch, P, cap) > 0) break;
  }
  return ks;
}

static size_t ws_need(int n_groups, int G, int k_t, int batch, const Policy& P) {
  return split_bytes(n_groups, G, plan_ksplit_fit(n_groups, G, k_t, batch, P), batch);
}

static int launch(int kind, GemvArgs& a, int n_groups, const Policy& P, hipStream_t s,
                  const char* what, void* ws = nullptr, size_t ws_bytes = 0) {
  const int B = round_batch(a.batch);
  int ks = plan_ksplit_fit(n_groups, a.G, a.k_t, a.batch, P);
  const size_t need = split_bytes(n_groups, a.G, ks, a.batch);
  if (ks > 1 && (need == 0 || ws == nullptr || ws_bytes < need || !Q4NX_ALIGNED(ws, 256)))
    ks = 1;   // no (or too small a) workspace: one workgroup per group
  a.ksplit = ks;
  if (ks > 1) {
    a.counters = (unsigned*)ws;
    a.part = (float*)((uint8_t*)ws + Q4NX_WS_COUNTER_BYTES);
    a.part_bytes = (uint32_t)(need - Q4NX_WS_COUNTER_BYTES);
  }
  const int kpp = (a.k_t + ks - 1) / ks;   // largest part
  const int tpw = plan_tpw_any(a.G, kpp, a.batch, P);
  Q4NX_REQUIRE(tpw > 0, Q4NX_ERR_SHAPE, "%s: K=%d is longer than one workgroup covers", what,
               a.k_t * 256);
  const int wm = (kpp + tpw - 1) / tpw;
  const int threads = a.G * wm * 64;
  const int blocks = n_groups * ks;
  if (kind == 4) {
    switch (B) {
      case 1: launch_b<4, 1>(a, tpw, blocks, threads, s); break;
      case 2: launch_b<4, 2>(a, tpw, blocks, threads, s); break;
      case 4: launch_b<4, 4>(a, tpw, blocks, threads, s); break;
      default: launch_b<4, 8>(a, tpw, blocks, threads, s); break;
    }
  } else {
    switch (B) {
      case 1: launch_b<8, 1>(a, tpw, blocks, threads, s); break;
      case 2: launch_b<8, 2>(a, tpw, blocks, threads, s); break;
      case 4: launch_b<8, 4>(a, tpw, blocks, threads, s); break;
      default: launch_b<8, 8>(a, tpw, blocks, threads, s); break;
    }
  }
  return check_launch(what);
}

static int check_common(const void* w, int n_tile_rows, int k_tiles, int batch, const char* what,
                        int max_batch = Q4NX_MAX_BATCH) {
  Q4NX_REQUIRE(w != nullptr && Q4NX_ALIGNED(w, 16), Q4NX_ERR_ARG,
               "%s: weights must be a non-null 16-byte aligned device pointer", what);
  Q4NX_REQUIRE(n_tile_rows > 0 && k_tiles > 0, Q4NX_ERR_SHAPE,
               "%s: n_tile_rows=%d k_tiles=%d must be positive (N %% 32 == 0, K %% 256 == 0)",
               what, n_tile_rows, k_tiles);
  Q4NX_REQUIRE(batch >= 1 && batch <= max_batch, Q4NX_ERR_SHAPE,
               "%s: batch=%d outside 1..%d (more rows need the matrix-core path)", what, batch,
               max_batch);
  return Q4NX_OK;
}

static int check_x(const void* x, int64_t x_stride, int k_tiles, const char* what) {
  Q4NX_REQUIRE(x != nullptr && Q4NX_ALIGNED(x, 16), Q4NX_ERR_ARG,
               "%s: x must be a non-null 16-byte aligned device pointer", what);
  Q4NX_REQUIRE(x_stride >= (int64_t)k_tiles * 256 && x_stride % 8 == 0, Q4NX_ERR_SHAPE,
               "%s: x_stride=%lld must be a multiple of 8 and >= K=%d", what,
               (long long)x_stride, k_tiles * 256);
  return Q4NX_OK;
}

static int check_ssq_in(const float* ssq_in, const uint16_t* norm_w, int k_tiles,
                        const char* what) {
  Q4NX_REQUIRE(ssq_in == nullptr || (norm_w != nullptr && Q4NX_ALIGNED(ssq_in, 16)),
               Q4NX_ERR_ARG, "%s: ssq_in goes with norm_w (16-byte aligned)", what);
  Q4NX_REQUIRE(ssq_in == nullptr || k_tiles <= 32, Q4NX_ERR_SHAPE,
               "%s: ssq_in supports K <= 8192, K=%d", what, k_tiles * 256);
  return Q4NX_OK;
}

// Whether a one-row call of G member tile-rows runs on the row-block kernels (gemv1.hip; q4,
// and q8 for a plain GEMV): the policy's choice, for the K they cover, with the producer's
// sums of squares for a norm.
static bool take_rowblock(int kind, int batch, int G, int k_tiles, const uint16_t* norm_w,
                          const float* ssq_in, const Policy& P) {
  return P.rowblock && (kind == Q4NX_KIND_Q4 || G == 1) && batch == 1 &&
         gemv1_fits(G, k_tiles, norm_w != nullptr) && (norm_w == nullptr || ssq_in != nullptr);
}

// Whether a launch of `batch` rows goes to the matrix-core kernels (gemm.hip): the policy's
// mfma_rows, and only for what they implement (an RMSNorm prologue there takes
// the producer's sums of squares, and room for the normalised rows in xn_out or the
// workspace).
static bool take_mfma(int kind, int batch, int k_tiles, const uint16_t* norm_w,
                      const float* ssq_in, const void* xn_out, size_t ws_bytes, const Policy& P) {
  if (!mfma_use(kind, batch, P)) return false;
  if (norm_w == nullptr) return true;
  return ssq_in != nullptr && (xn_out != nullptr || mfma_norm_fits(k_tiles, batch, ws_bytes));
}

static int gemv_plain(int kind, const uint8_t* w, const void* x, const uint16_t* norm_w,
                      float eps, const float* ssq_in, float* y, int n_tile_rows, int k_tiles,
                      int batch, int64_t x_stride, int64_t y_stride, const float* residual,
                      float* ssq_out, unsigned long long* argmax_keys, void* stream,
                      const char* what, void* ws, size_t ws_bytes, const q4nx_policy* policy) {
  Policy P;
  if (int rc = resolve_policy(policy, &P, what)) return rc;
  const bool mf = take_mfma(kind, batch, k_tiles, norm_w, ssq_in, nullptr, ws ? ws_bytes : 0, P);
  int rc = check_common(w, n_tile_rows, k_tiles, batch, what, mf ? INT_MAX : Q4NX_MAX_BATCH);
  if (rc) return rc;
  rc = check_x(x, x_stride, k_tiles, what);
  if (rc) return rc;
  rc = check_ssq_in(ssq_in, norm_w, k_tiles, what);
  if (rc) return rc;
  Q4NX_REQUIRE(ssq_out == nullptr || (y != nullptr && Q4NX_ALIGNED(ssq_out, 4)), Q4NX_ERR_ARG,
               "%s: ssq_out goes with y (4-byte aligned)", what);
  Q4NX_REQUIRE(norm_w == nullptr || Q4NX_ALIGNED(norm_w, 16), Q4NX_ERR_ARG,
               "%s: norm_w must be 16-byte aligned", what);
  Q4NX_REQUIRE((y != nullptr && Q4NX_ALIGNED(y, 4)) || (y == nullptr && argmax_keys != nullptr),
               Q4NX_ERR_ARG, "%s: y must be a 4-byte aligned device pointer", what);
  Q4NX_REQUIRE(y == nullptr || y_stride >= (int64_t)n_tile_rows * 32, Q4NX_ERR_SHAPE,
               "%s: y_stride=%lld < N=%d", what, (long long)y_stride, n_tile_rows * 32);
  Q4NX_REQUIRE(residual == nullptr || y != nullptr, Q4NX_ERR_ARG,
               "%s: a residual needs an output", what);
  Q4NX_REQUIRE(argmax_keys == nullptr || Q4NX_ALIGNED(argmax_keys, 8), Q4NX_ERR_ARG,
               "%s: argmax keys must be 8-byte aligned", what);
  if (mf) {
    GemmArgs g{};
    g.w[0] = w;
    g.n_tr[0] = n_tile_rows;
    g.k_t = k_tiles;
    g.m_rows = batch;
    if (norm_w) {
      g.hres = (const float*)x;
      g.norm_w = norm_w;
      g.eps = eps;
      g.ssq_in = ssq_in;
    } else {
      g.x = (const uint16_t*)x;
    }
    g.x_stride = x_stride;
    g.y = y;
    g.y_stride = y_stride;
    g.residual = residual;
    g.ssq_out = ssq_out;
    g.argmax_keys = argmax_keys;
    return mfma_launch(kind, GOP_PLAIN, g, n_tile_rows, ws, ws_bytes, P, (hipStream_t)stream,
                       what);
  }
  if (take_rowblock(kind, batch, 1, k_tiles, norm_w, ssq_in, P)) {
    Gemv1Args g{};
    g.w0 = w;
    g.k_t = k_tiles;
    g.n_groups = n_tile_rows;
    if (norm_w) {
      g.hres = (const float*)x;
      g.norm_w = norm_w;
      g.eps = eps;
      g.ssq_in = ssq_in;
    } else {
      g.x = (const uint16_t*)x;
    }
    g.y = y;
    g.residual = residual;
    g.ssq_out = ssq_out;
    g.keys = argmax_keys;
    return gemv1_launch(G1_PLAIN, g, (hipStream_t)stream, what, kind, P.gemv_tpw);
  }
  GemvArgs a{};
  a.w[0] = w;
  a.n_tr[0] = n_tile_rows;
  a.op = OP_PLAIN;
  a.G = 1;
  a.k_t = k_tiles;
  a.batch = batch;
  if (norm_w) {
    a.hres = (const float*)x;
    a.norm_w = norm_w;
    a.eps = eps;
    a.ssq_in = ssq_in;
  } else {
    a.x = (const uint16_t*)x;
  }
  a.x_stride = x_stride;
  a.y = y;
  a.y_stride = y_stride;
  a.residual = residual;
  a.ssq_out = ssq_out;
  a.argmax_keys = argmax_keys;
  return launch(kind, a, n_tile_rows, P, (hipStream_t)stream, what, ws, ws_bytes);
}

}  // namespace q4nx

using namespace q4nx;

extern "C" {

// Workspace of a split-K launch (0 when the launch has enough groups to fill the GPU, or runs
// on the row-block kernels). Without it the launches still run, one workgroup per group.
size_t q4nx_gemv_ws_bytes(int kind, int n_tile_rows, int k_tiles, int batch,
                          const q4nx_policy* policy) {
  Policy P;
  if (n_tile_rows < 1 || k_tiles < 1 || batch < 1 || !resolve_policy_quiet(policy, &P)) return 0;
  // either kernel may take the launch (the VALU one when the matrix-core one cannot)
  const bool rowblock = take_rowblock(kind, batch, 1, k_tiles, nullptr, nullptr, P);
  const size_t v = batch <= Q4NX_MAX_BATCH && !rowblock ? ws_need(n_tile_rows, 1, k_tiles, batch, P) : 0;
  const size_t m = mfma_use(kind, batch, P) ? mfma_ws_bytes(kind, GOP_PLAIN, n_tile_rows, k_tiles, batch, P) : 0;
  return v > m ? v : m;
}

int q4nx_gemv_q4(const uint8_t* w, const uint16_t* x, float* y, int n_tile_rows, int k_tiles,
                 int batch, int64_t x_stride, int64_t y_stride, const float* residual, void* ws,
                 size_t ws_bytes, const q4nx_policy* policy, void* stream) {
  return gemv_plain(4, w, x, nullptr, 0.f, nullptr, y, n_tile_rows, k_tiles, batch, x_stride,
                    y_stride, residual, nullptr, nullptr, stream, "q4nx_gemv_q4", ws, ws_bytes,
                    policy);
}

int q4nx_gemv_q8(const uint8_t* w, const uint16_t* x, float* y, int n_tile_rows, int k_tiles,
                 int batch, int64_t x_stride, int64_t y_stride, const float* residual, void* ws,
                 size_t ws_bytes, const q4nx_policy* policy, void* stream) {
  return gemv_plain(8, w, x, nullptr, 0.f, nullptr, y, n_tile_rows, k_tiles, batch, x_stride,
                    y_stride, residual, nullptr, nullptr, stream, "q4nx_gemv_q8", ws, ws_bytes,
                    policy);
}

int q4nx_gemv_ex(int kind, const uint8_t* w, int n_tile_rows, int k_tiles, const void* x,
                 int64_t x_stride, const uint16_t* norm_w, float eps, const float* ssq_in,
                 int batch, float* y, int64_t y_stride, const float* residual, float* ssq_out,
                 uint64_t* argmax_keys, void* ws, size_t ws_bytes, const q4nx_policy* policy,
                 void* stream) {
  Q4NX_REQUIRE(kind == Q4NX_KIND_Q4 || kind == Q4NX_KIND_Q8, Q4NX_ERR_ARG,
               "q4nx_gemv_ex: kind must be Q4NX_KIND_Q4 or Q4NX_KIND_Q8, got %d", kind);
  return gemv_plain(kind, w, x, norm_w, eps, ssq_in, y, n_tile_rows, k_tiles, batch, x_stride,
                    y_stride, residual, ssq_out, (unsigned long long*)argmax_keys, stream,
                    "q4nx_gemv_ex", ws, ws_bytes, policy);
}

int q4nx_gemv_attn_q4(const uint8_t* w, int n_tile_rows, const float* att_rec, int n_split,
                      int n_q_heads, int n_kv_heads, float* y, const float* residual,
                      float* ssq_out, void* stream) {
  const char* what = "q4nx_gemv_attn_q4";
  Q4NX_REQUIRE(n_q_heads > 0 && n_kv_heads > 0 && n_q_heads % n_kv_heads == 0 &&
                   n_q_heads % 4 == 0,
               Q4NX_ERR_SHAPE, "%s: n_q_heads=%d must be a multiple of 4 and of n_kv_heads=%d",
               what, n_q_heads, n_kv_heads);
  const int k_tiles = n_q_heads / 4;   // K = 64 per head
  Q4NX_REQUIRE(k_tiles <= kAttnRecMaxKTiles, Q4NX_ERR_SHAPE,
               "%s: %d query heads, at most %d (a wave per four heads, one workgroup)", what,
               n_q_heads, 4 * kAttnRecMaxKTiles);
  int rc = check_common(w, n_tile_rows, k_tiles, 1, what);
  if (rc) return rc;
  Q4NX_REQUIRE(att_rec != nullptr && Q4NX_ALIGNED(att_rec, 16), Q4NX_ERR_ARG,
               "%s: the split records must be a non-null 16-byte aligned device pointer", what);
  Q4NX_REQUIRE(n_split >= 1 && n_split <= kAttnRecMaxSplits, Q4NX_ERR_SHAPE,
               "%s: n_split=%d outside 1..%d", what, n_split, kAttnRecMaxSplits);
  Q4NX_REQUIRE(y != nullptr && Q4NX_ALIGNED(y, 4), Q4NX_ERR_ARG,
               "%s: y must be a 4-byte aligned device pointer", what);
  Q4NX_REQUIRE(ssq_out == nullptr || Q4NX_ALIGNED(ssq_out, 4), Q4NX_ERR_ARG,
               "%s: ssq_out must be 4-byte aligned", what);
  Gemv1Args g{};
  g.w0 = w;
  g.k_t = k_tiles;
  g.n_groups = n_tile_rows;
  g.att_rec = att_rec;
  g.att_split = n_split;
  g.att_g = n_q_heads / n_kv_heads;
  g.y = y;
  g.residual = residual;
  g.ssq_out = ssq_out;
  return gemv1_attn_launch(g, (hipStream_t)stream, what);
}

size_t q4nx_qkv_rope_ws_bytes(int n_q_heads, int n_kv_heads, int k_tiles, int batch,
                              const q4nx_policy* policy) {
  Policy P;
  if (n_q_heads < 1 || n_kv_heads < 1 || k_tiles < 1 || batch < 1 ||
      !resolve_policy_quiet(policy, &P))
    return 0;
  const int g = n_q_heads + 2 * n_kv_heads;
  // a call with a norm prologue needs ssq_in on the row-block kernels: size for the general
  // kernel too unless the shape fits them either way
  const bool rowblock = take_rowblock(Q4NX_KIND_Q4, batch, 2, k_tiles, nullptr, nullptr, P);
  const size_t v = batch <= Q4NX_MAX_BATCH && !rowblock ? ws_need(g, 2, k_tiles, batch, P) : 0;
  const size_t m = mfma_use(Q4NX_KIND_Q4, batch, P) ? mfma_ws_bytes(Q4NX_KIND_Q4, GOP_QKV, g, k_tiles, batch, P) : 0;
  return v > m ? v : m;
}

int q4nx_qkv_rope(const uint8_t* wq, const uint8_t* wk, const uint8_t* wv, int n_q_heads,
                  int n_kv_heads, int k_tiles, const void* x, int64_t x_stride,
                  const uint16_t* norm_w, float eps, const float* ssq_in, int batch,
                  const int32_t* positions,
                  const float* rope_tab, int max_pos, uint16_t* q_out, uint16_t* k_cache,
                  uint16_t* v_cache, int64_t kv_b_stride, int64_t kv_h_stride, float* raw_out,
                  uint16_t* xn_out, void* ws, size_t ws_bytes, const q4nx_policy* policy,
                  void* stream) {
  const char* what = "q4nx_qkv_rope";
  Policy P;
  if (int rc = resolve_policy(policy, &P, what)) return rc;
  const bool mf = take_mfma(Q4NX_KIND_Q4, batch, k_tiles, norm_w, ssq_in, xn_out, ws ? ws_bytes : 0, P);
  for (const void* p : {(const void*)wq, (const void*)wk, (const void*)wv}) {
    int rc = check_common(p, 2, k_tiles, batch, what, mf ? INT_MAX : Q4NX_MAX_BATCH);
    if (rc) return rc;
  }
  Q4NX_REQUIRE(n_q_heads > 0 && n_kv_heads > 0 && n_q_heads % n_kv_heads == 0, Q4NX_ERR_SHAPE,
               "%s: n_q_heads=%d must be a positive multiple of n_kv_heads=%d", what, n_q_heads,
               n_kv_heads);
  int rc = check_x(x, x_stride, k_tiles, what);
  if (rc) return rc;
  rc = check_ssq_in(ssq_in, norm_w, k_tiles, what);
  if (rc) return rc;
  Q4NX_REQUIRE(norm_w == nullptr || Q4NX_ALIGNED(norm_w, 16), Q4NX_ERR_ARG,
               "%s: norm_w must be 16-byte aligned", what);
  Q4NX_REQUIRE(xn_out == nullptr || Q4NX_ALIGNED(xn_out, 16), Q4NX_ERR_ARG,
               "%s: xn_out must be 16-byte aligned", what);
  Q4NX_REQUIRE(positions && rope_tab && q_out && k_cache && v_cache, Q4NX_ERR_ARG,
               "%s: positions, rope table, q_out and caches are required", what);
  Q4NX_REQUIRE(max_pos > 0 && kv_h_stride >= (int64_t)max_pos * 64 &&
                   kv_b_stride >= (int64_t)n_kv_heads * kv_h_stride,
               Q4NX_ERR_SHAPE, "%s: cache strides do not hold [n_kv][max_pos][64]", what);
  if (mf) {
    GemmArgs g{};
    g.w[0] = wq;
    g.w[1] = wk;
    g.w[2] = wv;
    g.n_tr[0] = n_q_heads * 2;
    g.n_tr[1] = n_kv_heads * 2;
    g.n_tr[2] = n_kv_heads * 2;
    g.grp_q = n_q_heads;
    g.grp_k = n_kv_heads;
    g.k_t = k_tiles;
    g.m_rows = batch;
    if (norm_w) {
      g.hres = (const float*)x;
      g.norm_w = norm_w;
      g.eps = eps;
      g.ssq_in = ssq_in;
      g.xn_out = xn_out;
    } else {
      g.x = (const uint16_t*)x;
    }
    g.x_stride = x_stride;
    g.q_out = q_out;
    g.k_cache = k_cache;
    g.v_cache = v_cache;
    g.kv_b_stride = kv_b_stride;
    g.kv_h_stride = kv_h_stride;
    g.pos = positions;
    g.rope_tab = rope_tab;
    g.max_pos = max_pos;
    g.n_q_heads = n_q_heads;
    g.n_kv_heads = n_kv_heads;
    g.raw_out = raw_out;
    return mfma_launch(Q4NX_KIND_Q4, GOP_QKV, g, n_q_heads + 2 * n_kv_heads, ws, ws_bytes, P,
                       (hipStream_t)stream, what);
  }
  if (take_rowblock(Q4NX_KIND_Q4, batch, 2, k_tiles, norm_w, ssq_in, P)) {
    Gemv1Args g{};
    g.w0 = wq;
    g.w1 = wk;
    g.w2 = wv;
    g.k_t = k_tiles;
    g.n_groups = n_q_heads + 2 * n_kv_heads;
    g.grp_q = n_q_heads;
    g.grp_k = n_kv_heads;
    if (norm_w) {
      g.hres = (const float*)x;
      g.norm_w = norm_w;
      g.eps = eps;
      g.ssq_in = ssq_in;
      g.xn_out = xn_out;
    } else {
      g.x = (const uint16_t*)x;
    }
    g.q_out = q_out;
    g.k_cache = k_cache;
    g.v_cache = v_cache;
    g.kv_h_stride = kv_h_stride;
    g.pos = positions;
    g.rope_tab = rope_tab;
    g.max_pos = max_pos;
    g.n_q_heads = n_q_heads;
    g.n_kv_heads = n_kv_heads;
    g.raw_out = raw_out;
    return gemv1_launch(G1_QKV, g, (hipStream_t)stream, what, 4, P.gemv_tpw);
  }
  GemvArgs a{};
  a.w[0] = wq;
  a.w[1] = wk;
  a.w[2] = wv;
  a.n_tr[0] = n_q_heads * 2;
  a.n_tr[1] = n_kv_heads * 2;
  a.n_tr[2] = n_kv_heads * 2;
  a.op = OP_QKV;
  a.G = 2;
  a.grp_q = n_q_heads;
  a.grp_k = n_kv_heads;
  a.k_t = k_tiles;
  a.batch = batch;
  if (norm_w) {
    a.hres = (const float*)x;
    a.norm_w = norm_w;
    a.eps = eps;
    a.ssq_in = ssq_in;
  } else {
    a.x = (const uint16_t*)x;
  }
  a.x_stride = x_stride;
  a.xn_out = xn_out;
  a.q_out = q_out;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.kv_b_stride = kv_b_stride;
  a.kv_h_stride = kv_h_stride;
  a.pos = positions;
  a.rope_tab = rope_tab;
  a.max_pos = max_pos;
  a.n_q_heads = n_q_heads;
  a.n_kv_heads = n_kv_heads;
  a.raw_out = raw_out;
  return launch(4, a, n_q_heads + 2 * n_kv_heads, P, (hipStream_t)stream, what, ws, ws_bytes);
}

size_t q4nx_gate_up_ws_bytes(int n_tile_rows, int k_tiles, int batch, const q4nx_policy* policy) {
  Policy P;
  if (n_tile_rows < 1 || k_tiles < 1 || batch < 1 || !resolve_policy_quiet(policy, &P)) return 0;
  const bool rowblock = take_rowblock(Q4NX_KIND_Q4, batch, 2, k_tiles, nullptr, nullptr, P);
  const size_t v = batch <= Q4NX_MAX_BATCH && !rowblock ? ws_need(n_tile_rows, 2, k_tiles, batch, P) : 0;
  const size_t m = mfma_use(Q4NX_KIND_Q4, batch, P) ? mfma_ws_bytes(Q4NX_KIND_Q4, GOP_GATEUP, n_tile_rows, k_tiles, batch, P) : 0;
  return v > m ? v : m;
}

int q4nx_gate_up_swiglu(const uint8_t* wg, const uint8_t* wu, int n_tile_rows, int k_tiles,
                        const void* x, int64_t x_stride, const uint16_t* norm_w, float eps,
                        const float* ssq_in, int batch, uint16_t* h_out, int64_t h_stride,
                        float* raw_out, uint16_t* xn_out, void* ws, size_t ws_bytes,
                        const q4nx_policy* policy, void* stream) {
  const char* what = "q4nx_gate_up_swiglu";
  Policy P;
  if (int rc = resolve_policy(policy, &P, what)) return rc;
  const bool mf = take_mfma(Q4NX_KIND_Q4, batch, k_tiles, norm_w, ssq_in, xn_out, ws ? ws_bytes : 0, P);
  for (const void* p : {(const void*)wg, (const void*)wu}) {
    int rc = check_common(p, n_tile_rows, k_tiles, batch, what, mf ? INT_MAX : Q4NX_MAX_BATCH);
    if (rc) return rc;
  }
  int rc = check_x(x, x_stride, k_tiles, what);
  if (rc) return rc;
  rc = check_ssq_in(ssq_in, norm_w, k_tiles, what);
  if (rc) return rc;
  Q4NX_REQUIRE(norm_w == nullptr || Q4NX_ALIGNED(norm_w, 16), Q4NX_ERR_ARG,
               "%s: norm_w must be 16-byte aligned", what);
  Q4NX_REQUIRE(xn_out == nullptr || Q4NX_ALIGNED(xn_out, 16), Q4NX_ERR_ARG,
               "%s: xn_out must be 16-byte aligned", what);
  Q4NX_REQUIRE(h_out != nullptr, Q4NX_ERR_ARG, "%s: h_out is required", what);
  Q4NX_REQUIRE(h_stride >= (int64_t)n_tile_rows * 32, Q4NX_ERR_SHAPE, "%s: bad h_stride", what);
  if (mf) {
    GemmArgs g{};
    g.w[0] = wg;
    g.w[1] = wu;
    g.n_tr[0] = n_tile_rows;
    g.n_tr[1] = n_tile_rows;
    g.k_t = k_tiles;
    g.m_rows = batch;
    if (norm_w) {
      g.hres = (const float*)x;
      g.norm_w = norm_w;
      g.eps = eps;
      g.ssq_in = ssq_in;
      g.xn_out = xn_out;
    } else {
      g.x = (const uint16_t*)x;
    }
    g.x_stride = x_stride;
    g.h_out = h_out;
    g.h_stride = h_stride;
    g.raw_out = raw_out;
    return mfma_launch(Q4NX_KIND_Q4, GOP_GATEUP, g, n_tile_rows, ws, ws_bytes, P,
                       (hipStream_t)stream, what);
  }
  if (take_rowblock(Q4NX_KIND_Q4, batch, 2, k_tiles, norm_w, ssq_in, P)) {
    Gemv1Args g{};
    g.w0 = wg;
    g.w1 = wu;
    g.k_t = k_tiles;
    g.n_groups = n_tile_rows;
    if (norm_w) {
      g.hres = (const float*)x;
      g.norm_w = norm_w;
      g.eps = eps;
      g.ssq_in = ssq_in;
      g.xn_out = xn_out;
    } else {
      g.x = (const uint16_t*)x;
    }
    g.h_out = h_out;
    g.raw_out = raw_out;
    return gemv1_launch(G1_GATEUP, g, (hipStream_t)stream, what, 4, P.gemv_tpw);
  }
  GemvArgs a{};
  a.w[0] = wg;
  a.w[1] = wu;
  a.n_tr[0] = n_tile_rows;
  a.n_tr[1] = n_tile_rows;
  a.op = OP_GATEUP;
  a.G = 2;
  a.k_t = k_tiles;
  a.batch = batch;
  if (norm_w) {
    a.hres = (const float*)x;
    a.norm_w = norm_w;
    a.eps = eps;
    a.ssq_in = ssq_in;
  } else {
    a.x = (const uint16_t*)x;
  }
  a.x_stride = x_stride;
  a.xn_out = xn_out;
  a.h_out = h_out;
  a.h_stride = h_stride;
  a.raw_out = raw_out;
  return launch(4, a, n_tile_rows, P, (hipStream_t)stream, what, ws, ws_bytes);
}

}  // extern "C"
