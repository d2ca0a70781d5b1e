// q4nx GEMV for gfx950: y = W x with W read directly in the q4nx tile layout.
//
// Replaces the per-core AIE kernels designs/granite_gemv/granite_gemv.h:109-300 (q4,
// Q4_1) and designs/lm_head/lm_head.h:53-113 (q8) with one launch over the whole tensor,
// plus the fused epilogues of granite_qkv_rope.h:30-71 and granite_swiglu_f32.h:27-51.
//
// Work decomposition
//   A workgroup owns one (group, member, K-split): `nt` consecutive K-tiles of one
//   tile-row. A group is the set of tile-rows an epilogue needs together: one tile-row
//   for a plain GEMV, the two tile-rows of one attention head for [q,k,v,RoPE] (RoPE
//   pairs dim i with i+32), or the same tile-row of gate and up for SwiGLU. Splits of a
//   group write fp32 partials to the workspace and the last workgroup to arrive (atomic
//   counter) sums them in split order and runs the epilogue, so results are
//   bit-reproducible run to run.
//
// Data path
//   The workgroup's tile bytes are contiguous; they go global -> LDS with
//   global_load_lds_dwordx4 (1 KB per wave instruction, fully coalesced). Two lanes own
//   one (row-block, 32-K group) "unit" of a tile, 16 K each, so the per-group scale and
//   minimum are applied once per 256 (q4) weights per lane and there is no cross-lane
//   traffic until the end.
//
// Arithmetic (exact inputs, fp32 accumulate)
//   x is converted to fp16 with one power-of-two scale per workgroup chosen from
//   max|x| over its K range (bf16 values convert exactly in fp16's normal range). A
//   4-bit code c placed in the low bits of an fp16 is the subnormal c * 2^-24, exactly;
//   v_dot2_f32_f16 then multiplies it by two x values with no rounding of the products.
//   For one byte b = lo | hi<<4 of two rows at one k, a v_perm_b32 builds
//   [b(k0), 0, b(k1), 0] = (lo + 16 hi) * 2^-24 for two k, and the same dword masked
//   with 0x000F000F gives lo alone: two dot2 per 4 weights recover both rows' sums
//   (hi = (full - lo) / 16). q8 codes are biased by 128 (xor 0x80) into 1..255 and the
//   bias is removed with 128 * sum(x).  The Q4_1 minimum factors out of the K sum
//   (granite_gemv.h:19-29): y_r += d_r * sum(c x) + m_r * sum(x) per 32-K group.

#include "common.h"

namespace q4nx {

enum GemvOp : int { OP_PLAIN = 0, OP_QKV = 1, OP_GATEUP = 2 };

struct GemvArgs {
  const uint8_t* w[3];
  int n_tr[3];
  int op;
  int G;          // tile-rows per group (1 or 2)
  int n_groups;
  int grp_q, grp_k;  // QKV: groups [0,grp_q) are q heads, [grp_q,grp_q+grp_k) k heads, rest v
  int k_t, nt, n_split, batch;
  // input: bf16 x, or fp32 residual h normalised with norm_w in the prologue
  const uint16_t* x;
  const float* hres;
  int64_t x_stride;
  const uint16_t* norm_w;
  float eps;
  uint16_t* xn_out;
  // plain
  float* y;
  int64_t y_stride;
  const float* residual;
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
  // split-K
  float* partial;
  unsigned* counters;
};

template <int KIND>
struct TileTraits;
template <>
struct TileTraits<4> {
  static constexpr int kBytes = kQ4TileBytes;
};
template <>
struct TileTraits<8> {
  static constexpr int kBytes = kQ8TileBytes;
};

constexpr int kLanesPerTile = 32;  // 16 units x 2 lanes
constexpr int kMaxNt = 8;

__host__ __device__ inline int lds_w_bytes(int kind, int nt) {
  return nt * (kind == 4 ? kQ4TileBytes : kQ8TileBytes);
}

// v_perm selector for result bytes [s1.b_i, 0, s0.b_i, 0]
__device__ __forceinline__ constexpr uint32_t sel_byte(int i) {
  return 0x0c040c00u + (uint32_t)i * 0x00010001u;
}

template <int KIND, int B>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  constexpr int TB = TileTraits<KIND>::kBytes;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;

  // ---- which (group, member, split) this workgroup owns
  const int blk = blockIdx.x;
  const int split = blk % a.n_split;
  const int gm = blk / a.n_split;
  const int member = gm % a.G;
  const int group = gm / a.G;
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
  const int kt0 = split * a.nt;
  const int ntiles = min(a.nt, a.k_t - kt0);
  const int K = a.k_t * kTileK;
  const int k_lo = kt0 * kTileK;           // first K of this workgroup
  const int nk = ntiles * kTileK;          // K values of this workgroup

  // ---- LDS carve-up
  uint8_t* sw = smem;                                                  // tiles
  uint32_t* sx = (uint32_t*)(smem + lds_w_bytes(KIND, a.nt));          // [B][nt*128] fp16 pairs
  float* sred = (float*)(sx + B * a.nt * (kTileK / 2));                // [nwaves][B][32]
  float* sgrp = sred + 8 * B * 32;                                     // [B][64]
  float* sscal = sgrp + B * 64;                                        // [8][B] scratch
  int* sflag = (int*)(sscal + 8 * B);

  // ---- 1. weights: global -> LDS, all issued up front
  {
    const uint8_t* src = a.w[seg] + ((size_t)tr * a.k_t + kt0) * TB;
    const int n_chunks = ntiles * TB / 16;
    const int n_inst = (n_chunks + 63) / 64;
    for (int i = wave; i < n_inst; i += nwaves) {
      const int c = i * 64 + lane;
      if (c < n_chunks) {
        __builtin_amdgcn_global_load_lds(
            (const void*)(src + (size_t)c * 16),
            (__attribute__((address_space(3))) void*)(sw + i * 1024), 16, 0, 0);
      }
    }
  }

  // ---- 2. activation prologue: [RMSNorm] -> bf16 -> fp16 with a power-of-two scale
  int xs_exp[B];  // true x = x' * 2^xs_exp
  {
    float inv_rms[B];
    if (a.norm_w != nullptr) {
      float ss[B];
#pragma unroll
      for (int b = 0; b < B; ++b) ss[b] = 0.f;
      for (int k = tid * 2; k < K; k += blockDim.x * 2) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
          if (b < a.batch) {
            float2 v = *(const float2*)(a.hres + b * a.x_stride + k);
            ss[b] = fmaf(v.x, v.x, ss[b]);
            ss[b] = fmaf(v.y, v.y, ss[b]);
          }
        }
      }
#pragma unroll
      for (int b = 0; b < B; ++b) {
        float s = wave_sum(ss[b]);
        if (lane == 0) sscal[wave * B + b] = s;
      }
      __syncthreads();
#pragma unroll
      for (int b = 0; b < B; ++b) {
        float s = 0.f;
        for (int w = 0; w < nwaves; ++w) s += sscal[w * B + b];
        inv_rms[b] = 1.0f / sqrtf(s / (float)K + a.eps);
      }
      __syncthreads();
    }

    // bf16 values of this workgroup's K range, two per thread-iteration
    float mx[B];
#pragma unroll
    for (int b = 0; b < B; ++b) mx[b] = 0.f;
    const int npairs = nk / 2;
    // threads >= 32 * nt, pairs <= 128 * nt: at most 4 pairs per thread
    constexpr int kPairsPerThread = 4;
    uint32_t xv[B][kPairsPerThread];
#pragma unroll
    for (int np = 0; np < kPairsPerThread; ++np) {
      const int p = tid + np * blockDim.x;
#pragma unroll
      for (int b = 0; b < B; ++b) xv[b][np] = 0u;
      if (p >= npairs) continue;
      const int k = k_lo + 2 * p;
#pragma unroll
      for (int b = 0; b < B; ++b) {
        uint32_t bits = 0;
        if (b < a.batch) {
          if (a.norm_w != nullptr) {
            float2 v = *(const float2*)(a.hres + b * a.x_stride + k);
            uint32_t wbits = *(const uint32_t*)(a.norm_w + k);
            uint16_t lo = f32_to_bf16((v.x * inv_rms[b]) * bf16lo(wbits));
            uint16_t hi = f32_to_bf16((v.y * inv_rms[b]) * bf16hi(wbits));
            bits = (uint32_t)lo | ((uint32_t)hi << 16);
            if (a.xn_out != nullptr && group == 0 && member == 0)
              *(uint32_t*)(a.xn_out + b * a.x_stride + k) = bits;
          } else {
            bits = *(const uint32_t*)(a.x + b * a.x_stride + k);
          }
        }
        xv[b][np] = bits;
        mx[b] = fmaxf(mx[b], fmaxf(fabsf(bf16lo(bits)), fabsf(bf16hi(bits))));
      }
    }
#pragma unroll
    for (int b = 0; b < B; ++b) {
      float m = wave_max(mx[b]);
      if (lane == 0) sscal[wave * B + b] = m;
    }
    __syncthreads();
    float to_half[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
      float m = 0.f;
      for (int w = 0; w < nwaves; ++w) m = fmaxf(m, sscal[w * B + b]);
      int e = 0;
      if (m > 0.f && m <= 3.0e38f) {
        (void)frexpf(m, &e);   // m < 2^e
        e -= 15;               // scaled max < 2^15
        e = e < -120 ? -120 : e;
      }
      to_half[b] = ldexpf(1.0f, -e);
      xs_exp[b] = e;
    }
#pragma unroll
    for (int np = 0; np < kPairsPerThread; ++np) {
      const int p = tid + np * blockDim.x;
      if (p >= npairs) continue;
#pragma unroll
      for (int b = 0; b < B; ++b) {
        uint32_t bits = xv[b][np];
        half2_t h;
        h.x = (_Float16)(bf16lo(bits) * to_half[b]);
        h.y = (_Float16)(bf16hi(bits) * to_half[b]);
        sx[b * (a.nt * kTileK / 2) + p] = h2_bits(h);
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // ---- 3. per-lane half-unit dot products
  const int j = tid >> 5;              // tile within the workgroup
  const int u = (tid >> 1) & 15;       // unit: rb*8 + kb (memory order)
  const int hh = tid & 1;              // which 16 K of the unit
  const int rb = u >> 3, kb = u & 7;
  const bool active = j < ntiles;
  const int jj = active ? j : 0;
  const uint8_t* tile = sw + jj * TB;
  const int pk0 = (jj * kTileK + kb * kGroup + hh * 16) >> 1;  // first x pair
  constexpr uint32_t kOne2 = 0x3C003C00u;                        // fp16 (1, 1)

  float acc[B][16];
  if (KIND == 4) {
    float lo[B][8], full[B][8], X[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
      X[b] = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) lo[b][i] = full[b][i] = 0.f;
    }
    const uint8_t* nib = tile + 1024 + rb * 2048 + kb * 256 + hh * 128;
    const int rot = tid >> 1;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int c = (s + rot) & 7;
      const uint4 q = *(const uint4*)(nib + c * 16);
      uint32_t xp[B];
#pragma unroll
      for (int b = 0; b < B; ++b) xp[b] = sx[b * (a.nt * kTileK / 2) + pk0 + c];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t T0 = perm(q.z, q.x, sel_byte(i));
        const uint32_t T1 = perm(q.w, q.y, sel_byte(i));
        const uint32_t L0 = T0 & 0x000F000Fu, L1 = T1 & 0x000F000Fu;
#pragma unroll
        for (int b = 0; b < B; ++b) {
          full[b][i] = dot2(T0, xp[b], full[b][i]);
          lo[b][i] = dot2(L0, xp[b], lo[b][i]);
          full[b][4 + i] = dot2(T1, xp[b], full[b][4 + i]);
          lo[b][4 + i] = dot2(L1, xp[b], lo[b][4 + i]);
        }
      }
#pragma unroll
      for (int b = 0; b < B; ++b) X[b] = dot2(xp[b], kOne2, X[b]);
    }
    // scale and minimum of this unit: d[g], m[g], g = kb*32 + rb*16 + r
    const int g0 = kb * 32 + rb * 16;
    const uint4 d0 = *(const uint4*)(tile + 2 * g0);
    const uint4 d1 = *(const uint4*)(tile + 2 * g0 + 16);
    const uint4 m0 = *(const uint4*)(tile + kMetaBytes + 2 * g0);
    const uint4 m1 = *(const uint4*)(tile + kMetaBytes + 2 * g0 + 16);
    const uint32_t dd[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
    const uint32_t mm[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
#pragma unroll
    for (int b = 0; b < B; ++b) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float se = lo[b][i] * 16777216.0f;             // 2^24
        const float so = (full[b][i] - lo[b][i]) * 1048576.0f;  // 2^20
        float ve = fmaf(bf16lo(dd[i]), se, bf16lo(mm[i]) * X[b]);
        float vo = fmaf(bf16hi(dd[i]), so, bf16hi(mm[i]) * X[b]);
        acc[b][2 * i] = active ? ve : 0.f;
        acc[b][2 * i + 1] = active ? vo : 0.f;
      }
    }
  } else {
    float sacc[B][16], X[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
      X[b] = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[b][r] = 0.f;
    }
    const uint8_t* cod = tile + kMetaBytes + u * 512 + hh * 256;
    const int rot = tid >> 1;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int p = (s + rot) & 7;
      const uint4 A = *(const uint4*)(cod + p * 32);
      const uint4 Bv = *(const uint4*)(cod + p * 32 + 16);
      uint32_t xp[B];
#pragma unroll
      for (int b = 0; b < B; ++b) xp[b] = sx[b * (a.nt * kTileK / 2) + pk0 + p];
      const uint32_t av[4] = {A.x ^ 0x80808080u, A.y ^ 0x80808080u, A.z ^ 0x80808080u,
                              A.w ^ 0x80808080u};
      const uint32_t bv[4] = {Bv.x ^ 0x80808080u, Bv.y ^ 0x80808080u, Bv.z ^ 0x80808080u,
                              Bv.w ^ 0x80808080u};
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t T = perm(bv[qd], av[qd], sel_byte(i));
#pragma unroll
          for (int b = 0; b < B; ++b) sacc[b][4 * qd + i] = dot2(T, xp[b], sacc[b][4 * qd + i]);
        }
      }
#pragma unroll
      for (int b = 0; b < B; ++b) X[b] = dot2(xp[b], kOne2, X[b]);
    }
    const int g0 = kb * 32 + rb * 16;
    const uint4 s0 = *(const uint4*)(tile + 2 * g0);
    const uint4 s1 = *(const uint4*)(tile + 2 * g0 + 16);
    const uint32_t sd[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const float bias = 128.0f * X[b];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float ve = fmaf(sacc[b][2 * i], 16777216.0f, -bias);
        const float vo = fmaf(sacc[b][2 * i + 1], 16777216.0f, -bias);
        acc[b][2 * i] = active ? bf16lo(sd[i]) * ve : 0.f;
        acc[b][2 * i + 1] = active ? bf16hi(sd[i]) * vo : 0.f;
      }
    }
  }

  // ---- 4. reduce: lanes with the same row-block, then waves, then splits
  // transpose-reduce over lane bits 0..3 (h, kb): afterwards lane holds row (lane & 15)
#pragma unroll
  for (int b = 0; b < B; ++b) {
    float v8[8];
    {
      const bool up = (lane & 8) != 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float keep = up ? acc[b][i + 8] : acc[b][i];
        const float send = up ? acc[b][i] : acc[b][i + 8];
        v8[i] = keep + __shfl_xor(send, 8);
      }
    }
    float v4[4];
    {
      const bool up = (lane & 4) != 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float keep = up ? v8[i + 4] : v8[i];
        const float send = up ? v8[i] : v8[i + 4];
        v4[i] = keep + __shfl_xor(send, 4);
      }
    }
    float v2[2];
    {
      const bool up = (lane & 2) != 0;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float keep = up ? v4[i + 2] : v4[i];
        const float send = up ? v4[i] : v4[i + 2];
        v2[i] = keep + __shfl_xor(send, 2);
      }
    }
    float v1;
    {
      const bool up = (lane & 1) != 0;
      const float keep = up ? v2[1] : v2[0];
      const float send = up ? v2[0] : v2[1];
      v1 = keep + __shfl_xor(send, 1);
    }
    v1 += __shfl_xor(v1, 32);
    if (lane < 32) sred[(wave * B + b) * 32 + lane] = v1;  // lane&31 = rb*16 + r
  }
  __syncthreads();

  const bool direct = (a.G == 1 && a.n_split == 1);
  // a workgroup can be a single wave, so every (b, row) loop strides by blockDim
  for (int e = tid; e < B * 32; e += blockDim.x) {
    const int b = e >> 5, r = e & 31;
    float s = 0.f;
    for (int w = 0; w < nwaves; ++w) s += sred[(w * B + b) * 32 + r];
    s *= ldexpf(1.0f, xs_exp[b]);
    if (direct) {
      sgrp[b * 64 + r] = s;
    } else {
      a.partial[(((size_t)group * a.G + member) * a.n_split + split) * (B * 32) + e] = s;
    }
  }
  if (!direct) {
    __threadfence();
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = atomicAdd(&a.counters[group], 1u);
      sflag[0] = (prev == (unsigned)(a.G * a.n_split - 1)) ? 1 : 0;
    }
    __syncthreads();
    if (sflag[0] == 0) return;
    __threadfence();
    for (int e = tid; e < a.G * B * 32; e += blockDim.x) {
      const int m = e / (B * 32), rest = e % (B * 32);
      const int b = rest >> 5, r = rest & 31;
      const float* p = a.partial + (((size_t)group * a.G + m) * a.n_split) * (B * 32) + rest;
      float s = 0.f;
      for (int sp = 0; sp < a.n_split; ++sp) s += p[sp * (B * 32)];
      sgrp[b * 64 + m * 32 + r] = s;
    }
    if (tid == 0) a.counters[group] = 0u;
  }
  __syncthreads();

  // ---- 5. epilogue on the whole group
  if (a.op == OP_PLAIN) {
    for (int e = tid; e < B * 32; e += blockDim.x) {
      const int b = e >> 5, r = e & 31;
      if (b < a.batch) {
        const int64_t n = (int64_t)tr * 32 + r;
        float v = sgrp[b * 64 + r];
        if (a.residual != nullptr) v += a.residual[b * a.y_stride + n];
        a.y[b * a.y_stride + n] = v;
      }
    }
  } else if (a.op == OP_GATEUP) {
    for (int e = tid; e < B * 32; e += blockDim.x) {
      const int b = e >> 5, r = e & 31;
      if (b < a.batch) {
        const int64_t n = (int64_t)group * 32 + r;
        const float gr = sgrp[b * 64 + r], ur = sgrp[b * 64 + 32 + r];
        const float g = bf16_to_f32(f32_to_bf16(gr));
        const float uu = bf16_to_f32(f32_to_bf16(ur));
        const float h = (g / (1.0f + expf(-g))) * uu;
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
        const float r0 = sgrp[b * 64 + d], r1 = sgrp[b * 64 + 32 + d];
        if (a.raw_out != nullptr) {
          const int64_t W = (int64_t)(a.n_q_heads + 2 * a.n_kv_heads) * 64;
          a.raw_out[b * W + seg_off + hg * 64 + d] = r0;
          a.raw_out[b * W + seg_off + hg * 64 + 32 + d] = r1;
        }
        const float x0 = bf16_to_f32(f32_to_bf16(r0));
        const float x1 = bf16_to_f32(f32_to_bf16(r1));
        const int p = a.pos[b];
        const bool pos_ok = p >= 0 && p < a.max_pos;
        if (seg == 2) {
          if (pos_ok) {
            uint16_t* dst = a.v_cache + b * a.kv_b_stride + hg * a.kv_h_stride + (int64_t)p * 64;
            dst[d] = f32_to_bf16(x0);
            dst[32 + d] = f32_to_bf16(x1);
          }
        } else if (pos_ok) {
          const float c = a.rope_tab[(int64_t)p * 64 + d];
          const float sn = a.rope_tab[(int64_t)p * 64 + 32 + d];
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
}

// ------------------------------------------------------------------ host side

static int g_split_tiles = 0;

constexpr size_t kMaxLds = 65536;

static int round_batch(int batch) { return batch <= 1 ? 1 : batch <= 2 ? 2 : batch <= 4 ? 4 : 8; }

static size_t lds_bytes(int kind, int nt, int B) {
  return (size_t)lds_w_bytes(kind, nt) + (size_t)B * nt * kTileK * 2 + 8 * B * 32 * 4 +
         B * 64 * 4 + 8 * B * 4 + 16;
}

// K-tiles per workgroup. Automatic: the largest divisor of k_t (<= 8) giving >= 512
// workgroups, else >= 256, else 1; then capped so the LDS carve-up fits in 64 KB.
static int choose_nt(int kind, int total_rows_in_groups, int k_t, int batch) {
  const int B = round_batch(batch);
  int nt = 0;
  if (g_split_tiles > 0) {
    nt = g_split_tiles < k_t ? g_split_tiles : k_t;
  } else {
    for (int target : {512, 256}) {
      for (int c = (k_t < kMaxNt ? k_t : kMaxNt); c >= 1 && nt == 0; --c) {
        if (k_t % c) continue;
        if ((long)total_rows_in_groups * (k_t / c) >= target) nt = c;
      }
      if (nt) break;
    }
    if (nt == 0) nt = 1;
  }
  if (nt > kMaxNt) nt = kMaxNt;
  while (nt > 1 && lds_bytes(kind, nt, B) > kMaxLds) --nt;
  return nt;
}

static size_t ws_bytes_for(int n_groups, int G, int n_split, int B) {
  if (G == 1 && n_split == 1) return 0;
  return (size_t)Q4NX_WS_COUNTER_BYTES + (size_t)n_groups * G * n_split * B * 32 * 4;
}

template <int KIND, int B>
static void launch_t(const GemvArgs& a, int blocks, int threads, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((gemv_kernel<KIND, B>), dim3(blocks), dim3(threads), lds, s, a);
}

static int launch(int kind, GemvArgs& a, void* ws, size_t ws_bytes, hipStream_t s,
                  const char* what) {
  const int B = round_batch(a.batch);
  a.n_split = (a.k_t + a.nt - 1) / a.nt;
  const size_t need = ws_bytes_for(a.n_groups, a.G, a.n_split, B);
  Q4NX_REQUIRE(need == 0 || (ws != nullptr && ws_bytes >= need), Q4NX_ERR_WS,
               "%s: workspace of %zu bytes needed, %zu given", what, need, ws_bytes);
  Q4NX_REQUIRE(ws == nullptr || Q4NX_ALIGNED(ws, 256), Q4NX_ERR_ARG,
               "%s: workspace must be 256-byte aligned", what);
  if (need) {
    Q4NX_REQUIRE((size_t)a.n_groups * 4 <= (size_t)Q4NX_WS_COUNTER_BYTES, Q4NX_ERR_SHAPE,
                 "%s: %d output groups exceed the workspace counter region", what, a.n_groups);
    a.counters = (unsigned*)ws;
    a.partial = (float*)((uint8_t*)ws + Q4NX_WS_COUNTER_BYTES);
  }
  const int blocks = a.n_groups * a.G * a.n_split;
  const int threads = ((a.nt * kLanesPerTile + 63) / 64) * 64;
  const size_t lds = lds_bytes(kind, a.nt, B);
  if (kind == 4) {
    switch (B) {
      case 1: launch_t<4, 1>(a, blocks, threads, lds, s); break;
      case 2: launch_t<4, 2>(a, blocks, threads, lds, s); break;
      case 4: launch_t<4, 4>(a, blocks, threads, lds, s); break;
      default: launch_t<4, 8>(a, blocks, threads, lds, s); break;
    }
  } else {
    switch (B) {
      case 1: launch_t<8, 1>(a, blocks, threads, lds, s); break;
      case 2: launch_t<8, 2>(a, blocks, threads, lds, s); break;
      case 4: launch_t<8, 4>(a, blocks, threads, lds, s); break;
      default: launch_t<8, 8>(a, blocks, threads, lds, s); break;
    }
  }
  return check_launch(what);
}

static int check_common(const void* w, int n_tile_rows, int k_tiles, int batch, const char* what) {
  Q4NX_REQUIRE(w != nullptr && Q4NX_ALIGNED(w, 16), Q4NX_ERR_ARG,
               "%s: weights must be a non-null 16-byte aligned device pointer", what);
  Q4NX_REQUIRE(n_tile_rows > 0 && k_tiles > 0, Q4NX_ERR_SHAPE,
               "%s: n_tile_rows=%d k_tiles=%d must be positive (N %% 32 == 0, K %% 256 == 0)",
               what, n_tile_rows, k_tiles);
  Q4NX_REQUIRE(batch >= 1 && batch <= Q4NX_MAX_BATCH, Q4NX_ERR_SHAPE,
               "%s: batch=%d outside 1..%d", what, batch, Q4NX_MAX_BATCH);
  return Q4NX_OK;
}

static int gemv_plain(int kind, const uint8_t* w, const uint16_t* x, float* y, int n_tile_rows,
                      int k_tiles, int batch, int64_t x_stride, int64_t y_stride,
                      const float* residual, void* ws, size_t ws_bytes, void* stream,
                      const char* what) {
  int rc = check_common(w, n_tile_rows, k_tiles, batch, what);
  if (rc) return rc;
  Q4NX_REQUIRE(x != nullptr && Q4NX_ALIGNED(x, 4) && y != nullptr && Q4NX_ALIGNED(y, 4),
               Q4NX_ERR_ARG, "%s: x and y must be non-null 4-byte aligned device pointers", what);
  Q4NX_REQUIRE(x_stride >= (int64_t)k_tiles * 256 && x_stride % 2 == 0, Q4NX_ERR_SHAPE,
               "%s: x_stride=%lld must be even and >= K=%d", what, (long long)x_stride,
               k_tiles * 256);
  Q4NX_REQUIRE(y_stride >= (int64_t)n_tile_rows * 32, Q4NX_ERR_SHAPE,
               "%s: y_stride=%lld < N=%d", what, (long long)y_stride, n_tile_rows * 32);
  GemvArgs a{};
  a.w[0] = w;
  a.n_tr[0] = n_tile_rows;
  a.op = OP_PLAIN;
  a.G = 1;
  a.n_groups = n_tile_rows;
  a.k_t = k_tiles;
  a.nt = choose_nt(kind, n_tile_rows, k_tiles, batch);
  a.batch = batch;
  a.x = x;
  a.x_stride = x_stride;
  a.y = y;
  a.y_stride = y_stride;
  a.residual = residual;
  return launch(kind, a, ws, ws_bytes, (hipStream_t)stream, what);
}

}  // namespace q4nx

using namespace q4nx;

extern "C" {

int q4nx_set_split_tiles(int tiles) {
  Q4NX_REQUIRE(tiles >= 0 && tiles <= kMaxNt, Q4NX_ERR_ARG, "split tiles %d outside 0..%d",
               tiles, kMaxNt);
  g_split_tiles = tiles;
  return Q4NX_OK;
}

size_t q4nx_gemv_ws_bytes(int kind, int n_tile_rows, int k_tiles, int batch) {
  if (n_tile_rows <= 0 || k_tiles <= 0 || batch < 1) return 0;
  const int nt = choose_nt(kind, n_tile_rows, k_tiles, batch);
  return ws_bytes_for(n_tile_rows, 1, (k_tiles + nt - 1) / nt, round_batch(batch));
}

int q4nx_gemv_q4(const uint8_t* w, const uint16_t* x, float* y, int n_tile_rows, int k_tiles,
                 int batch, int64_t x_stride, int64_t y_stride, const float* residual, void* ws,
                 size_t ws_bytes, void* stream) {
  return gemv_plain(4, w, x, y, n_tile_rows, k_tiles, batch, x_stride, y_stride, residual, ws,
                    ws_bytes, stream, "q4nx_gemv_q4");
}

int q4nx_gemv_q8(const uint8_t* w, const uint16_t* x, float* y, int n_tile_rows, int k_tiles,
                 int batch, int64_t x_stride, int64_t y_stride, const float* residual, void* ws,
                 size_t ws_bytes, void* stream) {
  return gemv_plain(8, w, x, y, n_tile_rows, k_tiles, batch, x_stride, y_stride, residual, ws,
                    ws_bytes, stream, "q4nx_gemv_q8");
}

size_t q4nx_qkv_rope_ws_bytes(int n_q_heads, int n_kv_heads, int k_tiles, int batch) {
  if (n_q_heads <= 0 || n_kv_heads <= 0 || k_tiles <= 0 || batch < 1) return 0;
  const int groups = n_q_heads + 2 * n_kv_heads;
  const int nt = choose_nt(4, groups * 2, k_tiles, batch);
  return ws_bytes_for(groups, 2, (k_tiles + nt - 1) / nt, round_batch(batch));
}

int q4nx_qkv_rope(const uint8_t* wq, const uint8_t* wk, const uint8_t* wv, int n_q_heads,
                  int n_kv_heads, int k_tiles, const void* x, int64_t x_stride,
                  const uint16_t* norm_w, float eps, int batch, const int32_t* positions,
                  const float* rope_tab, int max_pos, uint16_t* q_out, uint16_t* k_cache,
                  uint16_t* v_cache, int64_t kv_b_stride, int64_t kv_h_stride, float* raw_out,
                  uint16_t* xn_out, void* ws, size_t ws_bytes, void* stream) {
  const char* what = "q4nx_qkv_rope";
  for (const void* p : {(const void*)wq, (const void*)wk, (const void*)wv}) {
    int rc = check_common(p, 2, k_tiles, batch, what);
    if (rc) return rc;
  }
  Q4NX_REQUIRE(n_q_heads > 0 && n_kv_heads > 0 && n_q_heads % n_kv_heads == 0, Q4NX_ERR_SHAPE,
               "%s: n_q_heads=%d must be a positive multiple of n_kv_heads=%d", what, n_q_heads,
               n_kv_heads);
  Q4NX_REQUIRE(x != nullptr && Q4NX_ALIGNED(x, 8), Q4NX_ERR_ARG, "%s: x must be 8-byte aligned",
               what);
  Q4NX_REQUIRE(x_stride >= (int64_t)k_tiles * 256 && x_stride % 2 == 0, Q4NX_ERR_SHAPE,
               "%s: bad x_stride", what);
  Q4NX_REQUIRE(positions && rope_tab && q_out && k_cache && v_cache, Q4NX_ERR_ARG,
               "%s: positions, rope table, q_out and caches are required", what);
  Q4NX_REQUIRE(max_pos > 0 && kv_h_stride >= (int64_t)max_pos * 64 &&
                   kv_b_stride >= (int64_t)n_kv_heads * kv_h_stride,
               Q4NX_ERR_SHAPE, "%s: cache strides do not hold [n_kv][max_pos][64]", what);
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
  a.n_groups = n_q_heads + 2 * n_kv_heads;
  a.k_t = k_tiles;
  a.nt = choose_nt(4, a.n_groups * 2, k_tiles, batch);
  a.batch = batch;
  if (norm_w) {
    a.hres = (const float*)x;
    a.norm_w = norm_w;
    a.eps = eps;
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
  return launch(4, a, ws, ws_bytes, (hipStream_t)stream, what);
}

size_t q4nx_gate_up_ws_bytes(int n_tile_rows, int k_tiles, int batch) {
  if (n_tile_rows <= 0 || k_tiles <= 0 || batch < 1) return 0;
  const int nt = choose_nt(4, n_tile_rows * 2, k_tiles, batch);
  return ws_bytes_for(n_tile_rows, 2, (k_tiles + nt - 1) / nt, round_batch(batch));
}

int q4nx_gate_up_swiglu(const uint8_t* wg, const uint8_t* wu, int n_tile_rows, int k_tiles,
                        const void* x, int64_t x_stride, const uint16_t* norm_w, float eps,
                        int batch, uint16_t* h_out, int64_t h_stride, float* raw_out,
                        uint16_t* xn_out, void* ws, size_t ws_bytes, void* stream) {
  const char* what = "q4nx_gate_up_swiglu";
  for (const void* p : {(const void*)wg, (const void*)wu}) {
    int rc = check_common(p, n_tile_rows, k_tiles, batch, what);
    if (rc) return rc;
  }
  Q4NX_REQUIRE(x != nullptr && Q4NX_ALIGNED(x, 8) && h_out != nullptr, Q4NX_ERR_ARG,
               "%s: x (8-byte aligned) and h_out are required", what);
  Q4NX_REQUIRE(x_stride >= (int64_t)k_tiles * 256 && x_stride % 2 == 0, Q4NX_ERR_SHAPE,
               "%s: bad x_stride", what);
  Q4NX_REQUIRE(h_stride >= (int64_t)n_tile_rows * 32, Q4NX_ERR_SHAPE, "%s: bad h_stride", what);
  GemvArgs a{};
  a.w[0] = wg;
  a.w[1] = wu;
  a.n_tr[0] = n_tile_rows;
  a.n_tr[1] = n_tile_rows;
  a.op = OP_GATEUP;
  a.G = 2;
  a.n_groups = n_tile_rows;
  a.k_t = k_tiles;
  a.nt = choose_nt(4, n_tile_rows * 2, k_tiles, batch);
  a.batch = batch;
  if (norm_w) {
    a.hres = (const float*)x;
    a.norm_w = norm_w;
    a.eps = eps;
  } else {
    a.x = (const uint16_t*)x;
  }
  a.x_stride = x_stride;
  a.xn_out = xn_out;
  a.h_out = h_out;
  a.h_stride = h_stride;
  a.raw_out = raw_out;
  return launch(4, a, ws, ws_bytes, (hipStream_t)stream, what);
}

}  // extern "C"
