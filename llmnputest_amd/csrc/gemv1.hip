// Batch-1 q4 GEMV family for gfx950: y = W x for one token, W read in the q4nx tile layout.
//
// Replaces, for a single token, the per-core AIE kernels of
// designs/granite_gemv/granite_gemv.h:109-300 (Q4_1 GEMV) and the fused epilogues of
// granite_qkv_rope.h:30-71 and granite_swiglu_f32.h:27-51, with the RMSNorm of
// granite_rmsnorm.h:45-80 as a prologue and attention's split merge
// (granite_attention.h:193-212) as an alternative prologue of the o-projection.
//
// Work decomposition
//   A q4nx tile stores two 16-row blocks (rb) of 2048 code bytes each. One workgroup owns
//   one output group (one tile-row for a plain GEMV, the two tile-rows of an attention
//   head for [q,k,v,RoPE], the same tile-row of gate and up for SwiGLU) and ONE row block
//   of it: 16 (or 2 x 16) complete output rows, so no two workgroups ever share an output
//   and nothing is merged across workgroups. The two row blocks of a group go to
//   workgroups 8 apart, which the dispatcher places on the same XCD, so the tile metadata
//   both read is fetched into one L2. Each wave owns TPW consecutive K-tiles of one member
//   tile-row; the waves combine once through LDS, in wave order. [q,k,v,RoPE] has only 56
//   groups at the 3B shape, so its workgroups own half a row block (8 rows of each member,
//   224 workgroups): each lane still reads its 32 bytes (the sibling workgroup on the same
//   XCD reads the same lines, from L2) and uses the half it needs — 6.2 -> 5.5 us per launch,
//   bit-identical. The plain and gate/up launches measured slower that way (5.4 -> 6.3,
//   9.3 -> 11.4 us: their L1 traffic doubles for CUs they already fill).
//
// Data path
//   Lane l of a wave reads the 32 contiguous code bytes at rb * 2048 + 32 l of each of its
//   tiles: 4 K values x 16 rows (K-group l / 8, K offset 4 (l % 8)). Every load of a wave
//   (activations, the epilogue's inputs, codes, scales) is issued before the first wait,
//   the small ones of all waves ahead of any weight load, and nothing is loaded under a
//   branch, so the weight stream starts at once.
//
// Arithmetic (exact products, fp32 sums)
//   x is converted to fp16 with one power-of-two scale per 32-K group (bf16 values are exact
//   in fp16's range after scaling). A 4-bit code placed in bits 4-7 of an fp16 is the
//   subnormal c * 2^-20, and v_dot2_f32_f16 multiplies two of them by two x values exactly;
//   one v_perm_b32 builds [c(k), c(k+1)] for a row. The 16 row sums of a lane are reduced
//   over the 8 lanes of its K-group in three DPP steps (14 adds); each lane reads its bytes
//   into lane-dependent register slots so that two of the steps need no selects. Each lane
//   is left with two rows of one group, to which that group's scale and minimum are applied:
//   y_r += d_r * sum(c x) + m_r * sum(x) (the Q4_1 factoring, granite_gemv.h:19-29).
//
// The kernel's time is its launch, the weight stream and the VALU work of the waves that
// receive the last bytes, so the VALU count per K-tile is kept low: no register clears
// before the first dot products, no per-wave cross-row max, a fixed-order wave sum.

#include "common.h"
#include "gemv1.h"

namespace q4nx {

__device__ __forceinline__ constexpr uint32_t sel_pair(int i) {
  return 0x0c040c00u + (uint32_t)i * 0x00010001u;   // [s1.b_i, 0, s0.b_i, 0]
}

// a.x*b.x + a.y*b.y with no accumulator operand: the VOP3P form takes the constant 0, where
// the accumulating VOP2 form would first need a register cleared to zero
__device__ __forceinline__ float dot2_0(uint32_t a, uint32_t b) {
  float r;
  asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float dot2_acc(uint32_t a, uint32_t b, float acc, bool first) {
  return first ? dot2_0(a, b) : dot2(a, b, acc);
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}

// 64-bit max over aligned groups of 16 lanes (every lane of the group gets it).
__device__ __forceinline__ unsigned long long key_max16(unsigned long long k) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) {
    const unsigned long long t = __shfl_xor(k, o);
    k = t > k ? t : k;
  }
  return k;
}

// The 16 wave slots of each member (zero past its waves) in a fixed pairwise order: row r
// of each member, for thread r.
template <int G>
__device__ __forceinline__ void slot_sums(const float (*sred)[16][16], int r, float (&s)[G]) {
#pragma unroll
  for (int m = 0; m < G; ++m) {
    float v[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) v[c] = sred[m][c][r];
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
      for (int c = 0; c < w; ++c) v[c] = v[2 * c] + v[2 * c + 1];
    s[m] = v[0];
  }
}

// Epilogue of a plain or gate/up launch, run by the first wave: thread r < 16 finishes row r
// of the workgroup's 16-row block (tile-row tr, block rb).
template <int OP, int G>
__device__ __forceinline__ void finish_block(const Gemv1Args& a, const float (*sred)[16][16],
                                             int tid, int tr, int rb, float ep_res) {
  const int er = tid & 15;
  float s[G];
  slot_sums<G>(sred, er, s);
  const int64_t n = (int64_t)tr * 32 + rb * 16 + er;
  if constexpr (OP == G1_PLAIN) {
    float v = s[0];
    if (a.residual != nullptr) v += ep_res;
    if (tid < 16 && a.y != nullptr) a.y[n] = v;
    if (a.ssq_out != nullptr) {   // sum of squares of the block's 16 outputs
      const float q = group16_sum(tid < 16 ? v * v : 0.f);
      if (tid == 0) a.ssq_out[(int64_t)tr * 2 + rb] = q;
    }
    if (a.keys != nullptr) {      // (max, first row) of the block, order-preserving
      const unsigned long long kk = key_max16(tid < 16 ? argmax_key(v, (uint32_t)n) : 0ull);
      if (tid == 0) a.keys[(int64_t)tr * 2 + rb] = kk;
    }
  } else {
    static_assert(OP == G1_GATEUP, "plain or gate/up");
    if (tid < 16) {
      a.h_out[n] = f32_to_bf16(swiglu(round_bf16_op(s[0]), round_bf16_op(s[1])));
      if (a.raw_out != nullptr) {
        const int64_t N = (int64_t)a.n_groups * 32;
        a.raw_out[n] = s[0];
        a.raw_out[N + n] = s[1];
      }
    }
  }
}

template <int OP, int G, int TPW, int NSS, int XNS, int HB, int KIND>
__global__ __launch_bounds__(1024) void gemv1_kernel(Gemv1Args a) {
  constexpr bool NORM = NSS > 0;
  constexpr bool XREC = XNS > 0;
  // The two members of a normalised group ([q, k, v] heads' tile-row pairs, gate and up)
  // read the same activations: the member-0 wave of each K-chunk loads and normalises them
  // and hands the fp16 operands, their group sums and scale to the member-1 wave through
  // LDS, so half the waves load neither h nor the norm weights nor the sums of squares (at
  // two workgroups per CU a quarter of the bytes each CU takes in)
  constexpr bool SHARE = NORM && G == 2;
  __shared__ uint32_t xsh[SHARE ? 8 : 1][SHARE ? 3 * TPW + 1 : 1][64];
  static_assert(HB == 16 || (HB == 8 && OP == G1_QKV), "half row blocks: q/k/v only");
  static_assert(KIND == 4 || (KIND == 8 && OP == G1_PLAIN && !XREC && HB == 16),
                "q8 tiles: plain GEMV only");
  constexpr int TB = KIND == 8 ? kQ8TileBytes : kQ4TileBytes;
  constexpr int NW = KIND == 8 ? 4 : 2;   // 16-byte code loads per lane and K-tile
  __shared__ float sred[G][16][16];   // [member][wave of the member][row]

  // every argument read before the weight stream, in one round of scalar loads (the empty
  // asm consumes them all at once, so the compiler cannot spread them over dependent rounds)
  const uint8_t* const w0 = a.w0;
  const uint8_t* const w1 = a.w1;
  const uint8_t* const w2 = a.w2;
  const void* const xin = XREC ? (const void*)a.att_rec : NORM ? (const void*)a.hres : (const void*)a.x;
  const uint16_t* const norm_w = a.norm_w;
  const float* const ssq_in = a.ssq_in;
  const float* const residual = a.residual;
  const int32_t* const posp = a.pos;
  const int k_t = a.k_t, n_groups = a.n_groups, grp_q = a.grp_q, grp_k = a.grp_k;
  const int att_split = a.att_split, att_g = a.att_g;
  const float rcp_g = XREC ? __builtin_amdgcn_rcpf((float)att_g) : 0.f;
  asm volatile("" ::"s"(w0), "s"(w1), "s"(w2), "s"(xin), "s"(norm_w), "s"(ssq_in), "s"(residual),
               "s"(posp), "s"(k_t), "s"(n_groups), "s"(grp_q), "s"(grp_k), "s"(att_split),
               "s"(att_g));
  __builtin_amdgcn_sched_barrier(0);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int WM = (k_t + TPW - 1) / TPW;   // waves per member (the launch gives G * WM)
  const int member = (G == 2 && wave >= WM) ? 1 : 0, chunk = wave - member * WM;
  const bool own_x = !SHARE || member == 0;   // this wave loads its activations
  const int bi = blockIdx.x;
  // HB = 16: two workgroups per group (its row blocks); HB = 8: four (the halves of each
  // row block). A group's workgroups are 8 apart, so the dispatcher puts them on one XCD.
  int group, rb, half = 0;
  if constexpr (HB == 16) {
    if ((n_groups & 7) == 0) {
      group = (bi >> 4) * 8 + (bi & 7);
      rb = (bi >> 3) & 1;
    } else {
      group = bi >> 1;
      rb = bi & 1;
    }
  } else {
    int sub;
    if ((n_groups & 7) == 0) {
      group = (bi >> 5) * 8 + (bi & 7);
      sub = (bi >> 3) & 3;
    } else {
      group = bi >> 2;
      sub = bi & 3;
    }
    rb = sub >> 1;
    half = sub & 1;
  }
  const int r0 = rb * 16 + half * 8;   // first output row of this workgroup in the tile-row
  // member tile-row and its tensor
  int tr, seg = 0, hg = group;
  const uint8_t* wseg;
  if constexpr (OP == G1_PLAIN) {
    tr = group;
    wseg = w0;
  } else if constexpr (OP == G1_GATEUP) {
    tr = group;
    wseg = member ? w1 : w0;
  } else {
    seg = group < grp_q ? 0 : group < grp_q + grp_k ? 1 : 2;
    hg = group - (seg == 0 ? 0 : seg == 1 ? grp_q : grp_q + grp_k);
    tr = 2 * hg + member;
    wseg = seg == 0 ? w0 : seg == 1 ? w1 : w2;
  }
  const int K = k_t * kTileK;
  const int qq = lane & 7, gk = lane >> 3;
  const int k0 = gk * 32 + qq * 4;                 // this lane's first K inside a tile
  // The 8 lanes of a K-group reduce their row sums in three DPP steps (partners lane ^ 7,
  // lane ^ 2, lane ^ 1). Byte slot j of a lane's code dwords is read from byte j ^ gsw, so
  // the rows a lane keeps at the first two steps sit in the same registers in every lane and
  // those steps are single DPP adds; only the last step selects. The lane finishes row R
  // (and R + RS for a 16-row block) of its workgroup. A q4 byte holds two rows (its byte
  // index is row bits 1-2), a q8 byte one (row bits 0-1).
  const int b0 = lane & 1, b1 = (lane >> 1) & 1, b2 = (lane >> 2) & 1;
  const int gsw = 2 * b2 + (b1 ^ b2);
  constexpr int RS = KIND == 8 ? 4 : 1;
  const int R = KIND == 8 ? gsw + 8 * b0 : HB == 16 ? 2 * gsw + 8 * b0 : 2 * gsw + b0;
  const int mi = gk * 32 + (HB == 16 ? rb * 16 : r0) + R;   // meta index of row R
  const int kt0 = chunk * TPW;

  // ---- 1. every load of the wave
  uint2 xv[TPW];          // bf16 x[k .. k+3]
  float4 hv[TPW];         // fp32 h[k .. k+3] (RMSNorm prologue)
  uint2 nv[TPW];          // bf16 norm_w[k .. k+3]
  float4 sq[NORM ? NSS : 1];
  float4 racc[XREC ? XNS : 1];
  float2 rml[XREC ? (XNS + 15) / 16 : 1];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int k = min(kt0 + t, k_t - 1) * kTileK + k0;
    if constexpr (XREC) {
      // attention records of this lane's head (k / 64) and its four dims (k % 64 ..): split
      // i's record is i * att_g records past split 0's (the launch has XNS == att_split).
      // The kv head is an exact float quotient (h < 2^12 and att_g <= 64, so (h + 1/2) / att_g
      // stays at least 1/128 from an integer), and the loads take 32-bit byte offsets from the
      // uniform base (one launch's records are a few hundred KB).
      const int h = k >> 6;
      const int kvh = (int)(((float)h + 0.5f) * rcp_g);
      const int hh = h - kvh * att_g;
      const uint32_t o0 = (uint32_t)((kvh * XNS * att_g + hh) * kAttnRecFloats) * 4u;
      const uint32_t oa = o0 + (uint32_t)(k & 63) * 4u, ob = o0 + 64u * 4u;
      const uint32_t rs = (uint32_t)att_g * (kAttnRecFloats * 4u);   // uniform
#pragma unroll
      for (int i = 0; i < XNS; ++i) {
        const char* ri = (const char*)xin + (size_t)((uint32_t)i * rs);   // uniform base
        racc[i] = *(const float4*)(ri + oa);
      }
      // (m, l) of one split per lane: the 16 lanes of a head (a DPP row) hold splits
      // lane % 16 (+ 16), and the merge broadcasts them along the row, so the wave loads
      // 8 bytes per lane instead of 8 per lane and split (a third of the record bytes)
#pragma unroll
      for (int u = 0; u < (XNS + 15) / 16; ++u) {
        const uint32_t s = (uint32_t)min((lane & 15) + 16 * u, XNS - 1);
        rml[u] = *(const float2*)((const char*)xin + (s * rs + ob));
      }
    } else if constexpr (NORM) {
      if (own_x) {
        hv[t] = *(const float4*)((const float*)xin + k);
        nv[t] = *(const uint2*)(norm_w + k);
      }
    } else {
      xv[t] = *(const uint2*)((const uint16_t*)xin + k);
    }
  }
  if constexpr (NORM) {
    if (own_x) ssq_load<NSS>(ssq_in, lane, K / kSsqRows, sq);
  }
  // the epilogue's own inputs (thread r < 16 owns output row r of each member): the residual
  // (plain), the sequence position (q/k/v)
  const int er = tid & 15;
  float ep_res = 0.f;
  int ep_pos = 0;
  if constexpr (OP == G1_PLAIN) {
    const float* rp = residual != nullptr ? residual + (int64_t)tr * 32 + rb * 16 + er
                                            : (const float*)w0;
    ep_res = *rp;
  }
  // The position is one word for the whole workgroup: read through the scalar path. As a
  // vector load the compiler made it scalar with a readfirstlane placed before the barrier
  // below, whose wait (the in-order vector load counter) then held the weight stream back
  // until every activation load had arrived.
  if constexpr (OP == G1_QKV) ep_pos = *(const __attribute__((address_space(4))) int32_t*)posp;
  // The vector L1 returns a wave's loads in issue order, so a small activation load queued
  // behind other waves' weight misses waits for them. Every wave of the workgroup issues its
  // activation loads before any issues a weight load (an execution barrier only: nothing
  // waits for memory here).
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  uint4 wq[TPW][NW];
  uint32_t md[TPW], mm[TPW];
  {
    const uint8_t* rowp = wseg + (size_t)tr * k_t * TB;
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const uint8_t* tile = rowp + (size_t)min(kt0 + t, k_t - 1) * TB;
      const uint4* src = KIND == 8 ? (const uint4*)(tile + kMetaBytes + rb * 4096 + lane * 64)
                                   : (const uint4*)(tile + 2 * kMetaBytes + rb * 2048 + lane * 32);
#pragma unroll
      for (int c = 0; c < NW; ++c) wq[t][c] = src[c];
      if constexpr (KIND == 8) {   // the scales of rows R and R + 4
        md[t] = (uint32_t)*(const uint16_t*)(tile + 2 * mi) |
                ((uint32_t)*(const uint16_t*)(tile + 2 * (mi + RS)) << 16);
        mm[t] = 0;
      } else if constexpr (HB == 16) {
        md[t] = *(const uint32_t*)(tile + 2 * mi);
        mm[t] = *(const uint32_t*)(tile + kMetaBytes + 2 * mi);
      } else {
        md[t] = *(const uint16_t*)(tile + 2 * mi);
        mm[t] = *(const uint16_t*)(tile + kMetaBytes + 2 * mi);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // wave slots this workgroup has no wave for add zero in the fixed 16-term sum of step 6
  for (int i = tid; i < G * 256; i += G * WM * 64)
    if (((i >> 4) & 15) >= WM) sred[i >> 8][(i >> 4) & 15][i & 15] = 0.f;

  // ---- 2. activations: as given, RMSNorm of h, or merged attention records; bf16 bits
  uint2 xr[TPW];
  if constexpr (XREC) {   // the split merge of attention's own finish, in split order
    // M over the head's splits (a max: any order gives the same value), then split s's
    // weight exp2(m_s - M) from the lane that holds it, broadcast with l_s along the row
    constexpr int XMU = (XNS + 15) / 16;
    float mj[XMU], fj[XMU];
    float M = -INFINITY;
#pragma unroll
    for (int u = 0; u < XMU; ++u) {
      mj[u] = (lane & 15) + 16 * u < XNS ? rml[u].x : -INFINITY;
      M = fmaxf(M, mj[u]);
    }
    M = group16_max(M);
    // an empty head (every m = -inf) weighs its zero records by exp2(-inf) = 0
    const float Mb = M == -INFINITY ? 0.f : M;
#pragma unroll
    for (int u = 0; u < XMU; ++u) fj[u] = __builtin_amdgcn_exp2f(mj[u] - Mb);
    float L = 0.f, A0 = 0.f, A1 = 0.f, A2 = 0.f, A3 = 0.f;
    static_for<0, XNS>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      const float f = dpp<kDppRowBcast + (i & 15)>(fj[i / 16]);
      const float l = dpp<kDppRowBcast + (i & 15)>(rml[i / 16].y);
      L = fmaf(l, f, L);
      A0 = fmaf(racc[i].x, f, A0);
      A1 = fmaf(racc[i].y, f, A1);
      A2 = fmaf(racc[i].z, f, A2);
      A3 = fmaf(racc[i].w, f, A3);
    });
    const float o0 = L > 0.f ? attn_div(A0, L) : 0.f, o1 = L > 0.f ? attn_div(A1, L) : 0.f;
    const float o2 = L > 0.f ? attn_div(A2, L) : 0.f, o3 = L > 0.f ? attn_div(A3, L) : 0.f;
    xr[0] = make_uint2(pack_bf16x2_op(o0, o1), pack_bf16x2_op(o2, o3));
  } else if constexpr (NORM) {
    if (own_x) {
      const float inv = rms_inv(wave_sum(ssq_lane_sum<NSS>(sq, lane, K / kSsqRows)), K, a.eps);
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const float n0 = (hv[t].x * inv) * bf16lo(nv[t].x), n1 = (hv[t].y * inv) * bf16hi(nv[t].x);
        const float n2 = (hv[t].z * inv) * bf16lo(nv[t].y), n3 = (hv[t].w * inv) * bf16hi(nv[t].y);
        xr[t] = make_uint2(pack_bf16x2_op(n0, n1), pack_bf16x2_op(n2, n3));
        // the stored row keeps NaN payloads as every bf16 output does
        if (a.xn_out != nullptr && group == 0 && rb == 0 && member == 0 && kt0 + t < a.k_t)
          *(uint2*)(a.xn_out + (kt0 + t) * kTileK + k0) =
              make_uint2(pack_bf16x2(n0, n1), pack_bf16x2(n2, n3));
      }
    }
  } else {
#pragma unroll
    for (int t = 0; t < TPW; ++t) xr[t] = xv[t];
  }
  // RoPE cos/sin of this thread's output dim, now that the position is here
  float ep_c = 0.f, ep_s = 0.f;
  if constexpr (OP == G1_QKV) {
    const bool ok = ep_pos >= 0 && ep_pos < a.max_pos;
    const float* tb = ok ? a.rope_tab + (int64_t)ep_pos * 64 + r0 + (er & (HB - 1)) : a.rope_tab;
    ep_c = tb[0];
    ep_s = tb[32];
  }

  // ---- 3. fp16 conversion with one power-of-two scale 2^se per K-group of 8 lanes (the
  // lanes whose products are summed before the group's scale and minimum apply). The largest
  // |x| is taken on the bf16 bits: its exponent field E bounds it by 2^(E - 126), and
  // se = 141 - E brings it under 2^15, inside fp16's range. (A wave's clamped duplicate of
  // the last K-tile repeats values the wave already holds, so it never changes the max.)
  int se = 0;
  uint32_t xp[TPW][2];
  float Xs[TPW];
  if (own_x) {
    uint32_t am = 0;
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const uint32_t u = xr[t].x, v = xr[t].y;
      am = max(am, max(max(__builtin_amdgcn_ubfe(u, 0, 15), __builtin_amdgcn_ubfe(u, 16, 15)),
                       max(__builtin_amdgcn_ubfe(v, 0, 15), __builtin_amdgcn_ubfe(v, 16, 15))));
    }
    am = max(am, dpp_u<kDppXor1>(am));
    am = max(am, dpp_u<kDppXor2>(am));
    am = max(am, dpp_u<kDppHalfMirror>(am));
    se = min(141 - (int)(am >> 7), 120);   // zero / subnormal groups: 2^120
    const float xs = __uint_as_float((uint32_t)(se + 127) << 23);
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      half2_t h;
      h.x = (_Float16)(bf16lo(xr[t].x) * xs);
      h.y = (_Float16)(bf16hi(xr[t].x) * xs);
      xp[t][0] = h2_bits(h);
      h.x = (_Float16)(bf16lo(xr[t].y) * xs);
      h.y = (_Float16)(bf16hi(xr[t].y) * xs);
      xp[t][1] = h2_bits(h);
    }
    // sum of the K-group's x (the minimum's factor) per tile, with the activation scale undone
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      float X = dot2_0(xp[t][0], 0x3C003C00u);
      X = dot2(xp[t][1], 0x3C003C00u, X);
      X += dpp<kDppHalfMirror>(X);
      X += dpp<kDppXor2>(X);
      X += dpp<kDppXor1>(X);
      Xs[t] = __builtin_amdgcn_ldexpf(X, -se);
    }
  }
  if constexpr (SHARE) {   // member 0's chunk hands its converted activations to member 1's
    if (member == 0) {
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        xsh[chunk][3 * t][lane] = xp[t][0];
        xsh[chunk][3 * t + 1][lane] = xp[t][1];
        xsh[chunk][3 * t + 2][lane] = __float_as_uint(Xs[t]);
      }
      xsh[chunk][3 * TPW][lane] = (uint32_t)se;
    }
    __syncthreads();
    if (member == 1) {
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        xp[t][0] = xsh[chunk][3 * t][lane];
        xp[t][1] = xsh[chunk][3 * t + 1][lane];
        Xs[t] = __uint_as_float(xsh[chunk][3 * t + 2][lane]);
      }
      se = (int)xsh[chunk][3 * TPW][lane];
    }
  }
  const int ur = 20 - se;
  uint32_t sl[4];   // v_perm selectors of the lane's byte slots
#pragma unroll
  for (int j = 0; j < 4; ++j) sl[j] = sel_pair(j ^ gsw);
  // Everything above needs only the activations, which land before the weights: it runs
  // while the weight stream is still in flight, and the work after the last weight byte
  // is only the tile arithmetic below.
  __builtin_amdgcn_sched_barrier(0);

  // ---- 4. tiles (r * 2^20 undoes the codes' 2^-20; the sums carry the activation scale)
  float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const bool live = kt0 + t < a.k_t;   // always true for t = 0
    if constexpr (KIND == 8) {
      // q8: the 16 bytes of load c are rows 0-15 at k = k0 + c; biased by 128 (xor 0x80) a
      // code is the fp16 subnormal (c + 128) * 2^-24. pv[4 dw + j] is row 4 dw + (j ^ gsw).
      float pv[16] = {};
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const uint4 A = wq[t][2 * c], B = wq[t][2 * c + 1];
        const uint32_t av[4] = {A.x ^ 0x80808080u, A.y ^ 0x80808080u, A.z ^ 0x80808080u,
                                A.w ^ 0x80808080u};
        const uint32_t bv[4] = {B.x ^ 0x80808080u, B.y ^ 0x80808080u, B.z ^ 0x80808080u,
                                B.w ^ 0x80808080u};
        const uint32_t xc = xp[t][c];
#pragma unroll
        for (int dw = 0; dw < 4; ++dw)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            pv[4 * dw + j] = dot2_acc(perm(bv[dw], av[dw], sl[j]), xc, pv[4 * dw + j], c == 0);
      }
      // partners: lane ^ 7 holds row s ^ 2 of this lane's slot s in slot s + 2 (s bit 1 clear),
      // lane ^ 2 holds it in slot s + 1 (s bit 0 clear); then rows gsw + 4v in t4[v]
      float t8[8], t4[4], r2[2];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int sl8 = (u & 1) + 4 * (u >> 1);
        t8[u] = pv[sl8] + dpp<kDppHalfMirror>(pv[sl8 + 2]);
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) t4[v] = t8[2 * v] + dpp<kDppXor2>(t8[2 * v + 1]);
#pragma unroll
      for (int i = 0; i < 2; ++i) {   // lane ^ 1 keeps the other two of the four rows
        const float keep = b0 ? t4[i + 2] : t4[i], send = b0 ? t4[i] : t4[i + 2];
        r2[i] = keep + dpp<kDppXor1>(send);
      }
      // s * sum(c x) = s * (sum((c + 128) x) - 128 sum(x))
      const float Xb = 128.0f * Xs[t];
      const float c0 = bf16lo(md[t]) * (__builtin_amdgcn_ldexpf(r2[0], ur + 4) - Xb);
      const float c1 = bf16hi(md[t]) * (__builtin_amdgcn_ldexpf(r2[1], ur + 4) - Xb);
      acc0 = t == 0 ? c0 : acc0 + (live ? c0 : 0.f);
      acc1 = t == 0 ? c1 : acc1 + (live ? c1 : 0.f);
    } else if constexpr (HB == 16) {
      // pv[8 dw + 2 j + nib]: dword dw (rows 0-7 / 8-15), byte j ^ gsw, low / high nibble,
      // i.e. row 8 dw + 2 (j ^ gsw) + nib, summed over the lane's 4 K
      float pv[16] = {};
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        // dwords: rows 0-7 at k, rows 8-15 at k, rows 0-7 at k+1, rows 8-15 at k+1; the low
        // nibble of byte i is row 2i, the high nibble row 2i + 1. Both go to bits 4-7: a
        // code in bits 0-3 (the subnormal c * 2^-24, one mask instead of a shift and a mask)
        // measured 4x the error against the float64 oracle (5e-7 against 1.2e-7 of max|y|),
        // as v_dot2_f32_f16 keeps fewer bits of subnormals with leading zeros.
        const uint4 w = wq[t][c];
        const uint32_t Lx = (w.x << 4) & 0xF0F0F0F0u, Ly = (w.y << 4) & 0xF0F0F0F0u;
        const uint32_t Lz = (w.z << 4) & 0xF0F0F0F0u, Lw = (w.w << 4) & 0xF0F0F0F0u;
        const uint32_t Hx = w.x & 0xF0F0F0F0u, Hy = w.y & 0xF0F0F0F0u;
        const uint32_t Hz = w.z & 0xF0F0F0F0u, Hw = w.w & 0xF0F0F0F0u;
        const uint32_t xc = xp[t][c];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          pv[2 * j] = dot2_acc(perm(Lz, Lx, sl[j]), xc, pv[2 * j], c == 0);
          pv[2 * j + 1] = dot2_acc(perm(Hz, Hx, sl[j]), xc, pv[2 * j + 1], c == 0);
          pv[8 + 2 * j] = dot2_acc(perm(Lw, Ly, sl[j]), xc, pv[8 + 2 * j], c == 0);
          pv[8 + 2 * j + 1] = dot2_acc(perm(Hw, Hy, sl[j]), xc, pv[8 + 2 * j + 1], c == 0);
        }
      }
      // 16 rows over the 8 lanes of the K-group. Slot s holds row s ^ (2 gsw), and gsw
      // differs by 2 between lane and lane ^ 7 and by 1 between lane and lane ^ 2: the
      // partner's slot s + 4 (s + 2) holds the row of this lane's slot s.
      float t8[8], t4[4], r2[2];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int s = (u & 3) + 8 * (u >> 2);
        t8[u] = pv[s] + dpp<kDppHalfMirror>(pv[s + 4]);
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int u = (v & 1) + 4 * (v >> 1);
        t4[v] = t8[u] + dpp<kDppXor2>(t8[u + 2]);
      }
      // t4: rows 2 gsw, +1, +8, +9, the same in lane ^ 1, which keeps the other pair
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float keep = b0 ? t4[i + 2] : t4[i], send = b0 ? t4[i] : t4[i + 2];
        r2[i] = keep + dpp<kDppXor1>(send);
      }
      const float c0 = fmaf(bf16lo(md[t]), __builtin_amdgcn_ldexpf(r2[0], ur), bf16lo(mm[t]) * Xs[t]);
      const float c1 = fmaf(bf16hi(md[t]), __builtin_amdgcn_ldexpf(r2[1], ur), bf16hi(mm[t]) * Xs[t]);
      acc0 = t == 0 ? c0 : acc0 + (live ? c0 : 0.f);
      acc1 = t == 0 ? c1 : acc1 + (live ? c1 : 0.f);
    } else {
      // the 8 rows of this half: one dword at k and one at k + 1 of each 16-byte load;
      // pv[2 j + nib] is row 2 (j ^ gsw) + nib of the half
      float pv[8] = {};
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const uint4 w = wq[t][c];
        const uint32_t a0 = half ? w.y : w.x, a1 = half ? w.w : w.z;
        const uint32_t L0 = (a0 << 4) & 0xF0F0F0F0u, L1 = (a1 << 4) & 0xF0F0F0F0u;
        const uint32_t H0 = a0 & 0xF0F0F0F0u, H1 = a1 & 0xF0F0F0F0u;
        const uint32_t xc = xp[t][c];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          pv[2 * j] = dot2_acc(perm(L1, L0, sl[j]), xc, pv[2 * j], c == 0);
          pv[2 * j + 1] = dot2_acc(perm(H1, H0, sl[j]), xc, pv[2 * j + 1], c == 0);
        }
      }
      // 8 rows over the 8 lanes of the K-group, as above; lane ^ 1 shares rows 2 gsw, +1
      float t4[4], t2[2];
#pragma unroll
      for (int u = 0; u < 4; ++u) t4[u] = pv[u] + dpp<kDppHalfMirror>(pv[u + 4]);
#pragma unroll
      for (int v = 0; v < 2; ++v) t2[v] = t4[v] + dpp<kDppXor2>(t4[v + 2]);
      const float keep = b0 ? t2[1] : t2[0], send = b0 ? t2[0] : t2[1];
      const float r1 = keep + dpp<kDppXor1>(send);
      const float c0 = fmaf(bf16lo(md[t]), __builtin_amdgcn_ldexpf(r1, ur), bf16lo(mm[t]) * Xs[t]);
      acc0 = t == 0 ? c0 : acc0 + (live ? c0 : 0.f);
    }
  }

  // ---- 5. sum over the 8 K-groups (lane bits 3..5)
  if constexpr (HB == 16) {
    // v_permlane16_swap(a, b) leaves rows (a0, b0, a2, b2) and (a1, b1, a3, b3): their sum
    // carries row R's partial sums in the even 16-lane rows and row R + 1's in the odd ones
    const float v0 = acc0 + dpp<kDppRor8>(acc0), v1 = acc1 + dpp<kDppRor8>(acc1);
    const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(v0), __float_as_uint(v1),
                                                     false, false);
    const float p = xor32_sum(__uint_as_float(sw[0]) + __uint_as_float(sw[1]));
    if (lane < 8) sred[member][chunk][R] = p;
    else if (lane >= 16 && lane < 24) sred[member][chunk][R + RS] = p;
  } else {
    float v0 = acc0 + dpp<kDppRor8>(acc0);
    v0 = xor32_sum(xor16_sum(v0));
    if (lane < 8) sred[member][chunk][R] = v0;
  }
  __syncthreads();
  if (tid >= 64) return;

  // ---- 6, 7. the wave slots in a fixed order, then the epilogue
  if constexpr (OP != G1_QKV) {
    finish_block<OP, G>(a, sred, tid, tr, rb, ep_res);
  } else {   // QKV: dims d and d + 32 of one head, d = r0 + r (thread r < HB)
    float s[G];
    slot_sums<G>(sred, er & (HB - 1), s);
    if (tid < HB) {
      const int d = r0 + er;
      const int seg_off = seg == 0 ? 0 : seg == 1 ? a.n_q_heads * 64 : (a.n_q_heads + a.n_kv_heads) * 64;
      if (a.raw_out != nullptr) {
        a.raw_out[seg_off + hg * 64 + d] = s[0];
        a.raw_out[seg_off + hg * 64 + 32 + d] = s[1];
      }
      const float x0 = bf16_to_f32(f32_to_bf16(s[0]));
      const float x1 = bf16_to_f32(f32_to_bf16(s[1]));
      const int p = ep_pos;
      if (p >= 0 && p < a.max_pos) {
        if (seg == 2) {
          uint16_t* dst = a.v_cache + hg * a.kv_h_stride + (int64_t)p * 64;
          dst[d] = f32_to_bf16(x0);
          dst[32 + d] = f32_to_bf16(x1);
        } else {
          const float y0 = fmaf(x0, ep_c, -(x1 * ep_s));
          const float y1 = fmaf(x1, ep_c, x0 * ep_s);
          uint16_t* dst = seg == 0 ? a.q_out + hg * 64
                                   : a.k_cache + hg * a.kv_h_stride + (int64_t)p * 64;
          dst[d] = f32_to_bf16(y0);
          dst[32 + d] = f32_to_bf16(y1);
        }
      }
    }
  }
}

// ------------------------------------------------------------------ host side

// K-tiles per wave: the fewest (1, 2 or 4) that fit the group's K into 16 waves; 0 if none.
int gemv1_tpw(int G, int k_t) {
  for (int tpw = 1; tpw <= 4; tpw *= 2)
    if (G * ((k_t + tpw - 1) / tpw) <= 16) return tpw;
  return 0;
}

bool gemv1_fits(int G, int k_t, bool norm) {
  if (k_t < 1 || gemv1_tpw(G, k_t) == 0) return false;
  return !norm || k_t * kTileK / kSsqRows <= 512;
}

// blocks: workgroups of 16-row blocks (two per group); HB = 8 launches twice as many
template <int OP, int G, int TPW, int NSS, int XNS, int KIND = 4>
static void go(const Gemv1Args& a, int blocks, int threads, hipStream_t s) {
  constexpr int HB = OP == G1_QKV ? 8 : 16;
  hipLaunchKernelGGL((gemv1_kernel<OP, G, TPW, NSS, XNS, HB, KIND>),
                     dim3(HB == 8 ? 2 * blocks : blocks), dim3(threads), 0, s, a);
}

template <int OP, int G, int TPW, int KIND>
static void go_norm(const Gemv1Args& a, int blocks, int threads, hipStream_t s) {
  if (a.norm_w == nullptr) go<OP, G, TPW, 0, 0, KIND>(a, blocks, threads, s);
  else if (a.k_t * kTileK / kSsqRows <= 256) go<OP, G, TPW, 1, 0, KIND>(a, blocks, threads, s);
  else go<OP, G, TPW, 2, 0, KIND>(a, blocks, threads, s);
}

template <int OP, int G, int KIND = 4>
static void go_tpw(const Gemv1Args& a, int tpw, int blocks, int threads, hipStream_t s) {
  switch (tpw) {
    case 1: go_norm<OP, G, 1, KIND>(a, blocks, threads, s); break;
    case 2: go_norm<OP, G, 2, KIND>(a, blocks, threads, s); break;
    default: go_norm<OP, G, 4, KIND>(a, blocks, threads, s); break;
  }
}

int gemv1_launch(int op, const Gemv1Args& a, hipStream_t s, const char* what, int kind,
                 int tpw_req) {
  const int G = op == G1_PLAIN ? 1 : 2;
  const int tpw = tpw_req ? tpw_req : gemv1_tpw(G, a.k_t);
  Q4NX_REQUIRE(tpw > 0, Q4NX_ERR_SHAPE, "%s: K=%d is longer than one workgroup covers", what,
               a.k_t * kTileK);
  Q4NX_REQUIRE(G * ((a.k_t + tpw - 1) / tpw) <= 16, Q4NX_ERR_ARG,
               "%s: %d K-tiles per wave leave more than 16 waves per workgroup at K=%d", what,
               tpw, a.k_t * kTileK);
  Q4NX_REQUIRE(kind == 4 || (kind == 8 && op == G1_PLAIN), Q4NX_ERR_ARG,
               "%s: the row-block kernels take q8 tiles for a plain GEMV only", what);
  const int threads = G * ((a.k_t + tpw - 1) / tpw) * 64;
  const int blocks = 2 * a.n_groups;
  if (op == G1_PLAIN && kind == 8) go_tpw<G1_PLAIN, 1, 8>(a, tpw, blocks, threads, s);
  else if (op == G1_PLAIN) go_tpw<G1_PLAIN, 1>(a, tpw, blocks, threads, s);
  else if (op == G1_GATEUP) go_tpw<G1_GATEUP, 2>(a, tpw, blocks, threads, s);
  else go_tpw<G1_QKV, 2>(a, tpw, blocks, threads, s);
  return check_launch(what);
}

// The records prologue is compiled for each split count (its loads and merge unrolled
// exactly, with no masks).
template <int NS>
static void go_splits(const Gemv1Args& a, int blocks, int threads, hipStream_t s) {
  if constexpr (NS < kAttnRecMaxSplits) {
    if (a.att_split != NS) return go_splits<NS + 1>(a, blocks, threads, s);
  }
  go<G1_PLAIN, 1, 1, 0, NS>(a, blocks, threads, s);
}

// The o-projection from attention records: one K-tile (four heads) per wave.
int gemv1_attn_launch(const Gemv1Args& a, hipStream_t s, const char* what) {
  Q4NX_REQUIRE(a.k_t >= 1 && a.k_t <= kAttnRecMaxKTiles, Q4NX_ERR_SHAPE,
               "%s: %d K-tiles (at most %d)", what, a.k_t, kAttnRecMaxKTiles);
  Q4NX_REQUIRE(a.att_split >= 1 && a.att_split <= kAttnRecMaxSplits, Q4NX_ERR_SHAPE,
               "%s: %d splits (1..%d)", what, a.att_split, kAttnRecMaxSplits);
  const int blocks = 2 * a.n_groups, threads = a.k_t * 64;
  go_splits<1>(a, blocks, threads, s);
  return check_launch(what);
}

}  // namespace q4nx
