// GQA flash-decode attention for gfx950.
//
// Reference: designs/granite_gemv/granite_attention.h:80-213 (online softmax over 32-position
// KV blocks on one AIE core, one q head per design, scale*log2e folded in fp32 so the
// softmax is a pure exp2, :65-72) and its fp64 check granite_attention.py:163-167.
//
// One workgroup owns (sequence b, kv head, KV split): all Hq/Hkv query heads of the group
// share every K/V row it loads. Splits cover [0, max_len) in equal chunks so that every
// address is known at launch and the first loads go out before the sequence length has
// arrived; positions at or past the sequence's length are masked (and whole rounds past
// it are skipped). The last workgroup of a (b, kv head) merges the splits' (m, l, acc)
// exactly, in split order.
//
// Lanes: 8 lanes per KV position (8 head dims = 16 bytes each), 8 positions per wave step,
// so one wave instruction reads 1 KB of contiguous cache rows. A round is 4 steps per wave
// (128 positions per workgroup); the next round's loads are issued before the current one
// is computed. q.k is v_dot2_f32_bf16 (exact bf16 products, fp32 sums) completed across
// the 8 lanes with DPP; every lane then runs its own online softmax over the positions it
// saw (p.v in fp32) and the 32 lane states of the workgroup are merged once, in parallel,
// through LDS. Scores are scaled by scale*log2(e) so the softmax is exp2.

#include <atomic>
#include <math.h>

#include <mutex>

#include "common.h"
#include "policy.h"

namespace q4nx {

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* out;
  float* out_f32;
  const int32_t* lens;
  int batch, hq, hkv, n_split, chunk, max_len;
  int64_t kv_b_stride, kv_h_stride;
  float scale_l2;  // scale * log2(e)
  float* partial;  // [b*hkv + kvh][n_split][G][kPartStride]
  uint32_t partial_bytes;
  unsigned* counters;
  int publish_only;   // every split writes its record and ends; a later launch merges
};

typedef short bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kAttnWaves = 4;
constexpr int kAttnSteps = 4;                              // 8-position steps per round
constexpr int kAttnRound = kAttnWaves * kAttnSteps * 8;    // positions per workgroup round
constexpr int kAttnStates = kAttnWaves * 8;                // lane softmax states per WG
constexpr int kPartStride = kAttnRecFloats;                // acc[64], m, l, 2 pad (16 B rows)
constexpr int kMergeSplits = 20;   // splits merged per pass (loads in flight per output)

__device__ __forceinline__ float dot2bf(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                        __builtin_bit_cast(bf16x2_t, b), c, false);
}

// v_exp_f32: 2^x; results below 2^-126 flush to zero (they cannot move an fp32 sum of
// terms of which the largest is 1).
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

template <int G>
struct AttnLane {
  uint4 q[G];
  float m[G], l[G], acc[G][8];
};

template <int G>
__device__ __forceinline__ void attn_load(const uint16_t* kbase, const uint16_t* vbase, int r0,
                                          int stop, int wave, int pl, uint4 (&kr)[kAttnSteps],
                                          uint4 (&vr)[kAttnSteps]) {
#pragma unroll
  for (int s = 0; s < kAttnSteps; ++s) {
    const int t = r0 + (wave * kAttnSteps + s) * 8 + pl;
    const size_t row = (size_t)(t < stop ? t : 0) * 64;   // a valid row for masked lanes
    kr[s] = *(const uint4*)(kbase + row);
    vr[s] = *(const uint4*)(vbase + row);
  }
}

template <int G>
__device__ __forceinline__ void attn_round(AttnLane<G>& st, const uint4 (&kr)[kAttnSteps],
                                           const uint4 (&vr)[kAttnSteps], int r0, int end,
                                           int wave, int pl, float scale_l2) {
  float sc[kAttnSteps][G];
  uint4 vm[kAttnSteps];   // V rows, zero past the length (p = 0 there, and 0 * NaN is NaN)
#pragma unroll
  for (int s = 0; s < kAttnSteps; ++s) {
    const bool ok = r0 + (wave * kAttnSteps + s) * 8 + pl < end;
    vm[s] = ok ? vr[s] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float d = dot2bf(st.q[h].x, kr[s].x, 0.f);
      d = dot2bf(st.q[h].y, kr[s].y, d);
      d = dot2bf(st.q[h].z, kr[s].z, d);
      d = dot2bf(st.q[h].w, kr[s].w, d);
      // all-reduce over the 8 lanes of the position: every lane ends with the same sum
      d += dpp<kDppXor1>(d);
      d += dpp<kDppXor2>(d);
      d += dpp<kDppHalfMirror>(d);
      sc[s][h] = ok ? d * scale_l2 : -INFINITY;
    }
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float mr = sc[0][h];
#pragma unroll
    for (int s = 1; s < kAttnSteps; ++s) mr = fmaxf(mr, sc[s][h]);
    const float mn = fmaxf(st.m[h], mr);
    if (mn != -INFINITY) {
      const float corr = ex2(st.m[h] - mn);   // 0 while nothing was seen (m = -inf)
      st.l[h] *= corr;
#pragma unroll
      for (int i = 0; i < 8; ++i) st.acc[h][i] *= corr;
#pragma unroll
      for (int s = 0; s < kAttnSteps; ++s) {
        const float p = ex2(sc[s][h] - mn);   // masked positions: 2^-inf = 0
        st.l[h] += p;
        const uint32_t vv[4] = {vm[s].x, vm[s].y, vm[s].z, vm[s].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          st.acc[h][2 * i] = fmaf(p, bf16lo(vv[i]), st.acc[h][2 * i]);
          st.acc[h][2 * i + 1] = fmaf(p, bf16hi(vv[i]), st.acc[h][2 * i + 1]);
        }
      }
      st.m[h] = mn;
    }
  }
}

// One pass of the split merge for this thread's outputs (thread t of TH owns outputs t,
// t + TH, .. = (head e / 64, dim e % 64)): the (m, l, acc[dim]) of splits cs .. cs + ns - 1
// (ns <= P), all loaded at once (past ns the last record again, masked), then folded into the
// running (M, L, A) in split order.
template <int G, int P, int TH>
__device__ __forceinline__ void attn_merge_pass(const float* recs, int cs, int ns,
                                                float (&M)[(G * 64 + TH - 1) / TH],
                                                float (&L)[(G * 64 + TH - 1) / TH],
                                                float (&A)[(G * 64 + TH - 1) / TH]) {
  constexpr int kE = (G * 64 + TH - 1) / TH;
  float mv[kE][P], lv[kE][P], av[kE][P];
#pragma unroll
  for (int j = 0; j < kE; ++j) {
    const int e = min((int)threadIdx.x + TH * j, G * 64 - 1);
    const int h = e >> 6, d = e & 63;
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const float* r = recs + ((size_t)(cs + min(i, ns - 1)) * G + h) * kPartStride;
      mv[j][i] = load_sys(r + 64);
      lv[j][i] = load_sys(r + 65);
      av[j][i] = load_sys(r + d);
    }
  }
#pragma unroll
  for (int j = 0; j < kE; ++j) {
    float Mn = M[j];
#pragma unroll
    for (int i = 0; i < P; ++i)
      if (i < ns) Mn = fmaxf(Mn, mv[j][i]);
    if (Mn != -INFINITY) {
      const float g = ex2(M[j] - Mn);   // 0 while nothing was merged (M = -inf)
      float Ln = L[j] * g, An = A[j] * g;
#pragma unroll
      for (int i = 0; i < P; ++i)
        if (i < ns) {
          const float f = ex2(mv[j][i] - Mn);
          Ln = fmaf(lv[j][i], f, Ln);
          An = fmaf(av[j][i], f, An);
        }
      M[j] = Mn;
      L[j] = Ln;
      A[j] = An;
    }
  }
}

// The end both kernels share. s_fin[h] holds the workgroup's (acc[64], m, l) for query head
// h of the group. With one split that is the answer; otherwise the record is published and
// the last workgroup of the (sequence, kv head) to arrive merges every split's record
// exactly, in split order (kMergeSplits records per pass).
// TH: threads of the workgroup (each thread merges outputs tid, tid + TH, ..).
template <int G, int TH = 256>
__device__ __forceinline__ void attn_finish(const AttnArgs& a, float (*s_fin)[kPartStride],
                                            int* s_last, int bk, int split, int b, int kvh) {
  const int tid = threadIdx.x;
  if (a.publish_only || a.n_split > 1) {
    // publish this split's (acc, m, l), then the last workgroup of (b, kv head) merges (or,
    // publishing only, a later launch does)
    const __amdgpu_buffer_rsrc_t pr = make_rsrc(a.partial, a.partial_bytes);
    const uint32_t rec_bytes = G * kPartStride * 4;
    const uint32_t rec = (uint32_t)((size_t)bk * a.n_split + split) * rec_bytes;
    for (int e = tid; e < G * kPartStride / 4; e += TH)
      st16_sys(pr, rec + e * 16, ((const uint4*)&s_fin[0][0])[e]);
    if (a.publish_only) return;
    wait_vm();
    __syncthreads();
    if (tid == 0) {
      *s_last = ticket(&a.counters[bk], a.n_split) ? 1 : 0;
    }
    __syncthreads();
    if (!*s_last) return;

    // every thread merges its own output columns over the split records, straight from
    // memory: one round of loads per pass, no staging through LDS, no barriers
    constexpr int kE = (G * 64 + TH - 1) / TH;   // outputs per thread
    const float* recs = a.partial + (size_t)bk * a.n_split * G * kPartStride;
    float M[kE], L[kE], A[kE];
#pragma unroll
    for (int j = 0; j < kE; ++j) {
      M[j] = -INFINITY;
      L[j] = 0.f;
      A[j] = 0.f;
    }
    for (int cs = 0; cs < a.n_split; cs += kMergeSplits) {
      const int ns = min(kMergeSplits, a.n_split - cs);
      if (ns <= 8) attn_merge_pass<G, 8, TH>(recs, cs, ns, M, L, A);
      else attn_merge_pass<G, kMergeSplits, TH>(recs, cs, ns, M, L, A);
    }
#pragma unroll
    for (int j = 0; j < kE; ++j) {
      const int e = tid + TH * j;
      if (e < G * 64) {
        const int h = e >> 6, d = e & 63;
        s_fin[h][d] = A[j];
        if (d == 0) {
          s_fin[h][64] = M[j];
          s_fin[h][65] = L[j];
        }
      }
    }
    __syncthreads();
  }

  for (int e = tid; e < G * 64; e += TH) {
    const int h = e >> 6, d = e & 63;
    const float Ls = s_fin[h][65];
    const float o = Ls > 0.f ? attn_div(s_fin[h][d], Ls) : 0.f;   // an empty sequence: 0
    const size_t oi = ((size_t)b * a.hq + kvh * G + h) * 64 + d;
    if (a.out) a.out[oi] = f32_to_bf16(o);
    if (a.out_f32) a.out_f32[oi] = o;
  }
}

template <int G>
__global__ __launch_bounds__(256) void gqa_decode_kernel(AttnArgs a) {
  static_assert(G * 32 <= 256, "one thread per (head, lane state)");
  __shared__ float s_m[G][kAttnStates], s_f[G][kAttnStates];
  __shared__ __attribute__((aligned(16))) float s_acc[kAttnStates * G * 64];
  __shared__ __attribute__((aligned(16))) float s_fin[G][kPartStride];
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int blk = blockIdx.x;
  const int split = blk % a.n_split;
  const int bk = blk / a.n_split;  // b * hkv + kvh
  const int kvh = bk % a.hkv;
  const int b = bk / a.hkv;
  const int start = split * a.chunk;
  const int stop = min(start + a.chunk, a.max_len);

  const int dg = lane & 7;   // dims dg*8 .. +8
  const int pl = lane >> 3;  // position within the wave step
  const size_t head_off = (size_t)b * a.kv_b_stride + (size_t)kvh * a.kv_h_stride + dg * 8;
  const uint16_t* kbase = a.k + head_off;
  const uint16_t* vbase = a.v + head_off;

  // first round's K/V, q and the length all in flight together
  uint4 kA[kAttnSteps], vA[kAttnSteps], kB[kAttnSteps], vB[kAttnSteps];
  attn_load<G>(kbase, vbase, start, stop, wave, pl, kA, vA);
  AttnLane<G> st;
#pragma unroll
  for (int h = 0; h < G; ++h) {
    st.q[h] = *(const uint4*)(a.q + ((size_t)b * a.hq + kvh * G + h) * 64 + dg * 8);
    st.m[h] = -INFINITY;
    st.l[h] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) st.acc[h][i] = 0.f;
  }
  const int end = min(stop, max(0, a.lens[b]));
  const int nr = end > start ? (end - start + kAttnRound - 1) / kAttnRound : 0;
  for (int r = 0; r < nr; r += 2) {
    const int r0 = start + r * kAttnRound;
    if (r + 1 < nr) attn_load<G>(kbase, vbase, r0 + kAttnRound, stop, wave, pl, kB, vB);
    attn_round<G>(st, kA, vA, r0, end, wave, pl, a.scale_l2);
    if (r + 2 < nr) attn_load<G>(kbase, vbase, r0 + 2 * kAttnRound, stop, wave, pl, kA, vA);
    if (r + 1 < nr) attn_round<G>(st, kB, vB, r0 + kAttnRound, end, wave, pl, a.scale_l2);
  }

  // ---- merge the 32 lane states (4 waves x 8 position lanes) of the workgroup
  const int j = wave * 8 + pl;
#pragma unroll
  for (int h = 0; h < G; ++h) {
    if (dg == 0) {
      s_m[h][j] = st.m[h];
      s_f[h][j] = st.l[h];
    }
    float4* dst = (float4*)(s_acc + (j * G + h) * 64 + dg * 8);
    dst[0] = make_float4(st.acc[h][0], st.acc[h][1], st.acc[h][2], st.acc[h][3]);
    dst[1] = make_float4(st.acc[h][4], st.acc[h][5], st.acc[h][6], st.acc[h][7]);
  }
  __syncthreads();
  if (tid < G * 32) {   // thread (h, lane state jj): max, weights and the sum of l in parallel
    const int h = tid >> 5, jj = tid & 31;
    const float mj = s_m[h][jj], lj = s_f[h][jj];
    const float M = group32_max(mj);
    const float f = (M == -INFINITY) ? 0.f : ex2(mj - M);
    const float Ls = group32_sum(lj * f);
    s_f[h][jj] = f;
    if (jj == 0) {
      s_fin[h][64] = M;
      s_fin[h][65] = Ls;
      s_fin[h][66] = 0.f;
      s_fin[h][67] = 0.f;
    }
  }
  __syncthreads();
  for (int e = tid; e < G * 64; e += 256) {
    const int h = e >> 6, d = e & 63;
    float A = 0.f;
#pragma unroll 8
    for (int jj = 0; jj < kAttnStates; ++jj) A = fmaf(s_acc[(jj * G + h) * 64 + d], s_f[h][jj], A);
    s_fin[h][d] = A;
  }
  __syncthreads();

  attn_finish<G>(a, s_fin, &s_last, bk, split, b, kvh);
}

// ---------------------------------------------------------------- matrix-core kernel
//
// Same workgroups, splits, rounds (128 positions: 32 per wave) and split merge as above, but
// each wave scores and accumulates its 32 positions for all query heads of the group at once
// on v_mfma_f32_16x16x32_bf16 (the group's heads padded to 16 with zero rows):
//   S^T[pos][head]  = K[pos][:] . Q[head][:]      A = 16 K rows as stored (16 B per lane),
//                                                 B = Q^T; two MFMAs cover the 64 dims
//   O^T[dim][head] += V^T[dim][pos] . P^T[pos][head]
// Lane j + 16g of a score tile holds head j at positions 4g..4g+3 of the tile. The P.V
// contraction takes its 32 positions in exactly that order (slot 8g + e <-> position
// 16(e/4) + 4g + e%4), so P^T is already in place in the lanes; V^T is gathered to match:
// each lane loads dims 4j..4j+3 (8 B) of its 8 positions and v_perm splits them into four
// operands, operand u holding dims 4i + u, so every lane of an O^T tile belongs to one head
// and the online-softmax rescale is per lane. P enters as three bf16 terms p1 + p2 + p3
// (each the bf16 rounding of what the previous ones left), which carries it to fp32
// precision: products are exact and sums fp32, as on the VALU path. A head's running max is
// kept equal across its four lane groups, so the 32 positions share one scale; the four
// waves' states merge through LDS with one barrier.

struct MfmaLane {
  u32x4_t q[2];   // Q^T operands, dims 0..31 and 32..63
  f32x4_t o[4];   // O^T tiles: o[u][e] = head j, dim 16g + 4e + u
  float m, l;     // running max (scaled log2 units, same in every lane of the head); l of
                  // this lane's positions
};

__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
  const f32x2_v v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_v));
}

// K rows (tile t, dims half c) and the 8-byte V pieces of one wave's 32 positions from p0;
// positions at or past `stop` read zeros (cached loads: outside a buffer resource over the
// rows before stop, no memory access; batched decode +0.4 %) or row 0 (NT), masked later.
// NT: streaming (non-temporal) loads, for launches whose K/V is too large to stay in the
// caches.
template <bool NT>
__device__ __forceinline__ void attn_mfma_load(const uint16_t* kbase, const uint16_t* vbase,
                                               int p0, int stop, int j, int g,
                                               u32x4_t (&kr)[4], uint2 (&vr)[8]) {
  typedef uint32_t u32x2_v __attribute__((ext_vector_type(2)));
  if constexpr (!NT) {
    const __amdgpu_buffer_rsrc_t kr_ = make_rsrc(kbase, (uint32_t)stop * 128u);
    const __amdgpu_buffer_rsrc_t vr_ = make_rsrc(vbase, (uint32_t)stop * 128u);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint32_t o = (uint32_t)(p0 + 16 * t + j) * 128u + 16u * g;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const v4i_t v = __builtin_amdgcn_raw_buffer_load_b128(kr_, (int)(o + 64u * c), 0, 0);
        kr[2 * t + c] = u32x4_t{(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t o = (uint32_t)(p0 + 16 * (e >> 2) + 4 * g + (e & 3)) * 128u + 8u * j;
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(vr_, (int)o, 0, 0);
      vr[e] = make_uint2((uint32_t)v[0], (uint32_t)v[1]);
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int pos = p0 + 16 * t + j;
    const size_t row = (size_t)(pos < stop ? pos : 0) * 64;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const u32x4_t* p = (const u32x4_t*)(kbase + row + 32 * c + 8 * g);
      kr[2 * t + c] = NT ? __builtin_nontemporal_load(p) : *p;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int pos = p0 + 16 * (e >> 2) + 4 * g + (e & 3);
    const size_t row = (size_t)(pos < stop ? pos : 0) * 64;
    const u32x2_v* p = (const u32x2_v*)(vbase + row + 4 * j);
    const u32x2_v v2 = NT ? __builtin_nontemporal_load(p) : *p;
    vr[e] = make_uint2(v2.x, v2.y);
  }
}

__device__ __forceinline__ void attn_mfma_round(MfmaLane& st, const u32x4_t (&kr)[4],
                                                const uint2 (&vr)[8], int p0, int end, int g,
                                                float scale_l2) {
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
  f32x4_t s0 = mfma_bf16(kr[0], st.q[0], zero);
  f32x4_t s1 = mfma_bf16(kr[2], st.q[0], zero);
  s0 = mfma_bf16(kr[1], st.q[1], s0);
  s1 = mfma_bf16(kr[3], st.q[1], s1);
  float sc[8];
  bool ok[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    ok[e] = p0 + 16 * (e >> 2) + 4 * g + (e & 3) < end;
    sc[e] = ok[e] ? (e < 4 ? s0[e] : s1[e - 4]) * scale_l2 : -INFINITY;
  }
  float mr = sc[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) mr = fmaxf(mr, sc[e]);
  mr = xor32_max(xor16_max(mr));   // no LDS round trips (the swaps are VALU)
  const float mn = fmaxf(st.m, mr);
  const float mb = mn == -INFINITY ? 0.f : mn;   // nothing seen yet: every p and corr is 0
  const float corr = ex2(st.m - mb);
  float p[8], ls = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    p[e] = ex2(sc[e] - mb);
    ls += p[e];
  }
  st.l = fmaf(st.l, corr, ls);
  st.m = mn;
#pragma unroll
  for (int u = 0; u < 4; ++u) st.o[u] *= corr;
  u32x4_t pp[3];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    float x0 = p[2 * w], x1 = p[2 * w + 1];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      const uint32_t h = pk_bf16(x0, x1);
      pp[t][w] = h;
      x0 -= bf16lo(h);
      x1 -= bf16hi(h);
    }
  }
  uint2 v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = ok[e] ? vr[e] : make_uint2(0u, 0u);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    u32x4_t av;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t lo = u < 2 ? v[2 * w].x : v[2 * w].y;
      const uint32_t hi = u < 2 ? v[2 * w + 1].x : v[2 * w + 1].y;
      av[w] = perm(hi, lo, (u & 1) ? 0x07060302u : 0x05040100u);
    }
#pragma unroll
    for (int t = 0; t < 3; ++t) st.o[u] = mfma_bf16(av, pp[t], st.o[u]);
  }
}

// NW waves of 32 positions per round (4; 8 for launches whose splits are longer than a
// 4-wave round: one round of 256 positions instead of two of 128; 12 for splits of 513-768
// positions: two rounds of 384 instead of three of 256).
template <int G, bool NT, int NW = kAttnWaves>
__global__ __launch_bounds__(NW * 64) void gqa_mfma_kernel(AttnArgs a) {
  static_assert(G * 32 <= 256 && G <= 16, "one thread per (head, split) in the merge");
  constexpr int TH = NW * 64;
  constexpr int R = NW * 32;   // positions per workgroup round
  __shared__ __attribute__((aligned(16))) float s_o[NW * G * 64];   // wave states
  __shared__ __attribute__((aligned(16))) float s_fin[G][kPartStride];
  __shared__ float s_wm[NW][G], s_wl[NW][G];
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int blk = blockIdx.x;
  const int split = blk % a.n_split;
  const int bk = blk / a.n_split;  // b * hkv + kvh
  const int kvh = bk % a.hkv;
  const int b = bk / a.hkv;
  const int start = split * a.chunk;
  const int stop = min(start + a.chunk, a.max_len);
  const int j = lane & 15, g = lane >> 4;
  const size_t head_off = (size_t)b * a.kv_b_stride + (size_t)kvh * a.kv_h_stride;
  const uint16_t* kbase = a.k + head_off;
  const uint16_t* vbase = a.v + head_off;
  const int wo = wave * 32;

  // the length, q and the first two rounds' K/V all in flight together, in that order: the
  // in-order load counter then lets the first K/V round start when its own bytes are in, not
  // after the second's; three buffers, so that two rounds are in flight while one is computed (one wave per
  // SIMD at long contexts: nothing else hides a round's latency)
  const int len_b = a.lens[b];
  MfmaLane st;
  {
    // the group's G heads through a buffer resource; a padded head's lanes (j >= G) read
    // outside it: zero rows, with no memory access
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q + ((size_t)b * a.hq + kvh * G) * 64, G * 128);
    const uint32_t qo = j < G ? (uint32_t)(j * 128 + 16 * g) : 0x80000000u;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const v4i_t v = __builtin_amdgcn_raw_buffer_load_b128(qr, (int)(qo + 64 * c), 0, 0);
      st.q[c] = u32x4_t{(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
    }
  }
  asm volatile("" ::: "memory");
  u32x4_t kA[4], kB[4], kC[4];
  uint2 vA[8], vB[8], vC[8];
  attn_mfma_load<NT>(kbase, vbase, start + wo, stop, j, g, kA, vA);
  if (stop - start > R)   // a second round exists (known before the length is)
    attn_mfma_load<NT>(kbase, vbase, start + R + wo, stop, j, g, kB, vB);
  st.m = -INFINITY;
  st.l = 0.f;
#pragma unroll
  for (int u = 0; u < 4; ++u) st.o[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int end = min(stop, max(0, len_b));
  const int nr = end > start ? (end - start + R - 1) / R : 0;
  if constexpr (NW > 8) {
    // launched only for splits of at most two rounds (launch_attn), both in flight from the
    // start: two buffers, 88 VGPRs where the three-buffer loop takes 170
    if (nr > 0) attn_mfma_round(st, kA, vA, start + wo, end, g, a.scale_l2);
    if (nr > 1) attn_mfma_round(st, kB, vB, start + R + wo, end, g, a.scale_l2);
  } else
  for (int r = 0; r < nr; r += 3) {
    const int p0 = start + r * R + wo;   // this wave's first position of round r
    if (r + 2 < nr) attn_mfma_load<NT>(kbase, vbase, p0 + 2 * R, stop, j, g, kC, vC);
    attn_mfma_round(st, kA, vA, p0, end, g, a.scale_l2);
    if (r + 3 < nr) attn_mfma_load<NT>(kbase, vbase, p0 + 3 * R, stop, j, g, kA, vA);
    if (r + 1 < nr) attn_mfma_round(st, kB, vB, p0 + R, end, g, a.scale_l2);
    if (r + 4 < nr) attn_mfma_load<NT>(kbase, vbase, p0 + 4 * R, stop, j, g, kB, vB);
    if (r + 2 < nr) attn_mfma_round(st, kC, vC, p0 + 2 * R, end, g, a.scale_l2);
  }

  // ---- merge the waves: l over each head's lane groups, then (m, l, O) through LDS
  st.l = xor32_sum(xor16_sum(st.l));
  if (j < G) {
    if (g == 0) {
      s_wm[wave][j] = st.m;
      s_wl[wave][j] = st.l;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
      *(float4*)(s_o + (wave * G + j) * 64 + 16 * g + 4 * e) =
          make_float4(st.o[0][e], st.o[1][e], st.o[2][e], st.o[3][e]);
  }
  __syncthreads();
  for (int e = tid; e < G * 64; e += TH) {
    const int h = e >> 6, d = e & 63;
    float M = s_wm[0][h];
#pragma unroll
    for (int w = 1; w < NW; ++w) M = fmaxf(M, s_wm[w][h]);
    const float Mb = M == -INFINITY ? 0.f : M;
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = ex2(s_wm[w][h] - Mb);
      L = fmaf(s_wl[w][h], f, L);
      A = fmaf(s_o[(w * G + h) * 64 + d], f, A);
    }
    s_fin[h][d] = A;
    if (d == 0) {
      s_fin[h][64] = M;
      s_fin[h][65] = L;
      s_fin[h][66] = 0.f;
      s_fin[h][67] = 0.f;
    }
  }
  __syncthreads();
  attn_finish<G, TH>(a, s_fin, &s_last, bk, split, b, kvh);
}

// Positions per split as attn_run lays them out, and whether a matrix-core launch of `wgs`
// workgroups with splits that long runs on 8 waves: a split longer than one 4-wave round,
// when the launch fits one 8-wave workgroup per CU (170 VGPRs: two waves per SIMD; a larger
// grid keeps 4 waves and two workgroups per CU). Its rounds of positions per split.
constexpr long long kWideMaxWorkgroups = 256;   // compute units of an MI355X
static int split_chunk(int max_len, int s) { return ((max_len + s - 1) / s + 7) & ~7; }
static bool attn_wide(int chunk, long long wgs) {
  return chunk > kAttnRound && wgs <= kWideMaxWorkgroups;
}
static int attn_rounds(int chunk, bool wide) {
  const int r = wide ? 2 * kAttnRound : kAttnRound;
  return (chunk + r - 1) / r;
}

// Splits per (sequence, kv head), at least one round of positions each. VALU kernel: about
// 512 workgroups, at most 64 splits.
static int auto_split(int batch, int hkv, int max_len, bool mfma) {
  const int by_len = (max_len + kAttnRound - 1) / kAttnRound;   // rounds per (b, kv head)
  const int bh = batch * hkv;
  if (mfma) {
    // Up to two 8-wave rounds per (sequence, kv head) the whole length stays in one split:
    // the split merge's hand-off costs more than the longer workgroup (swept over batch 1-8,
    // L = 128-768, against every split count: L = 256 4.5 against 5.9 us, batch 8 at
    // L = 512 6.84 against 7.13 us); at batch 1 and L = 512 four splits are still ahead
    // (5.96 against 6.03 us), as they are everywhere past 512 positions.
    if (by_len <= 3 || (by_len == 4 && bh >= 16)) return 1;
    // A split's rounds pipeline through its three K/V buffers, and each split adds a record
    // to the merge: a split per round while the whole launch is short, then two rounds per
    // split up to 16 splits, 16 splits up to 128 rounds, then a split per 8 rounds up to 32;
    // at most 512 workgroups. Swept on MI355X at batch 1 and 8, 40 q / 8 kv heads,
    // L = 512-32768: within 5 % of the best count everywhere (batch 1, L = 4096: 16 splits,
    // 9.5 us against 10.9 us with the earlier policy's 24).
    const long long total = (long long)bh * by_len;
    int s;
    if (by_len <= 8 && total <= 256) s = by_len;
    else if (by_len <= 128) s = (by_len + 1) / 2 < 16 ? (by_len + 1) / 2 : 16;
    else s = by_len / 8;
    const int by_grid = 512 / bh;
    s = s > by_grid ? by_grid : s;
    s = s > 32 ? 32 : s;
    s = s < 1 ? 1 : s;
    // then the fewest splits that take no more rounds (each in its own wave count) and still
    // give 128 workgroups: the same time per workgroup with fewer records to merge (batch 8
    // at context 2048: 3 splits on 8 waves, 3425 against 3367 tok/s with 8 on 4 waves; batch
    // 8, L = 4096: 16.8 against 17.4 us). Below 128 workgroups fewer, longer ones finish
    // later (batch 1, L = 512: 2 splits on 8 waves 6.8 us, 4 splits on 4 waves 6.4 us).
    const int c0 = split_chunk(max_len, s);
    const int r0 = attn_rounds(c0, attn_wide(c0, (long long)bh * s));
    for (int t = 1; t < s; ++t) {
      if ((long long)bh * t < 128) continue;
      const int c = split_chunk(max_len, t);
      if (attn_rounds(c, attn_wide(c, (long long)bh * t)) <= r0) return t;
    }
    return s;
  }
  const int by_grid = (512 + bh - 1) / bh;
  int s = by_len < by_grid ? by_len : by_grid;
  s = s > 64 ? 64 : s;
  return s < 1 ? 1 : s;
}

template <int G>
static void launch_attn(const AttnArgs& a, bool mfma, dim3 grid, hipStream_t s) {
  // K/V of 64 MB or more per launch streams past the caches (measured: batch 8 at 32768
  // positions 101 -> 93 us); smaller launches, decode's included, keep cached loads
  const bool nt = (size_t)a.batch * a.hkv * a.max_len * 256 >= ((size_t)64 << 20);
  // 8 waves by attn_wide (published records and the merged answer then come from the same
  // kernel, bit for bit; batch 8 at context 2048 with 8 splits, 512 workgroups: 3379 tok/s on
  // 4 waves against 3169 on 8)
  const bool wide = attn_wide(a.chunk, (long long)grid.x);
  // a split of 513-768 positions: two rounds of 12 waves instead of three of 8 (batch 8 at
  // context 2112, 3 splits of 704: decode 3912 -> 3943 tok/s; 16 waves, two rounds of 512,
  // read 3855)
  if (mfma && !nt && wide && a.chunk > 2 * 2 * kAttnRound && a.chunk <= 2 * 3 * kAttnRound)
    hipLaunchKernelGGL((gqa_mfma_kernel<G, false, 12>), grid, dim3(768), 0, s, a);
  else if (mfma && nt && wide)
    hipLaunchKernelGGL((gqa_mfma_kernel<G, true, 8>), grid, dim3(512), 0, s, a);
  else if (mfma && nt) hipLaunchKernelGGL((gqa_mfma_kernel<G, true>), grid, dim3(256), 0, s, a);
  else if (mfma && wide)
    hipLaunchKernelGGL((gqa_mfma_kernel<G, false, 8>), grid, dim3(512), 0, s, a);
  else if (mfma) hipLaunchKernelGGL((gqa_mfma_kernel<G, false>), grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL(gqa_decode_kernel<G>, grid, dim3(256), 0, s, a);
}

static size_t partial_bytes(int batch, int hkv, int n_split, int G) {
  return (size_t)batch * hkv * n_split * G * kPartStride * 4;
}

// The allocation-free attention entry point's workspace: one library-owned array per GPU,
// laid out like a caller's workspace (arrival counters, then split records). The loader
// zero-fills it, and every launch leaves its counters at zero again. Host code never uses
// the array's name as an address: each device's copy is reached through the pointer that
// hipGetSymbolAddress returned for that device.
constexpr size_t kStaticScratchBytes = Q4NX_STATIC_SCRATCH_BYTES;
static_assert(kStaticScratchBytes % 256 == 0, "the scratch keeps the workspace alignment");
__device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices] = {};   // set once per device, under g_scratch_mu

// This device's copy of `scratch`, resolved on the first call made with the device current.
static int static_scratch(void** out, const char* what) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  Q4NX_REQUIRE(e == hipSuccess, Q4NX_ERR_LAUNCH, "%s: hipGetDevice: %s", what,
               hipGetErrorString(e));
  Q4NX_REQUIRE(dev >= 0 && dev < kMaxDevices, Q4NX_ERR_ARG, "%s: device %d beyond %d", what, dev,
               kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    Q4NX_REQUIRE(e == hipSuccess && p != nullptr, Q4NX_ERR_LAUNCH,
                 "%s: hipGetSymbolAddress(scratch) on device %d: %s", what, dev,
                 hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return Q4NX_OK;
}

}  // namespace q4nx

using namespace q4nx;

extern "C" {

size_t q4nx_gqa_decode_ws_bytes(int batch, int n_q_heads, int n_kv_heads, int max_len,
                                const q4nx_policy* policy) {
  Policy P;
  if (batch < 1 || n_kv_heads < 1 || n_q_heads < n_kv_heads || max_len < 1 ||
      !resolve_policy_quiet(policy, &P))
    return 0;
  const int ns = auto_split(batch, n_kv_heads, max_len, P.attn_mfma != 0);
  if (ns == 1) return 0;
  return (size_t)Q4NX_WS_COUNTER_BYTES +
         partial_bytes(batch, n_kv_heads, ns, n_q_heads / n_kv_heads);
}

static int attn_run(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                    uint16_t* out, float* out_f32, int batch, int n_q_heads, int n_kv_heads,
                    int head_dim, const int32_t* lens, int max_len, int64_t kv_b_stride,
                    int64_t kv_h_stride, float scale, int n_split, void* ws, size_t ws_bytes,
                    const q4nx_policy* policy, void* stream, bool publish_only,
                    const char* what) {
  Policy P;
  if (int rc = resolve_policy(policy, &P, what)) return rc;
  Q4NX_REQUIRE(q && k_cache && v_cache && lens && (publish_only || out || out_f32), Q4NX_ERR_ARG,
               "%s: q, caches, lens and an output are required", what);
  Q4NX_REQUIRE(Q4NX_ALIGNED(q, 16) && Q4NX_ALIGNED(k_cache, 16) && Q4NX_ALIGNED(v_cache, 16),
               Q4NX_ERR_ARG, "%s: q and caches must be 16-byte aligned", what);
  Q4NX_REQUIRE(head_dim == 64, Q4NX_ERR_SHAPE, "%s: head_dim=%d, only 64 is built", what,
               head_dim);
  Q4NX_REQUIRE(batch >= 1 && n_kv_heads >= 1 && n_q_heads % n_kv_heads == 0 &&
                   n_q_heads / n_kv_heads <= 8,
               Q4NX_ERR_SHAPE, "%s: Hq=%d must be a multiple (<= 8x) of Hkv=%d", what, n_q_heads,
               n_kv_heads);
  Q4NX_REQUIRE(max_len >= 1 && kv_h_stride >= (int64_t)max_len * 64 && kv_h_stride % 8 == 0 &&
                   kv_b_stride >= (int64_t)n_kv_heads * kv_h_stride && kv_b_stride % 8 == 0,
               Q4NX_ERR_SHAPE, "%s: cache strides do not hold [Hkv][max_len][64]", what);
  // a (sequence, kv head)'s rows are read with 32-bit byte offsets
  Q4NX_REQUIRE(max_len < (1 << 24), Q4NX_ERR_SHAPE, "%s: max_len=%d beyond 2^24 positions", what,
               max_len);
  AttnArgs a{};
  a.q = q;
  a.k = k_cache;
  a.v = v_cache;
  a.out = out;
  a.out_f32 = out_f32;
  a.lens = lens;
  a.batch = batch;
  a.hq = n_q_heads;
  a.hkv = n_kv_heads;
  a.max_len = max_len;
  a.kv_b_stride = kv_b_stride;
  a.kv_h_stride = kv_h_stride;
  a.scale_l2 = (float)((double)scale * 1.4426950408889634);
  Q4NX_REQUIRE(n_split >= 0 && n_split <= 4096, Q4NX_ERR_ARG, "%s: n_split=%d outside 0..4096",
               what, n_split);
  const bool mfma = P.attn_mfma != 0;
  a.n_split = n_split > 0 ? n_split : auto_split(batch, n_kv_heads, max_len, mfma);
  a.chunk = ((max_len + a.n_split - 1) / a.n_split + 7) & ~7;
  a.publish_only = publish_only ? 1 : 0;
  if (publish_only || a.n_split > 1) {
    const int G = n_q_heads / n_kv_heads;
    const size_t pb = partial_bytes(batch, n_kv_heads, a.n_split, G);
    Q4NX_REQUIRE(pb < (size_t)1 << 31, Q4NX_ERR_SHAPE, "%s: split partials exceed 2 GB", what);
    size_t need = (size_t)Q4NX_WS_COUNTER_BYTES + pb;
    Q4NX_REQUIRE(ws != nullptr && ws_bytes >= need && Q4NX_ALIGNED(ws, 256), Q4NX_ERR_WS,
                 "%s: workspace of %zu bytes (256-aligned) needed, %zu given", what, need,
                 ws_bytes);
    Q4NX_REQUIRE((size_t)batch * n_kv_heads * 4 <= (size_t)Q4NX_WS_COUNTER_BYTES, Q4NX_ERR_SHAPE,
                 "%s: batch*Hkv exceeds the workspace counter region", what);
    a.counters = (unsigned*)ws;
    a.partial = (float*)((uint8_t*)ws + Q4NX_WS_COUNTER_BYTES);
    a.partial_bytes = (uint32_t)pb;
  }
  const dim3 grid((unsigned)(batch * n_kv_heads * a.n_split));
  hipStream_t s = (hipStream_t)stream;
  switch (n_q_heads / n_kv_heads) {
    case 1: launch_attn<1>(a, mfma, grid, s); break;
    case 2: launch_attn<2>(a, mfma, grid, s); break;
    case 3: launch_attn<3>(a, mfma, grid, s); break;
    case 4: launch_attn<4>(a, mfma, grid, s); break;
    case 5: launch_attn<5>(a, mfma, grid, s); break;
    case 6: launch_attn<6>(a, mfma, grid, s); break;
    case 7: launch_attn<7>(a, mfma, grid, s); break;
    default: launch_attn<8>(a, mfma, grid, s); break;
  }
  return check_launch(what);
}

int q4nx_gqa_decode(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                    uint16_t* out, float* out_f32, int batch, int n_q_heads, int n_kv_heads,
                    int head_dim, const int32_t* lens, int max_len, int64_t kv_b_stride,
                    int64_t kv_h_stride, float scale, int n_split, void* ws, size_t ws_bytes,
                    const q4nx_policy* policy, void* stream) {
  return attn_run(q, k_cache, v_cache, out, out_f32, batch, n_q_heads, n_kv_heads, head_dim,
                  lens, max_len, kv_b_stride, kv_h_stride, scale, n_split, ws, ws_bytes, policy,
                  stream, false, "q4nx_gqa_decode");
}

int q4nx_gqa_decode_static(const uint16_t* q, const uint16_t* k_cache,
                           const uint16_t* v_cache, uint16_t* out, float* out_f32, int batch,
                           int n_q_heads, int n_kv_heads, int head_dim, const int32_t* lens,
                           int max_len, int64_t kv_b_stride, int64_t kv_h_stride, float scale,
                           int n_split, const q4nx_policy* policy, void* stream) {
  const char* what = "q4nx_gqa_decode_static";
  Policy P;
  if (int rc = resolve_policy(policy, &P, what)) return rc;
  Q4NX_REQUIRE(batch >= 1 && n_kv_heads >= 1 && n_q_heads >= n_kv_heads &&
                   n_q_heads % n_kv_heads == 0 && max_len >= 1 && n_split >= 0 &&
                   n_split <= 4096,
               Q4NX_ERR_SHAPE, "%s: batch=%d Hq=%d Hkv=%d max_len=%d n_split=%d", what, batch,
               n_q_heads, n_kv_heads, max_len, n_split);
  const int ns = n_split > 0 ? n_split : auto_split(batch, n_kv_heads, max_len, P.attn_mfma != 0);
  const size_t need = ns > 1 ? (size_t)Q4NX_WS_COUNTER_BYTES +
                                   partial_bytes(batch, n_kv_heads, ns, n_q_heads / n_kv_heads)
                             : 0;
  Q4NX_REQUIRE(need <= kStaticScratchBytes, Q4NX_ERR_WS,
               "%s: %d splits of batch %d x %d kv heads need %zu bytes of split records, more "
               "than the %zu of the static scratch (fewer splits or q4nx_gqa_decode with a "
               "workspace)",
               what, ns, batch, n_kv_heads, need, kStaticScratchBytes);
  void* ws = nullptr;
  if (int rc = static_scratch(&ws, what)) return rc;
  return attn_run(q, k_cache, v_cache, out, out_f32, batch, n_q_heads, n_kv_heads, head_dim,
                  lens, max_len, kv_b_stride, kv_h_stride, scale, ns, ws, kStaticScratchBytes,
                  policy, stream, false, what);
}

int q4nx_gqa_decode_splits(int batch, int n_q_heads, int n_kv_heads, int max_len,
                           const q4nx_policy* policy) {
  Policy P;
  if (batch < 1 || n_kv_heads < 1 || n_q_heads < n_kv_heads || max_len < 1 ||
      !resolve_policy_quiet(policy, &P))
    return 0;
  return auto_split(batch, n_kv_heads, max_len, P.attn_mfma != 0);
}

// Splits for records an o-projection merges: the attention policy's count, capped at 12.
// Every split adds a record that each o-projection workgroup reads (0.16 us a split at the
// 3B shape), so the pair is fastest with fewer, longer splits than attention alone: decode
// at one sequence, 40 q / 8 kv heads, measured best at 5 (context 512), 9 (2048) and 12
// (4000) splits.
constexpr int kRecordSplitCap = 12;

int q4nx_gqa_decode_records_splits(int batch, int n_q_heads, int n_kv_heads, int max_len,
                                   const q4nx_policy* policy) {
  const int ns = q4nx_gqa_decode_splits(batch, n_q_heads, n_kv_heads, max_len, policy);
  return ns < kRecordSplitCap ? ns : kRecordSplitCap;
}

int q4nx_gqa_decode_records(const uint16_t* q, const uint16_t* k_cache,
                            const uint16_t* v_cache, int batch, int n_q_heads, int n_kv_heads,
                            int head_dim, const int32_t* lens, int max_len, int64_t kv_b_stride,
                            int64_t kv_h_stride, float scale, int n_split, void* ws,
                            size_t ws_bytes, const q4nx_policy* policy, void* stream) {
  const char* what = "q4nx_gqa_decode_records";
  Q4NX_REQUIRE(n_split >= 1, Q4NX_ERR_ARG, "%s: n_split=%d must be given (>= 1)", what, n_split);
  return attn_run(q, k_cache, v_cache, nullptr, nullptr, batch, n_q_heads, n_kv_heads,
                  head_dim, lens, max_len, kv_b_stride, kv_h_stride, scale, n_split, ws,
                  ws_bytes, policy, stream, true, what);
}

}  // extern "C"
