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

#include <math.h>

#include "common.h"

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
};

typedef short bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kAttnWaves = 4;
constexpr int kAttnSteps = 4;                              // 8-position steps per round
constexpr int kAttnRound = kAttnWaves * kAttnSteps * 8;    // positions per workgroup round
constexpr int kAttnStates = kAttnWaves * 8;                // lane softmax states per WG
constexpr int kPartStride = 68;                            // acc[64], m, l, 2 pad (16 B rows)
constexpr int kMergeSplits = 16;                           // splits merged per LDS pass

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
#pragma unroll
  for (int s = 0; s < kAttnSteps; ++s) {
    const bool ok = r0 + (wave * kAttnSteps + s) * 8 + pl < end;
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
        const uint32_t vv[4] = {vr[s].x, vr[s].y, vr[s].z, vr[s].w};
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

template <int G>
__global__ __launch_bounds__(256) void gqa_decode_kernel(AttnArgs a) {
  static_assert(G * 32 <= 256, "one thread per (head, lane state)");
  __shared__ float s_m[G][kAttnStates], s_f[G][kAttnStates];
  __shared__ __attribute__((aligned(16))) float s_acc[kAttnStates * G * 64];  // also merge buffer
  __shared__ __attribute__((aligned(16))) float s_fin[G][kPartStride];
  __shared__ float s_g[G];
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

  if (a.n_split > 1) {
    // publish this split's (acc, m, l), then the last workgroup of (b, kv head) merges
    const __amdgpu_buffer_rsrc_t pr = make_rsrc(a.partial, a.partial_bytes);
    const uint32_t rec_bytes = G * kPartStride * 4;
    const uint32_t rec = (uint32_t)((size_t)bk * a.n_split + split) * rec_bytes;
    for (int e = tid; e < G * kPartStride / 4; e += 256)
      st16_sys(pr, rec + e * 16, ((const uint4*)&s_fin[0][0])[e]);
    wait_vm();
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = atomicAdd(&a.counters[bk], 1u);
      s_last = (prev == (unsigned)(a.n_split - 1)) ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;

    constexpr int kRec16 = G * kPartStride / 4;                     // uint4 per split record
    constexpr int kPer = (kMergeSplits * kRec16 + 255) / 256;       // loads per thread per pass
    const uint32_t base = (uint32_t)((size_t)bk * a.n_split) * rec_bytes;
    // running merged state: s_fin[h][64] = M, s_fin[h][65] = L, thread (h, d) holds A
    float Ar[2] = {0.f, 0.f};
    if (tid < G) {
      s_fin[tid][64] = -INFINITY;
      s_fin[tid][65] = 0.f;
    }
    for (int cs = 0; cs < a.n_split; cs += kMergeSplits) {
      const int ns = min(kMergeSplits, a.n_split - cs);
      const uint32_t src = base + (uint32_t)cs * rec_bytes;
      uint4 v[kPer];   // unconditional: past the buffer end the loads return 0
#pragma unroll
      for (int i = 0; i < kPer; ++i) v[i] = ld16_sys(pr, src + (tid + i * 256) * 16);
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int e = tid + i * 256;
        if (e < ns * kRec16) ((uint4*)s_acc)[e] = v[i];
      }
      __syncthreads();
      if (tid < G * 16) {   // thread (h, split sp of the pass): weights in parallel
        const int h = tid >> 4, sp = tid & 15;
        const float ms = sp < ns ? s_acc[(sp * G + h) * kPartStride + 64] : -INFINITY;
        const float ls = sp < ns ? s_acc[(sp * G + h) * kPartStride + 65] : 0.f;
        const float Mh = group16_max(fmaxf(ms, s_fin[h][64]));   // s_fin[h][64]: running M
        const float f = (Mh == -INFINITY) ? 0.f : ex2(ms - Mh);
        const float Lp = group16_sum(ls * f);
        s_f[h][sp] = f;
        if (sp == 0) {
          const float Mo = s_fin[h][64];
          const float g = (Mo == -INFINITY) ? 0.f : ex2(Mo - Mh);
          s_g[h] = g;
          s_fin[h][65] = fmaf(s_fin[h][65], g, Lp);
          s_fin[h][64] = Mh;
        }
      }
      __syncthreads();
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int e = tid + jj * 256;
        if (e < G * 64) {
          const int h = e >> 6, d = e & 63;
          float As = Ar[jj] * s_g[h];
          for (int sp = 0; sp < ns; ++sp)
            As = fmaf(s_acc[(sp * G + h) * kPartStride + d], s_f[h][sp], As);
          Ar[jj] = As;
        }
      }
      __syncthreads();
    }
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int e = tid + jj * 256;
      if (e < G * 64) s_fin[e >> 6][e & 63] = Ar[jj];
    }
    if (tid == 0)  // ready for the next call
      __hip_atomic_store(&a.counters[bk], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __syncthreads();
  }

  for (int e = tid; e < G * 64; e += 256) {
    const int h = e >> 6, d = e & 63;
    const float Ls = s_fin[h][65];
    const float o = Ls > 0.f ? s_fin[h][d] / Ls : 0.f;   // an empty sequence gives zeros
    const size_t oi = ((size_t)b * a.hq + kvh * G + h) * 64 + d;
    if (a.out) a.out[oi] = f32_to_bf16(o);
    if (a.out_f32) a.out_f32[oi] = o;
  }
}

// Splits per (sequence, kv head): enough workgroups to cover the GPU (about 512), at least
// one round of positions each, at most 64 so the merge stays short.
static int auto_split(int batch, int hkv, int max_len) {
  const int by_len = (max_len + kAttnRound - 1) / kAttnRound;
  const int by_grid = (512 + batch * hkv - 1) / (batch * hkv);
  int s = by_len < by_grid ? by_len : by_grid;
  s = s > 64 ? 64 : s;
  return s < 1 ? 1 : s;
}

static size_t partial_bytes(int batch, int hkv, int n_split, int G) {
  return (size_t)batch * hkv * n_split * G * kPartStride * 4;
}

}  // namespace q4nx

using namespace q4nx;

extern "C" {

size_t q4nx_gqa_decode_ws_bytes(int batch, int n_q_heads, int n_kv_heads, int max_len) {
  if (batch < 1 || n_kv_heads < 1 || n_q_heads < n_kv_heads || max_len < 1) return 0;
  const int ns = auto_split(batch, n_kv_heads, max_len);
  if (ns == 1) return 0;
  return (size_t)Q4NX_WS_COUNTER_BYTES +
         partial_bytes(batch, n_kv_heads, ns, n_q_heads / n_kv_heads);
}

int q4nx_gqa_decode(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                    uint16_t* out, float* out_f32, int batch, int n_q_heads, int n_kv_heads,
                    int head_dim, const int32_t* lens, int max_len, int64_t kv_b_stride,
                    int64_t kv_h_stride, float scale, int n_split, void* ws, size_t ws_bytes,
                    void* stream) {
  const char* what = "q4nx_gqa_decode";
  Q4NX_REQUIRE(q && k_cache && v_cache && lens && (out || out_f32), Q4NX_ERR_ARG,
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
  a.n_split = n_split > 0 ? n_split : auto_split(batch, n_kv_heads, max_len);
  a.chunk = ((max_len + a.n_split - 1) / a.n_split + 7) & ~7;
  if (a.n_split > 1) {
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
  const dim3 grid((unsigned)(batch * n_kv_heads * a.n_split)), block(256);
  hipStream_t s = (hipStream_t)stream;
  switch (n_q_heads / n_kv_heads) {
    case 1: hipLaunchKernelGGL(gqa_decode_kernel<1>, grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL(gqa_decode_kernel<2>, grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL(gqa_decode_kernel<3>, grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL(gqa_decode_kernel<4>, grid, block, 0, s, a); break;
    case 5: hipLaunchKernelGGL(gqa_decode_kernel<5>, grid, block, 0, s, a); break;
    case 6: hipLaunchKernelGGL(gqa_decode_kernel<6>, grid, block, 0, s, a); break;
    case 7: hipLaunchKernelGGL(gqa_decode_kernel<7>, grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL(gqa_decode_kernel<8>, grid, block, 0, s, a); break;
  }
  return check_launch(what);
}

}  // extern "C"
