// GQA flash-decode attention for gfx950.
//
// Reference: designs/granite_gemv/granite_attention.h:80-213 (online softmax over 32-position
// KV blocks on one AIE core, one q head per design, scale*log2e folded in fp32 so the
// softmax is a pure exp2, :65-72) and its fp64 check granite_attention.py:163-167.
//
// Here one workgroup owns (sequence b, kv head, KV split): all Hq/Hkv query heads of the
// group share every K/V row it loads, the KV length is split across workgroups, and the
// last workgroup of a (b, kv head) merges the splits' (m, l, acc) exactly, in split order.
// Lanes: 4 lanes per KV position (16 head dims each), 16 positions per wave per step.
// QK uses v_dot2_f32_bf16 (exact bf16 products, fp32 sums); PV and the softmax state are
// fp32; exp2 runs on scores already scaled by scale*log2(e).

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
  int batch, hq, hkv, chunk, n_split, max_len;
  int64_t kv_b_stride, kv_h_stride;
  float scale_l2;  // scale * log2(e)
  float* partial;  // [b*hkv + kvh][n_split][G][66]
  unsigned* counters;
};

typedef short bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kSplitChunk = 16;   // splits merged per LDS pass

__device__ __forceinline__ float dot2bf(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                        __builtin_bit_cast(bf16x2_t, b), c, false);
}

template <int G>
__global__ __launch_bounds__(256) void gqa_decode_kernel(AttnArgs a) {
  __shared__ float s_m[4][G], s_l[4][G];
  __shared__ float s_acc[4][G][64];
  __shared__ float s_fin[G][66];
  __shared__ float s_part[kSplitChunk * G * 66];
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int blk = blockIdx.x;
  const int split = blk % a.n_split;
  const int bk = blk / a.n_split;  // b * hkv + kvh
  const int kvh = bk % a.hkv;
  const int b = bk / a.hkv;
  const int L = min(a.lens[b], a.max_len);
  const int start = split * a.chunk;
  const int end = min(start + a.chunk, L);

  const int dg = lane & 3;   // dims dg*16 .. +16
  const int tl = lane >> 2;  // position within the wave's 16

  // q for the G heads of this kv head, this lane's 16 dims: 8 bf16 pairs per head
  uint32_t qv[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const uint4* qp = (const uint4*)(a.q + ((size_t)b * a.hq + kvh * G + h) * 64 + dg * 16);
    const uint4 q0 = qp[0], q1 = qp[1];
    qv[h][0] = q0.x; qv[h][1] = q0.y; qv[h][2] = q0.z; qv[h][3] = q0.w;
    qv[h][4] = q1.x; qv[h][5] = q1.y; qv[h][6] = q1.z; qv[h][7] = q1.w;
  }

  float m[G], l[G], acc[G][16];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[h][i] = 0.f;
  }

  const uint16_t* kbase = a.k + (size_t)b * a.kv_b_stride + (size_t)kvh * a.kv_h_stride + dg * 16;
  const uint16_t* vbase = a.v + (size_t)b * a.kv_b_stride + (size_t)kvh * a.kv_h_stride + dg * 16;

  // Two 16-position steps per trip, both steps' K/V loads issued before any arithmetic.
  for (int t0 = start + wave * 16; t0 < end; t0 += 128) {
    uint4 kk4[2][2], vv4[2][2];
    bool valid[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = t0 + u * 64 + tl;
      valid[u] = t < end;
      kk4[u][0] = kk4[u][1] = vv4[u][0] = vv4[u][1] = make_uint4(0, 0, 0, 0);
      if (valid[u]) {
        const uint4* kp = (const uint4*)(kbase + (size_t)t * 64);
        const uint4* vp = (const uint4*)(vbase + (size_t)t * 64);
        kk4[u][0] = kp[0];
        kk4[u][1] = kp[1];
        vv4[u][0] = vp[0];
        vv4[u][1] = vp[1];
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      if (t0 + u * 64 >= end) break;   // wave-uniform
      const uint32_t kk[8] = {kk4[u][0].x, kk4[u][0].y, kk4[u][0].z, kk4[u][0].w,
                              kk4[u][1].x, kk4[u][1].y, kk4[u][1].z, kk4[u][1].w};
      float s[G];
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) d = dot2bf(qv[h][i], kk[i], d);
        d += __shfl_xor(d, 1);
        d += __shfl_xor(d, 2);
        s[h] = valid[u] ? d * a.scale_l2 : -INFINITY;
      }
      const uint32_t vv[8] = {vv4[u][0].x, vv4[u][0].y, vv4[u][0].z, vv4[u][0].w,
                              vv4[u][1].x, vv4[u][1].y, vv4[u][1].z, vv4[u][1].w};
      float vf[16];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        vf[2 * i] = bf16lo(vv[i]);
        vf[2 * i + 1] = bf16hi(vv[i]);
      }
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float bm = s[h];
#pragma unroll
        for (int o = 4; o < 64; o <<= 1) bm = fmaxf(bm, __shfl_xor(bm, o));
        const float mn = fmaxf(m[h], bm);
        if (mn != m[h]) {  // wave-uniform: rescale what is accumulated
          const float corr = (m[h] == -INFINITY) ? 0.f : exp2f(m[h] - mn);
          l[h] *= corr;
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[h][i] *= corr;
          m[h] = mn;
        }
        const float p = (s[h] == -INFINITY) ? 0.f : exp2f(s[h] - m[h]);
        l[h] += p;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[h][i] = fmaf(p, vf[i], acc[h][i]);
      }
    }
  }

  // reduce over the 16 positions of the wave (lane bits 2..5)
#pragma unroll
  for (int h = 0; h < G; ++h) {
#pragma unroll
    for (int o = 4; o < 64; o <<= 1) {
      l[h] += __shfl_xor(l[h], o);
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[h][i] += __shfl_xor(acc[h][i], o);
    }
    if (lane < 4) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s_acc[wave][h][lane * 16 + i] = acc[h][i];
    }
    if (lane == 0) {
      s_m[wave][h] = m[h];
      s_l[wave][h] = l[h];
    }
  }
  __syncthreads();

  // merge the 4 waves: thread per (h, d)
  for (int e = tid; e < G * 64; e += 256) {
    const int h = e >> 6, d = e & 63;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, s_m[w][h]);
    float Ls = 0.f, As = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = (s_m[w][h] == -INFINITY) ? 0.f : exp2f(s_m[w][h] - M);
      Ls = fmaf(s_l[w][h], f, Ls);
      As = fmaf(s_acc[w][h][d], f, As);
    }
    s_fin[h][d] = As;
    if (d == 0) {
      s_fin[h][64] = M;
      s_fin[h][65] = Ls;
    }
  }
  __syncthreads();

  if (a.n_split > 1) {
    float* part = a.partial + ((size_t)bk * a.n_split + split) * (G * 66);
    for (int e = tid; e < G * 66; e += 256) store_sys(part + e, s_fin[e / 66][e % 66]);
    wait_vm();
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = atomicAdd(&a.counters[bk], 1u);
      s_last = (prev == (unsigned)(a.n_split - 1)) ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;
    // Merge all splits in split order, kSplitChunk at a time: every partial of the chunk
    // is loaded into LDS with many loads in flight, then each thread folds its (h, d).
    const float* base = a.partial + (size_t)bk * a.n_split * (G * 66);
    // running state of this thread's (h, d) outputs e = tid + j*256 (G*64 <= 512)
    float Mr[2] = {-INFINITY, -INFINITY}, Lr[2] = {0.f, 0.f}, Ar[2] = {0.f, 0.f};
    for (int cs = 0; cs < a.n_split; cs += kSplitChunk) {
      const int ns = min(kSplitChunk, a.n_split - cs);
      const float* src = base + (size_t)cs * G * 66;
      const int n = ns * G * 66;
      for (int e = tid; e < n; e += 4 * 256) {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (e + j * 256 < n) ? load_sys(src + e + j * 256) : 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (e + j * 256 < n) s_part[e + j * 256] = v[j];
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int e = tid + j * 256;
        if (e < G * 64) {
          const int h = e >> 6, d = e & 63;
          float M = Mr[j];
          for (int sp = 0; sp < ns; ++sp) M = fmaxf(M, s_part[(sp * G + h) * 66 + 64]);
          float Ls = Lr[j], As = Ar[j];
          if (Mr[j] != -INFINITY && M != Mr[j]) {
            const float f = exp2f(Mr[j] - M);
            Ls *= f;
            As *= f;
          }
          for (int sp = 0; sp < ns; ++sp) {
            const float* ps = s_part + (sp * G + h) * 66;
            const float f = (ps[64] == -INFINITY) ? 0.f : exp2f(ps[64] - M);
            Ls = fmaf(ps[65], f, Ls);
            As = fmaf(ps[d], f, As);
          }
          Mr[j] = M;
          Lr[j] = Ls;
          Ar[j] = As;
        }
      }
      __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int e = tid + j * 256;
      if (e < G * 64) {
        s_fin[e >> 6][e & 63] = Ar[j];
        if ((e & 63) == 0) s_fin[e >> 6][65] = Lr[j];
      }
    }
    if (tid == 0) a.counters[bk] = 0u;
    __syncthreads();
  }

  for (int e = tid; e < G * 64; e += 256) {
    const int h = e >> 6, d = e & 63;
    const float o = s_fin[h][d] / s_fin[h][65];
    const size_t oi = ((size_t)b * a.hq + kvh * G + h) * 64 + d;
    if (a.out) a.out[oi] = f32_to_bf16(o);
    if (a.out_f32) a.out_f32[oi] = o;
  }
}

static int auto_split(int batch, int hkv, int max_len) {
  int by_len = (max_len + 127) / 128;                  // >= 128 positions per split
  int by_grid = (1024 + batch * hkv - 1) / (batch * hkv);  // about 1024 workgroups
  int s = by_len < by_grid ? by_len : by_grid;
  return s < 1 ? 1 : s;
}

static int split_chunk(int max_len, int n_split) {
  int chunk = (max_len + n_split - 1) / n_split;
  return (chunk + 63) / 64 * 64;
}

}  // namespace q4nx

using namespace q4nx;

extern "C" {

size_t q4nx_gqa_decode_ws_bytes(int batch, int n_q_heads, int n_kv_heads, int max_len) {
  if (batch < 1 || n_kv_heads < 1 || n_q_heads < n_kv_heads || max_len < 1) return 0;
  const int ns = auto_split(batch, n_kv_heads, max_len);
  if (ns == 1) return 0;
  const int G = n_q_heads / n_kv_heads;
  return (size_t)Q4NX_WS_COUNTER_BYTES + (size_t)batch * n_kv_heads * ns * G * 66 * 4;
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
  a.n_split = n_split > 0 ? n_split : auto_split(batch, n_kv_heads, max_len);
  a.chunk = split_chunk(max_len, a.n_split);
  a.n_split = (max_len + a.chunk - 1) / a.chunk;
  if (a.n_split > 1) {
    const int G = n_q_heads / n_kv_heads;
    size_t need = (size_t)Q4NX_WS_COUNTER_BYTES + (size_t)batch * n_kv_heads * a.n_split * G * 66 * 4;
    Q4NX_REQUIRE(ws != nullptr && ws_bytes >= need && Q4NX_ALIGNED(ws, 256), Q4NX_ERR_WS,
                 "%s: workspace of %zu bytes (256-aligned) needed, %zu given", what, need,
                 ws_bytes);
    Q4NX_REQUIRE((size_t)batch * n_kv_heads * 4 <= (size_t)Q4NX_WS_COUNTER_BYTES, Q4NX_ERR_SHAPE,
                 "%s: batch*Hkv exceeds the workspace counter region", what);
    a.counters = (unsigned*)ws;
    a.partial = (float*)((uint8_t*)ws + Q4NX_WS_COUNTER_BYTES);
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
