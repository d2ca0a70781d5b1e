// Weight-stream floors of the batch-1 q4 GEMV: a null kernel and a plain streaming read.
//
// The reference tells "the kernel is slow" apart from "the memory path is slow" with a null
// design that keeps the GEMV's dataflow and does no arithmetic
// (designs/granite_gemv/granite_gemv.py:105-121, selected by --null at :315-321; the
// measured pair is quoted at granite_gemv32.py:13-19), and its CPU baseline times a STREAM
// read of the same weights beside the GEMV (cpu_baseline.cpp:157-166). These two kernels
// are the same two floors for the row-block GEMV of gemv1.hip:
//
//   gemv1_null_kernel   exactly gemv1_kernel's grid (two workgroups per tile-row, the pair
//                       8 apart), workgroup size, per-lane loads (activation, execution
//                       barrier, then 32 code bytes and the two rows' d and m per K-tile) and
//                       its 16 output stores per workgroup; in place of the arithmetic each
//                       lane folds what it loaded with XOR so that no load is dead.
//   stream_read_kernel  a plain read of a byte range: every lane four 16-byte loads, each
//                       load instruction of a wave covering 1 KB contiguous; a store only
//                       if the fold hits a fixed value, so the kernel writes (almost)
//                       nothing.
//
// Neither result means anything: the null kernel's y holds XOR folds of the loaded bits.

#include "common.h"
#include "gemv1.h"

namespace q4nx {

constexpr uint32_t kFoldMagic = 0x9E3779B9u;   // a fold equal to this stores (never in practice)

__device__ __forceinline__ uint32_t fold4(uint4 v) { return (v.x ^ v.y) ^ (v.z ^ v.w); }

template <int TPW>
__global__ __launch_bounds__(1024) void gemv1_null_kernel(const uint8_t* __restrict__ w,
                                                          const uint16_t* __restrict__ x,
                                                          float* __restrict__ y, int k_t,
                                                          int n_groups) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int chunk = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bi = blockIdx.x;
  int group, rb;   // gemv1_kernel's mapping for 16-row blocks
  if ((n_groups & 7) == 0) {
    group = (bi >> 4) * 8 + (bi & 7);
    rb = (bi >> 3) & 1;
  } else {
    group = bi >> 1;
    rb = bi & 1;
  }
  const int qq = lane & 7, gk = lane >> 3;
  const int k0 = gk * 32 + qq * 4;
  const int b0 = lane & 1, b1 = (lane >> 1) & 1, b2 = (lane >> 2) & 1;
  const int gsw = 2 * b2 + (b1 ^ b2);
  const int R = 2 * gsw + 8 * b0;
  const int mi = gk * 32 + rb * 16 + R;
  const int kt0 = chunk * TPW;

  uint2 xv[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) xv[t] = *(const uint2*)(x + min(kt0 + t, k_t - 1) * kTileK + k0);
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  uint4 wq[TPW][2];
  uint32_t md[TPW], mm[TPW];
  const uint8_t* rowp = w + (size_t)group * k_t * kQ4TileBytes;
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const uint8_t* tile = rowp + (size_t)min(kt0 + t, k_t - 1) * kQ4TileBytes;
    const uint4* src = (const uint4*)(tile + 2 * kMetaBytes + rb * 2048 + lane * 32);
    wq[t][0] = src[0];
    wq[t][1] = src[1];
    md[t] = *(const uint32_t*)(tile + 2 * mi);
    mm[t] = *(const uint32_t*)(tile + kMetaBytes + 2 * mi);
  }
  uint32_t f = 0;
#pragma unroll
  for (int t = 0; t < TPW; ++t)
    f ^= (fold4(wq[t][0]) ^ fold4(wq[t][1])) ^ ((md[t] ^ mm[t]) ^ (xv[t].x ^ xv[t].y));
  // the GEMV's 16 output stores per workgroup (first wave, lanes 0-15); every other lane
  // stores only on the fixed fold value
  if (chunk == 0 ? lane < 16 : f == kFoldMagic)
    y[(int64_t)group * 32 + rb * 16 + (lane & 15)] = __uint_as_float(f);
}

__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ p, int64_t n16,
                                                          uint32_t* __restrict__ sink) {
  const int64_t base = (int64_t)blockIdx.x * 1024 + threadIdx.x;
  uint4 v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = p[min(base + 256 * j, n16 - 1)];   // the tail re-reads
  const uint32_t f = (fold4(v[0]) ^ fold4(v[1])) ^ (fold4(v[2]) ^ fold4(v[3]));
  if (f == kFoldMagic) sink[threadIdx.x & 63] = f;
}

}  // namespace q4nx

using namespace q4nx;

extern "C" {

int q4nx_gemv_q4_null(const uint8_t* w, const uint16_t* x, float* y, int n_tile_rows,
                      int k_tiles, void* stream) {
  const char* what = "q4nx_gemv_q4_null";
  Q4NX_REQUIRE(w != nullptr && Q4NX_ALIGNED(w, 16), Q4NX_ERR_ARG,
               "%s: w must be a 16-byte aligned device pointer", what);
  Q4NX_REQUIRE(x != nullptr && Q4NX_ALIGNED(x, 8), Q4NX_ERR_ARG,
               "%s: x must be an 8-byte aligned device pointer", what);
  Q4NX_REQUIRE(y != nullptr && Q4NX_ALIGNED(y, 4), Q4NX_ERR_ARG,
               "%s: y must be a 4-byte aligned device pointer", what);
  Q4NX_REQUIRE(n_tile_rows >= 1, Q4NX_ERR_SHAPE, "%s: n_tile_rows=%d", what, n_tile_rows);
  const int tpw = gemv1_tpw(1, k_tiles);
  Q4NX_REQUIRE(k_tiles >= 1 && tpw > 0, Q4NX_ERR_SHAPE,
               "%s: k_tiles=%d (the row-block GEMV covers 1..64)", what, k_tiles);
  const dim3 grid(2 * n_tile_rows), block(((k_tiles + tpw - 1) / tpw) * 64);
  hipStream_t s = (hipStream_t)stream;
  if (tpw == 1) hipLaunchKernelGGL(gemv1_null_kernel<1>, grid, block, 0, s, w, x, y, k_tiles, n_tile_rows);
  else if (tpw == 2) hipLaunchKernelGGL(gemv1_null_kernel<2>, grid, block, 0, s, w, x, y, k_tiles, n_tile_rows);
  else hipLaunchKernelGGL(gemv1_null_kernel<4>, grid, block, 0, s, w, x, y, k_tiles, n_tile_rows);
  return check_launch(what);
}

int q4nx_stream_read(const void* buf, size_t bytes, uint32_t* sink, void* stream) {
  const char* what = "q4nx_stream_read";
  Q4NX_REQUIRE(buf != nullptr && Q4NX_ALIGNED(buf, 16), Q4NX_ERR_ARG,
               "%s: buf must be a 16-byte aligned device pointer", what);
  Q4NX_REQUIRE(sink != nullptr && Q4NX_ALIGNED(sink, 4), Q4NX_ERR_ARG,
               "%s: sink must be a 4-byte aligned device pointer (64 words)", what);
  Q4NX_REQUIRE(bytes >= 16 && bytes % 16 == 0 && bytes <= ((size_t)1 << 40), Q4NX_ERR_SHAPE,
               "%s: bytes=%zu (a positive multiple of 16)", what, bytes);
  const int64_t n16 = (int64_t)(bytes / 16);
  const int64_t blocks = (n16 + 1023) / 1024;
  Q4NX_REQUIRE(blocks <= INT32_MAX, Q4NX_ERR_SHAPE, "%s: bytes=%zu", what, bytes);
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, (const uint4*)buf, n16, sink);
  return check_launch(what);
}

}  // extern "C"
