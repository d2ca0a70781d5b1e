// q4nx tile dequantisation on gfx950, bit-exact against the reference.
//
// q4: w = fp32(code * d + m) (code*d is exact, one rounding for the add), then RNE to
//     bf16 -- tools/q4nx.py:97-101 and the on-core unpack
//     designs/q4nx_unpack/q4nx_unpack.cc:40-92.
// q8: w = code * s, exact in fp32 -- tools/q4nx.py:104-111, :140-143.
// Output either in weight-index order per tile (i = rb*4096 + k*16 + r) or un-tiled to
// the [N][K] matrix (tools/q4nx.py:146-149).
//
// One workgroup of 256 threads per tile; thread t owns the 32 weights of 2 consecutive
// k at 16 rows (one 16-byte chunk of q4 nibbles, two 16-byte chunks of q8 codes).

#include "common.h"

namespace q4nx {

template <int KIND, bool F32, bool UNTILE>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ tiles,
                                                      void* __restrict__ out, int k_tiles) {
  constexpr int TB = KIND == 4 ? kQ4TileBytes : kQ8TileBytes;
  const int t = blockIdx.x;                      // tile index = tr * k_tiles + kt
  const int tr = t / k_tiles, kt = t % k_tiles;
  const uint8_t* tile = tiles + (size_t)t * TB;
  const int c = threadIdx.x;                     // 0..255
  const int rb = c >> 7;                         // row block
  const int k = (c & 127) * 2;                   // first of two k
  const int kb = k >> 5;
  const int g0 = kb * 32 + rb * 16;              // meta index of row 0 of this row-block

  float w[32];  // [kk][r], kk = 0..1
  const uint4 s0 = *(const uint4*)(tile + 2 * g0);
  const uint4 s1 = *(const uint4*)(tile + 2 * g0 + 16);
  const uint32_t sc[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
  if (KIND == 4) {
    const uint4 m0 = *(const uint4*)(tile + kMetaBytes + 2 * g0);
    const uint4 m1 = *(const uint4*)(tile + kMetaBytes + 2 * g0 + 16);
    const uint32_t mn[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
    // weights rb*4096 + k*16 .. +31 -> bytes (rb*4096 + k*16)/2 .. +15
    const uint4 q = *(const uint4*)(tile + 1024 + rb * 2048 + k * 8);
    const uint32_t qq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t byte = (qq[kk * 2 + (r >> 3)] >> (8 * ((r & 7) >> 1))) & 0xFFu;
        const uint32_t code = (r & 1) ? (byte >> 4) : (byte & 0xFu);  // low nibble = even i
        const float d = (r & 1) ? bf16hi(sc[r >> 1]) : bf16lo(sc[r >> 1]);
        const float m = (r & 1) ? bf16hi(mn[r >> 1]) : bf16lo(mn[r >> 1]);
        w[kk * 16 + r] = fmaf((float)code, d, m);
      }
    }
  } else {
    const uint4 q0 = *(const uint4*)(tile + kMetaBytes + rb * 4096 + k * 16);
    const uint4 q1 = *(const uint4*)(tile + kMetaBytes + rb * 4096 + k * 16 + 16);
    const uint32_t qq[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int code = (int)(int8_t)((qq[kk * 4 + (r >> 2)] >> (8 * (r & 3))) & 0xFFu);
        const float s = (r & 1) ? bf16hi(sc[r >> 1]) : bf16lo(sc[r >> 1]);
        w[kk * 16 + r] = (float)code * s;
      }
    }
  }

  if (!UNTILE) {
    const size_t base = (size_t)t * 8192 + rb * 4096 + k * 16;
    if (F32) {
      float4* o = (float4*)((float*)out + base);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = make_float4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
    } else {
      uint4* o = (uint4*)((uint16_t*)out + base);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          v[j] = (uint32_t)f32_to_bf16(w[8 * i + 2 * j]) |
                 ((uint32_t)f32_to_bf16(w[8 * i + 2 * j + 1]) << 16);
        o[i] = make_uint4(v[0], v[1], v[2], v[3]);
      }
    }
  } else {
    const int64_t K = (int64_t)k_tiles * 256;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = (int64_t)tr * 32 + rb * 16 + r;
      const int64_t col = (int64_t)kt * 256 + k;
      if (F32) {
        *(float2*)((float*)out + row * K + col) = make_float2(w[r], w[16 + r]);
      } else {
        *(uint32_t*)((uint16_t*)out + row * K + col) =
            (uint32_t)f32_to_bf16(w[r]) | ((uint32_t)f32_to_bf16(w[16 + r]) << 16);
      }
    }
  }
}

template <int KIND>
static int dequant(const uint8_t* tiles, void* out, int n_tile_rows, int k_tiles, int out_f32,
                   int untile, void* stream, const char* what) {
  Q4NX_REQUIRE(tiles != nullptr && Q4NX_ALIGNED(tiles, 16) && out != nullptr &&
                   Q4NX_ALIGNED(out, 16),
               Q4NX_ERR_ARG, "%s: tiles and out must be non-null 16-byte aligned", what);
  Q4NX_REQUIRE(n_tile_rows > 0 && k_tiles > 0, Q4NX_ERR_SHAPE,
               "%s: n_tile_rows=%d k_tiles=%d must be positive", what, n_tile_rows, k_tiles);
  const int64_t n_tiles = (int64_t)n_tile_rows * k_tiles;
  Q4NX_REQUIRE(n_tiles < (1ll << 31), Q4NX_ERR_SHAPE, "%s: too many tiles", what);
  hipStream_t s = (hipStream_t)stream;
  dim3 grid((unsigned)n_tiles), block(256);
  if (out_f32) {
    if (untile) hipLaunchKernelGGL((dequant_kernel<KIND, true, true>), grid, block, 0, s, tiles, out, k_tiles);
    else hipLaunchKernelGGL((dequant_kernel<KIND, true, false>), grid, block, 0, s, tiles, out, k_tiles);
  } else {
    if (untile) hipLaunchKernelGGL((dequant_kernel<KIND, false, true>), grid, block, 0, s, tiles, out, k_tiles);
    else hipLaunchKernelGGL((dequant_kernel<KIND, false, false>), grid, block, 0, s, tiles, out, k_tiles);
  }
  return check_launch(what);
}

}  // namespace q4nx

extern "C" {

int q4nx_dequant_q4(const uint8_t* tiles, void* out, int n_tile_rows, int k_tiles, int out_f32,
                    int untile, void* stream) {
  return q4nx::dequant<4>(tiles, out, n_tile_rows, k_tiles, out_f32, untile, stream,
                          "q4nx_dequant_q4");
}

int q4nx_dequant_q8(const uint8_t* tiles, void* out, int n_tile_rows, int k_tiles, int out_f32,
                    int untile, void* stream) {
  return q4nx::dequant<8>(tiles, out, n_tile_rows, k_tiles, out_f32, untile, stream,
                          "q4nx_dequant_q8");
}

}  // extern "C"
