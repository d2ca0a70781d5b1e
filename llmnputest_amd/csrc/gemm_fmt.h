// q4nx tile formats as the matrix-core kernels stage and read them: per-kind tile sizes and
// the code -> bf16 operand conversions shared by the batched (gemm.hip) and prefill
// (gemm_pf.hip) contractions.
#pragma once

#include "common.h"

namespace q4nx {

typedef int i32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i32x2_t lds_i32x2_t;

// Per kind: tile bytes, where the codes start, the 16-byte loads per lane that stage a tile
// and the LDS slot it takes; a row-block workgroup (one of a tile's two 16-row blocks) stages
// the metadata and its block's codes only (kLoadsRB, kSlotRB).
template <int KIND>
struct GemmFmt;
template <>
struct GemmFmt<4> {
  static constexpr int kTile = kQ4TileBytes;
  static constexpr int kCodes = 2 * kMetaBytes;   // codes start after d and m
  static constexpr int kLoads = 5;                // 16-byte loads per lane per tile
  static constexpr int kSlot = kQ4TileBytes;      // LDS bytes per staged tile
  static constexpr int kBlockCodes = 2048;        // codes of one 16-row block
  static constexpr int kLoadsRB = 3;              // row-block staging: 1024 + 2048 bytes
  static constexpr int kSlotRB = 3072;
};
template <>
struct GemmFmt<8> {
  static constexpr int kTile = kQ8TileBytes;
  static constexpr int kCodes = kMetaBytes;
  static constexpr int kLoads = 9;                // 8704 B: the 9th load of lanes 32..63 is padding
  static constexpr int kSlot = 9216;
  static constexpr int kBlockCodes = 4096;
  static constexpr int kLoadsRB = 5;              // 512 + 4096 bytes; lanes 32..63 of the 5th: padding
  static constexpr int kSlotRB = 5120;
};

// 8 transposed code bytes (k-slots 0..7 of one row pair) -> bf16 16 + c for the even row (low
// nibbles) and the odd row (high nibbles). The bf16 bits of 16 + c are 0x41 : 0x80 | c << 3, so
// one shift and mask per word moves every byte's nibble to bits 3-6 under the 0x80, and one
// byte permute per operand word pairs two such bytes with the exponent byte 0x41.
__device__ __forceinline__ void q4_operands(i32x2_t r, u32x4_t& ev, u32x4_t& od) {
  const uint32_t w[2] = {(uint32_t)r.x, (uint32_t)r.y};
  // the mask and the 0x80 bytes as register operands, so each mask-and-set is one v_and_or_b32
  // (a three-operand instruction takes no literal constant)
  uint32_t msk, top;
  asm("v_mov_b32 %0, 0x78787878" : "=v"(msk));
  asm("v_mov_b32 %0, 0x80808080" : "=v"(top));
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t lo = ((w[h] << 3) & msk) | top;
    const uint32_t hi = ((w[h] >> 1) & msk) | top;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      // [b(2q), 0x41, b(2q+1), 0x41]
      const uint32_t sel = q ? 0x04030402u : 0x04010400u;
      ev[2 * h + q] = perm(0x41414141u, lo, sel);
      od[2 * h + q] = perm(0x41414141u, hi, sel);
    }
  }
}

// The 16 rows of one row-block as one operand, from the same 8 transposed code bytes in
// lanes c and c + 8 of each 16-lane group: lanes 0-7 take the low nibbles (rows 2p), lanes
// 8-15 the high nibbles (rows 2p + 1). Rotating each word right by `rot` (29: a left shift by
// 3; 1: a right shift by 1) puts the chosen nibble of every byte at bits 3-6, and the mask and
// byte permute finish bf16 16 + c as in q4_operands.
__device__ __forceinline__ u32x4_t q4_operand_rb(i32x2_t r, uint32_t rot) {
  const uint32_t w[2] = {(uint32_t)r.x, (uint32_t)r.y};
  uint32_t msk, top;
  asm("v_mov_b32 %0, 0x78787878" : "=v"(msk));
  asm("v_mov_b32 %0, 0x80808080" : "=v"(top));
  u32x4_t o;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t t = (__builtin_amdgcn_alignbit(w[h], w[h], rot) & msk) | top;
    o[2 * h] = perm(0x41414141u, t, 0x04010400u);
    o[2 * h + 1] = perm(0x41414141u, t, 0x04030402u);
  }
  return o;
}

// 8 transposed int8 codes -> bf16 of q + 128 (exact: at most 8 significant bits); the byte
// conversions compile to v_cvt_f32_ubyte0..3.
__device__ __forceinline__ u32x4_t q8_operand(i32x2_t r) {
  const uint32_t w[2] = {(uint32_t)r.x ^ 0x80808080u, (uint32_t)r.y ^ 0x80808080u};
  u32x4_t o;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t f0 = __float_as_uint((float)(w[h] & 0xFFu));
    const uint32_t f1 = __float_as_uint((float)((w[h] >> 8) & 0xFFu));
    const uint32_t f2 = __float_as_uint((float)((w[h] >> 16) & 0xFFu));
    const uint32_t f3 = __float_as_uint((float)((w[h] >> 24) & 0xFFu));
    o[2 * h] = perm(f1, f0, 0x07060302u);
    o[2 * h + 1] = perm(f3, f2, 0x07060302u);
  }
  return o;
}

}  // namespace q4nx
