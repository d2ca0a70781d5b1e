// Shared device/host helpers for the q4nx HIP kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/q4nx_hip.h"

namespace q4nx {

// ---------------------------------------------------------------- q4nx tile format
// tools/q4nx.py:46-56 and :7-18.
constexpr int kTileRows = 32;
constexpr int kTileK = 256;
constexpr int kGroup = 32;
constexpr int kQ4TileBytes = 5120;   // [bf16 d x256][bf16 m x256][4096 B nibbles]
constexpr int kQ8TileBytes = 8704;   // [bf16 s x256][8192 B int8]
constexpr int kMetaBytes = 512;      // one bf16 plane of 256 entries

// ---------------------------------------------------------------- bf16 / fp16 bits

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}
// lo / hi bf16 of a packed dword, as fp32
__device__ __forceinline__ float bf16lo(uint32_t d) { return __uint_as_float(d << 16); }
__device__ __forceinline__ float bf16hi(uint32_t d) { return __uint_as_float(d & 0xFFFF0000u); }

// fp32 -> bf16, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2_t as_h2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }
__device__ __forceinline__ uint32_t h2_bits(half2_t v) { return __builtin_bit_cast(uint32_t, v); }

// acc + a.x*b.x + a.y*b.y, fp16 inputs, fp32 accumulate (v_dot2c_f32_f16).
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), acc, false);
}

// v_perm_b32: bytes of {hi:s0, lo:s1} selected by `sel`, 0x0c selects zero.
__device__ __forceinline__ uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
  return __builtin_amdgcn_perm(s0, s1, sel);
}

// Cross-workgroup publication without flushing the XCD L2s: partial results go out with
// system-scope (L2-bypassing, write-through) stores, `wait_vm` waits until they are
// acknowledged, and the workgroup that reads them back uses system-scope loads. An
// agent-scope __threadfence() here would write back and invalidate the whole L2 of the
// XCD for every workgroup (buffer_wbl2 / buffer_inv), which costs tens of microseconds.
__device__ __forceinline__ void store_sys(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ float load_sys(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Sum over the wave (64 lanes) via xor shuffles.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

}  // namespace q4nx

// ---------------------------------------------------------------- host-side error plumbing
namespace q4nx {
void set_error(const char* fmt, ...);
int check_launch(const char* what);
}  // namespace q4nx

#define Q4NX_REQUIRE(cond, code, ...)         \
  do {                                        \
    if (!(cond)) {                            \
      ::q4nx::set_error(__VA_ARGS__);         \
      return (code);                          \
    }                                         \
  } while (0)

#define Q4NX_ALIGNED(p, a) ((((uintptr_t)(p)) & ((a) - 1)) == 0)
