// Shared device/host helpers for the q4nx HIP kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

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

// fp32 -> bf16, round to nearest even (v_cvt_pk_bf16_f32); a NaN keeps its upper payload
// bits and becomes quiet, as the software rounding (u >> 16) | 0x40 does.
typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
typedef float f32x2_v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_v v = {lo, hi};
  uint32_t r = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_v));
  const uint32_t ul = __float_as_uint(lo), uh = __float_as_uint(hi);
  if ((ul & 0x7FFFFFFFu) > 0x7F800000u) r = (r & 0xFFFF0000u) | ((ul >> 16) | 0x40u);
  if ((uh & 0x7FFFFFFFu) > 0x7F800000u) r = (r & 0x0000FFFFu) | (((uh >> 16) | 0x40u) << 16);
  return r;
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return (uint16_t)pack_bf16x2(f, 0.f); }
// The same rounding for operands that are consumed in place (a NaN stays a NaN, its payload
// is not kept): one instruction.
__device__ __forceinline__ uint32_t pack_bf16x2_op(float lo, float hi) {
  const f32x2_v v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_v));
}

// RMSNorm scale 1 / sqrt(ss / K + eps) from a row's sum of squares ss. Every kernel family
// computes it with this one sequence (v_rcp_f32, v_rsq_f32: 1 ulp each), so all of them
// normalise a row to the same bits.
__device__ __forceinline__ float rms_inv(float ss, int K, float eps) {
  return __builtin_amdgcn_rsqf(fmaf(ss, __builtin_amdgcn_rcpf((float)K), eps));
}
// x narrowed to bf16 and widened back, for values used in place (a NaN stays a NaN)
__device__ __forceinline__ float round_bf16_op(float x) { return bf16lo(pack_bf16x2_op(x, 0.f)); }

// silu(g) * u = g / (1 + e^-g) * u (granite_elementwise.h:80-108), with e^-g as 2^(-g log2 e)
// and a hardware reciprocal: every kernel family computes SwiGLU with this one sequence.
__device__ __forceinline__ float swiglu(float g, float u) {
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.44269504088896341f)) * u;
}

// a / l for the attention split merge (both the attention kernel's own merge and the
// o-projection's prologue use it, so the two paths agree bit for bit)
__device__ __forceinline__ float attn_div(float a, float l) {
  return a * __builtin_amdgcn_rcpf(l);
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2_t as_h2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }
__device__ __forceinline__ uint32_t h2_bits(half2_t v) { return __builtin_bit_cast(uint32_t, v); }

// acc + a.x*b.x + a.y*b.y, fp16 inputs, fp32 accumulate (v_dot2c_f32_f16).
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), acc, false);
}

// v_mfma_f32_16x16x32_bf16: D = A.B + C with A 16x32, B 32x16 (8 bf16 per lane each) and
// D 16x16 fp32 (4 per lane). Operand layout on gfx950: A[i][k] in lane i + 16(k/8), element
// k%8; B[k][j] in lane j + 16(k/8), element k%8; D[i][j] in lane j + 16(i/4), element i%4.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f32x4_t mfma_bf16(const u32x4_t& a, const u32x4_t& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// v_perm_b32: bytes of {hi:s0, lo:s1} selected by `sel`, 0x0c selects zero.
__device__ __forceinline__ uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
  return __builtin_amdgcn_perm(s0, s1, sel);
}

// 64-bit key whose unsigned order is numpy's argmax order: larger value first, NaN above
// everything, and on ties the smaller index (stored inverted in the low word).
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
  const uint32_t u = __float_as_uint(v);
  uint32_t ord;
  if ((u & 0x7fffffffu) > 0x7f800000u) ord = 0xffffffffu;
  else ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)ord << 32) | (unsigned long long)(0xffffffffu - idx);
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

// Arrival ticket of one of `parts` workgroups on a counter that starts at 0: true for the
// last to arrive. The increment wraps (atomicInc: old >= parts - 1 stores 0), so the last
// arrival leaves the counter at 0 for the next launch with no store of its own; a separate
// system-scope reset at the end of the merge cost 0.2-0.26 us per launch.
__device__ __forceinline__ bool ticket(unsigned* counter, int parts) {
  return atomicInc(counter, (unsigned)(parts - 1)) == (unsigned)(parts - 1);
}

// Attention split record: per (sequence, kv head, split, query head of the group) the fp32
// acc[64] of the split's positions, its running max m (scale*log2e units) at [64], its sum l
// at [65], two pad words; records of one (sequence, kv head) consecutive by split.
constexpr int kAttnRecFloats = 68;
// The o-projection that reads them directly (q4nx_gemv_attn_q4): at most this many splits and
// K-tiles (one 640-thread workgroup per tile-row, four activations per thread).
constexpr int kAttnRecMaxSplits = 18;
constexpr int kAttnRecMaxKTiles = 10;

// 16-byte system-coherent (sc0 sc1) loads and stores through a raw buffer resource over
// [base, base + bytes): the compiler tracks their completion like any other load, and
// out-of-range offsets read 0 / drop the store (the buffer unit's own bounds check).
typedef int v4i_t __attribute__((ext_vector_type(4)));
constexpr int kCacheSys = 0x11;  // sc0 | sc1
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ uint4 ld16_sys(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const v4i_t v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kCacheSys);
  return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
}
__device__ __forceinline__ void st16_sys(__amdgpu_buffer_rsrc_t r, uint32_t off, uint4 u) {
  const v4i_t v = {(int)u.x, (int)u.y, (int)u.z, (int)u.w};
  __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)off, 0, kCacheSys);
}

// Pins a value at this point of the program: arithmetic on it cannot be hoisted above,
// and (with the memory clobber) loads issued before stay before. Used so that waits for
// activation loads land after a wave has issued its weight stream.
__device__ __forceinline__ void pin(uint4& v) {
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w) : : "memory");
}
__device__ __forceinline__ void pin(float4& v) {
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w) : : "memory");
}

// v + (v of lane ^ 16), in every lane, with no LDS round trip: v_permlane16_swap exchanges
// the odd 16-lane rows of its first operand with the even rows of its second, so with v in
// both the two results hold rows (v0, v0, v2, v2) and (v1, v1, v3, v3). The sum is the same
// in both lanes of a pair (addition commutes), as with a shuffle.
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// The same across the two 32-lane halves: v_permlane32_swap gives (v_lo, v_lo) and (v_hi, v_hi).
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// DPP lane exchanges (a VALU operand modifier, no LDS traffic).
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i inside each 8 lanes
constexpr int kDppRor4 = 0x124;       // rotate by 4 inside each row of 16 lanes
constexpr int kDppRor8 = 0x128;       // rotate by 8 inside each row of 16 lanes
constexpr int kDppRowBcast = 0x150;   // + n: lane n of each row of 16 lanes to the whole row
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
// f(std::integral_constant<int, I>) for I = B .. E-1, each with I a constant expression.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// All-reduce over aligned groups of 16 or 32 lanes; every lane of the group ends with the
// bit-identical result (each step combines the same two values in either order).
__device__ __forceinline__ float group16_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  return fmaxf(v, dpp<kDppRor8>(v));
}
__device__ __forceinline__ float group16_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  return v + dpp<kDppRor8>(v);
}
__device__ __forceinline__ float group32_max(float v) {
  v = group16_max(v);
  return fmaxf(v, __shfl_xor(v, 16));
}
__device__ __forceinline__ float group32_sum(float v) { return xor16_sum(group16_sum(v)); }

// Sum / max over the wave: DPP inside each row of 16 lanes, then the four row results read
// into scalars and combined in a fixed order (every lane gets the same value).
__device__ __forceinline__ float lane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ float wave_sum(float v) {
  v = group16_sum(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
  v = group16_max(v);
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// RMSNorm from the producer's sums of squares: a row of x has n = K/16 partial sums (one per
// 16 entries; n is a multiple of 16 and the row 16-byte aligned). Lane l loads the float4s
// at entries 4(l + 64j), j < NQ (one load instruction each, so the 64 lanes of a wave touch
// each line of the row once), and adds them as (s.x + s.y) + (s.z + s.w) in j order;
// wave_sum of the lane sums is the row's total. Every consumer of the sums uses this order,
// so all kernel families normalise with the same bits.
constexpr int kSsqRows = 16;   // entries per partial sum of squares
template <int NQ>
__device__ __forceinline__ void ssq_load(const float* row, int lane, int n, float4 (&q)[NQ]) {
  // through a buffer resource over the row's n floats: lanes past its end read zeros with no
  // memory access (and ssq_lane_sum leaves them out)
  const __amdgpu_buffer_rsrc_t r = make_rsrc(row, (uint32_t)n * 4u);
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    const v4i_t v = __builtin_amdgcn_raw_buffer_load_b128(r, 16 * (lane + 64 * j), 0, 0);
    q[j] = make_float4(__int_as_float(v.x), __int_as_float(v.y), __int_as_float(v.z),
                       __int_as_float(v.w));
  }
}
template <int NQ>
__device__ __forceinline__ float ssq_lane_sum(const float4 (&q)[NQ], int lane, int n) {
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NQ; ++j)
    if (4 * (lane + 64 * j) < n) s += (q[j].x + q[j].y) + (q[j].z + q[j].w);
  return s;
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
