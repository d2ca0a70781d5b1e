// Prefill contraction on the matrix cores (gfx950): Y[m][n] = R[m][n] + sum_k W[n][k] X[m][k]
// for many rows of X (a prompt block), W read in the q4nx tile layout.
//
// Replaces, for prompt blocks, the torch fallback that reference/npu.py:118-122, 138-140 takes
// for more than one row, as the batched kernel (gemm.hip) does for smaller row counts.
//
// Arithmetic. With the Q4_1 factoring of granite_gemv.h:19-29 per 32-K group g and column n,
//   y[m][n] = sum_g d[n][g] P[m][n][g] + sum_g u[n][g] S[m][g]
//   P[m][n][g] = sum_{k in g} b[n][k] x[m][k]   b = 16 + c (q4) or q + 128 (q8): exact bf16
//   S[m][g]    = sum_{k in g} x[m][k]           fp32, from a pre-pass over x
//   u[n][g]    = m - 16 d (q4) or -128 s (q8)   exact in fp32
// P is one v_mfma_f32_16x16x32_bf16 per 16x16 block and group (exact products, fp32 sums) and
// its scale one fp32 FMA per output on the VALU. The minimum term is a contraction over the
// groups, 32 groups per MFMA, with S split into three bf16 terms (S = s1 + s2 + s3 exactly)
// and u into three (q4; u = u1 + u2 + u3) or one (q8: -128 s is a bf16 value): the products
// s1u1, s2u1, s3u1 (+ s1u2, s2u2, s1u3 for q4) carry it to fp32 precision. That is one MFMA
// per block and group plus 6/32 (q4) or 3/32 (q8) of one, where folding scale and minimum
// into hi/lo weight operands took three (q4) or two (q8). A one-hot row reproduces the fp32
// dequantised column bit for bit: d (16 + c) is exact, and so is its sum with u.
//
// Work decomposition: a workgroup of four waves takes one block of 16*MT rows of X and four
// tile-rows; wave w owns tile-row 4*blockIdx.x + w for the whole K, so nothing is merged
// across waves or workgroups. Each wave stages its tile in its own LDS slot (the transposing
// LDS read needs it there) while the next tile is in flight to registers. The block's x is
// loaded once for the four waves, by direct global-to-LDS loads into a ring of four step
// buffers, three steps ahead of their use (one barrier per step), laid out so that each
// m-tile's A operand is one conflict-free 16-byte LDS read per lane. The minimum term runs
// first, from the tile-row's scales and minima (re-read: a fifth of its bytes) and the
// pre-pass's sums, so the main loop carries no state for it. The outputs leave through the
// ring as 128-byte row segments.

#include "common.h"
#include "gemm.h"
#include "gemm_fmt.h"

namespace q4nx {

namespace {

constexpr int kPfWaves = 4;
constexpr int kPfChunkTiles = 4;   // K-tiles (32 groups) per minimum-term contraction
constexpr int kPfMT = 8;           // m-tiles (16 rows) per workgroup

// One 32-K step's weight operands of this lane's two columns: the codes as exact bf16 and
// the group's scale of each column.
struct PfOps {
  u32x4_t b[2];
  float d[2];
};

// What a step's operands are built from, read from the wave's tile slot: the transposed code
// bytes and the scales of the lane's two columns at group kb.
struct PfRaw {
  i32x2_t cb[2];
  uint32_t sc;
};

template <int KIND>
__device__ __forceinline__ void pf_read(const uint8_t* slot, int tr_off, int meta_off, int kb,
                                        PfRaw& r) {
  if constexpr (KIND == 4) {
    r.cb[0] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2_t*)(slot + tr_off + kb * 256));
    r.sc = *(const uint32_t*)(slot + kb * 64 + meta_off);
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h)
      r.cb[h] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          (lds_i32x2_t*)(slot + tr_off + h * 4096 + kb * 512));
    r.sc = (uint32_t) * (const uint16_t*)(slot + kb * 64 + meta_off) |
           ((uint32_t) * (const uint16_t*)(slot + kb * 64 + 32 + meta_off) << 16);
  }
}

template <int KIND>
__device__ __forceinline__ void pf_build(const PfRaw& r, PfOps& o) {
  if constexpr (KIND == 4) q4_operands(r.cb[0], o.b[0], o.b[1]);
  else {
    o.b[0] = q8_operand(r.cb[0]);
    o.b[1] = q8_operand(r.cb[1]);
  }
  o.d[0] = bf16lo(r.sc);
  o.d[1] = bf16hi(r.sc);
}

// s_waitcnt immediate that waits until at most n vector-memory operations are outstanding
// (vmcnt bits 3:0 and 15:14; expcnt and lgkmcnt left at their maxima, so they are not waited on)
constexpr int vm_wait(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) & 3) << 14; }

// (x0, x1) = t[0] + t[1] + t[2] exactly, as packed bf16 pairs (x0 in the low halves)
__device__ __forceinline__ void split3(float x0, float x1, uint32_t (&t)[3]) {
  t[0] = pack_bf16x2_op(x0, x1);
  const float r0 = x0 - bf16lo(t[0]), r1 = x1 - bf16hi(t[0]);
  t[1] = pack_bf16x2_op(r0, r1);
  t[2] = pack_bf16x2_op(r0 - bf16lo(t[1]), r1 - bf16hi(t[1]));
}

// Per-group sums of x in the A-operand order of the minimum term: for m-tile t (16 rows),
// chunk ch (32 groups) and term i, lane l holds rows 16 t + l % 16 at groups
// 32 ch + 8 (l / 16) + j, j = 0..7, as bf16: sums[((t * n_ch + ch) * 3 + i) * 64 + l].
// Rows past m_rows and groups past n_groups are zero. One workgroup per (m-tile, chunk):
// thread (row r, pair p) sums groups 2p, 2p + 1 of the chunk (128 contiguous bytes of x).
__global__ __launch_bounds__(256) void pf_sums_kernel(const uint16_t* __restrict__ x,
                                                      int64_t x_stride, int m_rows, int n_groups,
                                                      int n_ch, u32x4_t* __restrict__ sums) {
  __shared__ float sm[16][33];
  const int tid = threadIdx.x;
  const int t = blockIdx.x / n_ch, ch = blockIdx.x - t * n_ch;
  {
    const int r = tid >> 4, p = tid & 15;
    const int row = 16 * t + r;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int g = 32 * ch + 2 * p + e;
      float s = 0.f;
      if (row < m_rows && g < n_groups) {
        const u32x4_t* src = (const u32x4_t*)(x + (int64_t)row * x_stride + 32 * g);
        float q[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const u32x4_t w = src[i];
          q[i] = ((bf16lo(w[0]) + bf16hi(w[0])) + (bf16lo(w[1]) + bf16hi(w[1]))) +
                 ((bf16lo(w[2]) + bf16hi(w[2])) + (bf16lo(w[3]) + bf16hi(w[3])));
        }
        s = (q[0] + q[1]) + (q[2] + q[3]);
      }
      sm[r][2 * p + e] = s;
    }
  }
  __syncthreads();
  if (tid >= 64) return;
  const int r = tid & 15, g0 = 8 * (tid >> 4);
  u32x4_t o[3];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t tt[3];
    split3(sm[r][g0 + 2 * w], sm[r][g0 + 2 * w + 1], tt);
#pragma unroll
    for (int i = 0; i < 3; ++i) o[i][w] = tt[i];
  }
  u32x4_t* dst = sums + (size_t)blockIdx.x * 3 * 64 + tid;
#pragma unroll
  for (int i = 0; i < 3; ++i) dst[i * 64] = o[i];
}

template <int KIND, int MT>
__global__ __launch_bounds__(256) void gemm_pf_kernel(GemmArgs a, const u32x4_t* __restrict__ sums) {
  constexpr int SLOT = GemmFmt<KIND>::kSlot;
  constexpr int NLD = GemmFmt<KIND>::kLoads;
  constexpr int TB = GemmFmt<KIND>::kTile;
  constexpr int MB = 16 * MT;
  constexpr int UPT = MB * 4 / 256;        // 16-byte x units per thread and 32-K step
  constexpr int XB = MB * 4 * 16;          // bytes of one staged step of x
  constexpr int XD = 3;                    // steps of x in flight to LDS ahead of their step
  constexpr int NU = KIND == 4 ? 3 : 1;    // bf16 terms of u
  // The x ring: four step buffers, step t in buffer t % 4 (a position the unrolled steps of a
  // K-tile know at compile time), and the four waves' tile slots.
  __shared__ __attribute__((aligned(16))) uint8_t xr0[XB], xr1[XB], xr2[XB], xr3[XB];
  __shared__ __attribute__((aligned(16))) uint8_t slots[kPfWaves * SLOT];

  const int tid = threadIdx.x, l = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_tr = a.n_tr[0];
  const int tr = blockIdx.x * kPfWaves + wave;
  const bool live = tr < n_tr;                    // a wave past the last tile-row only helps
  const int trc = live ? tr : n_tr - 1;
  const int m0 = blockIdx.y * MB;
  const uint8_t* wr = a.w[0] + (size_t)trc * a.k_t * TB;
  uint8_t* slot = slots + wave * SLOT;            // this wave's weight tile
  const int c = l & 15, s = l >> 4;
  const int n_steps = a.k_t * 8;
  const int n_ch = (a.k_t + kPfChunkTiles - 1) / kPfChunkTiles;
  // this workgroup's per-group sums: m-tile mt, chunk ch, term i at sblk[((mt n_ch + ch) 3 + i) 64]
  const u32x4_t* sblk = sums + (size_t)blockIdx.y * MT * n_ch * 3 * 64 + l;

  const int tr_off = KIND == 4
      ? GemmFmt<4>::kCodes + (c & 1) * 2048 + (8 * s + (c >> 1)) * 8
      : GemmFmt<8>::kCodes + (8 * s + (c >> 1)) * 16 + (c & 1) * 8;
  const int meta_off = KIND == 4 ? 2 * ((c >> 3) * 16 + 2 * (c & 7)) : 2 * c;

  int ld_off[NLD];
#pragma unroll
  for (int i = 0; i < NLD; ++i)
    ld_off[i] = 16 * (64 * i + l) - ((KIND == 8 && i == NLD - 1 && l >= 32) ? 512 : 0);

  // x unit u of a step (16 bytes): m-tile u >> 6, k-slot group (u >> 4) & 3, row u & 15 —
  // staged at byte 16 u, where lane (row, group) of an m-tile's A operand reads it
  const uint16_t* xsrc[UPT];
#pragma unroll
  for (int j = 0; j < UPT; ++j) {
    const int u = tid + 256 * j;
    const int m = min(m0 + 16 * (u >> 6) + (u & 15), a.m_rows - 1);
    xsrc[j] = a.x + (int64_t)m * a.x_stride + 8 * ((u >> 4) & 3);
  }
  auto xring = [&](int b) -> uint8_t* { return b == 0 ? xr0 : b == 1 ? xr1 : b == 2 ? xr2 : xr3; };
  // x of a step straight from memory into its ring buffer (global_load_lds_dwordx4: lane l's
  // 16 bytes land at the wave's base in M0 + 16 l, which is this layout). Issued as inline
  // assembly: the compiler would otherwise wait for every direct load in flight before each
  // read of the ring. The waits at the end of each step order the loads instead (vmcnt
  // counts them, and loads complete in issue order, so a wait the compiler places for another
  // load can only wait longer than it needs).
  auto x_load = [&](int step, uint8_t* buf) {
    const int st = step < n_steps ? step : n_steps - 1;   // past the end: a re-read, never used
    const int k = (st >> 3) * 256 + (st & 7) * 32;
    const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)buf +
                          16 * 64 * wave;
#pragma unroll
    for (int j = 0; j < UPT; ++j)
      asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                   :: "v"(xsrc[j] + k), "s"(base + 16 * 256 * j) : "memory", "m0");
  };

  // Pipeline: during step s the MFMAs of s run while this wave builds the weight operands of
  // s + 1 from its tile slot and loads x of s + XD into the ring; one barrier ends each step.
  // The first steps' x and the first tile go out before the minimum term, whose own loads
  // then wait alongside them.
  u32x4_t pf[NLD];
#pragma unroll
  for (int i = 0; i < NLD; ++i) pf[i] = *(const u32x4_t*)(wr + ld_off[i]);
#pragma unroll
  for (int t = 0; t < XD; ++t) x_load(t, xring(t));

  // ---- the minimum term first: acc = sum_g u S over every chunk of 32 groups. The lane's
  // B operand holds u of its two columns at groups 32 ch + 8 s + j, read from the
  // tile-row's scales and minima (K-tile 4 ch + s, group j); its A operands are the
  // pre-pass's S terms of each m-tile.
  f32x4_t acc[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt][0] = acc[mt][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int ch = 0; ch < n_ch; ++ch) {
    const int kt = kPfChunkTiles * ch + s;
    float u[2][8];
    if (kt < a.k_t) {
      const uint8_t* tile = wr + (size_t)kt * TB;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if constexpr (KIND == 4) {
          const uint32_t dv = *(const uint32_t*)(tile + j * 64 + meta_off);
          const uint32_t mv = *(const uint32_t*)(tile + kMetaBytes + j * 64 + meta_off);
          u[0][j] = fmaf(-16.f, bf16lo(dv), bf16lo(mv));
          u[1][j] = fmaf(-16.f, bf16hi(dv), bf16hi(mv));
        } else {
#pragma unroll
          for (int h = 0; h < 2; ++h)
            u[h][j] = -128.f * bf16_to_f32(*(const uint16_t*)(tile + j * 64 + h * 32 + meta_off));
        }
      }
    } else {   // past K: groups whose S is zero
#pragma unroll
      for (int j = 0; j < 8; ++j) u[0][j] = u[1][j] = 0.f;
    }
    u32x4_t U[NU][2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        uint32_t tt[3];
        split3(u[h][2 * w], u[h][2 * w + 1], tt);
#pragma unroll
        for (int i = 0; i < NU; ++i) U[i][h][w] = tt[i];
      }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      u32x4_t S[3];
#pragma unroll
      for (int i = 0; i < 3; ++i) S[i] = sblk[((mt * n_ch + ch) * 3 + i) * 64];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        f32x4_t r = acc[mt][h];
        r = mfma_bf16(S[0], U[0][h], r);
        r = mfma_bf16(S[1], U[0][h], r);
        r = mfma_bf16(S[2], U[0][h], r);
        if constexpr (NU == 3) {
          r = mfma_bf16(S[0], U[1][h], r);
          r = mfma_bf16(S[1], U[1][h], r);
          r = mfma_bf16(S[0], U[2][h], r);
        }
        acc[mt][h] = r;
      }
    }
  }

  {
    // every load so far has landed (the minimum term waited for its own, issued after them)
    __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
    for (int i = 0; i < NLD; ++i) *(u32x4_t*)(slot + 16 * (64 * i + l)) = pf[i];
    const size_t off = (size_t)(a.k_t > 1 ? 1 : 0) * TB;
#pragma unroll
    for (int i = 0; i < NLD; ++i) pf[i] = *(const u32x4_t*)(wr + off + ld_off[i]);
  }
  __syncthreads();
  // the next step's operand data is read from LDS one step ahead (in the step before, ahead
  // of its MFMAs), and so is the first m-tile of its x, so no LDS latency is exposed
  PfOps ops[2];
  PfRaw raw;
  pf_read<KIND>(slot, tr_off, meta_off, 0, raw);
  pf_build<KIND>(raw, ops[0]);
  u32x4_t x0 = *(const u32x4_t*)(xr0 + 16 * l);
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};

  for (int kt = 0; kt < a.k_t; ++kt) {
#pragma unroll
    for (int kb = 0; kb < 8; ++kb) {
      const int step = kt * 8 + kb;
      const int cur = kb & 1, nxt = cur ^ 1;
      // ---- this step's groups: P on the matrix cores, its scale on the VALU
      x_load(step + XD, xring((kb + XD) & 3));
      const uint8_t* xb = xring(kb & 3);
      if (kb < 7) pf_read<KIND>(slot, tr_off, meta_off, kb + 1, raw);
      // Pipelined by m-tile, fenced so that the schedule holds: x of m-tile mt + 1 is read
      // from LDS, the two MFMAs of mt issue, then m-tile mt - 1's P is scaled on the VALU
      // while they run; two m-tiles' P are live at a time.
      {
        constexpr int XA = 1;        // m-tiles of x read ahead of their MFMAs
        constexpr int FENCE = 1;     // m-tiles between schedule fences
        u32x4_t xa[XA + 1];
        f32x4_t p[2][2];
        xa[0] = x0;
#pragma unroll
        for (int i = 1; i < XA; ++i) xa[i] = *(const u32x4_t*)(xb + 16 * (64 * i + l));
#pragma unroll
        for (int mt = 0; mt <= MT; ++mt) {
          if (mt + XA < MT)
            xa[(mt + XA) % (XA + 1)] = *(const u32x4_t*)(xb + 16 * (64 * (mt + XA) + l));
          if (mt < MT) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
              p[mt & 1][h] = mfma_bf16(xa[mt % (XA + 1)], ops[cur].b[h], zero);
          }
          if (mt > 0) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
              for (int e = 0; e < 4; ++e)
                acc[mt - 1][h][e] = fmaf(ops[cur].d[h], p[(mt - 1) & 1][h][e], acc[mt - 1][h][e]);
          }
          if (FENCE > 0 && mt % FENCE == FENCE - 1) __builtin_amdgcn_sched_barrier(0);
        }
      }
      // ---- the next step's operands (the next tile into the slot first at a tile boundary;
      // past the last step they are built from re-read data and not used)
      if (kb == 7) {
#pragma unroll
        for (int i = 0; i < NLD; ++i) *(u32x4_t*)(slot + 16 * (64 * i + l)) = pf[i];
        const size_t off = (size_t)(kt + 2 < a.k_t ? kt + 2 : a.k_t - 1) * TB;
#pragma unroll
        for (int i = 0; i < NLD; ++i) pf[i] = *(const u32x4_t*)(wr + off + ld_off[i]);
        pf_read<KIND>(slot, tr_off, meta_off, 0, raw);
      }
      pf_build<KIND>(raw, ops[nxt]);
      x0 = *(const u32x4_t*)(xring((kb + 1) & 3) + 16 * l);
      // This thread's direct loads of step + 2's x must have landed before the barrier, after
      // which everyone reads them. Loads complete in issue order, and issued after them are
      // only step + 3's x (at the start of this step) and the next tile's prefetch when this
      // step or the one before ended a K-tile (kb 7, after its x load): wait for all but those.
      // (A read of the buffer would make the compiler wait for every direct load in flight.)
      if (kb == 0 || kb == 7) __builtin_amdgcn_s_waitcnt(vm_wait(UPT + NLD));
      else __builtin_amdgcn_s_waitcnt(vm_wait(UPT));
      __syncthreads();
    }
  }

  // ---- outputs, through the x ring once every wave is done with it and the direct loads of
  // the steps past the end have landed (each wave waits for its own, then the barrier): wave w
  // stages half of its [MB][32] block at a time in buffer w (MB/2 rows of 128 bytes = XB;
  // row m = 16 mt + 4 s + e, column of operand h at lane c) and reads it back as 128-byte
  // row segments
  __builtin_amdgcn_s_waitcnt(vm_wait(0));
  __syncthreads();
  float* blk = (float*)xring(wave);
  const int q = l & 7, r0 = l >> 3;   // 8 lanes per 32-float row, 8 rows per pass
#pragma unroll
  for (int half = 0; half < 2; ++half) {
#pragma unroll
    for (int mt = half * MT / 2; mt < (half + 1) * MT / 2; ++mt)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int col = KIND == 4 ? (c >> 3) * 16 + 2 * (c & 7) + h : h * 16 + c;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          blk[(16 * (mt - half * MT / 2) + 4 * s + e) * 32 + col] = acc[mt][h][e];
      }
    if (live) {
#pragma unroll
      for (int p = 0; p < MB / 16; ++p) {
        const int r = 8 * p + r0, m = m0 + half * (MB / 2) + r;
        if (m < a.m_rows) {
          float4 v = *(const float4*)(blk + r * 32 + 4 * q);
          const int64_t o = (int64_t)m * a.y_stride + (int64_t)tr * 32 + 4 * q;
          if (a.residual != nullptr) {
            const float4 rr = *(const float4*)(a.residual + o);
            v.x += rr.x;
            v.y += rr.y;
            v.z += rr.z;
            v.w += rr.w;
          }
          *(float4*)(a.y + o) = v;
        }
      }
    }
  }
}

template <int KIND, int MT>
void pf_go(const GemmArgs& a, const u32x4_t* sums, hipStream_t st) {
  const dim3 grid((unsigned)((a.n_tr[0] + kPfWaves - 1) / kPfWaves),
                  (unsigned)((a.m_rows + 16 * MT - 1) / (16 * MT)));
  hipLaunchKernelGGL((gemm_pf_kernel<KIND, MT>), grid, dim3(256), 0, st, a, sums);
}

// m-tiles the sums cover (whole 128-row blocks, enough for either block size) and chunks of 32
// groups
int pf_mtiles(int m_rows) { return (m_rows + 16 * kPfMT - 1) / (16 * kPfMT) * kPfMT; }
int pf_chunks(int k_t) { return (k_t + kPfChunkTiles - 1) / kPfChunkTiles; }
size_t pf_align256(size_t b) { return (b + 255) & ~(size_t)255; }

// Workgroups of the prefill kernel with blocks of 16 * mt rows (four tile-rows each).
int pf_workgroups(int n_tile_rows, int m_rows, int mt) {
  return ((n_tile_rows + kPfWaves - 1) / kPfWaves) * ((m_rows + 16 * mt - 1) / (16 * mt));
}

// Row-block size of a launch: 128 rows from three workgroups per CU, else 64 rows from two;
// 0 when neither fills the chip (the batched kernel takes the launch). Measured at 2048 rows:
// q4 2560->8192 (1024 / 2048 workgroups) 541 / 535 TFLOP/s; q4 8192->2560 (320 / 640) 458 on
// 64-row blocks against 340 on the batched kernel; q8 248320x1024 at 512 rows (7760 / 15520)
// 425 / 364.
int pf_block_mtiles(int n_tile_rows, int m_rows) {
  if (m_rows < kPrefillRows) return 0;
  if (pf_workgroups(n_tile_rows, m_rows, kPfMT) >= 768) return kPfMT;
  if (pf_workgroups(n_tile_rows, m_rows, kPfMT / 2) >= 512) return kPfMT / 2;
  return 0;
}

}  // namespace

size_t pf_ws_bytes(int n_tile_rows, int k_t, int m_rows) {
  if (pf_block_mtiles(n_tile_rows, m_rows) == 0) return 0;
  return pf_align256((size_t)pf_mtiles(m_rows) * pf_chunks(k_t) * 3 * 64 * sizeof(u32x4_t));
}

// A plain contraction goes to the prefill kernel when it fills the chip (pf_block_mtiles), with
// no sums-of-squares or argmax epilogue (those stay on the batched kernel).
bool pf_use(int op, const GemmArgs& a) {
  return op == GOP_PLAIN && a.ssq_out == nullptr && a.argmax_keys == nullptr &&
         pf_ws_bytes(a.n_tr[0], a.k_t, a.m_rows) > 0;
}

void pf_launch(int kind, const GemmArgs& a, void* sums, hipStream_t st) {
  const int n_ch = pf_chunks(a.k_t);
  hipLaunchKernelGGL(pf_sums_kernel, dim3((unsigned)(pf_mtiles(a.m_rows) * n_ch)), dim3(256), 0,
                     st, a.x, a.x_stride, a.m_rows, a.k_t * 8, n_ch, (u32x4_t*)sums);
  const bool big = pf_block_mtiles(a.n_tr[0], a.m_rows) == kPfMT;
  const u32x4_t* sp = (const u32x4_t*)sums;
  if (kind == Q4NX_KIND_Q4) big ? pf_go<4, kPfMT>(a, sp, st) : pf_go<4, kPfMT / 2>(a, sp, st);
  else big ? pf_go<8, kPfMT>(a, sp, st) : pf_go<8, kPfMT / 2>(a, sp, st);
}

}  // namespace q4nx
