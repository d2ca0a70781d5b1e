// q4nx batched contraction on the matrix cores (gfx950): Y[m][n] = R[m][n] + sum_k W[n][k] X[m][k]
// for any number of rows m (batched decode, prefill), W read in the q4nx tile layout.
//
// Replaces the torch fallback that reference/npu.py:118-122, 138-140 takes for more than one
// row (prefill), and extends the batched design of designs/granite_gemv/granite_gemv.h:79-91
// (B tokens share one weight pass) from B <= 8 to any row count.
//
// Operands of v_mfma_f32_16x16x32_bf16 (verified layout: A[i][k] in lane i + 16(k/8), element
// k%8; B[k][j] in lane j + 16(k/8), element k%8; D[i][j] in lane j + 16(i/4), element i%4):
//   A = x rows (16 per m-tile), loaded straight from global memory: 16 contiguous bytes per
//       lane and 32-K group.
//   B = weight codes, 16 output rows per operand. A q4nx tile stores, per row-block of 16 rows
//       and per k, 8 bytes whose low nibble is row 2p and high nibble row 2p+1 (tools/q4nx.py:
//       46-56). The tile is copied to LDS as stored and read back with ds_read_b64_tr_b8,
//       which hands lane (8h + p) of each 16-lane group the byte of pair p at 8 consecutive k
//       of row-block h: one LDS read yields the codes of 32 rows x 8 k in two operands, the
//       low nibbles (even rows) and the high nibbles (odd rows). For q8 (16 bytes per k and
//       row-block) the same read yields one row-block's 16 rows.
//   Codes become exact bf16 values without a table: a q4 code c in bits 3-6 of 0x4180 is
//   16 + c; a q8 code q, biased to q + 128 in 0..255, converts with v_cvt_f32_ubyte.
// Per 32-K group g each MFMA product P = sum_k (c_k + o) x_k is exact-input, fp32-accumulated,
// and one more MFMA against ones gives S = sum_k x_k for every row; the Q4_1 identity
// (granite_gemv.h:19-29) y += d P + (m - o d) S (q4: o = 16) or s P - 128 s S (q8) is
// applied in fp32 per group. Waves along K combine through LDS in a fixed order; split-K
// across workgroups publishes parts with system-scope stores and the last arriver adds them
// in part order, as the GEMV does, so results are bit-reproducible.

#include <atomic>
#include "common.h"
#include "gemm.h"
#include "gemm_fmt.h"

namespace q4nx {

// One workgroup of NWV waves owns RT tile-rows x (16 MT WM) rows of X over the K-tiles of its
// part; WK waves split those K-tiles round-robin and WM = NWV / WK waves take different
// m-tiles. Each wave stages one tile per tile-row at a time in its own LDS slot while the next
// tile's bytes are in flight to registers. With one m-tile (decode batches) the workgroup has
// as many waves as its part has K-tiles (up to 10 or 16), so every wave issues all of its
// loads at once, as the one-row kernels do. RB (one m-tile, small grids): the two 16-row
// blocks of each group go to two workgroups, 8 apart (one XCD, so the metadata both stage
// comes from one L2), each staging the metadata and its block's codes only and taking one
// operand and one MFMA per tile-row and 32-K group.
template <int KIND, int OP, int RT, int MT, int WK, int NWV, bool RB = false>
__global__ __launch_bounds__(64 * NWV) void gemm_kernel(GemmArgs a) {
  constexpr int WM = NWV / WK;
  constexpr int NT = 64 * NWV;              // threads
  constexpr int SLOT = RB ? GemmFmt<KIND>::kSlotRB : GemmFmt<KIND>::kSlot;
  constexpr int NLD = RB ? GemmFmt<KIND>::kLoadsRB : GemmFmt<KIND>::kLoads;
  constexpr int TB = GemmFmt<KIND>::kTile;
  constexpr int MB = 16 * MT * WM;          // rows of X per workgroup
  constexpr int TW = RB ? 16 : 32;          // outputs per tile-row per workgroup
  constexpr int NW = RT * TW;               // outputs per row of X per workgroup
  static_assert(!RB || MT == 1, "row-block workgroups: one m-tile");
  static_assert(OP == GOP_PLAIN || RT == 2, "fused epilogues pair two tile-rows");
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ int s_last;
  __shared__ unsigned long long skey[OP == GOP_PLAIN ? MB * NW / 16 : 1];

  const int tid = threadIdx.x, l = tid & 63, wave = tid >> 6;
  const int wk = wave % WK, wm = wave / WK;
  const int unit = blockIdx.x / a.ksplit, kpart = blockIdx.x % a.ksplit;
  int group = unit, rb = 0;   // RB: the row block of the group's tile-rows
  if constexpr (RB) {
    if (((gridDim.x / a.ksplit) & 15) == 0) {
      group = (unit >> 4) * 8 + (unit & 7);
      rb = (unit >> 3) & 1;
    } else {
      group = unit >> 1;
      rb = unit & 1;
    }
  }
  const int mblk = blockIdx.y;
  const int m0 = mblk * MB + wm * 16 * MT;  // first row of this wave's m-tiles
  const int kbeg = kpart * a.kpp;
  const int kend = min(a.k_t, kbeg + a.kpp);
  const int n_it = kend - kbeg > wk ? (kend - kbeg - wk + WK - 1) / WK : 0;
  uint8_t* slot = lds + wave * RT * SLOT;

  // weight tile-rows of this group
  int seg = 0, hg = group;
  const uint8_t* wr[RT];
  if constexpr (OP == GOP_PLAIN) {
#pragma unroll
    for (int r = 0; r < RT; ++r) wr[r] = a.w[0] + (size_t)(group * RT + r) * a.k_t * TB;
  } else if constexpr (OP == GOP_GATEUP) {
#pragma unroll
    for (int r = 0; r < RT; ++r) wr[r] = a.w[r] + (size_t)group * a.k_t * TB;
  } else {
    if (group >= a.grp_q + a.grp_k) {
      seg = 2;
      hg = group - a.grp_q - a.grp_k;
    } else if (group >= a.grp_q) {
      seg = 1;
      hg = group - a.grp_q;
    }
#pragma unroll
    for (int r = 0; r < RT; ++r) wr[r] = a.w[seg] + (size_t)(2 * hg + r) * a.k_t * TB;
  }

  const int c = l & 15, s = l >> 4;         // operand column / k-slot group
  // ds_read_b64_tr_b8 row addresses: lane c of a 16-lane group addresses row (2j + h) with
  // j = c/2, h = c%2 -> k = 8s + j of row-block h (q4) or row half h (q8)
  // RB: the slot holds the metadata and one block's codes; for q4 both halves of a 16-lane
  // group address that block, so lanes c and c + 8 receive the same bytes (row pair c % 8)
  // and take their low / high nibbles
  const int tr_off = KIND == 4
      ? GemmFmt<4>::kCodes + (RB ? 0 : (c & 1) * 2048) + (8 * s + (c >> 1)) * 8
      : GemmFmt<8>::kCodes + (8 * s + (c >> 1)) * 16 + (c & 1) * 8;
  // this lane's output column within a tile-row, per operand: q4 even/odd row of pair p of
  // row-block h (c = 8h + p); q8 row c of row-block 0 / 1
  // (RB: q4 rows 2p, 2p + 1 of the block, the lane keeping row 2p + c / 8; q8 row c of it)
  const int meta_off = KIND == 4 ? 2 * ((RB ? rb : (c >> 3)) * 16 + 2 * (c & 7))
                                 : 2 * c + (RB ? rb * 32 : 0);
  const bool nib = RB && KIND == 4 && (c >> 3);   // RB q4: the high nibble's row
  const uint32_t rot = nib ? 1u : 29u;

  f32x4_t acc[RT][MT][2];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[r][mt][0] = acc[r][mt][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const u32x4_t ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};

  // this lane's 16-byte pieces of a tile: piece i at 16 (64 i + l); the last q8 piece of lanes
  // 32..63 re-reads bytes inside the tile (its LDS copy lands in the slot's padding)
  // (RB: staged piece i is the metadata below kCodes, then the block's codes)
  int ld_off[NLD];
#pragma unroll
  for (int i = 0; i < NLD; ++i) {
    const int o = 16 * (64 * i + l);
    if constexpr (RB) {
      constexpr int MC = GemmFmt<KIND>::kCodes, BC = GemmFmt<KIND>::kBlockCodes;
      ld_off[i] = o < MC ? o : MC + rb * BC + min(o - MC, BC - 16);
      // q4: each 64-byte group of d (and of m) holds row block 0's 32 bytes, then block 1's
      if (KIND == 4 && o < MC && ((l >> 1) & 1) != rb) ld_off[i] = -1;
    } else {
      ld_off[i] = o - ((KIND == 8 && i == NLD - 1 && l >= 32) ? 512 : 0);
    }
  }

  // RB q4: the weights through buffer resources over the tile-rows, so the other row
  // block's metadata (ld_off -1) reads out of range: zeros, no memory access
  __amdgpu_buffer_rsrc_t wrs[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) wrs[r] = make_rsrc(wr[r], (uint32_t)(a.k_t * TB));
  auto wload = [&](int r, size_t off, int i) -> u32x4_t {
    if constexpr (RB && KIND == 4) {
      const uint32_t o = ld_off[i] < 0 ? 0x80000000u : (uint32_t)(off + ld_off[i]);
      const v4i_t v = __builtin_amdgcn_raw_buffer_load_b128(wrs[r], (int)o, 0, 0);
      return u32x4_t{(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
    } else {
      return *(const u32x4_t*)(wr[r] + off + ld_off[i]);
    }
  };
  // The epilogue's own inputs are requested ahead of the weight stream: the residual of each
  // (row, output) this thread finishes (plain), the sequence positions and, once the weight
  // loads are out, their cos/sin (q/k/v). Loaded in the epilogue they put one (two, the table
  // read depending on the position) memory round trips after the last MFMA.
  constexpr int EIT_P = (MB * NW + NT - 1) / NT;   // plain epilogue iterations per thread
  constexpr int EIT_Q = (MB * TW + NT - 1) / NT;   // q/k/v epilogue iterations per thread
  constexpr bool PF_RES = OP == GOP_PLAIN && EIT_P <= 2;
  constexpr bool PF_POS = OP == GOP_QKV && EIT_Q <= 2;
  float ep_res[PF_RES ? EIT_P : 1] = {};
  int ep_pos[PF_POS ? EIT_Q : 1];
  bool ep_live[PF_POS ? EIT_Q : 1];
  float ep_cs[PF_POS ? EIT_Q : 1] = {}, ep_sn[PF_POS ? EIT_Q : 1] = {};
  if constexpr (PF_RES) {
    if (a.residual != nullptr) {
      const int64_t gn0 = (int64_t)(group * RT * 2 + rb) * 16;
#pragma unroll
      for (int i = 0; i < EIT_P; ++i) {
        const int e = i * NT + tid, gm = mblk * MB + e / NW;
        if (e < MB * NW && gm < a.m_rows) ep_res[i] = a.residual[gm * a.y_stride + gn0 + e % NW];
      }
    }
  }
  if constexpr (PF_POS) {
#pragma unroll
    for (int i = 0; i < EIT_Q; ++i) {
      const int e = i * NT + tid, gm = mblk * MB + e / TW;
      // every lane loads (a clamped row): no branch around the load and nothing computed
      // from it here, so the wait for it below counts exactly the weight loads after it
      ep_pos[i] = a.pos[min(gm, a.m_rows - 1)];
      ep_live[i] = e < MB * TW && gm < a.m_rows;
    }
  }
  asm volatile("" ::: "memory");
  const uint16_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = min(m0 + 16 * mt + c, a.m_rows - 1);
    xrow[mt] = a.x + (int64_t)m * a.x_stride + 8 * s;
  }
  // One m-tile (at most 16 rows): the operand rows past the batch load through a buffer
  // resource over the batch's rows at an offset outside it, which returns zeros without a
  // memory access, instead of re-reading the last row (batch-8 decode 3909 -> 3943 tok/s;
  // a branch around those lanes' loads measured slower). Their outputs are never stored.
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x, (uint32_t)((int64_t)a.m_rows * a.x_stride * 2));
  const uint32_t xoff = m0 + c < a.m_rows ? (uint32_t)(((int64_t)(m0 + c) * a.x_stride + 8 * s) * 2)
                                          : 0x80000000u;
  u32x4_t xa[8][MT];
  auto xload = [&](int kt) {
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if constexpr (MT == 1) {
          const v4i_t v = __builtin_amdgcn_raw_buffer_load_b128(
              xrs, (int)(xoff + (uint32_t)(kt * 512 + kb * 64)), 0, 0);
          xa[kb][mt] = u32x4_t{(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
        } else {
          xa[kb][mt] = *(const u32x4_t*)(xrow[mt] + kt * 256 + kb * 32);
        }
      }
  };
  // the first tile's weights, also in a wave with no tile (a clamped tile, never used): no
  // branch around the first loads, so the compiler's counts for the waits below stay exact
  // (after a branch they fall back to waiting for every load)
  u32x4_t pf[RT][NLD];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int i = 0; i < NLD; ++i) pf[r][i] = wload(r, (size_t)min(kbeg + wk, a.k_t - 1) * TB, i);
  asm volatile("" ::: "memory");
  // One m-tile: the first tile's activations right behind its weights, so that they are in
  // flight while the wave waits for the weights (issued after the tile's LDS store, their
  // latency followed the weights' in every one-tile wave, which is every wave of a decode
  // batch's launches; issued ahead of the weights they delayed the weight stream)
  // (a wave with no tile loads bytes it never uses: inside the rows' buffer, or zeros past it)
  if (MT == 1) xload(kbeg + wk);
  asm volatile("" ::: "memory");
  if constexpr (PF_POS) {
    if (seg != 2) {
#pragma unroll
      for (int i = 0; i < EIT_Q; ++i) {
        const int p = ep_live[i] ? ep_pos[i] : -1, d = rb * 16 + (i * NT + tid) % TW;
        if (p >= 0 && p < a.max_pos) {
          ep_cs[i] = a.rope_tab[(int64_t)p * 64 + d];
          ep_sn[i] = a.rope_tab[(int64_t)p * 64 + 32 + d];
        }
      }
    }
  }

  for (int it = 0; it < n_it; ++it) {
    const int kt = kbeg + wk + it * WK;
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int i = 0; i < NLD; ++i) *(u32x4_t*)(slot + r * SLOT + 16 * (64 * i + l)) = pf[r][i];
    // activations of this tile first, then the next tile's weights: the in-order load
    // counter then lets the arithmetic start before the next tile arrives
    if (MT != 1 || it > 0) xload(kt);
    asm volatile("" ::: "memory");
    if (it + 1 < n_it) {   // wave-uniform: a one-iteration wave issues no second tile
      const size_t off = (size_t)(kt + WK) * TB;
#pragma unroll
      for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int i = 0; i < NLD; ++i) pf[r][i] = wload(r, off, i);
    }
    asm volatile("" ::: "memory");

#pragma unroll
    for (int kb = 0; kb < 8; ++kb) {
      f32x4_t sx[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) sx[mt] = mfma_bf16(xa[kb][mt], ones, zero);
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        const uint8_t* sl = slot + r * SLOT;
        if constexpr (RB) {   // one operand: this workgroup's 16 rows
          u32x4_t op;
          float dd, mm;
          if constexpr (KIND == 4) {
            const i32x2_t cb = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                (lds_i32x2_t*)(sl + tr_off + kb * 256));
            op = q4_operand_rb(cb, rot);
            const uint32_t dv = *(const uint32_t*)(sl + kb * 64 + meta_off);
            const uint32_t mv = *(const uint32_t*)(sl + kMetaBytes + kb * 64 + meta_off);
            dd = nib ? bf16hi(dv) : bf16lo(dv);
            mm = fmaf(-16.f, dd, nib ? bf16hi(mv) : bf16lo(mv));
          } else {
            const i32x2_t cb = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                (lds_i32x2_t*)(sl + tr_off + kb * 512));
            op = q8_operand(cb);
            dd = bf16_to_f32(*(const uint16_t*)(sl + kb * 64 + meta_off));
            mm = -128.f * dd;
          }
          const f32x4_t p = mfma_bf16(xa[kb][0], op, zero);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            acc[r][0][0][e] = fmaf(mm, sx[0][e], fmaf(dd, p[e], acc[r][0][0][e]));
          continue;
        }
        u32x4_t op[2];
        float dd[2], mm[2];
        if constexpr (KIND == 4) {
          const i32x2_t cb = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
              (lds_i32x2_t*)(sl + tr_off + kb * 256));
          q4_operands(cb, op[0], op[1]);
          const uint32_t dv = *(const uint32_t*)(sl + kb * 64 + meta_off);
          const uint32_t mv = *(const uint32_t*)(sl + kMetaBytes + kb * 64 + meta_off);
          dd[0] = bf16lo(dv);
          dd[1] = bf16hi(dv);
          mm[0] = fmaf(-16.f, dd[0], bf16lo(mv));
          mm[1] = fmaf(-16.f, dd[1], bf16hi(mv));
        } else {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const i32x2_t cb = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                (lds_i32x2_t*)(sl + tr_off + h * 4096 + kb * 512));
            op[h] = q8_operand(cb);
            dd[h] = bf16_to_f32(*(const uint16_t*)(sl + kb * 64 + h * 32 + meta_off));
            mm[h] = -128.f * dd[h];
          }
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const f32x4_t p = mfma_bf16(xa[kb][mt], op[h], zero);
#pragma unroll
            for (int e = 0; e < 4; ++e)
              acc[r][mt][h][e] = fmaf(mm[h], sx[mt][e], fmaf(dd[h], p[e], acc[r][mt][h][e]));
          }
      }
    }
  }

  // ---- combine the waves: red[wave][m][n] (reuses the staging slots)
  __syncthreads();
  float* red = (float*)lds;
  constexpr int RED = 16 * MT * NW;          // floats per wave
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int h = 0; h < (RB ? 1 : 2); ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = 16 * mt + 4 * s + e;
          // RB: column c holds row 2 (c % 8) + c / 8 (q4) or row c (q8) of the block
          const int n = RB ? r * 16 + (KIND == 4 ? 2 * (c & 7) + (c >> 3) : c)
                           : r * 32 + (KIND == 4 ? (c >> 3) * 16 + 2 * (c & 7) + h : h * 16 + c);
          red[wave * RED + m * NW + n] = acc[r][mt][h][e];
        }
  __syncthreads();
  // the block's row m lives in the record of wave (m / 16MT, wk = 0), row m % 16MT; the other
  // K waves' records are added into it in wave order (each element has one owner thread)
  auto outp = [&](int m, int n) -> float* {
    return red + ((m / (16 * MT)) * WK) * RED + (m % (16 * MT)) * NW + n;
  };
  if constexpr (WK > 1) {
    for (int e = tid; e < MB * NW / 4; e += NT) {
      const int m = (4 * e) / NW, n = (4 * e) % NW;
      float* dst = outp(m, n);
      float4 v = *(const float4*)dst;
#pragma unroll
      for (int k = 1; k < WK; ++k) {
        const float4 u = *(const float4*)(dst + k * RED);
        v.x += u.x;
        v.y += u.y;
        v.z += u.z;
        v.w += u.w;
      }
      *(float4*)dst = v;
    }
    __syncthreads();
  }

  if (a.ksplit > 1) {
    const __amdgpu_buffer_rsrc_t pr = make_rsrc(a.part, a.part_bytes);
    const uint32_t nrec = MB * NW;           // floats per part record
    const int cnt = unit * gridDim.y + mblk;
    const uint32_t rec0 = (uint32_t)(cnt * a.ksplit) * nrec * 4u;
    for (int e = tid; e < (int)nrec / 4; e += NT)
      st16_sys(pr, rec0 + (uint32_t)kpart * nrec * 4u + 16u * e,
               *(const uint4*)outp((4 * e) / NW, (4 * e) % NW));
    wait_vm();
    __syncthreads();
    if (tid == 0) s_last = ticket(&a.counters[cnt], a.ksplit) ? 1 : 0;
    __syncthreads();
    if (!s_last) return;
    for (int e = tid; e < (int)nrec / 4; e += NT) {
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int p = 0; p < a.ksplit; ++p) {
        const uint4 u = ld16_sys(pr, rec0 + (uint32_t)p * nrec * 4u + 16u * e);
        v.x += __uint_as_float(u.x);
        v.y += __uint_as_float(u.y);
        v.z += __uint_as_float(u.z);
        v.w += __uint_as_float(u.w);
      }
      *(float4*)outp((4 * e) / NW, (4 * e) % NW) = v;
    }
    __syncthreads();
  }

  // ---- epilogues, one thread per (row, output) with 32 consecutive threads on one tile-row
  if constexpr (OP == GOP_PLAIN) {
    const int n_tr = a.n_tr[0];
    const int tr0 = group * RT;
    constexpr int NB = NW / 16;               // 16-row blocks per row of X
    const int blk0 = tr0 * 2 + rb;            // the first one's index along N
    if (a.argmax_keys != nullptr) {
      for (int e = tid; e < MB * NB; e += NT) skey[e] = 0ull;
      __syncthreads();
    }
    for (int e0 = 0; e0 < MB * NW; e0 += NT) {   // MB * NW is a multiple of NT
      const int e = e0 + tid;
      const int m = e / NW, n = e % NW;
      const int gm = mblk * MB + m;
      const bool live = gm < a.m_rows;
      const int64_t gn = (int64_t)blk0 * 16 + n;
      float v = 0.f;
      if (live) {
        v = *outp(m, n);
        if constexpr (PF_RES) v += ep_res[e0 / NT];
        else if (a.residual != nullptr) v += a.residual[gm * a.y_stride + gn];
        if (a.y != nullptr) a.y[gm * a.y_stride + gn] = v;
        if (a.argmax_keys != nullptr) atomicMax(&skey[m * NB + n / 16], argmax_key(v, (uint32_t)gn));
      }
      if (a.ssq_out != nullptr) {   // per 16-row block
        const float sq16 = group16_sum(v * v);
        if (live && (n & 15) == 0) a.ssq_out[(int64_t)gm * n_tr * 2 + blk0 + n / 16] = sq16;
      }
    }
    if (a.argmax_keys != nullptr) {
      __syncthreads();
      for (int e = tid; e < MB * NB; e += NT) {
        const int gm = mblk * MB + e / NB;
        if (gm < a.m_rows) a.argmax_keys[(int64_t)gm * n_tr * 2 + blk0 + e % NB] = skey[e];
      }
    }
  } else if constexpr (OP == GOP_GATEUP) {
    const int64_t N = (int64_t)a.n_tr[0] * 32;
    for (int e = tid; e < MB * TW; e += NT) {   // gate in columns [0, TW), up in [TW, 2 TW)
      const int m = e / TW, j = e % TW;
      const int gm = mblk * MB + m;
      if (gm >= a.m_rows) continue;
      const int64_t n = (int64_t)group * 32 + rb * 16 + j;
      const float gr = *outp(m, j), ur = *outp(m, TW + j);
      const float h = swiglu(round_bf16_op(gr), round_bf16_op(ur));
      a.h_out[gm * a.h_stride + n] = f32_to_bf16(h);
      if (a.raw_out != nullptr) {
        a.raw_out[gm * 2 * N + n] = gr;
        a.raw_out[gm * 2 * N + N + n] = ur;
      }
    }
  } else {   // QKV: one head of q, k or v (64 dims), RoPE pairs dim d with d + 32
    int seg_off = 0;
    if (seg == 1) seg_off = a.n_q_heads * 64;
    else if (seg == 2) seg_off = (a.n_q_heads + a.n_kv_heads) * 64;
    const int64_t Wd = (int64_t)(a.n_q_heads + 2 * a.n_kv_heads) * 64;
    // a head's dims d and d + 32 are rows d of its two tile-rows (RB: d in this block's 16)
    for (int e = tid; e < MB * TW; e += NT) {
      const int m = e / TW, d = rb * 16 + e % TW;
      const int gm = mblk * MB + m;
      if (gm >= a.m_rows) continue;
      const float r0 = *outp(m, e % TW), r1 = *outp(m, TW + e % TW);
      if (a.raw_out != nullptr) {
        a.raw_out[gm * Wd + seg_off + hg * 64 + d] = r0;
        a.raw_out[gm * Wd + seg_off + hg * 64 + 32 + d] = r1;
      }
      const float x0 = bf16_to_f32(f32_to_bf16(r0));
      const float x1 = bf16_to_f32(f32_to_bf16(r1));
      const int it = (e - tid) / NT;
      const int p = PF_POS ? ep_pos[PF_POS ? it : 0] : a.pos[gm];   // gm < m_rows here
      if (p < 0 || p >= a.max_pos) continue;
      if (seg == 2) {
        uint16_t* dst = a.v_cache + gm * a.kv_b_stride + hg * a.kv_h_stride + (int64_t)p * 64;
        dst[d] = f32_to_bf16(x0);
        dst[32 + d] = f32_to_bf16(x1);
      } else {
        const float cs = PF_POS ? ep_cs[PF_POS ? it : 0] : a.rope_tab[(int64_t)p * 64 + d];
        const float sn = PF_POS ? ep_sn[PF_POS ? it : 0] : a.rope_tab[(int64_t)p * 64 + 32 + d];
        const float y0 = fmaf(x0, cs, -(x1 * sn));
        const float y1 = fmaf(x1, cs, x0 * sn);
        uint16_t* dst = seg == 0
                            ? a.q_out + gm * (int64_t)a.n_q_heads * 64 + hg * 64
                            : a.k_cache + gm * a.kv_b_stride + hg * a.kv_h_stride + (int64_t)p * 64;
        dst[d] = f32_to_bf16(y0);
        dst[32 + d] = f32_to_bf16(y1);
      }
    }
  }
}

// RMSNorm of the input rows into bf16, once per launch, before a contraction that needs it:
// xn[m][k] = bf16((h[m][k] * r_m) * w[k]), r_m = 1/sqrt(sum(ssq[m]) / K + eps) with the K/16
// sums of squares added in the order every GEMV prologue uses (ssq_lane_sum, then
// wave_sum), so all kernel families see the same input. granite_rmsnorm.h:45-80. One
// workgroup per row; K % 256 == 0, K <= 8192.
__global__ __launch_bounds__(256) void xnorm_kernel(const float* __restrict__ h, int64_t h_stride,
                                                    const float* __restrict__ ssq,
                                                    const uint16_t* __restrict__ w, float eps,
                                                    int K, uint16_t* __restrict__ xn,
                                                    int64_t xn_stride) {
  constexpr int kMaxChunks = 4;   // 8-entry chunks per thread: K <= 8192
  const int m = blockIdx.x, tid = threadIdx.x, l = tid & 63;
  const int n_ss = K / kSsqRows, n_ch = K / 8;
  const float* hr = h + (int64_t)m * h_stride;
  // the row and the weights are requested before the sums of squares are added up, so the
  // kernel waits on memory once
  float4 a0[kMaxChunks], a1[kMaxChunks];
  uint4 wv[kMaxChunks];
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const int e = tid + 256 * i;
    if (e < n_ch) {
      a0[i] = *(const float4*)(hr + 8 * e);
      a1[i] = *(const float4*)(hr + 8 * e + 4);
      wv[i] = *(const uint4*)(w + 8 * e);
    }
  }
  const float* srow = ssq + (int64_t)m * n_ss;
  float4 sq[2];   // n_ss <= 512
  ssq_load<2>(srow, l, n_ss, sq);
  const float inv = rms_inv(wave_sum(ssq_lane_sum<2>(sq, l, n_ss)), K, eps);
  uint16_t* xr = xn + (int64_t)m * xn_stride;
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const int e = tid + 256 * i;
    if (e < n_ch) {
      uint4 o;
      o.x = pack_bf16x2((a0[i].x * inv) * bf16lo(wv[i].x), (a0[i].y * inv) * bf16hi(wv[i].x));
      o.y = pack_bf16x2((a0[i].z * inv) * bf16lo(wv[i].y), (a0[i].w * inv) * bf16hi(wv[i].y));
      o.z = pack_bf16x2((a1[i].x * inv) * bf16lo(wv[i].z), (a1[i].y * inv) * bf16hi(wv[i].z));
      o.w = pack_bf16x2((a1[i].z * inv) * bf16lo(wv[i].w), (a1[i].w * inv) * bf16hi(wv[i].w));
      *(uint4*)(xr + 8 * e) = o;
    }
  }
}

// ---------------------------------------------------------------- host side

struct GemmPlan {
  int rt, mt, wk, nwv, ksplit, kpp, mb, m_blocks, groups;
  bool rb;     // one m-tile: a workgroup per 16-row block of each group
  int units;   // workgroups along N (groups, or twice that with rb)
};

// Workgroup shape by row count: up to 16 rows the four waves split K; more rows go to more
// waves and, past 32, two m-tiles per wave. Past 64 rows (prefill) a workgroup takes two
// tile-rows, halving the x traffic (the fused epilogues always pair two tile-rows); q8 keeps
// one so the staging stays under 64 KB of LDS.
// n_units: tile-rows for PLAIN, output groups (of two tile-rows) for GATEUP and QKV.
static GemmPlan plan_gemm(int kind, int op, int n_units, int k_t, int m_rows, const Policy& P) {
  GemmPlan p{};
  p.nwv = 4;
  if (m_rows <= 16) {
    p.mt = 1; p.wk = 4;
  } else if (m_rows <= 32) {
    p.mt = 2; p.wk = 4;
  } else if (m_rows <= 64) {
    p.mt = 2; p.wk = 2;
  } else {
    p.mt = 2; p.wk = 1;
  }
  if (op != GOP_PLAIN) {
    p.rt = 2;
    p.groups = n_units;
  } else {
    p.rt = (m_rows > 64 && kind == Q4NX_KIND_Q4 && n_units % 2 == 0) ? 2 : 1;
    p.groups = n_units / p.rt;
  }
  p.mb = 16 * p.mt * (4 / p.wk);
  p.m_blocks = (m_rows + p.mb - 1) / p.mb;
  const int wgs = p.groups * p.m_blocks;
  // one m-tile on a grid that does not fill the chip by itself: as many waves per workgroup
  // as K-tiles in its part (below), so its K parts follow from that wave count
  const bool deep = p.mt == 1 && wgs < 512;
  const int cap = (p.rt == 1 && kind == Q4NX_KIND_Q4) ? 16 : 10;   // waves (LDS, registers)
  int ks = 1;
  const int forced = P.gemm_ksplit;
  if (forced > 0) {
    ks = forced;
  } else if (deep) {
    // measured at 8 rows (granite-3B decode): one tile-row per workgroup takes the fewest
    // parts whose K-tiles fit its waves (o 2560->2560 unsplit 6.1 us against 6.7 with 3
    // parts, down 8192->2560 in 2 parts 9.8 us); a pair of tile-rows stays whole when the
    // groups cover the chip ([gate, up] 10.2 us; split 2-3 ways 12-17 us) or when twice its
    // groups fit one workgroup per CU, which then runs row-block workgroups ([q, k, v]: whole
    // on 112 row-block workgroups 6.9 us, in 3 parts of 4 K-tiles 8.2 us, 2 parts 7.7), and
    // else takes parts of at most 4 K-tiles
    ks = p.rt == 1 ? (k_t + cap - 1) / cap
                   : (wgs >= 192 || 2 * wgs <= 256 ? 1 : (k_t + 3) / 4);
  } else if (wgs < 192 && k_t >= 4) {
    ks = (240 + wgs - 1) / wgs;
    const int cap = k_t / 2;                 // >= 2 K-tiles per workgroup
    ks = ks < cap ? ks : cap;
  }
  ks = ks > 8 ? 8 : (ks < 1 ? 1 : ks);
  ks = ks > k_t ? k_t : ks;
  p.kpp = (k_t + ks - 1) / ks;
  p.ksplit = (k_t + p.kpp - 1) / p.kpp;      // no empty parts
  // one m-tile: the fewest of 4, 8, 10 or 16 waves that give every wave at most one K-tile
  // of the part (16 only for one q4 tile-row: its LDS slots and registers), so all of a
  // wave's loads are in flight at once. A grid of 512 workgroups or more keeps 4 waves:
  // there the LDS of more waves would cost resident workgroups (the q8 lm_head 100352 x 2560
  // at 8 rows: 64 us with 4 waves, 84 us with 10).
  if (deep) {
    for (int w : {4, 8, 10, 16})
      if (w <= cap && (w >= p.kpp || w == cap)) {
        p.nwv = p.wk = w;
        break;
      }
  }
  // Row-block workgroups when the doubled grid still fits one workgroup per CU (measured at
  // 8 rows: the o-projection 2560->2560, 80 -> 160 workgroups, 6.79 -> 5.97 us and batch-8
  // decode 3736 -> 3790 tok/s; launches that already fill the chip lose, as each group's
  // activation loads, S sums and reduction are then done twice: [gate, up] 9.54 -> 12.47,
  // down 9.68 -> 14.65 us)
  p.rb = p.mt == 1 && 2 * p.groups * p.m_blocks * p.ksplit <= 256;
  p.units = p.groups * (p.rb ? 2 : 1);
  return p;
}

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// fp32 part records of a split-K launch (0 without a split or with too many counters)
static size_t split_part_bytes(const GemmPlan& p) {
  const size_t cnt = (size_t)p.units * p.m_blocks;
  if (p.ksplit <= 1 || cnt > Q4NX_WS_COUNTER_BYTES / 4) return 0;
  return cnt * p.ksplit * p.mb * p.rt * (p.rb ? 16 : 32) * 4;
}

// Workspace layout: arrival counters, the split-K part records, then (for an RMSNorm
// prologue) the normalised bf16 rows.
static size_t gemm_split_bytes(const GemmPlan& p) {
  const size_t part = split_part_bytes(p);
  return part ? Q4NX_WS_COUNTER_BYTES + align256(part) : 0;
}

template <int KIND, int OP, int RT, int MT, int WK, int NWV = 4>
static void gemm_launch_t(const GemmArgs& a, const GemmPlan& p, hipStream_t st) {
  constexpr int lds = NWV * RT * GemmFmt<KIND>::kSlot;
  static_assert(NWV * 16 * MT * RT * 32 * 4 <= lds, "reduction does not fit the staging slots");
  const dim3 grid((unsigned)(p.units * p.ksplit), (unsigned)p.m_blocks);
  if constexpr (MT == 1) {
    if (p.rb) {
      constexpr int lds_rb = NWV * RT * GemmFmt<KIND>::kSlotRB;
      static_assert(NWV * 16 * RT * 16 * 4 <= lds_rb, "reduction does not fit the staging slots");
      hipLaunchKernelGGL((gemm_kernel<KIND, OP, RT, MT, WK, NWV, true>), grid, dim3(64 * NWV),
                         lds_rb, st, a);
      return;
    }
  }
  hipLaunchKernelGGL((gemm_kernel<KIND, OP, RT, MT, WK, NWV>), grid, dim3(64 * NWV), lds, st, a);
}

template <int KIND, int OP>
static void gemm_launch_op(const GemmArgs& a, const GemmPlan& p, hipStream_t st) {
  constexpr int R1 = OP == GOP_PLAIN ? 1 : 2;
  if (p.mt == 1 && p.nwv == 8) gemm_launch_t<KIND, OP, R1, 1, 8, 8>(a, p, st);
  else if (p.mt == 1 && p.nwv == 10) gemm_launch_t<KIND, OP, R1, 1, 10, 10>(a, p, st);
  else if (p.mt == 1 && p.nwv == 16) {
    if constexpr (KIND == 4 && OP == GOP_PLAIN) gemm_launch_t<KIND, OP, 1, 1, 16, 16>(a, p, st);
  } else if (p.mt == 1) gemm_launch_t<KIND, OP, R1, 1, 4>(a, p, st);
  else if (p.wk == 4) gemm_launch_t<KIND, OP, (OP == GOP_PLAIN ? 1 : 2), 2, 4>(a, p, st);
  else if (p.wk == 2) gemm_launch_t<KIND, OP, (OP == GOP_PLAIN ? 1 : 2), 2, 2>(a, p, st);
  else if (OP != GOP_PLAIN || p.rt == 2) gemm_launch_t<KIND, OP, 2, 2, 1>(a, p, st);
  else if constexpr (OP == GOP_PLAIN) gemm_launch_t<KIND, OP, 1, 2, 1>(a, p, st);
}

// Whether `rows` rows of `kind` run on the matrix cores under the policy (mfma_rows: 0 never).
bool mfma_use(int kind, int rows, const Policy& P) {
  const int t = P.mfma_rows[kind == Q4NX_KIND_Q8 ? 1 : 0];
  return t > 0 && rows >= t;
}

size_t mfma_ws_bytes(int kind, int op, int n_units, int k_t, int m_rows, const Policy& P) {
  // room for the split-K records, for the normalised rows of an RMSNorm prologue and, for a
  // plain prompt block, for the prefill kernel's per-group sums of x
  const size_t split = split_part_bytes(plan_gemm(kind, op, n_units, k_t, m_rows, P));
  const size_t pf = op == GOP_PLAIN ? pf_ws_bytes(n_units, k_t, m_rows) : 0;
  return Q4NX_WS_COUNTER_BYTES + align256(split) + align256((size_t)m_rows * k_t * kTileK * 2) +
         pf;
}

bool mfma_norm_fits(int k_t, int m_rows, size_t ws_bytes) {
  return ws_bytes >= Q4NX_WS_COUNTER_BYTES + align256((size_t)m_rows * k_t * kTileK * 2);
}

// Launches the contraction described by `a` (weights, input, epilogue fields filled in);
// sets the split-K fields from the plan and the workspace. With norm_w set, the rows are
// normalised once into xn_out (when given) or the workspace, then contracted as bf16.
int mfma_launch(int kind, int op, GemmArgs& a, int n_units, void* ws, size_t ws_bytes,
                const Policy& P, hipStream_t st, const char* what) {
  Q4NX_REQUIRE(op == GOP_PLAIN || kind == Q4NX_KIND_Q4, Q4NX_ERR_ARG,
               "%s: fused epilogues take q4 tiles", what);
  const int K = a.k_t * kTileK;
  GemmPlan p = plan_gemm(kind, op, n_units, a.k_t, a.m_rows, P);
  size_t split = split_part_bytes(p);
  const size_t xn_b = a.norm_w != nullptr && a.xn_out == nullptr
                          ? align256((size_t)a.m_rows * K * 2) : 0;
  const bool ws_ok = ws != nullptr && Q4NX_ALIGNED(ws, 256);
  if (split && (!ws_ok || ws_bytes < Q4NX_WS_COUNTER_BYTES + align256(split) + xn_b)) {
    split = 0;   // no (or too small a) workspace: whole K per workgroup
    p.ksplit = 1;
    p.kpp = a.k_t;
  }
  if (a.norm_w != nullptr) {
    Q4NX_REQUIRE(a.ssq_in != nullptr, Q4NX_ERR_ARG,
                 "%s: the matrix-core RMSNorm prologue needs the sums of squares ssq_in", what);
    Q4NX_REQUIRE(K / kSsqRows <= 512, Q4NX_ERR_SHAPE, "%s: RMSNorm prologue supports K <= 8192", what);
    uint16_t* xn = a.xn_out;
    int64_t xs = a.x_stride;
    if (xn == nullptr) {
      Q4NX_REQUIRE(ws_ok && ws_bytes >= Q4NX_WS_COUNTER_BYTES + align256(split) + xn_b,
                   Q4NX_ERR_WS, "%s: workspace of %zu bytes needed for the normalised rows",
                   what, (size_t)(Q4NX_WS_COUNTER_BYTES + align256(split) + xn_b));
      xn = (uint16_t*)((uint8_t*)ws + Q4NX_WS_COUNTER_BYTES + align256(split));
      xs = K;
    }
    hipLaunchKernelGGL(xnorm_kernel, dim3(a.m_rows), dim3(256), 0, st, a.hres, a.x_stride,
                       a.ssq_in, a.norm_w, a.eps, K, xn, xs);
    a.x = xn;
    a.x_stride = xs;
  }
  // a prompt block: the prefill kernel, when the workspace holds its per-group sums of x
  // (past the counters, the split records and the normalised rows); else the batched kernel
  const size_t pf_off = Q4NX_WS_COUNTER_BYTES + align256(split) + xn_b;
  if (pf_use(op, a) && ws_ok && ws_bytes >= pf_off + pf_ws_bytes(a.n_tr[0], a.k_t, a.m_rows)) {
    pf_launch(kind, a, (uint8_t*)ws + pf_off, st);
    return check_launch(what);
  }
  // one m-tile reads x through a buffer resource with 32-bit byte offsets
  Q4NX_REQUIRE(p.mt != 1 || (int64_t)a.m_rows * a.x_stride * 2 < ((int64_t)1 << 31),
               Q4NX_ERR_SHAPE, "%s: %d rows of x at a stride of %lld span 2 GiB or more", what,
               a.m_rows, (long long)a.x_stride);
  a.ksplit = p.ksplit;
  a.kpp = p.kpp;
  if (p.ksplit > 1) {
    a.counters = (unsigned*)ws;
    a.part = (float*)((uint8_t*)ws + Q4NX_WS_COUNTER_BYTES);
    a.part_bytes = (uint32_t)split;
  }
  if (op == GOP_PLAIN) {
    if (kind == Q4NX_KIND_Q4) gemm_launch_op<4, GOP_PLAIN>(a, p, st);
    else gemm_launch_op<8, GOP_PLAIN>(a, p, st);
  } else if (op == GOP_GATEUP) {
    gemm_launch_op<4, GOP_GATEUP>(a, p, st);
  } else {
    gemm_launch_op<4, GOP_QKV>(a, p, st);
  }
  return check_launch(what);
}

}  // namespace q4nx

using namespace q4nx;

extern "C" {

size_t q4nx_gemm_ws_bytes(int kind, int n_tile_rows, int k_tiles, int m_rows,
                          const q4nx_policy* policy) {
  Policy P;
  if ((kind != Q4NX_KIND_Q4 && kind != Q4NX_KIND_Q8) || n_tile_rows < 1 || k_tiles < 1 ||
      m_rows < 1 || !resolve_policy_quiet(policy, &P))
    return 0;
  const size_t split = gemm_split_bytes(plan_gemm(kind, GOP_PLAIN, n_tile_rows, k_tiles, m_rows, P));
  const size_t pf = pf_ws_bytes(n_tile_rows, k_tiles, m_rows);
  // the prefill kernel's sums sit past the counters and the split records
  return pf ? (split ? split : Q4NX_WS_COUNTER_BYTES) + pf : split;
}

int q4nx_gemm(int kind, const uint8_t* w, int n_tile_rows, int k_tiles, const uint16_t* x,
              int64_t x_stride, int m_rows, float* y, int64_t y_stride, const float* residual,
              void* ws, size_t ws_bytes, const q4nx_policy* policy, void* stream) {
  const char* what = "q4nx_gemm";
  Policy P;
  if (int rc = resolve_policy(policy, &P, what)) return rc;
  Q4NX_REQUIRE(kind == Q4NX_KIND_Q4 || kind == Q4NX_KIND_Q8, Q4NX_ERR_ARG,
               "%s: kind must be Q4NX_KIND_Q4 or Q4NX_KIND_Q8, got %d", what, kind);
  Q4NX_REQUIRE(w != nullptr && Q4NX_ALIGNED(w, 16), Q4NX_ERR_ARG,
               "%s: weights must be a non-null 16-byte aligned device pointer", what);
  Q4NX_REQUIRE(n_tile_rows > 0 && k_tiles > 0, Q4NX_ERR_SHAPE,
               "%s: n_tile_rows=%d k_tiles=%d must be positive (N %% 32 == 0, K %% 256 == 0)",
               what, n_tile_rows, k_tiles);
  Q4NX_REQUIRE(m_rows >= 1, Q4NX_ERR_SHAPE, "%s: m_rows=%d must be positive", what, m_rows);
  Q4NX_REQUIRE(x != nullptr && Q4NX_ALIGNED(x, 16), Q4NX_ERR_ARG,
               "%s: x must be a non-null 16-byte aligned device pointer", what);
  Q4NX_REQUIRE(x_stride >= (int64_t)k_tiles * 256 && x_stride % 8 == 0, Q4NX_ERR_SHAPE,
               "%s: x_stride=%lld must be a multiple of 8 and >= K=%d", what,
               (long long)x_stride, k_tiles * 256);
  Q4NX_REQUIRE(y != nullptr && Q4NX_ALIGNED(y, 16), Q4NX_ERR_ARG,
               "%s: y must be a non-null 16-byte aligned device pointer", what);
  Q4NX_REQUIRE(y_stride >= (int64_t)n_tile_rows * 32 && y_stride % 4 == 0, Q4NX_ERR_SHAPE,
               "%s: y_stride=%lld must be a multiple of 4 and >= N=%d", what,
               (long long)y_stride, n_tile_rows * 32);
  Q4NX_REQUIRE(residual == nullptr || Q4NX_ALIGNED(residual, 16), Q4NX_ERR_ARG,
               "%s: residual must be 16-byte aligned", what);
  GemmArgs a{};
  a.w[0] = w;
  a.n_tr[0] = n_tile_rows;
  a.x = x;
  a.y = y;
  a.residual = residual;
  a.x_stride = x_stride;
  a.y_stride = y_stride;
  a.m_rows = m_rows;
  a.k_t = k_tiles;
  return mfma_launch(kind, GOP_PLAIN, a, n_tile_rows, ws, ws_bytes, P, (hipStream_t)stream, what);
}

}  // extern "C"
