// Prefill contraction on the matrix cores (gfx950): Y[m][n] = R[m][n] + sum_k W[n][k] X[m][k]
// for many rows of X (a prompt block), W read in the q4nx tile layout.
//
// Replaces, for prompt blocks, the torch fallback that reference/npu.py:118-122, 138-140 takes
// for more than one row, as the batched kernel (gemm.hip) does for smaller row counts.
//
// Why a second kernel. The batched kernel multiplies raw codes and applies each 32-K group's
// scale afterwards on the VALU: two fp32 FMAs per output and group against one MFMA per
// 16x16x32 block, which holds it near 15 % of the bf16 peak however many rows there are.
// Here the scale and the minimum go into the weight operands instead, exactly:
//   q4: c d has at most 12 significant bits (4 x 8), so it is the sum of two bf16 values,
//       hi = bf16(c d) and lo = c d - hi, and m is a bf16 value already: three MFMAs per
//       16x16x32 block (hi, lo, and m at every k of the group, all against the same x
//       operand) give sum_k (c_k d + m) x_k with exact products and fp32 accumulation, each
//       group's terms meeting in one accumulator as in the batched kernel's per-group
//       identity (granite_gemv.h:19-29).
//   q8: w = q s has at most 15 significant bits (8 x 8, the sign apart): hi + lo, two MFMAs.
// The operands of a tile-row are built once per 32-K step, for the next step while this
// step's MFMAs run, and used for all 128 rows of the workgroup's block. One-hot x reproduces
// the float32 dequantised column bit for bit: hi + lo is exactly c d, and m joins it in one
// rounding, as fp32(c d + m). What bounds it is the VALU: building the operands takes about
// 150 VALU instructions per wave and 32-K step (4 cycles each for a 64-wide wave) against
// 48 MFMAs (q4), so the matrix cores stay near a third busy and the q4 contraction runs at
// the batched kernel's rate; the q8 lm_head, two MFMAs per block and no minimum, runs near
// twice its rate.
//
// Work decomposition: a workgroup of four waves takes one block of 16*MT rows of X and four
// tile-rows; wave w owns tile-row 4*blockIdx.x + w for the whole K, so nothing is merged
// across waves or workgroups. Each wave stages its tile in its own LDS slot (the transposing
// LDS read needs it there) while the next tile is in flight to registers. The block's x is
// loaded once for the four waves: every thread carries its share of the next four 32-K steps
// in registers and stores one step into a ring of three LDS buffers per step (one barrier per
// step), laid out so that each m-tile's A operand is one conflict-free 16-byte LDS read per
// lane. The outputs leave through LDS as 128-byte row segments.

#include "common.h"
#include "gemm.h"
#include "gemm_fmt.h"

namespace q4nx {

namespace {

constexpr int kPfWaves = 4;
constexpr int kPfRowPad = 32;   // floats per staged output row (the block of four waves fits 64 KB)

// w0, w1 (each exact in at most 16 significant bits) as bf16 pairs with hi + lo == w exactly
__device__ __forceinline__ void split_pair(float w0, float w1, uint32_t& hi, uint32_t& lo) {
  const f32x2_v v = {w0, w1};
  hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_v));
  const f32x2_v r = {w0 - bf16lo(hi), w1 - bf16hi(hi)};
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, bf16x2_v));
}

// eight bf16 values 16 + c of an operand (as q4_operands builds them) -> c d, split
__device__ __forceinline__ void cd_split(const u32x4_t& op, float d, u32x4_t& hi, u32x4_t& lo) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t h, l;
    split_pair((bf16lo(op[i]) - 16.f) * d, (bf16hi(op[i]) - 16.f) * d, h, l);
    hi[i] = h;
    lo[i] = l;
  }
}

// eight int8 codes (LDS-transposed, as in q8_operand) times s, split
__device__ __forceinline__ void q8_scale_split(i32x2_t r, float s, u32x4_t& hi, u32x4_t& lo) {
  const uint32_t w[2] = {(uint32_t)r.x, (uint32_t)r.y};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const float f0 = (float)(int)(int8_t)(w[h] >> (16 * q));
      const float f1 = (float)(int)(int8_t)(w[h] >> (16 * q + 8));
      uint32_t hh, ll;
      split_pair(f0 * s, f1 * s, hh, ll);
      hi[2 * h + q] = hh;
      lo[2 * h + q] = ll;
    }
  }
}

// One 32-K step's weight operands of this lane's two columns: c d (q4) or q s (q8) as
// bf16 hi + lo, and (q4) the group minimum m at every k of the step.
struct PfOps {
  u32x4_t hi[2], lo[2], mb[2];
};

template <int KIND>
__device__ __forceinline__ void pf_ops(const uint8_t* slot, int tr_off, int meta_off, int kb,
                                       PfOps& o) {
  if constexpr (KIND == 4) {
    const i32x2_t cb =
        __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2_t*)(slot + tr_off + kb * 256));
    u32x4_t op[2];
    q4_operands(cb, op[0], op[1]);
    const uint32_t dv = *(const uint32_t*)(slot + kb * 64 + meta_off);
    const uint32_t mv = *(const uint32_t*)(slot + kMetaBytes + kb * 64 + meta_off);
    const float d0 = bf16lo(dv), d1 = bf16hi(dv);
    const uint32_t m0 = (mv & 0xFFFFu) * 0x10001u, m1 = (mv >> 16) * 0x10001u;
    o.mb[0] = u32x4_t{m0, m0, m0, m0};   // the group's minimum at every k
    o.mb[1] = u32x4_t{m1, m1, m1, m1};
    cd_split(op[0], d0, o.hi[0], o.lo[0]);
    cd_split(op[1], d1, o.hi[1], o.lo[1]);
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const i32x2_t cb = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          (lds_i32x2_t*)(slot + tr_off + h * 4096 + kb * 512));
      const float sc = bf16_to_f32(*(const uint16_t*)(slot + kb * 64 + h * 32 + meta_off));
      q8_scale_split(cb, sc, o.hi[h], o.lo[h]);
    }
  }
}

template <int KIND, int MT>
__global__ __launch_bounds__(256) void gemm_pf_kernel(GemmArgs a) {
  constexpr int SLOT = GemmFmt<KIND>::kSlot;
  constexpr int NLD = GemmFmt<KIND>::kLoads;
  constexpr int TB = GemmFmt<KIND>::kTile;
  constexpr int MB = 16 * MT;
  constexpr int UPT = MB * 4 / 256;        // 16-byte x units per thread and 32-K step
  constexpr int XB = MB * 4 * 16;          // bytes of one staged step of x
  constexpr int XD = 4;                    // steps of x in flight in registers (divides the 8 steps of a tile)
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

  const int tid = threadIdx.x, l = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_tr = a.n_tr[0];
  const int tr = blockIdx.x * kPfWaves + wave;
  const bool live = tr < n_tr;                    // a wave past the last tile-row only helps
  const int trc = live ? tr : n_tr - 1;
  const int m0 = blockIdx.y * MB;
  const uint8_t* wr = a.w[0] + (size_t)trc * a.k_t * TB;
  uint8_t* xbuf = lds;                            // three staged steps of x
  uint8_t* slot = lds + 3 * XB + wave * SLOT;     // this wave's weight tile
  const int c = l & 15, s = l >> 4;
  const int n_steps = a.k_t * 8;

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
  auto x_load = [&](u32x4_t (&g)[UPT], int step) {
    const int st = step < n_steps ? step : n_steps - 1;   // past the end: a re-read
    const int k = (st >> 3) * 256 + (st & 7) * 32;
#pragma unroll
    for (int j = 0; j < UPT; ++j) g[j] = *(const u32x4_t*)(xsrc[j] + k);
  };
  auto x_store = [&](const u32x4_t (&g)[UPT], int buf) {
#pragma unroll
    for (int j = 0; j < UPT; ++j) *(u32x4_t*)(xbuf + buf * XB + 16 * (tid + 256 * j)) = g[j];
  };
  auto x_read = [&](u32x4_t (&xa)[MT], int buf) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xa[mt] = *(const u32x4_t*)(xbuf + buf * XB + 16 * (64 * mt + l));
  };

  f32x4_t acc[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt][0] = acc[mt][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // Pipeline: during step s the MFMAs of s run while this wave builds the weight operands of
  // s + 1 from its tile slot, reads the x operands of s + 1 from LDS (staged during s - 1),
  // stages x of s + 2 and loads x of s + 2 + XD; one barrier ends each step.
  u32x4_t pf[NLD];
  u32x4_t gx[XD][UPT];   // x of steps s + 2 .. s + 1 + XD at step s, step t in gx[t % XD]
  {
    u32x4_t g0[UPT], g1[UPT];
    x_load(g0, 0);
    x_load(g1, 1);
#pragma unroll
    for (int t = 2; t < 2 + XD; ++t) x_load(gx[t % XD], t);
#pragma unroll
    for (int i = 0; i < NLD; ++i) pf[i] = *(const u32x4_t*)(wr + ld_off[i]);
#pragma unroll
    for (int i = 0; i < NLD; ++i) *(u32x4_t*)(slot + 16 * (64 * i + l)) = pf[i];
    {
      const size_t off = (size_t)(a.k_t > 1 ? 1 : 0) * TB;
#pragma unroll
      for (int i = 0; i < NLD; ++i) pf[i] = *(const u32x4_t*)(wr + off + ld_off[i]);
    }
    x_store(g0, 0);
    x_store(g1, 1);
  }
  __syncthreads();
  u32x4_t xa[2][MT];
  PfOps ops[2];
  x_read(xa[0], 0);
  pf_ops<KIND>(slot, tr_off, meta_off, 0, ops[0]);

  for (int kt = 0; kt < a.k_t; ++kt) {
#pragma unroll
    for (int kb = 0; kb < 8; ++kb) {
      const int step = kt * 8 + kb;
      const int cur = kb & 1, nxt = cur ^ 1;
      // ---- the MFMAs of this step
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          acc[mt][h] = mfma_bf16(xa[cur][mt], ops[cur].hi[h], acc[mt][h]);
          acc[mt][h] = mfma_bf16(xa[cur][mt], ops[cur].lo[h], acc[mt][h]);
          if constexpr (KIND == 4) acc[mt][h] = mfma_bf16(xa[cur][mt], ops[cur].mb[h], acc[mt][h]);
        }
      // ---- x of step + 2 into LDS, x of step + 2 + XD into the freed registers
      x_store(gx[(kb + 2) % XD], (step + 2) % 3);
      x_load(gx[(kb + 2) % XD], step + 2 + XD);
      // ---- the next step's operands (the next tile into the slot first at a tile boundary;
      // past the last step they are built from re-read data and not used)
      if (kb == 7) {
#pragma unroll
        for (int i = 0; i < NLD; ++i) *(u32x4_t*)(slot + 16 * (64 * i + l)) = pf[i];
        const size_t off = (size_t)(kt + 2 < a.k_t ? kt + 2 : a.k_t - 1) * TB;
#pragma unroll
        for (int i = 0; i < NLD; ++i) pf[i] = *(const u32x4_t*)(wr + off + ld_off[i]);
      }
      pf_ops<KIND>(slot, tr_off, meta_off, (kb + 1) & 7, ops[nxt]);
      x_read(xa[nxt], (step + 1) % 3);
      // step + 2's x is in LDS for everyone once all have passed here; the buffer it took was
      // last read during step - 1, before every thread passed the previous barrier
      __syncthreads();
    }
  }

  // ---- outputs: every wave has finished with LDS (the last barrier), then each writes its
  // [MB][32] block (row m = 16 mt + 4 s + e, column of operand h at lane c) and reads it
  // back as 128-byte row segments
  float* blk = (float*)lds + wave * MB * kPfRowPad;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int col = KIND == 4 ? (c >> 3) * 16 + 2 * (c & 7) + h : h * 16 + c;
#pragma unroll
      for (int e = 0; e < 4; ++e) blk[(16 * mt + 4 * s + e) * kPfRowPad + col] = acc[mt][h][e];
    }
  if (!live) return;
  const int q = l & 7, r0 = l >> 3;   // 8 lanes per 32-float row, 8 rows per pass
#pragma unroll
  for (int p = 0; p < MB / 8; ++p) {
    const int r = 8 * p + r0, m = m0 + r;
    if (m < a.m_rows) {
      float4 v = *(const float4*)(blk + r * kPfRowPad + 4 * q);
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

template <int KIND, int MT>
void pf_go(const GemmArgs& a, hipStream_t st) {
  constexpr int lds_slots = 3 * 16 * MT * 4 * 16 + kPfWaves * GemmFmt<KIND>::kSlot;
  constexpr int lds_out = kPfWaves * 16 * MT * kPfRowPad * 4;
  constexpr int lds = lds_slots > lds_out ? lds_slots : lds_out;
  const dim3 grid((unsigned)((a.n_tr[0] + kPfWaves - 1) / kPfWaves),
                  (unsigned)((a.m_rows + 16 * MT - 1) / (16 * MT)));
  hipLaunchKernelGGL((gemm_pf_kernel<KIND, MT>), grid, dim3(256), lds, st, a);
}

}  // namespace

// Workgroups of the prefill kernel for a launch (four tile-rows x 128 rows each).
static int pf_workgroups(const GemmArgs& a) {
  return ((a.n_tr[0] + kPfWaves - 1) / kPfWaves) * ((a.m_rows + 127) / 128);
}

// A plain contraction goes to the prefill kernel from kPrefillRows rows when it has at least
// two workgroups per CU, with no sums-of-squares or argmax epilogue (those stay on the
// batched kernel). Measured at 2048 rows: q4 2560->8192 (1024 workgroups) 373 against 366
// TFLOP/s on the batched kernel, q8 lm_head 248320x1024 at 512 rows 398 against 220; q4
// 8192->2560 (320 workgroups) 270 against 364, so smaller launches keep the batched kernel.
bool pf_use(int op, const GemmArgs& a) {
  return op == GOP_PLAIN && a.m_rows >= kPrefillRows && a.ssq_out == nullptr &&
         a.argmax_keys == nullptr && pf_workgroups(a) >= 512;
}

void pf_launch(int kind, const GemmArgs& a, hipStream_t st) {
  if (kind == Q4NX_KIND_Q4) pf_go<4, 8>(a, st);
  else pf_go<8, 8>(a, st);
}

}  // namespace q4nx
