/* q4nx_hip.h -- C ABI of libq4nx_hip.so, the MI355X (gfx950) decode hot path for
 * q4nx-tiled weights: dequantisation, the q4 (W4A16 Q4_1) and q8 (W8A16) GEMVs, RMSNorm,
 * RoPE, SwiGLU, the fused [q,k,v,RoPE] and [gate,up,SwiGLU] groups, GQA flash-decode
 * attention, and the small decode-step helpers (embedding row, argmax).
 *
 * Conventions for every entry point:
 *   - Device pointers are caller-owned and must stay valid until the stream work ends.
 *   - Every call is asynchronous on `stream` (a hipStream_t; NULL = the null stream).
 *   - bf16 values are passed as uint16_t bit patterns.
 *   - Return 0 (Q4NX_OK) on success, a negative Q4NX_ERR_* on an argument error or launch
 *     failure; q4nx_last_error() gives the message. Nothing throws across the ABI.
 *   - Tiled weights are raw q4nx bytes, [n_tile_rows][k_tiles][tile], exactly as stored
 *     in a .q4nx file (tools/q4nx.py:1-18): q4 tiles are 5120 B, q8 tiles 8704 B.
 *   - Workspaces (`ws`) are laid out as Q4NX_WS_COUNTER_BYTES of arrival counters
 *     followed by fp32 partial sums. They must be zero-filled once before their first
 *     use; every call leaves the counters at zero again, whatever the shapes of the
 *     calls that share the workspace. Calls that share a workspace must be ordered on
 *     one stream. Any entry point's ws_bytes query includes the counter region.
 *   - Entry points that choose between kernel families or work splits take a
 *     `const q4nx_policy *policy` (NULL = the defaults of q4nx_policy_init). The library
 *     keeps no mutable state of its own: calls with different policies, from any thread,
 *     never affect each other. A ws_bytes query must be given the policy of the call.
 *   - Sums of squares (ssq_in / ssq_out) and argmax keys are kept per 16-row block:
 *     [batch][N/16] for an output of N rows, [batch][K/16] for an input of K entries.
 *
 * The reference interface each entry point replaces is cited beside it (paths relative
 * to the reference repository).
 */
#ifndef Q4NX_HIP_H
#define Q4NX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q4NX_ABI_VERSION 2

#define Q4NX_OK 0
#define Q4NX_ERR_ARG (-1)     /* null or misaligned pointer, bad enum            */
#define Q4NX_ERR_SHAPE (-2)   /* K % 256, N % 32, Hq % Hkv, head_dim, batch ...  */
#define Q4NX_ERR_WS (-3)      /* workspace missing or too small                  */
#define Q4NX_ERR_LAUNCH (-4)  /* the HIP runtime refused the launch              */

#define Q4NX_KIND_Q4 4
#define Q4NX_KIND_Q8 8
#define Q4NX_KIND_BF16 16   /* a plain bf16 matrix (embedding tables) */

#define Q4NX_MAX_BATCH 8

/* Size of the counter region at the start of every workspace (16384 counters). */
#define Q4NX_WS_COUNTER_BYTES 65536
/* q4nx_gqa_decode_static's library-owned scratch per GPU: the counter region and 8 MiB
 * of split records. */
#define Q4NX_STATIC_SCRATCH_BYTES (Q4NX_WS_COUNTER_BYTES + (8 << 20))

int q4nx_abi_version(void);
/* Message of the last error on this thread ("" if none). */
const char *q4nx_last_error(void);

/* ---------------------------------------------------------------- launch policy
 * Which kernel family takes a call and how its work is split, passed per call. No reference
 * counterpart: each NPU design fixed its mapping when it was built (export_design.py). */
typedef struct q4nx_policy {
  int mfma_rows_q4;   /* q4 GEMV / fused groups: rows from which they run on the matrix
                         cores (the q4nx_gemm kernels); 0 = never. Default 2. */
  int mfma_rows_q8;   /* the same for q8. Default 2. */
  int rowblock;       /* 1 (default): one-row calls on the row-block kernels (one
                         workgroup per 16 output rows; q4, and q8 for a plain GEMV);
                         0: on the general VALU GEMV */
  int gemv_ksplit;    /* general VALU GEMV: workgroups per output group along K, 1..8;
                         0 = automatic (default) */
  int gemv_tiles_per_wave; /* K-tiles per wave, 1, 2 or 4, of the general VALU GEMV and of the
                         row-block kernels (where it must leave at most 16 waves per
                         workgroup, else Q4NX_ERR_ARG); 0 = automatic (default) */
  int gemm_ksplit;    /* matrix-core contraction: workgroups along K, 1..8; 0 = automatic */
  int attn_mfma;      /* 1 (default): attention on the matrix cores; 0: on the VALU kernel */
} q4nx_policy;
/* Fills *p with the defaults. */
void q4nx_policy_init(q4nx_policy *p);

/* ---------------------------------------------------------------- dequantisation
 * Replaces tools/q4nx.py:97-111 (dequant_q4 / dequant_q8, bf16 out) and :127-149
 * (_q4_tiles / _q8_tiles / _untile, fp32 out), and the on-core unpack
 * designs/q4nx_unpack/q4nx_unpack.cc:40-92. Bit-exact: w = fp32(code*d + m) (q4) or
 * code*s (q8), then RNE to bf16 when out_f32 == 0.
 *   untile == 0: out is [n_tiles][8192] in weight-index order (i = rb*4096 + k*16 + r)
 *   untile == 1: out is the [N][K] matrix, row = tr*32 + rb*16 + r, col = kt*256 + k */
int q4nx_dequant_q4(const uint8_t *tiles, void *out, int n_tile_rows, int k_tiles,
                    int out_f32, int untile, void *stream);
int q4nx_dequant_q8(const uint8_t *tiles, void *out, int n_tile_rows, int k_tiles,
                    int out_f32, int untile, void *stream);

/* ---------------------------------------------------------------- GEMV
 * y[b][n] = residual[b][n] + sum_k W[n][k] * x[b][k], fp32 accumulate, b < batch <= 8.
 * Replaces the per-core kernels designs/granite_gemv/granite_gemv.h:109-300
 * (granite_gemv_p{P}b{B}_k{N}(tiles, x, y)) and designs/lm_head/lm_head.h:53-113
 * (lmhead_q8_k{N}(tiles, x, y)), with the whole tensor in one launch.
 *   w: tile bytes, 16-byte aligned; x: bf16 [batch][x_stride]; y: fp32 [batch][y_stride];
 *   residual: fp32 [batch][y_stride] or NULL. K = 256*k_tiles, N = 32*n_tile_rows.
 *   ws: workspace of at least q4nx_gemv_ws_bytes(...) bytes (may be NULL when that is 0). */
size_t q4nx_gemv_ws_bytes(int kind, int n_tile_rows, int k_tiles, int batch,
                          const q4nx_policy *policy);
int q4nx_gemv_q4(const uint8_t *w, const uint16_t *x, float *y, int n_tile_rows,
                 int k_tiles, int batch, int64_t x_stride, int64_t y_stride,
                 const float *residual, void *ws, size_t ws_bytes,
                 const q4nx_policy *policy, void *stream);
int q4nx_gemv_q8(const uint8_t *w, const uint16_t *x, float *y, int n_tile_rows,
                 int k_tiles, int batch, int64_t x_stride, int64_t y_stride,
                 const float *residual, void *ws, size_t ws_bytes,
                 const q4nx_policy *policy, void *stream);

/* General form of the two above: y = residual + W * f(x), where f is the identity on a
 * bf16 x, or, when norm_w != NULL, RMSNorm(x; norm_w, eps) of an fp32 x rounded to bf16
 * in the prologue (granite_rmsnorm.h:45-80 fused into the GEMV). kind is Q4NX_KIND_Q4 or
 * Q4NX_KIND_Q8. argmax_keys (optional, uint64 [batch][N/16]) receives for every 16-row
 * block an order-preserving key of (max y over its rows, first such row);
 * q4nx_decode_advance reduces them. y may be NULL when only the keys are wanted.
 * ssq_out (optional, fp32 [batch][N/16]): sum of y^2 over each 16-row block.
 * ssq_in (optional, with norm_w; fp32 [batch][K/16], K <= 8192, 16-byte aligned): the same partial sums
 * for x, as the producer of x wrote them; the prologue then adds these (in a fixed order)
 * instead of reducing x across the workgroup (the one-row kernels need them with norm_w).
 * ws as for the GEMVs above (K split when the launch has few tile-rows). No reference
 * counterpart for the fusions: the reference runs the final norm and argmax on the host
 * (chat.py:74-78 through transformers' generate). */
int q4nx_gemv_ex(int kind, const uint8_t *w, int n_tile_rows, int k_tiles, const void *x,
                 int64_t x_stride, const uint16_t *norm_w, float eps, const float *ssq_in,
                 int batch, float *y, int64_t y_stride, const float *residual, float *ssq_out,
                 uint64_t *argmax_keys, void *ws, size_t ws_bytes,
                 const q4nx_policy *policy, void *stream);

/* The o-projection of a batch-1 decode step fed straight from attention's split records:
 * y = residual + W * bf16(merge(att_rec)), where merge(att_rec) is the attention output
 * q4nx_gqa_decode would have written for the same records (same operations, same order:
 * the results equal q4nx_gqa_decode followed by q4nx_gemv_ex bit for bit). W: q4 tiles
 * [n_tile_rows][n_q_heads/4]; K = 64 * n_q_heads <= 2560; att_rec: the records of
 * q4nx_gqa_decode_records at batch 1 (ws + Q4NX_WS_COUNTER_BYTES), n_split <= 18, which are
 * only read; y, residual, ssq_out as in q4nx_gemv_ex. One workgroup per 16 output rows, no K
 * split, no workspace. Fuses granite_attn_finish (granite_attention.h:193-212, 232-237) into the
 * o-projection GEMV of designs/granite_gemv/granite_gemv.h:79-91. */
int q4nx_gemv_attn_q4(const uint8_t *w, int n_tile_rows, const float *att_rec, int n_split,
                      int n_q_heads, int n_kv_heads, float *y, const float *residual,
                      float *ssq_out, void *stream);


/* ---------------------------------------------------------------- batched contraction (MFMA)
 * y[m][n] = residual[m][n] + sum_k W[n][k] * x[m][k] for m < m_rows, any m_rows >= 1, on the
 * matrix cores; fp32 out. Replaces the torch fallback reference/npu.py:118-122, 138-140
 * takes for prefill (more than one row), and carries the batched design of
 * designs/granite_gemv/granite_gemv.h:79-91 (tokens share one weight pass) past 8 rows.
 *   w: q4 or q8 tiles (kind), 16-byte aligned; x: bf16 [m_rows][x_stride], x_stride % 8 == 0;
 *   y, residual: fp32 [m_rows][y_stride], y_stride % 4 == 0, 16-byte aligned.
 *   ws: workspace of q4nx_gemm_ws_bytes(...) bytes, zeroed once (K is split across
 *   workgroups when the launch has few of them; a prompt block that fills the chip keeps
 *   per-group sums of x there for the prefill kernel); NULL, or a workspace smaller than
 *   q4nx_gemm_ws_bytes asks for, runs without either (a prompt block then takes the batched
 *   kernel, whole K per workgroup). */
size_t q4nx_gemm_ws_bytes(int kind, int n_tile_rows, int k_tiles, int m_rows,
                          const q4nx_policy *policy);
int q4nx_gemm(int kind, const uint8_t *w, int n_tile_rows, int k_tiles, const uint16_t *x,
              int64_t x_stride, int m_rows, float *y, int64_t y_stride, const float *residual,
              void *ws, size_t ws_bytes, const q4nx_policy *policy, void *stream);
/* The GEMV and fused entry points hand calls of policy->mfma_rows_q4 / _q8 rows or more to
 * these matrix-core kernels (fused prologue and epilogues included); there `batch` may
 * exceed Q4NX_MAX_BATCH, and an RMSNorm prologue needs ssq_in (launches without it stay on
 * the VALU kernel, batch <= 8). */

/* ---------------------------------------------------------------- elementwise
 * RMSNorm y = x * rsqrt(mean(x^2) + eps) * w, fp32 math, bf16 out (+ optional fp32
 * pre-rounding copy). Replaces designs/granite_gemv/granite_rmsnorm.h:82-87
 * (granite_rms_norm(x, w, y, cols)). x is bf16 (x_f32 == 0) or fp32 (x_f32 == 1),
 * [batch][cols]; cols % 2 == 0. */
int q4nx_rmsnorm(const void *x, int x_f32, const uint16_t *w, uint16_t *y,
                 float *y_f32, int cols, int batch, float eps, void *stream);

/* Half-split RoPE (rotate_half) on [batch][n_heads][head_dim] bf16 with the fp32
 * cos/sin table tab[pos][2][head_dim/2] built by q4nx_rope_table_host. Replaces
 * designs/granite_gemv/granite_elementwise.h:111-114 (granite_rope(x, cs, y, n_heads));
 * the per-position cos/sin come from the table instead of the caller. */
int q4nx_rope(const uint16_t *x, uint16_t *y, float *y_f32, int n_heads, int head_dim,
              int batch, const int32_t *positions, const float *tab, int max_pos,
              void *stream);

/* Host-side (no GPU): fp32 cos/sin table of pos * theta^(-2i/head_dim), computed in
 * float64 and rounded once, layout [max_pos][2][head_dim/2]. */
int q4nx_rope_table_host(float *tab, int max_pos, int head_dim, double theta);

/* y = bf16(silu(g) * u). g, u bf16 (in_f32 == 0) or fp32 GEMV accumulators narrowed to
 * bf16 first (in_f32 == 1). Replaces designs/granite_gemv/granite_elementwise.h:115-118
 * (granite_swiglu) and granite_swiglu_f32.h:132-137 (granite_swiglu_f32). */
int q4nx_swiglu(const void *g, const void *u, int in_f32, uint16_t *y, float *y_f32,
                int n, int batch, void *stream);

/* ---------------------------------------------------------------- fused groups
 * [q, k, v, RoPE] in one launch: q|k|v GEMVs over the same input, the q/k accumulators
 * narrowed to bf16 and rotated, v narrowed; q goes to q_out [batch][n_q*64], k and v
 * are written into the caches at positions[b]; a row whose position lies outside
 * [0, max_pos) writes neither its q nor the caches (raw_out still receives its GEMV outputs).
 * Replaces the fused design
 * designs/granite_gemv/granite_qkv.py:50-128 with its epilogue granite_qkv_rope.h:74-78.
 * Input: bf16 x [batch][x_stride], or, when norm_w != NULL, the fp32 residual h
 * [batch][x_stride] normalised in the prologue (RMSNorm with norm_w, eps).
 * Cache layout: k_cache[b][kv_head][l][64] with strides (kv_b_stride, kv_h_stride) in
 * elements; l < max_pos. raw_out (optional): fp32 [batch][(n_q+2*n_kv)*64] GEMV outputs
 * before narrowing. xn_out (optional): bf16 [batch][K] normalised input. ssq_in: as in
 * q4nx_gemv_ex. */
size_t q4nx_qkv_rope_ws_bytes(int n_q_heads, int n_kv_heads, int k_tiles, int batch,
                              const q4nx_policy *policy);
int q4nx_qkv_rope(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, int n_q_heads,
                  int n_kv_heads, int k_tiles, const void *x, int64_t x_stride,
                  const uint16_t *norm_w, float eps, const float *ssq_in, int batch,
                  const int32_t *positions,
                  const float *rope_tab, int max_pos, uint16_t *q_out, uint16_t *k_cache,
                  uint16_t *v_cache, int64_t kv_b_stride, int64_t kv_h_stride,
                  float *raw_out, uint16_t *xn_out, void *ws, size_t ws_bytes,
                  const q4nx_policy *policy, void *stream);

/* [gate, up, SwiGLU] in one launch: h[b][n] = bf16(silu(bf16(gate.x)) * bf16(up.x)).
 * Replaces designs/granite_gemv/granite_mlp.py:48-133 with granite_swiglu_f32.h. Input
 * as q4nx_qkv_rope (bf16 x, or fp32 residual + norm_w). raw_out (optional): fp32
 * [batch][2*N] gate|up accumulators; xn_out (optional) as above. */
size_t q4nx_gate_up_ws_bytes(int n_tile_rows, int k_tiles, int batch,
                             const q4nx_policy *policy);
int q4nx_gate_up_swiglu(const uint8_t *wg, const uint8_t *wu, int n_tile_rows,
                        int k_tiles, const void *x, int64_t x_stride,
                        const uint16_t *norm_w, float eps, const float *ssq_in, int batch,
                        uint16_t *h_out,
                        int64_t h_stride, float *raw_out, uint16_t *xn_out, void *ws,
                        size_t ws_bytes, const q4nx_policy *policy, void *stream);

/* ---------------------------------------------------------------- attention
 * GQA flash-decode: one query token per sequence, out[b][h] = softmax(scale * K q) V
 * over positions [0, lens[b]) of the caches, q head h reading kv head h / (Hq/Hkv); a
 * sequence with lens[b] <= 0 gets zeros, and lens[b] > max_len reads max_len positions.
 * Split-K over the KV length with an exact (m, l, acc) combine. Replaces
 * designs/granite_gemv/granite_attention.h:221-237 (granite_attn_block /
 * granite_attn_finish). head_dim must be 64. q: bf16 [B][Hq][64]; out: bf16 and/or fp32
 * [B][Hq][64]; caches as in q4nx_qkv_rope. n_split = 0 chooses automatically.
 * policy->attn_mfma picks the kernel: the matrix cores (scores and P.V on
 * v_mfma_f32_16x16x32_bf16, P carried as three bf16 terms) or the VALU kernel; both give
 * fp32-accurate results. */
size_t q4nx_gqa_decode_ws_bytes(int batch, int n_q_heads, int n_kv_heads, int max_len,
                                const q4nx_policy *policy);
int q4nx_gqa_decode(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                    uint16_t *out, float *out_f32, int batch, int n_q_heads,
                    int n_kv_heads, int head_dim, const int32_t *lens, int max_len,
                    int64_t kv_b_stride, int64_t kv_h_stride, float scale, int n_split,
                    void *ws, size_t ws_bytes, const q4nx_policy *policy, void *stream);
/* The split count q4nx_gqa_decode chooses for n_split = 0 under `policy`; 0 for an invalid
 * shape or policy. */
int q4nx_gqa_decode_splits(int batch, int n_q_heads, int n_kv_heads, int max_len,
                           const q4nx_policy *policy);
/* q4nx_gqa_decode without a workspace argument: it allocates nothing. No counterpart in the
 * reference; it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The arrival counters and
 * split records live in a library-owned device array of Q4NX_STATIC_SCRATCH_BYTES per GPU
 * (the workspace layout: counters, then records), held until the process ends. The loader
 * zero-fills it and every call leaves the counters at zero. The first call on a device
 * (made with it current, outside graph capture) looks up that device's copy of the array.
 * A call whose records would not fit (Q4NX_WS_COUNTER_BYTES + B*Hkv*n_split*(Hq/Hkv)*68*4
 * bytes, with n_split as chosen for n_split = 0) is refused with Q4NX_ERR_WS before
 * anything is launched. Every call on one GPU shares the array: calls ordered on one
 * stream are safe, calls that overlap on one GPU race. Arguments, results and bits as in
 * q4nx_gqa_decode at the same n_split and policy. */
int q4nx_gqa_decode_static(const uint16_t *q, const uint16_t *k_cache,
                           const uint16_t *v_cache, uint16_t *out, float *out_f32, int batch,
                           int n_q_heads, int n_kv_heads, int head_dim, const int32_t *lens,
                           int max_len, int64_t kv_b_stride, int64_t kv_h_stride, float scale,
                           int n_split, const q4nx_policy *policy, void *stream);
/* The split count to give q4nx_gqa_decode_records when q4nx_gemv_attn_q4 merges the
 * records: q4nx_gqa_decode_splits capped at 12 (every split is a record each o-projection
 * workgroup reads, so the pair runs fastest with fewer, longer splits). */
int q4nx_gqa_decode_records_splits(int batch, int n_q_heads, int n_kv_heads, int max_len,
                                   const q4nx_policy *policy);
/* The first half of q4nx_gqa_decode: every split of every (b, kv head) writes its record
 * (fp32 acc[64], m (log2 domain), l, 2 pad; 68 floats per q head) to the workspace at
 * ws + Q4NX_WS_COUNTER_BYTES, laid out [b][kv head][split][head in group][68], and ends;
 * nothing is merged, no counter is touched and no output is written. The second half is
 * the merge in q4nx_gemv_attn_q4 (batch 1). n_split >= 1 must be given (records for
 * n_split = 1 too). ws: Q4NX_WS_COUNTER_BYTES + B*Hkv*n_split*(Hq/Hkv)*68*4 bytes,
 * 256-byte aligned. Splits granite_attn_block / granite_attn_finish
 * (designs/granite_gemv/granite_attention.h:221-237) the way the reference does: the
 * blocks publish partials, a separate step combines them. */
int q4nx_gqa_decode_records(const uint16_t *q, const uint16_t *k_cache,
                            const uint16_t *v_cache, int batch, int n_q_heads, int n_kv_heads,
                            int head_dim, const int32_t *lens, int max_len,
                            int64_t kv_b_stride, int64_t kv_h_stride, float scale, int n_split,
                            void *ws, size_t ws_bytes, const q4nx_policy *policy,
                            void *stream);

/* ---------------------------------------------------------------- weight-stream floors
 * The null GEMV: exactly the grid, workgroup size and per-lane loads of the batch-1 q4 GEMV
 * (q4nx_gemv_q4 at batch 1 under the default policy: the row-block kernel) and its 16
 * output stores per workgroup, with no arithmetic: y receives XOR folds of the loaded bits,
 * not a GEMV. It times what the weight stream alone costs at a shape. Replaces the
 * reference's null design (designs/granite_gemv/granite_gemv.py:105-121, NULL_SRC; run by
 * --null at :315-321: "separates 'the kernel is slow' from 'the memory path is slow'").
 * Shapes as q4nx_gemv_q4; x 8-byte aligned; y fp32 [32*n_tile_rows]. */
int q4nx_gemv_q4_null(const uint8_t *w, const uint16_t *x, float *y, int n_tile_rows,
                      int k_tiles, void *stream);
/* A plain streaming read of bytes (a positive multiple of 16) at buf (16-byte aligned): every
 * byte loaded once, nothing written unless the fold of a workgroup's bytes hits a fixed
 * value (then one word of sink[64]). The device counterpart of the STREAM read floor of
 * designs/granite_gemv/cpu_baseline.cpp:157-166. */
int q4nx_stream_read(const void *buf, size_t bytes, uint32_t *sink, void *stream);

/* y[i] = bf16(x[i]), round to nearest even, NaN kept quiet: the device form of the bf16
 * rounding every kernel applies to its outputs (tools/q4nx.py:97-111 rounds the same way
 * on the host). */
int q4nx_round_bf16(const float *x, uint16_t *y, int64_t n, void *stream);

/* ---------------------------------------------------------------- decode-step helpers
 * h[b][:] = fp32 row tokens[b] of a [vocab][hidden] table: a plain bf16 matrix
 * (kind Q4NX_KIND_BF16, e.g. a stored model.embed_tokens.weight) or q4 / q8 tiles (a tied
 * lm_head used as the embedding, dequantised exactly as q4nx_dequant_* does);
 * ssq_out (optional, [batch][hidden/16]) as in q4nx_gemv_ex. A token outside [0, vocab)
 * gives a row of NaN, which every later result then shows. No reference counterpart: the reference has no token loop
 * (README.md:295-311); its Qwen path embeds through transformers. */
int q4nx_embed(int kind, const void *table, const int32_t *tokens, float *h, float *ssq_out,
               int vocab, int hidden, int batch, void *stream);
/* idx[b] = argmax_n logits[b][n] (first maximum), max[b] its value (optional). */
int q4nx_argmax(const float *logits, int n, int batch, int64_t stride, int32_t *idx,
                float *max_val, void *stream);
/* Greedy-loop bookkeeping in one small launch: tokens[b] = the row whose key is the
 * largest of keys[b][0..n_slots) (from q4nx_gemv_ex), pos[b] += 1, lens[b] = pos[b] + 1,
 * history[step][b] = tokens[b] while step < history_len; then step += 1. */
int q4nx_decode_advance(const uint64_t *keys, int n_slots, int32_t *tokens, int32_t *pos,
                        int32_t *lens, int32_t *history, int32_t *step, int history_len,
                        int batch, void *stream);
/* q4nx_decode_advance, then q4nx_embed of the new tokens into h / ssq_out (batch 1..64): a
 * greedy loop's next step starts from h with no embedding launch of its own. One launch at
 * batch 1; from batch 2 one workgroup per row, then a one-wave launch for the history and the
 * step counter. No reference counterpart (the reference has no token loop, README.md:295-311). */
int q4nx_decode_advance_embed(const uint64_t *keys, int n_slots, int32_t *tokens, int32_t *pos,
                              int32_t *lens, int32_t *history, int32_t *step, int history_len,
                              int batch, int kind, const void *table, int vocab, int hidden,
                              float *h, float *ssq_out, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* Q4NX_HIP_H */
