/*
 * libcujev_ops.so -- operator-level C ABI of the branch-forward hot path.
 *
 * The reference has no such library: its operator layer is the C launcher
 * header src/kernels/kernels.h:21-102, called only by the engine
 * (src/engine/forward.c:92-145). libcujev.so keeps exactly the 14 public
 * functions of include/cujev.h, so this separate library exposes the same
 * kernels one by one for kernel-level parity tests and benchmarks (the
 * reference has no kernel-level tests). Every entry point takes device
 * pointers, plain sizes and a HIP stream (hipStream_t passed as void*; NULL is
 * the default stream), launches asynchronously and returns a cujev_status:
 * CUJEV_ERR_INVALID_ARGUMENT for shapes the kernels do not support,
 * CUJEV_ERR_CUDA (4) for a launch error, whose text is in cujev_ops_last_error().
 *
 * bf16 buffers are raw uint16 bfloat16. Layouts:
 *   proj      fused projection rows, bf16 [N][stride]
 *   k cache   bf16 [Hkv][cache_stride][256]   token-major
 *   vt cache  bf16 [Hkv][256][cache_stride]   d-major (V transposed)
 *   cache_stride must be a multiple of 64 and at least
 *   cujev_ops_kv_stride(max tokens) so 64-key tiles stay inside.
 */
#ifndef CUJEV_OPS_H
#define CUJEV_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Cache stride (in tokens) the attention kernels need for `max_tokens`. */
int cujev_ops_kv_stride(int max_tokens);
const char *cujev_ops_last_error(void);

/* Replaces reference src/kernels/kernels.h:50-53 (k_gemm_bf16*): Y[N,M] =
 * X[N,K] . W[M,K]^T, bf16 inputs, fp32 accumulation, bf16 (f32out = 0) or fp32
 * output, through hipBLASLt. `workspace` (ws_bytes, e.g. 64 MiB) is device
 * memory the caller keeps for the process; plans are cached per shape. */
int cujev_op_gemm(const void *X, const void *W, void *Y, int f32out, int N, int M, int K,
                  void *workspace, size_t ws_bytes, void *stream);

/* No counterpart in the reference (cuBLAS picks its own algorithm there):
 * times every hipBLASLt solution that supports the cujev_op_gemm problem
 * (N, M, K, f32out) on these buffers (Y is overwritten) and returns the
 * fastest one's solution index with its time and the time of hipBLASLt's
 * heuristic first choice, in microseconds per launch. The indices feed the
 * tuned-algorithm table the engine reads at model open. */
int cujev_op_gemm_tune(const void *X, const void *W, void *Y, int f32out, int N, int M, int K,
                       void *workspace, size_t ws_bytes, void *stream, int *best_index,
                       float *best_us, float *heuristic_us);
/* Replaces reference src/kernels/kernels.h:50-53 (k_gemm_bf16) for few
 * tokens, the eval-time shape: Y[N,M] = X[N,K] . W[M,K]^T with N <= 96,
 * M % 64 == 0, K % 128 == 0, X rows of stride ldx, bf16 in, fp32
 * accumulation, weights streamed once by a hand-written kernel.
 *   splits == 1: bf16 Y, row stride ldy.
 *   1 < splits <= min(8, K/128): fp32 partial sums P[splits][N][M] (no Y); split
 *     s sums the 128-wide K chunks [s C / splits, (s+1) C / splits) of the
 *     C = K/128; sum them in split order (cujev_op_add_rmsnorm).
 *   gated (splits == 1): W is the fused [gate I | up I] weight (M = 2I) and
 *     Y receives act[N][I] = bf16(silu(bf16 gate) * bf16 up), which is the
 *     reference's GEMM + silu_mul pair (src/kernels/elementwise.cu:42-54). */
int cujev_op_gemm_small(const void *X, int ldx, const void *W, int N, int M, int K, int gated,
                        int splits, void *Y, int ldy, float *P, void *stream);
/* The weight layout cujev_op_gemm_small reads: Wt (M*K bf16, distinct from W)
 * receives W [M][K] (M % 16 == 0, K % 128 == 0) as one contiguous 4 KiB
 * block per 16 rows x 128 k, in the order the kernel's loads consume it;
 * the block of row group g and 128-wide K chunk c is number c * (M/16) + g.
 * Run once per weight; no counterpart in the reference, whose cuBLAS calls
 * read the plain rows. */
int cujev_op_gemm_small_tile(const void *W, int M, int K, void *Wt, void *stream);
/* Split count the engine uses for an (M, K) few-token GEMM; 0 = unsupported shape. */
int cujev_ops_gemm_small_splits(int M, int K);

/* Replaces reference src/kernels/kernels.h:50-53 (k_gemm_bf16) at prefill
 * token counts (any N >= 1): the operands and outputs of
 * cujev_op_gemm_small (tiled W from cujev_op_gemm_small_tile; bf16 Y, gated
 * act[N][M/2], or fp32 partials P[splits][N][M] to be summed in split order)
 * through a hand-tiled MFMA kernel. M % 16 == 0 (gated: M % 32 == 0),
 * K % 128 == 0, (K/128) % splits == 0, X and W under 4 GiB each. The tile is
 * 64 rg weight rows (gated: 32 rg gate rows and the same up rows) x 32 ng
 * tokens; (rg, ng) must be a pair cujev_ops_gemm_wide_plan can return. */
int cujev_op_gemm_wide(const void *X, int ldx, const void *W, int N, int M, int K, int gated,
                       int rg, int ng, int splits, void *Y, int ldy, float *P, void *stream);
/* The tile (rg, ng) and split count (<= max_splits) the engine uses for a
 * shape; 0 on success, -1 for an unsupported shape. */
int cujev_ops_gemm_wide_plan(int N, int M, int K, int gated, int max_splits, int *rg, int *ng,
                             int *splits);

/* Replaces reference src/kernels/kernels.h:40-43 (k_rmsnorm, k_add) fused:
 * row r reads source row src = rows ? rows[r] : r (R rows, else N);
 * v = x[src] + (y ? y[src] : yp ? bf16(sum_s yp[s][src]) : 0), written back
 * to x when something was added and rows == NULL; out[r] = bf16(v *
 * rsqrt(mean v^2 + eps) * w). y is bf16 [N][H]; yp is fp32 [splits][N][H]. */
int cujev_op_add_rmsnorm(float *x, const void *y, const float *yp, int splits, const float *w,
                         void *out, int N, int H, float eps, const int32_t *rows, int R,
                         void *stream);

/* hipBLASLt library version (solution indices are only valid for it). */
int cujev_ops_blaslt_version(void);

/* Fills the device RoPE table used by cujev_op_attn_prep: table[p][i] =
 * (cos a, sin a), a = fp32(fp32(theta^(-2i/rot)) * p), p < npos, i < rot/2
 * (npos * rot floats). Synchronous. Replaces the reference's per-launch
 * constant-memory inv_freq upload (src/kernels/attention.cu:87-96). */
int cujev_op_rope_table(double theta, int rot, int npos, float *table);

/* Replaces reference src/kernels/kernels.h:197-199 (k_attn_prep).
 * q_norm_w / k_norm_w: fp32 [256], already 1 + w. pos: int32 [N] (< npos of
 * the table). Writes q_out bf16 [N][Hq][256] scaled by q_scale (the engine
 * passes 256^-1/2 * log2 e), K rows n and V^T columns n of the caches. */
int cujev_op_attn_prep(const void *proj, int proj_stride, const float *q_norm_w,
                       const float *k_norm_w, const int32_t *pos, int N, int Hq, int Hkv,
                       int rot, const float *rope_table, float eps, float q_scale, void *q_out,
                       void *k_cache, void *vt_cache, int cache_stride, void *stream);

/* The same over Na + Nb tokens in one launch (no counterpart in the
 * reference; the engine's deferred-prefill pass writes the state's tokens
 * and the branches' this way): K rows / V^T columns of tokens [0, Na) go to
 * column n of (k_cache, vt_cache), those of the rest to column n - Na of
 * (k_cache2, vt_cache2); q_out rows are n throughout. The same bits as two
 * cujev_op_attn_prep calls. */
int cujev_op_attn_prep_pair(const void *proj, int proj_stride, const float *q_norm_w,
                            const float *k_norm_w, const int32_t *pos, int Na, int Nb, int Hq,
                            int Hkv, int rot, const float *rope_table, float eps, float q_scale,
                            void *q_out, void *k_cache, void *vt_cache, int cache_stride,
                            void *k_cache2, void *vt_cache2, int cache_stride2, void *stream);

/* Replaces reference src/kernels/kernels.h:203-206 (k_attention).
 * out bf16 [N][Hq*256] = sigmoid(gate) * softmax2(q.k) v over the state keys
 * [0,P) of (pk, pvt) and own keys [own_base[n], n] of (ok, ovt).
 * gate element (n, h, d) is at gate[n*gate_tok_stride + h*gate_head_stride + d]. */
int cujev_op_attention(const void *q, const void *gate, int gate_tok_stride, int gate_head_stride,
                       const void *pk, const void *pvt, int P, int p_stride, const void *ok,
                       const void *ovt, int o_stride, const int32_t *own_base, int N, int Hq,
                       int Hkv, void *out, void *stream);
/* Two such problems over one state cache in one launch (no counterpart in
 * the reference; the engine's deferred-prefill pass uses it for the state's
 * tokens and the branches' side by side). Rows [0, Na) of q, gate, own_base
 * and out are problem a (state keys [0, Pa), own keys in oka / ovta), rows
 * [Na, Na + Nb) problem b (state keys [0, Pb), own keys in okb / ovtb,
 * own_base counted from its first row). One pass each: the same bits as two
 * cujev_op_attention calls. */
int cujev_op_attention_pair(const void *q, const void *gate, int gate_tok_stride,
                            int gate_head_stride, const void *pk, const void *pvt, int p_stride,
                            const int32_t *own_base, void *out, int Hq, int Hkv, int Na, int Pa,
                            const void *oka, const void *ovta, int oa_stride, int Nb, int Pb,
                            const void *okb, const void *ovtb, int ob_stride, void *stream);
/* The same with a device workspace (no counterpart in the reference, whose
 * kernel has one pass): with few workgroups (N <= 256 tokens giving under
 * 128 of them) the key tiles are split over up to 16 workgroups
 * per token tile and their softmax partials merged by a second kernel. The
 * result equals one pass up to fp32 summation order. ws_bytes from
 * cujev_ops_attention_ws_bytes (0 = no split for this shape; a smaller ws
 * also runs one pass). */
int cujev_op_attention_ws(const void *q, const void *gate, int gate_tok_stride,
                          int gate_head_stride, const void *pk, const void *pvt, int P,
                          int p_stride, const void *ok, const void *ovt, int o_stride,
                          const int32_t *own_base, int N, int Hq, int Hkv, void *out, void *ws,
                          size_t ws_bytes, void *stream);
size_t cujev_ops_attention_ws_bytes(int N, int Hq, int Hkv, int P);

/* No counterpart in the reference. cujev_op_attention_ws for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): the same kernels and results, with the
 * key-split partials in a static device array the library holds, one per
 * GPU, until the process ends. It calls no hipMalloc / hipFree. Limit: the
 * partials of one call must fit CUJEV_OPS_ATTN_NOALLOC_SCRATCH_BYTES; every
 * shape the kernel accepts does (splits x N x Hq <= 32768 rows of 258
 * floats, since the kernel needs Hq = 4 Hkv), and a larger need is rejected
 * with status 6. Every call on one GPU shares the array, so calls that
 * overlap on one GPU (other streams, other threads) race; serialise them.
 * The stream must belong to the current device. */
#define CUJEV_OPS_ATTN_NOALLOC_SCRATCH_BYTES 33816576u /* 32.25 MiB */
int cujev_op_attention_noalloc(const void *q, const void *gate, int gate_tok_stride,
                               int gate_head_stride, const void *pk, const void *pvt, int P,
                               int p_stride, const void *ok, const void *ovt, int o_stride,
                               const int32_t *own_base, int N, int Hq, int Hkv, void *out,
                               void *stream);

/* Replaces reference src/kernels/kernels.h:214-215 (k_gdn_conv) and :221-223
 * (k_gdn_prep), fused. proj rows [q Hk*128 | k Hk*128 | v Hv*128 | z | b | a].
 * Conv (width 4) + SiLU with taps before a segment taken from conv_in [C][3]
 * (NULL = zeros); own_base[n] = first token of n's segment. Outputs fp32
 * q, k [N][Hk][128] (l2-normalised, q * 128^-1/2), v [N][Hv][128], fp32
 * g, beta [N][Hv] (the scan keeps q, k, v at about 16 significant bits). conv_out (may be NULL) gets the last three pre-conv inputs
 * of tokens [0, seg0_len) as [C][3]. conv_w fp32 [C][4]. */
int cujev_op_gdn_conv_prep(const void *proj, int proj_stride, const float *conv_w,
                           const float *conv_in, float *conv_out, int seg0_len,
                           const int32_t *own_base, const float *A_neg_exp,
                           const float *dt_bias, int N, int Hk, int Hv, void *q, void *k,
                           void *v, float *g, float *beta, void *stream);

/* Bytes of device scratch cujev_op_gdn_scan needs for num_chunks chunks of
 * N packed tokens. */
size_t cujev_ops_gdn_scratch_bytes(int num_chunks, int Hv, int N);

/* Replaces reference src/kernels/kernels.h:228-230 (k_gdn_scan) and :233-234
 * (k_gdn_norm_gate), fused. Chunk table (device int32): chunk_tok0/chunk_len
 * [num_chunks], seg_chunk0/seg_nchunk [num_segments]; each segment is cut into
 * chunks of 64 tokens from its start. S_in fp32 [Hv][128][128] (NULL = 0),
 * S_out (may be NULL) = final state of segment 0. y bf16 [N][Hv*128] is the
 * gated-RMSNorm output; z is read at z[n*z_stride + hv*128 + c].
 * max_seg_chunks: the largest seg_nchunk entry as the caller knows it (0 =
 * not given); 1 with S_out == NULL (branches continuing a state) selects a
 * path that reads S once per v-head for a group of segments.
 * chunk_starts (device uint64 [num_chunks], may be NULL): packs several whole
 * segments of at most 64 tokens into one chunk; bit t is set where token t of
 * the chunk starts a segment. Only with S_out == NULL: every segment continues
 * S_in, and seg_chunk0 / seg_nchunk / num_segments are not read.
 * q, k, v are cujev_op_gdn_conv_prep's fp32 outputs. Hv / Hk <= 4.
 * scratch: cujev_ops_gdn_scratch_bytes(num_chunks, Hv, N) bytes, 256-aligned. */
int cujev_op_gdn_scan(const void *q, const void *k, const void *v, const float *g,
                      const float *beta, const int32_t *chunk_tok0, const int32_t *chunk_len,
                      int num_chunks, const int32_t *seg_chunk0, const int32_t *seg_nchunk,
                      int num_segments, int max_seg_chunks, const uint64_t *chunk_starts,
                      const float *S_in, float *S_out, const void *z,
                      int z_stride, const float *norm_w, float eps, int Hk, int Hv, int N,
                      void *y, void *scratch, void *stream);

/* Replaces reference src/kernels/kernels.h:214-215 (k_gdn_conv), :221-223
 * (k_gdn_prep), :228-230 (k_gdn_scan) and :233-234 (k_gdn_norm_gate): the
 * GDN mixer from the in_proj rows to the gated-norm output in one call.
 * Arguments as cujev_op_gdn_conv_prep followed by cujev_op_gdn_scan (z is
 * read from proj at column C = (2Hk+Hv)*128); the result is bit-identical to
 * that pair, but q, k, v, g and beta are never written out. proj rows must be
 * 16-byte aligned (proj_stride % 8 == 0); conv_out must not alias conv_in. */
int cujev_op_gdn_layer(const void *proj, int proj_stride, const float *conv_w,
                       const float *conv_in, float *conv_out, int seg0_len,
                       const int32_t *own_base, const float *A_neg_exp, const float *dt_bias,
                       const int32_t *chunk_tok0, const int32_t *chunk_len, int num_chunks,
                       const int32_t *seg_chunk0, const int32_t *seg_nchunk, int num_segments,
                       int max_seg_chunks, const uint64_t *chunk_starts, const float *S_in,
                       float *S_out, const float *norm_w, float eps, int Hk, int Hv, int N,
                       void *y, void *scratch, void *stream);

/* No counterpart in the reference's kernel list; its semantics are the
 * reference's recurrent scan (src/kernels/gdn.cu:111-182) for eval branches:
 * cujev_op_gdn_layer's result for branches that each continue S_in with no
 * final state or conv tail written, computed token by token in fp32. The
 * chunk table must hold one chunk per segment (chunk_tok0 / chunk_len indexed
 * through seg_chunk0), every segment at most max_seg_len <= 32 tokens; the
 * scratch is cujev_ops_gdn_scratch_bytes(num_segments, Hv, N) bytes.
 * cujev_op_gdn_layer itself never takes this path; the engine does for small
 * evals. */
int cujev_op_gdn_recur(const void *proj, int proj_stride, const float *conv_w,
                       const float *conv_in, const float *A_neg_exp, const float *dt_bias,
                       const int32_t *chunk_tok0, const int32_t *chunk_len,
                       const int32_t *seg_chunk0, int num_segments, int max_seg_len,
                       const float *S_in, const float *norm_w, float eps, int Hk, int Hv, int N,
                       void *y, void *scratch, void *stream);

#ifdef __cplusplus
}
#endif
#endif
