/* Launchers of the gfx950 kernels: the operator layer between the host engine
 * and the device code. All pointers are device pointers, all launches go to
 * `stream`, every launcher returns the launch status. Row-major throughout.
 *
 * Role of the reference's src/kernels/kernels.h:21-102, with signatures of our
 * own (the only callers are this engine and the ops library). Data layouts in
 * HBM that differ from the reference are stated per launcher. */
#ifndef CUJEV_KERNELS_H
#define CUJEV_KERNELS_H

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t bf16_t; /* storage type of bfloat16 seen from C */

/* Token tiles of the attention kernel: 32 consecutive packed tokens per wave
 * group; K/V tiles are 64 keys. Caches are padded so aligned 64-key tiles
 * never leave the allocation. */
#define CUJEV_ATT_KEY_TILE 64
static inline int cujev_kv_stride(int max_tokens) { return (max_tokens + 63) / 64 * 64 + 64; }

/* RoPE table rope[p][i] = (cos a, sin a), a = fl32(fl32(1/theta^(2i/rot)) * p),
 * i < rot/2, p < npos: the fp32 angle transformers forms (inv_freq times the
 * position in fp32), its cos/sin evaluated in double and rounded once.
 * `out` has npos * rot floats (host memory). */
#include <math.h>
static inline void cujev_rope_table_host(double theta, int rot, int npos, float *out) {
    for (int i = 0; i < rot / 2; i++) {
        const float f = (float)(1.0 / pow(theta, 2.0 * i / rot));
        for (int p = 0; p < npos; p++) {
            const float a = f * (float)p;
            out[((size_t)p * (rot / 2) + i) * 2] = (float)cos((double)a);
            out[((size_t)p * (rot / 2) + i) * 2 + 1] = (float)sin((double)a);
        }
    }
}

/* ---- full attention -----------------------------------------------------
 * proj[N, proj_stride] bf16 is the fused projection row
 *   [Hq x (q 256 | gate 256)] [Hkv x K 256] [Hkv x V 256].
 * Per q-head: zero-centred RMSNorm (q_norm_w already holds 1+w), RoPE on the
 * first `rot` dims (rotate_half with the device table rope_table of
 * cujev_rope_table_host, indexed by pos[n]), times q_scale
 * (= head_dim^-1/2 * log2 e), rounded to bf16 -> q_out[N][Hq][256].
 * Per kv-head: the same for K -> k_cache[Hkv][cache_stride][256] row n;
 * V copied raw -> vt_cache[Hkv][256][cache_stride] column n (d-major).
 * The cache column of packed token n is n itself. */
hipError_t k_attn_prep(const bf16_t *proj, int proj_stride, const float *q_norm_w,
                       const float *k_norm_w, const int32_t *pos, int N, int Hq, int Hkv, int rot,
                       const float *rope_table, float eps, float q_scale, bf16_t *q_out,
                       bf16_t *k_cache, bf16_t *vt_cache, int cache_stride, hipStream_t stream);
/* The same over Na + Nb tokens in one launch: K / V^T of tokens [0, Na) go
 * to columns n of (k_cache, vt_cache), those of tokens [Na, Na + Nb) to
 * columns n - Na of (k_cache2, vt_cache2); q_out rows are n throughout. */
hipError_t k_attn_prep_pair(const bf16_t *proj, int proj_stride, const float *q_norm_w,
                            const float *k_norm_w, const int32_t *pos, int Na, int Nb, int Hq,
                            int Hkv, int rot, const float *rope_table, float eps, float q_scale,
                            bf16_t *q_out, bf16_t *k_cache, bf16_t *vt_cache, int cache_stride,
                            bf16_t *k_cache2, bf16_t *vt_cache2, int cache_stride2,
                            hipStream_t stream);

/* out[n, h*256 + d] = sigmoid(gate[n*gate_tok_stride + h*gate_head_stride + d])
 *                     * softmax_j(q[n,h] . k_j) v_j          (base-2 softmax)
 * over keys j in [0, P) of the state cache (pk / pvt, stride p_stride) and
 * the own keys j in [own_base[n], n] of (ok / ovt, stride o_stride).
 * q is bf16 [N][Hq][256] already scaled by head_dim^-1/2 * log2 e. GQA:
 * q-head h reads kv-head h / (Hq/Hkv); Hq/Hkv must be 4. */
hipError_t k_attention(const bf16_t *q, const bf16_t *gate, int gate_tok_stride,
                       int gate_head_stride, const bf16_t *pk, const bf16_t *pvt, int P,
                       int p_stride, const bf16_t *ok, const bf16_t *ovt, int o_stride,
                       const int32_t *own_base, int N, int Hq, int Hkv, bf16_t *out,
                       void *ws, size_t ws_bytes, hipStream_t stream);
/* With few workgroups (N <= CUJEV_ATTN_SPLIT_MAX_N tokens giving under 128
 * of them), k_attention splits the key tiles over
 * cujev_attention_splits() workgroups per token tile and merges their
 * softmax partials in a second kernel, when `ws` holds
 * cujev_attention_ws_bytes() bytes; otherwise (ws NULL) one pass. */
#define CUJEV_ATTN_SPLIT_MAX_N 256
#define CUJEV_ATTN_MAX_SPLITS 16
int cujev_attention_splits(int N, int Hkv, int P);
size_t cujev_attention_ws_bytes(int N, int Hq, int nsplit);
/* the largest workspace any N <= max_tokens can use */
size_t cujev_attention_ws_max(int max_tokens, int Hq, int Hkv);
/* Two k_attention problems over one state cache (pk, pvt) in one launch,
 * one pass each (no key split): rows [0, Na) of q, gate, own_base and out
 * are problem a (the cache's first Pa keys, own keys in oka / ovta), rows
 * [Na, Na + Nb) problem b (Pb keys, own keys in okb / ovtb; own_base
 * counted from its own first row). The workgroups of one run beside the
 * other's, so the launch takes about as long as the longer of the two. Same
 * results as two k_attention calls with ws NULL. */
hipError_t k_attention_pair(const bf16_t *q, const bf16_t *gate, int gate_tok_stride,
                            int gate_head_stride, const bf16_t *pk, const bf16_t *pvt,
                            int p_stride, const int32_t *own_base, bf16_t *out, int Hq, int Hkv,
                            int Na, int Pa, const bf16_t *oka, const bf16_t *ovta, int oa_stride,
                            int Nb, int Pb, const bf16_t *okb, const bf16_t *ovtb, int ob_stride,
                            hipStream_t stream);

/* ---- Gated DeltaNet -------------------------------------------------------
 * proj[N, proj_stride] bf16 is the fused row [q Hk*128 | k Hk*128 | v Hv*128 |
 * z Hv*128 | b Hv | a Hv]. Conv (width 4, no bias) + SiLU over the first
 * C = (2Hk+Hv)*128 columns; taps before a segment start (local index from
 * own_base) come from conv_in[C][3] (NULL = zeros). Then q,k l2-normalised
 * (q also * 128^-1/2) -> fp32 q,k [N][Hk][128], v fp32 [N][Hv][128],
 * g = A_neg_exp * softplus(a + dt_bias), beta = sigmoid(b) -> fp32 [N][Hv].
 * If conv_out != NULL the last three pre-conv inputs of the first segment
 * (tokens [0, seg0_len)) are written there as [C][3]. */
hipError_t k_gdn_conv_prep(const bf16_t *proj, int proj_stride, const float *conv_w,
                           const float *conv_in, float *conv_out, int seg0_len,
                           const int32_t *own_base, const float *A_neg_exp, const float *dt_bias,
                           int N, int Hk, int Hv, float *q, float *k, float *v, float *g,
                           float *beta, hipStream_t stream);

/* 64-token chunks of the packed segments; chunks never cross a segment. */
typedef struct cujev_chunks {
    const int32_t *chunk_tok0; /* [num_chunks] first packed token */
    const int32_t *chunk_len;  /* [num_chunks] 1..64              */
    const int32_t *seg_chunk0; /* [num_segments] first chunk      */
    const int32_t *seg_nchunk; /* [num_segments] chunk count      */
    int num_chunks;
    int num_segments;
    int max_seg_chunks; /* most chunks in one segment (host-side); 0 = not known */
    /* [num_chunks] or NULL: bit t set where token t of the chunk starts a
     * segment. Non-NULL packs whole segments (each <= 64 tokens) into chunks;
     * only for branches that all continue S_in with no final state written.
     * The segment arrays are then unused. */
    const uint64_t *chunk_starts;
    int max_seg_len; /* longest segment in tokens (host-side); 0 = not known */
} cujev_chunks;

/* Scratch of the chunked scan, written by the parallel first phase in the
 * MFMA operand-fragment order of the sequential second phase, so each of its
 * lanes reads 16 contiguous bytes per fragment and a wave reads 1 KiB runs.
 * Per (chunk, v-head):
 *   W          [64][128] as 16x16x32 A fragments (4 row blocks x 4 k-steps), bf16
 *   QK^T masked [64][64] as 16x16x32 A fragments (4 x 2), bf16 hi then lo
 *   U          [64][128] as 16x16 accumulator fragments per 32-column block, fp32
 *   G          [64] cumulative log-decay of each token (restarting at segment
 *              starts; past the chunk's end the last token's value)
 * Per (chunk, k-head), shared by the k-head's v-heads (their decays are
 * applied in the second phase):
 *   Q          [64][128] as 16x16x32 A fragments, bf16
 *   K^T        [128][64] as 32x32x16 A fragments (4 x 4), bf16 hi then lo
 * O is the fp32 output [N][Hv][128] before the gated norm. The per-k-head
 * arrays are sized per v-head (Hk <= Hv). */
typedef struct cujev_gdn_scratch {
    void *W;  /* bf16 [chunks][Hv][1024][8] */
    void *Q;  /* bf16 [chunks][Hk][1024][8] */
    void *QK; /* bf16 [chunks][Hv][2][512][8]  */
    void *KT; /* bf16 [chunks][Hk][2][1024][8] */
    float *U; /* fp32 [chunks][Hv][1024][8] */
    float *G; /* [chunks][Hv][64] */
    float *O; /* fp32 [N][Hv][128] */
} cujev_gdn_scratch;

static inline size_t cujev_align256(size_t x) { return (x + 255) / 256 * 256; }
static inline size_t cujev_gdn_scratch_bytes(int num_chunks, int Hv, int N) {
    const size_t ch = (size_t)num_chunks * Hv;
    return 2 * cujev_align256(ch * 64 * 128 * 2) /* W, Q */ +
           cujev_align256(ch * 64 * 64 * 2 * 2) /* QK hi + lo */ +
           cujev_align256(ch * 64 * 128 * 2 * 2) /* K^T hi + lo */ +
           cujev_align256(ch * 64 * 128 * 4) /* U */ + cujev_align256(ch * 64 * 4) +
           cujev_align256((size_t)N * Hv * 128 * 4);
}
/* Carve the scratch of cujev_gdn_scratch_bytes() starting at `base`. */
static inline cujev_gdn_scratch cujev_gdn_scratch_carve(void *base, int num_chunks, int Hv) {
    const size_t ch = (size_t)num_chunks * Hv;
    char *p = (char *)base;
    cujev_gdn_scratch s;
    s.W = p;
    p += cujev_align256(ch * 64 * 128 * 2);
    s.Q = p;
    p += cujev_align256(ch * 64 * 128 * 2);
    s.QK = p;
    p += cujev_align256(ch * 64 * 64 * 2 * 2);
    s.KT = p;
    p += cujev_align256(ch * 64 * 128 * 2 * 2);
    s.U = (float *)p;
    p += cujev_align256(ch * 64 * 128 * 4);
    s.G = (float *)p;
    p += cujev_align256(ch * 64 * 4);
    s.O = (float *)p;
    return s;
}

/* Chunked gated delta rule over every segment (N packed tokens), each from
 * S_in[Hv][128][128] (fp32, read-only; NULL = zeros); S_out (may be NULL)
 * receives the final state of segment 0. The output goes through the gated
 * RMSNorm: y[n, hv*128 + c] = bf16( bf16(o * rsqrt(mean o^2 + eps))
 *                                   * norm_w[c] * silu(z[n*z_stride + hv*128 + c]) ). */
hipError_t k_gdn_scan(const float *q, const float *k, const float *v, const float *g,
                      const float *beta, const cujev_chunks *chunks, const float *S_in,
                      float *S_out, const bf16_t *z, int z_stride, const float *norm_w, float eps,
                      int Hk, int Hv, bf16_t *y, const cujev_gdn_scratch *scratch, int N,
                      hipStream_t stream);

/* The whole GDN mixer after in_proj: k_gdn_conv_prep's conv + gates computed
 * inside the scan's first phase (q, k, v never leave the chip), then
 * k_gdn_scan's recurrence and gated norm with z read from proj at column
 * C = (2Hk+Hv)*128. Same arguments and results as k_gdn_conv_prep followed by
 * k_gdn_scan (bit for bit). proj rows must be 16-byte aligned; conv_out
 * must not alias conv_in. */
hipError_t k_gdn_layer(const bf16_t *proj, int proj_stride, const float *conv_w,
                       const float *conv_in, float *conv_out, int seg0_len,
                       const int32_t *own_base, const float *A_neg_exp, const float *dt_bias,
                       const cujev_chunks *chunks, const float *S_in, float *S_out,
                       const float *norm_w, float eps, int Hk, int Hv, bf16_t *y,
                       const cujev_gdn_scratch *scratch, int N, hipStream_t stream);
/* k_gdn_layer up to its gated norm: where that norm would be a launch of its
 * own, o (fp32 [N][Hv][128]) is left in scratch->O and *o_pending = 1, for
 * one k_gdn_norm_gate over several calls' rows; where the scan kernel
 * applies the norm itself, y is written and *o_pending = 0. */
hipError_t k_gdn_layer_o(const bf16_t *proj, int proj_stride, const float *conv_w,
                         const float *conv_in, float *conv_out, int seg0_len,
                         const int32_t *own_base, const float *A_neg_exp, const float *dt_bias,
                         const cujev_chunks *chunks, const float *S_in, float *S_out,
                         const float *norm_w, float eps, int Hk, int Hv, bf16_t *y,
                         const cujev_gdn_scratch *scratch, int N, hipStream_t stream,
                         int *o_pending);
/* The gated RMSNorm of k_gdn_scan over `rows` = tokens x Hv rows of o (fp32,
 * 128 each): y[n, hv*128 + c] from o[n][hv] and z[n*z_stride + hv*128 + c]. */
hipError_t k_gdn_norm_gate(const float *o, const bf16_t *z, int z_stride, const float *norm_w,
                           float eps, int rows, int Hv, bf16_t *y, hipStream_t stream);

/* Few-token branches (eval: every segment continues S_in, none writes a
 * final state or conv tail, no packed chunks, each at most
 * CUJEV_GDN_RECUR_MAX_LEN tokens) can run the recurrence token by token in
 * fp32 (the reference's own form) instead of the chunked scan: one kernel for
 * conv, gates and recurrence, then the gated norm. Returns 1 when k_gdn_layer
 * takes that path for these arguments (the engine keys its captured graphs
 * on it). CUJEV_GDN_RECUR=0 never takes it, =1 whenever eligible; by default
 * only while segments x heads x tokens stays within the latency-bound range. */
#define CUJEV_GDN_RECUR_MAX_LEN 32
int cujev_gdn_recur_chosen(const cujev_chunks *chunks, int Hv, int has_S_out, int has_conv_out);
/* The token-by-token path on its own (the chunk table must describe one
 * chunk per segment; max_seg_len as above). */
hipError_t k_gdn_recur(const bf16_t *proj, int proj_stride, const float *conv_w,
                       const float *conv_in, const float *A_neg_exp, const float *dt_bias,
                       const cujev_chunks *chunks, const float *S_in, const float *norm_w,
                       float eps, int Hk, int Hv, bf16_t *y, const cujev_gdn_scratch *scratch,
                       int N, hipStream_t stream);

/* ---- per-layer glue --------------------------------------------------------
 * x[N,H] fp32 residual = E[tokens] (bf16 table).  REF elementwise.cu:3-11. */
hipError_t k_embed(const int32_t *tokens, const bf16_t *E, float *x, int N, int H, hipStream_t s);

/* Fused residual add + RMSNorm (REF elementwise.cu:13-40). Output row r reads
 * source row src = rows ? rows[r] : r (R rows, else N). The added term is
 *   d = y[src]                                  (y != NULL, bf16), or
 *   d = bf16(sum_{s < splits} yp[s][src])        (yp != NULL: fp32 split-K
 *       partials [splits][N][H] of k_gemm_small, splits <= 8, summed in split order);
 *   v = x[src] + d;  x[src] = v when there is a d and !rows;
 *   out[r] = bf16(v * rsqrt(mean v^2 + eps) * w)   (w holds 1 + weight).
 * H must be a multiple of 4 and at most 4096. */
hipError_t k_add_rmsnorm(float *x, const bf16_t *y, const float *yp, int splits, const float *w,
                         bf16_t *out, int N, int H, float eps, const int32_t *rows, int R,
                         hipStream_t s);

/* dst row r = src row rows[r] for r < R (row_bytes each; rows, pitches and
 * pointers 16-byte aligned). */
hipError_t k_gather_rows(const void *src, size_t src_pitch, const int32_t *rows, int R, void *dst,
                         size_t dst_pitch, size_t row_bytes, hipStream_t s);

/* act[N,I] = bf16(silu(gu[:, :I]) * gu[:, I:])  (REF elementwise.cu:42-54). */
hipError_t k_silu_mul(const bf16_t *gu, bf16_t *act, int N, int I, hipStream_t s);

/* logits[b*ld + i] = h[b] . E[cand[b*cand_ld + i]], i < ncand[b]
 * (REF elementwise.cu:78-97). h bf16 [B,H], fp32 accumulation. */
hipError_t k_readout(const bf16_t *h, const bf16_t *E, const int32_t *cand, const int32_t *ncand,
                     int cand_ld, float *logits, int ld, int B, int H, hipStream_t s);

/* ---- weight-streaming GEMM for few tokens (gemm_small.hip) ---------------
 * Y[N, M] = X[N, K] . W[M, K]^T for N <= CUJEV_GEMM_SMALL_MAX_N, M % 64 == 0,
 * K % 128 == 0, X rows of stride ldx, W given in the tiled layout that
 * k_gemm_small_tile writes (same size as W). splits == 1 writes bf16 Y (row stride
 * ldy); 1 < splits <= K / 128 writes fp32 partial sums P[splits][N][M]
 * instead (split s sums the 128-wide chunks [s C / splits, (s+1) C /
 * splits) of the C = K / 128), to be summed by the consumer in split order.
 * gated (splits == 1): W is the fused [gate I | up I] (M = 2I) and Y gets
 * act[N][I] = bf16(silu(bf16 gate) * bf16 up). */
#define CUJEV_GEMM_SMALL_MAX_N 96 /* 6 token blocks of 16: register budget without spills */
#define CUJEV_GEMM_SMALL_MAX_SPLITS 8
int cujev_gemm_small_splits(int M, int K); /* suggested split count (<= MAX_SPLITS), 0 = shape unsupported */
hipError_t k_gemm_small(const bf16_t *X, int ldx, const bf16_t *W, int N, int M, int K, int gated,
                        int splits, bf16_t *Y, int ldy, float *P, hipStream_t stream);
/* W [M, K] (M % 16 == 0, K % 128 == 0) -> Wt, the tiled copy k_gemm_small
 * streams: one contiguous 4 KiB block per 16 rows x 128 k, block number
 * chunk * (M/16) + row group. */
hipError_t k_gemm_small_tile(const bf16_t *W, int M, int K, bf16_t *Wt, hipStream_t stream);

/* ---- tiled GEMM for prefill token counts (gemm_wide.hip) ------------------
 * Same operands and outputs as k_gemm_small (tiled W, X rows of stride ldx,
 * bf16 Y / gated act / fp32 partials P[splits][N][M]) for any N >= 1; M % 16
 * == 0 (gated: M % 32), K % 128 == 0, (K / 128) % splits == 0, X and W each
 * under 4 GiB. The tile is 64 RG weight rows (gated: 32 RG gate rows and the
 * same up rows) x 32 NG tokens; cujev_gemm_wide_plan picks RG, NG and a split
 * count <= max_splits (1 = no partials) for a shape and returns 0, or -1 for
 * an unsupported shape. CUJEV_WIDE_PLAN="RG,NG,S" forces a plan. */
int cujev_gemm_wide_plan(int N, int M, int K, int gated, int max_splits, int *RG, int *NG, int *S);
int cujev_gemm_wide_supported(int RG, int NG, int gated);
hipError_t k_gemm_wide(const bf16_t *X, int ldx, const bf16_t *Wt, int N, int M, int K, int gated,
                       int RG, int NG, int splits, bf16_t *Y, int ldy, float *P,
                       hipStream_t stream);

/* ---- projection GEMMs (hipBLASLt) ------------------------------------------
 * Y[N,M] = X[N,K] . W[M,K]^T, bf16 in, fp32 accumulate, bf16 (f32out = 0) or
 * fp32 out. REF elementwise.cu:56-75. `workspace` (ws_bytes) is device memory
 * owned by the caller. */
typedef struct cujev_gemm cujev_gemm;
int cujev_gemm_create(cujev_gemm **out, void *workspace, size_t ws_bytes);
void cujev_gemm_destroy(cujev_gemm *g);
hipError_t k_gemm(cujev_gemm *g, const bf16_t *X, const bf16_t *W, void *Y, int f32out, int N,
                  int M, int K, hipStream_t stream);
/* Tuned-algorithm table (text file, see gemm.cpp); returns entries loaded,
 * -1 unreadable, -2 made with another hipBLASLt version. */
int cujev_gemm_load_table(cujev_gemm *g, const char *path);
int cujev_gemm_version(cujev_gemm *g);
/* Exhaustive hipBLASLt search for one shape; records the winner. */
int cujev_gemm_tune(cujev_gemm *g, const bf16_t *X, const bf16_t *W, void *Y, int f32out, int N,
                    int M, int K, hipStream_t stream, int *best_index, float *best_us,
                    float *heuristic_us);

#ifdef __cplusplus
}
#endif
#endif
