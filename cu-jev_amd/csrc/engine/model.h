/* Model, state and workspace of the host engine.
 * Role of REF src/engine/model.h:15-98, with the MI355X data layout:
 *   state, per full layer   K   bf16 [Hkv][kv_stride(max_state)][256]
 *                           V^T bf16 [Hkv][256][kv_stride(max_state)]
 *   state, per GDN layer    S fp32 [Hv][128][128], conv tail fp32 [C][3]
 *   workspace               branch K / V^T in the same layouts, bf16 q,
 *                           GDN bf16 q/k/v + chunk scratch, fp32 residual. */
#ifndef CUJEV_MODEL_H
#define CUJEV_MODEL_H

#include "core/config.h"
#include "core/devmem.h"
#include "cujev.h"
#include "kernels/kernels.h"
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct cujev_layer {
    cujev_layer_type type;
    float *in_norm;   /* [H] fp32, 1 + w */
    float *post_norm; /* [H] fp32, 1 + w */
    /* full attention */
    bf16_t *w_qkv;          /* [Hq*512 + 2*Hkv*256, H] row-fused q|k|v */
    float *q_norm, *k_norm; /* [256], 1 + w */
    bf16_t *w_o;            /* [H, Hq*256] */
    /* gated delta net */
    bf16_t *w_in;     /* [C + V + 2Hv, H] row-fused qkv|z|b|a */
    float *conv_w;    /* [C][4] */
    float *A_neg_exp; /* [Hv] = -exp(A_log) */
    float *dt_bias;   /* [Hv] */
    float *g_norm;    /* [128] (not zero-centred) */
    bf16_t *w_out;    /* [H, V] */
    /* mlp */
    bf16_t *w_gate_up; /* [2I, H] row-fused gate|up */
    bf16_t *w_down;    /* [H, I] */
    /* the same projections tiled for the few-token GEMM (k_gemm_small_tile),
     * which streams them at the eval shapes; NULL where it does not apply */
    bf16_t *wt_qkv, *wt_o, *wt_in, *wt_out, *wt_gate_up, *wt_down;
} cujev_layer;

/* Captured eval forwards (see forward.c): one executable graph per launch
 * shape. Everything a launch argument depends on is in the key; the per-call
 * metadata lives in fixed device buffers, so a replay only needs the upload. */
#define CUJEV_GRAPH_SLOTS 8
typedef struct cujev_graph_slot {
    const struct cujev_state *st;
    int P, N, B, nc, maxc, has_cand;
    int packed; /* GDN chunk table packed (its metadata offsets differ) */
    int recur;  /* GDN layers run the token-by-token branch path */
    int seen; /* eager runs so far; -1: capture failed, this key stays eager */
    hipGraphExec_t exec;
    unsigned long long stamp;
} cujev_graph_slot;

struct cujev_model {
    cujev_config cfg;
    cujev_options opts;
    cujev_slab weights; /* bf16 matrices (plain and tiled), fp32 vectors */
    cujev_slab work;    /* per-call buffers sized for the largest call */
    cujev_gemm *gemm;
    hipStream_t stream;
    hipEvent_t ev0, ev1;
    cujev_timing timing;

    bf16_t *embed;     /* [V, H] */
    bf16_t *lm_head;   /* [V, H]; == embed when tied */
    float *final_norm; /* [H], 1 + w */
    cujev_layer layers[CUJEV_MAX_LAYERS];

    /* derived widths */
    int D, Hq, Hkv, Hk, Hv, K, V, C;
    int w_attn, w_gdn, w_proj;
    int max_tokens;     /* workspace rows: max(max_state, max_branch), or their
                         * sum when prefills are deferred */
    int defer_prefill;  /* CUJEV_DEFER_PREFILL at open: 1 = a prefill runs
                         * inside the state's next eval (one pass over both),
                         * 2 = it runs first in that eval, on its own */
    int max_chunks;     /* GDN chunks of one forward */
    int state_stride;   /* kv stride of the state caches */
    int branch_stride;  /* kv stride of the branch scratch */

    /* workspace (device) */
    float *x;        /* [N,H] fp32 residual */
    bf16_t *xb;      /* [N,H] normed input */
    bf16_t *proj;    /* [N, w_proj] */
    bf16_t *y;       /* [N,H] */
    float *ypart;    /* split-K partials [splits][N][H] of the residual projections */
    size_t ypart_bytes; /* >= the few-token GEMM's 8 x 96 x H floats; the prefill GEMM
                         * picks its split count to fit */
    void *attn_ws;   /* key-split partials of the attention for few-token evals */
    size_t attn_ws_bytes;
    bf16_t *q;       /* [N,Hq,256] prescaled */
    bf16_t *mix_out; /* [N, max(Hq*256, V)] */
    bf16_t *br_k, *br_vt;
    void *gdn_scratch;
    bf16_t *act;  /* [N, I] */
    bf16_t *hsel; /* [B, H] */
    /* the last layer past its mixer runs on the B rows that reach the
     * outputs, gathered here: residual fp32 [B][H], mixer output bf16
     * [B][max(Hq*256, V)] */
    float *xl;
    bf16_t *mixl;
    float *full_logits; /* [B, vocab] */
    void *gemm_ws;
    size_t gemm_ws_bytes;
    /* per-call metadata, one device block uploaded with one copy */
    int32_t *d_meta, *h_meta; /* h_meta is pinned host memory */
    size_t meta_ints;
    float *d_logits; /* [B, max_candidates] */
    float *rope;     /* [max positions][rot/2] (cos, sin) */
    int rope_positions;
    cujev_graph_slot graphs[CUJEV_GRAPH_SLOTS];
    unsigned long long graph_clock;
};

struct cujev_state {
    cujev_model *model;
    cujev_slab mem; /* K / V^T caches, S, conv tails */
    int num_tokens;
    /* a deferred prefill not yet run: its tokens (host, max_state_tokens
     * ints) and count; 0 when the device state is current */
    int32_t *pending;
    int pending_n;
    bf16_t **kv_k, **kv_vt; /* per layer, NULL for GDN layers */
    float **S;              /* per layer, NULL for full layers */
    float **conv;           /* per layer, NULL for full layers */
};

cujev_status cujev_model_load_weights(cujev_model *m, const char *dir);
cujev_status cujev_model_alloc_workspace(cujev_model *m);

/* FUSED: one pass over [pending prefill tokens ++ branch tokens]. The
 * token-parallel kernels (embedding, projections, norms) run once over all
 * of them, so each layer's weights are streamed once; the mixers run per
 * group, the state's first (writing the state), then the branches' (reading
 * it), as PREFILL and EVAL would. */
typedef enum { CUJEV_FWD_PREFILL = 0, CUJEV_FWD_EVAL = 1, CUJEV_FWD_FUSED = 2 } cujev_fwd_mode;

/* Run the network over N tokens in B segments (host arrays). PREFILL: one
 * segment, side outputs go to the state. EVAL: every segment sees the state's
 * prefix and itself. On return hsel[B,H] holds the final-norm output of every
 * segment's last token, and candidates (if any) were staged by the caller. */
cujev_status cujev_forward(cujev_model *m, cujev_state *st, cujev_fwd_mode mode,
                           const int32_t *tokens, int N, const int32_t *seg_start,
                           const int32_t *seg_len, int B);
/* Same, also uploading candidate ids (host [B][maxc]) and counts (host [B])
 * with the metadata; their device copies are returned in d_cand / d_ncand.
 * With candidates the readout runs too: d_logits[B][maxc] holds the
 * candidate logits. EVAL forwards are replayed from captured HIP graphs
 * once a launch shape repeats (CUJEV_GRAPHS=0 keeps them eager). An EVAL on
 * a state with a pending prefill runs FUSED when both fit the workspace (no
 * graph), else the prefill first and then the EVAL; either way the state is
 * current afterwards. */
cujev_status cujev_forward_with_candidates(cujev_model *m, cujev_state *st, cujev_fwd_mode mode,
                                           const int32_t *tokens, int N, const int32_t *seg_start,
                                           const int32_t *seg_len, int B, const int32_t *cand,
                                           const int32_t *ncand, int maxc, int32_t **d_cand,
                                           int32_t **d_ncand);

/* Drop the captured graphs that use `st` (all of them when st is NULL). */
void cujev_graphs_forget(cujev_model *m, const struct cujev_state *st);

#ifdef __cplusplus
}
#endif
#endif
