/* The forward pass: one function for both uses (REF src/engine/forward.c:1-149).
 *
 *   PREFILL  N tokens, one segment. Full-attention K and V^T go into the
 *            state's cache; each GDN layer's final S and conv tail go into
 *            the state.
 *   EVAL     N tokens in B segments (branches). Every token attends to the
 *            state's prefix plus its own segment; every GDN segment starts
 *            from the state's S and conv tail (read-only, never copied).
 *
 * Per-call metadata (positions, segment starts, final-norm rows, the GDN
 * chunk table, candidates) is built on the host and uploaded with ONE copy.
 * The residual add and the next RMSNorm are fused, so a layer is
 * 4 GEMMs + 4 (attention) or 3 (GDN) kernels + 2 norm/add passes.
 * CUJEV_DEBUG_SYNC=1 synchronises and checks after every stage
 * (REF src/engine/forward.c:21-41). */
#include "engine/model.h"
#include <math.h>

static int debug_sync_enabled(void) {
    static int cached = -1;
    if (cached < 0) {
        const char *e = getenv("CUJEV_DEBUG_SYNC");
        cached = e && *e && *e != '0';
    }
    return cached;
}

static cujev_status check(cujev_model *m, hipError_t launch, const char *what, int layer) {
    if (launch != hipSuccess)
        return cujev_raise(launch == hipErrorInvalidValue ? CUJEV_ERR_UNSUPPORTED : CUJEV_ERR_CUDA,
                          "%s (layer %d): %s", what, layer, hipGetErrorString(launch));
    if (!debug_sync_enabled())
        return CUJEV_OK;
    hipError_t e = hipStreamSynchronize(m->stream);
    if (e == hipSuccess)
        e = hipGetLastError();
    if (e != hipSuccess)
        return cujev_raise(CUJEV_ERR_CUDA, "%s (layer %d): %s", what, layer, hipGetErrorString(e));
    return CUJEV_OK;
}

#define K_TRY(call, what, layer) CJ_CHECK(check(m, (call), (what), (layer)))

/* Everything the launch sequence needs besides the model and the state.
 * Tokens come in up to two groups: the state's (PREFILL, and the first Ns of
 * a FUSED call) and the branches' (EVAL, and the rest of a FUSED call).
 * `chunks` is the GDN chunk table of the PREFILL or EVAL group; a FUSED call
 * has the branches' there and the state's in `schunks`. Token indices in a
 * table, and own-key bases, count from the start of their group. */
typedef struct {
    cujev_fwd_mode mode;
    int N, B, P, nc, maxc;
    int Ns, nc_s; /* FUSED: state tokens (first in the call) and their chunks */
    const int32_t *tok, *pos, *base, *rows, *cand, *ncand; /* device metadata */
    cujev_chunks chunks, schunks;
} fwd_launch;

/* Projection GEMMs Y[N,M] = X[N,K] W^T. For few tokens (the eval, N <= 96)
 * the hand-written weight-streaming kernel reads the pre-tiled copy of the
 * weight (its time is the HBM stream of W). Up to 1000 tokens the
 * hand-tiled prefill kernel (gemm_wide, same tiled copy) takes every
 * projection: measured on MI355X against hipBLASLt on the plain rows, with
 * cold weights, for the 4B shapes at 256-800 tokens it took 0.69-0.98 of
 * the time for qkv and in_proj, 0.55-0.74 for o_proj / out_proj and
 * 0.52-0.61 for down_proj (the last two split over K into fp32 partials
 * that the residual add sums), and 0.65-0.89 for the gated gate|up + silu.
 * At 1024 tokens hipBLASLt was faster for in_proj (69-72 against 77 us), so
 * above 1000 tokens the projections go to hipBLASLt, except gate|up, which
 * stays on the kernel up to 2048 tokens (0.84-1.03 of hipBLASLt + silu_mul
 * there); above that hipBLASLt + silu_mul measured faster for gate|up: a 4B
 * eval of 2560 tokens 25.48 -> 25.09 ms, and the 9B request with its
 * 4096-token eval 155.6 -> 150.9 ms.
 * CUJEV_SMALL_GEMM=0 / CUJEV_WIDE_GEMM=0 send those shapes to hipBLASLt. */
static int env_on(const char *name) {
    const char *e = getenv(name);
    return !(e && *e == '0');
}

static int small_gemm_ok(int N, int M, int K) {
    static int cached = -1;
    if (cached < 0)
        cached = env_on("CUJEV_SMALL_GEMM");
    return cached && N <= CUJEV_GEMM_SMALL_MAX_N && cujev_gemm_small_splits(M, K) > 0;
}

#define CUJEV_WIDE_GATED_MAX_N 2048
#define CUJEV_WIDE_MAX_N 1000
static int wide_gemm_on(void) {
    static int cached = -1;
    if (cached < 0)
        cached = env_on("CUJEV_WIDE_GEMM");
    return cached;
}

static hipError_t proj_gemm(cujev_model *m, const bf16_t *X, const bf16_t *W, const bf16_t *Wt,
                            bf16_t *Y, int N, int M, int K) {
    if (Wt && small_gemm_ok(N, M, K))
        return k_gemm_small(X, K, Wt, N, M, K, 0, 1, Y, M, NULL, m->stream);
    int rg, ng, sp;
    if (Wt && wide_gemm_on() && N <= CUJEV_WIDE_MAX_N &&
        cujev_gemm_wide_plan(N, M, K, 0, 1, &rg, &ng, &sp) == 0)
        return k_gemm_wide(X, K, Wt, N, M, K, 0, rg, ng, 1, Y, M, NULL, m->stream);
    return k_gemm(m->gemm, X, W, Y, 0, N, M, K, m->stream);
}

/* A projection whose output feeds the residual add (o_proj, out_proj,
 * down_proj: M = H). Returns through *y / *yp / *splits what the following
 * k_add_rmsnorm reads: bf16 rows, or split-K fp32 partials in m->ypart. */
static hipError_t resid_gemm(cujev_model *m, const bf16_t *X, const bf16_t *W, const bf16_t *Wt,
                             int N, int M, int K, const bf16_t **y, const float **yp,
                             int *splits) {
    *y = m->y;
    *yp = NULL;
    *splits = 0;
    if (Wt && small_gemm_ok(N, M, K)) {
        const int sp = cujev_gemm_small_splits(M, K);
        if (sp > 1) {
            *y = NULL;
            *yp = m->ypart;
            *splits = sp;
            return k_gemm_small(X, K, Wt, N, M, K, 0, sp, NULL, 0, m->ypart, m->stream);
        }
        return k_gemm_small(X, K, Wt, N, M, K, 0, 1, m->y, M, NULL, m->stream);
    }
    if (Wt && wide_gemm_on() && N <= CUJEV_WIDE_MAX_N) {
        size_t cap = m->ypart_bytes / ((size_t)N * M * 4);
        const int max_sp = cap > 8 ? 8 : (int)cap;
        int rg, ng, sp;
        if (max_sp >= 1 && cujev_gemm_wide_plan(N, M, K, 0, max_sp, &rg, &ng, &sp) == 0) {
            if (sp > 1) {
                *y = NULL;
                *yp = m->ypart;
                *splits = sp;
                return k_gemm_wide(X, K, Wt, N, M, K, 0, rg, ng, sp, NULL, 0, m->ypart,
                                   m->stream);
            }
            return k_gemm_wide(X, K, Wt, N, M, K, 0, rg, ng, 1, m->y, M, NULL, m->stream);
        }
    }
    return k_gemm(m->gemm, X, W, m->y, 0, N, M, K, m->stream);
}

/* gate|up projection + silu_mul into m->act [N][I] */
static hipError_t gate_up_gemm(cujev_model *m, const cujev_layer *ly, int N, int I, int H) {
    if (ly->wt_gate_up && small_gemm_ok(N, 2 * I, H))
        return k_gemm_small(m->xb, H, ly->wt_gate_up, N, 2 * I, H, 1, 1, m->act, I, NULL,
                            m->stream);
    int rg, ng, sp;
    if (ly->wt_gate_up && wide_gemm_on() && N <= CUJEV_WIDE_GATED_MAX_N &&
        cujev_gemm_wide_plan(N, 2 * I, H, 1, 1, &rg, &ng, &sp) == 0)
        return k_gemm_wide(m->xb, H, ly->wt_gate_up, N, 2 * I, H, 1, rg, ng, 1, m->act, I, NULL,
                           m->stream);
    hipError_t e = proj_gemm(m, m->xb, ly->w_gate_up, NULL, m->proj, N, 2 * I, H);
    return e != hipSuccess ? e : k_silu_mul(m->proj, m->act, N, I, m->stream);
}

/* The kernels of one forward (and the candidate readout); no host sync. */
static cujev_status launch_all(cujev_model *m, cujev_state *st, const fwd_launch *a) {
    const cujev_config *c = &m->cfg;
    const int H = c->hidden_size, I = c->intermediate_size, N = a->N, B = a->B, P = a->P;
    const cujev_fwd_mode mode = a->mode;
    const float eps = c->rms_norm_eps;
    hipStream_t s = m->stream;
    const float q_scale = (1.0f / sqrtf((float)m->D)) * 1.4426950408889634f;
    /* the groups: ns state tokens (rows [0, ns)), then nb branch tokens */
    const int ns = mode == CUJEV_FWD_PREFILL ? N : mode == CUJEV_FWD_FUSED ? a->Ns : 0;
    const int nb = N - ns;
    const cujev_chunks *sch = mode == CUJEV_FWD_FUSED ? &a->schunks : &a->chunks;
    /* GDN scratch. FUSED: the state group's chunk arrays, then o for all N
     * rows (the branch group's rows after the state's, so one gated norm
     * covers both), then the branch group's chunk arrays. */
    const cujev_gdn_scratch gws_s =
        cujev_gdn_scratch_carve(m->gdn_scratch, mode == CUJEV_FWD_FUSED ? a->nc_s : a->nc, m->Hv);
    cujev_gdn_scratch gws_b = gws_s;
    if (mode == CUJEV_FWD_FUSED) {
        gws_b = cujev_gdn_scratch_carve((char *)gws_s.O + cujev_align256((size_t)N * m->Hv * 128 * 4),
                                        a->nc, m->Hv);
        gws_b.O = gws_s.O + (size_t)ns * m->Hv * 128;
    }
    const size_t qrow = (size_t)m->Hq * m->D; /* q and attention-output row width */

    K_TRY(k_embed(a->tok, m->embed, m->x, N, H, s), "embed", -1);
    K_TRY(k_add_rmsnorm(m->x, NULL, NULL, 0, m->layers[0].in_norm, m->xb, N, H, eps, NULL, 0, s),
          "norm", 0);

    for (int l = 0; l < c->num_layers; l++) {
        cujev_layer *ly = &m->layers[l];
        const bf16_t *ry; /* what the residual add reads: bf16 rows or split-K partials */
        const float *ryp;
        int rsp;
        /* Past the last layer's mixer only each segment's last token reaches
         * the outputs: the state's rows need nothing more (a PREFILL ends
         * there), and the branches' final rows go on alone. */
        const int last = l + 1 == c->num_layers;
        const bf16_t *w_res, *wt_res; /* the mixer's output projection */
        int k_res;
        if (ly->type == CUJEV_LAYER_FULL) {
            K_TRY(proj_gemm(m, m->xb, ly->w_qkv, ly->wt_qkv, m->proj, N, m->w_attn, H), "gemm qkv",
                  l);
            /* state tokens: K and V^T into the state's cache, causal over it;
             * branch tokens: into the branch scratch, over the state's P keys
             * and their own */
            const bf16_t *bproj = m->proj + (size_t)ns * m->w_attn;
            if (ns && nb) /* FUSED: one launch, each group into its cache */
                K_TRY(k_attn_prep_pair(m->proj, m->w_attn, ly->q_norm, ly->k_norm, a->pos, ns, nb,
                                       m->Hq, m->Hkv, c->rotary_dim, m->rope, eps, q_scale, m->q,
                                       st->kv_k[l], st->kv_vt[l], m->state_stride, m->br_k,
                                       m->br_vt, m->branch_stride, s),
                      "attn_prep", l);
            else if (ns)
                K_TRY(k_attn_prep(m->proj, m->w_attn, ly->q_norm, ly->k_norm, a->pos, ns, m->Hq,
                                  m->Hkv, c->rotary_dim, m->rope, eps, q_scale, m->q, st->kv_k[l],
                                  st->kv_vt[l], m->state_stride, s),
                      "attn_prep", l);
            else
                K_TRY(k_attn_prep(bproj, m->w_attn, ly->q_norm, ly->k_norm, a->pos + ns, nb, m->Hq,
                                  m->Hkv, c->rotary_dim, m->rope, eps, q_scale,
                                  m->q + (size_t)ns * qrow, m->br_k, m->br_vt, m->branch_stride,
                                  s),
                      "attn_prep", l);
            /* whose attention output is read: the state's rows only before
             * the last layer */
            const int att_s = ns && !last, att_b = nb > 0;
            if (att_s && att_b) /* FUSED: both groups in one launch, side by side */
                K_TRY(k_attention_pair(m->q, m->proj + m->D, m->w_attn, 2 * m->D, st->kv_k[l],
                                       st->kv_vt[l], m->state_stride, a->base, m->mix_out, m->Hq,
                                       m->Hkv, ns, 0, st->kv_k[l], st->kv_vt[l], m->state_stride,
                                       nb, P, m->br_k, m->br_vt, m->branch_stride, s),
                      "attention", l);
            else if (att_s)
                K_TRY(k_attention(m->q, m->proj + m->D, m->w_attn, 2 * m->D, st->kv_k[l],
                                  st->kv_vt[l], 0, m->state_stride, st->kv_k[l], st->kv_vt[l],
                                  m->state_stride, a->base, ns, m->Hq, m->Hkv, m->mix_out,
                                  m->attn_ws, m->attn_ws_bytes, s),
                      "attention", l);
            else if (att_b)
                K_TRY(k_attention(m->q + (size_t)ns * qrow, bproj + m->D, m->w_attn, 2 * m->D,
                                  st->kv_k[l], st->kv_vt[l], P, m->state_stride, m->br_k,
                                  m->br_vt, m->branch_stride, a->base + ns, nb, m->Hq, m->Hkv,
                                  m->mix_out + (size_t)ns * qrow, m->attn_ws, m->attn_ws_bytes,
                                  s),
                      "attention", l);
            w_res = ly->w_o, wt_res = ly->wt_o, k_res = m->Hq * m->D;
        } else {
            K_TRY(proj_gemm(m, m->xb, ly->w_in, ly->wt_in, m->proj, N, m->w_gdn, H), "gemm in", l);
            /* state tokens write the state's final S and conv tail; branch
             * tokens continue from them (read-only) */
            /* o of both groups is left in scratch and normed by one launch
             * where neither group's scan applied the norm itself */
            int pend_s = 0, pend_b = 0;
            if (ns)
                K_TRY(k_gdn_layer_o(m->proj, m->w_gdn, ly->conv_w, NULL, st->conv[l], ns, a->base,
                                    ly->A_neg_exp, ly->dt_bias, sch, NULL, st->S[l], ly->g_norm,
                                    eps, m->Hk, m->Hv, m->mix_out, &gws_s, ns, s, &pend_s),
                      "gdn_layer", l);
            if (nb)
                K_TRY(k_gdn_layer_o(m->proj + (size_t)ns * m->w_gdn, m->w_gdn, ly->conv_w,
                                    st->conv[l], NULL, nb, a->base + ns, ly->A_neg_exp,
                                    ly->dt_bias, &a->chunks, st->S[l], NULL, ly->g_norm, eps,
                                    m->Hk, m->Hv, m->mix_out + (size_t)ns * m->V, &gws_b, nb, s,
                                    &pend_b),
                      "gdn_layer", l);
            const bf16_t *z = m->proj + m->C; /* the gate z, after the conv channels */
            const int zs = m->w_gdn;
            if (pend_s && pend_b)
                K_TRY(k_gdn_norm_gate(gws_s.O, z, zs, ly->g_norm, eps, N * m->Hv, m->Hv,
                                      m->mix_out, s),
                      "gdn_norm", l);
            else if (pend_s)
                K_TRY(k_gdn_norm_gate(gws_s.O, z, zs, ly->g_norm, eps, ns * m->Hv, m->Hv,
                                      m->mix_out, s),
                      "gdn_norm", l);
            else if (pend_b)
                K_TRY(k_gdn_norm_gate(gws_b.O, z + (size_t)ns * zs, zs, ly->g_norm, eps,
                                      nb * m->Hv, m->Hv, m->mix_out + (size_t)ns * m->V, s),
                      "gdn_norm", l);
            w_res = ly->w_out, wt_res = ly->wt_out, k_res = m->V;
        }
        if (last && mode == CUJEV_FWD_PREFILL)
            break;
        int n = N; /* rows past the mixer */
        const bf16_t *mix = m->mix_out;
        float *x = m->x;
        if (last) { /* the segments' last tokens, gathered */
            K_TRY(k_gather_rows(m->mix_out, (size_t)k_res * 2, a->rows, B, m->mixl,
                                (size_t)k_res * 2, (size_t)k_res * 2, s),
                  "gather", l);
            K_TRY(k_gather_rows(m->x, (size_t)H * 4, a->rows, B, m->xl, (size_t)H * 4,
                                (size_t)H * 4, s),
                  "gather", l);
            n = B, mix = m->mixl, x = m->xl;
        }
        K_TRY(resid_gemm(m, mix, w_res, wt_res, n, H, k_res, &ry, &ryp, &rsp), "gemm o/out", l);
        K_TRY(k_add_rmsnorm(x, ry, ryp, rsp, ly->post_norm, m->xb, n, H, eps, NULL, 0, s),
              "add+norm", l);
        K_TRY(gate_up_gemm(m, ly, n, I, H), "gemm gate_up", l);
        K_TRY(resid_gemm(m, m->act, ly->w_down, ly->wt_down, n, H, I, &ry, &ryp, &rsp),
              "gemm down", l);
        K_TRY(k_add_rmsnorm(x, ry, ryp, rsp, last ? m->final_norm : m->layers[l + 1].in_norm,
                            last ? m->hsel : m->xb, n, H, eps, NULL, 0, s),
              last ? "final norm" : "add+norm", l);
    }
    if (a->cand)
        K_TRY(k_readout(m->hsel, m->lm_head, a->cand, a->ncand, a->maxc, m->d_logits, a->maxc, B,
                        H, s),
              "readout", -1);
    return CUJEV_OK;
}

/* ---- captured eval forwards ----------------------------------------------
 * A launch shape is (state, P, N, B, chunks, candidate width). Its first eval
 * runs eagerly (this also creates the hipBLASLt plans of its GEMM shapes,
 * which time candidates with host syncs); the second is captured into a HIP
 * graph and every later one replays it. Graph nodes are kernels only (no
 * memset nodes). At most CUJEV_GRAPH_SLOTS shapes are kept (least recently
 * used goes first); a state's graphs are dropped with the state. */
/* Pack eval branches into shared chunks when B * Hv exceeds this many
 * (segment, head) units; CUJEV_GDN_PACK_MIN_UNITS overrides it (read on every
 * forward; negative = never pack). */
static int gdn_pack_min_units(void) {
    const char *e = getenv("CUJEV_GDN_PACK_MIN_UNITS");
    return e && *e ? atoi(e) : 512;
}

static int graphs_enabled(void) {
    static int cached = -1;
    if (cached < 0) {
        const char *e = getenv("CUJEV_GRAPHS");
        cached = !(e && *e == '0');
    }
    return cached && !debug_sync_enabled();
}

void cujev_graphs_forget(cujev_model *m, const struct cujev_state *st) {
    for (int i = 0; i < CUJEV_GRAPH_SLOTS; i++) {
        cujev_graph_slot *g = &m->graphs[i];
        if (g->st && (!st || g->st == st)) {
            if (g->exec)
                hipGraphExecDestroy(g->exec);
            memset(g, 0, sizeof *g);
        }
    }
}

static cujev_status run_eval(cujev_model *m, cujev_state *st, const fwd_launch *a) {
    if (!graphs_enabled())
        return launch_all(m, st, a);
    cujev_graph_slot *g = NULL, *victim = &m->graphs[0];
    const int has_cand = a->cand != NULL;
    /* a packed and an unpacked table can have the same chunk count, but
     * their metadata sits at other offsets of the uploaded block */
    const int packed = a->chunks.chunk_starts != NULL;
    /* same shape, other GDN kernels: the segment lengths pick the path */
    const int recur = cujev_gdn_recur_chosen(&a->chunks, m->Hv, 0, 0);
    for (int i = 0; i < CUJEV_GRAPH_SLOTS; i++) {
        cujev_graph_slot *x = &m->graphs[i];
        if (x->st == st && x->P == a->P && x->N == a->N && x->B == a->B && x->nc == a->nc &&
            x->maxc == a->maxc && x->has_cand == has_cand && x->packed == packed &&
            x->recur == recur) {
            g = x;
            break;
        }
        if (!x->st || (victim->st && x->stamp < victim->stamp))
            victim = x;
    }
    if (!g) {
        if (victim->exec)
            hipGraphExecDestroy(victim->exec);
        memset(victim, 0, sizeof *victim);
        g = victim;
        g->st = st;
        g->P = a->P;
        g->N = a->N;
        g->B = a->B;
        g->nc = a->nc;
        g->maxc = a->maxc;
        g->has_cand = has_cand;
        g->packed = packed;
        g->recur = recur;
    }
    g->stamp = ++m->graph_clock;
    if (g->exec) {
        hipError_t e = hipGraphLaunch(g->exec, m->stream);
        return e == hipSuccess ? CUJEV_OK
                               : cujev_raise(CUJEV_ERR_CUDA, "hipGraphLaunch: %s",
                                            hipGetErrorString(e));
    }
    if (g->seen == 0 || g->seen < 0) {
        if (g->seen == 0)
            g->seen = 1;
        return launch_all(m, st, a);
    }
    /* second sighting: capture */
    hipError_t e = hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) {
        g->seen = -1;
        return launch_all(m, st, a);
    }
    cujev_status s = launch_all(m, st, a);
    hipGraph_t graph = NULL;
    e = hipStreamEndCapture(m->stream, &graph);
    if (s != CUJEV_OK) {
        if (graph)
            hipGraphDestroy(graph);
        return s;
    }
    hipGraphExec_t exec = NULL;
    if (e == hipSuccess)
        e = hipGraphInstantiate(&exec, graph, NULL, NULL, 0);
    if (graph)
        hipGraphDestroy(graph);
    if (e != hipSuccess) { /* not capturable here: this shape stays eager */
        cujev_note(1, "eval graph capture failed (%s); shape N=%d B=%d runs eagerly",
                  hipGetErrorString(e), a->N, a->B);
        (void)hipGetLastError();
        g->seen = -1;
        return launch_all(m, st, a);
    }
    g->exec = exec;
    e = hipGraphLaunch(exec, m->stream);
    return e == hipSuccess ? CUJEV_OK
                           : cujev_raise(CUJEV_ERR_CUDA, "hipGraphLaunch: %s", hipGetErrorString(e));
}

/* GDN chunk rows of B segments (starts counted within their group): each
 * segment's 64-token chunks in order. Returns the number of chunks. */
static int fill_chunk_table(int32_t *h, size_t o_ctok, size_t o_clen, size_t o_sc0, size_t o_snc,
                            const int32_t *seg_start, const int32_t *seg_len, int B) {
    int ci = 0;
    for (int b = 0; b < B; b++) {
        h[o_sc0 + b] = ci;
        for (int t = 0; t < seg_len[b]; t += 64) {
            h[o_ctok + ci] = seg_start[b] + t;
            h[o_clen + ci] = seg_len[b] - t < 64 ? seg_len[b] - t : 64;
            ci++;
        }
        h[o_snc + b] = ci - h[o_sc0 + b];
    }
    return ci;
}

/* One forward over Ns state tokens (FUSED only, stok) followed by Nt tokens
 * in B segments (the prefill's one segment, or the branches). */
static cujev_status forward_call(cujev_model *m, cujev_state *st, cujev_fwd_mode mode,
                                 const int32_t *stok, int Ns, const int32_t *tokens, int Nt,
                                 const int32_t *seg_start, const int32_t *seg_len, int B,
                                 const int32_t *cand, const int32_t *ncand, int maxc,
                                 int32_t **d_cand, int32_t **d_ncand) {
    const int N = Ns + Nt;
    const int P = mode == CUJEV_FWD_EVAL ? st->num_tokens : Ns;

    /* ---- metadata: one packed block, one upload ---- */
    int nc = 0;
    for (int b = 0; b < B; b++)
        nc += (seg_len[b] + 63) / 64;
    const int nc_s = (Ns + 63) / 64;
    if (nc + nc_s > m->max_chunks)
        return cujev_raise(CUJEV_ERR_CAPACITY, "%d GDN chunks exceed %d", nc + nc_s,
                          m->max_chunks);
    /* Eval branches that each fit a 64-token chunk: consecutive whole
     * segments share a chunk (they all continue the stored state and write
     * none back), so a scan chunk holds up to 64 tokens however short the
     * branches are. Only when the branches already give the scan more
     * (segment, head) units than about two workgroups per CU: below that,
     * packing would only lengthen each workgroup's serial chain. npk =
     * packed chunks, 0 when not packing. */
    int npk = 0;
    const int pack_min = gdn_pack_min_units();
    if (mode != CUJEV_FWD_PREFILL && pack_min >= 0 && B * m->Hv > pack_min) {
        int fill = 64, end = -1;
        for (int b = 0; b < B; b++) {
            if (seg_len[b] > 64) {
                npk = 0;
                break;
            }
            if (seg_len[b] <= 0)
                continue;
            if (fill + seg_len[b] > 64 || seg_start[b] != end) {
                npk++;
                fill = 0;
            }
            fill += seg_len[b];
            end = seg_start[b] + seg_len[b];
        }
    }
    const int fused = mode == CUJEV_FWD_FUSED;
    int32_t *h = m->h_meta;
    size_t o = 0;
    const size_t o_cst = o; o += 2 * (size_t)npk; /* uint64 segment-start masks, 8-byte aligned */
    const size_t o_tok = o; o += (size_t)N;
    const size_t o_pos = o; o += (size_t)N;
    const size_t o_base = o; o += (size_t)N;
    const size_t o_rows = o; o += (size_t)B;
    const size_t o_ctok = o; o += (size_t)nc;
    const size_t o_clen = o; o += (size_t)nc;
    const size_t o_sc0 = o; o += (size_t)B;
    const size_t o_snc = o; o += (size_t)B;
    const size_t o_sctok = o; o += (size_t)nc_s; /* FUSED: the state's one-segment table */
    const size_t o_sclen = o; o += (size_t)nc_s;
    const size_t o_ssc0 = o; o += fused;
    const size_t o_ssnc = o; o += fused;
    const size_t o_cand = o; o += cand ? (size_t)B * maxc : 0;
    const size_t o_ncand = o; o += cand ? (size_t)B : 0;
    if (o > m->meta_ints)
        return cujev_raise(CUJEV_ERR_CAPACITY, "per-call metadata exceeds its buffer");
    if (Ns) { /* state tokens: positions 0.., one causal segment from 0 */
        memcpy(h + o_tok, stok, (size_t)Ns * 4);
        for (int t = 0; t < Ns; t++) {
            h[o_pos + t] = t;
            h[o_base + t] = 0;
        }
        const int32_t s0 = 0, sl = Ns;
        fill_chunk_table(h, o_sctok, o_sclen, o_ssc0, o_ssnc, &s0, &sl, 1);
    }
    memcpy(h + o_tok + Ns, tokens, (size_t)Nt * 4);
    for (int b = 0; b < B; b++) {
        for (int t = 0; t < seg_len[b]; t++) {
            const int n = Ns + seg_start[b] + t;
            h[o_pos + n] = P + t;
            h[o_base + n] = seg_start[b];
        }
        h[o_rows + b] = Ns + seg_start[b] + seg_len[b] - 1;
    }
    fill_chunk_table(h, o_ctok, o_clen, o_sc0, o_snc, seg_start, seg_len, B);
    if (npk) { /* the chunk rows now describe packed chunks */
        int pc = -1, end = -1;
        uint64_t mask = 0;
        for (int b = 0; b < B; b++) {
            if (seg_len[b] <= 0)
                continue;
            if (pc < 0 || h[o_clen + pc] + seg_len[b] > 64 || seg_start[b] != end) {
                if (pc >= 0)
                    memcpy(h + o_cst + 2 * pc, &mask, 8);
                pc++;
                h[o_ctok + pc] = seg_start[b];
                h[o_clen + pc] = 0;
                mask = 0;
            }
            mask |= 1ull << h[o_clen + pc];
            h[o_clen + pc] += seg_len[b];
            end = seg_start[b] + seg_len[b];
        }
        memcpy(h + o_cst + 2 * pc, &mask, 8);
    }
    if (cand) {
        memcpy(h + o_cand, cand, (size_t)B * maxc * 4);
        memcpy(h + o_ncand, ncand, (size_t)B * 4);
    }
    HIP_CHECK(hipMemcpyAsync(m->d_meta, h, o * 4, hipMemcpyHostToDevice, m->stream));
    const int32_t *d = m->d_meta;
    if (d_cand) {
        *d_cand = cand ? m->d_meta + o_cand : NULL;
        *d_ncand = cand ? m->d_meta + o_ncand : NULL;
    }
    fwd_launch a;
    memset(&a, 0, sizeof a);
    a.mode = mode;
    a.N = N;
    a.B = B;
    a.P = P;
    a.nc = nc;
    a.Ns = Ns;
    a.nc_s = nc_s;
    a.maxc = cand ? maxc : 0;
    a.tok = d + o_tok;
    a.pos = d + o_pos;
    a.base = d + o_base;
    a.rows = d + o_rows;
    a.cand = cand ? d + o_cand : NULL;
    a.ncand = cand ? d + o_ncand : NULL;
    int max_snc = 0, max_len = 0;
    for (int b = 0; b < B; b++) {
        max_snc = h[o_snc + b] > max_snc ? h[o_snc + b] : max_snc;
        max_len = seg_len[b] > max_len ? seg_len[b] : max_len;
    }
    const cujev_chunks chunks = {d + o_ctok, d + o_clen, d + o_sc0, d + o_snc, nc, B, max_snc,
                                 NULL, max_len};
    a.chunks = chunks;
    if (npk) {
        a.nc = a.chunks.num_chunks = npk;
        a.chunks.chunk_starts = (const uint64_t *)(d + o_cst);
    }
    if (fused) {
        const cujev_chunks sc = {d + o_sctok, d + o_sclen, d + o_ssc0, d + o_ssnc, nc_s, 1, nc_s,
                                 NULL, Ns};
        a.schunks = sc;
    }
    return mode == CUJEV_FWD_EVAL ? run_eval(m, st, &a) : launch_all(m, st, &a);
}

cujev_status cujev_forward_with_candidates(cujev_model *m, cujev_state *st, cujev_fwd_mode mode,
                                           const int32_t *tokens, int N, const int32_t *seg_start,
                                           const int32_t *seg_len, int B, const int32_t *cand,
                                           const int32_t *ncand, int maxc, int32_t **d_cand,
                                           int32_t **d_ncand) {
    if (mode == CUJEV_FWD_FUSED)
        return cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "FUSED comes from a pending prefill");
    if (mode == CUJEV_FWD_EVAL && st->pending_n > 0) {
        /* a deferred prefill: one pass over both when they fit the
         * workspace, else the prefill on its own first */
        const int Ns = st->pending_n;
        int nc = 0;
        for (int b = 0; b < B; b++)
            nc += (seg_len[b] + 63) / 64;
        st->pending_n = 0;
        cujev_status s;
        if (m->defer_prefill == 1 && Ns + N <= m->max_tokens &&
            nc + (Ns + 63) / 64 <= m->max_chunks) {
            s = forward_call(m, st, CUJEV_FWD_FUSED, st->pending, Ns, tokens, N, seg_start,
                             seg_len, B, cand, ncand, maxc, d_cand, d_ncand);
            if (s != CUJEV_OK)
                st->num_tokens = 0; /* the state is not usable */
            return s;
        }
        const int32_t s0 = 0, sl = Ns;
        s = forward_call(m, st, CUJEV_FWD_PREFILL, NULL, 0, st->pending, Ns, &s0, &sl, 1, NULL,
                         NULL, 0, NULL, NULL);
        /* the eval rewrites the pinned metadata block the prefill's upload reads */
        if (s == CUJEV_OK && hipStreamSynchronize(m->stream) != hipSuccess)
            s = cujev_raise(CUJEV_ERR_CUDA, "deferred prefill failed");
        if (s != CUJEV_OK) {
            st->num_tokens = 0;
            return s;
        }
    }
    return forward_call(m, st, mode, NULL, 0, tokens, N, seg_start, seg_len, B, cand, ncand, maxc,
                        d_cand, d_ncand);
}

cujev_status cujev_forward(cujev_model *m, cujev_state *st, cujev_fwd_mode mode,
                           const int32_t *tokens, int N, const int32_t *seg_start,
                           const int32_t *seg_len, int B) {
    return cujev_forward_with_candidates(m, st, mode, tokens, N, seg_start, seg_len, B, NULL, NULL,
                                         0, NULL, NULL);
}
