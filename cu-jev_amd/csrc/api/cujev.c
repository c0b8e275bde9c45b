/* The public C ABI (include/cujev.h): argument checks, model/state lifetime,
 * branch packing, candidate readout, timing. Behaviour of REF
 * src/api/cujev.c:11-327: same validation order and status codes, same
 * capacity rules, one stream per model, every call synchronous. */
#include <dlfcn.h>
#include "engine/model.h"
#include <math.h>

#define API __attribute__((visibility("default")))

API void cujev_options_default(cujev_options *o) {
    if (!o)
        return;
    memset(o, 0, sizeof *o);
    o->device = 0;
    o->max_state_tokens = 8192;
    o->max_branch_tokens = 4096;
    o->max_branches = 256;
    o->max_candidates = 256;
}

/* Tuned hipBLASLt algorithms: CUJEV_GEMM_TABLE, else
 * gemm_table_gfx950_hipblaslt<version>.txt next to this library, for the
 * hipBLASLt the process actually loaded (a process that imported torch first
 * runs on torch's bundled copy, others on the system one). A missing or
 * foreign-version table leaves every shape on hipBLASLt's heuristic. */
static void load_gemm_table(cujev_model *m) {
    char buf[4096];
    const char *path = getenv("CUJEV_GEMM_TABLE");
    if (!path) {
        Dl_info info;
        if (!dladdr((void *)load_gemm_table, &info) || !info.dli_fname)
            return;
        snprintf(buf, sizeof buf, "%s", info.dli_fname);
        char *slash = strrchr(buf, '/');
        const size_t dir = slash ? (size_t)(slash - buf + 1) : 0;
        snprintf(buf + dir, sizeof buf - dir, "gemm_table_gfx950_hipblaslt%d.txt",
                 cujev_gemm_version(m->gemm));
        path = buf;
    }
    const int n = cujev_gemm_load_table(m->gemm, path);
    if (n >= 0)
        cujev_note(m->opts.verbose, "gemm table: %d tuned shapes from %s", n, path);
    else if (n == -2)
        cujev_note(1, "gemm table %s was made with another hipBLASLt version; ignored", path);
}

API void cujev_model_close(cujev_model *m) {
    if (!m)
        return;
    if (m->stream)
        hipStreamSynchronize(m->stream);
    cujev_graphs_forget(m, NULL);
    cujev_gemm_destroy(m->gemm);
    if (m->h_meta)
        hipHostFree(m->h_meta);
    cujev_slab_release(&m->work);
    cujev_slab_release(&m->weights);
    if (m->ev0)
        hipEventDestroy(m->ev0);
    if (m->ev1)
        hipEventDestroy(m->ev1);
    if (m->stream)
        hipStreamDestroy(m->stream);
    free(m);
}

API cujev_status cujev_model_open(const char *dir, const cujev_options *opts, cujev_model **out) {
    if (!dir || !out)
        return cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "null argument");
    *out = NULL;
    cujev_model *m = (cujev_model *)calloc(1, sizeof *m);
    if (!m)
        return cujev_raise(CUJEV_ERR_OOM, "model struct");
    if (opts)
        m->opts = *opts;
    else
        cujev_options_default(&m->opts);
    if (m->opts.max_state_tokens <= 0 || m->opts.max_branch_tokens <= 0 ||
        m->opts.max_branches <= 0 || m->opts.max_candidates < 0) {
        free(m);
        return cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "capacities must be positive");
    }
    /* config first: fails before any device call */
    cujev_status s = cujev_config_load(dir, &m->cfg);
    if (s != CUJEV_OK) {
        free(m);
        return s;
    }
    const cujev_config *c = &m->cfg;
    m->D = c->head_dim;
    m->Hq = c->num_heads;
    m->Hkv = c->num_kv_heads;
    m->Hk = c->lin_num_k_heads;
    m->Hv = c->lin_num_v_heads;
    m->K = m->Hk * c->lin_k_dim;
    m->V = m->Hv * c->lin_v_dim;
    m->C = 2 * m->K + m->V;
    m->w_attn = m->Hq * 2 * m->D + 2 * m->Hkv * m->D;
    m->w_gdn = m->C + m->V + 2 * m->Hv;
    m->w_proj = m->w_attn;
    if (m->w_gdn > m->w_proj)
        m->w_proj = m->w_gdn;
    if (2 * c->intermediate_size > m->w_proj)
        m->w_proj = 2 * c->intermediate_size;
    m->max_tokens = m->opts.max_state_tokens > m->opts.max_branch_tokens
                        ? m->opts.max_state_tokens
                        : m->opts.max_branch_tokens;
    /* CUJEV_DEFER_PREFILL=1: a prefill only stages its tokens and runs inside
     * the state's next eval, as one pass over state and branch tokens (each
     * layer's weights streamed once for both); the workspace then holds both.
     * =2 stages too, but the eval runs the prefill on its own first. */
    {
        const char *e = getenv("CUJEV_DEFER_PREFILL");
        m->defer_prefill = e && (*e == '1' || *e == '2') ? *e - '0' : 0;
    }
    if (m->defer_prefill)
        m->max_tokens = m->opts.max_state_tokens + m->opts.max_branch_tokens;
    m->state_stride = cujev_kv_stride(m->opts.max_state_tokens);
    m->branch_stride = cujev_kv_stride(m->opts.max_branch_tokens);
    m->rope_positions = m->opts.max_state_tokens + m->opts.max_branch_tokens;

    hipError_t e = hipSetDevice(m->opts.device);
    if (e != hipSuccess) {
        const int dev = m->opts.device;
        free(m);
        return cujev_raise(CUJEV_ERR_CUDA, "hipSetDevice(%d): %s", dev, hipGetErrorString(e));
    }
    if ((e = hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking)) != hipSuccess ||
        (e = hipEventCreate(&m->ev0)) != hipSuccess || (e = hipEventCreate(&m->ev1)) != hipSuccess) {
        cujev_model_close(m);
        return cujev_raise(CUJEV_ERR_CUDA, "stream/event creation: %s", hipGetErrorString(e));
    }
    s = cujev_model_load_weights(m, dir);
    if (s == CUJEV_OK)
        s = cujev_model_alloc_workspace(m);
    if (s == CUJEV_OK && cujev_gemm_create(&m->gemm, m->gemm_ws, m->gemm_ws_bytes) != 0)
        s = cujev_raise(CUJEV_ERR_CUDA, "hipblasLtCreate failed");
    if (s == CUJEV_OK)
        load_gemm_table(m);
    if (s == CUJEV_OK && (e = hipStreamSynchronize(m->stream)) != hipSuccess)
        s = cujev_raise(CUJEV_ERR_CUDA, "%s", hipGetErrorString(e));
    if (s != CUJEV_OK) {
        cujev_model_close(m);
        return s;
    }
    *out = m;
    return CUJEV_OK;
}

API cujev_status cujev_model_info_get(const cujev_model *m, cujev_model_info *o) {
    if (!m || !o)
        return cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "null argument");
    memset(o, 0, sizeof *o);
    snprintf(o->name, sizeof o->name, "%s", m->cfg.name);
    o->hidden_size = m->cfg.hidden_size;
    o->num_layers = m->cfg.num_layers;
    o->num_full_attention_layers = m->cfg.num_full_layers;
    o->vocab_size = m->cfg.vocab_size;
    o->max_state_tokens = m->opts.max_state_tokens;
    o->max_branch_tokens = m->opts.max_branch_tokens;
    o->max_branches = m->opts.max_branches;
    o->device_bytes_weights = cujev_slab_used(&m->weights);
    o->device_bytes_workspace = cujev_slab_used(&m->work);
    return CUJEV_OK;
}

API void cujev_state_destroy(cujev_state *st) {
    if (!st)
        return;
    if (st->model) {
        hipStreamSynchronize(st->model->stream);
        cujev_graphs_forget(st->model, st);
    }
    cujev_slab_release(&st->mem);
    free(st->pending);
    free(st->kv_k);
    free(st->kv_vt);
    free(st->S);
    free(st->conv);
    free(st);
}

API cujev_status cujev_state_create(cujev_model *m, cujev_state **out) {
    if (!m || !out)
        return cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "null argument");
    *out = NULL;
    cujev_state *st = (cujev_state *)calloc(1, sizeof *st);
    if (!st)
        return cujev_raise(CUJEV_ERR_OOM, "state struct");
    st->model = m;
    const int L = m->cfg.num_layers;
    st->kv_k = (bf16_t **)calloc((size_t)L, sizeof(bf16_t *));
    st->kv_vt = (bf16_t **)calloc((size_t)L, sizeof(bf16_t *));
    st->S = (float **)calloc((size_t)L, sizeof(float *));
    st->conv = (float **)calloc((size_t)L, sizeof(float *));
    if (!st->kv_k || !st->kv_vt || !st->S || !st->conv) {
        cujev_state_destroy(st);
        return cujev_raise(CUJEV_ERR_OOM, "state tables");
    }
    const size_t kv_bytes = (size_t)m->Hkv * m->state_stride * m->D * 2;
    const size_t S_bytes = (size_t)m->Hv * 128 * 128 * 4;
    const size_t conv_bytes = (size_t)m->C * 3 * 4;
    /* pass 0 plans the slab, pass 1 carves it */
    for (int pass = 0; pass < 2; pass++) {
        for (int l = 0; l < L; l++) {
            if (m->cfg.layer_types[l] == CUJEV_LAYER_FULL) {
                st->kv_k[l] = (bf16_t *)cujev_slab_take(&st->mem, kv_bytes);
                st->kv_vt[l] = (bf16_t *)cujev_slab_take(&st->mem, kv_bytes);
            } else {
                st->S[l] = (float *)cujev_slab_take(&st->mem, S_bytes);
                st->conv[l] = (float *)cujev_slab_take(&st->mem, conv_bytes);
            }
        }
        if (pass == 0) {
            const cujev_status s = cujev_slab_commit(&st->mem, "state");
            if (s != CUJEV_OK) {
                cujev_state_destroy(st);
                return s;
            }
        }
    }
    /* finite everywhere: attention tiles read masked keys past the prefix */
    hipError_t e = hipMemset(st->mem.base, 0, cujev_slab_used(&st->mem));
    if (e != hipSuccess) {
        cujev_state_destroy(st);
        return cujev_raise(CUJEV_ERR_CUDA, "hipMemset state: %s", hipGetErrorString(e));
    }
    *out = st;
    return CUJEV_OK;
}

API int cujev_state_num_tokens(const cujev_state *st) { return st ? st->num_tokens : 0; }

API cujev_status cujev_state_prefill(cujev_model *m, cujev_state *st, const int32_t *tokens, int N) {
    if (!m || !st || !tokens || N <= 0)
        return cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "bad prefill arguments");
    if (st->model != m)
        return cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "state belongs to another model");
    if (N > m->opts.max_state_tokens)
        return cujev_raise(CUJEV_ERR_CAPACITY, "state of %d tokens exceeds max_state_tokens=%d", N,
                          m->opts.max_state_tokens);
    for (int i = 0; i < N; i++)
        if (tokens[i] < 0 || tokens[i] >= m->cfg.vocab_size)
            return cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "token id %d out of range", tokens[i]);
    st->pending_n = 0;
    if (m->defer_prefill) { /* staged; the next eval runs it */
        if (!st->pending) {
            st->pending = (int32_t *)malloc((size_t)m->opts.max_state_tokens * 4);
            if (!st->pending)
                return cujev_raise(CUJEV_ERR_OOM, "deferred prefill staging");
        }
        memcpy(st->pending, tokens, (size_t)N * 4);
        st->pending_n = N;
        st->num_tokens = N;
        m->timing.prefill_ms = 0.f;
        m->timing.prefill_tokens = N;
        cujev_error_reset();
        return CUJEV_OK;
    }
    const int32_t ss = 0, sl = N;
    st->num_tokens = 0;
    HIP_CHECK(hipEventRecord(m->ev0, m->stream));
    cujev_status s = cujev_forward(m, st, CUJEV_FWD_PREFILL, tokens, N, &ss, &sl, 1);
    if (s != CUJEV_OK) {
        hipStreamSynchronize(m->stream);
        return s;
    }
    HIP_CHECK(hipEventRecord(m->ev1, m->stream));
    HIP_CHECK(hipStreamSynchronize(m->stream));
    HIP_CHECK(hipGetLastError());
    hipEventElapsedTime(&m->timing.prefill_ms, m->ev0, m->ev1);
    m->timing.prefill_tokens = N;
    st->num_tokens = N;
    cujev_error_reset();
    return CUJEV_OK;
}

/* Concatenate branch tokens; seg_start/seg_len are [B]. REF src/api/cujev.c:189-217. */
static cujev_status pack_branches(cujev_model *m, const cujev_branch *br, int B, int32_t **tok,
                                  int32_t *seg_start, int32_t *seg_len, int *N_out) {
    long long N = 0;
    for (int b = 0; b < B; b++) {
        if (br[b].num_tokens <= 0 || !br[b].tokens)
            return cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "branch %d has no tokens", b);
        if (br[b].num_candidates < 0 || (br[b].num_candidates > 0 && !br[b].candidates))
            return cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "branch %d: bad candidates", b);
        if (br[b].num_candidates > m->opts.max_candidates)
            return cujev_raise(CUJEV_ERR_CAPACITY, "branch %d: %d candidates > max_candidates=%d",
                              b, br[b].num_candidates, m->opts.max_candidates);
        seg_start[b] = (int32_t)N;
        seg_len[b] = br[b].num_tokens;
        N += br[b].num_tokens;
    }
    if (N > m->opts.max_branch_tokens)
        return cujev_raise(CUJEV_ERR_CAPACITY, "%lld branch tokens exceed max_branch_tokens=%d", N,
                          m->opts.max_branch_tokens);
    int32_t *t = (int32_t *)malloc((size_t)N * 4);
    if (!t)
        return cujev_raise(CUJEV_ERR_OOM, "token staging");
    for (int b = 0; b < B; b++)
        memcpy(t + seg_start[b], br[b].tokens, (size_t)br[b].num_tokens * 4);
    for (long long i = 0; i < N; i++)
        if (t[i] < 0 || t[i] >= m->cfg.vocab_size) {
            const int32_t bad = t[i];
            free(t);
            return cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "token id %d out of range", bad);
        }
    *tok = t;
    *N_out = (int)N;
    return CUJEV_OK;
}

static cujev_status check_eval_args(cujev_model *m, cujev_state *st, const cujev_branch *br,
                                    int B) {
    if (!m || !st || !br || B <= 0)
        return cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "bad eval arguments");
    if (st->model != m)
        return cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "state belongs to another model");
    if (st->num_tokens == 0)
        return cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "state has not been prefilled");
    if (B > m->opts.max_branches)
        return cujev_raise(CUJEV_ERR_CAPACITY, "%d branches > max_branches=%d", B,
                          m->opts.max_branches);
    return CUJEV_OK;
}

API cujev_status cujev_eval(cujev_model *m, cujev_state *st, const cujev_branch *br, int B,
                            float *logits_out, int ld) {
    CJ_CHECK(check_eval_args(m, st, br, B));
    if (!logits_out)
        return cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "logits_out is NULL");
    int32_t *seg = (int32_t *)malloc((size_t)B * 2 * 4);
    if (!seg)
        return cujev_raise(CUJEV_ERR_OOM, "segment table");
    int32_t *seg_start = seg, *seg_len = seg + B;
    int32_t *tok = NULL, *cand = NULL, *ncand = NULL;
    int N = 0, maxc = 0;
    cujev_status s = pack_branches(m, br, B, &tok, seg_start, seg_len, &N);
    if (s != CUJEV_OK)
        goto out;
    for (int b = 0; b < B; b++)
        if (br[b].num_candidates > maxc)
            maxc = br[b].num_candidates;
    if (ld < maxc) {
        s = cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "ld=%d < max candidates=%d", ld, maxc);
        goto out;
    }
    if (maxc > 0) {
        cand = (int32_t *)calloc((size_t)B * maxc + B, 4);
        if (!cand) {
            s = cujev_raise(CUJEV_ERR_OOM, "candidate staging");
            goto out;
        }
        ncand = cand + (size_t)B * maxc;
        for (int b = 0; b < B; b++) {
            ncand[b] = br[b].num_candidates;
            for (int i = 0; i < br[b].num_candidates; i++) {
                const int32_t id = br[b].candidates[i];
                if (id < 0 || id >= m->cfg.vocab_size) {
                    s = cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "candidate id %d out of range", id);
                    goto out;
                }
                cand[(size_t)b * maxc + i] = id;
            }
        }
    }
    {
        hipError_t e = hipEventRecord(m->ev0, m->stream);
        if (e != hipSuccess) {
            s = cujev_raise(CUJEV_ERR_CUDA, "hipEventRecord: %s", hipGetErrorString(e));
            goto out;
        }
        int32_t *d_cand = NULL, *d_ncand = NULL;
        s = cujev_forward_with_candidates(m, st, CUJEV_FWD_EVAL, tok, N, seg_start, seg_len, B,
                                          cand, ncand, maxc, &d_cand, &d_ncand);
        if (s != CUJEV_OK)
            goto sync_out;
        if (maxc > 0) { /* the forward ran the readout into d_logits[B][maxc] */
            e = hipMemcpy2DAsync(logits_out, (size_t)ld * 4, m->d_logits, (size_t)maxc * 4,
                                 (size_t)maxc * 4, (size_t)B, hipMemcpyDeviceToHost, m->stream);
            if (e != hipSuccess) {
                s = cujev_raise(CUJEV_ERR_CUDA, "readout: %s", hipGetErrorString(e));
                goto sync_out;
            }
        }
        if ((e = hipEventRecord(m->ev1, m->stream)) != hipSuccess ||
            (e = hipStreamSynchronize(m->stream)) != hipSuccess) {
            s = cujev_raise(CUJEV_ERR_CUDA, "eval: %s", hipGetErrorString(e));
            goto out;
        }
        hipEventElapsedTime(&m->timing.eval_ms, m->ev0, m->ev1);
        m->timing.eval_tokens = N;
        m->timing.eval_branches = B;
        cujev_error_reset();
        goto out;
    }
sync_out:
    hipStreamSynchronize(m->stream);
out:
    free(tok);
    free(cand);
    free(seg);
    return s;
}

API cujev_status cujev_eval_full_logits(cujev_model *m, cujev_state *st, const cujev_branch *br,
                                        int B, float *logits_out) {
    CJ_CHECK(check_eval_args(m, st, br, B));
    if (!logits_out)
        return cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "logits_out is NULL");
    int32_t *seg = (int32_t *)malloc((size_t)B * 2 * 4);
    if (!seg)
        return cujev_raise(CUJEV_ERR_OOM, "segment table");
    int32_t *tok = NULL;
    int N = 0;
    const int V = m->cfg.vocab_size, H = m->cfg.hidden_size;
    cujev_status s = pack_branches(m, br, B, &tok, seg, seg + B, &N);
    if (s == CUJEV_OK) {
        hipEventRecord(m->ev0, m->stream);
        s = cujev_forward(m, st, CUJEV_FWD_EVAL, tok, N, seg, seg + B, B);
        hipError_t e = hipSuccess;
        if (s == CUJEV_OK) {
            e = k_gemm(m->gemm, m->hsel, m->lm_head, m->full_logits, 1, B, V, H, m->stream);
            if (e == hipSuccess)
                e = hipMemcpyAsync(logits_out, m->full_logits, (size_t)B * V * 4,
                                   hipMemcpyDeviceToHost, m->stream);
            if (e == hipSuccess)
                e = hipEventRecord(m->ev1, m->stream);
        }
        hipError_t e2 = hipStreamSynchronize(m->stream);
        if (s == CUJEV_OK && e == hipSuccess)
            e = e2;
        if (s == CUJEV_OK && e != hipSuccess)
            s = cujev_raise(CUJEV_ERR_CUDA, "full logits: %s", hipGetErrorString(e));
        if (s == CUJEV_OK) {
            hipEventElapsedTime(&m->timing.eval_ms, m->ev0, m->ev1);
            m->timing.eval_tokens = N;
            m->timing.eval_branches = B;
            cujev_error_reset();
        }
    }
    free(tok);
    free(seg);
    return s;
}

API void cujev_last_timing(const cujev_model *m, cujev_timing *out) {
    if (m && out)
        *out = m->timing;
}
