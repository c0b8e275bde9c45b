/* Weight upload and workspace sizing.
 *
 * Behaviour of REF src/engine/model.c:161-247 (which tensors, the "model." or
 * "model.language_model." prefix, tied embeddings, row-fused q|k|v, qkv|z|b|a
 * and gate|up, +1 on the zero-centred norms, A_neg_exp = -exp(A_log)) and
 * :249-313 (one workspace for the largest call). Matrices are uploaded
 * as bf16 (F16/F32 converted with round-to-nearest-even), vectors as fp32.
 * The weight and workspace slabs are sized by a planning pass of the same
 * code that carves them (core/devmem.h), so their sizes are exact. */
#include "engine/model.h"
#include "core/safetensors.h"
#include <math.h>

static float bf16_bits_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float f16_bits_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    int exp = (h >> 10) & 0x1f;
    uint32_t mant = h & 0x3ff, u;
    if (exp == 0x1f) {
        u = sign | 0x7f800000u | (mant << 13);
    } else if (exp == 0) {
        if (mant == 0) {
            u = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do {
                mant <<= 1;
                e++;
            } while (!(mant & 0x400));
            mant &= 0x3ff;
            u = sign | ((uint32_t)(127 - 15 - e) << 23) | (mant << 13);
        }
    } else {
        u = sign | ((uint32_t)(exp - 15 + 127) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint16_t f32_to_bf16_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) /* NaN stays NaN */
        return (uint16_t)((u >> 16) | 0x40);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

static float elem_f32(const st_tensor *t, size_t i) {
    switch (t->dtype) {
    case ST_F32: return ((const float *)t->data)[i];
    case ST_BF16: return bf16_bits_to_f32(((const uint16_t *)t->data)[i]);
    default: return f16_bits_to_f32(((const uint16_t *)t->data)[i]);
    }
}

/* One walk over the checkpoint's tensors. The walk runs twice: while the
 * weight slab is planning it only sizes the uploads, then it uploads. Names
 * are resolved inside a scope: the checkpoint's text-model prefix
 * ("model." or "model.language_model."), plus "layers.<l>." inside a layer. */
typedef struct loader {
    cujev_model *m;
    const st_bundle *b;
    const char *prefix;
    char scope[128];    /* prefix + current layer's "layers.<l>." */
    uint16_t *conv;     /* host staging for F16/F32 -> bf16 conversion */
    size_t conv_cap;
} loader;

static void scope_top(loader *L) { snprintf(L->scope, sizeof L->scope, "%s", L->prefix); }
static void scope_layer(loader *L, int layer) {
    snprintf(L->scope, sizeof L->scope, "%slayers.%d.", L->prefix, layer);
}

/* The tensor `leaf` of the current scope; FORMAT if absent, UNSUPPORTED if
 * its dtype is none of BF16 / F16 / F32. */
static cujev_status need(loader *L, const char *leaf, const st_tensor **out) {
    char full[256];
    snprintf(full, sizeof full, "%s%s", L->scope, leaf);
    const st_tensor *t = st_lookup(L->b, full);
    *out = t;
    if (!t)
        return cujev_raise(CUJEV_ERR_FORMAT, "checkpoint has no tensor %s", full);
    if (t->dtype == ST_OTHER)
        return cujev_raise(CUJEV_ERR_UNSUPPORTED, "tensor %s: dtype is not BF16/F16/F32", full);
    return CUJEV_OK;
}

static int planning(const loader *L) { return cujev_slab_planning(&L->m->weights); }

static void *take(loader *L, size_t bytes) { return cujev_slab_take(&L->m->weights, bytes); }

/* Row-concatenation of 2-D tensors [rows_i, K] -> one bf16 [sum rows, K]. */
/* The output projections (o_proj, out_proj, down_proj) write the residual:
 * their row count must be hidden_size, since the tiled copy and every GEMM on
 * them run over exactly H rows. */
static cujev_status need_rows(const st_tensor *t, int H, int layer) {
    if (t->ndim != 2 || t->shape[0] != H)
        return cujev_raise(CUJEV_ERR_FORMAT, "layer %d: tensor %s: expected [%d, *]", layer,
                           t->name, H);
    return CUJEV_OK;
}

static cujev_status upload_fused(loader *L, const st_tensor **parts, int nparts, int K,
                                 bf16_t **out) {
    size_t rows = 0;
    for (int i = 0; i < nparts; i++) {
        if (parts[i]->ndim != 2 || parts[i]->shape[1] != K)
            return cujev_raise(CUJEV_ERR_FORMAT, "tensor %s: expected [*, %d]", parts[i]->name, K);
        rows += (size_t)parts[i]->shape[0];
    }
    bf16_t *d = (bf16_t *)take(L, rows * (size_t)K * 2);
    if (planning(L))
        return CUJEV_OK;
    if (!d)
        return cujev_raise(CUJEV_ERR_OOM, "weight slab exhausted");
    size_t off = 0;
    for (int i = 0; i < nparts; i++) {
        const st_tensor *t = parts[i];
        const size_t n = t->numel;
        if (t->dtype == ST_BF16) {
            HIP_CHECK(hipMemcpy(d + off, t->data, n * 2, hipMemcpyHostToDevice));
        } else {
            const size_t step = (size_t)1 << 24;
            if (L->conv_cap < step) {
                free(L->conv);
                L->conv = (uint16_t *)malloc(step * 2);
                if (!L->conv)
                    return cujev_raise(CUJEV_ERR_OOM, "host conversion buffer");
                L->conv_cap = step;
            }
            for (size_t s = 0; s < n; s += step) {
                const size_t c = n - s < step ? n - s : step;
                for (size_t j = 0; j < c; j++)
                    L->conv[j] = f32_to_bf16_bits(elem_f32(t, s + j));
                HIP_CHECK(hipMemcpy(d + off + s, L->conv, c * 2, hipMemcpyHostToDevice));
            }
        }
        off += n;
    }
    *out = d;
    return CUJEV_OK;
}

/* Small fp32 vector, optionally +add or -exp(x). */
/* The tiled copy of an uploaded projection that the few-token GEMM streams
 * (one contiguous 4 KiB block per 16 rows x 128 k), for the shapes it
 * supports; *out stays NULL otherwise. */
static cujev_status upload_tiled(loader *L, const bf16_t *w, int M, int K, bf16_t **out) {
    *out = NULL;
    if (cujev_gemm_small_splits(M, K) <= 0)
        return CUJEV_OK;
    bf16_t *d = (bf16_t *)take(L, (size_t)M * K * 2);
    if (planning(L))
        return CUJEV_OK;
    if (!d)
        return cujev_raise(CUJEV_ERR_OOM, "weight slab exhausted");
    HIP_CHECK(k_gemm_small_tile(w, M, K, d, L->m->stream));
    *out = d;
    return CUJEV_OK;
}

static cujev_status upload_f32(loader *L, const st_tensor *t, float add, int negexp, size_t expect,
                               float **out) {
    const size_t n = t->numel;
    if (expect && n != expect)
        return cujev_raise(CUJEV_ERR_FORMAT, "tensor %s: %zu elements, expected %zu", t->name, n,
                          expect);
    float *d = (float *)take(L, n * 4);
    if (planning(L))
        return CUJEV_OK;
    if (!d)
        return cujev_raise(CUJEV_ERR_OOM, "weight slab exhausted");
    float *h = (float *)malloc(n * 4);
    if (!h)
        return cujev_raise(CUJEV_ERR_OOM, "host vector");
    for (size_t i = 0; i < n; i++) {
        const float v = elem_f32(t, i);
        h[i] = negexp ? -expf(v) : v + add;
    }
    hipError_t e = hipMemcpy(d, h, n * 4, hipMemcpyHostToDevice);
    free(h);
    if (e != hipSuccess)
        return cujev_raise(CUJEV_ERR_CUDA, "hipMemcpy: %s", hipGetErrorString(e));
    *out = d;
    return CUJEV_OK;
}

static cujev_status walk(loader *L) {
    cujev_model *m = L->m;
    const cujev_config *c = &m->cfg;
    const int H = c->hidden_size;
    const st_tensor *t, *parts[4];
    scope_top(L);
    CJ_CHECK(need(L, "embed_tokens.weight", &t));
    if (t->ndim != 2 || t->shape[0] != c->vocab_size || t->shape[1] != H)
        return cujev_raise(CUJEV_ERR_FORMAT, "embed_tokens shape mismatch");
    CJ_CHECK(upload_fused(L, &t, 1, H, &m->embed));
    m->lm_head = m->embed;
    if (!c->tie_word_embeddings) {
        const st_tensor *lm = st_lookup(L->b, "lm_head.weight"); /* outside the prefix */
        if (!lm)
            return cujev_raise(CUJEV_ERR_FORMAT,
                              "tie_word_embeddings is false but lm_head.weight is missing");
        if (lm->ndim != 2 || lm->shape[0] != c->vocab_size)
            return cujev_raise(CUJEV_ERR_FORMAT, "lm_head shape mismatch");
        CJ_CHECK(upload_fused(L, &lm, 1, H, &m->lm_head));
    }
    CJ_CHECK(need(L, "norm.weight", &t));
    CJ_CHECK(upload_f32(L, t, 1.f, 0, (size_t)H, &m->final_norm));
    for (int l = 0; l < c->num_layers; l++) {
        cujev_layer *ly = &m->layers[l];
        ly->type = c->layer_types[l];
        scope_layer(L, l);
        CJ_CHECK(need(L, "input_layernorm.weight", &t));
        CJ_CHECK(upload_f32(L, t, 1.f, 0, (size_t)H, &ly->in_norm));
        CJ_CHECK(need(L, "post_attention_layernorm.weight", &t));
        CJ_CHECK(upload_f32(L, t, 1.f, 0, (size_t)H, &ly->post_norm));
        if (ly->type == CUJEV_LAYER_FULL) {
            CJ_CHECK(need(L, "self_attn.q_proj.weight", &parts[0]));
            CJ_CHECK(need(L, "self_attn.k_proj.weight", &parts[1]));
            CJ_CHECK(need(L, "self_attn.v_proj.weight", &parts[2]));
            if (parts[0]->shape[0] != (int64_t)m->Hq * 2 * m->D ||
                parts[1]->shape[0] != (int64_t)m->Hkv * m->D ||
                parts[2]->shape[0] != (int64_t)m->Hkv * m->D)
                return cujev_raise(CUJEV_ERR_FORMAT, "layer %d: attention projection shapes", l);
            CJ_CHECK(upload_fused(L, parts, 3, H, &ly->w_qkv));
            CJ_CHECK(upload_tiled(L, ly->w_qkv, m->w_attn, H, &ly->wt_qkv));
            CJ_CHECK(need(L, "self_attn.o_proj.weight", &t));
            CJ_CHECK(need_rows(t, H, l));
            CJ_CHECK(upload_fused(L, &t, 1, m->Hq * m->D, &ly->w_o));
            CJ_CHECK(upload_tiled(L, ly->w_o, H, m->Hq * m->D, &ly->wt_o));
            CJ_CHECK(need(L, "self_attn.q_norm.weight", &t));
            CJ_CHECK(upload_f32(L, t, 1.f, 0, (size_t)m->D, &ly->q_norm));
            CJ_CHECK(need(L, "self_attn.k_norm.weight", &t));
            CJ_CHECK(upload_f32(L, t, 1.f, 0, (size_t)m->D, &ly->k_norm));
        } else {
            CJ_CHECK(need(L, "linear_attn.in_proj_qkv.weight", &parts[0]));
            CJ_CHECK(need(L, "linear_attn.in_proj_z.weight", &parts[1]));
            CJ_CHECK(need(L, "linear_attn.in_proj_b.weight", &parts[2]));
            CJ_CHECK(need(L, "linear_attn.in_proj_a.weight", &parts[3]));
            if (parts[0]->shape[0] != m->C || parts[1]->shape[0] != m->V ||
                parts[2]->shape[0] != m->Hv || parts[3]->shape[0] != m->Hv)
                return cujev_raise(CUJEV_ERR_FORMAT, "layer %d: GDN projection shapes", l);
            CJ_CHECK(upload_fused(L, parts, 4, H, &ly->w_in));
            CJ_CHECK(upload_tiled(L, ly->w_in, m->w_gdn, H, &ly->wt_in));
            CJ_CHECK(need(L, "linear_attn.out_proj.weight", &t));
            CJ_CHECK(need_rows(t, H, l));
            CJ_CHECK(upload_fused(L, &t, 1, m->V, &ly->w_out));
            CJ_CHECK(upload_tiled(L, ly->w_out, H, m->V, &ly->wt_out));
            CJ_CHECK(need(L, "linear_attn.conv1d.weight", &t));
            CJ_CHECK(upload_f32(L, t, 0.f, 0, (size_t)m->C * 4, &ly->conv_w));
            CJ_CHECK(need(L, "linear_attn.A_log", &t));
            CJ_CHECK(upload_f32(L, t, 0.f, 1, (size_t)m->Hv, &ly->A_neg_exp));
            CJ_CHECK(need(L, "linear_attn.dt_bias", &t));
            CJ_CHECK(upload_f32(L, t, 0.f, 0, (size_t)m->Hv, &ly->dt_bias));
            CJ_CHECK(need(L, "linear_attn.norm.weight", &t));
            CJ_CHECK(upload_f32(L, t, 0.f, 0, 128, &ly->g_norm));
        }
        CJ_CHECK(need(L, "mlp.gate_proj.weight", &parts[0]));
        CJ_CHECK(need(L, "mlp.up_proj.weight", &parts[1]));
        if (parts[0]->shape[0] != c->intermediate_size || parts[1]->shape[0] != c->intermediate_size)
            return cujev_raise(CUJEV_ERR_FORMAT, "layer %d: MLP shapes", l);
        CJ_CHECK(upload_fused(L, parts, 2, H, &ly->w_gate_up));
        CJ_CHECK(upload_tiled(L, ly->w_gate_up, 2 * c->intermediate_size, H, &ly->wt_gate_up));
        CJ_CHECK(need(L, "mlp.down_proj.weight", &t));
        CJ_CHECK(need_rows(t, H, l));
        CJ_CHECK(upload_fused(L, &t, 1, c->intermediate_size, &ly->w_down));
        CJ_CHECK(upload_tiled(L, ly->w_down, H, c->intermediate_size, &ly->wt_down));
    }
    return CUJEV_OK;
}

cujev_status cujev_model_load_weights(cujev_model *m, const char *dir) {
    st_bundle b;
    CJ_CHECK(st_bundle_open(dir, &b));
    loader L;
    memset(&L, 0, sizeof L);
    L.m = m;
    L.b = &b;
    L.prefix = st_lookup(&b, "model.language_model.embed_tokens.weight") ? "model.language_model."
                                                                          : "model.";
    cujev_status s = walk(&L); /* planning pass: sizes only */
    if (s == CUJEV_OK) {
        cujev_note(m->opts.verbose, "weights: %.2f GiB from %d tensors in %d shard(s)",
                   m->weights.planned / 1073741824.0, b.num_tensors, b.num_files);
        s = cujev_slab_commit(&m->weights, "weights");
    }
    if (s == CUJEV_OK)
        s = walk(&L); /* upload pass */
    if (s == CUJEV_OK && hipStreamSynchronize(m->stream) != hipSuccess) /* the tiling kernels */
        s = cujev_raise(CUJEV_ERR_CUDA, "weight tiling failed");
    free(L.conv);
    st_bundle_release(&b);
    return s;
}

cujev_status cujev_model_alloc_workspace(cujev_model *m) {
    const cujev_config *c = &m->cfg;
    const size_t N = (size_t)m->max_tokens, H = (size_t)c->hidden_size,
                 I = (size_t)c->intermediate_size;
    const size_t B = (size_t)(m->opts.max_branches > 0 ? m->opts.max_branches : 1);
    const size_t mixw = (size_t)((m->Hq * m->D > m->V) ? m->Hq * m->D : m->V);
    const size_t mix = N * mixw;
    const size_t br_kv = (size_t)m->Hkv * m->branch_stride * m->D * 2;
    m->max_chunks = m->max_tokens / 64 + (int)B + 1;
    /* + 8: a FUSED call's second (one-segment) chunk table heads */
    m->meta_ints = 3 * N + 3 * B + 4 * (size_t)m->max_chunks + B * (size_t)m->opts.max_candidates + B + 8;
    m->gemm_ws_bytes = (size_t)64 << 20;
    m->attn_ws_bytes = cujev_attention_ws_max(m->max_tokens, m->Hq, m->Hkv);
    /* split-K partials: the few-token GEMM's at most 8 splits of 96 tokens,
     * and 64 MiB (or what 8 splits of all N tokens need, if less) for the
     * prefill GEMM, which fits its split count to it */
    {
        const size_t small = (size_t)CUJEV_GEMM_SMALL_MAX_SPLITS * CUJEV_GEMM_SMALL_MAX_N * H * 4;
        size_t wide = (size_t)64 << 20;
        if (wide > 8 * N * H * 4)
            wide = 8 * N * H * 4;
        m->ypart_bytes = small > wide ? small : wide;
    }
    struct {
        void **p;
        size_t bytes;
    } parts[] = {
        {(void **)&m->x, N * H * 4},
        {(void **)&m->xb, N * H * 2},
        {(void **)&m->proj, N * (size_t)m->w_proj * 2},
        {(void **)&m->y, N * H * 2},
        {(void **)&m->ypart, m->ypart_bytes},
        {&m->attn_ws, m->attn_ws_bytes},
        {(void **)&m->q, N * (size_t)m->Hq * m->D * 2},
        {(void **)&m->mix_out, mix * 2},
        {(void **)&m->br_k, br_kv},
        {(void **)&m->br_vt, br_kv},
        /* + 4 KiB: a FUSED call carves the chunk arrays of its two token
         * groups apart, each rounded up on its own */
        {(void **)&m->gdn_scratch,
         cujev_gdn_scratch_bytes(m->max_chunks, m->Hv, m->max_tokens) + 4096},
        {(void **)&m->act, N * I * 2},
        {(void **)&m->hsel, B * H * 2},
        {(void **)&m->xl, B * H * 4},
        {(void **)&m->mixl, B * mixw * 2},
        {(void **)&m->full_logits, B * (size_t)c->vocab_size * 4},
        {(void **)&m->gemm_ws, m->gemm_ws_bytes},
        {(void **)&m->d_meta, m->meta_ints * 4},
        {(void **)&m->d_logits, B * (size_t)(m->opts.max_candidates > 0 ? m->opts.max_candidates : 1) * 4},
        {(void **)&m->rope, (size_t)m->rope_positions * c->rotary_dim * 4},
    };
    const int np = (int)(sizeof parts / sizeof parts[0]);
    for (int i = 0; i < np; i++) /* planning pass */
        cujev_slab_take(&m->work, parts[i].bytes);
    CJ_CHECK(cujev_slab_commit(&m->work, "workspace"));
    for (int i = 0; i < np; i++) {
        *parts[i].p = cujev_slab_take(&m->work, parts[i].bytes);
        if (!*parts[i].p)
            return cujev_raise(CUJEV_ERR_OOM, "workspace slab undersized");
    }
    /* Branch K/V scratch must hold finite values everywhere: 64-key tiles read
     * past the valid keys (masked to p = 0, and 0 * NaN would be NaN). */
    HIP_CHECK(hipMemset(m->br_k, 0, br_kv));
    HIP_CHECK(hipMemset(m->br_vt, 0, br_kv));
    HIP_CHECK(hipHostMalloc((void **)&m->h_meta, m->meta_ints * 4, hipHostMallocDefault));
    {
        const size_t rb = (size_t)m->rope_positions * c->rotary_dim * 4;
        float *h = (float *)malloc(rb);
        if (!h)
            return cujev_raise(CUJEV_ERR_OOM, "RoPE table");
        cujev_rope_table_host(c->rope_theta, c->rotary_dim, m->rope_positions, h);
        hipError_t e = hipMemcpy(m->rope, h, rb, hipMemcpyHostToDevice);
        free(h);
        if (e != hipSuccess)
            return cujev_raise(CUJEV_ERR_CUDA, "RoPE table upload: %s", hipGetErrorString(e));
    }
    cujev_note(m->opts.verbose, "workspace: %.2f GiB for %zu tokens, %zu branches",
              cujev_slab_used(&m->work) / 1073741824.0, N, B);
    return CUJEV_OK;
}
