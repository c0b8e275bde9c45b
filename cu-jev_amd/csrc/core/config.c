/* config.json -> cujev_config. Behaviour of REF src/core/config.c:42-144:
 * "text_config" if present (multimodal checkpoints) else the top level;
 * model_type must start with "qwen3_5"; RoPE from "rope_parameters" or the top
 * level (theta 10000, partial factor 1 by default); layer_types required; the
 * kernels' specialisations (k = v = 128, head_dim 256, rotary 64, 4 q-heads
 * per kv-head, conv 4) are enforced here, before any device call. */
#include "core/config.h"
#include "core/json.h"
#include "core/devmem.h"

static int geti(const js_node *o, const char *k, int dflt) {
    const js_node *v = js_get(o, k);
    return js_is(v, JS_NUM) ? (int)v->num : dflt;
}
static double getd(const js_node *o, const char *k, double dflt) {
    const js_node *v = js_get(o, k);
    return js_is(v, JS_NUM) ? v->num : dflt;
}
static int getb(const js_node *o, const char *k, int dflt) {
    const js_node *v = js_get(o, k);
    return js_is(v, JS_BOOL) ? v->boolean : dflt;
}

cujev_status cujev_config_parse(const char *text, size_t len, const char *what, cujev_config *c) {
    char err[256];
    js_doc *doc = js_parse(text, len, err, sizeof err);
    if (!doc)
        return cujev_raise(CUJEV_ERR_FORMAT, "%s: invalid JSON (%s)", what, err);
    const js_node *root = js_root(doc);
    const js_node *t = js_get(root, "text_config");
    if (!js_is(t, JS_OBJ))
        t = root;
    memset(c, 0, sizeof *c);
    cujev_status st = CUJEV_OK;

    const js_node *mt = js_get(t, "model_type");
    if (!js_is(mt, JS_STR) || strncmp(mt->str, "qwen3_5", 7) != 0) {
        st = cujev_raise(CUJEV_ERR_UNSUPPORTED, "model_type %s is not qwen3_5",
                        js_is(mt, JS_STR) ? mt->str : "(missing)");
        goto done;
    }
    c->hidden_size = geti(t, "hidden_size", 0);
    c->intermediate_size = geti(t, "intermediate_size", 0);
    c->num_layers = geti(t, "num_hidden_layers", 0);
    c->vocab_size = geti(t, "vocab_size", 0);
    c->rms_norm_eps = (float)getd(t, "rms_norm_eps", 1e-6);
    c->tie_word_embeddings = getb(t, "tie_word_embeddings", getb(root, "tie_word_embeddings", 0));
    c->num_heads = geti(t, "num_attention_heads", 0);
    c->num_kv_heads = geti(t, "num_key_value_heads", 0);
    c->head_dim = geti(t, "head_dim", c->hidden_size / (c->num_heads ? c->num_heads : 1));
    c->lin_num_k_heads = geti(t, "linear_num_key_heads", 0);
    c->lin_num_v_heads = geti(t, "linear_num_value_heads", 0);
    c->lin_k_dim = geti(t, "linear_key_head_dim", 0);
    c->lin_v_dim = geti(t, "linear_value_head_dim", 0);
    c->lin_conv_kernel = geti(t, "linear_conv_kernel_dim", 4);
    {
        const js_node *rp = js_get(t, "rope_parameters");
        const js_node *src = js_is(rp, JS_OBJ) ? rp : t;
        c->rope_theta = getd(src, "rope_theta", 10000.0);
        c->rotary_dim = (int)(c->head_dim * getd(src, "partial_rotary_factor", 1.0));
    }
    {
        const js_node *lt = js_get(t, "layer_types");
        if (!js_is(lt, JS_ARR) || lt->count != c->num_layers || c->num_layers > CUJEV_MAX_LAYERS) {
            st = cujev_raise(CUJEV_ERR_FORMAT, "%s: layer_types missing or wrong length", what);
            goto done;
        }
        int i = 0;
        for (const js_node *e = lt->child; e; e = e->next, i++) {
            if (!js_is(e, JS_STR)) {
                st = cujev_raise(CUJEV_ERR_FORMAT, "%s: layer_types[%d] is not a string", what, i);
                goto done;
            }
            if (strcmp(e->str, "full_attention") == 0) {
                c->layer_types[i] = CUJEV_LAYER_FULL;
                c->num_full_layers++;
            } else if (strcmp(e->str, "linear_attention") == 0) {
                c->layer_types[i] = CUJEV_LAYER_LINEAR;
                c->num_linear_layers++;
            } else {
                st = cujev_raise(CUJEV_ERR_UNSUPPORTED, "layer type %s", e->str);
                goto done;
            }
        }
    }
    if (c->hidden_size <= 0 || c->num_layers <= 0 || c->vocab_size <= 0 || c->num_heads <= 0 ||
        c->num_kv_heads <= 0 || c->lin_num_v_heads <= 0 || c->lin_num_k_heads <= 0 ||
        c->intermediate_size <= 0) {
        st = cujev_raise(CUJEV_ERR_FORMAT, "%s: missing required fields", what);
        goto done;
    }
    if (c->lin_num_v_heads % c->lin_num_k_heads != 0 || c->num_heads % c->num_kv_heads != 0) {
        st = cujev_raise(CUJEV_ERR_UNSUPPORTED, "head counts must divide");
        goto done;
    }
    if (c->lin_k_dim != 128 || c->lin_v_dim != 128 || c->head_dim != 256 || c->rotary_dim != 64) {
        st = cujev_raise(CUJEV_ERR_UNSUPPORTED,
                        "kernels are specialised for k=v=128, head_dim=256, rotary=64 "
                        "(got %d/%d/%d/%d)",
                        c->lin_k_dim, c->lin_v_dim, c->head_dim, c->rotary_dim);
        goto done;
    }
    if (c->num_heads / c->num_kv_heads != 4) {
        st = cujev_raise(CUJEV_ERR_UNSUPPORTED,
                        "attention kernel needs 4 q-heads per kv-head (got %d)",
                        c->num_heads / c->num_kv_heads);
        goto done;
    }
    if (c->lin_conv_kernel != 4) {
        st = cujev_raise(CUJEV_ERR_UNSUPPORTED, "conv kernel %d (need 4)", c->lin_conv_kernel);
        goto done;
    }
    if (c->hidden_size % 8 || c->intermediate_size % 4 || c->hidden_size > 16384) {
        st = cujev_raise(CUJEV_ERR_UNSUPPORTED, "hidden %d / intermediate %d not supported",
                        c->hidden_size, c->intermediate_size);
        goto done;
    }
    {
        const char *size = c->hidden_size == 1024   ? "0.8B"
                           : c->hidden_size == 2048 ? "2B"
                           : c->hidden_size == 2560 ? "4B"
                           : c->hidden_size == 4096 ? "9B"
                           : c->hidden_size == 5120 ? "27B"
                                                    : NULL;
        if (size)
            snprintf(c->name, sizeof c->name, "Qwen3.5-%s", size);
        else
            snprintf(c->name, sizeof c->name, "Qwen3.5-h%d-L%d", c->hidden_size, c->num_layers);
    }
done:
    js_free(doc);
    return st;
}

cujev_status cujev_config_load(const char *dir, cujev_config *c) {
    char path[4096];
    snprintf(path, sizeof path, "%s/config.json", dir);
    FILE *f = fopen(path, "rb");
    if (!f)
        return cujev_raise(CUJEV_ERR_IO, "cannot read %s", path);
    fseek(f, 0, SEEK_END);
    long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    if (n < 0) {
        fclose(f);
        return cujev_raise(CUJEV_ERR_IO, "cannot read %s", path);
    }
    char *buf = (char *)malloc((size_t)n + 1);
    if (!buf) {
        fclose(f);
        return cujev_raise(CUJEV_ERR_OOM, "config buffer");
    }
    size_t got = fread(buf, 1, (size_t)n, f);
    fclose(f);
    if (got != (size_t)n) {
        free(buf);
        return cujev_raise(CUJEV_ERR_IO, "short read of %s", path);
    }
    buf[n] = 0;
    cujev_status s = cujev_config_parse(buf, (size_t)n, path, c);
    free(buf);
    return s;
}
