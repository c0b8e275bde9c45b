#include "core/json.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* Nodes and strings come from a list of big blocks freed together. */
typedef struct js_block {
    struct js_block *prev;
    size_t used, cap;
    char data[];
} js_block;

struct js_doc {
    js_block *blocks;
    js_node *root;
};

typedef struct {
    const char *p, *end;
    js_doc *doc;
    char *err;
    size_t errlen;
    int depth;
} js_parser;

static void *js_alloc(js_doc *d, size_t n) {
    n = (n + 15) & ~(size_t)15;
    if (!d->blocks || d->blocks->used + n > d->blocks->cap) {
        size_t cap = n > (1u << 16) ? n : (1u << 16);
        js_block *b = (js_block *)malloc(sizeof(js_block) + cap);
        if (!b)
            return NULL;
        b->prev = d->blocks;
        b->used = 0;
        b->cap = cap;
        d->blocks = b;
    }
    void *r = d->blocks->data + d->blocks->used;
    d->blocks->used += n;
    return r;
}

static int fail(js_parser *P, const char *msg) {
    if (P->err && P->errlen)
        snprintf(P->err, P->errlen, "JSON: %s at byte %ld", msg, (long)(P->end - P->p));
    return 0;
}

static void skip_ws(js_parser *P) {
    while (P->p < P->end && (*P->p == ' ' || *P->p == '\t' || *P->p == '\n' || *P->p == '\r'))
        P->p++;
}

static int hexval(char c) {
    if (c >= '0' && c <= '9')
        return c - '0';
    if (c >= 'a' && c <= 'f')
        return c - 'a' + 10;
    if (c >= 'A' && c <= 'F')
        return c - 'A' + 10;
    return -1;
}

static int put_utf8(char *o, unsigned cp) {
    if (cp < 0x80) {
        o[0] = (char)cp;
        return 1;
    }
    if (cp < 0x800) {
        o[0] = (char)(0xC0 | (cp >> 6));
        o[1] = (char)(0x80 | (cp & 0x3F));
        return 2;
    }
    if (cp < 0x10000) {
        o[0] = (char)(0xE0 | (cp >> 12));
        o[1] = (char)(0x80 | ((cp >> 6) & 0x3F));
        o[2] = (char)(0x80 | (cp & 0x3F));
        return 3;
    }
    o[0] = (char)(0xF0 | (cp >> 18));
    o[1] = (char)(0x80 | ((cp >> 12) & 0x3F));
    o[2] = (char)(0x80 | ((cp >> 6) & 0x3F));
    o[3] = (char)(0x80 | (cp & 0x3F));
    return 4;
}

static int read_hex4(js_parser *P, unsigned *cp) {
    if (P->end - P->p < 4)
        return 0;
    unsigned v = 0;
    for (int i = 0; i < 4; i++) {
        int h = hexval(P->p[i]);
        if (h < 0)
            return 0;
        v = v * 16 + (unsigned)h;
    }
    P->p += 4;
    *cp = v;
    return 1;
}

/* Parses a string starting at the opening quote. */
static int parse_string(js_parser *P, const char **out) {
    P->p++; /* opening quote */
    const char *s = P->p;
    size_t raw = 0;
    while (s < P->end && *s != '"') {
        if (*s == '\\')
            s++;
        s++;
        raw++;
    }
    if (s >= P->end)
        return fail(P, "unterminated string");
    /* unescaped length <= raw bytes scanned * 4 (\\u escapes expand at most to 4) */
    char *o = (char *)js_alloc(P->doc, (size_t)(s - P->p) + 1);
    if (!o)
        return fail(P, "out of memory");
    char *w = o;
    while (*P->p != '"') {
        char c = *P->p++;
        if ((unsigned char)c < 0x20)
            return fail(P, "control character in string");
        if (c != '\\') {
            *w++ = c;
            continue;
        }
        if (P->p >= P->end)
            return fail(P, "bad escape");
        char e = *P->p++;
        switch (e) {
        case '"': *w++ = '"'; break;
        case '\\': *w++ = '\\'; break;
        case '/': *w++ = '/'; break;
        case 'b': *w++ = '\b'; break;
        case 'f': *w++ = '\f'; break;
        case 'n': *w++ = '\n'; break;
        case 'r': *w++ = '\r'; break;
        case 't': *w++ = '\t'; break;
        case 'u': {
            unsigned cp;
            if (!read_hex4(P, &cp))
                return fail(P, "bad \\u escape");
            if (cp >= 0xD800 && cp < 0xDC00) { /* surrogate pair */
                unsigned lo;
                if (P->end - P->p < 6 || P->p[0] != '\\' || P->p[1] != 'u')
                    return fail(P, "lone surrogate");
                P->p += 2;
                if (!read_hex4(P, &lo) || lo < 0xDC00 || lo >= 0xE000)
                    return fail(P, "bad surrogate pair");
                cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
            }
            w += put_utf8(w, cp);
            break;
        }
        default:
            return fail(P, "bad escape");
        }
    }
    P->p++; /* closing quote */
    *w = 0;
    *out = o;
    (void)raw;
    return 1;
}

static int parse_value(js_parser *P, js_node *n);

static int parse_number(js_parser *P, js_node *n) {
    const char *s = P->p;
    if (s < P->end && *s == '-')
        s++;
    if (s >= P->end || !((*s >= '0' && *s <= '9')))
        return fail(P, "bad number");
    while (s < P->end && ((*s >= '0' && *s <= '9') || *s == '.' || *s == 'e' || *s == 'E' ||
                          *s == '+' || *s == '-'))
        s++;
    char buf[64];
    size_t L = (size_t)(s - P->p);
    if (L >= sizeof buf)
        return fail(P, "number too long");
    memcpy(buf, P->p, L);
    buf[L] = 0;
    char *endp;
    n->num = strtod(buf, &endp);
    if (endp != buf + L)
        return fail(P, "bad number");
    n->type = JS_NUM;
    P->p = s;
    return 1;
}

static int literal(js_parser *P, const char *word) {
    size_t L = strlen(word);
    if ((size_t)(P->end - P->p) < L || memcmp(P->p, word, L) != 0)
        return 0;
    P->p += L;
    return 1;
}

static int parse_container(js_parser *P, js_node *n, int is_obj) {
    if (++P->depth > 64)
        return fail(P, "nesting too deep");
    P->p++; /* [ or { */
    n->type = is_obj ? JS_OBJ : JS_ARR;
    js_node **tail = &n->child;
    skip_ws(P);
    if (P->p < P->end && *P->p == (is_obj ? '}' : ']')) {
        P->p++;
        P->depth--;
        return 1;
    }
    for (;;) {
        js_node *c = (js_node *)js_alloc(P->doc, sizeof(js_node));
        if (!c)
            return fail(P, "out of memory");
        memset(c, 0, sizeof *c);
        skip_ws(P);
        if (is_obj) {
            if (P->p >= P->end || *P->p != '"')
                return fail(P, "expected member name");
            if (!parse_string(P, &c->key))
                return 0;
            skip_ws(P);
            if (P->p >= P->end || *P->p != ':')
                return fail(P, "expected ':'");
            P->p++;
        }
        if (!parse_value(P, c))
            return 0;
        *tail = c;
        tail = &c->next;
        n->count++;
        skip_ws(P);
        if (P->p < P->end && *P->p == ',') {
            P->p++;
            continue;
        }
        if (P->p < P->end && *P->p == (is_obj ? '}' : ']')) {
            P->p++;
            break;
        }
        return fail(P, is_obj ? "expected ',' or '}'" : "expected ',' or ']'");
    }
    P->depth--;
    return 1;
}

static int parse_value(js_parser *P, js_node *n) {
    skip_ws(P);
    if (P->p >= P->end)
        return fail(P, "unexpected end");
    switch (*P->p) {
    case '{': return parse_container(P, n, 1);
    case '[': return parse_container(P, n, 0);
    case '"': n->type = JS_STR; return parse_string(P, &n->str);
    case 't':
        if (!literal(P, "true"))
            return fail(P, "bad literal");
        n->type = JS_BOOL;
        n->boolean = 1;
        return 1;
    case 'f':
        if (!literal(P, "false"))
            return fail(P, "bad literal");
        n->type = JS_BOOL;
        return 1;
    case 'n':
        if (!literal(P, "null"))
            return fail(P, "bad literal");
        n->type = JS_NULL;
        return 1;
    default: return parse_number(P, n);
    }
}

js_doc *js_parse(const char *text, size_t len, char *err, size_t errlen) {
    js_doc *d = (js_doc *)calloc(1, sizeof *d);
    if (!d)
        return NULL;
    js_parser P = {text, text + len, d, err, errlen, 0};
    js_node *root = (js_node *)js_alloc(d, sizeof(js_node));
    if (!root) {
        js_free(d);
        return NULL;
    }
    memset(root, 0, sizeof *root);
    if (!parse_value(&P, root)) {
        js_free(d);
        return NULL;
    }
    skip_ws(&P);
    while (P.p < P.end && *P.p == 0) /* tolerate NUL padding */
        P.p++;
    skip_ws(&P);
    if (P.p != P.end) {
        fail(&P, "trailing characters");
        js_free(d);
        return NULL;
    }
    d->root = root;
    return d;
}

const js_node *js_root(const js_doc *d) { return d ? d->root : NULL; }

void js_free(js_doc *d) {
    if (!d)
        return;
    js_block *b = d->blocks;
    while (b) {
        js_block *p = b->prev;
        free(b);
        b = p;
    }
    free(d);
}

const js_node *js_get(const js_node *obj, const char *key) {
    if (!obj || obj->type != JS_OBJ)
        return NULL;
    for (const js_node *c = obj->child; c; c = c->next)
        if (strcmp(c->key, key) == 0)
            return c;
    return NULL;
}

const js_node *js_at(const js_node *arr, int i) {
    if (!arr || arr->type != JS_ARR || i < 0)
        return NULL;
    const js_node *c = arr->child;
    while (c && i--)
        c = c->next;
    return c;
}

int js_is(const js_node *n, js_type t) { return n && n->type == t; }
