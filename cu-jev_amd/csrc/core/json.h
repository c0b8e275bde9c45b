/* Minimal JSON reader for config.json and safetensors headers (the reference
 * vendors cJSON for this; this is an independent recursive-descent parser).
 * The whole document becomes one tree allocated from a single block. */
#ifndef CUJEV_JSON_H
#define CUJEV_JSON_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum { JS_NULL, JS_BOOL, JS_NUM, JS_STR, JS_ARR, JS_OBJ } js_type;

typedef struct js_node {
    js_type type;
    int boolean;
    double num;
    const char *str;       /* JS_STR: NUL-terminated, unescaped (UTF-8) */
    const char *key;       /* member name when the parent is an object */
    struct js_node *child; /* first element / member */
    struct js_node *next;  /* next sibling */
    int count;             /* number of children */
} js_node;

typedef struct js_doc js_doc;

/* Parse `len` bytes. Returns NULL on error and writes a message to err. */
js_doc *js_parse(const char *text, size_t len, char *err, size_t errlen);
const js_node *js_root(const js_doc *d);
void js_free(js_doc *d);

const js_node *js_get(const js_node *obj, const char *key); /* NULL if absent */
const js_node *js_at(const js_node *arr, int i);
int js_is(const js_node *n, js_type t);

#ifdef __cplusplus
}
#endif
#endif
