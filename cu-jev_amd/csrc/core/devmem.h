/* Planned device slabs: one hipMalloc per lifetime object (the model's
 * weights, its workspace, one state), sized by a planning pass over the very
 * code that later carves it, so the size is exact by construction.
 *
 *   cujev_slab s = {0};                 planning mode
 *   walk(&s);                           every cujev_slab_take() returns NULL
 *                                       and only adds its request to the plan
 *   cujev_slab_commit(&s, "weights");   one hipMalloc of the planned bytes
 *   walk(&s);                           the same takes now return the pieces,
 *                                       in order, each 256-byte aligned
 *   cujev_slab_release(&s);
 *
 * Pieces start on 256-byte boundaries: 16-byte vector accesses and the
 * buffer-load descriptors of the kernels need at least that, and whole
 * 256-byte lines keep every piece's first and last lines private to it. */
#ifndef CUJEV_DEVMEM_H
#define CUJEV_DEVMEM_H

#include "core/status.h"

#ifdef __cplusplus
extern "C" {
#endif

#define CUJEV_SLAB_ALIGN 256

typedef struct cujev_slab {
    unsigned char *base; /* NULL while planning */
    size_t planned;      /* bytes the planning pass asked for */
    size_t cursor;       /* bytes carved so far (after commit) */
} cujev_slab;

static inline int cujev_slab_planning(const cujev_slab *s) { return s->base == NULL; }

/* Planning: records `bytes`, returns NULL. Carving: the next piece, or NULL
 * when the carving pass asks for more than was planned. */
void *cujev_slab_take(cujev_slab *s, size_t bytes);
/* Allocates the planned bytes (CUJEV_ERR_OOM with `what` in the message on
 * failure); the slab then carves from its start. */
cujev_status cujev_slab_commit(cujev_slab *s, const char *what);
/* Bytes handed out by the carving pass (0 while planning). */
static inline size_t cujev_slab_used(const cujev_slab *s) { return s->base ? s->cursor : 0; }
void cujev_slab_release(cujev_slab *s);

#ifdef __cplusplus
}
#endif
#endif
