/* Planned device slabs (see devmem.h). */
#include "core/devmem.h"
#include <hip/hip_runtime_api.h>

void *cujev_slab_take(cujev_slab *s, size_t bytes) {
    const size_t piece = cujev_round_up(bytes ? bytes : 1, CUJEV_SLAB_ALIGN);
    if (!s->base) {
        s->planned += piece;
        return NULL;
    }
    if (piece > s->planned - s->cursor)
        return NULL;
    void *p = s->base + s->cursor;
    s->cursor += piece;
    return p;
}

cujev_status cujev_slab_commit(cujev_slab *s, const char *what) {
    if (s->base)
        return cujev_raise(CUJEV_ERR_INVALID_ARGUMENT, "%s: slab committed twice", what);
    void *p = NULL;
    const size_t bytes = s->planned ? s->planned : CUJEV_SLAB_ALIGN;
    const hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess || !p)
        return cujev_raise(CUJEV_ERR_OOM, "%s: %zu bytes of device memory: %s", what, bytes,
                           hipGetErrorString(e));
    s->base = (unsigned char *)p;
    s->planned = bytes;
    s->cursor = 0;
    return CUJEV_OK;
}

void cujev_slab_release(cujev_slab *s) {
    if (s->base)
        hipFree(s->base);
    s->base = NULL;
    s->planned = s->cursor = 0;
}
