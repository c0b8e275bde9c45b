#include "core/util.h"
#include <hip/hip_runtime_api.h>

static __thread char g_last_error[1024];

cujev_status cujev_fail(cujev_status s, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
    return s;
}

void cujev_clear_error(void) { g_last_error[0] = 0; }

__attribute__((visibility("default"))) const char *cujev_last_error(void) { return g_last_error; }

void cujev_log(int verbose, const char *fmt, ...) {
    if (!verbose)
        return;
    va_list ap;
    va_start(ap, fmt);
    fputs("[cujev] ", stderr);
    vfprintf(stderr, fmt, ap);
    fputc('\n', stderr);
    va_end(ap);
}

__attribute__((visibility("default"))) const char *cujev_status_string(cujev_status s) {
    switch (s) {
    case CUJEV_OK: return "ok";
    case CUJEV_ERR_INVALID_ARGUMENT: return "invalid argument";
    case CUJEV_ERR_IO: return "i/o error";
    case CUJEV_ERR_FORMAT: return "format error";
    case CUJEV_ERR_CUDA: return "device runtime error";
    case CUJEV_ERR_OOM: return "out of memory";
    case CUJEV_ERR_CAPACITY: return "capacity exceeded";
    case CUJEV_ERR_UNSUPPORTED: return "unsupported";
    }
    return "unknown";
}

__attribute__((visibility("default"))) const char *cujev_version(void) { return "0.1.0"; }

cujev_status cujev_arena_init(cujev_arena *a, size_t bytes) {
    a->base = NULL;
    a->size = a->used = 0;
    hipError_t e = hipMalloc(&a->base, bytes);
    if (e != hipSuccess) {
        a->base = NULL;
        return cujev_fail(CUJEV_ERR_OOM, "hipMalloc(%zu bytes): %s", bytes, hipGetErrorString(e));
    }
    a->size = bytes;
    return CUJEV_OK;
}

void *cujev_arena_alloc(cujev_arena *a, size_t bytes) {
    size_t off = cujev_align_up(a->used, 256);
    if (!a->base || off + bytes > a->size)
        return NULL;
    a->used = off + bytes;
    return (char *)a->base + off;
}

void cujev_arena_free(cujev_arena *a) {
    if (a->base)
        hipFree(a->base);
    a->base = NULL;
    a->size = a->used = 0;
}
