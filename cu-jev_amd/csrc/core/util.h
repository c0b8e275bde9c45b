/* Errors, logging and the device bump arena of the host engine.
 * Role of REF src/core/util.h:17-29 (thread-local last error, stderr log,
 * one-allocation arena), on the HIP runtime. */
#ifndef CUJEV_UTIL_H
#define CUJEV_UTIL_H

#include "cujev.h"
#include <stdarg.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Record the message returned by cujev_last_error() and return `s`. */
cujev_status cujev_fail(cujev_status s, const char *fmt, ...)
    __attribute__((format(printf, 2, 3)));
void cujev_clear_error(void);
void cujev_log(int verbose, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

/* One hipMalloc carved into 256-byte aligned pieces. */
typedef struct cujev_arena {
    void *base;
    size_t size;
    size_t used;
} cujev_arena;

cujev_status cujev_arena_init(cujev_arena *a, size_t bytes);
void *cujev_arena_alloc(cujev_arena *a, size_t bytes); /* NULL when full */
void cujev_arena_free(cujev_arena *a);

static inline size_t cujev_align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

#define CUJEV_TRY(expr)                                                                          \
    do {                                                                                         \
        cujev_status _s = (expr);                                                                \
        if (_s != CUJEV_OK)                                                                      \
            return _s;                                                                           \
    } while (0)

/* HIP runtime call -> CUJEV_ERR_CUDA with the runtime's message. */
#define HIP_TRY(expr)                                                                            \
    do {                                                                                         \
        hipError_t _e = (expr);                                                                  \
        if (_e != hipSuccess)                                                                    \
            return cujev_fail(CUJEV_ERR_CUDA, "%s: %s", #expr, hipGetErrorString(_e));           \
    } while (0)

#ifdef __cplusplus
}
#endif
#endif
