/* Status reporting of the host engine.
 *
 * Every failing host function returns a cujev_status and leaves a message in
 * a per-thread error record that cujev_last_error() (public ABI) reads back.
 * The record is reset at the start of every successful public call's
 * completion path, so a stale message never outlives the next success. */
#ifndef CUJEV_STATUS_H
#define CUJEV_STATUS_H

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

/* Records `code` and the formatted message for this thread; returns `code`
 * so a caller can write `return cujev_raise(...)`. */
cujev_status cujev_raise(cujev_status code, const char *fmt, ...)
    __attribute__((format(printf, 2, 3)));
/* Clears this thread's record (message "" , code CUJEV_OK). */
void cujev_error_reset(void);
/* Code of this thread's last recorded error (CUJEV_OK after a reset). */
cujev_status cujev_error_code(void);

/* One line "cujev: <message>" on stderr when `enabled`. */
void cujev_note(int enabled, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

static inline size_t cujev_round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

/* Propagate a non-OK status. */
#define CJ_CHECK(expr)                                                                           \
    do {                                                                                         \
        const cujev_status cj_s_ = (expr);                                                       \
        if (cj_s_ != CUJEV_OK)                                                                   \
            return cj_s_;                                                                        \
    } while (0)

/* A HIP runtime call whose failure becomes CUJEV_ERR_CUDA (the device-error
 * code of the ABI) with the runtime's own description. */
#define HIP_CHECK(expr)                                                                          \
    do {                                                                                         \
        const hipError_t cj_e_ = (expr);                                                         \
        if (cj_e_ != hipSuccess)                                                                 \
            return cujev_raise(CUJEV_ERR_CUDA, "%s failed: %s", #expr,                           \
                               hipGetErrorString(cj_e_));                                        \
    } while (0)

#ifdef __cplusplus
}
#endif
#endif
