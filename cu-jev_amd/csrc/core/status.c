/* Per-thread error record, status names, version string, stderr notes. */
#include "core/status.h"

#define CJ_EXPORT __attribute__((visibility("default")))

typedef struct err_record {
    cujev_status code;
    char text[1024];
} err_record;

static _Thread_local err_record tl_err;

/* Indexed by cujev_status; holes (none today) read as unknown. */
static const char *const k_status_names[] = {
    [CUJEV_OK] = "ok",
    [CUJEV_ERR_INVALID_ARGUMENT] = "invalid argument",
    [CUJEV_ERR_IO] = "i/o error",
    [CUJEV_ERR_FORMAT] = "format error",
    [CUJEV_ERR_CUDA] = "device runtime error",
    [CUJEV_ERR_OOM] = "out of memory",
    [CUJEV_ERR_CAPACITY] = "capacity exceeded",
    [CUJEV_ERR_UNSUPPORTED] = "unsupported",
};

cujev_status cujev_raise(cujev_status code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    const int n = vsnprintf(tl_err.text, sizeof tl_err.text, fmt, ap);
    va_end(ap);
    if (n < 0)
        tl_err.text[0] = '\0';
    tl_err.code = code;
    return code;
}

void cujev_error_reset(void) {
    tl_err.code = CUJEV_OK;
    tl_err.text[0] = '\0';
}

cujev_status cujev_error_code(void) { return tl_err.code; }

void cujev_note(int enabled, const char *fmt, ...) {
    if (!enabled)
        return;
    char line[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(line, sizeof line, fmt, ap);
    va_end(ap);
    fprintf(stderr, "cujev: %s\n", line);
}

CJ_EXPORT const char *cujev_last_error(void) { return tl_err.text; }

CJ_EXPORT const char *cujev_status_string(cujev_status s) {
    const unsigned i = (unsigned)s;
    if (i < sizeof k_status_names / sizeof k_status_names[0] && k_status_names[i])
        return k_status_names[i];
    return "unknown";
}

#define CJ_STR_(x) #x
#define CJ_STR(x) CJ_STR_(x)
CJ_EXPORT const char *cujev_version(void) {
    return CJ_STR(CUJEV_VERSION_MAJOR) "." CJ_STR(CUJEV_VERSION_MINOR) "." CJ_STR(
        CUJEV_VERSION_PATCH);
}
