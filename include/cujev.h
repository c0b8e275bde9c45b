/*
 * libcujev.so -- public C ABI of the MI355X shared-prefix decision engine.
 *
 * Drop-in for the reference's include/cujev/cujev.h:1-137. Every type below
 * has the same size, field order and enum values as the reference, because
 * existing ctypes callers (python/cujev/_lib.py:17-59, :103-130 in the
 * reference) bind to them by layout. The library exports exactly these 14
 * functions; everything else is hidden.
 *
 * Execution model:
 *   cujev_state_prefill  runs the shared prefix once and keeps, per layer, what
 *                        later tokens need: the K/V cache of every full
 *                        attention layer, the recurrent matrix S and the conv
 *                        tail of every Gated DeltaNet layer.
 *   cujev_eval           runs B independent branches packed into one token
 *                        stream. Each branch token attends to the prefix plus
 *                        its own branch, never to a sibling. At the last token of
 *                        each branch it returns the logits of the requested
 *                        candidate ids. Nothing is decoded.
 *
 * All calls are synchronous (they end with a stream synchronisation), use one
 * HIP stream per model and are not re-entrant for one model.
 */
#ifndef CUJEV_H
#define CUJEV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CUJEV_VERSION_MAJOR 0
#define CUJEV_VERSION_MINOR 1
#define CUJEV_VERSION_PATCH 0

typedef struct cujev_model cujev_model;
typedef struct cujev_state cujev_state;

/* Same values as reference include/cujev/cujev.h:37-46. CUJEV_ERR_CUDA (4) is
 * kept as the name and value of "device runtime error" (HIP here). */
typedef enum cujev_status {
    CUJEV_OK = 0,
    CUJEV_ERR_INVALID_ARGUMENT = 1,
    CUJEV_ERR_IO = 2,
    CUJEV_ERR_FORMAT = 3,
    CUJEV_ERR_CUDA = 4,
    CUJEV_ERR_OOM = 5,
    CUJEV_ERR_CAPACITY = 6,
    CUJEV_ERR_UNSUPPORTED = 7,
} cujev_status;

/* 6 x int, 24 bytes (reference include/cujev/cujev.h:48-55). */
typedef struct cujev_options {
    int device;            /* HIP device ordinal, default 0 */
    int max_state_tokens;  /* prefix capacity, default 8192 */
    int max_branch_tokens; /* branch tokens of one eval, default 4096 */
    int max_branches;      /* default 256 */
    int max_candidates;    /* per branch, default 256 */
    int verbose;           /* log to stderr */
} cujev_options;

/* char[64] + 7 int + 2 size_t, 112 bytes on LP64
 * (reference include/cujev/cujev.h:58-69). */
typedef struct cujev_model_info {
    char name[64];
    int hidden_size;
    int num_layers;
    int num_full_attention_layers;
    int vocab_size;
    int max_state_tokens;
    int max_branch_tokens;
    int max_branches;
    size_t device_bytes_weights;
    size_t device_bytes_workspace;
} cujev_model_info;

/* One branch: its own tokens (appended after the prefix) and the vocabulary
 * ids whose logits are wanted at its last token. 32 bytes on LP64
 * (reference include/cujev/cujev.h:74-79). */
typedef struct cujev_branch {
    const int32_t *tokens;
    int num_tokens;
    const int32_t *candidates;
    int num_candidates;
} cujev_branch;

/* Reference include/cujev/cujev.h:81. Fills 8192 / 4096 / 256 / 256, device 0. */
void cujev_options_default(cujev_options *opts);

/* Reference include/cujev/cujev.h:85-86. Loads config.json + *.safetensors of a
 * Qwen3.5 checkpoint directory (text model only). opts may be NULL. */
cujev_status cujev_model_open(const char *checkpoint_dir, const cujev_options *opts,
                              cujev_model **out);
/* Reference include/cujev/cujev.h:87. NULL is a no-op. */
void cujev_model_close(cujev_model *model);
/* Reference include/cujev/cujev.h:88. */
cujev_status cujev_model_info_get(const cujev_model *model, cujev_model_info *out);

/* Reference include/cujev/cujev.h:92-93. A state is reusable across evals. */
cujev_status cujev_state_create(cujev_model *model, cujev_state **out);
void cujev_state_destroy(cujev_state *state);

/* Reference include/cujev/cujev.h:96-98. Overwrites whatever the state held. */
cujev_status cujev_state_prefill(cujev_model *model, cujev_state *state, const int32_t *tokens,
                                 int num_tokens);
int cujev_state_num_tokens(const cujev_state *state);

/* Reference include/cujev/cujev.h:108-109.
 *   logits_out: row-major [num_branches][ld]; entry (b, i) is the raw logit of
 *               branches[b].candidates[i] at the last token of branch b.
 *               Entries i >= num_candidates of a row are left untouched.
 *   ld        : row stride in floats, >= max num_candidates. */
cujev_status cujev_eval(cujev_model *model, cujev_state *state, const cujev_branch *branches,
                        int num_branches, float *logits_out, int ld);

/* Reference include/cujev/cujev.h:115-117. Full-vocabulary logits at the last
 * token of every branch, row-major [num_branches][vocab_size]. */
cujev_status cujev_eval_full_logits(cujev_model *model, cujev_state *state,
                                    const cujev_branch *branches, int num_branches,
                                    float *logits_out);

/* 2 float + 3 int, 20 bytes (reference include/cujev/cujev.h:120-127).
 * GPU milliseconds of the last prefill / eval on this model. */
typedef struct cujev_timing {
    float prefill_ms;
    float eval_ms;
    int prefill_tokens;
    int eval_tokens;
    int eval_branches;
} cujev_timing;
void cujev_last_timing(const cujev_model *model, cujev_timing *out);

/* Reference include/cujev/cujev.h:129-132. */
const char *cujev_status_string(cujev_status s);
const char *cujev_last_error(void); /* thread-local; "" if none */
const char *cujev_version(void);

#ifdef __cplusplus
}
#endif
#endif /* CUJEV_H */
