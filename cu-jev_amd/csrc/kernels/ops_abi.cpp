/* libcujev_ops.so: the operator-level C ABI (include/cujev_ops.h). Thin
 * argument checks around the launchers of kernels.h. */
#include "../../../include/cujev_ops.h"
#include "kernels.h"
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <mutex>
#include <stdio.h>
#include <stdlib.h>

#define EXPORT extern "C" __attribute__((visibility("default")))

static thread_local char g_err[512];

static int fail(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return status;
}

static int launched(hipError_t e, const char *what) {
    if (e == hipErrorInvalidValue)
        return fail(1, "%s: unsupported shape", what);
    if (e != hipSuccess)
        return fail(4, "%s: %s", what, hipGetErrorString(e));
    g_err[0] = 0;
    return 0;
}

EXPORT int cujev_ops_kv_stride(int max_tokens) { return cujev_kv_stride(max_tokens); }

/* One hipBLASLt context per process for the GEMM entry point; its workspace
 * is the caller's. */
static cujev_gemm *g_gemm = nullptr;
static void *g_gemm_ws = nullptr;

EXPORT int cujev_op_gemm(const void *X, const void *W, void *Y, int f32out, int N, int M, int K,
                         void *workspace, size_t ws_bytes, void *stream) {
    if (N < 0 || M <= 0 || K <= 0 || !X || !W || !Y)
        return fail(1, "gemm: bad arguments");
    if (!g_gemm || g_gemm_ws != workspace) {
        if (g_gemm)
            cujev_gemm_destroy(g_gemm);
        g_gemm = nullptr;
        if (cujev_gemm_create(&g_gemm, workspace, ws_bytes) != 0)
            return fail(4, "gemm: hipblasLtCreate failed");
        g_gemm_ws = workspace;
    }
    return launched(k_gemm(g_gemm, (const bf16_t *)X, (const bf16_t *)W, Y, f32out, N, M, K,
                           (hipStream_t)stream),
                    "gemm");
}
EXPORT int cujev_op_gemm_tune(const void *X, const void *W, void *Y, int f32out, int N, int M,
                              int K, void *workspace, size_t ws_bytes, void *stream,
                              int *best_index, float *best_us, float *heuristic_us) {
    if (N <= 0 || M <= 0 || K <= 0 || !X || !W || !Y || !best_index || !best_us || !heuristic_us)
        return fail(1, "gemm_tune: bad arguments");
    if (!g_gemm || g_gemm_ws != workspace) {
        if (g_gemm)
            cujev_gemm_destroy(g_gemm);
        g_gemm = nullptr;
        if (cujev_gemm_create(&g_gemm, workspace, ws_bytes) != 0)
            return fail(4, "gemm_tune: hipblasLtCreate failed");
        g_gemm_ws = workspace;
    }
    if (cujev_gemm_tune(g_gemm, (const bf16_t *)X, (const bf16_t *)W, Y, f32out, N, M, K,
                        (hipStream_t)stream, best_index, best_us, heuristic_us) != 0)
        return fail(4, "gemm_tune: no supported hipBLASLt algorithm ran");
    return 0;
}

EXPORT int cujev_ops_gemm_small_splits(int M, int K) { return cujev_gemm_small_splits(M, K); }

EXPORT int cujev_op_gemm_small(const void *X, int ldx, const void *W, int N, int M, int K,
                               int gated, int splits, void *Y, int ldy, float *P, void *stream) {
    if (N < 0 || N > CUJEV_GEMM_SMALL_MAX_N || M <= 0 || K <= 0 || !X || !W ||
        splits > CUJEV_GEMM_SMALL_MAX_SPLITS || ldx < K ||
        (splits == 1 && ldy < (gated ? M / 2 : M)))
        return fail(1, "gemm_small: bad arguments");
    return launched(k_gemm_small((const bf16_t *)X, ldx, (const bf16_t *)W, N, M, K, gated, splits,
                                 (bf16_t *)Y, ldy, P, (hipStream_t)stream),
                    "gemm_small");
}

EXPORT int cujev_op_gemm_wide(const void *X, int ldx, const void *W, int N, int M, int K,
                              int gated, int rg, int ng, int splits, void *Y, int ldy, float *P,
                              void *stream) {
    if (N < 0 || M <= 0 || K <= 0 || !X || !W || ldx < K || splits < 1 ||
        (splits == 1 && (!Y || ldy < (gated ? M / 2 : M))) || (splits > 1 && !P))
        return fail(1, "gemm_wide: bad arguments");
    return launched(k_gemm_wide((const bf16_t *)X, ldx, (const bf16_t *)W, N, M, K, gated, rg, ng,
                                splits, (bf16_t *)Y, ldy, P, (hipStream_t)stream),
                    "gemm_wide");
}

EXPORT int cujev_ops_gemm_wide_plan(int N, int M, int K, int gated, int max_splits, int *rg,
                                    int *ng, int *splits) {
    if (!rg || !ng || !splits)
        return -1;
    return cujev_gemm_wide_plan(N, M, K, gated, max_splits, rg, ng, splits);
}

EXPORT int cujev_op_gemm_small_tile(const void *W, int M, int K, void *Wt, void *stream) {
    if (!W || !Wt || W == Wt || M <= 0 || K <= 0 || M % 16 || K % 128)
        return fail(1, "gemm_small_tile: bad arguments");
    return launched(k_gemm_small_tile((const bf16_t *)W, M, K, (bf16_t *)Wt, (hipStream_t)stream),
                    "gemm_small_tile");
}

EXPORT int cujev_op_add_rmsnorm(float *x, const void *y, const float *yp, int splits,
                                const float *w, void *out, int N, int H, float eps,
                                const int32_t *rows, int R, void *stream) {
    if (N < 0 || H <= 0 || !x || !w || !out || (rows && R < 0))
        return fail(1, "add_rmsnorm: bad arguments");
    return launched(k_add_rmsnorm(x, (const bf16_t *)y, yp, splits, w, (bf16_t *)out, N, H, eps,
                                  rows, R, (hipStream_t)stream),
                    "add_rmsnorm");
}

EXPORT int cujev_ops_blaslt_version(void) {
    cujev_gemm *g = nullptr;
    if (cujev_gemm_create(&g, nullptr, 0) != 0)
        return -1;
    const int v = cujev_gemm_version(g);
    cujev_gemm_destroy(g);
    return v;
}

EXPORT const char *cujev_ops_last_error(void) { return g_err; }

EXPORT int cujev_op_rope_table(double theta, int rot, int npos, float *table) {
    if (rot <= 0 || rot > 64 || rot % 8 || npos <= 0 || !table)
        return fail(1, "rope_table: bad arguments");
    const size_t bytes = (size_t)npos * rot * 4;
    float *h = (float *)malloc(bytes);
    if (!h)
        return fail(5, "rope_table: host buffer");
    cujev_rope_table_host(theta, rot, npos, h);
    hipError_t e = hipMemcpy(table, h, bytes, hipMemcpyHostToDevice);
    free(h);
    return launched(e, "rope_table");
}

EXPORT int cujev_op_attn_prep(const void *proj, int proj_stride, const float *q_norm_w,
                              const float *k_norm_w, const int32_t *pos, int N, int Hq, int Hkv,
                              int rot, const float *rope_table, float eps, float q_scale,
                              void *q_out, void *k_cache, void *vt_cache, int cache_stride,
                              void *stream) {
    if (N < 0 || Hkv <= 0 || rot <= 0 || rot > 64 || cache_stride % 64 || !rope_table)
        return fail(1, "attn_prep: bad arguments");
    return launched(k_attn_prep((const bf16_t *)proj, proj_stride, q_norm_w, k_norm_w, pos, N, Hq,
                                Hkv, rot, rope_table, eps, q_scale, (bf16_t *)q_out,
                                (bf16_t *)k_cache, (bf16_t *)vt_cache, cache_stride,
                                (hipStream_t)stream),
                    "attn_prep");
}

EXPORT int cujev_op_attn_prep_pair(const void *proj, int proj_stride, const float *q_norm_w,
                                   const float *k_norm_w, const int32_t *pos, int Na, int Nb,
                                   int Hq, int Hkv, int rot, const float *rope_table, float eps,
                                   float q_scale, void *q_out, void *k_cache, void *vt_cache,
                                   int cache_stride, void *k_cache2, void *vt_cache2,
                                   int cache_stride2, void *stream) {
    if (Na < 0 || Nb < 0 || Hkv <= 0 || rot <= 0 || rot > 64 || cache_stride % 64 ||
        cache_stride2 % 64 || !rope_table)
        return fail(1, "attn_prep_pair: bad arguments");
    return launched(k_attn_prep_pair((const bf16_t *)proj, proj_stride, q_norm_w, k_norm_w, pos,
                                     Na, Nb, Hq, Hkv, rot, rope_table, eps, q_scale,
                                     (bf16_t *)q_out, (bf16_t *)k_cache, (bf16_t *)vt_cache,
                                     cache_stride, (bf16_t *)k_cache2, (bf16_t *)vt_cache2,
                                     cache_stride2, (hipStream_t)stream),
                    "attn_prep_pair");
}

EXPORT int cujev_op_attention(const void *q, const void *gate, int gate_tok_stride,
                              int gate_head_stride, const void *pk, const void *pvt, int P,
                              int p_stride, const void *ok, const void *ovt, int o_stride,
                              const int32_t *own_base, int N, int Hq, int Hkv, void *out,
                              void *stream) {
    if (N < 0 || P < 0 || Hkv <= 0)
        return fail(1, "attention: bad arguments");
    return launched(k_attention((const bf16_t *)q, (const bf16_t *)gate, gate_tok_stride,
                                gate_head_stride, (const bf16_t *)pk, (const bf16_t *)pvt, P,
                                p_stride, (const bf16_t *)ok, (const bf16_t *)ovt, o_stride,
                                own_base, N, Hq, Hkv, (bf16_t *)out, nullptr, 0,
                                (hipStream_t)stream),
                    "attention");
}

EXPORT int cujev_op_attention_pair(const void *q, const void *gate, int gate_tok_stride,
                                   int gate_head_stride, const void *pk, const void *pvt,
                                   int p_stride, const int32_t *own_base, void *out, int Hq,
                                   int Hkv, int Na, int Pa, const void *oka, const void *ovta,
                                   int oa_stride, int Nb, int Pb, const void *okb,
                                   const void *ovtb, int ob_stride, void *stream) {
    if (Na < 0 || Nb < 0 || Pa < 0 || Pb < 0 || Hkv <= 0)
        return fail(1, "attention_pair: bad arguments");
    return launched(k_attention_pair((const bf16_t *)q, (const bf16_t *)gate, gate_tok_stride,
                                     gate_head_stride, (const bf16_t *)pk, (const bf16_t *)pvt,
                                     p_stride, own_base, (bf16_t *)out, Hq, Hkv, Na, Pa,
                                     (const bf16_t *)oka, (const bf16_t *)ovta, oa_stride, Nb, Pb,
                                     (const bf16_t *)okb, (const bf16_t *)ovtb, ob_stride,
                                     (hipStream_t)stream),
                    "attention_pair");
}

EXPORT size_t cujev_ops_attention_ws_bytes(int N, int Hq, int Hkv, int P) {
    return cujev_attention_ws_bytes(N, Hq, cujev_attention_splits(N, Hkv, P));
}

EXPORT int cujev_op_attention_ws(const void *q, const void *gate, int gate_tok_stride,
                                 int gate_head_stride, const void *pk, const void *pvt, int P,
                                 int p_stride, const void *ok, const void *ovt, int o_stride,
                                 const int32_t *own_base, int N, int Hq, int Hkv, void *out,
                                 void *ws, size_t ws_bytes, void *stream) {
    if (N < 0 || P < 0 || Hkv <= 0)
        return fail(1, "attention: bad arguments");
    return launched(k_attention((const bf16_t *)q, (const bf16_t *)gate, gate_tok_stride,
                                gate_head_stride, (const bf16_t *)pk, (const bf16_t *)pvt, P,
                                p_stride, (const bf16_t *)ok, (const bf16_t *)ovt, o_stride,
                                own_base, N, Hq, Hkv, (bf16_t *)out, ws, ws_bytes,
                                (hipStream_t)stream),
                    "attention");
}

/* ---- attention with no allocation ----------------------------------------
 * The key-split partials of cujev_op_attention_noalloc live in `scratch`, a
 * file-scope device array (each GPU the library runs on holds its own copy
 * until the process ends). Host code never uses the array's name as an
 * address: on its first call on a device, with that device current, the
 * entry point asks the runtime for that device's address of the array and
 * keeps it per device. Every call on one GPU shares the array: calls that
 * overlap on one GPU race. Nothing in it has to start at zero (every split
 * writes l and mu of each of its rows; o is read only where l > 0). */
static __device__ __align__(256) unsigned char scratch[CUJEV_OPS_ATTN_NOALLOC_SCRATCH_BYTES];

#define CUJEV_OPS_MAX_DEVICES 64
static std::mutex g_scratch_mu;
static void *g_scratch_dev[CUJEV_OPS_MAX_DEVICES]; /* per device ordinal */

static int scratch_address(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return fail(4, "attention_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= CUJEV_OPS_MAX_DEVICES)
        return fail(7, "attention_noalloc: device %d is beyond the %d this library tracks", dev,
                    CUJEV_OPS_MAX_DEVICES);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(4, "attention_noalloc: hipGetSymbolAddress(scratch) on device %d: %s",
                        dev, hipGetErrorString(e));
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return 0;
}

EXPORT int cujev_op_attention_noalloc(const void *q, const void *gate, int gate_tok_stride,
                                      int gate_head_stride, const void *pk, const void *pvt,
                                      int P, int p_stride, const void *ok, const void *ovt,
                                      int o_stride, const int32_t *own_base, int N, int Hq,
                                      int Hkv, void *out, void *stream) {
    if (N < 0 || P < 0 || Hkv <= 0)
        return fail(1, "attention_noalloc: bad arguments");
    const size_t need = cujev_attention_ws_bytes(N, Hq, cujev_attention_splits(N, Hkv, P));
    if (need > CUJEV_OPS_ATTN_NOALLOC_SCRATCH_BYTES)
        return fail(6,
                    "attention_noalloc: N=%d, Hq=%d, Hkv=%d, P=%d needs %zu bytes of key-split "
                    "partials; the static scratch holds %zu",
                    N, Hq, Hkv, P, need, (size_t)CUJEV_OPS_ATTN_NOALLOC_SCRATCH_BYTES);
    void *ws = nullptr;
    const int st = scratch_address(&ws);
    if (st != 0)
        return st;
    return launched(k_attention((const bf16_t *)q, (const bf16_t *)gate, gate_tok_stride,
                                gate_head_stride, (const bf16_t *)pk, (const bf16_t *)pvt, P,
                                p_stride, (const bf16_t *)ok, (const bf16_t *)ovt, o_stride,
                                own_base, N, Hq, Hkv, (bf16_t *)out, ws,
                                CUJEV_OPS_ATTN_NOALLOC_SCRATCH_BYTES, (hipStream_t)stream),
                    "attention_noalloc");
}

EXPORT int cujev_op_gdn_conv_prep(const void *proj, int proj_stride, const float *conv_w,
                                  const float *conv_in, float *conv_out, int seg0_len,
                                  const int32_t *own_base, const float *A_neg_exp,
                                  const float *dt_bias, int N, int Hk, int Hv, void *q, void *k,
                                  void *v, float *g, float *beta, void *stream) {
    if (N < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk || (conv_out && (seg0_len < 0 || seg0_len > N)))
        return fail(1, "gdn_conv_prep: bad arguments");
    return launched(k_gdn_conv_prep((const bf16_t *)proj, proj_stride, conv_w, conv_in, conv_out,
                                    seg0_len, own_base, A_neg_exp, dt_bias, N, Hk, Hv,
                                    (float *)q, (float *)k, (float *)v, g, beta,
                                    (hipStream_t)stream),
                    "gdn_conv_prep");
}

EXPORT int cujev_op_gdn_layer(const void *proj, int proj_stride, const float *conv_w,
                              const float *conv_in, float *conv_out, int seg0_len,
                              const int32_t *own_base, const float *A_neg_exp,
                              const float *dt_bias, const int32_t *chunk_tok0,
                              const int32_t *chunk_len, int num_chunks, const int32_t *seg_chunk0,
                              const int32_t *seg_nchunk, int num_segments, int max_seg_chunks,
                              const uint64_t *chunk_starts, const float *S_in, float *S_out,
                              const float *norm_w, float eps, int Hk, int Hv, int N, void *y,
                              void *scratch, void *stream) {
    if (num_chunks < 0 || num_segments < 0 || N < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk ||
        !scratch || (conv_out && (seg0_len < 0 || seg0_len > N)))
        return fail(1, "gdn_layer: bad arguments");
    if (proj_stride % 8 || ((uintptr_t)proj & 15))
        return fail(1, "gdn_layer: projection rows must be 16-byte aligned");
    if (chunk_starts && S_out)
        return fail(1, "gdn_layer: packed segments write no final state");
    cujev_chunks ck = {chunk_tok0, chunk_len,   seg_chunk0,     seg_nchunk,
                       num_chunks, num_segments, max_seg_chunks, chunk_starts};
    cujev_gdn_scratch ws = cujev_gdn_scratch_carve(scratch, num_chunks, Hv);
    return launched(k_gdn_layer((const bf16_t *)proj, proj_stride, conv_w, conv_in, conv_out,
                                seg0_len, own_base, A_neg_exp, dt_bias, &ck, S_in, S_out, norm_w,
                                eps, Hk, Hv, (bf16_t *)y, &ws, N, (hipStream_t)stream),
                    "gdn_layer");
}

EXPORT int cujev_op_gdn_recur(const void *proj, int proj_stride, const float *conv_w,
                              const float *conv_in, const float *A_neg_exp, const float *dt_bias,
                              const int32_t *chunk_tok0, const int32_t *chunk_len,
                              const int32_t *seg_chunk0, int num_segments, int max_seg_len,
                              const float *S_in, const float *norm_w, float eps, int Hk, int Hv,
                              int N, void *y, void *scratch, void *stream) {
    if (num_segments < 0 || N < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk || !scratch || !y ||
        max_seg_len < 1 || max_seg_len > CUJEV_GDN_RECUR_MAX_LEN)
        return fail(1, "gdn_recur: bad arguments");
    if (proj_stride % 8 || ((uintptr_t)proj & 15))
        return fail(1, "gdn_recur: projection rows must be 16-byte aligned");
    cujev_chunks ck = {chunk_tok0, chunk_len, seg_chunk0, nullptr, num_segments,
                       num_segments, 1, nullptr, max_seg_len};
    cujev_gdn_scratch ws = cujev_gdn_scratch_carve(scratch, num_segments, Hv);
    return launched(k_gdn_recur((const bf16_t *)proj, proj_stride, conv_w, conv_in, A_neg_exp,
                                dt_bias, &ck, S_in, norm_w, eps, Hk, Hv, (bf16_t *)y, &ws, N,
                                (hipStream_t)stream),
                    "gdn_recur");
}

EXPORT size_t cujev_ops_gdn_scratch_bytes(int num_chunks, int Hv, int N) {
    return cujev_gdn_scratch_bytes(num_chunks, Hv, N);
}

EXPORT int cujev_op_gdn_scan(const void *q, const void *k, const void *v, const float *g,
                             const float *beta, const int32_t *chunk_tok0,
                             const int32_t *chunk_len, int num_chunks, const int32_t *seg_chunk0,
                             const int32_t *seg_nchunk, int num_segments, int max_seg_chunks,
                             const uint64_t *chunk_starts, const float *S_in, float *S_out,
                             const void *z, int z_stride,
                             const float *norm_w, float eps, int Hk, int Hv, int N, void *y,
                             void *scratch, void *stream) {
    if (num_chunks < 0 || num_segments < 0 || N < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk || !scratch)
        return fail(1, "gdn_scan: bad arguments");
    if (chunk_starts && S_out)
        return fail(1, "gdn_scan: packed segments write no final state");
    cujev_chunks ck = {chunk_tok0, chunk_len,   seg_chunk0,     seg_nchunk,
                       num_chunks, num_segments, max_seg_chunks, chunk_starts};
    cujev_gdn_scratch ws = cujev_gdn_scratch_carve(scratch, num_chunks, Hv);
    return launched(k_gdn_scan((const float *)q, (const float *)k, (const float *)v, g, beta,
                               &ck, S_in, S_out, (const bf16_t *)z, z_stride, norm_w, eps, Hk, Hv,
                               (bf16_t *)y, &ws, N, (hipStream_t)stream),
                    "gdn_scan");
}
