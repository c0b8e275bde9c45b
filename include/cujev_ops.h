/*
 * libcujev_ops.so -- operator-level C ABI of the branch-forward hot path.
 *
 * The reference has no such library: its operator layer is the C launcher
 * header src/kernels/kernels.h:21-102, called only by the engine
 * (src/engine/forward.c:92-145). libcujev.so keeps exactly the 14 public
 * functions of include/cujev.h, so this separate library exposes the same
 * kernels one by one for kernel-level parity tests and benchmarks (the
 * reference has no kernel-level tests). Every entry point takes device
 * pointers, plain sizes and a HIP stream (hipStream_t passed as void*; NULL is
 * the default stream), launches asynchronously and returns a cujev_status:
 * CUJEV_ERR_INVALID_ARGUMENT for shapes the kernels do not support,
 * CUJEV_ERR_CUDA (4) for a launch error, whose text is in cujev_ops_last_error().
 *
 * bf16 buffers are raw uint16 bfloat16. Layouts:
 *   proj      fused projection rows, bf16 [N][stride]
 *   k cache   bf16 [Hkv][cache_stride][256]   token-major
 *   vt cache  bf16 [Hkv][256][cache_stride]   d-major (V transposed)
 *   cache_stride must be a multiple of 64 and at least
 *   cujev_ops_kv_stride(max tokens) so 64-key tiles stay inside.
 */
#ifndef CUJEV_OPS_H
#define CUJEV_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Cache stride (in tokens) the attention kernels need for `max_tokens`. */
int cujev_ops_kv_stride(int max_tokens);
const char *cujev_ops_last_error(void);

/* Replaces reference src/kernels/kernels.h:197-199 (k_attn_prep).
 * q_norm_w / k_norm_w: fp32 [256], already 1 + w. pos: int32 [N].
 * Writes q_out bf16 [N][Hq][256] scaled by q_scale (the engine passes
 * 256^-1/2 * log2 e), K rows n and V^T columns n of the caches. */
int cujev_op_attn_prep(const void *proj, int proj_stride, const float *q_norm_w,
                       const float *k_norm_w, const int32_t *pos, int N, int Hq, int Hkv,
                       int rot, double theta, float eps, float q_scale, void *q_out,
                       void *k_cache, void *vt_cache, int cache_stride, void *stream);

/* Replaces reference src/kernels/kernels.h:203-206 (k_attention).
 * out bf16 [N][Hq*256] = sigmoid(gate) * softmax2(q.k) v over the state keys
 * [0,P) of (pk, pvt) and own keys [own_base[n], n] of (ok, ovt).
 * gate element (n, h, d) is at gate[n*gate_tok_stride + h*gate_head_stride + d]. */
int cujev_op_attention(const void *q, const void *gate, int gate_tok_stride, int gate_head_stride,
                       const void *pk, const void *pvt, int P, int p_stride, const void *ok,
                       const void *ovt, int o_stride, const int32_t *own_base, int N, int Hq,
                       int Hkv, void *out, void *stream);

#ifdef __cplusplus
}
#endif
#endif
