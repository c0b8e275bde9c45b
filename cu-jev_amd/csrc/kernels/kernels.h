/* Launchers of the gfx950 kernels: the operator layer between the host engine
 * and the device code. All pointers are device pointers, all launches go to
 * `stream`, every launcher returns the launch status. Row-major throughout.
 *
 * Role of the reference's src/kernels/kernels.h:21-102, with signatures of our
 * own (the only callers are this engine and the ops library). Data layouts in
 * HBM that differ from the reference are stated per launcher. */
#ifndef CUJEV_KERNELS_H
#define CUJEV_KERNELS_H

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t bf16_t; /* storage type of bfloat16 seen from C */

/* Token tiles of the attention kernel: 32 consecutive packed tokens per wave
 * group; K/V tiles are 64 keys. Caches are padded so aligned 64-key tiles
 * never leave the allocation. */
#define CUJEV_ATT_KEY_TILE 64
static inline int cujev_kv_stride(int max_tokens) { return (max_tokens + 63) / 64 * 64 + 64; }

/* ---- full attention -----------------------------------------------------
 * proj[N, proj_stride] bf16 is the fused projection row
 *   [Hq x (q 256 | gate 256)] [Hkv x K 256] [Hkv x V 256].
 * Per q-head: zero-centred RMSNorm (q_norm_w already holds 1+w), RoPE on the
 * first `rot` dims (rotate_half, angle pos*inv_freq[i]), times q_scale
 * (= head_dim^-1/2 * log2 e), rounded to bf16 -> q_out[N][Hq][256].
 * Per kv-head: the same for K -> k_cache[Hkv][cache_stride][256] row n;
 * V copied raw -> vt_cache[Hkv][256][cache_stride] column n (d-major).
 * The cache column of packed token n is n itself. inv_freq has rot/2 floats
 * in host memory. */
hipError_t k_attn_prep(const bf16_t *proj, int proj_stride, const float *q_norm_w,
                       const float *k_norm_w, const int32_t *pos, int N, int Hq, int Hkv, int rot,
                       const float *inv_freq_host, float eps, float q_scale, bf16_t *q_out,
                       bf16_t *k_cache, bf16_t *vt_cache, int cache_stride, hipStream_t stream);

/* out[n, h*256 + d] = sigmoid(gate[n*gate_tok_stride + h*gate_head_stride + d])
 *                     * softmax_j(q[n,h] . k_j) v_j          (base-2 softmax)
 * over keys j in [0, P) of the state cache (pk / pvt, stride p_stride) and
 * the own keys j in [own_base[n], n] of (ok / ovt, stride o_stride).
 * q is bf16 [N][Hq][256] already scaled by head_dim^-1/2 * log2 e. GQA:
 * q-head h reads kv-head h / (Hq/Hkv); Hq/Hkv must be 4. */
hipError_t k_attention(const bf16_t *q, const bf16_t *gate, int gate_tok_stride,
                       int gate_head_stride, const bf16_t *pk, const bf16_t *pvt, int P,
                       int p_stride, const bf16_t *ok, const bf16_t *ovt, int o_stride,
                       const int32_t *own_base, int N, int Hq, int Hkv, bf16_t *out,
                       hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif
