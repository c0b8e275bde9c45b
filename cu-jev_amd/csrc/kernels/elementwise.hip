/* Per-layer glue kernels of the forward pass (gfx950).
 *
 * Semantics: REF src/kernels/elementwise.cu:3-11 (embed), :13-30 (rmsnorm with
 * optional row gather), :32-40 (residual add), :42-54 (silu * up), :78-97
 * (candidate readout). The residual add and the following RMSNorm are fused
 * into one pass here (same arithmetic: fp32 add, then the norm of the sum). */
#include "common.h"
#include "kernels.h"

namespace CUJEV_KNS {
namespace {

constexpr int NT = 256;

/* x[n, :] = float(E[tok[n], :]) */
__global__ __launch_bounds__(NT) void embed_kernel(const int32_t *__restrict__ tok,
                                                   const bf16 *__restrict__ E, float *__restrict__ x,
                                                   int H) {
    const int n = blockIdx.x;
    const bf16 *row = E + (size_t)tok[n] * H;
    float *dst = x + (size_t)n * H;
    for (int i = threadIdx.x * 4; i < H; i += NT * 4) {
        bf16x4 v = *(const bf16x4 *)(row + i);
        *(float4 *)(dst + i) = make_float4(bf2f(v[0]), bf2f(v[1]), bf2f(v[2]), bf2f(v[3]));
    }
}

/* dst row r = src row rows[r], 16-byte pieces (the last layer's rows that
 * reach the outputs) */
__global__ __launch_bounds__(NT) void gather_rows_kernel(const unsigned char *__restrict__ src,
                                                         size_t src_pitch,
                                                         const int32_t *__restrict__ rows,
                                                         unsigned char *__restrict__ dst,
                                                         size_t dst_pitch, int pieces) {
    const uint4 *s = (const uint4 *)(src + (size_t)rows[blockIdx.x] * src_pitch);
    uint4 *d = (uint4 *)(dst + (size_t)blockIdx.x * dst_pitch);
    for (int i = threadIdx.x; i < pieces; i += NT)
        d[i] = s[i];
}

/* One block per output row r (source row rows ? rows[r] : r):
 *   v = x[src] + d (d from bf16 y, or bf16 of the split-K partial sum of yp);
 *   x[src] = v when there is a d and !rows;
 *   out[r] = bf16(v * rsqrt(mean v^2 + eps) * w)
 * Thread t holds the float4 groups t + 256k (k < 4, H <= 4096). Every load
 * (x, the added term, w) is issued before the reduction, with indices clamped
 * into the row: one memory round trip per row. */
constexpr int RN_K = 4;
template <int SPLITS> /* 0: bf16 y or nothing; > 0: that many fp32 partials, all loads up front */
__global__ __launch_bounds__(NT) void add_rmsnorm_kernel(float *__restrict__ x,
                                                         const bf16 *__restrict__ y,
                                                         const float *__restrict__ yp, int splits,
                                                         size_t split_stride,
                                                         const float *__restrict__ w,
                                                         bf16 *__restrict__ out, int H, float eps,
                                                         const int32_t *__restrict__ rows) {
    __shared__ float scratch[NT / 64];
    const int r = blockIdx.x;
    const int src = rows ? rows[r] : r;
    const int ng = H / 4;
    float *xr = x + (size_t)src * H;
    float4 v[RN_K], ww[RN_K];
#pragma unroll
    for (int k = 0; k < RN_K; k++) {
        const int g = min((int)threadIdx.x + k * NT, ng - 1);
        v[k] = *(const float4 *)(xr + 4 * g);
        ww[k] = *(const float4 *)(w + 4 * g);
    }
    const bool add = y || yp;
    if (add) {
        float4 d[RN_K];
        if (y) {
#pragma unroll
            for (int k = 0; k < RN_K; k++) {
                const int g = min((int)threadIdx.x + k * NT, ng - 1);
                const bf16x4 b = *(const bf16x4 *)(y + (size_t)src * H + 4 * g);
                d[k] = make_float4(bf2f(b[0]), bf2f(b[1]), bf2f(b[2]), bf2f(b[3]));
            }
        } else {
#pragma unroll
            for (int k = 0; k < RN_K; k++)
                d[k] = make_float4(0.f, 0.f, 0.f, 0.f);
            float4 t[SPLITS > 0 ? SPLITS : 1][RN_K];
#pragma unroll
            for (int sp = 0; sp < SPLITS; sp++)
#pragma unroll
                for (int k = 0; k < RN_K; k++) {
                    const int g = min((int)threadIdx.x + k * NT, ng - 1);
                    t[sp][k] = *(const float4 *)(yp + sp * split_stride + (size_t)src * H + 4 * g);
                }
#pragma unroll
            for (int sp = 0; sp < SPLITS; sp++) /* split order: deterministic */
#pragma unroll
                for (int k = 0; k < RN_K; k++)
                    d[k].x += t[sp][k].x, d[k].y += t[sp][k].y, d[k].z += t[sp][k].z,
                        d[k].w += t[sp][k].w;
#pragma unroll
            for (int k = 0; k < RN_K; k++) /* the GEMM output's bf16 rounding */
                d[k] = make_float4(bf2f(f2bf(d[k].x)), bf2f(f2bf(d[k].y)), bf2f(f2bf(d[k].z)),
                                   bf2f(f2bf(d[k].w)));
        }
#pragma unroll
        for (int k = 0; k < RN_K; k++)
            v[k].x += d[k].x, v[k].y += d[k].y, v[k].z += d[k].z, v[k].w += d[k].w;
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < RN_K; k++) {
        const int g = threadIdx.x + k * NT;
        if (g < ng) {
            ss += v[k].x * v[k].x + v[k].y * v[k].y + v[k].z * v[k].z + v[k].w * v[k].w;
            if (add && !rows)
                *(float4 *)(xr + 4 * g) = v[k];
        }
    }
    ss = block_sum(ss, scratch);
    const float inv = rsqrtf(ss / H + eps);
    bf16 *orow = out + (size_t)r * H;
#pragma unroll
    for (int k = 0; k < RN_K; k++) {
        const int g = threadIdx.x + k * NT;
        if (g < ng)
            *(bf16x4 *)(orow + 4 * g) =
                bf16x4{f2bf(v[k].x * inv * ww[k].x), f2bf(v[k].y * inv * ww[k].y),
                       f2bf(v[k].z * inv * ww[k].z), f2bf(v[k].w * inv * ww[k].w)};
    }
}

/* act[n, i] = bf16(silu(gu[n, i]) * gu[n, I + i]) */
__global__ __launch_bounds__(NT) void silu_mul_kernel(const bf16 *__restrict__ gu,
                                                      bf16 *__restrict__ act, int I) {
    const int n = blockIdx.y;
    const int i = (blockIdx.x * NT + threadIdx.x) * 4;
    if (i >= I)
        return;
    const bf16 *row = gu + (size_t)n * 2 * I;
    bf16x4 g = *(const bf16x4 *)(row + i), u = *(const bf16x4 *)(row + I + i);
    bf16x4 o;
#pragma unroll
    for (int e = 0; e < 4; e++)
        o[e] = f2bf(silu_f(bf2f(g[e])) * bf2f(u[e]));
    *(bf16x4 *)(act + (size_t)n * I + i) = o;
}

/* logits[b*ld + i] = h[b] . E[cand[b*cand_ld + i]] for i < ncand[b]; one wave
 * per (branch, candidate), 4 per block. */
__global__ __launch_bounds__(NT) void readout_kernel(const bf16 *__restrict__ h,
                                                     const bf16 *__restrict__ E,
                                                     const int32_t *__restrict__ cand,
                                                     const int32_t *__restrict__ ncand, int cand_ld,
                                                     float *__restrict__ logits, int ld, int H) {
    const int b = blockIdx.y;
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (i >= ncand[b])
        return;
    const bf16 *hr = h + (size_t)b * H;
    const bf16 *er = E + (size_t)cand[(size_t)b * cand_ld + i] * H;
    float acc = 0.f;
    for (int j = lane * 8; j < H; j += 64 * 8) {
        bf16x8 a = *(const bf16x8 *)(hr + j), e = *(const bf16x8 *)(er + j);
#pragma unroll
        for (int k = 0; k < 8; k++)
            acc += bf2f(a[k]) * bf2f(e[k]);
    }
    acc = wave_sum(acc);
    if (lane == 0)
        logits[(size_t)b * ld + i] = acc;
}

} // namespace
} // namespace CUJEV_KNS
using namespace CUJEV_KNS;

extern "C" hipError_t k_embed(const int32_t *tokens, const bf16_t *E, float *x, int N, int H,
                              hipStream_t s) {
    if (N <= 0)
        return hipSuccess;
    if (H % 4)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(embed_kernel, dim3((unsigned)N), dim3(NT), 0, s, tokens, (const bf16 *)E, x,
                       H);
    return hipGetLastError();
}

extern "C" hipError_t k_add_rmsnorm(float *x, const bf16_t *y, const float *yp, int splits,
                                    const float *w, bf16_t *out, int N, int H, float eps,
                                    const int32_t *rows, int R, hipStream_t s) {
    const int nrows = rows ? R : N;
    if (nrows <= 0)
        return hipSuccess;
    if (H % 4 || H > RN_K * 4 * NT || (yp && (y || splits < 1)))
        return hipErrorInvalidValue;
#define CUJEV_RN_LAUNCH(S)                                                                   \
    hipLaunchKernelGGL(add_rmsnorm_kernel<S>, dim3((unsigned)nrows), dim3(NT), 0, s, x,       \
                       (const bf16 *)y, yp, splits, (size_t)N * H, w, (bf16 *)out, H, eps, rows)
    switch (yp ? splits : 0) {
    case 0: CUJEV_RN_LAUNCH(0); break;
    case 1: CUJEV_RN_LAUNCH(1); break;
    case 2: CUJEV_RN_LAUNCH(2); break;
    case 3: CUJEV_RN_LAUNCH(3); break;
    case 4: CUJEV_RN_LAUNCH(4); break;
    case 5: CUJEV_RN_LAUNCH(5); break;
    case 6: CUJEV_RN_LAUNCH(6); break;
    case 7: CUJEV_RN_LAUNCH(7); break;
    case 8: CUJEV_RN_LAUNCH(8); break;
    default: return hipErrorInvalidValue;
    }
#undef CUJEV_RN_LAUNCH
    return hipGetLastError();
}

extern "C" hipError_t k_gather_rows(const void *src, size_t src_pitch, const int32_t *rows, int R,
                                    void *dst, size_t dst_pitch, size_t row_bytes,
                                    hipStream_t s) {
    if (R <= 0)
        return hipSuccess;
    if (row_bytes % 16 || src_pitch % 16 || dst_pitch % 16 || ((uintptr_t)src & 15) ||
        ((uintptr_t)dst & 15))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)R), dim3(NT), 0, s,
                       (const unsigned char *)src, src_pitch, rows, (unsigned char *)dst,
                       dst_pitch, (int)(row_bytes / 16));
    return hipGetLastError();
}

extern "C" hipError_t k_silu_mul(const bf16_t *gu, bf16_t *act, int N, int I, hipStream_t s) {
    if (N <= 0)
        return hipSuccess;
    if (I % 4)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)CEIL_DIV(I / 4, NT), (unsigned)N), dim3(NT),
                       0, s, (const bf16 *)gu, (bf16 *)act, I);
    return hipGetLastError();
}

extern "C" hipError_t k_readout(const bf16_t *h, const bf16_t *E, const int32_t *cand,
                                const int32_t *ncand, int cand_ld, float *logits, int ld, int B,
                                int H, hipStream_t s) {
    if (B <= 0 || cand_ld <= 0)
        return hipSuccess;
    if (H % 8)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(readout_kernel, dim3((unsigned)CEIL_DIV(cand_ld, 4), (unsigned)B), dim3(NT),
                       0, s, (const bf16 *)h, (const bf16 *)E, cand, ncand, cand_ld, logits, ld, H);
    return hipGetLastError();
}
