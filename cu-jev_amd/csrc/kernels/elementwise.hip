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

/* One block per output row r (source row rows ? rows[r] : r):
 *   v = x[src] (+ y[src] if y);  if (y && !rows) x[src] = v;
 *   out[r] = bf16(v * rsqrt(mean v^2 + eps) * w) */
__global__ __launch_bounds__(NT) void add_rmsnorm_kernel(float *__restrict__ x,
                                                         const bf16 *__restrict__ y,
                                                         const float *__restrict__ w,
                                                         bf16 *__restrict__ out, int H, float eps,
                                                         const int32_t *__restrict__ rows) {
    __shared__ float scratch[NT / 64];
    const int r = blockIdx.x;
    const int src = rows ? rows[r] : r;
    float *xr = x + (size_t)src * H;
    const bf16 *yr = y ? y + (size_t)src * H : nullptr;
    const bool write_back = y && !rows;
    /* H <= 16 * 4 * NT: keep the row in registers */
    float4 v[16];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const int i = (threadIdx.x + k * NT) * 4;
        if (i < H) {
            float4 a = *(const float4 *)(xr + i);
            if (yr) {
                bf16x4 b = *(const bf16x4 *)(yr + i);
                a.x += bf2f(b[0]);
                a.y += bf2f(b[1]);
                a.z += bf2f(b[2]);
                a.w += bf2f(b[3]);
                if (write_back)
                    *(float4 *)(xr + i) = a;
            }
            v[k] = a;
            ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
        }
    }
    ss = block_sum(ss, scratch);
    const float inv = rsqrtf(ss / H + eps);
    bf16 *orow = out + (size_t)r * H;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const int i = (threadIdx.x + k * NT) * 4;
        if (i < H) {
            const float4 ww = *(const float4 *)(w + i);
            bf16x4 o;
            o[0] = f2bf(v[k].x * inv * ww.x);
            o[1] = f2bf(v[k].y * inv * ww.y);
            o[2] = f2bf(v[k].z * inv * ww.z);
            o[3] = f2bf(v[k].w * inv * ww.w);
            *(bf16x4 *)(orow + i) = o;
        }
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

extern "C" hipError_t k_add_rmsnorm(float *x, const bf16_t *y, const float *w, bf16_t *out, int N,
                                    int H, float eps, const int32_t *rows, int R, hipStream_t s) {
    const int nrows = rows ? R : N;
    if (nrows <= 0)
        return hipSuccess;
    if (H % 4 || H > 16 * 4 * NT)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3((unsigned)nrows), dim3(NT), 0, s, x,
                       (const bf16 *)y, w, (bf16 *)out, H, eps, rows);
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
