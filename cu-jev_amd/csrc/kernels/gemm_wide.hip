/* Tiled MFMA GEMM for token counts past the few-token kernel (the prefill):
 * Y[N, M] = X[N, K] . W[M, K]^T, bf16 in, fp32 accumulate, W in the tiled
 * layout k_gemm_small_tile writes (the copy the few-token kernel streams, so
 * no third copy of the weights). The reference runs these projections
 * through cuBLAS GemmEx (src/kernels/elementwise.cu:56-75).
 *
 * At a few hundred tokens a library's 256x256-class tiles leave most of the
 * 256 CUs idle on the 2560-wide residual projections and pad the token
 * dimension by up to a third. Here the tile is chosen per shape, the
 * residual projections split K into fp32 partials that the residual add +
 * RMSNorm sums, and the grid is one round of workgroups:
 *
 *  - 4 waves stacked along M, one per SIMD (or 8, two per SIMD, each with
 *    half the row groups: gw_eight_waves). A wave owns RG row groups of
 *    16 weight rows and all NG token groups of 16 of the tile: RG x NG
 *    accumulators of v_mfma_f32_16x16x32_bf16 (W as the A operand). Tile
 *    64 RG x 16 NG. A wave's weight rows are its own (no fragment is loaded
 *    twice); the token fragments are shared through LDS.
 *  - K advances in 128-wide chunks of 4 k steps. A wave's A fragment for one
 *    row group and step is one contiguous 1 KiB piece of the tiled W (one
 *    16-byte buffer load per lane), loaded one chunk ahead into a ring of 4
 *    register slots.
 *  - X goes through LDS, double buffered by chunk. Each wave loads its
 *    share of chunk c+1 into registers while chunk c-1 computes and writes
 *    it into the free buffer at the start of chunk c. Every load
 *    instruction reads four whole 256-byte token rows (16 lanes per row):
 *    loading the B fragments directly (16 tokens x 16 bytes at a 32-byte
 *    stride per instruction) measured 10-15 % slower on the prefill shapes,
 *    bound by the scattered addresses rather than the bytes. The LDS image
 *    of a chunk is token-major, 256 bytes per token, with the 16-byte piece
 *    p of token t in slot p ^ (t % 16), so that the B fragment reads (16
 *    tokens at one k piece per quarter wave) hit 16 distinct 4-bank groups.
 *    Lane l of step i reads k = 64 (i/2) + 16 (l/16) + 8 (i%2) + 0..7 of the
 *    chunk, the k assignment of the tiled W, so the product is the plain
 *    dot product.
 *  - All loads go to registers, so the compiler's in-order vmcnt waits
 *    hold. (Loading X with buffer_load ... lds measured faster still, but
 *    those loads can complete out of order with the W loads to registers:
 *    a partial vmcnt wait then does not cover the W operand, and on
 *    multi-round grids the products came out wrong.)
 *  - One barrier per chunk. Loads are unconditional (chunk indices clamped,
 *    rows past N read as zero through the buffer range, row groups past M
 *    clamped and never stored).
 *  - Outputs: bf16 Y (row stride ldy); GATED: W = [gate I | up I], a wave
 *    holds RG/2 gate row groups and the same RG/2 up row groups and writes
 *    act = bf16(silu(bf16 gate) * bf16 up) [N][I]; PART: fp32 partial sums
 *    P[split][N][M] of the split's K range.
 *  - Workgroup b runs item (b % 8) * per_xcd + b / 8: the 8 XCDs take
 *    contiguous item ranges, and consecutive items (the token blocks of one
 *    weight block) share that weight block in the XCD's L2. */
#include <stdio.h>
#include <stdlib.h>

#include "common.h"
#include "kernels.h"

namespace CUJEV_KNS {
namespace {

constexpr int GW_THREADS = 256;

constexpr int GW_KC = 128;

enum { GW_PLAIN = 0, GW_GATED = 1, GW_PART = 2 };

/* A tile of 64 RG rows runs as 8 waves of RG/2 row groups (two per SIMD,
 * which hides part of each other's wait for late weight loads: 2-3 % at the
 * prefill shapes) where the halves are whole (gated: whole gate/up pairs)
 * and the wave's registers fit without scratch; else as 4 waves of RG. Each
 * output is summed by one wave in the same k order either way. */
constexpr bool gw_eight_waves(int rg, int ng, int mode) {
    return rg % 2 == 0 && (mode != GW_GATED || rg % 4 == 0) && ng % 2 == 0 && !(rg == 4 && ng == 12);
}

DEV __amdgpu_buffer_rsrc_t gw_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}
DEV bf16x8 gw_load(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    return __builtin_bit_cast(bf16x8, v);
}
typedef __attribute__((address_space(3))) unsigned char lds_u8;
DEV bf16x8 gw_lds_read(const unsigned char *base, uint32_t off) {
    return *(const __attribute__((address_space(3))) bf16x8 *)((const lds_u8 *)base + off);
}
DEV void gw_lds_write(unsigned char *base, uint32_t off, bf16x8 v) {
    *(__attribute__((address_space(3))) bf16x8 *)((lds_u8 *)base + off) = v;
}

template <int RG, int NG, int MODE, int WV>
__global__ __launch_bounds__(64 * WV, 1) void gemm_wide_kernel(
    const bf16 *__restrict__ X, int ldx, const bf16 *__restrict__ Wt, int N, int M, int K,
    int nch, int mblocks, int nblocks, int splits, int per_xcd, bf16 *__restrict__ Y, int ldy,
    float *__restrict__ P) {
    static_assert(MODE != GW_GATED || RG % 2 == 0, "gated tiles pair gate and up row groups");
    static_assert(WV == 4 || WV == 8, "4 or 8 waves stacked along M");
    static_assert((4 * NG) % WV == 0, "whole X pieces per thread");
    constexpr int BN = 16 * NG;       /* tokens per tile */
    constexpr int SPT = 4 * NG / WV;  /* X pieces a thread stages per chunk */
    constexpr int XBUF = BN * 256;    /* bytes of one X chunk: BN tokens x 128 k */
    __shared__ __attribute__((aligned(1024))) unsigned char xl[2 * XBUF];

    const int item = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
    if (item >= mblocks * nblocks * splits)
        return;
    const int nb = item % nblocks, rest = item / nblocks;
    const int sp = rest % splits, mb = rest / splits;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, c16 = lane & 15;
    const int G = M >> 4;              /* row groups in the tiled W */
    const int c0 = sp * nch;           /* first chunk of this split */

    /* this wave's row groups: gidx (unclamped, for the stores) and the
     * clamped byte offsets of their blocks at chunk 0 */
    int gidx[RG];
    uint32_t wofs[RG];
    if constexpr (MODE == GW_GATED) {
        constexpr int H = RG / 2;
        const int GI = G >> 1;
#pragma unroll
        for (int r = 0; r < H; r++) {
            gidx[r] = (mb * WV + wave) * H + r;
            const int gc = min(gidx[r], GI - 1);
            wofs[r] = (uint32_t)gc * 4096u;
            gidx[r + H] = gidx[r];
            wofs[r + H] = (uint32_t)(gc + GI) * 4096u;
        }
    } else {
#pragma unroll
        for (int r = 0; r < RG; r++) {
            gidx[r] = (mb * WV + wave) * RG + r;
            wofs[r] = (uint32_t)min(gidx[r], G - 1) * 4096u;
        }
    }
    const __amdgpu_buffer_rsrc_t wr = gw_rsrc(Wt, (uint32_t)((size_t)M * K * 2));
    const uint32_t wchunk = (uint32_t)G * 4096u; /* bytes per 128-k chunk of the tiled W */
    const uint32_t wlane = (uint32_t)lane * 16u;
    auto ldw = [&](int cl, int i, int r) {
        const uint32_t c = (uint32_t)(c0 + min(cl, nch - 1));
        return gw_load(wr, wlane, c * wchunk + wofs[r] + (uint32_t)i * 1024u);
    };

    /* X staging: instruction s of wave w loads local tokens 4 (w + WV s) +
     * 0..3 into registers, one 256-byte row per 16 lanes (lane l: 16-byte
     * piece l % 16 of token 4 (w + WV s) + l / 16), and writes piece p of
     * token t to slot p ^ (t % 16) of that token's 256-byte LDS row. t % 16
     * does not depend on s (4 WV is a multiple of 16). */
    const __amdgpu_buffer_rsrc_t xr = gw_rsrc(X, (uint32_t)((size_t)N * ldx * 2));
    const int tl0 = 4 * wave + (lane >> 4);
    const uint32_t xoff = (uint32_t)(nb * BN + tl0) * (uint32_t)ldx * 2u + (uint32_t)(c16 * 16);
    const uint32_t xstride = (uint32_t)(4 * WV) * (uint32_t)ldx * 2u; /* between instructions */
    const uint32_t xdst = (uint32_t)(tl0 * 256 + ((c16 ^ (tl0 & 15)) * 16));
    auto ldx_chunk = [&](int cl, bf16x8 (&xs)[SPT]) {
        const uint32_t kb = (uint32_t)(c0 + min(cl, nch - 1)) * (GW_KC * 2);
#pragma unroll
        for (int s = 0; s < SPT; s++)
            xs[s] = gw_load(xr, xoff + (uint32_t)s * xstride, kb);
    };
    auto stx_chunk = [&](int buf, const bf16x8 (&xs)[SPT]) {
#pragma unroll
        for (int s = 0; s < SPT; s++)
            gw_lds_write(xl, (uint32_t)(buf * XBUF + WV * s * 1024) + xdst, xs[s]);
    };
    /* B fragment (token group j, step i) of buffer b: lane l reads token
     * 16 j + l%16, piece 8 (i/2) + 2 (l/16) + i%2, from its swizzled slot */
    uint32_t boff[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        boff[i] = (uint32_t)(c16 * 256 + (((8 * (i >> 1) + 2 * q + (i & 1)) ^ c16) * 16));
    auto ldb = [&](int buf, int i, bf16x8 (&b)[NG]) {
#pragma unroll
        for (int j = 0; j < NG; j++)
            b[j] = gw_lds_read(xl, (uint32_t)(buf * XBUF + j * 4096) + boff[i]);
    };

    floatx4 acc[RG][NG];
#pragma unroll
    for (int r = 0; r < RG; r++)
#pragma unroll
        for (int j = 0; j < NG; j++)
            acc[r][j] = floatx4{};

    /* prologue in the order the loop's waits assume: at the top of every
     * chunk the 12 newest loads in flight are the W prefetches issued after
     * the staged X */
    bf16x8 w[4][RG];
    bf16x8 xs[SPT];
    ldx_chunk(0, xs);
    stx_chunk(0, xs);
    ldx_chunk(1, xs);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < RG; r++)
            w[i][r] = ldw(0, i, r);
    lds_barrier();

    bf16x8 b0[NG], b1[NG];
    /* The scheduling barriers pin the order the pipeline depends on: the X
     * loads of chunk c+2 at the top of chunk c and each step's W prefetch
     * right after its MFMAs; left alone the scheduler sinks every load to
     * the end of the chunk, where the next chunk waits for it at once. */
    for (int c = 0; c < nch; c++) {
        const int cur = c & 1;
        stx_chunk(cur ^ 1, xs); /* chunk c+1 into the buffer chunk c-1 used */
        ldx_chunk(c + 2, xs);
        ldb(cur, 0, b0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            bf16x8 (&b)[NG] = (i & 1) ? b1 : b0;
            bf16x8 (&bn)[NG] = (i & 1) ? b0 : b1;
            if (i < 3)
                ldb(cur, i + 1, bn); /* next step's B, read while these MFMAs run */
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < RG; r++)
#pragma unroll
                for (int j = 0; j < NG; j++)
                    acc[r][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w[i][r], b[j], acc[r][j],
                                                                        0, 0, 0);
#pragma unroll
            for (int r = 0; r < RG; r++)
                w[i][r] = ldw(c + 1, i, r);
            __builtin_amdgcn_sched_barrier(0);
        }
        lds_barrier();
    }

    /* acc[r][j]: token nb BN + 16 j + l%16, rows 16 g_r + 4 (l/16) + 0..3 */
    const int n0 = nb * BN + c16;
    if constexpr (MODE == GW_GATED) {
        constexpr int H = RG / 2;
        const int I = M >> 1;
#pragma unroll
        for (int r = 0; r < H; r++) {
            const int i0 = 16 * gidx[r] + 4 * q;
            if (i0 >= I)
                continue;
#pragma unroll
            for (int j = 0; j < NG; j++) {
                const int n = n0 + 16 * j;
                bf16x4 a;
#pragma unroll
                for (int e = 0; e < 4; e++)
                    a[e] = f2bf(silu_f(bf2f(f2bf(acc[r][j][e]))) * bf2f(f2bf(acc[r + H][j][e])));
                if (n < N)
                    *(bf16x4 *)(Y + (size_t)n * ldy + i0) = a;
            }
        }
    } else {
#pragma unroll
        for (int r = 0; r < RG; r++) {
            const int m = 16 * gidx[r] + 4 * q;
            if (m >= M)
                continue;
#pragma unroll
            for (int j = 0; j < NG; j++) {
                const int n = n0 + 16 * j;
                if (n >= N)
                    continue;
                if constexpr (MODE == GW_PART)
                    *(floatx4 *)(P + ((size_t)sp * N + n) * M + m) = acc[r][j];
                else
                    *(bf16x4 *)(Y + (size_t)n * ldy + m) =
                        bf16x4{f2bf(acc[r][j][0]), f2bf(acc[r][j][1]), f2bf(acc[r][j][2]),
                               f2bf(acc[r][j][3])};
            }
        }
    }
}

template <int MODE>
hipError_t launch_mode(int RG, int NG, dim3 grid, hipStream_t s, const bf16 *X, int ldx,
                       const bf16 *W, int N, int M, int K, int nch, int mblocks, int nblocks,
                       int splits, int per_xcd, bf16 *Y, int ldy, float *P) {
#define CUJEV_GW_CASE(rg, ng)                                                                \
    if (RG == rg && NG == ng) {                                                              \
        if constexpr (gw_eight_waves(rg, ng, MODE))                                         \
            hipLaunchKernelGGL((gemm_wide_kernel<rg / 2, ng, MODE, 8>), grid, dim3(512), 0, s, \
                               X, ldx, W, N, M, K, nch, mblocks, nblocks, splits, per_xcd, Y,  \
                               ldy, P);                                                      \
        else                                                                                 \
            hipLaunchKernelGGL((gemm_wide_kernel<rg, ng, MODE, 4>), grid, dim3(GW_THREADS), 0, \
                               s, X, ldx, W, N, M, K, nch, mblocks, nblocks, splits, per_xcd, \
                               Y, ldy, P);                                                   \
        return hipGetLastError();                                                            \
    }
    CUJEV_GW_CASE(2, 8)
    CUJEV_GW_CASE(2, 12)
    CUJEV_GW_CASE(4, 6)
    CUJEV_GW_CASE(4, 8)
    CUJEV_GW_CASE(4, 10)
    CUJEV_GW_CASE(4, 12)
    CUJEV_GW_CASE(6, 4)
    CUJEV_GW_CASE(6, 6)
    CUJEV_GW_CASE(6, 8)
    CUJEV_GW_CASE(8, 4)
    CUJEV_GW_CASE(8, 6)
    if constexpr (MODE != GW_GATED) {
        CUJEV_GW_CASE(3, 8)
        CUJEV_GW_CASE(3, 12)
    }
#undef CUJEV_GW_CASE
    return hipErrorInvalidValue;
}

} // namespace
} // namespace CUJEV_KNS

using namespace CUJEV_KNS;

extern "C" int cujev_gemm_wide_supported(int RG, int NG, int gated) {
    switch (RG) {
    case 2: return NG == 8 || NG == 12;
    case 3: return !gated && (NG == 8 || NG == 12);
    case 4: return NG == 6 || NG == 8 || NG == 10 || NG == 12;
    case 6: return NG == 4 || NG == 6 || NG == 8;
    case 8: return NG == 4 || NG == 6;
    default: return 0;
    }
}

/* Estimated microseconds of a plan, a linear model fitted to measured
 * launches on MI355X (the 4B prefill shapes at 256-2048 tokens, every tile
 * and split, cold weights; mean error 7 %; on the GEMM time alone its pick
 * is the measured best in 32 of 35 shape/token cases and within 11 % in
 * the rest): per
 * round of 256 workgroups, the MFMA cycles of one wave, the W and X bytes a
 * workgroup loads over its K range and the bytes its waves read from LDS,
 * plus a fixed cost per round; with splits, the fp32 partials' write and
 * the residual add's read of them (about 5 TB/s). */
static double plan_us(int N, int M, int K, int gated, int RG, int NG, int S) {
    const int rows = gated ? M / 2 : M;
    const int bm = gated ? 32 * RG : 64 * RG;
    const long mb = (rows + bm - 1) / bm, nb = (N + 16 * NG - 1) / (16 * NG);
    const long items = mb * nb * S;
    const double rounds = (double)((items + 255) / 256);
    const double nch = (double)K / GW_KC / S;
    const double mfma = nch * 4 * RG * NG * 16;
    const double wbytes = nch * 16384.0 * RG;
    const double xbytes = nch * 256.0 * 16 * NG;
    const double lds = nch * 16384.0 * NG;
    double us = rounds * (2.667e-4 * mfma + 8.406e-6 * wbytes + 1.016e-6 * xbytes +
                          4.065e-6 * lds + 4.685);
    if (S > 1) {
        const double mb_part = (double)S * N * M * 4 / 1e6;
        us += 0.1863 * mb_part + 0.2 * mb_part;
    }
    return us;
}

extern "C" int cujev_gemm_wide_plan(int N, int M, int K, int gated, int max_splits, int *RG,
                                    int *NG, int *S) {
    if (N <= 0 || M % 16 || K % GW_KC || (gated && M % 32))
        return -1;
    const char *force = getenv("CUJEV_WIDE_PLAN");
    if (force) {
        int a, b, c;
        if (sscanf(force, "%d,%d,%d", &a, &b, &c) == 3 && cujev_gemm_wide_supported(a, b, gated) &&
            c >= 1 && c <= (max_splits < 1 ? 1 : max_splits) && (K / GW_KC) % c == 0) {
            *RG = a, *NG = b, *S = c;
            return 0;
        }
    }
    double best = 1e30;
    for (int rg = 2; rg <= 8; rg++)
        for (int ng = 4; ng <= 12; ng += 2)
            for (int s = 1; s <= (max_splits < 1 ? 1 : max_splits); s++) {
                if (!cujev_gemm_wide_supported(rg, ng, gated) || (K / GW_KC) % s)
                    continue;
                const double t = plan_us(N, M, K, gated, rg, ng, s);
                if (t < best * 0.999) {
                    best = t;
                    *RG = rg, *NG = ng, *S = s;
                }
            }
    return best < 1e29 ? 0 : -1;
}

extern "C" hipError_t k_gemm_wide(const bf16_t *X, int ldx, const bf16_t *Wt, int N, int M, int K,
                                  int gated, int RG, int NG, int splits, bf16_t *Y, int ldy,
                                  float *P, hipStream_t stream) {
    if (N <= 0)
        return hipSuccess;
    if (M % 16 || K % GW_KC || splits < 1 || (K / GW_KC) % splits || ldx < K ||
        !cujev_gemm_wide_supported(RG, NG, gated) || (gated && (splits != 1 || M % 32)) ||
        (splits > 1 && !P) || (splits == 1 && !Y) ||
        (size_t)N * ldx * 2 > 0xffffffffull || (size_t)M * K * 2 > 0xffffffffull)
        return hipErrorInvalidValue;
    const int rows = gated ? M / 2 : M, bm = gated ? 32 * RG : 64 * RG;
    const int mblocks = (rows + bm - 1) / bm, nblocks = (N + 16 * NG - 1) / (16 * NG);
    const int items = mblocks * nblocks * splits, per_xcd = (items + 7) / 8;
    const dim3 grid((unsigned)(8 * per_xcd));
    const int nch = K / GW_KC / splits;
    const bf16 *x = (const bf16 *)X, *w = (const bf16 *)Wt;
    if (gated)
        return launch_mode<GW_GATED>(RG, NG, grid, stream, x, ldx, w, N, M, K, nch, mblocks,
                                     nblocks, 1, per_xcd, (bf16 *)Y, ldy, nullptr);
    if (splits > 1)
        return launch_mode<GW_PART>(RG, NG, grid, stream, x, ldx, w, N, M, K, nch, mblocks,
                                    nblocks, splits, per_xcd, nullptr, 0, P);
    return launch_mode<GW_PLAIN>(RG, NG, grid, stream, x, ldx, w, N, M, K, nch, mblocks, nblocks,
                                 1, per_xcd, (bf16 *)Y, ldy, nullptr);
}
