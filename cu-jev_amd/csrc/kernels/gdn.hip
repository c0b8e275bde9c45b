/* Gated DeltaNet for gfx950: fused conv/gates, chunked WY/UT delta rule on
 * bf16 MFMA with an fp32 recurrent state, gated RMSNorm fused into the scan.
 *
 * Semantics: REF src/kernels/gdn.cu:4-24 (conv), :26-43 (conv tail), :57-96
 * (prep), :111-182 (scan, recurrent form), :193-216 (gated norm); math of
 * transformers' torch_chunk_gated_delta_rule (modeling_qwen3_5.py:249-327).
 *
 * Pipeline per layer (all tokens of all segments in one launch each):
 *   gdn_conv_prep  (two-call form) conv(4) + SiLU, l2norm(q,k) with
 *                  q * 128^-1/2, g, beta -> fp32 q,k [N][Hk][128],
 *                  v [N][Hv][128], g, beta. The one-call layer computes the
 *                  same inside gdn_chunk_a.
 *   gdn_chunk_a    per (64-token chunk, k-head), fully parallel, for every
 *                  v-head of the k-head: G = cumsum g,
 *                  A = tril(beta_i k_i.k_j e^{G_i-G_j}, -1),
 *                  T = (I+A)^-1 by blocked forward substitution (fp32),
 *                  W = T diag(beta e^G) K, U = T diag(beta) V,
 *                  QKm = tril(q_i.k_j e^{G_i-G_j}), and once per k-head Q
 *                  and K^T  -> HBM in phase B's fragment order (bf16; U
 *                  fp32; QKm and K^T as bf16 hi + lo pairs).
 *   gdn_chunk_b    per (segment, v-head), sequential over the segment's
 *                  chunks; a workgroup owns 32 columns of S (fp32, registers):
 *                  V' = U - W S;  O = e^G (Q S) + QKm V';
 *                  S = e^{G_last} S + K^T (e^{G_last-G} V')  (bf16 MFMA, V'
 *                  and the two operands above as hi + lo products), O fp32,
 *                  then y = w * bf16(rmsnorm(O)) * silu(z) to bf16.
 * Every segment starts from S_in (the state's S, read-only) or 0 and the
 * conv taps before a segment come from the state's conv tail (or 0): branches
 * never copy the state.
 *
 * MFMA operand layouts (v_mfma_f32_32x32x16_bf16): A lane l = row l%32,
 * k 8(l/32)..+8; B lane l = col l%32, same k; C lane l = col l%32, rows
 * 8(r/4) + 4(l/32) + r%4. An accumulator used again as a B operand supplies
 * its k values in that row order, so the matching A operand is read as two
 * 4-element pieces at k offsets 4h and 8+4h of each 16-wide step. */
#include <stdlib.h>

#include "common.h"
#include "kernels.h"

namespace CUJEV_KNS {
namespace {

constexpr int DK = 128; /* key head dim   */
constexpr int DV = 128; /* value head dim */
constexpr int CH = 64;  /* chunk length   */

/* ---------------------------------------------------------------------- */
/* conv + gates                                                            */
/* ---------------------------------------------------------------------- */
/* One group of 16 lanes = one 128-channel head slice of PREP_T consecutive
 * tokens; lane s holds channels 8s..8s+7. Every load the group needs (the
 * PREP_T + 3 pre-conv rows, conv weights, the state's conv tail, segment
 * starts, b and a) is issued first, unconditionally (row indices clamped
 * into the batch; a load skipped on some path would make every later use
 * wait for all loads in flight), then the 4-tap window slides over the rows
 * in registers. Groups are numbered token block fastest, 16 per 256-thread
 * workgroup. Groups of head h < Hv also produce g and beta of v-head h. */
constexpr int PREP_T = 8;

template <bool VEC, bool TAIL>
__global__ __launch_bounds__(256) void gdn_conv_prep_kernel(
    const bf16 *__restrict__ proj, int ps, const float *__restrict__ conv_w,
    const float *__restrict__ conv_in, const int32_t *__restrict__ own_base,
    const float *__restrict__ A_neg_exp, const float *__restrict__ dt_bias, int N, int Hk, int Hv,
    float *__restrict__ qo, float *__restrict__ ko, float *__restrict__ vo, float *__restrict__ go,
    float *__restrict__ bo) {
    const int nheads = 2 * Hk + Hv;
    const int ntb = (N + PREP_T - 1) / PREP_T;
    const int grp = blockIdx.x * 16 + (threadIdx.x >> 4);
    const int s = threadIdx.x & 15;
    if (grp >= ntb * nheads)
        return; /* whole 16-lane groups leave together */
    const int head = grp / ntb, n0 = (grp - head * ntb) * PREP_T;
    const int C = nheads * DK;
    const int c0 = head * DK + 8 * s;

    /* ---- loads ---- */
    bf16x8 x[PREP_T + 3];
#pragma unroll
    for (int r = 0; r < PREP_T + 3; r++) {
        const int row = min(max(n0 - 3 + r, 0), N - 1);
        const bf16 *src = proj + (size_t)row * ps + c0;
        if constexpr (VEC) {
            x[r] = *(const bf16x8 *)src;
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++)
                x[r][e] = src[e];
        }
    }
    float w[8][4];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float4 t = *(const float4 *)(conv_w + (size_t)(c0 + e) * 4);
        w[e][0] = t.x, w[e][1] = t.y, w[e][2] = t.z, w[e][3] = t.w;
    }
    float tail[24]; /* conv_in[c0 + e][j] at 3e + j */
    if constexpr (TAIL) {
#pragma unroll
        for (int i = 0; i < 6; i++) {
            const float4 t = *(const float4 *)(conv_in + (size_t)c0 * 3 + 4 * i);
            tail[4 * i] = t.x, tail[4 * i + 1] = t.y, tail[4 * i + 2] = t.z, tail[4 * i + 3] = t.w;
        }
    }
    const int nt = min(n0 + (s & (PREP_T - 1)), N - 1); /* lane s: token n0 + s%8 */
    const int base_s = own_base[nt];
    const int hg = min(head, Hv - 1);
    const bf16 *ab = proj + (size_t)nt * ps + C + Hv * DV; /* b then a */
    const float bv = bf2f(ab[hg]), av = bf2f(ab[Hv + hg]);
    const float aneg = A_neg_exp[hg], dtb = dt_bias[hg];

    /* ---- gates ---- */
    if (head < Hv && s < PREP_T && n0 + s < N) {
        bo[(size_t)(n0 + s) * Hv + head] = sigmoid_f(bv);
        go[(size_t)(n0 + s) * Hv + head] = aneg * softplus_f(av + dtb);
    }

    /* ---- conv + SiLU (+ l2 norm) ---- */
    float *dst;
    float scale = 1.f;
    const bool norm = head < 2 * Hk;
    if (head < Hk) {
        dst = qo + (size_t)head * DK;
        scale = 0.08838834764831845f; /* 128^-1/2 */
    } else if (head < 2 * Hk) {
        dst = ko + (size_t)(head - Hk) * DK;
    } else {
        dst = vo + (size_t)(head - 2 * Hk) * DV;
    }
    const int tok_stride = head < 2 * Hk ? Hk * DK : Hv * DV;
    const int gl0 = threadIdx.x & 48; /* first lane of this group */
#pragma unroll
    for (int j = 0; j < PREP_T; j++) {
        const int n = n0 + j;
        const int local = n - __shfl(base_s, gl0 + j, 64);
        if (n >= N)
            continue; /* uniform over the group; no loads below */
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; e++)
            y[e] = 0.f;
        if (local >= 3) { /* every tap inside the segment */
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int e = 0; e < 8; e++)
                    y[e] = fmaf(w[e][i], bf2f(x[j + i][e]), y[e]);
        } else { /* taps before the segment start: the state's tail or 0 */
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tau = local - 3 + i; /* local index of the tap */
                const float mx = tau >= 0 ? 1.f : 0.f;
                const float m0 = tau == -3 ? 1.f : 0.f, m1 = tau == -2 ? 1.f : 0.f,
                            m2 = tau == -1 ? 1.f : 0.f;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    float xi = mx * bf2f(x[j + i][e]);
                    if constexpr (TAIL)
                        xi += m0 * tail[3 * e] + m1 * tail[3 * e + 1] + m2 * tail[3 * e + 2];
                    y[e] = fmaf(w[e][i], xi, y[e]);
                }
            }
        }
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            y[e] = silu_f(y[e]);
            ss += y[e] * y[e];
        }
        float inv = 1.f;
        if (norm) {
#pragma unroll
            for (int o = 1; o < 16; o <<= 1)
                ss += __shfl_xor(ss, o, 64);
            inv = rsqrtf(ss + 1e-6f) * scale;
        }
        float *d = dst + (size_t)n * tok_stride + 8 * s;
        *(float4 *)d = make_float4(y[0] * inv, y[1] * inv, y[2] * inv, y[3] * inv);
        *(float4 *)(d + 4) = make_float4(y[4] * inv, y[5] * inv, y[6] * inv, y[7] * inv);
    }
}

/* Last three pre-conv inputs of segment 0 -> conv_out[C][3] (prefill). */
__global__ void gdn_conv_tail_kernel(const bf16 *__restrict__ proj, int ps,
                                     const float *__restrict__ conv_in, float *__restrict__ conv_out,
                                     int seg_len, int C) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C)
        return;
#pragma unroll
    for (int j = 0; j < 3; j++) {
        const int t = seg_len - 3 + j;
        float x;
        if (t >= 0)
            x = bf2f(proj[(size_t)t * ps + c]);
        else
            x = conv_in ? conv_in[(size_t)c * 3 + t + 3] : 0.f;
        conv_out[(size_t)c * 3 + j] = x;
    }
}

/* ---------------------------------------------------------------------- */
/* phase A: intra-chunk WY/UT factors, written in phase B's operand layouts */
/* ---------------------------------------------------------------------- */
/* One workgroup (8 waves) per (chunk, k-head, pair of the k-head's v-heads):
 *   1. q and k rows of the k-head (conv + SiLU + l2 norm and q * 128^-1/2,
 *      or read from gdn_conv_prep's fp32 output) staged in LDS as bf16
 *      pairs hi + lo (hi = bf16(x), lo = bf16(x - hi): x to ~16 bits); the
 *      gates of both v-heads: G = cumsum g (restarted at segment starts;
 *      leaves for phase B), beta e^G, beta;
 *   2. raw K K^T (hi parts) and Q K^T (hi.hi + hi.lo + lo.hi MFMAs) in fp32,
 *      shared by both v-heads; q (bf16) leaves once per k-head;
 *   then waves 0-3 serve the first v-head and waves 4-7 the second, side by
 *   side:
 *   3. the masked QK^T (hi + lo) leaves; A = tril(beta_i e^{G_i-G_j}
 *      k_i.k_j, -1) (fp32); K^T from the exact k rows leaves as hi + lo,
 *      once per k-head (phase B scales V' by e^{G_last-G} instead, and
 *      Q S by e^G, so the k-head's v-heads share Q and K^T);
 *   4. the v rows of both v-heads (hi + lo) where the q rows and the raw
 *      products were; T = (I + A)^-1 in place (fp32, blocked forward
 *      substitution);
 *   5. W = T (beta e^G K) (bf16) and U = T (beta V) with V exact (hi and lo
 *      MFMAs; U kept fp32), staged row-major, then stored in the fragment
 *      order phase B reads.
 * Which operands carry lo parts follows from where a bf16 rounding moves
 * the layer output: q and k in QK^T, v in U, k in K^T, and U, QK^T, K^T
 * and V' themselves each cost about as much as the reference's own bf16
 * round trip in the gated norm; K K^T, W, T, Q and the bf16 copy of S that
 * the W S and Q S products read each cost under a tenth of that.
 * A chunk may hold several whole segments (chunk_starts marks where each
 * begins): G restarts at every segment start and A and QK^T are kept
 * block-diagonal, so the segments do not see each other. This is valid for
 * branches that all continue one state and write no final state: phase B
 * then needs nothing per segment. */
constexpr int PA_THREADS = 512;
constexpr int PA_STAGE1 = 8 * 16 * 4 + 3 * 128; /* floats of one slice's conv weights + tail */

struct __attribute__((aligned(16))) PairA_Smem {
    bf16 Kh[CH][DK + 8], Kl[CH][DK + 8]; /* k rows, hi and lo parts                   */
    /* X: q rows (hi, lo); then the first v-head's v rows; then its U staging
     * (fp32 [CH][DV + 4]). Y: raw k_i.k_j and q_i.k_j (fp32 [CH][CH + 4]
     * each); then the second v-head's v rows; then its U staging. */
    bf16 Xh[CH][DK + 8], Xl[CH][DK + 8];
    bf16 Yh[CH][DK + 8], Yl[CH][DK + 8];
    float AT[2][CH][CH + 4];             /* A, then T in place; then W staging    */
    float cs[2 * PA_STAGE1];             /* conv weights and tails of two slices  */
    float G[2][CH], sK[2][CH], sV[2][CH]; /* per v-head of the pair */
    int Sid[CH]; /* segment of each token inside a packed chunk (1-based) */
};
static_assert(sizeof(PairA_Smem) <= 160 * 1024, "phase A fits one CU's LDS");
static_assert(2 * sizeof(bf16) * CH * (DK + 8) >= sizeof(float) * CH * (DV + 4), "U staging");
static_assert(sizeof(bf16) * CH * (DK + 8) >= sizeof(float) * CH * (CH + 4), "raw products");
static_assert(sizeof(float) * CH * (CH + 4) >= sizeof(bf16) * CH * (DK + 8), "W staging");

DEV bf16x8 ld8(const bf16 *p) { return *(const bf16x8 *)p; }
DEV float4 rd4(const float *p) { return *(const float4 *)p; }
DEV void wr4(float *p, float4 v) { *(float4 *)p = v; }
DEV float4 f4fma(float a, float4 b, float4 c) {
    return make_float4(fmaf(a, b.x, c.x), fmaf(a, b.y, c.y), fmaf(a, b.z, c.z), fmaf(a, b.w, c.w));
}
/* x, through an empty asm: the compiler cannot treat what is derived from it
 * as loop-invariant (keeps per-iteration index math inside a loop instead
 * of hoisting dozens of indices out of it into scratch memory). */
DEV int opaque(int x) {
    asm volatile("" : "+v"(x));
    return x;
}
/* hi = bf16(x), lo = bf16(x - hi) */
struct bfpair {
    bf16 hi, lo;
};
DEV bfpair split2(float x) {
    const bf16 hi = f2bf(x);
    return {hi, f2bf(x - bf2f(hi))};
}

/* X[r][c0..c0+3] = sum_{k<n} P[r][k] Q[k][c0..c0+3] over fp32 LDS rows of pitch CH+4 */
template <int n>
DEV float4 row_times(const float *P, const float *Qm) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k4 = 0; k4 < n; k4 += 4) {
        const float4 p = rd4(P + k4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float pe = e == 0 ? p.x : e == 1 ? p.y : e == 2 ? p.z : p.w;
            acc = f4fma(pe, rd4(Qm + (k4 + e) * (CH + 4)), acc);
        }
    }
    return acc;
}

/* The pre-conv inputs of the fused front end (gdn_conv_prep's arguments). */
struct ConvSrc {
    const bf16 *proj;
    int ps;
    const float *conv_w, *conv_in;
    const int32_t *own_base;
    const float *A_neg_exp, *dt_bias;
    int N;
};

/* The state's new conv tail (prefill): extra workgroups of the phase B grid
 * copy it, beside the recurrence, which leaves most CUs idle. */
struct TailJob {
    const bf16 *proj;
    int ps;
    const float *conv_in;
    float *conv_out; /* NULL: no tail */
    int seg0_len, C;
};

/* Conv weights and the state's tail (the same for every token block) of
 * `nsl` 128-channel slices starting at channel c0[sl] -> LDS:
 * cw[(sl*8 + e)*16 + s] float4 and ct[(sl*3 + j)*128 + e*16 + s] for
 * channel 8s + e of slice sl. */
template <bool TAIL>
DEV void conv_stage(const ConvSrc &cv, const int *c0, int nsl, int tid, int nthr, float *cw,
                    float *ct) {
    for (int i = tid; i < nsl * DK; i += nthr) {
        const int sl = i / DK, c = i % DK, cg = c0[sl] + c;
        const int slot = (sl * 8 + (c & 7)) * 16 + (c >> 3);
        *(float4 *)&cw[slot * 4] = *(const float4 *)(cv.conv_w + (size_t)cg * 4);
        if constexpr (TAIL) {
#pragma unroll
            for (int j = 0; j < 3; j++)
                ct[(sl * 3 + j) * 128 + (c & 7) * 16 + (c >> 3)] = cv.conv_in[(size_t)cg * 3 + j];
        }
    }
}

/* 32-bit element offsets (rows x stride stays far below 2^31): one register
 * per row address instead of two. */
DEV void conv_rows(const ConvSrc &cv, int c0, int n0, bf16x8 (&x)[7]) {
#pragma unroll
    for (int i = 0; i < 7; i++) {
        const int row = min(max(n0 - 3 + i, 0), cv.N - 1);
        x[i] = ld8(cv.proj + (unsigned)(row * cv.ps + c0));
    }
}

/* Sum over each row of 16 lanes with DPP moves (no LDS round trip). The
 * quad steps leave identical sums in the 4 lanes of a quad, so the half-row
 * and row mirrors read the same values as xor 4 and xor 8 would: the result
 * equals the xor butterfly's bit for bit. */
template <int CTRL> DEV float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL,
                                                              0xf, 0xf, false));
}
DEV float sum16_dpp(float v) {
    v += dpp<0xB1>(v);  /* quad_perm [1,0,3,2]: lane ^ 1 */
    v += dpp<0x4E>(v);  /* quad_perm [2,3,0,1]: lane ^ 2 */
    v += dpp<0x141>(v); /* row_half_mirror: the other quad of 8 */
    v += dpp<0x140>(v); /* row_mirror: the other half of 16 */
    return v;
}

/* One 128-channel slice of 4 consecutive tokens (token block tb of the
 * chunk) through conv + SiLU (+ l2 norm and scale), with gdn_conv_prep's
 * arithmetic step for step; the fp32 results go to LDS as hi + lo. Lane s
 * of the 16-lane group owns channels 8s..8s+7; sl indexes the staged
 * weights / tail. */
template <bool TAIL>
DEV void conv_slice(const bf16x8 (&x)[7], const int (&base)[4], const float *cw, const float *ct,
                    int sl, bool norm, float scale, int t0, int L, int tb, int s,
                    bf16 (*dh)[DK + 8], bf16 (*dl)[DK + 8]) {
    float w[8][4];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float4 t = *(const float4 *)&cw[((sl * 8 + e) * 16 + s) * 4];
        w[e][0] = t.x, w[e][1] = t.y, w[e][2] = t.z, w[e][3] = t.w;
    }
    float xf[7][8];
#pragma unroll
    for (int i = 0; i < 7; i++)
#pragma unroll
        for (int e = 0; e < 8; e++)
            xf[i][e] = bf2f(x[i][e]);
    /* All 4 tokens in one segment (the usual case): rows before its start
     * are replaced by the tail (or 0) once, and every token takes the plain
     * 4-tap path. This is exactly the masked form below, whose single
     * nonzero term is that same value. */
    const int n0 = t0 + 4 * tb;
    const bool one_seg = base[0] == base[3];
    if (one_seg && n0 - 3 < base[0]) {
#pragma unroll
        for (int i = 0; i < 7; i++) {
            const int k = n0 - 3 + i - base[0] + 3; /* tail slot of the row */
            if (k < 3) {
#pragma unroll
                for (int e = 0; e < 8; e++)
                    xf[i][e] = TAIL && k >= 0 ? ct[(sl * 3 + max(k, 0)) * 128 + e * 16 + s] : 0.f;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int tt = 4 * tb + j, local = t0 + tt - base[j];
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; e++)
            y[e] = 0.f;
        if (one_seg || local >= 3) { /* every tap inside the segment */
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int e = 0; e < 8; e++)
                    y[e] = fmaf(w[e][i], xf[j + i][e], y[e]);
        } else { /* taps before the segment start: the state's tail or 0 */
            float tail[3][8];
#pragma unroll
            for (int q = 0; q < 3; q++)
#pragma unroll
                for (int e = 0; e < 8; e++)
                    tail[q][e] = TAIL ? ct[(sl * 3 + q) * 128 + e * 16 + s] : 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tau = local - 3 + i;
                const float mx = tau >= 0 ? 1.f : 0.f;
                const float m0 = tau == -3 ? 1.f : 0.f, m1 = tau == -2 ? 1.f : 0.f,
                            m2 = tau == -1 ? 1.f : 0.f;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    float xi = mx * xf[j + i][e];
                    if constexpr (TAIL)
                        xi += m0 * tail[0][e] + m1 * tail[1][e] + m2 * tail[2][e];
                    y[e] = fmaf(w[e][i], xi, y[e]);
                }
            }
        }
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            y[e] = silu_f(y[e]);
            ss += y[e] * y[e];
        }
        float inv = 1.f;
        if (norm) {
            ss = sum16_dpp(ss);
            inv = rsqrtf(ss + 1e-6f) * scale;
        }
        bf16x8 oh, ol;
#pragma unroll
        for (int e = 0; e < 8; e++)
            { const bfpair sp_ = split2(tt < L ? y[e] * inv : 0.f); oh[e] = sp_.hi; ol[e] = sp_.lo; }
        *(bf16x8 *)&dh[tt][8 * s] = oh;
        *(bf16x8 *)&dl[tt][8 * s] = ol;
    }
}

/* fp32 rows [CH][128] of gdn_conv_prep's output (row stride `rs` floats,
 * rows t >= L zero) -> LDS hi + lo, over `nthr` threads. */
DEV void rows_f32(const float *src, size_t rs, int L, int tid, int nthr, bf16 (*dh)[DK + 8],
                  bf16 (*dl)[DK + 8]) {
    for (int i = tid; i < CH * 16; i += nthr) {
        const int t = i >> 4, c8 = (i & 15) * 8;
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
        if (t < L) {
            a = *(const float4 *)(src + t * rs + c8);
            b = *(const float4 *)(src + t * rs + c8 + 4);
        }
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        bf16x8 oh, ol;
#pragma unroll
        for (int e = 0; e < 8; e++)
            { const bfpair sp_ = split2(v[e]); oh[e] = sp_.hi; ol[e] = sp_.lo; }
        *(bf16x8 *)&dh[t][c8] = oh;
        *(bf16x8 *)&dl[t][c8] = ol;
    }
}

/* SRC 0: q, k, v, g, beta read from gdn_conv_prep's outputs (fp32); 1: computed
 * here from the pre-conv projection rows (zeros before a segment); 2: the
 * same with the state's conv tail before each segment. Grid: (chunk,
 * k-head x pairs of its v-heads); npairs = ceil(Hv / Hk / 2). */
template <int SRC>
__global__ __launch_bounds__(PA_THREADS, 1) void gdn_chunk_a_kernel(
    const float *__restrict__ qh, const float *__restrict__ kh_, const float *__restrict__ vh,
    const float *__restrict__ g, const float *__restrict__ beta, ConvSrc cv,
    const int32_t *__restrict__ chunk_tok0, const int32_t *__restrict__ chunk_len,
    const uint64_t *__restrict__ chunk_starts, int Hk, int Hv, int npairs,
    bf16 *__restrict__ Wo, bf16 *__restrict__ Qo, bf16 *__restrict__ QKo,
    bf16 *__restrict__ KTo, float *__restrict__ Uo, float *__restrict__ Go) {
    __shared__ PairA_Smem sm;
    const int ch = blockIdx.x, hk = blockIdx.y / npairs, pr = blockIdx.y - hk * npairs;
    const int rep = Hv / Hk;
    const int hv0 = hk * rep + 2 * pr;   /* the pair's first v-head */
    const int nh = min(2, rep - 2 * pr); /* 1 or 2 v-heads */
    const int t0 = chunk_tok0[ch], L = chunk_len[ch];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, col = lane & 31;
    const int grp = tid >> 4, s16 = tid & 15; /* 32 groups of 16 lanes */
    const int nblk = (L + 3) >> 2;            /* 4-token blocks holding tokens */
    const int C = (2 * Hk + Hv) * DK;
    /* the v-head of this wave's group (waves 0-3: first, 4-7: second) */
    const int hg = wave >> 2, w4 = wave & 3;
    const bool hact = hg < nh;
    const size_t cbg = (size_t)ch * Hv + hv0 + hg;
    /* segments packed into the chunk: bit t set where token t starts one */
    const uint64_t starts = chunk_starts ? chunk_starts[ch] | 1ull : 1ull;
    const uint64_t upto = lane == 63 ? ~0ull : (2ull << lane) - 1;
    bf16(*Vh)[DK + 8] = hg ? sm.Yh : sm.Xh; /* this group's v rows (step 4 on) */
    bf16(*Vl)[DK + 8] = hg ? sm.Yl : sm.Xl;
    float(*KK)[CH + 4] = reinterpret_cast<float(*)[CH + 4]>(&sm.Yh[0][0]);
    float(*QK)[CH + 4] = reinterpret_cast<float(*)[CH + 4]>(&sm.Yl[0][0]);
    float(*AT)[CH + 4] = sm.AT[hg];

    /* ---- 1. q and k rows (hi + lo); gates of the pair (waves 4, 5) ---- */
    if constexpr (SRC == 0) {
        rows_f32(qh + ((size_t)t0 * Hk + hk) * DK, (size_t)Hk * DK, L, tid, PA_THREADS, sm.Xh,
                 sm.Xl);
        rows_f32(kh_ + ((size_t)t0 * Hk + hk) * DK, (size_t)Hk * DK, L, tid, PA_THREADS, sm.Kh,
                 sm.Kl);
    } else {
        constexpr bool TAIL = SRC == 2;
        /* (slice, 4-token block) tasks, one per 16-lane group: every
         * pre-conv row in flight first, then weights and tail into LDS */
        const int ntask = 2 * nblk;
        bf16x8 xr[7];
        int base[4];
        if (grp < ntask) {
            const int sl = grp / nblk, n0 = t0 + 4 * (grp - sl * nblk);
            conv_rows(cv, (sl == 0 ? hk : Hk + hk) * DK + 8 * s16, n0, xr);
#pragma unroll
            for (int j = 0; j < 4; j++)
                base[j] = cv.own_base[min(n0 + j, cv.N - 1)];
        }
        const int c0s[2] = {hk * DK, (Hk + hk) * DK};
        conv_stage<TAIL>(cv, c0s, 2, tid, PA_THREADS, sm.cs, sm.cs + 2 * 8 * 16 * 4);
        const int zrows = CH - 4 * nblk; /* rows of blocks without tokens: zeros */
        for (int i = tid; i < 4 * zrows * 16; i += PA_THREADS) {
            const int a = i / (zrows * 16), rem = i - a * zrows * 16;
            bf16(*z)[DK + 8] = a == 0 ? sm.Xh : a == 1 ? sm.Xl : a == 2 ? sm.Kh : sm.Kl;
            *(bf16x8 *)&z[4 * nblk + (rem >> 4)][8 * (rem & 15)] = bf16x8{};
        }
        lds_barrier();
        if (grp < ntask) {
            const int sl = grp / nblk, tb = grp - sl * nblk;
            conv_slice<TAIL>(xr, base, sm.cs, sm.cs + 2 * 8 * 16 * 4, sl, true,
                             sl == 0 ? 0.08838834764831845f /* 128^-1/2 */ : 1.f, t0, L, tb, s16,
                             sl == 0 ? sm.Xh : sm.Kh, sl == 0 ? sm.Xl : sm.Kl);
        }
    }
    if (wave == 7)
        sm.Sid[lane] = __builtin_popcountll(starts & upto);
    if (wave >= 4 && wave - 4 < nh) {
        const int r = wave - 4, hv = hv0 + r;
        float gv = 0.f, bv = 0.f;
        if (lane < L) {
            if constexpr (SRC == 0) {
                gv = g[(size_t)(t0 + lane) * Hv + hv];
                bv = beta[(size_t)(t0 + lane) * Hv + hv];
            } else {
                const bf16 *ab = cv.proj + (size_t)(t0 + lane) * cv.ps + C + Hv * DV;
                bv = sigmoid_f(bf2f(ab[hv]));
                gv = cv.A_neg_exp[hv] * softplus_f(bf2f(ab[Hv + hv]) + cv.dt_bias[hv]);
            }
        }
        /* st = first token of this lane's segment, en = its last */
        const int st = 63 - __builtin_clzll(starts & upto);
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) { /* cumulative sum restarted per segment */
            const float up = __shfl_up(gv, o, 64);
            if (lane - o >= st)
                gv += up;
        }
        sm.G[r][lane] = gv;
        sm.sK[r][lane] = bv * fast_exp(gv);
        sm.sV[r][lane] = bv;
        /* past the chunk's end g = 0: those lanes repeat the last token's G,
         * so G[63] is the chunk's total log-decay */
        Go[((size_t)ch * Hv + hv) * 64 + lane] = gv;
    }
    lds_barrier();

    /* ---- 2. raw Q K^T (split) on waves 0-2, K K^T on waves 3, 6, 7: the
     * lower 32x32 tiles (0,0), (1,0), (1,1) | q of the k-head, once per
     * k-head (waves 4-7 of its first workgroup, 16x16x32 A-fragment order:
     * entry i holds row 16(i/256) + i%16, columns 32((i/64)%4) +
     * 8((i/16)%4) .. +7; phase B applies each v-head's e^G to Q S) | every
     * group: the pre-conv rows of its v-conv task (slice = v-head grp/16,
     * block grp%16) ---- */
    constexpr bool CONV = SRC != 0;
    bf16x8 vr[7];
    int vbase[4];
    const int vsl = grp >> 4, vtb = grp & 15;
    const bool vtask = CONV && vsl < nh && vtb < nblk;
    if constexpr (CONV) {
        if (vtask) {
            const int n0 = t0 + 4 * vtb;
            conv_rows(cv, (2 * Hk + hv0 + vsl) * DK + 8 * s16, n0, vr);
#pragma unroll
            for (int j = 0; j < 4; j++)
                vbase[j] = cv.own_base[min(n0 + j, cv.N - 1)];
        }
    }
    {
        const bool isqk = wave < 3;
        const int job = wave < 3 ? wave : wave == 3 ? 0 : wave >= 6 ? wave - 5 : -1;
        floatx16 acc = {};
        const int ti = job == 0 ? 0 : 1, tj = job == 2 ? 1 : 0;
        if (job >= 0) {
#pragma unroll
            for (int ks = 0; ks < DK / 16; ks++) {
                const int c = 16 * ks + 8 * h;
                const bf16x8 bkh = ld8(&sm.Kh[32 * tj + col][c]);
                if (isqk) {
                    const bf16x8 aqh = ld8(&sm.Xh[32 * ti + col][c]);
                    const bf16x8 aql = ld8(&sm.Xl[32 * ti + col][c]);
                    const bf16x8 bkl = ld8(&sm.Kl[32 * tj + col][c]);
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aqh, bkh, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aqh, bkl, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aql, bkh, acc, 0, 0, 0);
                } else {
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ld8(&sm.Kh[32 * ti + col][c]),
                                                                  bkh, acc, 0, 0, 0);
                }
            }
        }
        if (wave >= 4 && pr == 0) { /* q rounded once: its hi part */
            const int u = tid - 256, t = u & 15, c8 = 32 * ((u >> 6) & 3) + 8 * ((u >> 4) & 3);
            const size_t ck = (size_t)ch * Hk + hk;
#pragma unroll
            for (int j = 0; j < 4; j++)
                *(bf16x8 *)(Qo + (ck * 1024 + u + 256 * j) * 8) = ld8(&sm.Xh[16 * j + t][c8]);
        }
        /* the raw products go where the second v-head's v rows will be */
        if (job >= 0) {
            float(*dst)[CH + 4] = isqk ? QK : KK;
#pragma unroll
            for (int r = 0; r < 16; r++)
                dst[32 * ti + 8 * (r >> 2) + 4 * h + (r & 3)][32 * tj + col] = acc[r];
        }
    }
    lds_barrier();

    bf16x8 eye[2]; /* B operand of the identity, k = 16s + 8h + e */
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
        for (int e = 0; e < 8; e++)
            eye[s][e] = f2bf(16 * s + 8 * h + e == col ? 1.f : 0.f);
    /* token of accumulator slot r of 32-row tile tb */
    auto tok = [&](int tb, int r) { return 32 * tb + 8 * (r >> 2) + 4 * h + (r & 3); };
    const float *Gg = sm.G[hg];

    /* ---- 3. per group (its v-head): masked QK^T hi + lo and A; the first
     * group of a k-head's first workgroup: K^T hi + lo for dk block 32 w4
     * (phase B applies each v-head's e^{G_last-G} to V'); the v-conv
     * weights ---- */
    if (hact) {
        const int u = tid & 255;
        /* masked QK^T = tril(q_i.k_j e^{G_i-G_j}) within a segment, as hi
         * and lo 16x16x32 A fragments: entry i holds row 16(i/128) + i%16,
         * columns 32((i/64)%2) + 8((i/16)%4) .. +7 */
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int i = u + 256 * j;
            const int rr = 16 * (i >> 7) + (i & 15), c8 = 32 * ((i >> 6) & 1) + 8 * ((i >> 4) & 3);
            const float Gi = Gg[rr];
            const int Si = sm.Sid[rr];
            const float4 q0 = rd4(&QK[rr][c8]), q1 = rd4(&QK[rr][c8 + 4]);
            const float qv[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
            bf16x8 oh, ol;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int cj = c8 + e;
                const bool keep = rr >= cj && Si == sm.Sid[cj];
                const bfpair sp = split2(keep ? qv[e] * fast_exp(fminf(Gi - Gg[cj], 0.f)) : 0.f);
                oh[e] = sp.hi;
                ol[e] = sp.lo;
            }
            *(bf16x8 *)(QKo + (cbg * 1024 + i) * 8) = oh;
            *(bf16x8 *)(QKo + (cbg * 1024 + 512 + i) * 8) = ol;
        }
        /* A = tril(beta_i e^{G_i-G_j} k_i.k_j, -1) within a segment, zero
         * elsewhere (the inverse reads the upper part of its blocks): row
         * u/4, columns 16(u%4) .. +15 */
        {
            const int ri = u >> 2, c16b = 16 * (u & 3);
            const float Gi = Gg[ri], bi = sm.sV[hg][ri];
            const int Si = sm.Sid[ri];
#pragma unroll
            for (int c4 = 0; c4 < 16; c4 += 4) {
                const float4 kk = rd4(&KK[ri][c16b + c4]);
                const float kv[4] = {kk.x, kk.y, kk.z, kk.w};
                float a[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int cj = c16b + c4 + e;
                    const bool keep = ri > cj && Si == sm.Sid[cj];
                    a[e] = keep ? bi * kv[e] * fast_exp(fminf(Gi - Gg[cj], 0.f)) : 0.f;
                }
                wr4(&AT[ri][c16b + c4], make_float4(a[0], a[1], a[2], a[3]));
            }
        }
    }
    if (hg == 0 && pr == 0) {
        /* K^T as 32x32x16 A fragments (row dk = 32 w4 + l%32, tokens 16s +
         * 8(l/32)..+7) from the exact k rows (identity products of hi and
         * lo); the lane pair (l, l^32) trades halves */
        const size_t ck = (size_t)ch * Hk + hk;
        floatx16 dK[2];
#pragma unroll
        for (int tb = 0; tb < 2; tb++) {
            dK[tb] = floatx16{};
#pragma unroll
            for (int s = 0; s < 2; s++) {
                const int c = 32 * w4 + 16 * s + 8 * h;
                dK[tb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ld8(&sm.Kh[32 * tb + col][c]),
                                                                 eye[s], dK[tb], 0, 0, 0);
                dK[tb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ld8(&sm.Kl[32 * tb + col][c]),
                                                                 eye[s], dK[tb], 0, 0, 0);
            }
        }
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int tb = s >> 1, r0 = 8 * (s & 1);
            bf16 vh_[8], vl_[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const bfpair sp = split2(dK[tb][r0 + e]);
                vh_[e] = sp.hi;
                vl_[e] = sp.lo;
            }
#pragma unroll
            for (int part = 0; part < 2; part++) {
                const bf16 *v = part ? vl_ : vh_;
                uint32_t p0[2], p1[2];
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    p0[e] = __builtin_bit_cast(uint32_t, bf16x2{v[2 * e], v[2 * e + 1]});
                    p1[e] = __builtin_bit_cast(uint32_t, bf16x2{v[4 + 2 * e], v[5 + 2 * e]});
                }
                uint32_t o[4];
#pragma unroll
                for (int e = 0; e < 2; e++) { /* h=0 holds tokens +0..3 | +8..11 */
                    const uint32_t x1 = (uint32_t)__shfl_xor((int)p1[e], 32, 64);
                    const uint32_t x0 = (uint32_t)__shfl_xor((int)p0[e], 32, 64);
                    o[e] = h ? x1 : p0[e];
                    o[2 + e] = h ? p1[e] : x0;
                }
                *(u32x4 *)(KTo + (ck * 2048 + part * 1024 + (w4 * 4 + s) * 64 + lane) * 8) =
                    u32x4{o[0], o[1], o[2], o[3]};
            }
        }
    }
    if constexpr (CONV) {
        int c0s[2] = {(2 * Hk + hv0) * DK, (2 * Hk + hv0 + 1) * DK};
        conv_stage<SRC == 2>(cv, c0s, nh, tid, PA_THREADS, sm.cs, sm.cs + 2 * 8 * 16 * 4);
    }
    lds_barrier(); /* the q rows and the raw products are no longer read */

    /* ---- 4. the v rows of both v-heads (hi + lo) | T = (I + A)^-1 ----
     * 4a: wave w4 of each group inverts diagonal block w4 of its A, lane
     * c < 16 owning column c; the block is read (all lanes, broadcast)
     * before any lane writes it. */
    if constexpr (SRC == 0) {
        for (int r = 0; r < nh; r++)
            rows_f32(vh + ((size_t)t0 * Hv + hv0 + r) * DV, (size_t)Hv * DV, L, tid, PA_THREADS,
                     r ? sm.Yh : sm.Xh, r ? sm.Yl : sm.Xl);
    } else {
        const int zrows = CH - 4 * nblk;
        for (int i = tid; i < 2 * nh * zrows * 16; i += PA_THREADS) {
            const int a = i / (zrows * 16), rem = i - a * zrows * 16;
            bf16(*z)[DK + 8] = a == 0 ? sm.Xh : a == 1 ? sm.Xl : a == 2 ? sm.Yh : sm.Yl;
            *(bf16x8 *)&z[4 * nblk + (rem >> 4)][8 * (rem & 15)] = bf16x8{};
        }
        if (vtask)
            conv_slice<SRC == 2>(vr, vbase, sm.cs, sm.cs + 2 * 8 * 16 * 4, vsl, false, 1.f, t0, L,
                                 vtb, s16, vsl ? sm.Yh : sm.Xh, vsl ? sm.Yl : sm.Xl);
    }
    if (hact && lane < 16) {
        const int b0 = 16 * w4, c = lane;
        float t[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            float acc = 0.f;
#pragma unroll
            for (int k4 = 0; k4 < i; k4 += 4) {
                const float4 a = rd4(&AT[b0 + i][b0 + k4]);
                acc = fmaf(a.x, t[k4], acc);
                if (k4 + 1 < i)
                    acc = fmaf(a.y, t[k4 + 1], acc);
                if (k4 + 2 < i)
                    acc = fmaf(a.z, t[k4 + 2], acc);
                if (k4 + 3 < i)
                    acc = fmaf(a.w, t[k4 + 3], acc);
            }
            t[i] = (i == c ? 1.f : 0.f) - acc;
        }
#pragma unroll
        for (int i = 0; i < 16; i++)
            if (i >= c)
                AT[b0 + i][b0 + c] = t[i];
    }
    lds_barrier();
    /* 4b: inside 32x32 diagonal block p (wave w4 = p): T_10 = -T_11 (A_10
     * T_00), 16x16 blocks; lane = (row l/4, columns 4(l%4)..+3) */
    if (hact && w4 < 2) {
        const int p0 = 32 * w4, rr = lane >> 2, c0 = 4 * (lane & 3);
        float *a10 = &AT[p0 + 16 + rr][p0];
        const float4 x = row_times<16>(a10, &AT[p0][p0 + c0]);
        wr4(a10 + c0, x);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const float4 y = row_times<16>(&AT[p0 + 16 + rr][p0 + 16], &AT[p0 + 16][p0 + c0]);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wr4(a10 + c0, make_float4(-y.x, -y.y, -y.z, -y.w));
    }
    lds_barrier();
    /* 4c: T_10 = -T_11 (A_10 T_00) with 32x32 blocks; lane = (row 8 w4 +
     * l/8, columns 4(l%8)..+3). A chunk of at most 32 tokens has A_10 = 0
     * and so T_10 = 0, which the array already holds. Every wave passes the
     * same barriers. */
    if (L > 32) {
        const int rr = 32 + 8 * w4 + (lane >> 3), c0 = 4 * (lane & 7);
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        if (hact)
            x = row_times<32>(&AT[rr][0], &AT[0][c0]);
        lds_barrier();
        if (hact)
            wr4(&AT[rr][c0], x);
        lds_barrier();
        float4 y = x;
        if (hact)
            y = row_times<32>(&AT[rr][32], &AT[32][c0]);
        lds_barrier();
        if (hact)
            wr4(&AT[rr][c0], make_float4(-y.x, -y.y, -y.z, -y.w));
        lds_barrier();
    }

    /* ---- 5. per group: W = T (beta e^G K) (dk block 32 w4, K hi) and
     * U = T (beta V) (dv block 32 w4, V hi + lo) ---- */
    {
        const float *sKr = sm.sK[hg], *sVr = sm.sV[hg];
        floatx16 accw[2] = {}, accu[2] = {};
        if (hact) {
            floatx16 dX[2], dV[2]; /* rows 32tb.. of K (V), columns 32 w4.. */
#pragma unroll
            for (int tb = 0; tb < 2; tb++) {
                dX[tb] = dV[tb] = floatx16{};
#pragma unroll
                for (int s = 0; s < 2; s++) {
                    const int c = 32 * w4 + 16 * s + 8 * h;
                    dX[tb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ld8(&sm.Kh[32 * tb + col][c]),
                                                                     eye[s], dX[tb], 0, 0, 0);
                    dV[tb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ld8(&Vh[32 * tb + col][c]),
                                                                     eye[s], dV[tb], 0, 0, 0);
                    dV[tb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ld8(&Vl[32 * tb + col][c]),
                                                                     eye[s], dV[tb], 0, 0, 0);
                }
            }
            /* B operands: token k-steps ks (tile ks/2, rows 8(ks%2)..) times
             * beta e^G (K) or beta (V, kept as hi + lo) */
            bf16x8 xk[4], xvh[4], xvl[4];
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                const int tb = ks >> 1, r0 = 8 * (ks & 1);
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int t = tok(tb, r0 + e);
                    xk[ks][e] = f2bf(dX[tb][r0 + e] * sKr[t]);
                    const bfpair sp = split2(dV[tb][r0 + e] * sVr[t]);
                    xvh[ks][e] = sp.hi;
                    xvl[ks][e] = sp.lo;
                }
            }
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
#pragma unroll
                for (int mi = 0; mi < 2; mi++) {
                    /* T row 32mi + col, columns in the accumulator order */
                    const float *tr = &AT[32 * mi + col][16 * ks + 4 * h];
                    const float4 a0 = rd4(tr), a1 = rd4(tr + 8);
                    const bf16x8 a = {f2bf(a0.x), f2bf(a0.y), f2bf(a0.z), f2bf(a0.w),
                                      f2bf(a1.x), f2bf(a1.y), f2bf(a1.z), f2bf(a1.w)};
                    accw[mi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, xk[ks], accw[mi], 0, 0, 0);
                    accu[mi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, xvh[ks], accu[mi], 0, 0, 0);
                    accu[mi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, xvl[ks], accu[mi], 0, 0, 0);
                }
            }
        }
        lds_barrier(); /* every wave is done with T and the v rows */
        if (hact) {
            bf16(*Wst)[DK + 8] = reinterpret_cast<bf16(*)[DK + 8]>(&AT[0][0]);
            float(*Ust)[DV + 4] = reinterpret_cast<float(*)[DV + 4]>(&Vh[0][0]);
#pragma unroll
            for (int mi = 0; mi < 2; mi++)
#pragma unroll
                for (int rr = 0; rr < 16; rr++) {
                    Wst[tok(mi, rr)][32 * w4 + col] = f2bf(accw[mi][rr]);
                    Ust[tok(mi, rr)][32 * w4 + col] = accu[mi][rr];
                }
        }
    }
    lds_barrier();
    /* ---- 6. W in the fragment order of Q; U (fp32) as 16x16
     * accumulator fragments: entry i = (32-column block i/256, row block
     * (i/64)%4, lane i%64) holds rows 16((i/64)%4) + 4((i/16)%4) + 0..3 of
     * columns 32(i/256) + i%16 (values 0..3) and +16 (values 4..7) ---- */
    if (hact) {
        bf16(*Wst)[DK + 8] = reinterpret_cast<bf16(*)[DK + 8]>(&AT[0][0]);
        float(*Ust)[DV + 4] = reinterpret_cast<float(*)[DV + 4]>(&Vh[0][0]);
        const int u = tid & 255;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i = u + 256 * j;
            const int t = 16 * (i >> 8) + (i & 15), c8 = 32 * ((i >> 6) & 3) + 8 * ((i >> 4) & 3);
            *(bf16x8 *)(Wo + (cbg * 1024 + i) * 8) = ld8(&Wst[t][c8]);
            const int tu = 16 * ((i >> 6) & 3) + 4 * ((i >> 4) & 3), cu = 32 * (i >> 8) + (i & 15);
            float *dst = Uo + (cbg * 1024 + i) * 8;
            *(float4 *)dst = make_float4(Ust[tu][cu], Ust[tu + 1][cu], Ust[tu + 2][cu],
                                         Ust[tu + 3][cu]);
            *(float4 *)(dst + 4) = make_float4(Ust[tu][cu + 16], Ust[tu + 1][cu + 16],
                                               Ust[tu + 2][cu + 16], Ust[tu + 3][cu + 16]);
        }
    }
}

/* ---------------------------------------------------------------------- */
/* phase B: the state recurrence over chunks                                */
/* ---------------------------------------------------------------------- */
/* The columns of S evolve independently, so a (segment, v-head) is spread
 * over NCB workgroups of 32 state columns each. A workgroup has two sets of
 * four waves, one of each per SIMD, which meet at two barriers per chunk:
 *   chain wave w (S rows 32w..32w+31 in one fp32 32x32 accumulator, chunk
 *   tokens 16w..16w+15):
 *     S (bf16) -> LDS as S^T;                                   barrier 1
 *     V'_w = U_w - W_w S (16x16x32, 8 MFMAs), as hi + lo (bf16)
 *       -> LDS as V'^T, and e^{G_last-G} V'_w likewise as D^T;  barrier 2
 *     S_w = e^{G_last} S_w + K^T_w D (32x32x16; hi.hi, hi.lo, lo.hi:
 *       12 MFMAs)
 *   output wave w (chunk tokens 16w..16w+15):
 *                                                               barrier 1
 *     O_w(c-1) += QKm_w V'(c-1) (12 MFMAs), O (fp32) out through a
 *       per-wave LDS tile; O_w(c) = e^G (Q_w S) (8 MFMAs) from the same
 *       S^T;                                                    barrier 2
 *     V'^T(c) read into registers.
 *   Holding chunk c's QKm V' products until after the next barrier 1 leaves
 *   the matrix cores to the chain's S update between barrier 2 and barrier 1
 *   (config 2: 115.3 -> 112.9-114.6 us per layer).
 * The output waves keep their products off the recurrence's critical path:
 * each LDS buffer is written by the chain waves only after the barrier
 * that follows the output waves' last read of it (S^T(c+1) after barrier 2
 * of chunk c, V'^T(c+1) after barrier 1 of chunk c+1), so one copy of each
 * suffices.
 * Phase A stored every operand in fragment order, so each lane loads its
 * fragments with 16-byte reads straight into registers, one chunk ahead, in
 * parts between its MFMA groups: issued as one burst, the texture unit's
 * time for all of them would be spent before a barrier and added to the
 * chain. The NCB workgroups of one unit share those operands; block
 * numbering puts them on one XCD (blockIdx % 8 picks the XCD), so their L2
 * serves the repeats. */
constexpr int NCB = DV / 32;
constexpr int CB_THREADS = 512;

struct ChainOps {
    bf16x8 w[4], kgh[4], kgl[4];
    float4 u[2];
    float4 g; /* G of this lane's 4 V' rows */
    float gl;
};
struct OutOps {
    bf16x8 qg[4], qkh[2], qkl[2];
    float4 g; /* G of this lane's 4 O rows */
};

__global__ __launch_bounds__(CB_THREADS) void gdn_chunk_b_kernel(
    const bf16x8 *__restrict__ Wi, const bf16x8 *__restrict__ Qi, const bf16x8 *__restrict__ QKi,
    const bf16x8 *__restrict__ KTi, const float4 *__restrict__ Ui, const float *__restrict__ Gi,
    const int32_t *__restrict__ chunk_tok0, const int32_t *__restrict__ chunk_len,
    const int32_t *__restrict__ seg_chunk0, const int32_t *__restrict__ seg_nchunk,
    const float *__restrict__ S_in, float *__restrict__ S_out, int Hv, int Hk, int units,
    float *__restrict__ o, TailJob tail) {
    __shared__ __attribute__((aligned(16))) bf16 sT[32][DK + 8];   /* S^T [column][dk]        */
    __shared__ __attribute__((aligned(16))) bf16 vTh[32][CH + 8];  /* V'^T hi [column][token] */
    __shared__ __attribute__((aligned(16))) bf16 vTl[32][CH + 8];  /* V'^T lo                 */
    /* (e^{G_last-G} V')^T hi and lo: the S update's operand */
    __shared__ __attribute__((aligned(16))) bf16 dTh[32][CH + 8];
    __shared__ __attribute__((aligned(16))) bf16 dTl[32][CH + 8];
    __shared__ __attribute__((aligned(16))) float ost[4][16][36];  /* per output wave O tile  */

    const int bid = blockIdx.x;
    const int nmain = NCB * ((units + 7) / 8) * 8;
    if (bid >= nmain) { /* conv tail: CB_THREADS channels per workgroup */
        const int c = (bid - nmain) * CB_THREADS + threadIdx.x;
        if (c < tail.C) {
            float tv[3];
#pragma unroll
            for (int j = 0; j < 3; j++) {
                const int t = tail.seg0_len - 3 + j;
                tv[j] = t >= 0 ? bf2f(tail.proj[(size_t)t * tail.ps + c])
                               : (tail.conv_in ? tail.conv_in[(size_t)c * 3 + t + 3] : 0.f);
            }
#pragma unroll
            for (int j = 0; j < 3; j++)
                tail.conv_out[(size_t)c * 3 + j] = tv[j];
        }
        return;
    }
    const int un = (bid & 7) + 8 * ((bid >> 3) / NCB), cbk = (bid >> 3) % NCB;
    if (un >= units)
        return;
    const int seg = un / Hv, hv = un - seg * Hv, hk = hv / (Hv / Hk);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int w4 = wave & 3;
    const int h = lane >> 5, c32 = lane & 31, q4 = lane >> 4, c16 = lane & 15;
    const int col0 = 32 * cbk;
    const int c0 = seg_chunk0[seg], nc = seg_nchunk[seg];
    /* A segment's chunks are consecutive 64-token slices: token offsets
     * follow from the first chunk, the length from the last. The loads are
     * unconditional (past the end they repeat the last chunk) so the
     * compiler's wait counts stay exact: a load skipped on one path makes
     * the next use wait for every load in flight. */
    const int tok_seg = nc > 0 ? chunk_tok0[c0] : 0;
    const int len_last = nc > 0 ? chunk_len[c0 + nc - 1] : 0;
    auto cl = [&](int ci) { return c0 + min(ci, nc - 1); };
    /* S^T as the 16x16x32 B operand: k step s, column block jb */
    auto read_sb = [&](bf16x8 (&sb)[4][2]) {
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int jb = 0; jb < 2; jb++)
                sb[s][jb] = *(const bf16x8 *)&sT[16 * jb + c16][32 * s + 8 * q4];
    };

    if (wave < 4) {
        /* ---- chain waves: the recurrence ---- */
        floatx16 S; /* rows 32 w4 + 8(r/4) + 4h + r%4, column col0 + c32 */
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int dk = 32 * w4 + 8 * (r >> 2) + 4 * h + (r & 3);
            S[r] = S_in ? S_in[((size_t)hv * DK + dk) * DV + col0 + c32] : 0.f;
        }
        /* consume S here, before any operand prefetch is in flight: S then
         * enters the chunk loop as a VALU result, and the loop's waits only
         * cover the operand set a step uses */
#pragma unroll
        for (int r = 0; r < 16; r++)
            S[r] += 0.f;
        struct Ptr {
            const bf16x8 *w, *kg;
            const float4 *u;
            const float *g;
        };
        auto ptrs = [&](int ch) {
            const size_t cb = (size_t)ch * Hv + hv, ck = (size_t)ch * Hk + hk;
            Ptr p;
            p.w = Wi + cb * 1024 + w4 * 256 + lane;
            p.kg = KTi + ck * 2048 + w4 * 256 + lane;
            p.u = Ui + (cb * 1024 + (cbk * 4 + w4) * 64 + lane) * 2;
            p.g = Gi + cb * 64;
            return p;
        };
        auto load_part = [&](const Ptr &p, ChainOps &op, int part) {
            if (part == 0) {
#pragma unroll
                for (int s = 0; s < 4; s++)
                    op.w[s] = p.w[64 * s];
            } else if (part == 1) {
                op.u[0] = p.u[0];
                op.u[1] = p.u[1];
                op.g = *(const float4 *)(p.g + 16 * w4 + 4 * q4);
                op.gl = p.g[63];
            } else {
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    op.kgh[s] = p.kg[64 * s];
                    op.kgl[s] = p.kg[1024 + 64 * s];
                }
            }
        };
        auto step = [&](const ChainOps &op, int chn, ChainOps &nx) {
            const Ptr np = ptrs(chn);
            const float dec = fast_exp(op.gl);
#pragma unroll
            for (int j = 0; j < 4; j++)
                *(bf16x4 *)&sT[c32][32 * w4 + 8 * j + 4 * h] = bf16x4{
                    f2bf(S[4 * j]), f2bf(S[4 * j + 1]), f2bf(S[4 * j + 2]), f2bf(S[4 * j + 3])};
            lds_barrier(); /* 1: S^T of this chunk */
            bf16x8 sb[4][2];
            read_sb(sb);
            floatx4 V[2] = {};
#pragma unroll
            for (int s = 0; s < 4; s++)
#pragma unroll
                for (int jb = 0; jb < 2; jb++)
                    V[jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(op.w[s], sb[s][jb], V[jb], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            load_part(np, nx, 0);
            __builtin_amdgcn_sched_barrier(0);
            const float uf[8] = {op.u[0].x, op.u[0].y, op.u[0].z, op.u[0].w,
                                 op.u[1].x, op.u[1].y, op.u[1].z, op.u[1].w};
            /* each row's decay to the chunk's end: V' enters the S update as
             * e^{G_last-G} V', and O as it is */
            const float gv[4] = {op.g.x, op.g.y, op.g.z, op.g.w};
            float dg[4];
#pragma unroll
            for (int i = 0; i < 4; i++)
                dg[i] = fast_exp(op.gl - gv[i]);
#pragma unroll
            for (int jb = 0; jb < 2; jb++) {
                bf16x4 ph, pl, dh, dl;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float vp = uf[4 * jb + i] - V[jb][i];
                    const bfpair sp_ = split2(vp);
                    ph[i] = sp_.hi;
                    pl[i] = sp_.lo;
                    const bfpair sd_ = split2(vp * dg[i]);
                    dh[i] = sd_.hi;
                    dl[i] = sd_.lo;
                }
                *(bf16x4 *)&vTh[16 * jb + c16][16 * w4 + 4 * q4] = ph;
                *(bf16x4 *)&vTl[16 * jb + c16][16 * w4 + 4 * q4] = pl;
                *(bf16x4 *)&dTh[16 * jb + c16][16 * w4 + 4 * q4] = dh;
                *(bf16x4 *)&dTl[16 * jb + c16][16 * w4 + 4 * q4] = dl;
            }
            __builtin_amdgcn_sched_barrier(0);
            load_part(np, nx, 1);
            __builtin_amdgcn_sched_barrier(0);
            lds_barrier(); /* 2: V'^T of this chunk */
            bf16x8 vbh[4], vbl[4];
#pragma unroll
            for (int s = 0; s < 4; s++) {
                vbh[s] = *(const bf16x8 *)&dTh[c32][16 * s + 8 * h];
                vbl[s] = *(const bf16x8 *)&dTl[c32][16 * s + 8 * h];
            }
            S = S * dec;
#pragma unroll
            for (int s = 0; s < 4; s++) {
                S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op.kgh[s], vbh[s], S, 0, 0, 0);
                S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op.kgh[s], vbl[s], S, 0, 0, 0);
                S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op.kgl[s], vbh[s], S, 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            load_part(np, nx, 2);
            __builtin_amdgcn_sched_barrier(0);
        };
        if (nc > 0) {
            ChainOps A, B;
#pragma unroll
            for (int part = 0; part < 3; part++)
                load_part(ptrs(cl(0)), A, part);
            for (int ci = 0; ci < nc; ci += 2) {
                step(A, cl(ci + 1), B);
                if (ci + 1 >= nc)
                    break;
                step(B, cl(ci + 2), A);
            }
        }
        if (S_out && seg == 0) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int dk = 32 * w4 + 8 * (r >> 2) + 4 * h + (r & 3);
                S_out[((size_t)hv * DK + dk) * DV + col0 + c32] = S[r];
            }
        }
        return;
    }

    /* ---- output waves: O of chunk tokens 16 w4 .. +15 ---- */
    struct Ptr {
        const bf16x8 *qg, *qk;
        const float *g;
    };
    auto ptrs = [&](int ch) {
        const size_t cb = (size_t)ch * Hv + hv, ck = (size_t)ch * Hk + hk;
        Ptr p;
        p.qg = Qi + ck * 1024 + w4 * 256 + lane;
        p.qk = QKi + cb * 1024 + w4 * 128 + lane;
        p.g = Gi + cb * 64 + 16 * w4 + 4 * q4;
        return p;
    };
    auto load_part = [&](const Ptr &p, OutOps &op, int part) {
        if (part == 0) {
#pragma unroll
            for (int s = 0; s < 4; s++)
                op.qg[s] = p.qg[64 * s];
            op.g = *(const float4 *)p.g;
        } else {
#pragma unroll
            for (int s = 0; s < 2; s++) {
                op.qkh[s] = p.qk[64 * s];
                op.qkl[s] = p.qk[512 + 64 * s];
            }
        }
    };
    /* The QKm V' products and the store of chunk c's O wait until after
     * barrier 1 of chunk c+1: between barrier 2 and the next barrier 1 the
     * chain's S update then has the SIMD's matrix core to itself. V'^T(c) is
     * held in registers across the barrier (the chain rewrites the LDS copy
     * in chunk c+1), and chunk c's QKm fragments stay in the operand set the
     * next step would refill until they are used. */
    floatx4 Op[2] = {};
    bf16x8 v2h[2][2], v2l[2][2];
    auto finish = [&](int ch, const OutOps &pq) {
        const int ci = ch - c0;
        const int t0 = tok_seg + CH * ci, L = ci + 1 < nc ? CH : len_last;
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int jb = 0; jb < 2; jb++) {
                Op[jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pq.qkh[s], v2h[s][jb], Op[jb], 0, 0, 0);
                Op[jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pq.qkh[s], v2l[s][jb], Op[jb], 0, 0, 0);
                Op[jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pq.qkl[s], v2h[s][jb], Op[jb], 0, 0, 0);
            }
#pragma unroll
        for (int jb = 0; jb < 2; jb++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                ost[w4][4 * q4 + i][16 * jb + c16] = Op[jb][i];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const int r = lane >> 2, c8 = 8 * (lane & 3);
        const float4 o0 = *(const float4 *)&ost[w4][r][c8];
        const float4 o1 = *(const float4 *)&ost[w4][r][c8 + 4];
        if (16 * w4 + r < L) {
            float *dst = o + ((size_t)(t0 + 16 * w4 + r) * Hv + hv) * DV + col0 + c8;
            *(float4 *)dst = o0;
            *(float4 *)(dst + 4) = o1;
        }
    };
    auto step = [&](int ch, const OutOps &op, int chn, OutOps &nx) {
        const Ptr np = ptrs(chn);
        lds_barrier(); /* 1 */
        bf16x8 sb[4][2];
        read_sb(sb);
        if (ch > c0)
            finish(ch - 1, nx); /* nx still holds chunk ch-1's operands */
        floatx4 O[2] = {};
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int jb = 0; jb < 2; jb++)
                O[jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(op.qg[s], sb[s][jb], O[jb], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        load_part(np, nx, 0);
        load_part(np, nx, 1);
        __builtin_amdgcn_sched_barrier(0);
        {
            const float gv[4] = {op.g.x, op.g.y, op.g.z, op.g.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float eg = fast_exp(gv[i]);
                O[0][i] *= eg;
                O[1][i] *= eg;
            }
        }
        lds_barrier(); /* 2 */
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int jb = 0; jb < 2; jb++) {
                v2h[s][jb] = *(const bf16x8 *)&vTh[16 * jb + c16][32 * s + 8 * q4];
                v2l[s][jb] = *(const bf16x8 *)&vTl[16 * jb + c16][32 * s + 8 * q4];
            }
        Op[0] = O[0];
        Op[1] = O[1];
    };
    if (nc > 0) {
        OutOps A, B;
        load_part(ptrs(cl(0)), A, 0);
        load_part(ptrs(cl(0)), A, 1);
        for (int ci = 0; ci < nc; ci += 2) {
            step(c0 + ci, A, cl(ci + 1), B);
            if (ci + 1 >= nc)
                break;
            step(c0 + ci + 1, B, cl(ci + 2), A);
        }
        finish(c0 + nc - 1, ((nc - 1) & 1) ? B : A);
    }
}

/* ---------------------------------------------------------------------- */
/* phase B for one-chunk segments with no state written back (eval branches) */
/* ---------------------------------------------------------------------- */
/* Every segment starts from the same S_in and nothing carries over between
 * them, so a workgroup takes one v-head and spw consecutive segments (as many
 * as keep about SB_WGS workgroups busy). Wave w (of 8: short per-wave chains,
 * since a few branches give few workgroups) owns state columns 16w..16w+15:
 * its S^T fragments (bf16) are read once into registers, then per segment it
 * computes those columns of
 *   V' = U - W S (hi + lo),  O = e^G (Q S) + QKm V'
 * for the 16-row blocks that hold tokens (the fragments and split products
 * of gdn_chunk_b_kernel), and the workgroup applies the gated RMSNorm of
 * gdn_norm_gate_kernel to the segment's fp32 rows. */
constexpr int SB_WGS = 512;
constexpr int SB_THREADS = 512; /* 8 waves, 16 state columns each */

__global__ __launch_bounds__(SB_THREADS) void gdn_short_b_kernel(
    const bf16x8 *__restrict__ Wi, const bf16x8 *__restrict__ Qi, const bf16x8 *__restrict__ QKi,
    const float4 *__restrict__ Ui, const float *__restrict__ Gi,
    const int32_t *__restrict__ chunk_tok0, const int32_t *__restrict__ chunk_len,
    const int32_t *__restrict__ seg_chunk0, const int32_t *__restrict__ seg_nchunk, int nseg,
    int spw, const float *__restrict__ S_in, int Hv, int Hk, const bf16 *__restrict__ z, int zs,
    const float *__restrict__ nw, float eps, bf16 *__restrict__ y) {
    /* S^T staging at the start, then each segment's fp32 O rows */
    __shared__ __attribute__((aligned(16))) unsigned char so_raw[sizeof(bf16) * DV * (DK + 8)];
    __shared__ __attribute__((aligned(16))) bf16 vTh[DV][CH + 8]; /* V'^T hi [column][token] */
    __shared__ __attribute__((aligned(16))) bf16 vTl[DV][CH + 8]; /* V'^T lo                 */
    bf16(*sT)[DK + 8] = reinterpret_cast<bf16(*)[DK + 8]>(so_raw);
    float(*ob)[DV + 4] = reinterpret_cast<float(*)[DV + 4]>(so_raw);
    static_assert(sizeof(float) * CH * (DV + 4) <= sizeof(bf16) * DV * (DK + 8), "O staging");

    const int hv = blockIdx.y, sg0 = blockIdx.x * spw, hk = hv / (Hv / Hk);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q4 = lane >> 4, c16 = lane & 15;
    const int col0 = 16 * wave; /* this wave's 16 state columns */

    /* S^T: thread reads S[dk0..dk0+7][dv4..dv4+3] (16-byte rows) and writes
     * the 4 columns' 8-element runs */
    {
        const int dv4 = 4 * (tid & 31), dk0 = 8 * (tid >> 5);
        float4 r[8];
#pragma unroll
        for (int e = 0; e < 8; e++)
            r[e] = S_in ? *(const float4 *)(S_in + ((size_t)hv * DK + dk0 + e) * DV + dv4)
                        : float4{0.f, 0.f, 0.f, 0.f};
        bf16x8 c[4];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            c[0][e] = f2bf(r[e].x);
            c[1][e] = f2bf(r[e].y);
            c[2][e] = f2bf(r[e].z);
            c[3][e] = f2bf(r[e].w);
        }
#pragma unroll
        for (int j = 0; j < 4; j++)
            *(bf16x8 *)&sT[dv4 + j][dk0] = c[j];
    }
    /* V'^T rows past a segment's last 16-row block may be read by the QKm
     * step (times an exact zero of the causal mask): keep them finite */
    for (int i = tid; i < DV * (CH + 8) / 8; i += SB_THREADS) {
        ((bf16x8 *)&vTh[0][0])[i] = bf16x8{};
        ((bf16x8 *)&vTl[0][0])[i] = bf16x8{};
    }
    lds_barrier();
    bf16x8 sb[4]; /* this wave's S^T fragments, the same for every segment */
#pragma unroll
    for (int s = 0; s < 4; s++)
        sb[s] = *(const bf16x8 *)&sT[col0 + c16][32 * s + 8 * q4];
    lds_barrier(); /* sT's space now holds O */

    float wl[8];
#pragma unroll
    for (int e = 0; e < 8; e++)
        wl[e] = nw[8 * (tid & 15) + e];

    for (int j = 0; j < spw; j++) {
        const int seg = sg0 + j;
        if (seg >= nseg)
            break;
        /* without a segment table every unit is one (packed) chunk */
        if (seg_chunk0 && seg_nchunk[seg] <= 0)
            continue;
        const int ch = seg_chunk0 ? seg_chunk0[seg] : seg;
        const int t0 = chunk_tok0[ch], L = chunk_len[ch];
        const int nrb = (L + 15) >> 4, nks = (L + 31) >> 5;
        const size_t cb = (size_t)ch * Hv + hv, ck = (size_t)ch * Hk + hk;

        floatx4 O[4];
#pragma unroll
        for (int rb = 0; rb < 4; rb++) {
            O[rb] = floatx4{};
            if (rb >= nrb)
                continue;
            bf16x8 w[4], qg[4];
#pragma unroll
            for (int s = 0; s < 4; s++) {
                w[s] = Wi[cb * 1024 + rb * 256 + 64 * s + lane];
                qg[s] = Qi[ck * 1024 + rb * 256 + 64 * s + lane];
            }
            const float4 gq = *(const float4 *)(Gi + cb * 64 + 16 * rb + 4 * q4);
            /* U fragment of the 32-column block holding these 16 columns:
             * values 0..3 its first 16 columns, 4..7 the second */
            const float4 *up = Ui + (cb * 1024 + ((wave >> 1) * 4 + rb) * 64 + lane) * 2;
            const float4 uu = up[wave & 1];
            floatx4 V = {};
#pragma unroll
            for (int s = 0; s < 4; s++) {
                V = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w[s], sb[s], V, 0, 0, 0);
                O[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qg[s], sb[s], O[rb], 0, 0, 0);
            }
            /* O = e^G (Q S) + QKm V' */
            O[rb][0] *= fast_exp(gq.x);
            O[rb][1] *= fast_exp(gq.y);
            O[rb][2] *= fast_exp(gq.z);
            O[rb][3] *= fast_exp(gq.w);
            const float uf[4] = {uu.x, uu.y, uu.z, uu.w};
            bf16x4 ph, pl;
#pragma unroll
            for (int i = 0; i < 4; i++)
                { const bfpair sp_ = split2(uf[i] - V[i]); ph[i] = sp_.hi; pl[i] = sp_.lo; }
            *(bf16x4 *)&vTh[col0 + c16][16 * rb + 4 * q4] = ph;
            *(bf16x4 *)&vTl[col0 + c16][16 * rb + 4 * q4] = pl;
        }
        /* the wave reads back only its own columns of V'^T: LDS order suffices */
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int rb = 0; rb < 4; rb++) {
            if (rb >= nrb)
                continue;
#pragma unroll
            for (int s = 0; s < 2; s++) {
                if (s >= nks)
                    continue;
                const bf16x8 qkh = QKi[cb * 1024 + rb * 128 + 64 * s + lane];
                const bf16x8 qkl = QKi[cb * 1024 + 512 + rb * 128 + 64 * s + lane];
                const bf16x8 vh_ = *(const bf16x8 *)&vTh[col0 + c16][32 * s + 8 * q4];
                const bf16x8 vl_ = *(const bf16x8 *)&vTl[col0 + c16][32 * s + 8 * q4];
                O[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qkh, vh_, O[rb], 0, 0, 0);
                O[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qkh, vl_, O[rb], 0, 0, 0);
                O[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qkl, vh_, O[rb], 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
                ob[16 * rb + 4 * q4 + i][col0 + c16] = O[rb][i];
        }
        lds_barrier();
        /* gated RMSNorm, 16 lanes per token row (as gdn_norm_gate_kernel) */
        for (int r0 = 0; r0 < L; r0 += SB_THREADS / 16) {
            const int t = r0 + (tid >> 4), sl = tid & 15;
            if (t < L) { /* whole 16-lane groups */
                const float4 o0 = *(const float4 *)&ob[t][8 * sl];
                const float4 o1 = *(const float4 *)&ob[t][8 * sl + 4];
                const float ov[8] = {o0.x, o0.y, o0.z, o0.w, o1.x, o1.y, o1.z, o1.w};
                const size_t n = (size_t)t0 + t;
                const bf16 *zr = z + n * zs + hv * DV + 8 * sl;
                float ss = 0.f;
#pragma unroll
                for (int e = 0; e < 8; e++)
                    ss += ov[e] * ov[e];
#pragma unroll
                for (int m = 1; m < 16; m <<= 1)
                    ss += __shfl_xor(ss, m, 64);
                const float inv = rsqrtf(ss * (1.f / DV) + eps);
                bf16x8 res;
#pragma unroll
                for (int e = 0; e < 8; e++)
                    res[e] = f2bf(bf2f(f2bf(ov[e] * inv)) * wl[e] * silu_f(bf2f(zr[e])));
                *(bf16x8 *)(y + (n * Hv + hv) * DV + 8 * sl) = res;
            }
        }
        lds_barrier(); /* ob and vT are rewritten by the next segment */
    }
}

/* y = bf16( w * bf16(o * rsqrt(mean o^2 + eps)) * silu(z) ) from the fp32
 * output o: 16 lanes per (token, v-head) row, 8 columns a lane.
 * REF src/kernels/gdn.cu:193-216. */
/* ---------------------------------------------------------------------- */
/* few-token branches: the recurrence token by token, fp32                 */
/* ---------------------------------------------------------------------- */
/* For an eval of a few short branches the chunked scan is one round of
 * workgroups whose serial chains (conv, products, inverse, operand stores,
 * then phase B) set the time. Here each workgroup owns one (segment, v-head,
 * block of RC_COLS state columns), so a handful of branches still fills the
 * chip, and runs the reference's recurrence (src/kernels/gdn.cu:140-176) in
 * fp32 registers:
 *   kS = S^T k;  v' = beta (v - e^g kS);  S = e^g S + k v'^T;  o = S^T q
 * Wave w owns state columns 8w..8w+7 of the block whole: lane (c = l%8,
 * r = l/8) holds rows 16r..16r+15 of column c, so k.S and q.S finish inside
 * the wave (one DPP rotate and two permlane swaps) and the token loop has no
 * barrier and no LDS traffic but the broadcast reads of k and q.
 * Before it, the workgroup stages the segment's pre-conv rows (its k-head's
 * q and k slices, its v columns) in LDS with every load in flight at once;
 * thread t then runs channel t's causal conv + SiLU over the tokens with
 * its weights and the state's tail in registers (gdn_conv_prep's
 * arithmetic), and 8 lanes per (token, q|k) row apply the l2-norm and q's
 * scale. o (fp32) goes to the gated norm kernel. */
constexpr int RC_THREADS = 256;
constexpr int RC_COLS = 32;
constexpr int RC_MAXL = CUJEV_GDN_RECUR_MAX_LEN;
constexpr int RC_CH = 2 * DK + RC_COLS; /* q, k and this block's v channels */

struct RecurSmem {
    float q[RC_MAXL][DK];
    float k[RC_MAXL][DK];
    float v[RC_MAXL][RC_COLS];
    bf16 x[RC_MAXL][RC_CH]; /* pre-conv rows of the segment's tokens */
    float g[RC_MAXL], beta[RC_MAXL];
    float kq[RC_MAXL]; /* k_j . q_j */
};

/* sum over the 8 lanes l, l^8, ..., l^56 (lane bits 3..5) */
DEV float sum_lanes8(float v) {
    v += dpp<0x128>(v); /* row_ror:8 = lane ^ 8 inside a row of 16 */
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]); /* + lane ^ 16 */
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]); /* + lane ^ 32 */
}

template <bool TAIL>
__global__ __launch_bounds__(RC_THREADS, 2) void gdn_recur_kernel(
    ConvSrc cv, const int32_t *__restrict__ chunk_tok0, const int32_t *__restrict__ chunk_len,
    const int32_t *__restrict__ seg_chunk0, int Hk, int Hv, int units,
    const float *__restrict__ S_in, float *__restrict__ o) {
    __shared__ __attribute__((aligned(16))) RecurSmem sm;
    const int cb = blockIdx.x & 3, unit = blockIdx.x >> 2;
    if (unit >= units)
        return;
    const int seg = unit / Hv, hv = unit - seg * Hv, hk = hv / (Hv / Hk);
    const int c0 = seg_chunk0[seg];
    const int t0 = chunk_tok0[c0], L = min(chunk_len[c0], RC_MAXL);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int C = (2 * Hk + Hv) * DK;
    /* channel slot -> projection column: q slice, k slice, this block's v */
    auto gch = [&](int ch) {
        return ch < DK       ? hk * DK + ch
               : ch < 2 * DK ? (Hk + hk) * DK + ch - DK
                             : (2 * Hk + hv) * DK + RC_COLS * cb + ch - 2 * DK;
    };

    /* ---- every global load first (one memory latency, not one per stage):
     * the segment's rows into registers, the gates' inputs, this thread's
     * conv weights and tail, and its slice of the state ---- */
    constexpr int XP = CEIL_DIV(RC_MAXL * (RC_CH / 8), RC_THREADS); /* row pieces per thread */
    const int npieces = L * (RC_CH / 8);
    bf16x8 xr[XP];
#pragma unroll
    for (int k = 0; k < XP; k++) {
        const int i = tid + k * RC_THREADS;
        if (i < npieces) {
            const int rr = i / (RC_CH / 8), ch = 8 * (i - rr * (RC_CH / 8));
            xr[k] = ld8(cv.proj + (size_t)(t0 + rr) * cv.ps + gch(ch));
        }
    }
    float b_raw = 0.f, a_raw = 0.f;
    if (tid < L) {
        const bf16 *ab = cv.proj + (size_t)(t0 + tid) * cv.ps + C + Hv * DV;
        b_raw = bf2f(ab[hv]);
        a_raw = bf2f(ab[Hv + hv]);
    }
    const float A_neg = cv.A_neg_exp[hv], dtb = cv.dt_bias[hv];
    /* thread t convolves q/k channel t, and v channel t when t < RC_COLS */
    const int gq = gch(tid), gv = gch(2 * DK + (tid & (RC_COLS - 1)));
    const float4 wq = *(const float4 *)(cv.conv_w + (size_t)gq * 4);
    const float4 wv = *(const float4 *)(cv.conv_w + (size_t)gv * 4);
    float tq[3], tv[3];
#pragma unroll
    for (int j = 0; j < 3; j++) {
        tq[j] = TAIL ? cv.conv_in[(size_t)gq * 3 + j] : 0.f;
        tv[j] = TAIL ? cv.conv_in[(size_t)gv * 3 + j] : 0.f;
    }
    const int c = lane & 7, r = lane >> 3, colw = 8 * wave + c;
    float S[16];
#pragma unroll
    for (int i = 0; i < 16; i++)
        S[i] = S_in ? S_in[((size_t)hv * DK + 16 * r + i) * DV + RC_COLS * cb + colw] : 0.f;
#pragma unroll
    for (int k = 0; k < XP; k++) {
        const int i = tid + k * RC_THREADS;
        if (i < npieces) {
            const int rr = i / (RC_CH / 8), ch = 8 * (i - rr * (RC_CH / 8));
            *(bf16x8 *)&sm.x[rr][ch] = xr[k];
        }
    }
    if (tid < L) {
        sm.beta[tid] = sigmoid_f(b_raw);
        sm.g[tid] = A_neg * softplus_f(a_raw + dtb);
    }
    lds_barrier();

    /* ---- conv + SiLU, a sliding window per channel: the channel's inputs
     * of every row slot are read first (rows past L hold no token and are
     * not used), so the window runs on registers ---- */
    {
        float xin[RC_MAXL];
#pragma unroll
        for (int j = 0; j < RC_MAXL; j++)
            xin[j] = bf2f(sm.x[j][tid]);
        float x3 = tq[0], x2 = tq[1], x1 = tq[2]; /* inputs of tokens -3, -2, -1 */
        float *dst = tid < DK ? &sm.q[0][tid] : &sm.k[0][tid - DK];
#pragma unroll
        for (int j = 0; j < RC_MAXL; j++) {
            if (j < L) {
                const float x0 = xin[j];
                float y = fmaf(wq.x, x3, 0.f);
                y = fmaf(wq.y, x2, y);
                y = fmaf(wq.z, x1, y);
                y = fmaf(wq.w, x0, y);
                dst[j * DK] = silu_f(y);
                x3 = x2, x2 = x1, x1 = x0;
            }
        }
    }
    if (tid < 4 * RC_COLS) { /* v: channel tid % 32, token quarter tid / 32 */
        const int cc = tid & (RC_COLS - 1), per = (L + 3) >> 2;
        const int j0 = (tid >> 5) * per, j1 = min(L, j0 + per);
        auto xin = [&](int j) { /* input of token j, the tail before 0 */
            return j >= 0 ? bf2f(sm.x[j][2 * DK + cc]) : tv[j + 3];
        };
        float x3 = xin(j0 - 3), x2 = xin(j0 - 2), x1 = xin(j0 - 1);
        for (int j = j0; j < j1; j++) {
            const float x0 = bf2f(sm.x[j][2 * DK + cc]);
            float y = fmaf(wv.x, x3, 0.f);
            y = fmaf(wv.y, x2, y);
            y = fmaf(wv.z, x1, y);
            y = fmaf(wv.w, x0, y);
            sm.v[j][cc] = silu_f(y);
            x3 = x2, x2 = x1, x1 = x0;
        }
    }
    lds_barrier();
    /* ---- per token, 8 lanes: the l2-norms of q and k (q also * 128^-1/2)
     * and k.q from the same registers ---- */
    for (int base = 0; base < L; base += RC_THREADS / 8) {
        const int j = base + (tid >> 3), part = tid & 7;
        if (j < L) { /* whole 8-lane groups */
            float *qp = sm.q[j] + 16 * part, *kp = sm.k[j] + 16 * part;
            float4 a[4], b[4];
            float sq = 0.f, sk = 0.f, d = 0.f;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                a[e] = *(const float4 *)(qp + 4 * e);
                b[e] = *(const float4 *)(kp + 4 * e);
                sq += a[e].x * a[e].x + a[e].y * a[e].y + a[e].z * a[e].z + a[e].w * a[e].w;
                sk += b[e].x * b[e].x + b[e].y * b[e].y + b[e].z * b[e].z + b[e].w * b[e].w;
                d += a[e].x * b[e].x + a[e].y * b[e].y + a[e].z * b[e].z + a[e].w * b[e].w;
            }
            sq += dpp<0xB1>(sq), sk += dpp<0xB1>(sk), d += dpp<0xB1>(d);    /* lane ^ 1 */
            sq += dpp<0x4E>(sq), sk += dpp<0x4E>(sk), d += dpp<0x4E>(d);    /* lane ^ 2 */
            sq += dpp<0x141>(sq), sk += dpp<0x141>(sk), d += dpp<0x141>(d); /* other quad */
            const float iq = rsqrtf(sq + 1e-6f) * 0.08838834764831845f;
            const float ik = rsqrtf(sk + 1e-6f);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                *(float4 *)(qp + 4 * e) =
                    make_float4(a[e].x * iq, a[e].y * iq, a[e].z * iq, a[e].w * iq);
                *(float4 *)(kp + 4 * e) =
                    make_float4(b[e].x * ik, b[e].y * ik, b[e].z * ik, b[e].w * ik);
            }
            if (part == 0)
                sm.kq[j] = d * iq * ik;
        }
    }
    lds_barrier();

    /* ---- the recurrence: no barrier, the waves run free ----
     * S is kept as sigma * St (sigma = the product of the decays so far), so
     * a token costs three FMAs per state element: k.St and q.St in one pass,
     * then St += k (v' / sigma). With kS = sigma k.St and qS = sigma q.St of
     * the previous state,
     *   v' = beta (v - e^g kS),  o = e^g qS + v' (k.q)   (= S_new^T q).
     * When sigma would drop below 2^-40 the token applies its decay to St
     * directly and sigma restarts at 1. */
    float *orow = o + (size_t)hv * DV + RC_COLS * cb + colw;
    float sigma = 1.f;
    /* a token's operands from LDS; read one token ahead of its use (they do
     * not depend on the state), two buffers alternating */
    struct StepOps {
        float kq[16], qq[16];
        float g, beta, v, kqd;
    };
    auto load_ops = [&](int j, StepOps &op) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float4 a = *(const float4 *)&sm.k[j][16 * r + 4 * e];
            const float4 b = *(const float4 *)&sm.q[j][16 * r + 4 * e];
            op.kq[4 * e] = a.x, op.kq[4 * e + 1] = a.y, op.kq[4 * e + 2] = a.z, op.kq[4 * e + 3] = a.w;
            op.qq[4 * e] = b.x, op.qq[4 * e + 1] = b.y, op.qq[4 * e + 2] = b.z, op.qq[4 * e + 3] = b.w;
        }
        op.g = sm.g[j], op.beta = sm.beta[j], op.v = sm.v[j][colw], op.kqd = sm.kq[j];
    };
    auto step = [&](int j, const StepOps &op) {
        const float eg = fast_exp(op.g);
        float pk[4] = {0.f, 0.f, 0.f, 0.f}, pq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 16; i++) {
            pk[i & 3] = fmaf(op.kq[i], S[i], pk[i & 3]);
            pq[i & 3] = fmaf(op.qq[i], S[i], pq[i & 3]);
        }
        const float kS = sigma * sum_lanes8((pk[0] + pk[1]) + (pk[2] + pk[3]));
        const float qS = sigma * sum_lanes8((pq[0] + pq[1]) + (pq[2] + pq[3]));
        const float vn = op.beta * (op.v - eg * kS);
        const float os = fmaf(eg, qS, vn * op.kqd);
        if (r == 0)
            orow[(size_t)(t0 + j) * Hv * DV] = os;
        const float sn = sigma * eg;
        if (sn < 0x1p-40f) { /* wave-uniform: fold the decay into St */
#pragma unroll
            for (int i = 0; i < 16; i++)
                S[i] = fmaf(sn, S[i], op.kq[i] * vn);
            sigma = 1.f;
        } else {
            const float w = vn * __builtin_amdgcn_rcpf(sn);
#pragma unroll
            for (int i = 0; i < 16; i++)
                S[i] = fmaf(op.kq[i], w, S[i]);
            sigma = sn;
        }
    };
    StepOps opa, opb;
    load_ops(0, opa);
    for (int j = 0; j < L; j += 2) { /* past the end: row L - 1 again, unused */
        load_ops(min(j + 1, L - 1), opb);
        step(j, opa);
        if (j + 1 >= L)
            break;
        load_ops(min(j + 2, L - 1), opa);
        step(j + 1, opb);
    }
}

template <bool VEC>
__global__ __launch_bounds__(256) void gdn_norm_gate_kernel(const float *__restrict__ o,
                                                            const bf16 *__restrict__ z, int zs,
                                                            const float *__restrict__ w, float eps,
                                                            int rows, int Hv,
                                                            bf16 *__restrict__ y) {
    const int row = blockIdx.x * 16 + (threadIdx.x >> 4);
    const int s = threadIdx.x & 15;
    if (row >= rows)
        return; /* whole 16-lane groups leave together */
    const int n = row / Hv, hv = row - n * Hv;
    const float4 o0 = *(const float4 *)(o + (size_t)row * DV + 8 * s);
    const float4 o1 = *(const float4 *)(o + (size_t)row * DV + 8 * s + 4);
    const float ov[8] = {o0.x, o0.y, o0.z, o0.w, o1.x, o1.y, o1.z, o1.w};
    const bf16 *zr = z + (size_t)n * zs + hv * DV + 8 * s;
    bf16x8 zv;
    if constexpr (VEC) {
        zv = *(const bf16x8 *)zr;
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++)
            zv[e] = zr[e];
    }
    float wl[8];
#pragma unroll
    for (int e = 0; e < 8; e++)
        wl[e] = w[8 * s + e];
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++)
        ss += ov[e] * ov[e];
#pragma unroll
    for (int m = 1; m < 16; m <<= 1)
        ss += __shfl_xor(ss, m, 64);
    const float inv = rsqrtf(ss * (1.f / DV) + eps);
    bf16x8 r;
#pragma unroll
    for (int e = 0; e < 8; e++)
        r[e] = f2bf(bf2f(f2bf(ov[e] * inv)) * wl[e] * silu_f(bf2f(zv[e])));
    *(bf16x8 *)(y + (size_t)row * DV + 8 * s) = r;
}

} // namespace
} // namespace CUJEV_KNS
using namespace CUJEV_KNS;

extern "C" hipError_t k_gdn_conv_prep(const bf16_t *proj, int proj_stride, const float *conv_w,
                                      const float *conv_in, float *conv_out, int seg0_len,
                                      const int32_t *own_base, const float *A_neg_exp,
                                      const float *dt_bias, int N, int Hk, int Hv, float *q,
                                      float *k, float *v, float *g, float *beta,
                                      hipStream_t stream) {
    if (N <= 0)
        return hipSuccess;
    if (Hk <= 0 || Hv % Hk != 0)
        return hipErrorInvalidValue;
    const int nheads = 2 * Hk + Hv;
    const int groups = CEIL_DIV(N, PREP_T) * nheads;
    const bool vec = proj_stride % 8 == 0 && ((uintptr_t)proj & 15) == 0;
    auto kern = vec ? (conv_in ? gdn_conv_prep_kernel<true, true> : gdn_conv_prep_kernel<true, false>)
                    : (conv_in ? gdn_conv_prep_kernel<false, true> : gdn_conv_prep_kernel<false, false>);
    hipLaunchKernelGGL(kern, dim3((unsigned)CEIL_DIV(groups, 16)), dim3(256), 0, stream,
                       (const bf16 *)proj, proj_stride, conv_w, conv_in, own_base, A_neg_exp,
                       dt_bias, N, Hk, Hv, q, k, v, g, beta);
    if (conv_out) {
        const int C = nheads * DK;
        hipLaunchKernelGGL(gdn_conv_tail_kernel, dim3((unsigned)CEIL_DIV(C, 256)), dim3(256), 0,
                           stream, (const bf16 *)proj, proj_stride, conv_in, conv_out, seg0_len, C);
    }
    return hipGetLastError();
}

/* Phase B and the gated norm after phase A (either front end). */
/* norm == false leaves o in ws->O for k_gdn_norm_gate (*o_pending = 1)
 * where a separate norm launch would follow; the short-segment kernel
 * applies the norm itself either way (*o_pending = 0). */
static hipError_t gdn_phase_b(const cujev_chunks *ck, const float *S_in, float *S_out,
                              const bf16_t *z, int z_stride, const float *norm_w, float eps,
                              int Hk, int Hv, bf16_t *y, const cujev_gdn_scratch *ws, int N,
                              const TailJob &tail, hipStream_t stream, bool norm = true,
                              int *o_pending = nullptr) {
    if (o_pending)
        *o_pending = 0;
    const bool packed = ck->chunk_starts != nullptr;
    if (!S_out && (packed || ck->max_seg_chunks == 1)) {
        /* packed: the units are the chunks, each scanned from S_in */
        const int units = packed ? ck->num_chunks : ck->num_segments;
        const int spw = max(1, CEIL_DIV(units * Hv, SB_WGS));
        if (tail.conv_out)
            hipLaunchKernelGGL(gdn_conv_tail_kernel, dim3((unsigned)CEIL_DIV(tail.C, 256)),
                               dim3(256), 0, stream, tail.proj, tail.ps, tail.conv_in,
                               tail.conv_out, tail.seg0_len, tail.C);
        hipLaunchKernelGGL(gdn_short_b_kernel, dim3((unsigned)CEIL_DIV(units, spw), (unsigned)Hv),
                           dim3(SB_THREADS), 0, stream, (const bf16x8 *)ws->W, (const bf16x8 *)ws->Q,
                           (const bf16x8 *)ws->QK, (const float4 *)ws->U, ws->G, ck->chunk_tok0,
                           ck->chunk_len, packed ? nullptr : ck->seg_chunk0,
                           packed ? nullptr : ck->seg_nchunk, units, spw, S_in, Hv, Hk,
                           (const bf16 *)z, z_stride, norm_w, eps, (bf16 *)y);
        return hipGetLastError();
    }
    if (packed)
        return hipErrorInvalidValue; /* packed segments write no final state */
    const int units = ck->num_segments * Hv;
    const int ntail = tail.conv_out ? CEIL_DIV(tail.C, CB_THREADS) : 0;
    hipLaunchKernelGGL(gdn_chunk_b_kernel, dim3((unsigned)(NCB * CEIL_DIV(units, 8) * 8 + ntail)),
                       dim3(CB_THREADS), 0, stream, (const bf16x8 *)ws->W, (const bf16x8 *)ws->Q,
                       (const bf16x8 *)ws->QK, (const bf16x8 *)ws->KT, (const float4 *)ws->U,
                       ws->G, ck->chunk_tok0, ck->chunk_len, ck->seg_chunk0, ck->seg_nchunk,
                       S_in, S_out, Hv, Hk, units, ws->O, tail);
    if (!norm) {
        if (o_pending)
            *o_pending = 1;
        return hipGetLastError();
    }
    return k_gdn_norm_gate(ws->O, z, z_stride, norm_w, eps, N * Hv, Hv, y, stream);
}

extern "C" hipError_t k_gdn_scan(const float *q, const float *k, const float *v, const float *g,
                                 const float *beta, const cujev_chunks *ck, const float *S_in,
                                 float *S_out, const bf16_t *z, int z_stride, const float *norm_w,
                                 float eps, int Hk, int Hv, bf16_t *y, const cujev_gdn_scratch *ws,
                                 int N, hipStream_t stream) {
    if (ck->num_chunks <= 0 || N <= 0)
        return hipSuccess;
    if (Hk <= 0 || Hv % Hk != 0 || (ck->chunk_starts && S_out))
        return hipErrorInvalidValue;
    const int npairs = CEIL_DIV(Hv / Hk, 2);
    hipLaunchKernelGGL(gdn_chunk_a_kernel<0>, dim3((unsigned)ck->num_chunks, (unsigned)(Hk * npairs)),
                       dim3(PA_THREADS), 0, stream, q, k, v, g, beta, ConvSrc{}, ck->chunk_tok0,
                       ck->chunk_len, ck->chunk_starts, Hk, Hv, npairs, (bf16 *)ws->W, (bf16 *)ws->Q,
                       (bf16 *)ws->QK, (bf16 *)ws->KT, ws->U, ws->G);
    return gdn_phase_b(ck, S_in, S_out, z, z_stride, norm_w, eps, Hk, Hv, y, ws, N, TailJob{},
                       stream);
}

extern "C" int cujev_gdn_recur_chosen(const cujev_chunks *ck, int Hv, int has_S_out,
                                      int has_conv_out) {
    if (has_S_out || has_conv_out || ck->chunk_starts || ck->max_seg_chunks != 1 ||
        ck->max_seg_len <= 0 || ck->max_seg_len > RC_MAXL || ck->num_segments <= 0)
        return 0;
    static int mode = -2;
    if (mode == -2) {
        const char *e = getenv("CUJEV_GDN_RECUR");
        mode = e && *e == '0' ? 0 : e && *e == '1' ? 1 : -1;
    }
    if (mode >= 0)
        return mode;
    /* the token loop is latency-bound while there are at most about two
     * workgroups per CU, each with few tokens */
    return (long)ck->num_segments * Hv <= 256 && ck->max_seg_len <= RC_MAXL;
}

static hipError_t gdn_recur(const bf16_t *proj, int proj_stride, const float *conv_w,
                            const float *conv_in, const float *A_neg_exp, const float *dt_bias,
                            const cujev_chunks *ck, const float *S_in, const float *norm_w,
                            float eps, int Hk, int Hv, bf16_t *y, const cujev_gdn_scratch *ws,
                            int N, hipStream_t stream, bool norm) {
    if (N <= 0 || ck->num_segments <= 0)
        return hipSuccess;
    if (Hk <= 0 || Hv % Hk != 0 || proj_stride % 8 != 0 || ((uintptr_t)proj & 15) != 0 ||
        ck->chunk_starts || ck->max_seg_chunks != 1 || ck->max_seg_len <= 0 ||
        ck->max_seg_len > RC_MAXL)
        return hipErrorInvalidValue;
    const ConvSrc cv{(const bf16 *)proj, proj_stride, conv_w, conv_in, nullptr,
                     A_neg_exp,          dt_bias,     N};
    const int units = ck->num_segments * Hv;
    hipLaunchKernelGGL(conv_in ? gdn_recur_kernel<true> : gdn_recur_kernel<false>,
                       dim3((unsigned)(4 * units)), dim3(RC_THREADS), 0, stream, cv,
                       ck->chunk_tok0, ck->chunk_len, ck->seg_chunk0, Hk, Hv, units, S_in, ws->O);
    if (!norm)
        return hipGetLastError();
    const int C = (2 * Hk + Hv) * DK;
    return k_gdn_norm_gate(ws->O, proj + C, proj_stride, norm_w, eps, N * Hv, Hv, y, stream);
}

extern "C" hipError_t k_gdn_recur(const bf16_t *proj, int proj_stride, const float *conv_w,
                                  const float *conv_in, const float *A_neg_exp,
                                  const float *dt_bias, const cujev_chunks *ck, const float *S_in,
                                  const float *norm_w, float eps, int Hk, int Hv, bf16_t *y,
                                  const cujev_gdn_scratch *ws, int N, hipStream_t stream) {
    return gdn_recur(proj, proj_stride, conv_w, conv_in, A_neg_exp, dt_bias, ck, S_in, norm_w,
                     eps, Hk, Hv, y, ws, N, stream, true);
}

static hipError_t gdn_layer(const bf16_t *proj, int proj_stride, const float *conv_w,
                            const float *conv_in, float *conv_out, int seg0_len,
                            const int32_t *own_base, const float *A_neg_exp, const float *dt_bias,
                            const cujev_chunks *ck, const float *S_in, float *S_out,
                            const float *norm_w, float eps, int Hk, int Hv, bf16_t *y,
                            const cujev_gdn_scratch *ws, int N, hipStream_t stream, bool norm,
                            int *o_pending) {
    if (o_pending)
        *o_pending = 0;
    if (N <= 0)
        return hipSuccess;
    if (Hk <= 0 || Hv % Hk != 0 || (ck->chunk_starts && S_out) || proj_stride % 8 != 0 ||
        ((uintptr_t)proj & 15) != 0)
        return hipErrorInvalidValue;
    const int C = (2 * Hk + Hv) * DK;
    if (ck->num_chunks <= 0) {
        if (conv_out)
            hipLaunchKernelGGL(gdn_conv_tail_kernel, dim3((unsigned)CEIL_DIV(C, 256)), dim3(256),
                               0, stream, (const bf16 *)proj, proj_stride, conv_in, conv_out,
                               seg0_len, C);
        return hipGetLastError();
    }
    if (cujev_gdn_recur_chosen(ck, Hv, S_out != nullptr, conv_out != nullptr)) {
        if (o_pending)
            *o_pending = !norm;
        return gdn_recur(proj, proj_stride, conv_w, conv_in, A_neg_exp, dt_bias, ck, S_in,
                         norm_w, eps, Hk, Hv, y, ws, N, stream, norm);
    }
    const ConvSrc cv{(const bf16 *)proj, proj_stride, conv_w, conv_in, own_base,
                     A_neg_exp,          dt_bias,     N};
    /* the conv tail rides along with phase B */
    const TailJob tail{(const bf16 *)proj, proj_stride, conv_in, conv_out, seg0_len, C};
    const int npairs = CEIL_DIV(Hv / Hk, 2);
    hipLaunchKernelGGL(conv_in ? gdn_chunk_a_kernel<2> : gdn_chunk_a_kernel<1>,
                       dim3((unsigned)ck->num_chunks, (unsigned)(Hk * npairs)), dim3(PA_THREADS), 0,
                       stream,
                       (const float *)nullptr, (const float *)nullptr, (const float *)nullptr,
                       (const float *)nullptr, (const float *)nullptr, cv, ck->chunk_tok0,
                       ck->chunk_len, ck->chunk_starts, Hk, Hv, npairs, (bf16 *)ws->W,
                       (bf16 *)ws->Q, (bf16 *)ws->QK, (bf16 *)ws->KT, ws->U, ws->G);
    return gdn_phase_b(ck, S_in, S_out, proj + C, proj_stride, norm_w, eps, Hk, Hv, y, ws, N, tail,
                       stream, norm, o_pending);
}

extern "C" hipError_t k_gdn_layer(const bf16_t *proj, int proj_stride, const float *conv_w,
                                  const float *conv_in, float *conv_out, int seg0_len,
                                  const int32_t *own_base, const float *A_neg_exp,
                                  const float *dt_bias, const cujev_chunks *ck, const float *S_in,
                                  float *S_out, const float *norm_w, float eps, int Hk, int Hv,
                                  bf16_t *y, const cujev_gdn_scratch *ws, int N,
                                  hipStream_t stream) {
    return gdn_layer(proj, proj_stride, conv_w, conv_in, conv_out, seg0_len, own_base, A_neg_exp,
                     dt_bias, ck, S_in, S_out, norm_w, eps, Hk, Hv, y, ws, N, stream, true,
                     nullptr);
}

extern "C" hipError_t k_gdn_layer_o(const bf16_t *proj, int proj_stride, const float *conv_w,
                                    const float *conv_in, float *conv_out, int seg0_len,
                                    const int32_t *own_base, const float *A_neg_exp,
                                    const float *dt_bias, const cujev_chunks *ck,
                                    const float *S_in, float *S_out, const float *norm_w,
                                    float eps, int Hk, int Hv, bf16_t *y,
                                    const cujev_gdn_scratch *ws, int N, hipStream_t stream,
                                    int *o_pending) {
    return gdn_layer(proj, proj_stride, conv_w, conv_in, conv_out, seg0_len, own_base, A_neg_exp,
                     dt_bias, ck, S_in, S_out, norm_w, eps, Hk, Hv, y, ws, N, stream, false,
                     o_pending);
}

extern "C" hipError_t k_gdn_norm_gate(const float *o, const bf16_t *z, int z_stride,
                                      const float *norm_w, float eps, int rows, int Hv, bf16_t *y,
                                      hipStream_t stream) {
    if (rows <= 0)
        return hipSuccess;
    const bool zvec = z_stride % 8 == 0 && ((uintptr_t)z & 15) == 0;
    hipLaunchKernelGGL(zvec ? gdn_norm_gate_kernel<true> : gdn_norm_gate_kernel<false>,
                       dim3((unsigned)CEIL_DIV(rows, 16)), dim3(256), 0, stream, o,
                       (const bf16 *)z, z_stride, norm_w, eps, rows, Hv, (bf16 *)y);
    return hipGetLastError();
}
