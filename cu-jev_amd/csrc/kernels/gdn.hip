/* Gated DeltaNet for gfx950: fused conv/gates, chunked WY/UT delta rule on
 * bf16 MFMA with an fp32 recurrent state, gated RMSNorm fused into the scan.
 *
 * Semantics: REF src/kernels/gdn.cu:4-24 (conv), :26-43 (conv tail), :57-96
 * (prep), :111-182 (scan, recurrent form), :193-216 (gated norm); math of
 * transformers' torch_chunk_gated_delta_rule (modeling_qwen3_5.py:249-327).
 *
 * Pipeline per layer (all tokens of all segments in one launch each):
 *   gdn_conv_prep  conv(4) + SiLU, l2norm(q,k) with q * 128^-1/2, g, beta
 *                  -> bf16 q,k [N][Hk][128], v [N][Hv][128]; fp32 g, beta.
 *   gdn_chunk_a    per (64-token chunk, v-head), fully parallel:
 *                  G = cumsum g, A = tril(beta_i k_i.k_j e^{G_i-G_j}, -1),
 *                  T = (I+A)^-1 by blocked forward substitution (fp32),
 *                  W = T diag(beta e^G) K, U = T diag(beta) V (bf16 MFMA),
 *                  QKm = tril(q_i.k_j e^{G_i-G_j})           -> bf16 in HBM.
 *   gdn_chunk_b    per (segment, v-head), sequential over the segment's
 *                  chunks; wave w owns 32 columns of S (fp32, registers):
 *                  V' = U - W S;  O = (Q e^G) S + QKm V';
 *                  S = e^{G_last} S + (K e^{G_last-G})^T V'  (bf16 MFMA),
 *                  then y = w * bf16(rmsnorm(O)) * silu(z) straight to bf16.
 * Every segment starts from S_in (the state's S, read-only) or 0 and the
 * conv taps before a segment come from the state's conv tail (or 0): branches
 * never copy the state.
 *
 * MFMA operand layouts (v_mfma_f32_32x32x16_bf16): A lane l = row l%32,
 * k 8(l/32)..+8; B lane l = col l%32, same k; C lane l = col l%32, rows
 * 8(r/4) + 4(l/32) + r%4. An accumulator used again as a B operand supplies
 * its k values in that row order, so the matching A operand is read as two
 * 4-element pieces at k offsets 4h and 8+4h of each 16-wide step. */
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
    bf16 *__restrict__ qo, bf16 *__restrict__ ko, bf16 *__restrict__ vo, float *__restrict__ go,
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
    bf16 *dst;
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
        bf16x8 out;
#pragma unroll
        for (int e = 0; e < 8; e++)
            out[e] = f2bf(y[e] * inv);
        *(bf16x8 *)(dst + (size_t)n * tok_stride + 8 * s) = out;
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
/* One workgroup (4 waves) per (chunk, v-head), LDS under 80 KiB so two
 * share a CU:
 *   1. q, k (k-head), v rows -> LDS; wave 0 forms G = cumsum g and the
 *      per-token scales beta e^G, beta, e^{G_last - G}.
 *   2. K K^T and Q K^T (bf16 MFMA); A = tril(beta_i e^{G_i-G_j} k_i.k_j, -1)
 *      (fp32) and the masked QK^T (bf16) -> LDS; Q e^G and QK^T leave.
 *   3. T = (I + A)^-1 in place, fp32: the four 16x16 diagonal blocks by
 *      forward substitution, then T_10 = -T_11 (A_10 T_00) inside each 32x32
 *      diagonal block, then the same at 64 with 32x32 blocks.
 *   4. W = T (beta e^G K), U = T (beta V) on MFMA. Their B operands need
 *      tokens on the k axis: D = K I (an exact identity product) gives that
 *      layout in registers, rows in the accumulator order 4h+0..3, 8+4h+0..3
 *      of every 16, so T is read with its columns in that order. The same
 *      D tiles scaled by e^{G_last - G} are (k e^{G_last-G})^T, stored
 *      straight from registers after one cross-half exchange.
 *   5. W and U staged row-major in the freed q / v rows, then stored in
 *      fragment order.
 * A chunk may hold several whole segments (chunk_starts marks where each
 * begins): G restarts at every segment start and A and QK^T are kept
 * block-diagonal, so the segments do not see each other. This is valid for
 * branches that all continue one state and write no final state: phase B then
 * needs nothing per segment. */
struct __attribute__((aligned(16))) ChunkA_Smem {
    bf16 K[CH][DK + 8];   /* k rows                     */
    bf16 Q[CH][DK + 8];   /* q rows, later W            */
    bf16 V[CH][DV + 8];   /* v rows, later U            */
    float AT[CH][CH + 4]; /* A, then T in place (rows 16-byte aligned) */
    bf16 QK[CH][CH + 8];  /* masked QK^T staging        */
    float G[CH], sK[CH], sKg[CH], sV[CH];
    int Sid[CH]; /* segment of each token inside a packed chunk (1-based) */
};
static_assert(sizeof(ChunkA_Smem) <= 80 * 1024, "two phase-A workgroups per CU");

DEV bf16x8 ld8(const bf16 *p) { return *(const bf16x8 *)p; }
typedef __attribute__((address_space(3))) float4 lds_f4;
DEV float4 rd4(const float *p) { return *(const float4 *)p; }
DEV void wr4(float *p, float4 v) { *(float4 *)p = v; }
DEV float4 f4fma(float a, float4 b, float4 c) {
    return make_float4(fmaf(a, b.x, c.x), fmaf(a, b.y, c.y), fmaf(a, b.z, c.z), fmaf(a, b.w, c.w));
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
 * copy it, beside the recurrence, which leaves half the CUs idle. */
struct TailJob {
    const bf16 *proj;
    int ps;
    const float *conv_in;
    float *conv_out; /* NULL: no tail */
    int seg0_len, C;
};

/* The three 128-channel slices a phase-A workgroup needs (q and k of its
 * k-head, v of its v-head) through conv + SiLU (+ l2 norm and scale), with
 * gdn_conv_prep_kernel's arithmetic step for step. Thread = (token block
 * tid/16 of 4 tokens, channels 8(tid%16)..+7 of every slice). The 7
 * pre-conv rows of each slice are loaded first; the conv weights and the
 * state's tail (the same for all token blocks) go through LDS once:
 * cw[slice][e][s] float4 and ct[slice][j][e][s] for channel 8s + e. */
DEV int slice_c0(int sl, int Hk, int hk, int hv) {
    return sl == 0 ? hk * DK : sl == 1 ? (Hk + hk) * DK : (2 * Hk + hv) * DK;
}

template <bool TAIL>
DEV void conv_stage(const ConvSrc &cv, int Hk, int hk, int hv, int tid, float *cw, float *ct) {
    for (int i = tid; i < 3 * DK; i += 256) {
        const int sl = i / DK, c = i % DK, cg = slice_c0(sl, Hk, hk, hv) + c;
        const int slot = (sl * 8 + (c & 7)) * 16 + (c >> 3);
        *(float4 *)&cw[slot * 4] = *(const float4 *)(cv.conv_w + (size_t)cg * 4);
        if constexpr (TAIL) {
#pragma unroll
            for (int j = 0; j < 3; j++)
                ct[(sl * 3 + j) * 128 + (c & 7) * 16 + (c >> 3)] = cv.conv_in[(size_t)cg * 3 + j];
        }
    }
}

DEV void conv_rows(const ConvSrc &cv, int c0, int n0, bf16x8 (&x)[7]) {
#pragma unroll
    for (int i = 0; i < 7; i++) {
        const int row = min(max(n0 - 3 + i, 0), cv.N - 1);
        x[i] = ld8(cv.proj + (size_t)row * cv.ps + c0);
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

template <bool TAIL>
DEV void conv_slice(const bf16x8 (&x)[7], const int (&base)[4], const float *cw, const float *ct,
                    int sl, bool norm, float scale, int t0, int L, int tb, int s,
                    bf16 (*dst)[DK + 8]) {
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
        bf16x8 out;
#pragma unroll
        for (int e = 0; e < 8; e++)
            out[e] = f2bf(tt < L ? y[e] * inv : 0.f);
        *(bf16x8 *)&dst[tt][8 * s] = out;
    }
}

/* SRC 0: q, k, v, g, beta read from gdn_conv_prep's outputs; 1: computed
 * here from the pre-conv projection rows (zeros before a segment); 2: the
 * same with the state's conv tail before each segment. */
template <int SRC>
__global__ __launch_bounds__(256, 2) void gdn_chunk_a_kernel(
    const bf16 *__restrict__ qh, const bf16 *__restrict__ kh_, const bf16 *__restrict__ vh,
    const float *__restrict__ g, const float *__restrict__ beta, ConvSrc cv,
    const int32_t *__restrict__ chunk_tok0, const int32_t *__restrict__ chunk_len,
    const uint64_t *__restrict__ chunk_starts, int Hk, int Hv,
    bf16 *__restrict__ Wo, bf16 *__restrict__ Qgo, bf16 *__restrict__ QKo,
    bf16 *__restrict__ KgTo, bf16 *__restrict__ Uo, float *__restrict__ Glo) {
    __shared__ ChunkA_Smem sm;
    const int ch = blockIdx.x, hv = blockIdx.y;
    const int hk = hv / (Hv / Hk);
    const int t0 = chunk_tok0[ch], L = chunk_len[ch];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, col = lane & 31;
    const size_t cb = (size_t)ch * Hv + hv;

    /* ---- 1. rows and gates ---- */
    {
        float gv = 0.f, bv = 0.f;
        if constexpr (SRC == 0) {
            bf16x8 kv[4], qv[4], vv[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int i = tid + 256 * j, t = i >> 4, c8 = (i & 15) * 8;
                kv[j] = qv[j] = vv[j] = bf16x8{};
                if (t < L) {
                    kv[j] = ld8(kh_ + ((size_t)(t0 + t) * Hk + hk) * DK + c8);
                    qv[j] = ld8(qh + ((size_t)(t0 + t) * Hk + hk) * DK + c8);
                    vv[j] = ld8(vh + ((size_t)(t0 + t) * Hv + hv) * DV + c8);
                }
            }
            if (wave == 0 && lane < L) {
                gv = g[(size_t)(t0 + lane) * Hv + hv];
                bv = beta[(size_t)(t0 + lane) * Hv + hv];
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int i = tid + 256 * j, t = i >> 4, c8 = (i & 15) * 8;
                *(bf16x8 *)&sm.K[t][c8] = kv[j];
                *(bf16x8 *)&sm.Q[t][c8] = qv[j];
                *(bf16x8 *)&sm.V[t][c8] = vv[j];
            }
        } else {
            constexpr bool TAIL = SRC == 2;
            const int C = (2 * Hk + Hv) * DK;
            if (wave == 0 && lane < L) {
                const bf16 *ab = cv.proj + (size_t)(t0 + lane) * cv.ps + C + Hv * DV; /* b, a */
                bv = sigmoid_f(bf2f(ab[hv]));
                gv = cv.A_neg_exp[hv] * softplus_f(bf2f(ab[Hv + hv]) + cv.dt_bias[hv]);
            }
            /* (slice, 4-token block) tasks over the 16-lane groups: only
             * blocks holding tokens are computed, so a short chunk spreads
             * its few tasks over all groups (64 tokens: one block, three
             * slices per group). All pre-conv rows go in flight first, then
             * the weights and tail into LDS (the A/T area is free until
             * step 2). */
            const int nblk = (L + 3) >> 2, ntask = 3 * nblk;
            const int grp = tid >> 4, s16 = tid & 15;
            bf16x8 xr[3][7];
            int base[3][4];
#pragma unroll
            for (int r = 0; r < 3; r++) {
                const int t = grp + 16 * r;
                if (t < ntask) {
                    const int sl = t / nblk, n0 = t0 + 4 * (t - sl * nblk);
                    conv_rows(cv, slice_c0(sl, Hk, hk, hv) + 8 * s16, n0, xr[r]);
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        base[r][j] = cv.own_base[min(n0 + j, cv.N - 1)];
                }
            }
            float *cw = &sm.AT[0][0], *ct = cw + 3 * 8 * 16 * 4;
            conv_stage<TAIL>(cv, Hk, hk, hv, tid, cw, ct);
            /* rows of token blocks without tokens: zeros */
            const int zrows = CH - 4 * nblk;
            for (int i = tid; i < 3 * zrows * 16; i += 256) {
                const int a = i / (zrows * 16), rem = i - a * zrows * 16;
                bf16(*z)[DK + 8] = a == 0 ? sm.Q : a == 1 ? sm.K : sm.V;
                *(bf16x8 *)&z[4 * nblk + (rem >> 4)][8 * (rem & 15)] = bf16x8{};
            }
            lds_barrier();
#pragma unroll
            for (int r = 0; r < 3; r++) {
                const int t = grp + 16 * r;
                if (t < ntask) {
                    const int sl = t / nblk, tb = t - sl * nblk;
                    conv_slice<TAIL>(xr[r], base[r], cw, ct, sl, sl < 2,
                                     sl == 0 ? 0.08838834764831845f /* 128^-1/2 */ : 1.f, t0, L,
                                     tb, s16, sl == 0 ? sm.Q : sl == 1 ? sm.K : sm.V);
                }
            }
        }
        if (wave == 0) {
            /* segments packed into the chunk: st = first token of this
             * lane's segment, en = its last (63 for the chunk's last one) */
            const uint64_t starts = chunk_starts ? chunk_starts[ch] | 1ull : 1ull;
            const uint64_t upto = lane == 63 ? ~0ull : (2ull << lane) - 1;
            const int st = 63 - __builtin_clzll(starts & upto);
            const uint64_t later = starts & ~upto;
            const int en = later ? __builtin_ctzll(later) - 1 : 63;
            /* cumulative sum restarted at each segment start */
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const float up = __shfl_up(gv, o, 64);
                if (lane - o >= st)
                    gv += up;
            }
            const float gl = __shfl(gv, en, 64);
            sm.Sid[lane] = __builtin_popcountll(starts & upto);
            sm.G[lane] = gv;
            sm.sK[lane] = bv * fast_exp(gv);
            sm.sKg[lane] = fast_exp(gl - gv);
            sm.sV[lane] = bv;
            Glo[cb * 64 + lane] = gl; /* one copy per lane of phase B's waves */
        }
    }
    lds_barrier();

    /* ---- 2. K K^T, Q K^T; wave w owns the 32x32 tile (w>>1, w&1) ---- */
    {
        const int ti = wave >> 1, tj = wave & 1;
        floatx16 kk = {}, qk = {};
        if (ti >= tj) {
#pragma unroll
            for (int ks = 0; ks < DK / 16; ks++) {
                const int c = 16 * ks + 8 * h;
                const bf16x8 ak = *(const bf16x8 *)&sm.K[32 * ti + col][c];
                const bf16x8 aq = *(const bf16x8 *)&sm.Q[32 * ti + col][c];
                const bf16x8 bk = *(const bf16x8 *)&sm.K[32 * tj + col][c];
                kk = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ak, bk, kk, 0, 0, 0);
                qk = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aq, bk, qk, 0, 0, 0);
            }
        }
        const int j = 32 * tj + col;
        const float Gj = sm.G[j];
        const int Sj = sm.Sid[j];
        /* rows i = 32ti + 8m + 4h + 0..3: their G and beta four at a time,
         * read unconditionally (a read under the mask becomes a branch) */
        float Gi[16], Bi[16];
        int Si[16];
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const float4 a = rd4(&sm.G[32 * ti + 8 * m + 4 * h]);
            const float4 b = rd4(&sm.sV[32 * ti + 8 * m + 4 * h]);
            const int4 c = *(const int4 *)&sm.Sid[32 * ti + 8 * m + 4 * h];
            Gi[4 * m] = a.x, Gi[4 * m + 1] = a.y, Gi[4 * m + 2] = a.z, Gi[4 * m + 3] = a.w;
            Bi[4 * m] = b.x, Bi[4 * m + 1] = b.y, Bi[4 * m + 2] = b.z, Bi[4 * m + 3] = b.w;
            Si[4 * m] = c.x, Si[4 * m + 1] = c.y, Si[4 * m + 2] = c.z, Si[4 * m + 3] = c.w;
        }
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int i = 32 * ti + 8 * (r >> 2) + 4 * h + (r & 3);
            const float dec = fast_exp(fminf(Gi[r] - Gj, 0.f));
            const bool same = Si[r] == Sj; /* tokens of one segment interact */
            sm.AT[i][j] = i > j && same ? Bi[r] * kk[r] * dec : 0.f;
            sm.QK[i][j] = f2bf(i >= j && same ? qk[r] * dec : 0.f);
        }
    }
    lds_barrier();
    /* q e^G and the masked QK^T leave in 16x16x32 A-fragment order: entry
     * i = (row block w, k-step s, lane l) holds row 16w + l%16, columns
     * 32s + 8(l/16)..+7 */
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int i = tid + 256 * j;
        const int t = 16 * (i >> 8) + (i & 15), c8 = 32 * ((i >> 6) & 3) + 8 * ((i >> 4) & 3);
        const float eg = fast_exp(sm.G[t]);
        const bf16x8 qv = *(const bf16x8 *)&sm.Q[t][c8];
        bf16x8 r;
#pragma unroll
        for (int e = 0; e < 8; e++)
            r[e] = f2bf(bf2f(qv[e]) * eg);
        *(bf16x8 *)(Qgo + (cb * 1024 + i) * 8) = r;
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int i = tid + 256 * j;
        const int r = 16 * (i >> 7) + (i & 15), c8 = 32 * ((i >> 6) & 1) + 8 * ((i >> 4) & 3);
        *(bf16x8 *)(QKo + (cb * 512 + i) * 8) = *(const bf16x8 *)&sm.QK[r][c8];
    }

    /* ---- 3. T = (I + A)^-1 in place ----
     * 3a: wave w inverts diagonal block w, lane c < 16 owning column c; the
     * block is read (all lanes, broadcast) before any lane writes it. */
    if (lane < 16) {
        const int b0 = 16 * wave, c = lane;
        float t[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            float acc = 0.f;
#pragma unroll
            for (int k4 = 0; k4 < i; k4 += 4) {
                const float4 a = rd4(&sm.AT[b0 + i][b0 + k4]);
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
        /* stores only after every read of the block: the reads can all be
         * issued up front (a store in the loop would keep them in order) */
#pragma unroll
        for (int i = 0; i < 16; i++)
            if (i >= c)
                sm.AT[b0 + i][b0 + c] = t[i];
    }
    lds_barrier();
    /* 3b: inside 32x32 diagonal block p (wave p): T_10 = -T_11 (A_10 T_00),
     * 16x16 blocks; lane = (row l/4, columns 4(l%4)..+3) */
    if (wave < 2) {
        const int p0 = 32 * wave, r = lane >> 2, c0 = 4 * (lane & 3);
        float *a10 = &sm.AT[p0 + 16 + r][p0];
        const float4 x = row_times<16>(a10, &sm.AT[p0][p0 + c0]);
        wr4(a10 + c0, x);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const float4 y = row_times<16>(&sm.AT[p0 + 16 + r][p0 + 16], &sm.AT[p0 + 16][p0 + c0]);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wr4(a10 + c0, make_float4(-y.x, -y.y, -y.z, -y.w));
    }
    lds_barrier();
    /* 3c: T_10 = -T_11 (A_10 T_00) with 32x32 blocks; lane = (row 8w + l/8,
     * columns 4(l%8)..+3). A chunk of at most 32 tokens has A_10 = 0 and so
     * T_10 = 0, which the A/T array already holds; only padding rows read it. */
    if (L > 32) {
        const int r = 32 + 8 * wave + (lane >> 3), c0 = 4 * (lane & 7);
        const float4 x = row_times<32>(&sm.AT[r][0], &sm.AT[0][c0]);
        lds_barrier();
        wr4(&sm.AT[r][c0], x);
        lds_barrier();
        const float4 y = row_times<32>(&sm.AT[r][32], &sm.AT[32][c0]);
        lds_barrier();
        wr4(&sm.AT[r][c0], make_float4(-y.x, -y.y, -y.z, -y.w));
    }
    lds_barrier();

    /* ---- 4. W = T (beta e^G K), U = T (beta V), (k e^{Glast-G})^T ----
     * wave w: dk (= dv) block 32w, both 32-row halves of W and U. */
    {
        bf16x8 eye[2]; /* B operand of the identity, k = 16s + 8h + e */
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int e = 0; e < 8; e++)
                eye[s][e] = f2bf(16 * s + 8 * h + e == col ? 1.f : 0.f);
        floatx16 dK[2], dV[2]; /* D[tb] = rows 32tb.. of K (V), columns 32w.. */
#pragma unroll
        for (int tb = 0; tb < 2; tb++) {
            dK[tb] = dV[tb] = floatx16{};
#pragma unroll
            for (int s = 0; s < 2; s++) {
                const int c = 32 * wave + 16 * s + 8 * h;
                dK[tb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    *(const bf16x8 *)&sm.K[32 * tb + col][c], eye[s], dK[tb], 0, 0, 0);
                dV[tb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    *(const bf16x8 *)&sm.V[32 * tb + col][c], eye[s], dV[tb], 0, 0, 0);
            }
        }
        /* token of accumulator slot r of tile tb */
        auto tok = [&](int tb, int r) { return 32 * tb + 8 * (r >> 2) + 4 * h + (r & 3); };
        /* per-token scales of this lane's accumulator slots: slot r of tile tb
         * is token 32tb + 8(r/4) + 4h + r%4, four consecutive tokens a read */
        float sk[2][16], sv[2][16], skg[2][16];
#pragma unroll
        for (int tb = 0; tb < 2; tb++)
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const int t = 32 * tb + 8 * m + 4 * h;
                const float4 a = rd4(&sm.sK[t]), b = rd4(&sm.sV[t]), c = rd4(&sm.sKg[t]);
                sk[tb][4 * m] = a.x, sk[tb][4 * m + 1] = a.y, sk[tb][4 * m + 2] = a.z, sk[tb][4 * m + 3] = a.w;
                sv[tb][4 * m] = b.x, sv[tb][4 * m + 1] = b.y, sv[tb][4 * m + 2] = b.z, sv[tb][4 * m + 3] = b.w;
                skg[tb][4 * m] = c.x, skg[tb][4 * m + 1] = c.y, skg[tb][4 * m + 2] = c.z, skg[tb][4 * m + 3] = c.w;
            }
        bf16x8 xk[4], xv[4];
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int tb = ks >> 1, r0 = 8 * (ks & 1);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                xk[ks][e] = f2bf(dK[tb][r0 + e] * sk[tb][r0 + e]);
                xv[ks][e] = f2bf(dV[tb][r0 + e] * sv[tb][r0 + e]);
            }
        }
        /* (k e^{Glast-G})^T as 32x32x16 A fragments (row dk = 32w + l%32,
         * tokens 16s + 8(l/32)..+7): the lane pair (l, l^32) trades halves */
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int tb = s >> 1, r0 = 8 * (s & 1);
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; e++)
                v[e] = dK[tb][r0 + e] * skg[tb][r0 + e];
            /* h=0 holds tokens +0..3 | +8..11, h=1 holds +4..7 | +12..15 */
            uint32_t p0[2], p1[2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                p0[e] = __builtin_bit_cast(uint32_t, bf16x2{f2bf(v[2 * e]), f2bf(v[2 * e + 1])});
                p1[e] = __builtin_bit_cast(uint32_t, bf16x2{f2bf(v[4 + 2 * e]), f2bf(v[5 + 2 * e])});
            }
            uint32_t o[4];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const uint32_t x1 = (uint32_t)__shfl_xor((int)p1[e], 32, 64);
                const uint32_t x0 = (uint32_t)__shfl_xor((int)p0[e], 32, 64);
                o[e] = h ? x1 : p0[e];
                o[2 + e] = h ? p1[e] : x0;
            }
            *(u32x4 *)(KgTo + (cb * 1024 + (wave * 4 + s) * 64 + lane) * 8) =
                u32x4{o[0], o[1], o[2], o[3]};
        }
        floatx16 w[2] = {}, u[2] = {};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
#pragma unroll
            for (int mi = 0; mi < 2; mi++) {
                const float *tr = &sm.AT[32 * mi + col][16 * ks + 4 * h];
                const float4 a0 = rd4(tr), a1 = rd4(tr + 8);
                const bf16x8 a = {f2bf(a0.x), f2bf(a0.y), f2bf(a0.z), f2bf(a0.w),
                                  f2bf(a1.x), f2bf(a1.y), f2bf(a1.z), f2bf(a1.w)};
                w[mi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, xk[ks], w[mi], 0, 0, 0);
                u[mi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, xv[ks], u[mi], 0, 0, 0);
            }
        }
        lds_barrier(); /* every wave is done with the v rows */
#pragma unroll
        for (int mi = 0; mi < 2; mi++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int i = tok(mi, r);
                sm.Q[i][32 * wave + col] = f2bf(w[mi][r]);
                sm.V[i][32 * wave + col] = f2bf(u[mi][r]);
            }
        }
    }
    lds_barrier();
    /* ---- 5. W in the fragment order of q e^G; U as 16x16 accumulator
     * fragments: entry i = (32-column block cbk, row block w, lane l) holds
     * rows 16w + 4(l/16) + 0..3 of columns 32cbk + l%16 (values 0..3) and
     * 32cbk + 16 + l%16 (values 4..7) ---- */
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int i = tid + 256 * j;
        const int t = 16 * (i >> 8) + (i & 15), c8 = 32 * ((i >> 6) & 3) + 8 * ((i >> 4) & 3);
        *(bf16x8 *)(Wo + (cb * 1024 + i) * 8) = *(const bf16x8 *)&sm.Q[t][c8];
        const int tu = 16 * ((i >> 6) & 3) + 4 * ((i >> 4) & 3), cu = 32 * (i >> 8) + (i & 15);
        bf16x8 r;
#pragma unroll
        for (int e = 0; e < 8; e++)
            r[e] = sm.V[tu + (e & 3)][cu + 16 * (e >> 2)];
        *(bf16x8 *)(Uo + (cb * 1024 + i) * 8) = r;
    }
}

/* ---------------------------------------------------------------------- */
/* phase B: the state recurrence over chunks                                */
/* ---------------------------------------------------------------------- */
/* The columns of S evolve independently, so a (segment, v-head) is spread
 * over NCB workgroups of 32 state columns each, and inside a workgroup the
 * four waves split rows: wave w holds S rows 32w..32w+31 (fp32, one 32x32
 * accumulator) and chunk tokens 16w..16w+15. Per chunk:
 *   S (bf16) -> LDS as S^T; barrier
 *   V'_w = U_w - W_w S,  O_w = (Q e^G)_w S          (16x16x32, 16 MFMAs)
 *   V'_w (bf16) -> LDS as V'^T; barrier
 *   S_w = e^{G_last} S_w + (K e^{G_last-G})^T_w V'  (32x32x16, 4 MFMAs)
 *   O_w += QKm_w V'                                  (16x16x32, 4 MFMAs)
 * Phase A stored every operand in fragment order, so each lane loads its
 * fragments with 16-byte reads straight into registers, two chunks ahead.
 * The NCB workgroups of one unit share those operands; block numbering puts
 * them on one XCD (blockIdx % 8 picks the XCD), so their L2 serves the
 * repeats. */
constexpr int NCB = DV / 32;

struct BOps {
    bf16x8 w[4], qg[4], qk[2], kg[4], u;
    float gl;
};

__global__ __launch_bounds__(256) void gdn_chunk_b_kernel(
    const bf16x8 *__restrict__ Wi, const bf16x8 *__restrict__ Qgi, const bf16x8 *__restrict__ QKi,
    const bf16x8 *__restrict__ KgTi, const bf16x8 *__restrict__ Ui, const float *__restrict__ Gli,
    const int32_t *__restrict__ chunk_tok0, const int32_t *__restrict__ chunk_len,
    const int32_t *__restrict__ seg_chunk0, const int32_t *__restrict__ seg_nchunk,
    const float *__restrict__ S_in, float *__restrict__ S_out, int Hv, int units,
    bf16 *__restrict__ o, TailJob tail) {
    __shared__ __attribute__((aligned(16))) bf16 sT[32][DK + 8];  /* S^T [column][dk]     */
    __shared__ __attribute__((aligned(16))) bf16 vT[32][CH + 8];  /* V'^T [column][token] */
    __shared__ __attribute__((aligned(16))) bf16 ost[4][16][40];  /* per-wave O tile      */

    const int bid = blockIdx.x;
    const int nmain = NCB * ((units + 7) / 8) * 8;
    if (bid >= nmain) { /* conv tail: 256 channels per workgroup */
        const int c = (bid - nmain) * 256 + threadIdx.x;
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
    const int u = (bid & 7) + 8 * ((bid >> 3) / NCB), cbk = (bid >> 3) % NCB;
    if (u >= units)
        return;
    const int seg = u / Hv, hv = u - seg * Hv;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane >> 5, c32 = lane & 31, q4 = lane >> 4, c16 = lane & 15;
    const int col0 = 32 * cbk;

    floatx16 S; /* rows 32 wave + 8(r/4) + 4h + r%4, column col0 + c32 */
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int dk = 32 * wave + 8 * (r >> 2) + 4 * h + (r & 3);
        S[r] = S_in ? S_in[((size_t)hv * DK + dk) * DV + col0 + c32] : 0.f;
    }
    /* consume S here, before any operand prefetch is in flight: S then enters
     * the chunk loop as a VALU result, and the loop's waits only cover the
     * operand set a step uses (a pending load there would turn the loop-head
     * wait into vmcnt(0), draining the prefetches every round) */
#pragma unroll
    for (int r = 0; r < 16; r++)
        S[r] += 0.f;
    const int c0 = seg_chunk0[seg], nc = seg_nchunk[seg];

    auto load = [&](int ch, BOps &op) {
        const size_t cb = (size_t)ch * Hv + hv;
        const bf16x8 *w = Wi + cb * 1024 + wave * 256 + lane;
        const bf16x8 *qg = Qgi + cb * 1024 + wave * 256 + lane;
        const bf16x8 *kg = KgTi + cb * 1024 + wave * 256 + lane;
        const bf16x8 *qk = QKi + cb * 512 + wave * 128 + lane;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            op.w[s] = w[64 * s];
            op.kg[s] = kg[64 * s];
        }
        op.u = Ui[cb * 1024 + (cbk * 4 + wave) * 64 + lane];
        op.gl = Gli[cb * 64 + lane];
#pragma unroll
        for (int s = 0; s < 4; s++)
            op.qg[s] = qg[64 * s];
#pragma unroll
        for (int s = 0; s < 2; s++)
            op.qk[s] = qk[64 * s];
    };

    /* A segment's chunks are consecutive 64-token slices: token offsets
     * follow from the first chunk, the length from the last. The log-decay
     * travels with the operand set (phase A stores it once per lane). */
    const int tok_seg = nc > 0 ? chunk_tok0[c0] : 0;
    const int len_last = nc > 0 ? chunk_len[c0 + nc - 1] : 0;

    auto step = [&](int ch, const BOps &op) {
        const int ci = ch - c0;
        const int t0 = tok_seg + CH * ci, L = ci + 1 < nc ? CH : len_last;
        const float dec = fast_exp(op.gl);
#pragma unroll
        for (int j = 0; j < 4; j++)
            *(bf16x4 *)&sT[c32][32 * wave + 8 * j + 4 * h] =
                bf16x4{f2bf(S[4 * j]), f2bf(S[4 * j + 1]), f2bf(S[4 * j + 2]), f2bf(S[4 * j + 3])};
        lds_barrier();
        /* every LDS operand of a stage is read before its MFMAs: one wait */
        bf16x8 sb[4][2];
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int jb = 0; jb < 2; jb++)
                sb[s][jb] = *(const bf16x8 *)&sT[16 * jb + c16][32 * s + 8 * q4];
        floatx4 V[2] = {}, O[2] = {};
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int jb = 0; jb < 2; jb++)
                V[jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(op.w[s], sb[s][jb], V[jb], 0, 0, 0);
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int jb = 0; jb < 2; jb++)
                O[jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(op.qg[s], sb[s][jb], O[jb], 0, 0, 0);
#pragma unroll
        for (int jb = 0; jb < 2; jb++) {
            bf16x4 p;
#pragma unroll
            for (int i = 0; i < 4; i++)
                p[i] = f2bf(bf2f(op.u[4 * jb + i]) - V[jb][i]);
            *(bf16x4 *)&vT[16 * jb + c16][16 * wave + 4 * q4] = p;
        }
        lds_barrier();
        bf16x8 vb[4], vb2[2][2];
#pragma unroll
        for (int s = 0; s < 4; s++)
            vb[s] = *(const bf16x8 *)&vT[c32][16 * s + 8 * h];
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int jb = 0; jb < 2; jb++)
                vb2[s][jb] = *(const bf16x8 *)&vT[16 * jb + c16][32 * s + 8 * q4];
        S = S * dec;
#pragma unroll
        for (int s = 0; s < 4; s++)
            S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op.kg[s], vb[s], S, 0, 0, 0);
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int jb = 0; jb < 2; jb++)
                O[jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(op.qk[s], vb2[s][jb], O[jb], 0, 0, 0);
        /* O (bf16) through this wave's LDS tile: 16-byte stores, 64 bytes a row */
#pragma unroll
        for (int jb = 0; jb < 2; jb++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                ost[wave][4 * q4 + i][16 * jb + c16] = f2bf(O[jb][i]);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const int r = lane >> 2, c8 = 8 * (lane & 3);
        const bf16x8 ov = *(const bf16x8 *)&ost[wave][r][c8];
        if (16 * wave + r < L)
            *(bf16x8 *)(o + ((size_t)(t0 + 16 * wave + r) * Hv + hv) * DV + col0 + c8) = ov;
    };

    /* three operand sets in rotation: chunk ci + 2 loads while ci runs. The
     * loads are unconditional (past the end they repeat the last chunk) so
     * the compiler's wait counts stay exact: a load skipped on one path makes
     * the next use wait for every load in flight. */
    if (nc > 0) {
        auto cl = [&](int ci) { return c0 + min(ci, nc - 1); };
        BOps A, B, C;
        load(cl(0), A);
        load(cl(1), B);
        for (int ci = 0; ci < nc; ci += 3) {
            load(cl(ci + 2), C);
            step(c0 + ci, A);
            if (ci + 1 >= nc)
                break;
            load(cl(ci + 3), A);
            step(c0 + ci + 1, B);
            if (ci + 2 >= nc)
                break;
            load(cl(ci + 4), B);
            step(c0 + ci + 2, C);
        }
    }
    if (S_out && seg == 0) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int dk = 32 * wave + 8 * (r >> 2) + 4 * h + (r & 3);
            S_out[((size_t)hv * DK + dk) * DV + col0 + c32] = S[r];
        }
    }
}

/* ---------------------------------------------------------------------- */
/* phase B for one-chunk segments with no state written back (eval branches) */
/* ---------------------------------------------------------------------- */
/* Every segment starts from the same S_in and nothing carries over between
 * them, so a workgroup takes one v-head and spw consecutive segments (as many
 * as keep about SB_WGS workgroups busy): S^T (bf16) goes to LDS once, then
 * per segment wave w (of 8: short per-wave chains, since a few branches
 * give few workgroups) computes columns 16w..16w+15 of
 *   V' = U - W S,  O = (Q e^G) S + QKm V'
 * for the 16-row blocks that hold tokens (the same 16x16x32 steps and
 * operand fragments as gdn_chunk_b_kernel), and the workgroup applies the
 * gated RMSNorm of gdn_norm_gate_kernel to the segment's rows. */
constexpr int SB_WGS = 512;
constexpr int SB_THREADS = 512; /* 8 waves, 16 state columns each */

__global__ __launch_bounds__(SB_THREADS) void gdn_short_b_kernel(
    const bf16x8 *__restrict__ Wi, const bf16x8 *__restrict__ Qgi, const bf16x8 *__restrict__ QKi,
    const bf16x8 *__restrict__ Ui, const int32_t *__restrict__ chunk_tok0,
    const int32_t *__restrict__ chunk_len, const int32_t *__restrict__ seg_chunk0,
    const int32_t *__restrict__ seg_nchunk, int nseg, int spw, const float *__restrict__ S_in,
    int Hv,
    const bf16 *__restrict__ z, int zs, const float *__restrict__ nw, float eps,
    bf16 *__restrict__ y) {
    __shared__ __attribute__((aligned(16))) bf16 sT[DV][DK + 8]; /* S^T [column][dk]       */
    __shared__ __attribute__((aligned(16))) bf16 vT[DV][CH + 8]; /* V'^T [column][token]   */
    __shared__ __attribute__((aligned(16))) bf16 ob[CH][DV + 8]; /* O (bf16) [token][column] */

    const int hv = blockIdx.y, sg0 = blockIdx.x * spw;
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
    for (int i = tid; i < DV * (CH + 8) / 8; i += SB_THREADS)
        ((bf16x8 *)&vT[0][0])[i] = bf16x8{};
    lds_barrier();

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
        const size_t cb = (size_t)ch * Hv + hv;

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
                qg[s] = Qgi[cb * 1024 + rb * 256 + 64 * s + lane];
            }
            /* U fragment of the 32-column block holding these 16 columns:
             * values 0..3 its first 16 columns, 4..7 the second */
            const bf16x8 u = Ui[cb * 1024 + ((wave >> 1) * 4 + rb) * 64 + lane];
            const int jh = 4 * (wave & 1);
            floatx4 V = {};
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const bf16x8 sb = *(const bf16x8 *)&sT[col0 + c16][32 * s + 8 * q4];
                V = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w[s], sb, V, 0, 0, 0);
                O[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qg[s], sb, O[rb], 0, 0, 0);
            }
            bf16x4 p;
#pragma unroll
            for (int i = 0; i < 4; i++)
                p[i] = f2bf(bf2f(u[jh + i]) - V[i]);
            *(bf16x4 *)&vT[col0 + c16][16 * rb + 4 * q4] = p;
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
                const bf16x8 qk = QKi[cb * 512 + rb * 128 + 64 * s + lane];
                const bf16x8 vb = *(const bf16x8 *)&vT[col0 + c16][32 * s + 8 * q4];
                O[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qk, vb, O[rb], 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
                ob[16 * rb + 4 * q4 + i][col0 + c16] = f2bf(O[rb][i]);
        }
        lds_barrier();
        /* gated RMSNorm, 16 lanes per token row (as gdn_norm_gate_kernel) */
        for (int r0 = 0; r0 < L; r0 += SB_THREADS / 16) {
            const int t = r0 + (tid >> 4), sl = tid & 15;
            if (t < L) { /* whole 16-lane groups */
                const bf16x8 ov = *(const bf16x8 *)&ob[t][8 * sl];
                const size_t n = (size_t)t0 + t;
                const bf16 *zr = z + n * zs + hv * DV + 8 * sl;
                float ss = 0.f;
#pragma unroll
                for (int e = 0; e < 8; e++)
                    ss += bf2f(ov[e]) * bf2f(ov[e]);
#pragma unroll
                for (int m = 1; m < 16; m <<= 1)
                    ss += __shfl_xor(ss, m, 64);
                const float inv = rsqrtf(ss * (1.f / DV) + eps);
                bf16x8 res;
#pragma unroll
                for (int e = 0; e < 8; e++)
                    res[e] = f2bf(bf2f(f2bf(bf2f(ov[e]) * inv)) * wl[e] * silu_f(bf2f(zr[e])));
                *(bf16x8 *)(y + (n * Hv + hv) * DV + 8 * sl) = res;
            }
        }
        lds_barrier(); /* ob and vT are rewritten by the next segment */
    }
}

/* y = bf16( w * bf16(o * rsqrt(mean o^2 + eps)) * silu(z) ): 16 lanes per
 * (token, v-head) row, 8 columns a lane. REF src/kernels/gdn.cu:193-216. */
template <bool VEC>
__global__ __launch_bounds__(256) void gdn_norm_gate_kernel(const bf16 *__restrict__ o,
                                                            const bf16 *__restrict__ z, int zs,
                                                            const float *__restrict__ w, float eps,
                                                            int rows, int Hv,
                                                            bf16 *__restrict__ y) {
    const int row = blockIdx.x * 16 + (threadIdx.x >> 4);
    const int s = threadIdx.x & 15;
    if (row >= rows)
        return; /* whole 16-lane groups leave together */
    const int n = row / Hv, hv = row - n * Hv;
    const bf16x8 ov = *(const bf16x8 *)(o + (size_t)row * DV + 8 * s);
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
        ss += bf2f(ov[e]) * bf2f(ov[e]);
#pragma unroll
    for (int m = 1; m < 16; m <<= 1)
        ss += __shfl_xor(ss, m, 64);
    const float inv = rsqrtf(ss * (1.f / DV) + eps);
    bf16x8 r;
#pragma unroll
    for (int e = 0; e < 8; e++)
        r[e] = f2bf(bf2f(f2bf(bf2f(ov[e]) * inv)) * wl[e] * silu_f(bf2f(zv[e])));
    *(bf16x8 *)(y + (size_t)row * DV + 8 * s) = r;
}

} // namespace
} // namespace CUJEV_KNS
using namespace CUJEV_KNS;

extern "C" hipError_t k_gdn_conv_prep(const bf16_t *proj, int proj_stride, const float *conv_w,
                                      const float *conv_in, float *conv_out, int seg0_len,
                                      const int32_t *own_base, const float *A_neg_exp,
                                      const float *dt_bias, int N, int Hk, int Hv, bf16_t *q,
                                      bf16_t *k, bf16_t *v, float *g, float *beta,
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
                       dt_bias, N, Hk, Hv, (bf16 *)q, (bf16 *)k, (bf16 *)v, g, beta);
    if (conv_out) {
        const int C = nheads * DK;
        hipLaunchKernelGGL(gdn_conv_tail_kernel, dim3((unsigned)CEIL_DIV(C, 256)), dim3(256), 0,
                           stream, (const bf16 *)proj, proj_stride, conv_in, conv_out, seg0_len, C);
    }
    return hipGetLastError();
}

/* Phase B and the gated norm after phase A (either front end). */
static hipError_t gdn_phase_b(const cujev_chunks *ck, const float *S_in, float *S_out,
                              const bf16_t *z, int z_stride, const float *norm_w, float eps,
                              int Hv, bf16_t *y, const cujev_gdn_scratch *ws, int N,
                              const TailJob &tail, hipStream_t stream) {
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
                           dim3(SB_THREADS), 0, stream, (const bf16x8 *)ws->W, (const bf16x8 *)ws->Qg,
                           (const bf16x8 *)ws->QK, (const bf16x8 *)ws->U, ck->chunk_tok0,
                           ck->chunk_len, packed ? nullptr : ck->seg_chunk0,
                           packed ? nullptr : ck->seg_nchunk, units, spw, S_in, Hv,
                           (const bf16 *)z, z_stride, norm_w, eps, (bf16 *)y);
        return hipGetLastError();
    }
    if (packed)
        return hipErrorInvalidValue; /* packed segments write no final state */
    const int units = ck->num_segments * Hv;
    const int ntail = tail.conv_out ? CEIL_DIV(tail.C, 256) : 0;
    hipLaunchKernelGGL(gdn_chunk_b_kernel, dim3((unsigned)(NCB * CEIL_DIV(units, 8) * 8 + ntail)),
                       dim3(256), 0, stream, (const bf16x8 *)ws->W, (const bf16x8 *)ws->Qg,
                       (const bf16x8 *)ws->QK, (const bf16x8 *)ws->KgT, (const bf16x8 *)ws->U,
                       ws->Glast, ck->chunk_tok0, ck->chunk_len, ck->seg_chunk0, ck->seg_nchunk,
                       S_in, S_out, Hv, units, (bf16 *)ws->O, tail);
    const int rows = N * Hv;
    const bool zvec = z_stride % 8 == 0 && ((uintptr_t)z & 15) == 0;
    hipLaunchKernelGGL(zvec ? gdn_norm_gate_kernel<true> : gdn_norm_gate_kernel<false>,
                       dim3((unsigned)CEIL_DIV(rows, 16)), dim3(256), 0, stream,
                       (const bf16 *)ws->O, (const bf16 *)z, z_stride, norm_w, eps, rows, Hv,
                       (bf16 *)y);
    return hipGetLastError();
}

extern "C" hipError_t k_gdn_scan(const bf16_t *q, const bf16_t *k, const bf16_t *v, const float *g,
                                 const float *beta, const cujev_chunks *ck, const float *S_in,
                                 float *S_out, const bf16_t *z, int z_stride, const float *norm_w,
                                 float eps, int Hk, int Hv, bf16_t *y, const cujev_gdn_scratch *ws,
                                 int N, hipStream_t stream) {
    if (ck->num_chunks <= 0 || N <= 0)
        return hipSuccess;
    if (Hk <= 0 || Hv % Hk != 0 || (ck->chunk_starts && S_out))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(gdn_chunk_a_kernel<0>, dim3((unsigned)ck->num_chunks, (unsigned)Hv),
                       dim3(256), 0, stream, (const bf16 *)q, (const bf16 *)k, (const bf16 *)v, g,
                       beta, ConvSrc{}, ck->chunk_tok0, ck->chunk_len, ck->chunk_starts, Hk, Hv,
                       (bf16 *)ws->W, (bf16 *)ws->Qg, (bf16 *)ws->QK, (bf16 *)ws->KgT,
                       (bf16 *)ws->U, ws->Glast);
    return gdn_phase_b(ck, S_in, S_out, z, z_stride, norm_w, eps, Hv, y, ws, N, TailJob{},
                       stream);
}

extern "C" hipError_t k_gdn_layer(const bf16_t *proj, int proj_stride, const float *conv_w,
                                  const float *conv_in, float *conv_out, int seg0_len,
                                  const int32_t *own_base, const float *A_neg_exp,
                                  const float *dt_bias, const cujev_chunks *ck, const float *S_in,
                                  float *S_out, const float *norm_w, float eps, int Hk, int Hv,
                                  bf16_t *y, const cujev_gdn_scratch *ws, int N,
                                  hipStream_t stream) {
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
    const ConvSrc cv{(const bf16 *)proj, proj_stride, conv_w, conv_in, own_base,
                     A_neg_exp,          dt_bias,     N};
    /* the conv tail rides along with phase B */
    const TailJob tail{(const bf16 *)proj, proj_stride, conv_in, conv_out, seg0_len, C};
    hipLaunchKernelGGL(conv_in ? gdn_chunk_a_kernel<2> : gdn_chunk_a_kernel<1>,
                       dim3((unsigned)ck->num_chunks, (unsigned)Hv), dim3(256), 0, stream,
                       (const bf16 *)nullptr, (const bf16 *)nullptr, (const bf16 *)nullptr,
                       (const float *)nullptr, (const float *)nullptr, cv, ck->chunk_tok0,
                       ck->chunk_len, ck->chunk_starts, Hk, Hv, (bf16 *)ws->W, (bf16 *)ws->Qg,
                       (bf16 *)ws->QK, (bf16 *)ws->KgT, (bf16 *)ws->U, ws->Glast);
    return gdn_phase_b(ck, S_in, S_out, proj + C, proj_stride, norm_w, eps, Hv, y, ws, N, tail,
                       stream);
}
