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
 * tokens; lane s holds channels 8s..8s+7. The PREP_T + 3 pre-conv rows the
 * group needs are loaded once (16 bytes per lane and row when the projection
 * rows allow it) and the 4-tap window slides over them in registers. Groups
 * are numbered token block fastest, 16 per 256-thread workgroup. Groups of
 * head h < Hv also produce g and beta of v-head h for their tokens. */
constexpr int PREP_T = 8;

template <bool VEC>
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

    if (head < Hv && s < PREP_T && n0 + s < N) {
        const int n = n0 + s;
        const bf16 *ab = proj + (size_t)n * ps + C + Hv * DV; /* b then a */
        const float bv = bf2f(ab[head]), av = bf2f(ab[Hv + head]);
        bo[(size_t)n * Hv + head] = sigmoid_f(bv);
        go[(size_t)n * Hv + head] = A_neg_exp[head] * softplus_f(av + dt_bias[head]);
    }

    float w[8][4];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float4 t = *(const float4 *)(conv_w + (size_t)(c0 + e) * 4);
        w[e][0] = t.x;
        w[e][1] = t.y;
        w[e][2] = t.z;
        w[e][3] = t.w;
    }
    bf16x8 x[PREP_T + 3];
#pragma unroll
    for (int r = 0; r < PREP_T + 3; r++) {
        const int row = n0 - 3 + r;
        x[r] = bf16x8{};
        if (row >= 0 && row < N) {
            const bf16 *src = proj + (size_t)row * ps + c0;
            if constexpr (VEC) {
                x[r] = *(const bf16x8 *)src;
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++)
                    x[r][e] = src[e];
            }
        }
    }
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
#pragma unroll
    for (int j = 0; j < PREP_T; j++) {
        const int n = n0 + j;
        if (n >= N)
            break; /* uniform over the group */
        const int local = n - own_base[n];
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; e++)
            y[e] = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tau = local - 3 + i; /* local index of the tap */
            if (tau >= 0) {
#pragma unroll
                for (int e = 0; e < 8; e++)
                    y[e] += w[e][i] * bf2f(x[j + i][e]);
            } else if (conv_in) {
#pragma unroll
                for (int e = 0; e < 8; e++)
                    y[e] += w[e][i] * conv_in[(size_t)(c0 + e) * 3 + tau + 3];
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
/* Phase B feeds S and V' (accumulators) back into MFMAs as B operands. An
 * accumulator supplies the k values of a 16-wide step in the order
 * 4h+0..3, 8+4h+0..3 (lane half h), so every A operand phase B reads is stored
 * with bits 2 and 3 of its column index swapped inside each 16-column group:
 * the 8 consecutive stored values at 16ks + 8h are then exactly the matching
 * original columns and one 16-byte read fetches them. */
DEV int swap23(int j) { return (j & ~12) | ((j & 4) << 1) | ((j & 8) >> 1); }

struct __attribute__((aligned(16))) ChunkA_Smem {
    bf16 K[CH][DK + 8];  /* k rows                                            */
    bf16 Q[CH][DK + 8];  /* q rows; later W staged for coalesced stores       */
    bf16 V[CH][DV + 8];  /* v rows; later masked QK^T staged                  */
    bf16 Kt[DK][CH + 8]; /* (beta e^G k)^T, later (k e^{Glast-G})^T swapped   */
    bf16 Vt[DV][CH + 8]; /* (beta v)^T                                        */
    float A[CH][CH + 1]; /* strictly lower A                                  */
    float T[CH][CH + 1]; /* (I + A)^-1                                        */
    float M[3][16][17];  /* block products                                    */
    float G[CH], B[CH];
};

DEV bf16x8 ld8(const bf16 *p) { return *(const bf16x8 *)p; }
DEV void st4(bf16 *p, bf16 a, bf16 b, bf16 c, bf16 d) { *(bf16x4 *)p = bf16x4{a, b, c, d}; }

__global__ __launch_bounds__(256) void gdn_chunk_a_kernel(
    const bf16 *__restrict__ qh, const bf16 *__restrict__ kh_, const bf16 *__restrict__ vh,
    const float *__restrict__ g, const float *__restrict__ beta,
    const int32_t *__restrict__ chunk_tok0, const int32_t *__restrict__ chunk_len, int Hk, int Hv,
    bf16 *__restrict__ Wo, bf16 *__restrict__ Qgo, bf16 *__restrict__ QKo,
    bf16 *__restrict__ KgTo, bf16 *__restrict__ Uo, float *__restrict__ Glo) {
    __shared__ ChunkA_Smem sm;
    const int ch = blockIdx.x, hv = blockIdx.y;
    const int hk = hv / (Hv / Hk);
    const int t0 = chunk_tok0[ch], L = chunk_len[ch];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int h = lane >> 5, col = lane & 31;
    const size_t cb = (size_t)ch * Hv + hv;

    /* gates and cumulative log-decay (zero past L, so G stays at G[L-1]) */
    if (wave == 0) {
        float gv = lane < L ? g[(size_t)(t0 + lane) * Hv + hv] : 0.f;
        const float bv = lane < L ? beta[(size_t)(t0 + lane) * Hv + hv] : 0.f;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float up = __shfl_up(gv, o, 64);
            if (lane >= o)
                gv += up;
        }
        sm.G[lane] = gv;
        sm.B[lane] = bv;
    }
    /* q, k, v rows (zero past L), 16-byte coalesced */
    for (int i = tid; i < CH * (DK / 8); i += 256) {
        const int t = i >> 4, c8 = (i & 15) * 8;
        bf16x8 kv = {}, qv = {}, vv = {};
        if (t < L) {
            kv = ld8(kh_ + ((size_t)(t0 + t) * Hk + hk) * DK + c8);
            qv = ld8(qh + ((size_t)(t0 + t) * Hk + hk) * DK + c8);
            vv = ld8(vh + ((size_t)(t0 + t) * Hv + hv) * DV + c8);
        }
        *(bf16x8 *)&sm.K[t][c8] = kv;
        *(bf16x8 *)&sm.Q[t][c8] = qv;
        *(bf16x8 *)&sm.V[t][c8] = vv;
    }
    __syncthreads();
    const float Glast = sm.G[CH - 1];
    /* q e^G straight to HBM (16 lanes per row: coalesced) */
    for (int i = tid; i < CH * (DK / 8); i += 256) {
        const int t = i >> 4, c8 = (i & 15) * 8;
        const float eg = fast_exp(sm.G[t]);
        bf16x8 qv = *(const bf16x8 *)&sm.Q[t][c8];
        bf16 *qrow = Qgo + cb * CH * DK + t * DK;
        st4(qrow + swap23(c8), f2bf(bf2f(qv[0]) * eg), f2bf(bf2f(qv[1]) * eg),
            f2bf(bf2f(qv[2]) * eg), f2bf(bf2f(qv[3]) * eg));
        st4(qrow + swap23(c8 + 4), f2bf(bf2f(qv[4]) * eg), f2bf(bf2f(qv[5]) * eg),
            f2bf(bf2f(qv[6]) * eg), f2bf(bf2f(qv[7]) * eg));
    }
    /* (beta e^G k)^T and (beta v)^T: consecutive lanes take consecutive
     * tokens so the transposed 2-byte writes hit consecutive addresses */
    for (int i = tid; i < CH * (DK / 8); i += 256) {
        const int t = i & 63, c8 = (i >> 6) * 8;
        const float sk = sm.B[t] * fast_exp(sm.G[t]), sv = sm.B[t];
        bf16x8 kv = *(const bf16x8 *)&sm.K[t][c8];
        bf16x8 vv = *(const bf16x8 *)&sm.V[t][c8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            sm.Kt[c8 + e][t] = f2bf(bf2f(kv[e]) * sk);
            sm.Vt[c8 + e][t] = f2bf(bf2f(vv[e]) * sv);
        }
    }
    __syncthreads(); /* V rows are free from here on: QK^T staging */

    /* K K^T and Q K^T: wave w owns the 32x32 tile (w>>1, w&1) of both */
    {
        const int ti = wave >> 1, tj = wave & 1;
        floatx16 kk = {}, qk = {};
#pragma unroll
        for (int ks = 0; ks < DK / 16; ks++) {
            const int c = 16 * ks + 8 * h;
            bf16x8 ak = *(const bf16x8 *)&sm.K[32 * ti + col][c];
            bf16x8 aq = *(const bf16x8 *)&sm.Q[32 * ti + col][c];
            bf16x8 bk = *(const bf16x8 *)&sm.K[32 * tj + col][c];
            kk = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ak, bk, kk, 0, 0, 0);
            qk = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aq, bk, qk, 0, 0, 0);
        }
        const int j = 32 * tj + col;
        const float Gj = sm.G[j];
        bf16 *qks = &sm.V[0][0] + swap23(j); /* [64][72] bf16 staging */
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int i = 32 * ti + 8 * (r >> 2) + 4 * h + (r & 3);
            const float dec = i >= j ? fast_exp(sm.G[i] - Gj) : 0.f;
            sm.A[i][j] = i > j ? sm.B[i] * kk[r] * dec : 0.f;
            qks[i * (CH + 8)] = f2bf(i >= j ? qk[r] * dec : 0.f);
        }
    }
    __syncthreads();
    /* masked QK^T rows to HBM; T = (I + A)^-1 diagonal blocks by forward
     * substitution (wave w inverts block w, lane c < 16 owns column c) */
    for (int i = tid; i < CH * (CH / 8); i += 256) {
        const int r = i >> 3, c8 = (i & 7) * 8;
        *(bf16x8 *)(QKo + cb * CH * CH + r * CH + c8) = *(const bf16x8 *)(&sm.V[0][0] + r * (CH + 8) + c8);
    }
    if (lane < 16) {
        const int b0 = 16 * wave, c = lane;
        float t[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < i; k++)
                acc += sm.A[b0 + i][b0 + k] * t[k];
            t[i] = (i == c ? 1.f : 0.f) - acc;
        }
#pragma unroll
        for (int i = 0; i < 16; i++)
            sm.T[b0 + i][b0 + c] = t[i];
    }
    /* ... then the strictly lower blocks by distance from the diagonal:
     * T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj */
    for (int lvl = 1; lvl < 4; lvl++) {
        __syncthreads();
        const int nb = 4 - lvl;
        for (int e = tid; e < nb * 256; e += 256) {
            const int b = e >> 8, r = (e >> 4) & 15, c = e & 15;
            const int bj = b, bi = b + lvl;
            float acc = 0.f;
            for (int bk = bj; bk < bi; bk++)
#pragma unroll
                for (int x = 0; x < 16; x++)
                    acc += sm.A[16 * bi + r][16 * bk + x] * sm.T[16 * bk + x][16 * bj + c];
            sm.M[b][r][c] = acc;
        }
        __syncthreads();
        for (int e = tid; e < nb * 256; e += 256) {
            const int b = e >> 8, r = (e >> 4) & 15, c = e & 15;
            const int bj = b, bi = b + lvl;
            float acc = 0.f;
#pragma unroll
            for (int x = 0; x < 16; x++)
                acc += sm.T[16 * bi + r][16 * bi + x] * sm.M[b][x][c];
            sm.T[16 * bi + r][16 * bj + c] = -acc;
        }
    }
    for (int e = tid; e < CH * CH; e += 256) {
        const int i = e >> 6, j = e & 63;
        if ((j >> 4) > (i >> 4))
            sm.T[i][j] = 0.f;
    }
    __syncthreads();

    /* W = T (beta e^G K), U = T (beta V): wave w owns rows 32(w>>1).. and
     * columns 64(w&1)..+64 of both. W is staged (swapped columns) in the q
     * rows' LDS for coalesced stores; U goes out in accumulator-fragment
     * order, i.e. exactly the 16 values lane l of phase B's wave (column
     * block) needs, contiguous. */
    {
        const int mi = wave >> 1, nh = wave & 1;
        floatx16 w[2] = {}, u[2] = {};
#pragma unroll
        for (int ks = 0; ks < CH / 16; ks++) {
            const int k0 = 16 * ks + 8 * h;
            bf16x8 a;
#pragma unroll
            for (int e = 0; e < 8; e++)
                a[e] = f2bf(sm.T[32 * mi + col][k0 + e]);
#pragma unroll
            for (int nj = 0; nj < 2; nj++) {
                const int c = 64 * nh + 32 * nj + col;
                bf16x8 bk = *(const bf16x8 *)&sm.Kt[c][k0];
                bf16x8 bv = *(const bf16x8 *)&sm.Vt[c][k0];
                w[nj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bk, w[nj], 0, 0, 0);
                u[nj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bv, u[nj], 0, 0, 0);
            }
        }
#pragma unroll
        for (int nj = 0; nj < 2; nj++) {
            const int c = swap23(64 * nh + 32 * nj + col);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int i = 32 * mi + 8 * (r >> 2) + 4 * h + (r & 3);
                sm.Q[i][c] = f2bf(w[nj][r]);
            }
            const int wblk = 2 * nh + nj; /* phase B's wave owning these 32 columns */
            bf16 *uo = Uo + (((cb * 4 + wblk) * 2 + mi) * 64 + lane) * 16;
            bf16x8 lo, hi;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                lo[e] = f2bf(u[nj][e]);
                hi[e] = f2bf(u[nj][8 + e]);
            }
            *(bf16x8 *)uo = lo;
            *(bf16x8 *)(uo + 8) = hi;
        }
    }
    __syncthreads(); /* everyone is done with Kt; W is staged */
    for (int i = tid; i < CH * (DK / 8); i += 256) {
        const int t = i >> 4, c8 = (i & 15) * 8;
        *(bf16x8 *)(Wo + cb * CH * DK + t * DK + c8) = *(const bf16x8 *)&sm.Q[t][c8];
    }
    /* (k e^{Glast - G})^T with swapped token columns, then rows to HBM */
    for (int i = tid; i < CH * (DK / 8); i += 256) {
        const int t = i & 63, c8 = (i >> 6) * 8;
        const float ek = fast_exp(Glast - sm.G[t]);
        bf16x8 kv = *(const bf16x8 *)&sm.K[t][c8];
        const int ts = swap23(t);
#pragma unroll
        for (int e = 0; e < 8; e++)
            sm.Kt[c8 + e][ts] = f2bf(bf2f(kv[e]) * ek);
    }
    __syncthreads();
    for (int i = tid; i < DK * (CH / 8); i += 256) {
        const int r = i >> 3, c8 = (i & 7) * 8;
        *(bf16x8 *)(KgTo + cb * DK * CH + r * CH + c8) = *(const bf16x8 *)&sm.Kt[r][c8];
    }
    if (tid == 0)
        Glo[cb] = Glast;
}

/* ---------------------------------------------------------------------- */
/* phase B: the state recurrence over chunks                                */
/* ---------------------------------------------------------------------- */
/* One LDS stage holds the shared A operands of one chunk, 16-byte chunks
 * XOR-swizzled per row for conflict-free ds_read_b128:
 *   W   [64][128]  at 0        Qg [64][128] at 16 KiB
 *   QK  [64][64]   at 32 KiB   KgT [128][64] at 40 KiB        (56 KiB) */
constexpr int B_W = 0, B_QG = 16384, B_QK = 32768, B_KGT = 40960, B_BUF = 57344;
constexpr int B_CHUNKS = B_BUF / 16;     /* 3584 */
constexpr int B_PER = B_CHUNKS / 256;    /* 14 per thread */

DEV int swz16(int r) { return r & 15; }
DEV int swz8(int r) { return (r & 7) ^ ((r >> 3) & 1); }

/* global source and LDS offset of 16-byte chunk f of one stage */
DEV void stage_addr(int f, const bf16 *W, const bf16 *Qg, const bf16 *QK, const bf16 *KgT,
                    const bf16 *&src, int &dst) {
    if (f < 2048) {
        const int g = f & 1023, row = g >> 4, c = g & 15;
        src = (f < 1024 ? W : Qg) + row * DK + c * 8;
        dst = (f < 1024 ? B_W : B_QG) + row * 256 + ((c ^ swz16(row)) << 4);
    } else if (f < 2560) {
        const int g = f - 2048, row = g >> 3, c = g & 7;
        src = QK + row * CH + c * 8;
        dst = B_QK + row * 128 + ((c ^ swz8(row)) << 4);
    } else {
        const int g = f - 2560, row = g >> 3, c = g & 7;
        src = KgT + row * CH + c * 8;
        dst = B_KGT + row * 128 + ((c ^ swz8(row)) << 4);
    }
}

DEV bf16x8 acc_as_b(const floatx16 &c, int s) {
    bf16x8 b;
#pragma unroll
    for (int e = 0; e < 8; e++)
        b[e] = f2bf(c[8 * s + e]);
    return b;
}

__global__ __launch_bounds__(256) void gdn_chunk_b_kernel(
    const bf16 *__restrict__ Wi, const bf16 *__restrict__ Qgi, const bf16 *__restrict__ QKi,
    const bf16 *__restrict__ KgTi, const bf16 *__restrict__ Ui, const float *__restrict__ Gli,
    const int32_t *__restrict__ chunk_tok0, const int32_t *__restrict__ chunk_len,
    const int32_t *__restrict__ seg_chunk0, const int32_t *__restrict__ seg_nchunk,
    const float *__restrict__ S_in, float *__restrict__ S_out, int Hv, float *__restrict__ o) {
    __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * B_BUF];
    const int seg = blockIdx.x, hv = blockIdx.y;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int h = lane >> 5, col = lane & 31;
    const int dv = 32 * wave + col; /* this lane's state column */

    floatx16 S[4]; /* S[:, dv], rows 32ti + 8(r/4) + 4h + r%4 */
#pragma unroll
    for (int ti = 0; ti < 4; ti++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int dk = 32 * ti + 8 * (r >> 2) + 4 * h + (r & 3);
            S[ti][r] = S_in ? S_in[((size_t)hv * DK + dk) * DV + dv] : 0.f;
        }
    }
    const int c0 = seg_chunk0[seg], nc = seg_nchunk[seg];

    u32x4 stage[B_PER];
    bf16x8 ucur[4], unext[4];
    auto fetch = [&](int ch) {
        const size_t cb = (size_t)ch * Hv + hv;
        const bf16 *W = Wi + cb * CH * DK, *Qg = Qgi + cb * CH * DK, *QK = QKi + cb * CH * CH,
                   *KgT = KgTi + cb * DK * CH;
#pragma unroll
        for (int j = 0; j < B_PER; j++) {
            const bf16 *src;
            int dst;
            stage_addr(tid + 256 * j, W, Qg, QK, KgT, src, dst);
            stage[j] = *(const u32x4 *)src;
        }
        const bf16 *up = Ui + (cb * 4 + wave) * 2 * 64 * 16 + lane * 16;
        unext[0] = ld8(up);
        unext[1] = ld8(up + 8);
        unext[2] = ld8(up + 64 * 16);
        unext[3] = ld8(up + 64 * 16 + 8);
    };
    auto store = [&](unsigned char *buf) {
#pragma unroll
        for (int j = 0; j < B_PER; j++) {
            const bf16 *src;
            int dst;
            stage_addr(tid + 256 * j, nullptr, nullptr, nullptr, nullptr, src, dst);
            *(u32x4 *)(buf + dst) = stage[j];
        }
    };

    if (nc > 0) {
        fetch(c0);
        store(smem);
#pragma unroll
        for (int e = 0; e < 4; e++)
            ucur[e] = unext[e];
        __syncthreads();
    }
    for (int ci = 0; ci < nc; ci++) {
        const int ch = c0 + ci;
        const int t0 = chunk_tok0[ch], L = chunk_len[ch];
        const float Glast = Gli[(size_t)ch * Hv + hv];
        const bool more = ci + 1 < nc;
        if (more)
            fetch(ch + 1);
        const unsigned char *buf = smem + (ci & 1) * B_BUF;

        bf16x8 Sb[8];
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
            Sb[ks] = acc_as_b(S[ks >> 1], ks & 1);

        /* V' = U - W S   (tokens x dv) */
        floatx16 Vn[2];
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
            floatx16 acc = {};
            const int r = 32 * mt + col;
#pragma unroll
            for (int ks = 0; ks < 8; ks++) {
                bf16x8 a = *(const bf16x8 *)(buf + B_W + r * 256 + (((2 * ks + h) ^ swz16(r)) << 4));
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, Sb[ks], acc, 0, 0, 0);
            }
#pragma unroll
            for (int e = 0; e < 8; e++) {
                Vn[mt][e] = bf2f(ucur[2 * mt][e]) - acc[e];
                Vn[mt][8 + e] = bf2f(ucur[2 * mt + 1][e]) - acc[8 + e];
            }
        }
        bf16x8 Vb[4];
#pragma unroll
        for (int ks = 0; ks < 4; ks++)
            Vb[ks] = acc_as_b(Vn[ks >> 1], ks & 1);

        /* O = (Q e^G) S + QKm V' -> fp32 o[token][hv][dv] */
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
            floatx16 acc = {};
            const int r = 32 * mt + col;
#pragma unroll
            for (int ks = 0; ks < 8; ks++) {
                bf16x8 a = *(const bf16x8 *)(buf + B_QG + r * 256 + (((2 * ks + h) ^ swz16(r)) << 4));
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, Sb[ks], acc, 0, 0, 0);
            }
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                bf16x8 a = *(const bf16x8 *)(buf + B_QK + r * 128 + (((2 * ks + h) ^ swz8(r)) << 4));
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, Vb[ks], acc, 0, 0, 0);
            }
#pragma unroll
            for (int rr = 0; rr < 16; rr++) {
                const int t = 32 * mt + 8 * (rr >> 2) + 4 * h + (rr & 3);
                if (t < L)
                    o[((size_t)(t0 + t) * Hv + hv) * DV + dv] = acc[rr];
            }
        }

        /* S = e^{G_last} S + (K e^{G_last - G})^T V' */
        const float dec = fast_exp(Glast);
#pragma unroll
        for (int ti = 0; ti < 4; ti++) {
            floatx16 acc = S[ti] * dec;
            const int r = 32 * ti + col;
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                bf16x8 a = *(const bf16x8 *)(buf + B_KGT + r * 128 + (((2 * ks + h) ^ swz8(r)) << 4));
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, Vb[ks], acc, 0, 0, 0);
            }
            S[ti] = acc;
        }

        if (more) {
            store(smem + ((ci + 1) & 1) * B_BUF);
#pragma unroll
            for (int e = 0; e < 4; e++)
                ucur[e] = unext[e];
        }
        __syncthreads();
    }
    if (S_out && seg == 0) {
#pragma unroll
        for (int ti = 0; ti < 4; ti++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int dk = 32 * ti + 8 * (r >> 2) + 4 * h + (r & 3);
                S_out[((size_t)hv * DK + dk) * DV + dv] = S[ti][r];
            }
        }
    }
}

/* y = bf16( w * bf16(o * rsqrt(mean o^2 + eps)) * silu(z) ): one wave per
 * (token, v-head) row, lane = 2 columns. REF src/kernels/gdn.cu:193-216. */
__global__ __launch_bounds__(256) void gdn_norm_gate_kernel(const float *__restrict__ o,
                                                            const bf16 *__restrict__ z, int zs,
                                                            const float *__restrict__ w, float eps,
                                                            int rows, int Hv,
                                                            bf16 *__restrict__ y) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows)
        return;
    const int n = row / Hv, hv = row % Hv;
    const float2 v = *(const float2 *)(o + (size_t)row * DV + 2 * lane);
    const float ss = wave_sum(v.x * v.x + v.y * v.y);
    const float inv = rsqrtf(ss * (1.f / DV) + eps);
    const bf16 *zr = z + (size_t)n * zs + hv * DV + 2 * lane;
    const float n0 = bf2f(f2bf(v.x * inv)) * w[2 * lane];
    const float n1 = bf2f(f2bf(v.y * inv)) * w[2 * lane + 1];
    bf16 *yr = y + (size_t)row * DV + 2 * lane;
    yr[0] = f2bf(n0 * silu_f(bf2f(zr[0])));
    yr[1] = f2bf(n1 * silu_f(bf2f(zr[1])));
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
    auto kern = vec ? gdn_conv_prep_kernel<true> : gdn_conv_prep_kernel<false>;
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

extern "C" hipError_t k_gdn_scan(const bf16_t *q, const bf16_t *k, const bf16_t *v, const float *g,
                                 const float *beta, const cujev_chunks *ck, const float *S_in,
                                 float *S_out, const bf16_t *z, int z_stride, const float *norm_w,
                                 float eps, int Hk, int Hv, bf16_t *y, const cujev_gdn_scratch *ws,
                                 int N, hipStream_t stream) {
    if (ck->num_chunks <= 0 || N <= 0)
        return hipSuccess;
    if (Hk <= 0 || Hv % Hk != 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(gdn_chunk_a_kernel, dim3((unsigned)ck->num_chunks, (unsigned)Hv), dim3(256),
                       0, stream, (const bf16 *)q, (const bf16 *)k, (const bf16 *)v, g, beta,
                       ck->chunk_tok0, ck->chunk_len, Hk, Hv, (bf16 *)ws->W, (bf16 *)ws->Qg,
                       (bf16 *)ws->QK, (bf16 *)ws->KgT, (bf16 *)ws->U, ws->Glast);
    hipLaunchKernelGGL(gdn_chunk_b_kernel, dim3((unsigned)ck->num_segments, (unsigned)Hv),
                       dim3(256), 0, stream, (const bf16 *)ws->W, (const bf16 *)ws->Qg,
                       (const bf16 *)ws->QK, (const bf16 *)ws->KgT, (const bf16 *)ws->U, ws->Glast,
                       ck->chunk_tok0, ck->chunk_len, ck->seg_chunk0, ck->seg_nchunk, S_in, S_out,
                       Hv, ws->O);
    const int rows = N * Hv;
    hipLaunchKernelGGL(gdn_norm_gate_kernel, dim3((unsigned)CEIL_DIV(rows, 4)), dim3(256), 0,
                       stream, ws->O, (const bf16 *)z, z_stride, norm_w, eps, rows, Hv, (bf16 *)y);
    return hipGetLastError();
}
