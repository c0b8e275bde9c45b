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
    int local_of[PREP_T]; /* all segment offsets fetched up front, not per step */
#pragma unroll
    for (int j = 0; j < PREP_T; j++)
        local_of[j] = n0 + j < N ? n0 + j - own_base[n0 + j] : 0;
#pragma unroll
    for (int j = 0; j < PREP_T; j++) {
        const int n = n0 + j;
        if (n >= N)
            continue; /* uniform over the group */
        const int local = local_of[j];
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
    lds_barrier();
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
    lds_barrier(); /* V rows are free from here on: QK^T staging */

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
    lds_barrier();
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
        lds_barrier();
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
        lds_barrier();
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
    lds_barrier();

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
    lds_barrier(); /* everyone is done with Kt; W is staged */
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
    lds_barrier();
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
 *   QK  [64][64]   at 32 KiB   KgT [128][64] at 40 KiB
 *   U   wave w's accumulator fragments at 56 KiB + 4 KiB w, as
 *       [row block][half][lane][8]: 16-byte lane stride      (72 KiB)
 * A stage moves HBM -> LDS by buffer_load ... lds: lane l of a wave writes
 * its 16 bytes at LDS base + 16 l, so the swizzle is applied on the global
 * side (the lane landing on slot p of row r fetches chunk p ^ swz(r)). Wave
 * w issues 14 loads per stage, load j covering W/Qg rows 4(4j + w)..+3 or
 * QK/KgT rows 8(4j' + w)..+7; with that numbering every lane's offset inside
 * a load is the same for all j. Wave w also loads its own 4 KiB of U. */
constexpr int B_W = 0, B_QG = 16384, B_QK = 32768, B_KGT = 40960, B_U = 57344, B_BUF = 73728;

typedef __attribute__((address_space(3))) void *lds_ptr;
typedef __attribute__((address_space(3))) const unsigned char lds_u8;
DEV bf16x8 lds_read16(lds_u8 *base, uint32_t off) {
    return *(__attribute__((address_space(3))) const bf16x8 *)(base + off);
}
DEV __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}
DEV int swz16(int r) { return r & 15; }
DEV int swz8(int r) { return (r & 7) ^ ((r >> 3) & 1); }

DEV bf16x8 acc_as_b(const floatx16 &c, int s) {
    bf16x8 b;
#pragma unroll
    for (int e = 0; e < 8; e++)
        b[e] = f2bf(c[8 * s + e]);
    return b;
}

/* Per chunk, wave w (state columns 32w..32w+31) computes, in two straight-line
 * MFMA blocks with the A operands read from LDS six fragments ahead:
 *   block 1  V' = U - W S  and  O = (Q e^G) S           (4 chains, 32 MFMAs)
 *   block 2  O += QKm V'  and  S = e^{G_last} S + (K e^{G_last-G})^T V'
 *                                                        (6 chains, 24 MFMAs)
 * while the next chunk's stage streams into the other LDS buffer. */
constexpr int B_RING = 5;
constexpr int O_LDS = 136; /* fp32 row pitch of the transposed O tile: rows 4 apart sit 32 banks apart */

__global__ __launch_bounds__(256) void gdn_chunk_b_kernel(
    const bf16 *__restrict__ Wi, const bf16 *__restrict__ Qgi, const bf16 *__restrict__ QKi,
    const bf16 *__restrict__ KgTi, const bf16 *__restrict__ Ui, const float *__restrict__ Gli,
    const int32_t *__restrict__ chunk_tok0, const int32_t *__restrict__ chunk_len,
    const int32_t *__restrict__ seg_chunk0, const int32_t *__restrict__ seg_nchunk,
    const float *__restrict__ S_in, float *__restrict__ S_out, int Hv, int num_chunks,
    float *__restrict__ o) {
    __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * B_BUF];
    const int seg = blockIdx.x, hv = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, col = lane & 31;
    const int dv = 32 * wave + col; /* this lane's state column */
    lds_u8 *lds = (lds_u8 *)smem;

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

    /* stage loads: one resource per operand array (all chunks, all heads) */
    const uint32_t big = (uint32_t)num_chunks * Hv * CH * DK * 2; /* W, Qg, KgT bytes */
    const __amdgpu_buffer_rsrc_t rW = make_rsrc(Wi, big), rQg = make_rsrc(Qgi, big),
                                 rQK = make_rsrc(QKi, big / 2), rKgT = make_rsrc(KgTi, big);
    /* U of (chunk, head, wave): [row block mt][lane][16] in HBM; LDS slot
     * (mt, half, lane) holds elements 8 half .. 8 half + 7 of lane's row */
    const __amdgpu_buffer_rsrc_t rU = make_rsrc(Ui, big);
    const int l16 = lane >> 4, l8 = lane >> 3;
    const uint32_t off16 = l16 * 256 + (((lane & 15) ^ (4 * (wave & 3) + l16)) << 4);
    const uint32_t off8 = l8 * 128 + (((lane & 7) ^ (l8 ^ (wave & 1))) << 4);
    /* load j (0..17) of a stage: 14 of W/Qg/QK/KgT, then 4 of U */
    auto issue_load = [&](int j, int ch, unsigned char *buf) {
        const uint32_t cb = (uint32_t)(ch * Hv + hv);
        if (j >= 14) { /* U: j - 14 = 2 mt + half */
            const int q = j - 14;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rU, (lds_ptr)(buf + B_U + wave * 4096 + q * 1024), 16, lane * 32 + (q & 1) * 16,
                (cb * 4 + wave) * 4096 + (q >> 1) * 2048, 0, 0);
            return;
        }
        {
            if (j < 8) { /* W (j < 4) or Qg: rows 4 idx .. +3, 1 KiB */
                const int idx = 4 * (j & 3) + wave;
                const uint32_t lo = (uint32_t)idx * 1024;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    j < 4 ? rW : rQg, (lds_ptr)(buf + (j < 4 ? B_W : B_QG) + lo), 16, off16,
                    cb * (CH * DK * 2) + lo, 0, 0);
            } else { /* QK (j < 10) or KgT: rows 8 idx .. +7, 1 KiB */
                const int idx = 4 * (j < 10 ? j - 8 : j - 10) + wave;
                const uint32_t lo = (uint32_t)idx * 1024;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    j < 10 ? rQK : rKgT, (lds_ptr)(buf + (j < 10 ? B_QK : B_KGT) + lo), 16,
                    off8, cb * (j < 10 ? CH * CH * 2 : DK * CH * 2) + lo, 0, 0);
            }
        }
    };
    /* A-operand read sequence of one chunk: 32 block-1 reads (W then Qg of
     * k-step ks for row blocks 0, 1), then 24 block-2 reads (QK of row blocks
     * 0, 1 and KgT of row blocks 0..3 for each k-step). */
    auto addr_of = [&](int i, uint32_t buf) -> uint32_t {
        if (i < 32) {
            const int ks = i >> 2, mt = (i >> 1) & 1, q = i & 1; /* q: 0 W, 1 Qg */
            const int r = 32 * mt + col;
            return buf + (q ? B_QG : B_W) + r * 256 + (((2 * ks + h) ^ swz16(r)) << 4);
        }
        const int k = i - 32, ks = k / 6, u = k % 6;
        if (u < 2) {
            const int r = 32 * u + col;
            return buf + B_QK + r * 128 + (((2 * ks + h) ^ swz8(r)) << 4);
        }
        const int r = 32 * (u - 2) + col;
        return buf + B_KGT + r * 128 + (((2 * ks + h) ^ swz8(r)) << 4);
    };

    if (nc > 0) {
#pragma unroll
        for (int j = 0; j < 18; j++)
            issue_load(j, c0, smem);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        lds_barrier();
    }
    for (int ci = 0; ci < nc; ci++) {
        const int ch = c0 + ci;
        const int t0 = chunk_tok0[ch], L = chunk_len[ch];
        const float dec = fast_exp(Gli[(size_t)ch * Hv + hv]);
        const bool more = ci + 1 < nc;
        const uint32_t buf = (ci & 1) * B_BUF;
        unsigned char *nbuf = smem + (buf ^ B_BUF);

        bf16x8 Sb[8];
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
            Sb[ks] = acc_as_b(S[ks >> 1], ks & 1);

        bf16x8 ring[B_RING];
#pragma unroll
        for (int i = 0; i < B_RING; i++)
            ring[i] = lds_read16(lds, addr_of(i, buf));
        floatx16 Vacc[2] = {}, Oacc[2] = {};
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const bf16x8 a = ring[i % B_RING];
            ring[i % B_RING] = lds_read16(lds, addr_of(i + B_RING, buf));
            if (i % 3 == 0 && more)
                issue_load(i / 3, ch + 1, nbuf);
            const int ks = i >> 2, mt = (i >> 1) & 1;
            if (i & 1)
                Oacc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, Sb[ks], Oacc[mt], 0, 0, 0);
            else
                Vacc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, Sb[ks], Vacc[mt], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        /* V' = U - W S */
        bf16x8 Vb[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const bf16x8 u = lds_read16(lds, buf + B_U + wave * 4096 + j * 1024 + lane * 16);
#pragma unroll
            for (int e = 0; e < 8; e++)
                Vb[j][e] = f2bf(bf2f(u[e]) - Vacc[j >> 1][8 * (j & 1) + e]);
        }
#pragma unroll
        for (int ti = 0; ti < 4; ti++)
            S[ti] = S[ti] * dec;
#pragma unroll
        for (int i = 32; i < 56; i++) {
            const bf16x8 a = ring[i % B_RING];
            if (i + B_RING < 56)
                ring[i % B_RING] = lds_read16(lds, addr_of(i + B_RING, buf));
            if (i % 3 == 0 && i / 3 < 18 && more)
                issue_load(i / 3, ch + 1, nbuf);
            const int k = i - 32, ks = k / 6, u = k % 6;
            if (u < 2)
                Oacc[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, Vb[ks], Oacc[u], 0, 0, 0);
            else
                S[u - 2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, Vb[ks], S[u - 2], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        /* the next stage has landed (waited before the stores below, which
         * also count against vmcnt) */
        if (more)
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        /* O -> fp32 o[token][hv][dv], transposed through this chunk's (now
         * consumed) stage buffer so every store is 16 bytes of a row */
        lds_barrier();
        __attribute__((address_space(3))) float *ot =
            (__attribute__((address_space(3))) float *)(smem + buf);
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
#pragma unroll
            for (int rr = 0; rr < 16; rr++) {
                const int t = 32 * mt + 8 * (rr >> 2) + 4 * h + (rr & 3);
                ot[t * O_LDS + dv] = Oacc[mt][rr];
            }
        }
        lds_barrier();
#pragma unroll
        for (int p = 0; p < 8; p++) { /* rows 16 wave + 2p + h, 32 lanes x 16 B */
            const int t = 16 * wave + 2 * p + h;
            if (t < L) {
                const floatx4 v = *(__attribute__((address_space(3))) const floatx4 *)(
                    ot + t * O_LDS + 4 * col);
                *(floatx4 *)(o + ((size_t)(t0 + t) * Hv + hv) * DV + 4 * col) = v;
            }
        }
        lds_barrier(); /* the o stores keep streaming */
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
                       Hv, ck->num_chunks, ws->O);
    const int rows = N * Hv;
    hipLaunchKernelGGL(gdn_norm_gate_kernel, dim3((unsigned)CEIL_DIV(rows, 4)), dim3(256), 0,
                       stream, ws->O, (const bf16 *)z, z_stride, norm_w, eps, rows, Hv, (bf16 *)y);
    return hipGetLastError();
}
