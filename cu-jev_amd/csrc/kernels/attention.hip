/* Shared-prefix gated GQA attention for gfx950 (CDNA4), plus its Q/K/V prep.
 *
 * Semantics follow the reference's src/kernels/attention.cu:11-100 (prep) and
 * :138-332 (attention): zero-centred RMSNorm on q and k, RoPE on the first 64
 * dims, q scaled by head_dim^-1/2 * log2 e before its bf16 rounding, base-2
 * online softmax with P rounded to bf16 for the PV product and l accumulated
 * in fp32 from the unrounded p, fully masked rows give 0, output times
 * sigmoid(gate). The math is transformers' Qwen3_5Attention
 * (modeling_qwen3_5.py:656-701).
 *
 * The kernel is designed for CDNA4, not translated:
 *  - One workgroup owns one kv-head and 32*TG consecutive packed tokens; its
 *    4*TG waves are (token group) x (the 4 q-heads of the kv-group). Every
 *    64-key K/V tile staged in LDS therefore serves 128*TG query rows of
 *    possibly several branches: the state keys are identical for all of them.
 *  - The MFMA is v_mfma_f32_32x32x16_bf16 computing S^T = K Q^T (keys on the
 *    M side, queries on N), so each lane holds 16 keys of ONE query: row max
 *    and row sum are in-lane plus one lane^32 exchange.
 *  - K rows are fed to the A operand in a permuted order (bits 2 and 3 of the
 *    row swapped) so that the S^T accumulator of a lane is exactly the 8
 *    consecutive keys the B operand of O^T += V^T P^T needs: P goes from the
 *    accumulator to the next MFMA without any cross-lane movement.
 *  - V is kept d-major in HBM (vt cache [Hkv][256][stride]) so the V^T A
 *    operand is a 16-byte LDS read; the prep kernel writes it that way.
 *  - LDS tiles are XOR-swizzled for conflict-free ds_read_b128; the next tile
 *    is fetched to registers while the current one is multiplied (one barrier
 *    per tile).
 *  - blockIdx -> (kv-head, token tile) is XCD-aware: the 8 XCDs (own L2 each)
 *    are split among the kv-heads so the WGs sharing an L2 stream the same
 *    K/V. Tiles run last-to-first so the longest causal rows start first. */
#include "common.h"
#include "kernels.h"

namespace CUJEV_KNS {
namespace {

constexpr int D = 256;
constexpr int BK = 64;                   /* keys per tile */
constexpr int QW = 32;                   /* query tokens per wave */
constexpr int K_BYTES = BK * D * 2;      /* 32 KiB: K tile [64][256]    */
constexpr int V_BYTES = D * BK * 2;      /* 32 KiB: V^T tile [256][64]  */
constexpr int BUF_BYTES = K_BYTES + V_BYTES;

/* 16-byte chunk swizzles: the 16 lanes of one ds_read_b128 phase hit 16
 * distinct 16-byte bank groups (and any 8 consecutive lanes 8 distinct ones). */
DEV int swz_k(int key) { return ((key & 4) << 1) | ((key & 8) >> 1) | (key & 3); }
DEV int swz_v(int d) { return (d & 7) ^ ((d >> 3) & 1); }
/* MFMA row m of the S^T tile holds key perm_row(m) of its 32-key block. */
DEV int perm_row(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }

struct TileSrc {
    const bf16 *k;  /* K rows of this kv-head */
    const bf16 *vt; /* V^T rows of this kv-head */
    int kbase;      /* first key of the tile (multiple of 64) */
    int stride;     /* cache stride in tokens */
};

template <int NT>
DEV void fetch_tile(const TileSrc &s, u32x4 (&stage)[2 * 2048 / NT]) {
    constexpr int PER = 2048 / NT; /* 16-byte chunks per thread per operand */
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int idx = t + NT * j;
        const int row = idx >> 5, c = idx & 31;
        stage[j] = *(const u32x4 *)(s.k + (size_t)(s.kbase + row) * D + c * 8);
    }
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int idx = t + NT * j;
        const int d = idx >> 3, c = idx & 7;
        stage[PER + j] = *(const u32x4 *)(s.vt + (size_t)d * s.stride + s.kbase + c * 8);
    }
}

template <int NT>
DEV void store_tile(unsigned char *buf, const u32x4 (&stage)[2 * 2048 / NT]) {
    constexpr int PER = 2048 / NT;
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int idx = t + NT * j;
        const int row = idx >> 5, c = idx & 31;
        *(u32x4 *)(buf + row * 512 + ((c ^ swz_k(row)) << 4)) = stage[j];
    }
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int idx = t + NT * j;
        const int d = idx >> 3, c = idx & 7;
        *(u32x4 *)(buf + K_BYTES + d * 128 + ((c ^ swz_v(d)) << 4)) = stage[PER + j];
    }
}

template <int TG>
__global__ __launch_bounds__(256 * TG) void attention_kernel(
    const bf16 *__restrict__ q, const bf16 *__restrict__ gate, int gts, int ghs,
    const bf16 *__restrict__ pk, const bf16 *__restrict__ pvt, int P, int p_stride,
    const bf16 *__restrict__ ok, const bf16 *__restrict__ ovt, int o_stride,
    const int32_t *__restrict__ own_base, int N, int Hq, int Hkv, int ntile, bf16 *__restrict__ out) {
    constexpr int NT = 256 * TG;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * BUF_BYTES];

    /* ---- XCD-aware work mapping ---- */
    int kh, tile;
    {
        const int bid = blockIdx.x;
        if (8 % Hkv == 0) {
            const int G = 8 / Hkv, xcd = bid & 7, slot = bid >> 3;
            kh = xcd / G;
            tile = slot * G + xcd % G;
        } else {
            kh = bid % Hkv;
            tile = bid / Hkv;
        }
        if (tile >= ntile)
            return;
        tile = ntile - 1 - tile;
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int hq = wave & 3, tg = wave >> 2;
    const int head = kh * 4 + hq;
    const int h = lane >> 5, col = lane & 31;
    const int n0 = tile * (QW * TG);
    const int n = n0 + tg * QW + col; /* this lane's query token */
    const bool qvalid = n < N;

    /* ---- Q^T B-operand fragments, resident for the whole kernel ---- */
    bf16x8 qf[16];
    {
        const bf16 *qp = q + ((size_t)(qvalid ? n : 0) * Hq + head) * D + 8 * h;
#pragma unroll
        for (int ks = 0; ks < 16; ks++) {
            u32x4 raw = qvalid ? *(const u32x4 *)(qp + 16 * ks) : u32x4{0, 0, 0, 0};
            qf[ks] = __builtin_bit_cast(bf16x8, raw);
        }
    }
    const int base_n = qvalid ? own_base[n] : 0x7fffffff;

    /* ---- key tiles: state [0,P) then own [own_lo, own_hi] (64-aligned) ---- */
    const int own_lo = own_base[n0];
    const int own_hi = min(n0 + QW * TG, N) - 1;
    const int nst = (P + BK - 1) / BK;
    const int own_t0 = own_lo / BK;
    const int ntl = nst + own_hi / BK - own_t0 + 1;
    const bf16 *pk_h = pk + (size_t)kh * p_stride * D, *pv_h = pvt + (size_t)kh * D * p_stride;
    const bf16 *ok_h = ok + (size_t)kh * o_stride * D, *ov_h = ovt + (size_t)kh * D * o_stride;
    auto src_of = [&](int i) {
        TileSrc s;
        if (i < nst) {
            s.k = pk_h; s.vt = pv_h; s.kbase = i * BK; s.stride = p_stride;
        } else {
            s.k = ok_h; s.vt = ov_h; s.kbase = (own_t0 + i - nst) * BK; s.stride = o_stride;
        }
        return s;
    };

    floatx16 o[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
        o[i] = floatx16{};
    float m_run = -INFINITY, l_run = 0.f;

    u32x4 stage[2 * 2048 / NT];
    fetch_tile<NT>(src_of(0), stage);
    store_tile<NT>(smem, stage);
    __syncthreads();

    const int arow0 = perm_row(col), arow1 = 32 + perm_row(col);
    for (int i = 0; i < ntl; i++) {
        const bool more = i + 1 < ntl;
        if (more)
            fetch_tile<NT>(src_of(i + 1), stage);
        const unsigned char *kt = smem + (i & 1) * BUF_BYTES;
        const unsigned char *vt = kt + K_BYTES;

        /* S^T = K Q^T for 64 keys x this wave's 32 queries */
        floatx16 s0 = floatx16{}, s1 = floatx16{};
#pragma unroll
        for (int ks = 0; ks < 16; ks++) {
            const int c = 2 * ks + h;
            bf16x8 a0 = *(const bf16x8 *)(kt + arow0 * 512 + ((c ^ swz_k(arow0)) << 4));
            bf16x8 a1 = *(const bf16x8 *)(kt + arow1 * 512 + ((c ^ swz_k(arow1)) << 4));
            s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, qf[ks], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, qf[ks], s1, 0, 0, 0);
        }

        /* mask: key of accumulator slot r of block t is 32t + 16(r>>3) + 8h + (r&7) */
        const TileSrc cur = src_of(i);
        const bool own = i >= nst;
        if (own || cur.kbase + BK > P) {
            const int k8 = cur.kbase + 8 * h;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int j0 = k8 + 16 * (r >> 3) + (r & 7), j1 = j0 + 32;
                const bool v0 = own ? (j0 >= base_n && j0 <= n) : (j0 < P);
                const bool v1 = own ? (j1 >= base_n && j1 <= n) : (j1 < P);
                s0[r] = v0 ? s0[r] : -INFINITY;
                s1[r] = v1 ? s1[r] : -INFINITY;
            }
        }

        /* online softmax (base 2); rescale only when some row max moved */
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++)
            mx = fmaxf(mx, fmaxf(s0[r], s1[r]));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run, mx);
        const bool moved = m_new > m_run;
        if (__any(moved)) {
            const float alpha = moved ? fast_exp2(m_run - m_new) : 1.f;
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < 8; dt++)
                o[dt] *= alpha;
        }
        m_run = m_new;
        const float mu = m_run == -INFINITY ? 0.f : m_run;
        bf16x8 pf[4];
        float lsum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const float p0 = fast_exp2(s0[r] - mu), p1 = fast_exp2(s1[r] - mu);
            lsum += p0 + p1;
            pf[(r >> 3)][r & 7] = f2bf(p0);
            pf[2 + (r >> 3)][r & 7] = f2bf(p1);
        }
        l_run += lsum;

        /* O^T += V^T P^T */
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int c = 2 * s + h;
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                const int d = 32 * dt + col;
                bf16x8 a = *(const bf16x8 *)(vt + d * 128 + ((c ^ swz_v(d)) << 4));
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pf[s], o[dt], 0, 0, 0);
            }
        }

        if (more)
            store_tile<NT>(smem + ((i + 1) & 1) * BUF_BYTES, stage);
        __syncthreads();
    }

    /* ---- epilogue: normalise, gate, store ---- */
    if (!qvalid)
        return;
    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    const bf16 *g = gate + (size_t)n * gts + (size_t)head * ghs;
    bf16 *dst = out + ((size_t)n * Hq + head) * D;
#pragma unroll
    for (int dt = 0; dt < 8; dt++) {
#pragma unroll
        for (int gq = 0; gq < 4; gq++) {
            const int d0 = 32 * dt + 8 * gq + 4 * h;
            bf16x4 gv = *(const bf16x4 *)(g + d0);
            bf16x4 r;
#pragma unroll
            for (int e = 0; e < 4; e++)
                r[e] = f2bf(o[dt][4 * gq + e] * inv * sigmoid_f(bf2f(gv[e])));
            *(bf16x4 *)(dst + d0) = r;
        }
    }
}

/* ---- prep: norm + RoPE + scale for q, norm + RoPE for k, V transposed ----
 * Workgroup = 16 consecutive tokens x one kv-group: waves 0-3 the 4 q-heads,
 * wave 4 the k-head, all five waves the V transpose. A wave normalises one
 * 256-wide row per step, lane l holding dims 4l..4l+3; RoPE pairs dim i with
 * i + rot/2, i.e. lane l with lane l ^ (rot/8). cos/sin come from a table
 * rope[pos][rot/2] of (cos, sin) pairs built once on the host. */
constexpr int PREP_TOK = 16;

__global__ __launch_bounds__(320) void attn_prep_kernel(
    const bf16 *__restrict__ proj, int ps, const float *__restrict__ qw, const float *__restrict__ kw,
    const int32_t *__restrict__ pos, int N, int Hq, int Hkv, int rot,
    const float2 *__restrict__ rope, float eps, float q_scale, bf16 *__restrict__ q_out,
    bf16 *__restrict__ kc, bf16 *__restrict__ vtc, int cs) {
    __shared__ bf16 vs[256][PREP_TOK + 8]; /* V^T staging [d][token] */
    const int n0 = blockIdx.x * PREP_TOK, kh = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nt = min(PREP_TOK, N - n0);
    const int half_lanes = rot / 8; /* lanes holding the first rot/2 dims */
    const int hr = rot / 2;

    const float *w = wave < 4 ? qw : kw;
    float wl[4];
#pragma unroll
    for (int e = 0; e < 4; e++)
        wl[e] = w[4 * lane + e];
    const bool rotates = lane < 2 * half_lanes;
    const bool first = lane < half_lanes;
    const int fi0 = first ? 4 * lane : 4 * lane - hr;
    for (int t = 0; t < nt; t++) {
        const int nn = n0 + t;
        const bf16 *src = wave < 4 ? proj + (size_t)nn * ps + (kh * 4 + wave) * 512
                                   : proj + (size_t)nn * ps + Hq * 512 + kh * 256;
        bf16x4 raw = *(const bf16x4 *)(src + 4 * lane);
        float x[4];
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            x[e] = bf2f(raw[e]);
            ss += x[e] * x[e];
        }
        ss = wave_sum(ss);
        const float rinv = rsqrtf(ss * (1.f / 256.f) + eps);
#pragma unroll
        for (int e = 0; e < 4; e++)
            x[e] = x[e] * rinv * wl[e];
        float partner[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
            partner[e] = __shfl_xor(x[e], half_lanes, 64);
        if (rotates) {
            const float2 *cs_row = rope + (size_t)pos[nn] * hr + fi0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float2 c = cs_row[e];
                x[e] = first ? x[e] * c.x - partner[e] * c.y : x[e] * c.x + partner[e] * c.y;
            }
        }
        bf16x4 o;
        if (wave < 4) {
#pragma unroll
            for (int e = 0; e < 4; e++)
                o[e] = f2bf(x[e] * q_scale);
            *(bf16x4 *)(q_out + ((size_t)nn * Hq + kh * 4 + wave) * 256 + 4 * lane) = o;
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                o[e] = f2bf(x[e]);
            *(bf16x4 *)(kc + ((size_t)kh * cs + nn) * 256 + 4 * lane) = o;
        }
    }

    /* V: [16 tokens][256] -> LDS [256][16] -> 256 vt rows of 16 columns */
    for (int idx = threadIdx.x; idx < PREP_TOK * 32; idx += 320) {
        const int t = idx >> 5, c = idx & 31;
        if (t < nt) {
            bf16x8 v = *(const bf16x8 *)(proj + (size_t)(n0 + t) * ps + Hq * 512 + Hkv * 256 +
                                         kh * 256 + 8 * c);
#pragma unroll
            for (int e = 0; e < 8; e++)
                vs[8 * c + e][t] = v[e];
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < 256 * 2; idx += 320) {
        const int d = idx >> 1, c = idx & 1;
        bf16 *dst = vtc + ((size_t)kh * 256 + d) * cs + n0 + 8 * c;
        if (8 * c + 8 <= nt) {
            *(bf16x8 *)dst = *(const bf16x8 *)&vs[d][8 * c];
        } else {
            for (int e = 0; e < 8 && 8 * c + e < nt; e++)
                dst[e] = vs[d][8 * c + e];
        }
    }
}

} // namespace
} // namespace CUJEV_KNS
using namespace CUJEV_KNS;

extern "C" hipError_t k_attn_prep(const bf16_t *proj, int proj_stride, const float *q_norm_w,
                                  const float *k_norm_w, const int32_t *pos, int N, int Hq, int Hkv,
                                  int rot, const float *rope_table, float eps, float q_scale,
                                  bf16_t *q_out, bf16_t *k_cache, bf16_t *vt_cache, int cache_stride,
                                  hipStream_t stream) {
    if (N <= 0)
        return hipSuccess;
    if (Hq != 4 * Hkv || rot > 64 || rot % 8 != 0)
        return hipErrorInvalidValue;
    dim3 grid((unsigned)CEIL_DIV(N, PREP_TOK), (unsigned)Hkv);
    hipLaunchKernelGGL(attn_prep_kernel, grid, dim3(320), 0, stream, (const bf16 *)proj,
                       proj_stride, q_norm_w, k_norm_w, pos, N, Hq, Hkv, rot,
                       (const float2 *)rope_table, eps, q_scale, (bf16 *)q_out, (bf16 *)k_cache,
                       (bf16 *)vt_cache, cache_stride);
    return hipGetLastError();
}

extern "C" hipError_t k_attention(const bf16_t *q, const bf16_t *gate, int gate_tok_stride,
                                  int gate_head_stride, const bf16_t *pk, const bf16_t *pvt, int P,
                                  int p_stride, const bf16_t *ok, const bf16_t *ovt, int o_stride,
                                  const int32_t *own_base, int N, int Hq, int Hkv, bf16_t *out,
                                  hipStream_t stream) {
    if (N <= 0)
        return hipSuccess;
    if (Hq != 4 * Hkv || P < 0 || p_stride % 64 != 0 || o_stride % 64 != 0)
        return hipErrorInvalidValue;
    constexpr int TG = 1;
    const int ntile = CEIL_DIV(N, QW * TG);
    int nblk;
    if (8 % Hkv == 0) {
        const int G = 8 / Hkv;
        nblk = CEIL_DIV(ntile, G) * G * Hkv;
    } else {
        nblk = ntile * Hkv;
    }
    hipLaunchKernelGGL(attention_kernel<TG>, dim3((unsigned)nblk), dim3(256 * TG), 0, stream,
                       (const bf16 *)q, (const bf16 *)gate, gate_tok_stride, gate_head_stride,
                       (const bf16 *)pk, (const bf16 *)pvt, P, p_stride, (const bf16 *)ok,
                       (const bf16 *)ovt, o_stride, own_base, N, Hq, Hkv, ntile, (bf16 *)out);
    return hipGetLastError();
}
