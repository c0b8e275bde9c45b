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
 *  - One workgroup owns one kv-head and 32 consecutive packed tokens; its 4
 *    waves are the 4 q-heads of the kv-group. Every 64-key K/V tile staged in
 *    LDS therefore serves 128 query rows of possibly several branches: the
 *    state keys are identical for all of them.
 *  - The MFMA is v_mfma_f32_32x32x16_bf16 computing S^T = K Q^T (keys on the
 *    M side, queries on N), so each lane holds 16 keys of ONE query: row max
 *    and row sum are in-lane plus one v_permlane32_swap.
 *  - K rows are fed to the A operand in a permuted order (bits 2 and 3 of the
 *    row swapped) so that the S^T accumulator of a lane is exactly the 8
 *    consecutive keys the B operand of O^T += V^T P^T needs: P goes from the
 *    accumulator to the next MFMA without any cross-lane movement.
 *  - V is kept d-major in HBM (vt cache [Hkv][256][stride]) so the V^T A
 *    operand is a 16-byte LDS read; the prep kernel writes it that way.
 *  - Tiles move HBM -> LDS with buffer_load ... lds (no staging registers),
 *    XOR-swizzled for conflict-free ds_read_b128. K and V^T have separate
 *    double buffers: while a wave runs the softmax of tile i interleaved with
 *    the S^T MFMAs of tile i+1 and then the PV MFMAs of tile i, the V^T of
 *    tile i+1 and the K of tile i+2 are in flight. One barrier per tile;
 *    the last two PV MFMAs of a tile run after it, while the next tile's
 *    first K reads come back (their operands are read before it).
 *  - The softmax shift mu stays 0 while the running max is within 2^+-64
 *    of it, so S accumulators start at the MFMA's inline zero and scores need
 *    no per-tile shift; only rows whose scores leave that range pay for a
 *    subtraction (and, when mu moves, the O/l rescale).
 *  - blockIdx -> (kv-head, token tile) is XCD-aware: the 8 XCDs (own L2 each)
 *    are split among the kv-heads so the WGs sharing an L2 stream the same
 *    K/V. Tiles run last-to-first so the longest causal rows start first. */
#include "common.h"
#include "kernels.h"

#include <type_traits>

namespace CUJEV_KNS {
namespace {

constexpr int D = 256;
constexpr int BK = 64;              /* keys per tile */
constexpr int QW = 32;              /* query tokens per wave */
constexpr int K_BYTES = BK * D * 2; /* 32 KiB: K tile [64][256]    */
constexpr int V_BYTES = D * BK * 2; /* 32 KiB: V^T tile [256][64]  */
/* LDS: V^T buffers first, K buffers after, so every ds_read offset of a
 * buffer fits the 16-bit immediate from one per-lane base register. */
constexpr int V_OFF = 0, K_OFF = 2 * V_BYTES, LDS_BYTES = 2 * V_BYTES + 2 * K_BYTES;
/* Shift of the base-2 softmax: mu cancels in o / l, so any reference mu
 * gives the same softmax and only has to keep p = 2^(s - mu) in range. It
 * stays 0 while the running max m is within +-SHIFT_RANGE of it (p <= 2^64,
 * the largest p >= 2^-64) and moves to m when m leaves that window,
 * rescaling o and l. The bf16 rounding of p then happens at other points
 * than the reference's (which rounds 2^(s - m) against the running max): the
 * two roundings agree only where m - mu is a whole number, and otherwise
 * differ by up to one bf16 ulp of p, an equally valid rounding. */
constexpr float SHIFT_RANGE = 64.f;

/* 16-byte chunk swizzles: the 16 lanes of one ds_read_b128 phase hit 16
 * distinct 16-byte bank groups (and any 8 consecutive lanes 8 distinct ones). */
DEV int swz_k(int key) { return ((key & 4) << 1) | ((key & 8) >> 1) | (key & 3); }
DEV int swz_v(int d) { return (d & 7) ^ ((d >> 3) & 1); }
/* MFMA row m of the S^T tile holds key perm_row(m) of its 32-key block. */
DEV int perm_row(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }

typedef __attribute__((address_space(3))) void *lds_ptr;
typedef __attribute__((address_space(3))) const unsigned char lds_u8;
/* 16-byte LDS read at a byte offset from the start of the tile buffers */
DEV bf16x8 lds_read16(lds_u8 *base, uint32_t off) {
    return *(__attribute__((address_space(3))) const bf16x8 *)(base + off);
}

/* Tiles go HBM -> LDS directly (buffer_load_dwordx4 ... lds): lane l of a
 * wave writes the 16 bytes it fetched at LDS base + 16 l, so the swizzle is
 * applied on the global side: the lane landing on chunk slot p of LDS row r
 * fetches chunk p ^ swz(r). Per tile and operand each of the 4 waves issues 8
 * such loads: K load j of wave w covers rows 8j + 2w + {0,1}; V^T load j covers
 * d rows 8(4j + w) .. +7. No registers hold the tile in flight, and the buffer
 * form only counts against vmcnt, so LDS reads keep their own fine-grained
 * waits. Each operand of a kv-head has its own buffer resource whose size is
 * the cache slice, so the hardware range check covers every load. */
struct TileSrc {
    __amdgpu_buffer_rsrc_t k;  /* K rows [stride][256] of this kv-head */
    __amdgpu_buffer_rsrc_t vt; /* V^T rows [256][stride] of this kv-head */
    int kbase;                 /* first key of the tile (multiple of 64) */
    uint32_t voff;             /* this lane's byte offset inside a V^T load */
    int vrow_bytes;            /* V^T row pitch in bytes */
};

DEV __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}

DEV void issue_k1(const TileSrc &s, unsigned char *kbuf, const uint32_t (&koff)[2], int wave, int j) {
    const int r0 = 8 * j + 2 * wave;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(s.k, (lds_ptr)(kbuf + r0 * 512), 16, koff[j & 1],
                                             (s.kbase + r0) * 512, 0, 0);
}

DEV void issue_v1(const TileSrc &s, unsigned char *vbuf, int wave, int j) {
    const int d0 = 8 * (4 * j + wave);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(s.vt, (lds_ptr)(vbuf + d0 * 128), 16, s.voff,
                                             d0 * s.vrow_bytes + s.kbase * 2, 0, 0);
}

DEV void issue_k(const TileSrc &s, unsigned char *kbuf, const uint32_t (&koff)[2], int wave) {
#pragma unroll
    for (int j = 0; j < 8; j++)
        issue_k1(s, kbuf, koff, wave, j);
}

DEV void issue_v(const TileSrc &s, unsigned char *vbuf, int wave) {
#pragma unroll
    for (int j = 0; j < 8; j++)
        issue_v1(s, vbuf, wave, j);
}

DEV void wait_tile_loads() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

/* s_waitcnt on the LDS count alone (gfx9 encoding: lgkmcnt in bits 11:8,
 * vmcnt and expcnt at their maxima): one wait covers the operands of two
 * MFMAs, so the compiler adds none of its own before the second. */
#define WAIT_LGKM_(n) __builtin_amdgcn_s_waitcnt(0xC07F | ((n) << 8))
DEV void wait_lgkm(int n) { /* n is a constant once the loops are unrolled */
    switch (n) {
    case 0: WAIT_LGKM_(0); break;
    case 1: WAIT_LGKM_(1); break;
    case 2: WAIT_LGKM_(2); break;
    case 3: WAIT_LGKM_(3); break;
    case 4: WAIT_LGKM_(4); break;
    case 5: WAIT_LGKM_(5); break;
    case 6: WAIT_LGKM_(6); break;
    default: WAIT_LGKM_(0); break;
    }
}

/* One workgroup = 4 waves = the 4 q-heads of kv-head kh x 32 packed tokens.
 * Per key tile i the loop overlaps, in each wave, the S^T MFMAs of tile i+1
 * with the softmax of tile i, then runs the PV MFMAs of tile i, while the
 * V^T of tile i+1 and the K of tile i+2 stream into the idle buffers. */
/* Key-split partials (SPLIT): split s of a (token, q-head) row keeps the
 * unnormalised o[256], l and the shift mu of its share of the key tiles. */
struct AttnPart {
    float *o;  /* [nsplit][N][Hq][256] */
    float *l;  /* [nsplit][N][Hq]      */
    float *mu; /* [nsplit][N][Hq]      */
    int nsplit;
};

/* The second problem of a paired launch: N packed tokens starting row0
 * rows after the first problem's, over the shared state cache's first P
 * keys and their own keys in (ok, ovt) (see k_attention). */
struct AttnJob {
    const bf16 *ok, *ovt;
    int row0, P, o_stride, N;
};

/* PAIR (attention_pair): workgroups [0, nblk_a) serve the problem of the
 * leading arguments, the rest a second one over the same state cache, given
 * by jb (its rows start jb.row0 rows further into q, gate, own_base and
 * out; nblk_a is a multiple of 8 where Hkv divides 8, so both keep the XCD
 * mapping). Without PAIR, jb and nblk_a are unused. */
template <bool SPLIT, bool PAIR>
__global__ __launch_bounds__(256) void attention_kernel(
    const bf16 *__restrict__ q, const bf16 *__restrict__ gate, int gts, int ghs,
    const bf16 *__restrict__ pk, const bf16 *__restrict__ pvt, int P, int p_stride,
    const bf16 *__restrict__ ok, const bf16 *__restrict__ ovt, int o_stride,
    const int32_t *__restrict__ own_base, int N, int Hq, int Hkv, int ntile, bf16 *__restrict__ out,
    AttnPart part, AttnJob jb, int nblk_a) {
    __shared__ __attribute__((aligned(1024))) unsigned char smem[LDS_BYTES];
    int bid = blockIdx.x;
    if (PAIR && bid >= nblk_a) {
        bid -= nblk_a;
        q += (size_t)jb.row0 * Hq * D, gate += (size_t)jb.row0 * gts;
        own_base += jb.row0, out += (size_t)jb.row0 * Hq * D;
        P = jb.P, ok = jb.ok, ovt = jb.ovt, o_stride = jb.o_stride, N = jb.N;
        ntile = (N + QW - 1) / QW;
    }

    /* ---- XCD-aware work mapping ---- */
    int kh, tile;
    {
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
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int head = kh * 4 + wave;
    const int h = lane >> 5, col = lane & 31;
    const int n0 = tile * QW;
    const int n = n0 + col; /* this lane's query token */
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
    const int own_hi = min(n0 + QW, N) - 1;
    const int nst = (P + BK - 1) / BK;
    const int own_t0 = own_lo / BK;
    const int ntl_all = nst + own_hi / BK - own_t0 + 1;
    /* SPLIT: this workgroup's contiguous share [tb, tb + ntl) of the tiles */
    const int split = SPLIT ? (int)blockIdx.y : 0;
    const int tb = SPLIT ? split * ntl_all / part.nsplit : 0;
    const int ntl = SPLIT ? (split + 1) * ntl_all / part.nsplit - tb : ntl_all;
    if (SPLIT && ntl <= 0) { /* no tiles: an empty partial */
        if (qvalid && h == 0) {
            const size_t r = ((size_t)split * N + n) * Hq + head;
            part.l[r] = 0.f;
            part.mu[r] = 0.f;
        }
        return;
    }

    uint32_t koff[2];
#pragma unroll
    for (int par = 0; par < 2; par++) {
        const int hi = lane >> 5, row = 8 * par + 2 * wave + hi;
        koff[par] = hi * 512 + (((lane & 31) ^ swz_k(row)) << 4);
    }
    const int vl = lane >> 3, vc = ((lane & 7) ^ ((lane >> 3) ^ (wave & 1))) << 4;
    TileSrc st, ow;
    const uint32_t p_bytes = (uint32_t)p_stride * D * 2, o_bytes = (uint32_t)o_stride * D * 2;
    st.k = make_rsrc(pk + (size_t)kh * p_stride * D, p_bytes);
    st.vt = make_rsrc(pvt + (size_t)kh * D * p_stride, p_bytes);
    st.vrow_bytes = p_stride * 2;
    st.voff = vl * st.vrow_bytes + vc;
    ow.k = make_rsrc(ok + (size_t)kh * o_stride * D, o_bytes);
    ow.vt = make_rsrc(ovt + (size_t)kh * D * o_stride, o_bytes);
    ow.vrow_bytes = o_stride * 2;
    ow.voff = vl * ow.vrow_bytes + vc;
    auto src_of = [&](int i) {
        i += tb;
        TileSrc s = i < nst ? st : ow;
        s.kbase = i < nst ? i * BK : (own_t0 + i - nst) * BK;
        return s;
    };

    /* per-lane LDS read addresses; the rest of each address is an immediate */
    const int arow = perm_row(col); /* key rows arow and 32 + arow */
    lds_u8 *lds = (lds_u8 *)smem;
    const int xk = h ^ swz_k(arow);
    uint32_t ka[8];
#pragma unroll
    for (int c8 = 0; c8 < 8; c8++)
        ka[c8] = K_OFF + arow * 512 + (((2 * c8) ^ xk) << 4);
    const int xv = h ^ swz_v(col);
    uint32_t va[4];
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++)
        va[s4] = V_OFF + col * 128 + (((2 * s4) ^ xv) << 4);

    floatx16 o[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
        o[i] = floatx16{};
    /* m_run: running max of the scores (log2 units); mu_run: the shift */
    float m_run = -INFINITY, l_run = 0.f, mu_run = 0.f;

    constexpr int QD = 3; /* S^T A-operand reads in flight, in k-steps */
    constexpr int VD = 4; /* V^T A-operand reads in flight, in MFMAs   */
#ifndef ATT_HB
#define ATT_HB 2
#endif
    constexpr int HB = ATT_HB; /* PV MFMAs held back past the barrier */
    static_assert(HB <= VD && HB <= 8, "held-back operands are read before the barrier, in P block 3");
    bf16x8 vd[HB], pd = {};
#pragma unroll
    for (int t = 0; t < HB; t++)
        vd[t] = bf16x8{};
    auto kaddr = [&](int ks, int buf) { return ka[ks & 7] + (ks >> 3) * 256 + buf * K_BYTES; };
    auto vaddr = [&](int t, int buf) { return va[t >> 3] + (t & 7) * 4096 + buf * V_BYTES; };

    /* prologue: K0, V0, K1 in flight; S^T of tile 0 */
    issue_k(src_of(0), smem + K_OFF, koff, wave);
    issue_v(src_of(0), smem + V_OFF, wave);
    if (ntl > 1)
        issue_k(src_of(1), smem + K_OFF + K_BYTES, koff, wave);
    wait_tile_loads();
    __syncthreads();
    floatx16 sa0 = floatx16{}, sa1 = floatx16{}, sb0, sb1;
#pragma unroll
    for (int ks = 0; ks < 16; ks++) {
        sa0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lds_read16(lds, kaddr(ks, 0)), qf[ks], sa0, 0, 0, 0);
        sa1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lds_read16(lds, kaddr(ks, 0) + 16384), qf[ks],
                                                      sa1, 0, 0, 0);
    }
    __syncthreads(); /* K buffer 0 is refilled in the first step */

    /* One key tile i with unshifted scores S = (s0, s1). With a next tile,
     * its S^T MFMAs run in the same straight-line block as this tile's
     * softmax: per k-step two MFMAs, the LDS reads QD k-steps ahead and a
     * slice of the softmax VALU work, pinned in that order by scheduling
     * barriers. The PV MFMAs of tile i follow with their reads VD ahead. */
    auto step = [&](auto has_next, int i, floatx16 &s0, floatx16 &s1, floatx16 &n0_, floatx16 &n1_,
                    int kbuf_next, int vbuf) {
        constexpr bool NEXT = decltype(has_next)::value;
        /* This step's tile loads go out one per k-step of the S^T loop below,
         * between its MFMAs: K of tile i+2 (source clamped to the last tile;
         * past the end the load refills a buffer that is not read again) and
         * V^T of tile i+1. Both target buffers were last read before the
         * barrier that ended the previous step. An LDS read issued after a
         * buffer_load ... lds of the same wave completes only once that load
         * has landed; in this loop the operand reads run QD k-steps ahead of
         * their MFMAs, which hides most of that (the PV reads, VD MFMAs
         * ahead, would not). */
        const TileSrc sk = src_of(min(i + 2, ntl - 1));
        const TileSrc sv = src_of(min(i + 1, ntl - 1));
        unsigned char *const kdst = smem + K_OFF + (kbuf_next ^ 1) * K_BYTES;
        unsigned char *const vdst = smem + V_OFF + (vbuf ^ 1) * V_BYTES;

        /* mask: key of accumulator slot r of block t is 32t + 16(r>>3) + 8h + (r&7) */
        const int gi = i + tb; /* index in the full tile list */
        const bool own = gi >= nst;
        const int kbase = own ? (own_t0 + gi - nst) * BK : gi * BK;
        if (own || kbase + BK > P) {
            const int lo = own ? base_n : 0, hi = own ? n : P - 1;
            const int k8 = kbase + 8 * h;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int j0 = k8 + 16 * (r >> 3) + (r & 7), j1 = j0 + 32;
                s0[r] = (j0 >= lo && j0 <= hi) ? s0[r] : -INFINITY;
                s1[r] = (j1 >= lo && j1 <= hi) ? s1[r] : -INFINITY;
            }
        }

        bf16x8 r0[QD], r1[QD];
        if constexpr (NEXT) {
#pragma unroll
            for (int ks = 0; ks < QD; ks++) {
                r0[ks] = lds_read16(lds, kaddr(ks, kbuf_next));
                r1[ks] = lds_read16(lds, kaddr(ks, kbuf_next) + 16384);
            }
        }
        /* The previous tile's last HB PV MFMAs, held back past the barrier
         * (their V^T operands were read before it) so the matrix core works
         * while the reads above come back. Zero operands before the first
         * tile. */
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < HB; t++)
            o[(32 - HB + t) & 7] =
                __builtin_amdgcn_mfma_f32_32x32x16_bf16(vd[t], pd, o[(32 - HB + t) & 7], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        /* Softmax of tile i with the exponentials taken for the shift 0 (the
         * common case): score pairs 0-7 (P blocks 0 and 1) between the S^T
         * MFMAs of tile i+1, pairs 8-15 (blocks 2 and 3) between the PV MFMAs
         * of tile i ahead of their use, and the max of the raw scores along
         * the S^T loop. Whether the scores need a shift is decided after that
         * loop, when the max is long complete; only then (rarely) are they
         * shifted in place and pairs 0-7 redone; pairs 8-15 read the shifted
         * scores anyway. */
        float mx = -INFINITY, lsum = 0.f;
        bf16x8 pf[4];
        /* The empty asm keeps each pair in its slot: the compiler would
         * otherwise sink the exponentials towards their first use. */
        auto pair = [&](int q2) {
            const int v = 2 * q2;
            const float x0 = v < 16 ? s0[v] : s1[v - 16];
            const float x1 = v < 16 ? s0[v + 1] : s1[v - 15];
            const float p0 = fast_exp2(x0), p1 = fast_exp2(x1);
            lsum += p0 + p1;
            bf16x2 pk = {f2bf(p0), f2bf(p1)};
            asm volatile("" : "+v"(pk), "+v"(lsum));
            const int blk = (v < 16 ? 0 : 2) + ((v & 15) >> 3), e = v & 7;
            pf[blk][e] = pk[0];
            pf[blk][e + 1] = pk[1];
        };
#pragma unroll
        for (int ks = 0; ks < 16; ks++) {
            if constexpr (NEXT) {
                const bf16x8 a0 = r0[ks % QD], a1 = r1[ks % QD];
                if (ks + QD < 16) {
                    r0[ks % QD] = lds_read16(lds, kaddr(ks + QD, kbuf_next));
                    r1[ks % QD] = lds_read16(lds, kaddr(ks + QD, kbuf_next) + 16384);
                }
                wait_lgkm(2 * ((ks + QD < 16 ? ks + QD : 15) - ks));
                n0_ = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, qf[ks], ks == 0 ? floatx16{} : n0_, 0, 0, 0);
                n1_ = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, qf[ks], ks == 0 ? floatx16{} : n1_, 0, 0, 0);
                if (ks < 8)
                    issue_k1(sk, kdst, koff, wave, ks);
                else
                    issue_v1(sv, vdst, wave, ks - 8);
            }
            mx = fmaxf(mx, fmaxf(s0[ks], s1[ks]));
            if ((ks & 1) == 0)
                pair(ks >> 1);
            __builtin_amdgcn_sched_barrier(0);
        }
        {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx),
                                                             false, false);
            mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
            const float m_new = fmaxf(m_run, mx);
            const bool move = m_new != -INFINITY && fabsf(m_new - mu_run) > SHIFT_RANGE;
            const float mu_new = move ? m_new : mu_run;
            if (__builtin_expect(__any(move || mu_new != 0.f), 0)) {
                /* rare: scores out of range of 2^0 */
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    s0[r] -= mu_new;
                    s1[r] -= mu_new;
                }
                lsum = 0.f;
#pragma unroll
                for (int q2 = 0; q2 < 8; q2++)
                    pair(q2);
                /* a move down only happens before any key counted (l = o = 0) */
                const float alpha = fast_exp2(fminf(mu_run - mu_new, 0.f));
                if (__any(move)) {
                    l_run *= alpha;
#pragma unroll
                    for (int dt = 0; dt < 8; dt++)
                        o[dt] *= alpha;
                }
            }
            m_run = m_new;
            mu_run = mu_new;
        }

        /* O^T += V^T P^T; with a next tile the last HB MFMAs wait for the
         * next step (their operands in vd, pd) */
        constexpr int TPV = NEXT ? 32 - HB : 32;
        bf16x8 vr[VD];
#pragma unroll
        for (int t = 0; t < VD; t++)
            vr[t] = lds_read16(lds, vaddr(t, vbuf));
#pragma unroll
        for (int t = 0; t < TPV; t++) {
            const bf16x8 a = vr[t % VD];
            if (t + VD < 32)
                vr[t % VD] = lds_read16(lds, vaddr(t + VD, vbuf));
            if ((t & 1) == 0)
                wait_lgkm((t + VD < 32 ? t + VD : 31) - t - 1);
            o[t & 7] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pf[t >> 3], o[t & 7], 0, 0, 0);
            if (t < 16 && (t & 1) == 0)
                pair(8 + (t >> 1));
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (NEXT) {
#pragma unroll
            for (int t = 0; t < HB; t++)
                vd[t] = vr[(32 - HB + t) % VD]; /* the reads of MFMAs 32 - HB .. 31 */
            pd = pf[3];
        }
        l_run += lsum;
        wait_tile_loads();
        __syncthreads();
    };

    /* unrolled by two so buffer indices are compile-time; the last tile has
     * no successor */
    const std::true_type more{};
    const std::false_type last{};
    int i = 0;
    for (; i + 2 < ntl; i += 2) {
        step(more, i, sa0, sa1, sb0, sb1, 1, 0);
        step(more, i + 1, sb0, sb1, sa0, sa1, 0, 1);
    }
    if (ntl - i == 2) {
        step(more, i, sa0, sa1, sb0, sb1, 1, 0);
        step(last, i + 1, sb0, sb1, sa0, sa1, 0, 1);
    } else {
        step(last, i, sa0, sa1, sb0, sb1, 1, 0);
    }

    /* ---- epilogue: normalise, gate, store ---- */
    if (!qvalid)
        return;
    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    if constexpr (SPLIT) { /* the unnormalised partial; the merge gates it */
        const size_t r = ((size_t)split * N + n) * Hq + head;
        float *po = part.o + r * D;
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
            for (int gq = 0; gq < 4; gq++)
                *(float4 *)(po + 32 * dt + 8 * gq + 4 * h) =
                    make_float4(o[dt][4 * gq], o[dt][4 * gq + 1], o[dt][4 * gq + 2],
                                o[dt][4 * gq + 3]);
        if (h == 0) {
            part.l[r] = l_tot;
            part.mu[r] = mu_run;
        }
        return;
    }
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

/* Merge of the key-split partials: per (token, q-head) row, with mu the
 * largest shift among the splits that saw keys, o = sum_s 2^(mu_s - mu) o_s
 * and l likewise (the same p = 2^(s - mu) for every split, up to fp32 sum
 * order); out = o / l * sigmoid(gate). One wave per row, 4 dims a lane. */
__global__ __launch_bounds__(256) void attention_merge_kernel(AttnPart part,
                                                              const bf16 *__restrict__ gate,
                                                              int gts, int ghs, int N, int Hq,
                                                              bf16 *__restrict__ out) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= N * Hq)
        return;
    const int n = row / Hq, head = row % Hq;
    const size_t rs = (size_t)N * Hq;
    /* every split's l, mu and o slice in flight before any arithmetic */
    float ls[CUJEV_ATTN_MAX_SPLITS], ms[CUJEV_ATTN_MAX_SPLITS];
    float4 os[CUJEV_ATTN_MAX_SPLITS];
#pragma unroll
    for (int sp = 0; sp < CUJEV_ATTN_MAX_SPLITS; sp++) {
        ls[sp] = 0.f, ms[sp] = 0.f, os[sp] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (sp < part.nsplit) { /* uniform */
            ls[sp] = part.l[sp * rs + row];
            ms[sp] = part.mu[sp * rs + row];
            os[sp] = *(const float4 *)(part.o + (sp * rs + row) * D + 4 * lane);
        }
    }
    float mu = -INFINITY;
#pragma unroll
    for (int sp = 0; sp < CUJEV_ATTN_MAX_SPLITS; sp++)
        if (sp < part.nsplit && ls[sp] > 0.f)
            mu = fmaxf(mu, ms[sp]);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    float l = 0.f;
#pragma unroll
    for (int sp = 0; sp < CUJEV_ATTN_MAX_SPLITS; sp++) {
        /* a split without visible keys adds nothing (its o was not written) */
        if (!(sp < part.nsplit && ls[sp] > 0.f))
            continue;
        const float w = fast_exp2(ms[sp] - mu);
        const float4 v = os[sp];
        acc.x = fmaf(w, v.x, acc.x), acc.y = fmaf(w, v.y, acc.y);
        acc.z = fmaf(w, v.z, acc.z), acc.w = fmaf(w, v.w, acc.w);
        l = fmaf(w, ls[sp], l);
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const bf16x4 gv = *(const bf16x4 *)(gate + (size_t)n * gts + (size_t)head * ghs + 4 * lane);
    const float a[4] = {acc.x, acc.y, acc.z, acc.w};
    bf16x4 r;
#pragma unroll
    for (int e = 0; e < 4; e++)
        r[e] = f2bf(a[e] * inv * sigmoid_f(bf2f(gv[e])));
    *(bf16x4 *)(out + (size_t)row * D + 4 * lane) = r;
}

/* ---- prep: norm + RoPE + scale for q, norm + RoPE for k, V transposed ----
 * Workgroup = 16 consecutive tokens x one kv-group: waves 0-3 the 4 q-heads,
 * wave 4 the k-head, all five waves the V transpose. A wave normalises one
 * 256-wide row per step, lane l holding dims 4l..4l+3; RoPE pairs dim i with
 * i + rot/2, i.e. lane l with lane l ^ (rot/8). cos/sin come from a table
 * rope[pos][rot/2] of (cos, sin) pairs built once on the host. */
/* Tokens per prep workgroup: each wave walks its tokens one after another
 * (a 256-wide reduction and a RoPE exchange per token), so the per-token chain,
 * not the data, sets the time; 4 tokens keep it short and the grid wide. */
constexpr int PREP_TOK = 4;

/* Tokens [0, Na) write K / V^T to (kc, vtc, cs) columns n, the rest (from
 * workgroup nblk_a on) to (kc2, vtc2, cs2) columns n - Na; a one-cache
 * launch passes Na = N and nblk_a = gridDim.x. */
__global__ __launch_bounds__(320) void attn_prep_kernel(
    const bf16 *__restrict__ proj, int ps, const float *__restrict__ qw, const float *__restrict__ kw,
    const int32_t *__restrict__ pos, int N, int Hq, int Hkv, int rot,
    const float2 *__restrict__ rope, float eps, float q_scale, bf16 *__restrict__ q_out,
    bf16 *__restrict__ kc, bf16 *__restrict__ vtc, int cs, int Na, int nblk_a,
    bf16 *__restrict__ kc2, bf16 *__restrict__ vtc2, int cs2) {
    __shared__ bf16 vs[256][PREP_TOK + 8]; /* V^T staging [d][token] */
    int blk = blockIdx.x, nend = Na, col0 = 0;
    if (blk >= nblk_a) {
        blk -= nblk_a, nend = N, col0 = Na;
        kc = kc2, vtc = vtc2, cs = cs2;
    }
    const int n0 = col0 + blk * PREP_TOK, kh = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nt = min(PREP_TOK, nend - n0);
    const int half_lanes = rot / 8; /* lanes holding the first rot/2 dims */
    const int hr = rot / 2;

    const float *w = wave < 4 ? qw : kw;
    float wl[4];
#pragma unroll
    for (int e = 0; e < 4; e++)
        wl[e] = w[4 * lane + e];
    const bool rotates = lane < 2 * half_lanes;
    const bool first = lane < half_lanes;
    const int fi0 = rotates ? (first ? 4 * lane : 4 * lane - hr) : 0;
    /* Every load is issued before any math, unconditionally (token indices
     * clamped into the block; a load skipped on some path would make each
     * later use wait for all loads in flight): the 16 rows, the positions
     * (lane t holds token t's), each token's 4 (cos, sin) pairs, and the V
     * rows of the transpose. */
    const bf16 *src0 = wave < 4 ? proj + (kh * 4 + wave) * 512 : proj + Hq * 512 + kh * 256;
    bf16x4 raw[PREP_TOK];
#pragma unroll
    for (int t = 0; t < PREP_TOK; t++)
        raw[t] = *(const bf16x4 *)(src0 + (size_t)(n0 + min(t, nt - 1)) * ps + 4 * lane);
    const int pos_lane = pos[n0 + min(lane, nt - 1)];
    float4 rc[PREP_TOK][2]; /* (cos, sin) of dims fi0 .. fi0 + 3 */
#pragma unroll
    for (int t = 0; t < PREP_TOK; t++) {
        const int p = __builtin_amdgcn_readlane(pos_lane, t);
        const float4 *row = (const float4 *)(rope + (size_t)p * hr + fi0);
        rc[t][0] = row[0];
        rc[t][1] = row[1];
    }
    bf16x8 vrow[2]; /* V transpose items idx = tid, tid + 320 */
    const bf16 *vsrc = proj + Hq * 512 + Hkv * 256 + kh * 256;
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int idx = min((int)threadIdx.x + 320 * k, PREP_TOK * 32 - 1);
        const int t = min(idx >> 5, nt - 1), c = idx & 31;
        vrow[k] = *(const bf16x8 *)(vsrc + (size_t)(n0 + t) * ps + 8 * c);
    }

#pragma unroll
    for (int t = 0; t < PREP_TOK; t++) {
        if (t >= nt) /* no break: the loop must unroll so raw[t], rc[t] stay in registers */
            continue;
        const int nn = n0 + t;
        float x[4];
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            x[e] = bf2f(raw[t][e]);
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
            const float cz[8] = {rc[t][0].x, rc[t][0].y, rc[t][0].z, rc[t][0].w,
                                 rc[t][1].x, rc[t][1].y, rc[t][1].z, rc[t][1].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float c = cz[2 * e], sn = cz[2 * e + 1];
                x[e] = first ? x[e] * c - partner[e] * sn : x[e] * c + partner[e] * sn;
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
            *(bf16x4 *)(kc + ((size_t)kh * cs + nn - col0) * 256 + 4 * lane) = o;
        }
    }

    /* V: [PREP_TOK tokens][256] -> LDS [256][PREP_TOK] -> 256 vt rows of
     * PREP_TOK columns */
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int idx = threadIdx.x + 320 * k;
        if (idx < PREP_TOK * 32) {
            const int t = idx >> 5, c = idx & 31;
#pragma unroll
            for (int e = 0; e < 8; e++)
                vs[8 * c + e][t] = vrow[k][e];
        }
    }
    __syncthreads();
    constexpr int VP = PREP_TOK < 8 ? PREP_TOK : 8; /* tokens per vt store */
    constexpr int NPC = PREP_TOK / VP;
    typedef __bf16 bf16xVP __attribute__((ext_vector_type(VP)));
    for (int idx = threadIdx.x; idx < 256 * NPC; idx += 320) {
        const int d = idx / NPC, c = idx % NPC;
        bf16 *dst = vtc + ((size_t)kh * 256 + d) * cs + (n0 - col0) + VP * c;
        if (VP * c + VP <= nt) {
            *(bf16xVP *)dst = *(const bf16xVP *)&vs[d][VP * c];
        } else {
            for (int e = 0; e < VP && VP * c + e < nt; e++)
                dst[e] = vs[d][VP * c + e];
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
    const int nblk = CEIL_DIV(N, PREP_TOK);
    hipLaunchKernelGGL(attn_prep_kernel, dim3((unsigned)nblk, (unsigned)Hkv), dim3(320), 0, stream,
                       (const bf16 *)proj, proj_stride, q_norm_w, k_norm_w, pos, N, Hq, Hkv, rot,
                       (const float2 *)rope_table, eps, q_scale, (bf16 *)q_out, (bf16 *)k_cache,
                       (bf16 *)vt_cache, cache_stride, N, nblk, (bf16 *)k_cache,
                       (bf16 *)vt_cache, cache_stride);
    return hipGetLastError();
}

extern "C" hipError_t k_attn_prep_pair(const bf16_t *proj, int proj_stride,
                                       const float *q_norm_w, const float *k_norm_w,
                                       const int32_t *pos, int Na, int Nb, int Hq, int Hkv,
                                       int rot, const float *rope_table, float eps, float q_scale,
                                       bf16_t *q_out, bf16_t *k_cache, bf16_t *vt_cache,
                                       int cache_stride, bf16_t *k_cache2, bf16_t *vt_cache2,
                                       int cache_stride2, hipStream_t stream) {
    if (Na < 0 || Nb < 0)
        return hipErrorInvalidValue;
    if (Na + Nb <= 0)
        return hipSuccess;
    if (Hq != 4 * Hkv || rot > 64 || rot % 8 != 0)
        return hipErrorInvalidValue;
    const int na = CEIL_DIV(Na, PREP_TOK), nb = CEIL_DIV(Nb, PREP_TOK);
    hipLaunchKernelGGL(attn_prep_kernel, dim3((unsigned)(na + nb), (unsigned)Hkv), dim3(320), 0,
                       stream, (const bf16 *)proj, proj_stride, q_norm_w, k_norm_w, pos, Na + Nb,
                       Hq, Hkv, rot, (const float2 *)rope_table, eps, q_scale, (bf16 *)q_out,
                       (bf16 *)k_cache, (bf16 *)vt_cache, cache_stride, Na, na, (bf16 *)k_cache2,
                       (bf16 *)vt_cache2, cache_stride2);
    return hipGetLastError();
}

extern "C" int cujev_attention_splits(int N, int Hkv, int P) {
    const int wgs = CEIL_DIV(N, QW) * Hkv;
    /* at most as many shares as a token tile has key tiles (state + own) */
    const int ntl_max = CEIL_DIV(P, BK) + CEIL_DIV(N, BK) + 1;
    if (N <= 0 || P < 0 || N > CUJEV_ATTN_SPLIT_MAX_N || wgs >= 128)
        return 1;
    int s = 256 / wgs;
    s = s > ntl_max ? ntl_max : s;
    s = s > CUJEV_ATTN_MAX_SPLITS ? CUJEV_ATTN_MAX_SPLITS : s;
    return s < 1 ? 1 : s;
}

extern "C" size_t cujev_attention_ws_bytes(int N, int Hq, int nsplit) {
    return nsplit > 1 ? (size_t)nsplit * N * Hq * (D + 2) * sizeof(float) : 0;
}

extern "C" size_t cujev_attention_ws_max(int max_tokens, int Hq, int Hkv) {
    size_t best = 0;
    const int nmax = max_tokens < CUJEV_ATTN_SPLIT_MAX_N ? max_tokens : CUJEV_ATTN_SPLIT_MAX_N;
    for (int n = 1; n <= nmax; n++) { /* P large: the most shares */
        const size_t b = cujev_attention_ws_bytes(n, Hq, cujev_attention_splits(n, Hkv, 1 << 20));
        best = b > best ? b : best;
    }
    return best;
}

/* Workgroups of one job: ntile token tiles x Hkv kv-heads, rounded up so
 * that every XCD group of the mapping is whole (a multiple of 8 when Hkv
 * divides 8). */
static int attention_blocks(int ntile, int Hkv) {
    if (8 % Hkv == 0) {
        const int G = 8 / Hkv;
        return CEIL_DIV(ntile, G) * G * Hkv;
    }
    return ntile * Hkv;
}

extern "C" hipError_t k_attention(const bf16_t *q, const bf16_t *gate, int gate_tok_stride,
                                  int gate_head_stride, const bf16_t *pk, const bf16_t *pvt, int P,
                                  int p_stride, const bf16_t *ok, const bf16_t *ovt, int o_stride,
                                  const int32_t *own_base, int N, int Hq, int Hkv, bf16_t *out,
                                  void *ws, size_t ws_bytes, hipStream_t stream) {
    if (N <= 0)
        return hipSuccess;
    if (Hq != 4 * Hkv || P < 0 || p_stride % 64 != 0 || o_stride % 64 != 0)
        return hipErrorInvalidValue;
    const int ntile = CEIL_DIV(N, QW);
    const int nblk = attention_blocks(ntile, Hkv);
    /* Few workgroups (an eval of a few branches: 4 kv-heads x 3 token tiles
     * at 80 tokens): split the key tiles over blockIdx.y so that about 256
     * workgroups run, when the workspace holds the partials. */
    const int nsplit = cujev_attention_splits(N, Hkv, P);
    if (nsplit > 1 && ws && ws_bytes >= cujev_attention_ws_bytes(N, Hq, nsplit)) {
        const size_t rows = (size_t)nsplit * N * Hq;
        AttnPart part{(float *)ws, (float *)ws + rows * D, (float *)ws + rows * (D + 1), nsplit};
        hipLaunchKernelGGL((attention_kernel<true, false>), dim3((unsigned)nblk, (unsigned)nsplit),
                           dim3(256), 0, stream, (const bf16 *)q, (const bf16 *)gate,
                           gate_tok_stride, gate_head_stride, (const bf16 *)pk, (const bf16 *)pvt,
                           P, p_stride, (const bf16 *)ok, (const bf16 *)ovt, o_stride, own_base, N,
                           Hq, Hkv, ntile, (bf16 *)out, part, AttnJob{}, 0);
        hipLaunchKernelGGL(attention_merge_kernel, dim3((unsigned)CEIL_DIV(N * Hq, 4)), dim3(256),
                           0, stream, part, (const bf16 *)gate, gate_tok_stride, gate_head_stride,
                           N, Hq, (bf16 *)out);
        return hipGetLastError();
    }
    hipLaunchKernelGGL((attention_kernel<false, false>), dim3((unsigned)nblk), dim3(256), 0, stream,
                       (const bf16 *)q, (const bf16 *)gate, gate_tok_stride, gate_head_stride,
                       (const bf16 *)pk, (const bf16 *)pvt, P, p_stride, (const bf16 *)ok,
                       (const bf16 *)ovt, o_stride, own_base, N, Hq, Hkv, ntile, (bf16 *)out,
                       AttnPart{}, AttnJob{}, 0);
    return hipGetLastError();
}

extern "C" hipError_t k_attention_pair(const bf16_t *q, const bf16_t *gate, int gate_tok_stride,
                                       int gate_head_stride, const bf16_t *pk, const bf16_t *pvt,
                                       int p_stride, const int32_t *own_base, bf16_t *out, int Hq,
                                       int Hkv, int Na, int Pa, const bf16_t *oka,
                                       const bf16_t *ovta, int oa_stride, int Nb, int Pb,
                                       const bf16_t *okb, const bf16_t *ovtb, int ob_stride,
                                       hipStream_t stream) {
    if (Na <= 0 || Nb <= 0)
        return Na > 0 ? k_attention(q, gate, gate_tok_stride, gate_head_stride, pk, pvt, Pa,
                                    p_stride, oka, ovta, oa_stride, own_base, Na, Hq, Hkv, out,
                                    nullptr, 0, stream)
                      : k_attention(q, gate, gate_tok_stride, gate_head_stride, pk, pvt, Pb,
                                    p_stride, okb, ovtb, ob_stride, own_base, Nb, Hq, Hkv, out,
                                    nullptr, 0, stream);
    if (Hq != 4 * Hkv || Pa < 0 || Pb < 0 || p_stride % 64 || oa_stride % 64 || ob_stride % 64)
        return hipErrorInvalidValue;
    const int ta = CEIL_DIV(Na, QW), tb = CEIL_DIV(Nb, QW);
    const AttnJob jb{(const bf16 *)okb, (const bf16 *)ovtb, Na, Pb, ob_stride, Nb};
    const int na = attention_blocks(ta, Hkv), nb = attention_blocks(tb, Hkv);
    hipLaunchKernelGGL((attention_kernel<false, true>), dim3((unsigned)(na + nb)), dim3(256), 0,
                       stream, (const bf16 *)q, (const bf16 *)gate, gate_tok_stride,
                       gate_head_stride, (const bf16 *)pk, (const bf16 *)pvt, Pa, p_stride,
                       (const bf16 *)oka, (const bf16 *)ovta, oa_stride, own_base, Na, Hq, Hkv, ta,
                       (bf16 *)out, AttnPart{}, jb, na);
    return hipGetLastError();
}
