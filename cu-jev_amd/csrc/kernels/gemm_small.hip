/* Weight-streaming GEMM for few tokens (gfx950): Y[N, M] = X[N, K] . W[M, K]^T
 * with N <= 96, bf16 in, fp32 accumulate. This is the eval-time shape of
 * every projection (the reference runs them through cuBLAS GemmEx,
 * src/kernels/elementwise.cu:56-75): the weights are read exactly once and
 * the time is the HBM stream of W, so the kernel is built around keeping
 * that stream full rather than around MFMA tiling.
 *
 *  - A workgroup owns 64 consecutive rows of W (16 per wave) and a K range;
 *    every wave streams its 16 rows straight from HBM into registers, three
 *    128-wide K chunks ahead of the MFMAs (v_mfma_f32_16x16x32_bf16 with W
 *    as the A operand, 16 tokens per B fragment).
 *  - W comes pre-tiled (k_gemm_small_tile, once per weight): the 16 rows x
 *    128 k of one wave and chunk are one contiguous 4 KiB block laid out in
 *    the order the wave's four 16-byte loads consume it, so every load
 *    instruction reads 1 KiB of consecutive bytes; blocks are chunk-major. Streaming the plain
 *    [M][K] rows (16 rows x 64 bytes per instruction) runs at two thirds of
 *    that rate.
 *  - X (tiny, L2-resident) goes to an LDS ring by buffer DMA, the same three
 *    chunks ahead, and is shared by the computing waves. One more wave
 *    issues all of those DMAs and waits for them before each step's
 *    barrier: an LDS
 *    read completes only after every buffer_load ... lds its own wave issued
 *    earlier has landed, so DMAs issued by the computing waves would hold
 *    their B-operand reads behind each prefetch.
 *  - A lane's 16 A-operand values for one 64-wide k step are 32 contiguous
 *    bytes of its W row (k = 64j + 16(l/16) + 0..15); the two MFMAs of the
 *    step take the halves, and the B fragments are read from LDS with the
 *    same k assignment, so the product is the plain dot product.
 *  - What sets the time is each CU's share of the bytes it requests: its
 *    weight rows plus a copy of X for its K range (at N = 80, 400 KiB for a
 *    2560-wide K, as much as the rows of a 64-row workgroup). A CU moves
 *    about 40 GB/s of such requests, so the grid is one workgroup per CU at
 *    most: two on one CU double its share and the kernel's time.
 *  - Short M (the 2560-wide outputs) splits K over blockIdx.y, as many ways
 *    as fill the CUs (the splits' chunk counts may differ by one). Splits
 *    write fp32 partials P[split][N][M] that the consumer (the residual add
 *    + RMSNorm) sums in a fixed order: results are deterministic, and the
 *    sum is rounded to bf16 like a bf16-output GEMM.
 *  - GATED=true is the fused gate|up projection (W rows [gate I | up I]):
 *    a workgroup takes 16 H gate rows and the same up rows (H = 2 with 4
 *    computing waves; H = 3 with 6 when 32-row halves would need more than
 *    256 workgroups), the up accumulators cross to the gate waves through
 *    LDS, and the output is act = bf16(silu(bf16 gate) * bf16 up) [N][I]
 *    directly, the rounding points of a bf16 GEMM followed by the
 *    activation pass.
 * All loads are unconditional (indices clamped into range): a load skipped
 * on one path would make the next use wait for every load in flight. */
#include "common.h"
#include "kernels.h"

namespace CUJEV_KNS {
namespace {

constexpr int SG_BM = 64;  /* W rows per workgroup (not gated) */
constexpr int SG_KC = 128; /* K per chunk          */
constexpr int SG_NS = 4;   /* pipeline depth: chunk c + 3 loads while c computes */

DEV bf16x8 ldg8(const bf16 *p) { return *(const bf16x8 *)p; }
typedef __attribute__((address_space(3))) void *lds_ptr;

/* Target builtins live in plain device functions: a template kernel that
 * names them directly gets no host-side launch stub. */
/* s_waitcnt with only the vector-memory count constrained (gfx9 encoding:
 * vmcnt bits 3:0 and 15:14; expcnt and lgkmcnt left at their maxima). The
 * counts used are 8 NB, NB = 1..6; others wait for everything. */
#define SG_VM(v) __builtin_amdgcn_s_waitcnt(((v) & 15) | (((v) >> 4) << 14) | (7 << 4) | (15 << 8))
DEV void sg_wait_vm(int vm) {
    switch (vm) {
    case 8: SG_VM(8); break;
    case 16: SG_VM(16); break;
    case 24: SG_VM(24); break;
    case 32: SG_VM(32); break;
    case 40: SG_VM(40); break;
    case 48: SG_VM(48); break;
    default: SG_VM(0); break;
    }
}
#undef SG_VM
/* 16 bytes per lane from base + voff + soff into LDS at dst + 16 * lane;
 * bytes past `bytes` read as zero */
DEV void sg_dma16(const void *base, uint32_t bytes, unsigned char *dst, uint32_t voff, int soff) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)dst, 16, voff, soff, 0, 0);
}
DEV bf16x8 sg_lds16(const unsigned char *base, uint32_t off) {
    return *(__attribute__((address_space(3))) const bf16x8 *)(
        (__attribute__((address_space(3))) const unsigned char *)base + off);
}

/* CW computing waves (4, or 6 for the gated projection's 48 + 48 rows) and
 * the X loader wave */
template <int NB, bool GATED, bool PART, int CW>
__global__ __launch_bounds__((CW + 1) * 64, 2) void gemm_small_kernel(
    const bf16 *__restrict__ X, int ldx, const bf16 *__restrict__ W, int N, int K,
    bf16 *__restrict__ Y, int ldy, float *__restrict__ P, int M) {
    static_assert(CW == 4 || (GATED && CW == 6), "4 computing waves, or 6 when gated");
    constexpr int H = CW / 2; /* gated: gate (and up) row groups per workgroup */
    /* X ring: SG_NS stages of NB*16 token rows x 128 k, rows of 256 bytes
     * with the 16-byte slots XOR-swizzled by (row & 15) */
    constexpr int XSTAGE = NB * 16 * 256;
    __shared__ __attribute__((aligned(1024))) unsigned char xs[SG_NS * XSTAGE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, c16 = lane & 15;
    /* split s of S takes chunks [s C / S, (s+1) C / S) of the C = K / 128 */
    const int split = blockIdx.y, nsplit = gridDim.y, ctot = K / SG_KC;
    const int cb0 = split * ctot / nsplit, nch = (split + 1) * ctot / nsplit - cb0;
    const int kb = cb0 * SG_KC;
    /* this wave's first W row (GATED: M = 2I, 32 gate rows + the same 32 up rows) */
    const int wr0 = GATED ? blockIdx.x * 16 * H + 16 * (wave % H) + (wave / H) * (M / 2)
                          : blockIdx.x * SG_BM + 16 * wave;

    /* tiled W: block (chunk, row group wr0/16) of 2048 elements, chunk-major
     * (G = M/16 row groups per chunk); load i of lane l is elements 512 i +
     * 8 l .. +7 of the block */
    const size_t G = (size_t)(M >> 4);
    const bf16 *wblk = W + ((size_t)(kb / SG_KC) * G + (wr0 >> 4)) * 2048 + lane * 8;
    auto load_w = [&](int c, bf16x8 (&wf)[4]) {
        const bf16 *p = wblk + (size_t)2048 * G * min(c, nch - 1);
#pragma unroll
        for (int i = 0; i < 4; i++)
            wf[i] = ldg8(p + 512 * i);
    };
    /* the number of steps (one barrier each), rounds of 4 */
    const int nsteps = (nch + 3) / 4 * 4;
    if (wave == CW) {
        /* X loader. A chunk -> LDS by buffer DMA: instruction i fills token
         * rows 4i + 0..3; lane l lands on slot l%16 of row 4i + l/16 and
         * fetches the chunk's 16-byte piece (l%16) ^ (row & 15). Rows >= N
         * lie past the buffer's range and read as zeros. Step c: wait for
         * chunk c (chunks c+1 and c+2, 8 NB DMAs, may stay in flight), the
         * barrier, then chunk c+3 into the stage chunk c-1 used. */
        const uint32_t xbytes = (uint32_t)N * ldx * 2;
        uint32_t xoff[4 * NB];
#pragma unroll
        for (int i = 0; i < 4 * NB; i++) {
            const int r = 4 * i + (lane >> 4);
            xoff[i] = (uint32_t)r * ldx * 2 + (uint32_t)(((lane & 15) ^ (r & 15)) * 16);
        }
        auto load_x = [&](int c) {
            unsigned char *st = xs + (c % SG_NS) * XSTAGE;
            const int kbyte = (kb + SG_KC * min(c, nch - 1)) * 2;
#pragma unroll
            for (int i = 0; i < 4 * NB; i++)
                sg_dma16(X, xbytes, st + 4 * i * 256, xoff[i], kbyte);
        };
        load_x(0);
        load_x(1);
        load_x(2);
        for (int c = 0; c < nsteps; c++) {
            sg_wait_vm(8 * NB);
            lds_barrier();
            load_x(c + 3);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); /* no DMA into LDS outlives the kernel */
        if constexpr (GATED) { /* the epilogue's two barriers */
            lds_barrier();
            lds_barrier();
        }
        return;
    }

    floatx4 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
        acc[nb] = floatx4{};
    auto compute = [&](int c, const bf16x8 (&wf)[4]) {
        const uint32_t st = (c % SG_NS) * XSTAGE + c16 * 256;
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int hf = 0; hf < 2; hf++) {
                const uint32_t slot = (uint32_t)(((8 * j + 2 * q + hf) ^ c16) << 4);
                bf16x8 b[NB];
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
                    b[nb] = sg_lds16(xs, st + nb * 16 * 256 + slot);
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
                    acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[2 * j + hf], b[nb],
                                                                      acc[nb], 0, 0, 0);
            }
    };

    /* Each step c: the barrier (after it chunk c's X is in LDS and the
     * stage chunk c-1 used is free), load W of c+3, compute c. W lives in
     * the register ring w0..w3 (slot c % 4); the compiler waits for each W
     * register before its MFMA. Whole rounds of 4 steps, no early exit: past
     * the end the loads repeat the last chunk and only the MFMAs are
     * skipped. */
    bf16x8 w0[4], w1[4], w2[4], w3[4];
    load_w(0, w0);
    load_w(1, w1);
    load_w(2, w2);
    auto step = [&](int c, const bf16x8 (&wcur)[4], bf16x8 (&wfill)[4]) {
        lds_barrier();
        load_w(c + 3, wfill);
        __builtin_amdgcn_sched_barrier(0); /* keep the prefetches here */
        if (c < nch)
            compute(c, wcur);
    };
    for (int c = 0; c < nsteps; c += 4) {
        step(c, w0, w3);
        step(c + 1, w1, w0);
        step(c + 2, w2, w1);
        step(c + 3, w3, w2);
    }

    /* acc[nb]: token 16 nb + c16, rows wr0 + 4q .. +3 */
    if constexpr (GATED) {
        /* up waves (H..CW-1) hand their accumulators to the gate waves */
        lds_barrier();
        floatx4 *xch = (floatx4 *)xs; /* [H][NB][64] */
        if (wave >= H) {
#pragma unroll
            for (int nb = 0; nb < NB; nb++)
                xch[((wave - H) * NB + nb) * 64 + lane] = acc[nb];
        }
        lds_barrier();
        if (wave < H) {
            const int m = blockIdx.x * 16 * H + 16 * wave + 4 * q;
#pragma unroll
            for (int nb = 0; nb < NB; nb++) {
                const int n = 16 * nb + c16;
                const floatx4 u = xch[(wave * NB + nb) * 64 + lane];
                bf16x4 a;
#pragma unroll
                for (int e = 0; e < 4; e++)
                    a[e] = f2bf(silu_f(bf2f(f2bf(acc[nb][e]))) * bf2f(f2bf(u[e])));
                if (n < N)
                    *(bf16x4 *)(Y + (size_t)n * ldy + m) = a;
            }
        }
        return;
    }
    const int m = wr0 + 4 * q;
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        const int n = 16 * nb + c16;
        if (n >= N)
            continue;
        if constexpr (PART) {
            *(floatx4 *)(P + ((size_t)split * N + n) * M + m) = acc[nb];
        } else {
            *(bf16x4 *)(Y + (size_t)n * ldy + m) =
                bf16x4{f2bf(acc[nb][0]), f2bf(acc[nb][1]), f2bf(acc[nb][2]), f2bf(acc[nb][3])};
        }
    }
}

/* W [M][K] -> the tiled layout the kernel streams: block b = (c, g), g = row
 * group of 16, c = 128-wide K chunk, at b = c (M/16) + g (chunk-major: the
 * workgroups, which move through K together, read one contiguous region at a
 * time); element 512 i +
 * 8 l + e of the block is W[16 g + l%16][128 c + 64 (i/2) + 16 (l/16) +
 * 8 (i%2) + e] (the A operand of lane l = row l%16, k 16 (l/16) + 8 hf.., for
 * the two MFMAs of k step 64 j, i = 2 j + hf). One thread per 16 bytes. */
__global__ __launch_bounds__(256) void gemm_small_tile_kernel(const bf16 *__restrict__ W, int M,
                                                              int K, bf16 *__restrict__ Wt) {
    const size_t piece = (size_t)blockIdx.x * 256 + threadIdx.x; /* 8 elements each */
    const size_t total = (size_t)M * K / 8;
    if (piece >= total)
        return;
    const int l = (int)(piece & 63), i = (int)((piece >> 6) & 3);
    const size_t b = piece >> 8;
    const int G = M / 16;
    const int g = (int)(b % G), c = (int)(b / G);
    const int row = 16 * g + (l & 15);
    const int k = SG_KC * c + 64 * (i >> 1) + 16 * (l >> 4) + 8 * (i & 1);
    *(bf16x8 *)(Wt + piece * 8) = ldg8(W + (size_t)row * K + k);
}

template <bool GATED, bool PART, int CW>
hipError_t launch_nb(int NB, dim3 grid, hipStream_t s, const bf16 *X, int ldx, const bf16 *W,
                     int N, int K, bf16 *Y, int ldy, float *P, int M) {
#define CUJEV_SG_CASE(nb)                                                                    \
    case nb:                                                                                 \
        hipLaunchKernelGGL((gemm_small_kernel<nb, GATED, PART, CW>), grid,                     \
                           dim3((CW + 1) * 64), 0, s, X, ldx, W, N, K, Y, ldy, P, M);          \
        break;
    switch (NB) {
        CUJEV_SG_CASE(1)
        CUJEV_SG_CASE(2)
        CUJEV_SG_CASE(3)
        CUJEV_SG_CASE(4)
        CUJEV_SG_CASE(5)
        CUJEV_SG_CASE(6)
    default:
        return hipErrorInvalidValue;
    }
#undef CUJEV_SG_CASE
    return hipGetLastError();
}

} // namespace
} // namespace CUJEV_KNS
using namespace CUJEV_KNS;

extern "C" int cujev_gemm_small_splits(int M, int K) {
    if (M <= 0 || K <= 0 || M % SG_BM || K % SG_KC)
        return 0;
    const int rowblocks = M / SG_BM, chunks = K / SG_KC;
    /* about one workgroup per CU; the splits' chunk counts may differ by one */
    int s = (256 + rowblocks / 2) / rowblocks;
    s = s < 1 ? 1 : s > chunks ? chunks : s;
    return s > CUJEV_GEMM_SMALL_MAX_SPLITS ? CUJEV_GEMM_SMALL_MAX_SPLITS : s;
}

extern "C" hipError_t k_gemm_small_tile(const bf16_t *W, int M, int K, bf16_t *Wt,
                                        hipStream_t stream) {
    if (M <= 0 || K <= 0 || M % 16 || K % SG_KC || W == Wt)
        return hipErrorInvalidValue;
    const size_t pieces = (size_t)M * K / 8;
    hipLaunchKernelGGL(gemm_small_tile_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256),
                       0, stream, (const bf16 *)W, M, K, (bf16 *)Wt);
    return hipGetLastError();
}

extern "C" hipError_t k_gemm_small(const bf16_t *X, int ldx, const bf16_t *W, int N, int M, int K,
                                   int gated, int splits, bf16_t *Y, int ldy, float *P,
                                   hipStream_t stream) {
    if (N <= 0)
        return hipSuccess;
    if (N > CUJEV_GEMM_SMALL_MAX_N || M % SG_BM || K % SG_KC || splits < 1 ||
        splits > K / SG_KC || (splits > 1 && (!P || gated)) || (splits == 1 && !Y))
        return hipErrorInvalidValue;
    const int NB = (N + 15) / 16;
    const bf16 *x = (const bf16 *)X, *w = (const bf16 *)W;
    if (splits > 1)
        return launch_nb<false, true, 4>(NB, dim3((unsigned)(M / SG_BM), (unsigned)splits), stream,
                                         x, ldx, w, N, K, nullptr, 0, P, M);
    if (gated) {
        /* More than one workgroup per CU (each streams its own copy of X as
         * well as its rows) would double some CUs' share: past 256
         * workgroups of 32 + 32 rows, take 48 + 48 when that divides. */
        const int I = M / 2;
        if (I / 32 > 256 && I % 48 == 0)
            return launch_nb<true, false, 6>(NB, dim3((unsigned)(I / 48)), stream, x, ldx, w, N, K,
                                             (bf16 *)Y, ldy, nullptr, M);
        return launch_nb<true, false, 4>(NB, dim3((unsigned)(I / 32)), stream, x, ldx, w, N, K,
                                         (bf16 *)Y, ldy, nullptr, M);
    }
    return launch_nb<false, false, 4>(NB, dim3((unsigned)(M / SG_BM)), stream, x, ldx, w, N, K,
                                      (bf16 *)Y, ldy, nullptr, M);
}
