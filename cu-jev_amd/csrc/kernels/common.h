/* Device helpers shared by the gfx950 kernels.
 *
 * Semantics of silu / sigmoid / softplus (threshold 20) follow the reference's
 * src/kernels/common.cuh:7-13; the implementations are written for CDNA4
 * (v_exp_f32 / v_rcp_f32 via builtins, wave64 reductions). */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define CUJEV_LOG2E 1.4426950408889634f

#define DEV __device__ __forceinline__

/* Kernels live in this namespace. The engine library and the operator
 * library compile the same sources under different names, so profiles tell
 * their launches apart. */
#ifndef CUJEV_KNS
#define CUJEV_KNS cujev
#endif

DEV float bf2f(bf16 x) { return (float)x; }
DEV bf16 f2bf(float x) { return (bf16)x; } /* round to nearest even */

/* 2^x on the transcendental unit; exact -inf -> 0. */
DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
DEV float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * CUJEV_LOG2E); }
/* 1/(1+e^-x) with the hardware reciprocal (v_rcp_f32, about 1 ulp) rather
 * than an IEEE division sequence. */
DEV float sigmoid_f(float x) { return __builtin_amdgcn_rcpf(1.f + fast_exp(-x)); }
DEV float silu_f(float x) { return x * __builtin_amdgcn_rcpf(1.f + fast_exp(-x)); }
/* log(1+e^x), linear above 20 like torch.nn.functional.softplus. */
DEV float softplus_f(float x) { return x > 20.f ? x : log1pf(expf(x)); }

/* Workgroup barrier for LDS traffic only: this wave's LDS operations are
 * complete (so its writes are visible and its reads have returned), then
 * s_barrier. Unlike __syncthreads() it does not wait for the wave's global
 * stores to reach memory, so stores issued before it keep streaming. Global
 * data another wave reads needs __syncthreads(); LDS written by buffer
 * loads (...lds) needs an explicit vmcnt wait first. */
DEV void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

/* Wave64 reductions (butterfly over all 64 lanes). */
DEV float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        v += __shfl_xor(v, o, 64);
    return v;
}
DEV float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

/* Sum over a block of `nw` waves; scratch holds >= nw floats. Result is
 * broadcast to every thread. */
DEV float block_sum(float v, float *scratch) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    __syncthreads();
    if (lane == 0)
        scratch[w] = v;
    __syncthreads();
    float r = 0.f;
    for (int i = 0; i < nw; i++)
        r += scratch[i];
    return r;
}

#define CEIL_DIV(a, b) (((a) + (b) - 1) / (b))
