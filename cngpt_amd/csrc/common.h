// common.h - shared device helpers for the gfx950 kernels of cngpt_amd.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define CNGPT_WAVE 64

// Guarded 16-byte load that always reads *p (the caller clamps the index to
// a valid address) and returns zero when !ok. Unlike `ok ? *p : 0`, which
// masks the load off for lanes without ok, it costs a real access per lane;
// it serves where the masked-off lanes are few and a fixed instruction
// sequence keeps register pressure down (LayerNorm rows).
__device__ __forceinline__ f32x4 ld4_or0(const f32x4* p, bool ok) {
    const f32x4 v = *p;
    return ok ? v : f32x4{0.f, 0.f, 0.f, 0.f};
}

// Butterfly sum / max over the 64 lanes of a wavefront.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Sum / max over the 64 lanes with DPP lane moves inside each row of 16
// (xor 1, xor 2, half-row mirror, row mirror) and the four row results read
// as scalars: a few cycles per step instead of an LDS round trip per
// shuffle. Every lane of the wavefront must be active. The result is the
// same in every lane.
#define CNGPT_DPP(v, ctrl)                                                                  \
    __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, (v)), (ctrl), \
                                                       0xF, 0xF, false))
__device__ __forceinline__ float row_sum16(float v) {
    v += CNGPT_DPP(v, 0xB1);   // quad_perm [1,0,3,2]
    v += CNGPT_DPP(v, 0x4E);   // quad_perm [2,3,0,1]
    v += CNGPT_DPP(v, 0x141);  // row_half_mirror
    v += CNGPT_DPP(v, 0x140);  // row_mirror
    return v;
}
// LDS pointer type of the direct global -> LDS loads (global_load_lds).
typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt vmcnt(N), expcnt and lgkmcnt left alone (GFX9 encoding: vmcnt
// in bits 3:0 and 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (7 << 4) | (0xF << 8));
}

// wait_vmcnt<n>() for 0 <= n < N <= 8 where n is a constant only once the
// caller's loop is unrolled (the switch then folds to the one wait)
template <int N>
__device__ __forceinline__ void wait_vmcnt_dyn(int n) {
    static_assert(N <= 8, "counts up to 7");
    switch (n) {
        case 0: wait_vmcnt<0>(); break;
        case 1: wait_vmcnt<1>(); break;
        case 2: wait_vmcnt<2>(); break;
        case 3: wait_vmcnt<3>(); break;
        case 4: wait_vmcnt<4>(); break;
        case 5: wait_vmcnt<5>(); break;
        case 6: wait_vmcnt<6>(); break;
        default: wait_vmcnt<7>(); break;
    }
}

// 16 bytes per lane from global memory into LDS at lds + 16 * lane
// (global_load_lds_dwordx4, lds wavefront-uniform), issued as assembly so
// that the compiler tracks neither the load nor the LDS it writes: it would
// otherwise wait for every such load in flight before the first LDS read
// that it cannot prove disjoint, and a ring of such loads carried across
// loop trips in registers would lose its prefetch to a wait for every load
// at the top of each trip. The caller's explicit vmcnt waits cover them.
// M0 (the LDS base) is restored for the compiler's own use.
__device__ __forceinline__ void lds_dma16(const void* g, const float* lds) {
    const unsigned la = (unsigned)(size_t)(const __attribute__((address_space(3))) float*)lds;
    int m0s;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "global_load_lds_dwordx4 %2, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(m0s)
        : "s"(la), "v"(g)
        : "memory");
}

__device__ __forceinline__ float lane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v = row_sum16(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, CNGPT_DPP(v, 0xB1));
    v = fmaxf(v, CNGPT_DPP(v, 0x4E));
    v = fmaxf(v, CNGPT_DPP(v, 0x141));
    v = fmaxf(v, CNGPT_DPP(v, 0x140));
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// GELU, tanh form (the formula of the reference's ops.h:56-58):
// 0.5 x (1 + tanh(u)), u = sqrt(2/pi) (x + 0.044715 x^3), evaluated as
// x / (1 + exp(-2u)) (1 + tanh(u) = 2 / (1 + exp(-2u))): one hardware exp
// and one reciprocal instead of a library tanh, a few ulp from it. Large
// negative x give exp(-2u) = inf and the limit -0.
__device__ __forceinline__ float gelu_tanh(float x) {
    const float k0 = 0.7978845608028654f;  // sqrt(2/pi)
    const float k1 = 0.044715f;
    const float u = k0 * (x + k1 * (x * x * x));
    return x * __builtin_amdgcn_rcpf(1.0f + __expf(-2.0f * u));
}

// Epilogues shared by the GEMM and GEMV kernels.
enum EpiMode : int {
    EPI_STORE = 0,      // Y = acc
    EPI_BIAS = 1,       // Y = acc + b
    EPI_BIAS_GELU = 2,  // Y = gelu(acc + b)
    EPI_RESID = 3,      // Y = (Y + acc) + b   (residual folded in, beta = 1)
};

template <int EPI>
__device__ __forceinline__ float apply_epi(float acc, const float* __restrict__ bias, int col,
                                           const float* yold) {
    if (EPI == EPI_STORE) return acc;
    if (EPI == EPI_BIAS) return acc + bias[col];
    if (EPI == EPI_BIAS_GELU) return gelu_tanh(acc + bias[col]);
    return (*yold + acc) + bias[col];
}
