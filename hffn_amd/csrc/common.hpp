// Shared device helpers of the HFFN kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hffn {

constexpr int kWave = 64;

// exp(y) as the hardware base-2 exponential of y log2(e) carried in two floats: the product's rounding error and the
// tail of log2(e) are put back by a first-order factor, so that it loses nothing against expf to the rounding of a
// large |y|.
__device__ __forceinline__ float exp_split(float y) {
    constexpr float kLog2e = 1.44269502162933349609375f, kLog2eTail = 1.925963033500011e-8f, kLn2 = 0.69314718055994531f;
    const float h = y * kLog2e;
    const float l = fmaf(y, kLog2eTail, fmaf(y, kLog2e, -h));  // y log2(e) = h + l to about 2^-48 |h|
    return __builtin_amdgcn_exp2f(h) * fmaf(l, kLn2, 1.0f);
}

// Exact GELU (erf form, PyTorch's approximate="none"; `gelu` of
// runtime/gpu/nvidia/common/kernels/hffn_cuda/kernels.py:87-89), written as z/2 erfc(-z/sqrt 2) so that negative z
// keep their relative accuracy (no 1 + erf cancellation), with erfc from the Chebyshev fit of Press, Teukolsky,
// Vetterling and Flannery, Numerical Recipes (2nd ed., section 6.2, "erfcc"; fractional error below 1.2e-7 for
// every argument): for x >= 0, erfc(x) = t exp(-x^2 + P(t)) with t = 1 / (1 + x / 2), and erfc(-x) = 2 - erfc(x).
// Branch-free, so that a wave evaluates many independent GELUs back to back. The reciprocal is the hardware one
// (1 ulp) refined by a Newton step; the exponential is exp_split.
// erfc(a) for a >= 0:
__device__ __forceinline__ float erfc_nonneg(float a) {
    const float d = fmaf(0.5f, a, 1.0f);
    const float t0 = __builtin_amdgcn_rcpf(d);
    const float t = fmaf(t0, fmaf(-d, t0, 1.0f), t0);
    float p = 0.17087277f;
    p = fmaf(p, t, -0.82215223f);
    p = fmaf(p, t, 1.48851587f);
    p = fmaf(p, t, -1.13520398f);
    p = fmaf(p, t, 0.27886807f);
    p = fmaf(p, t, -0.18628806f);
    p = fmaf(p, t, 0.09678418f);
    p = fmaf(p, t, 0.37409196f);
    p = fmaf(p, t, 1.00002368f);
    p = fmaf(p, t, -1.26551223f);
    return t * exp_split(fmaf(-a, a, p));
}

__device__ __forceinline__ float gelu(float z) {
    const float x = -z * 0.70710678118654752f;
    const float tail = erfc_nonneg(fabsf(x));  // erfc(|x|)
    return 0.5f * z * (x >= 0.0f ? tail : 2.0f - tail);
}

// d gelu / dz = Phi(z) + z phi(z) (the form of PyTorch's GELU backward, approximate="none"; `gelu_grad` of
// runtime/gpu/nvidia/ffn/training/kernels_train.py:111-113), Phi(z) = erfc(-z/sqrt 2)/2 as in gelu and
// phi(z) = exp(-z^2/2)/sqrt(2 pi).
__device__ __forceinline__ float gelu_grad(float z) {
    const float x = -z * 0.70710678118654752f;
    const float tail = erfc_nonneg(fabsf(x));
    const float cdf = 0.5f * (x >= 0.0f ? tail : 2.0f - tail);
    const float pdf = 0.39894228040143268f * exp_split((-0.5f * z) * z);
    return fmaf(z, pdf, cdf);
}

// Value loads: float32 store, or bfloat16 bits widened exactly to float32.
__device__ __forceinline__ float widen(float v) { return v; }
__device__ __forceinline__ float widen(uint16_t v) { return __uint_as_float(static_cast<uint32_t>(v) << 16); }

// Sum over the 64 lanes of a wave; every lane receives the same total (fixed xor-butterfly order,
// so the result does not depend on scheduling).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
    return v;
}

__device__ __forceinline__ uint32_t uniform(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
}

template <int N>
__device__ __forceinline__ void load_vec(const float* p, float (&out)[N]) {
    if constexpr (N == 1) {
        out[0] = *p;
    } else if constexpr (N == 2) {
        const float2 v = *reinterpret_cast<const float2*>(p);
        out[0] = v.x; out[1] = v.y;
    } else if constexpr (N == 4) {
        const float4 v = *reinterpret_cast<const float4*>(p);
        out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
    } else {
        static_assert(N == 8, "vector loads of 1, 2, 4 or 8 floats");
        const float4 v = *reinterpret_cast<const float4*>(p);
        const float4 u = *reinterpret_cast<const float4*>(p + 4);
        out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
        out[4] = u.x; out[5] = u.y; out[6] = u.z; out[7] = u.w;
    }
}

// s_waitcnt vmcnt(N) lgkmcnt(0): at most N vector-memory loads of this wave still in flight, its LDS accesses done.
template <int N>
__device__ __forceinline__ void wait_loads() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

// 16 bytes per lane from global memory straight into LDS (global_load_lds_dwordx4): lane l reads base + offset_l
// (base wave-uniform, in scalar registers; offset_l a 32-bit byte offset in a vector register) and its bytes land at
// lds + 16 l. Inactive lanes transfer nothing. Written as inline assembly so that the compiler, which cannot tell the
// transfers' LDS destinations apart, does not wait for every transfer in flight before each LDS read; the kernel
// orders them itself (wait_loads, then a barrier).
__device__ __forceinline__ void dma16(const void* base, uint32_t offset, const void* lds) {
    const uint32_t to = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(
        static_cast<int>(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)))));  // low 32 bits: the LDS address
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(offset), "s"(base), "s"(to)
                 : "memory", "m0");
}

// The same with 4 bytes per lane (lane l's land at lds + 4 l).
__device__ __forceinline__ void dma4(const void* base, uint32_t offset, const void* lds) {
    const uint32_t to = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(
        static_cast<int>(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)))));
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(offset), "s"(base), "s"(to)
                 : "memory", "m0");
}

}  // namespace hffn
