// Shared device helpers of the HFFN kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hffn {

constexpr int kWave = 64;

// Exact GELU (erf form, PyTorch's approximate="none"), with the device erff of the ROCm math
// library (OCML). Matches `gelu` of runtime/gpu/nvidia/common/kernels/hffn_cuda/kernels.py:87-89.
__device__ __forceinline__ float gelu(float z) {
    return 0.5f * z * (1.0f + erff(z * 0.70710678118654752f));
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

}  // namespace hffn
