// Training kernels of the HFFN layer on CDNA4 (wave64): the two sampled products of the backward (the gradients of
// the compact weights; lanes over tokens in 256-token tiles, or lanes over slots up to 8 tokens), the fixed-order sum
// of their token-tile partials, the compact AdamW and a value gather. The other two backward quantities are gathers
// with the forward's shapes: gz is the up kernel (edges up to 8 tokens, else rows) over the hidden-major down support
// with a gelu' epilogue, gx the down kernel (edges or rows) over the input-major up support with no bias. Semantics
// follow runtime/gpu/nvidia/ffn/training/kernels_train.py:101-258; every result is written by exactly one lane, with
// no atomics, so the bits repeat run to run.
#include "common.hpp"
#include "launch.hpp"

namespace hffn {
namespace {

constexpr uint32_t kBlock = 256;
constexpr uint32_t kWaves = kBlock / kWave;
constexpr uint32_t kTokensPerLane = kGradTile / kWave;  // 4: one 16-byte load per lane and row
static_assert(kTokensPerLane == 4, "the lanes of a tile hold 4 consecutive tokens");

uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

// Sampled product, owner-row form (grad_down over the output-major down edges with row = gy_t and mat = act; grad_up
// over the hidden-major up slots with row = gz and mat = x_t; kernels_train.py:115-137 and 162-184). One wave per
// owner o and token tile k; lane l holds row[o, t] for its 4 consecutive tokens t = 256 k + 4 l + j. Per slot q the
// lane forms sum_j row[o, t] * mat[idx[q], t] (ascending j, tokens past n skipped) and the wave adds the lanes with
// the fixed xor butterfly. The slots are taken 4 at a time, so that 4 row reads are in flight per wave.
__global__ __launch_bounds__(kBlock) void grad_sddmm_kernel(const float* __restrict__ row, const float* __restrict__ mat,
                                                           const int32_t* __restrict__ off, const int16_t* __restrict__ idx,
                                                           float* __restrict__ g, float* __restrict__ gb, uint32_t rows,
                                                           uint32_t n, uint32_t ld, uint32_t stride) {
    const uint32_t o = blockIdx.x * kWaves + uniform(threadIdx.x / kWave), lane = threadIdx.x % kWave;
    if (o >= rows) return;
    const uint32_t t0 = blockIdx.y * kGradTile + lane * kTokensPerLane;
    const size_t part = static_cast<size_t>(blockIdx.y) * stride;
    const bool active = t0 < n;
    float own[kTokensPerLane] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (active) load_vec<kTokensPerLane>(row + static_cast<size_t>(o) * ld + t0, own);
    float sum = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < kTokensPerLane; ++j) {
        if (t0 + j >= n) own[j] = 0.0f;
        sum += own[j];
    }
    const float total = wave_sum(sum);
    if (lane == 0) gb[part + o] = total;
    const int32_t begin = off[o], end = off[o + 1];
    const auto dot = [&](const float (&m)[kTokensPerLane]) {
        float s = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < kTokensPerLane; ++j) s = t0 + j < n ? fmaf(own[j], m[j], s) : s;
        return s;
    };
    int32_t q = begin;
    for (; q + 4 <= end; q += 4) {
        float m[4][kTokensPerLane] = {};
        if (active) {
#pragma unroll
            for (int u = 0; u < 4; ++u)
                load_vec<kTokensPerLane>(mat + static_cast<size_t>(static_cast<uint16_t>(idx[q + u])) * ld + t0, m[u]);
        }
        float s[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) s[u] = wave_sum(dot(m[u]));
        if (lane == 0) {
#pragma unroll
            for (int u = 0; u < 4; ++u) g[part + q + u] = s[u];
        }
    }
    for (; q < end; ++q) {
        float m[kTokensPerLane] = {};
        if (active) load_vec<kTokensPerLane>(mat + static_cast<size_t>(static_cast<uint16_t>(idx[q])) * ld + t0, m);
        const float s = wave_sum(dot(m));
        if (lane == 0) g[part + q] = s;
    }
}

// Sampled product for n <= 8 tokens (one pass): lanes over the slots of owner o (slot q = begin + lane + 64 k), the n
// values of row o in registers (the same for every lane); each lane forms its slot's sum over the tokens in ascending
// order and writes it, so no cross-lane reduction is needed. Lane 0 writes gb.
template <int NT>
__global__ __launch_bounds__(kBlock) void grad_sddmm_edges_kernel(const float* __restrict__ row, const float* __restrict__ mat,
                                                                 const int32_t* __restrict__ off, const int16_t* __restrict__ idx,
                                                                 float* __restrict__ g, float* __restrict__ gb, uint32_t rows,
                                                                 uint32_t n, uint32_t ld) {
    const uint32_t o = blockIdx.x * kWaves + uniform(threadIdx.x / kWave), lane = threadIdx.x % kWave;
    if (o >= rows) return;
    float own[NT];
    load_vec<NT>(row + static_cast<size_t>(o) * ld, own);
    float sum = 0.0f;
#pragma unroll
    for (uint32_t t = 0; t < NT; ++t) sum = t < n ? sum + own[t] : sum;
    if (lane == 0) gb[o] = sum;
    const int32_t end = off[o + 1];
    for (int32_t q = off[o] + static_cast<int32_t>(lane); q < end; q += kWave) {
        float m[NT];
        load_vec<NT>(mat + static_cast<size_t>(static_cast<uint16_t>(idx[q])) * ld, m);
        float s = 0.0f;
#pragma unroll
        for (uint32_t t = 0; t < NT; ++t) s = t < n ? fmaf(own[t], m[t], s) : s;
        g[q] = s;
    }
}

// ws [tiles, stride]: columns [0, c1) g_down, [c1, c2) gb_down, [c2, c3) g_up, [c3, stride) gb_up. One thread per
// column: ((ws[0][j] + ws[1][j]) + ws[2][j]) + ... in ascending tile order (kernels_train.py:186-199).
__global__ __launch_bounds__(kBlock) void reduce_tiles_kernel(const float* __restrict__ ws, uint32_t stride, uint32_t tiles,
                                                             uint32_t c1, uint32_t c2, uint32_t c3, float* __restrict__ g_down,
                                                             float* __restrict__ gb_down, float* __restrict__ g_up,
                                                             float* __restrict__ gb_up) {
    const uint32_t j = blockIdx.x * kBlock + threadIdx.x;
    if (j >= stride) return;
    float s = ws[j];
    for (uint32_t k = 1; k < tiles; ++k) s += ws[static_cast<size_t>(k) * stride + j];
    if (j < c1) g_down[j] = s;
    else if (j < c2) gb_down[j - c1] = s;
    else if (j < c3) g_up[j - c2] = s;
    else gb_up[j - c3] = s;
}

// Compact AdamW in the order of PyTorch's AdamW (kernels_train.py:233-247): decoupled decay, then the moments, then
// the bias-corrected step; the step-dependent scalars come from the host (float64 there). A thread takes four
// consecutive entries with 16-byte loads and stores (the first `quads` threads, when all four arrays are 16-byte
// aligned), one entry otherwise (the rest); the same arithmetic per entry either way.
struct AdamScalars {
    float lr_decay, beta1, one_minus_beta1, beta2, one_minus_beta2, step_size, bias2_sqrt, eps;
};

__device__ __forceinline__ void adamw_entry(float& p, float g, float& m, float& v, const AdamScalars& a) {
    p -= a.lr_decay * p;
    m = a.beta1 * m + a.one_minus_beta1 * g;
    v = a.beta2 * v + a.one_minus_beta2 * g * g;
    p = p - a.step_size * m / (sqrtf(v) / a.bias2_sqrt + a.eps);
}

__global__ __launch_bounds__(kBlock) void adamw_kernel(float* __restrict__ p, const float* __restrict__ g, float* __restrict__ m,
                                                      float* __restrict__ v, uint32_t count, uint32_t quads, AdamScalars a) {
    const uint32_t i = blockIdx.x * kBlock + threadIdx.x;
    if (i < quads) {
        float4 pi = reinterpret_cast<const float4*>(p)[i];
        const float4 gi = reinterpret_cast<const float4*>(g)[i];
        float4 mi = reinterpret_cast<const float4*>(m)[i], vi = reinterpret_cast<const float4*>(v)[i];
        adamw_entry(pi.x, gi.x, mi.x, vi.x, a);
        adamw_entry(pi.y, gi.y, mi.y, vi.y, a);
        adamw_entry(pi.z, gi.z, mi.z, vi.z, a);
        adamw_entry(pi.w, gi.w, mi.w, vi.w, a);
        reinterpret_cast<float4*>(m)[i] = mi;
        reinterpret_cast<float4*>(v)[i] = vi;
        reinterpret_cast<float4*>(p)[i] = pi;
        return;
    }
    const uint32_t j = 4 * quads + (i - quads);
    if (j >= count) return;
    float pj = p[j], mj = m[j], vj = v[j];
    adamw_entry(pj, g[j], mj, vj, a);
    m[j] = mj;
    v[j] = vj;
    p[j] = pj;
}

__global__ __launch_bounds__(kBlock) void gather_values_kernel(const float* __restrict__ src, const int32_t* __restrict__ pos,
                                                              float* __restrict__ dst, uint32_t count) {
    const uint32_t i = blockIdx.x * kBlock + threadIdx.x;
    if (i < count) dst[i] = src[pos[i]];
}

}  // namespace

hipError_t launch_grad_sddmm(const float* row, const float* mat, const int32_t* off, const int16_t* idx, float* g, float* gb,
                             uint32_t rows, uint32_t n, uint32_t ld, uint32_t stride, hipStream_t stream) {
    hipLaunchKernelGGL(grad_sddmm_kernel, dim3(ceil_div(rows, kWaves), grad_tiles(n)), dim3(kBlock), 0, stream, row, mat, off, idx,
                       g, gb, rows, n, ld, stride);
    return hipGetLastError();
}

hipError_t launch_grad_sddmm_edges(const float* row, const float* mat, const int32_t* off, const int16_t* idx, float* g, float* gb,
                                   uint32_t rows, uint32_t n, uint32_t ld, hipStream_t stream) {
    const dim3 grid(ceil_div(rows, kWaves)), block(kBlock);
    switch (edges_tokens(n)) {
        case 1: hipLaunchKernelGGL(grad_sddmm_edges_kernel<1>, grid, block, 0, stream, row, mat, off, idx, g, gb, rows, n, ld); break;
        case 2: hipLaunchKernelGGL(grad_sddmm_edges_kernel<2>, grid, block, 0, stream, row, mat, off, idx, g, gb, rows, n, ld); break;
        case 4: hipLaunchKernelGGL(grad_sddmm_edges_kernel<4>, grid, block, 0, stream, row, mat, off, idx, g, gb, rows, n, ld); break;
        default: hipLaunchKernelGGL(grad_sddmm_edges_kernel<8>, grid, block, 0, stream, row, mat, off, idx, g, gb, rows, n, ld); break;
    }
    return hipGetLastError();
}

hipError_t launch_reduce_tiles(const float* ws, uint32_t stride, uint32_t tiles, uint32_t c1, uint32_t c2, uint32_t c3,
                               float* g_down, float* gb_down, float* g_up, float* gb_up, hipStream_t stream) {
    hipLaunchKernelGGL(reduce_tiles_kernel, dim3(ceil_div(stride, kBlock)), dim3(kBlock), 0, stream, ws, stride, tiles, c1, c2, c3,
                       g_down, gb_down, g_up, gb_up);
    return hipGetLastError();
}

hipError_t launch_adamw(float* p, const float* g, float* m, float* v, uint32_t count, float lr_decay, float beta1,
                        float one_minus_beta1, float beta2, float one_minus_beta2, float step_size, float bias2_sqrt, float eps,
                        hipStream_t stream) {
    const bool aligned = (reinterpret_cast<uintptr_t>(p) | reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(m) |
                          reinterpret_cast<uintptr_t>(v)) % 16 == 0;
    const uint32_t quads = aligned ? count / 4 : 0, threads = quads + (count - 4 * quads);
    const AdamScalars a{lr_decay, beta1, one_minus_beta1, beta2, one_minus_beta2, step_size, bias2_sqrt, eps};
    hipLaunchKernelGGL(adamw_kernel, dim3(ceil_div(threads, kBlock)), dim3(kBlock), 0, stream, p, g, m, v, count, quads, a);
    return hipGetLastError();
}

hipError_t launch_gather_values(const float* src, const int32_t* pos, float* dst, uint32_t count, hipStream_t stream) {
    hipLaunchKernelGGL(gather_values_kernel, dim3(ceil_div(count, kBlock)), dim3(kBlock), 0, stream, src, pos, dst, count);
    return hipGetLastError();
}

}  // namespace hffn
