// Lane-per-token ("rows") gather kernels of the HFFN forward on CDNA4 (wave64), and the layout transpose:
// up projection with fused bias + exact GELU, and the atomics-free down projection over the output-major store.
// One wave per neuron/output; the lanes own consecutive tokens (TPL per lane, vector loads), the wave walks the row's
// slots in order with wave-uniform index/value loads, and each slot is one coalesced read of a feature-major input
// row. (The lane-per-slot decode shapes are in edges.hip.)
// Every activation and every output is written by exactly one lane: no atomics, bitwise
// repeatable. Semantics follow runtime/gpu/nvidia/common/kernels/hffn_cuda/kernels.py:1-22.
#include "common.hpp"
#include "launch.hpp"

namespace hffn {
namespace {

constexpr uint32_t kBlock = 256;
constexpr uint32_t kWaves = kBlock / kWave;

// ------------------------------------------------------------------------------------------- up, rows
// EPI kGelu: act = gelu(b + acc), and z = b + acc where z is not null (the training forward keeps it). EPI kGeluGrad
// (the backward's gz): act = acc * gelu'(z), z read, b unused.
enum RowsEpilogue : int { kGelu = 0, kGeluGrad = 1 };

template <int TPL, typename V, int EPI>
__global__ __launch_bounds__(kBlock) void up_rows_kernel(const float* __restrict__ x_t, const int32_t* __restrict__ off,
                                                        const int16_t* __restrict__ idx, const V* __restrict__ w,
                                                        const float* __restrict__ b, float* __restrict__ act,
                                                        float* __restrict__ z, uint32_t h, uint32_t n, uint32_t ld) {
    const uint32_t r = blockIdx.x * kWaves + uniform(threadIdx.x / kWave);
    if (r >= h) return;
    const uint32_t t0 = (blockIdx.y * kWave + threadIdx.x % kWave) * TPL;
    if (t0 >= n) return;
    const int32_t begin = off[r], end = off[r + 1];
    const float* base = x_t + t0;
    float acc[TPL];
#pragma unroll
    for (int j = 0; j < TPL; ++j) acc[j] = 0.0f;
    int32_t e = begin;
    for (; e + 8 <= end; e += 8) {
        float xv[8][TPL];
        float wv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const uint32_t i = static_cast<uint16_t>(idx[e + u]);
            wv[u] = widen(w[e + u]);
            load_vec<TPL>(base + static_cast<size_t>(i) * ld, xv[u]);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
            for (int j = 0; j < TPL; ++j) acc[j] = fmaf(wv[u], xv[u][j], acc[j]);
    }
    for (; e < end; ++e) {
        const uint32_t i = static_cast<uint16_t>(idx[e]);
        const float wv = widen(w[e]);
        float xv[TPL];
        load_vec<TPL>(base + static_cast<size_t>(i) * ld, xv);
#pragma unroll
        for (int j = 0; j < TPL; ++j) acc[j] = fmaf(wv, xv[j], acc[j]);
    }
    float* out = act + static_cast<size_t>(r) * ld + t0;
    float* zr = z ? z + static_cast<size_t>(r) * ld + t0 : nullptr;
    if constexpr (EPI == kGelu) {
        const float bias = b[r];
#pragma unroll
        for (int j = 0; j < TPL; ++j)
            if (t0 + j < n) {
                const float pre = bias + acc[j];
                if (zr) zr[j] = pre;
                out[j] = gelu(pre);
            }
    } else {
#pragma unroll
        for (int j = 0; j < TPL; ++j)
            if (t0 + j < n) out[j] = acc[j] * gelu_grad(zr[j]);
    }
}

// ----------------------------------------------------------------------------------------- down, rows
template <int TPL, typename V>
__global__ __launch_bounds__(kBlock) void down_rows_kernel(const float* __restrict__ act, const int32_t* __restrict__ off,
                                                          const int16_t* __restrict__ hid, const V* __restrict__ v,
                                                          const float* __restrict__ bias, float* __restrict__ y_t,
                                                          uint32_t d, uint32_t n, uint32_t ld) {
    const uint32_t o = blockIdx.x * kWaves + uniform(threadIdx.x / kWave);
    if (o >= d) return;
    const uint32_t t0 = (blockIdx.y * kWave + threadIdx.x % kWave) * TPL;
    if (t0 >= n) return;
    const int32_t begin = off[o], end = off[o + 1];
    const float* base = act + t0;
    float acc[TPL];
#pragma unroll
    for (int j = 0; j < TPL; ++j) acc[j] = 0.0f;
    int32_t q = begin;
    for (; q + 8 <= end; q += 8) {
        float av[8][TPL];
        float vv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const uint32_t hh = static_cast<uint16_t>(hid[q + u]);
            vv[u] = widen(v[q + u]);
            load_vec<TPL>(base + static_cast<size_t>(hh) * ld, av[u]);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
            for (int j = 0; j < TPL; ++j) acc[j] = fmaf(vv[u], av[u][j], acc[j]);
    }
    for (; q < end; ++q) {
        const uint32_t hh = static_cast<uint16_t>(hid[q]);
        const float vv = widen(v[q]);
        float av[TPL];
        load_vec<TPL>(base + static_cast<size_t>(hh) * ld, av);
#pragma unroll
        for (int j = 0; j < TPL; ++j) acc[j] = fmaf(vv, av[j], acc[j]);
    }
    const float bo = bias ? bias[o] : 0.0f;  // no bias: the backward's gx
    float* out = y_t + static_cast<size_t>(o) * ld + t0;
#pragma unroll
    for (int j = 0; j < TPL; ++j)
        if (t0 + j < n) out[j] = acc[j] + bo;
}

// ------------------------------------------------------------------------------------------ transpose
__global__ __launch_bounds__(kBlock) void transpose_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                          uint32_t rows, uint32_t cols, uint32_t in_ld, uint32_t out_ld) {
    __shared__ float tile[64][65];
    const uint32_t r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
    const uint32_t tx = threadIdx.x % 64, ty = threadIdx.x / 64;
    for (uint32_t k = ty; k < 64; k += kWaves) {
        const uint32_t r = r0 + k, c = c0 + tx;
        if (r < rows && c < cols) tile[k][tx] = in[static_cast<size_t>(r) * in_ld + c];
    }
    __syncthreads();
    for (uint32_t k = ty; k < 64; k += kWaves) {
        const uint32_t c = c0 + k, r = r0 + tx;
        if (c < cols && r < rows) out[static_cast<size_t>(c) * out_ld + r] = tile[tx][k];
    }
}

uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

template <typename V, int EPI>
hipError_t up_rows_typed(const float* x_t, const int32_t* off, const int16_t* idx, const V* w, const float* b, float* act,
                         float* z, uint32_t h, uint32_t n, uint32_t ld, hipStream_t stream) {
    const dim3 block(kBlock);
    if (n >= 256) {
        hipLaunchKernelGGL((up_rows_kernel<4, V, EPI>), dim3(ceil_div(h, kWaves), ceil_div(n, 4 * kWave)), block, 0, stream, x_t, off, idx, w, b, act, z, h, n, ld);
    } else if (n >= 128) {
        hipLaunchKernelGGL((up_rows_kernel<2, V, EPI>), dim3(ceil_div(h, kWaves), ceil_div(n, 2 * kWave)), block, 0, stream, x_t, off, idx, w, b, act, z, h, n, ld);
    } else {
        hipLaunchKernelGGL((up_rows_kernel<1, V, EPI>), dim3(ceil_div(h, kWaves), ceil_div(n, kWave)), block, 0, stream, x_t, off, idx, w, b, act, z, h, n, ld);
    }
    return hipGetLastError();
}

template <typename V>
hipError_t down_rows_typed(const float* act, const int32_t* off, const int16_t* hid, const V* v, const float* bias, float* y_t,
                           uint32_t d, uint32_t n, uint32_t ld, hipStream_t stream) {
    const dim3 block(kBlock);
    if (n >= 256) {
        hipLaunchKernelGGL((down_rows_kernel<4, V>), dim3(ceil_div(d, kWaves), ceil_div(n, 4 * kWave)), block, 0, stream, act, off, hid, v, bias, y_t, d, n, ld);
    } else if (n >= 128) {
        hipLaunchKernelGGL((down_rows_kernel<2, V>), dim3(ceil_div(d, kWaves), ceil_div(n, 2 * kWave)), block, 0, stream, act, off, hid, v, bias, y_t, d, n, ld);
    } else {
        hipLaunchKernelGGL((down_rows_kernel<1, V>), dim3(ceil_div(d, kWaves), ceil_div(n, kWave)), block, 0, stream, act, off, hid, v, bias, y_t, d, n, ld);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_transpose(const float* in, float* out, uint32_t rows, uint32_t cols, uint32_t in_ld, uint32_t out_ld,
                            hipStream_t stream) {
    hipLaunchKernelGGL(transpose_kernel, dim3(ceil_div(cols, 64), ceil_div(rows, 64)), dim3(kBlock), 0, stream, in, out, rows,
                       cols, in_ld, out_ld);
    return hipGetLastError();
}

hipError_t launch_up_rows(int vt, const float* x_t, const int32_t* off, const int16_t* idx, const void* w, const float* b,
                          float* act, float* z, uint32_t, uint32_t h, uint32_t n, uint32_t ld, hipStream_t stream) {
    if (vt == kBF16) return up_rows_typed<uint16_t, kGelu>(x_t, off, idx, static_cast<const uint16_t*>(w), b, act, z, h, n, ld, stream);
    return up_rows_typed<float, kGelu>(x_t, off, idx, static_cast<const float*>(w), b, act, z, h, n, ld, stream);
}

hipError_t launch_grad_hidden_rows(const float* gy_t, const int32_t* off, const int16_t* idx, const float* v, const float* z,
                                   float* gz, uint32_t h, uint32_t n, uint32_t ld, hipStream_t stream) {
    return up_rows_typed<float, kGeluGrad>(gy_t, off, idx, v, nullptr, gz, const_cast<float*>(z), h, n, ld, stream);
}

hipError_t launch_down_rows(int vt, const float* act, const int32_t* off, const int16_t* hid, const void* v,
                            const float* bias, float* y_t, uint32_t d, uint32_t n, uint32_t ld, hipStream_t stream) {
    if (vt == kBF16) return down_rows_typed(act, off, hid, static_cast<const uint16_t*>(v), bias, y_t, d, n, ld, stream);
    return down_rows_typed(act, off, hid, static_cast<const float*>(v), bias, y_t, d, n, ld, stream);
}

}  // namespace hffn
