// Gather kernels of the HFFN forward on CDNA4 (wave64): up projection with fused bias + exact GELU,
// and the atomics-free down projection over the output-major store.
//
// Two shapes of each:
//  * "edges" (decode, n <= 8): one wave per neuron (up) or per output (down); the 64 lanes stride
//    that row's slots, every lane keeps one partial sum per token, and a fixed xor butterfly adds
//    the 64 partials. The input of the up kernel is staged in LDS (token-major), so each slot
//    costs one coalesced index/value load from HBM and n LDS reads.
//  * "rows" (n > 8): one wave per neuron/output; the lanes own consecutive tokens (TPL per lane,
//    vector loads), the wave walks the row's slots in order with wave-uniform index/value loads,
//    and each slot is one coalesced read of a feature-major input row.
// Every activation and every output is written by exactly one lane: no atomics, bitwise
// repeatable. Semantics follow runtime/gpu/nvidia/common/kernels/hffn_cuda/kernels.py:1-22.
#include "common.hpp"
#include "launch.hpp"

namespace hffn {
namespace {

constexpr uint32_t kBlock = 256;
constexpr uint32_t kWaves = kBlock / kWave;

// ------------------------------------------------------------------------------------------ up, edges
// Tokens are taken NT at a time (every n is valid; the policy uses this shape for n <= 8).
template <int NT, typename V>
__global__ __launch_bounds__(kBlock) void up_edges_kernel(const float* __restrict__ x, const int32_t* __restrict__ off,
                                                         const int16_t* __restrict__ idx, const V* __restrict__ w,
                                                         const float* __restrict__ b, float* __restrict__ act,
                                                         uint32_t d, uint32_t h, uint32_t n, uint32_t ld,
                                                         uint32_t per_block) {
    extern __shared__ float xs[];  // [NT][d]: tokens c0 .. c0 + NT - 1, rows past n are zero
    const uint32_t wave = uniform(threadIdx.x / kWave), lane = threadIdx.x % kWave;
    const uint32_t r0 = blockIdx.x * per_block;
    const uint32_t r1 = min(h, r0 + per_block);
    for (uint32_t c0 = 0; c0 < n; c0 += NT) {
        const uint32_t valid = min(n - c0, static_cast<uint32_t>(NT)) * d;
        const float* chunk = x + static_cast<size_t>(c0) * d;
        if (c0) __syncthreads();
        for (uint32_t i = threadIdx.x; i < NT * d; i += kBlock) xs[i] = i < valid ? chunk[i] : 0.0f;
        __syncthreads();
        for (uint32_t r = r0 + wave; r < r1; r += kWaves) {
            const int32_t begin = off[r], end = off[r + 1];
            float acc[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
            int32_t e = begin + static_cast<int32_t>(lane);
            for (; e + 3 * kWave < end; e += 4 * kWave) {
                uint32_t i[4];
                float wv[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    i[u] = static_cast<uint16_t>(idx[e + u * kWave]);
                    wv[u] = widen(w[e + u * kWave]);
                }
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int t = 0; t < NT; ++t) acc[t] = fmaf(wv[u], xs[t * d + i[u]], acc[t]);
            }
            for (; e < end; e += kWave) {
                const uint32_t i = static_cast<uint16_t>(idx[e]);
                const float wv = widen(w[e]);
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = fmaf(wv, xs[t * d + i], acc[t]);
            }
            float mine = 0.0f;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float s = wave_sum(acc[t]);
                if (lane == static_cast<uint32_t>(t)) mine = s;
            }
            if (lane < NT && c0 + lane < n) act[static_cast<size_t>(r) * ld + c0 + lane] = gelu(b[r] + mine);
        }
    }
}

// ------------------------------------------------------------------------------------------- up, rows
template <int TPL, typename V>
__global__ __launch_bounds__(kBlock) void up_rows_kernel(const float* __restrict__ x_t, const int32_t* __restrict__ off,
                                                        const int16_t* __restrict__ idx, const V* __restrict__ w,
                                                        const float* __restrict__ b, float* __restrict__ act,
                                                        uint32_t h, uint32_t n, uint32_t ld) {
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
    const float bias = b[r];
    float* out = act + static_cast<size_t>(r) * ld + t0;
#pragma unroll
    for (int j = 0; j < TPL; ++j)
        if (t0 + j < n) out[j] = gelu(bias + acc[j]);
}

// ---------------------------------------------------------------------------------------- down, edges
// Tokens NT at a time; act rows are read as NT-float vectors (ld is a multiple of NT).
template <int NT, typename V>
__global__ __launch_bounds__(kBlock) void down_edges_kernel(const float* __restrict__ act, const int32_t* __restrict__ off,
                                                           const int16_t* __restrict__ hid, const V* __restrict__ v,
                                                           const float* __restrict__ bias, float* __restrict__ y,
                                                           uint32_t d, uint32_t n, uint32_t ld, uint32_t per_block) {
    const uint32_t wave = uniform(threadIdx.x / kWave), lane = threadIdx.x % kWave;
    const uint32_t o0 = blockIdx.x * per_block;
    const uint32_t o1 = min(d, o0 + per_block);
    for (uint32_t o = o0 + wave; o < o1; o += kWaves) {
        const int32_t begin = off[o], end = off[o + 1];
        const float bo = bias[o];
        for (uint32_t c0 = 0; c0 < n; c0 += NT) {
            const float* base = act + c0;
            float acc[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
            int32_t q = begin + static_cast<int32_t>(lane);
            for (; q + kWave < end; q += 2 * kWave) {
                const uint32_t h0 = static_cast<uint16_t>(hid[q]), h1 = static_cast<uint16_t>(hid[q + kWave]);
                const float v0 = widen(v[q]), v1 = widen(v[q + kWave]);
                float a0[NT], a1[NT];
                load_vec<NT>(base + static_cast<size_t>(h0) * ld, a0);
                load_vec<NT>(base + static_cast<size_t>(h1) * ld, a1);
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = fmaf(v0, a0[t], acc[t]);
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = fmaf(v1, a1[t], acc[t]);
            }
            if (q < end) {
                const uint32_t h0 = static_cast<uint16_t>(hid[q]);
                const float v0 = widen(v[q]);
                float a0[NT];
                load_vec<NT>(base + static_cast<size_t>(h0) * ld, a0);
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = fmaf(v0, a0[t], acc[t]);
            }
            float mine = 0.0f;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float s = wave_sum(acc[t]);
                if (lane == static_cast<uint32_t>(t)) mine = s;
            }
            if (lane < NT && c0 + lane < n) y[static_cast<size_t>(c0 + lane) * d + o] = mine + bo;
        }
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
    const float bo = bias[o];
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

// Rows per block of the edges kernels: about 1024 blocks, a multiple of the 4 waves.
uint32_t rows_per_block(uint32_t rows) {
    uint32_t per = ceil_div(rows, 1024);
    return ceil_div(per, kWaves) * kWaves;
}

template <typename V>
hipError_t up_edges_typed(const float* x, const int32_t* off, const int16_t* idx, const V* w, const float* b, float* act,
                          uint32_t d, uint32_t h, uint32_t n, uint32_t ld, hipStream_t stream) {
    const uint32_t per = rows_per_block(h);
    const dim3 grid(ceil_div(h, per)), block(kBlock);
    if (n <= 1) {
        hipLaunchKernelGGL((up_edges_kernel<1, V>), grid, block, 1 * d * sizeof(float), stream, x, off, idx, w, b, act, d, h, n, ld, per);
    } else if (n <= 2) {
        hipLaunchKernelGGL((up_edges_kernel<2, V>), grid, block, 2 * d * sizeof(float), stream, x, off, idx, w, b, act, d, h, n, ld, per);
    } else if (n <= 4) {
        hipLaunchKernelGGL((up_edges_kernel<4, V>), grid, block, 4 * d * sizeof(float), stream, x, off, idx, w, b, act, d, h, n, ld, per);
    } else {
        hipLaunchKernelGGL((up_edges_kernel<8, V>), grid, block, 8 * d * sizeof(float), stream, x, off, idx, w, b, act, d, h, n, ld, per);
    }
    return hipGetLastError();
}

template <typename V>
hipError_t up_rows_typed(const float* x_t, const int32_t* off, const int16_t* idx, const V* w, const float* b, float* act,
                         uint32_t h, uint32_t n, uint32_t ld, hipStream_t stream) {
    const dim3 block(kBlock);
    if (n >= 256) {
        hipLaunchKernelGGL((up_rows_kernel<4, V>), dim3(ceil_div(h, kWaves), ceil_div(n, 4 * kWave)), block, 0, stream, x_t, off, idx, w, b, act, h, n, ld);
    } else if (n >= 128) {
        hipLaunchKernelGGL((up_rows_kernel<2, V>), dim3(ceil_div(h, kWaves), ceil_div(n, 2 * kWave)), block, 0, stream, x_t, off, idx, w, b, act, h, n, ld);
    } else {
        hipLaunchKernelGGL((up_rows_kernel<1, V>), dim3(ceil_div(h, kWaves), ceil_div(n, kWave)), block, 0, stream, x_t, off, idx, w, b, act, h, n, ld);
    }
    return hipGetLastError();
}

template <typename V>
hipError_t down_edges_typed(const float* act, const int32_t* off, const int16_t* hid, const V* v, const float* bias, float* y,
                            uint32_t d, uint32_t n, uint32_t ld, hipStream_t stream) {
    const uint32_t per = rows_per_block(d);
    const dim3 grid(ceil_div(d, per)), block(kBlock);
    if (n <= 1) {
        hipLaunchKernelGGL((down_edges_kernel<1, V>), grid, block, 0, stream, act, off, hid, v, bias, y, d, n, ld, per);
    } else if (n <= 2) {
        hipLaunchKernelGGL((down_edges_kernel<2, V>), grid, block, 0, stream, act, off, hid, v, bias, y, d, n, ld, per);
    } else if (n <= 4) {
        hipLaunchKernelGGL((down_edges_kernel<4, V>), grid, block, 0, stream, act, off, hid, v, bias, y, d, n, ld, per);
    } else {
        hipLaunchKernelGGL((down_edges_kernel<8, V>), grid, block, 0, stream, act, off, hid, v, bias, y, d, n, ld, per);
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

hipError_t launch_up_edges(int vt, const float* x, const int32_t* off, const int16_t* idx, const void* w, const float* b,
                           float* act, uint32_t d, uint32_t h, uint32_t n, uint32_t ld, hipStream_t stream) {
    if (vt == kBF16) return up_edges_typed(x, off, idx, static_cast<const uint16_t*>(w), b, act, d, h, n, ld, stream);
    return up_edges_typed(x, off, idx, static_cast<const float*>(w), b, act, d, h, n, ld, stream);
}

hipError_t launch_up_rows(int vt, const float* x_t, const int32_t* off, const int16_t* idx, const void* w, const float* b,
                          float* act, uint32_t, uint32_t h, uint32_t n, uint32_t ld, hipStream_t stream) {
    if (vt == kBF16) return up_rows_typed(x_t, off, idx, static_cast<const uint16_t*>(w), b, act, h, n, ld, stream);
    return up_rows_typed(x_t, off, idx, static_cast<const float*>(w), b, act, h, n, ld, stream);
}

hipError_t launch_down_edges(int vt, const float* act, const int32_t* off, const int16_t* hid, const void* v,
                             const float* bias, float* y, uint32_t d, uint32_t n, uint32_t ld, hipStream_t stream) {
    if (vt == kBF16) return down_edges_typed(act, off, hid, static_cast<const uint16_t*>(v), bias, y, d, n, ld, stream);
    return down_edges_typed(act, off, hid, static_cast<const float*>(v), bias, y, d, n, ld, stream);
}

hipError_t launch_down_rows(int vt, const float* act, const int32_t* off, const int16_t* hid, const void* v,
                            const float* bias, float* y_t, uint32_t d, uint32_t n, uint32_t ld, hipStream_t stream) {
    if (vt == kBF16) return down_rows_typed(act, off, hid, static_cast<const uint16_t*>(v), bias, y_t, d, n, ld, stream);
    return down_rows_typed(act, off, hid, static_cast<const float*>(v), bias, y_t, d, n, ld, stream);
}

}  // namespace hffn
