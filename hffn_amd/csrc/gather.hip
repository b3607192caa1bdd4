// Lane-per-token ("rows") gather kernels of the HFFN forward on CDNA4 (wave64), and the layout transpose:
// up projection with fused bias + exact GELU, and the atomics-free down projection over the output-major store.
// One wave per neuron/output; the lanes own consecutive tokens (TPL per lane, vector loads), the wave walks the row's
// slots in order, and each slot is one coalesced read of a feature-major input row. The slots' indices and values
// are read 64 at a time (one coalesced load per lane) and broadcast from their lanes, and the input rows of a batch of
// slots are all requested before the first is used: a walk costs a memory round trip per batch, not per slot, while
// each output stays the sequential sum in stored slot order. (The lane-per-slot decode shapes are in edges.hip.)
// Every activation and every output is written by exactly one lane: no atomics, bitwise
// repeatable. Semantics follow runtime/gpu/nvidia/common/kernels/hffn_cuda/kernels.py:1-22.
#include "common.hpp"
#include "launch.hpp"

namespace hffn {
namespace {

constexpr uint32_t kBlock = 256;
constexpr uint32_t kWaves = kBlock / kWave;

// The wave's walk of one row's slots [begin, end) for the TPL tokens of each lane (base: the lane's first token in the
// feature-major input, rows ld apart). Lane l holds slot e0 + l of the current 64 (the next 64 are requested after the
// first batch's inputs); a batch takes kBatch slots, broadcasting each slot's index from its lane, requesting every
// input row of the batch, then adding the products one slot after the other in stored order. A slot past the row's end
// repeats the row's last slot and is not added.
template <int TPL, typename V>
__device__ __forceinline__ void walk_row(const float* __restrict__ base, const int16_t* __restrict__ idx, const V* __restrict__ w,
                                         int32_t begin, int32_t end, uint32_t ld, uint32_t lane, float (&acc)[TPL]) {
    constexpr int32_t kBatch = TPL == 4 ? 16 : 32;
#pragma unroll
    for (int j = 0; j < TPL; ++j) acc[j] = 0.0f;
    if (begin >= end) return;
    const int32_t last = end - 1;
    int32_t at = min(begin + static_cast<int32_t>(lane), last);
    int32_t my_i = static_cast<uint16_t>(idx[at]);
    float my_w = widen(w[at]);
    for (int32_t e0 = begin; e0 < end; e0 += kWave) {
        const int32_t count = min(static_cast<int32_t>(kWave), end - e0);
        float xv[kBatch][TPL];
        auto request = [&](int32_t u0) {
#pragma unroll
            for (int32_t u = 0; u < kBatch; ++u) {
                const uint32_t i = static_cast<uint32_t>(__builtin_amdgcn_readlane(my_i, min(u0 + u, count - 1)));
                load_vec<TPL>(base + static_cast<size_t>(i) * ld, xv[u]);
            }
        };
        auto add = [&](int32_t u0) {
#pragma unroll
            for (int32_t u = 0; u < kBatch; ++u)
                if (u0 + u < count) {
                    const float wv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_w), u0 + u));
#pragma unroll
                    for (int j = 0; j < TPL; ++j) acc[j] = fmaf(wv, xv[u][j], acc[j]);
                }
        };
        request(0);
        at = min(e0 + static_cast<int32_t>(kWave + lane), last);  // the next 64 slots, behind the first batch's inputs
        const int32_t next_i = static_cast<uint16_t>(idx[at]);
        const float next_w = widen(w[at]);
        add(0);
        for (int32_t u0 = kBatch; u0 < count; u0 += kBatch) {
            request(u0);
            add(u0);
        }
        my_i = next_i;
        my_w = next_w;
    }
}

// The same walk for one token per lane, pipelined over chunks of 64 slots: lane l holds slot c0 + l's index and
// weight; chunk k + 1's input rows and chunk k + 2's slots are requested before chunk k's products are added, so each
// chunk costs one memory round trip, overlapped with the previous chunk's adds (two chunks of inputs in registers,
// 128 VGPRs: the lane-per-token kernels run few waves per CU). The sum is the same running sum in stored slot order.
template <typename V>
__device__ __forceinline__ float walk_row_pipelined(const float* __restrict__ base, const int16_t* __restrict__ idx,
                                                    const V* __restrict__ w, int32_t begin, int32_t end, uint32_t ld,
                                                    uint32_t lane) {
    float acc = 0.0f;
    if (begin >= end) return acc;
    const int32_t last = end - 1;
    const auto slot = [&](int32_t c0) { return min(c0 + static_cast<int32_t>(lane), last); };
    const auto request = [&](float (&xv)[kWave], int32_t my_i, int32_t c0) {
        const int32_t count = min(static_cast<int32_t>(kWave), end - c0);
#pragma unroll
        for (int32_t u = 0; u < kWave; ++u) {
            const uint32_t i = static_cast<uint32_t>(__builtin_amdgcn_readlane(my_i, min(u, count - 1)));
            xv[u] = base[static_cast<size_t>(i) * ld];
        }
    };
    const auto add = [&](const float (&xv)[kWave], float my_w, int32_t c0) {
        const int32_t count = min(static_cast<int32_t>(kWave), end - c0);
#pragma unroll
        for (int32_t u = 0; u < kWave; ++u)
            if (u < count) acc = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_w), u)), xv[u], acc);
    };
    float xa[kWave], xb[kWave];
    int32_t c0 = begin;
    int32_t i_a = static_cast<uint16_t>(idx[slot(c0)]);
    float w_a = widen(w[slot(c0)]);
    request(xa, i_a, c0);
    int32_t i_b = static_cast<uint16_t>(idx[slot(c0 + kWave)]);  // the next chunk's slots, behind this chunk's inputs
    float w_b = widen(w[slot(c0 + kWave)]);
    while (true) {
        // chunk c0's inputs requested into xa (its weights w_a), the next chunk's slots into (i_b, w_b)
        const bool more = c0 + kWave < end;
        int32_t i_c = 0;
        float w_c = 0.0f;
        if (more) {
            request(xb, i_b, c0 + kWave);
            i_c = static_cast<uint16_t>(idx[slot(c0 + 2 * kWave)]);
            w_c = widen(w[slot(c0 + 2 * kWave)]);
        }
        add(xa, w_a, c0);
        if (!more) break;
        c0 += kWave;
        // chunk c0's inputs in xb (weights w_b), the next chunk's slots in (i_c, w_c): the same with the buffers' roles
        // exchanged
        const bool again = c0 + kWave < end;
        int32_t i_d = 0;
        float w_d = 0.0f;
        if (again) {
            request(xa, i_c, c0 + kWave);
            i_d = static_cast<uint16_t>(idx[slot(c0 + 2 * kWave)]);
            w_d = widen(w[slot(c0 + 2 * kWave)]);
        }
        add(xb, w_b, c0);
        if (!again) break;
        c0 += kWave;
        w_a = w_c;  // chunk c0's inputs in xa, requested with i_c
        i_b = i_d;
        w_b = w_d;
    }
    return acc;
}

// ------------------------------------------------------------------------------------------- up, rows
// EPI kGelu: act = gelu(b + acc), and z = b + acc where z is not null (the training forward keeps it). EPI kGeluGrad
// (the backward's gz): act = acc * gelu'(z), z read, b unused.
enum RowsEpilogue : int { kGelu = 0, kGeluGrad = 1 };

template <int TPL, typename V, int EPI, bool PIPE = false>
__global__ __launch_bounds__(kBlock) void up_rows_kernel(const float* __restrict__ x_t, const int32_t* __restrict__ off,
                                                        const int16_t* __restrict__ idx, const V* __restrict__ w,
                                                        const float* __restrict__ b, float* __restrict__ act,
                                                        float* __restrict__ z, uint32_t h, uint32_t n, uint32_t ld) {
    static_assert(!PIPE || TPL == 1, "the pipelined walk takes one token per lane");
    const uint32_t r = blockIdx.x * kWaves + uniform(threadIdx.x / kWave);
    if (r >= h) return;
    // every lane walks (the slots are spread over the wave's lanes); a lane past the tokens reads token 0 and stores nothing
    const uint32_t t0 = (blockIdx.y * kWave + threadIdx.x % kWave) * TPL;
    const bool live = t0 < n;
    const float bias = EPI == kGelu ? b[r] : 0.0f;  // requested with the row's first slots
    float acc[TPL];
    if constexpr (PIPE) acc[0] = walk_row_pipelined(x_t + (live ? t0 : 0), idx, w, off[r], off[r + 1], ld, threadIdx.x % kWave);
    else walk_row<TPL>(x_t + (live ? t0 : 0), idx, w, off[r], off[r + 1], ld, threadIdx.x % kWave, acc);
    if (!live) return;
    float* out = act + static_cast<size_t>(r) * ld + t0;
    float* zr = z ? z + static_cast<size_t>(r) * ld + t0 : nullptr;
    if constexpr (EPI == kGelu) {
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
template <int TPL, typename V, bool PIPE = false>
__global__ __launch_bounds__(kBlock) void down_rows_kernel(const float* __restrict__ act, const int32_t* __restrict__ off,
                                                          const int16_t* __restrict__ hid, const V* __restrict__ v,
                                                          const float* __restrict__ bias, float* __restrict__ y,
                                                          uint32_t d, uint32_t n, uint32_t ld, uint32_t os, uint32_t ts) {
    static_assert(!PIPE || TPL == 1, "the pipelined walk takes one token per lane");
    const uint32_t o = blockIdx.x * kWaves + uniform(threadIdx.x / kWave);
    if (o >= d) return;
    const uint32_t t0 = (blockIdx.y * kWave + threadIdx.x % kWave) * TPL;
    const bool live = t0 < n;
    const float bo = bias ? bias[o] : 0.0f;  // no bias: the backward's gx; requested with the row's first slots
    float acc[TPL];
    if constexpr (PIPE) acc[0] = walk_row_pipelined(act + (live ? t0 : 0), hid, v, off[o], off[o + 1], ld, threadIdx.x % kWave);
    else walk_row<TPL>(act + (live ? t0 : 0), hid, v, off[o], off[o + 1], ld, threadIdx.x % kWave, acc);
    if (!live) return;
    float* out = y + static_cast<size_t>(o) * os + static_cast<size_t>(t0) * ts;  // y[o, t] at o os + t ts
#pragma unroll
    for (int j = 0; j < TPL; ++j)
        if (t0 + j < n) out[static_cast<size_t>(j) * ts] = acc[j] + bo;
}

// ------------------------------------------------------------------------------------------ transpose
// out[c, r] = in[r, c] through an LDS tile of kTransRows x kTransCols (padded by one float per row). A full tile whose
// rows start on 16-byte boundaries on both sides (strides multiples of 4 floats, aligned pointers) moves float4s: thread
// t reads 16 bytes of input rows t / 16 and t / 16 + 16 (16 threads per 256-byte row run) and writes 16 bytes of output
// rows t / 8 and t / 8 + 32 (4 input rows each), every load issued before the first LDS write; any other tile moves
// floats. 256 blocks for a 512 x 1024 transpose, one per CU.
constexpr uint32_t kTransRows = 32, kTransCols = 64;
__global__ __launch_bounds__(kBlock) void transpose_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                          uint32_t rows, uint32_t cols, uint32_t in_ld, uint32_t out_ld,
                                                          uint32_t vectors) {
    static_assert(kBlock == 256 && kTransRows * kTransCols / 4 == 2 * kBlock, "two float4 per thread each way");
    __shared__ float tile[kTransRows][kTransCols + 1];
    const uint32_t r0 = blockIdx.y * kTransRows, c0 = blockIdx.x * kTransCols, t = threadIdx.x;
    if (vectors && r0 + kTransRows <= rows && c0 + kTransCols <= cols) {
        float4 v[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t r = t / 16 + 16 * j, c = (t % 16) * 4;
            v[j] = *reinterpret_cast<const float4*>(in + static_cast<size_t>(r0 + r) * in_ld + c0 + c);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t r = t / 16 + 16 * j, c = (t % 16) * 4;
            tile[r][c] = v[j].x;
            tile[r][c + 1] = v[j].y;
            tile[r][c + 2] = v[j].z;
            tile[r][c + 3] = v[j].w;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t c = t / 8 + 32 * j, r = (t % 8) * 4;
            const float4 w = make_float4(tile[r][c], tile[r + 1][c], tile[r + 2][c], tile[r + 3][c]);
            *reinterpret_cast<float4*>(out + static_cast<size_t>(c0 + c) * out_ld + r0 + r) = w;
        }
        return;
    }
    for (uint32_t k = t; k < kTransRows * kTransCols; k += kBlock) {
        const uint32_t r = k / kTransCols, c = k % kTransCols;
        if (r0 + r < rows && c0 + c < cols) tile[r][c] = in[static_cast<size_t>(r0 + r) * in_ld + c0 + c];
    }
    __syncthreads();
    for (uint32_t k = t; k < kTransRows * kTransCols; k += kBlock) {
        const uint32_t c = k / kTransRows, r = k % kTransRows;
        if (c0 + c < cols && r0 + r < rows) out[static_cast<size_t>(c0 + c) * out_ld + r0 + r] = tile[r][c];
    }
}

uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

// Below 256 tokens: the pipelined walk (one token per lane) where the grid's waves fit one round at its occupancy (3
// waves per SIMD on 256 CUs, 150 VGPRs): there each wave's chain of round trips bounds the kernel (the 70M layer's 512
// outputs at 128 tokens: its down kernel 1024 waves, the call 44.1 -> 38.9 us); with more waves the plain walk's
// occupancy (8 per SIMD) hides the latency better (the 1.4B layer at 128 tokens: 222 us plain, 267 us pipelined).
// Two tokens per lane pipelined in 32-slot chunks, where only that grid fits one round, measured slower (the 410M
// outputs at 200 tokens 259 -> 281 us, the 1.4B outputs at 128 tokens 221 -> 242 us) or no faster (the 70M neurons at 128).
constexpr uint64_t kPipelinedWaves = 3 * 4 * 256;
bool pipelined(uint32_t rows, uint32_t n) { return static_cast<uint64_t>(rows) * ceil_div(n, kWave) <= kPipelinedWaves; }

template <typename V, int EPI>
hipError_t up_rows_typed(const float* x_t, const int32_t* off, const int16_t* idx, const V* w, const float* b, float* act,
                         float* z, uint32_t h, uint32_t n, uint32_t ld, hipStream_t stream) {
    const dim3 block(kBlock);
    if (n >= 256) {
        hipLaunchKernelGGL((up_rows_kernel<4, V, EPI>), dim3(ceil_div(h, kWaves), ceil_div(n, 4 * kWave)), block, 0, stream, x_t, off, idx, w, b, act, z, h, n, ld);
    } else if (pipelined(h, n)) {
        hipLaunchKernelGGL((up_rows_kernel<1, V, EPI, true>), dim3(ceil_div(h, kWaves), ceil_div(n, kWave)), block, 0, stream, x_t, off, idx, w, b, act, z, h, n, ld);
    } else if (n >= 128) {
        hipLaunchKernelGGL((up_rows_kernel<2, V, EPI>), dim3(ceil_div(h, kWaves), ceil_div(n, 2 * kWave)), block, 0, stream, x_t, off, idx, w, b, act, z, h, n, ld);
    } else {
        hipLaunchKernelGGL((up_rows_kernel<1, V, EPI>), dim3(ceil_div(h, kWaves), ceil_div(n, kWave)), block, 0, stream, x_t, off, idx, w, b, act, z, h, n, ld);
    }
    return hipGetLastError();
}

template <typename V>
hipError_t down_rows_typed(const float* act, const int32_t* off, const int16_t* hid, const V* v, const float* bias, float* y_t,
                           uint32_t d, uint32_t n, uint32_t ld, uint32_t os, uint32_t ts, hipStream_t stream) {
    const dim3 block(kBlock);
    if (n >= 256) {
        hipLaunchKernelGGL((down_rows_kernel<4, V>), dim3(ceil_div(d, kWaves), ceil_div(n, 4 * kWave)), block, 0, stream, act, off, hid, v, bias, y_t, d, n, ld, os, ts);
    } else if (pipelined(d, n)) {
        hipLaunchKernelGGL((down_rows_kernel<1, V, true>), dim3(ceil_div(d, kWaves), ceil_div(n, kWave)), block, 0, stream, act, off, hid, v, bias, y_t, d, n, ld, os, ts);
    } else if (n >= 128) {
        hipLaunchKernelGGL((down_rows_kernel<2, V>), dim3(ceil_div(d, kWaves), ceil_div(n, 2 * kWave)), block, 0, stream, act, off, hid, v, bias, y_t, d, n, ld, os, ts);
    } else {
        hipLaunchKernelGGL((down_rows_kernel<1, V>), dim3(ceil_div(d, kWaves), ceil_div(n, kWave)), block, 0, stream, act, off, hid, v, bias, y_t, d, n, ld, os, ts);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_transpose(const float* in, float* out, uint32_t rows, uint32_t cols, uint32_t in_ld, uint32_t out_ld,
                            hipStream_t stream) {
    const uint32_t vectors = in_ld % 4 == 0 && out_ld % 4 == 0 && reinterpret_cast<uintptr_t>(in) % 16 == 0 &&
                             reinterpret_cast<uintptr_t>(out) % 16 == 0;
    hipLaunchKernelGGL(transpose_kernel, dim3(ceil_div(cols, kTransCols), ceil_div(rows, kTransRows)), dim3(kBlock), 0, stream, in,
                       out, rows, cols, in_ld, out_ld, vectors);
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
                            const float* bias, float* y, uint32_t d, uint32_t n, uint32_t ld, hipStream_t stream, bool token_major) {
    const uint32_t os = token_major ? 1 : ld, ts = token_major ? d : 1;  // y [n, d] or [d, ld]
    if (vt == kBF16) return down_rows_typed(act, off, hid, static_cast<const uint16_t*>(v), bias, y, d, n, ld, os, ts, stream);
    return down_rows_typed(act, off, hid, static_cast<const float*>(v), bias, y, d, n, ld, os, ts, stream);
}

}  // namespace hffn
