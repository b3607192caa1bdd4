// Decode-shaped ("edges") kernels of the HFFN forward on CDNA4: lanes over a row's slots, tokens in registers.
//
// Up:   act[r, t] = gelu(b_up[r] + sum_e w[e] x[t, idx[e]]),   one row per neuron r (up store).
// Down: y[t, o]   = b_down[o] + sum_q v[q] act[hid[q], t],     one row per output o (output-major store).
//
// A row is read as groups of consecutive slots per lane, each value load 16 bytes (1 KB of one contiguous range per
// wave instruction): float32 groups of 4 slots with an 8-byte index load, bfloat16 groups of 8 with a 16-byte index
// load (half the instructions of 4-slot groups: the 1.4B-shape pair at one token 14.0 -> 13.0 us). Groups are aligned
// to the group size, so a group may straddle the row's ends and its outside slots are skipped. A wave requests its
// first G groups per lane (1-3 rounds of 64 groups, from the average segment) before its block stages the
// inputs in LDS (by DMA, every transfer issued before any is waited for), so the store streams while the block waits:
// one memory round trip for the row offsets, then one for the slots and the inputs together.
// Long rows are split over P waves of the block (each takes a contiguous segment cut on the group grid); the P
// partial sums are added in segment order. Within a wave the 64 lane partials are added by a fixed xor butterfly. Inputs are
// staged in LDS when they fit (x for up, act for down at small n), otherwise act is gathered from L2.
// Tokens are processed NT at a time (NT = 1, 2, 4 or 8); every activation and output is written by one lane: no
// atomics, bitwise repeatable, and a token's result does not depend on the other tokens of the call.
#include <algorithm>

#include "common.hpp"
#include "edges.hpp"
#include "launch.hpp"

namespace hffn {
namespace {

using namespace edges;

constexpr uint32_t kBlock = 256;
constexpr uint32_t kWaves = kBlock / kWave;

// ------------------------------------------------------------------------------------------------- up
template <int NT, int P, typename V, int WAVES, bool GRAD, int G>
__global__ __launch_bounds__(WAVES * kWave) void up_edges_kernel(const float* __restrict__ x, const int32_t* __restrict__ off,
                                                                const int16_t* __restrict__ idx, const V* __restrict__ w,
                                                                const float* __restrict__ b, float* __restrict__ act,
                                                                float* __restrict__ z, uint32_t d, uint32_t h, uint32_t n,
                                                                uint32_t ld, int32_t nnz, uint32_t per_block) {
    extern __shared__ float smem[];  // x of NT tokens, [d][NT]; then the segment totals [WAVES][NT]
    float* xs = smem;
    float* totals = smem + static_cast<size_t>(d) * NT;
    constexpr uint32_t kRowsPerPass = WAVES / P;
    const uint32_t wave = uniform(threadIdx.x / kWave), lane = threadIdx.x % kWave;
    const uint32_t row_in_pass = wave / P, part = wave % P;
    const uint32_t r0 = blockIdx.x * per_block;
    const uint32_t r1 = min(h, r0 + per_block);
    for (uint32_t c0 = 0; c0 < n; c0 += NT) {
        const uint32_t tokens = min(n - c0, static_cast<uint32_t>(NT));
        // the first row's slots (and bias) are requested before the block stages x and waits for it
        Slots<V, G> cur;
        request_row<P>(cur, off, idx, w, r0 + row_in_pass, r1, part, nnz, lane);
        float b_cur = GRAD ? 0.0f : row_bias(b, r0 + row_in_pass, r1);
        if (c0) __syncthreads();
        stage_inputs<NT, WAVES>(xs, x + static_cast<size_t>(c0) * d, d, 1, d, tokens, wave, lane);
        wait_loads<0>();
        __syncthreads();
        const StagedInput input{xs};
        for (uint32_t base = r0; base < r1; base += kRowsPerPass) {  // uniform trip count across the block
            const uint32_t r = base + row_in_pass;
            // the wave's next row is requested before this row's sums, so its slots stream meanwhile
            Slots<V, G> next;
            request_row<P>(next, off, idx, w, r + kRowsPerPass, r1, part, nnz, lane);
            const float b_next = GRAD ? 0.0f : row_bias(b, r + kRowsPerPass, r1);
            float acc[NT];
            if (r < r1) {
                row_partials<NT>(cur.seg, idx, w, cur.pb, cur.pe, nnz, input, lane, acc);
            } else {
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
            }
            const float total = row_total<NT, P>(acc, lane, part, row_in_pass, totals);
            if (r < r1 && part == 0 && lane < tokens) {
                const size_t at = static_cast<size_t>(r) * ld + c0 + lane;
                if constexpr (GRAD) {  // the backward's gz: z holds the forward's pre-activations
                    act[at] = total * gelu_grad(z[at]);
                } else {
                    const float pre = b_cur + total;
                    if (z) z[at] = pre;  // the training forward keeps the pre-activation
                    act[at] = gelu(pre);
                }
            }
            cur = next;
            b_cur = b_next;
        }
    }
}

// ----------------------------------------------------------------------------------------------- down
template <int NT, int P, typename V, bool STAGE, int WAVES, int G>
__global__ __launch_bounds__(WAVES * kWave) void down_edges_kernel(const float* __restrict__ act, const int32_t* __restrict__ off,
                                                           const int16_t* __restrict__ hid, const V* __restrict__ v,
                                                           const float* __restrict__ bias, float* __restrict__ y, uint32_t d,
                                                           uint32_t h, uint32_t n, uint32_t ld, int32_t nnz, uint32_t per_block) {
    extern __shared__ float smem[];  // STAGE: act of NT tokens, [h][NT]; then the segment totals [WAVES][NT]
    float* as = smem;
    float* totals = smem + (STAGE ? static_cast<size_t>(h) * NT : 0);
    constexpr uint32_t kRowsPerPass = WAVES / P;
    const uint32_t wave = uniform(threadIdx.x / kWave), lane = threadIdx.x % kWave;
    const uint32_t row_in_pass = wave / P, part = wave % P;
    const uint32_t o0 = blockIdx.x * per_block;
    const uint32_t o1 = min(d, o0 + per_block);
    for (uint32_t c0 = 0; c0 < n; c0 += NT) {
        const uint32_t tokens = min(n - c0, static_cast<uint32_t>(NT));
        Slots<V, G> cur;
        request_row<P>(cur, off, hid, v, o0 + row_in_pass, o1, part, nnz, lane);
        float b_cur = row_bias(bias, o0 + row_in_pass, o1);
        if constexpr (STAGE) {
            if (c0) __syncthreads();
            stage_inputs<NT, WAVES>(as, act + c0, h, ld, 1, tokens, wave, lane);
            wait_loads<0>();
            __syncthreads();
        }
        for (uint32_t base = o0; base < o1; base += kRowsPerPass) {
            const uint32_t o = base + row_in_pass;
            Slots<V, G> next;
            request_row<P>(next, off, hid, v, o + kRowsPerPass, o1, part, nnz, lane);
            const float b_next = row_bias(bias, o + kRowsPerPass, o1);
            float acc[NT];
            if (o < o1) {
                if constexpr (STAGE) row_partials<NT>(cur.seg, hid, v, cur.pb, cur.pe, nnz, StagedInput{as}, lane, acc);
                else row_partials<NT>(cur.seg, hid, v, cur.pb, cur.pe, nnz, GlobalInput{act + c0, ld}, lane, acc);
            } else {
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
            }
            const float total = row_total<NT, P>(acc, lane, part, row_in_pass, totals);
            if (o < o1 && part == 0 && lane < tokens) y[static_cast<size_t>(c0 + lane) * d + o] = bias ? total + b_cur : total;
            cur = next;
            b_cur = b_next;
        }
    }
}

uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

// Waves per row: one per 512 slots of the average row, at most 4.
int parts_for(uint32_t nnz, uint32_t rows) {
    const uint32_t average = rows ? nnz / rows : 0;
    return average >= 1536 ? 4 : average >= 768 ? 2 : 1;
}

// Groups a lane holds at once: as many rounds of 64 groups as a wave's average segment takes, 1 to 3 (a longer
// segment's rest is loaded a chunk at a time after the first chunk's sums; a lane's group past its segment is a load
// of the store's group 0). The lanes meet their slots in the same order for any count: it does not change the bits.
template <typename V>
int groups_for(uint32_t nnz, uint32_t rows, int parts) {
    const uint64_t average = rows ? nnz / (static_cast<uint64_t>(rows) * parts) : 0, round = Group<V>::kSlots * kWave;
    return static_cast<int>(std::min<uint64_t>(3, std::max<uint64_t>(1, (average + round - 1) / round)));
}

// Rows per block: about `blocks` blocks, a multiple of the rows one pass of the block takes.
uint32_t rows_per_block(uint32_t rows, int parts, uint32_t waves = kWaves, uint32_t blocks = 1024) {
    const uint32_t pass = waves / parts;
    const uint32_t per = max(1u, ceil_div(rows, blocks));
    return ceil_div(per, pass) * pass;
}

// Up stages of more than 64 KB (wide d_model at 8 tokens) need the kernel's dynamic LDS limit raised (once per
// kernel: the limit is remembered per instantiation).
template <auto Kernel>
hipError_t allow_lds(size_t lds) {
    static size_t allowed = 65536;
    if (lds <= allowed) return hipSuccess;
    const hipError_t status = hipFuncSetAttribute(reinterpret_cast<const void*>(Kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                                  static_cast<int>(lds));
    if (status == hipSuccess) allowed = lds;
    return status;
}

// Every block stages x of its NT tokens (d * NT floats from L2): from 4 tokens on, blocks of 16 waves (a quarter as
// many blocks) cut that traffic by 4. Below 4 tokens a row of one wave (P = 1) is the wave's only row, so that no
// wave's second row waits behind its first: 4-wave blocks up to 4096 rows, 16-wave blocks above (at most 512 blocks
// staging x; on the 1.4B shape at one token 7.4 -> 6.3 us against two rows per wave of 4-wave blocks).
template <int NT, int P, typename V, int WAVES, bool GRAD, int G>
hipError_t up_launch(const float* x, const int32_t* off, const int16_t* idx, const V* w, const float* b, float* act, float* z, uint32_t d,
                     uint32_t h, uint32_t n, uint32_t ld, uint32_t nnz, hipStream_t stream) {
    const uint32_t per = NT < 4 && P == 1 ? WAVES : rows_per_block(h, P, WAVES, WAVES == kWaves ? 1024 : 256);
    const size_t lds = (static_cast<size_t>(d) * NT + WAVES * NT) * sizeof(float);
    if (const hipError_t status = allow_lds<up_edges_kernel<NT, P, V, WAVES, GRAD, G>>(lds); status != hipSuccess) return status;
    hipLaunchKernelGGL((up_edges_kernel<NT, P, V, WAVES, GRAD, G>), dim3(ceil_div(h, per)), dim3(WAVES * kWave), lds, stream, x, off, idx, w,
                       b, act, z, d, h, n, ld, static_cast<int32_t>(nnz), per);
    return hipGetLastError();
}

template <int NT, int P, typename V, int WAVES, bool GRAD>
hipError_t up_waves(const float* x, const int32_t* off, const int16_t* idx, const V* w, const float* b, float* act, float* z, uint32_t d,
                    uint32_t h, uint32_t n, uint32_t ld, uint32_t nnz, hipStream_t stream) {
    switch (groups_for<V>(nnz, h, P)) {
        case 1: return up_launch<NT, P, V, WAVES, GRAD, 1>(x, off, idx, w, b, act, z, d, h, n, ld, nnz, stream);
        case 2: return up_launch<NT, P, V, WAVES, GRAD, 2>(x, off, idx, w, b, act, z, d, h, n, ld, nnz, stream);
        default: return up_launch<NT, P, V, WAVES, GRAD, 3>(x, off, idx, w, b, act, z, d, h, n, ld, nnz, stream);
    }
}

template <int NT, int P, typename V, bool GRAD>
hipError_t up_shape(const float* x, const int32_t* off, const int16_t* idx, const V* w, const float* b, float* act, float* z,
                    uint32_t d, uint32_t h, uint32_t n, uint32_t ld, uint32_t nnz, hipStream_t stream) {
    if constexpr (NT >= 4) return up_waves<NT, P, V, 16, GRAD>(x, off, idx, w, b, act, z, d, h, n, ld, nnz, stream);
    else if (P == 1 && h > 4096) return up_waves<NT, P, V, 16, GRAD>(x, off, idx, w, b, act, z, d, h, n, ld, nnz, stream);
    else return up_waves<NT, P, V, kWaves, GRAD>(x, off, idx, w, b, act, z, d, h, n, ld, nnz, stream);
}

// With act staged in LDS (small n), blocks of 16 waves take 4x the rows of 4-wave blocks, so each block's staging
// of the whole act serves 4x the slots.
template <int NT, int P, typename V, int G>
hipError_t down_launch(const float* act, const int32_t* off, const int16_t* hid, const V* v, const float* bias, float* y,
                       uint32_t d, uint32_t h, uint32_t n, uint32_t ld, uint32_t nnz, hipStream_t stream) {
    const bool stage = static_cast<size_t>(h) * NT * sizeof(float) <= kEdgesStageBytes;
    if (stage) {
        constexpr uint32_t waves = 16;
        const uint32_t per = rows_per_block(d, P, waves, 256);
        const size_t lds = (static_cast<size_t>(h) * NT + waves * NT) * sizeof(float);
        if (const hipError_t status = allow_lds<down_edges_kernel<NT, P, V, true, waves, G>>(lds); status != hipSuccess) return status;
        hipLaunchKernelGGL((down_edges_kernel<NT, P, V, true, waves, G>), dim3(ceil_div(d, per)), dim3(waves * kWave), lds, stream,
                           act, off, hid, v, bias, y, d, h, n, ld, static_cast<int32_t>(nnz), per);
    } else {
        const uint32_t per = rows_per_block(d, P);
        const size_t lds = static_cast<size_t>(kWaves) * NT * sizeof(float);
        hipLaunchKernelGGL((down_edges_kernel<NT, P, V, false, kWaves, G>), dim3(ceil_div(d, per)), dim3(kBlock), lds, stream, act,
                           off, hid, v, bias, y, d, h, n, ld, static_cast<int32_t>(nnz), per);
    }
    return hipGetLastError();
}

template <int NT, int P, typename V>
hipError_t down_shape(const float* act, const int32_t* off, const int16_t* hid, const V* v, const float* bias, float* y,
                      uint32_t d, uint32_t h, uint32_t n, uint32_t ld, uint32_t nnz, hipStream_t stream) {
    switch (groups_for<V>(nnz, d, P)) {
        case 1: return down_launch<NT, P, V, 1>(act, off, hid, v, bias, y, d, h, n, ld, nnz, stream);
        case 2: return down_launch<NT, P, V, 2>(act, off, hid, v, bias, y, d, h, n, ld, nnz, stream);
        default: return down_launch<NT, P, V, 3>(act, off, hid, v, bias, y, d, h, n, ld, nnz, stream);
    }
}

template <int NT, typename V, bool GRAD>
hipError_t up_parts(int parts, const float* x, const int32_t* off, const int16_t* idx, const V* w, const float* b, float* act,
                    float* z, uint32_t d, uint32_t h, uint32_t n, uint32_t ld, uint32_t nnz, hipStream_t stream) {
    if (parts == 4) return up_shape<NT, 4, V, GRAD>(x, off, idx, w, b, act, z, d, h, n, ld, nnz, stream);
    if (parts == 2) return up_shape<NT, 2, V, GRAD>(x, off, idx, w, b, act, z, d, h, n, ld, nnz, stream);
    return up_shape<NT, 1, V, GRAD>(x, off, idx, w, b, act, z, d, h, n, ld, nnz, stream);
}

template <int NT, typename V>
hipError_t down_parts(int parts, const float* act, const int32_t* off, const int16_t* hid, const V* v, const float* bias,
                      float* y, uint32_t d, uint32_t h, uint32_t n, uint32_t ld, uint32_t nnz, hipStream_t stream) {
    if (parts == 4) return down_shape<NT, 4>(act, off, hid, v, bias, y, d, h, n, ld, nnz, stream);
    if (parts == 2) return down_shape<NT, 2>(act, off, hid, v, bias, y, d, h, n, ld, nnz, stream);
    return down_shape<NT, 1>(act, off, hid, v, bias, y, d, h, n, ld, nnz, stream);
}

template <typename V, bool GRAD = false>
hipError_t up_typed(const float* x, const int32_t* off, const int16_t* idx, const V* w, const float* b, float* act, float* z,
                    uint32_t d, uint32_t h, uint32_t n, uint32_t ld, uint32_t nnz, hipStream_t stream) {
    const int parts = parts_for(nnz, h);
    switch (edges_tokens(n)) {
        case 1: return up_parts<1, V, GRAD>(parts, x, off, idx, w, b, act, z, d, h, n, ld, nnz, stream);
        case 2: return up_parts<2, V, GRAD>(parts, x, off, idx, w, b, act, z, d, h, n, ld, nnz, stream);
        case 4: return up_parts<4, V, GRAD>(parts, x, off, idx, w, b, act, z, d, h, n, ld, nnz, stream);
        default: return up_parts<8, V, GRAD>(parts, x, off, idx, w, b, act, z, d, h, n, ld, nnz, stream);
    }
}

template <typename V>
hipError_t down_typed(const float* act, const int32_t* off, const int16_t* hid, const V* v, const float* bias, float* y,
                      uint32_t d, uint32_t h, uint32_t n, uint32_t ld, uint32_t nnz, hipStream_t stream) {
    const int parts = parts_for(nnz, d);
    switch (edges_tokens(n)) {
        case 1: return down_parts<1>(parts, act, off, hid, v, bias, y, d, h, n, ld, nnz, stream);
        case 2: return down_parts<2>(parts, act, off, hid, v, bias, y, d, h, n, ld, nnz, stream);
        case 4: return down_parts<4>(parts, act, off, hid, v, bias, y, d, h, n, ld, nnz, stream);
        default: return down_parts<8>(parts, act, off, hid, v, bias, y, d, h, n, ld, nnz, stream);
    }
}

}  // namespace

hipError_t launch_up_edges(int vt, const float* x, const int32_t* off, const int16_t* idx, const void* w, const float* b,
                           float* act, float* z, uint32_t d, uint32_t h, uint32_t n, uint32_t ld, uint32_t nnz, hipStream_t stream) {
    if (vt == kBF16) return up_typed(x, off, idx, static_cast<const uint16_t*>(w), b, act, z, d, h, n, ld, nnz, stream);
    return up_typed(x, off, idx, static_cast<const float*>(w), b, act, z, d, h, n, ld, nnz, stream);
}

hipError_t launch_grad_hidden_edges(const float* gy, const int32_t* off, const int16_t* idx, const float* v, const float* z,
                                    float* gz, uint32_t d, uint32_t h, uint32_t n, uint32_t ld, uint32_t nnz, hipStream_t stream) {
    return up_typed<float, true>(gy, off, idx, v, nullptr, gz, const_cast<float*>(z), d, h, n, ld, nnz, stream);
}

hipError_t launch_down_edges(int vt, const float* act, const int32_t* off, const int16_t* hid, const void* v,
                             const float* bias, float* y, uint32_t d, uint32_t h, uint32_t n, uint32_t ld, uint32_t nnz,
                             hipStream_t stream) {
    if (vt == kBF16) return down_typed(act, off, hid, static_cast<const uint16_t*>(v), bias, y, d, h, n, ld, nnz, stream);
    return down_typed(act, off, hid, static_cast<const float*>(v), bias, y, d, h, n, ld, nnz, stream);
}

}  // namespace hffn
