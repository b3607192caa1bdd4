// Decode-sized projections straight from the compact store (gfx950, wave64): 1-64 tokens, every stored slot read from
// HBM once per call, the dot products on MFMA over tiles densified in LDS.
//
// A side has R rows (up: the d_ff neurons over K = d_model inputs; down: the d_model outputs of the output-major store
// over K = d_ff neurons), each row's slots sorted by index. A block takes a tile of 16 rows and one 1024-wide chunk of
// K (blockIdx.y); an index table built at load gives each row's first slot in every chunk (tiles_index_kernel). The
// block
//   1. loads its rows' slots of the chunk (each wave two rows, lanes over slots) while it zero-fills the LDS tile;
//   2. scatters them into the dense tile [16 rows][1024 k]: float32 weights scaled by the power of two of their
//      row's largest magnitude in the chunk and split into fp16 hi and lo planes; bfloat16 weights as they are;
//   3. multiplies: each of the 8 waves takes 128 k of the chunk; per 32-k step lane (r, c) = (lane % 16, lane / 16)
//      reads row r's 8 weights at k-run c from LDS (the B operand) and token r's 8 inputs at the same k from global
//      memory (the A operand), for each 16-token tile. float32 weights: the inputs are scaled by the token's power of
//      two over the 32-k step and split into fp16 hi and lo, D = x_hi w_hi + x_hi w_lo + x_lo w_hi on
//      v_mfma_f32_16x16x32_f16, and the token's power of two is undone exactly. bfloat16 weights: each input is split
//      exactly into three bfloat16 parts (8 significant bits each, by truncation), D = (x_1 + x_2 + x_3) w on
//      v_mfma_f32_16x16x32_bf16, every product exact in fp32;
//   4. adds the 8 waves' sums in wave order (LDS), undoes the row's power of two, and writes the output with the
//      epilogue (bias, and GELU for the up side), or, when K spans several chunks, a partial per chunk that
//      tiles_reduce_kernel adds in chunk order before the epilogue.
// Every output is a fixed-order sum over fixed groups: no atomics, the bits repeat run to run and a token's result does
// not depend on the other tokens of the call. The inputs (x, or act for the down side) and outputs are token-major
// [n, K] and [n, R].
#include <algorithm>

#include "common.hpp"
#include "launch.hpp"

namespace hffn {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kRows = 16;                 // rows per tile: one MFMA operand width
constexpr uint32_t kChunk = kTilesChunk;       // k per block
constexpr uint32_t kWaves = 16;                // one row of the tile per wave
constexpr uint32_t kThreads = kWaves * kWave;
constexpr uint32_t kStep = 32;                 // k per MFMA
constexpr uint32_t kLdsRow = kChunk;           // halves per LDS row
constexpr uint32_t kGroups = (kChunk + 3 + 4 * kWave - 1) / (4 * kWave);  // 4-slot groups per lane: a row holds at
                                                                      // most kChunk slots of a chunk, plus alignment
constexpr uint32_t kWaveSteps = kChunk / 32 / kWaves;                  // 32-k steps per wave
constexpr uint32_t kTokenTile = 16;

template <typename V> struct TilePlanes;
template <> struct TilePlanes<float> { static constexpr uint32_t count = 2; };     // fp16 hi, lo
template <> struct TilePlanes<uint16_t> { static constexpr uint32_t count = 1; };  // bfloat16 bits

// Half offset of (row r, k) in a tile plane: the 16-byte runs of 8 k are XOR-swizzled by the row, so the 8 lanes of one
// LDS pass (rows r..r+7, the same run) read 8 distinct bank groups.
__device__ __forceinline__ uint32_t tile_at(uint32_t r, uint32_t k) { return r * kLdsRow + (((k >> 3) ^ (r & 7)) << 3) + (k & 7); }

__device__ __forceinline__ int binade_of(uint32_t magnitude_bits) {
    return magnitude_bits == 0 ? 0 : static_cast<int>((magnitude_bits >> 23) & 0xff) - 127;
}

// A row segment's slots of one chunk, loaded 4 at a time (16-byte fp32 / 8-byte bf16 value loads, 8-byte index loads):
// group j of lane l starts at slot (b & ~3) + 4 l + 256 j; the slots of a group outside [b, e) are ignored, and the
// store's last group, when it crosses nnz, is read slot by slot.
template <typename V> struct Quad;
template <> struct Quad<float> {
    using type = float4;
    __device__ static float at(const float4& q, int s) { return s == 0 ? q.x : s == 1 ? q.y : s == 2 ? q.z : q.w; }
};
template <> struct Quad<uint16_t> {
    using type = uint2;
    __device__ static float at(const uint2& q, int s) {
        const uint32_t word = s < 2 ? q.x : q.y;
        return __uint_as_float(s % 2 == 0 ? word << 16 : word & 0xffff0000u);
    }
};

__device__ __forceinline__ uint32_t quad_index(const uint2& q, int s) {
    const uint32_t word = s < 2 ? q.x : q.y;
    return s % 2 == 0 ? (word & 0xffffu) : (word >> 16);
}

template <typename V, int TT, bool UP>
__global__ __launch_bounds__(kThreads) void tiles_kernel(const float* __restrict__ in,           // [n, K]
                                                         const int16_t* __restrict__ idx,        // slots' k
                                                         const V* __restrict__ val,              // slots' weights
                                                         const int32_t* __restrict__ table,      // offsets, then binades
                                                         const float* __restrict__ bias,         // [R]
                                                         float* __restrict__ out,                // [n, R]
                                                         float* __restrict__ partials,           // [chunks, n, R]
                                                         uint32_t rows, uint32_t K, uint32_t n, int32_t nnz) {
    constexpr uint32_t kPlanes = TilePlanes<V>::count;
    constexpr uint32_t kTileHalves = kPlanes * kRows * kLdsRow;
    constexpr uint32_t kHalfSums = kWaves / 2 * TT * kTokenTile * kRows;  // floats of half the waves' sums
    // the tile, then (reusing its LDS) half the waves' sums followed by the row binades
    constexpr uint32_t kLdsBytes = (kTileHalves * 2 > kHalfSums * 4 + kRows * 4 ? kTileHalves * 2 : kHalfSums * 4 + kRows * 4);
    __shared__ __align__(16) unsigned char lds[kLdsBytes];
    uint16_t* tile = reinterpret_cast<uint16_t*>(lds);  // [plane][row][kLdsRow], swizzled runs
    float* sums = reinterpret_cast<float*>(lds);        // [wave % 8][token][row], after the products
    int* row_binade = reinterpret_cast<int*>(sums + kHalfSums);
    using Q = typename Quad<V>::type;

    const uint32_t lane = threadIdx.x % kWave, wave = uniform(threadIdx.x / kWave);
    const uint32_t chunks = gridDim.y, chunk = blockIdx.y;
    const uint32_t row0 = blockIdx.x * kRows, k0 = chunk * kChunk;
    const uint32_t width = min(kChunk, K - k0);  // k of this chunk (a multiple of 8)
    const uint32_t r = lane % 16, c = lane / 16;

    // 1. request the wave's first inputs and its row segment, zero the tile while they arrive
    const uint32_t row = row0 + wave;
    int32_t b = 0, e = 0, binade = 0;  // binade: the power of two of the segment's largest |weight| (float32 stores)
    if (row < rows) {
        b = table[static_cast<size_t>(row) * (chunks + 1) + chunk];
        e = table[static_cast<size_t>(row) * (chunks + 1) + chunk + 1];
        if constexpr (kPlanes == 2) binade = table[static_cast<size_t>(rows) * (chunks + 1) + static_cast<size_t>(row) * chunks + chunk];
    }
    const uint32_t steps = (width + kStep - 1) / kStep;
    const uint32_t per_wave = (steps + kWaves - 1) / kWaves;  // at most kWaveSteps
    const uint32_t s0 = min(steps, wave * per_wave), s1 = min(steps, s0 + per_wave);
    // The inputs of the wave's two 32-k steps: the first requested before the slots, the second after the scatter (when
    // the slot registers are free). Loaded without branches: an input outside the call (token >= n, k beyond the
    // chunk) loads x[0, 0..7] and is zeroed at use.
    auto request = [&](uint32_t q, float (&xv)[TT][8]) -> uint32_t {
        uint32_t live = 0;  // bit tt: token tile tt of step q is inside the call
        const uint32_t kk = (s0 + q) * kStep + c * 8;
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
            const uint32_t t = tt * kTokenTile + r;
            const bool inside = s0 + q < s1 && t < n && kk < width;
            live |= static_cast<uint32_t>(inside) << tt;
            load_vec<8>(in + (inside ? static_cast<size_t>(t) * K + k0 + kk : 0), xv[tt]);
        }
        return live;
    };
    float xv0[TT][8];
    const uint32_t live0 = request(0, xv0);
    const int32_t first = (b & ~3) + 4 * static_cast<int32_t>(lane);
    Q wq[kGroups];
    uint2 iq[kGroups];
#pragma unroll
    for (uint32_t j = 0; j < kGroups; ++j) {
        wq[j] = Q{};
        iq[j] = make_uint2(0, 0);
    }
    if (e + 4 <= nnz) {
        // Whole-group loads, all issued at once and without branches (a branch around each load makes the compiler wait
        // for it): a group past the segment reloads the segment's last group, (e & ~3) + 4 <= nnz, and is masked at use.
        const int32_t last = e & ~3;
#pragma unroll
        for (uint32_t j = 0; j < kGroups; ++j) {
            const int32_t g = min(first + static_cast<int32_t>(j * 4 * kWave), last);
            wq[j] = *reinterpret_cast<const Q*>(val + g);
            iq[j] = *reinterpret_cast<const uint2*>(idx + g);
        }
    } else {  // the segment ending within 4 slots of the store's end: slot by slot
#pragma unroll
        for (uint32_t j = 0; j < kGroups; ++j) {
            const int32_t g = first + static_cast<int32_t>(j * 4 * kWave);
            V v4[4] = {V(0), V(0), V(0), V(0)};
            uint16_t i4[4] = {0, 0, 0, 0};
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (g + q < e) {
                    v4[q] = val[g + q];
                    i4[q] = static_cast<uint16_t>(idx[g + q]);
                }
            wq[j] = *reinterpret_cast<const Q*>(v4);
            iq[j] = make_uint2(i4[0] | (static_cast<uint32_t>(i4[1]) << 16), i4[2] | (static_cast<uint32_t>(i4[3]) << 16));
        }
    }
    for (uint32_t i = threadIdx.x; i < kTileHalves / 8; i += kThreads) reinterpret_cast<uint4*>(tile)[i] = make_uint4(0, 0, 0, 0);
    __syncthreads();  // the tile is zero (this waits for the LDS only: the loads stay in flight)

    // 2. scatter the row into the tile, each group as its loads arrive
    const uint32_t groups = e > b ? static_cast<uint32_t>((e - (b & ~3) + 4 * kWave - 1) / (4 * kWave)) : 0;
#pragma unroll
    for (uint32_t j = 0; j < kGroups; ++j) {
        if (j >= groups) break;
        const int32_t g = first + static_cast<int32_t>(j * 4 * kWave);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t at = quad_index(iq[j], q) - k0;
            if (g + q >= b && g + q < e && at < width) {
                const float weight = Quad<V>::at(wq[j], q);
                if constexpr (kPlanes == 2) {
                    const float s = ldexpf(weight, -binade);
                    const _Float16 hi = static_cast<_Float16>(s);
                    const _Float16 lo = static_cast<_Float16>(s - static_cast<float>(hi));
                    tile[tile_at(wave, at)] = __builtin_bit_cast(uint16_t, hi);
                    tile[kRows * kLdsRow + tile_at(wave, at)] = __builtin_bit_cast(uint16_t, lo);
                } else {
                    tile[tile_at(wave, at)] = static_cast<uint16_t>(__float_as_uint(weight) >> 16);
                }
            }
        }
    }
    float xv1[TT][8];
    const uint32_t live1 = request(1, xv1);
    __syncthreads();

    // 3. products over the wave's two 32-k steps
    static_assert(kWaveSteps == 2, "two 32-k steps per wave");
    uint4 bh[2], bl[2];
#pragma unroll
    for (uint32_t q = 0; q < 2; ++q) {
        const uint16_t* b_at = tile + tile_at(r, min(s0 + q, steps - 1) * kStep + c * 8);
        bh[q] = *reinterpret_cast<const uint4*>(b_at);
        bl[q] = make_uint4(0, 0, 0, 0);
        if constexpr (kPlanes == 2) bl[q] = *reinterpret_cast<const uint4*>(b_at + kRows * kLdsRow);
    }
    floatx4 acc[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
        float v[2][8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[0][i] = (live0 >> tt) & 1u ? xv0[tt][i] : 0.0f;
            v[1][i] = (live1 >> tt) & 1u ? xv1[tt][i] : 0.0f;
        }
        if constexpr (kPlanes == 2) {
            // the token's power of two over the wave's 64 k: its inputs sit in lanes r, r + 16, r + 32, r + 48
            uint32_t m = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) m = max(m, max(__float_as_uint(v[0][i]), __float_as_uint(v[1][i])) & 0x7fffffffu);
            m = max(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), 16, kWave)));
            m = max(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), 32, kWave)));
            const int ex = binade_of(m);
            floatx4 d = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                half8 xh, xl;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float sv = ldexpf(v[q][i], -ex);
                    const _Float16 hv = static_cast<_Float16>(sv);
                    xh[i] = hv;
                    xl[i] = static_cast<_Float16>(sv - static_cast<float>(hv));
                }
                const half8 wh = __builtin_bit_cast(half8, bh[q]), wl = __builtin_bit_cast(half8, bl[q]);
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, wh, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, wl, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, wh, d, 0, 0, 0);
            }
            // D register i holds token 4c + i of the tile: undo its power of two (held by lane 4c + i)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[tt][i] = ldexpf(d[i], __shfl(ex, static_cast<int>(4 * c + i), kWave));
        } else {
            acc[tt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                uint32_t p1[4], p2[4], p3[4];  // pairs of bfloat16: the three parts of the 8 inputs
#pragma unroll
                for (int i = 0; i < 8; i += 2) {
                    uint32_t part[3][2];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const float x0 = v[q][i + h];
                        const uint32_t b1 = __float_as_uint(x0) & 0xffff0000u;
                        const float rest = x0 - __uint_as_float(b1);
                        const uint32_t b2 = __float_as_uint(rest) & 0xffff0000u;
                        const uint32_t b3 = __float_as_uint(rest - __uint_as_float(b2));  // <= 8 significant bits left
                        part[0][h] = b1 >> 16;
                        part[1][h] = b2 >> 16;
                        part[2][h] = b3 >> 16;
                    }
                    p1[i / 2] = part[0][0] | (part[0][1] << 16);
                    p2[i / 2] = part[1][0] | (part[1][1] << 16);
                    p3[i / 2] = part[2][0] | (part[2][1] << 16);
                }
                const bf16x8 wb = __builtin_bit_cast(bf16x8, bh[q]);
                acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, p1), wb, acc[tt], 0, 0, 0);
                acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, p2), wb, acc[tt], 0, 0, 0);
                acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, p3), wb, acc[tt], 0, 0, 0);
            }
        }
    }
    __syncthreads();  // the tile is read: its LDS now holds the waves' sums

    // 4. the 16 waves' sums in a fixed order (wave w + 8 into wave w, then waves 0..7), the row's power of two, then
    // the output or this chunk's partial
    const uint32_t half = wave % (kWaves / 2);
    float* mine = sums + half * TT * kTokenTile * kRows;
    if (wave >= kWaves / 2) {
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) mine[(tt * kTokenTile + 4 * c + i) * kRows + r] = acc[tt][i];
    }
    if (lane == 0) row_binade[wave] = binade;
    __syncthreads();
    if (wave < kWaves / 2) {
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float* cell = mine + (tt * kTokenTile + 4 * c + i) * kRows + r;
                *cell = acc[tt][i] + *cell;
            }
    }
    __syncthreads();
    for (uint32_t o = threadIdx.x; o < TT * kTokenTile * kRows; o += kThreads) {
        const uint32_t t = o / kRows, rr = o % kRows, out_row = row0 + rr;
        if (t >= n) break;
        if (out_row >= rows) continue;
        float s = sums[t * kRows + rr];
#pragma unroll
        for (uint32_t q = 1; q < kWaves / 2; ++q) s += sums[(q * TT * kTokenTile + t) * kRows + rr];
        s = ldexpf(s, row_binade[rr]);
        if (chunks > 1) {
            partials[(static_cast<size_t>(chunk) * n + t) * rows + out_row] = s;
        } else {
            const float z = s + bias[out_row];
            out[static_cast<size_t>(t) * rows + out_row] = UP ? gelu(z) : z;
        }
    }
}

// out[t, r] = epilogue(bias[r] + the chunks' partials added in chunk order); one thread per output.
template <bool UP>
__global__ __launch_bounds__(256) void tiles_reduce_kernel(const float* __restrict__ partials, uint32_t chunks,
                                                           const float* __restrict__ bias, float* __restrict__ out,
                                                           uint32_t rows, uint32_t n) {
    const uint32_t o = blockIdx.x * 256 + threadIdx.x;
    if (o >= n * rows) return;
    const size_t stride = static_cast<size_t>(n) * rows;
    float s = partials[o];
    for (uint32_t k = 1; k < chunks; ++k) s += partials[k * stride + o];
    const float z = s + bias[o % rows];
    out[o] = UP ? gelu(z) : z;
}

// The index table of one side: offsets[r][c] = the first slot of row r whose index is at least c * kChunk
// (c = 0 .. chunks), then, for float32 values, binades[r][c] = the power of two of the largest |weight| of row r's slots
// in chunk c (c < chunks; 0 for an empty segment). One thread per row.
template <typename V>
__global__ __launch_bounds__(256) void tiles_index_kernel(const int32_t* __restrict__ offsets, const int16_t* __restrict__ idx,
                                                          const V* __restrict__ val, uint32_t rows, uint32_t chunks,
                                                          int32_t* __restrict__ table) {
    const uint32_t r = blockIdx.x * 256 + threadIdx.x;
    if (r >= rows) return;
    const int32_t end = offsets[r + 1];
    int32_t lo = offsets[r];
    table[static_cast<size_t>(r) * (chunks + 1)] = lo;
    for (uint32_t c = 1; c <= chunks; ++c) {
        // the first slot in [lo, end) whose index reaches c * kChunk, else end (indices ascend within the row)
        int32_t a = lo, z = end;
        while (a < z) {
            const int32_t mid = a + (z - a) / 2;
            if (static_cast<uint32_t>(static_cast<uint16_t>(idx[mid])) < c * kChunk) a = mid + 1; else z = mid;
        }
        table[static_cast<size_t>(r) * (chunks + 1) + c] = a;
        if constexpr (sizeof(V) == 4) {
            uint32_t m = 0;
            for (int32_t s = lo; s < a; ++s) m = max(m, __float_as_uint(val[s]) & 0x7fffffffu);
            table[static_cast<size_t>(rows) * (chunks + 1) + static_cast<size_t>(r) * chunks + c - 1] = binade_of(m);
        }
        lo = a;
    }
}

uint32_t chunks_of(uint32_t K) { return (K + kChunk - 1) / kChunk; }

template <typename V, bool UP>
hipError_t tiles_side(const float* in, const int16_t* idx, const void* val, const int32_t* table, const float* bias, float* out,
                      float* partials, uint32_t rows, uint32_t K, uint32_t n, uint32_t nnz, hipStream_t stream) {
    const uint32_t chunks = chunks_of(K);
    const dim3 grid((rows + kRows - 1) / kRows, chunks), block(kThreads);
    const V* v = static_cast<const V*>(val);
    if (n <= kTokenTile)
        hipLaunchKernelGGL((tiles_kernel<V, 1, UP>), grid, block, 0, stream, in, idx, v, table, bias, out, partials, rows, K, n,
                           static_cast<int32_t>(nnz));
    else if (n <= 2 * kTokenTile)
        hipLaunchKernelGGL((tiles_kernel<V, 2, UP>), grid, block, 0, stream, in, idx, v, table, bias, out, partials, rows, K, n,
                           static_cast<int32_t>(nnz));
    else
        hipLaunchKernelGGL((tiles_kernel<V, 4, UP>), grid, block, 0, stream, in, idx, v, table, bias, out, partials, rows, K, n,
                           static_cast<int32_t>(nnz));
    if (hipError_t status = hipGetLastError(); status != hipSuccess || chunks == 1) return status;
    hipLaunchKernelGGL(tiles_reduce_kernel<UP>, dim3((n * rows + 255) / 256), dim3(256), 0, stream, partials, chunks, bias, out, rows, n);
    return hipGetLastError();
}

}  // namespace

uint32_t tiles_index_entries(uint32_t rows, uint32_t K) { return rows * (2 * chunks_of(K) + 1); }

size_t tiles_workspace_bytes(uint32_t n, uint32_t d, uint32_t h) {
    const size_t up = chunks_of(d) > 1 ? size_t(chunks_of(d)) * n * h : 0;
    const size_t down = chunks_of(h) > 1 ? size_t(chunks_of(h)) * n * d : 0;
    return std::max<size_t>(std::max(up, down) * sizeof(float), 256);
}

hipError_t launch_tiles_index(int vt, const int32_t* offsets, const int16_t* idx, const void* val, uint32_t rows, uint32_t K,
                              int32_t* table, hipStream_t stream) {
    const dim3 grid((rows + 255) / 256);
    if (vt == kBF16) {
        hipLaunchKernelGGL(tiles_index_kernel<uint16_t>, grid, dim3(256), 0, stream, offsets, idx, static_cast<const uint16_t*>(val), rows,
                           chunks_of(K), table);
    } else {
        hipLaunchKernelGGL(tiles_index_kernel<float>, grid, dim3(256), 0, stream, offsets, idx, static_cast<const float*>(val), rows,
                           chunks_of(K), table);
    }
    return hipGetLastError();
}

hipError_t launch_tiles_forward(int vt, const float* x, const int16_t* up_idx, const void* up_val, const int32_t* up_table,
                                const float* b_up, const int16_t* out_hidden, const void* out_val, const int32_t* down_table,
                                const float* b_down, float* act, float* work, float* y, uint32_t d, uint32_t h, uint32_t nnz_up,
                                uint32_t nnz_down, uint32_t n, hipStream_t stream) {
    const hipError_t status = vt == kBF16 ? tiles_side<uint16_t, true>(x, up_idx, up_val, up_table, b_up, act, work, h, d, n, nnz_up, stream)
                                          : tiles_side<float, true>(x, up_idx, up_val, up_table, b_up, act, work, h, d, n, nnz_up, stream);
    if (status != hipSuccess) return status;
    return vt == kBF16 ? tiles_side<uint16_t, false>(act, out_hidden, out_val, down_table, b_down, y, work, d, h, n, nnz_down, stream)
                       : tiles_side<float, false>(act, out_hidden, out_val, down_table, b_down, y, work, d, h, n, nnz_down, stream);
}

}  // namespace hffn
