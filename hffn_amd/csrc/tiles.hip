// Decode-sized projections (gfx950, wave64): 1-64 tokens from the tiled store, every stored slot read from HBM once per
// call, the dot products on MFMA over tiles densified in LDS.
//
// A side has R rows (up: the d_ff neurons over K = d_model inputs; down: the d_model outputs of the output-major store
// over K = d_ff neurons). Its tiled store is a copy of the compact store built on the device at load
// (tiles_count/scan/place kernels): the slots of one 16-row tile and one 512-wide sub-chunk of K (an item) are
// consecutive, items in tile-major, sub-chunk-minor order, in 8-slot groups of interleaved 16-bit fields:
//   bfloat16 weights: [8 positions][8 weights]                    32 bytes, two 16-byte loads
//   float32 weights:  [8 positions][8 fp16 hi][8 fp16 lo]          48 bytes, three 16-byte loads
// with position = (row in the tile) << 12 | (k mod 4096). A float32 weight w of row r is kept as hi + lo ~ w 2^-e(r),
// e(r) the power of two of the row's largest |weight|. An item is padded to whole groups by repeating its last slot
// (which writes a tile cell again with the value it already holds). The table: every item's first group, the number
// of groups, then (float32) e(r) per row.
//
// A block of 16 waves takes TR 16-row tiles and S sub-chunks (a chunk of 512 S of K). Its groups are one contiguous
// range per tile, read once, 16 bytes per lane per load. The block
//   1. requests the inputs of each wave's 32 S k (first token tile) and its groups, and zeroes the tile;
//   2. scatters the groups into the dense tile [16 TR rows][512 S k] (two fp16 planes, or one bfloat16 plane);
//   3. multiplies: wave w takes S 32-k steps; lane (r, c) = (lane % 16, lane / 16) holds row r's 8 weights at k-run c
//      (B operand, from LDS) and token r's 8 inputs at the same k (A operand). float32: the inputs are scaled by the
//      token's power of two over the wave's k and split into fp16 hi and lo, D += x_hi w_hi + x_hi w_lo + x_lo w_hi
//      on v_mfma_f32_16x16x32_f16; bfloat16: each input is split exactly into three bfloat16 parts (8 significant
//      bits each, by truncation), D += (x_1 + x_2 + x_3) w on v_mfma_f32_16x16x32_bf16, every product exact;
//   4. adds the 16 waves' sums in a fixed order (LDS), undoes the powers of two, and writes the output with the
//      epilogue (bias, and GELU for the up side), or, when K spans several chunks, a partial per chunk that
//      tiles_reduce_kernel adds in chunk order before the epilogue.
// The block shape (TR, S) of each side is the one of least estimated time (tiles_shape); it depends on the side's shape
// and density only, never on the token count. Every output is a fixed-order sum over fixed groups: no atomics, the bits repeat run to run and a
// token's result does not depend on the other tokens of the call. Inputs and outputs are token-major [n, K], [n, R].
#include <algorithm>
#include <cmath>

#include "common.hpp"
#include "launch.hpp"

namespace hffn {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kRows = 16;                // rows per tile: one MFMA operand width
constexpr uint32_t kSub = 512;                // k per sub-chunk (one item of the store)
constexpr uint32_t kSuper = 4096;             // k span of a position's 12-bit field
constexpr uint32_t kWaves = 16;
constexpr uint32_t kThreads = kWaves * kWave;
constexpr uint32_t kStep = 32;                // k per MFMA
constexpr uint32_t kTokenTile = 16;
constexpr uint32_t kGroupSlots = 8;
constexpr uint32_t kTileBudget = 128 * 1024;  // LDS bytes of a block's dense tile
constexpr uint32_t kCUs = 256;                // MI355X compute units: one round of blocks

template <typename V> struct Planes;
template <> struct Planes<float> { static constexpr uint32_t count = 2; };     // fp16 hi, lo
template <> struct Planes<uint16_t> { static constexpr uint32_t count = 1; };  // bfloat16 bits

constexpr uint32_t planes_of(int vt) { return vt == kBF16 ? 1 : 2; }
constexpr uint32_t group_bytes(uint32_t planes) { return 16 * (1 + planes); }

// 16-bit field u (0..7) of an 8-field run
__device__ __forceinline__ uint32_t field(const uint4& q, int u) {
    const uint32_t word = u < 2 ? q.x : u < 4 ? q.y : u < 6 ? q.z : q.w;
    return u % 2 == 0 ? (word & 0xffffu) : (word >> 16);
}

__device__ __forceinline__ int binade_of(uint32_t magnitude_bits) {
    return magnitude_bits == 0 ? 0 : static_cast<int>((magnitude_bits >> 23) & 0xff) - 127;
}

// Half offset of (row r, k) in a tile plane of W k per row: the 16-byte runs of 8 k are XOR-swizzled by the row, so
// the 16 lanes of one LDS pass (rows r..r+15, the same run) read 16 distinct bank groups.
template <uint32_t W>
__device__ __forceinline__ uint32_t tile_at(uint32_t r, uint32_t k) {
    return r * W + (((k >> 3) ^ (r & 15)) << 3) + (k & 7);
}

template <typename V, int TT, int S, int TR>
constexpr bool shape_fits() {
    return TR * S * Planes<V>::count * kRows * kSub * 2 <= kTileBudget;
}

// One 8-slot piece of a row of the compact store, slots [8 q, 8 q + 8): its 8 indices (one 16-byte load) and values
// (one or two 16-byte loads), without branches, so that a wave's pieces are in flight together. A piece across the end
// of the arrays (the store's last, when nnz is not a multiple of 8) loads piece 0 here (nnz >= 8), and load_tail then
// reads it slot by slot, the slots past nnz zero.
template <typename V>
__device__ __forceinline__ void load_piece(const int16_t* __restrict__ idx, const V* __restrict__ val, int32_t q, int32_t nnz,
                                           uint4 (&pc)[1 + Planes<V>::count]) {
    constexpr uint32_t P = Planes<V>::count;
    const int32_t s = 8 * q, at = s + 8 <= nnz ? s : 0;
    pc[0] = *reinterpret_cast<const uint4*>(idx + at);
#pragma unroll
    for (uint32_t p = 0; p < P; ++p) pc[1 + p] = reinterpret_cast<const uint4*>(val + at)[p];
}

template <typename V>
__device__ __forceinline__ void load_tail(const int16_t* __restrict__ idx, const V* __restrict__ val, int32_t q, int32_t nnz,
                                          uint4 (&pc)[1 + Planes<V>::count]) {
    // composed in 32-bit words (two 16-bit indices or bfloat16 values per word, one float32 value), as the whole-piece
    // loads deliver them
    const int32_t s = 8 * q;
    uint32_t ids[4] = {0, 0, 0, 0}, vals[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int u = 0; u < 8; ++u)
        if (s + u < nnz) {
            ids[u / 2] |= static_cast<uint32_t>(static_cast<uint16_t>(idx[s + u])) << (16 * (u % 2));
            if constexpr (Planes<V>::count == 1) vals[u / 2] |= static_cast<uint32_t>(val[s + u]) << (16 * (u % 2));
            else vals[u] = __float_as_uint(val[s + u]);
        }
    pc[0] = make_uint4(ids[0], ids[1], ids[2], ids[3]);
    pc[1] = make_uint4(vals[0], vals[1], vals[2], vals[3]);
    if constexpr (Planes<V>::count == 2) pc[2] = make_uint4(vals[4], vals[5], vals[6], vals[7]);
}

// Value u (0..7) of a piece: float32 (fields 4 per uint4) or bfloat16 bits.
__device__ __forceinline__ float piece_value(const uint4 (&pc)[3], int u) {
    const uint4& q = pc[1 + u / 4];
    return __uint_as_float(u % 4 == 0 ? q.x : u % 4 == 1 ? q.y : u % 4 == 2 ? q.z : q.w);
}

template <typename V, int TT, int S, int TR, bool COMPACT>
__global__ __launch_bounds__(kThreads) void tiles_kernel(const float* __restrict__ in,         // [n, K]
                                                         const uint4* __restrict__ store,      // groups
                                                         const int32_t* __restrict__ table,    // items' first groups
                                                         const int32_t* __restrict__ binades,  // rows' powers of two
                                                         const float* __restrict__ bias,       // [R]
                                                         float* __restrict__ out,              // [n, R]
                                                         float* __restrict__ partials,         // [chunks, n, R]
                                                         uint32_t rows, uint32_t K, uint32_t n, uint32_t subchunks,
                                                         uint32_t up, const int16_t* __restrict__ cidx, const V* __restrict__ cval,
                                                         int32_t nnz) {
    constexpr uint32_t P = Planes<V>::count;
    constexpr uint32_t W = S * kSub;  // k per block
    constexpr uint32_t kTileRows = TR * kRows;
    constexpr uint32_t kPlane = kTileRows * W;  // halves per plane
    constexpr uint32_t kWaveSums = TR * TT * kTokenTile * kRows;
    constexpr uint32_t kTileBytes = P * kPlane * 2, kSumBytes = kWaves / 2 * kWaveSums * 4;
    static_assert(kTileBytes <= kTileBudget, "block shape beyond the LDS budget");
    __shared__ __align__(16) unsigned char lds[kTileBytes > kSumBytes ? kTileBytes : kSumBytes];
    uint16_t* tile = reinterpret_cast<uint16_t*>(lds);  // [plane][row][W], swizzled runs
    float* sums = reinterpret_cast<float*>(lds);        // [wave % 8][tr][tt][token][row], after the products

    const uint32_t lane = threadIdx.x % kWave, wave = uniform(threadIdx.x / kWave);
    const uint32_t r = lane % 16, c = lane / 16;
    const uint32_t chunk = blockIdx.y, tile0 = blockIdx.x * TR, tiles = (rows + kRows - 1) / kRows;
    const uint32_t kb = chunk * W, width = min(W, K - kb), kbase = kb % kSuper;
    const uint32_t j0 = chunk * S, j1 = min(j0 + S, subchunks);

    // the epilogue's per-row constants of this thread's outputs (output o = threadIdx.x + kThreads i: row o % the block's
    // rows), requested first so that their round trip overlaps the store's; a row past the side reads the last row's
    constexpr uint32_t kOutputs = TT * kTokenTile * kTileRows, kOuts = (kOutputs + kThreads - 1) / kThreads;
    int32_t out_e[kOuts];
    float out_b[kOuts];
#pragma unroll
    for (uint32_t i = 0; i < kOuts; ++i) {
        const uint32_t row = min(tile0 * kRows + (threadIdx.x + i * kThreads) % kTileRows, rows - 1);
        out_e[i] = 0;
        out_b[i] = 0.0f;
        if constexpr (P == 2) out_e[i] = binades[row];
        if (gridDim.y == 1) out_b[i] = bias[row];
    }

    // 1. the block's group ranges (one per tile; a tile past the side owns none)
    int32_t first[TR], count[TR], total = 0;
    // compact: the slot range [s0, s1) of each of the wave's rows (row 16 tr + wave of the block) in this chunk, and
    // (float32) the row's power of two
    int32_t s0[TR], s1[TR], row_e[TR];
#pragma unroll
    for (int tr = 0; tr < TR; ++tr) {
        first[tr] = 0;
        count[tr] = 0;
        if constexpr (COMPACT) {
            const uint32_t row = (tile0 + tr) * kRows + wave;
            s0[tr] = s1[tr] = 0;
            row_e[tr] = 0;
            if (row < rows) {
                s0[tr] = table[row * (subchunks + 1) + j0];
                s1[tr] = table[row * (subchunks + 1) + j1];
                if constexpr (P == 2) row_e[tr] = binades[row];
            }
        } else if (tile0 + tr < tiles) {
            first[tr] = table[(tile0 + tr) * subchunks + j0];
            count[tr] = table[(tile0 + tr) * subchunks + j1] - first[tr];
        }
        total += count[tr];
    }
    // The wave's inputs of one token tile (its S steps), requested without branches: an input outside the call
    // (token >= n, or k beyond the chunk) loads x[0, 0..7] and is zeroed at use. The first tile's are requested now.
    float xv[S][8];
    uint32_t live = 0;  // bit q: step q's inputs are inside the call
    auto request = [&](int tt) {
        live = 0;
#pragma unroll
        for (int q = 0; q < S; ++q) {
            const uint32_t kk = (wave * S + q) * kStep + c * 8, t = tt * kTokenTile + r;
            const bool inside = t < n && kk < width;
            live |= static_cast<uint32_t>(inside) << q;
            load_vec<8>(in + (inside ? static_cast<size_t>(t) * K + kb + kk : 0), xv[q]);
        }
    };
    request(0);
    // The g-th group of the block and the first tile row it belongs to (clamped into the block's ranges: a lane past
    // the end reloads the last group and skips it; an empty block reads the group at its range start, which the
    // store's one spare group at its end keeps valid). A later tile with cum <= g overrides an earlier one, so a tile
    // without groups is passed over.
    auto load_group = [&](int32_t g, uint4 (&part)[1 + P]) -> uint32_t {
        g = min(g, max(total, 1) - 1);
        int32_t at = first[0] + g, cum = 0;
        uint32_t row_base = 0;
#pragma unroll
        for (int tr = 1; tr < TR; ++tr) {
            cum += count[tr - 1];
            if (g >= cum) {
                at = first[tr] + (g - cum);
                row_base = tr * kRows;
            }
        }
        const uint4* p = store + static_cast<size_t>(at) * (1 + P);
#pragma unroll
        for (uint32_t i = 0; i < 1 + P; ++i) part[i] = p[i];
        return row_base;
    };
    auto scatter = [&](int32_t g, const uint4 (&part)[1 + P], uint32_t row_base) {
        if (g >= total) return;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const uint32_t pos = field(part[0], u);
            const uint32_t k = (pos & (kSuper - 1)) - kbase;
            if (k < width) {
                const uint32_t at = tile_at<W>(row_base + (pos >> 12), k);
#pragma unroll
                for (uint32_t p = 0; p < P; ++p) tile[p * kPlane + at] = static_cast<uint16_t>(field(part[1 + p], u));
            }
        }
    };
    if constexpr (COMPACT) {
        // 1'. the wave's rows' 8-slot pieces as one list (row tr's pieces q0[tr] .. q0[tr] + count - 1 after those of
        // rows 0 .. tr - 1), over the lanes: piece g of the list in lane g % 64, round g / 64. The first two rounds are
        // requested before the tile is zeroed.
        int32_t q0[TR], cum[TR], pieces = 0;
#pragma unroll
        for (int tr = 0; tr < TR; ++tr) {
            q0[tr] = s0[tr] >> 3;
            cum[tr] = pieces;
            pieces += s0[tr] < s1[tr] ? ((s1[tr] + 7) >> 3) - q0[tr] : 0;
        }
        auto locate = [&](int32_t g, int& tr, int32_t& q) {  // a later row with cum <= g overrides: empty rows are passed
            tr = 0;
#pragma unroll
            for (int t = 1; t < TR; ++t)
                if (g >= cum[t]) tr = t;
            q = q0[tr] + (g - cum[tr]);
        };
        // without branches: a lane past the wave's pieces loads the wave's last piece again (and places nothing); a
        // piece across nnz is completed by fix_tail
        auto fetch = [&](int32_t g, int& tr, int32_t& q, uint4 (&part)[3]) {
            locate(min(g, max(pieces, 1) - 1), tr, q);
            if (nnz >= 8) load_piece(cidx, cval, q, nnz, reinterpret_cast<uint4(&)[1 + P]>(part));
        };
        auto fix_tail = [&](int32_t g, int32_t q, uint4 (&part)[3]) {
            if (g < pieces && (nnz < 8 || 8 * q + 8 > nnz)) load_tail(cidx, cval, q, nnz, reinterpret_cast<uint4(&)[1 + P]>(part));
        };
        // 2'. scatter: a piece's slots inside its row's range, at (row, index - kb); float32 weights split into fp16
        // hi + lo = w 2^-e(row), as the tile would hold them from any source
        auto place = [&](int32_t g, int tr, int32_t q, const uint4 (&part)[3]) {
            if (g >= pieces) return;
            const uint32_t rr = tr * kRows + wave;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int32_t slot = 8 * q + u;
                if (slot >= s0[tr] && slot < s1[tr]) {
                    const uint32_t at = tile_at<W>(rr, field(part[0], u) - kb);
                    if constexpr (P == 1) {
                        tile[at] = static_cast<uint16_t>(field(part[1], u));
                    } else {
                        const float sv = ldexpf(piece_value(part, u), -row_e[tr]);
                        const _Float16 hi = static_cast<_Float16>(sv);
                        tile[at] = __builtin_bit_cast(uint16_t, hi);
                        tile[kPlane + at] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(sv - static_cast<float>(hi)));
                    }
                }
            }
        };
        const int32_t ga_at = static_cast<int32_t>(lane), gb_at = ga_at + kWave;
        uint4 pa[3], pb[3];
        int tra = 0, trb = 0;
        int32_t qa = 0, qb = 0;
        locate(min(ga_at, max(pieces, 1) - 1), tra, qa);
        locate(min(gb_at, max(pieces, 1) - 1), trb, qb);
        if (nnz >= 8) {  // both rounds' pieces in one block of loads, none of them used before all are requested
            load_piece(cidx, cval, qa, nnz, reinterpret_cast<uint4(&)[1 + P]>(pa));
            load_piece(cidx, cval, qb, nnz, reinterpret_cast<uint4(&)[1 + P]>(pb));
            __builtin_amdgcn_sched_barrier(0);
        }
        bool tail = false;  // wave-uniform: some row's pieces reach past the last whole piece of the store
#pragma unroll
        for (int tr = 0; tr < TR; ++tr) {
            const int32_t count = (tr + 1 < TR ? cum[tr + 1] : pieces) - cum[tr];
            tail |= count > 0 && 8 * (q0[tr] + count) > (nnz & ~7);
        }
        if (tail) {
            fix_tail(ga_at, qa, pa);
            fix_tail(gb_at, qb, pb);
        }
        for (uint32_t i = threadIdx.x; i < kTileBytes / 16; i += kThreads) reinterpret_cast<uint4*>(tile)[i] = make_uint4(0, 0, 0, 0);
        __syncthreads();  // the tile is zero (this waits for the LDS only: the loads stay in flight)
        place(ga_at, tra, qa, pa);
        place(gb_at, trb, qb, pb);
        for (int32_t g = ga_at + 2 * kWave; g - static_cast<int32_t>(lane) < pieces; g += kWave) {
            uint4 pc[3];
            int tr = 0;
            int32_t q = 0;
            fetch(g, tr, q, pc);
            fix_tail(g, q, pc);
            place(g, tr, q, pc);
        }
        __syncthreads();
    } else {
    uint4 ga[1 + P], gb[1 + P];
    const uint32_t rows_a = load_group(threadIdx.x, ga), rows_b = load_group(threadIdx.x + kThreads, gb);
    for (uint32_t i = threadIdx.x; i < kTileBytes / 16; i += kThreads) reinterpret_cast<uint4*>(tile)[i] = make_uint4(0, 0, 0, 0);
    __syncthreads();  // the tile is zero (this waits for the LDS only: the loads stay in flight)

    // 2. scatter, the first two rounds of groups as they arrive, then any further rounds
    scatter(threadIdx.x, ga, rows_a);
    scatter(threadIdx.x + kThreads, gb, rows_b);
    for (int32_t g = 2 * kThreads + threadIdx.x; g - static_cast<int32_t>(threadIdx.x) < total; g += kThreads) {
        uint4 gc[1 + P];
        scatter(g, gc, load_group(g, gc));
    }
    __syncthreads();
    }

    // 3. products over the wave's S steps, one token tile after the other. With few steps (2; 4 for bfloat16) the
    // tile's A operands are all formed before the next tile's inputs are requested (their arrival overlaps the
    // products); otherwise each step's are formed just before its products (registers) and the next inputs requested
    // after them.
    floatx4 acc[TT][TR];
    // the A operands of step q of the current tile: fp16 hi/lo, or the three bfloat16 parts of each input
    auto split = [&](int q, int ex, uint32_t (&aq)[3][4]) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (live >> q) & 1u ? xv[q][i] : 0.0f;
        if constexpr (P == 2) {
            half8 xh, xl;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float sv = ldexpf(v[i], -ex);
                const _Float16 hv = static_cast<_Float16>(sv);
                xh[i] = hv;
                xl[i] = static_cast<_Float16>(sv - static_cast<float>(hv));
            }
            const uint4 h4 = __builtin_bit_cast(uint4, xh), l4 = __builtin_bit_cast(uint4, xl);
            aq[0][0] = h4.x; aq[0][1] = h4.y; aq[0][2] = h4.z; aq[0][3] = h4.w;
            aq[1][0] = l4.x; aq[1][1] = l4.y; aq[1][2] = l4.z; aq[1][3] = l4.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; i += 2) {
                uint32_t part[3][2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float x0 = v[i + h];
                    const uint32_t b1 = __float_as_uint(x0) & 0xffff0000u;
                    const float rest = x0 - __uint_as_float(b1);
                    const uint32_t b2 = __float_as_uint(rest) & 0xffff0000u;
                    const uint32_t b3 = __float_as_uint(rest - __uint_as_float(b2));  // <= 8 significant bits left
                    part[0][h] = b1 >> 16;
                    part[1][h] = b2 >> 16;
                    part[2][h] = b3 >> 16;
                }
#pragma unroll
                for (int j = 0; j < 3; ++j) aq[j][i / 2] = part[j][0] | (part[j][1] << 16);
            }
        }
    };
    auto multiply = [&](int q, const uint32_t (&aq)[3][4], floatx4 (&d)[TR]) {
        const uint32_t kq = (wave * S + q) * kStep + c * 8;
#pragma unroll
        for (int tr = 0; tr < TR; ++tr) {
            const uint16_t* at = tile + tile_at<W>(tr * kRows + r, kq);
            if constexpr (P == 2) {
                const half8 wh = __builtin_bit_cast(half8, *reinterpret_cast<const uint4*>(at));
                const half8 wl = __builtin_bit_cast(half8, *reinterpret_cast<const uint4*>(at + kPlane));
                const half8 xh = __builtin_bit_cast(half8, aq[0]), xl = __builtin_bit_cast(half8, aq[1]);
                d[tr] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, wh, d[tr], 0, 0, 0);
                d[tr] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, wl, d[tr], 0, 0, 0);
                d[tr] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, wh, d[tr], 0, 0, 0);
            } else {
                const bf16x8 wb = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(at));
#pragma unroll
                for (int j = 0; j < 3; ++j)
                    d[tr] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, aq[j]), wb, d[tr], 0, 0, 0);
            }
        }
    };
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
#pragma unroll
        for (int tr = 0; tr < TR; ++tr) acc[tt][tr] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        int ex = 0;  // float32: the token's power of two over the wave's k (lanes r, r + 16, r + 32, r + 48 hold it)
        if constexpr (P == 2) {
            uint32_t m = 0;
#pragma unroll
            for (int q = 0; q < S; ++q)
#pragma unroll
                for (int i = 0; i < 8; ++i) m = max(m, ((live >> q) & 1u ? __float_as_uint(xv[q][i]) : 0u) & 0x7fffffffu);
            m = max(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), 16, kWave)));
            m = max(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), 32, kWave)));
            ex = binade_of(m);
        }
        if constexpr (S <= 2 || (S <= 4 && P == 1)) {
            uint32_t a[S][3][4];
#pragma unroll
            for (int q = 0; q < S; ++q) split(q, ex, a[q]);
            if (tt + 1 < TT) request(tt + 1);
#pragma unroll
            for (int q = 0; q < S; ++q) multiply(q, a[q], acc[tt]);
        } else {
#pragma unroll
            for (int q = 0; q < S; ++q) {
                uint32_t aq[3][4];
                split(q, ex, aq);
                multiply(q, aq, acc[tt]);
            }
            if (tt + 1 < TT) request(tt + 1);
        }
        if constexpr (P == 2) {
            // D register i holds token 4c + i of the tile: undo its power of two (held by lane 4c + i)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int e = __shfl(ex, static_cast<int>(4 * c + i), kWave);
#pragma unroll
                for (int tr = 0; tr < TR; ++tr) acc[tt][tr][i] = ldexpf(acc[tt][tr][i], e);
            }
        }
    }
    __syncthreads();  // the tile is read: its LDS now holds the waves' sums

    // 4. the 16 waves' sums in a fixed order (wave w + 8 into wave w, then waves 0..7), the row's power of two, then the
    // output or this chunk's partial
    float* mine = sums + (wave % (kWaves / 2)) * kWaveSums;
    auto cell = [](int tr, int tt, uint32_t token, uint32_t row) { return ((tr * TT + tt) * kTokenTile + token) * kRows + row; };
    if (wave >= kWaves / 2) {
#pragma unroll
        for (int tr = 0; tr < TR; ++tr)
#pragma unroll
            for (int tt = 0; tt < TT; ++tt)
#pragma unroll
                for (int i = 0; i < 4; ++i) mine[cell(tr, tt, 4 * c + i, r)] = acc[tt][tr][i];
    }
    __syncthreads();
    if (wave < kWaves / 2) {
#pragma unroll
        for (int tr = 0; tr < TR; ++tr)
#pragma unroll
            for (int tt = 0; tt < TT; ++tt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float* at = mine + cell(tr, tt, 4 * c + i, r);
                    *at = acc[tt][tr][i] + *at;
                }
    }
    __syncthreads();
#pragma unroll
    for (uint32_t i = 0; i < kOuts; ++i) {
        const uint32_t o = threadIdx.x + i * kThreads;
        if (o >= kOutputs) break;
        const uint32_t t = o / kTileRows, rr = o % kTileRows, row = tile0 * kRows + rr;
        if (t >= n) break;
        if (row >= rows) continue;
        const uint32_t at = cell(rr / kRows, t / kTokenTile, t % kTokenTile, rr % kRows);
        float s = sums[at];
#pragma unroll
        for (uint32_t h = 1; h < kWaves / 2; ++h) s += sums[h * kWaveSums + at];
        if constexpr (P == 2) s = ldexpf(s, out_e[i]);
        if (gridDim.y > 1) {
            partials[(static_cast<size_t>(chunk) * n + t) * rows + row] = s;
        } else {
            const float z = s + out_b[i];
            out[static_cast<size_t>(t) * rows + row] = up ? gelu(z) : z;
        }
    }
}

// out[t, r] = epilogue(bias[r] + the chunks' partials added in chunk order); one thread per output.
__global__ __launch_bounds__(256) void tiles_reduce_kernel(const float* __restrict__ partials, uint32_t chunks,
                                                           const float* __restrict__ bias, float* __restrict__ out,
                                                           uint32_t rows, uint32_t n, uint32_t up) {
    const uint32_t o = blockIdx.x * 256 + threadIdx.x;
    if (o >= n * rows) return;
    const size_t stride = static_cast<size_t>(n) * rows;
    // every load of a batch of 8 chunks (and the bias) is issued before the first is added: one memory round trip per
    // batch; a chunk past the last reloads the last one and is not added
    const float b = bias[o % rows];
    float s = partials[o];
    for (uint32_t k0 = 1; k0 < chunks; k0 += 8) {
        float p[8];
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) p[u] = partials[min(k0 + u, chunks - 1) * stride + o];
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u)
            if (k0 + u < chunks) s += p[u];
    }
    const float z = s + b;
    out[o] = up ? gelu(z) : z;
}

// ---------------------------------------------------------------------------------------------- building the store

// The first slot of [lo, hi) whose index reaches k (indices ascend within a row), else hi.
__device__ int32_t first_reaching(const int16_t* __restrict__ idx, int32_t lo, int32_t hi, uint32_t k) {
    while (lo < hi) {
        const int32_t mid = lo + (hi - lo) / 2;
        if (static_cast<uint32_t>(static_cast<uint16_t>(idx[mid])) < k) lo = mid + 1; else hi = mid;
    }
    return lo;
}

// table[item] = the groups of item (tile t, sub-chunk j): its 16 rows' slots with index in [512 j, 512 j + 512).
__global__ __launch_bounds__(256) void tiles_count_kernel(const int32_t* __restrict__ offsets, const int16_t* __restrict__ idx,
                                                          uint32_t rows, uint32_t subchunks, uint32_t items,
                                                          int32_t* __restrict__ table) {
    const uint32_t item = blockIdx.x * 256 + threadIdx.x;
    if (item >= items) return;
    const uint32_t t = item / subchunks, j = item % subchunks;
    int32_t slots = 0;
    for (uint32_t rr = 0; rr < kRows && t * kRows + rr < rows; ++rr) {
        const int32_t lo = offsets[t * kRows + rr], hi = offsets[t * kRows + rr + 1];
        slots += first_reaching(idx, lo, hi, (j + 1) * kSub) - first_reaching(idx, lo, hi, j * kSub);
    }
    table[item] = (slots + kGroupSlots - 1) / kGroupSlots;
}

// Exclusive prefix sum of table[0, items) in place, table[items] = the total; one block.
__global__ __launch_bounds__(1024) void tiles_scan_kernel(int32_t* __restrict__ table, uint32_t items) {
    __shared__ int32_t part[1024];
    const uint32_t per = (items + 1023) / 1024;
    const uint32_t b = min(items, threadIdx.x * per), e = min(items, b + per);
    int32_t s = 0;
    for (uint32_t i = b; i < e; ++i) s += table[i];
    part[threadIdx.x] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        int32_t run = 0;
        for (uint32_t i = 0; i < 1024; ++i) {
            const int32_t v = part[i];
            part[i] = run;
            run += v;
        }
        table[items] = run;
    }
    __syncthreads();
    int32_t run = part[threadIdx.x];
    for (uint32_t i = b; i < e; ++i) {
        const int32_t v = table[i];
        table[i] = run;
        run += v;
    }
}

// binades[r] = the power of two of row r's largest |weight| (0 for a row without a non-zero weight); float32 stores.
// One wave per row: the lanes' maxima over the row's slots (64 apart), then a wave maximum.
__global__ __launch_bounds__(256) void tiles_binade_kernel(const int32_t* __restrict__ offsets, const float* __restrict__ val,
                                                           uint32_t rows, int32_t* __restrict__ binades) {
    const uint32_t r = blockIdx.x * 4 + threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (r >= rows) return;
    uint32_t m = 0;
    for (int32_t s = offsets[r] + static_cast<int32_t>(lane); s < offsets[r + 1]; s += kWave) m = max(m, __float_as_uint(val[s]) & 0x7fffffffu);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = max(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), o, kWave)));
    if (lane == 0) binades[r] = binade_of(m);
}

// One wave per item: its rows' slots in row order, then the padding (the item's last slot again).
template <typename V>
__global__ __launch_bounds__(256) void tiles_place_kernel(const int32_t* __restrict__ offsets, const int16_t* __restrict__ idx,
                                                          const V* __restrict__ val, const int32_t* __restrict__ table,
                                                          const int32_t* __restrict__ binades, uint32_t rows, uint32_t subchunks,
                                                          uint32_t items, uint16_t* __restrict__ store) {
    constexpr uint32_t P = Planes<V>::count;
    const uint32_t item = blockIdx.x * 4 + threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (item >= items) return;
    const uint32_t t = item / subchunks, j = item % subchunks;
    int32_t lo = 0, len = 0;
    if (lane < kRows && t * kRows + lane < rows) {
        const int32_t a = offsets[t * kRows + lane], z = offsets[t * kRows + lane + 1];
        lo = first_reaching(idx, a, z, j * kSub);
        len = first_reaching(idx, a, z, (j + 1) * kSub) - lo;
    }
    const int64_t base = static_cast<int64_t>(table[item]) * kGroupSlots;
    const int32_t slots = (table[item + 1] - table[item]) * static_cast<int32_t>(kGroupSlots);
    auto put = [&](int64_t o, uint32_t rr, int32_t s) {
        uint16_t* g = store + (o / kGroupSlots) * kGroupSlots * (1 + P);
        const uint32_t u = static_cast<uint32_t>(o % kGroupSlots);
        g[u] = static_cast<uint16_t>((rr << 12) | (static_cast<uint32_t>(static_cast<uint16_t>(idx[s])) & (kSuper - 1)));
        if constexpr (P == 1) {
            g[kGroupSlots + u] = val[s];
        } else {
            const float sv = ldexpf(val[s], -binades[t * kRows + rr]);
            const _Float16 hi = static_cast<_Float16>(sv);
            g[kGroupSlots + u] = __builtin_bit_cast(uint16_t, hi);
            g[2 * kGroupSlots + u] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(sv - static_cast<float>(hi)));
        }
    };
    int32_t done = 0, last = -1;
    uint32_t last_row = 0;
    for (uint32_t rr = 0; rr < kRows; ++rr) {
        const int32_t seg_lo = __shfl(lo, static_cast<int>(rr), kWave), seg_len = __shfl(len, static_cast<int>(rr), kWave);
        for (int32_t i = static_cast<int32_t>(lane); i < seg_len; i += kWave) put(base + done + i, rr, seg_lo + i);
        if (seg_len > 0) {
            last = seg_lo + seg_len - 1;
            last_row = rr;
        }
        done += seg_len;
    }
    if (last >= 0)
        for (int32_t o = done + static_cast<int32_t>(lane); o < slots; o += kWave) put(base + o, last_row, last);
}

// ---------------------------------------------------------------------------------------------- launches

// table[r (subchunks + 1) + j] = the first slot of row r whose index reaches 512 j (j = subchunks: the row's end).
__global__ __launch_bounds__(256) void tiles_bounds_kernel(const int32_t* __restrict__ offsets, const int16_t* __restrict__ idx,
                                                           uint32_t rows, uint32_t subchunks, int32_t* __restrict__ table) {
    const uint32_t e = blockIdx.x * 256 + threadIdx.x;
    if (e >= rows * (subchunks + 1)) return;
    const uint32_t r = e / (subchunks + 1), j = e % (subchunks + 1);
    const int32_t lo = offsets[r], hi = offsets[r + 1];
    table[e] = j == 0 ? lo : j == subchunks ? hi : first_reaching(idx, lo, hi, j * kSub);
}

struct Side {
    const float* in;
    const uint4* store;
    const int32_t* table;
    const int32_t* binades;
    const float* bias;
    float* out;
    float* partials;
    uint32_t rows, K, n, subchunks, up;
    uint64_t nnz;
    const int16_t* cidx;  // the compact rows (COMPACT launches)
    const void* cval;
};

template <typename V, int TT, int S, int TR, bool COMPACT>
bool launch_shape(const Side& a, const TilesShape& shape, hipStream_t stream) {
    if constexpr (!shape_fits<V, TT, S, TR>()) {
        return false;
    } else {
        if (shape.s != S || shape.tr != TR) return false;
        hipLaunchKernelGGL((tiles_kernel<V, TT, S, TR, COMPACT>), dim3(shape.blocks, shape.chunks), dim3(kThreads), 0, stream, a.in, a.store,
                           a.table, a.binades, a.bias, a.out, a.partials, a.rows, a.K, a.n, a.subchunks, a.up, a.cidx,
                           static_cast<const V*>(a.cval), static_cast<int32_t>(a.nnz));
        return true;
    }
}

template <typename V, int TT, bool COMPACT>
bool launch_tokens(const Side& a, const TilesShape& shape, hipStream_t stream) {
    return launch_shape<V, TT, 2, 1, COMPACT>(a, shape, stream) || launch_shape<V, TT, 4, 1, COMPACT>(a, shape, stream) ||
           launch_shape<V, TT, 8, 1, COMPACT>(a, shape, stream) || launch_shape<V, TT, 2, 2, COMPACT>(a, shape, stream) ||
           launch_shape<V, TT, 4, 2, COMPACT>(a, shape, stream) || launch_shape<V, TT, 2, 4, COMPACT>(a, shape, stream);
}

template <typename V, bool COMPACT = false>
hipError_t tiles_side(const Side& a, hipStream_t stream) {
    const TilesShape shape = tiles_shape(Planes<V>::count == 1 ? kBF16 : kF32, a.rows, a.K, a.nnz);
    const bool launched = a.n <= kTokenTile       ? launch_tokens<V, 1, COMPACT>(a, shape, stream)
                          : a.n <= 2 * kTokenTile ? launch_tokens<V, 2, COMPACT>(a, shape, stream)
                                                  : launch_tokens<V, 4, COMPACT>(a, shape, stream);
    if (!launched) return hipErrorInvalidValue;
    if (hipError_t status = hipGetLastError(); status != hipSuccess || shape.chunks == 1) return status;
    hipLaunchKernelGGL(tiles_reduce_kernel, dim3((a.n * a.rows + 255) / 256), dim3(256), 0, stream, a.partials, shape.chunks, a.bias, a.out,
                       a.rows, a.n, a.up);
    return hipGetLastError();
}

uint32_t items_of(uint32_t rows, uint32_t K) { return ((rows + kRows - 1) / kRows) * ((K + kSub - 1) / kSub); }

}  // namespace

// The block shape of a side: the (TR, S) of least estimated time, from a model of one block fitted to per-block
// timestamps of the 410M (float32, 50 %) and 1.4B (bfloat16, 20 %) sides at 16 tokens on MI355X: the loads take
// 0.8 us + 25 ns per KB of groups and inputs (the inputs of the 16 token rows of the chunk, 32 S KB), the products
// 0.3 + 0.4 S us (the inputs' split dominates), the epilogue 0.6 + 0.15 TR us; rounds of blocks over the CUs add up,
// and a side whose blocks split K pays a reduce pass (3 us). A block of a side split over K reads each of its 16 TR
// rows' slots in the chunk as a separate run of the compact arrays (the runs of a block that spans K are consecutive):
// 0.1 us per run, from the compact-row blocks' timestamps (the 1.4B down side's loads and scatter 2.5 us with 64 runs
// of 205 slots, 1.4 us from the tiled store's 4 ranges). Both stores take the same shape, so they give the same bits.
TilesShape tiles_shape(int vt, uint32_t rows, uint32_t K, uint64_t nnz) {
    constexpr double kRunUs = 0.1;
    const uint32_t planes = planes_of(vt), slot_bytes = vt == kBF16 ? 4 : 6;
    const uint32_t tiles = (rows + kRows - 1) / kRows, subchunks = (K + kSub - 1) / kSub;
    const double density = static_cast<double>(nnz) / (static_cast<double>(rows) * K);
    TilesShape best{0, 0, 0, 0};
    double best_us = 1e30;
    for (uint32_t tr = 1; tr <= 4; tr *= 2)
        for (uint32_t s = 2; s <= 8; s *= 2) {
            if (tr * s * planes * kRows * kSub * 2 > kTileBudget) continue;
            const uint32_t chunks = (subchunks + s - 1) / s, blocks = (tiles + tr - 1) / tr;
            const double rounds = std::ceil(static_cast<double>(blocks) * chunks / kCUs);
            const double width = std::min<double>(s * kSub, K);
            const double load_kb = (kRows * tr * width * density * slot_bytes + kTokenTile * width * 4) / 1024;
            const double runs = chunks > 1 ? kRows * tr : 0.0;
            const double block_us = 0.8 + 0.025 * load_kb + 0.3 + 0.4 * s + 0.6 + 0.15 * tr + kRunUs * runs;
            const double us = rounds * block_us + (chunks > 1 ? 3.0 : 0.0);
            if (us < best_us) {
                best_us = us;
                best = TilesShape{tr, s, chunks, blocks};
            }
        }
    return best;
}

TilesStoreSize tiles_store_size(int vt, uint32_t rows, uint32_t K, uint64_t nnz) {
    const uint64_t items = items_of(rows, K);
    const uint64_t groups = (nnz + kGroupSlots - 1) / kGroupSlots + items + 1;  // padding at most one group per item, one spare
    return TilesStoreSize{groups * group_bytes(planes_of(vt)), items + 1 + (vt == kBF16 ? 0 : rows)};
}

size_t tiles_workspace_bytes(int vt, uint32_t n, uint32_t d, uint32_t h, uint64_t nnz_up, uint64_t nnz_down) {
    const TilesShape up = tiles_shape(vt, h, d, nnz_up), down = tiles_shape(vt, d, h, nnz_down);
    const size_t a = up.chunks > 1 ? static_cast<size_t>(up.chunks) * n * h : 0;
    const size_t b = down.chunks > 1 ? static_cast<size_t>(down.chunks) * n * d : 0;
    return std::max<size_t>(std::max(a, b) * sizeof(float), 256);
}

hipError_t launch_tiles_build(int vt, const int32_t* offsets, const int16_t* idx, const void* val, uint32_t rows, uint32_t K, void* store,
                              int32_t* table, hipStream_t stream) {
    const uint32_t items = items_of(rows, K), subchunks = (K + kSub - 1) / kSub;
    int32_t* binades = table + items + 1;
    hipLaunchKernelGGL(tiles_count_kernel, dim3((items + 255) / 256), dim3(256), 0, stream, offsets, idx, rows, subchunks, items, table);
    hipLaunchKernelGGL(tiles_scan_kernel, dim3(1), dim3(1024), 0, stream, table, items);
    const dim3 place((items + 3) / 4);
    if (vt == kBF16) {
        hipLaunchKernelGGL(tiles_place_kernel<uint16_t>, place, dim3(256), 0, stream, offsets, idx, static_cast<const uint16_t*>(val), table,
                           binades, rows, subchunks, items, static_cast<uint16_t*>(store));
    } else {
        hipLaunchKernelGGL(tiles_binade_kernel, dim3((rows + 3) / 4), dim3(256), 0, stream, offsets, static_cast<const float*>(val), rows,
                           binades);
        hipLaunchKernelGGL(tiles_place_kernel<float>, place, dim3(256), 0, stream, offsets, idx, static_cast<const float*>(val), table,
                           binades, rows, subchunks, items, static_cast<uint16_t*>(store));
    }
    return hipGetLastError();
}

uint64_t tiles_table_entries(int vt, uint32_t rows, uint32_t K) {
    return static_cast<uint64_t>(rows) * ((K + kSub - 1) / kSub + 1) + (vt == kBF16 ? 0 : rows);
}

hipError_t launch_tiles_table(int vt, const int32_t* offsets, const int16_t* idx, const void* val, uint32_t rows, uint32_t K,
                              int32_t* table, hipStream_t stream) {
    const uint32_t subchunks = (K + kSub - 1) / kSub, entries = rows * (subchunks + 1);
    hipLaunchKernelGGL(tiles_bounds_kernel, dim3((entries + 255) / 256), dim3(256), 0, stream, offsets, idx, rows, subchunks, table);
    if (vt != kBF16)
        hipLaunchKernelGGL(tiles_binade_kernel, dim3((rows + 3) / 4), dim3(256), 0, stream, offsets, static_cast<const float*>(val), rows,
                           table + entries);
    return hipGetLastError();
}

hipError_t launch_tiles_compact(int vt, const float* x, const int16_t* up_idx, const void* up_val, const int32_t* up_table,
                                const float* b_up, const int16_t* out_hidden, const void* out_val, const int32_t* down_table,
                                const float* b_down, float* act, float* work, float* y, uint32_t d, uint32_t h, uint64_t nnz_up,
                                uint64_t nnz_down, uint32_t n, hipStream_t stream) {
    const uint32_t up_sub = (d + kSub - 1) / kSub, down_sub = (h + kSub - 1) / kSub;
    const Side up{x, nullptr, up_table, up_table + static_cast<size_t>(h) * (up_sub + 1), b_up, act, work, h, d, n, up_sub, 1, nnz_up,
                  up_idx, up_val};
    const Side down{act, nullptr, down_table, down_table + static_cast<size_t>(d) * (down_sub + 1), b_down, y, work, d, h, n, down_sub, 0,
                    nnz_down, out_hidden, out_val};
    const hipError_t status = vt == kBF16 ? tiles_side<uint16_t, true>(up, stream) : tiles_side<float, true>(up, stream);
    if (status != hipSuccess) return status;
    return vt == kBF16 ? tiles_side<uint16_t, true>(down, stream) : tiles_side<float, true>(down, stream);
}

hipError_t launch_tiles_forward(int vt, const float* x, const void* up_store, const int32_t* up_table, const float* b_up,
                                const void* down_store, const int32_t* down_table, const float* b_down, float* act, float* work,
                                float* y, uint32_t d, uint32_t h, uint64_t nnz_up, uint64_t nnz_down, uint32_t n, hipStream_t stream) {
    const uint32_t up_items = items_of(h, d), down_items = items_of(d, h);
    const Side up{x, static_cast<const uint4*>(up_store), up_table, up_table + up_items + 1, b_up, act, work, h, d, n,
                  (d + kSub - 1) / kSub, 1, nnz_up, nullptr, nullptr};
    const Side down{act, static_cast<const uint4*>(down_store), down_table, down_table + down_items + 1, b_down, y, work, d, h, n,
                    (h + kSub - 1) / kSub, 0, nnz_down, nullptr, nullptr};
    const hipError_t status = vt == kBF16 ? tiles_side<uint16_t>(up, stream) : tiles_side<float>(up, stream);
    if (status != hipSuccess) return status;
    return vt == kBF16 ? tiles_side<uint16_t>(down, stream) : tiles_side<float>(down, stream);
}

}  // namespace hffn
