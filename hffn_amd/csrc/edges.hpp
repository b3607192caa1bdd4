// Device pieces of the lane-per-slot ("edges") kernels (edges.hip): a row's slots read in groups of consecutive slots
// per lane, every value load 16 bytes and each wave instruction 1 KB of one contiguous range: float32 groups of 4 slots
// (a 16-byte value load and an 8-byte index load), bfloat16 groups of 8 (a 16-byte value load and a 16-byte index
// load: half the load instructions of 4-slot groups; 8 float32 values per lane would split a wave's value loads into
// two 2 KB ranges of half-used lines). The groups of a wave are strided by 64 groups, the lane partials of NT tokens
// are added by a fixed xor butterfly, and a long row split in P segments (one wave each) is added in segment order.
// Every kernel that runs a row through these pieces with the same P produces the same bits (the number of groups a
// lane holds at once does not change them).
#pragma once

#include "common.hpp"

namespace hffn {
namespace edges {

__device__ __forceinline__ uint32_t word_at(const uint4& q, int w) { return w == 0 ? q.x : w == 1 ? q.y : w == 2 ? q.z : q.w; }
__device__ __forceinline__ uint32_t word_at(const uint2& q, int w) { return w == 0 ? q.x : q.y; }

// A group of a value type: its slots, its value and index loads, value s and index s of a loaded group, and a group
// composed slot by slot (the store's last, partial group).
template <typename V> struct Group;
template <> struct Group<float> {
    static constexpr int kSlots = 4;
    using type = float4;
    using ids = uint2;
    __device__ static type load(const float* p) { return *reinterpret_cast<const float4*>(p); }
    __device__ static float at(const type& g, int s) { return s == 0 ? g.x : s == 1 ? g.y : s == 2 ? g.z : g.w; }
    __device__ static type compose(const float (&v)[kSlots]) { return make_float4(v[0], v[1], v[2], v[3]); }
};
template <> struct Group<uint16_t> {
    static constexpr int kSlots = 8;
    using type = uint4;
    using ids = uint4;
    __device__ static type load(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }
    __device__ static float at(const type& g, int s) {
        const uint32_t word = word_at(g, s / 2);
        return __uint_as_float((s % 2 == 0 ? word << 16 : word & 0xffff0000u));
    }
    __device__ static type compose(const uint16_t (&v)[kSlots]) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = v[2 * i] | (static_cast<uint32_t>(v[2 * i + 1]) << 16);
        return make_uint4(w[0], w[1], w[2], w[3]);
    }
};

template <typename Ids>
__device__ __forceinline__ uint32_t index_at(const Ids& g, int s) {
    const uint32_t word = word_at(g, s / 2);
    return s % 2 == 0 ? (word & 0xffffu) : (word >> 16);
}

// The index group of `S` slots from 16-bit indices packed two per word.
template <int S>
__device__ __forceinline__ auto compose_ids(const uint16_t (&i)[S]) {
    if constexpr (S == 4) {
        return make_uint2(i[0] | (static_cast<uint32_t>(i[1]) << 16), i[2] | (static_cast<uint32_t>(i[3]) << 16));
    } else {
        static_assert(S == 8, "groups of 4 or 8 slots");
        return make_uint4(i[0] | (static_cast<uint32_t>(i[1]) << 16), i[2] | (static_cast<uint32_t>(i[3]) << 16),
                          i[4] | (static_cast<uint32_t>(i[5]) << 16), i[6] | (static_cast<uint32_t>(i[7]) << 16));
    }
}

// Where a token's input for feature i lives: LDS [i][NT] (staged) or global [i * ld] + t (act of the down kernel).
struct StagedInput {
    const float* lds;
    template <int NT> __device__ void load(uint32_t i, float (&v)[NT]) const { load_vec<NT>(lds + i * NT, v); }
};
struct GlobalInput {
    const float* base;  // act + c0
    uint32_t ld;
    template <int NT> __device__ void load(uint32_t i, float (&v)[NT]) const {
        load_vec<NT>(base + static_cast<size_t>(i) * ld, v);
    }
};

// A wave's slots of one row segment [pb, pe), held in registers: up to G groups per lane, loaded before the inputs are
// staged so that the store's bytes are in flight while the block waits for its inputs.
template <typename V, int G>
struct Segment {
    typename Group<V>::type vals[G];
    typename Group<V>::ids ids[G];
    int32_t first;  // slot of this lane's group 0
};

// Issues the loads of groups [chunk * G, chunk * G + G) of this lane (groups strided by the wave). The whole groups
// (below pe and nnz) are loaded as one value and one index load each, all issued back to back with no branch between
// them, so they are in flight together (a lane without a whole group reads the store's group 0, which it never uses).
// A group that crosses nnz is loaded slot by slot, only in a wave whose segment reaches past the last whole group of
// the store (nnz not a multiple of the group).
template <typename V, int G>
__device__ __forceinline__ void load_segment(Segment<V, G>& seg, const int16_t* __restrict__ idx, const V* __restrict__ val,
                                             int32_t pb, int32_t pe, int32_t nnz, uint32_t lane, uint32_t chunk) {
    constexpr int S = Group<V>::kSlots;
    using Ids = typename Group<V>::ids;
    seg.first = (pb & ~(S - 1)) + S * static_cast<int32_t>(lane) + static_cast<int32_t>(chunk) * G * S * kWave;
    if (nnz >= S) {
#pragma unroll
        for (int k = 0; k < G; ++k) {
            const int32_t g = seg.first + k * S * kWave;
            const int32_t at = g < pe && g + S <= nnz ? g : 0;
            seg.vals[k] = Group<V>::load(val + at);
            seg.ids[k] = *reinterpret_cast<const Ids*>(idx + at);
        }
    }
    if (pe > (nnz & ~(S - 1))) {
#pragma unroll
        for (int k = 0; k < G; ++k) {
            const int32_t g = seg.first + k * S * kWave;
            if (g < pe && g + S > nnz) {
                uint16_t is[S] = {};
                V vs[S] = {};
                for (int s = 0; s < S; ++s)
                    if (g + s < nnz) {
                        is[s] = static_cast<uint16_t>(idx[g + s]);
                        vs[s] = val[g + s];
                    }
                seg.ids[k] = compose_ids<S>(is);
                seg.vals[k] = Group<V>::compose(vs);
            }
        }
    }
}

// Stages NT tokens of `rows` inputs into LDS [rows][NT] by DMA (global_load_lds, 4 bytes per lane): element (r, t)
// from src[r * rstride + min(t, tokens - 1) * tstride] (a padded token repeats the block's last token; its sums are
// never written). Every transfer of the block is issued before any is waited for; the caller waits (wait_loads<0>)
// and synchronises the block before reading the stage.
template <int NT, int WAVES>
__device__ __forceinline__ void stage_inputs(float* lds, const float* src, uint32_t rows, uint32_t rstride, uint32_t tstride,
                                             uint32_t tokens, uint32_t wave, uint32_t lane) {
    const uint32_t total = rows * NT;
    // Inputs already in LDS order (one token's contiguous row, or tokens interleaved with stride NT, as the packed
    // activations are), from a 16-byte aligned source, a multiple of 4 floats: 16 bytes per lane, a quarter of the
    // transfers. With fewer tokens than NT the padded tokens' columns are staged as they lie (never written by the up
    // kernel): only the padded tokens' sums read them, and those are never written.
    const bool contiguous = (NT == 1 && rstride == 1) || (rstride == NT && tstride == 1);
    if (contiguous && total % 4 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0) {
        for (uint32_t base = wave * kWave * 4; base < total; base += WAVES * kWave * 4)
            if (base + lane * 4 < total) dma16(src + base, lane * 16, lds + base);
        return;
    }
    for (uint32_t base = wave * kWave; base < total; base += WAVES * kWave) {
        const uint32_t r0 = base / NT;  // the piece's first row: its address is the wave-uniform base of the transfer
        const float* from = src + static_cast<size_t>(r0) * rstride;
        const uint32_t i = base + lane;
        if (i < total) {
            const uint32_t r = i / NT - r0, t = min(i % NT, tokens - 1);
            dma4(from, (r * rstride + t * tstride) * static_cast<uint32_t>(sizeof(float)), lds + base);
        }
    }
}

template <int NT, typename V, int G, typename Input>
__device__ __forceinline__ void accumulate_segment(const Segment<V, G>& seg, int32_t pb, int32_t pe, const Input& input,
                                                   float (&acc)[NT]) {
    constexpr int S = Group<V>::kSlots;
#pragma unroll
    for (int k = 0; k < G; ++k) {
        const int32_t g = seg.first + k * S * kWave;
        if (g < pe) {
#pragma unroll
            for (int s = 0; s < S; ++s) {
                if (g + s >= pb && g + s < pe) {
                    float xv[NT];
                    input.template load<NT>(index_at(seg.ids[k], s), xv);
                    const float w = Group<V>::at(seg.vals[k], s);
#pragma unroll
                    for (int t = 0; t < NT; ++t) acc[t] = fmaf(w, xv[t], acc[t]);
                }
            }
        }
    }
}

// Partial sums of one wave over slots [pb, pe) of a row, NT tokens, G groups per lane at a time (a chunk of 64 G
// groups): the first chunk's loads come from `first` (issued by the caller before the inputs were staged); the next
// chunks are loaded here.
template <int NT, typename V, int G, typename Input>
__device__ __forceinline__ void row_partials(const Segment<V, G>& first, const int16_t* __restrict__ idx,
                                             const V* __restrict__ val, int32_t pb, int32_t pe, int32_t nnz,
                                             const Input& input, uint32_t lane, float (&acc)[NT]) {
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
    accumulate_segment<NT>(first, pb, pe, input, acc);
    constexpr int S = Group<V>::kSlots;
    const int32_t span = G * S * kWave;
    for (uint32_t chunk = 1; (pb & ~(S - 1)) + static_cast<int32_t>(chunk) * span < pe; ++chunk) {
        Segment<V, G> seg;
        load_segment(seg, idx, val, pb, pe, nnz, lane, chunk);
        accumulate_segment<NT>(seg, pb, pe, input, acc);
    }
}

// Adds the wave's lane partials, then (P > 1) the block's P segment totals of the row in segment order; returns, in
// lane t < NT of the row's first wave, the row total of token t (other lanes: unspecified).
template <int NT, int P>
__device__ __forceinline__ float row_total(float (&acc)[NT], uint32_t lane, uint32_t part, uint32_t row_in_block,
                                           float* __restrict__ totals /* LDS [kWaves][NT] */) {
    float mine = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float s = wave_sum(acc[t]);
        if (lane == static_cast<uint32_t>(t)) mine = s;
    }
    if constexpr (P > 1) {
        const uint32_t wave = row_in_block * P + part;
        if (lane < NT) totals[wave * NT + lane] = mine;
        __syncthreads();
        if (part == 0 && lane < NT) {
            float s = totals[(row_in_block * P) * NT + lane];
#pragma unroll
            for (int p = 1; p < P; ++p) s += totals[(row_in_block * P + p) * NT + lane];
            mine = s;
        }
        __syncthreads();
    }
    return mine;
}

// Segment [pb, pe) of part `part` of a row [begin, end) split in P: the parts cut the row on the grid of S-slot
// groups, so each starts on a group boundary and no group is shared by two waves.
template <int P, int S>
__device__ __forceinline__ void segment(int32_t begin, int32_t end, uint32_t part, int32_t& pb, int32_t& pe) {
    if constexpr (P == 1) {
        pb = begin;
        pe = end;
    } else {
        const int32_t base = begin & ~(S - 1);
        const int32_t seg = ((end - base + P - 1) / P + S - 1) & ~(S - 1);
        const int32_t start = base + static_cast<int32_t>(part) * seg;
        pb = max(begin, min(end, start));
        pe = min(end, start + seg);
    }
}

// Row r's bias (0 past the rows, or without biases), requested with the row's slots so that the epilogue does not
// wait for it.
__device__ __forceinline__ float row_bias(const float* __restrict__ b, uint32_t r, uint32_t rows) {
    return b != nullptr && r < rows ? b[r] : 0.0f;
}

// A wave's first chunk of one row segment, requested ahead of its use.
template <typename V, int G>
struct Slots {
    Segment<V, G> seg;
    int32_t pb = 0, pe = 0;  // empty unless requested
};

// Requests the first chunk of part `part` of row r (nothing when r >= rows).
template <int P, typename V, int G>
__device__ __forceinline__ void request_row(Slots<V, G>& s, const int32_t* __restrict__ off, const int16_t* __restrict__ idx,
                                            const V* __restrict__ val, uint32_t r, uint32_t rows, uint32_t part, int32_t nnz,
                                            uint32_t lane) {
    if (r < rows) {
        segment<P, Group<V>::kSlots>(off[r], off[r + 1], part, s.pb, s.pe);
        load_segment(s.seg, idx, val, s.pb, s.pe, nnz, lane, 0);
    }
}


}  // namespace edges
}  // namespace hffn
