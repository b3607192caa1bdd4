// Tile-densified MFMA path of the HFFN forward (gfx950, v_mfma_f32_32x32x16_f16).
//
// At high density and large token counts a tile of neurons has a nearly dense union support, so the layer is two
// contractions: Z[N, d_ff] = X[N, d_model] W_up^T, A = gelu(Z + b_up), Y[N, d_model] = A W_down^T + b_down.
// The weights are densified once at load into fp16 "planes" (hi and lo parts, each row scaled by a power of two so
// that its largest entry lies in [1, 2)); activations are split the same way on the fly while they are staged in
// LDS, with one power of two per token row. Each product is  a_hi b_hi + a_hi b_lo + a_lo b_hi  accumulated in fp32
// by the MFMA units (the lo*lo term, ~2^-22 relative, is dropped; bf16 weights are exact in the hi plane and take
// the first two terms). The powers of two are undone exactly in the epilogue.
//
// Plane layout (K-chunk-major): k is cut into 32-wide k-tiles and each k-tile into four 16-byte chunks of 8 halves;
// for k-tile kt, part p (0 hi, 1 lo) and chunk c, the chunks of all rows follow one another:
//   planes[((((kt * 2 + p) * 4 + c) * rows + n) * 8 + k % 8]   with c = (k % 32) / 8.
// A block's B tile of BN rows is 8 runs of BN * 16 contiguous bytes, and LDS keeps the same order, so the MFMA
// operand reads (32 lanes on 32 consecutive rows of one chunk) and the staging writes touch consecutive 16-byte
// blocks: no LDS bank conflicts, no padding.
//
// GEMM blocks: 4 waves in 2 x 2, each wave a (32 MI) x (32 NI) tile of 32x32 MFMA accumulators; the k loop stages
// 32-wide k-tiles through double-buffered LDS (one barrier per k-tile, the next tile's global loads in flight during
// the current tile's MFMAs). The grid is one-dimensional and remapped so that each of the 8 XCDs works on one compact
// group of output tiles (its L2 then holds the A rows and B columns those tiles share). A down projection with very
// few output tiles splits K over 2 blocks per tile; the block that finishes a tile last (an integer counter per tile)
// adds the partials in split order, so the result does not depend on which block ends first.
//
// The up epilogue applies bias and exact GELU, writes the activations token-major [N, d_ff] in fp32, and, per token
// row and block of BN neurons, the binade of the largest activation; the down kernel takes, per token, the largest of
// those binades as its row scale.
#include "common.hpp"
#include "launch.hpp"

namespace hffn {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kBK = 32;          // k per staged step, one plane k-tile
constexpr int kRuns = 8;         // (part, chunk) runs of a k-tile
constexpr uint32_t kXcds = 8;    // MI355X: 8 XCDs, workgroups dispatched round-robin over them
constexpr uint32_t kGroupM = 4;  // output-tile rows per group of the tile order

// floor(log2(m)) of a non-negative float given by its bits; 0 for zero (any scale is exact for zeros).
__device__ __forceinline__ int binade_of_bits(uint32_t bits) {
    return bits == 0 ? 0 : static_cast<int>((bits >> 23) & 0xff) - 127;
}

__device__ __forceinline__ uint32_t abs_bits(float v) { return __float_as_uint(v) & 0x7fffffffu; }

__device__ __forceinline__ void split(float v, _Float16& hi, _Float16& lo) {
    hi = static_cast<_Float16>(v);
    lo = static_cast<_Float16>(v - static_cast<float>(hi));
}

// ------------------------------------------------------------------------------------------ row binades
// e[row] = binade of max |x[row, :]| ; one wave per row.
__global__ __launch_bounds__(kThreads) void row_binade_kernel(const float* __restrict__ x, uint32_t rows, uint32_t cols,
                                                             int32_t* __restrict__ e) {
    const uint32_t row = blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
    if (row >= rows) return;
    const uint32_t lane = threadIdx.x % kWave;
    const float* p = x + static_cast<size_t>(row) * cols;
    uint32_t m = 0;
    for (uint32_t c = lane; c < cols; c += kWave) m = max(m, abs_bits(p[c]));
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) m = max(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), s, kWave)));
    if (lane == 0) e[row] = binade_of_bits(m);
}

// --------------------------------------------------------------------------------------------- densify
// One block per row n of the dense matrix (a neuron of W_up, or an output of W_down^T) with its slots
// [off[n], off[n+1]) at columns idx[] (distinct within a row; the host checks it). Writes the whole row of both
// planes (zeros outside the support) and its binade.
template <typename V>
__global__ __launch_bounds__(kThreads) void densify_kernel(const int32_t* __restrict__ off, const int16_t* __restrict__ idx,
                                                          const V* __restrict__ val, uint32_t rows, uint32_t k,
                                                          _Float16* __restrict__ planes, int32_t* __restrict__ exps) {
    __shared__ uint32_t part[kThreads / kWave];
    const uint32_t n = blockIdx.x;
    const int32_t begin = off[n], end = off[n + 1];
    uint32_t m = 0;
    for (int32_t s = begin + static_cast<int32_t>(threadIdx.x); s < end; s += kThreads) m = max(m, abs_bits(widen(val[s])));
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) m = max(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), s, kWave)));
    if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = m;
    // zero this row's 16-byte chunk in every (k-tile, part, chunk) run
    const uint32_t runs = k / kBK * kRuns;
    for (uint32_t i = threadIdx.x; i < runs; i += kThreads)
        *reinterpret_cast<uint4*>(planes + (static_cast<size_t>(i) * rows + n) * 8) = make_uint4(0, 0, 0, 0);
    __syncthreads();
    uint32_t mx = 0;
#pragma unroll
    for (int w = 0; w < kThreads / kWave; ++w) mx = max(mx, part[w]);
    const int e = binade_of_bits(mx);
    for (int32_t s = begin + static_cast<int32_t>(threadIdx.x); s < end; s += kThreads) {
        const uint32_t c = static_cast<uint16_t>(idx[s]);
        _Float16 hi, lo;
        split(ldexpf(widen(val[s]), -e), hi, lo);
        const size_t run = static_cast<size_t>(c / kBK) * kRuns + (c % kBK) / 8;  // part 0
        planes[(run * rows + n) * 8 + c % 8] = hi;
        planes[((run + 4) * rows + n) * 8 + c % 8] = lo;
    }
    if (threadIdx.x == 0) exps[n] = e;
}

// ------------------------------------------------------------------------------------------------ GEMM
enum class Epi { Up, Down };

struct Tile {
    uint32_t m, n, split;
};

// Workgroup id -> (row tile, column tile, k split). The first 8 * floor(T / 8) ids are dealt so that XCD j (ids
// j, j + 8, ...) takes the j-th contiguous run of the tile order; the tile order walks groups of kGroupM tile rows
// column by column, so a run is a compact block of tiles.
__device__ __forceinline__ Tile tile_of(uint32_t id, uint32_t tiles_m, uint32_t tiles_n, uint32_t splits) {
    const uint32_t total = tiles_m * tiles_n * splits;
    const uint32_t per = total / kXcds;
    uint32_t t = id < kXcds * per ? (id % kXcds) * per + id / kXcds : id;
    const uint32_t per_split = tiles_m * tiles_n;
    Tile tile;
    tile.split = t / per_split;
    t %= per_split;
    const uint32_t group = t / (kGroupM * tiles_n);
    const uint32_t first = group * kGroupM;
    const uint32_t rows = min(tiles_m - first, kGroupM);
    const uint32_t within = t % (kGroupM * tiles_n);
    tile.m = first + within % rows;
    tile.n = within / rows;
    return tile;
}

template <int ARPT, int BRPT>
struct StageRegs {
    float4 a[ARPT][2];
    uint4 b[BRPT];
};

// Global loads of k-tile kt: 8 floats of A from rows row0 + 16 j (zeros past M), BRPT 16-byte chunks of B.
template <int ARPT, int BRPT>
__device__ __forceinline__ void load_stage(StageRegs<ARPT, BRPT>& r, const float* a_src, uint32_t row0, uint32_t M, uint32_t K,
                                           const _Float16* b_src, size_t b_stride, uint32_t kt) {
#pragma unroll
    for (int j = 0; j < ARPT; ++j) {
        if (row0 + 16 * j < M) {
            const float* p = a_src + static_cast<size_t>(16 * j) * K + kt * kBK;
            r.a[j][0] = *reinterpret_cast<const float4*>(p);
            r.a[j][1] = *reinterpret_cast<const float4*>(p + 4);
        } else {
            r.a[j][0] = make_float4(0.f, 0.f, 0.f, 0.f);
            r.a[j][1] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
#pragma unroll
    for (int j = 0; j < BRPT; ++j) r.b[j] = *reinterpret_cast<const uint4*>(b_src + kt * b_stride + 32 * j * 8);
}

// LDS stores of a staged k-tile: A split into hi/lo halves with its row's power of two, B copied.
template <int BM, int BN, int ARPT, int BRPT>
__device__ __forceinline__ void store_stage(const StageRegs<ARPT, BRPT>& r, _Float16* s_a, _Float16* s_b, uint32_t a_chunk,
                                            uint32_t a_row0, const int32_t* row_e, uint32_t b_run, uint32_t b_row) {
#pragma unroll
    for (int j = 0; j < ARPT; ++j) {
        const uint32_t row = a_row0 + 16 * j;
        const float scale = ldexpf(1.0f, -row_e[row]);
        const float v[8] = {r.a[j][0].x, r.a[j][0].y, r.a[j][0].z, r.a[j][0].w, r.a[j][1].x, r.a[j][1].y, r.a[j][1].z, r.a[j][1].w};
        half8 h, l;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            _Float16 hh, ll;
            split(v[e] * scale, hh, ll);
            h[e] = hh;
            l[e] = ll;
        }
        *reinterpret_cast<half8*>(s_a + (a_chunk * BM + row) * 8) = h;
        *reinterpret_cast<half8*>(s_a + ((4 + a_chunk) * BM + row) * 8) = l;
    }
#pragma unroll
    for (int j = 0; j < BRPT; ++j) *reinterpret_cast<uint4*>(s_b + (b_run * BN + b_row + 32 * j) * 8) = r.b[j];
}

template <Epi EPI, int MI, int NI, bool LO_B, int SPLITS>
__global__ __launch_bounds__(kThreads) void gemm_split_kernel(
    const float* __restrict__ a,          // [M, K] fp32 row-major
    const int32_t* __restrict__ a_exp,    // Up: [M] row binades; Down: [M, a_blocks] block binades (max taken here)
    uint32_t a_blocks,
    const _Float16* __restrict__ planes,  // tile-major planes of B [Ncol, K]
    const int32_t* __restrict__ b_exp,    // [Ncol]
    const float* __restrict__ bias,       // [Ncol]
    float* __restrict__ out,              // [M, Ncol] fp32 row-major
    int32_t* __restrict__ out_exp,        // Up: [M, Ncol / BN] activation block binades
    float* __restrict__ partials,         // SPLITS > 1: [SPLITS, M, Ncol] scaled partial sums
    int32_t* __restrict__ counters,       // SPLITS > 1: [tiles], zero between calls
    uint32_t M, uint32_t Ncol, uint32_t K) {
    constexpr int BM = 64 * MI, BN = 64 * NI;
    constexpr int ARPT = BM / 64;                    // A rows per staging thread (16 rows x 4 chunks per wave pass)
    constexpr int BRPT = BN / 32;                    // B rows per staging thread (32 rows x 8 runs per block pass)

    // [buffer][part][chunk][row][8 halves]
    __shared__ __attribute__((aligned(16))) _Float16 s_a[2][kRuns * BM * 8];
    __shared__ __attribute__((aligned(16))) _Float16 s_b[2][kRuns * BN * 8];
    __shared__ int32_t row_e[BM];
    __shared__ uint32_t row_max[2][BM];
    __shared__ int32_t last;

    const uint32_t tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    const uint32_t wm = wave / 2, wn = wave % 2;
    const uint32_t tiles_m = (M + BM - 1) / BM, tiles_n = Ncol / BN;
    const Tile tile = tile_of(blockIdx.x, tiles_m, tiles_n, SPLITS);
    const uint32_t m0 = tile.m * BM, n0 = tile.n * BN;
    const uint32_t ktiles = K / kBK;
    const uint32_t k_begin = tile.split * ktiles / SPLITS, k_end = (tile.split + 1) * ktiles / SPLITS;

    if (tid < BM) {
        const uint32_t row = m0 + tid;
        int e = 0;
        if (row < M) {
            if constexpr (EPI == Epi::Up) {
                e = a_exp[row];
            } else {
                e = -1000;
                for (uint32_t b = 0; b < a_blocks; ++b) e = max(e, a_exp[static_cast<size_t>(row) * a_blocks + b]);
            }
        }
        row_e[tid] = e;
    }
    __syncthreads();

    // staging assignments. A: lane l of wave w converts chunk l / 16 (8 floats) of rows w * 16 * ARPT + l % 16 + 16 j;
    // B: thread t copies run t / 32 of rows t % 32 + 32 j.
    const uint32_t a_chunk = lane / 16, a_row0 = wave * 16 * ARPT + lane % 16;
    const float* a_src = a + static_cast<size_t>(m0 + a_row0) * K + a_chunk * 8;
    const uint32_t b_run = tid / 32, b_row = tid % 32;
    const _Float16* b_src = planes + (static_cast<size_t>(b_run) * Ncol + n0 + b_row) * 8;
    const size_t b_stride = static_cast<size_t>(kRuns) * Ncol * 8;  // halves per k-tile
    StageRegs<ARPT, BRPT> regs;

    floatx16 acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    if (k_begin < k_end) {
        load_stage<ARPT, BRPT>(regs, a_src, m0 + a_row0, M, K, b_src, b_stride, k_begin);
        store_stage<BM, BN, ARPT, BRPT>(regs, s_a[0], s_b[0], a_chunk, a_row0, row_e, b_run, b_row);
        if (k_begin + 1 < k_end) load_stage<ARPT, BRPT>(regs, a_src, m0 + a_row0, M, K, b_src, b_stride, k_begin + 1);
        __syncthreads();
    }
    for (uint32_t kt = k_begin; kt < k_end; ++kt) {
        const int buf = (kt - k_begin) & 1;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const uint32_t chunk = kk * 2 + lane / 32;
            half8 ah[MI], al[MI], bh[NI], bl[NI];
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                const uint32_t r = wm * (BM / 2) + i * 32 + lane % 32;
                ah[i] = *reinterpret_cast<const half8*>(s_a[buf] + (chunk * BM + r) * 8);
                al[i] = *reinterpret_cast<const half8*>(s_a[buf] + ((4 + chunk) * BM + r) * 8);
            }
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                const uint32_t r = wn * (BN / 2) + j * 32 + lane % 32;
                bh[j] = *reinterpret_cast<const half8*>(s_b[buf] + (chunk * BN + r) * 8);
                if constexpr (LO_B) bl[j] = *reinterpret_cast<const half8*>(s_b[buf] + ((4 + chunk) * BN + r) * 8);
            }
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NI; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bh[j], acc[i][j], 0, 0, 0);
                    if constexpr (LO_B) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bl[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], bh[j], acc[i][j], 0, 0, 0);
                }
        }
        if (kt + 1 < k_end) {
            store_stage<BM, BN, ARPT, BRPT>(regs, s_a[buf ^ 1], s_b[buf ^ 1], a_chunk, a_row0, row_e, b_run, b_row);
            if (kt + 2 < k_end) load_stage<ARPT, BRPT>(regs, a_src, m0 + a_row0, M, K, b_src, b_stride, kt + 2);
        }
        __syncthreads();
    }

    // epilogue: accumulator r of lane l of tile (i, j) holds row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32
    if constexpr (EPI == Epi::Up) {
        uint32_t lane_max[MI][16];
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) lane_max[i][r] = 0;
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const uint32_t col = n0 + wn * (BN / 2) + j * 32 + lane % 32;
            const int ce = b_exp[col];
            const float cb = bias[col];
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t m = wm * (BM / 2) + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
                    const float v = gelu(ldexpf(acc[i][j][r], row_e[m] + ce) + cb);
                    lane_max[i][r] = max(lane_max[i][r], abs_bits(v));
                    if (m0 + m < M) out[static_cast<size_t>(m0 + m) * Ncol + col] = v;
                }
        }
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                uint32_t v = lane_max[i][r];
#pragma unroll
                for (int s = 16; s >= 1; s >>= 1) v = max(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), s, kWave)));
                if (lane % 32 == 0) row_max[wn][wm * (BM / 2) + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4] = v;
            }
        __syncthreads();
        if (tid < BM && m0 + tid < M)
            out_exp[static_cast<size_t>(m0 + tid) * tiles_n + tile.n] = binade_of_bits(max(row_max[0][tid], row_max[1][tid]));
    } else if constexpr (SPLITS == 1) {
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const uint32_t col = n0 + wn * (BN / 2) + j * 32 + lane % 32;
            const int ce = b_exp[col];
            const float cb = bias[col];
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t m = wm * (BM / 2) + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
                    if (m0 + m < M) out[static_cast<size_t>(m0 + m) * Ncol + col] = ldexpf(acc[i][j][r], row_e[m] + ce) + cb;
                }
        }
    } else {
        // every split writes its scaled partial, then the block that completes the tile adds them in split order
        const size_t plane_size = static_cast<size_t>(M) * Ncol;
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const uint32_t col = n0 + wn * (BN / 2) + j * 32 + lane % 32;
            const int ce = b_exp[col];
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t m = wm * (BM / 2) + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
                    acc[i][j][r] = ldexpf(acc[i][j][r], row_e[m] + ce);
                    if (m0 + m < M) partials[tile.split * plane_size + static_cast<size_t>(m0 + m) * Ncol + col] = acc[i][j][r];
                }
        }
        __threadfence();
        __syncthreads();
        if (tid == 0) {
            const uint32_t counter = tile.m * tiles_n + tile.n;
            const int32_t arrived = atomicAdd(&counters[counter], 1);
            last = arrived == SPLITS - 1;
            if (last) counters[counter] = 0;  // every split of this tile has arrived: ready for the next call
        }
        __syncthreads();
        if (!last) return;
        __threadfence();
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const uint32_t col = n0 + wn * (BN / 2) + j * 32 + lane % 32;
            const float cb = bias[col];
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t m = wm * (BM / 2) + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
                    if (m0 + m >= M) continue;
                    const size_t at = static_cast<size_t>(m0 + m) * Ncol + col;
                    float total = 0.0f;
#pragma unroll
                    for (int s = 0; s < SPLITS; ++s) {
                        const float p = s == static_cast<int>(tile.split)
                                            ? acc[i][j][r]
                                            : __hip_atomic_load(partials + s * plane_size + at, __ATOMIC_RELAXED,
                                                                __HIP_MEMORY_SCOPE_AGENT);
                        total = s == 0 ? p : total + p;
                    }
                    out[at] = total + cb;
                }
        }
    }
}

uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

struct Shape {
    int mi, ni, splits;  // wave tile (32 mi) x (32 ni), block tile (64 mi) x (64 ni), k splits
};

constexpr int kMaxSplits = 4;

// Measured on the Pythia-410M layer at N = 2048: up 128 x 128 blocks (80 us); down 64 x 128 blocks without a k
// split (91 us; 128 x 128 with 2 splits: 131 us, the fixup's device-scope fences write back the L2). K is split only
// when a down projection has fewer than 64 blocks.
Shape up_shape(uint32_t, uint32_t) { return {2, 2, 1}; }

Shape down_shape(uint32_t m, uint32_t ncol, uint32_t k) {
    const uint32_t tiles = ceil_div(m, 64) * (ncol / 128);
    return {1, 2, tiles < 64 && k >= 2048 ? 2 : 1};
}

template <Epi EPI, bool LO_B, int MI, int NI, int SPLITS>
hipError_t launch_gemm(const float* a, const int32_t* a_exp, uint32_t a_blocks, const _Float16* planes, const int32_t* b_exp,
                       const float* bias, float* out, int32_t* out_exp, float* partials, int32_t* counters, uint32_t M,
                       uint32_t Ncol, uint32_t K, hipStream_t stream) {
    const uint32_t tiles = ceil_div(M, 64 * MI) * (Ncol / (64 * NI));
    hipLaunchKernelGGL((gemm_split_kernel<EPI, MI, NI, LO_B, SPLITS>), dim3(tiles * SPLITS), dim3(kThreads), 0, stream, a, a_exp,
                       a_blocks, planes, b_exp, bias, out, out_exp, partials, counters, M, Ncol, K);
    return hipGetLastError();
}

// The instantiated shapes: up (mi, ni) in {(2,2), (2,4), (4,2), (1,2)} without splits; down (2,2) and (1,2) with
// 1, 2 or 4 splits and (2,4) with 1 or 2.
template <Epi EPI, bool LO_B>
hipError_t gemm(Shape shape, const float* a, const int32_t* a_exp, uint32_t a_blocks, const _Float16* planes, const int32_t* b_exp,
                const float* bias, float* out, int32_t* out_exp, float* partials, int32_t* counters, uint32_t M, uint32_t Ncol,
                uint32_t K, hipStream_t stream) {
#define HFFN_GEMM(MI, NI, S)                                                                                                \
    if (shape.mi == MI && shape.ni == NI && shape.splits == S)                                                              \
        return launch_gemm<EPI, LO_B, MI, NI, S>(a, a_exp, a_blocks, planes, b_exp, bias, out, out_exp, partials, counters, \
                                                 M, Ncol, K, stream);
    if constexpr (EPI == Epi::Up) {
        HFFN_GEMM(2, 2, 1)
        HFFN_GEMM(2, 4, 1)
        HFFN_GEMM(4, 2, 1)
        HFFN_GEMM(1, 2, 1)
    } else {
        HFFN_GEMM(2, 2, 1)
        HFFN_GEMM(2, 2, 2)
        HFFN_GEMM(2, 2, 4)
        HFFN_GEMM(1, 2, 1)
        HFFN_GEMM(1, 2, 2)
        HFFN_GEMM(1, 2, 4)
        HFFN_GEMM(2, 4, 1)
        HFFN_GEMM(2, 4, 2)
    }
#undef HFFN_GEMM
    return hipErrorInvalidValue;
}

// Workspace layout (int32 words unless stated): split counters [down tiles of the largest token count, 64 x 64 tiles]
// | x binades [M] | activation block binades [M, d_ff / 64] | (256-byte aligned) float partials [4, M, d_model].
// The counters come first and are sized for every M and tile shape, so a call at any M finds them where the previous
// call, at any other M, left them (at zero).
struct Workspace {
    size_t counters, x_binades, act_binades, partials, bytes;
};

Workspace workspace_layout(uint32_t m, uint32_t d, uint32_t h) {
    Workspace w{};
    w.counters = 0;
    const size_t counter_words = static_cast<size_t>(ceil_div(kMaxTokens, 64)) * (d / 64);
    w.x_binades = w.counters + counter_words;
    w.act_binades = w.x_binades + m;
    const size_t partial_start = (w.act_binades + static_cast<size_t>(m) * (h / 64)) * 4;
    w.partials = (partial_start + 255) / 256 * 256;  // bytes
    w.bytes = w.partials + static_cast<size_t>(kMaxSplits) * m * d * 4;
    return w;
}

}  // namespace

size_t dense_plane_halves(uint32_t rows, uint32_t k) { return static_cast<size_t>(rows) * k * 2; }

bool mfma_shape_supported(uint32_t d, uint32_t h) { return d % 256 == 0 && h % 256 == 0; }

size_t mfma_workspace_bytes(uint32_t n, uint32_t d, uint32_t h) { return workspace_layout(n, d, h).bytes; }

hipError_t launch_densify(int vt, const int32_t* off, const int16_t* idx, const void* val, uint32_t rows, uint32_t k,
                          void* planes, int32_t* exps, hipStream_t stream) {
    if (vt == kBF16)
        hipLaunchKernelGGL((densify_kernel<uint16_t>), dim3(rows), dim3(kThreads), 0, stream, off, idx,
                           static_cast<const uint16_t*>(val), rows, k, static_cast<_Float16*>(planes), exps);
    else
        hipLaunchKernelGGL((densify_kernel<float>), dim3(rows), dim3(kThreads), 0, stream, off, idx,
                           static_cast<const float*>(val), rows, k, static_cast<_Float16*>(planes), exps);
    return hipGetLastError();
}

hipError_t launch_mfma_up(int vt, const float* x, const void* planes, const int32_t* w_exp, const float* b_up, float* act,
                          void* workspace, uint32_t n, uint32_t d, uint32_t h, hipStream_t stream) {
    const Workspace w = workspace_layout(n, d, h);
    int32_t* words = static_cast<int32_t*>(workspace);
    hipLaunchKernelGGL(row_binade_kernel, dim3(ceil_div(n, kThreads / kWave)), dim3(kThreads), 0, stream, x, n, d,
                       words + w.x_binades);
    if (hipError_t status = hipGetLastError(); status != hipSuccess) return status;
    const auto* p = static_cast<const _Float16*>(planes);
    const Shape shape = up_shape(n, h);
    if (vt == kBF16)
        return gemm<Epi::Up, false>(shape, x, words + w.x_binades, 1, p, w_exp, b_up, act, words + w.act_binades, nullptr,
                                    nullptr, n, h, d, stream);
    return gemm<Epi::Up, true>(shape, x, words + w.x_binades, 1, p, w_exp, b_up, act, words + w.act_binades, nullptr, nullptr,
                               n, h, d, stream);
}

hipError_t launch_mfma_down(int vt, const float* act, const void* planes, const int32_t* v_exp, const float* b_down, float* y,
                            void* workspace, uint32_t n, uint32_t d, uint32_t h, hipStream_t stream) {
    const Workspace w = workspace_layout(n, d, h);
    int32_t* words = static_cast<int32_t*>(workspace);
    float* partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + w.partials);
    const auto* p = static_cast<const _Float16*>(planes);
    const Shape shape = down_shape(n, d, h);
    const uint32_t blocks = h / (64 * up_shape(n, h).ni);
    if (vt == kBF16)
        return gemm<Epi::Down, false>(shape, act, words + w.act_binades, blocks, p, v_exp, b_down, y, nullptr, partials,
                                      words + w.counters, n, d, h, stream);
    return gemm<Epi::Down, true>(shape, act, words + w.act_binades, blocks, p, v_exp, b_down, y, nullptr, partials,
                                 words + w.counters, n, d, h, stream);
}

}  // namespace hffn
