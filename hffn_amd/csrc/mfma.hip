// Tile-densified MFMA path of the HFFN forward (gfx950, v_mfma_f32_32x32x16_f16).
//
// At high density and large token counts a tile of neurons has a nearly dense union support, so the layer is two
// contractions: Z[N, d_ff] = X[N, d_model] W_up^T, A = gelu(Z + b_up), Y[N, d_model] = A W_down^T + b_down.
// Every operand enters the MFMA units as a pair of fp16 "planes" (hi and lo parts) scaled by powers of two: the
// weights are densified once at load (one power of two per row, so that its largest entry lies in [1, 2)); the input
// X is split by a small kernel before the up GEMM (one power of two per token); the activations are split by the up
// GEMM's epilogue (one power of two per token and 128-neuron block). Each product is  a_hi b_hi + a_hi b_lo +
// a_lo b_hi  accumulated in fp32 (the lo*lo term, ~2^-22 relative, is dropped; bf16 weights take the first and last
// terms on the hi plane only, which holds them exactly down to 2^-14 of their row's largest magnitude; below that
// fp16 subnormals keep fewer bits, at most ~2^-25 of that magnitude per weight). The powers of two are undone
// exactly: the down GEMM rescales its accumulators at each 128-wide k block by the ratio of the blocks' powers of
// two, and the epilogues apply the last.
//
// Plane layout (K-chunk-major): k is cut into 32-wide k-tiles and each k-tile into four 16-byte chunks of 8 halves;
// for k-tile kt, part p (0 hi, 1 lo) and chunk c, the chunks of all rows follow one another:
//   planes[((((kt * 2 + p) * 4 + c) * rows + n) * 8 + k % 8]   with c = (k % 32) / 8.
// A block's tile of B rows is 8 runs of B * 16 contiguous bytes, and LDS keeps the same order, so the MFMA operand
// reads (32 lanes on 32 consecutive rows of one chunk) and the staging writes touch consecutive 16-byte blocks: no
// LDS bank conflicts, no padding. Token planes have a row count padded to kRowPad (rows past N are zeros in X and
// hold gelu(b_up) in A; their outputs are never stored); a call of at most 64 or 128 tokens writes and reads only
// the first 64 or 128 rows (rows_live).
//
// Two GEMM kernels: the streamed one (gemm_dma_kernel: 256 x 128 tiles whose k-tiles go from global memory straight
// into LDS, K split 2-32 ways by an estimate of the rounds of blocks and the partials' cost, partials added by
// separate passes; a down GEMM may take its first column tiles over all of K and split only the others) takes every
// shape whose tiles and splits give enough blocks; the register-staged one below (gemm_planes_kernel) remains for
// narrower layers at small N.
//
// Register-staged GEMM blocks: 4 waves in 2 x 2, each wave a (32 MI) x (32 NI) tile of 32x32 MFMA accumulators; the k loop stages
// 32-wide k-tiles of both planes through double-buffered LDS with plain 16-byte copies (one barrier per k-tile, the
// next tile's global loads in flight during the current tile's MFMAs). The grid is one-dimensional and remapped so
// that each of the 8 XCDs works on one compact group of output tiles (its L2 then holds the A rows and B columns
// those tiles share). A down projection with very few output tiles splits K over 2 blocks per tile; the block that
// finishes a tile last (an integer counter per tile) adds the partials in split order, so the result does not depend
// on which block ends first.
#include "common.hpp"
#include "launch.hpp"

namespace hffn {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // 16 bytes of plane: 8 halves

constexpr int kThreads = 256;
constexpr int kBK = 32;          // k per staged step, one plane k-tile
constexpr int kRuns = 8;         // (part, chunk) runs of a k-tile
constexpr uint32_t kXcds = 8;    // MI355X: 8 XCDs, workgroups dispatched round-robin over them
constexpr uint32_t kGroupM = 4;  // output-tile rows per group of the tile order
constexpr uint32_t kRowPad = 256;  // token planes hold a multiple of this many rows
constexpr uint32_t kActBlock = 128;  // neurons per activation power of two (the up GEMM's column tile)
constexpr uint32_t kKtPerActBlock = kActBlock / kBK;

// Every plane row (a token's inputs, a weight row, a token's activation block) is stored as hi + lo = v * 2^-e, e
// its power of two. e puts the row's largest |v| at 2^kPlaneLift .. 2^(kPlaneLift + 1) (below fp16's 65504 with room
// to spare), far above fp16's smallest normal 2^-14: lo, the residual of hi (at most 2^-11 of |hi|), is then a
// normal fp16 for every entry down to 2^-(kPlaneLift + 3) of the row's largest, and below that its absolute error
// (2^-25 after scaling) is 2^-(25 + kPlaneLift) of the largest. Scaled products stay below 2^26 per term, so fp32
// accumulation has no overflow at any K. Whoever reads a plane undoes e exactly (ldexp), so the lift is invisible
// outside the planes.
constexpr int kPlaneLift = 12;
// binades are clamped to +-kBinadeClamp before the lift: 2^(kBinadeClamp + kPlaneLift) is a finite float scale, and an
// activation block's binade fits an int8 (a row of only tiny entries, below 2^-100, keeps less than fp32's precision)
constexpr int kBinadeClamp = 100;

// floor(log2(m)) - kPlaneLift of a non-negative float given by its bits (clamped); -kPlaneLift for zero (any scale is
// exact for zeros). inf and NaN give the clamp's top, which scales them to themselves.
__device__ __forceinline__ int binade_of_bits(uint32_t bits) {
    const int e = bits == 0 ? 0 : static_cast<int>((bits >> 23) & 0xff) - 127;
    return min(max(e, -kBinadeClamp), kBinadeClamp) - kPlaneLift;
}

// Power of two of an activation block (a token's kActBlock neurons): binade_of_bits of its largest |v| rounded up to a
// multiple of kActBinadeStep (kPlaneLift is one, so the rounding is that of the true binade). The block's largest
// value scaled lies in 2^(kPlaneLift - 3) .. 2^(kPlaneLift + 1); neighbouring blocks of a token then mostly share their
// power of two, and the down GEMM has nothing to rescale between them. Range: -112 .. 88, an int8.
constexpr int kActBinadeStep = 4;
static_assert(kPlaneLift % kActBinadeStep == 0, "the lift keeps activation binades on their grid");
static_assert(kBinadeClamp + kPlaneLift + kActBinadeStep < 128, "activation binades fit an int8");
__device__ __forceinline__ int act_binade(uint32_t bits) {
    const int e = binade_of_bits(bits);
    return e >= 0 ? (e + kActBinadeStep - 1) / kActBinadeStep * kActBinadeStep : -(-e / kActBinadeStep * kActBinadeStep);
}

// Activation block binades are int8 (multiples of kActBinadeStep, -112 .. 88), block-major [d_ff / kActBlock][rows_pad]:
// the down GEMM transfers each activation block's binades of its 256 rows, one contiguous 256-byte run, straight into
// LDS. They travel through the GEMMs' int32 binade pointers (Up: out_exp; Down: a_exp), read and written as bytes.
__device__ __forceinline__ size_t act_exp_at(uint32_t rows_pad, uint32_t m, uint32_t block) {
    return static_cast<size_t>(block) * rows_pad + m;
}
__device__ __forceinline__ const int8_t* act_exps(const int32_t* p) { return reinterpret_cast<const int8_t*>(p); }
__device__ __forceinline__ int8_t* act_exps(int32_t* p) { return reinterpret_cast<int8_t*>(p); }

__device__ __forceinline__ uint32_t abs_bits(float v) { return __float_as_uint(v) & 0x7fffffffu; }

__device__ __forceinline__ void split(float v, _Float16& hi, _Float16& lo) {
    hi = static_cast<_Float16>(v);
    lo = static_cast<_Float16>(v - static_cast<float>(hi));
}

// Index of element (row, k) of part p (0 hi, 1 lo) in planes of `rows` rows.
__device__ __forceinline__ size_t plane_at(uint32_t rows, uint32_t row, uint32_t k, uint32_t p) {
    return ((static_cast<size_t>(k / kBK) * kRuns + p * 4 + (k % kBK) / 8) * rows + row) * 8 + k % 8;
}

// ------------------------------------------------------------------------------------------ input planes
// X [M, K] fp32 (row stride ld; entries at k >= k_real read as zeros) -> planes of X [rows_pad, K] and e[row] =
// binade of max |x[row, :]| (rows M .. 8 * gridDim.x: zeros, e = -kPlaneLift; K a multiple of 256). A block takes 8 rows; its wave w takes k in [w K/4, (w + 1) K/4) in steps of 64,
// up to 4 steps (a chunk) at a time: in a step, lane l holds 8 consecutive k (piece l / 8) of row l % 8, so that the
// 8 lanes of a row read 256 contiguous bytes of it and the 8 lanes of a piece write the 8 rows' 16 bytes of one
// 128-byte run of the planes. First the row maxima (lanes, then the 4 waves through LDS), then the split; a wave
// whose range is one chunk keeps its values in registers, longer ranges are read again (from L2).
constexpr uint32_t kSplitBlockRows = 8;
constexpr uint32_t kSplitChunk = 256;  // k per chunk: 4 steps of 64
__global__ __launch_bounds__(kThreads) void split_rows_kernel(const float* __restrict__ x, uint32_t M, uint32_t rows_pad,
                                                             uint32_t K, uint32_t ld, uint32_t k_real, _Float16* __restrict__ planes,
                                                             int32_t* __restrict__ e) {
    constexpr uint32_t kWaves = kThreads / kWave;
    __shared__ uint32_t part[kWaves][kSplitBlockRows];
    const uint32_t lane = threadIdx.x % kWave, wave = uniform(threadIdx.x / kWave);
    const uint32_t r = lane % kSplitBlockRows, piece = lane / kSplitBlockRows;
    const uint32_t row = blockIdx.x * kSplitBlockRows + r;
    const uint32_t span = K / kWaves, k_begin = wave * span, k_end = k_begin + span;
    const float* src = x + static_cast<size_t>(row) * ld;
    const bool real = row < M;
    float v[4][8];
    const auto load_chunk = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
            const uint32_t k = k0 + 64 * i + 8 * piece;
            if (real && k0 + 64 * i < k_end && k < k_real) {
                const float* q = src + k;
                if (k + 8 <= k_real) {
                    a = *reinterpret_cast<const float4*>(q);
                    b = *reinterpret_cast<const float4*>(q + 4);
                } else {  // a piece across the end of the real columns: only those are read (the row may end there)
                    const uint32_t valid = k_real - k;
                    a.x = q[0];
                    if (valid > 1) a.y = q[1];
                    if (valid > 2) a.z = q[2];
                    if (valid > 3) a.w = q[3];
                    if (valid > 4) b.x = q[4];
                    if (valid > 5) b.y = q[5];
                    if (valid > 6) b.z = q[6];
                }
            }
            v[i][0] = a.x; v[i][1] = a.y; v[i][2] = a.z; v[i][3] = a.w;
            v[i][4] = b.x; v[i][5] = b.y; v[i][6] = b.z; v[i][7] = b.w;
        }
    };
    uint32_t m = 0;
    for (uint32_t k0 = k_begin; k0 < k_end; k0 += kSplitChunk) {
        load_chunk(k0);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int q = 0; q < 8; ++q) m = max(m, abs_bits(v[i][q]));
    }
#pragma unroll
    for (int s = kSplitBlockRows; s < kWave; s <<= 1) m = max(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), s, kWave)));
    if (piece == 0) part[wave][r] = m;
    __syncthreads();
    uint32_t mx = part[0][r];
#pragma unroll
    for (uint32_t w = 1; w < kWaves; ++w) mx = max(mx, part[w][r]);
    const int be = binade_of_bits(mx);
    if (wave == 0 && piece == 0) e[row] = be;
    const float scale = ldexpf(1.0f, -be);
    for (uint32_t k0 = k_begin; k0 < k_end; k0 += kSplitChunk) {
        if (span > kSplitChunk) load_chunk(k0);  // one chunk: still in registers
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (k0 + 64 * i >= k_end) break;
            half8 h, l;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                _Float16 hh, ll;
                split(v[i][q] * scale, hh, ll);
                h[q] = hh;
                l[q] = ll;
            }
            const uint32_t k = k0 + 64 * i + 8 * piece;
            *reinterpret_cast<half8*>(planes + plane_at(rows_pad, row, k, 0)) = h;
            *reinterpret_cast<half8*>(planes + plane_at(rows_pad, row, k, 1)) = l;
        }
    }
}

// --------------------------------------------------------------------------------------------- densify
// Row n of the dense matrix (a neuron of W_up, or an output of W_down^T) has its slots [off[n], off[n+1]) at columns
// idx[] (distinct within a row; the host checks it); densifying writes the whole row of both planes (zeros outside
// the support) and its binade. A block takes kDensRows consecutive rows and kDensChunk columns (blockIdx.y): the rows'
// maxima (two waves per row, over all their slots), then their hi/lo parts in its columns assembled in LDS (zeroed
// meanwhile, then each slot of the chunk in its column) and written out whole: for every 16-byte chunk run the block's rows are
// kDensRows consecutive 16-byte pieces, one 128-byte line per (run, row group). The rows are padded by 16 bytes in
// LDS so that the eight rows of a chunk fall in different banks; the tile (66 KB) leaves room for two blocks per CU.
constexpr uint32_t kDensRows = 8, kDensChunk = 2048, kDensThreads = 1024, kDensPad = 8;
template <typename V>
__global__ __launch_bounds__(kDensThreads) void densify_kernel(const int32_t* __restrict__ off, const int16_t* __restrict__ idx,
                                                              const V* __restrict__ val, uint32_t rows, uint32_t k,
                                                              _Float16* __restrict__ planes, int32_t* __restrict__ exps) {
    const auto value = [&](int32_t s) { return widen(val[s]); };
    static_assert(kDensRows * 16 == 128, "a row group's pieces of one chunk run fill one 128-byte line");
    __shared__ __attribute__((aligned(16))) _Float16 tile[2][kDensRows][kDensChunk + kDensPad];
    __shared__ uint32_t row_max[2][kDensRows];
    constexpr uint32_t kWaves = kDensThreads / kWave;
    static_assert(kWaves == 2 * kDensRows, "two waves per row");
    const uint32_t tid = threadIdx.x, lane = tid % kWave, wave = uniform(tid / kWave);
    const uint32_t row = wave % kDensRows, half = wave / kDensRows;  // wave-uniform
    const uint32_t r0 = blockIdx.x * kDensRows, n = r0 + row;
    const uint32_t c0 = blockIdx.y * kDensChunk;
    const uint32_t width = min(kDensChunk, k - c0), pieces = width / 8;  // width: a multiple of 32
    // the block's tile zeroed while the slots are in flight
    for (uint32_t i = tid; i < 2 * kDensRows * pieces; i += kDensThreads) {
        const uint32_t part = i / (kDensRows * pieces), rr = (i / pieces) % kDensRows, j = i % pieces;
        *reinterpret_cast<uint4*>(&tile[part][rr][j * 8]) = make_uint4(0, 0, 0, 0);
    }
    // Waves w and w + kDensRows take row r0 + w, slots interleaved by 64 (lane l of half h: begin + 64 h + l + 128 q).
    // A row of at most kHeld slots per lane is read once, into registers, for both its maximum and its scatter; a
    // longer row is read twice, kBatch slots per lane in flight. The two halves' maxima meet in LDS.
    constexpr int kHeld = 16, kBatch = 16, kStride = 2 * kWave;
    const int32_t begin = n < rows ? off[n] : 0, end = n < rows ? off[n + 1] : 0;
    const int32_t first = begin + static_cast<int32_t>(half * kWave + lane);
    const bool held = end - begin <= kHeld * kStride;  // wave-uniform
    uint32_t hc[kHeld];
    float hw[kHeld];
    uint32_t m = 0;
    if (held) {
#pragma unroll
        for (int q = 0; q < kHeld; ++q) {
            const int32_t s = first + q * kStride;
            const bool in = s < end;
            hc[q] = in ? static_cast<uint16_t>(idx[s]) : 0xFFFFFFFFu;
            hw[q] = in ? value(s) : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < kHeld; ++q) m = max(m, abs_bits(hw[q]));
    } else {
        // a batch's loads all issued before the first is used: a slot past the row reads the row's last slot again
        // (a value of the row: the maximum is unchanged)
        for (int32_t s0 = first; s0 < end; s0 += kBatch * kStride) {
            float w[kBatch];
#pragma unroll
            for (int q = 0; q < kBatch; ++q) w[q] = value(min(s0 + q * kStride, end - 1));
#pragma unroll
            for (int q = 0; q < kBatch; ++q) m = max(m, abs_bits(w[q]));
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = max(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), o, kWave)));
    if (lane == 0) row_max[half][row] = m;
    __syncthreads();  // the tile is zeroed, the halves' maxima are in
    const int e = binade_of_bits(max(row_max[0][row], row_max[1][row]));
    const auto place = [&](uint32_t c, float w) {
        if (c < c0 || c >= c0 + width) return;  // another column block's slot, or past the row
        _Float16 hi, lo;
        split(ldexpf(w, -e), hi, lo);
        tile[0][row][c - c0] = hi;
        tile[1][row][c - c0] = lo;
    };
    if (held) {
#pragma unroll
        for (int q = 0; q < kHeld; ++q) place(hc[q], hw[q]);
    } else {
        for (int32_t s0 = first; s0 < end; s0 += kBatch * kStride) {
            uint32_t c[kBatch];
            float w[kBatch];
#pragma unroll
            for (int q = 0; q < kBatch; ++q) {  // past the row: its last slot again (placed again, the same cell and value)
                const int32_t at = min(s0 + q * kStride, end - 1);
                c[q] = static_cast<uint16_t>(idx[at]);
                w[q] = value(at);
            }
#pragma unroll
            for (int q = 0; q < kBatch; ++q) place(c[q], w[q]);
        }
    }
    __syncthreads();
    for (uint32_t i = tid; i < 2 * pieces * kDensRows; i += kDensThreads) {
        const uint32_t rr = i % kDensRows, j = (i / kDensRows) % pieces, part = i / (kDensRows * pieces);
        if (r0 + rr < rows)
            *reinterpret_cast<uint4*>(planes + plane_at(rows, r0 + rr, c0 + j * 8, part)) =
                *reinterpret_cast<const uint4*>(&tile[part][rr][j * 8]);
    }
    if (blockIdx.y == 0 && half == 0 && lane == 0 && n < rows) exps[n] = e;
}

// ------------------------------------------------------------------------------------------------ GEMM
// Up: the up GEMM with the GELU epilogue writing activation planes. Down: the down GEMM writing y or split partials.
// UpSplit: the up GEMM over a k split, writing fp32 partial sums (no bias, no GELU) for act_planes_kernel.
enum class Epi { Up, Down, UpSplit };

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

// One k-tile of a block's operands in flight: ARPT 16-byte chunks of the A planes and BRPT of the B planes per thread.
template <int ARPT, int BRPT>
struct StageRegs {
    u32x4 a[ARPT];
    u32x4 b[BRPT];
};

// Global loads of k-tile kt: thread t copies run t / 32 (part, chunk) of rows t % 32 + 32 j of each operand.
template <int ARPT, int BRPT>
__device__ __forceinline__ void load_stage(StageRegs<ARPT, BRPT>& r, const _Float16* a_src, size_t a_stride, const _Float16* b_src,
                                           size_t b_stride, uint32_t kt) {
#pragma unroll
    for (int j = 0; j < ARPT; ++j) r.a[j] = *reinterpret_cast<const u32x4*>(a_src + kt * a_stride + 32 * j * 8);
#pragma unroll
    for (int j = 0; j < BRPT; ++j) r.b[j] = *reinterpret_cast<const u32x4*>(b_src + kt * b_stride + 32 * j * 8);
}

template <int BM, int BN, int ARPT, int BRPT>
__device__ __forceinline__ void store_stage(const StageRegs<ARPT, BRPT>& r, _Float16* s_a, _Float16* s_b, uint32_t run,
                                            uint32_t row) {
#pragma unroll
    for (int j = 0; j < ARPT; ++j) *reinterpret_cast<u32x4*>(s_a + (run * BM + row + 32 * j) * 8) = r.a[j];
#pragma unroll
    for (int j = 0; j < BRPT; ++j) *reinterpret_cast<u32x4*>(s_b + (run * BN + row + 32 * j) * 8) = r.b[j];
}

// Row m (within the block tile) of accumulator register r of tile row i of wave row wm, lane `lane`: accumulator r
// of a 32x32 tile holds row 8 (r / 4) + 4 (lane / 32) + r % 4 and column lane % 32.
template <int BM>
__device__ __forceinline__ uint32_t acc_row(uint32_t wm, int i, int r, uint32_t lane) {
    return wm * (BM / 2) + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
}

// The same for waves of WR rows each (the streamed GEMM's 4- or 8-wave blocks).
template <uint32_t WR>
__device__ __forceinline__ uint32_t wave_row(uint32_t wm, int i, int r, uint32_t lane) {
    return wm * WR + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
}

// C[M, Ncol] = A[M, K] B[Ncol, K]^T from planes. Up: A = X planes (power of two per row), epilogue bias + GELU,
// writes the activation planes (K-chunk-major over the d_ff neurons) and one power of two per (row, BN block).
// Down: A = activation planes (power of two per row and kActBlock-wide k block), epilogue bias, writes Y fp32.
template <Epi EPI, int MI, int NI, bool LO_B, int SPLITS>
__global__ __launch_bounds__(kThreads) void gemm_planes_kernel(
    const _Float16* __restrict__ a_planes,  // [K / 32][8][rows_pad][8]
    const int32_t* __restrict__ a_exp,      // Up: [rows_pad]; Down: [K / kActBlock, rows_pad] (act_exp_at)
    const _Float16* __restrict__ b_planes,  // [K / 32][8][Ncol][8]
    const int32_t* __restrict__ b_exp,      // [Ncol]
    const float* __restrict__ bias,         // [Ncol]
    float* __restrict__ out,                // Down: [M, Ncol] fp32 row-major
    _Float16* __restrict__ out_planes,      // Up: activation planes [Ncol / 32][8][rows_pad][8]
    int32_t* __restrict__ out_exp,          // Up: [Ncol / BN, rows_pad] activation block binades (act_exp_at)
    float* __restrict__ partials,           // SPLITS > 1: [SPLITS, M, Ncol] partial sums
    int32_t* __restrict__ counters,         // SPLITS > 1: [tiles], zero between calls
    uint32_t M, uint32_t rows_pad, uint32_t Ncol, uint32_t K) {
    constexpr int BM = 64 * MI, BN = 64 * NI;
    constexpr int ARPT = BM / 32, BRPT = BN / 32;  // chunks per thread and k-tile (8 runs x 32 rows per block pass)

    // staged k-tiles, [buffer][part][chunk][row][8 halves] of A then of B; the up epilogue reuses it for its output
    __shared__ __attribute__((aligned(16))) _Float16 smem[2 * kRuns * (BM + BN) * 8];
    const auto s_a = [&](uint32_t buffer) { return smem + buffer * (kRuns * BM * 8); };
    const auto s_b = [&](uint32_t buffer) { return smem + 2 * kRuns * BM * 8 + buffer * (kRuns * BN * 8); };
    __shared__ int32_t row_e[2][BM];  // Up: [0] the row binades; Down: the row binades of the current / next k block
    __shared__ uint32_t row_max[2][BM];
    __shared__ int32_t last;

    const uint32_t tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    const uint32_t wm = wave / 2, wn = wave % 2;
    const uint32_t tiles_m = rows_pad / BM, tiles_n = Ncol / BN;
    const Tile tile = tile_of(blockIdx.x, tiles_m, tiles_n, SPLITS);
    const uint32_t m0 = tile.m * BM, n0 = tile.n * BN;
    const uint32_t ktiles = K / kBK;
    const uint32_t k_begin = tile.split * ktiles / SPLITS, k_end = (tile.split + 1) * ktiles / SPLITS;

    if (tid < BM) {
        if constexpr (EPI == Epi::Up) row_e[0][tid] = a_exp[m0 + tid];
        else row_e[(k_begin / kKtPerActBlock) & 1][tid] = act_exps(a_exp)[act_exp_at(rows_pad, m0 + tid, k_begin / kKtPerActBlock)];
    }

    const uint32_t run = tid / 32, row = tid % 32;
    const _Float16* a_src = a_planes + (static_cast<size_t>(run) * rows_pad + m0 + row) * 8;
    const _Float16* b_src = b_planes + (static_cast<size_t>(run) * Ncol + n0 + row) * 8;
    const size_t a_stride = static_cast<size_t>(kRuns) * rows_pad * 8, b_stride = static_cast<size_t>(kRuns) * Ncol * 8;
    StageRegs<ARPT, BRPT> regs;

    floatx16 acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    int32_t next_e = 0;  // Down: binades of the activation block of the k-tile in flight, when it starts one
    if (k_begin < k_end) {
        load_stage<ARPT, BRPT>(regs, a_src, a_stride, b_src, b_stride, k_begin);
        store_stage<BM, BN, ARPT, BRPT>(regs, s_a(0), s_b(0), run, row);
        if (k_begin + 1 < k_end) {
            load_stage<ARPT, BRPT>(regs, a_src, a_stride, b_src, b_stride, k_begin + 1);
            if constexpr (EPI == Epi::Down) {
                if ((k_begin + 1) % kKtPerActBlock == 0 && tid < BM)
                    next_e = act_exps(a_exp)[act_exp_at(rows_pad, m0 + tid, (k_begin + 1) / kKtPerActBlock)];
            }
        }
    }
    __syncthreads();
    for (uint32_t kt = k_begin; kt < k_end; ++kt) {
        const int buf = (kt - k_begin) & 1;
        if constexpr (EPI == Epi::Down) {
            // a new activation block: bring the accumulators to its power of two (exact), and fetch the next one's
            if (kt % kKtPerActBlock == 0 && kt != k_begin) {
                const uint32_t kb = kt / kKtPerActBlock;
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const uint32_t m = acc_row<BM>(wm, i, r, lane);
                        const float f = ldexpf(1.0f, row_e[(kb - 1) & 1][m] - row_e[kb & 1][m]);
#pragma unroll
                        for (int j = 0; j < NI; ++j) acc[i][j][r] *= f;
                    }
            }
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const uint32_t chunk = kk * 2 + lane / 32;
            half8 ah[MI], al[MI], bh[NI], bl[NI];
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                const uint32_t r = wm * (BM / 2) + i * 32 + lane % 32;
                ah[i] = *reinterpret_cast<const half8*>(s_a(buf) + (chunk * BM + r) * 8);
                al[i] = *reinterpret_cast<const half8*>(s_a(buf) + ((4 + chunk) * BM + r) * 8);
            }
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                const uint32_t r = wn * (BN / 2) + j * 32 + lane % 32;
                bh[j] = *reinterpret_cast<const half8*>(s_b(buf) + (chunk * BN + r) * 8);
                if constexpr (LO_B) bl[j] = *reinterpret_cast<const half8*>(s_b(buf) + ((4 + chunk) * BN + r) * 8);
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
            store_stage<BM, BN, ARPT, BRPT>(regs, s_a(buf ^ 1), s_b(buf ^ 1), run, row);
            if constexpr (EPI == Epi::Down) {
                // the next activation block's binades travel with the stage loads: requested with k-tile 4 kb, they
                // reach LDS with its store, one barrier before the rescale at k-tile 4 kb reads them
                if ((kt + 1) % kKtPerActBlock == 0 && tid < BM) row_e[((kt + 1) / kKtPerActBlock) & 1][tid] = next_e;
            }
            if (kt + 2 < k_end) {
                load_stage<ARPT, BRPT>(regs, a_src, a_stride, b_src, b_stride, kt + 2);
                if constexpr (EPI == Epi::Down) {
                    if ((kt + 2) % kKtPerActBlock == 0 && tid < BM)
                        next_e = act_exps(a_exp)[act_exp_at(rows_pad, m0 + tid, (kt + 2) / kKtPerActBlock)];
                }
            }
        }
        __syncthreads();
    }
    const int e_last = EPI == Epi::Up ? 0 : static_cast<int>(((k_end - 1) / kKtPerActBlock) & 1);

    if constexpr (EPI == Epi::Up) {
        // v = gelu(z + b): first its largest |v| per row over the tile's BN neurons (one tile row at a time, to keep
        // few registers live), then v again, split with that row's power of two into the activation planes
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            uint32_t lane_max[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) lane_max[r] = 0;
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                const uint32_t col = n0 + wn * (BN / 2) + j * 32 + lane % 32;
                const int ce = b_exp[col];
                const float cb = bias[col];
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    lane_max[r] = max(lane_max[r],
                                      abs_bits(gelu(ldexpf(acc[i][j][r], row_e[0][acc_row<BM>(wm, i, r, lane)] + ce) + cb)));
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                uint32_t v = lane_max[r];
#pragma unroll
                for (int s = 16; s >= 1; s >>= 1) v = max(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), s, kWave)));
                if (lane % 32 == 0) row_max[wn][acc_row<BM>(wm, i, r, lane)] = v;
            }
        }
        __syncthreads();
        if (tid < BM) {
            const int e = act_binade(max(row_max[0][tid], row_max[1][tid]));
            row_e[1][tid] = e;
            act_exps(out_exp)[act_exp_at(rows_pad, m0 + tid, tile.n)] = static_cast<int8_t>(e);
        }
        // the planes go out through LDS, half the block's rows (one wave row) at a time: the waves of that row store
        // v as fp32 [row][col], then every thread splits 8 consecutive columns of one row and writes 16 bytes per
        // part, 64 consecutive rows of one chunk per wave (1 KB contiguous)
        constexpr uint32_t R = BM / 2, kLd = BN + 8;
        static_assert(R * kLd * sizeof(float) <= sizeof(smem), "the epilogue tile fits the staging LDS");
        float* tile_v = reinterpret_cast<float*>(smem);
#pragma unroll
        for (uint32_t half = 0; half < 2; ++half) {
            __syncthreads();
            if (wm == half) {
#pragma unroll
                for (int j = 0; j < NI; ++j) {
                    const uint32_t c = wn * (BN / 2) + j * 32 + lane % 32;
                    const int ce = b_exp[n0 + c];
                    const float cb = bias[n0 + c];
#pragma unroll
                    for (int i = 0; i < MI; ++i)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const uint32_t m = acc_row<BM>(wm, i, r, lane);
                            tile_v[(m - half * R) * kLd + c] = gelu(ldexpf(acc[i][j][r], row_e[0][m] + ce) + cb);
                        }
                }
            }
            __syncthreads();
            for (uint32_t q = tid; q < R * (BN / 8); q += kThreads) {
                const uint32_t m = q % R, chunk = q / R, k = n0 + chunk * 8;
                const float scale = ldexpf(1.0f, -row_e[1][half * R + m]);
                const float* src = tile_v + m * kLd + chunk * 8;
                half8 h, l;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    _Float16 hh, ll;
                    split(src[e] * scale, hh, ll);
                    h[e] = hh;
                    l[e] = ll;
                }
                *reinterpret_cast<half8*>(out_planes + plane_at(rows_pad, m0 + half * R + m, k, 0)) = h;
                *reinterpret_cast<half8*>(out_planes + plane_at(rows_pad, m0 + half * R + m, k, 1)) = l;
            }
        }
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
                    const uint32_t m = acc_row<BM>(wm, i, r, lane);
                    if (m0 + m < M) out[static_cast<size_t>(m0 + m) * Ncol + col] = ldexpf(acc[i][j][r], row_e[e_last][m] + ce) + cb;
                }
        }
    } else {
        // every split writes its partial (powers of two undone), then the block that completes the tile adds them in
        // split order
        const size_t plane_size = static_cast<size_t>(M) * Ncol;
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const uint32_t col = n0 + wn * (BN / 2) + j * 32 + lane % 32;
            const int ce = b_exp[col];
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t m = acc_row<BM>(wm, i, r, lane);
                    acc[i][j][r] = ldexpf(acc[i][j][r], row_e[e_last][m] + ce);
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
                    const uint32_t m = acc_row<BM>(wm, i, r, lane);
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

// ------------------------------------------------------------------------------- streamed GEMM (LDS DMA)
// The large-N GEMM: 256 x 128 block tiles of 8 waves (4 x 2, 64 x 64 outputs each: two waves per SIMD, so that one
// wave's barrier and transfer waits are covered by the other's MFMAs), one block per CU, and k-tiles streamed
// straight from global memory into a ring of kDmaStages LDS stages by global_load_lds (16 bytes per lane, no
// registers on the way). In the middle of k-tile kt (its first 16-wide step multiplied, its second read into
// registers) the block waits for stage kt + 1, meets at a barrier and requests stage kt + kDmaStages into the slot of
// kt; each stage is thus requested kDmaStages - 1 k-tiles before its wait, and the MFMAs never wait for LDS reads.
// Before the first k-tile the lower half of the waves requests the first stages while the upper half loads the
// activation binades of the tile's rows and k range (the down GEMM). Same products and order as gemm_planes_kernel.
constexpr int kDmaStages = 3;
constexpr int kDmaBM = 256, kDmaBN = 128;
constexpr int kDmaWaves = 8;  // waves per block: two per SIMD, 64 x 64 outputs each
constexpr uint32_t kDmaMaxActBlocks = 40;  // activation blocks of one down split held in LDS (int8 binades)
constexpr uint32_t kDmaLoRuns = 32;        // activation blocks more per ring slot with bfloat16 weights (its B lo plane)

// Workgroup barrier without the memory fence of __syncthreads (whose release would also wait for every LDS DMA in
// flight); LDS visibility is ensured by the wait_loads before it.
__device__ __forceinline__ void block_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// LIVE < BM (one row tile of up to LIVE tokens): only the first LIVE rows of A are transferred and multiplied; the
// waves whose rows are all padding only transfer and meet at the barriers. The live rows get the same
// products in the same order as with LIVE = BM, and the padding rows' accumulators stay zero, as zero A rows leave
// them, so the results are bitwise those of the full tile.
template <Epi EPI, bool LO_B, int LIVE>
__global__ __launch_bounds__(64 * kDmaWaves) void gemm_dma_kernel(
    const _Float16* __restrict__ a_planes,  // [K / 32][8][rows_pad][8]
    const int32_t* __restrict__ a_exp,      // Up: [rows_pad]; Down: [K / kActBlock, rows_pad] (act_exp_at)
    const _Float16* __restrict__ b_planes,  // [K / 32][8][Ncol][8]
    const int32_t* __restrict__ b_exp,      // [Ncol]
    const float* __restrict__ bias,         // [Ncol]
    float* __restrict__ out,                // Down: y [M, Ncol] (splits == 1) or partials [splits, M, Ncol]; UpSplit: partials
    _Float16* __restrict__ out_planes,      // Up: activation planes [Ncol / 32][8][rows_pad][8]
    int32_t* __restrict__ out_exp,          // Up: [Ncol / BN, rows_pad] activation block binades (act_exp_at)
    uint32_t M, uint32_t rows_pad, uint32_t Ncol, uint32_t K, uint32_t splits,
    uint32_t whole_n,                       // Down: column tiles below whole_n take all of K and write y into `out`
    float* __restrict__ part) {             // Down, whole_n > 0: the other column tiles' partials [splits, M, Ncol - whole_n BN]
    // 8 waves in 4 x 2, 64 x 64 outputs each (two waves per SIMD)
    constexpr int W = kDmaWaves, MI = 2, NI = 2, BM = kDmaBM, BN = kDmaBN, S = kDmaStages;
    constexpr uint32_t kT = 64 * W, kWaveRows = 32 * MI, kHalf = W / 2;
    static_assert(kWaveRows * (W / 2) == BM, "the waves cover the block's rows");
    static_assert(kHalf * kWave == BM, "the upper half of the waves holds a thread per block row");
    static_assert(LIVE == BM || LIVE == 128 || LIVE == 64, "live rows: the whole tile, its first half or first quarter");
    constexpr uint32_t kStage = kRuns * (BM + BN) * 8;  // halves per stage
    // Down: the activation binades of up to kDmaMaxActBlocks blocks sit in e_tab; with bfloat16 weights the B lo plane of
    // every ring slot (8 KB, never transferred) holds 32 blocks more, so that a tile can take all of a wide K
    constexpr uint32_t kLoRegion = kRuns * BM * 8 + kRuns / 2 * BN * 8, kLoRuns = kRuns / 2 * BN * 8 * 2 / BM;
    constexpr uint32_t kMaxActBlocks = LO_B ? kDmaMaxActBlocks : kDmaMaxActBlocks + S * kLoRuns;
    static_assert(kLoRuns == kDmaLoRuns, "the host's plan counts the ring's spare runs alike");
    constexpr int kRowRuns = LIVE / 64;                  // 64-row runs of A transferred per (part, chunk)
    // runs of B transferred per k-tile: both planes, or the hi plane alone when the lo plane is not read (LO_B false)
    constexpr int kRunsB = LO_B ? kRuns : kRuns / 2;
    constexpr int kLoadsA = kRowRuns * kRuns / W, kLoadsB = BN * kRunsB / kWave / W;  // DMA instructions per wave
    static_assert(kLoadsA * W == kRowRuns * kRuns && kLoadsB * W == BN * kRunsB / kWave, "the transfers divide over the waves");
    constexpr int kLoads = kLoadsA + kLoadsB;
    static_assert(kLoads * S + (kMaxActBlocks + W - 1) / W < 64, "the prologue's transfers of a wave fit vmcnt");
    // multiplied 32-row tiles of a live wave (its rows start at wm * kWaveRows; LIVE is a multiple of kWaveRows)
    constexpr int MIL = LIVE >= static_cast<int>(kWaveRows) ? MI : LIVE / 32;

    __shared__ __attribute__((aligned(16))) _Float16 smem[S * kStage];
    __shared__ __attribute__((aligned(16))) int32_t e_row[1][BM];  // Up: x binades
    __shared__ __attribute__((aligned(16))) int8_t e_tab[EPI == Epi::Down ? kDmaMaxActBlocks : 1][EPI == Epi::Down ? BM : 1];  // Down: [block][row]
    // Down: the BM binades of the k range's activation block c (c < kMaxActBlocks): a row of e_tab, or a 256-byte run in
    // the unused B lo plane of ring slot (c - kDmaMaxActBlocks) / kLoRuns
    const auto etab = [&](uint32_t c) -> int8_t* {
        if (LO_B || c < kDmaMaxActBlocks) return &e_tab[c][0];
        const uint32_t o = c - kDmaMaxActBlocks;
        return reinterpret_cast<int8_t*>(smem + (o / kLoRuns) * kStage + kLoRegion) + (o % kLoRuns) * BM;
    };

    const uint32_t tid = threadIdx.x, lane = tid % kWave, wave = uniform(tid / kWave);
    const uint32_t wm = wave / 2, wn = wave % 2;
    // wave-uniform: this wave's rows hold tokens (a constant for a full tile)
    const bool live = LIVE == BM || wm * kWaveRows < static_cast<uint32_t>(LIVE);
    const uint32_t tiles_m = rows_pad / BM, tiles_n = Ncol / BN;
    // the first tiles_m * whole_n blocks: column tiles 0 .. whole_n - 1 over all of K (one round of long blocks first);
    // the others: the remaining column tiles, K split `splits` ways (whole_n 0: every tile split alike)
    const uint32_t whole_blocks = tiles_m * whole_n;
    const bool whole = blockIdx.x < whole_blocks;
    Tile tile = whole ? tile_of(blockIdx.x, tiles_m, whole_n, 1) : tile_of(blockIdx.x - whole_blocks, tiles_m, tiles_n - whole_n, splits);
    if (!whole) tile.n += whole_n;
    const uint32_t nsplit = whole ? 1 : splits;
    const uint32_t m0 = tile.m * BM, n0 = tile.n * BN;
    const uint32_t ktiles = K / kBK;
    const uint32_t k_begin = tile.split * ktiles / nsplit, k_end = (tile.split + 1) * ktiles / nsplit;
    const uint32_t kb0 = k_begin / kKtPerActBlock;

    // piece q of wave w's share of a stage: a run of 64 rows (1 KB) of A (pieces below kLoadsA), then of B; its
    // element offsets within a k-tile's planes and within a ring slot
    const auto piece = [&](uint32_t w, int q, uint32_t& src, uint32_t& dst) {
        if (q < kLoadsA) {
            const uint32_t at = w * kLoadsA + q, run = at / kRowRuns, rb = at % kRowRuns;
            src = (run * rows_pad + m0 + rb * 64) * 8;
            dst = (run * BM + rb * 64) * 8;
        } else {
            const uint32_t at = w * kLoadsB + (q - kLoadsA), run = at / (BN / 64), rb = at % (BN / 64);
            src = (run * Ncol + n0 + rb * 64) * 8;
            dst = kRuns * BM * 8 + (run * BN + rb * 64) * 8;
        }
    };
    // this wave's pieces, computed once: the lanes' byte offsets from the k-tile's base (vector registers) and the
    // LDS offsets (wave-uniform), so that a transfer in the k loop takes the k-tile's base pointer of its operand
    const size_t a_kt = static_cast<size_t>(kRuns) * rows_pad * 8, b_kt = static_cast<size_t>(kRuns) * Ncol * 8;
    uint32_t src_lane[kLoads], dst_off[kLoads];
#pragma unroll
    for (int q = 0; q < kLoads; ++q) {
        uint32_t src;
        piece(wave, q, src, dst_off[q]);
        src_lane[q] = src * 2 + lane * 16;
    }
    const auto issue_piece = [&](uint32_t kt, uint32_t slot, int q) {
        const _Float16* base = q < kLoadsA ? a_planes + kt * a_kt : b_planes + kt * b_kt;
        dma16(base, src_lane[q], smem + slot * kStage + dst_off[q]);
    };
    const auto issue = [&](uint32_t kt, uint32_t slot) {
#pragma unroll
        for (int q = 0; q < kLoads; ++q) issue_piece(kt, slot, q);
    };

    // Prologue: every wave requests its pieces of the first stages, after the binades of the tile's rows, which go
    // straight into LDS as well (Up: the x binades, one 1 KB run; Down: the split's activation blocks, one 256-byte run
    // of int8 each, block c from wave c % W). vmcnt retires in order within a wave, so once the first stage has landed
    // so have they: the block meets once, and no wave holds a register for them. (Loaded into registers by half of the
    // waves and reduced to change masks there, the down GEMM's binades kept the block 6.5 us in its prologue, where
    // the first stage lands in 2.5-3 us.)
    const uint32_t steps = k_end - k_begin;  // at least 1
    if constexpr (EPI == Epi::Down) {
        const uint32_t blocks = (k_end - k_begin) / kKtPerActBlock;  // at least one: K is split on activation blocks
        const int8_t* tab = act_exps(a_exp);
        for (uint32_t c = wave; c < blocks; c += W)
            dma4(tab + act_exp_at(rows_pad, m0, kb0 + c), lane * 4, etab(c));
    } else {
        if (wave == 0) dma16(a_exp + m0, lane * 16, &e_row[0][0]);
    }
#pragma unroll
    for (int s = 0; s < S; ++s)
        if (static_cast<uint32_t>(s) < steps) issue(k_begin + s, s);
    // stage k_begin has landed (later stages may be in flight), and with it the binades; then the block meets
    if (steps >= 3) wait_loads<2 * kLoads>();
    else if (steps == 2) wait_loads<kLoads>();
    else wait_loads<0>();
    block_barrier();

    floatx16 acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // operand fragments of one 16-wide k step (chunk pair kk of a k-tile)
    struct Frags {
        half8 ah[MI], al[MI], bh[NI], bl[NI];
    };
    const auto load = [&](Frags& f, uint32_t slot, int kk) {
        if (!live) return;
        const _Float16* s_a = smem + slot * kStage;
        const _Float16* s_b = s_a + kRuns * BM * 8;
        const uint32_t chunk = kk * 2 + lane / 32;
#pragma unroll
        for (int i = 0; i < MIL; ++i) {
            const uint32_t r = wm * kWaveRows + i * 32 + lane % 32;
            f.ah[i] = *reinterpret_cast<const half8*>(s_a + (chunk * BM + r) * 8);
            f.al[i] = *reinterpret_cast<const half8*>(s_a + ((4 + chunk) * BM + r) * 8);
        }
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const uint32_t r = wn * (BN / 2) + j * 32 + lane % 32;
            f.bh[j] = *reinterpret_cast<const half8*>(s_b + (chunk * BN + r) * 8);
            if constexpr (LO_B) f.bl[j] = *reinterpret_cast<const half8*>(s_b + ((4 + chunk) * BN + r) * 8);
        }
    };
    const auto multiply = [&](const Frags& f) {
        if (!live) return;
#pragma unroll
        for (int i = 0; i < MIL; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.ah[i], f.bh[j], acc[i][j], 0, 0, 0);
                if constexpr (LO_B) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.ah[i], f.bl[j], acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.al[i], f.bh[j], acc[i][j], 0, 0, 0);
            }
    };
    // The same products with stage kt's transfers spread among them, one after every few MFMAs: a transfer's issue
    // holds the wave while the CU's address unit takes the other waves' transfers, and in-order issue would
    // otherwise keep the MFMA unit idle behind a burst of them. sched_barrier pins the order.
    constexpr int kProducts = LO_B ? 3 : 2, kMfmas = MI * NI * kProducts;
    static_assert(kMfmas >= kLoads, "at most one transfer per MFMA");
    const auto multiply_issuing = [&](const Frags& f, uint32_t kt, uint32_t slot, bool transfer) {
        if constexpr (LIVE < BM) {  // few MFMAs: the stage's transfers go out first, in one burst
            if (transfer) issue(kt, slot);
            __builtin_amdgcn_sched_barrier(0);
            multiply(f);
            return;
        }
#pragma unroll
        for (int p = 0; p < kProducts; ++p)  // product-major: consecutive MFMAs accumulate into different tiles
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NI; ++j) {
                    const half8& a = p == kProducts - 1 ? f.al[i] : f.ah[i];
                    const half8& b = (LO_B && p == 1) ? f.bl[j] : f.bh[j];
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[i][j], 0, 0, 0);
                    const int m = (p * MI + i) * NI + j;  // MFMAs issued so far, less one
                    if ((m + 1) * kLoads % kMfmas < kLoads) {   // kLoads transfers evenly over kMfmas MFMAs
                        __builtin_amdgcn_sched_barrier(0);
                        if (transfer) issue_piece(kt, slot, (m + 1) * kLoads / kMfmas - 1);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
    };

    // Software pipeline over half k-tiles: the fragments of the next 16-wide step are read from LDS while the MFMAs
    // of the current one run, and the block meets once per k-tile, between its two steps (after every wave has read
    // all of k-tile kt and before anyone reads k-tile kt + 1), where the slot of kt is refilled with kt + kDmaStages.
    // The first stages went out in the prologue.
    // a new activation block at k-tile kt: bring the accumulators to its power of two (exact), when some row of the
    // wave changes it (lane l checks the wave's row l; binades are multiples of kActBinadeStep, so changes are rare;
    // checked here rather than for all blocks after the prologue, which measured 0.5 % slower); accumulator registers
    // 4g .. 4g + 3 hold 4 consecutive rows, so one 4-byte read per block and group
    const auto rescale = [&](uint32_t kt) {
        if constexpr (EPI == Epi::Down) {
            const uint32_t kb = kt / kKtPerActBlock - kb0;
            if (kt % kKtPerActBlock != 0 || kt == k_begin || !live) return;
            const uint32_t own = wm * kWaveRows + lane;
            if (__builtin_amdgcn_ballot_w64(etab(kb - 1)[own] != etab(kb)[own]) != 0) {
#pragma unroll
                for (int i = 0; i < MIL; ++i)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const uint32_t m = wave_row<kWaveRows>(wm, i, 4 * g, lane);
                        const uint32_t before = *reinterpret_cast<const uint32_t*>(etab(kb - 1) + m);
                        const uint32_t now = *reinterpret_cast<const uint32_t*>(etab(kb) + m);
#pragma unroll
                        for (int b = 0; b < 4; ++b) {
                            const int d = static_cast<int8_t>(before >> (8 * b)) - static_cast<int8_t>(now >> (8 * b));
                            const float f = ldexpf(1.0f, d);
#pragma unroll
                            for (int j = 0; j < NI; ++j) acc[i][j][4 * g + b] *= f;
                        }
                    }
            }
        }
    };
    // A wave raises its issue priority (s_setprio) for the MFMA run that carries the stage's transfers, so that of the two
    // waves of a SIMD the one with products ready issues ahead of the other's LDS reads (same box, alternating builds:
    // the 2.8B layer's up GEMM 415-427 -> 401-402 us and down GEMM 466-468 -> 444-458 us, the 410M layer's up GEMM
    // ~56 -> 54.5 us; the raised priority around the other MFMA run gave nothing on the down GEMM and lost ~2 % on the
    // up GEMM).
    const auto raise_priority = [] { __builtin_amdgcn_s_setprio(1); };
    const auto lower_priority = [] {
        __builtin_amdgcn_sched_barrier(0);  // the MFMA run ends here
        __builtin_amdgcn_s_setprio(0);
    };
    Frags f0, f1;
    load(f0, 0, 0);
    // every k-tile but the last (peeled, so that no path reaches the second step's MFMAs without the barrier's wait
    // for the first step's reads: the compiler's own LDS waits then never hold them for the reads just issued)
    // (sched_barrier keeps each step's LDS reads ahead of the MFMAs they overlap)
    for (uint32_t kt = k_begin; kt + 1 < k_end; ++kt) {
        const uint32_t it = kt - k_begin, slot = it % S;
        rescale(kt);
        wait_loads<63>();  // this step's reads, issued a step ago, are in: the next reads do not hold its MFMAs
        load(f1, slot, 1);
        __builtin_amdgcn_sched_barrier(0);
        multiply(f0);
        if (kt + 2 < k_end) wait_loads<kLoads>();  // stage kt + 1 has landed, kt + 2 may be in flight
        else wait_loads<0>();
        wait_loads<63>();  // the same LDS wait on every path, where the compiler's wait tracking sees it
        block_barrier();
        load(f0, (it + 1) % S, 0);
        __builtin_amdgcn_sched_barrier(0);
        raise_priority();
        multiply_issuing(f1, kt + S, slot, kt + S < k_end);  // straight-line MFMAs: one set of accumulators
        lower_priority();
    }
    rescale(k_end - 1);
    wait_loads<63>();
    load(f1, (steps - 1) % S, 1);
    __builtin_amdgcn_sched_barrier(0);
    multiply(f0);
    multiply(f1);
    __syncthreads();

    if constexpr (EPI == Epi::Up) {
        // v = gelu(z + b) once per element into an fp32 [BM][BN] tile in LDS; then thread t takes block row t: the
        // largest |v| of the row over the tile's BN neurons gives its power of two, and the row goes out split, 16
        // bytes per part and chunk (the 256 threads write 256 consecutive rows of one chunk: 4 KB contiguous)
        constexpr uint32_t kLd = BN + 4;
        static_assert(BM * kLd * sizeof(float) <= sizeof(smem), "the epilogue tile fits the staging LDS");
        float* tile_v = reinterpret_cast<float*>(smem);
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const uint32_t c = wn * (BN / 2) + j * 32 + lane % 32;
            const int ce = b_exp[n0 + c];
            const float cb = bias[n0 + c];
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t m = wave_row<kWaveRows>(wm, i, r, lane);
                    tile_v[m * kLd + c] = gelu(ldexpf(acc[i][j][r], e_row[0][m] + ce) + cb);
                }
        }
        __syncthreads();
        // H threads per block row (1 with 4 waves, 2 with 8: lanes h of a row are adjacent), each a BN / H-wide part
        constexpr uint32_t H = kT / BM;
        const uint32_t row = tid / H, part = tid % H;
        const float* row_v = tile_v + row * kLd;
        uint32_t largest = 0;
#pragma unroll 8
        for (uint32_t c = part * (BN / H); c < (part + 1) * (BN / H); c += 4) {
            const float4 v = *reinterpret_cast<const float4*>(row_v + c);
            largest = max(largest, max(max(abs_bits(v.x), abs_bits(v.y)), max(abs_bits(v.z), abs_bits(v.w))));
        }
#pragma unroll
        for (uint32_t off = 1; off < H; off <<= 1)
            largest = max(largest, static_cast<uint32_t>(__shfl_xor(static_cast<int>(largest), static_cast<int>(off), kWave)));
        const int e = act_binade(largest);
        if (part == 0) act_exps(out_exp)[act_exp_at(rows_pad, m0 + row, tile.n)] = static_cast<int8_t>(e);
        const float scale = ldexpf(1.0f, -e);
#pragma unroll 4
        for (uint32_t chunk = part * (BN / 8 / H); chunk < (part + 1) * (BN / 8 / H); ++chunk) {
            const float4 u = *reinterpret_cast<const float4*>(row_v + chunk * 8);
            const float4 w = *reinterpret_cast<const float4*>(row_v + chunk * 8 + 4);
            const float v[8] = {u.x, u.y, u.z, u.w, w.x, w.y, w.z, w.w};
            half8 h, l;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                _Float16 hh, ll;
                split(v[q] * scale, hh, ll);
                h[q] = hh;
                l[q] = ll;
            }
            *reinterpret_cast<half8*>(out_planes + plane_at(rows_pad, m0 + row, n0 + chunk * 8, 0)) = h;
            *reinterpret_cast<half8*>(out_planes + plane_at(rows_pad, m0 + row, n0 + chunk * 8, 1)) = l;
        }
    } else {
        // y (Down, one split) or this split's partial, powers of two undone: through an fp32 [BM][BN] tile in LDS, so
        // that every thread writes 16 bytes (a wave: two rows of BN columns)
        constexpr uint32_t kLd = BN + 4;
        static_assert(BM * kLd * sizeof(float) <= sizeof(smem), "the epilogue tile fits the staging LDS");
        float* tile_v = reinterpret_cast<float*>(smem);
        const uint32_t kb_last = (k_end - 1) / kKtPerActBlock - kb0;
        // the last activation block's binades held in a ring slot (a wide k range), which the tile below overwrites,
        // are first copied to e_row (block-uniform condition)
        const bool last_in_ring = EPI == Epi::Down && kb_last >= kDmaMaxActBlocks;
        if (last_in_ring) {
            if (tid < BM) e_row[0][tid] = etab(kb_last)[tid];
            __syncthreads();
        }
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const uint32_t c = wn * (BN / 2) + j * 32 + lane % 32;
            const int ce = b_exp[n0 + c];
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t m = wave_row<kWaveRows>(wm, i, r, lane);
                    const int ea = EPI == Epi::Down && !last_in_ring ? static_cast<int>(e_tab[kb_last][m]) : e_row[0][m];
                    tile_v[m * kLd + c] = ldexpf(acc[i][j][r], ea + ce);
                }
        }
        __syncthreads();
        // y (whole k range) or this split's partial: [splits, M, Ncol], or with whole_n > 0 [splits, M, Ncol - whole_n BN]
        // over the split column tiles only
        const uint32_t ld = nsplit > 1 && whole_n > 0 ? Ncol - whole_n * BN : Ncol, c0 = n0 - (ld == Ncol ? 0 : whole_n * BN);
        float* target = nsplit == 1 ? out : (whole_n > 0 ? part : out) + static_cast<size_t>(tile.split) * M * ld;
        const bool add_bias = EPI == Epi::Down && nsplit == 1 && bias != nullptr;  // no bias: the training gx product
        for (uint32_t q = tid; q < BM * (BN / 4); q += kT) {
            const uint32_t m = q / (BN / 4), c = (q % (BN / 4)) * 4;
            if (m0 + m >= M) break;  // rows ascend with q
            float4 v = *reinterpret_cast<const float4*>(tile_v + m * kLd + c);
            if (add_bias) {
                const float4 b = *reinterpret_cast<const float4*>(bias + n0 + c);
                v.x += b.x; v.y += b.y; v.z += b.z; v.w += b.w;
            }
            *reinterpret_cast<float4*>(target + static_cast<size_t>(m0 + m) * ld + c0 + c) = v;
        }
    }
}

// y[m, c0 + c] = sum over splits (in split order) of partials[s, m, c] + bias[c0 + c] for the partials' width columns
// (y rows of Ncol); 4 columns per thread.
__global__ __launch_bounds__(kThreads) void reduce_splits_kernel(const float* __restrict__ partials, const float* __restrict__ bias,
                                                                float* __restrict__ y, uint32_t M, uint32_t Ncol, uint32_t splits,
                                                                uint32_t width, uint32_t c0) {
    const size_t quads = static_cast<size_t>(M) * width / 4;
    const size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= quads) return;
    const size_t m = i / (width / 4), c = c0 + (i % (width / 4)) * 4;
    const float4* p = reinterpret_cast<const float4*>(partials);
    float4 t = p[i];
    for (uint32_t s0 = 1; s0 < splits; s0 += 8) {  // 8 loads in flight, added in split order
        float4 u[8];
#pragma unroll
        for (uint32_t q = 0; q < 8; ++q)
            if (s0 + q < splits) u[q] = p[(s0 + q) * quads + i];
#pragma unroll
        for (uint32_t q = 0; q < 8; ++q)
            if (s0 + q < splits) {
                t.x += u[q].x; t.y += u[q].y; t.z += u[q].z; t.w += u[q].w;
            }
    }
    if (bias != nullptr) {  // none for the training gx product
        const float4 b = *reinterpret_cast<const float4*>(bias + c);
        t.x += b.x; t.y += b.y; t.z += b.z; t.w += b.w;
    }
    *reinterpret_cast<float4*>(y + m * Ncol + c) = t;
}

// Activation planes from the up GEMM's k-split partial sums (Epi::UpSplit): v = gelu(sum over the splits, in split
// order, of partials[s, m, n] + b_up[n]); rows m >= M hold gelu(b_up[n]), as the zero rows of x give in the fused
// epilogue. Then, per token and 128-neuron block, the binade of the largest |v| and the hi/lo planes, as
// gemm_dma_kernel<Up> writes them. A wave takes 4 rows of one 128-neuron block: 16 lanes per row, 8 consecutive
// neurons per lane (one 16-byte chunk per part); the block's maximum is a 16-lane xor butterfly.
constexpr uint32_t kActRowsPerBlock = kThreads / 16;
__global__ __launch_bounds__(kThreads) void act_planes_kernel(const float* __restrict__ partials, uint32_t splits,
                                                             const float* __restrict__ b_up, _Float16* __restrict__ planes,
                                                             int8_t* __restrict__ exps, uint32_t M, uint32_t rows_pad, uint32_t H) {
    const uint32_t m = blockIdx.x * kActRowsPerBlock + threadIdx.x / 16, sub = threadIdx.x % 16;
    const uint32_t nb = blockIdx.y, n = nb * kActBlock + sub * 8;
    const float4 b0 = *reinterpret_cast<const float4*>(b_up + n), b1 = *reinterpret_cast<const float4*>(b_up + n + 4);
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (m < M) {
        for (uint32_t s0 = 0; s0 < splits; s0 += 4) {  // 8 loads in flight, added in split order
            float4 u[4], w[4];
#pragma unroll
            for (uint32_t q = 0; q < 4; ++q)
                if (s0 + q < splits) {
                    const float* p = partials + (static_cast<size_t>(s0 + q) * M + m) * H + n;
                    u[q] = *reinterpret_cast<const float4*>(p);
                    w[q] = *reinterpret_cast<const float4*>(p + 4);
                }
#pragma unroll
            for (uint32_t q = 0; q < 4; ++q)
                if (s0 + q < splits) {
                    v[0] += u[q].x; v[1] += u[q].y; v[2] += u[q].z; v[3] += u[q].w;
                    v[4] += w[q].x; v[5] += w[q].y; v[6] += w[q].z; v[7] += w[q].w;
                }
        }
    }
    const float b[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    uint32_t largest = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        v[q] = gelu(v[q] + b[q]);
        largest = max(largest, abs_bits(v[q]));
    }
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) largest = max(largest, static_cast<uint32_t>(__shfl_xor(static_cast<int>(largest), off, kWave)));
    const int e = act_binade(largest);
    if (sub == 0) exps[act_exp_at(rows_pad, m, nb)] = static_cast<int8_t>(e);
    const float scale = ldexpf(1.0f, -e);
    half8 hi, lo;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        _Float16 hh, ll;
        split(v[q] * scale, hh, ll);
        hi[q] = hh;
        lo[q] = ll;
    }
    *reinterpret_cast<half8*>(planes + plane_at(rows_pad, m, n, 0)) = hi;
    *reinterpret_cast<half8*>(planes + plane_at(rows_pad, m, n, 1)) = lo;
}

// Training epilogues of the split up-shaped products [tokens, d_ff] (the sums of the split partials, in split order):
//   Forward: z = b_up + sum, act = gelu(z): z and act hidden-major [d_ff, ld], act also as planes with its block
//            binades (read by the down GEMM);
//   GradZ:   gz = sum * gelu'(z), z read hidden-major: gz hidden-major and as planes with block binades (read by the gx
//            GEMM).
// Blocks and threads as act_planes_kernel (16 tokens x one 128-neuron block; 16 threads per token, 8 neurons each). The
// hidden-major rows go through LDS tiles [128 neurons][16 tokens]: thread i takes neuron i / 4 and tokens 4 (i % 4) ..
// + 3, 16 bytes at a time (ld and the block's first token are multiples of 4, so a vector that starts below ld ends
// below it); only tokens below M are written.
enum class TrainPost { Forward, GradZ };
template <TrainPost MODE>
__global__ __launch_bounds__(kThreads) void train_planes_kernel(const float* __restrict__ partials, uint32_t splits,
                                                               const float* __restrict__ b_up, const float* __restrict__ z_in,
                                                               float* __restrict__ out_a, float* __restrict__ out_b,
                                                               _Float16* __restrict__ planes, int8_t* __restrict__ exps, uint32_t M,
                                                               uint32_t rows_pad, uint32_t H, uint32_t ld) {
    constexpr uint32_t R = kActRowsPerBlock;
    static_assert(R == 16 && kActBlock * 4 % kThreads == 0, "16 tokens a block; the tile rows divide over the threads");
    __shared__ float ta[kActBlock][R + 1], tb[kActBlock][R + 1];  // Forward: z, act; GradZ: z, gz
    const uint32_t ml = threadIdx.x / 16, sub = threadIdx.x % 16;
    const uint32_t m0 = blockIdx.x * R, m = m0 + ml;
    const uint32_t nb = blockIdx.y, n0 = nb * kActBlock, n = n0 + sub * 8;
    if constexpr (MODE == TrainPost::GradZ) {
        for (uint32_t i = threadIdx.x; i < kActBlock * 4; i += kThreads) {
            const uint32_t r = i / 4, c = (i % 4) * 4;
            float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m0 + c < ld) q = *reinterpret_cast<const float4*>(z_in + static_cast<size_t>(n0 + r) * ld + m0 + c);
            ta[r][c] = q.x, ta[r][c + 1] = q.y, ta[r][c + 2] = q.z, ta[r][c + 3] = q.w;
        }
        __syncthreads();
    }
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (m < M) {
        for (uint32_t s0 = 0; s0 < splits; s0 += 4) {  // 8 loads in flight, added in split order
            float4 u[4], w[4];
#pragma unroll
            for (uint32_t q = 0; q < 4; ++q)
                if (s0 + q < splits) {
                    const float* p = partials + (static_cast<size_t>(s0 + q) * M + m) * H + n;
                    u[q] = *reinterpret_cast<const float4*>(p);
                    w[q] = *reinterpret_cast<const float4*>(p + 4);
                }
#pragma unroll
            for (uint32_t q = 0; q < 4; ++q)
                if (s0 + q < splits) {
                    v[0] += u[q].x; v[1] += u[q].y; v[2] += u[q].z; v[3] += u[q].w;
                    v[4] += w[q].x; v[5] += w[q].y; v[6] += w[q].z; v[7] += w[q].w;
                }
        }
    }
    uint32_t largest = 0;
    if constexpr (MODE == TrainPost::Forward) {
        const float4 b0 = *reinterpret_cast<const float4*>(b_up + n), b1 = *reinterpret_cast<const float4*>(b_up + n + 4);
        const float b[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float z = v[q] + b[q];
            ta[sub * 8 + q][ml] = z;
            v[q] = gelu(z);
            tb[sub * 8 + q][ml] = v[q];
            largest = max(largest, abs_bits(v[q]));
        }
    } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            v[q] *= gelu_grad(ta[sub * 8 + q][ml]);
            tb[sub * 8 + q][ml] = v[q];
            largest = max(largest, abs_bits(v[q]));
        }
    }
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) largest = max(largest, static_cast<uint32_t>(__shfl_xor(static_cast<int>(largest), off, kWave)));
    const int e = act_binade(largest);
    if (sub == 0) exps[act_exp_at(rows_pad, m, nb)] = static_cast<int8_t>(e);
    const float scale = ldexpf(1.0f, -e);
    half8 hi, lo;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        _Float16 hh, ll;
        split(v[q] * scale, hh, ll);
        hi[q] = hh;
        lo[q] = ll;
    }
    *reinterpret_cast<half8*>(planes + plane_at(rows_pad, m, n, 0)) = hi;
    *reinterpret_cast<half8*>(planes + plane_at(rows_pad, m, n, 1)) = lo;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < kActBlock * 4; i += kThreads) {
        const uint32_t r = i / 4, c = (i % 4) * 4;
        const size_t at = static_cast<size_t>(n0 + r) * ld + m0 + c;
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
            if (m0 + c + q >= M) break;
            if constexpr (MODE == TrainPost::Forward) {
                out_a[at + q] = ta[r][c + q];
                out_b[at + q] = tb[r][c + q];
            } else {
                out_a[at + q] = tb[r][c + q];
            }
        }
    }
}

uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

struct Shape {
    int mi, ni, splits;  // wave tile (32 mi) x (32 ni), block tile (64 mi) x (64 ni), k splits
};

constexpr int kMaxSplits = 4;

uint32_t rows_padded(uint32_t m) { return ceil_div(m, kRowPad) * kRowPad; }

// Rows of the token and activation planes that a call of m tokens reads: one row tile of at most 64 or 128 tokens
// runs the live-row GEMMs (gemm_dma_kernel<..., 64 or 128>), which read only its first 64 or 128 rows; otherwise every
// padded row. The split and activation-plane passes write these rows only.
uint32_t rows_live(uint32_t m) { return m <= 64 ? 64 : m <= 128 ? 128 : rows_padded(m); }

// Up: 128 x 128 blocks (the column tile is the activation block). Down: 64 x 128 blocks without a k split; K is
// split only when a down projection has fewer than 64 blocks (the fixup's device-scope fences write back the L2).
Shape up_shape(uint32_t, uint32_t) { return {2, 2, 1}; }

Shape down_shape(uint32_t m, uint32_t ncol, uint32_t k) {
    const uint32_t tiles = rows_padded(m) / 64 * (ncol / 128);
    return {1, 2, tiles < 64 && k >= 2048 ? 2 : 1};
}

template <Epi EPI, bool LO_B, int MI, int NI, int SPLITS>
hipError_t launch_gemm(const _Float16* a_planes, const int32_t* a_exp, const _Float16* b_planes, const int32_t* b_exp,
                       const float* bias, float* out, _Float16* out_planes, int32_t* out_exp, float* partials, int32_t* counters,
                       uint32_t M, uint32_t Ncol, uint32_t K, hipStream_t stream) {
    static_assert(EPI == Epi::Down || 64 * NI == kActBlock, "the up GEMM's column tile is the activation block");
    const uint32_t rows_pad = rows_padded(M);
    const uint32_t tiles = rows_pad / (64 * MI) * (Ncol / (64 * NI));
    hipLaunchKernelGGL((gemm_planes_kernel<EPI, MI, NI, LO_B, SPLITS>), dim3(tiles * SPLITS), dim3(kThreads), 0, stream, a_planes,
                       a_exp, b_planes, b_exp, bias, out, out_planes, out_exp, partials, counters, M, rows_pad, Ncol, K);
    return hipGetLastError();
}

// The instantiated shapes: up (mi, ni) in {(2,2), (4,2), (1,2)} without splits; down (2,2) and (1,2) with 1, 2 or 4
// splits and (2,4) with 1 or 2.
template <Epi EPI, bool LO_B>
hipError_t gemm(Shape shape, const _Float16* a_planes, const int32_t* a_exp, const _Float16* b_planes, const int32_t* b_exp,
                const float* bias, float* out, _Float16* out_planes, int32_t* out_exp, float* partials, int32_t* counters,
                uint32_t M, uint32_t Ncol, uint32_t K, hipStream_t stream) {
#define HFFN_GEMM(MI, NI, S)                                                                                                   \
    if (shape.mi == MI && shape.ni == NI && shape.splits == S)                                                                 \
        return launch_gemm<EPI, LO_B, MI, NI, S>(a_planes, a_exp, b_planes, b_exp, bias, out, out_planes, out_exp, partials,   \
                                                 counters, M, Ncol, K, stream);
    if constexpr (EPI == Epi::Up) {
        HFFN_GEMM(2, 2, 1)
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

// The streamed kernel takes a GEMM when its 256 x 128 tiles times its k splits give at least kDmaMinBlocks blocks
// (an up projection) or kDmaMinDownBlocks (a down projection, whose split count is bounded by the activation blocks
// of narrow layers); the split partials are added by reduce_splits_kernel (down) or act_planes_kernel (up).
constexpr uint32_t kDmaMinBlocks = 128;
constexpr uint32_t kDmaMinDownBlocks = 64;

uint32_t dma_tiles(uint32_t m, uint32_t ncol) { return rows_padded(m) / kDmaBM * (ncol / kDmaBN); }

// Splits of the streamed down GEMM by estimated time, over the split counts (powers of two up to kDmaMaxSplits) that
// cut K on activation blocks, hold a split's binades in LDS and give at least kDmaMinDownBlocks blocks: the blocks
// run in rounds of one per CU (the LDS ring takes a CU), each block kDmaKtileUs per k-tile plus kDmaBlockUs of
// prologue and epilogue; a split count above 1 adds its partials' round trip (written, then read by
// reduce_splits_kernel) and that kernel's launch. The partials are priced on the padded rows, so every token count
// of one padded row count takes the same splits and a token's sums do not depend on the call's other tokens.
// Constants measured on MI355X (256 x 128 blocks of 8 waves: a k-tile 1.29-1.46 us, prologue + epilogue 7-9 us,
// partials at ~4 TB/s). 0: not streamed.
constexpr uint32_t kDmaMaxSplits = 32;
constexpr uint32_t kCus = 256;
constexpr double kDmaKtileUs = 1.35, kDmaBlockUs = 8.0, kPartialBytesPerUs = 4.0e6, kReduceUs = 4.0;
uint32_t dma_down_splits(uint32_t m, uint32_t ncol, uint32_t k) {
    const uint32_t tiles = dma_tiles(m, ncol), ktiles = k / kBK;
    uint32_t best = 0;
    double best_us = 0.0;
    for (uint32_t splits = 1; splits <= kDmaMaxSplits; splits *= 2) {
        if (k % (kActBlock * splits) != 0 || k / kActBlock / splits > kDmaMaxActBlocks || tiles * splits < kDmaMinDownBlocks)
            continue;
        const double rounds = ceil_div(tiles * splits, kCus);
        double us = rounds * (static_cast<double>(ktiles) / splits * kDmaKtileUs + kDmaBlockUs);
        if (splits > 1) us += 8.0 * splits * rows_padded(m) * ncol / kPartialBytesPerUs + kReduceUs;
        if (best == 0 || us < best_us) best = splits, best_us = us;
    }
    return best;
}

// The streamed down GEMM's plan: `splits` k splits of every column tile (whole_n 0), or, where that is estimated faster,
// the first whole_n column tiles over all of K (one round of long blocks, writing y) and the others in `splits` k
// splits, whose partials cover only their columns. A wide K takes the whole-K tiles only where a tile holds all of its
// activation blocks' binades in LDS (bfloat16 weights leave the ring's B lo plane free for them). Priced as
// dma_down_splits: the split blocks that the CUs without a whole tile finish meanwhile, then whole rounds of the rest.
// MI355X, 2.8B shape at 4096 tokens (16 x 20 tiles, 320 k-tiles): 16 whole column tiles and 4 column tiles in 4 splits
// (256 + 256 blocks) against 4 splits of all 20 (1280 blocks), a fifth of the partials.
struct DownPlan {
    uint32_t splits, whole_n;
};
DownPlan dma_down_plan(uint32_t m, uint32_t ncol, uint32_t k, bool bf16) {
    const uint32_t uniform = dma_down_splits(m, ncol, k);
    DownPlan plan{uniform, 0};
    const uint32_t tiles_m = rows_padded(m) / kDmaBM, tiles_n = ncol / kDmaBN, ktiles = k / kBK;
    const uint32_t max_blocks = bf16 ? kDmaMaxActBlocks + kDmaStages * kDmaLoRuns : kDmaMaxActBlocks;
    if (uniform == 0 || k % kActBlock != 0 || k / kActBlock > max_blocks) return plan;
    const double partial_us = 8.0 * rows_padded(m) / kPartialBytesPerUs;  // per split and column
    double best_us = ceil_div(tiles_m * tiles_n * uniform, kCus) * (static_cast<double>(ktiles) / uniform * kDmaKtileUs + kDmaBlockUs) +
                     (uniform > 1 ? partial_us * uniform * ncol + kReduceUs : 0.0);
    const double whole_us = ktiles * kDmaKtileUs + kDmaBlockUs;
    for (uint32_t whole_n = 1; whole_n < tiles_n && tiles_m * whole_n <= kCus; ++whole_n)
        for (uint32_t splits = 2; splits <= kDmaMaxSplits; splits *= 2) {
            if (k % (kActBlock * splits) != 0 || k / kActBlock / splits > kDmaMaxActBlocks) continue;
            const double split_us = static_cast<double>(ktiles) / splits * kDmaKtileUs + kDmaBlockUs;
            const uint32_t free_cus = kCus - tiles_m * whole_n, pieces = tiles_m * (tiles_n - whole_n) * splits;
            const uint32_t meanwhile = free_cus * static_cast<uint32_t>(whole_us / split_us);
            const double span = pieces <= meanwhile ? max(whole_us, ceil_div(pieces, free_cus) * split_us)
                                                    : whole_us + ceil_div(pieces - meanwhile, kCus) * split_us;
            const double us = span + partial_us * splits * (tiles_n - whole_n) * kDmaBN + kReduceUs;
            if (us < best_us) plan = {splits, whole_n}, best_us = us;
        }
    return plan;
}

// Splits of the streamed up GEMM: 1 when its tiles alone fill the chip, else doubled (up to 8, each split at least
// one k-tile) until ~192 blocks; the partial sums then go through act_planes_kernel. 0: not streamed.
constexpr uint32_t kDmaMaxUpSplits = 8;
uint32_t dma_up_splits(uint32_t m, uint32_t ncol, uint32_t k) {
    const uint32_t tiles = dma_tiles(m, ncol);
    if (tiles >= kDmaMinBlocks) return 1;
    uint32_t splits = 1;
    while (splits < kDmaMaxUpSplits && tiles * splits < 192 && k % (kBK * splits * 2) == 0) splits *= 2;
    return tiles * splits >= kDmaMinBlocks ? splits : 0;
}

// Sampled products of the training backward from a dense product: G[rows, cols] = A[rows, n] B[cols, n]^T by the
// streamed GEMM (Epi::UpSplit partials [splits, rows, cols], powers of two undone), then one wave per owner row o:
// g[q] = sum over the splits (in split order) of G[o, idx[q]] for the row's slots q, and gb[o] = sum_t A[o, t]
// (lanes over the tokens, then the fixed xor butterfly).
__global__ __launch_bounds__(kThreads) void gather_dense_kernel(const float* __restrict__ partials, uint32_t splits,
                                                               const float* __restrict__ a, uint32_t ld, uint32_t n,
                                                               const int32_t* __restrict__ off, const int16_t* __restrict__ idx,
                                                               float* __restrict__ g, float* __restrict__ gb, uint32_t rows,
                                                               uint32_t cols) {
    const uint32_t o = blockIdx.x * (kThreads / kWave) + uniform(threadIdx.x / kWave), lane = threadIdx.x % kWave;
    if (o >= rows) return;
    // (kBatch loads per lane in flight; each lane's sums in the order of its tokens and splits)
    constexpr int kBatch = 16;
    float s = 0.0f;
    const float* arow = a + static_cast<size_t>(o) * ld;
    for (uint32_t t0 = lane; t0 < n; t0 += kBatch * kWave) {
        float v[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) v[j] = t0 + j * kWave < n ? arow[t0 + j * kWave] : 0.0f;
#pragma unroll
        for (int j = 0; j < kBatch; ++j)
            if (t0 + j * kWave < n) s += v[j];
    }
    s = wave_sum(s);
    if (lane == 0) gb[o] = s;
    const size_t plane = static_cast<size_t>(rows) * cols;
    const float* row = partials + static_cast<size_t>(o) * cols;
    const int32_t end = off[o + 1];
    // a batch's loads all issued before the first is used (no branch between them): a slot past the row reads the
    // row's last slot again, and its sum is not written
    for (int32_t q0 = off[o] + static_cast<int32_t>(lane); q0 < end; q0 += kBatch * kWave) {
        uint32_t c[kBatch];
        float v[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) c[j] = static_cast<uint16_t>(idx[min(q0 + j * static_cast<int32_t>(kWave), end - 1)]);
#pragma unroll
        for (int j = 0; j < kBatch; ++j) v[j] = row[c[j]];
        for (uint32_t sp = 1; sp < splits; ++sp) {
            float u[kBatch];
#pragma unroll
            for (int j = 0; j < kBatch; ++j) u[j] = row[sp * plane + c[j]];
#pragma unroll
            for (int j = 0; j < kBatch; ++j) v[j] += u[j];
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j)
            if (q0 + j * static_cast<int32_t>(kWave) < end) g[q0 + j * kWave] = v[j];
    }
}

// One row tile of at most 64 or 128 tokens takes the kernel that transfers and multiplies only those rows.
template <Epi EPI, bool LO_B>
hipError_t launch_dma(const _Float16* a_planes, const int32_t* a_exp, const _Float16* b_planes, const int32_t* b_exp,
                      const float* bias, float* out, _Float16* out_planes, int32_t* out_exp, uint32_t M, uint32_t Ncol, uint32_t K,
                      uint32_t splits, hipStream_t stream, uint32_t whole_n = 0, float* part = nullptr) {
    const uint32_t tiles_m = rows_padded(M) / kDmaBM, tiles_n = Ncol / kDmaBN;
    const dim3 grid(tiles_m * whole_n + tiles_m * (tiles_n - whole_n) * splits), block(64 * kDmaWaves);
    const uint32_t rows_pad = rows_padded(M), live = rows_live(M);
    if (live == 64)
        hipLaunchKernelGGL((gemm_dma_kernel<EPI, LO_B, 64>), grid, block, 0, stream, a_planes, a_exp, b_planes, b_exp, bias, out,
                           out_planes, out_exp, M, rows_pad, Ncol, K, splits, whole_n, part);
    else if (live == 128)
        hipLaunchKernelGGL((gemm_dma_kernel<EPI, LO_B, 128>), grid, block, 0, stream, a_planes, a_exp, b_planes, b_exp, bias, out,
                           out_planes, out_exp, M, rows_pad, Ncol, K, splits, whole_n, part);
    else
        hipLaunchKernelGGL((gemm_dma_kernel<EPI, LO_B, kDmaBM>), grid, block, 0, stream, a_planes, a_exp, b_planes, b_exp, bias, out,
                           out_planes, out_exp, M, rows_pad, Ncol, K, splits, whole_n, part);
    return hipGetLastError();
}

template <bool LO_B>
hipError_t dma_down(DownPlan plan, const _Float16* a_planes, const int32_t* a_exp, const _Float16* b_planes, const int32_t* b_exp,
                    const float* bias, float* y, float* partials, uint32_t M, uint32_t Ncol, uint32_t K, hipStream_t stream) {
    if (plan.splits == 1)
        return launch_dma<Epi::Down, LO_B>(a_planes, a_exp, b_planes, b_exp, bias, y, nullptr, nullptr, M, Ncol, K, 1, stream);
    const hipError_t status =
        plan.whole_n > 0 ? launch_dma<Epi::Down, LO_B>(a_planes, a_exp, b_planes, b_exp, bias, y, nullptr, nullptr, M, Ncol, K,
                                                       plan.splits, stream, plan.whole_n, partials)
                         : launch_dma<Epi::Down, LO_B>(a_planes, a_exp, b_planes, b_exp, bias, partials, nullptr, nullptr, M, Ncol, K,
                                                       plan.splits, stream);
    if (status != hipSuccess) return status;
    const uint32_t c0 = plan.whole_n * kDmaBN, width = Ncol - c0;
    const size_t quads = static_cast<size_t>(M) * width / 4;
    hipLaunchKernelGGL(reduce_splits_kernel, dim3(static_cast<uint32_t>((quads + kThreads - 1) / kThreads)), dim3(kThreads), 0, stream,
                       partials, bias, y, M, Ncol, plan.splits, width, c0);
    return hipGetLastError();
}

// Workspace layout (int32 words unless stated; rows = M padded to kRowPad): split counters [down tiles of the
// largest token count, 64 x 64 tiles] | x binades [rows] | activation block binades [rows, d_ff / kActBlock] |
// (256-byte aligned, bytes) x planes [rows * d_model * 2 halves] | activation planes [rows * d_ff * 2 halves] |
// float partials (partial_floats: the largest [splits, M, d_model] or [splits, M, d_ff] of any N up to M). The counters
// come first and are sized for every M and tile shape, so a call at
// any M finds them where the previous call, at any other M, left them (at zero).
struct Workspace {
    size_t counters, x_binades, act_binades, x_planes, act_planes, partials, bytes;
};

// Floats of split partial sums any call of up to m tokens may need (the register-staged down GEMM's kMaxSplits, or
// the streamed GEMMs' splits for every padded row count up to m's): a workspace sized for m serves every smaller n.
size_t partial_floats(uint32_t m, uint32_t d, uint32_t h) {
    size_t most = static_cast<size_t>(kMaxSplits) * m * d;
    for (uint32_t rows = kRowPad; rows <= rows_padded(m); rows += kRowPad) {
        const size_t tokens = min(m, rows);
        most = max(most, static_cast<size_t>(dma_down_splits(rows, d, h)) * tokens * d);
        for (const bool bf16 : {false, true}) {
            const DownPlan plan = dma_down_plan(rows, d, h, bf16);
            most = max(most, static_cast<size_t>(plan.splits) * tokens * (d - plan.whole_n * kDmaBN));
        }
        const uint32_t up = dma_up_splits(rows, h, d);
        if (up > 1) most = max(most, static_cast<size_t>(up) * tokens * h);
    }
    return most;
}

// The training products run the up-shaped GEMMs (the forward's up projection, gz) as split products with partials at
// every split count, one included: their partials need the largest [max(1, splits), M, d_ff] of any N up to M too.
size_t train_partial_floats(uint32_t m, uint32_t d, uint32_t h) {
    size_t most = partial_floats(m, d, h);
    for (uint32_t rows = kRowPad; rows <= rows_padded(m); rows += kRowPad)
        most = max(most, static_cast<size_t>(max(1u, dma_up_splits(rows, h, d))) * min(m, rows) * h);
    return most;
}

Workspace workspace_layout(uint32_t m, uint32_t d, uint32_t h, bool training = false) {
    const size_t rows = rows_padded(m);
    Workspace w{};
    w.counters = 0;
    const size_t counter_words = static_cast<size_t>(ceil_div(kMaxTokens, 64)) * (d / 64);
    // both binade tables start on 256-byte boundaries: the streamed GEMM transfers them into LDS 16 or 4 bytes a lane
    w.x_binades = (w.counters + counter_words + 63) / 64 * 64;
    w.act_binades = (w.x_binades + rows + 63) / 64 * 64;
    const size_t words_end = (w.act_binades + rows * (h / kActBlock) / 4) * 4;  // int8 activation binades
    w.x_planes = (words_end + 255) / 256 * 256;  // bytes from here on
    w.act_planes = w.x_planes + rows * d * 4;
    w.partials = w.act_planes + rows * h * 4;
    w.bytes = w.partials + (training ? train_partial_floats(m, d, h) : partial_floats(m, d, h)) * 4;
    return w;
}

}  // namespace

size_t dense_plane_halves(uint32_t rows, uint32_t k) { return static_cast<size_t>(rows) * k * 2; }

bool mfma_shape_supported(uint32_t d, uint32_t h) { return d % 256 == 0 && h % 256 == 0; }

bool mfma_streamed(uint32_t n, uint32_t d, uint32_t h) { return dma_up_splits(n, h, d) != 0 && dma_down_splits(n, d, h) != 0; }

// Workspace of the dense sampled product (bytes, 256-aligned parts): the planes of A [rows, k_pad] and B [cols,
// k_pad] (tokens padded to a multiple of 256, split_rows' k granularity), their row binades and the GEMM's partials.
namespace {
struct GradDenseLayout {
    size_t a_planes, b_planes, a_exp, b_exp, partials, bytes;
    uint32_t k_pad, splits;
};
size_t align256(size_t v) { return (v + 255) / 256 * 256; }
GradDenseLayout grad_dense_layout(uint32_t rows, uint32_t cols, uint32_t n) {
    GradDenseLayout l{};
    l.k_pad = ceil_div(n, 256) * 256;
    l.splits = dma_up_splits(rows, cols, l.k_pad);
    l.a_planes = 0;
    l.b_planes = align256(l.a_planes + dense_plane_halves(rows, l.k_pad) * 2);
    l.a_exp = align256(l.b_planes + dense_plane_halves(cols, l.k_pad) * 2);
    l.b_exp = align256(l.a_exp + static_cast<size_t>(rows) * 4);
    l.partials = align256(l.b_exp + static_cast<size_t>(cols) * 4);
    l.bytes = l.partials + static_cast<size_t>(l.splits) * rows * cols * 4;
    return l;
}
}  // namespace

size_t grad_dense_workspace_bytes(uint32_t rows, uint32_t cols, uint32_t n) {
    if (rows % kRowPad != 0 || cols % kDmaBN != 0) return 0;
    const GradDenseLayout l = grad_dense_layout(rows, cols, n);
    return l.splits == 0 ? 0 : l.bytes;
}

hipError_t launch_grad_dense(const float* row, const float* mat, const int32_t* off, const int16_t* idx, float* g, float* gb,
                             uint32_t rows, uint32_t cols, uint32_t n, uint32_t ld, void* workspace, hipStream_t stream) {
    const GradDenseLayout l = grad_dense_layout(rows, cols, n);
    char* w = static_cast<char*>(workspace);
    auto* a_planes = reinterpret_cast<_Float16*>(w + l.a_planes);
    auto* b_planes = reinterpret_cast<_Float16*>(w + l.b_planes);
    auto* a_exp = reinterpret_cast<int32_t*>(w + l.a_exp);
    auto* b_exp = reinterpret_cast<int32_t*>(w + l.b_exp);
    auto* partials = reinterpret_cast<float*>(w + l.partials);
    hipLaunchKernelGGL(split_rows_kernel, dim3(rows / kSplitBlockRows), dim3(kThreads), 0, stream, row, rows, rows, l.k_pad, ld, n,
                       a_planes, a_exp);
    hipLaunchKernelGGL(split_rows_kernel, dim3(cols / kSplitBlockRows), dim3(kThreads), 0, stream, mat, cols, cols, l.k_pad, ld, n,
                       b_planes, b_exp);
    if (hipError_t status = hipGetLastError(); status != hipSuccess) return status;
    if (hipError_t status = launch_dma<Epi::UpSplit, true>(a_planes, a_exp, b_planes, b_exp, nullptr, partials, nullptr, nullptr, rows,
                                                           cols, l.k_pad, l.splits, stream);
        status != hipSuccess)
        return status;
    hipLaunchKernelGGL(gather_dense_kernel, dim3(ceil_div(rows, kThreads / kWave)), dim3(kThreads), 0, stream, partials, l.splits, row,
                       ld, n, off, idx, g, gb, rows, cols);
    return hipGetLastError();
}

size_t mfma_workspace_bytes(uint32_t n, uint32_t d, uint32_t h) { return workspace_layout(n, d, h).bytes; }

hipError_t launch_densify(int vt, const int32_t* off, const int16_t* idx, const void* val, uint32_t rows, uint32_t k,
                          void* planes, int32_t* exps, hipStream_t stream) {
    const dim3 grid(ceil_div(rows, kDensRows), ceil_div(k, kDensChunk)), block(kDensThreads);
    if (vt == kBF16)
        hipLaunchKernelGGL((densify_kernel<uint16_t>), grid, block, 0, stream, off, idx, static_cast<const uint16_t*>(val), rows, k,
                           static_cast<_Float16*>(planes), exps);
    else
        hipLaunchKernelGGL((densify_kernel<float>), grid, block, 0, stream, off, idx, static_cast<const float*>(val), rows, k,
                           static_cast<_Float16*>(planes), exps);
    return hipGetLastError();
}

hipError_t launch_mfma_split(const float* x, void* workspace, uint32_t n, uint32_t d, uint32_t h, hipStream_t stream) {
    const Workspace w = workspace_layout(n, d, h);
    int32_t* words = static_cast<int32_t*>(workspace);
    auto* x_planes = reinterpret_cast<_Float16*>(static_cast<char*>(workspace) + w.x_planes);
    hipLaunchKernelGGL(split_rows_kernel, dim3(rows_live(n) / kSplitBlockRows), dim3(kThreads), 0, stream, x, n, rows_padded(n), d, d,
                       d, x_planes, words + w.x_binades);  // 8 rows per block
    return hipGetLastError();
}

hipError_t launch_mfma_up(int vt, const float* x, const void* planes, const int32_t* w_exp, const float* b_up, void* workspace,
                          uint32_t n, uint32_t d, uint32_t h, hipStream_t stream) {
    if (hipError_t status = launch_mfma_split(x, workspace, n, d, h, stream); status != hipSuccess) return status;
    return launch_mfma_up_planes(vt, planes, w_exp, b_up, workspace, n, d, h, stream);
}

hipError_t launch_mfma_up_planes(int vt, const void* planes, const int32_t* w_exp, const float* b_up, void* workspace, uint32_t n,
                                 uint32_t d, uint32_t h, hipStream_t stream) {
    const Workspace w = workspace_layout(n, d, h);
    int32_t* words = static_cast<int32_t*>(workspace);
    char* bytes = static_cast<char*>(workspace);
    auto* x_planes = reinterpret_cast<_Float16*>(bytes + w.x_planes);
    auto* act_planes = reinterpret_cast<_Float16*>(bytes + w.act_planes);
    const auto* p = static_cast<const _Float16*>(planes);
    if (const uint32_t splits = dma_up_splits(n, h, d); splits > 1) {
        float* partials = reinterpret_cast<float*>(bytes + w.partials);
        const hipError_t status =
            vt == kBF16 ? launch_dma<Epi::UpSplit, false>(x_planes, words + w.x_binades, p, w_exp, nullptr, partials, nullptr, nullptr, n,
                                                          h, d, splits, stream)
                        : launch_dma<Epi::UpSplit, true>(x_planes, words + w.x_binades, p, w_exp, nullptr, partials, nullptr, nullptr, n,
                                                         h, d, splits, stream);
        if (status != hipSuccess) return status;
        hipLaunchKernelGGL(act_planes_kernel, dim3(rows_live(n) / kActRowsPerBlock, h / kActBlock), dim3(kThreads), 0, stream, partials,
                           splits, b_up, act_planes, reinterpret_cast<int8_t*>(words + w.act_binades), n, rows_padded(n), h);
        return hipGetLastError();
    }
    if (dma_tiles(n, h) >= kDmaMinBlocks) {
        if (vt == kBF16)
            return launch_dma<Epi::Up, false>(x_planes, words + w.x_binades, p, w_exp, b_up, nullptr, act_planes, words + w.act_binades,
                                              n, h, d, 1, stream);
        return launch_dma<Epi::Up, true>(x_planes, words + w.x_binades, p, w_exp, b_up, nullptr, act_planes, words + w.act_binades, n,
                                         h, d, 1, stream);
    }
    const Shape shape = up_shape(n, h);
    if (vt == kBF16)
        return gemm<Epi::Up, false>(shape, x_planes, words + w.x_binades, p, w_exp, b_up, nullptr, act_planes, words + w.act_binades,
                                    nullptr, nullptr, n, h, d, stream);
    return gemm<Epi::Up, true>(shape, x_planes, words + w.x_binades, p, w_exp, b_up, nullptr, act_planes, words + w.act_binades,
                               nullptr, nullptr, n, h, d, stream);
}

hipError_t launch_mfma_down(int vt, const void* planes, const int32_t* v_exp, const float* b_down, float* y, void* workspace,
                            uint32_t n, uint32_t d, uint32_t h, hipStream_t stream) {
    const Workspace w = workspace_layout(n, d, h);
    int32_t* words = static_cast<int32_t*>(workspace);
    char* bytes = static_cast<char*>(workspace);
    const auto* act_planes = reinterpret_cast<const _Float16*>(bytes + w.act_planes);
    float* partials = reinterpret_cast<float*>(bytes + w.partials);
    const auto* p = static_cast<const _Float16*>(planes);
    if (const DownPlan plan = dma_down_plan(n, d, h, vt == kBF16); plan.splits != 0) {
        if (vt == kBF16)
            return dma_down<false>(plan, act_planes, words + w.act_binades, p, v_exp, b_down, y, partials, n, d, h, stream);
        return dma_down<true>(plan, act_planes, words + w.act_binades, p, v_exp, b_down, y, partials, n, d, h, stream);
    }
    const Shape shape = down_shape(n, d, h);
    if (vt == kBF16)
        return gemm<Epi::Down, false>(shape, act_planes, words + w.act_binades, p, v_exp, b_down, y, nullptr, nullptr, partials,
                                      words + w.counters, n, d, h, stream);
    return gemm<Epi::Down, true>(shape, act_planes, words + w.act_binades, p, v_exp, b_down, y, nullptr, nullptr, partials,
                                 words + w.counters, n, d, h, stream);
}

size_t train_mfma_workspace_bytes(uint32_t n, uint32_t d, uint32_t h) { return workspace_layout(n, d, h, true).bytes; }

// Training forward on the planes (fp32 weights): x split into planes, the up projection as a split product (partials
// at every split count) whose epilogue (train_planes_kernel<Forward>) writes z, act (hidden-major) and the activation
// planes, then the inference down GEMM: y. x_t = x transposed for the sampled product of g_up. The workspace is laid
// out as the MFMA workspace with the training partials (train_mfma_workspace_bytes).
hipError_t launch_train_forward(const float* x, const void* up_planes, const int32_t* up_exp, const float* b_up, const void* down_planes,
                                const int32_t* down_exp, const float* b_down, void* workspace, float* x_t, float* act, float* z, float* y,
                                uint32_t n, uint32_t d, uint32_t h, uint32_t ld, hipStream_t stream) {
    const Workspace w = workspace_layout(n, d, h, true);
    int32_t* words = static_cast<int32_t*>(workspace);
    char* bytes = static_cast<char*>(workspace);
    auto* x_planes = reinterpret_cast<_Float16*>(bytes + w.x_planes);
    auto* act_planes = reinterpret_cast<_Float16*>(bytes + w.act_planes);
    float* partials = reinterpret_cast<float*>(bytes + w.partials);
    if (hipError_t status = launch_transpose(x, x_t, n, d, d, ld, stream); status != hipSuccess) return status;
    hipLaunchKernelGGL(split_rows_kernel, dim3(rows_live(n) / kSplitBlockRows), dim3(kThreads), 0, stream, x, n, rows_padded(n), d, d,
                       d, x_planes, words + w.x_binades);
    if (hipError_t status = hipGetLastError(); status != hipSuccess) return status;
    const uint32_t splits = max(1u, dma_up_splits(n, h, d));
    if (hipError_t status = launch_dma<Epi::UpSplit, true>(x_planes, words + w.x_binades, static_cast<const _Float16*>(up_planes), up_exp,
                                                           nullptr, partials, nullptr, nullptr, n, h, d, splits, stream);
        status != hipSuccess)
        return status;
    hipLaunchKernelGGL(train_planes_kernel<TrainPost::Forward>, dim3(rows_live(n) / kActRowsPerBlock, h / kActBlock), dim3(kThreads), 0,
                       stream, partials, splits, b_up, nullptr, z, act, act_planes, reinterpret_cast<int8_t*>(words + w.act_binades), n,
                       rows_padded(n), h, ld);
    if (hipError_t status = hipGetLastError(); status != hipSuccess) return status;
    return launch_mfma_down(kF32, down_planes, down_exp, b_down, y, workspace, n, d, h, stream);
}

// Training backward products on the planes: gy split into planes; gz = (gy W_down) * gelu'(z) as a split product over
// the planes of W_down^T [d_ff rows, d_model k] whose epilogue (train_planes_kernel<GradZ>) writes gz hidden-major and
// as planes; gx = gz W_up by the down GEMM over the planes of W_up^T [d_model rows, d_ff k], without bias.
hipError_t launch_train_backward(const float* gy, const float* z, const void* down_t_planes, const int32_t* down_t_exp,
                                 const void* up_t_planes, const int32_t* up_t_exp, void* workspace, float* gz, float* gx, uint32_t n,
                                 uint32_t d, uint32_t h, uint32_t ld, hipStream_t stream) {
    const Workspace w = workspace_layout(n, d, h, true);
    int32_t* words = static_cast<int32_t*>(workspace);
    char* bytes = static_cast<char*>(workspace);
    auto* gy_planes = reinterpret_cast<_Float16*>(bytes + w.x_planes);
    auto* gz_planes = reinterpret_cast<_Float16*>(bytes + w.act_planes);
    float* partials = reinterpret_cast<float*>(bytes + w.partials);
    hipLaunchKernelGGL(split_rows_kernel, dim3(rows_live(n) / kSplitBlockRows), dim3(kThreads), 0, stream, gy, n, rows_padded(n), d, d,
                       d, gy_planes, words + w.x_binades);
    if (hipError_t status = hipGetLastError(); status != hipSuccess) return status;
    const uint32_t splits = max(1u, dma_up_splits(n, h, d));
    if (hipError_t status = launch_dma<Epi::UpSplit, true>(gy_planes, words + w.x_binades, static_cast<const _Float16*>(down_t_planes),
                                                           down_t_exp, nullptr, partials, nullptr, nullptr, n, h, d, splits, stream);
        status != hipSuccess)
        return status;
    hipLaunchKernelGGL(train_planes_kernel<TrainPost::GradZ>, dim3(rows_live(n) / kActRowsPerBlock, h / kActBlock), dim3(kThreads), 0,
                       stream, partials, splits, nullptr, z, gz, nullptr, gz_planes, reinterpret_cast<int8_t*>(words + w.act_binades), n,
                       rows_padded(n), h, ld);
    if (hipError_t status = hipGetLastError(); status != hipSuccess) return status;
    return launch_mfma_down(kF32, up_t_planes, up_t_exp, nullptr, gx, workspace, n, d, h, stream);
}

}  // namespace hffn
