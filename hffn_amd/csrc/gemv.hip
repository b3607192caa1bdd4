// Decode-sized projections over the densified planes (gfx950, wave64): both projections of the layer for 1-64 tokens
// on v_mfma_f32_16x16x32_f16, one kernel per projection (and, for a large side whose row tiles alone leave CUs idle,
// a small second kernel adding its k splits). A decode call is bound by reading the weights once; the MFMA units
// deliver the operands, so the cost per token stays small (an fp32 FMA GEMV spends its time feeding every lane the
// inputs of every token).
//
// Planes as the MFMA path keeps them (mfma.hip): planes[(((kt*2 + p)*4 + c)*rows + r)*8 + k % 8], kt = k / 32,
// c = (k % 32) / 8, p = 0 hi / 1 lo, one power of two per row. A block takes 16 rows (neurons) over the whole K or
// one of 2-8 k splits (blockIdx.y); its W waves (16 when the row tiles, times the splits, do not outnumber the CUs
// and K has a 32-k tile for each; 4 when the row tiles outnumber the CUs; else 8)
// split that range in W spans of whole 32-k tiles. Per tile, lane (r, c) = (lane % 16, lane / 16) holds row r's
// chunk c of both planes as the B operand (the 16 lanes of a chunk read 256 contiguous bytes), and the 8 inputs of
// token r at the same k as the A operand, scaled by the token's power of two over the tile and split into fp16 hi and
// lo: D[token, row] = x_hi w_hi + x_hi w_lo + x_lo w_hi (x_hi w_hi + x_lo w_hi for bf16 weights, read from the hi
// plane only: exact for entries down to 2^-14 of their row's largest magnitude; below, fp16 subnormals keep fewer
// bits, an error of at most ~2^-25 of that magnitude per weight), accumulated in fp32 with the token's power of two
// undone exactly. The waves' sums are added in wave order
// (then the splits' partials in split order by gemv_reduce_kernel), then the row's power of two is undone; every
// output is written by one thread, the sums do not depend on the other tokens of the call, and the bits repeat run to
// run.
//
// Up: act[t, r] = gelu(b_up[r] + sum_k W_up[r, k] x[t, k]) (token-major act); down: y[t, o] = b_down[o] +
// sum_r W_down[o, r] act[t, r].
#include <algorithm>
#include <mutex>

#include "../../include/hffn_amd.h"
#include "common.hpp"
#include "launch.hpp"

namespace hffn {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kGemvRows = 16;   // rows per block: one MFMA column tile
constexpr uint32_t kGemvTile = 16;   // tokens per MFMA row tile
constexpr uint32_t kGemvK = 32;      // k per MFMA, one plane k-tile
constexpr uint32_t kGemvMinBlocks = 256;  // blocks of one round (one per CU); fewer row tiles call for splits or 16 waves

// Power of two of a token's 32 inputs of a k-tile: floor(log2(m)) - 12, clamped, so that the largest scaled input lies
// in 2^12 .. 2^13 and lo stays a normal fp16 down to 2^-15 of it (the weight planes are lifted the same way: scaled
// products stay below 2^26); -12 for zero.
__device__ __forceinline__ int gemv_binade(uint32_t bits) {
    const int e = bits == 0 ? 0 : static_cast<int>((bits >> 23) & 0xff) - 127;
    return min(max(e, -100), 100) - 12;
}

template <int W, int TT, bool LO_B, bool UP>
__global__ __launch_bounds__(W* kWave) void gemv_mfma_kernel(const float* __restrict__ in,        // [n, K]
                                                                 const _Float16* __restrict__ planes,  // [K/32][8][rows][8]
                                                                 const int32_t* __restrict__ exps,     // [rows]
                                                                 const float* __restrict__ bias,       // [rows]
                                                                 float* __restrict__ out,              // [n, rows]
                                                                 float* __restrict__ partials,  // [splits, n, rows] when split
                                                                 uint32_t rows, uint32_t K, uint32_t n) {
    constexpr uint32_t kTokens = TT * kGemvTile;
    constexpr uint32_t kThreads = W * kWave;
    // k-tiles whose loads are issued together, within the VGPR budget (128 per lane with 16 waves, 256 with 8)
    constexpr uint32_t kChunk = W >= 16 ? (TT >= 4 ? 1 : 4 / TT) : (TT >= 4 ? 4 : 8);
    __shared__ float sums[W][kTokens][kGemvRows];
    const uint32_t lane = threadIdx.x % kWave, wave = uniform(threadIdx.x / kWave);
    const uint32_t r = lane % 16, c = lane / 16;
    const uint32_t row = blockIdx.x * kGemvRows + r;  // < rows: the grid covers rows exactly (rows % 16 == 0)
    const uint32_t splits = gridDim.y;  // k splits of the row tile (blockIdx.y); K % (32 W splits) == 0
    const uint32_t tiles = K / kGemvK / W / splits, kt0 = (blockIdx.y * W + wave) * tiles;
    const size_t run = static_cast<size_t>(rows) * 8;  // halves between consecutive runs
    const _Float16* wbase = planes + static_cast<size_t>(c) * run + static_cast<size_t>(row) * 8;
    floatx4 acc[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) acc[tt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t j0 = 0; j0 < tiles; j0 += kChunk) {
        const uint32_t count = min(tiles - j0, kChunk);
        half8 wh[kChunk], wl[kChunk];
        float v[kChunk][TT][8];
#pragma unroll
        for (uint32_t j = 0; j < kChunk; ++j) {
            if (j >= count) break;
            const _Float16* p = wbase + static_cast<size_t>(kt0 + j0 + j) * 8 * run;
            wh[j] = *reinterpret_cast<const half8*>(p);
            if constexpr (LO_B) wl[j] = *reinterpret_cast<const half8*>(p + 4 * run);
        }
#pragma unroll
        for (uint32_t j = 0; j < kChunk; ++j) {
            if (j >= count) break;
            const uint32_t k = (kt0 + j0 + j) * kGemvK + c * 8;
#pragma unroll
            for (int tt = 0; tt < TT; ++tt) {
                const uint32_t t = tt * kGemvTile + r;
                if (t < n) load_vec<8>(in + static_cast<size_t>(t) * K + k, v[j][tt]);
                else {
#pragma unroll
                    for (int i = 0; i < 8; ++i) v[j][tt][i] = 0.0f;
                }
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < kChunk; ++j) {
            if (j >= count) break;
#pragma unroll
            for (int tt = 0; tt < TT; ++tt) {
                // the token's power of two over this 32-k tile: its 32 inputs sit in lanes r, r + 16, r + 32, r + 48
                uint32_t m = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) m = max(m, __float_as_uint(v[j][tt][i]) & 0x7fffffffu);
                m = max(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), 16, kWave)));
                m = max(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), 32, kWave)));
                const int e = gemv_binade(m);
                const float scale = ldexpf(1.0f, -e);
                half8 xh, xl;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float s = v[j][tt][i] * scale;
                    const _Float16 h = static_cast<_Float16>(s);
                    xh[i] = h;
                    xl[i] = static_cast<_Float16>(s - static_cast<float>(h));
                }
                floatx4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, wh[j], floatx4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                if constexpr (LO_B) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, wl[j], d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, wh[j], d, 0, 0, 0);
                // D register i holds token 4c + i: undo that token's power of two (held by lane 4c + i) exactly
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[tt][i] += ldexpf(d[i], __shfl(e, static_cast<int>(4 * c + i), kWave));
            }
        }
    }
    // D register i of token tile tt: token tt*16 + 4c + i, row r
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) sums[wave][tt * kGemvTile + 4 * c + i][r] = acc[tt][i];
    __syncthreads();
    for (uint32_t o = threadIdx.x; o < kTokens * kGemvRows; o += kThreads) {
        const uint32_t t = o / kGemvRows, rr = o % kGemvRows, out_row = blockIdx.x * kGemvRows + rr;
        if (t >= n) break;
        float s = sums[0][t][rr];
#pragma unroll
        for (uint32_t w = 1; w < W; ++w) s += sums[w][t][rr];
        if (splits > 1) {
            partials[(static_cast<size_t>(blockIdx.y) * n + t) * rows + out_row] = s;
        } else {
            const float z = ldexpf(s, exps[out_row]) + bias[out_row];
            out[static_cast<size_t>(t) * rows + out_row] = UP ? gelu(z) : z;
        }
    }
}

// out[t, r] = epilogue(sum of the k splits' partials in split order); one thread per output.
template <bool UP>
__global__ __launch_bounds__(256) void gemv_reduce_kernel(const float* __restrict__ partials, uint32_t splits,
                                                          const int32_t* __restrict__ exps, const float* __restrict__ bias,
                                                          float* __restrict__ out, uint32_t rows, uint32_t n) {
    const uint32_t o = blockIdx.x * 256 + threadIdx.x;
    if (o >= n * rows) return;
    const uint32_t row = o % rows;
    const size_t stride = static_cast<size_t>(n) * rows;
    float s = partials[o];
    for (uint32_t k = 1; k < splits; ++k) s += partials[k * stride + o];
    const float z = ldexpf(s, exps[row]) + bias[row];
    out[o] = UP ? gelu(z) : z;
}

// k splits of a projection whose row tiles alone leave CUs idle: the most (up to 8) that still fit one round of
// kGemvMinBlocks blocks of 8 waves, each wave keeping at least one 32-k tile; none for a side of less than
// kGemvSplitBytes of planes, where the second kernel costs more than the split gains.
constexpr size_t kGemvSplitBytes = size_t(8) << 20;
uint32_t gemv_splits(uint32_t rows, uint32_t K, uint32_t weight_bytes) {
    constexpr uint32_t kMaxSplits = 8;
    if (static_cast<size_t>(rows) * K * weight_bytes < kGemvSplitBytes) return 1;
    uint32_t splits = 1;
    while (splits < kMaxSplits && rows / kGemvRows * splits * 2 <= kGemvMinBlocks && K % (2 * splits * 8 * kGemvK) == 0) splits *= 2;
    return splits;
}

template <int W, bool LO_B, bool UP>
void gemv_launch(const float* in, const _Float16* planes, const int32_t* exps, const float* bias, float* out, float* partials,
                 uint32_t splits, uint32_t rows, uint32_t K, uint32_t n, hipStream_t stream) {
    const dim3 grid(rows / kGemvRows, splits), block(W * kWave);
    if (n <= kGemvTile)
        hipLaunchKernelGGL((gemv_mfma_kernel<W, 1, LO_B, UP>), grid, block, 0, stream, in, planes, exps, bias, out, partials, rows, K, n);
    else if (n <= 2 * kGemvTile)
        hipLaunchKernelGGL((gemv_mfma_kernel<W, 2, LO_B, UP>), grid, block, 0, stream, in, planes, exps, bias, out, partials, rows, K, n);
    else
        hipLaunchKernelGGL((gemv_mfma_kernel<W, 4, LO_B, UP>), grid, block, 0, stream, in, planes, exps, bias, out, partials, rows, K, n);
}

// k splits (added by gemv_reduce_kernel) where gemv_splits finds them worth a second kernel; 16 waves per block
// while the blocks do not outnumber the CUs (more load streams per CU) and K allows, 4 waves when the row tiles do
// outnumber them (2-3 blocks of 4 waves then share a CU, so every block is resident from the start), else 8.
template <bool LO_B, bool UP>
hipError_t gemv_side(const float* in, const void* planes, const int32_t* exps, const float* bias, float* out, float* partials,
                     uint32_t rows, uint32_t K, uint32_t n, hipStream_t stream) {
    const auto* p = static_cast<const _Float16*>(planes);
    const uint32_t splits = gemv_splits(rows, K, LO_B ? 4 : 2);
    if (splits > 1) {
        if (K % (16 * kGemvK * splits) == 0) gemv_launch<16, LO_B, UP>(in, p, exps, bias, out, partials, splits, rows, K, n, stream);
        else gemv_launch<8, LO_B, UP>(in, p, exps, bias, out, partials, splits, rows, K, n, stream);
        if (hipError_t status = hipGetLastError(); status != hipSuccess) return status;
        hipLaunchKernelGGL(gemv_reduce_kernel<UP>, dim3((n * rows + 255) / 256), dim3(256), 0, stream, partials, splits, exps, bias, out,
                           rows, n);
    } else if (rows / kGemvRows <= kGemvMinBlocks && K % (16 * kGemvK) == 0) {
        gemv_launch<16, LO_B, UP>(in, p, exps, bias, out, partials, 1, rows, K, n, stream);
    } else if (rows / kGemvRows > kGemvMinBlocks) {
        gemv_launch<4, LO_B, UP>(in, p, exps, bias, out, partials, 1, rows, K, n, stream);
    } else {
        gemv_launch<8, LO_B, UP>(in, p, exps, bias, out, partials, 1, rows, K, n, stream);
    }
    return hipGetLastError();
}

// The k-split partials of the allocation-free entry point: one array per GPU, alive until the process ends. Splits
// are taken only while rows / 16 * splits <= kGemvMinBlocks, so a split side holds at most 16 * kGemvMinBlocks rows'
// worth of partials for kGemvMaxTokens tokens: 64 * 4096 floats (1 MiB) for every shape.
constexpr size_t kScratchFloats = size_t(kGemvMaxTokens) * kGemvRows * kGemvMinBlocks;
static __device__ __align__(256) float scratch[kScratchFloats];
static_assert(sizeof(scratch) == HFFN_GEMV_STATIC_SCRATCH_BYTES, "the header states the scratch size");

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch[kMaxDevices] = {};  // device address of `scratch` on each GPU, looked up once per GPU

}  // namespace

size_t gemv_scratch_bytes() { return kScratchFloats * sizeof(float); }

hipError_t gemv_scratch_address(float** address) {
    int device = 0;
    if (const hipError_t status = hipGetDevice(&device); status != hipSuccess) return status;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    const std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch[device]) {
        void* found = nullptr;
        if (const hipError_t status = hipGetSymbolAddress(&found, HIP_SYMBOL(scratch)); status != hipSuccess) return status;
        g_scratch[device] = static_cast<float*>(found);
    }
    *address = g_scratch[device];
    return hipSuccess;
}

size_t gemv_workspace_bytes(uint32_t d, uint32_t h) {
    const size_t up = gemv_splits(h, d, 4), down = gemv_splits(d, h, 4);  // fp32 weights split at least as often
    const size_t floats = std::max(up > 1 ? up * kGemvMaxTokens * h : 0, down > 1 ? down * kGemvMaxTokens * d : 0);
    return std::max<size_t>(floats * sizeof(float), 256);
}

hipError_t launch_gemv_forward(int vt, const float* x, const void* up_planes, const int32_t* up_exps, const float* b_up,
                               const void* down_planes, const int32_t* down_exps, const float* b_down, float* act, float* work,
                               float* y, uint32_t d, uint32_t h, uint32_t n, hipStream_t stream) {
    const hipError_t status = vt == kBF16 ? gemv_side<false, true>(x, up_planes, up_exps, b_up, act, work, h, d, n, stream)
                                          : gemv_side<true, true>(x, up_planes, up_exps, b_up, act, work, h, d, n, stream);
    if (status != hipSuccess) return status;
    return vt == kBF16 ? gemv_side<false, false>(act, down_planes, down_exps, b_down, y, work, d, h, n, stream)
                       : gemv_side<true, false>(act, down_planes, down_exps, b_down, y, work, d, h, n, stream);
}

}  // namespace hffn
