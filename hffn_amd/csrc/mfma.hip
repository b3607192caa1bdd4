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
// Plane layout (tile-major, for 128-byte transactions): for k-tile kt (32 wide) and row n, 32 hi halves then 32 lo
// halves, i.e. planes[((kt * rows + n) * 2 + part) * 32 + k % 32]; a block's B tile of BN rows is one contiguous
// run of BN * 128 bytes.
//
// Kernels: row_binade (per-row power of two of the fp32 input), densify (load time), gemm_split<Up|Down>.
// The up epilogue applies bias and exact GELU, writes the activations token-major [N, d_ff] in fp32, and, per token
// row and block of BN neurons, the binade of the largest activation; the down kernel takes, per token, the largest
// of those binades as its row scale. No atomics: every output is written by one lane.
#include "common.hpp"
#include "launch.hpp"

namespace hffn {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kBK = 32;          // k per staged step, one plane k-tile
constexpr int kRow = kBK + 8;    // halves per LDS row: 80-byte stride keeps 16-byte lane reads conflict-free

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
    // zero this row in every k-tile (64 halves per tile: hi then lo)
    const uint32_t tiles = k / kBK;
    for (uint32_t i = threadIdx.x; i < tiles * 64; i += kThreads) {
        const uint32_t kt = i / 64, j = i % 64;
        planes[(static_cast<size_t>(kt) * rows + n) * 64 + j] = static_cast<_Float16>(0.0f);
    }
    __syncthreads();
    uint32_t mx = 0;
#pragma unroll
    for (int w = 0; w < kThreads / kWave; ++w) mx = max(mx, part[w]);
    const int e = binade_of_bits(mx);
    for (int32_t s = begin + static_cast<int32_t>(threadIdx.x); s < end; s += kThreads) {
        const uint32_t c = static_cast<uint16_t>(idx[s]);
        _Float16 hi, lo;
        split(ldexpf(widen(val[s]), -e), hi, lo);
        _Float16* row = planes + (static_cast<size_t>(c / kBK) * rows + n) * 64 + c % kBK;
        row[0] = hi;
        row[32] = lo;
    }
    if (threadIdx.x == 0) exps[n] = e;
}

// ------------------------------------------------------------------------------------------------ GEMM
enum class Epi { Up, Down };

template <Epi EPI, int BM, int BN, bool LO_B>
__global__ __launch_bounds__(kThreads) void gemm_split_kernel(
    const float* __restrict__ a,          // [M, K] fp32 row-major
    const int32_t* __restrict__ a_exp,    // Up: [M] row binades; Down: [M, a_blocks] block binades (max taken here)
    uint32_t a_blocks,
    const _Float16* __restrict__ planes,  // tile-major planes of B [Ncol, K]
    const int32_t* __restrict__ b_exp,    // [Ncol]
    const float* __restrict__ bias,       // [Ncol]
    float* __restrict__ out,              // [M, Ncol] fp32 row-major
    int32_t* __restrict__ out_exp,        // Up: [M, Ncol / BN] activation block binades
    uint32_t M, uint32_t Ncol, uint32_t K) {
    static_assert(BM == 64 || BM == 128, "BM");
    static_assert(BN == 64 || BN == 128, "BN");
    constexpr int MI = BM / 64, NI = BN / 64;        // 32x32 MFMA tiles per wave (2x2 waves)
    constexpr int TPR = kThreads / BM;               // staging threads per A row
    constexpr int FPT = kBK / TPR;                   // floats per staging thread (16 or 8)
    constexpr int BBYTES = BN * 128 / kThreads;      // bytes of B per staging thread (64 or 32)

    __shared__ __attribute__((aligned(16))) _Float16 a_hi[BM * kRow], a_lo[BM * kRow], b_hi[BN * kRow], b_lo[BN * kRow];
    __shared__ int32_t row_e[BM];
    __shared__ uint32_t row_max[2][BM];

    const uint32_t tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    const uint32_t wm = wave / 2, wn = wave % 2;
    const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

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

    // staging assignments
    const uint32_t a_row = tid / TPR, a_col = (tid % TPR) * FPT;
    const bool a_valid = m0 + a_row < M;
    const float* a_src = a + static_cast<size_t>(m0 + (a_valid ? a_row : 0)) * K + a_col;
    const float a_scale = ldexpf(1.0f, -row_e[a_row]);
    const char* b_base = reinterpret_cast<const char*>(planes) + static_cast<size_t>(n0) * 128 + tid * BBYTES;
    const size_t b_stride = static_cast<size_t>(Ncol) * 128;  // bytes per k-tile
    // B staging target: BN=128 -> row tid/2, part tid%2, 32 halves; BN=64 -> row tid/4, part (tid/2)%2, 16 halves at (tid%2)*16
    const uint32_t b_row = BN == 128 ? tid / 2 : tid / 4;
    const uint32_t b_part = BN == 128 ? tid % 2 : (tid / 2) % 2;
    const uint32_t b_col = BN == 128 ? 0 : (tid % 2) * 16;
    _Float16* b_dst = (b_part == 0 ? b_hi : b_lo) + b_row * kRow + b_col;

    float4 a_reg[FPT / 4];
    uint4 b_reg[BBYTES / 16];

    auto load = [&](uint32_t kt) {
        if (a_valid) {
#pragma unroll
            for (int i = 0; i < FPT / 4; ++i) a_reg[i] = *reinterpret_cast<const float4*>(a_src + kt * kBK + 4 * i);
        } else {
#pragma unroll
            for (int i = 0; i < FPT / 4; ++i) a_reg[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        const uint4* src = reinterpret_cast<const uint4*>(b_base + kt * b_stride);
#pragma unroll
        for (int i = 0; i < BBYTES / 16; ++i) b_reg[i] = src[i];
    };
    auto stage = [&]() {
        _Float16* hi_dst = a_hi + a_row * kRow + a_col;
        _Float16* lo_dst = a_lo + a_row * kRow + a_col;
#pragma unroll
        for (int i = 0; i < FPT / 8; ++i) {
            half8 h, l;
            const float v[8] = {a_reg[2 * i].x, a_reg[2 * i].y, a_reg[2 * i].z, a_reg[2 * i].w,
                                a_reg[2 * i + 1].x, a_reg[2 * i + 1].y, a_reg[2 * i + 1].z, a_reg[2 * i + 1].w};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                _Float16 hh, ll;
                split(v[j] * a_scale, hh, ll);
                h[j] = hh;
                l[j] = ll;
            }
            *reinterpret_cast<half8*>(hi_dst + 8 * i) = h;
            *reinterpret_cast<half8*>(lo_dst + 8 * i) = l;
        }
#pragma unroll
        for (int i = 0; i < BBYTES / 16; ++i) *reinterpret_cast<uint4*>(b_dst + 8 * i) = b_reg[i];
    };

    floatx16 acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const uint32_t ktiles = K / kBK;
    load(0);
    for (uint32_t kt = 0; kt < ktiles; ++kt) {
        stage();
        __syncthreads();
        if (kt + 1 < ktiles) load(kt + 1);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const uint32_t koff = kk * 16 + 8 * (lane / 32);
            half8 ah[MI], al[MI], bh[NI], bl[NI];
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                const uint32_t r = wm * (BM / 2) + i * 32 + lane % 32;
                ah[i] = *reinterpret_cast<const half8*>(a_hi + r * kRow + koff);
                al[i] = *reinterpret_cast<const half8*>(a_lo + r * kRow + koff);
            }
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                const uint32_t r = wn * (BN / 2) + j * 32 + lane % 32;
                bh[j] = *reinterpret_cast<const half8*>(b_hi + r * kRow + koff);
                if constexpr (LO_B) bl[j] = *reinterpret_cast<const half8*>(b_lo + r * kRow + koff);
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
        __syncthreads();
    }

    // epilogue: accumulator r of lane l of tile (i, j) holds row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32
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
                float v = ldexpf(acc[i][j][r], row_e[m] + ce) + cb;
                if constexpr (EPI == Epi::Up) {
                    v = gelu(v);
                    lane_max[i][r] = max(lane_max[i][r], abs_bits(v));
                }
                if (m0 + m < M) out[static_cast<size_t>(m0 + m) * Ncol + col] = v;
            }
    }
    if constexpr (EPI == Epi::Up) {
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
            out_exp[static_cast<size_t>(m0 + tid) * (Ncol / BN) + blockIdx.x] = binade_of_bits(max(row_max[0][tid], row_max[1][tid]));
    }
}

uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

template <Epi EPI, bool LO_B>
hipError_t gemm(int bm, int bn, const float* a, const int32_t* a_exp, uint32_t a_blocks, const _Float16* planes, const int32_t* b_exp,
                const float* bias, float* out, int32_t* out_exp, uint32_t M, uint32_t Ncol, uint32_t K, hipStream_t stream) {
    const dim3 block(kThreads);
    const dim3 grid(Ncol / bn, ceil_div(M, bm));
    if (bm == 128 && bn == 128)
        hipLaunchKernelGGL((gemm_split_kernel<EPI, 128, 128, LO_B>), grid, block, 0, stream, a, a_exp, a_blocks, planes, b_exp, bias, out, out_exp, M, Ncol, K);
    else if (bm == 64 && bn == 128)
        hipLaunchKernelGGL((gemm_split_kernel<EPI, 64, 128, LO_B>), grid, block, 0, stream, a, a_exp, a_blocks, planes, b_exp, bias, out, out_exp, M, Ncol, K);
    else if (bm == 128 && bn == 64)
        hipLaunchKernelGGL((gemm_split_kernel<EPI, 128, 64, LO_B>), grid, block, 0, stream, a, a_exp, a_blocks, planes, b_exp, bias, out, out_exp, M, Ncol, K);
    else
        hipLaunchKernelGGL((gemm_split_kernel<EPI, 64, 64, LO_B>), grid, block, 0, stream, a, a_exp, a_blocks, planes, b_exp, bias, out, out_exp, M, Ncol, K);
    return hipGetLastError();
}

}  // namespace

size_t dense_plane_halves(uint32_t rows, uint32_t k) { return static_cast<size_t>(rows) * k * 2; }

uint32_t mfma_block_cols(uint32_t ncol) { return ncol % 128 == 0 ? 128 : 64; }

uint32_t mfma_block_rows(uint32_t m, uint32_t ncol) {
    // 128-row tiles unless that leaves most of the 256 CUs without a block
    const uint32_t bn = mfma_block_cols(ncol);
    return ceil_div(m, 128) * (ncol / bn) >= 256 ? 128 : 64;
}

hipError_t launch_row_binades(const float* x, uint32_t rows, uint32_t cols, int32_t* e, hipStream_t stream) {
    hipLaunchKernelGGL(row_binade_kernel, dim3(ceil_div(rows, kThreads / kWave)), dim3(kThreads), 0, stream, x, rows, cols, e);
    return hipGetLastError();
}

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

hipError_t launch_mfma_up(int vt, const float* x, const int32_t* x_exp, const void* planes, const int32_t* w_exp,
                          const float* b_up, float* act, int32_t* act_exp, uint32_t n, uint32_t d, uint32_t h,
                          hipStream_t stream) {
    const uint32_t bn = mfma_block_cols(h), bm = mfma_block_rows(n, h);
    const auto* p = static_cast<const _Float16*>(planes);
    if (vt == kBF16) return gemm<Epi::Up, false>(bm, bn, x, x_exp, 1, p, w_exp, b_up, act, act_exp, n, h, d, stream);
    return gemm<Epi::Up, true>(bm, bn, x, x_exp, 1, p, w_exp, b_up, act, act_exp, n, h, d, stream);
}

hipError_t launch_mfma_down(int vt, const float* act, const int32_t* act_exp, const void* planes, const int32_t* v_exp,
                            const float* b_down, float* y, uint32_t n, uint32_t d, uint32_t h, hipStream_t stream) {
    const uint32_t bn = mfma_block_cols(d), bm = mfma_block_rows(n, d);
    const uint32_t blocks = h / mfma_block_cols(h);
    const auto* p = static_cast<const _Float16*>(planes);
    if (vt == kBF16) return gemm<Epi::Down, false>(bm, bn, act, act_exp, blocks, p, v_exp, b_down, y, nullptr, n, d, h, stream);
    return gemm<Epi::Down, true>(bm, bn, act, act_exp, blocks, p, v_exp, b_down, y, nullptr, n, d, h, stream);
}

}  // namespace hffn
