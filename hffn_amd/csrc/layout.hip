// Output-major transpose of the hidden-major down store, built on the device once at load.
//
// Result (runtime/gpu/nvidia/common/kernels/hffn_cuda/runtime.py:55-67): for output o, the slots s
// with down_idx[s] == o in increasing s (a stable counting sort by output), i.e.
//   out_offsets = [0, cumsum(bincount(down_idx, d))],
//   out_hidden[p] = hidden neuron owning slot order[p], out_val[p] = down_val[order[p]].
// Three kernels, no floating point, deterministic by construction:
//   count  one block per chunk of consecutive slots counts each output in LDS;
//   scan   one block turns the [chunk, output] counts into the first position of every
//          (chunk, output) run and writes out_offsets;
//   place  one wave per chunk walks its slots 64 at a time; a slot's place is its run start plus
//          the number of earlier slots of the chunk with the same output (lane ranks by
//          readlane, then one cursor update per output by the last lane that holds it).
#include "common.hpp"
#include "launch.hpp"

namespace hffn {
namespace {

constexpr uint32_t kMaxChunks = 1024;
constexpr uint32_t kMinChunk = 2048;

__global__ __launch_bounds__(256) void count_kernel(const int16_t* __restrict__ idx, uint32_t nnz, uint32_t d,
                                                    uint32_t chunk, int32_t* __restrict__ counts) {
    extern __shared__ int32_t bins[];
    for (uint32_t o = threadIdx.x; o < d; o += blockDim.x) bins[o] = 0;
    __syncthreads();
    const uint32_t s0 = blockIdx.x * chunk;
    const uint32_t s1 = min(nnz, s0 + chunk);
    for (uint32_t s = s0 + threadIdx.x; s < s1; s += blockDim.x) atomicAdd(&bins[static_cast<uint16_t>(idx[s])], 1);
    __syncthreads();
    for (uint32_t o = threadIdx.x; o < d; o += blockDim.x) counts[static_cast<size_t>(blockIdx.x) * d + o] = bins[o];
}

// One block of 1024 threads; thread k owns outputs [k * per, (k + 1) * per).
__global__ __launch_bounds__(1024) void scan_kernel(int32_t* __restrict__ counts, uint32_t chunks, uint32_t d,
                                                    int32_t* __restrict__ out_offsets) {
    __shared__ int32_t sums[1024];
    const uint32_t per = (d + blockDim.x - 1) / blockDim.x;
    const uint32_t o0 = min(d, threadIdx.x * per), o1 = min(d, o0 + per);
    int32_t mine = 0;
    for (uint32_t o = o0; o < o1; ++o) {
        int32_t total = 0;
        for (uint32_t c = 0; c < chunks; ++c) total += counts[static_cast<size_t>(c) * d + o];
        out_offsets[o + 1] = total;  // per-output total, replaced below by the prefix
        mine += total;
    }
    sums[threadIdx.x] = mine;
    __syncthreads();
    if (threadIdx.x == 0) {
        int32_t running = 0;
        for (uint32_t k = 0; k < blockDim.x; ++k) {
            const int32_t value = sums[k];
            sums[k] = running;
            running += value;
        }
        out_offsets[0] = 0;
    }
    __syncthreads();
    int32_t start = sums[threadIdx.x];
    for (uint32_t o = o0; o < o1; ++o) {
        const int32_t total = out_offsets[o + 1];
        int32_t run = start;
        for (uint32_t c = 0; c < chunks; ++c) {
            int32_t* cell = counts + static_cast<size_t>(c) * d + o;
            const int32_t count = *cell;
            *cell = run;
            run += count;
        }
        start += total;
        out_offsets[o + 1] = start;
    }
}

// Hidden neuron owning slot s: the last r with offsets[r] <= s (zero-degree neurons skipped).
__device__ __forceinline__ uint32_t owner(const int32_t* __restrict__ offsets, uint32_t h, int32_t s) {
    uint32_t lo = 0, hi = h;  // offsets[lo] <= s < offsets[hi]
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) / 2;
        if (offsets[mid] <= s) lo = mid; else hi = mid;
    }
    return lo;
}

template <typename V>
__global__ __launch_bounds__(64) void place_kernel(const int32_t* __restrict__ down_offsets, const int16_t* __restrict__ idx,
                                                   const V* __restrict__ val, uint32_t h, uint32_t nnz, uint32_t d,
                                                   uint32_t chunk, const int32_t* __restrict__ runs,
                                                   int16_t* __restrict__ out_hidden, V* __restrict__ out_val) {
    extern __shared__ int32_t cursor[];
    for (uint32_t o = threadIdx.x; o < d; o += kWave) cursor[o] = runs[static_cast<size_t>(blockIdx.x) * d + o];
    __syncthreads();
    const uint32_t lane = threadIdx.x;
    const uint32_t s0 = blockIdx.x * chunk;
    const uint32_t s1 = min(nnz, s0 + chunk);
    for (uint32_t base = s0; base < s1; base += kWave) {
        const uint32_t s = base + lane;
        const bool valid = s < s1;
        const int32_t o = valid ? static_cast<int32_t>(static_cast<uint16_t>(idx[s])) : -1;
        int32_t rank = 0;
        bool last = true;
        for (int j = 0; j < kWave; ++j) {
            const int32_t other = __builtin_amdgcn_readlane(o, j);
            if (other == o) {
                if (j < static_cast<int>(lane)) ++rank;
                if (j > static_cast<int>(lane)) last = false;
            }
        }
        int32_t position = 0;
        if (valid) position = cursor[o] + rank;
        __syncthreads();
        if (valid) {
            out_hidden[position] = static_cast<int16_t>(owner(down_offsets, h, static_cast<int32_t>(s)));
            out_val[position] = val[s];
            if (last) cursor[o] = position + 1;
        }
        __syncthreads();
    }
}

uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

uint32_t chunk_size(uint32_t nnz) { return max(kMinChunk, ceil_div(nnz, kMaxChunks)); }

}  // namespace

uint32_t output_major_chunks(uint32_t nnz) { return max(1u, ceil_div(nnz, chunk_size(nnz))); }

hipError_t launch_output_major(int vt, const int32_t* down_offsets, const int16_t* down_idx, const void* down_val,
                               uint32_t d, uint32_t h, uint32_t nnz, int32_t* out_offsets, int16_t* out_hidden,
                               void* out_val, int32_t* counts, hipStream_t stream) {
    const uint32_t chunk = chunk_size(nnz);
    const uint32_t chunks = output_major_chunks(nnz);
    const size_t lds = static_cast<size_t>(d) * sizeof(int32_t);
    hipLaunchKernelGGL(count_kernel, dim3(chunks), dim3(256), lds, stream, down_idx, nnz, d, chunk, counts);
    hipError_t status = hipGetLastError();
    if (status != hipSuccess) return status;
    hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(1024), 0, stream, counts, chunks, d, out_offsets);
    status = hipGetLastError();
    if (status != hipSuccess || nnz == 0) return status;
    if (vt == kBF16) {
        hipLaunchKernelGGL((place_kernel<uint16_t>), dim3(chunks), dim3(kWave), lds, stream, down_offsets, down_idx,
                           static_cast<const uint16_t*>(down_val), h, nnz, d, chunk, counts, out_hidden,
                           static_cast<uint16_t*>(out_val));
    } else {
        hipLaunchKernelGGL((place_kernel<float>), dim3(chunks), dim3(kWave), lds, stream, down_offsets, down_idx,
                           static_cast<const float*>(down_val), h, nnz, d, chunk, counts, out_hidden,
                           static_cast<float*>(out_val));
    }
    return hipGetLastError();
}

}  // namespace hffn
