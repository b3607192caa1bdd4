// The plain-read floor of the decode measurements: a streaming read of `bytes` with nothing else in the kernel, each
// wave taking one contiguous span (64 lanes x 16 bytes per load, four loads in flight per lane), one word per wave
// written to a sink so that the loads are kept. bench.py times it on the same bytes as a decode call reads, as one
// launch per side and as one launch for both, beside the call itself. No counterpart in the reference.
#include "common.hpp"
#include "launch.hpp"

namespace hffn {
namespace {

constexpr uint32_t kProbeWaves = 4;  // per block of 256 threads

__global__ __launch_bounds__(kProbeWaves * kWave) void read_probe_kernel(const uint4* __restrict__ data, uint64_t n16,
                                                                       uint32_t* __restrict__ sink) {
    const uint64_t waves = static_cast<uint64_t>(gridDim.x) * kProbeWaves;
    const uint64_t wave = static_cast<uint64_t>(blockIdx.x) * kProbeWaves + threadIdx.x / kWave;
    const uint32_t lane = threadIdx.x % kWave;
    const uint64_t span = (n16 + waves - 1) / waves;
    const uint64_t begin = wave * span, end = min(n16, begin + span);
    uint32_t acc = 0;
    for (uint64_t i = begin + lane; i < end; i += 4 * kWave) {
        uint4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = data[min(i + u * kWave, end - 1)];  // past the span: its last element again
#pragma unroll
        for (int u = 0; u < 4; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
#pragma unroll
    for (int m = kWave / 2; m >= 1; m >>= 1) acc ^= static_cast<uint32_t>(__shfl_xor(static_cast<int>(acc), m, kWave));
    if (lane == 0) sink[wave] = acc;
}

}  // namespace

hipError_t launch_read_probe(const void* data, uint64_t bytes, uint32_t* sink, uint32_t blocks, hipStream_t stream) {
    hipLaunchKernelGGL(read_probe_kernel, dim3(blocks), dim3(kProbeWaves * kWave), 0, stream, static_cast<const uint4*>(data),
                       bytes / 16, sink);
    return hipGetLastError();
}

}  // namespace hffn
