// LDS read-bandwidth probe: a measurement kernel for the benchmark's
// roofline, built into its own library (libramnet_lds_probe.so). It is not
// part of the operator ABI and no operator calls it.
//
// Every thread streams 16-byte reads from a 32 KiB LDS table, consecutive
// lanes on consecutive 16-byte words, so a wave's ds_read_b128 touches every
// bank equally (no bank conflicts): the rate it reaches is the CU's LDS read
// peak, the ceiling of the segment scan's slot-row traffic.
#include <hip/hip_runtime.h>

#include <stdint.h>

namespace {

constexpr int kThreads = 256;
constexpr int kWords = 2048;  // uint4 words: 32 KiB of LDS per workgroup

__global__ __launch_bounds__(kThreads) void lds_read_probe_kernel(uint32_t *sink, int iters) {
    __shared__ uint4 table[kWords];
    const int t = static_cast<int>(threadIdx.x);
    for (int i = t; i < kWords; i += kThreads)
        table[i] = make_uint4(i, i * 3u + 1u, i * 5u + 2u, i * 7u + 3u);
    __syncthreads();
    uint4 acc = make_uint4(0u, 0u, 0u, 0u);
    // rotating the start by blockIdx keeps the sum data-dependent
    int idx = (t + static_cast<int>(blockIdx.x)) & (kWords - 1);
#pragma unroll 8
    for (int it = 0; it < iters; ++it) {
        const uint4 v = table[idx];
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
        idx = (idx + kThreads) & (kWords - 1);
    }
    // the sum is never this value; the store keeps the loads alive
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u)
        sink[blockIdx.x * kThreads + t] = acc.x;
}

}  // namespace

extern "C" {

// Bytes one launch reads from LDS: blocks * 256 threads * 16 B * iters.
int64_t ramnet_lds_probe_bytes(int blocks, int iters) {
    return static_cast<int64_t>(blocks) * kThreads * 16 * iters;
}

// Launches the probe on `stream` (sink: blocks * 256 uint32, never written in
// practice). Returns 0, or a nonzero hipError_t.
int ramnet_lds_probe(int blocks, int iters, uint32_t *sink, void *stream) {
    if (blocks <= 0 || iters <= 0 || !sink)
        return static_cast<int>(hipErrorInvalidValue);
    hipLaunchKernelGGL(lds_read_probe_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), sink, iters);
    return static_cast<int>(hipGetLastError());
}

}  // extern "C"
