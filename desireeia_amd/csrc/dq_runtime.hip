// dq_runtime.hip - library version, device query, and the streaming-read
// probe the benchmark uses to measure the device's read ceiling at a GEMV's
// size (a read of N bytes with no arithmetic: what a bandwidth-bound kernel
// of that size can at best approach on this device).
#include "dq_common.h"

extern "C" int dq_version(void) { return 1; }

extern "C" int dq_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

namespace {

// Wave w of the grid reads the chunks w, w + n_waves, ... of D kilobytes: D
// loads of 16 bytes per lane, all issued before any is used, each load
// instruction covering one contiguous kilobyte. The loaded words are folded
// into one value per lane, stored only if it equals a value the caller chose
// never to occur, so no load can be removed.
template <int D>
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ src, size_t n_chunks,
                                                          uint32_t* __restrict__ sink, uint32_t never) {
    const int lane = threadIdx.x & 63;
    const size_t wave = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const size_t n_waves = ((size_t)gridDim.x * blockDim.x) >> 6;
    uint32_t acc = 0;
    for (size_t c = wave; c < n_chunks; c += n_waves) {
        const uint4* p = src + c * (64 * D) + lane;
        uint4 v[D];
#pragma unroll
        for (int i = 0; i < D; ++i) v[i] = p[64 * i];
#pragma unroll
        for (int i = 0; i < D; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    }
    if (acc == never) sink[0] = acc;
}

}  // namespace

extern "C" int dq_stream_read(const void* d_src, size_t bytes, uint32_t waves_per_cu, uint32_t depth_kb,
                              uint32_t* d_sink, uint32_t never, void* stream) {
    if (!d_src || !d_sink || waves_per_cu == 0 || waves_per_cu > 32) return DQ_ERR_INVALID_ARG;
    if (waves_per_cu > 4 && waves_per_cu % 4) return DQ_ERR_NOT_SUPPORTED;  // whole 4-wave workgroups per CU
    if (depth_kb != 4 && depth_kb != 8 && depth_kb != 16) return DQ_ERR_NOT_SUPPORTED;
    const size_t chunk = (size_t)depth_kb * 1024;
    if (bytes % chunk || reinterpret_cast<uintptr_t>(d_src) % 16) return DQ_ERR_NOT_SUPPORTED;
    if (bytes == 0) return DQ_OK;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return DQ_ERR_IO;
    // waves_per_cu waves on every CU: workgroups of 4 waves, or one workgroup
    // of waves_per_cu waves per CU below 4
    const unsigned wg_waves = waves_per_cu >= 4 ? 4u : waves_per_cu;
    const unsigned grid = (unsigned)((size_t)cus * waves_per_cu / wg_waves);
    const unsigned threads = 64u * wg_waves;
    const auto* src = static_cast<const uint4*>(d_src);
    const hipStream_t st = (hipStream_t)stream;
    const size_t n = bytes / chunk;
    if (depth_kb == 4) stream_read_kernel<4><<<grid, threads, 0, st>>>(src, n, d_sink, never);
    else if (depth_kb == 8) stream_read_kernel<8><<<grid, threads, 0, st>>>(src, n, d_sink, never);
    else stream_read_kernel<16><<<grid, threads, 0, st>>>(src, n, d_sink, never);
    return dq_launch_status();
}
