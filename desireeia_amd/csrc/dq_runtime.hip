// dq_runtime.hip - library version, device query, and two probes the
// benchmark uses: the streaming read that measures the device's read ceiling
// at a GEMV's size (a read of N bytes with no arithmetic: what a
// bandwidth-bound kernel of that size can at best approach on this device),
// and the LDS read probe whose bank-conflict counts show which lanes a
// 16-byte LDS read serves together (the fragment swizzles depend on it).
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

constexpr int PROBE_LDS = 65536;  // bytes of LDS the probe reads

// One wave per workgroup: lane l reads 16 bytes at LDS byte offset
// offs[l] + it * stride (wrapped into the 64 KiB buffer, 16-byte aligned) for
// it = 0 .. iters - 1, one ds_read_b128 per iteration; the loaded words are
// folded and stored only if they equal `never`. With stride 0 every
// iteration repeats the same access pattern (the stride, a kernel argument,
// keeps the compiler from hoisting the read out of the loop).
__global__ __launch_bounds__(64) void lds_read_probe_kernel(const int32_t* __restrict__ offs, int iters, int stride,
                                                            uint32_t* __restrict__ sink, uint32_t never) {
    __shared__ __align__(16) uint8_t buf[PROBE_LDS];
    for (int i = threadIdx.x; i < PROBE_LDS / 4; i += 64) reinterpret_cast<uint32_t*>(buf)[i] = i * 2654435761u;
    __syncthreads();
    const int off = offs[threadIdx.x];
    uint4 acc = {0u, 0u, 0u, 0u};
    for (int it = 0; it < iters; ++it) {
        const uint4 v = *reinterpret_cast<const uint4*>(buf + ((off + it * stride) & (PROBE_LDS - 16)));
        acc.x ^= v.x, acc.y += v.y, acc.z ^= v.z, acc.w += v.w;
    }
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == never) sink[0] = acc.x;
}

}  // namespace

extern "C" int dq_lds_read_probe(const int32_t* d_offsets, uint32_t iters, uint32_t n_wg, int32_t stride,
                                 uint32_t* d_sink, uint32_t never, void* stream) {
    if (!d_offsets || !d_sink || n_wg == 0 || n_wg > 65535 || iters > (1u << 20)) return DQ_ERR_INVALID_ARG;
    lds_read_probe_kernel<<<n_wg, 64, 0, (hipStream_t)stream>>>(d_offsets, (int)iters, stride, d_sink, never);
    return dq_launch_status();
}

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
