// kore_hbm_probe.hip - read-bandwidth reference for the benchmark (part of
// libkore_qmv_bench.so, not of the kore drop-in boundary).
//
// A plain streaming read: `grid` workgroups of 256 threads walk the buffer in
// 16-byte chunks with a grid-wide stride, four loads in flight per thread,
// and fold what they read into one word per thread (so nothing is optimised
// away).  Timed back to back with HIP events, it tells what one launch of a
// given size can stream on this device, the yardstick for the HBM-bound
// kernels (their roofline fraction is quoted against the published 8 TB/s).
// kqb_floor_probe times the launch pattern of one decode layer with nothing
// but the layer's bytes read: one launch reading them once (every load issued
// up front) and one dependent empty launch, buffers rotated like the layers.
#include <hip/hip_runtime.h>

#include <cstdint>

#define KQB_API extern "C" __attribute__((visibility("default")))

namespace {

__global__ __launch_bounds__(256) void read_kernel(const uint4 *__restrict__ p, int64_t n, uint32_t *__restrict__ out) {
    uint32_t acc = 0;
    const int64_t stride = (int64_t)gridDim.x * 256;
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    for (; i + 3 * stride < n; i += 4 * stride) {
        const uint4 a = p[i], b = p[i + stride], c = p[i + 2 * stride], d = p[i + 3 * stride];
        acc ^= a.x ^ b.y ^ c.z ^ d.w;
    }
    for (; i < n; i += stride) acc ^= p[i].x;
    out[(int64_t)blockIdx.x * 256 + threadIdx.x] = acc;
}

__global__ void empty_kernel(uint32_t *out) {
    if (threadIdx.x == 0xFFFF) out[0] = 1;
}

// One round of loads per thread: PER 16-byte chunks at a grid-wide stride, all
// requested before the first is used (the grid covers the buffer once), so a
// launch is one memory round trip plus the stream of its bytes.
template <int PER>
__global__ __launch_bounds__(256) void read_once_kernel(const uint4 *__restrict__ p, int64_t n,
                                                        uint32_t *__restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    const int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
    uint4 v[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) v[j] = p[min(i0 + j * stride, n - 1)];
    uint32_t acc = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) acc ^= v[j].x ^ v[j].w;
    if (i0 < n) out[i0] = acc;
}

}  // namespace

// reps launches reading `bytes` (a multiple of 16) starting at buf + (r % rot) * bytes
// for launch r (rot copies rotate so no launch finds the previous one's bytes in
// the caches); sink: grid * 256 words.  us_per_launch: event time / reps.
// grid = 0 times `reps` empty single-wave launches instead.
KQB_API int kqb_read_probe(const void *buf, int64_t bytes, int rot, int grid, int reps, uint32_t *sink,
                           float *us_per_launch) {
    if (!buf || !sink || !us_per_launch || reps <= 0 || rot <= 0 || bytes % 16) return -1;
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -4;
    const uint8_t *b = (const uint8_t *)buf;
    auto launch = [&](int r) {
        if (grid > 0)
            hipLaunchKernelGGL(read_kernel, dim3(grid), dim3(256), 0, 0, (const uint4 *)(b + (r % rot) * bytes),
                               bytes / 16, sink);
        else
            hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, 0, sink);
    };
    for (int r = 0; r < 4; ++r) launch(r);
    int rc = hipDeviceSynchronize() == hipSuccess ? 0 : -4;
    if (!rc) {
        (void)hipEventRecord(e0, 0);
        for (int r = 0; r < reps; ++r) launch(r);
        (void)hipEventRecord(e1, 0);
        float ms = 0;
        if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess) rc = -4;
        *us_per_launch = ms * 1000.0f / reps;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc;
}

// The floor of a decode layer's launch pattern: reps rounds, each one launch of
// read_once_kernel<per> over `bytes` (a multiple of 16) at buf + (r % rot) *
// bytes, followed (with_launch != 0) by one dependent single-wave launch,
// back to back on one stream, timed with HIP events: us_per_round = event
// time / reps.  sink: at least bytes / 16 words.
KQB_API int kqb_floor_probe(const void *buf, int64_t bytes, int rot, int per, int with_launch, int reps,
                            uint32_t *sink, float *us_per_round) {
    if (!buf || !sink || !us_per_round || reps <= 0 || rot <= 0 || bytes <= 0 || bytes % 16) return -1;
    if (per != 1 && per != 2 && per != 4 && per != 8) return -1;
    const int64_t n = bytes / 16;
    const int grid = (int)((n + 256LL * per - 1) / (256LL * per));
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -4;
    const uint8_t *b = (const uint8_t *)buf;
    auto launch = [&](int r) {
        const uint4 *src = (const uint4 *)(b + (r % rot) * bytes);
        switch (per) {
            case 1: hipLaunchKernelGGL(read_once_kernel<1>, dim3(grid), dim3(256), 0, 0, src, n, sink); break;
            case 2: hipLaunchKernelGGL(read_once_kernel<2>, dim3(grid), dim3(256), 0, 0, src, n, sink); break;
            case 4: hipLaunchKernelGGL(read_once_kernel<4>, dim3(grid), dim3(256), 0, 0, src, n, sink); break;
            default: hipLaunchKernelGGL(read_once_kernel<8>, dim3(grid), dim3(256), 0, 0, src, n, sink); break;
        }
        if (with_launch) hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, 0, sink);
    };
    for (int r = 0; r < 2 * rot; ++r) launch(r);
    int rc = hipDeviceSynchronize() == hipSuccess ? 0 : -4;
    if (!rc) {
        (void)hipEventRecord(e0, 0);
        for (int r = 0; r < reps; ++r) launch(r);
        (void)hipEventRecord(e1, 0);
        float ms = 0;
        if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess) rc = -4;
        *us_per_round = ms * 1000.0f / reps;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc;
}
