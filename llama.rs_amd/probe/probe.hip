// probe.hip — liblrs_probe.so, a measurement library kept apart from the
// product (liblrs.so): a kernel that does nothing but stream reads.  The read
// rate it reaches at a given byte count is the practical ceiling of the
// decode matvecs, which must also unpack, multiply and reduce.  bench.py
// (--workload stream) is its only user.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <cstdint>

namespace {

typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;

// one word per workgroup keeps the loads live
constexpr uint32_t READ_MAX_WG = 4096;
__device__ uint32_t g_read_sink[READ_MAX_WG];

template <bool NT>
__global__ __launch_bounds__(1024) void k_read(const u32x4 *__restrict__ p, size_t n16) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    uint32_t acc = 0;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    // four independent 16-byte loads per thread in flight
    for (; i + 3 * stride < n16; i += 4 * stride) {
        u32x4 v[4];
#pragma unroll
        for (int j = 0; j < 4; j++)
            v[j] = NT ? __builtin_nontemporal_load(p + i + j * stride) : p[i + j * stride];
#pragma unroll
        for (int j = 0; j < 4; j++) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
    for (; i < n16; i += stride) {
        const u32x4 v = NT ? __builtin_nontemporal_load(p + i) : p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc ^= __shfl_xor(acc, o, 64);
    if (threadIdx.x == 0) g_read_sink[blockIdx.x] = acc;  // one wavefront's word
}

// Workgroups of `threads` threads stride over the window together
// (consecutive workgroups read consecutive 16 * threads bytes), each thread
// with four 16-byte loads in flight.
hipError_t launch_read(const void *src, size_t bytes, bool nt, uint32_t workgroups,
                       uint32_t threads, hipStream_t s) {
    const size_t n16 = bytes / 16;
    const uint32_t grid = (uint32_t)std::min<size_t>(workgroups, (n16 + threads - 1) / threads);
    const u32x4 *p = reinterpret_cast<const u32x4 *>(src);
    if (nt)
        hipLaunchKernelGGL(k_read<true>, dim3(grid), dim3(threads), 0, s, p, n16);
    else
        hipLaunchKernelGGL(k_read<false>, dim3(grid), dim3(threads), 0, s, p, n16);
    return hipGetLastError();
}

}  // namespace

extern "C" {

// Average µs of one read pass over a window of `window` bytes (a positive
// multiple of 16) of device memory on `device`.  Pass i reads window
// i % n_windows of the arena at `base` (n_windows * window bytes), so with an
// arena larger than the memory-side cache no window is cached when it is read
// again.  `workgroups` 1..4096 (0 = 1024), `threads` a multiple of 64 up to
// 1024 (0 = 256), nontemporal 0 / 1 picks plain or non-temporal loads.
// plain_first = 0: two untimed passes, then `reads` passes back to back
// between two events on a stream of the library's own.  plain_first = 1:
// each timed pass is preceded by an untimed plain read of the same window
// (the memory-side cache warm) and timed on its own.
// Returns 0, -1 for an invalid argument (nothing launched), or a hipError_t.
int lrsp_read_time(int device, const void *base, size_t window, uint32_t n_windows,
                   int nontemporal, uint32_t workgroups, uint32_t threads, uint32_t reads,
                   int plain_first, float *us) {
    if (!workgroups) workgroups = 1024;
    if (!threads) threads = 256;
    if (!base || !us || window == 0 || window % 16 || n_windows == 0 || reads == 0 ||
        workgroups > READ_MAX_WG || threads % 64 || threads > 1024)
        return -1;
    hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) return (int)e;
    hipStream_t s = nullptr;
    hipEvent_t ev[2] = {nullptr, nullptr};
    e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreate(&ev[0]);
    if (e == hipSuccess) e = hipEventCreate(&ev[1]);
    const char *b = static_cast<const char *>(base);
    const bool nt = nontemporal != 0;
    double total_ms = 0.0;
    if (e == hipSuccess && !plain_first) {
        for (uint32_t i = 0; i < 2 && e == hipSuccess; i++)
            e = launch_read(b + (size_t)(i % n_windows) * window, window, nt, workgroups, threads, s);
        if (e == hipSuccess) e = hipEventRecord(ev[0], s);
        for (uint32_t i = 0; i < reads && e == hipSuccess; i++)
            e = launch_read(b + (size_t)(i % n_windows) * window, window, nt, workgroups, threads, s);
        if (e == hipSuccess) e = hipEventRecord(ev[1], s);
        if (e == hipSuccess) e = hipEventSynchronize(ev[1]);
        float ms = 0.f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev[0], ev[1]);
        total_ms = ms;
    } else {
        for (uint32_t i = 0; i < reads && e == hipSuccess; i++) {
            const char *w = b + (size_t)(i % n_windows) * window;
            e = launch_read(w, window, false, workgroups, threads, s);
            if (e == hipSuccess) e = hipEventRecord(ev[0], s);
            if (e == hipSuccess) e = launch_read(w, window, nt, workgroups, threads, s);
            if (e == hipSuccess) e = hipEventRecord(ev[1], s);
            if (e == hipSuccess) e = hipEventSynchronize(ev[1]);
            float ms = 0.f;
            if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev[0], ev[1]);
            total_ms += ms;
        }
    }
    if (s) (void)hipStreamSynchronize(s);
    if (ev[0]) (void)hipEventDestroy(ev[0]);
    if (ev[1]) (void)hipEventDestroy(ev[1]);
    if (s) (void)hipStreamDestroy(s);
    if (e != hipSuccess) return (int)e;
    *us = (float)(total_ms * 1e3 / reads);
    return 0;
}

}  // extern "C"
