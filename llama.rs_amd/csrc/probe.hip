// probe.hip — a kernel that does nothing but stream reads (lrs_read_dev):
// the read rate it reaches at a given byte count is the practical ceiling
// of the decode matvecs, which must also unpack, multiply and reduce.
#include "lrs_internal.h"

#include <algorithm>

namespace lrs {

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

// Workgroups of `threads` threads stride over the buffer together
// (consecutive workgroups read consecutive 16 * threads bytes), each thread
// with four 16-byte loads in flight.  The best workgroup count depends on the
// size (on MI355X 512 of 256 threads for >= 100 MB, 2048 for ~20 MB), so the
// caller picks it (0 = 1024; threads 0 = 256).
hipError_t launch_read(const void *src, size_t bytes, bool nontemporal, uint32_t workgroups,
                       uint32_t threads, hipStream_t s) {
    if (!threads) threads = 256;
    if (!src || bytes == 0 || bytes % 16 || workgroups > READ_MAX_WG || threads % 64 ||
        threads > 1024)
        return hipErrorInvalidValue;
    const size_t n16 = bytes / 16;
    const uint32_t grid =
        (uint32_t)std::min<size_t>(workgroups ? workgroups : 1024, (n16 + threads - 1) / threads);
    const u32x4 *p = reinterpret_cast<const u32x4 *>(src);
    if (nontemporal)
        hipLaunchKernelGGL(k_read<true>, dim3(grid), dim3(threads), 0, s, p, n16);
    else
        hipLaunchKernelGGL(k_read<false>, dim3(grid), dim3(threads), 0, s, p, n16);
    return hipGetLastError();
}

}  // namespace lrs
