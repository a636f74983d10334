// Device helpers shared by the kernels that write activation packs
// (mq_args.h) or greedy argmax keys.
#pragma once

#include "lrs_internal.h"

namespace lrs {

// DPP lane exchange within a row of 16 lanes
template <int CTRL>
__device__ __forceinline__ float pk_dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// pack stores: plain, or (AG) agent-scope stores, written through to memory,
// for a reader in the same launch on another XCD
template <bool AG>
__device__ __forceinline__ void st_dig(int8_t *p, int v) {
    if constexpr (AG)
        __hip_atomic_store(p, (int8_t)v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        *p = (int8_t)v;
}
template <bool AG>
__device__ __forceinline__ void st_meta(float *p, float a, float b, float c, float d) {
    if constexpr (AG) {
        __hip_atomic_store(p, a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(p + 1, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(p + 2, c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(p + 3, d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        *reinterpret_cast<float4 *>(p) = make_float4(a, b, c, d);
    }
}

// Packs one 32-element block held one element per lane by the 32 lanes of a
// half wavefront (lane i of the half = element i).  Writes the 3 digit bytes
// of the element and, from lane 0 of the half, the block's meta.  The max and
// the 16-element sums reduce over rows of 16 lanes with DPP (quad_perm
// [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror), then one exchange
// between the two rows of the half.
// With store false the half wavefront computes the block but writes nothing
// (a half past the end of the pack, kept in step with the rest of the wave).
// AG: agent-scope stores (st_dig / st_meta).
template <bool AG = false>
__device__ __forceinline__ void pack_half(float v, uint32_t blk, XPack p, bool store = true) {
    const uint32_t i = threadIdx.x & 31;
    float amax = fabsf(v);
    amax = fmaxf(amax, pk_dpp<0xB1>(amax));
    amax = fmaxf(amax, pk_dpp<0x4E>(amax));
    amax = fmaxf(amax, pk_dpp<0x141>(amax));
    amax = fmaxf(amax, pk_dpp<0x140>(amax));
    amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
    if (p.q8) {
        // Model::forward's input of a Q8_0 weight (weights.rs:113-117):
        // quantize_q8_0_avx2 (ops.rs:284-340), IEEE divisions, half to even
        const float d = amax > 0.f ? amax / 127.0f : 0.f;
        const float di = d > 0.f ? 1.0f / d : 0.f;
        const float r = fminf(fmaxf(__builtin_rintf(v * di), -128.f), 127.f);
        if (!store) return;
        int8_t *dg = p.dig + (size_t)blk * 96 + i;
        st_dig<AG>(dg, 0);
        st_dig<AG>(dg + 32, 0);
        st_dig<AG>(dg + 64, (int)r);
        if (i == 0) st_meta<AG>(p.meta + 4 * (size_t)blk, (float)(_Float16)d, 0.f, 0.f, 0.f);
        return;
    }
    float r16 = v;  // sum of this lane's 16-element run
    r16 += pk_dpp<0xB1>(r16);
    r16 += pk_dpp<0x4E>(r16);
    r16 += pk_dpp<0x141>(r16);
    r16 += pk_dpp<0x140>(r16);
    const float other = __shfl_xor(r16, 16, 64);
    int e;
    frexpf(amax, &e);
    if (e < -100) e = -100;  // blocks this small pack as zero
    const int X = __float2int_rn(v * ldexpf(1.0f, 21 - e));
    const int d2 = (int)(int8_t)(X & 255);
    const int X1 = (X - d2) >> 8;
    const int d1 = (int)(int8_t)(X1 & 255);
    const int d0 = (X1 - d1) >> 8;
    if (!store) return;
    int8_t *dg = p.dig + (size_t)blk * 96 + i;
    st_dig<AG>(dg, d0);
    st_dig<AG>(dg + 32, d1);
    st_dig<AG>(dg + 64, d2);
    // r16 = sum of elements 0..15, other = sum of 16..31
    if (i == 0) st_meta<AG>(p.meta + 4 * (size_t)blk, ldexpf(1.0f, e - 21), r16 + other, r16, other);
}

// Sum over the 32 lanes of a half wavefront, in every lane of the half (the
// same DPP rows of 16, then one exchange between the rows): the producers of
// the residual x store sum(x^2) per 32-element block with it, so that a
// fused RMSNorm reads n / 32 block sums instead of the n elements.
__device__ __forceinline__ float half_sum(float v) {
    v += pk_dpp<0xB1>(v);
    v += pk_dpp<0x4E>(v);
    v += pk_dpp<0x141>(v);
    v += pk_dpp<0x140>(v);
    return v + __shfl_xor(v, 16, 64);
}

// orderable 64-bit argmax key of value v at index r: the larger value wins,
// ties go to the smaller index (the first max of ops.rs:1035-1045); NaN
// never wins
__device__ __forceinline__ unsigned long long amax_key(float v, uint32_t r) {
    if (v != v) return 0ull;
    const uint32_t b = __float_as_uint(v);
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)o << 32) | (0xFFFFFFFFu - r);
}

}  // namespace lrs
