// Device helpers of the decode attention shared by the split kernel, the
// combine kernel (attention.hip) and the launch that runs the combine ahead
// of the o-projection (mq.hip).
#pragma once

#include "mq_args.h"
#include "pack_dev.h"

namespace lrs {

constexpr uint32_t ATT_BLOCK = 16;  // positions per block; split s owns blocks s, s + splits, ...

// the splits that hold positions of a context of L positions (the others
// have no work and write no partial)
__device__ __forceinline__ uint32_t attn_live_splits(uint32_t L, uint32_t splits) {
    const uint32_t b = (L + ATT_BLOCK - 1) / ATT_BLOCK;
    return b < splits ? b : splits;
}

// sum over aligned groups of N lanes (N = 8, 16, 32) in every lane: DPP
// within a row of 16 (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror,
// row_mirror), a lane shuffle across rows
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
// max over each row of 16 lanes, in every lane of the row
__device__ __forceinline__ float row_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    return fmaxf(v, dpp_f<0x140>(v));
}
// max over aligned groups of N lanes (N = 8, 16, 32) in every lane
template <int N>
__device__ __forceinline__ float group_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    if constexpr (N >= 16) v = fmaxf(v, dpp_f<0x140>(v));
    if constexpr (N >= 32) v = fmaxf(v, __shfl_xor(v, 16, 64));
    return v;
}
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    if constexpr (N >= 16) v += dpp_f<0x140>(v);  // row_mirror
    if constexpr (N >= 32) v += __shfl_xor(v, 16, 64);
    return v;
}

// Merges the split partials [splits][hd + 4] (acc[hd] relative to the split
// max, m, l) of query head h into the head's output and packs it as hd / 32
// blocks of `out` (the identity of attention_split.comp + attn_reduce.comp:
// out = sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s over the splits that
// hold positions).  The head's partial block goes to LDS in one round trip
// (global_load_lds, every thread of the workgroup loading, issued before the
// position arrives); then wave 0 forms the split weights and thread d < hd
// owns dim d.  Gated attention (gate non-null, gate_quant.comp): the output
// is multiplied by sigmoid(gate[h * gstride + d]).  AG: the pack is written
// with agent-scope stores, for a reader in the same launch.  CP: cache
// policy of the partials' loads (agent scope when the splits ran in the
// same launch).
// pl: LDS for splits * (hd + 4) floats (16-byte aligned); wsh: 64 floats;
// red: 1 float.  splits <= 64; hd a multiple of 64, at most blockDim.x.
template <bool AG, int CP = 0>
__device__ __forceinline__ void attn_combine_head(const float *__restrict__ part, uint32_t splits,
                                                  uint32_t hd, const uint32_t *__restrict__ step,
                                                  const float *__restrict__ gate, uint32_t gstride,
                                                  XPack out, uint32_t h, float *pl, float *wsh,
                                                  float *red) {
    typedef __attribute__((address_space(3))) void lds_v;
    const uint32_t ST = hd + 4;
    const uint32_t d = threadIdx.x, lane = d & 63, wave = d >> 6;
    const uint8_t *src = reinterpret_cast<const uint8_t *>(part + (size_t)h * splits * ST);
    const uint32_t bytes = splits * ST * 4;  // multiple of 16
    for (uint32_t base = wave * 1024; base < bytes; base += blockDim.x * 16) {
        const uint32_t off = base + lane * 16;
        if (off < bytes)
            __builtin_amdgcn_global_load_lds(src + off, (lds_v *)(reinterpret_cast<uint8_t *>(pl) + base), 16, 0, CP);
    }
    // the output gate of (head h, dim d), loaded with the partials
    const float gv = gate && d < hd ? gate[(size_t)h * gstride + d] : 0.f;
    // the splits that hold positions (the split kernel wrote no partial for
    // the others; what their slots hold is not used)
    splits = attn_live_splits(step[1] + 1, splits);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // wave 0: M = max over the splits, weights, denominator
    if (wave == 0) {
        const float ms = lane < splits ? pl[lane * ST + hd] : -INFINITY;
        float M = row_max(ms);  // rows of 16 by DPP, then across the rows
        M = fmaxf(M, __shfl_xor(M, 16, 64));
        M = fmaxf(M, __shfl_xor(M, 32, 64));
        const float w = ms == -INFINITY ? 0.f : expf(ms - M);  // empty splits weigh 0
        float den = group_sum<16>(lane < splits ? w * pl[lane * ST + hd + 1] : 0.f);
        den += __shfl_xor(den, 16, 64);
        den += __shfl_xor(den, 32, 64);
        if (lane < splits) wsh[lane] = w;
        if (lane == 0) red[0] = den;
    }
    __syncthreads();
    if (d < hd) {  // whole wavefronts
        const float den = red[0];
        float num = 0.f;
        for (uint32_t s = 0; s < splits; s++) num = fmaf(wsh[s], pl[s * ST + d], num);
        float o = num / den;
        if (gate) o = o * (1.0f / (1.0f + expf(-gv)));
        pack_half<AG>(o, (h * hd + d) >> 5, out);
    }
}

}  // namespace lrs
