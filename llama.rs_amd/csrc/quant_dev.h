// Device-side dequant helpers shared by quant.hip and model.hip.
// Element-exact restatement of ggml_cpu::dequant_to_f32
// (crates/ggml-cpu/src/dequant.rs:58-258): same f32 operation order, no FMA
// (explicit __fmul_rn / __fsub_rn).
#pragma once

#include "lrs_internal.h"

namespace lrs {

__device__ __forceinline__ float h2f(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}

__device__ __forceinline__ uint16_t rd16(const uint8_t *p) {
    return (uint16_t)(p[0] | ((uint16_t)p[1] << 8));
}

// K-quant 6-bit (scale, min) of sub-block j: dequant.rs:101-110
__device__ __forceinline__ void scale_min_k4(uint32_t j, const uint8_t *s, uint32_t &sc,
                                             uint32_t &m) {
    if (j < 4) {
        sc = s[j] & 63;
        m = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

// GGUF byte o of GGUF block blk of row `row` of a resident weight
__device__ __forceinline__ uint8_t gbyte(const WeightView &w, uint32_t row, uint32_t blk, uint32_t o) {
    if (is_tiled(w.type)) return w.q[toff(w.type, w.n_in, row, blk, o)];
    return w.q[((size_t)row * w.nb + blk) * (size_t)block_bytes(w.type) + o];
}

// element e (0..255) of one GGUF block of a block type (Q8_0, Q4_0, Q4_K,
// Q5_K, Q6_K) whose byte o is B(o)
template <typename BF>
__device__ __forceinline__ float deq_block_elem(uint32_t type, uint32_t e, BF B) {
    switch (type) {
    case T_Q8_0:
        // dequant.rs:58-76
        return __fmul_rn((float)(int8_t)B(2 + e), h2f((uint16_t)(B(0) | (B(1) << 8))));
    case T_Q4_K:
    case T_Q5_K: {
        // dequant.rs:112-150 / 157-203
        const bool q5 = type == T_Q5_K;
        const float dv = h2f((uint16_t)(B(0) | (B(1) << 8)));
        const float mv = h2f((uint16_t)(B(2) | (B(3) << 8)));
        const uint32_t grp = e >> 6, within = e & 63, l = within & 31, hi = within >> 5;
        const uint32_t sub = 2 * grp + hi;
        uint8_t sb[12];
        for (int k = 0; k < 12; k++) sb[k] = B(4 + k);
        uint32_t sc, m;
        scale_min_k4(sub, sb, sc, m);
        const uint8_t byte = B((q5 ? 48 : 16) + 32 * grp + l);
        uint32_t q = hi ? (byte >> 4) : (byte & 15);
        if (q5) q += ((B(16 + l) >> sub) & 1) ? 16 : 0;
        const float d1 = __fmul_rn(dv, (float)sc);
        const float m1 = __fmul_rn(mv, (float)m);
        return __fsub_rn(__fmul_rn(d1, (float)q), m1);
    }
    case T_Q6_K: {
        // dequant.rs:205-258
        const float dv = h2f((uint16_t)(B(208) | (B(209) << 8)));
        const uint32_t half = e >> 7, within = e & 127, quarter = within >> 5, l = within & 31;
        const uint8_t qlb = B(64 * half + l + 32 * (quarter & 1));
        const uint32_t lo = quarter < 2 ? (qlb & 15) : (qlb >> 4);
        const uint32_t hi2 = (B(128 + 32 * half + l) >> (2 * quarter)) & 3;
        const int q = (int)(lo | (hi2 << 4)) - 32;
        const float s = (float)(int8_t)B(192 + 8 * half + (l >> 4) + 2 * quarter);
        return __fmul_rn(__fmul_rn(dv, s), (float)q);
    }
    case T_Q4_0: {
        // dequant.rs:77-99
        const int x = e < 16 ? (int)(B(2 + e) & 15) - 8 : (int)(B(2 + e - 16) >> 4) - 8;
        return __fmul_rn((float)x, h2f((uint16_t)(B(0) | (B(1) << 8))));
    }
    default:
        return 0.0f;
    }
}

// element e (0..255) of GGUF block b (= row * nb + block in row) of a resident weight
__device__ __forceinline__ float deq_elem(const WeightView &w, uint64_t b, uint32_t e) {
    if (w.type == T_F16) return h2f(reinterpret_cast<const uint16_t *>(w.q)[b]);
    if (w.type == T_F32) return reinterpret_cast<const float *>(w.q)[b];
    const uint32_t row = (uint32_t)(b / w.nb), blk = (uint32_t)(b % w.nb);
    return deq_block_elem(w.type, e, [&](uint32_t o) { return gbyte(w, row, blk, o); });
}

}  // namespace lrs
