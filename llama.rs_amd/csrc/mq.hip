// mq.hip — fused dequantize x matvec on the gfx950 matrix cores.
//
// Replaces shaders/q{8_0,4_k,5_k,6_k}_matvec.comp of llama.rs (dispatched by
// matmul.rs:36-430 and build_plan resident_forward.rs:3678-3752).  The
// reference quantizes the activation to int8 (one f32 scale per 32) and uses
// dot4 instructions; here the activation is kept to 22 significant bits per
// 32-element block (the pack of mq_args.h: three exact int8 digits), the
// integer products run on v_mfma_i32_16x16x64_i8 with exact i32 sums per
// quant sub-block, and only the per-sub-block scale arithmetic is f32.  The
// result matches dequant + f32 dot (ops.rs:78-101) to ~1e-6 relative.
//
// Work decomposition (wave64).  Weights are in the tiled layout of tiled.h:
// one contiguous chunk per (16-row tile, unit), lane n + 16 g reading piece
// (g, n).  One MFMA multiplies the 16 rows of a tile (B operand, column n =
// row n) by 16 "slots" of the activation (A operand, row m = slot): slot m
// carries one digit of the activation restricted to one quant sub-block, so
// output register i of lane (n, G) is the exact integer sum over sub-block
// c(G) of quant * digit i.  The lane then applies d * scale (and the min /
// offset term with the f32 block sums) in f32.
//
// Per type and unit (one K-quant super-block, or 64 Q8_0 elements):
//   Q4_K / Q5_K  2 halves x 2 MFMAs (low nibbles, high nibbles); within a
//                half lane group g holds qs bytes 16g..16g+15 = elements
//                16(g&1).. of sub-blocks 2(g>>1) (low) and 2(g>>1)+1 (high)
//   Q6_K         4 MFMAs (one per 32-element quarter of each half); lane group
//                g = (half g>>1, is g&1) holds the 16-element run of each quarter
//   Q8_0         1 MFMA; lane group g holds bytes 16(g&1).. of block g>>1
//
// A workgroup is TG tile groups x KS K-slices of wavefronts.  A tile group is
// TPW tiles that share the activation (two consecutive tiles, or the gate
// and up tiles of the same outputs).  The input pack is copied to LDS once
// per workgroup (global_load_lds, no VGPR staging) while the first units of
// every wavefront are already in flight; each wavefront streams its K-slice
// with P units of loads in flight, then the K-slices are summed through LDS
// and an epilogue writes the outputs (store, q/k/v with bias + RoPE + f16 KV
// append, residual add, SwiGLU) and, for the residual and SwiGLU epilogues,
// the pack of the next op's input.  The plain matvec (k_mqx) instead packs
// its f32 input inside each workgroup and runs up to NC input columns over
// every weight load (each column bit-identical to a one-column call).
#include "attn_dev.h"
#include "attn_split_dev.h"
#include "dn_dev.h"
#include "lrs_internal.h"
#include "mq_args.h"
#include "pack_dev.h"

#include <cmath>

namespace lrs {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ float hf16(uint32_t h) {
    _Float16 v;
    const uint16_t b = (uint16_t)h;
    __builtin_memcpy(&v, &b, 2);
    return (float)v;
}
// weight bytes are read once per token: non-temporal loads
__device__ __forceinline__ uint4 ld16(const uint8_t *p) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const v4u t = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ v4i asv(uint4 u) {
    v4i r = {(int)u.x, (int)u.y, (int)u.z, (int)u.w};
    return r;
}
__device__ __forceinline__ v4i mfma8(v4i a, v4i b) {
    const v4i z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, z, 0, 0, 0);
}
// exact digit sums -> f32 (digit weights 65536, 256, 1)
__device__ __forceinline__ float cfold(v4i c) {
    return fmaf((float)c[0], 65536.f, fmaf((float)c[1], 256.f, (float)c[2]));
}

// ---------------------------------------------------------------------------
// activation pack
// ---------------------------------------------------------------------------
// x-pack of x (times nw when given) for blocks [0, nxb); elements >= n pack
// as zero (padding of the K dimension to whole units)
// xsq (optional): sum(x^2) of each 32-element block
__global__ __launch_bounds__(256) void k_xpack(const float *__restrict__ x,
                                               const float *__restrict__ nw, uint32_t n,
                                               uint32_t nxb, XPack p, float *__restrict__ xsq) {
    const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= 32 * nxb) return;  // whole half-waves leave together
    float v = 0.f, xv = 0.f;
    if (e < n) {
        xv = x[e];
        v = nw ? xv * nw[e] : xv;
    }
    pack_half(v, e >> 5, p);
    if (xsq) {
        const float sq = half_sum(xv * xv);
        if ((e & 31) == 0) xsq[e >> 5] = sq;
    }
}

hipError_t launch_xpack(const float *x, const float *nw, uint32_t n, uint32_t nxb, XPack p,
                        hipStream_t s, float *xsq) {
    const uint32_t threads = 32 * nxb;
    hipLaunchKernelGGL(k_xpack, dim3((threads + 255) / 256), dim3(256), 0, s, x, nw, n, nxb, p,
                       xsq);
    return hipGetLastError();
}

// rmsnorm_and_scale (ops.rs:56-66) of x, then the Q8_0 rounding of the
// result (p.q8 set): the input of a Q8_0 weight after an RMSNorm in
// Model::forward (weights.rs:113-117, quantize_q8_0_split).  Every workgroup
// reduces the sum of squares of the whole vector itself (n is a few thousand
// elements), then packs its 256 elements; n is a multiple of 256.
__global__ __launch_bounds__(256) void k_q8norm(const float *__restrict__ x,
                                                const float *__restrict__ w, uint32_t n,
                                                float eps, XPack p) {
    __shared__ float part[4];
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += 256) {
        const float v = x[i];
        ss += v * v;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float scale = 1.0f / sqrtf(tot / (float)n + eps);
    const uint32_t e = blockIdx.x * 256 + threadIdx.x;
    const float v = (x[e] * scale) * w[e];
    pack_half(v, e >> 5, p);
}

hipError_t launch_q8norm(const float *x, const float *w, uint32_t n, float eps, XPack p,
                         hipStream_t s) {
    if (n % 256 || !p.q8) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_q8norm, dim3(n / 256), dim3(256), 0, s, x, w, n, eps, p);
    return hipGetLastError();
}

// Q8_0 activation quantization of the reference's CPU forward for Q8_0
// weights: quantize_q8_0 (ops.rs:343-368, round half away from zero) and
// quantize_q8_0_avx2 (ops.rs:284-340, round half to even; its saturating
// packs clamp like the scalar clamp).  Per 32 elements d = max|x| / 127,
// q = round(x * (1 / d)) clamped to [-128, 127], d kept as f16; the quotients
// use the f32 d, and both divisions are IEEE (correctly rounded).  One lane
// per element, a half wavefront per block (max by DPP within rows of 16,
// then one exchange).  Writes the GGUF Q8_0 bytes (q8, n / 32 blocks) and/or
// the pack the matvec reads: digits (0, 0, q) and scale f16(d) widened, so
// the matrix-core dot of a Q8_0 weight block is the exact i32 sum(qw * qx)
// times dw * dx (the sums of the pack are unused for Q8_0 weights).
__global__ __launch_bounds__(256) void k_q8act(const float *__restrict__ x, uint32_t n,
                                               uint32_t nxb, int half_even, uint8_t *q8,
                                               XPack p) {
    const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= 32 * nxb) return;  // whole half-waves leave together
    const uint32_t b = e >> 5, i = e & 31;
    const float v = e < n ? x[e] : 0.f;
    float amax = fabsf(v);
    amax = fmaxf(amax, pk_dpp<0xB1>(amax));
    amax = fmaxf(amax, pk_dpp<0x4E>(amax));
    amax = fmaxf(amax, pk_dpp<0x141>(amax));
    amax = fmaxf(amax, pk_dpp<0x140>(amax));
    amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
    const float d = amax > 0.f ? amax / 127.0f : 0.f;
    const float di = d > 0.f ? 1.0f / d : 0.f;
    const float t = v * di;
    float r = half_even ? __builtin_rintf(t) : roundf(t);
    r = fminf(fmaxf(r, -128.f), 127.f);
    const int8_t q = (int8_t)(int)r;
    const _Float16 dh = (_Float16)d;
    if (q8 && e < n) {
        uint8_t *o = q8 + 34 * (size_t)b;
        o[2 + i] = (uint8_t)q;
        if (i == 0) {
            uint16_t hb;
            __builtin_memcpy(&hb, &dh, 2);
            o[0] = (uint8_t)(hb & 0xFF);
            o[1] = (uint8_t)(hb >> 8);
        }
    }
    if (p.dig) {
        int8_t *dg = p.dig + (size_t)b * 96 + i;
        dg[0] = 0;
        dg[32] = 0;
        dg[64] = q;
        if (i == 0)
            *reinterpret_cast<float4 *>(p.meta + 4 * (size_t)b) = make_float4((float)dh, 0.f, 0.f, 0.f);
    }
}

hipError_t launch_q8act(const float *x, uint32_t n, uint32_t nxb, int half_even, uint8_t *q8,
                        XPack p, hipStream_t s) {
    const uint32_t threads = 32 * nxb;
    hipLaunchKernelGGL(k_q8act, dim3((threads + 255) / 256), dim3(256), 0, s, x, n, nxb,
                       half_even, q8, p);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// per-type unit registers and loads (tiled layout, tiled.h)
// ---------------------------------------------------------------------------
template <uint32_t T>
struct WReg;
template <>
struct WReg<T_Q4_K> {
    uint4 hd, qa, qb;
};
template <>
struct WReg<T_Q5_K> {
    uint4 hd, qh, qa, qb;
};
template <>
struct WReg<T_Q6_K> {
    uint4 sc, la, lb, qh;
    uint32_t d;
};
template <>
struct WReg<T_Q8_0> {
    uint4 qs;
    uint32_t d;
};

// c = chunk of the unit; lane = n + 16 g
template <uint32_t T>
__device__ __forceinline__ void wload(WReg<T> &r, const uint8_t *__restrict__ c, uint32_t lane) {
    const uint32_t n = lane & 15, g = lane >> 4;
    if constexpr (T == T_Q4_K) {
        r.hd = ld16(c + 16 * n);
        r.qa = ld16(c + 256 + 16 * lane);
        r.qb = ld16(c + 1280 + 16 * lane);
    } else if constexpr (T == T_Q5_K) {
        r.hd = ld16(c + 16 * n);
        r.qh = ld16(c + 256 + 16 * (16 * (g & 1) + n));
        r.qa = ld16(c + 768 + 16 * lane);
        r.qb = ld16(c + 1792 + 16 * lane);
    } else if constexpr (T == T_Q6_K) {
        r.sc = ld16(c + 16 * n);
        r.la = ld16(c + 256 + 16 * lane);
        r.lb = ld16(c + 1280 + 16 * lane);
        r.qh = ld16(c + 2304 + 16 * lane);
        r.d = *reinterpret_cast<const uint16_t *>(c + 3328 + 2 * n);
    } else {
        r.qs = ld16(c + 16 * lane);
        r.d = *reinterpret_cast<const uint16_t *>(c + 1024 + 4 * n + 2 * (g >> 1));
    }
}

// LDS layout of the staged input pack: digits [nxb][96], 16 zero bytes, then
// meta [nxb] float4
struct LPack {
    uint32_t zero, meta;  // byte offsets
};

// per-lane constants of the A-operand (slot) mapping
template <uint32_t T>
struct ALane {
    uint32_t base, step;  // LDS byte offset of this lane's digits for unit 0, step per unit
    uint32_t c;           // Q4_K/Q5_K: sub-block of this lane's C slots within a half
};

template <uint32_t T>
__device__ __forceinline__ ALane<T> alane(uint32_t lane, const LPack &lp) {
    const uint32_t m = lane & 15, g = lane >> 4;
    ALane<T> a;
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        // slot m: nibble half s = m>>3, sub-block pair sigma = (m>>2)&1, digit m&3;
        // block 4h + 2 sigma + s, elements 16 (g&1) ..
        const uint32_t s = m >> 3, sg = (m >> 2) & 1, d = m & 3;
        const bool act = d < 3 && sg == (g >> 1);
        a.base = act ? (2 * sg + s) * 96 + 32 * d + 16 * (g & 1) : lp.zero;
        a.step = act ? 2 * 384 : 0;  // per super-block (2 halves of 4 blocks)
        a.c = 2 * (g & 1) + (g >> 1);
    } else if constexpr (T == T_Q6_K) {
        // slot m: run group m>>2 (= g of the weights), digit m&3;
        // block 8S + 4 (g>>1) + quarter, elements 16 (g&1) ..
        const bool act = (m >> 2) == g && (m & 3) < 3;
        a.base = act ? 4 * (g >> 1) * 96 + 32 * (m & 3) + 16 * (g & 1) : lp.zero;
        a.step = act ? 8 * 96 : 0;
        a.c = 0;
    } else {
        const bool act = (m >> 2) == g && (m & 3) < 3;
        a.base = act ? (g >> 1) * 96 + 32 * (m & 3) + 16 * (g & 1) : lp.zero;
        a.step = act ? 2 * 96 : 0;
        a.c = 0;
    }
    return a;
}

__device__ __forceinline__ v4i lds_a(const uint8_t *lds, uint32_t off) {
    return asv(*reinterpret_cast<const uint4 *>(lds + off));
}

// one unit u of TPW tiles: acc += sum d*sc*(x.q), accm += sum dmin*m*sum(x)
template <uint32_t T, int TPW>
__device__ __forceinline__ void udot(const WReg<T> (&w)[TPW], uint32_t u, const uint8_t *lds,
                                     const LPack &lp, const ALane<T> &al, uint32_t lane,
                                     float (&acc)[TPW], float (&accm)[TPW]) {
    const uint32_t g = lane >> 4;
    const uint32_t M = 0x0F0F0F0Fu;
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        const uint32_t c8 = 8 * al.c;
        float dsc[TPW][2], dmm[TPW][2];
#pragma unroll
        for (int t = 0; t < TPW; t++) {
            // 6-bit scale / min of sub-blocks c and 4 + c (dequant.rs:101-110)
            const uint4 h = w[t].hd;
            const float d = hf16(h.x & 0xFFFFu), dm = hf16(h.x >> 16);
            const uint32_t s0 = h.y >> c8, s4 = h.z >> c8, s8 = h.w >> c8;
            const uint32_t sc0 = s0 & 63u, m0 = s4 & 63u;
            const uint32_t sc1 = (s8 & 15u) | (((s0 >> 6) & 3u) << 4);
            const uint32_t m1 = ((s8 >> 4) & 15u) | (((s4 >> 6) & 3u) << 4);
            dsc[t][0] = d * (float)sc0;
            dsc[t][1] = d * (float)sc1;
            dmm[t][0] = dm * (float)m0;
            dmm[t][1] = dm * (float)m1;
        }
#pragma unroll
        for (int p = 0; p < 2; p++) {
            const uint32_t hh = 2 * u + p;  // half index in the row
            const v4i A = lds_a(lds, al.base + u * al.step + (al.step ? 384 * p : 0));
            const float2 mt =
                *reinterpret_cast<const float2 *>(lds + lp.meta + 16 * (4 * hh + al.c));
#pragma unroll
            for (int t = 0; t < TPW; t++) {
                const uint4 q = p ? w[t].qb : w[t].qa;
                uint4 lo = make_uint4(q.x & M, q.y & M, q.z & M, q.w & M);
                uint4 hi = make_uint4((q.x >> 4) & M, (q.y >> 4) & M, (q.z >> 4) & M, (q.w >> 4) & M);
                if constexpr (T == T_Q5_K) {
                    // fifth bit: bit 2j (low) / 2j+1 (high) of qh[l], j = 2p + (g>>1)
                    // (dequant.rs:157-203)
                    const uint32_t j2 = 2 * (2 * p + (g >> 1));
                    const uint4 qh = w[t].qh;
                    const uint32_t B1 = 0x01010101u;
                    lo.x |= ((qh.x >> j2) & B1) << 4;
                    lo.y |= ((qh.y >> j2) & B1) << 4;
                    lo.z |= ((qh.z >> j2) & B1) << 4;
                    lo.w |= ((qh.w >> j2) & B1) << 4;
                    hi.x |= ((qh.x >> (j2 + 1)) & B1) << 4;
                    hi.y |= ((qh.y >> (j2 + 1)) & B1) << 4;
                    hi.z |= ((qh.z >> (j2 + 1)) & B1) << 4;
                    hi.w |= ((qh.w >> (j2 + 1)) & B1) << 4;
                }
                const v4i C1 = mfma8(A, asv(lo));
                const v4i C2 = mfma8(A, asv(hi));
                const float cf = g >= 2 ? cfold(C2) : cfold(C1);
                acc[t] = fmaf(dsc[t][p], mt.x * cf, acc[t]);
                accm[t] = fmaf(dmm[t][p], mt.y, accm[t]);
            }
        }
    } else if constexpr (T == T_Q6_K) {
        // dequant.rs:205-258: q = (ql nibble | qh 2 bits << 4) - 32, run scale sc[8 half + 2 quarter + is]
        const uint32_t bsel = 8 * (g & 1);
        float dsc[TPW][4];
#pragma unroll
        for (int t = 0; t < TPW; t++) {
            const float d = hf16(w[t].d);
            const uint32_t lo = (g >> 1) ? w[t].sc.z : w[t].sc.x;
            const uint32_t hi = (g >> 1) ? w[t].sc.w : w[t].sc.y;
            dsc[t][0] = d * (float)(int)(int8_t)((lo >> bsel) & 255u);
            dsc[t][1] = d * (float)(int)(int8_t)((lo >> (bsel + 16)) & 255u);
            dsc[t][2] = d * (float)(int)(int8_t)((hi >> bsel) & 255u);
            dsc[t][3] = d * (float)(int)(int8_t)((hi >> (bsel + 16)) & 255u);
        }
        const uint32_t mq0 = lp.meta + 16 * (8 * u + 4 * (g >> 1));
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const v4i A = lds_a(lds, al.base + u * al.step + (al.step ? 96 * q : 0));
            const float4 mt = *reinterpret_cast<const float4 *>(lds + mq0 + 16 * q);
            const float rs = (g & 1) ? mt.w : mt.z;
            const float xo = fmaf(-32.f, rs, 0.f);
#pragma unroll
            for (int t = 0; t < TPW; t++) {
                const uint4 ql = (q & 1) ? w[t].lb : w[t].la;
                const uint4 qh = w[t].qh;
                const uint32_t H = 0x30303030u;
                uint4 b;
                if (q == 0) {
                    b = make_uint4((ql.x & M) | ((qh.x << 4) & H), (ql.y & M) | ((qh.y << 4) & H),
                                   (ql.z & M) | ((qh.z << 4) & H), (ql.w & M) | ((qh.w << 4) & H));
                } else if (q == 1) {
                    b = make_uint4((ql.x & M) | ((qh.x << 2) & H), (ql.y & M) | ((qh.y << 2) & H),
                                   (ql.z & M) | ((qh.z << 2) & H), (ql.w & M) | ((qh.w << 2) & H));
                } else if (q == 2) {
                    b = make_uint4(((ql.x >> 4) & M) | (qh.x & H), ((ql.y >> 4) & M) | (qh.y & H),
                                   ((ql.z >> 4) & M) | (qh.z & H), ((ql.w >> 4) & M) | (qh.w & H));
                } else {
                    b = make_uint4(((ql.x >> 4) & M) | ((qh.x >> 2) & H), ((ql.y >> 4) & M) | ((qh.y >> 2) & H),
                                   ((ql.z >> 4) & M) | ((qh.z >> 2) & H), ((ql.w >> 4) & M) | ((qh.w >> 2) & H));
                }
                const float cf = cfold(mfma8(A, asv(b)));
                acc[t] = fmaf(dsc[t][q], fmaf(mt.x, cf, xo), acc[t]);
            }
        }
    } else {
        // Q8_0 (dequant.rs:58-76): q * d, one d per 32-element block
        const v4i A = lds_a(lds, al.base + u * al.step);
        const float xs = *reinterpret_cast<const float *>(lds + lp.meta + 16 * (2 * u + (g >> 1)));
#pragma unroll
        for (int t = 0; t < TPW; t++) {
            const float cf = cfold(mfma8(A, asv(w[t].qs)));
            acc[t] = fmaf(hf16(w[t].d), xs * cf, acc[t]);
        }
    }
}

// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------
__device__ __forceinline__ float silu_mul(float g, float u) {
    // ops.rs:978-988: silu(g) = g / (1 + exp(-g)), then * up
    return (g / (1.0f + expf(-g))) * u;
}

// cache policy of a load that must see agent-scope stores made in the same
// launch by another XCD (sc1: the memory model's agent-scope load)
constexpr int CPOL_SC1 = 16;

// copies `bytes` (multiple of 16) from global memory to LDS, 16 B per lane,
// with cache policy CP
template <int CP = 0>
__device__ __forceinline__ void copy_to_lds(const uint8_t *__restrict__ g, uint8_t *lds,
                                            uint32_t bytes) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    for (uint32_t base = wave * 1024; base < bytes; base += nw * 1024) {
        const uint32_t off = base + lane * 16;
        if (off < bytes) __builtin_amdgcn_global_load_lds(g + off, (lds_void *)(lds + base), 16, 0, CP);
    }
}

// polls of a matvec workgroup waiting for its input pack (k_mq_ao) before it
// gives up (MqArgs::wait_polls 0): each is a memory round trip plus a short
// sleep (~0.5-2 us), so 40-130 ms in all, against the few microseconds the
// producers take
constexpr uint32_t MQ_WAIT_POLLS = 1u << 16;

// one wavefront waits until flags row[0..n) (n <= 64) are all non-zero (lane
// i polls flag i: one load per poll for the wavefront), then clears them
// for the next launch; after `polls` polls (0: MQ_WAIT_POLLS) it sets *werr
// to 1 and goes on
__device__ __forceinline__ void wait_flags(uint32_t *row, uint32_t n, uint32_t polls, uint32_t *werr) {
    const uint32_t lane = threadIdx.x & 63;
    uint32_t *f = row + lane;
    const bool mine = lane < n;
    const uint32_t limit = polls ? polls : MQ_WAIT_POLLS;
    uint32_t k = 0;
    for (;;) {
        const uint32_t v = mine ? __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 1u;
        if (__all(v != 0u)) break;
        if (++k >= limit) {
            if (lane == 0) __hip_atomic_store(werr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    if (mine) __hip_atomic_store(f, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// body for the segments [s_lo, s_hi) of type T (one workgroup).  NC > 1 or
// XF (MQ_STORE only): NC input columns share each weight load, their packs
// side by side in LDS; with XF the workgroup packs the f32 columns a.xf
// itself instead of copying a pack made by a previous launch.  WT: the pack
// is written by producers in the same launch; the workgroup issues its
// weight loads and the epilogue's operand loads, then waits for its flag
// (a.wflag) and stages the pack with agent-scope loads.
template <uint32_t T, int TPW, int TG, int KS, int P, int EPI, int NC = 1, bool XF = false,
          bool WT = false>
__device__ __forceinline__ void mq_body(const MqArgs &a, uint32_t si, uint8_t *lds, float *red) {
    static_assert(NC == 1 || EPI == MQ_STORE, "several columns: store epilogue only");
    constexpr int W = TG * KS;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t tg = wave / KS, ks = wave % KS;
    const MqSeg &sg = a.seg[si];
    const bool pair = sg.w2 != nullptr;
    const uint32_t units = tunits(T, a.n_in);
    const size_t tstride = (size_t)units * tchunk_bytes(T);
    // output tiles of this workgroup: TG tile groups of TPW tiles (pairs: one
    // output tile per group, its gate and up weights)
    const uint32_t otiles_wg = pair ? TG : TG * TPW;
    // MQ_RESID / MQ_SWIGLU split over K: workgroup b is slice b % xs of
    // output block b / xs (past the xfull whole blocks when those are set)
    const uint32_t xs_all = ((EPI == MQ_RESID || EPI == MQ_SWIGLU) && a.xsplit > 1) ? a.xsplit : 1u;
    const uint32_t wrel = blockIdx.x - sg.wg0;
    const bool whole = xs_all == 1 || wrel < a.xfull;
    const uint32_t XSN = whole ? 1u : xs_all;
    const uint32_t blk = whole ? wrel : a.xfull + (wrel - a.xfull) / xs_all;
    const uint32_t xsl = whole ? 0u : (wrel - a.xfull) % xs_all;
    const uint32_t tile0 = blk * otiles_wg;
    const uint32_t ntiles = ttiles(sg.rows);
    const uint8_t *wt[TPW];
#pragma unroll
    for (int t = 0; t < TPW; t++) {
        uint32_t tile = pair ? tile0 + tg : tile0 + tg * TPW + t;
        if (tile >= ntiles) tile = ntiles - 1;  // duplicate reads, results dropped
        wt[t] = (pair && t == 1 ? sg.w2 : sg.w) + (size_t)tile * tstride;
    }
    // this workgroup's units [ub, ue) (all of them without the split); the
    // input pack is staged from block ub * BPU on, so LDS offsets use u - ub
    const uint32_t ub = xsl * units / XSN, ue = (xsl + 1) * units / XSN, nu = ue - ub;
    constexpr uint32_t BPU = T == T_Q8_0 ? 2u : 8u;  // pack blocks per unit
    const uint32_t nxl = XSN > 1 ? nu * BPU : a.nxb;  // pack blocks staged
    const uint32_t u_lo = ub + ks * nu / KS, u_hi = ub + (ks + 1) * nu / KS;

    // XF: the first B input elements per thread of column 0 are loaded ahead
    // of the weight prefetch, so packing them waits for these loads only
    constexpr int B = 8;
    float xv0[B];
    constexpr uint32_t NT = 64 * W;  // threads of the workgroup
    if constexpr (XF) {
        // branch-free (index wrapped into the input, then select) so that
        // the wait before packing counts exactly these loads; wrapped, not
        // clamped: every workgroup's lanes past the input would otherwise
        // all read the input's last line
#pragma unroll
        for (int k = 0; k < B; k++) {
            const uint32_t e = threadIdx.x + k * NT;
            const float t = a.xf[e < a.n_in ? e : e % a.n_in];
            xv0[k] = e < a.n_in ? t : 0.f;
        }
    }

    // prefetch the first P units of this wavefront
    WReg<T> wr[P][TPW];
    if constexpr (XF) {
        // unconditional (a unit past this wavefront's range reads an in-range
        // unit whose registers are never consumed), for the same reason
#pragma unroll
        for (int i = 0; i < P; i++) {
            const uint32_t uu = u_lo + i < units ? u_lo + i : units - 1;
#pragma unroll
            for (int t = 0; t < TPW; t++) wload<T>(wr[i][t], wt[t] + (size_t)uu * tchunk_bytes(T), lane);
        }
    } else {
#pragma unroll
        for (int i = 0; i < P; i++)
            if (u_lo + i < u_hi) {
#pragma unroll
                for (int t = 0; t < TPW; t++) wload<T>(wr[i][t], wt[t] + (size_t)(u_lo + i) * tchunk_bytes(T), lane);
            }
    }

    // stage the input pack(s): digits of column c at c * nxb * 96, 16 zero
    // bytes, then the meta of column c at + c * nxb * 16; fused RMSNorm: sum
    // of the block sums of squares
    LPack lp;
    lp.zero = NC * nxl * 96;
    lp.meta = lp.zero + 16;
    if constexpr (XF) {
        // pack_half per 32-element block (lane i of a half wavefront =
        // element i); elements past n_in pack as zero.  B elements per
        // thread are loaded before any is packed: the LDS stores of the pack
        // would otherwise keep each load behind the previous store.
        const uint32_t ne = 32 * a.nxb;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            XPack xl;
            xl.dig = reinterpret_cast<int8_t *>(lds + c * a.nxb * 96);
            xl.meta = reinterpret_cast<float *>(lds + lp.meta + c * a.nxb * 16);
            xl.q8 = 0;
            const float *xc = a.xf + (size_t)c * a.n_in;
            uint32_t e0 = threadIdx.x;
            if (c == 0) {
                // the batch loaded ahead of the weights; every lane computes
                // (no branch for the compiler to sink those loads into), the
                // half-waves past the pack store nothing
#pragma unroll
                for (int k = 0; k < B; k++) {
                    // batches past the input store nothing: skipped whole
                    // (a branch uniform over the workgroup)
                    if (k * NT >= ne) break;
                    const uint32_t e = e0 + k * NT;
                    pack_half(xv0[k], e < ne ? e >> 5 : 0, xl, e < ne);
                }
                e0 += B * NT;
            }
            for (; e0 < ne; e0 += B * NT) {
                float v[B];
#pragma unroll
                for (int k = 0; k < B; k++) {
                    const uint32_t e = e0 + k * NT;
                    v[k] = e < a.n_in ? xc[e] : 0.f;
                }
#pragma unroll
                for (int k = 0; k < B; k++) {
                    const uint32_t e = e0 + k * NT;
                    if (e < ne) pack_half(v[k], e >> 5, xl);  // whole half-waves
                }
            }
        }
    } else if constexpr (!WT) {
        const uint32_t bb0 = XSN > 1 ? ub * BPU : 0u;
        copy_to_lds(reinterpret_cast<const uint8_t *>(a.xin.dig) + (size_t)bb0 * 96, lds, nxl * 96);
        copy_to_lds(reinterpret_cast<const uint8_t *>(a.xin.meta + 4 * (size_t)bb0), lds + lp.meta,
                    nxl * 16);
    }
    if (threadIdx.x < 4) reinterpret_cast<uint32_t *>(lds + lp.zero)[threadIdx.x] = 0u;
    // the epilogue's operands of this thread's output (thread i owns output i
    // of the workgroup): loaded here, with the weights, so that no load is
    // left for after the main loop (the position and RoPE frequency, the
    // bias, the residual and its norm weight)
    const uint32_t eo = threadIdx.x, erow = tile0 * 16 + eo;
    const bool evalid = eo < otiles_wg * 16 && erow < sg.rows;
    float e_bias = 0.f, e_x = 0.f, e_nw = 1.f, e_freq = 0.f, e_cs = 1.f, e_sn = 0.f;
    uint32_t e_pos = 0;
    if (sg.bias && evalid) e_bias = sg.bias[erow];
    if constexpr (EPI == MQ_QKV) {
        e_pos = a.step[1];
        const uint32_t dd = erow % a.head_dim;
        if (evalid && sg.kind < 2 && dd < a.rope_dim) {
            if (a.rope) {
                e_cs = a.rope[2 * (dd >> 1)];
                e_sn = a.rope[2 * (dd >> 1) + 1];
            } else {
                e_freq = a.freq[dd >> 1];
            }
        }
    }
    if constexpr (EPI == MQ_RESID) {
        if (evalid) {
            e_x = a.x[erow];
            if (a.nw) e_nw = a.nw[erow];
        }
    }
    float ss = 0.f;
    if (a.xsq) {
        // the block sums of squares x's producer wrote (n_in / 32 of them)
        for (uint32_t b = threadIdx.x; b < a.n_in / 32; b += blockDim.x) ss += a.xsq[b];
        // the wavefront's sum now, while the weight and pack loads are in
        // flight, not in the epilogue
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    }
    // grouped RMS factor (below): the sum of squares of this thread's first
    // block's group, loaded with the weights
    const uint32_t gb0 = XSN > 1 ? ub * BPU : 0u;  // first staged block
    float gs0 = 0.f;
    if (a.gss && threadIdx.x < nxl) {
        const uint32_t g = (threadIdx.x + gb0) / a.gblk;
        for (uint32_t r = 0; r < a.gblk; r++) gs0 += a.gss[g * a.gblk + r];
    }
    if constexpr (WT) {
        // every load above is in flight; wavefront 0 waits for this
        // workgroup's n_wait producer flags (lane i polls flag i, one load
        // per poll for the wavefront; bounded), clears them for the next
        // launch, then the workgroup stages the pack with loads that see the
        // producers' stores
        if (wave == 0) wait_flags(a.wflag + 64 * (size_t)wrel, a.n_wait, a.wait_polls, a.werr);
        __syncthreads();
        copy_to_lds<CPOL_SC1>(reinterpret_cast<const uint8_t *>(a.xin.dig), lds, nxl * 96);
        copy_to_lds<CPOL_SC1>(reinterpret_cast<const uint8_t *>(a.xin.meta), lds + lp.meta, nxl * 16);
    }
    if constexpr (XF) {
        // the pack was written to LDS from registers: wait for those stores
        // only (lgkmcnt(0)), not for the weight loads in flight, so the
        // matrix-core work starts on each unit as it arrives (the compiler
        // waits for a unit's registers before their first use)
        __builtin_amdgcn_s_waitcnt(0xC07F);
    } else {
        // the pack arrives in LDS through global_load_lds, counted by vmcnt
        // behind the weight loads issued before it
        __builtin_amdgcn_s_waitcnt(0);
    }
    __syncthreads();
    if (a.gss) {
        // the producer packed each group without its RMS factor; the pack is
        // linear in the block scale and sums, so the factor scales the meta
        for (uint32_t b = threadIdx.x; b < nxl; b += blockDim.x) {
            const uint32_t g = (b + gb0) / a.gblk;
            float t = 0.f;
            if (b == threadIdx.x) {
                t = gs0;
            } else {
                for (uint32_t r = 0; r < a.gblk; r++) t += a.gss[g * a.gblk + r];
            }
            const float f = 1.0f / sqrtf(t / a.gn + a.eps);
            float4 *mb = reinterpret_cast<float4 *>(lds + lp.meta + 16 * b);
            const float4 v = *mb;
            *mb = make_float4(v.x * f, v.y * f, v.z * f, v.w * f);
        }
        __syncthreads();
    }

    // column 0 reads the pack through lp/al; each further column c the same
    // slot mapping over its own pack (the zero slot is shared).  Column 0
    // stays out of the arrays: routed through them, the one-column kernels
    // need more than 128 VGPRs and spill inside the main loop.
    const ALane<T> al = alane<T>(lane, lp);
    LPack lpc[NC];
    ALane<T> alc[NC];
#pragma unroll
    for (int c = 1; c < NC; c++) {
        lpc[c].zero = lp.zero;
        lpc[c].meta = lp.meta + c * a.nxb * 16;
        alc[c] = al;
        if (al.base != lp.zero) alc[c].base = al.base + c * a.nxb * 96;
    }
    float acc[NC][TPW], accm[NC][TPW];
#pragma unroll
    for (int c = 0; c < NC; c++)
#pragma unroll
        for (int t = 0; t < TPW; t++) acc[c][t] = accm[c][t] = 0.f;

    // XF with every unit of the wavefront already in flight (the prefetch
    // covered its range): no refills and no loop, so the wait before each
    // unit's work is for that unit's registers alone, and the first units
    // are consumed while the last are still arriving (through the loop below
    // the compiler waits for every load before the first unit)
    bool all_in_flight = false;
    if constexpr (XF) all_in_flight = u_hi - u_lo <= (uint32_t)P;
    if (all_in_flight) {
#pragma unroll
        for (int i = 0; i < P; i++)
            if (u_lo + i < u_hi) {
                udot<T, TPW>(wr[i], u_lo + i - ub, lds, lp, al, lane, acc[0], accm[0]);
#pragma unroll
                for (int c = 1; c < NC; c++)
                    udot<T, TPW>(wr[i], u_lo + i - ub, lds, lpc[c], alc[c], lane, acc[c], accm[c]);
            }
    } else {
        // steady state: every unit's successor P units ahead is in range, so the
        // loads are unconditional and each register set is refilled in place
        // right after its unit is consumed (P units stay in flight; a
        // conditional refill would make the compiler copy the sets at the loop
        // back-edge and wait for every load there)
        uint32_t u0 = u_lo;
        for (; u0 + 2 * P <= u_hi; u0 += P) {
#pragma unroll
            for (int i = 0; i < P; i++) {
                udot<T, TPW>(wr[i], u0 + i - ub, lds, lp, al, lane, acc[0], accm[0]);
#pragma unroll
                for (int c = 1; c < NC; c++)
                    udot<T, TPW>(wr[i], u0 + i - ub, lds, lpc[c], alc[c], lane, acc[c], accm[c]);
#pragma unroll
                for (int t = 0; t < TPW; t++)
                    wload<T>(wr[i][t], wt[t] + (size_t)(u0 + P + i) * tchunk_bytes(T), lane);
                // keep the refill here: the scheduler would otherwise sink every
                // refill to the end of the loop body and drain the queue first
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // tail: fewer than 2P units left, the last refills
#pragma unroll
        for (int i = 0; i < P; i++) {
            if (u0 + i < u_hi) {
                udot<T, TPW>(wr[i], u0 + i - ub, lds, lp, al, lane, acc[0], accm[0]);
#pragma unroll
                for (int c = 1; c < NC; c++)
                    udot<T, TPW>(wr[i], u0 + i - ub, lds, lpc[c], alc[c], lane, acc[c], accm[c]);
                if (u0 + P + i < u_hi) {
#pragma unroll
                    for (int t = 0; t < TPW; t++)
                        wload<T>(wr[i][t], wt[t] + (size_t)(u0 + P + i) * tchunk_bytes(T), lane);
                }
            }
        }
        u0 += P;
#pragma unroll
        for (int i = 0; i < P; i++)
            if (u0 + i < u_hi) {
                udot<T, TPW>(wr[i], u0 + i - ub, lds, lp, al, lane, acc[0], accm[0]);
#pragma unroll
                for (int c = 1; c < NC; c++)
                    udot<T, TPW>(wr[i], u0 + i - ub, lds, lpc[c], alc[c], lane, acc[c], accm[c]);
            }
    }

    // row sums: lanes n, n+16, n+32, n+48 hold sub-block classes of row n
    // red layout: [NC][W][TPW][16] partials, then [W] sums of squares
#pragma unroll
    for (int c = 0; c < NC; c++) {
        float v[TPW];
#pragma unroll
        for (int t = 0; t < TPW; t++) {
            v[t] = acc[c][t] - accm[c][t];
            v[t] += __shfl_xor(v[t], 16, 64);
            v[t] += __shfl_xor(v[t], 32, 64);
        }
        if (lane < 16) {
#pragma unroll
            for (int t = 0; t < TPW; t++) red[((c * W + wave) * TPW + t) * 16 + lane] = v[t];
        }
    }
    if (lane == 0) red[NC * W * TPW * 16 + wave] = ss;
    __syncthreads();

    // ---- epilogue: thread i owns output i of the workgroup ----
    float s = 1.0f;
    if (a.xsq) {
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < W; w++) tot += red[NC * W * TPW * 16 + w];
        // ops.rs:56-66: 1 / sqrt(mean(x^2) + eps)
        s = 1.0f / sqrtf(tot / (float)a.n_in + a.eps);
    }
    const uint32_t i = threadIdx.x;
    const uint32_t nout = otiles_wg * 16;  // outputs of the workgroup
    // threads past the outputs leave; pack epilogues keep whole half-waves
    // (one 32-element block each), the argmax keeps whole wavefronts
    constexpr bool PACK = EPI == MQ_RESID || EPI == MQ_SWIGLU;
    const uint32_t lim = PACK ? ((nout + 31) & ~31u) : EPI == MQ_STORE ? ((nout + 63) & ~63u) : nout;
    // value of output i (column c): sum of the KS K-slice partials of its
    // tile group
    auto partial = [&](uint32_t grp, uint32_t t, uint32_t n, int c = 0) {
        float r = 0.f;
#pragma unroll
        for (int k = 0; k < KS; k++) r += red[((c * W + grp * KS + k) * TPW + t) * 16 + n];
        return r;
    };
    const uint32_t row = tile0 * 16 + i;
    const bool valid = i < nout && row < sg.rows;
    const uint32_t ii = i < nout ? i : nout - 1;
    const uint32_t grp = pair ? (ii >> 4) : (ii >> 4) / TPW;
    const uint32_t tt = pair ? 0 : (ii >> 4) % TPW;
    // the K-slice sums of output i: (value) or, for SwiGLU, (gate, up)
    float ysum = 0.f, usum = 0.f;
    if constexpr (EPI == MQ_RESID || EPI == MQ_SWIGLU) {
        if constexpr (EPI == MQ_SWIGLU) {
            ysum = partial(ii >> 4, 0, ii & 15);
            usum = partial(ii >> 4, TPW - 1, ii & 15);
        } else {
            ysum = partial(grp, tt, ii & 15);
        }
        if (XSN > 1) {
            // every thread reaches both barriers; slices other than the last
            // to arrive leave after counting themselves.  Partials go out as
            // agent-scope stores (written through to memory), and the wait
            // for their completion comes before the count, so the last
            // arriver's agent-scope loads see every slice's partials.
            // Slice k of block b: [32 values] or [32 gate][32 up] floats.
            constexpr uint32_t NXV = EPI == MQ_SWIGLU ? 64u : 32u;
            float *mine = a.xpart + ((size_t)blk * XSN + xsl) * NXV;
            if (i < nout) {
                __hip_atomic_store(mine + i, ysum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if constexpr (EPI == MQ_SWIGLU)
                    __hip_atomic_store(mine + 32 + i, usum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the stores are complete
            __syncthreads();
            uint32_t *flag = reinterpret_cast<uint32_t *>(red + NC * W * TPW * 16 + W);
            if (threadIdx.x == 0) {
                const uint32_t before =
                    __hip_atomic_fetch_add(a.xcnt + blk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const uint32_t last = before == XSN - 1;
                // every slice has counted itself: ready for the next launch
                if (last) __hip_atomic_store(a.xcnt + blk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                *flag = last;
            }
            __syncthreads();
            if (*flag == 0) return;
            if (i < nout) {
                // the slices in order, whichever arrived last
                float r = 0.f, ru = 0.f;
                for (uint32_t k = 0; k < XSN; k++) {
                    const float *pk = a.xpart + ((size_t)blk * XSN + k) * NXV;
                    r += k == xsl ? ysum : __hip_atomic_load(pk + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if constexpr (EPI == MQ_SWIGLU)
                        ru += k == xsl ? usum
                                       : __hip_atomic_load(pk + 32 + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                ysum = r;
                usum = ru;
            }
        }
    }
    if (i >= lim) return;
    if constexpr (EPI == MQ_SWIGLU) {
        const float gv = s * ysum, uv = s * usum;
        const float act = valid ? silu_mul(gv, uv) : 0.f;
        pack_half(act, row >> 5, a.xout);
        return;
    }
    float y = s * (EPI == MQ_RESID ? ysum : partial(grp, tt, ii & 15));
    if (sg.bias && valid) y = y + e_bias;
    if constexpr (NC > 1) {
        // several columns: column c's outputs at out + c * ostride
        if (valid) {
            sg.out[row] = y;
#pragma unroll
            for (int c = 1; c < NC; c++) {
                float yc = s * partial(grp, tt, ii & 15, c);
                if (sg.bias) yc = yc + e_bias;
                sg.out[(size_t)c * a.ostride + row] = yc;
            }
        }
    } else if constexpr (EPI == MQ_STORE) {
        if (valid) sg.out[row] = y;
        if (a.amax) {
            unsigned long long key = valid ? amax_key(y, row) : 0ull;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                const unsigned long long k2 = __shfl_xor(key, o, 64);
                key = k2 > key ? k2 : key;
            }
            // one key per wavefront of outputs, reduced by the finish kernel
            if (lane == 0) a.amax[(size_t)blockIdx.x * ((otiles_wg * 16 + 63) / 64) + wave] = key;
        }
    } else if constexpr (EPI == MQ_QKV) {
        const uint32_t pos = e_pos;
        // adjacent-pair RoPE (ops.rs:952-975) on q and k: theta = pos * freq[d/2]
        const float yo = __shfl_xor(y, 1, 64);
        const uint32_t dd = row % a.head_dim;
        if (sg.kind < 2 && dd < a.rope_dim) {
            float sn = e_sn, cs = e_cs;
            if (!a.rope) {
                const float th = (float)pos * e_freq;
                sincosf(th, &sn, &cs);
            }
            y = (row & 1) ? yo * sn + y * cs : y * cs - yo * sn;
        }
        if (valid) {
            if (sg.kind == 0) {
                sg.out[row] = y;
            } else {
                const uint32_t hh = row / a.head_dim;
                sg.kv[((size_t)hh * a.ctx + pos) * a.head_dim + dd] = (_Float16)y;
            }
        }
    } else {  // MQ_RESID
        float xn = 0.f;
        if (valid) {
            xn = e_x + y;
            a.x[row] = xn;
        }
        const float pv = valid ? (a.nw ? xn * e_nw : xn) : 0.f;
        pack_half(pv, row >> 5, a.xout);
        if (a.xsq_out) {
            const float sq = half_sum(xn * xn);
            if ((i & 31) == 0 && valid) a.xsq_out[row >> 5] = sq;
        }
    }
}

// two workgroups of up to 8 wavefronts per CU (at most 128 VGPRs), else one
template <int W>
constexpr int mq_waves_per_eu() { return W <= 8 ? (2 * W + 3) / 4 : (W + 3) / 4; }

template <uint32_t T0, uint32_t T1, int TPW, int TG, int KS, int P, int EPI>
__global__ __launch_bounds__(64 * TG * KS)
__attribute__((amdgpu_waves_per_eu(mq_waves_per_eu<TG * KS>()))) void k_mq(MqArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float red[TG * KS * TPW * 16 + TG * KS + 1];
    uint32_t si = 0;
#pragma unroll
    for (int s = 1; s < MQ_MAX_SEG; s++)
        if ((uint32_t)s < a.n_seg && blockIdx.x >= a.seg[s].wg0) si = s;
    if (T0 == T1 || si < a.n_seg0)
        mq_body<T0, TPW, TG, KS, P, EPI>(a, si, lds, red);
    else
        mq_body<T1, TPW, TG, KS, P, EPI>(a, si, lds, red);
}

// The attention combine and the o-projection in one launch.  Workgroups
// [0, c.n_prod) merge one query head's split partials each into the o input
// pack (attn_combine_head, agent-scope stores), wait for those stores to
// complete, then raise their flag in every o workgroup's row of the flag
// matrix (a.wflag).  The o workgroups (from c.n_prod on: seg[0].wg0)
// prefetch all their weight units (P covers a wavefront's share of K), so
// the weight stream runs while the producers do; then they wait for their
// row of flags and stage the pack (mq_body, WT).  Workgroups are dispatched
// in id order, so no producer waits behind a consumer; a consumer's wait is
// bounded all the same (a.werr).
template <uint32_t T, int TPW, int TG, int KS, int P>
__global__ __launch_bounds__(64 * TG * KS)
__attribute__((amdgpu_waves_per_eu(mq_waves_per_eu<TG * KS>()))) void k_mq_ao(MqArgs a, AoArgs c) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float red[TG * KS * TPW * 16 + TG * KS + 1];
    __shared__ float wsh[64];
    if (blockIdx.x < c.n_prod) {
        attn_combine_head<true>(c.part, c.splits, c.head_dim, a.step, c.gate, c.gstride, a.xin,
                                blockIdx.x, reinterpret_cast<float *>(lds), wsh, red);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wavefront's pack stores are complete
        __syncthreads();
        if (!c.no_signal)
            for (uint32_t t = threadIdx.x; t < c.n_cons; t += blockDim.x)
                __hip_atomic_store(a.wflag + 64 * (size_t)t + blockIdx.x, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    mq_body<T, TPW, TG, KS, P, MQ_RESID, 1, false, true>(a, 0, lds, red);
}

// The attention split, the combine and the o-projection in one launch, so
// that o's weight stream runs while the splits and the combine do.
// Workgroups [0, splits * n_kv) are the splits (threads 0..ATT_THREADS-1;
// the rest leave at once): partials with agent-scope stores, then, once
// they are complete, flag sp in the rows of the group's REP query heads
// (c.sflag).  Workgroups [.., + c.n_prod) are the combine of k_mq_ao, each
// first waiting (wavefront 0, bounded) for its head's live splits and
// loading their partials with agent-scope loads; the o workgroups follow
// (mq_body, WT).  Every wait is on workgroups with lower ids, which are
// dispatched first.
template <uint32_t T, int TPW, int TG, int KS, int P, int HD, int REP, bool QP, bool DQ>
__global__ __launch_bounds__(64 * TG * KS) void k_mq_sao(MqArgs a, AoArgs c, AttnArgs s) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float red[TG * KS * TPW * 16 + TG * KS + 1];
    __shared__ float wsh[64];
    static_assert(64 * TG * KS >= ATT_THREADS, "the split role takes ATT_THREADS threads");
    const uint32_t nsw = s.splits * s.n_kv;
    if (blockIdx.x < nsw) {
        if (threadIdx.x >= ATT_THREADS) return;  // whole wavefronts
        const uint32_t sp = blockIdx.x % s.splits, kh = blockIdx.x / s.splits;
        if (!attn_split<HD, REP, QP, DQ, true>(s, sp, kh, *reinterpret_cast<AttnLds<HD, REP, QP, DQ> *>(lds)))
            return;  // no position in this split: no partial, no flag
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wavefront's partial stores are complete
        __syncthreads();
        if (!c.no_signal && threadIdx.x < REP)
            __hip_atomic_store(c.sflag + 64 * (size_t)(kh * REP + threadIdx.x) + sp, 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    if (blockIdx.x < nsw + c.n_prod) {
        const uint32_t h = blockIdx.x - nsw;
        if (threadIdx.x < 64)
            wait_flags(c.sflag + 64 * (size_t)h, attn_live_splits(a.step[1] + 1, c.splits), a.wait_polls,
                       a.werr);
        __syncthreads();
        attn_combine_head<true, CPOL_SC1>(c.part, c.splits, c.head_dim, a.step, c.gate, c.gstride, a.xin, h,
                                          reinterpret_cast<float *>(lds), wsh, red);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wavefront's pack stores are complete
        __syncthreads();
        if (!c.no_signal)
            for (uint32_t t = threadIdx.x; t < c.n_cons; t += blockDim.x)
                __hip_atomic_store(a.wflag + 64 * (size_t)t + h, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    mq_body<T, TPW, TG, KS, P, MQ_RESID, 1, false, true>(a, 0, lds, red);
}

// The delta-net projections (MQ_STORE over ssm_qkv and ssm_gate) with the
// layer's gate projections in the same launch: the workgroups past the
// matvec's (n_mq of them), one per value head, compute the head's
// {e^g, beta} with threads 0..255 exactly as the step kernel would, which
// then reads two floats instead of 40 KB of gate rows per workgroup.
template <uint32_t T0, uint32_t T1, int TPW, int TG, int KS, int P>
__global__ __launch_bounds__(64 * TG * KS)
__attribute__((amdgpu_waves_per_eu(mq_waves_per_eu<TG * KS>()))) void k_mq_gates(MqArgs a, DnGateArgs g,
                                                                                    uint32_t n_mq) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float red[TG * KS * TPW * 16 + TG * KS + 1];
    static_assert(TG * KS * 64 >= DN_GATE_THREADS && sizeof(red) >= 12 * sizeof(float), "gate role");
    if (blockIdx.x >= n_mq) {
        const uint32_t hh = blockIdx.x - n_mq;
        float(*r4)[4] = reinterpret_cast<float(*)[4]>(red);
        if (threadIdx.x < DN_GATE_THREADS)
            dn_gate_two_rounds(g.x, g.attn_norm, g.alpha + (size_t)hh * g.n_embd,
                               g.beta + (size_t)hh * g.n_embd, g.n_embd, threadIdx.x, r4);
        __syncthreads();
        if (threadIdx.x == 0) g.out[hh] = dn_gate_final(r4, g.a[hh], g.dt[hh], g.n_embd, g.eps);
        return;
    }
    uint32_t si = 0;
#pragma unroll
    for (int s = 1; s < MQ_MAX_SEG; s++)
        if ((uint32_t)s < a.n_seg && blockIdx.x >= a.seg[s].wg0) si = s;
    if (T0 == T1 || si < a.n_seg0)
        mq_body<T0, TPW, TG, KS, P, MQ_STORE>(a, si, lds, red);
    else
        mq_body<T1, TPW, TG, KS, P, MQ_STORE>(a, si, lds, red);
}

// plain matvec of NC f32 input columns (a.xf), packed by each workgroup
template <uint32_t T, int TPW, int TG, int KS, int P, int NC>
__global__ __launch_bounds__(64 * TG * KS)
__attribute__((amdgpu_waves_per_eu(mq_waves_per_eu<TG * KS>()))) void k_mqx(MqArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float red[NC * TG * KS * TPW * 16 + TG * KS + 1];
    mq_body<T, TPW, TG, KS, P, MQ_STORE, NC, true>(a, 0, lds, red);
}

// ---------------------------------------------------------------------------
// launch
// ---------------------------------------------------------------------------
using MqFn = void (*)(MqArgs);

template <uint32_t T0, uint32_t T1, int EPI>
static MqFn pick(const MqGeom &g) {
#define LRS_MQ_CASE(TPW, TG, KS, P)                                                   \
    if (g.tpw == TPW && g.tg == TG && g.ks == KS && g.p == P) return k_mq<T0, T1, TPW, TG, KS, P, EPI>;
    LRS_MQ_CASE(1, 1, 4, 2)
    LRS_MQ_CASE(1, 1, 4, 3)
    LRS_MQ_CASE(1, 2, 4, 2)
    LRS_MQ_CASE(1, 2, 2, 2)
    LRS_MQ_CASE(2, 4, 2, 2)
    LRS_MQ_CASE(2, 2, 4, 2)
    LRS_MQ_CASE(1, 2, 6, 2)
    LRS_MQ_CASE(1, 2, 6, 1)
    LRS_MQ_CASE(1, 2, 8, 1)
    LRS_MQ_CASE(1, 2, 8, 2)
    LRS_MQ_CASE(2, 2, 2, 1)
    LRS_MQ_CASE(2, 2, 2, 2)
    LRS_MQ_CASE(1, 2, 4, 1)
    LRS_MQ_CASE(1, 2, 2, 1)
    // Q8_0 units are 64 elements: deeper prefetch over more K-slices
    if constexpr (T0 == T_Q8_0 && T1 == T_Q8_0 && EPI == MQ_STORE) {
        LRS_MQ_CASE(1, 1, 16, 4)
    }
#undef LRS_MQ_CASE
    return nullptr;
}

template <int EPI>
static MqFn pick_types(uint32_t t0, uint32_t t1, const MqGeom &g) {
    if (t0 == t1) {
        switch (t0) {
        case T_Q4_K: return pick<T_Q4_K, T_Q4_K, EPI>(g);
        case T_Q5_K: return pick<T_Q5_K, T_Q5_K, EPI>(g);
        case T_Q6_K: return pick<T_Q6_K, T_Q6_K, EPI>(g);
        case T_Q8_0: return pick<T_Q8_0, T_Q8_0, EPI>(g);
        default: return nullptr;
        }
    }
    if ((EPI == MQ_QKV || EPI == MQ_STORE) && t0 == T_Q4_K && t1 == T_Q6_K)
        return pick<T_Q4_K, T_Q6_K, EPI>(g);
    return nullptr;
}

bool mq_geom_supported(const MqGeom &g) {
    return pick<T_Q4_K, T_Q4_K, MQ_STORE>(g) != nullptr;
}

using MqGatesFn = void (*)(MqArgs, DnGateArgs, uint32_t);
static MqGatesFn pick_gates(uint32_t t0, uint32_t t1, const MqGeom &g) {
    if (t0 == T_Q4_K && t1 == T_Q4_K && g.tpw == 1 && g.tg == 2 && g.ks == 4 && g.p == 2 && g.xs <= 1)
        return k_mq_gates<T_Q4_K, T_Q4_K, 1, 2, 4, 2>;
    return nullptr;
}

bool mq_gates_supported(uint32_t t0, uint32_t t1, const MqGeom &g) {
    return pick_gates(t0, t1, g) != nullptr;
}

hipError_t launch_mq(const MqArgs &in, uint32_t t0, uint32_t t1, MqGeom g, int epi, hipStream_t s,
                     uint32_t *wgs_out, uint32_t *keys_per_wg, const DnGateArgs *gates) {
    MqArgs a = in;
    if (a.n_seg == 0 || a.n_seg > MQ_MAX_SEG) return hipErrorInvalidValue;
    if (t0 == t1) a.n_seg0 = a.n_seg;
    // K split across workgroups: one segment, residual epilogue, 32-row
    // output blocks, at least one unit per K-slice of every workgroup
    const uint32_t xs = g.xs > 1 ? (uint32_t)g.xs : 1u;
    if (xs > 1) {
        // 32 outputs per workgroup: 2 tiles (residual) or 2 tile pairs (SwiGLU)
        const bool resid = epi == MQ_RESID && !a.seg[0].w2 && g.tg * g.tpw == 2;
        const bool swiglu = epi == MQ_SWIGLU && a.seg[0].w2 && g.tpw == 2 && g.tg == 2;
        if (!(resid || swiglu) || a.n_seg != 1 || !a.xpart || !a.xcnt || t0 != t1 || xs > 8 ||
            tunits(t0, a.n_in) < xs * (uint32_t)g.ks)
            return hipErrorInvalidValue;
    }
    a.xsplit = xs;
    a.xfull = xs > 1 ? (uint32_t)g.xfull : 0u;
    uint32_t wgs = 0;
    for (uint32_t i = 0; i < a.n_seg; i++) {
        const bool pair = a.seg[i].w2 != nullptr;
        const uint32_t per = pair ? (uint32_t)g.tg : (uint32_t)(g.tg * g.tpw);
        if (pair && g.tpw != 2) return hipErrorInvalidValue;
        a.seg[i].wg0 = wgs;
        const uint32_t blocks = (ttiles(a.seg[i].rows) + per - 1) / per;
        if (a.xfull >= blocks) return hipErrorInvalidValue;
        wgs += a.xfull + (blocks - a.xfull) * xs;
    }
    // output packs need whole 32-row blocks per workgroup
    if (epi == MQ_RESID || epi == MQ_SWIGLU) {
        for (uint32_t i = 0; i < a.n_seg; i++) {
            const uint32_t outs = 16 * (a.seg[i].w2 ? g.tg : g.tg * g.tpw);
            if (outs % 32 || a.seg[i].rows % outs) return hipErrorInvalidValue;
        }
    }
    MqFn fn = nullptr;
    switch (epi) {
    case MQ_STORE: fn = pick_types<MQ_STORE>(t0, t1, g); break;
    case MQ_QKV: fn = pick_types<MQ_QKV>(t0, t1, g); break;
    case MQ_RESID: fn = pick_types<MQ_RESID>(t0, t1, g); break;
    case MQ_SWIGLU: fn = pick_types<MQ_SWIGLU>(t0, t1, g); break;
    default: return hipErrorInvalidValue;
    }
    if (!fn) return hipErrorNotSupported;
    // staged pack: all nxb blocks, or the largest slice's blocks
    const uint32_t units = tunits(t0, a.n_in), bpu = t0 == T_Q8_0 ? 2u : 8u;
    const size_t nxl = xs > 1 && !a.xfull ? (size_t)((units + xs - 1) / xs) * bpu : a.nxb;
    const size_t lds = nxl * 96 + 16 + nxl * 16;
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    if (wgs_out) *wgs_out = wgs;
    if (keys_per_wg) {
        const uint32_t outs = (uint32_t)(g.tg * g.tpw) * 16;
        *keys_per_wg = (outs + 63) / 64;
    }
    if (gates) {
        MqGatesFn gf = epi == MQ_STORE && !a.amax ? pick_gates(t0, t1, g) : nullptr;
        if (!gf) return hipErrorNotSupported;
        if (gates->n_embd % 4 || gates->n_embd > 4 * DN_GATE_THREADS * DN_GI || !gates->out)
            return hipErrorInvalidValue;
        hipLaunchKernelGGL(gf, dim3(wgs + gates->v_heads), dim3(64 * g.tg * g.ks), lds, s, a, *gates,
                           wgs);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(fn, dim3(wgs), dim3(64 * g.tg * g.ks), lds, s, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// attention combine + o-projection (k_mq_ao): shape (1, 2, 4, P), one 32-row
// block per matvec workgroup, P = a wavefront's share of the units (at least
// 2; at most 6 for Q4_K, 4 for Q5_K and 3 for Q6_K, whose units hold more
// registers: the largest P that compiles without spilling)
// ---------------------------------------------------------------------------
using MqAoFn = void (*)(MqArgs, AoArgs);
constexpr int AO_TG = 2, AO_KS = 4;

static int ao_units_per_wave(uint32_t t, uint32_t n_in) {
    const uint32_t w = (tunits(t, n_in) + AO_KS - 1) / AO_KS;
    return w < 2 ? 2 : (int)w;
}

template <uint32_t T>
static MqAoFn pick_ao_p(int p) {
    switch (p) {
    case 2: return k_mq_ao<T, 1, AO_TG, AO_KS, 2>;
    case 3: return k_mq_ao<T, 1, AO_TG, AO_KS, 3>;
    case 4: if constexpr (T != T_Q6_K) return k_mq_ao<T, 1, AO_TG, AO_KS, 4>; else return nullptr;
    case 5: if constexpr (T == T_Q4_K) return k_mq_ao<T, 1, AO_TG, AO_KS, 5>; else return nullptr;
    case 6: if constexpr (T == T_Q4_K) return k_mq_ao<T, 1, AO_TG, AO_KS, 6>; else return nullptr;
    default: return nullptr;
    }
}

static MqAoFn pick_ao(uint32_t t, uint32_t n_in) {
    const int p = ao_units_per_wave(t, n_in);
    switch (t) {
    case T_Q4_K: return pick_ao_p<T_Q4_K>(p);
    case T_Q5_K: return pick_ao_p<T_Q5_K>(p);
    case T_Q6_K: return pick_ao_p<T_Q6_K>(p);
    default: return nullptr;
    }
}

static size_t ao_lds(uint32_t nxb, uint32_t head_dim, uint32_t splits) {
    const size_t mq = (size_t)nxb * 96 + 16 + (size_t)nxb * 16;
    const size_t cb = (size_t)splits * (head_dim + 4) * sizeof(float);
    return mq > cb ? mq : cb;
}

bool mq_ao_supported(uint32_t t, uint32_t n_in, uint32_t rows, uint32_t head_dim, uint32_t splits,
                     uint32_t n_head) {
    return pick_ao(t, n_in) != nullptr && rows % 32 == 0 && rows > 0 && n_head >= 1 && n_head <= 64 &&
           (head_dim == 64 || head_dim == 128 || head_dim == 256) && splits >= 1 && splits <= 64 &&
           ao_lds(pack_blocks(t, n_in), head_dim, splits) <= 160 * 1024;
}

// ---------------------------------------------------------------------------
// attention split + combine + o-projection (k_mq_sao): the o weight in Q4_K,
// shape (1, 2, 4, P) as k_mq_ao; the head shapes built (HD, REP, QK-norm +
// RoPE in the split or the dense model's shared q split, P)
// ---------------------------------------------------------------------------
using MqSaoFn = void (*)(MqArgs, AoArgs, AttnArgs);
struct SaoShape {
    uint32_t hd, rep;
    bool qp, dq;
    int p;
    MqSaoFn fn;
    size_t lds;
};
#define LRS_SAO(HD, REP, QP, DQ, P)                                                                  \
    SaoShape{HD, REP, QP, DQ, P, k_mq_sao<T_Q4_K, 1, AO_TG, AO_KS, P, HD, REP, QP, DQ>,               \
             sizeof(AttnLds<HD, REP, QP, DQ>)}
static const SaoShape SAO_SHAPES[] = {
    LRS_SAO(128, 5, false, true, 5),  // 32B shape: 40 / 8 heads x 128, o 5120 wide
    LRS_SAO(256, 6, true, false, 6),  // the hybrid's gated attention: 24 / 4 x 256, o 6144 wide
    LRS_SAO(64, 2, false, true, 2),   LRS_SAO(64, 2, true, false, 2),  LRS_SAO(128, 5, false, true, 2),
    LRS_SAO(128, 8, false, true, 2),  LRS_SAO(256, 8, false, true, 2), LRS_SAO(256, 6, true, false, 2),
};
#undef LRS_SAO

static const SaoShape *pick_sao(uint32_t t, uint32_t n_in, uint32_t hd, uint32_t rep, bool qp, bool dq) {
    if (t != T_Q4_K) return nullptr;
    const int p = ao_units_per_wave(t, n_in);
    for (const SaoShape &x : SAO_SHAPES)
        if (x.hd == hd && x.rep == rep && x.qp == qp && x.dq == (dq && !qp) && x.p == p) return &x;
    return nullptr;
}

bool attn_ao_supported(uint32_t t, uint32_t n_in, uint32_t rows, uint32_t head_dim, uint32_t splits,
                       uint32_t n_head, uint32_t n_kv, bool qp, bool dq) {
    if (n_kv == 0 || n_head % n_kv || !mq_ao_supported(t, n_in, rows, head_dim, splits, n_head)) return false;
    const SaoShape *x = pick_sao(t, n_in, head_dim, n_head / n_kv, qp, dq);
    return x && (qp || dq) && x->lds <= 160 * 1024;
}

hipError_t launch_attn_ao(const float *q, const _Float16 *kc, const _Float16 *vc, uint32_t n_kv,
                          uint32_t ctx, const QkPrep *qp, bool dq, const MqArgs &in, const AoArgs &cin,
                          uint32_t t, hipStream_t s) {
    MqArgs a = in;
    AoArgs c = cin;
    const uint32_t n_head = c.n_prod;
    if (a.n_seg != 1 || a.seg[0].w2 || !a.wflag || !a.werr || !c.part || !c.sflag || a.xin.q8 ||
        n_head == 0 || a.nxb != pack_blocks(t, a.n_in) || !a.step)
        return hipErrorInvalidValue;
    if (!attn_ao_supported(t, a.n_in, a.seg[0].rows, c.head_dim, c.splits, n_head, n_kv, qp != nullptr, dq))
        return hipErrorNotSupported;
    const SaoShape *x = pick_sao(t, a.n_in, c.head_dim, n_head / n_kv, qp != nullptr, dq);
    AttnArgs at = {};
    at.q = q;
    at.kc = kc;
    at.vc = vc;
    at.part = const_cast<float *>(c.part);
    at.step = a.step;
    at.n_head = n_head;
    at.n_kv = n_kv;
    at.ctx = ctx;
    at.splits = c.splits;
    at.scale = 1.0f / sqrtf((float)c.head_dim);
    if (qp) {
        if (!qp->qg || !qp->kb || !qp->vb || !qp->q_norm || !qp->k_norm || !qp->rope || !qp->kc || !qp->vc)
            return hipErrorInvalidValue;
        at.qp = *qp;
    }
    const uint32_t nsw = c.splits * n_kv;
    a.n_seg0 = 1;
    a.xsplit = 1;
    a.xfull = 0;
    a.seg[0].wg0 = nsw + n_head;
    c.n_cons = a.seg[0].rows / 32;  // one 32-row block (two tiles) per workgroup
    a.n_wait = n_head;
    const size_t ml = ao_lds(a.nxb, c.head_dim, c.splits);
    hipLaunchKernelGGL(x->fn, dim3(nsw + n_head + c.n_cons), dim3(64 * AO_TG * AO_KS), ml > x->lds ? ml : x->lds,
                       s, a, c, at);
    return hipGetLastError();
}

hipError_t launch_mq_ao(const MqArgs &in, const AoArgs &cin, uint32_t t, hipStream_t s) {
    MqArgs a = in;
    AoArgs c = cin;
    if (a.n_seg != 1 || a.seg[0].w2 || !a.wflag || !a.werr || !c.part || a.xin.q8 ||
        c.n_prod == 0 || a.nxb != pack_blocks(t, a.n_in))
        return hipErrorInvalidValue;
    if (!mq_ao_supported(t, a.n_in, a.seg[0].rows, c.head_dim, c.splits, c.n_prod))
        return hipErrorNotSupported;
    MqAoFn fn = pick_ao(t, a.n_in);
    a.n_seg0 = 1;
    a.xsplit = 1;
    a.xfull = 0;
    a.seg[0].wg0 = c.n_prod;
    c.n_cons = a.seg[0].rows / 32;  // one 32-row block (two tiles) per workgroup
    a.n_wait = c.n_prod;
    hipLaunchKernelGGL(fn, dim3(c.n_prod + c.n_cons), dim3(64 * AO_TG * AO_KS),
                       ao_lds(a.nxb, c.head_dim, c.splits), s, a, c);
    return hipGetLastError();
}

}  // namespace lrs

namespace lrs {

// reduces per-wavefront argmax keys into the next step {token, pos + 1, n}
__global__ __launch_bounds__(1024) void k_argmax_finish(const unsigned long long *__restrict__ keys,
                                                        uint32_t n, uint32_t *__restrict__ step,
                                                        uint32_t *__restrict__ out,
                                                        uint32_t out_cap) {
    __shared__ unsigned long long kb[16];
    unsigned long long best = 0ull;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) best = keys[i] > best ? keys[i] : best;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const unsigned long long k = __shfl_xor(best, o, 64);
        best = k > best ? k : best;
    }
    if ((threadIdx.x & 63) == 0) kb[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < blockDim.x / 64; w++) best = kb[w] > best ? kb[w] : best;
        // no key (every logit NaN): index 0, like a first-max scan that never moves
        const uint32_t idx = best ? 0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull) : 0u;
        const uint32_t k = step[2];
        if (out && k < out_cap) out[k] = idx;
        step[0] = idx;
        step[1] = step[1] + 1;
        step[2] = k + 1;
    }
}

hipError_t launch_argmax_finish(const unsigned long long *keys, uint32_t n, uint32_t *step,
                                uint32_t *out, uint32_t out_cap, hipStream_t s) {
    hipLaunchKernelGGL(k_argmax_finish, dim3(1), dim3(1024), 0, s, keys, n, step, out, out_cap);
    return hipGetLastError();
}

static MqGeom g_store_override = {0, 0, 0, 0};

int set_matvec_geom(int tpw, int tg, int ks) {
    if (tpw == 0 && tg == 0 && ks == 0) {
        g_store_override = {0, 0, 0, 0};
        return 0;
    }
    const MqGeom g = {tpw, tg, ks, 2};
    if (!mq_geom_supported(g)) return -1;
    g_store_override = g;
    return 0;
}

// launch shape of a plain matvec (and the output head): enough wavefronts
// to cover 256 CUs, K split inside the workgroup when rows are few
MqGeom store_geom(uint32_t t, uint32_t n_in, uint32_t n_out) {
    (void)n_in;
    if (g_store_override.tpw) return g_store_override;
    // Q8_0 (config 1, 4096 x 4096): one tile x 16 K-slices with 4 of its
    // 64-element units in flight per wavefront (every unit of a wavefront in
    // one round of loads): 7.0 us per in-launch-packed matvec against 7.6 at
    // 8 K-slices x 6 units and 9.3 at the K-quant shape
    if (t == T_Q8_0) return {1, 1, 16, 4};
    const uint32_t tiles = ttiles(n_out);
    if (tiles >= 1024) return {1, 2, 2, 2};
    if (tiles >= 256) return {1, 2, 4, 2};
    return {1, 1, 4, 2};
}

// matmul_q8_0_actq (ops.rs:728-886): each column's activation rounded to
// Q8_0 (k_q8act), then the matrix-core matvec over that pack
hipError_t launch_matvec_actq(WeightView w, const float *x, float *y, uint32_t cols, void *pack,
                              int half_even, hipStream_t s) {
    if (w.type != T_Q8_0) return hipErrorInvalidValue;
    const uint32_t nxb = pack_blocks(w.type, w.n_in);
    const XPack xp = xpack_at(pack, nxb);
    for (uint32_t c = 0; c < cols; c++) {
        hipError_t e = launch_q8act(x + (size_t)c * w.n_in, w.n_in, nxb, half_even, nullptr, xp, s);
        if (e != hipSuccess) return e;
        MqArgs a = {};
        a.n_seg = 1;
        a.seg[0].w = w.q;
        a.seg[0].rows = w.n_out;
        a.seg[0].out = y + (size_t)c * w.n_out;
        a.n_in = w.n_in;
        a.nxb = nxb;
        a.xin = xp;
        e = launch_mq(a, w.type, w.type, store_geom(w.type, w.n_in, w.n_out), MQ_STORE, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// ---- plain matvec of f32 columns packed in the kernel (k_mqx) ----
template <uint32_t T, int TPW, int TG, int KS, int P>
static MqFn pick_nc(int nc) {
    switch (nc) {
    case 1: return k_mqx<T, TPW, TG, KS, P, 1>;
    case 2: return k_mqx<T, TPW, TG, KS, P, 2>;
    case 4: return k_mqx<T, TPW, TG, KS, P, 4>;
    case 8:
        if constexpr (T == T_Q8_0) return k_mqx<T, TPW, TG, KS, P, 8>;
        return nullptr;
    default: return nullptr;
    }
}

// the launch shapes store_geom picks (without a tuning override)
template <uint32_t T>
static MqFn pick_x_geom(const MqGeom &g, int nc) {
    if constexpr (T == T_Q8_0) {
        if (g.tpw == 1 && g.tg == 1 && g.ks == 16 && g.p == 4) return pick_nc<T, 1, 1, 16, 4>(nc);
    } else {
        if (g.tpw == 1 && g.tg == 2 && g.ks == 2 && g.p == 2) return pick_nc<T, 1, 2, 2, 2>(nc);
        if (g.tpw == 1 && g.tg == 2 && g.ks == 4 && g.p == 2) return pick_nc<T, 1, 2, 4, 2>(nc);
        if (g.tpw == 1 && g.tg == 1 && g.ks == 4 && g.p == 2) return pick_nc<T, 1, 1, 4, 2>(nc);
    }
    return nullptr;
}

static MqFn pick_x(uint32_t t, const MqGeom &g, int nc) {
    switch (t) {
    case T_Q4_K: return pick_x_geom<T_Q4_K>(g, nc);
    case T_Q5_K: return pick_x_geom<T_Q5_K>(g, nc);
    case T_Q6_K: return pick_x_geom<T_Q6_K>(g, nc);
    case T_Q8_0: return pick_x_geom<T_Q8_0>(g, nc);
    default: return nullptr;
    }
}

// LDS bytes of k_mqx with nc columns of nxb pack blocks each; launches keep
// 8 KB of the 160 KB for the kernel's static partial-sum array
static size_t mqx_lds(uint32_t nxb, int nc) { return (size_t)nc * nxb * 112 + 16; }
static constexpr size_t MQX_LDS_MAX = 152 * 1024;

// In-kernel packing costs every workgroup the pack of the whole input; it
// pays for Q8_0 (its short units leave the prologue exposed either way), for
// several columns (each weight load serves up to 8) and for inputs whose pack
// is one batch of 8 elements per thread, loaded ahead of the weights.  Wider
// single K-quant columns take the staged form (a pack launch, then the matvec
// copying that pack to LDS), which measures faster there.
bool matvec_packs_in_kernel(WeightView w, uint32_t cols) {
    if (!is_tiled(w.type)) return false;
    const MqGeom g = store_geom(w.type, w.n_in, w.n_out);
    const uint32_t nxb = pack_blocks(w.type, w.n_in);
    if (!pick_x(w.type, g, 1) || mqx_lds(nxb, 1) > MQX_LDS_MAX) return false;
    return w.type == T_Q8_0 || cols > 1 || 32 * nxb <= 8 * 64 * (uint32_t)(g.tg * g.ks);
}

hipError_t launch_matvec(WeightView w, const float *x, float *y, uint32_t cols, void *pack,
                         hipStream_t s) {
    if (!is_tiled(w.type)) return hipErrorInvalidValue;
    const uint32_t nxb = pack_blocks(w.type, w.n_in);
    const MqGeom g = store_geom(w.type, w.n_in, w.n_out);
    if (matvec_packs_in_kernel(w, cols)) {
        // up to 8 columns per launch share every weight load; each column's
        // arithmetic is the single-column kernel's (same K-slices, same
        // order), so the results do not depend on the grouping
        // K-quants: at most 4 columns (8 need more than 128 VGPRs, fewer waves)
        const int nc_max = w.type == T_Q8_0 ? 8 : 4;
        for (uint32_t c0 = 0; c0 < cols;) {
            int nc = nc_max;
            while (nc > 1 && ((uint32_t)nc > cols - c0 || mqx_lds(nxb, nc) > MQX_LDS_MAX)) nc >>= 1;
            MqArgs a = {};
            a.n_seg = a.n_seg0 = 1;
            a.seg[0].w = w.q;
            a.seg[0].rows = w.n_out;
            a.seg[0].out = y + (size_t)c0 * w.n_out;
            a.seg[0].wg0 = 0;
            a.n_in = w.n_in;
            a.nxb = nxb;
            a.xf = x + (size_t)c0 * w.n_in;
            a.ostride = w.n_out;
            const uint32_t per = (uint32_t)(g.tg * g.tpw);
            const uint32_t wgs = (ttiles(w.n_out) + per - 1) / per;
            hipLaunchKernelGGL(pick_x(w.type, g, nc), dim3(wgs), dim3(64 * g.tg * g.ks),
                               mqx_lds(nxb, nc), s, a);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
            c0 += (uint32_t)nc;
        }
        return hipSuccess;
    }
    if (!pack) return hipErrorInvalidValue;
    return launch_matvec_staged(w, x, y, cols, pack, s);
}

// the two-launch form: pack each column into `pack`, then the matvec over it
hipError_t launch_matvec_staged(WeightView w, const float *x, float *y, uint32_t cols, void *pack,
                                hipStream_t s) {
    if (!is_tiled(w.type)) return hipErrorInvalidValue;
    const uint32_t nxb = pack_blocks(w.type, w.n_in);
    const XPack xp = xpack_at(pack, nxb);
    for (uint32_t c = 0; c < cols; c++) {
        hipError_t e = launch_xpack(x + (size_t)c * w.n_in, nullptr, w.n_in, nxb, xp, s);
        if (e != hipSuccess) return e;
        MqArgs a = {};
        a.n_seg = 1;
        a.seg[0].w = w.q;
        a.seg[0].rows = w.n_out;
        a.seg[0].out = y + (size_t)c * w.n_out;
        a.n_in = w.n_in;
        a.nxb = nxb;
        a.xin = xp;
        e = launch_mq(a, w.type, w.type, store_geom(w.type, w.n_in, w.n_out), MQ_STORE, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace lrs
