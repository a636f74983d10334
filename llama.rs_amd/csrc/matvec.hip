// matvec.hip — fused dequantize x matvec for GGUF Q8_0 / Q4_K / Q5_K / Q6_K
// weights with f32 activations, gfx950 (wave64).
//
// Replaces shaders/q{8_0,4_k,5_k,6_k}_matvec.comp of llama.rs
// (crates/llama-vulkan/shaders, dispatched from matmul.rs:36-430 and
// build_plan resident_forward.rs:3678-3752) with a different numerical
// contract: the activation stays f32 (the reference quantizes it to int8), so
// y matches dequant + f32 dot (ops.rs:78-101) to ~1e-7 relative.
//
// Work decomposition.  A row is cut into "units" of contiguous elements: 64
// for Q4_K / Q5_K (one 32-byte qs group = two sub-blocks), 32 for Q8_0 (one
// block), 128 for Q6_K (one half super-block: 64 B ql + 32 B qh + 8 scales).
// A wavefront owns 64/LPR row groups of R rows; the LPR lanes of a group take
// every LPR-th unit, so within a load instruction consecutive lanes read
// consecutive 128-bit pieces of a row.  Each lane prefetches the weights of
// its next unit before it computes the current one.
//
// The activation is staged per workgroup in LDS (in K-tiles of at most
// MV_TILE elements), optionally RMS-normalised on the way in (the fused
// rmsnorm_and_scale of ops.rs:56-66), together with the sum of every
// 16-element run (used by the K-quant min / offset terms).  The LDS copy is
// padded by 4 floats per unit, so the 16 lanes of a group that read 16
// consecutive units hit 16 distinct 16-byte bank groups.  Each lane converts
// nibbles with v_cvt_f32_ubyte{0..3}, keeps one partial sum per 16-element run
// and applies the run's 6-bit scale / min once per run.  Partial sums are
// reduced across the LPR lanes; an epilogue fuses bias, adjacent-pair RoPE,
// the f16 KV-cache append, SwiGLU, or the residual add into the same launch.
#include "lrs_internal.h"
#include "mv_args.h"

#include <cstdio>
#include <cstdlib>

namespace lrs {

__device__ __forceinline__ float hf(uint32_t h16) {
    _Float16 v;
    uint16_t b = (uint16_t)h16;
    __builtin_memcpy(&v, &b, 2);
    return (float)v;
}

// byte K of v as float, one v_cvt_f32_ubyteK (the compiler would otherwise
// turn a masked byte into v_bfe_u32 + v_cvt_f32_ubyte0)
template <int K>
__device__ __forceinline__ float cvtub(uint32_t v) {
    float r;
    if constexpr (K == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
    else if constexpr (K == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
    else if constexpr (K == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
    else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// acc += byte_K(m) * x, as one v_cvt_f32_ubyteK + v_fmac_f32 pair: keeping
// the pair together stops the scheduler from converting a whole unit's
// nibbles ahead of time (64 live VGPRs) and keeps occupancy up
template <int K>
__device__ __forceinline__ float fma_ub(float acc, uint32_t m, float x) {
    float t;
    if constexpr (K == 0)
        asm("v_cvt_f32_ubyte0 %1, %2\n\tv_fmac_f32 %0, %1, %3" : "+v"(acc), "=&v"(t) : "v"(m), "v"(x));
    else if constexpr (K == 1)
        asm("v_cvt_f32_ubyte1 %1, %2\n\tv_fmac_f32 %0, %1, %3" : "+v"(acc), "=&v"(t) : "v"(m), "v"(x));
    else if constexpr (K == 2)
        asm("v_cvt_f32_ubyte2 %1, %2\n\tv_fmac_f32 %0, %1, %3" : "+v"(acc), "=&v"(t) : "v"(m), "v"(x));
    else
        asm("v_cvt_f32_ubyte3 %1, %2\n\tv_fmac_f32 %0, %1, %3" : "+v"(acc), "=&v"(t) : "v"(m), "v"(x));
    return acc;
}

// acc += sum_k byte_k(m) * x[k]
__device__ __forceinline__ float dot4b(uint32_t m, float4 x, float acc) {
    acc = fma_ub<0>(acc, m, x.x);
    acc = fma_ub<1>(acc, m, x.y);
    acc = fma_ub<2>(acc, m, x.z);
    acc = fma_ub<3>(acc, m, x.w);
    return acc;
}

__device__ __forceinline__ uint4 ldq(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }
__device__ __forceinline__ uint32_t u4get(const uint4 &v, int k) {
    return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w;
}
__device__ __forceinline__ float f4get(const float4 &v, int k) {
    return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w;
}
__device__ __forceinline__ float sext8(uint32_t v, int k) {  // signed byte k as float
    return (float)((int32_t)(v << (24 - 8 * k)) >> 24);
}

template <uint32_t T>
__host__ __device__ constexpr uint32_t unit_elems() {
    return T == T_Q6_K ? 128u : T == T_Q8_0 ? 32u : 64u;
}
template <uint32_t T>
__host__ __device__ constexpr uint32_t unit_shift() {
    return T == T_Q6_K ? 7u : T == T_Q8_0 ? 5u : 6u;
}
template <uint32_t T>
__host__ __device__ constexpr uint32_t qbytes() {
    return T == T_Q8_0 ? Q8_QBYTES : T == T_Q6_K ? Q6_QBYTES : T == T_Q5_K ? 176u : 144u;
}
// padded LDS index: 4 floats of padding after every unit
template <uint32_t T>
__device__ __forceinline__ uint32_t xphys(uint32_t i) {
    return i + 4u * (i >> unit_shift<T>());
}

// ---------------------------------------------------------------------------
// raw weight registers of one unit of one row
// ---------------------------------------------------------------------------
template <uint32_t T>
struct URaw;
template <>
struct URaw<T_Q4_K> {
    uint4 hd, q0, q1;
};
template <>
struct URaw<T_Q5_K> {
    uint4 hd, q0, q1, h0, h1;
};
template <>
struct URaw<T_Q6_K> {
    uint4 l0, l1, l2, l3, h0, h1;
    uint2 sc;
    uint32_t d;
};
template <>
struct URaw<T_Q8_0> {
    uint4 q0, q1;
    uint32_t d;
};

// e = first element of the unit within the row
template <uint32_t T>
__device__ __forceinline__ void uload(URaw<T> &r, const uint8_t *__restrict__ q,
                                      const uint16_t *__restrict__ dv, size_t rowblk, uint32_t e) {
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        const size_t bi = rowblk + (e >> 8);
        const uint8_t *blk = q + bi * qbytes<T>();
        const uint32_t j = (e >> 6) & 3;
        constexpr uint32_t QS = T == T_Q5_K ? 48 : 16;
        r.hd = ldq(blk);
        r.q0 = ldq(blk + QS + 32 * j);
        r.q1 = ldq(blk + QS + 32 * j + 16);
        if constexpr (T == T_Q5_K) {
            r.h0 = ldq(blk + 16);
            r.h1 = ldq(blk + 32);
        }
    } else if constexpr (T == T_Q6_K) {
        const size_t bi = rowblk + (e >> 8);
        const uint8_t *blk = q + bi * Q6_QBYTES;
        const uint32_t hfl = (e >> 7) & 1;
        r.l0 = ldq(blk + 64 * hfl);
        r.l1 = ldq(blk + 64 * hfl + 16);
        r.l2 = ldq(blk + 64 * hfl + 32);
        r.l3 = ldq(blk + 64 * hfl + 48);
        r.h0 = ldq(blk + 128 + 32 * hfl);
        r.h1 = ldq(blk + 128 + 32 * hfl + 16);
        r.sc = *reinterpret_cast<const uint2 *>(blk + 192 + 8 * hfl);
        r.d = dv[bi];
    } else {
        const size_t bi = rowblk + (e >> 5);
        const uint8_t *blk = q + bi * Q8_QBYTES;
        r.q0 = ldq(blk);
        r.q1 = ldq(blk + 16);
        r.d = dv[bi];
    }
}

// acc += sum over a 16-float run of bytes(w0..w3) * x
__device__ __forceinline__ float run16(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                       const float4 (&x)[4], float t) {
    t = dot4b(w0, x[0], t);
    t = dot4b(w1, x[1], t);
    t = dot4b(w2, x[2], t);
    t = dot4b(w3, x[3], t);
    return t;
}

__device__ __forceinline__ void ldrun(float4 (&x)[4], const float *__restrict__ p) {
    const float4 *p4 = reinterpret_cast<const float4 *>(p);
#pragma unroll
    for (int i = 0; i < 4; i++) x[i] = p4[i];
}

// dot of one unit for R rows (run-major: one 16-float activation run is live
// at a time and serves all R rows); xu = padded LDS pointer of the unit's
// first element, su = its 16-element run sums, e = unit's first element
template <uint32_t T, int R>
__device__ __forceinline__ void udot(const URaw<T> (&w)[R], const float *__restrict__ xu,
                                     const float *__restrict__ su, uint32_t e, float (&acc)[R]) {
    const uint32_t M = 0x0F0F0F0Fu;
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        // qs group j (bytes 32j..32j+31): low nibbles = sub-block 2j (runs 0,1),
        // high nibbles = sub-block 2j+1 (runs 2,3) -- dequant.rs:112-203
        const uint32_t j = (e >> 6) & 3, sh = 16 * (j & 1);
        float tl[R], th[R];
        float4 x[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            ldrun(x, xu + 16 * q);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint4 &qq = (q & 1) ? w[r].q1 : w[r].q0;
                uint32_t b[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const uint32_t v = u4get(qq, k);
                    b[k] = (q < 2 ? v : (v >> 4)) & M;
                    if constexpr (T == T_Q5_K) {
                        // fifth bit: bit s of qh[l] (dequant.rs:157-203)
                        const uint32_t hb = u4get((q & 1) ? w[r].h1 : w[r].h0, k);
                        b[k] |= ((hb >> (2 * j + (q >> 1))) & 0x01010101u) << 4;
                    }
                }
                if (q == 0) tl[r] = run16(b[0], b[1], b[2], b[3], x, 0.f);
                else if (q == 1) tl[r] = run16(b[0], b[1], b[2], b[3], x, tl[r]);
                else if (q == 2) th[r] = run16(b[0], b[1], b[2], b[3], x, 0.f);
                else th[r] = run16(b[0], b[1], b[2], b[3], x, th[r]);
            }
            __builtin_amdgcn_sched_barrier(0);  // keep one activation run live
        }
        const float4 s4 = *reinterpret_cast<const float4 *>(su);
        const float xl = s4.x + s4.y, xh = s4.z + s4.w;
#pragma unroll
        for (int r = 0; r < R; r++) {
            // 6-bit scale/min of sub-blocks 2j, 2j+1 (dequant.rs:101-110)
            const uint32_t A = w[r].hd.y >> sh, B = w[r].hd.z >> sh, Cc = w[r].hd.w >> sh;
            const bool hiform = j >= 2;
            const uint32_t scp = hiform ? ((Cc & 0x0F0Fu) | ((A >> 2) & 0x3030u)) : (A & 0x3F3Fu);
            const uint32_t mp = hiform ? (((Cc >> 4) & 0x0F0Fu) | ((B >> 2) & 0x3030u)) : (B & 0x3F3Fu);
            const float d = hf(w[r].hd.x & 0xFFFFu), dm = hf(w[r].hd.x >> 16);
            float sv = cvtub<0>(scp) * tl[r];
            sv = fmaf(cvtub<1>(scp), th[r], sv);
            float mv = cvtub<0>(mp) * xl;
            mv = fmaf(cvtub<1>(mp), xh, mv);
            acc[r] = fmaf(d, sv, fmaf(-dm, mv, acc[r]));
        }
    } else if constexpr (T == T_Q6_K) {
        // half super-block: run k = elements 16k..16k+15, scale sc[k]
        // (dequant.rs:205-258: q1..q4 from ql low/high nibbles + qh bit pairs)
        const uint32_t M3 = 0x03030303u;
        float v[R];
#pragma unroll
        for (int r = 0; r < R; r++) v[r] = 0.f;
        float4 x[4];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            ldrun(x, xu + 16 * k);
            const float xs = su[k];
            const int qsh = 2 * (k >> 1);  // qh bit pair: 0,2,4,6
            const bool hin = k >= 4;
#pragma unroll
            for (int r = 0; r < R; r++) {
                // ql bytes: runs 0,1,4,5 -> ql[0..31]; 2,3,6,7 -> ql[32..63]
                const uint4 &ql = (k & 2) ? ((k & 1) ? w[r].l3 : w[r].l2) : ((k & 1) ? w[r].l1 : w[r].l0);
                const uint4 &qh = (k & 1) ? w[r].h1 : w[r].h0;
                uint32_t b[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t wl = u4get(ql, i), wh = u4get(qh, i);
                    b[i] = ((hin ? (wl >> 4) : wl) & M) | (((wh >> qsh) & M3) << 4);
                }
                const float t = run16(b[0], b[1], b[2], b[3], x, 0.f);
                const float sc = sext8(k < 4 ? w[r].sc.x : w[r].sc.y, k & 3);
                v[r] = fmaf(sc, fmaf(-32.f, xs, t), v[r]);
            }
            __builtin_amdgcn_sched_barrier(0);  // keep one activation run live
        }
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = fmaf(hf(w[r].d & 0xFFFFu), v[r], acc[r]);
    } else {
        // one Q8_0 block (dequant.rs:58-76); q+128 via xor 0x80
        const uint32_t X = 0x80808080u;
        float t[R];
        float4 x[4];
#pragma unroll
        for (int q = 0; q < 2; q++) {
            ldrun(x, xu + 16 * q);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint4 &qq = q ? w[r].q1 : w[r].q0;
                t[r] = run16(qq.x ^ X, qq.y ^ X, qq.z ^ X, qq.w ^ X, x, q ? t[r] : 0.f);
            }
        }
        const float2 s2 = *reinterpret_cast<const float2 *>(su);
        const float xsum = s2.x + s2.y;
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = fmaf(hf(w[r].d & 0xFFFFu), fmaf(-128.f, xsum, t[r]), acc[r]);
    }
}

// ---------------------------------------------------------------------------
// cross-lane sum within aligned groups of L lanes
// ---------------------------------------------------------------------------
template <int L>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = L / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float silu_mul(float g, float u) {
    // ops.rs:978-988: silu(g) = g / (1 + exp(-g)), then * up
    const float den = 1.0f + expf(-g);
    return (g / den) * u;
}

// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------
// orderable 64-bit argmax key of logit v at row r: larger value wins, ties go
// to the smaller row (the first max, ops.rs:1035-1045); NaN never wins
__device__ __forceinline__ unsigned long long amax_key(float v, uint32_t r) {
    if (v != v) return 0ull;
    const uint32_t b = __float_as_uint(v);
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)o << 32) | (0xFFFFFFFFu - r);
}

// Segments [s_lo, s_hi) of `a` are processed by blocks of this shape; the
// block's global index selects the segment.
template <uint32_t T, int LPR, int R, int WAVES>
__device__ __forceinline__ void mv_body(const MvArgs &a, uint32_t s_lo, uint32_t s_hi) {
    extern __shared__ float lds[];
    __shared__ float red[WAVES];
    __shared__ unsigned long long kred[WAVES];
    constexpr uint32_t UE = unit_elems<T>();
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t li = lane % LPR, g = lane / LPR;
    constexpr uint32_t RPW = (64 / LPR) * R;  // logical rows per wave
    constexpr uint32_t RPB = RPW * WAVES;     // logical rows per block
    constexpr uint32_t EPB = T == T_Q8_0 ? 32u : 256u;  // elements per quant block

    // segment of this block (uniform)
    uint32_t si = s_lo;
#pragma unroll
    for (int s = 1; s < MV_MAX_SEG; s++)
        if ((uint32_t)s > s_lo && (uint32_t)s < s_hi && blockIdx.x >= a.seg[s].block0) si = s;
    const MvSeg &sg = a.seg[si];
    const uint32_t rows = sg.rows;
    const uint32_t row0 = (blockIdx.x - sg.block0) * RPB + wave * RPW + g * R;

    // physical row source of each logical row (dual: even -> q0, odd -> q1)
    size_t rblk[R];
    const uint8_t *rq[R];
    const uint16_t *rd[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        uint32_t lr = row0 + r;
        if (lr >= rows) lr = rows - 1;
        const bool odd = sg.dual && (lr & 1u);
        const uint32_t pr = sg.dual ? (lr >> 1) : lr;
        rq[r] = odd ? sg.q1 : sg.q0;
        rd[r] = odd ? sg.d1 : sg.d0;
        rblk[r] = (size_t)pr * a.nb;
    }

    const uint32_t tile = a.tile;  // elements per K-tile (multiple of UE)
    float *xs = lds;                                   // padded copy of the tile
    float *sums = lds + tile + 4 * (tile / UE);        // 16-element run sums

    for (uint32_t col = 0; col < a.cols; col++) {
        const float *xg = a.x + (size_t)col * a.n_in;
        float scale = 1.0f;
        if (a.norm_w) {
            float ss = 0.f;
            for (uint32_t i = 4 * threadIdx.x; i < a.n_in; i += 4 * blockDim.x) {
                const float4 v = *reinterpret_cast<const float4 *>(xg + i);
                ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
            }
            ss = group_sum<64>(ss);
            if (lane == 0) red[wave] = ss;
            __syncthreads();
            float tot = 0.f;
#pragma unroll
            for (int i = 0; i < WAVES; i++) tot += red[i];
            // ops.rs:56-66: scale = 1 / sqrt(mean(x^2) + eps); out = x*scale*w
            scale = 1.0f / sqrtf(tot / (float)a.n_in + a.eps);
        }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.f;

        for (uint32_t k0 = 0; k0 < a.n_in; k0 += tile) {
            const uint32_t tlen = min(tile, a.n_in - k0);
            const uint32_t nu = tlen / UE;
            // prefetch this lane's first unit of the tile before staging x
            URaw<T> wc[R], wn[R];
            uint32_t u = li;
            if (u < nu) {
#pragma unroll
                for (int r = 0; r < R; r++) uload<T>(wc[r], rq[r], rd[r], rblk[r], k0 + u * UE);
            }
            if (u + LPR < nu) {
#pragma unroll
                for (int r = 0; r < R; r++) uload<T>(wn[r], rq[r], rd[r], rblk[r], k0 + (u + LPR) * UE);
            }
            // stage (normalised) x and its 16-element run sums
            if (k0 > 0) __syncthreads();  // previous tile fully consumed
            for (uint32_t run = threadIdx.x; run < tlen / 16; run += blockDim.x) {
                const uint32_t i = 16 * run;
                float4 v[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    v[k] = *reinterpret_cast<const float4 *>(xg + k0 + i + 4 * k);
                    if (a.norm_w) {
                        const float4 nw = *reinterpret_cast<const float4 *>(a.norm_w + k0 + i + 4 * k);
                        v[k].x = (v[k].x * scale) * nw.x;
                        v[k].y = (v[k].y * scale) * nw.y;
                        v[k].z = (v[k].z * scale) * nw.z;
                        v[k].w = (v[k].w * scale) * nw.w;
                    }
                }
                float s = 0.f;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
                    *reinterpret_cast<float4 *>(xs + xphys<T>(i + 4 * k)) = v[k];
                }
                sums[run] = s;
            }
            __syncthreads();

            // prefetch distance 2: the loads of units u+LPR and u+2*LPR are in
            // flight while unit u computes
            for (; u < nu; u += 2 * LPR) {
                udot<T, R>(wc, xs + xphys<T>(u * UE), sums + u * (UE / 16), k0 + u * UE, acc);
                if (u + 2 * LPR < nu) {
#pragma unroll
                    for (int r = 0; r < R; r++) uload<T>(wc[r], rq[r], rd[r], rblk[r], k0 + (u + 2 * LPR) * UE);
                }
                const uint32_t un = u + LPR;
                if (un >= nu) break;
                udot<T, R>(wn, xs + xphys<T>(un * UE), sums + un * (UE / 16), k0 + un * UE, acc);
                if (un + 2 * LPR < nu) {
#pragma unroll
                    for (int r = 0; r < R; r++) uload<T>(wn[r], rq[r], rd[r], rblk[r], k0 + (un + 2 * LPR) * UE);
                }
            }
        }
        (void)EPB;
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = group_sum<LPR>(acc[r]);

        unsigned long long key = 0ull;  // greedy: this lane's best (logit, row)
        if (li == 0) {
            const uint32_t pos = a.step ? a.step[1] : 0u;
            float v[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t lr = row0 + r;
                v[r] = acc[r];
                if (sg.bias && lr < rows) v[r] = v[r] + sg.bias[lr];
            }
            if (sg.rope) {
                // ops.rs:952-975 adjacent pairs (x[2i], x[2i+1]), theta = pos*freq[i]
#pragma unroll
                for (int r = 0; r + 1 < R; r += 2) {
                    const uint32_t lr = row0 + r;
                    const uint32_t dd = lr % a.head_dim;
                    if (dd < a.rope_dim) {
                        const float th = (float)(pos + col) * a.freq[dd >> 1];
                        float sn, cs;
                        sincosf(th, &sn, &cs);
                        const float x0 = v[r], x1 = v[r + 1];
                        v[r] = x0 * cs - x1 * sn;
                        v[r + 1] = x0 * sn + x1 * cs;
                    }
                }
            }
            float *out = sg.out ? sg.out + (size_t)col * a.y_stride : nullptr;
            if (sg.epi == EPI_SWIGLU) {
#pragma unroll
                for (int r = 0; r + 1 < R; r += 2) {
                    const uint32_t lr = row0 + r;
                    if (lr + 1 < rows) out[lr >> 1] = silu_mul(v[r], v[r + 1]);
                }
            } else if (sg.epi == EPI_KV) {
                // f16 cache, head-major [kv_head][ctx][head_dim] (kv_pack.comp)
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t lr = row0 + r;
                    if (lr < rows) {
                        const uint32_t hh = lr / a.head_dim, dd = lr % a.head_dim;
                        const size_t o = ((size_t)hh * a.ctx + pos + col) * a.head_dim + dd;
                        sg.kv[o] = (_Float16)v[r];
                    }
                }
            } else if (sg.epi == EPI_ACCUM) {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t lr = row0 + r;
                    if (lr < rows) out[lr] = out[lr] + v[r];
                }
            } else {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t lr = row0 + r;
                    if (lr < rows) out[lr] = v[r];
                }
            }
            if (a.amax) {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t lr = row0 + r;
                    if (lr < rows) {
                        const unsigned long long k = amax_key(v[r], lr);
                        key = k > key ? k : key;
                    }
                }
            }
        }
        if (a.amax) {
            // per-block argmax of the logits; k_argmax_finish reduces the blocks
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                const unsigned long long k = __shfl_xor(key, o, 64);
                key = k > key ? k : key;
            }
            if (lane == 0) kred[wave] = key;
            __syncthreads();
            if (threadIdx.x == 0) {
                unsigned long long b = kred[0];
#pragma unroll
                for (int w = 1; w < WAVES; w++) b = kred[w] > b ? kred[w] : b;
                a.amax[blockIdx.x] = b;
            }
        }
        __syncthreads();  // LDS and red[] are reused by the next column
    }
}

template <uint32_t T, int LPR, int R, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void k_mv(MvArgs a) {
    mv_body<T, LPR, R, WAVES>(a, 0, a.n_seg);
}

// two weight types in one launch: segments [0, n_seg0) of type T0 (blocks of
// shape L0 x R0), then [n_seg0, n_seg) of type T1 (L1 x R1); the activation
// and its norm are shared (q/k Q4_K with v Q6_K in the Q4_K_M mix)
template <uint32_t T0, int L0, int R0, uint32_t T1, int L1, int R1, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void k_mv2(MvArgs a) {
    if (blockIdx.x < a.seg[a.n_seg0].block0)
        mv_body<T0, L0, R0, WAVES>(a, 0, a.n_seg0);
    else
        mv_body<T1, L1, R1, WAVES>(a, a.n_seg0, a.n_seg);
}

// ---------------------------------------------------------------------------
// dispatch
// ---------------------------------------------------------------------------
using KFn = void (*)(MvArgs);

template <uint32_t T, int LPR, int R>
static KFn pick_w(int w) {
    switch (w) {
    case 2: return k_mv<T, LPR, R, 2>;
    case 8: return k_mv<T, LPR, R, 8>;
    default: return k_mv<T, LPR, R, 4>;
    }
}
template <uint32_t T, int LPR>
static KFn pick_r(int r, int w) {
    switch (r) {
    case 1: return pick_w<T, LPR, 1>(w);
    case 4: return pick_w<T, LPR, 4>(w);
    default: return pick_w<T, LPR, 2>(w);
    }
}
template <uint32_t T>
static KFn pick_lpr(int lpr, int r, int w) {
    switch (lpr) {
    case 8: return pick_r<T, 8>(r, w);
    case 16: return pick_r<T, 16>(r, w);
    case 64: return pick_r<T, 64>(r, w);
    default: return pick_r<T, 32>(r, w);
    }
}

static MvGeom g_override = {-1, 0, 0};

int set_matvec_geom(int lpr, int r, int waves) {
    if (lpr == 0 && r == 0 && waves == 0) {
        g_override = {0, 0, 0};
        return 0;
    }
    if ((lpr != 8 && lpr != 16 && lpr != 32 && lpr != 64) || (r != 1 && r != 2 && r != 4) ||
        (waves != 2 && waves != 4 && waves != 8))
        return -1;
    g_override = {lpr, r, waves};
    return 0;
}

// Geometry: lanes per row so that each lane owns several units (a deep
// stream of 128-bit loads), 2 rows per group when an epilogue pairs rows
// (RoPE / SwiGLU) or the x reuse pays, 4 waves per workgroup.
MvGeom choose_geom(uint32_t t, uint32_t n_in, uint32_t rows, bool pairs) {
    if (g_override.lpr < 0) {
        g_override = {0, 0, 0};
        if (const char *s = getenv("LRS_MATVEC_GEOM")) {
            int a = 0, b = 0, c = 0;
            if (sscanf(s, "%d,%d,%d", &a, &b, &c) == 3) set_matvec_geom(a, b, c);
        }
    }
    MvGeom gm;
    if (g_override.lpr > 0) {
        gm = g_override;
        if (pairs && gm.r < 2) gm.r = 2;
    } else {
        // one row per lane group (two when an epilogue pairs rows); lanes per
        // row = the smallest power of two in [8, 64] that still puts ~8
        // wavefronts on every CU (2048 waves), measured best on MI355X
        const int r = pairs ? 2 : 1;
        const uint64_t want = 2048ull * 64ull * (uint64_t)r;
        int lpr = 8;
        while (lpr < 64 && (uint64_t)rows * (uint64_t)lpr < want) lpr *= 2;
        gm = {lpr, r, 4};
        (void)t;
        (void)n_in;
    }
    return gm;
}

hipError_t launch_mv(const MvArgs &args_in, MvGeom gm, uint32_t type, hipStream_t s,
                     uint32_t *blocks_out) {
    MvArgs a = args_in;
    const uint32_t rpb = (uint32_t)(gm.waves * (64 / gm.lpr) * gm.r);
    uint32_t blocks = 0;
    for (uint32_t i = 0; i < a.n_seg; i++) {
        a.seg[i].block0 = blocks;
        blocks += (a.seg[i].rows + rpb - 1) / rpb;
    }
    const uint32_t ue = type == T_Q6_K ? 128u : type == T_Q8_0 ? 32u : 64u;
    if (a.n_in % ue) return hipErrorInvalidValue;
    a.tile = a.n_in <= MV_TILE ? a.n_in : MV_TILE;
    const size_t lds = ((size_t)a.tile + 4 * (a.tile / ue) + a.tile / 16) * sizeof(float);
    KFn fn = nullptr;
    switch (type) {
    case T_Q4_K: fn = pick_lpr<T_Q4_K>(gm.lpr, gm.r, gm.waves); break;
    case T_Q5_K: fn = pick_lpr<T_Q5_K>(gm.lpr, gm.r, gm.waves); break;
    case T_Q6_K: fn = pick_lpr<T_Q6_K>(gm.lpr, gm.r, gm.waves); break;
    case T_Q8_0: fn = pick_lpr<T_Q8_0>(gm.lpr, gm.r, gm.waves); break;
    default: return hipErrorInvalidValue;
    }
    if (a.amax && (a.cols != 1 || blocks > a.amax_cap)) return hipErrorInvalidValue;
    if (blocks_out) *blocks_out = blocks;
    hipLaunchKernelGGL(fn, dim3(blocks), dim3(64 * gm.waves), lds, s, a);
    return hipGetLastError();
}

template <int L0, int L1>
static KFn pick_q4k_q6k() {
    return k_mv2<T_Q4_K, L0, 2, T_Q6_K, L1, 1, 4>;
}

// Segments [0, n_seg0) of type t0 (row pairs: RoPE) and [n_seg0, n_seg) of
// type t1 in one launch.  Instantiated for Q4_K + Q6_K (the Q4_K_M q/k + v);
// hipErrorNotSupported for other pairs (the caller launches them apart).
hipError_t launch_mv2(const MvArgs &args_in, uint32_t t0, MvGeom g0, uint32_t t1, MvGeom g1,
                      hipStream_t s) {
    if (t0 != T_Q4_K || t1 != T_Q6_K || g0.r != 2 || g1.r != 1 || g0.waves != 4 ||
        g1.waves != 4 || (g0.lpr != 32 && g0.lpr != 64) || (g1.lpr != 32 && g1.lpr != 64) ||
        args_in.n_seg0 == 0 || args_in.n_seg0 >= args_in.n_seg)
        return hipErrorNotSupported;
    MvArgs a = args_in;
    uint32_t blocks = 0;
    for (uint32_t i = 0; i < a.n_seg; i++) {
        const MvGeom &g = i < a.n_seg0 ? g0 : g1;
        const uint32_t rpb = (uint32_t)(g.waves * (64 / g.lpr) * g.r);
        a.seg[i].block0 = blocks;
        blocks += (a.seg[i].rows + rpb - 1) / rpb;
    }
    if (a.n_in % 128 || a.amax) return hipErrorInvalidValue;
    a.tile = a.n_in <= MV_TILE ? a.n_in : MV_TILE;
    // LDS of the wider layout (Q4_K pads every 64 elements, Q6_K every 128)
    const size_t lds = ((size_t)a.tile + 4 * (a.tile / 64) + a.tile / 16) * sizeof(float);
    KFn fn = g0.lpr == 32 ? (g1.lpr == 32 ? pick_q4k_q6k<32, 32>() : pick_q4k_q6k<32, 64>())
                          : (g1.lpr == 32 ? pick_q4k_q6k<64, 32>() : pick_q4k_q6k<64, 64>());
    hipLaunchKernelGGL(fn, dim3(blocks), dim3(256), lds, s, a);
    return hipGetLastError();
}

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

hipError_t launch_matvec(WeightView w, const float *x, float *y, uint32_t cols, const float *bias,
                         hipStream_t s) {
    MvArgs a = {};
    a.n_seg = 1;
    a.seg[0].q0 = a.seg[0].q1 = w.q;
    a.seg[0].d0 = a.seg[0].d1 = w.d;
    a.seg[0].rows = w.n_out;
    a.seg[0].bias = bias;
    a.seg[0].out = y;
    a.seg[0].epi = EPI_STORE;
    a.n_in = w.n_in;
    a.nb = w.nb;
    a.x = x;
    a.cols = cols;
    a.y_stride = w.n_out;
    return launch_mv(a, choose_geom(w.type, w.n_in, w.n_out, false), w.type, s);
}

}  // namespace lrs
