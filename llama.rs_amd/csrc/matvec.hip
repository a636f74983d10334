// matvec.hip — fused dequantize x matvec for GGUF Q8_0 / Q4_K / Q5_K / Q6_K
// weights with f32 activations, gfx950 (wave64).
//
// Replaces shaders/q{8_0,4_k,5_k,6_k}_matvec.comp of llama.rs
// (crates/llama-vulkan/shaders, dispatched from matmul.rs:36-430 and
// resident_forward.rs:3678-3752) with a different numerical contract: the
// activation stays f32 (the reference quantizes it to int8), so y matches
// dequant + f32 dot (ops.rs:78-101) to ~1e-7 relative instead of ~1e-2.
//
// Geometry: a wavefront owns (64/LPR) row groups of R rows; the LPR lanes of a
// group stride over the row's 32-weight "units" (Q8_0 block, Q6_K ql chunk,
// or for Q4_K/Q5_K a pair of 16-byte qs chunks that share one 12-byte scale
// decode).  Every lane keeps its unit's activations in registers and applies
// them to R rows, so x is read once per R rows.  Quant bytes arrive in 128-bit
// loads; nibbles become floats with v_cvt_f32_ubyte{0..3}; scales/mins are
// unpacked in registers; the LPR partial sums are reduced across lanes.
#include "lrs_internal.h"

#include <cstdlib>
#include <cstdio>

namespace lrs {

__device__ __forceinline__ float hf(uint32_t h16) {
    _Float16 v;
    uint16_t b = (uint16_t)h16;
    __builtin_memcpy(&v, &b, 2);
    return (float)v;
}

#define UB0(v) ((float)((v) & 0xFFu))
#define UB1(v) ((float)(((v) >> 8) & 0xFFu))
#define UB2(v) ((float)(((v) >> 16) & 0xFFu))
#define UB3(v) ((float)((v) >> 24))

__device__ __forceinline__ float dot4b(uint32_t m, float4 x, float acc) {
    acc = fmaf(UB0(m), x.x, acc);
    acc = fmaf(UB1(m), x.y, acc);
    acc = fmaf(UB2(m), x.z, acc);
    acc = fmaf(UB3(m), x.w, acc);
    return acc;
}

__device__ __forceinline__ float4 ldx(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ uint4 ldq(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }
__device__ __forceinline__ float hsum4(float4 v) { return (v.x + v.y) + (v.z + v.w); }
__device__ __forceinline__ uint32_t u4get(const uint4 &v, int k) {
    return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w;
}

template <uint32_t T>
__host__ __device__ constexpr uint32_t units_per_block() {
    return T == T_Q8_0 ? 1u : T == T_Q6_K ? 8u : 4u;
}

// ---------------------------------------------------------------------------
// Q4_K / Q5_K unit: qs chunks c0 (sub-blocks 2j, 2j+1) and c0+4 (2j+4, 2j+5)
// of super-block sb; j = c0>>1, h = c0&1.  dequant.rs:101-203 layout.
// ---------------------------------------------------------------------------
template <uint32_t T, int R>
__device__ __forceinline__ void unit_q45k(const WeightView &w, const float *__restrict__ x,
                                          uint32_t u, uint32_t row0, float (&acc)[R]) {
    constexpr bool Q5 = T == T_Q5_K;
    constexpr uint32_t BB = Q5 ? 176 : 144, QS = Q5 ? 48 : 16;
    const uint32_t sb = u >> 2, c0 = u & 3, j = c0 >> 1, h = c0 & 1;
    const float *xb = x + sb * 256 + 64 * j + 16 * h;
    float4 xr[4][4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        xr[0][k] = ldx(xb + 4 * k);
        xr[1][k] = ldx(xb + 32 + 4 * k);
        xr[2][k] = ldx(xb + 128 + 4 * k);
        xr[3][k] = ldx(xb + 160 + 4 * k);
    }
    float xs[4];
#pragma unroll
    for (int q = 0; q < 4; q++)
        xs[q] = (hsum4(xr[q][0]) + hsum4(xr[q][1])) + (hsum4(xr[q][2]) + hsum4(xr[q][3]));
    const uint32_t sh = 16 * j;
#pragma unroll
    for (int r = 0; r < R; r++) {
        uint32_t row = row0 + r;
        if (row >= w.n_out) row = w.n_out - 1;
        const uint8_t *blk = w.q + ((size_t)row * w.nb + sb) * BB;
        const uint4 hd = ldq(blk);
        const uint4 qa = ldq(blk + QS + 16 * c0);
        const uint4 qb = ldq(blk + QS + 16 * (c0 + 4));
        uint4 qh = make_uint4(0, 0, 0, 0);
        if constexpr (Q5) qh = ldq(blk + 16 + 16 * h);
        const float d = hf(hd.x & 0xFFFFu), dm = hf(hd.x >> 16);
        const uint32_t A = hd.y >> sh, B = hd.z >> sh, C = hd.w >> sh;
        const uint32_t scl = A & 0x3F3Fu, ml = B & 0x3F3Fu;
        const uint32_t sch = (C & 0x0F0Fu) | ((A >> 2) & 0x3030u);
        const uint32_t mh = ((C >> 4) & 0x0F0Fu) | ((B >> 2) & 0x3030u);
        float t0 = 0.f, t1 = 0.f, t2 = 0.f, t3 = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t wa = u4get(qa, k), wb = u4get(qb, k);
            uint32_t l0 = wa & 0x0F0F0F0Fu, l1 = (wa >> 4) & 0x0F0F0F0Fu;
            uint32_t l2 = wb & 0x0F0F0F0Fu, l3 = (wb >> 4) & 0x0F0F0F0Fu;
            if constexpr (Q5) {
                const uint32_t hb = u4get(qh, k);
                l0 |= ((hb >> (2 * j)) & 0x01010101u) << 4;
                l1 |= ((hb >> (2 * j + 1)) & 0x01010101u) << 4;
                l2 |= ((hb >> (2 * j + 4)) & 0x01010101u) << 4;
                l3 |= ((hb >> (2 * j + 5)) & 0x01010101u) << 4;
            }
            t0 = dot4b(l0, xr[0][k], t0);
            t1 = dot4b(l1, xr[1][k], t1);
            t2 = dot4b(l2, xr[2][k], t2);
            t3 = dot4b(l3, xr[3][k], t3);
        }
        float s = UB0(scl) * t0;
        s = fmaf(UB1(scl), t1, s);
        s = fmaf(UB0(sch), t2, s);
        s = fmaf(UB1(sch), t3, s);
        float m = UB0(ml) * xs[0];
        m = fmaf(UB1(ml), xs[1], m);
        m = fmaf(UB0(mh), xs[2], m);
        m = fmaf(UB1(mh), xs[3], m);
        acc[r] = fmaf(d, s, acc[r]);
        acc[r] = fmaf(-dm, m, acc[r]);
    }
}

// ---------------------------------------------------------------------------
// Q6_K unit: 16-byte ql chunk c of super-block sb (dequant.rs:205-258)
//   hf = c>>2 (128-half), p = (c&3)>>1 (ql[l] vs ql[l+32]), is = c&1 (l/16)
//   low nibbles  -> elements 128hf + 32p + 16is + i,  qh bits 2p..2p+1,
//                   scale 8hf + is + 2p
//   high nibbles -> elements 128hf + 64 + 32p + 16is + i, qh bits 4+2p..,
//                   scale 8hf + is + 4 + 2p
// ---------------------------------------------------------------------------
template <int R>
__device__ __forceinline__ void unit_q6k(const WeightView &w, const float *__restrict__ x,
                                         uint32_t u, uint32_t row0, float (&acc)[R]) {
    const uint32_t sb = u >> 3, c = u & 7, hfl = c >> 2, p = (c & 3) >> 1, is = c & 1;
    const float *xb = x + sb * 256 + 128 * hfl + 32 * p + 16 * is;
    float4 xl[4], xh[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        xl[k] = ldx(xb + 4 * k);
        xh[k] = ldx(xb + 64 + 4 * k);
    }
    const float xsl = (hsum4(xl[0]) + hsum4(xl[1])) + (hsum4(xl[2]) + hsum4(xl[3]));
    const float xsh = (hsum4(xh[0]) + hsum4(xh[1])) + (hsum4(xh[2]) + hsum4(xh[3]));
    const uint32_t bsh = 8 * (is + 2 * p);
#pragma unroll
    for (int r = 0; r < R; r++) {
        uint32_t row = row0 + r;
        if (row >= w.n_out) row = w.n_out - 1;
        const size_t bi = (size_t)row * w.nb + sb;
        const uint8_t *blk = w.q + bi * Q6_QBYTES;
        const uint4 ql = ldq(blk + 64 * hfl + 16 * (c & 3));
        const uint4 qh = ldq(blk + 128 + 32 * hfl + 16 * is);
        const uint2 sc = *reinterpret_cast<const uint2 *>(blk + 192 + 8 * hfl);
        const float d = hf(w.d[bi]);
        float tl = 0.f, th = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t wl = u4get(ql, k), wh = u4get(qh, k);
            const uint32_t lo = (wl & 0x0F0F0F0Fu) | (((wh >> (2 * p)) & 0x03030303u) << 4);
            const uint32_t hi = ((wl >> 4) & 0x0F0F0F0Fu) | (((wh >> (4 + 2 * p)) & 0x03030303u) << 4);
            tl = dot4b(lo, xl[k], tl);
            th = dot4b(hi, xh[k], th);
        }
        const float sl = (float)((int32_t)(sc.x << (24 - bsh)) >> 24);
        const float shh = (float)((int32_t)(sc.y << (24 - bsh)) >> 24);
        float v = sl * fmaf(-32.f, xsl, tl);
        v = fmaf(shh, fmaf(-32.f, xsh, th), v);
        acc[r] = fmaf(d, v, acc[r]);
    }
}

// ---------------------------------------------------------------------------
// Q8_0 unit: one 32-weight block (dequant.rs:58-76); q+128 via xor 0x80
// ---------------------------------------------------------------------------
template <int R>
__device__ __forceinline__ void unit_q80(const WeightView &w, const float *__restrict__ x,
                                         uint32_t u, uint32_t row0, float (&acc)[R]) {
    const float *xb = x + 32 * u;
    float4 xv[8];
#pragma unroll
    for (int k = 0; k < 8; k++) xv[k] = ldx(xb + 4 * k);
    float xs = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) xs += hsum4(xv[k]);
#pragma unroll
    for (int r = 0; r < R; r++) {
        uint32_t row = row0 + r;
        if (row >= w.n_out) row = w.n_out - 1;
        const size_t bi = (size_t)row * w.nb + u;
        const uint4 q0 = ldq(w.q + bi * Q8_QBYTES);
        const uint4 q1 = ldq(w.q + bi * Q8_QBYTES + 16);
        const float d = hf(w.d[bi]);
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            t = dot4b(u4get(q0, k) ^ 0x80808080u, xv[k], t);
            t = dot4b(u4get(q1, k) ^ 0x80808080u, xv[4 + k], t);
        }
        acc[r] = fmaf(d, fmaf(-128.f, xs, t), acc[r]);
    }
}

// ---------------------------------------------------------------------------
// kernel
// ---------------------------------------------------------------------------
template <uint32_t T, int LPR, int R, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void k_matvec(WeightView w, const float *__restrict__ x,
                                                       float *__restrict__ y,
                                                       const float *__restrict__ bias,
                                                       uint32_t cols) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t li = lane % LPR, g = lane / LPR;
    constexpr uint32_t RPW = (64 / LPR) * R;
    const uint32_t row0 = (blockIdx.x * WAVES + wave) * RPW + g * R;
    const uint32_t n_units = w.nb * units_per_block<T>();
    for (uint32_t col = 0; col < cols; col++) {
        const float *xc = x + (size_t)col * w.n_in;
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.f;
        for (uint32_t u = li; u < n_units; u += LPR) {
            if constexpr (T == T_Q4_K || T == T_Q5_K) unit_q45k<T, R>(w, xc, u, row0, acc);
            else if constexpr (T == T_Q6_K) unit_q6k<R>(w, xc, u, row0, acc);
            else unit_q80<R>(w, xc, u, row0, acc);
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            float v = acc[r];
#pragma unroll
            for (int o = LPR / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
            acc[r] = v;
        }
        if (li == 0) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t row = row0 + r;
                if (row < w.n_out) {
                    float v = acc[r];
                    if (bias) v = v + bias[row];
                    y[(size_t)col * w.n_out + row] = v;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// dispatch table
// ---------------------------------------------------------------------------
using KFn = void (*)(WeightView, const float *, float *, const float *, uint32_t);

template <uint32_t T, int LPR, int R>
static KFn pick_waves(int waves) {
    switch (waves) {
    case 1: return k_matvec<T, LPR, R, 1>;
    case 2: return k_matvec<T, LPR, R, 2>;
    default: return k_matvec<T, LPR, R, 4>;
    }
}

template <uint32_t T, int LPR>
static KFn pick_r(int r, int waves) {
    switch (r) {
    case 1: return pick_waves<T, LPR, 1>(waves);
    case 4: return pick_waves<T, LPR, 4>(waves);
    default: return pick_waves<T, LPR, 2>(waves);
    }
}

template <uint32_t T>
static KFn pick_lpr(int lpr, int r, int waves) {
    switch (lpr) {
    case 16: return pick_r<T, 16>(r, waves);
    case 64: return pick_r<T, 64>(r, waves);
    default: return pick_r<T, 32>(r, waves);
    }
}

struct MvGeom {
    int lpr, r, waves;
};

// lanes per row: the largest of {64,32,16} that divides the unit count, else
// the one with the least idle lanes in the last pass
static MvGeom g_override = {-1, 0, 0};

int set_matvec_geom(int lpr, int r, int waves) {
    if (lpr == 0 && r == 0 && waves == 0) {
        g_override = {0, 0, 0};
        return 0;
    }
    if ((lpr != 16 && lpr != 32 && lpr != 64) || (r != 1 && r != 2 && r != 4) ||
        (waves != 1 && waves != 2 && waves != 4))
        return -1;
    g_override = {lpr, r, waves};
    return 0;
}

static MvGeom choose_geom(uint32_t t, uint32_t n_in, uint32_t n_out) {
    if (g_override.lpr < 0) {
        g_override = {0, 0, 0};
        if (const char *s = getenv("LRS_MATVEC_GEOM")) {
            int a = 0, b = 0, c = 0;
            if (sscanf(s, "%d,%d,%d", &a, &b, &c) == 3) set_matvec_geom(a, b, c);
        }
    }
    if (g_override.lpr > 0) return g_override;
    const uint32_t upb = t == T_Q8_0 ? 1 : t == T_Q6_K ? 8 : 4;
    const uint32_t units = n_in / (uint32_t)block_elems(t) * upb;
    int best = 32;
    double best_eff = -1;
    for (int lpr : {64, 32, 16}) {
        uint32_t passes = (units + lpr - 1) / lpr;
        double eff = (double)units / (double)(passes * lpr);
        if (eff > best_eff + 1e-9) { best_eff = eff; best = lpr; }
    }
    (void)n_out;
    return {best, 2, 4};
}

hipError_t launch_matvec(WeightView w, const float *x, float *y, uint32_t cols,
                         const float *bias, hipStream_t s) {
    MvGeom g = choose_geom(w.type, w.n_in, w.n_out);
    KFn fn = nullptr;
    switch (w.type) {
    case T_Q4_K: fn = pick_lpr<T_Q4_K>(g.lpr, g.r, g.waves); break;
    case T_Q5_K: fn = pick_lpr<T_Q5_K>(g.lpr, g.r, g.waves); break;
    case T_Q6_K: fn = pick_lpr<T_Q6_K>(g.lpr, g.r, g.waves); break;
    case T_Q8_0: fn = pick_lpr<T_Q8_0>(g.lpr, g.r, g.waves); break;
    default: return hipErrorInvalidValue;
    }
    const uint32_t rows_per_block = (uint32_t)(g.waves * (64 / g.lpr) * g.r);
    const uint32_t grid = (w.n_out + rows_per_block - 1) / rows_per_block;
    hipLaunchKernelGGL(fn, dim3(grid), dim3(64 * g.waves), 0, s, w, x, y, bias, cols);
    return hipGetLastError();
}

}  // namespace lrs
