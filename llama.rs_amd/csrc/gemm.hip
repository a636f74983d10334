// gemm.hip — dequantize x GEMM for batched prefill on the gfx950 matrix cores.
//
// Y[m][n] = sum_k A[m][k] * W[n][k]: A = M tokens x K activations (f32 in
// HBM), W = a resident N x K GGUF weight (Q4_K or Q6_K).  Replaces the
// reference's prefill GEMM (shaders/mul_mm.comp, dispatched by
// matmul::dispatch_mul_mm_q4k, crates/llama-vulkan/src/matmul.rs:433-465),
// which quantizes A to int8; here both operands go to the MFMA units as bf16
// (v_mfma_f32_32x32x16_bf16, f32 accumulate):
//   PREC 1  A and dequant(W) rounded to bf16 once
//   PREC 3  both split into bf16 hi + lo, three products (hi*hi + hi*lo +
//           lo*hi): ~2^-16 relative per product, for prefill whose logits must
//           match the f32 reference
//
// Tiling.  A 256-thread workgroup owns a 128 (tokens) x 128 (weight rows)
// output tile; each of its 4 wavefronts a 64 x 64 quarter = 2 x 2 MFMA tiles
// of 32 x 32.  K advances 64 at a time (one Q4_K qs group / a quarter of a
// Q6_K super-block): every thread stages 32 activations (f32 -> bf16) and
// dequantizes 32 weights of one row (bit-exact f32 dequant as in dequant.rs,
// then bf16) into a double-buffered LDS tile, and each wavefront issues 4 K16
// steps x 4 tiles of MFMA.  LDS rows are padded to 72 bf16 so the 32 lanes
// that read 32 different rows at one K offset hit distinct banks.
#include "lrs_internal.h"
#include "quant_dev.h"

namespace lrs {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;

constexpr int GM_BM = 128, GM_BN = 128, GM_BK = 64;
constexpr int GM_LD = GM_BK + 8;  // padded LDS row (bf16 elements)

struct GemmArgs {
    const __bf16 *ahi, *alo;  // A [M][K] as bf16 (hi, and lo = bf16(a - hi) for PREC 3)
    float *y;                 // [M][ldy]
    const uint8_t *q;         // weight, tiled layout (tiled.h)
    uint32_t M, N, K, units, ldy;
    uint32_t accum;           // 1: y += A W^T (residual add), 0: y = A W^T
    uint32_t nm, nn;          // output tiles along M and N
};

__device__ __forceinline__ uint4 ldq16(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }

// Raw GGUF bytes a thread needs for 32 consecutive weights of row n starting
// at element e (e % 32 == 0): loaded one K-step ahead, dequantized after the
// current step's matrix-core work has been issued
template <uint32_t T> struct WRaw;
template <> struct WRaw<T_Q4_K> { uint4 hd, q0, q1; };
template <> struct WRaw<T_Q6_K> { uint4 l0, l1, h0, h1; uint32_t sc, d; };

template <uint32_t T>
__device__ __forceinline__ void wload(const GemmArgs &g, uint32_t n, uint32_t e, WRaw<T> &w) {
    const uint32_t o = e & 255, r = n & 15;  // offset inside the super-block, row in the tile
    const uint8_t *c = g.q + ((size_t)(n >> 4) * g.units + (e >> 8)) * tchunk_bytes(T);
    if constexpr (T == T_Q4_K) {
        const uint32_t j = o >> 6;  // qs group
        // qs bytes 32j..32j+31 = pieces (g, r) with g = 2(j&1), 2(j&1)+1 of half j>>1
        const uint8_t *qp = c + 256 + 1024 * (j >> 1) + 16 * (16 * (2 * (j & 1)) + r);
        w.hd = ldq16(c + 16 * r);
        w.q0 = ldq16(qp);
        w.q1 = ldq16(qp + 256);
    } else {  // T_Q6_K
        const uint32_t h = o >> 7, quarter = (o >> 5) & 3;  // elements 128h + 32 quarter + l
        // ql[64h + 32(quarter&1) + l] and qh[32h + l]: pieces g = 2h (l < 16), 2h+1 (l >= 16)
        const uint8_t *ql = c + 256 + 1024 * (quarter & 1) + 16 * (16 * (2 * h) + r);
        const uint8_t *qh = c + 2304 + 16 * (16 * (2 * h) + r);
        w.l0 = ldq16(ql);
        w.l1 = ldq16(ql + 256);
        w.h0 = ldq16(qh);
        w.h1 = ldq16(qh + 256);
        w.sc = *reinterpret_cast<const uint16_t *>(c + 16 * r + 8 * h + 2 * quarter);
        w.d = *reinterpret_cast<const uint16_t *>(c + 3328 + 2 * r);
    }
}

// the 32 weights in f32, exactly as ggml_cpu::dequant (dequant.rs:101-258)
template <uint32_t T>
__device__ __forceinline__ void wdeq(const WRaw<T> &w, uint32_t e, float (&v)[32]) {
    const uint32_t o = e & 255;
    if constexpr (T == T_Q4_K) {
        const uint32_t j = o >> 6, hi = (o >> 5) & 1;  // qs group, high nibbles
        // get_scale_min_k4 (dequant.rs:101-110): scale bytes 0-3, 4-7, 8-11 are
        // header words y, z, w; sub-block jj reads byte jj & 3 of each
        const uint32_t jj = 2 * j + hi, sh = 8 * (jj & 3);
        const uint32_t by = (w.hd.y >> sh) & 0xFF, bz = (w.hd.z >> sh) & 0xFF,
                       bw = (w.hd.w >> sh) & 0xFF;
        const uint32_t sc = jj < 4 ? (by & 63) : ((bw & 0xF) | ((by >> 6) << 4));
        const uint32_t m = jj < 4 ? (bz & 63) : ((bw >> 4) | ((bz >> 6) << 4));
        const float dv = h2f((uint16_t)(w.hd.x & 0xFFFF)), mv = h2f((uint16_t)(w.hd.x >> 16));
        const float d1 = __fmul_rn(dv, (float)sc), m1 = __fmul_rn(mv, (float)m);
        const uint32_t qw[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const uint32_t byte = (qw[i >> 2] >> (8 * (i & 3))) & 0xFF;
            const uint32_t q = hi ? (byte >> 4) : (byte & 15);
            v[i] = __fsub_rn(__fmul_rn(d1, (float)q), m1);
        }
    } else {  // T_Q6_K
        const uint32_t quarter = (o >> 5) & 3;
        const float dv = h2f((uint16_t)w.d);
        const float ds0 = __fmul_rn(dv, (float)(int8_t)(w.sc & 0xFF));
        const float ds1 = __fmul_rn(dv, (float)(int8_t)(w.sc >> 8));
        const uint32_t lw[8] = {w.l0.x, w.l0.y, w.l0.z, w.l0.w, w.l1.x, w.l1.y, w.l1.z, w.l1.w};
        const uint32_t hw[8] = {w.h0.x, w.h0.y, w.h0.z, w.h0.w, w.h1.x, w.h1.y, w.h1.z, w.h1.w};
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const uint32_t lb = (lw[i >> 2] >> (8 * (i & 3))) & 0xFF;
            const uint32_t hb = (hw[i >> 2] >> (8 * (i & 3))) & 0xFF;
            const uint32_t lo = quarter < 2 ? (lb & 15) : (lb >> 4);
            const int q = (int)(lo | (((hb >> (2 * quarter)) & 3) << 4)) - 32;
            v[i] = __fmul_rn(i < 16 ? ds0 : ds1, (float)q);
        }
    }
}

__device__ __forceinline__ __bf16 to_bf16(float v) { return (__bf16)v; }

// stores 32 values as bf16 (hi) and, for PREC 3, the bf16 remainders (lo)
template <int PREC>
__device__ __forceinline__ void put32(__bf16 *hi, __bf16 *lo, const float (&v)[32]) {
#pragma unroll
    for (int c = 0; c < 4; c++) {
        bf16x8 h, l;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float x = v[8 * c + i];
            h[i] = to_bf16(x);
            if constexpr (PREC == 3) l[i] = to_bf16(x - (float)h[i]);
        }
        *reinterpret_cast<bf16x8 *>(hi + 8 * c) = h;
        if constexpr (PREC == 3) *reinterpret_cast<bf16x8 *>(lo + 8 * c) = l;
    }
}

// Software pipeline over K: step k's operands sit in LDS buffer k & 1 while
// step k+1's activations (already bf16, split once per GEMM input by
// k_split_bf16) and raw weight bytes are in flight to registers; the
// wavefronts issue step k's MFMAs, then dequantize step k+1 into the other
// buffer (VALU work that overlaps the matrix cores), then one barrier.
//
// Tile order: workgroup b runs on XCD b % 8 (round-robin dispatch); the
// tiles are numbered M-block-major and XCD x takes the x-th contiguous run
// of them, so the workgroups of one XCD share one or two activation blocks,
// which stay in that XCD's L2.
template <uint32_t T, int PREC>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs g) {
    constexpr int NS = PREC == 3 ? 2 : 1;  // hi (+ lo) planes
    __shared__ __attribute__((aligned(16))) __bf16 As[2][NS][GM_BM * GM_LD];
    __shared__ __attribute__((aligned(16))) __bf16 Ws[2][NS][GM_BN * GM_LD];
    const uint32_t ntile = g.nm * g.nn, per = (ntile + 7) / 8;
    const uint32_t t = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (t >= ntile) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t m0 = (t / g.nn) * GM_BM, n0 = (t % g.nn) * GM_BN;
    const uint32_t wm = wave >> 1, wn = wave & 1;  // wave's 64 x 64 quarter
    // staging roles: thread t handles row t/2, half t%2 (32 of the 64 K)
    const uint32_t sr = tid >> 1, sh = (tid & 1) * 32;
    const uint32_t am = min(m0 + sr, g.M - 1), wr = min(n0 + sr, g.N - 1);
    const size_t aoff = (size_t)am * g.K + sh;

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    // two register sets: step k + 2 is loaded while step k is multiplied and
    // step k + 1 dequantized
    u32x4 a0[NS][4], a1[NS][4];
    WRaw<T> w0, w1;
#define LRS_GFETCH(A, W, K0)                                                                  \
    do {                                                                                      \
        _Pragma("unroll") for (int p = 0; p < NS; p++) {                                       \
            const u32x4 *ap = reinterpret_cast<const u32x4 *>((p == 0 ? g.ahi : g.alo) + aoff + (K0)); \
            _Pragma("unroll") for (int c = 0; c < 4; c++) A[p][c] = ap[c];                    \
        }                                                                                     \
        wload<T>(g, wr, (K0) + sh, W);                                                        \
    } while (0)
#define LRS_GSTAGE(BUF, A, W, K0)                                                             \
    do {                                                                                      \
        _Pragma("unroll") for (int p = 0; p < NS; p++)                                         \
            _Pragma("unroll") for (int c = 0; c < 4; c++)                                      \
                *reinterpret_cast<u32x4 *>(&As[BUF][p][sr * GM_LD + sh + 8 * c]) = A[p][c];    \
        float v_[32];                                                                         \
        wdeq<T>(W, (K0) + sh, v_);                                                            \
        put32<PREC>(&Ws[BUF][0][sr * GM_LD + sh], &Ws[BUF][NS - 1][sr * GM_LD + sh], v_);     \
    } while (0)
    auto mma = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < GM_BK / 16; ks++) {
            const uint32_t kk = 16 * ks + 8 * (lane >> 5);
            bf16x8 a[NS][2], b[NS][2];
#pragma unroll
            for (int p = 0; p < NS; p++)
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    a[p][u] = *reinterpret_cast<const bf16x8 *>(&As[buf][p][(64 * wm + 32 * u + (lane & 31)) * GM_LD + kk]);
                    b[p][u] = *reinterpret_cast<const bf16x8 *>(&Ws[buf][p][(64 * wn + 32 * u + (lane & 31)) * GM_LD + kk]);
                }
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    if constexpr (PREC == 3) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1][i], b[0][j], acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0][i], b[1][j], acc[i][j], 0, 0, 0);
                    }
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0][i], b[0][j], acc[i][j], 0, 0, 0);
                }
        }
    };

    // nk is even (K % 128 == 0): two steps per trip, no branch in the loop;
    // the last trip's look-ahead loads repeat the final step (unused)
    const uint32_t nk = g.K / GM_BK;
    LRS_GFETCH(a0, w0, 0);
    LRS_GFETCH(a1, w1, GM_BK);
    LRS_GSTAGE(0, a0, w0, 0);
    __syncthreads();
    for (uint32_t k = 0; k < nk; k += 2) {
        LRS_GFETCH(a0, w0, min(k + 2, nk - 1) * GM_BK);
        mma(0);
        LRS_GSTAGE(1, a1, w1, (k + 1) * GM_BK);
        __syncthreads();
        LRS_GFETCH(a1, w1, min(k + 3, nk - 1) * GM_BK);
        mma(1);
        LRS_GSTAGE(0, a0, w0, min(k + 2, nk - 1) * GM_BK);
        __syncthreads();
    }
#undef LRS_GFETCH
#undef LRS_GSTAGE
    // D layout: lane l, register r -> row 8(r/4) + 4(l/32) + r%4, column l%32
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t n = n0 + 64 * wn + 32 * j + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t m = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < g.M && n < g.N) {
                    float *o = g.y + (size_t)m * g.ldy + n;
                    *o = g.accum ? *o + acc[i][j][r] : acc[i][j][r];
                }
            }
        }
}

// a -> bf16 hi (round to nearest even) and, if lo, bf16(a - hi): the
// activation planes of the GEMM, 4 elements per thread
__global__ __launch_bounds__(256) void k_split_bf16(const float *__restrict__ a, size_t n4,
                                                    __bf16 *__restrict__ hi, __bf16 *__restrict__ lo) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const float4 v = reinterpret_cast<const float4 *>(a)[i];
    typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
    bf16x4 h, l;
    h[0] = to_bf16(v.x);
    h[1] = to_bf16(v.y);
    h[2] = to_bf16(v.z);
    h[3] = to_bf16(v.w);
    reinterpret_cast<bf16x4 *>(hi)[i] = h;
    if (lo) {
        l[0] = to_bf16(v.x - (float)h[0]);
        l[1] = to_bf16(v.y - (float)h[1]);
        l[2] = to_bf16(v.z - (float)h[2]);
        l[3] = to_bf16(v.w - (float)h[3]);
        reinterpret_cast<bf16x4 *>(lo)[i] = l;
    }
}

hipError_t launch_split_bf16(const float *a, size_t n, __bf16 *hi, __bf16 *lo, hipStream_t s) {
    if (n % 4) return hipErrorInvalidValue;
    const size_t n4 = n / 4;
    hipLaunchKernelGGL(k_split_bf16, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, a, n4, hi, lo);
    return hipGetLastError();
}

hipError_t launch_gemm(WeightView w, const __bf16 *ahi, const __bf16 *alo, float *y, uint32_t M,
                       uint32_t ldy, int prec, hipStream_t s, bool accum) {
    if (M == 0 || w.n_in % (2 * GM_BK) || (prec == 3 && !alo)) return hipErrorInvalidValue;
    GemmArgs g;
    g.ahi = ahi;
    g.alo = alo;
    g.y = y;
    g.q = w.q;
    g.M = M;
    g.N = w.n_out;
    g.K = w.n_in;
    g.units = tunits(w.type, w.n_in);
    g.ldy = ldy;
    g.accum = accum ? 1u : 0u;
    g.nm = (M + GM_BM - 1) / GM_BM;
    g.nn = (w.n_out + GM_BN - 1) / GM_BN;
    const uint32_t grid = 8 * ((g.nm * g.nn + 7) / 8);
    void (*fn)(GemmArgs) = nullptr;
    if (w.type == T_Q4_K) fn = prec == 3 ? k_gemm<T_Q4_K, 3> : k_gemm<T_Q4_K, 1>;
    else if (w.type == T_Q6_K) fn = prec == 3 ? k_gemm<T_Q6_K, 3> : k_gemm<T_Q6_K, 1>;
    else return hipErrorNotSupported;
    hipLaunchKernelGGL(fn, dim3(grid), dim3(256), 0, s, g);
    return hipGetLastError();
}

}  // namespace lrs
