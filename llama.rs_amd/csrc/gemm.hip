// gemm.hip — dequantize x GEMM for batched prefill on the gfx950 matrix cores.
//
// Y[m][n] = sum_k A[m][k] * W[n][k]: A = M tokens x K activations (f32 in
// HBM), W = a resident N x K GGUF weight (Q4_K, Q5_K, Q6_K or Q8_0).  Replaces the
// reference's prefill GEMM (shaders/mul_mm.comp, dispatched by
// matmul::dispatch_mul_mm_q4k, crates/llama-vulkan/src/matmul.rs:433-465),
// which quantizes A to int8; here both operands go to the MFMA units as bf16
// (v_mfma_f32_32x32x16_bf16, f32 accumulate):
//   PREC 1  A and dequant(W) rounded to bf16 once
//   PREC 3  both split into bf16 hi + lo, three products (hi*hi + hi*lo +
//           lo*hi): ~2^-16 relative per product, for prefill whose logits must
//           match the f32 reference
//
// Tiling.  A 512-thread workgroup owns a BM (tokens) x 128 (weight rows)
// output tile: BM = 256 for bf16 operands at M >= 512 (each wavefront a
// 64 x 64 part = 4 MFMA tiles of 32 x 32), else 128 (64 x 32 parts, 2
// tiles).  K advances 64 at a time: every thread stages BM / 8 activations
// (bf16, split from f32 once per GEMM input) and dequantizes 16 weights of
// one row (f32 dequant as in dequant.rs, the K-quant min term in the same
// fused multiply-add as the scale, then bf16) into a double-buffered LDS
// tile, and each wavefront issues 4 K16 steps of MFMA over its tiles.  LDS
// rows are padded to 72 bf16 so the 32 lanes that read 32 different rows at
// one K offset hit distinct banks.
#include "lrs_internal.h"
#include "quant_dev.h"

namespace lrs {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;

constexpr int GM_BN = 128, GM_BK = 64;
constexpr int GM_LD = GM_BK + 8;  // padded LDS row (bf16 elements)

// one weight of a launch: weights that share the input (a prompt block's q,
// k and v projections) run as one launch over their concatenated output
// tiles, segment s owning tiles [nt0, next segment's nt0) along N
constexpr int GM_MAX_SEG = 3;
struct GemmSeg {
    const uint8_t *q;  // weight, tiled layout (tiled.h)
    float *y;          // [M][ldy]
    uint32_t N, ldy, nt0;
};

struct GemmArgs {
    const __bf16 *ahi, *alo;  // A [M][K] as bf16 (hi, and lo = bf16(a - hi) for PREC 3)
    GemmSeg seg[GM_MAX_SEG];
    uint32_t nseg, nseg0;     // segments; the first nseg0 have the kernel's type T0, the rest T1
    uint32_t M, K;
    uint32_t accum;           // 1: y += A W^T (residual add), 0: y = A W^T
    uint32_t nm, nn;          // output tiles along M and N (all segments)
    uint32_t ks;              // K slices (one segment): slice z writes part + z*M*N (then a reduce)
    float *part;
};

__device__ __forceinline__ u32x4 ldq16(const uint8_t *p) { return *reinterpret_cast<const u32x4 *>(p); }

// Raw GGUF bytes a thread needs for 16 consecutive weights of row n starting
// at element e (e % 16 == 0), loaded three K-steps ahead and dequantized
// after the current step's matrix-core work has been issued
template <uint32_t T> struct WRaw;
template <> struct WRaw<T_Q4_K> { u32x4 hd, qs; };
template <> struct WRaw<T_Q6_K> { u32x4 ql, qh; uint32_t sc, d; };
template <> struct WRaw<T_Q5_K> { u32x4 hd, qh, qs; };
template <> struct WRaw<T_Q8_0> { u32x4 qs; uint32_t d; };

// rowq = the first chunk of the row's 16-row tile (hoisted out of the K
// loop: per step only the 32-bit unit offset changes); r = row in the tile
template <uint32_t T>
__device__ __forceinline__ void wload(const uint8_t *rowq, uint32_t r, uint32_t e, WRaw<T> &w) {
    const uint32_t o = e & 255;  // offset inside the super-block
    const uint32_t l0 = o & 16;  // first or second 16 of a 32-element run
    const uint8_t *c = rowq + (e / tunit_elems(T)) * tchunk_bytes(T);
    if constexpr (T == T_Q8_0) {
        // 64-element units of two blocks: piece g = 2 block + 16-byte half,
        // then the 16 rows' f16 d of both blocks (tiled.h)
        const uint32_t o6 = e & 63, b = o6 >> 5, pg = 2 * b + ((o6 >> 4) & 1);
        w.qs = ldq16(c + 16 * (16 * pg + r));
        w.d = *reinterpret_cast<const uint16_t *>(c + 1024 + 4 * r + 2 * b);
    } else if constexpr (T == T_Q5_K) {
        // as Q4_K with qs after the qh halves; qh[l0 .. l0 + 16) of row r is
        // half l0 / 16 of the row's qh (dequant.rs:157-203)
        const uint32_t j = o >> 6, pg = 2 * (j & 1) + (l0 >> 4);
        w.hd = ldq16(c + 16 * r);
        w.qh = ldq16(c + 256 + 16 * (16 * (l0 >> 4) + r));
        w.qs = ldq16(c + 768 + 1024 * (j >> 1) + 16 * (16 * pg + r));
    } else if constexpr (T == T_Q4_K) {
        // qs[32j + l0 ..+16), j = o / 64: piece (g, r), g = 2(j&1) + l0/16, of half j>>1
        const uint32_t j = o >> 6, pg = 2 * (j & 1) + (l0 >> 4);
        w.hd = ldq16(c + 16 * r);
        w.qs = ldq16(c + 256 + 1024 * (j >> 1) + 16 * (16 * pg + r));
    } else {  // T_Q6_K
        // elements 128h + 32 quarter + l: ql[64h + 32(quarter&1) + l], qh[32h + l],
        // pieces g = 2h + l0/16; scale byte 8h + l0/16 + 2 quarter
        const uint32_t h = o >> 7, quarter = (o >> 5) & 3, pg = 2 * h + (l0 >> 4);
        w.ql = ldq16(c + 256 + 1024 * (quarter & 1) + 16 * (16 * pg + r));
        w.qh = ldq16(c + 2304 + 16 * (16 * pg + r));
        w.sc = c[16 * r + 8 * h + (l0 >> 4) + 2 * quarter];
        w.d = *reinterpret_cast<const uint16_t *>(c + 3328 + 2 * r);
    }
}

// the 16 weights in f32 as ggml_cpu::dequant (dequant.rs:101-258) computes
// them with one fused multiply-add each: Q6_K a*q - 32a is a*(q - 32)
// rounded once, bit-exact; Q4_K / Q5_K a*q - b skips the reference's
// rounding of a*q (half an ulp of the product), which the bf16 rounding
// that follows absorbs:
// wprep decodes the run's scale (and min), wdeq4 the weights 4c..4c+3, so the
// dequant can be spread between the matrix-core ops of a pipeline step
struct DeqPrep {
    float a, b;    // Q4_K / Q5_K: d * sc, dmin * m; Q6_K: d * scale; Q8_0: d
    uint32_t sel;  // Q4_K / Q5_K: high nibbles; Q6_K: quarter of the half
    uint32_t sub;  // Q5_K: sub-block (its bit of qh)
};
template <uint32_t T>
__device__ __forceinline__ DeqPrep wprep(const WRaw<T> &w, uint32_t e) {
    const uint32_t o = e & 255;
    DeqPrep p;
    p.sub = 0;
    if constexpr (T == T_Q8_0) {
        p.a = h2f((uint16_t)w.d);
        p.b = 0.f;
        p.sel = 0;
    } else if constexpr (T == T_Q4_K || T == T_Q5_K) {
        const uint32_t j = o >> 6, hi = (o >> 5) & 1;  // qs group, high nibbles
        // get_scale_min_k4 (dequant.rs:101-110): scale bytes 0-3, 4-7, 8-11 are
        // header words y, z, w; sub-block jj reads byte jj & 3 of each
        const uint32_t jj = 2 * j + hi, sh = 8 * (jj & 3);
        const uint32_t by = (w.hd.y >> sh) & 0xFF, bz = (w.hd.z >> sh) & 0xFF,
                       bw = (w.hd.w >> sh) & 0xFF;
        // both forms, then a mask select: a conditional here compiles to a
        // divergent branch, which splits the step's MFMA / VALU interleaving
        const uint32_t lowm = 0u - (uint32_t)(jj < 4);
        const uint32_t sc = ((by & 63) & lowm) | (((bw & 0xF) | ((by >> 6) << 4)) & ~lowm);
        const uint32_t m = ((bz & 63) & lowm) | (((bw >> 4) | ((bz >> 6) << 4)) & ~lowm);
        const float dv = h2f((uint16_t)(w.hd.x & 0xFFFF)), mv = h2f((uint16_t)(w.hd.x >> 16));
        p.a = __fmul_rn(dv, (float)sc);
        p.b = __fmul_rn(mv, (float)m);
        p.sel = hi;
        p.sub = jj;
    } else {  // T_Q6_K
        p.a = __fmul_rn(h2f((uint16_t)w.d), (float)(int8_t)(w.sc & 0xFF));
        p.b = 0.f;
        p.sel = (o >> 5) & 3;
    }
    return p;
}
template <uint32_t T>
__device__ __forceinline__ void wdeq4(const WRaw<T> &w, const DeqPrep &p, int c, float (&v)[16]) {
    if constexpr (T == T_Q8_0) {
        // dequant.rs:58-76: q * d
        const uint32_t qw = c == 0 ? w.qs.x : c == 1 ? w.qs.y : c == 2 ? w.qs.z : w.qs.w;
#pragma unroll
        for (int i = 0; i < 4; i++)
            v[4 * c + i] = __fmul_rn((float)(int8_t)((qw >> (8 * i)) & 0xFF), p.a);
    } else if constexpr (T == T_Q4_K || T == T_Q5_K) {
        // the four quants as bytes of one word (nibble select and, for Q5_K,
        // the fifth bits: a few ops per 4 weights), then per weight one byte
        // conversion and one fused a * q - b
        const uint32_t qw = c == 0 ? w.qs.x : c == 1 ? w.qs.y : c == 2 ? w.qs.z : w.qs.w;
        uint32_t q4 = (qw >> (4 * p.sel)) & 0x0F0F0F0Fu;
        if constexpr (T == T_Q5_K) {
            const uint32_t hw = c == 0 ? w.qh.x : c == 1 ? w.qh.y : c == 2 ? w.qh.z : w.qh.w;
            q4 |= ((hw >> p.sub) & 0x01010101u) << 4;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) v[4 * c + i] = fmaf(p.a, (float)((q4 >> (8 * i)) & 0xFF), -p.b);
    } else {  // T_Q6_K: q = (ql nibble | qh 2 bits << 4) - 32
        const uint32_t lw = c == 0 ? w.ql.x : c == 1 ? w.ql.y : c == 2 ? w.ql.z : w.ql.w;
        const uint32_t hw = c == 0 ? w.qh.x : c == 1 ? w.qh.y : c == 2 ? w.qh.z : w.qh.w;
        const uint32_t q4 = ((lw >> (4 * (p.sel >> 1))) & 0x0F0F0F0Fu) |
                            (((hw >> (2 * p.sel)) & 0x03030303u) << 4);
        const float o = -32.0f * p.a;  // exact: a power-of-two multiple
#pragma unroll
        for (int i = 0; i < 4; i++) v[4 * c + i] = fmaf(p.a, (float)((q4 >> (8 * i)) & 0xFF), o);
    }
}

__device__ __forceinline__ __bf16 to_bf16(float v) { return (__bf16)v; }

// stores 16 values as bf16 (hi) and, for PREC 3, the bf16 remainders (lo)
template <int PREC>
__device__ __forceinline__ void put16(__bf16 *hi, __bf16 *lo, const float (&v)[16]) {
#pragma unroll
    for (int c = 0; c < 2; c++) {
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

// 512 threads = 8 wavefronts, each a 64 (tokens) x 32 (rows) part of the
// 128 x 128 tile (2 MFMA tiles of 32 x 32).  Software pipeline over K: step
// k's operands sit in LDS buffer k & 1; the activations (already bf16, split
// once per GEMM input by k_split_bf16) and raw weight bytes of steps k+1..k+3
// are in flight to four rotating register sets; each step the wavefronts
// load step k+3, issue step k's MFMAs, then dequantize step k+1 into the
// other buffer (VALU work that overlaps the matrix cores), then one barrier.
// K-quant rows are whole super-blocks (K % 256 == 0), so the loop runs four
// steps per trip with no tail.  One call computes the output tile (m0, n0
// of segment sg) of K slice kz with the weight of type T, over the
// workgroup's LDS stages As / Ws.
template <uint32_t T, int PREC, int BM>
__device__ __forceinline__ void gemm_tile(const GemmArgs &g, const GemmSeg &sg, uint32_t kz,
                                          uint32_t m0, uint32_t n0,
                                          __bf16 (*As)[PREC == 3 ? 2 : 1][BM * GM_LD],
                                          __bf16 (*Ws)[PREC == 3 ? 2 : 1][GM_BN * GM_LD]) {
    constexpr int NS = PREC == 3 ? 2 : 1;  // hi (+ lo) planes
    // wavefront grid: WM x WN = 8 wavefronts, each (BM / WM) x (128 / WN) of
    // the tile in MT x NT MFMA tiles of 32 x 32 (the 256-token tile uses 4 x 2
    // wavefronts of 64 x 64: fewer LDS operand reads per matrix-core op)
    constexpr int WM = BM == 256 ? 4 : 2, WN = 8 / WM;
    constexpr int MT = BM / WM / 32, NT = GM_BN / WN / 32;
    constexpr int AR = BM / 128;           // activation rows staged per thread
    const uint32_t kspan = g.K / g.ks;     // a multiple of 256
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t wm = wave / WN, wn = wave % WN;
    // staging roles: thread t handles row t/4, K quarter t%4 (16 of the 64)
    const uint32_t sr = tid >> 2, sq = (tid & 3) * 16;
    const uint32_t wr = min(n0 + sr, sg.N - 1);
    size_t aoff[AR];  // activation rows sr, sr + 128, ...
#pragma unroll
    for (int j = 0; j < AR; j++)
        aoff[j] = (size_t)min(m0 + sr + 128 * j, g.M - 1) * g.K + sq + (size_t)kz * kspan;
    const uint32_t kbase = kz * kspan;  // weight element offset of the slice
    const uint8_t *rowq = sg.q + (size_t)(wr >> 4) * tunits(T, g.K) * tchunk_bytes(T);

    f32x16 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int jn = 0; jn < NT; jn++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][jn][r] = 0.f;

    u32x4 a0[NS][AR][2], a1[NS][AR][2], a2[NS][AR][2], a3[NS][AR][2];
    WRaw<T> w0, w1, w2, w3;
#define LRS_GFETCH(A, W, K0)                                                                  \
    do {                                                                                      \
        _Pragma("unroll") for (int p = 0; p < NS; p++)                                         \
            _Pragma("unroll") for (int j = 0; j < AR; j++) {                                   \
                const u32x4 *ap = reinterpret_cast<const u32x4 *>((p == 0 ? g.ahi : g.alo) + aoff[j] + (K0)); \
                A[p][j][0] = ap[0];                                                           \
                A[p][j][1] = ap[1];                                                           \
            }                                                                                 \
        wload<T>(rowq, wr & 15, kbase + (K0) + sq, W);                                       \
    } while (0)
#define LRS_GSTAGE(BUF, A, W, K0)                                                             \
    do {                                                                                      \
        _Pragma("unroll") for (int p = 0; p < NS; p++)                                         \
            _Pragma("unroll") for (int j = 0; j < AR; j++) {                                   \
                *reinterpret_cast<u32x4 *>(&As[BUF][p][(sr + 128 * j) * GM_LD + sq]) = A[p][j][0];     \
                *reinterpret_cast<u32x4 *>(&As[BUF][p][(sr + 128 * j) * GM_LD + sq + 8]) = A[p][j][1]; \
            }                                                                                 \
        float v_[16];                                                                         \
        const DeqPrep dp_ = wprep<T>(W, kbase + (K0) + sq);                                   \
        _Pragma("unroll") for (int c = 0; c < 4; c++) wdeq4<T>(W, dp_, c, v_);                \
        put16<PREC>(&Ws[BUF][0][sr * GM_LD + sq], &Ws[BUF][NS - 1][sr * GM_LD + sq], v_);     \
    } while (0)
    // operand fragments of sub-step ks (K16) from LDS buffer buf
    auto frag = [&](int buf, int ks, bf16x8 (&a)[NS][MT], bf16x8 (&b)[NS][NT]) __attribute__((always_inline)) {
        const uint32_t kk = 16 * ks + 8 * (lane >> 5);
#pragma unroll
        for (int p = 0; p < NS; p++) {
#pragma unroll
            for (int u = 0; u < MT; u++)
                a[p][u] = *reinterpret_cast<const bf16x8 *>(&As[buf][p][((BM / WM) * wm + 32 * u + (lane & 31)) * GM_LD + kk]);
#pragma unroll
            for (int u = 0; u < NT; u++)
                b[p][u] = *reinterpret_cast<const bf16x8 *>(&Ws[buf][p][((GM_BN / WN) * wn + 32 * u + (lane & 31)) * GM_LD + kk]);
        }
    };
    auto mfma = [&](const bf16x8 (&a)[NS][MT], const bf16x8 (&b)[NS][NT]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < MT; i++)
#pragma unroll
            for (int jn = 0; jn < NT; jn++) {
                if constexpr (PREC == 3) {
                    acc[i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1][i], b[0][jn], acc[i][jn], 0, 0, 0);
                    acc[i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0][i], b[1][jn], acc[i][jn], 0, 0, 0);
                }
                acc[i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0][i], b[0][jn], acc[i][jn], 0, 0, 0);
            }
    };
    // one pipeline step: step k's four K16 sub-steps from buffer buf (the
    // fragments of sub-step ks+1 read while sub-step ks's matrix-core ops
    // run), step k+1's activations copied into the other buffer first and
    // its weights dequantized a quarter after each sub-step, so the VALU
    // work overlaps the matrix cores
#define LRS_GSTEP(BUF, A, W, K0)                                                              \
    do {                                                                                      \
        _Pragma("unroll") for (int p = 0; p < NS; p++)                                         \
            _Pragma("unroll") for (int j = 0; j < AR; j++) {                                   \
                *reinterpret_cast<u32x4 *>(&As[1 - (BUF)][p][(sr + 128 * j) * GM_LD + sq]) = A[p][j][0];     \
                *reinterpret_cast<u32x4 *>(&As[1 - (BUF)][p][(sr + 128 * j) * GM_LD + sq + 8]) = A[p][j][1]; \
            }                                                                                 \
        const DeqPrep dp_ = wprep<T>(W, kbase + (K0) + sq);                                   \
        float v_[16];                                                                         \
        bf16x8 fa0[NS][MT], fb0[NS][NT], fa1[NS][MT], fb1[NS][NT];                            \
        frag(BUF, 0, fa0, fb0);                                                               \
        frag(BUF, 1, fa1, fb1);                                                               \
        mfma(fa0, fb0);                                                                       \
        wdeq4<T>(W, dp_, 0, v_);                                                              \
        frag(BUF, 2, fa0, fb0);                                                               \
        mfma(fa1, fb1);                                                                       \
        wdeq4<T>(W, dp_, 1, v_);                                                              \
        frag(BUF, 3, fa1, fb1);                                                               \
        mfma(fa0, fb0);                                                                       \
        wdeq4<T>(W, dp_, 2, v_);                                                              \
        mfma(fa1, fb1);                                                                       \
        wdeq4<T>(W, dp_, 3, v_);                                                              \
        put16<PREC>(&Ws[1 - (BUF)][0][sr * GM_LD + sq], &Ws[1 - (BUF)][NS - 1][sr * GM_LD + sq], v_); \
    } while (0)

    const uint32_t nk = kspan / GM_BK;  // a multiple of 4
    auto kc = [&](uint32_t k) { return min(k, nk - 1) * GM_BK; };  // look-ahead past the end repeats the last step (unused)
    LRS_GFETCH(a0, w0, 0);
    LRS_GFETCH(a1, w1, kc(1));
    LRS_GFETCH(a2, w2, kc(2));
    LRS_GSTAGE(0, a0, w0, 0);
    __syncthreads();
    for (uint32_t k = 0; k < nk; k += 4) {
        LRS_GFETCH(a3, w3, kc(k + 3));
        LRS_GSTEP(0, a1, w1, kc(k + 1));
        __syncthreads();
        LRS_GFETCH(a0, w0, kc(k + 4));
        LRS_GSTEP(1, a2, w2, kc(k + 2));
        __syncthreads();
        LRS_GFETCH(a1, w1, kc(k + 5));
        LRS_GSTEP(0, a3, w3, kc(k + 3));
        __syncthreads();
        LRS_GFETCH(a2, w2, kc(k + 6));
        LRS_GSTEP(1, a0, w0, kc(k + 4));
        __syncthreads();
    }
#undef LRS_GFETCH
#undef LRS_GSTAGE
#undef LRS_GSTEP
    // D layout: lane l, register r -> row 8(r/4) + 4(l/32) + r%4, column l%32
#pragma unroll
    for (int jn = 0; jn < NT; jn++) {
        const uint32_t n = n0 + (GM_BN / WN) * wn + 32 * jn + (lane & 31);
#pragma unroll
        for (int i = 0; i < MT; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t m = m0 + (BM / WM) * wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < g.M && n < sg.N) {
                    if (g.ks > 1) {
                        g.part[((size_t)kz * g.M + m) * sg.N + n] = acc[i][jn][r];
                    } else {
                        float *o = sg.y + (size_t)m * sg.ldy + n;
                        *o = g.accum ? *o + acc[i][jn][r] : acc[i][jn][r];
                    }
                }
            }
    }
}

// workgroup b takes output tile t0 of the (K slice, M block, N tile) order;
// the segment of its N tile picks the weight and the type (T0 for the first
// nseg0 segments, T1 after them); MS = the most segments the instance takes
// (1: single-weight launches).  Tile order: workgroup b runs on XCD b % 8
// (round-robin dispatch); the tiles are numbered M-block-major and XCD x
// takes the x-th contiguous run of them, so the workgroups of one XCD share
// one or two activation blocks, which stay in that XCD's L2.
template <uint32_t T0, uint32_t T1, int PREC, int BM, int MS>
__global__ __launch_bounds__(512) void k_gemm(GemmArgs g) {
    constexpr int NS = PREC == 3 ? 2 : 1;
    __shared__ __attribute__((aligned(16))) __bf16 As[2][NS][BM * GM_LD];
    __shared__ __attribute__((aligned(16))) __bf16 Ws[2][NS][GM_BN * GM_LD];
    const uint32_t ntile = g.nm * g.nn * g.ks, per = (ntile + 7) / 8;
    const uint32_t t0 = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (t0 >= ntile) return;
    const uint32_t kz = t0 / (g.nm * g.nn), t = t0 % (g.nm * g.nn);  // K slice, output tile
    const uint32_t nt = t % g.nn;
    uint32_t si = 0;
#pragma unroll
    for (int i = 1; i < MS; i++)
        if ((uint32_t)i < g.nseg && nt >= g.seg[i].nt0) si = i;
    const GemmSeg sg = g.seg[si];
    const uint32_t m0 = (t / g.nn) * BM, n0 = (nt - sg.nt0) * GM_BN;
    if (T0 == T1 || si < g.nseg0)
        gemm_tile<T0, PREC, BM>(g, sg, kz, m0, n0, As, Ws);
    else
        gemm_tile<T1, PREC, BM>(g, sg, kz, m0, n0, As, Ws);
}

// y[m][n] (+)= sum over the K slices of part[z][m][n], slices in order
__global__ __launch_bounds__(256) void k_reduce_ks(const float *__restrict__ part, float *__restrict__ y,
                                                   uint32_t M, uint32_t N, uint32_t ldy, uint32_t ks,
                                                   uint32_t accum) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)M * N) return;
    const uint32_t m = (uint32_t)(i / N), n = (uint32_t)(i % N);
    float v = part[i];
    for (uint32_t z = 1; z < ks; z++) v += part[(size_t)z * M * N + i];
    float *o = y + (size_t)m * ldy + n;
    *o = accum ? *o + v : v;
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

// K slices for a GEMM with fewer output tiles than CUs (the long-K o / down
// projections): the slice count ks divides K into whole super-blocks and
// minimises the rounds of 256 workgroups (one per CU) each slice-sized unit
// of work takes, ceil(tiles * ks / 256) / ks, plus a small charge for the
// reduction pass; ties keep fewer slices
// token tile: 256 for bf16 operands at M >= 512 (twice the MFMA work per
// dequantized weight: the dequant, not the matrix cores, bounds the 128-row
// tile), else 128; the hi/lo form keeps 128 (its LDS would not fit)
static uint32_t gemm_bm(uint32_t M, int prec) { return prec == 1 && M >= 512 ? 256u : 128u; }

static uint32_t ksplit_for(uint32_t tiles, uint32_t K) {
    const uint32_t units = K / 256;
    uint32_t best = 1;
    if (tiles >= 256) return 1;  // a full round already; partial traffic would cost more
    double best_cost = 1.0;
    for (uint32_t ks = 2; ks <= 8; ks++) {
        if (units % ks || units / ks < 4) continue;
        const double cost = (double)((tiles * ks + 255) / 256) / ks + 0.05;
        if (cost < best_cost - 1e-9) {
            best_cost = cost;
            best = ks;
        }
    }
    return best;
}

uint32_t gemm_out_tiles(uint32_t M, uint32_t N, int prec) {
    const uint32_t bm = gemm_bm(M, prec);
    return ((M + bm - 1) / bm) * ((N + GM_BN - 1) / GM_BN);
}

uint32_t gemm_ksplit(uint32_t M, uint32_t N, uint32_t K, int prec) {
    const uint32_t bm = gemm_bm(M, prec);
    return ksplit_for(((M + bm - 1) / bm) * ((N + GM_BN - 1) / GM_BN), K);
}

// scratch of the K-sliced form (at most 8 * M * N floats)
size_t gemm_work_bytes(uint32_t M, uint32_t N, uint32_t K, int prec) {
    const uint32_t ks = gemm_ksplit(M, N, K, prec);
    return ks > 1 ? (size_t)ks * M * N * sizeof(float) : 0;
}

using GemmFn = void (*)(GemmArgs);

// the kernel for weight types t0 (the first segments) and t1 (the rest)
template <uint32_t T0>
static GemmFn pick_gemm_t0(uint32_t t1, uint32_t nseg, int prec, uint32_t bm) {
#define LRS_GEMM_PICK(T1, MS)                                                             \
    return prec == 3 ? k_gemm<T0, T1, 3, 128, MS>                                         \
                     : bm == 256 ? k_gemm<T0, T1, 1, 256, MS> : k_gemm<T0, T1, 1, 128, MS>
    if (t1 == T0 && nseg == 1) { LRS_GEMM_PICK(T0, 1); }
    if (t1 == T0) { LRS_GEMM_PICK(T0, GM_MAX_SEG); }
    // a prompt block's q / k with a Q6_K v (the K-quant mixes)
    if constexpr (T0 == T_Q4_K || T0 == T_Q5_K)
        if (t1 == T_Q6_K) { LRS_GEMM_PICK(T_Q6_K, GM_MAX_SEG); }
#undef LRS_GEMM_PICK
    return nullptr;
}
static GemmFn pick_gemm(uint32_t t0, uint32_t t1, uint32_t nseg, int prec, uint32_t bm) {
    switch (t0) {
    case T_Q4_K: return pick_gemm_t0<T_Q4_K>(t1, nseg, prec, bm);
    case T_Q5_K: return pick_gemm_t0<T_Q5_K>(t1, nseg, prec, bm);
    case T_Q6_K: return pick_gemm_t0<T_Q6_K>(t1, nseg, prec, bm);
    case T_Q8_0: return pick_gemm_t0<T_Q8_0>(t1, nseg, prec, bm);
    default: return nullptr;
    }
}

bool gemm_segs_supported(const WeightView *w, uint32_t nseg) {
    if (nseg == 0 || nseg > (uint32_t)GM_MAX_SEG) return false;
    uint32_t nseg0 = 1;
    while (nseg0 < nseg && w[nseg0].type == w[0].type) nseg0++;
    for (uint32_t i = 0; i < nseg; i++) {
        if (w[i].n_in != w[0].n_in || !is_tiled(w[i].type)) return false;
        if (i >= nseg0 && w[i].type != w[nseg0].type) return false;  // at most two types, in two runs
    }
    return pick_gemm(w[0].type, w[nseg - 1].type, nseg, 3, 128) != nullptr;
}

hipError_t launch_gemm_segs(const WeightView *w, float *const *y, const uint32_t *ldy, uint32_t nseg,
                            const __bf16 *ahi, const __bf16 *alo, uint32_t M, int prec,
                            hipStream_t s, bool accum, float *work, uint32_t *ks_out) {
    if (M == 0 || nseg == 0 || nseg > (uint32_t)GM_MAX_SEG || (prec == 3 && !alo))
        return hipErrorInvalidValue;
    if (!gemm_segs_supported(w, nseg) || w[0].n_in % (4 * GM_BK)) return hipErrorInvalidValue;
    const uint32_t bm = gemm_bm(M, prec);
    GemmArgs g = {};
    g.ahi = ahi;
    g.alo = alo;
    g.nseg = nseg;
    g.nseg0 = 1;
    while (g.nseg0 < nseg && w[g.nseg0].type == w[0].type) g.nseg0++;
    uint32_t nt = 0;
    for (uint32_t i = 0; i < nseg; i++) {
        g.seg[i].q = w[i].q;
        g.seg[i].y = y[i];
        g.seg[i].N = w[i].n_out;
        g.seg[i].ldy = ldy[i];
        g.seg[i].nt0 = nt;
        nt += (w[i].n_out + GM_BN - 1) / GM_BN;
    }
    g.M = M;
    g.K = w[0].n_in;
    g.accum = accum ? 1u : 0u;
    g.nm = (M + bm - 1) / bm;
    g.nn = nt;
    // K slices write [M][N] partials of one weight: one-segment launches only
    g.ks = work && nseg == 1 ? ksplit_for(g.nm * g.nn, g.K) : 1;
    g.part = work;
    const GemmFn fn = pick_gemm(w[0].type, w[nseg - 1].type, nseg, prec, bm);
    if (!fn) return hipErrorNotSupported;
    const uint32_t grid = 8 * ((g.nm * g.nn * g.ks + 7) / 8);
    hipLaunchKernelGGL(fn, dim3(grid), dim3(512), 0, s, g);
    if (ks_out) {
        *ks_out = g.ks;  // the caller reduces the slices (launch_reduce_norm_rows)
    } else if (g.ks > 1) {
        const size_t n = (size_t)M * g.seg[0].N;
        hipLaunchKernelGGL(k_reduce_ks, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, work,
                           y[0], M, g.seg[0].N, ldy[0], g.ks, g.accum);
    }
    return hipGetLastError();
}

hipError_t launch_gemm(WeightView w, const __bf16 *ahi, const __bf16 *alo, float *y, uint32_t M,
                       uint32_t ldy, int prec, hipStream_t s, bool accum, float *work,
                       uint32_t *ks_out) {
    if (!is_tiled(w.type)) return hipErrorNotSupported;
    return launch_gemm_segs(&w, &y, &ldy, 1, ahi, alo, M, prec, s, accum, work, ks_out);
}

}  // namespace lrs
