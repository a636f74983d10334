/*
 * lrs_oracle.c — CPU restatement of llama.rs's reference CPU path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker and the CPU baseline); the
 * product library never links, loads or falls back to this file.  Built with
 * -ffp-contract=off -fno-fast-math so that every a*b+c rounds twice, like the
 * Rust reference.  Each function names the reference file:line it follows.
 */
#include "lrs_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* types.rs:30-78                                                            */
/* ------------------------------------------------------------------------- */
int64_t lrso_block_size(uint32_t type) {
    switch (type) {
    case LRSO_F32: case LRSO_F16: return 1;
    case LRSO_Q4_0: case LRSO_Q8_0: return 32;
    case LRSO_Q4_K: case LRSO_Q5_K: case LRSO_Q6_K: return 256;
    default: return -1;
    }
}

int64_t lrso_type_size(uint32_t type) {
    switch (type) {
    case LRSO_F32: return 4;
    case LRSO_F16: return 2;
    case LRSO_Q4_0: return 18;
    case LRSO_Q8_0: return 34;
    case LRSO_Q4_K: return 144;
    case LRSO_Q5_K: return 176;
    case LRSO_Q6_K: return 210;
    default: return -1;
    }
}

/* ------------------------------------------------------------------------- */
/* binary16 <-> binary32 (the `half` crate, Cargo.lock: half 2.7.1)          */
/* ------------------------------------------------------------------------- */
static float bits_f32(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static uint32_t f32_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

float lrso_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (exp == 0) {
        if (man == 0) return bits_f32(sign);
        /* subnormal: value = man * 2^-24, renormalise */
        int e = -1;
        do { man <<= 1; e++; } while ((man & 0x400u) == 0);
        man &= 0x3FFu;
        return bits_f32(sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13));
    }
    if (exp == 31) return bits_f32(sign | 0x7F800000u | (man << 13));
    return bits_f32(sign | ((exp - 15 + 127) << 23) | (man << 13));
}

uint16_t lrso_f32_to_f16(float f) {
    uint32_t x = f32_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFF) {
        if (man) return (uint16_t)(sign | 0x7E00u | (man >> 13));
        return (uint16_t)(sign | 0x7C00u);
    }
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

static float rd_f16(const uint8_t *p) {
    return lrso_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
}

/* ------------------------------------------------------------------------- */
/* dequant.rs                                                                */
/* ------------------------------------------------------------------------- */

/* dequant.rs:58-76: out = (q as f32) * d */
static void deq_q8_0(const uint8_t *b, float *out) {
    float d = rd_f16(b);
    for (int i = 0; i < 32; i++) out[i] = (float)(int8_t)b[2 + i] * d;
}

/* dequant.rs:77-99 */
static void deq_q4_0(const uint8_t *b, float *out) {
    float d = rd_f16(b);
    for (int j = 0; j < 16; j++) {
        uint8_t q = b[2 + j];
        int x0 = (int)(q & 0x0F) - 8;
        int x1 = (int)(q >> 4) - 8;
        out[j] = (float)x0 * d;
        out[j + 16] = (float)x1 * d;
    }
}

/* dequant.rs:101-110 */
static void scale_min_k4(int j, const uint8_t *s, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* dequant.rs:112-150: out = d1*q - m1f with d1 = d*sc, m1f = dmin*m */
static void deq_q4_k(const uint8_t *b, float *out) {
    float d_val = rd_f16(b);
    float min_val = rd_f16(b + 2);
    const uint8_t *scales = b + 4;
    const uint8_t *qs = b + 16;
    int is = 0;
    for (int js = 0; js < 256; js += 64) {
        uint8_t sc1, m1, sc2, m2;
        scale_min_k4(is, scales, &sc1, &m1);
        scale_min_k4(is + 1, scales, &sc2, &m2);
        float d1 = d_val * (float)sc1;
        float m1f = min_val * (float)m1;
        float d2 = d_val * (float)sc2;
        float m2f = min_val * (float)m2;
        for (int l = 0; l < 32; l++) {
            uint8_t q = qs[l];
            float t1 = d1 * (float)(q & 0xF);
            float t2 = d2 * (float)(q >> 4);
            out[js + l] = t1 - m1f;
            out[js + l + 32] = t2 - m2f;
        }
        qs += 32;
        is += 2;
    }
}

/* dequant.rs:157-203: Q4_K plus a 5th bit from qh */
static void deq_q5_k(const uint8_t *b, float *out) {
    float d_val = rd_f16(b);
    float min_val = rd_f16(b + 2);
    const uint8_t *scales = b + 4;
    const uint8_t *qh = b + 16;
    const uint8_t *qs = b + 48;
    int is = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int js = 0; js < 256; js += 64) {
        uint8_t sc1, m1, sc2, m2;
        scale_min_k4(is, scales, &sc1, &m1);
        scale_min_k4(is + 1, scales, &sc2, &m2);
        float d1 = d_val * (float)sc1;
        float m1f = min_val * (float)m1;
        float d2 = d_val * (float)sc2;
        float m2f = min_val * (float)m2;
        for (int l = 0; l < 32; l++) {
            uint8_t q = qs[l];
            uint8_t hi1 = (qh[l] & u1) ? 16 : 0;
            uint8_t hi2 = (qh[l] & u2) ? 16 : 0;
            float t1 = d1 * (float)((q & 0xF) + hi1);
            float t2 = d2 * (float)((q >> 4) + hi2);
            out[js + l] = t1 - m1f;
            out[js + l + 32] = t2 - m2f;
        }
        qs += 32;
        is += 2;
        u1 = (uint8_t)(u1 << 2);
        u2 = (uint8_t)(u2 << 2);
    }
}

/* dequant.rs:205-258: out = (d*s)*q, q = 6-bit - 32 */
static void deq_q6_k(const uint8_t *b, float *out) {
    const uint8_t *ql_full = b;
    const uint8_t *qh_full = b + 128;
    const uint8_t *sc_full = b + 192;
    float d_val = rd_f16(b + 208);
    for (int half = 0; half < 2; half++) {
        const uint8_t *ql = ql_full + 64 * half;
        const uint8_t *qh = qh_full + 32 * half;
        const int8_t *sc = (const int8_t *)(sc_full + 8 * half);
        float *o = out + 128 * half;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (int)(int8_t)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
            int q2 = (int)(int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)(int8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)(int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            float s0 = (float)sc[is];
            float s2 = (float)sc[is + 2];
            float s4 = (float)sc[is + 4];
            float s6 = (float)sc[is + 6];
            float ds0 = d_val * s0, ds2 = d_val * s2, ds4 = d_val * s4, ds6 = d_val * s6;
            o[l] = ds0 * (float)q1;
            o[l + 32] = ds2 * (float)q2;
            o[l + 64] = ds4 * (float)q3;
            o[l + 96] = ds6 * (float)q4;
        }
    }
}

/* dequant.rs:10-21 (dispatch) */
int64_t lrso_dequant(uint32_t type, const uint8_t *bytes, size_t len, float *out) {
    int64_t ts = lrso_type_size(type), bs = lrso_block_size(type);
    if (ts < 0) return -2;
    if (len % (size_t)ts != 0) return -1;
    size_t nb = len / (size_t)ts;
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = bytes + i * (size_t)ts;
        float *o = out + i * (size_t)bs;
        switch (type) {
        case LRSO_F32: { float v; memcpy(&v, b, 4); o[0] = v; break; }
        case LRSO_F16: o[0] = rd_f16(b); break;
        case LRSO_Q8_0: deq_q8_0(b, o); break;
        case LRSO_Q4_0: deq_q4_0(b, o); break;
        case LRSO_Q4_K: deq_q4_k(b, o); break;
        case LRSO_Q5_K: deq_q5_k(b, o); break;
        case LRSO_Q6_K: deq_q6_k(b, o); break;
        default: return -2;
        }
    }
    return (int64_t)(nb * (size_t)bs);
}

/* ------------------------------------------------------------------------- */
/* parallel-for over row chunks of 32 (ops.rs:76, 83-92)                     */
/* ------------------------------------------------------------------------- */
typedef void (*row_fn)(void *ctx, uint32_t row0, uint32_t row1);
typedef struct {
    row_fn fn; void *ctx; uint32_t n; uint32_t chunk;
    uint32_t next; pthread_mutex_t mu;
} par_job;

static void *par_worker(void *arg) {
    par_job *j = (par_job *)arg;
    for (;;) {
        pthread_mutex_lock(&j->mu);
        uint32_t r0 = j->next;
        j->next = r0 + j->chunk;
        pthread_mutex_unlock(&j->mu);
        if (r0 >= j->n) break;
        uint32_t r1 = r0 + j->chunk < j->n ? r0 + j->chunk : j->n;
        j->fn(j->ctx, r0, r1);
    }
    return NULL;
}

static void par_rows(row_fn fn, void *ctx, uint32_t n, int n_threads) {
    if (n_threads <= 1 || n < 64) { fn(ctx, 0, n); return; }
    par_job j; j.fn = fn; j.ctx = ctx; j.n = n; j.chunk = 32; j.next = 0;
    pthread_mutex_init(&j.mu, NULL);
    pthread_t th[256];
    int nt = n_threads > 256 ? 256 : n_threads;
    for (int t = 1; t < nt; t++) pthread_create(&th[t], NULL, par_worker, &j);
    par_worker(&j);
    for (int t = 1; t < nt; t++) pthread_join(th[t], NULL);
    pthread_mutex_destroy(&j.mu);
}

/* ------------------------------------------------------------------------- */
/* matvec: dequant + ops::matmul (ops.rs:78-101)                              */
/* ------------------------------------------------------------------------- */
typedef struct {
    uint32_t type; const uint8_t *w; size_t row_bytes; uint32_t n_in, n_out;
    const float *x; float *y; uint32_t cols;
} mv_ctx;

/* Each output is the sequential left fold of ops.rs:89-91.  Columns are taken
 * eight at a time with eight independent accumulators over an interleaved
 * copy of x (xt[i][c]): every accumulator still adds its products in index
 * order, so the results are bit-identical to one column at a time, with
 * eight times the instruction-level parallelism for batched prompts. */
typedef struct {
    uint32_t type; const uint8_t *w; size_t row_bytes; uint32_t n_in, n_out;
    const float *x; float *y; uint32_t cols;
    const float *xt;  /* [cols/8][n_in][8] */
} mv_ctx8;

static void mv_rows(void *p, uint32_t r0, uint32_t r1) {
    mv_ctx8 *c = (mv_ctx8 *)p;
    float *row = (float *)malloc(sizeof(float) * c->n_in);
    const uint32_t full = c->xt ? c->cols / 8 * 8 : 0;
    for (uint32_t j = r0; j < r1; j++) {
        lrso_dequant(c->type, c->w + (size_t)j * c->row_bytes, c->row_bytes, row);
        for (uint32_t t0 = 0; t0 < full; t0 += 8) {
            const float *xg = c->xt + (size_t)t0 * c->n_in;
            float acc[8];
            for (int k = 0; k < 8; k++) acc[k] = -0.0f;
            for (uint32_t i = 0; i < c->n_in; i++) {
                const float wi = row[i];
                const float *xi = xg + 8 * (size_t)i;
                for (int k = 0; k < 8; k++) {
                    const float p2 = wi * xi[k];
                    acc[k] = acc[k] + p2;
                }
            }
            for (int k = 0; k < 8; k++) c->y[(size_t)(t0 + k) * c->n_out + j] = acc[k];
        }
        for (uint32_t t = full; t < c->cols; t++) {
            const float *xr = c->x + (size_t)t * c->n_in;
            float acc = -0.0f; /* f32 Iterator::sum starts from -0.0 */
            for (uint32_t i = 0; i < c->n_in; i++) {
                float p2 = row[i] * xr[i];
                acc = acc + p2;
            }
            c->y[(size_t)t * c->n_out + j] = acc;
        }
    }
    free(row);
}

int lrso_matvec(uint32_t type, const uint8_t *w, size_t w_len, uint32_t n_in,
                uint32_t n_out, const float *x, float *y, uint32_t cols,
                int n_threads) {
    int64_t bs = lrso_block_size(type), ts = lrso_type_size(type);
    if (bs < 0) return -2;
    if (n_in % (uint32_t)bs != 0) return -1;
    size_t row_bytes = (size_t)(n_in / (uint32_t)bs) * (size_t)ts;
    if (w_len != row_bytes * n_out) return -1;
    float *xt = NULL;
    if (cols >= 8) {
        const uint32_t groups = cols / 8;
        xt = (float *)malloc(sizeof(float) * (size_t)groups * 8 * n_in);
        if (!xt) return -3;
        for (uint32_t g = 0; g < groups; g++)
            for (uint32_t k = 0; k < 8; k++) {
                const float *xr = x + (size_t)(8 * g + k) * n_in;
                float *dst = xt + (size_t)g * 8 * n_in + k;
                for (uint32_t i = 0; i < n_in; i++) dst[8 * (size_t)i] = xr[i];
            }
    }
    mv_ctx8 c = {type, w, row_bytes, n_in, n_out, x, y, cols, xt};
    par_rows(mv_rows, &c, n_out, n_threads);
    free(xt);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* int8-activation path of Model::forward for Q8_0 weights                   */
/* ------------------------------------------------------------------------- */
/* quantize_q8_0 (ops.rs:343-368: scalar, f32::round = half away from zero)
 * and quantize_q8_0_avx2 (ops.rs:284-340: cvtps2dq under the default MXCSR =
 * half to even; the saturating packs clamp like the scalar clamp): per 32
 * elements d = max|x| / 127, q = round(x * (1 / d)) in [-128, 127], d stored
 * as f16 (the quotients use the f32 d, not its f16 rounding).  out: n / 32
 * GGUF Q8_0 blocks of 34 bytes. */
int lrso_quantize_q8_0(const float *x, uint32_t n, int half_even, uint8_t *out) {
    if (n % 32) return -1;
    for (uint32_t b = 0; b < n / 32; b++) {
        const float *blk = x + 32 * (size_t)b;
        float m = 0.0f; /* fold(0.0, f32::max) over |x| */
        for (int i = 0; i < 32; i++) {
            const float a = fabsf(blk[i]);
            m = a > m ? a : m;
        }
        const float d = m > 0.0f ? m / 127.0f : 0.0f;
        const float di = d > 0.0f ? 1.0f / d : 0.0f;
        const uint16_t h = lrso_f32_to_f16(d);
        uint8_t *o = out + 34 * (size_t)b;
        o[0] = (uint8_t)(h & 0xFF);
        o[1] = (uint8_t)(h >> 8);
        for (int i = 0; i < 32; i++) {
            const float t = blk[i] * di;
            float r = half_even ? nearbyintf(t) : roundf(t);
            if (r < -128.0f) r = -128.0f;
            if (r > 127.0f) r = 127.0f;
            o[2 + i] = (uint8_t)(int8_t)(int)r;
        }
    }
    return 0;
}

/* matmul_q8_0_actq (ops.rs:728-886) for one column with the scalar block dot
 * q8_0_q8_0_dot_scalar (ops.rs:704-724): acc += dw * dx * (float)sum(qw * qx)
 * block by block from 0.0; x is quantized first (quantize_q8_0_split,
 * ops.rs:371-384). */
typedef struct {
    const uint8_t *w, *xq; uint32_t nb; float *y;
} actq_ctx;

static void actq_rows(void *p, uint32_t r0, uint32_t r1) {
    const actq_ctx *c = (const actq_ctx *)p;
    for (uint32_t r = r0; r < r1; r++) {
        const uint8_t *wr = c->w + (size_t)r * c->nb * 34;
        float acc = 0.0f;
        for (uint32_t b = 0; b < c->nb; b++) {
            const uint8_t *bw = wr + 34 * (size_t)b, *bx = c->xq + 34 * (size_t)b;
            const float dw = lrso_f16_to_f32((uint16_t)(bw[0] | (bw[1] << 8)));
            const float dx = lrso_f16_to_f32((uint16_t)(bx[0] | (bx[1] << 8)));
            int32_t dot = 0;
            for (int i = 0; i < 32; i++) dot += (int32_t)(int8_t)bw[2 + i] * (int32_t)(int8_t)bx[2 + i];
            const float s = dw * dx;
            acc = acc + s * (float)dot;
        }
        c->y[r] = acc;
    }
}

int lrso_matvec_q8_0_actq_mt(const uint8_t *w, size_t w_len, uint32_t n_in, uint32_t n_out,
                             const float *x, int half_even, float *y, int n_threads) {
    if (n_in % 32) return -1;
    const uint32_t nb = n_in / 32;
    if (w_len != (size_t)nb * 34 * n_out) return -1;
    uint8_t *xq = (uint8_t *)malloc((size_t)nb * 34 + 1);
    if (!xq) return -3;
    lrso_quantize_q8_0(x, n_in, half_even, xq);
    actq_ctx c = {w, xq, nb, y};
    par_rows(actq_rows, &c, n_out, n_threads);
    free(xq);
    return 0;
}

int lrso_matvec_q8_0_actq(const uint8_t *w, size_t w_len, uint32_t n_in, uint32_t n_out,
                          const float *x, int half_even, float *y) {
    return lrso_matvec_q8_0_actq_mt(w, w_len, n_in, n_out, x, half_even, y, 1);
}

/* ------------------------------------------------------------------------- */
/* synthetic blocks                                                          */
/* ------------------------------------------------------------------------- */
static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

uint64_t lrso_hash(uint64_t seed, uint64_t block, uint32_t j) {
    return mix64(seed * 0x9E3779B97F4A7C15ULL + block * 0xD1B54A32D192ED03ULL +
                 (uint64_t)j * 0x8CB92BA72F3D8DD7ULL + 0x2545F4914F6CDD1DULL);
}

/* u in [0,1) with 24 bits; lo + (hi-lo)*u in f32, two roundings */
static float h_unif(uint64_t h, float lo, float hi) {
    float u = (float)(uint32_t)(h >> 40) * (1.0f / 16777216.0f);
    float span = hi - lo;
    float t = span * u;
    return lo + t;
}
static uint8_t h_byte(uint64_t h) { return (uint8_t)(h >> 56); }
static void put_f16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)(v & 0xFF); p[1] = (uint8_t)(v >> 8); }

/* 6-bit (sc, m) pairs -> 12 packed bytes, the inverse of dequant.rs:101-110 */
static void pack_scale_min_k4(const uint8_t sc[8], const uint8_t m[8], uint8_t s[12]) {
    for (int j = 0; j < 4; j++) {
        s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
    }
}

static void gen_block(uint32_t type, uint64_t seed, uint64_t blk, int mode,
                      float d_lo, float d_hi, uint8_t *o) {
    switch (type) {
    case LRSO_Q8_0: {
        put_f16(o, lrso_f32_to_f16(h_unif(lrso_hash(seed, blk, 0), d_lo, d_hi)));
        for (uint32_t i = 0; i < 32; i++) {
            uint64_t h = lrso_hash(seed, blk, 1 + i);
            int q = (int)(((h >> 32) * 255ULL) >> 32) - 127;
            o[2 + i] = (uint8_t)(int8_t)q;
        }
        break;
    }
    case LRSO_Q4_0: {
        put_f16(o, lrso_f32_to_f16(h_unif(lrso_hash(seed, blk, 0), d_lo, d_hi)));
        for (uint32_t i = 2; i < 18; i++) o[i] = h_byte(lrso_hash(seed, blk, i));
        break;
    }
    case LRSO_Q4_K:
    case LRSO_Q5_K: {
        uint32_t tsz = type == LRSO_Q4_K ? 144 : 176;
        float d = lrso_f16_to_f32(lrso_f32_to_f16(h_unif(lrso_hash(seed, blk, 0), d_lo, d_hi)));
        put_f16(o, lrso_f32_to_f16(d));
        if (mode == 1) {
            float mult = type == LRSO_Q4_K ? 7.5f : 15.5f;
            put_f16(o + 2, lrso_f32_to_f16(d * mult));
            uint8_t sc[8];
            for (uint32_t j = 0; j < 8; j++) sc[j] = h_byte(lrso_hash(seed, blk, 4 + j)) & 63;
            pack_scale_min_k4(sc, sc, o + 4);
        } else {
            put_f16(o + 2, lrso_f32_to_f16(h_unif(lrso_hash(seed, blk, 1), d_lo, d_hi)));
            for (uint32_t i = 4; i < 16; i++) o[i] = h_byte(lrso_hash(seed, blk, i));
        }
        for (uint32_t i = 16; i < tsz; i++) o[i] = h_byte(lrso_hash(seed, blk, i));
        break;
    }
    case LRSO_Q6_K: {
        for (uint32_t i = 0; i < 192; i++) o[i] = h_byte(lrso_hash(seed, blk, i));
        for (uint32_t i = 192; i < 208; i++) {
            int s = (int)(lrso_hash(seed, blk, i) >> 57) - 64;
            o[i] = (uint8_t)(int8_t)s;
        }
        put_f16(o + 208, lrso_f32_to_f16(h_unif(lrso_hash(seed, blk, 208), d_lo, d_hi)));
        break;
    }
    default: break;
    }
}

int lrso_gen_blocks(uint32_t type, uint64_t seed, uint64_t block0,
                    uint64_t n_blocks, int mode, float d_lo, float d_hi,
                    uint8_t *out) {
    int64_t ts = lrso_type_size(type);
    if (ts < 0 || lrso_block_size(type) == 1) return -2;
    for (uint64_t b = 0; b < n_blocks; b++)
        gen_block(type, seed, block0 + b, mode, d_lo, d_hi, out + b * (uint64_t)ts);
    return 0;
}

void lrso_gen_uniform(uint64_t seed, uint64_t n, float lo, float hi, float *out) {
    for (uint64_t i = 0; i < n; i++) out[i] = h_unif(lrso_hash(seed, i, 0), lo, hi);
}

void lrso_gen_normal(uint64_t seed, uint64_t n, float *out) {
    for (uint64_t i = 0; i < n; i += 2) {
        uint64_t h1 = lrso_hash(seed, i / 2, 1), h2 = lrso_hash(seed, i / 2, 2);
        double u1 = ((double)(h1 >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        double u2 = (double)(h2 >> 11) * (1.0 / 9007199254740992.0);
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(r * cos(6.283185307179586 * u2));
        if (i + 1 < n) out[i + 1] = (float)(r * sin(6.283185307179586 * u2));
    }
}

/* ------------------------------------------------------------------------- */
/* ops.rs / attention.rs                                                     */
/* ------------------------------------------------------------------------- */
void lrso_rmsnorm_scale(const float *x, const float *w, uint32_t n_tok,
                        uint32_t dim, float eps, float *out) {
    for (uint32_t t = 0; t < n_tok; t++) {
        const float *r = x + (size_t)t * dim;
        float *o = out + (size_t)t * dim;
        float ss = -0.0f;
        for (uint32_t i = 0; i < dim; i++) { float sq = r[i] * r[i]; ss = ss + sq; }
        float mean = ss / (float)dim;
        float scale = 1.0f / sqrtf(mean + eps);
        for (uint32_t i = 0; i < dim; i++) { float a = r[i] * scale; o[i] = a * w[i]; }
    }
}

void lrso_freq_table(float freq_base, uint32_t rope_dim, float *out) {
    for (uint32_t i = 0; i < rope_dim / 2; i++) {
        float e = -2.0f * (float)i;
        e = e / (float)rope_dim;
        out[i] = powf(freq_base, e);
    }
}

void lrso_rope_norm(float *x, uint32_t n_tok, uint32_t n_head, uint32_t head_dim,
                    uint32_t rope_dim, const float *freq, uint32_t pos0) {
    for (uint32_t t = 0; t < n_tok; t++) {
        float pos = (float)(pos0 + t);
        for (uint32_t h = 0; h < n_head; h++) {
            float *b = x + ((size_t)t * n_head + h) * head_dim;
            for (uint32_t i = 0; i < rope_dim / 2; i++) {
                float theta = pos * freq[i];
                float s = sinf(theta), c = cosf(theta);
                float a = b[2 * i], bb = b[2 * i + 1];
                float ac = a * c, bs = bb * s, as = a * s, bc = bb * c;
                b[2 * i] = ac - bs;
                b[2 * i + 1] = as + bc;
            }
        }
    }
}

float lrso_silu(float x) { return x * lrso_sigmoid(x); }

void lrso_swiglu(const float *g, const float *u, uint32_t n, float *out) {
    for (uint32_t i = 0; i < n; i++) {
        /* ops.rs:978-981: x / (1 + exp(-x)) */
        float den = 1.0f + expf(-g[i]);
        float s = g[i] / den;
        out[i] = s * u[i];
    }
}

void lrso_softmax(float *z, uint32_t n) {
    float mx = -INFINITY;
    for (uint32_t i = 0; i < n; i++) mx = fmaxf(mx, z[i]);
    float sum = 0.0f;
    for (uint32_t i = 0; i < n; i++) { z[i] = expf(z[i] - mx); sum += z[i]; }
    if (sum > 0.0f)
        for (uint32_t i = 0; i < n; i++) z[i] /= sum;
}

uint32_t lrso_argmax(const float *v, uint32_t n) {
    uint32_t best = 0;
    float bv = -INFINITY;
    for (uint32_t i = 0; i < n; i++)
        if (v[i] > bv) { bv = v[i]; best = i; }
    return best;
}

void lrso_attention(const float *q, const float *k_cache, const float *v_cache,
                    uint32_t n_tok, uint32_t pos0, uint32_t n_head,
                    uint32_t n_head_kv, uint32_t head_dim, float *out) {
    uint32_t n_embd = n_head * head_dim, kv_dim = n_head_kv * head_dim;
    uint32_t n_rep = n_head / n_head_kv;
    float scale = 1.0f / sqrtf((float)head_dim);
    float *scores = (float *)malloc(sizeof(float) * (pos0 + n_tok));
    memset(out, 0, sizeof(float) * (size_t)n_tok * n_embd);
    for (uint32_t t = 0; t < n_tok; t++) {
        uint32_t abs_pos = pos0 + t;
        for (uint32_t h = 0; h < n_head; h++) {
            uint32_t kv_h = h / n_rep;
            const float *qv = q + ((size_t)t * n_head + h) * head_dim;
            for (uint32_t j = 0; j <= abs_pos; j++) {
                const float *kv = k_cache + (size_t)j * kv_dim + (size_t)kv_h * head_dim;
                float dot = -0.0f;
                for (uint32_t d = 0; d < head_dim; d++) { float p = qv[d] * kv[d]; dot = dot + p; }
                scores[j] = dot * scale;
            }
            lrso_softmax(scores, abs_pos + 1);
            float *ov = out + ((size_t)t * n_head + h) * head_dim;
            for (uint32_t j = 0; j <= abs_pos; j++) {
                const float *vv = v_cache + (size_t)j * kv_dim + (size_t)kv_h * head_dim;
                for (uint32_t d = 0; d < head_dim; d++) { float p = scores[j] * vv[d]; ov[d] = ov[d] + p; }
            }
        }
    }
    free(scores);
}

/* ------------------------------------------------------------------------- */
/* model forward (model.rs:99-266)                                           */
/* ------------------------------------------------------------------------- */
struct lrso_model {
    lrso_config c;
    lrso_tensor embd, onorm, out;
    lrso_layer *layers;
    float *freq;
    float *kc, *vc;     /* [n_layer][ctx][kv_dim] */
    uint32_t len;
    int kv_f16, n_threads;
    int q8_actq; /* Q8_0 weights through quantize_q8_0_split + matmul_q8_0_actq */
};

static int tensor_ok(const lrso_tensor *t, uint32_t n_in, uint32_t n_out) {
    int64_t bs = lrso_block_size(t->type), ts = lrso_type_size(t->type);
    if (bs < 0 || !t->bytes) return 0;
    if (n_in % (uint32_t)bs) return 0;
    return t->len == (size_t)(n_in / (uint32_t)bs) * (size_t)ts * n_out;
}

lrso_model *lrso_model_create(const lrso_config *cfg, const lrso_tensor *token_embd,
                              const lrso_layer *layers, const lrso_tensor *output_norm,
                              const lrso_tensor *output, int kv_f16, int n_threads) {
    const lrso_config *c = cfg;
    uint32_t kv_dim = c->n_head_kv * c->head_dim;
    if (c->n_head % c->n_head_kv) return NULL;
    if (!tensor_ok(token_embd, c->n_embd, c->vocab)) return NULL;
    if (!tensor_ok(output, c->n_embd, c->vocab)) return NULL;
    if (!tensor_ok(output_norm, c->n_embd, 1)) return NULL;
    for (uint32_t l = 0; l < c->n_layer; l++) {
        const lrso_layer *L = &layers[l];
        if (!tensor_ok(&L->attn_q, c->n_embd, c->n_head * c->head_dim) ||
            !tensor_ok(&L->attn_k, c->n_embd, kv_dim) ||
            !tensor_ok(&L->attn_v, c->n_embd, kv_dim) ||
            !tensor_ok(&L->attn_output, c->n_head * c->head_dim, c->n_embd) ||
            !tensor_ok(&L->ffn_gate, c->n_embd, c->n_ff) ||
            !tensor_ok(&L->ffn_up, c->n_embd, c->n_ff) ||
            !tensor_ok(&L->ffn_down, c->n_ff, c->n_embd) ||
            !tensor_ok(&L->attn_norm, c->n_embd, 1) ||
            !tensor_ok(&L->ffn_norm, c->n_embd, 1))
            return NULL;
    }
    lrso_model *m = (lrso_model *)calloc(1, sizeof(lrso_model));
    m->c = *c;
    m->embd = *token_embd; m->onorm = *output_norm; m->out = *output;
    m->layers = (lrso_layer *)malloc(sizeof(lrso_layer) * c->n_layer);
    memcpy(m->layers, layers, sizeof(lrso_layer) * c->n_layer);
    m->freq = (float *)malloc(sizeof(float) * (c->rope_dim / 2 + 1));
    lrso_freq_table(c->freq_base, c->rope_dim, m->freq);
    size_t cap = (size_t)c->n_layer * c->ctx * kv_dim;
    m->kc = (float *)calloc(cap, sizeof(float));
    m->vc = (float *)calloc(cap, sizeof(float));
    m->kv_f16 = kv_f16;
    m->n_threads = n_threads;
    m->q8_actq = 1;
    return m;
}

void lrso_model_set_q8_actq(lrso_model *m, int on) { m->q8_actq = on; }

static float *tensor_f32(const lrso_tensor *t, uint32_t n) {
    float *o = (float *)malloc(sizeof(float) * n);
    lrso_dequant(t->type, t->bytes, t->len, o);
    return o;
}

/* RawTensor::matmul_into (weights.rs:109-124): a Q8_0 weight whose n_in is a
 * multiple of 32 takes the int8-activation path, each token's activation
 * rounded by quantize_q8_0_split (ops.rs:371-384; on x86 with AVX2, the
 * half-to-even quantize_q8_0_avx2, ops.rs:284-340 and :347-352) and
 * multiplied by matmul_q8_0_actq (ops.rs:728-886); every other weight is
 * dequantized to f32 and multiplied by ops::matmul (ops.rs:78-101). */
static void mm(lrso_model *m, const lrso_tensor *t, const float *x, uint32_t n_in,
               uint32_t n_out, uint32_t n_tok, float *y) {
    if (m->q8_actq && t->type == LRSO_Q8_0 && n_in % 32 == 0) {
        for (uint32_t k = 0; k < n_tok; k++)
            lrso_matvec_q8_0_actq_mt(t->bytes, t->len, n_in, n_out, x + (size_t)k * n_in, 1,
                                     y + (size_t)k * n_out, m->n_threads);
        return;
    }
    lrso_matvec(t->type, t->bytes, t->len, n_in, n_out, x, y, n_tok, m->n_threads);
}

static void add_bias(float *x, const lrso_tensor *b, uint32_t dim, uint32_t n_tok) {
    if (!b->bytes) return;
    float *bv = tensor_f32(b, dim);
    for (uint32_t t = 0; t < n_tok; t++)
        for (uint32_t i = 0; i < dim; i++) x[(size_t)t * dim + i] += bv[i];
    free(bv);
}

static int forward_impl(lrso_model *m, const uint32_t *tokens, uint32_t n_tok,
                        uint32_t n_layers_run, float *logits) {
    const lrso_config *c = &m->c;
    uint32_t E = c->n_embd, QD = c->n_head * c->head_dim, KV = c->n_head_kv * c->head_dim;
    uint32_t pos0 = m->len;
    if (n_tok == 0) return -1;
    if (pos0 + n_tok > c->ctx) return -3;
    for (uint32_t t = 0; t < n_tok; t++)
        if (tokens[t] >= c->vocab) return -4;
    /* embedding_lookup on the dequantized table (ops.rs:11-26, model.rs:109-110) */
    size_t row_bytes = m->embd.len / c->vocab;
    float *x = (float *)malloc(sizeof(float) * (size_t)n_tok * E);
    for (uint32_t t = 0; t < n_tok; t++)
        lrso_dequant(m->embd.type, m->embd.bytes + (size_t)tokens[t] * row_bytes, row_bytes,
                     x + (size_t)t * E);
    float *h = (float *)malloc(sizeof(float) * (size_t)n_tok * E);
    float *q = (float *)malloc(sizeof(float) * (size_t)n_tok * QD);
    float *k = (float *)malloc(sizeof(float) * (size_t)n_tok * KV);
    float *v = (float *)malloc(sizeof(float) * (size_t)n_tok * KV);
    float *att = (float *)malloc(sizeof(float) * (size_t)n_tok * QD);
    float *o = (float *)malloc(sizeof(float) * (size_t)n_tok * E);
    float *g = (float *)malloc(sizeof(float) * (size_t)n_tok * c->n_ff);
    float *u = (float *)malloc(sizeof(float) * (size_t)n_tok * c->n_ff);
    uint32_t nl = n_layers_run < c->n_layer ? n_layers_run : c->n_layer;
    for (uint32_t l = 0; l < nl; l++) {
        lrso_layer *L = &m->layers[l];
        float *an = tensor_f32(&L->attn_norm, E);
        float *fn = tensor_f32(&L->ffn_norm, E);
        lrso_rmsnorm_scale(x, an, n_tok, E, c->rms_eps, h);
        mm(m, &L->attn_q, h, E, QD, n_tok, q);
        mm(m, &L->attn_k, h, E, KV, n_tok, k);
        mm(m, &L->attn_v, h, E, KV, n_tok, v);
        add_bias(q, &L->bq, QD, n_tok);
        add_bias(k, &L->bk, KV, n_tok);
        add_bias(v, &L->bv, KV, n_tok);
        lrso_rope_norm(q, n_tok, c->n_head, c->head_dim, c->rope_dim, m->freq, pos0);
        lrso_rope_norm(k, n_tok, c->n_head_kv, c->head_dim, c->rope_dim, m->freq, pos0);
        /* KvCache::append (attention.rs:36-47) */
        float *kl = m->kc + (size_t)l * c->ctx * KV, *vl = m->vc + (size_t)l * c->ctx * KV;
        for (size_t i = 0; i < (size_t)n_tok * KV; i++) {
            float kk = k[i], vv = v[i];
            if (m->kv_f16) {
                kk = lrso_f16_to_f32(lrso_f32_to_f16(kk));
                vv = lrso_f16_to_f32(lrso_f32_to_f16(vv));
            }
            kl[(size_t)pos0 * KV + i] = kk;
            vl[(size_t)pos0 * KV + i] = vv;
        }
        lrso_attention(q, kl, vl, n_tok, pos0, c->n_head, c->n_head_kv, c->head_dim, att);
        mm(m, &L->attn_output, att, QD, E, n_tok, o);
        for (size_t i = 0; i < (size_t)n_tok * E; i++) x[i] += o[i];
        lrso_rmsnorm_scale(x, fn, n_tok, E, c->rms_eps, h);
        mm(m, &L->ffn_gate, h, E, c->n_ff, n_tok, g);
        mm(m, &L->ffn_up, h, E, c->n_ff, n_tok, u);
        lrso_swiglu(g, u, n_tok * c->n_ff, g);
        mm(m, &L->ffn_down, g, c->n_ff, E, n_tok, o);
        for (size_t i = 0; i < (size_t)n_tok * E; i++) x[i] += o[i];
        free(an); free(fn);
    }
    int rc = 0;
    if (logits) {
        /* cache.advance, final norm, head on the last token (model.rs:254-265) */
        float *on = tensor_f32(&m->onorm, E);
        lrso_rmsnorm_scale(x, on, n_tok, E, c->rms_eps, h);
        mm(m, &m->out, h + (size_t)(n_tok - 1) * E, E, c->vocab, 1, logits);
        free(on);
    }
    if (n_layers_run >= c->n_layer) m->len += n_tok;
    free(x); free(h); free(q); free(k); free(v); free(att); free(o); free(g); free(u);
    return rc;
}

int lrso_model_forward(lrso_model *m, const uint32_t *tokens, uint32_t n_tok,
                       float *logits) {
    return forward_impl(m, tokens, n_tok, m->c.n_layer, logits);
}

int lrso_model_forward_partial(lrso_model *m, const uint32_t *tokens, uint32_t n_tok,
                               uint32_t n_layers_run) {
    return forward_impl(m, tokens, n_tok, n_layers_run, NULL);
}

uint32_t lrso_model_len(const lrso_model *m) { return m->len; }
void lrso_model_reset(lrso_model *m) { m->len = 0; }
void lrso_model_destroy(lrso_model *m) {
    if (!m) return;
    free(m->layers); free(m->freq); free(m->kc); free(m->vc); free(m);
}

/* ------------------------------------------------------------------------- */
/* delta_net.rs:13-131                                                        */
/* ------------------------------------------------------------------------- */
float lrso_softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }
float lrso_sigmoid(float x) { float den = 1.0f + expf(-x); return 1.0f / den; }

void lrso_l2_norm_rows(float *x, uint32_t n_rows, uint32_t dim, float eps) {
    for (uint32_t r = 0; r < n_rows; r++) {
        float *row = x + (size_t)r * dim;
        float s = -0.0f;
        for (uint32_t i = 0; i < dim; i++) { float sq = row[i] * row[i]; s = s + sq; }
        float inv = 1.0f / sqrtf(s + eps);
        for (uint32_t i = 0; i < dim; i++) row[i] *= inv;
    }
}

void lrso_conv1d_step(float *state, const float *x, const float *w,
                      uint32_t channels, uint32_t d_conv, float *out) {
    uint32_t ps = d_conv - 1;
    for (uint32_t c = 0; c < channels; c++) {
        float *win = state + (size_t)c * ps;
        const float *ker = w + (size_t)c * d_conv;
        float acc = -0.0f;
        for (uint32_t t = 0; t < ps; t++) { float p = win[t] * ker[t]; acc = acc + p; }
        float last = x[c] * ker[d_conv - 1];
        acc = acc + last;
        out[c] = acc;
        if (ps > 0) {
            memmove(win, win + 1, sizeof(float) * (ps - 1));
            win[ps - 1] = x[c];
        }
    }
}

void lrso_delta_net_step(float *state, const float *q, const float *k,
                         const float *v, float g, float beta, uint32_t d,
                         float *out) {
    float decay = expf(g);
    for (size_t i = 0; i < (size_t)d * d; i++) state[i] *= decay;
    float *delta = (float *)malloc(sizeof(float) * d);
    for (uint32_t j = 0; j < d; j++) {
        const float *row = state + (size_t)j * d;
        float pred = -0.0f;
        for (uint32_t i = 0; i < d; i++) { float p = row[i] * k[i]; pred = pred + p; }
        float diff = v[j] - pred;
        delta[j] = diff * beta;
    }
    for (uint32_t j = 0; j < d; j++) {
        float *row = state + (size_t)j * d;
        for (uint32_t i = 0; i < d; i++) { float p = delta[j] * k[i]; row[i] = row[i] + p; }
    }
    float esc = 1.0f / sqrtf((float)d);
    for (uint32_t j = 0; j < d; j++) {
        const float *row = state + (size_t)j * d;
        float s = -0.0f;
        for (uint32_t i = 0; i < d; i++) { float p = row[i] * q[i]; s = s + p; }
        out[j] = s * esc;
    }
    free(delta);
}

/* ------------------------------------------------------------------------- */
/* hybrid attention + gated delta-net model (qwen35).  No CPU forward exists  */
/* in the reference (runner.rs:164): this follows the GPU plan's op order,    */
/* resident_forward.rs:3826-4103 and plano_delta :2252-2470.                  */
/* ------------------------------------------------------------------------- */
struct lrso_hybrid {
    lrso_hybrid_config c;
    lrso_tensor embd, onorm, out;
    lrso_hybrid_layer *layers;
    float *freq;
    float *kc, *vc;   /* [n_attn_layers][ctx][kv_dim] */
    float *state;     /* [n_dn_layers][v_heads][d][d], state[j*d+i] = S[i][j] */
    float *win;       /* [n_dn_layers][conv_dim][d_conv-1] */
    uint32_t *slot;   /* layer -> index among the layers of its kind */
    uint32_t n_attn, n_dn, len;
    int kv_f16, n_threads;
};

static int hy_full(const lrso_hybrid_config *c, uint32_t l) {
    /* LlamaConfig::eh_linear (config.rs:25-35) */
    return (l + 1) % c->full_attn_interval == 0;
}

static uint32_t hy_conv_dim(const lrso_hybrid_config *c) {
    return 2 * c->dn_k_heads * c->dn_state + c->dn_v_heads * c->dn_state;
}

lrso_hybrid *lrso_hybrid_create(const lrso_hybrid_config *cfg, const lrso_tensor *token_embd,
                                const lrso_hybrid_layer *layers,
                                const lrso_tensor *output_norm, const lrso_tensor *output,
                                int kv_f16, int n_threads) {
    const lrso_hybrid_config *c = cfg;
    const lrso_config *b = &c->base;
    if (!c->full_attn_interval || !c->dn_k_heads || !c->dn_v_heads || !c->dn_state ||
        c->dn_conv < 1 || c->dn_v_heads % c->dn_k_heads || b->n_head % b->n_head_kv)
        return NULL;
    const uint32_t E = b->n_embd, HD = b->head_dim, QD = b->n_head * HD, KV = b->n_head_kv * HD;
    const uint32_t d = c->dn_state, KD = c->dn_k_heads * d, VD = c->dn_v_heads * d;
    const uint32_t CD = hy_conv_dim(c);
    if (!tensor_ok(token_embd, E, b->vocab) || !tensor_ok(output, E, b->vocab) ||
        !tensor_ok(output_norm, E, 1))
        return NULL;
    (void)KD;
    for (uint32_t l = 0; l < b->n_layer; l++) {
        const lrso_hybrid_layer *L = &layers[l];
        if (!tensor_ok(&L->attn_norm, E, 1) || !tensor_ok(&L->post_norm, E, 1) ||
            !tensor_ok(&L->ffn_gate, E, b->n_ff) || !tensor_ok(&L->ffn_up, E, b->n_ff) ||
            !tensor_ok(&L->ffn_down, b->n_ff, E))
            return NULL;
        if (hy_full(c, l)) {
            if (!tensor_ok(&L->attn_q, E, 2 * QD) || !tensor_ok(&L->attn_k, E, KV) ||
                !tensor_ok(&L->attn_v, E, KV) || !tensor_ok(&L->attn_output, QD, E) ||
                !tensor_ok(&L->q_norm, HD, 1) || !tensor_ok(&L->k_norm, HD, 1))
                return NULL;
        } else {
            if (!tensor_ok(&L->ssm_qkv, E, CD) || !tensor_ok(&L->ssm_gate, E, VD) ||
                !tensor_ok(&L->ssm_out, VD, E) || !tensor_ok(&L->ssm_alpha, E, c->dn_v_heads) ||
                !tensor_ok(&L->ssm_beta, E, c->dn_v_heads) ||
                !tensor_ok(&L->ssm_a, c->dn_v_heads, 1) || !tensor_ok(&L->ssm_dt, c->dn_v_heads, 1) ||
                !tensor_ok(&L->ssm_conv, c->dn_conv, CD) || !tensor_ok(&L->ssm_norm, d, 1))
                return NULL;
        }
    }
    lrso_hybrid *m = (lrso_hybrid *)calloc(1, sizeof(lrso_hybrid));
    m->c = *c;
    m->embd = *token_embd; m->onorm = *output_norm; m->out = *output;
    m->layers = (lrso_hybrid_layer *)malloc(sizeof(lrso_hybrid_layer) * b->n_layer);
    memcpy(m->layers, layers, sizeof(lrso_hybrid_layer) * b->n_layer);
    m->slot = (uint32_t *)malloc(sizeof(uint32_t) * b->n_layer);
    for (uint32_t l = 0; l < b->n_layer; l++)
        m->slot[l] = hy_full(c, l) ? m->n_attn++ : m->n_dn++;
    /* freq[i] = 1 / base^(2i/rope_dim) (gpu.rs:540-547) */
    m->freq = (float *)malloc(sizeof(float) * (b->rope_dim / 2 + 1));
    for (uint32_t i = 0; i < b->rope_dim / 2; i++) {
        float ex = (float)(2 * i) / (float)b->rope_dim;
        m->freq[i] = 1.0f / powf(b->freq_base, ex);
    }
    m->kc = (float *)calloc((size_t)m->n_attn * b->ctx * KV + 1, sizeof(float));
    m->vc = (float *)calloc((size_t)m->n_attn * b->ctx * KV + 1, sizeof(float));
    m->state = (float *)calloc((size_t)m->n_dn * c->dn_v_heads * d * d + 1, sizeof(float));
    m->win = (float *)calloc((size_t)m->n_dn * CD * (c->dn_conv - 1) + 1, sizeof(float));
    m->kv_f16 = kv_f16;
    m->n_threads = n_threads;
    return m;
}

/* RMSNorm of one head in place, dn_norm.comp mode 2: x * (1/sqrt(mean(x^2)+eps)) * w */
static void hy_head_rms(float *x, uint32_t dim, const float *w, float eps) {
    float ss = -0.0f;
    for (uint32_t i = 0; i < dim; i++) { float sq = x[i] * x[i]; ss = ss + sq; }
    float s = 1.0f / sqrtf(ss / (float)dim + eps);
    for (uint32_t i = 0; i < dim; i++) { float v = x[i] * s; x[i] = v * w[i]; }
}

/* adjacent-pair RoPE of one head (rope.comp / ops.rs:952-975) */
static void hy_rope_head(float *b, uint32_t rope_dim, const float *freq, uint32_t pos) {
    for (uint32_t i = 0; i < rope_dim / 2; i++) {
        float theta = (float)pos * freq[i];
        float s = sinf(theta), c = cosf(theta);
        float a = b[2 * i], bb = b[2 * i + 1];
        float ac = a * c, bs = bb * s, as = a * s, bc = bb * c;
        b[2 * i] = ac - bs;
        b[2 * i + 1] = as + bc;
    }
}

static float hy_silu(float v) { float den = 1.0f + expf(-v); return v / den; }

/* n_tok consecutive tokens (positions m->len ..) through the full-attention
 * mixer of layer l; h, o [n_tok][n_embd].  The projections take all the
 * tokens as matvec columns (bit-identical to one column at a time, the
 * batched-column invariance of lrso_matvec); each token then runs in order,
 * so token t's attention sees the cache rows of the tokens before it. */
static void hy_attn(lrso_hybrid *m, uint32_t l, const float *h, uint32_t n_tok, float *o) {
    const lrso_config *b = &m->c.base;
    const lrso_hybrid_layer *L = &m->layers[l];
    const uint32_t E = b->n_embd, HD = b->head_dim, QD = b->n_head * HD, KV = b->n_head_kv * HD;
    float *qg = (float *)malloc(sizeof(float) * 2 * QD * n_tok);
    float *k = (float *)malloc(sizeof(float) * KV * n_tok);
    float *v = (float *)malloc(sizeof(float) * KV * n_tok);
    float *q = (float *)malloc(sizeof(float) * QD);
    float *att = (float *)malloc(sizeof(float) * QD * n_tok);
    float *qn = tensor_f32(&L->q_norm, HD), *kn = tensor_f32(&L->k_norm, HD);
    lrso_matvec(L->attn_q.type, L->attn_q.bytes, L->attn_q.len, E, 2 * QD, h, qg, n_tok, m->n_threads);
    lrso_matvec(L->attn_k.type, L->attn_k.bytes, L->attn_k.len, E, KV, h, k, n_tok, m->n_threads);
    lrso_matvec(L->attn_v.type, L->attn_v.bytes, L->attn_v.len, E, KV, h, v, n_tok, m->n_threads);
    const size_t sl = (size_t)m->slot[l] * b->ctx * KV;
    float *kl = m->kc + sl, *vl = m->vc + sl;
    for (uint32_t t = 0; t < n_tok; t++) {
        const uint32_t pos = m->len + t;
        float *qgt = qg + (size_t)t * 2 * QD, *kt = k + (size_t)t * KV, *vt = v + (size_t)t * KV;
        float *at = att + (size_t)t * QD;
        /* QK-norm (dn_norm mode 2, Q heads 2*head_dim apart) then RoPE */
        for (uint32_t hh = 0; hh < b->n_head; hh++) {
            float *qh = qgt + (size_t)hh * 2 * HD;
            hy_head_rms(qh, HD, qn, b->rms_eps);
            hy_rope_head(qh, b->rope_dim, m->freq, pos);
            memcpy(q + (size_t)hh * HD, qh, sizeof(float) * HD);
        }
        for (uint32_t hh = 0; hh < b->n_head_kv; hh++) {
            hy_head_rms(kt + (size_t)hh * HD, HD, kn, b->rms_eps);
            hy_rope_head(kt + (size_t)hh * HD, b->rope_dim, m->freq, pos);
        }
        for (uint32_t i = 0; i < KV; i++) {
            float kk = kt[i], vv = vt[i];
            if (m->kv_f16) {
                kk = lrso_f16_to_f32(lrso_f32_to_f16(kk));
                vv = lrso_f16_to_f32(lrso_f32_to_f16(vv));
            }
            kl[(size_t)pos * KV + i] = kk;
            vl[(size_t)pos * KV + i] = vv;
        }
        lrso_attention(q, kl, vl, 1, pos, b->n_head, b->n_head_kv, HD, at);
        /* gate_quant.comp: att * sigmoid(gate), gate = second half of the head's Q rows */
        for (uint32_t hh = 0; hh < b->n_head; hh++)
            for (uint32_t i = 0; i < HD; i++) {
                float g = qgt[(size_t)hh * 2 * HD + HD + i];
                at[(size_t)hh * HD + i] *= 1.0f / (1.0f + expf(-g));
            }
    }
    lrso_matvec(L->attn_output.type, L->attn_output.bytes, L->attn_output.len, QD, E, att, o,
                n_tok, m->n_threads);
    free(qg); free(q); free(k); free(v); free(att); free(qn); free(kn);
}

/* n_tok consecutive tokens through the gated delta-net mixer of layer l
 * (plano_delta order); h, o [n_tok][n_embd].  Projections batched as in
 * hy_attn; the conv, gates and the delta rule run token by token. */
static void hy_delta(lrso_hybrid *m, uint32_t l, const float *h, uint32_t n_tok, float *o) {
    const lrso_hybrid_config *c = &m->c;
    const lrso_config *b = &c->base;
    const lrso_hybrid_layer *L = &m->layers[l];
    const uint32_t E = b->n_embd, d = c->dn_state, KD = c->dn_k_heads * d, VD = c->dn_v_heads * d;
    const uint32_t CD = hy_conv_dim(c), NV = c->dn_v_heads;
    float *qkv = (float *)malloc(sizeof(float) * CD * n_tok);
    float *cv = (float *)malloc(sizeof(float) * CD);
    float *z = (float *)malloc(sizeof(float) * VD * n_tok);
    float *y = (float *)malloc(sizeof(float) * VD * n_tok);
    float *al = tensor_f32(&L->ssm_alpha, E * NV), *be = tensor_f32(&L->ssm_beta, E * NV);
    float *sa = tensor_f32(&L->ssm_a, NV), *dt = tensor_f32(&L->ssm_dt, NV);
    float *cw = tensor_f32(&L->ssm_conv, CD * c->dn_conv), *nw = tensor_f32(&L->ssm_norm, d);
    lrso_matvec(L->ssm_qkv.type, L->ssm_qkv.bytes, L->ssm_qkv.len, E, CD, h, qkv, n_tok, m->n_threads);
    lrso_matvec(L->ssm_gate.type, L->ssm_gate.bytes, L->ssm_gate.len, E, VD, h, z, n_tok, m->n_threads);
    float *win = m->win + (size_t)m->slot[l] * CD * (c->dn_conv - 1);
    float *st = m->state + (size_t)m->slot[l] * NV * d * d;
    for (uint32_t t = 0; t < n_tok; t++) {
        const float *ht = h + (size_t)t * E, *zt = z + (size_t)t * VD;
        float *yt = y + (size_t)t * VD;
        /* causal conv with state, then SiLU (dn_conv.comp; delta_net.rs:51-78) */
        lrso_conv1d_step(win, qkv + (size_t)t * CD, cw, CD, c->dn_conv, cv);
        for (uint32_t i = 0; i < CD; i++) cv[i] = hy_silu(cv[i]);
        /* L2 norm of q and k per key head (dn_l2_qk.comp, eps = rms_eps) */
        lrso_l2_norm_rows(cv, 2 * c->dn_k_heads, d, b->rms_eps);
        for (uint32_t hh = 0; hh < NV; hh++) {
            /* gates (dn_gates.comp): g = a * softplus(alpha.h + dt), beta = sigmoid(beta.h) */
            float pa = -0.0f, pb = -0.0f;
            for (uint32_t i = 0; i < E; i++) {
                float p1 = al[(size_t)hh * E + i] * ht[i], p2 = be[(size_t)hh * E + i] * ht[i];
                pa = pa + p1;
                pb = pb + p2;
            }
            float g = sa[hh] * lrso_softplus(pa + dt[hh]);
            float beta = 1.0f / (1.0f + expf(-pb));
            /* value head hh reads key head hh % k_heads (delta_net.comp:75-85) */
            const uint32_t kh = hh % c->dn_k_heads;
            lrso_delta_net_step(st + (size_t)hh * d * d, cv + (size_t)kh * d, cv + KD + (size_t)kh * d,
                                cv + 2 * KD + (size_t)hh * d, g, beta, d, yt + (size_t)hh * d);
            /* gated RMSNorm (dn_norm mode 1): (y * 1/sqrt(mean(y^2)+eps)) * (w * silu(z)) */
            float *yh = yt + (size_t)hh * d;
            const float *zh = zt + (size_t)hh * d;
            float ss = -0.0f;
            for (uint32_t i = 0; i < d; i++) { float sq = yh[i] * yh[i]; ss = ss + sq; }
            float s = 1.0f / sqrtf(ss / (float)d + b->rms_eps);
            for (uint32_t i = 0; i < d; i++) {
                float vv = yh[i] * s;
                float gz = nw[i] * hy_silu(zh[i]);
                yh[i] = vv * gz;
            }
        }
    }
    lrso_matvec(L->ssm_out.type, L->ssm_out.bytes, L->ssm_out.len, VD, E, y, o, n_tok, m->n_threads);
    free(qkv); free(cv); free(z); free(y); free(al); free(be); free(sa); free(dt); free(cw); free(nw);
}

/* The tokens go through the model layer by layer (every token of layer l
 * before layer l + 1), each op's per-token arithmetic unchanged, so the
 * result equals feeding them one at a time. */
int lrso_hybrid_forward(lrso_hybrid *m, const uint32_t *tokens, uint32_t n_tok, float *logits) {
    const lrso_config *b = &m->c.base;
    const uint32_t E = b->n_embd;
    if (n_tok == 0) return -1;
    if (m->len + n_tok > b->ctx) return -3;
    for (uint32_t t = 0; t < n_tok; t++)
        if (tokens[t] >= b->vocab) return -4;
    size_t row_bytes = m->embd.len / b->vocab;
    float *x = (float *)malloc(sizeof(float) * E * n_tok);
    float *h = (float *)malloc(sizeof(float) * E * n_tok);
    float *o = (float *)malloc(sizeof(float) * E * n_tok);
    float *g = (float *)malloc(sizeof(float) * b->n_ff * n_tok);
    float *u = (float *)malloc(sizeof(float) * b->n_ff * n_tok);
    for (uint32_t t = 0; t < n_tok; t++)
        lrso_dequant(m->embd.type, m->embd.bytes + (size_t)tokens[t] * row_bytes, row_bytes,
                     x + (size_t)t * E);
    const size_t xe = (size_t)E * n_tok;
    for (uint32_t l = 0; l < b->n_layer; l++) {
        lrso_hybrid_layer *L = &m->layers[l];
        float *an = tensor_f32(&L->attn_norm, E), *pn = tensor_f32(&L->post_norm, E);
        lrso_rmsnorm_scale(x, an, n_tok, E, b->rms_eps, h);
        if (hy_full(&m->c, l)) hy_attn(m, l, h, n_tok, o);
        else hy_delta(m, l, h, n_tok, o);
        for (size_t i = 0; i < xe; i++) x[i] += o[i];
        lrso_rmsnorm_scale(x, pn, n_tok, E, b->rms_eps, h);
        lrso_matvec(L->ffn_gate.type, L->ffn_gate.bytes, L->ffn_gate.len, E, b->n_ff, h, g, n_tok,
                    m->n_threads);
        lrso_matvec(L->ffn_up.type, L->ffn_up.bytes, L->ffn_up.len, E, b->n_ff, h, u, n_tok,
                    m->n_threads);
        lrso_swiglu(g, u, b->n_ff * n_tok, g);
        lrso_matvec(L->ffn_down.type, L->ffn_down.bytes, L->ffn_down.len, b->n_ff, E, g, o, n_tok,
                    m->n_threads);
        for (size_t i = 0; i < xe; i++) x[i] += o[i];
        free(an); free(pn);
    }
    m->len += n_tok;
    if (logits) {
        float *on = tensor_f32(&m->onorm, E);
        lrso_rmsnorm_scale(x + (size_t)(n_tok - 1) * E, on, 1, E, b->rms_eps, h);
        lrso_matvec(m->out.type, m->out.bytes, m->out.len, E, b->vocab, h, logits, 1, m->n_threads);
        free(on);
    }
    free(x); free(h); free(o); free(g); free(u);
    return 0;
}

uint32_t lrso_hybrid_len(const lrso_hybrid *m) { return m->len; }

void lrso_hybrid_reset(lrso_hybrid *m) {
    const lrso_hybrid_config *c = &m->c;
    m->len = 0;
    memset(m->state, 0, sizeof(float) * ((size_t)m->n_dn * c->dn_v_heads * c->dn_state * c->dn_state));
    memset(m->win, 0, sizeof(float) * ((size_t)m->n_dn * hy_conv_dim(c) * (c->dn_conv - 1)));
}

void lrso_hybrid_destroy(lrso_hybrid *m) {
    if (!m) return;
    free(m->layers); free(m->slot); free(m->freq); free(m->kc); free(m->vc);
    free(m->state); free(m->win); free(m);
}
