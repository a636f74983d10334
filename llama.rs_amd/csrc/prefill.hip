// prefill.hip — the per-token ops of a batched prompt block (n tokens at
// positions pos0 .. pos0+n-1) around the matrix-core GEMMs of gemm.hip:
// RMSNorm per row and SwiGLU (both written straight to the bf16 input
// planes of the next GEMM), bias + RoPE + f16 KV append after the q/k/v
// GEMMs, causal GQA attention over the cache.  The formulas of the decode
// kernels (Model::forward, crates/llama-model/src/model.rs:99-266; ops.rs:
// 56-66, 952-988; attention.rs:76-166), which is what the reference's
// prefill_residente (gpu.rs:673-697) drives in blocks of batch_size() tokens;
// the attention runs on the matrix cores (f16 hi/lo operands, f32
// accumulation), so its summation order differs from the per-token kernel.
#include "lrs_internal.h"

namespace lrs {

// bf16 hi of v and the bf16 of the remainder (the GEMM input planes)
__device__ __forceinline__ void split_store(float v, __bf16 *hi, __bf16 *lo) {
    const __bf16 h = (__bf16)v;
    *hi = h;
    *lo = (__bf16)(v - (float)h);
}

// Y[r] = (X[r] * scale_r) * w, scale_r = 1 / sqrt(mean(X[r]^2) + eps); with
// hi, the same values also as bf16 hi / lo planes (lo = hi + gridDim.x * E)
__global__ __launch_bounds__(256) void k_rmsnorm_rows(const float *__restrict__ X,
                                                      const float *__restrict__ w, float eps,
                                                      uint32_t E, float *__restrict__ Y,
                                                      __bf16 *__restrict__ hi) {
    __shared__ float red[4];
    const float *x = X + (size_t)blockIdx.x * E;
    float *y = Y ? Y + (size_t)blockIdx.x * E : nullptr;
    float ss = 0.f;
    for (uint32_t i = 4 * threadIdx.x; i < E; i += 4 * blockDim.x) {
        const float4 v = *reinterpret_cast<const float4 *>(x + i);
        ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float scale = 1.0f / sqrtf(tot / (float)E + eps);
    const size_t plane = (size_t)gridDim.x * E, r0 = (size_t)blockIdx.x * E;
    for (uint32_t i = threadIdx.x; i < E; i += blockDim.x) {
        const float v = (x[i] * scale) * w[i];
        if (Y) y[i] = v;
        if (hi) split_store(v, hi + r0 + i, hi + plane + r0 + i);
    }
}

// X += the ks K-slice partials part[z][row][E] (summed in slice order, then
// added to X, as k_reduce_ks does), then k_rmsnorm_rows over the new rows
// (same sum-of-squares order, so the same scale): the residual add of a
// K-split o / down GEMM and the norm after it in one pass over the rows
__global__ __launch_bounds__(256) void k_reduce_norm_rows(const float *__restrict__ part,
                                                          uint32_t ks, float *__restrict__ X,
                                                          const float *__restrict__ w, float eps,
                                                          uint32_t E, float *__restrict__ Y,
                                                          __bf16 *__restrict__ hi) {
    __shared__ float red[4];
    const size_t plane = (size_t)gridDim.x * E, r0 = (size_t)blockIdx.x * E;
    float *x = X + r0;
    float ss = 0.f;
    for (uint32_t i = 4 * threadIdx.x; i < E; i += 4 * blockDim.x) {
        float4 p = *reinterpret_cast<const float4 *>(part + r0 + i);
        for (uint32_t z = 1; z < ks; z++) {
            const float4 q = *reinterpret_cast<const float4 *>(part + z * plane + r0 + i);
            p.x += q.x;
            p.y += q.y;
            p.z += q.z;
            p.w += q.w;
        }
        float4 v = *reinterpret_cast<const float4 *>(x + i);
        v.x += p.x;
        v.y += p.y;
        v.z += p.z;
        v.w += p.w;
        *reinterpret_cast<float4 *>(x + i) = v;
        ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float scale = 1.0f / sqrtf(tot / (float)E + eps);
    // each thread reads back the elements it stored above
    for (uint32_t i = 4 * threadIdx.x; i < E; i += 4 * blockDim.x) {
        const float4 v = *reinterpret_cast<const float4 *>(x + i);
        const float4 g = *reinterpret_cast<const float4 *>(w + i);
        const float4 o = {(v.x * scale) * g.x, (v.y * scale) * g.y, (v.z * scale) * g.z,
                          (v.w * scale) * g.w};
        if (Y) *reinterpret_cast<float4 *>(Y + r0 + i) = o;
        if (hi) {
            split_store(o.x, hi + r0 + i, hi + plane + r0 + i);
            split_store(o.y, hi + r0 + i + 1, hi + plane + r0 + i + 1);
            split_store(o.z, hi + r0 + i + 2, hi + plane + r0 + i + 2);
            split_store(o.w, hi + r0 + i + 3, hi + plane + r0 + i + 3);
        }
    }
}

// q/k/v GEMM outputs -> bias, adjacent-pair RoPE on q and k at position
// pos0 + token, q to f32, k and v to the f16 cache.  One thread per pair.
struct QkvPost {
    const float *qt, *kt, *vt;     // [n][qd], [n][kvd], [n][kvd]
    const float *bq, *bk, *bv;     // biases or null
    const float *freq;             // [rope_dim / 2]
    float *q;                      // [n][qd]
    _Float16 *kc, *vc;             // this layer's caches [n_kv][ctx][hd]
    uint32_t n, pos0, qd, kvd, hd, rope_dim, ctx;
};

__global__ void k_qkv_post(QkvPost a) {
    const uint32_t b = blockIdx.y;
    const uint32_t np = (a.qd + 2 * a.kvd) / 2;  // pairs per token
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= np || b >= a.n) return;
    const uint32_t e = 2 * i, pos = a.pos0 + b;
    const float *src;
    const float *bias;
    uint32_t off;
    int kind;  // 0 q, 1 k, 2 v
    if (e < a.qd) {
        kind = 0, off = e, src = a.qt + (size_t)b * a.qd, bias = a.bq;
    } else if (e < a.qd + a.kvd) {
        kind = 1, off = e - a.qd, src = a.kt + (size_t)b * a.kvd, bias = a.bk;
    } else {
        kind = 2, off = e - a.qd - a.kvd, src = a.vt + (size_t)b * a.kvd, bias = a.bv;
    }
    float x0 = src[off], x1 = src[off + 1];
    if (bias) {
        x0 = x0 + bias[off];
        x1 = x1 + bias[off + 1];
    }
    const uint32_t dd = off % a.hd;
    if (kind < 2 && dd < a.rope_dim) {
        // ops.rs:952-975: theta = pos * freq[dd / 2]
        const float th = (float)pos * a.freq[dd >> 1];
        float sn, cs;
        sincosf(th, &sn, &cs);
        const float r0 = x0 * cs - x1 * sn, r1 = x0 * sn + x1 * cs;
        x0 = r0;
        x1 = r1;
    }
    if (kind == 0) {
        a.q[(size_t)b * a.qd + off] = x0;
        a.q[(size_t)b * a.qd + off + 1] = x1;
    } else {
        _Float16 *c = kind == 1 ? a.kc : a.vc;
        const uint32_t hh = off / a.hd;
        const size_t o = ((size_t)hh * a.ctx + pos) * a.hd + dd;
        c[o] = (_Float16)x0;
        c[o + 1] = (_Float16)x1;
    }
}

// Causal GQA attention of the block: token b (position pos0 + b) attends to
// cache positions 0..pos0+b (attention.rs:76-166 per token).
struct AttnPre {
    const float *q;                 // [n][n_head * hd]
    const _Float16 *kc, *vc;        // [n_kv][ctx][hd]
    float *out;                     // [n][n_head * hd]
    uint32_t n, pos0, n_head, n_kv, ctx;
    float scale;
};

// On the matrix cores: workgroup (32-token query block,
// KV head, group of NW query heads of the GQA group), one wavefront per query
// head: NW = the whole group for head_dim <= 128; at head_dim 256 at most 4
// wavefronts (the query and output registers of a wavefront exceed half the
// register file, so one wavefront per SIMD).  Per chunk of 32 cache positions each wavefront forms the transposed
// score tile S^T = K Q^T (32 positions x 32 queries) with
// v_mfma_f32_32x32x16_f16: K is the f16 cache (exact), Q is split into f16
// hi + lo after scaling each query by a power of two (2^-e >= 1 / max |q|),
// so the products carry 22 bits of q.  In that layout a lane owns one query
// and 16 of the chunk's positions, so the online softmax (running max m,
// sum l) needs one cross-lane step per reduction.  The probabilities, split
// into f16 hi + lo, are the B operand of O^T += V^T P^T straight from the
// score registers: the K index of that product is the position order in
// which the score layout holds them (4 positions of the lane's half, then the
// 4 positions 8 further), and V^T is read from LDS in the same order.
// K is staged with global_load_lds into an XOR-swizzled row layout
// (conflict-free 16-byte reads), V into a transposed, padded layout: through
// registers, or at head_dim 256 (no registers to spare) through a row-major
// LDS copy transposed after each chunk.  The next chunk's loads are in flight
// during the current chunk's matrix work.
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void_t;

template <int HD, int NW>
__global__ __launch_bounds__(64 * NW) void k_attn_pf_mma(AttnPre a) {
    constexpr int NT = 64 * NW;
    constexpr int KS = HD / 16;           // K-steps of S^T (16 dims each)
    constexpr int OT = HD / 32;           // O^T tiles of 32 dims
    constexpr int NPR = HD / 8;           // 16-byte pieces per K / V row
    constexpr int NPC = 32 * NPR;         // pieces per chunk
    constexpr int VLD = 36;               // V^T row (f16): 72 B, conflict-free 8-byte reads
    constexpr int NVP = (NPC + NT - 1) / NT;
    constexpr bool VLDS = HD > 128;       // V staged through LDS instead of registers
    __shared__ __attribute__((aligned(16))) _Float16 Ks[2][32 * HD];
    __shared__ __attribute__((aligned(16))) _Float16 Vt[2][HD * VLD];
    __shared__ __attribute__((aligned(16))) _Float16 Vraw[VLDS ? 32 * HD : 8];
    const uint32_t rep = a.n_head / a.n_kv, ng = (rep + NW - 1) / NW;
    const uint32_t qb = blockIdx.x, kh = blockIdx.y / ng;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, hf = lane >> 5;
    const uint32_t hl = (blockIdx.y % ng) * NW + wave;  // query head within the group
    const bool hact = hl < rep;                         // an idle wavefront stages and stores nothing
    const uint32_t h = kh * rep + (hact ? hl : rep - 1);
    const uint32_t q0 = qb * 32, qi = q0 + (lane & 31);
    const uint32_t qr = qi < a.n ? qi : a.n - 1;  // lanes past the block compute a copy, store nothing
    const uint32_t qpos = a.pos0 + qr;
    const uint32_t kend = a.pos0 + min(q0 + 32, a.n);  // positions 0..kend-1 are attended
    const uint32_t nch = (kend + 31) / 32;
    const _Float16 *kb = a.kc + (size_t)kh * a.ctx * HD;
    const _Float16 *vb = a.vc + (size_t)kh * a.ctx * HD;

    // K chunk c -> Ks[buf]: LDS slot s (16 B) holds row s / NPR, piece
    // (s % NPR) ^ (row % NPR); wavefront instruction i fills slots 64i..64i+63
    auto stage_k = [&](uint32_t c, uint32_t buf) {
        for (uint32_t i = wave; i < NPC / 64; i += NW) {
            const uint32_t sl = 64 * i + lane, row = sl / NPR, pc = (sl % NPR) ^ (row % NPR);
            const uint32_t kp = min(32 * c + row, kend - 1);  // past the end: any finite row (masked)
            __builtin_amdgcn_global_load_lds(kb + (size_t)kp * HD + 8 * pc,
                                             (lds_void_t *)(Ks[buf] + 64 * 8 * i), 16, 0, 0);
        }
    };
    // V chunk c: piece p = (row p % 32, dims 8 (p / 32)..), through registers
    // (load_v, store_v) or, at head_dim 256, global_load_lds into Vraw slot p
    // and an LDS transpose (vraw_to_vt)
    uint4 vr[VLDS ? 1 : NVP];
    auto stage_vraw = [&](uint32_t c) {
        for (uint32_t i = wave; i < NPC / 64; i += NW) {
            const uint32_t p = 64 * i + lane, row = p % 32, kp = min(32 * c + row, kend - 1);
            __builtin_amdgcn_global_load_lds(vb + (size_t)kp * HD + 8 * (p / 32),
                                             (lds_void_t *)(Vraw + 64 * 8 * i), 16, 0, 0);
        }
    };
    auto vraw_to_vt = [&](uint32_t buf) {
        for (uint32_t p = tid; p < (uint32_t)NPC; p += NT) {
            const uint4 v = *reinterpret_cast<const uint4 *>(Vraw + 8 * p);
            const _Float16 *hv = reinterpret_cast<const _Float16 *>(&v);
            const uint32_t row = p % 32, d0 = 8 * (p / 32);
#pragma unroll
            for (int e = 0; e < 8; e++) Vt[buf][(d0 + e) * VLD + row] = hv[e];
        }
    };
    auto load_v = [&](uint32_t c) {
#pragma unroll
        for (int j = 0; j < (VLDS ? 1 : NVP); j++) {
            const uint32_t p = tid + NT * j;
            if (p < (uint32_t)NPC) {
                const uint32_t row = p % 32, kp = min(32 * c + row, kend - 1);
                vr[j] = *reinterpret_cast<const uint4 *>(vb + (size_t)kp * HD + 8 * (p / 32));
            }
        }
    };
    auto store_v = [&](uint32_t buf) {
#pragma unroll
        for (int j = 0; j < (VLDS ? 1 : NVP); j++) {
            const uint32_t p = tid + NT * j;
            if (p < (uint32_t)NPC) {
                const uint32_t row = p % 32, d0 = 8 * (p / 32);
                const _Float16 *hv = reinterpret_cast<const _Float16 *>(&vr[j]);
#pragma unroll
                for (int e = 0; e < 8; e++) Vt[buf][(d0 + e) * VLD + row] = hv[e];
            }
        }
    };

    // this lane's query: dims 16 k + 8 hf .. + 7 of every K-step, scaled by
    // 2^-e (e from the head's max |q|, both halves), split into f16 hi + lo
    f16x8_t qh[KS], ql[KS];
    float qsc;
    {
        const float *qp = a.q + ((size_t)qr * a.n_head + h) * HD + 8 * hf;
        float qv[KS][8];
        float qm = 0.f;
#pragma unroll
        for (int k = 0; k < KS; k++) {
            const float4 x0 = *reinterpret_cast<const float4 *>(qp + 16 * k);
            const float4 x1 = *reinterpret_cast<const float4 *>(qp + 16 * k + 4);
            qv[k][0] = x0.x; qv[k][1] = x0.y; qv[k][2] = x0.z; qv[k][3] = x0.w;
            qv[k][4] = x1.x; qv[k][5] = x1.y; qv[k][6] = x1.z; qv[k][7] = x1.w;
#pragma unroll
            for (int e = 0; e < 8; e++) qm = fmaxf(qm, fabsf(qv[k][e]));
        }
        qm = fmaxf(qm, __shfl_xor(qm, 32, 64));
        int ex;
        frexpf(qm, &ex);
        ex = ex < -60 ? -60 : ex;
        qsc = ldexpf(1.0f, ex) * a.scale;
#pragma unroll
        for (int k = 0; k < KS; k++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float x = ldexpf(qv[k][e], -ex);
                const _Float16 xh = (_Float16)x;
                qh[k][e] = xh;
                ql[k][e] = (_Float16)(x - (float)xh);
            }
    }

    f32x16_t o[OT];
#pragma unroll
    for (int t = 0; t < OT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[t][r] = 0.f;
    float m = -INFINITY, l = 0.f;

    stage_k(0, 0);
    if constexpr (VLDS) {
        stage_vraw(0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        vraw_to_vt(0);
    } else {
        load_v(0);
        store_v(0);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (uint32_t c = 0; c < nch; c++) {
        const uint32_t cur = c & 1;
        const bool more = c + 1 < nch;
        if (more) {
            stage_k(c + 1, cur ^ 1);
            if constexpr (VLDS)
                stage_vraw(c + 1);
            else
                load_v(c + 1);
        }
        // S^T = K Q^T: lane (query l%32) gets positions 8(r/4) + 4 hf + r%4
        f32x16_t sc;
#pragma unroll
        for (int r = 0; r < 16; r++) sc[r] = 0.f;
        const uint32_t krow = lane & 31;
#pragma unroll
        for (int k = 0; k < KS; k++) {
            const uint32_t sl = krow * NPR + ((2 * k + hf) ^ (krow % NPR));
            const f16x8_t kf = *reinterpret_cast<const f16x8_t *>(Ks[cur] + 8 * sl);
            sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, ql[k], sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qh[k], sc, 0, 0, 0);
        }
        // online softmax of this query over the chunk (causal mask)
        float cmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const uint32_t kp = 32 * c + 8 * (r >> 2) + 4 * hf + (r & 3);
            sc[r] = kp <= qpos ? sc[r] * qsc : -INFINITY;
            cmax = fmaxf(cmax, sc[r]);
        }
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
        const float mn = fmaxf(m, cmax);  // finite: position 0 is in the first chunk
        const float alpha = expf(m - mn);
        float ps = 0.f;
        f16x8_t ph[2], pl[2];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const float p = expf(sc[r] - mn);
            ps += p;
            const _Float16 x = (_Float16)p;
            ph[r >> 3][r & 7] = x;
            pl[r >> 3][r & 7] = (_Float16)(p - (float)x);
        }
        ps += __shfl_xor(ps, 32, 64);
        l = l * alpha + ps;
        m = mn;
        // O^T (dims x queries) = alpha O^T + V^T P^T; K slot j of step s is
        // position 16 s + 4 hf + j (j < 4) or 16 s + 8 + 4 hf + j - 4
#pragma unroll
        for (int t = 0; t < OT; t++) {
#pragma unroll
            for (int r = 0; r < 16; r++) o[t][r] *= alpha;
            const _Float16 *vrow = Vt[cur] + (32 * t + (lane & 31)) * VLD + 4 * hf;
#pragma unroll
            for (int st = 0; st < 2; st++) {
                const f16x4_t v0 = *reinterpret_cast<const f16x4_t *>(vrow + 16 * st);
                const f16x4_t v1 = *reinterpret_cast<const f16x4_t *>(vrow + 16 * st + 8);
                const f16x8_t va = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pl[st], o[t], 0, 0, 0);
                o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, ph[st], o[t], 0, 0, 0);
            }
        }
        if constexpr (!VLDS) {
            if (more) store_v(cur ^ 1);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if constexpr (VLDS) {
            if (more) {
                vraw_to_vt(cur ^ 1);
                __syncthreads();
            }
        }
    }
    // out[token][head][dim]: lane holds dims 32 t + 8 (r/4) + 4 hf + r%4
    if (qi < a.n && hact) {
        const float inv = 1.0f / l;
        float *op = a.out + ((size_t)qi * a.n_head + h) * HD;
#pragma unroll
        for (int t = 0; t < OT; t++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                *reinterpret_cast<float4 *>(op + 32 * t + 8 * g + 4 * hf) =
                    make_float4(o[t][4 * g] * inv, o[t][4 * g + 1] * inv, o[t][4 * g + 2] * inv,
                                o[t][4 * g + 3] * inv);
    }
}

hipError_t launch_rmsnorm_rows(const float *X, const float *w, float eps, uint32_t E, uint32_t n,
                               float *Y, hipStream_t s, __bf16 *hi) {
    if (E % 4 || (!Y && !hi)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3(n), dim3(256), 0, s, X, w, eps, E, Y, hi);
    return hipGetLastError();
}

hipError_t launch_reduce_norm_rows(const float *part, uint32_t ks, float *X, const float *w,
                                   float eps, uint32_t E, uint32_t n, float *Y, __bf16 *hi,
                                   hipStream_t s) {
    if (E % 4 || ks == 0 || (!Y && !hi)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_reduce_norm_rows, dim3(n), dim3(256), 0, s, part, ks, X, w, eps, E, Y, hi);
    return hipGetLastError();
}

hipError_t launch_qkv_post(const float *qt, const float *kt, const float *vt, const float *bq,
                           const float *bk, const float *bv, const float *freq, float *q,
                           _Float16 *kc, _Float16 *vc, uint32_t n, uint32_t pos0, uint32_t qd,
                           uint32_t kvd, uint32_t hd, uint32_t rope_dim, uint32_t ctx,
                           hipStream_t s) {
    QkvPost a = {qt, kt, vt, bq, bk, bv, freq, q, kc, vc, n, pos0, qd, kvd, hd, rope_dim, ctx};
    const uint32_t np = (qd + 2 * kvd) / 2;
    hipLaunchKernelGGL(k_qkv_post, dim3((np + 255) / 256, n), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_attn_prefill(const float *q, const _Float16 *kc, const _Float16 *vc, float *out,
                               uint32_t n, uint32_t pos0, uint32_t n_head, uint32_t n_kv,
                               uint32_t hd, uint32_t ctx, hipStream_t s) {
    if (n == 0 || n_kv == 0 || n_head % n_kv || n_head / n_kv > 8) return hipErrorInvalidValue;
    AttnPre a = {q, kc, vc, out, n, pos0, n_head, n_kv, ctx, 1.0f / sqrtf((float)hd)};
    const uint32_t rep = n_head / n_kv;
    // wavefronts per workgroup: the whole group, or at head_dim 256 an even
    // share of it in groups of at most 4
    const uint32_t nw = hd == 256 ? (rep + (rep + 3) / 4 - 1) / ((rep + 3) / 4) : rep;
    void (*fn)(AttnPre) = nullptr;
#define LRS_PF_NW(W)                                                                     \
    case W:                                                                              \
        fn = hd == 64 ? k_attn_pf_mma<64, W> : hd == 128 ? k_attn_pf_mma<128, W> : nullptr; \
        break;
    if (hd == 64 || hd == 128) {
        switch (nw) {
            LRS_PF_NW(1) LRS_PF_NW(2) LRS_PF_NW(3) LRS_PF_NW(4)
            LRS_PF_NW(5) LRS_PF_NW(6) LRS_PF_NW(7) LRS_PF_NW(8)
        }
    } else if (hd == 256) {
        switch (nw) {
        case 1: fn = k_attn_pf_mma<256, 1>; break;
        case 2: fn = k_attn_pf_mma<256, 2>; break;
        case 3: fn = k_attn_pf_mma<256, 3>; break;
        case 4: fn = k_attn_pf_mma<256, 4>; break;
        }
    }
#undef LRS_PF_NW
    if (!fn) return hipErrorInvalidValue;
    const uint32_t ng = (rep + nw - 1) / nw;
    hipLaunchKernelGGL(fn, dim3((n + 31) / 32, n_kv * ng), dim3(64 * nw), 0, s, a);
    return hipGetLastError();
}

// silu(G) * U (ops.rs:978-988: g / (1 + e^-g) * u), stored as the bf16 hi / lo
// planes of the down projection's input
__global__ __launch_bounds__(256) void k_swiglu_split(const float *__restrict__ G,
                                                      const float *__restrict__ U, size_t n4,
                                                      __bf16 *__restrict__ hi,
                                                      __bf16 *__restrict__ lo) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const float4 g = reinterpret_cast<const float4 *>(G)[i];
    const float4 u = reinterpret_cast<const float4 *>(U)[i];
    const float y[4] = {(g.x / (1.0f + expf(-g.x))) * u.x, (g.y / (1.0f + expf(-g.y))) * u.y,
                        (g.z / (1.0f + expf(-g.z))) * u.z, (g.w / (1.0f + expf(-g.w))) * u.w};
    typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
    bf16x4 h, l;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        h[k] = (__bf16)y[k];
        l[k] = (__bf16)(y[k] - (float)h[k]);
    }
    reinterpret_cast<bf16x4 *>(hi)[i] = h;
    reinterpret_cast<bf16x4 *>(lo)[i] = l;
}

hipError_t launch_swiglu_split(const float *G, const float *U, size_t n, __bf16 *hi,
                               hipStream_t s) {
    if (n % 4) return hipErrorInvalidValue;
    const size_t n4 = n / 4;
    hipLaunchKernelGGL(k_swiglu_split, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, G, U,
                       n4, hi, hi + n);
    return hipGetLastError();
}

}  // namespace lrs
