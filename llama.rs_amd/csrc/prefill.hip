// prefill.hip — the per-token ops of a batched prompt block (n tokens at
// positions pos0 .. pos0+n-1) around the matrix-core GEMMs of gemm.hip:
// RMSNorm per row, bias + RoPE + f16 KV append after the q/k/v GEMMs,
// causal GQA attention over the cache, SwiGLU.  Same formulas and operation
// order as the decode kernels (Model::forward, crates/llama-model/src/
// model.rs:99-266; ops.rs:56-66, 952-988; attention.rs:76-166), which is what
// the reference's prefill_residente (gpu.rs:673-697) drives in blocks of
// batch_size() tokens.
#include "lrs_internal.h"

namespace lrs {

// Y[r] = (X[r] * scale_r) * w, scale_r = 1 / sqrt(mean(X[r]^2) + eps)
__global__ __launch_bounds__(256) void k_rmsnorm_rows(const float *__restrict__ X,
                                                      const float *__restrict__ w, float eps,
                                                      uint32_t E, float *__restrict__ Y) {
    __shared__ float red[4];
    const float *x = X + (size_t)blockIdx.x * E;
    float *y = Y + (size_t)blockIdx.x * E;
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
    for (uint32_t i = threadIdx.x; i < E; i += blockDim.x) y[i] = (x[i] * scale) * w[i];
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

// Causal GQA attention of token b (position pos0 + b) over cache positions
// 0..pos0+b, online softmax over chunks of 64 positions staged in LDS (K
// transposed so that lane = position reads conflict-free).  One workgroup per
// (token, KV head); wavefront w handles query heads w, w+4, ... of the group.
struct AttnPre {
    const float *q;                 // [n][n_head * hd]
    const _Float16 *kc, *vc;        // [n_kv][ctx][hd]
    float *out;                     // [n][n_head * hd]
    uint32_t n, pos0, n_head, n_kv, ctx;
    float scale;
};

template <int HD>
__global__ __launch_bounds__(256) void k_attn_prefill(AttnPre a) {
    constexpr int CH = 64;
    constexpr int DPL = HD / 64;  // dims per lane in the V sum
    __shared__ float kt[HD][CH + 1];
    __shared__ _Float16 vs[CH][HD];
    __shared__ float qs[8][HD];
    __shared__ float ps[4][CH];
    const uint32_t b = blockIdx.x, kh = blockIdx.y;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t rep = a.n_head / a.n_kv, h0 = kh * rep;
    const uint32_t L = a.pos0 + b + 1;
    const size_t qrow = (size_t)b * a.n_head * HD;
    for (uint32_t i = tid; i < rep * HD; i += 256) qs[i / HD][i % HD] = a.q[qrow + (size_t)h0 * HD + i];

    float m[2], l[2], acc[2][DPL];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        m[s] = -INFINITY;
        l[s] = 0.f;
#pragma unroll
        for (int k = 0; k < DPL; k++) acc[s][k] = 0.f;
    }
    const _Float16 *kbase = a.kc + (size_t)kh * a.ctx * HD;
    const _Float16 *vbase = a.vc + (size_t)kh * a.ctx * HD;
    for (uint32_t c0 = 0; c0 < L; c0 += CH) {
        const uint32_t nc = min((uint32_t)CH, L - c0);
        __syncthreads();  // the previous chunk is consumed (and q is staged)
        for (uint32_t i = tid; i < CH * HD; i += 256) {
            const uint32_t j = i / HD, d = i % HD;
            const bool ok = j < nc;
            kt[d][j] = ok ? (float)kbase[(size_t)(c0 + j) * HD + d] : 0.f;
            vs[j][d] = ok ? vbase[(size_t)(c0 + j) * HD + d] : (_Float16)0.f;
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const uint32_t r = wave + 4 * s;
            if (r >= rep) continue;
            // score of position c0 + lane
            float sc = 0.f;
#pragma unroll 8
            for (int d = 0; d < HD; d++) sc = fmaf(qs[r][d], kt[d][lane], sc);
            sc = lane < nc ? sc * a.scale : -INFINITY;
            float mc = sc;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) mc = fmaxf(mc, __shfl_xor(mc, o, 64));
            const float mn = fmaxf(m[s], mc);
            const float alpha = expf(m[s] - mn);  // m = -inf at the first chunk: 0
            const float p = lane < nc ? expf(sc - mn) : 0.f;
            float ls = p;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) ls += __shfl_xor(ls, o, 64);
            l[s] = l[s] * alpha + ls;
            m[s] = mn;
            ps[wave][lane] = p;
            // V sum: lane owns dims DPL*lane .. DPL*lane + DPL - 1 (wave-local
            // LDS row: written and read by this wavefront only)
#pragma unroll
            for (int k = 0; k < DPL; k++) acc[s][k] *= alpha;
            for (uint32_t j = 0; j < nc; j++) {
                const float pj = ps[wave][j];
#pragma unroll
                for (int k = 0; k < DPL; k++) acc[s][k] = fmaf(pj, (float)vs[j][DPL * lane + k], acc[s][k]);
            }
        }
    }
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const uint32_t r = wave + 4 * s;
        if (r >= rep) continue;
#pragma unroll
        for (int k = 0; k < DPL; k++)
            a.out[qrow + (size_t)(h0 + r) * HD + DPL * lane + k] = acc[s][k] / l[s];
    }
}

// G = silu(G) * U elementwise (ops.rs:978-988)
__global__ void k_swiglu_rows(float *__restrict__ G, const float *__restrict__ U, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        const float g = G[i];
        const float den = 1.0f + expf(-g);
        G[i] = (g / den) * U[i];
    }
}

hipError_t launch_rmsnorm_rows(const float *X, const float *w, float eps, uint32_t E, uint32_t n,
                               float *Y, hipStream_t s) {
    if (E % 4) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3(n), dim3(256), 0, s, X, w, eps, E, Y);
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
    if (n_head / n_kv > 8) return hipErrorInvalidValue;
    AttnPre a = {q, kc, vc, out, n, pos0, n_head, n_kv, ctx, 1.0f / sqrtf((float)hd)};
    dim3 grid(n, n_kv);
    switch (hd) {
    case 64: hipLaunchKernelGGL(k_attn_prefill<64>, grid, dim3(256), 0, s, a); break;
    case 128: hipLaunchKernelGGL(k_attn_prefill<128>, grid, dim3(256), 0, s, a); break;
    case 256: hipLaunchKernelGGL(k_attn_prefill<256>, grid, dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_swiglu_rows(float *G, const float *U, size_t n, hipStream_t s) {
    size_t g = (n + 255) / 256;
    if (g > 65536) g = 65536;
    hipLaunchKernelGGL(k_swiglu_rows, dim3((unsigned)g), dim3(256), 0, s, G, U, n);
    return hipGetLastError();
}

}  // namespace lrs
