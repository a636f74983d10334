// attention.hip — batch-1 causal GQA decode attention over the f16 KV cache.
//
// Math of attention.rs:76-166: scores q.k * 1/sqrt(head_dim) over positions
// 0..pos, softmax, weighted sum of V; query head h reads KV head
// h / (n_head / n_head_kv).  The cache holds f16 K and V, as the reference
// GPU path keeps them (kv_pack.comp).
//
// One workgroup of 16 wavefronts per query head, all positions, one launch,
// in three phases over the positions 0..pos:
//   scores   a "lane group" of HD/8 lanes owns one position at a time (8 dims
//            = one 16-byte piece of the K row per lane; the 64 lane groups
//            take positions g, g+64, ..., with the next positions' loads in
//            flight); q is split into f16 hi + lo halves so v_dot2_f32_f16
//            forms q.k from exact f16 products to 22 bits of q; scores to LDS
//   softmax  max and sum over the LDS scores (one exp per position)
//   values   the same lane groups accumulate p * V over their positions; the
//            groups of a wavefront are summed with cross-lane adds, the 16
//            wavefronts through LDS
// and the output is written as the activation pack of the o-projection.
// A single pass replaces the split + combine pair of the reference
// (attention_split.comp + attn_reduce.comp): no second launch, no partials
// in HBM.
#include "lrs_internal.h"
#include "pack_dev.h"

namespace lrs {

constexpr int ATT_THREADS = 1024;
constexpr int ATT_WAVES = ATT_THREADS / 64;
constexpr int ATT_DEPTH = 4;  // positions per lane group with K and V loads in flight

struct AttnArgs {
    const float *q;           // [n_head * HD], RoPE applied
    const _Float16 *kc, *vc;  // this layer's caches [n_kv][ctx][HD]
    XPack out;                // pack of the [n_head * HD] output
    const uint32_t *step;     // {token, pos}: attends positions 0..pos
    uint32_t n_head, n_kv, ctx;
    float scale;
};

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2_t as_h2(uint32_t v) {
    half2_t r;
    __builtin_memcpy(&r, &v, 4);
    return r;
}

// block-wide reduction of one float (max or sum) through LDS
template <bool MAX>
__device__ __forceinline__ float block_reduce(float v, float *red) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float t = __shfl_xor(v, o, 64);
        v = MAX ? fmaxf(v, t) : v + t;
    }
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();  // red[] may still be read by an earlier reduction
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < ATT_WAVES; w++) r = MAX ? fmaxf(r, red[w]) : r + red[w];
    return r;
}

template <int HD>
__global__ __launch_bounds__(ATT_THREADS) void k_attn(AttnArgs a) {
    constexpr int LP = HD / 8;              // lanes per position
    constexpr int NG = ATT_THREADS / LP;    // lane groups per workgroup
    extern __shared__ float sc[];           // [ctx] scores, then probabilities
    __shared__ float red[ATT_WAVES];
    __shared__ float sacc[ATT_WAVES][HD];
    const uint32_t tid = threadIdx.x, sub = tid % LP, grp = tid / LP;
    const uint32_t lane = tid & 63, wave = tid >> 6;
    const uint32_t h = blockIdx.x, kh = h / (a.n_head / a.n_kv);
    const uint32_t L = a.step[1] + 1;
    const _Float16 *kb = a.kc + (size_t)kh * a.ctx * HD + 8 * sub;
    const _Float16 *vb = a.vc + (size_t)kh * a.ctx * HD + 8 * sub;

    // K and V of the first ATT_DEPTH positions of every lane group in flight
    // at once (all of them up to 64 * ATT_DEPTH positions)
    uint4 kr[ATT_DEPTH], vr[ATT_DEPTH];
#pragma unroll
    for (int i = 0; i < ATT_DEPTH; i++) {
        const uint32_t p = grp + i * NG;
        if (p < L) kr[i] = *reinterpret_cast<const uint4 *>(kb + (size_t)p * HD);
    }
#pragma unroll
    for (int i = 0; i < ATT_DEPTH; i++) {
        const uint32_t p = grp + i * NG;
        if (p < L) vr[i] = *reinterpret_cast<const uint4 *>(vb + (size_t)p * HD);
    }
    // q / 2^e as f16 hi + lo pairs (dims 8 sub .. 8 sub + 7), 2^e >= max |q|
    // of the head so both halves stay in f16 range; the score is rescaled
    // by 2^e * scale (exact power of two, then the reference's 1/sqrt(HD))
    half2_t qh[4], ql[4];
    float sscale;
    {
        const float4 *qp = reinterpret_cast<const float4 *>(a.q + (size_t)h * HD + 8 * sub);
        const float4 x0 = qp[0], x1 = qp[1];
        float qv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        float qm = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) qm = fmaxf(qm, fabsf(qv[i]));
#pragma unroll
        for (int o = LP / 2; o >= 1; o >>= 1) qm = fmaxf(qm, __shfl_xor(qm, o, 64));
        int e;
        frexpf(qm, &e);
        e = e < -60 ? -60 : e;
#pragma unroll
        for (int i = 0; i < 8; i++) qv[i] = ldexpf(qv[i], -e);
        sscale = ldexpf(1.0f, e);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const _Float16 h0 = (_Float16)qv[2 * i], h1 = (_Float16)qv[2 * i + 1];
            qh[i] = half2_t{h0, h1};
            ql[i] = half2_t{(_Float16)(qv[2 * i] - (float)h0), (_Float16)(qv[2 * i + 1] - (float)h1)};
        }
    }

    // ---- scores ----
    float smax = -INFINITY;
    for (uint32_t p0 = grp; p0 < L; p0 += ATT_DEPTH * NG) {
#pragma unroll
        for (int i = 0; i < ATT_DEPTH; i++) {
            const uint32_t p = p0 + i * NG;
            if (p < L) {  // uniform within the lane group
                const uint4 k = kr[i];
                const uint32_t pn = p + ATT_DEPTH * NG;
                if (pn < L) kr[i] = *reinterpret_cast<const uint4 *>(kb + (size_t)pn * HD);
                const uint32_t kw[4] = {k.x, k.y, k.z, k.w};
                float s = 0.f;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    s = __builtin_amdgcn_fdot2(ql[j], as_h2(kw[j]), s, false);
                    s = __builtin_amdgcn_fdot2(qh[j], as_h2(kw[j]), s, false);
                }
#pragma unroll
                for (int o = LP / 2; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
                s = (s * sscale) * a.scale;  // attention.rs: (q.k) / sqrt(head_dim)
                if (sub == 0) sc[p] = s;
                smax = fmaxf(smax, s);
            }
        }
    }

    // ---- softmax (attention.rs:120-140) ----
    const float M = block_reduce<true>(smax, red);  // also orders the score stores
    float lsum = 0.f;
    for (uint32_t p = tid; p < L; p += ATT_THREADS) {
        const float e = expf(sc[p] - M);
        sc[p] = e;
        lsum += e;
    }
    const float den = block_reduce<false>(lsum, red);  // also orders the exp stores

    // ---- values ----
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; e++) acc[e] = 0.f;
    for (uint32_t p0 = grp; p0 < L; p0 += ATT_DEPTH * NG) {
#pragma unroll
        for (int i = 0; i < ATT_DEPTH; i++) {
            const uint32_t p = p0 + i * NG;
            if (p < L) {
                const uint4 v = vr[i];
                const uint32_t pn = p + ATT_DEPTH * NG;
                if (pn < L) vr[i] = *reinterpret_cast<const uint4 *>(vb + (size_t)pn * HD);
                const float pe = sc[p];
                const _Float16 *vh = reinterpret_cast<const _Float16 *>(&v);
#pragma unroll
                for (int e = 0; e < 8; e++) acc[e] = fmaf(pe, (float)vh[e], acc[e]);
            }
        }
    }
    // lane groups of a wavefront hold the same dims: sum them, then the waves
#pragma unroll
    for (int o = LP; o < 64; o <<= 1)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] += __shfl_xor(acc[e], o, 64);
    if (lane < LP) {
#pragma unroll
        for (int e = 0; e < 8; e++) sacc[wave][8 * lane + e] = acc[e];
    }
    __syncthreads();
    if (tid >= HD) return;  // whole half-waves remain for the pack (HD % 32 == 0)
    float num = 0.f;
#pragma unroll
    for (int w = 0; w < ATT_WAVES; w++) num += sacc[w][tid];
    pack_half(num / den, (h * HD + tid) >> 5, a.out);
}

hipError_t launch_attention(const float *q, const _Float16 *kc, const _Float16 *vc, XPack out,
                            const uint32_t *step, uint32_t n_head, uint32_t n_kv,
                            uint32_t head_dim, uint32_t ctx, hipStream_t s) {
    AttnArgs a;
    a.q = q;
    a.kc = kc;
    a.vc = vc;
    a.out = out;
    a.step = step;
    a.n_head = n_head;
    a.n_kv = n_kv;
    a.ctx = ctx;
    a.scale = 1.0f / sqrtf((float)head_dim);
    if (n_kv == 0 || n_head % n_kv) return hipErrorInvalidValue;
    const size_t lds = (size_t)ctx * sizeof(float);  // scores of every position
    if (lds > 128 * 1024) return hipErrorInvalidValue;
    switch (head_dim) {
    case 64: hipLaunchKernelGGL(k_attn<64>, dim3(n_head), dim3(ATT_THREADS), lds, s, a); break;
    case 128: hipLaunchKernelGGL(k_attn<128>, dim3(n_head), dim3(ATT_THREADS), lds, s, a); break;
    case 256: hipLaunchKernelGGL(k_attn<256>, dim3(n_head), dim3(ATT_THREADS), lds, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace lrs
