// attention.hip — batch-1 causal GQA decode attention over the f16 KV cache.
//
// Math of attention.rs:76-166: scores q.k * 1/sqrt(head_dim) over positions
// 0..pos, softmax, weighted sum of V; query head h reads KV head
// h / (n_head / n_head_kv).  The cache holds f16 K and V, as the reference
// GPU path keeps them (kv_pack.comp).
//
// Split over positions ("flash decode"): workgroup (split s, KV head kh)
// takes the blocks of ATT_BLOCK positions s, s + S, s + 2S, ... (S = splits)
// of 0..pos for all REP query heads of the GQA group (K and V are read once
// for the group).  The blocks a split owns do not depend on pos, so every
// workgroup issues its first K/V (and q) loads before the position arrives
// from the step buffer; pos only masks.  A "lane group" of HD/8 lanes owns
// one position at a time (8 dims = one 16-byte piece of the K and V rows per
// lane; lane group g takes the split's positions g, g+NG, ... in block order,
// with the next positions' loads in flight):
//   score    q is split into f16 hi + lo halves so v_dot2_f32_f16 forms q.k
//            from exact f16 products to 22 bits of q; the row sum over the
//            lane group is four DPP adds
//   update   online softmax per lane group: running max m, sum l and
//            accumulator e^(s - m) V, rescaled when the max moves
// The lane groups' states are merged through LDS with the same rescaling
// (out = sum_g e^(m_g - M) acc_g / sum_g e^(m_g - M) l_g) into each head's
// (acc, m, l) partial of the split.  A second kernel, one workgroup per query
// head, merges the splits the same way (the identity of attention_split.comp
// + attn_reduce.comp) and writes the output as the activation pack of the
// o-projection; it loads every split's partial while the position is in
// flight and weighs only the splits that hold positions.  The split spreads
// the K/V stream over ~256 workgroups: one CU streams only ~35 GB/s.
#include "attn_dev.h"
#include "lrs_internal.h"
#include "pack_dev.h"

namespace lrs {

constexpr int ATT_THREADS = 256;
constexpr int ATT_DEPTH = 4;    // positions per lane group with K and V loads in flight

struct AttnArgs {
    const float *q;           // [n_head * HD], RoPE applied
    const _Float16 *kc, *vc;  // this layer's caches [n_kv][ctx][HD]
    float *part;              // [n_head][splits][HD + 4]: acc[HD], m, l
    const uint32_t *step;     // {token, pos}: attends positions 0..pos
    uint32_t n_head, n_kv, ctx, splits;
    float scale;
};

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2_t as_h2(uint32_t v) {
    half2_t r;
    __builtin_memcpy(&r, &v, 4);
    return r;
}

template <int HD, int REP>
__global__ __launch_bounds__(ATT_THREADS) void k_attn(AttnArgs a) {
    constexpr int LP = HD / 8;              // lanes per position
    constexpr int NG = ATT_THREADS / LP;    // lane groups per workgroup
    static_assert(REP * NG <= ATT_THREADS, "one thread per (query head, lane group) in the merge");
    __shared__ float sm[NG][REP], sl[NG][REP], sw[NG][REP];
    __shared__ float sacc[NG][REP][HD];
    const uint32_t tid = threadIdx.x, sub = tid % LP, grp = tid / LP;
    const uint32_t sp = blockIdx.x, kh = blockIdx.y, h0 = kh * REP;
    const uint32_t S = a.splits * ATT_BLOCK;  // positions between two blocks of a split
    // position of this lane group's k-th slot: slot t = k NG + grp of the
    // split is position t % ATT_BLOCK of the split's block t / ATT_BLOCK
    auto slot_pos = [&](uint32_t k) {
        const uint32_t t = k * NG + grp;
        return sp * ATT_BLOCK + (t / ATT_BLOCK) * S + t % ATT_BLOCK;
    };
    const _Float16 *kb = a.kc + (size_t)kh * a.ctx * HD + 8 * sub;
    const _Float16 *vb = a.vc + (size_t)kh * a.ctx * HD + 8 * sub;

    // q of the REP heads, and K and V of this lane group's slots in the
    // split's first block, before the position is known (slots past the
    // position are in the cache allocation and are never used; the later
    // blocks wait for the position, so a short context reads no more than
    // one block per split)
    float4 qx[REP][2];
#pragma unroll
    for (int r = 0; r < REP; r++) {
        const float4 *qp = reinterpret_cast<const float4 *>(a.q + (size_t)(h0 + r) * HD + 8 * sub);
        qx[r][0] = qp[0];
        qx[r][1] = qp[1];
    }
    uint4 kr[ATT_DEPTH], vr[ATT_DEPTH];
#pragma unroll
    for (int i = 0; i < ATT_DEPTH; i++) {
        const uint32_t p = slot_pos(i);
        if (i * NG + grp < ATT_BLOCK && p < a.ctx) {
            kr[i] = *reinterpret_cast<const uint4 *>(kb + (size_t)p * HD);
            vr[i] = *reinterpret_cast<const uint4 *>(vb + (size_t)p * HD);
        }
    }
    const uint32_t L = a.step[1] + 1;
    if (sp * ATT_BLOCK >= L) return;  // no position in this split (the combine skips it)
#pragma unroll
    for (int i = 0; i < ATT_DEPTH; i++) {
        const uint32_t p = slot_pos(i);
        if (i * NG + grp >= ATT_BLOCK && p < L) {
            kr[i] = *reinterpret_cast<const uint4 *>(kb + (size_t)p * HD);
            vr[i] = *reinterpret_cast<const uint4 *>(vb + (size_t)p * HD);
        }
    }

    // q / 2^e as f16 hi + lo pairs (dims 8 sub .. 8 sub + 7), 2^e >= max |q|
    // of the head so both halves stay in f16 range; the score is rescaled
    // by 2^e * scale (exact power of two, then the reference's 1/sqrt(HD))
    half2_t qh[REP][4], ql[REP][4];
    float sscale[REP];
#pragma unroll
    for (int r = 0; r < REP; r++) {
        const float4 x0 = qx[r][0], x1 = qx[r][1];
        float qv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        float qm = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) qm = fmaxf(qm, fabsf(qv[i]));
        qm = group_max<LP>(qm);
        int e;
        frexpf(qm, &e);
        e = e < -60 ? -60 : e;
#pragma unroll
        for (int i = 0; i < 8; i++) qv[i] = ldexpf(qv[i], -e);
        sscale[r] = ldexpf(1.0f, e) * a.scale;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const _Float16 x0h = (_Float16)qv[2 * i], x1h = (_Float16)qv[2 * i + 1];
            qh[r][i] = half2_t{x0h, x1h};
            ql[r][i] = half2_t{(_Float16)(qv[2 * i] - (float)x0h), (_Float16)(qv[2 * i + 1] - (float)x1h)};
        }
    }

    // online softmax over this lane group's positions (attention.rs:120-166)
    float m[REP], l[REP], acc[REP][8];
#pragma unroll
    for (int r = 0; r < REP; r++) {
        m[r] = -INFINITY;
        l[r] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) acc[r][e] = 0.f;
    }
    // slot positions grow with the slot, so the first slot past L ends the walk
    for (uint32_t k0 = 0; slot_pos(k0) < L; k0 += ATT_DEPTH) {
#pragma unroll
        for (int i = 0; i < ATT_DEPTH; i++) {
            const uint32_t p = slot_pos(k0 + i);
            if (p < L) {  // uniform within the lane group
                const uint4 k = kr[i], v = vr[i];
                const uint32_t pn = slot_pos(k0 + i + ATT_DEPTH);
                if (pn < L) {
                    kr[i] = *reinterpret_cast<const uint4 *>(kb + (size_t)pn * HD);
                    vr[i] = *reinterpret_cast<const uint4 *>(vb + (size_t)pn * HD);
                }
                const uint32_t kw[4] = {k.x, k.y, k.z, k.w};
                const _Float16 *vh = reinterpret_cast<const _Float16 *>(&v);
                float vf[8];
#pragma unroll
                for (int e = 0; e < 8; e++) vf[e] = (float)vh[e];
#pragma unroll
                for (int r = 0; r < REP; r++) {
                    float s = 0.f;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        s = __builtin_amdgcn_fdot2(ql[r][j], as_h2(kw[j]), s, false);
                        s = __builtin_amdgcn_fdot2(qh[r][j], as_h2(kw[j]), s, false);
                    }
                    s = group_sum<LP>(s) * sscale[r];  // attention.rs: (q.k) / sqrt(head_dim)
                    const float mn = fmaxf(m[r], s);
                    const float c = expf(m[r] - mn), pe = expf(s - mn);
                    l[r] = fmaf(l[r], c, pe);
#pragma unroll
                    for (int e = 0; e < 8; e++) acc[r][e] = fmaf(pe, vf[e], acc[r][e] * c);
                    m[r] = mn;
                }
            }
        }
    }
    // merge the lane groups' states through LDS
    if (sub == 0) {
#pragma unroll
        for (int r = 0; r < REP; r++) {
            sm[grp][r] = m[r];
            sl[grp][r] = l[r];
        }
    }
#pragma unroll
    for (int r = 0; r < REP; r++)
#pragma unroll
        for (int e = 0; e < 8; e++) sacc[grp][r][8 * sub + e] = acc[r][e];
    __syncthreads();
    if (tid < REP * NG) {
        // thread (head r, lane group g), whole groups of NG aligned lanes:
        // split max M of head r, weight e^(m_g - M) of group g (0 for a group
        // with no position) and the denominator sum_g w_g l_g
        const uint32_t r = tid / NG, g = tid % NG;
        const float mg = sm[g][r];
        const float M = group_max<NG>(mg);
        const float w = mg == -INFINITY ? 0.f : expf(mg - M);
        sw[g][r] = w;
        const float den = group_sum<NG>(w * sl[g][r]);
        if (g == 0) {
            float *pp = a.part + ((size_t)(h0 + r) * a.splits + sp) * (HD + 4);
            pp[HD] = M;
            pp[HD + 1] = den;
        }
    }
    __syncthreads();
    for (uint32_t i = tid; i < REP * HD; i += ATT_THREADS) {
        const uint32_t r = i / HD, d = i % HD;
        float num = 0.f;
#pragma unroll
        for (int g = 0; g < NG; g++) num = fmaf(sw[g][r], sacc[g][r][d], num);
        a.part[((size_t)(h0 + r) * a.splits + sp) * (HD + 4) + d] = num;  // relative to the split max
    }
}

// combine of the split partials of head blockIdx.x (attn_combine_head)
template <int HD>
__global__ __launch_bounds__(HD) void k_attn_combine(const float *__restrict__ part, uint32_t splits,
                                                     const uint32_t *__restrict__ step,
                                                     const float *__restrict__ gate,
                                                     uint32_t gstride, XPack out) {
    extern __shared__ __attribute__((aligned(16))) float pl[];  // [splits][HD + 4]
    __shared__ float wsh[64], red[1];
    attn_combine_head<false>(part, splits, HD, step, gate, gstride, out, blockIdx.x, pl, wsh, red);
}

// split count: at most one workgroup per CU (256 >= splits x KV heads), at
// most 40 (measured on the decode benches at 511..640 positions: 8 KV heads
// x 128 dims run 32 splits, 40 / 48 / 64 are slower there, 16 ties; 4 KV
// heads x 256 dims take 11.8 us with 32 splits, 10.3 with 40, 10.4 with 48,
// and 64 is slower).  Blocks of 16 positions: a context of L < 16 * splits
// positions runs ceil(L / 16) splits (measured on the config-3 decode as
// contiguous ranges of at least 16 positions per split: 32 and 64 are no
// faster at 512 positions, 128 and 256 slower)

uint32_t attn_splits(uint32_t n_kv) {
    const uint32_t S = 256 / n_kv;
    return S < 1 ? 1 : S > 40 ? 40 : S;
}

using AttnFn = void (*)(AttnArgs);
template <int HD>
static AttnFn pick_rep(uint32_t rep) {
    switch (rep) {
    case 1: return k_attn<HD, 1>;
    case 2: return k_attn<HD, 2>;
    case 3: return k_attn<HD, 3>;
    case 4: return k_attn<HD, 4>;
    case 5: return k_attn<HD, 5>;
    case 6: return k_attn<HD, 6>;
    case 7: return k_attn<HD, 7>;
    case 8: return k_attn<HD, 8>;
    default: return nullptr;
    }
}

hipError_t launch_attention(const float *q, const _Float16 *kc, const _Float16 *vc, float *part,
                            XPack out, const uint32_t *step, uint32_t n_head, uint32_t n_kv,
                            uint32_t head_dim, uint32_t ctx, uint32_t splits, hipStream_t s,
                            const float *gate, uint32_t gstride, bool combine) {
    AttnArgs a;
    a.q = q;
    a.kc = kc;
    a.vc = vc;
    a.part = part;
    a.step = step;
    a.n_head = n_head;
    a.n_kv = n_kv;
    a.ctx = ctx;
    a.splits = splits;
    a.scale = 1.0f / sqrtf((float)head_dim);
    if (n_kv == 0 || n_head % n_kv || splits == 0) return hipErrorInvalidValue;
    const uint32_t rep = n_head / n_kv;
    const dim3 grid(splits, n_kv);
    AttnFn fn = nullptr;
    switch (head_dim) {
    case 64: fn = pick_rep<64>(rep); break;
    case 128: fn = pick_rep<128>(rep); break;
    case 256: fn = pick_rep<256>(rep); break;
    default: return hipErrorInvalidValue;
    }
    if (!fn) return hipErrorInvalidValue;
    hipLaunchKernelGGL(fn, grid, dim3(ATT_THREADS), 0, s, a);
    if (!combine) return hipGetLastError();  // the o launch merges the splits (k_mq_ao)
    const size_t cl = (size_t)splits * (head_dim + 4) * sizeof(float);
    switch (head_dim) {
    case 64: hipLaunchKernelGGL(k_attn_combine<64>, dim3(n_head), dim3(64), cl, s, part, splits, step, gate, gstride, out); break;
    case 128: hipLaunchKernelGGL(k_attn_combine<128>, dim3(n_head), dim3(128), cl, s, part, splits, step, gate, gstride, out); break;
    default: hipLaunchKernelGGL(k_attn_combine<256>, dim3(n_head), dim3(256), cl, s, part, splits, step, gate, gstride, out); break;
    }
    return hipGetLastError();
}

}  // namespace lrs
