// The decode attention's split step (one workgroup: split sp of KV head kh),
// shared by the split kernel (attention.hip) and the launch that runs the
// split, the combine and the o-projection together (mq.hip).  The design is
// described at the top of attention.hip.
#pragma once

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
    QkPrep qp;                // QP kernels: the QK-norm + RoPE inputs
};

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2_t as_h2(uint32_t v) {
    half2_t r;
    __builtin_memcpy(&r, &v, 4);
    return r;
}

// QK-norm (dn_norm mode 2) + adjacent-pair RoPE (rope.comp) of one HD-wide
// row held 8 dims per lane by a lane group of LP lanes (v: dims 8 sub ..
// 8 sub + 7): v <- (v / rms(row)) * w, then (v_2i, v_2i+1) rotated by the
// angle whose cosine / sine are cs[i] / sn[i] (cos 1, sin 0 past rope_dim:
// y0 * 1 - y1 * 0 = y0 exactly, as no rotation)
template <int LP>
__device__ __forceinline__ void qk_norm_rope(float (&v)[8], const float (&w)[8], const float (&cs)[4],
                                             const float (&sn)[4], uint32_t hd, float eps) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) ss += v[e] * v[e];
    ss = group_sum<LP>(ss);
    const float sc = 1.0f / sqrtf(ss / (float)hd + eps);
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = (v[e] * sc) * w[e];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float y0 = v[2 * i], y1 = v[2 * i + 1];
        v[2 * i] = y0 * cs[i] - y1 * sn[i];
        v[2 * i + 1] = y1 * cs[i] + y0 * sn[i];
    }
}

// q / 2^e as f16 hi + lo pairs (dims 8 sub .. 8 sub + 7 of one head), 2^e
// >= max |q| of the head so both halves stay in f16 range; returns the
// score factor 2^e * scale (exact power of two, then the reference's
// 1/sqrt(HD))
template <int LP>
__device__ __forceinline__ float q_split(float (&qv)[8], half2_t (&qh)[4], half2_t (&ql)[4], float scale) {
    float qm = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) qm = fmaxf(qm, fabsf(qv[i]));
    qm = group_max<LP>(qm);
    int e;
    frexpf(qm, &e);
    e = e < -60 ? -60 : e;
#pragma unroll
    for (int i = 0; i < 8; i++) qv[i] = ldexpf(qv[i], -e);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const _Float16 x0h = (_Float16)qv[2 * i], x1h = (_Float16)qv[2 * i + 1];
        qh[i] = half2_t{x0h, x1h};
        ql[i] = half2_t{(_Float16)(qv[2 * i] - (float)x0h), (_Float16)(qv[2 * i + 1] - (float)x1h)};
    }
    return ldexpf(1.0f, e) * scale;
}

typedef const float __attribute__((address_space(1))) gfloat;  // global memory
typedef float f4v __attribute__((ext_vector_type(4)));
template <typename T>
__device__ __forceinline__ void ld8(float (&v)[8], T *p) {
    typedef std::conditional_t<std::is_same_v<T, gfloat>, const __attribute__((address_space(1))) f4v,
                               const f4v>
        V;
    const f4v a = reinterpret_cast<V *>(p)[0], b = reinterpret_cast<V *>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// LDS of one split workgroup
template <int HD, int REP, bool QP, bool DQ>
struct AttnLds {
    static constexpr int LP = HD / 8, NG = ATT_THREADS / LP;
    static constexpr bool DIST = QP || DQ;
    float sm[NG][REP], sl[NG][REP], sw[NG][REP];
    float sacc[NG][REP][HD];
    // DIST: the query heads' hi / lo pairs and score factors; QP: the current K / V row
    uint4 sqp[DIST ? REP : 1][2][LP];
    float ssc[DIST ? REP : 1];
    uint4 skv[QP ? 2 : 1][LP];
};

// a partial's store: AG, agent scope (written through to memory, for a
// reader in the same launch)
template <bool AG>
__device__ __forceinline__ void st_part(float *p, float v) {
    if constexpr (AG) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *p = v;
}

// QP: the hybrid's gated attention with its QK-norm + RoPE in the split (no
// separate launch).  Lane group g < REP normalises and rotates query head
// h0 + g from the projection's rows (a.qp.qg: query then gate, 2 HD per
// head) and splits it into the f16 hi / lo pairs of the scores; lane group
// REP, in the split that owns the current position's block, builds that
// position's K / V row from a.qp.kb / vb (k normalised and rotated), rounded
// to f16 as the cache holds it, and writes it to the cache (no other split
// reads that position).  Both go through LDS to every lane group; the
// current row replaces what its slot's load returned.  The rotation's
// cosines / sines for the position come from a.qp.rope (written by the
// token's first kernel), so every lane group does one row's work.  DQ (q
// already normalised and rotated, the dense model): lane group g < REP
// alone splits query head g into its f16 pairs and shares them through LDS,
// as QP does; without either, every lane group splits every head itself.
//
// Split sp of KV head kh (threads 0..ATT_THREADS-1 of the workgroup): the
// REP query heads' partials of the split's positions; false (nothing
// written) when the split holds no position
template <int HD, int REP, bool QP, bool DQ, bool AG>
__device__ __forceinline__ bool attn_split(const AttnArgs &a, uint32_t sp, uint32_t kh,
                                           AttnLds<HD, REP, QP, DQ> &sh) {
    constexpr int LP = HD / 8;              // lanes per position
    constexpr int NG = ATT_THREADS / LP;    // lane groups per workgroup
    // DIST: lane group g < REP splits query head g alone and shares it
    // through LDS (QP always; DQ: the same for the dense model's q)
    constexpr bool DIST = QP || DQ;
    static_assert(REP * NG <= ATT_THREADS, "one thread per (query head, lane group) in the merge");
    static_assert(!QP || REP < NG, "QP: a lane group per query head and one for k");
    auto &sm = sh.sm, &sl = sh.sl, &sw = sh.sw;
    auto &sacc = sh.sacc;
    auto &sqp = sh.sqp;
    auto &ssc = sh.ssc;
    auto &skv = sh.skv;
    const uint32_t tid = threadIdx.x, sub = tid % LP, grp = tid / LP;
    const uint32_t h0 = kh * REP;
    const uint32_t S = a.splits * ATT_BLOCK;  // positions between two blocks of a split
    // position of this lane group's k-th slot: slot t = k NG + grp of the
    // split is position t % ATT_BLOCK of the split's block t / ATT_BLOCK
    auto slot_pos = [&](uint32_t k) {
        const uint32_t t = k * NG + grp;
        return sp * ATT_BLOCK + (t / ATT_BLOCK) * S + t % ATT_BLOCK;
    };
    const _Float16 *kb = a.kc + (size_t)kh * a.ctx * HD + 8 * sub;
    const _Float16 *vb = a.vc + (size_t)kh * a.ctx * HD + 8 * sub;

    // q of the REP heads (QP: this lane group's row and its inputs), and K
    // and V of this lane group's slots in the split's first block, before
    // the position is known (slots past the position are in the cache
    // allocation and are never used; the later blocks wait for the
    // position, so a short context reads no more than one block per split)
    const uint32_t pos0 = DIST ? a.step[1] : 0;
    float4 qx[DIST ? 1 : REP][2];
    const uint32_t role = grp < REP ? grp : REP;  // DIST: query head, or REP = k (QP) / none
    float rw[8] = {}, nw[8] = {}, vnew[8] = {}, cs[4] = {}, sn[4] = {};
    if constexpr (DIST) __builtin_assume(tid < ATT_THREADS);
    if constexpr (QP) {
        // the pointers as values (else the compiler selects between the
        // argument slots and loads the pointer per lane before the data),
        // kept global so the loads count on the vector memory counter alone
        uint64_t qg = (uint64_t)a.qp.qg, kbp = (uint64_t)a.qp.kb, qn = (uint64_t)a.qp.q_norm,
                 kn = (uint64_t)a.qp.k_norm;
        __asm__("" : "+s"(qg), "+s"(kbp), "+s"(qn), "+s"(kn));
        const gfloat *row = role < REP ? (const gfloat *)qg + (size_t)(h0 + role) * 2 * HD
                                       : (const gfloat *)kbp + (size_t)kh * HD;
        ld8(rw, row + 8 * sub);
        ld8(nw, (const gfloat *)(role < REP ? qn : kn) + 8 * sub);
        ld8(vnew, a.qp.vb + (size_t)kh * HD + 8 * sub);
        const float4 *rp = reinterpret_cast<const float4 *>(a.qp.rope + 4 * sub);  // {cos, sin} x 4
        const float4 r0 = rp[0], r1 = rp[1];
        cs[0] = r0.x; sn[0] = r0.y; cs[1] = r0.z; sn[1] = r0.w;
        cs[2] = r1.x; sn[2] = r1.y; cs[3] = r1.z; sn[3] = r1.w;
    } else if constexpr (DQ) {
        // this lane group's head (groups past REP load the last one, unused)
        const uint32_t hq = role < REP ? role : REP - 1;
        ld8(rw, a.q + (size_t)(h0 + hq) * HD + 8 * sub);
    } else {
#pragma unroll
        for (int r = 0; r < REP; r++) {
            const float4 *qp = reinterpret_cast<const float4 *>(a.q + (size_t)(h0 + r) * HD + 8 * sub);
            qx[r][0] = qp[0];
            qx[r][1] = qp[1];
        }
    }
    uint4 kr[ATT_DEPTH], vr[ATT_DEPTH];
#pragma unroll
    for (int i = 0; i < ATT_DEPTH; i++) {
        const uint32_t p = slot_pos(i);
        if (DIST && (i + 1) * NG <= ATT_BLOCK) {
            // DIST: slots of the first block in every lane group, loaded with
            // no branch (position clamped into the cache), so the row loads
            // before them can be waited for alone and the q work (QP: the
            // QK-norm + RoPE) overlaps these loads
            const uint32_t pc = p < a.ctx ? p : a.ctx - 1;
            kr[i] = *reinterpret_cast<const uint4 *>(kb + (size_t)pc * HD);
            vr[i] = *reinterpret_cast<const uint4 *>(vb + (size_t)pc * HD);
        } else if (i * NG + grp < ATT_BLOCK && p < a.ctx) {
            kr[i] = *reinterpret_cast<const uint4 *>(kb + (size_t)p * HD);
            vr[i] = *reinterpret_cast<const uint4 *>(vb + (size_t)p * HD);
        }
    }
    // DIST: the position was read first (a scalar load); the barrier keeps
    // the compiler from sinking the loads above below the exit, which
    // would issue them only once the position is known
    if constexpr (DIST) __asm__ volatile("" ::: "memory");
    const uint32_t L = (DIST ? pos0 : a.step[1]) + 1;
    if (sp * ATT_BLOCK >= L) return false;  // no position in this split (the combine skips it)
    const bool owner = QP && ((L - 1) / ATT_BLOCK) % a.splits == sp;  // uniform over the workgroup
    // (QP: the current position's slot, if loaded here, is replaced below)
#pragma unroll
    for (int i = 0; i < ATT_DEPTH; i++) {
        const uint32_t p = slot_pos(i);
        if (i * NG + grp >= ATT_BLOCK && p < L) {
            kr[i] = *reinterpret_cast<const uint4 *>(kb + (size_t)p * HD);
            vr[i] = *reinterpret_cast<const uint4 *>(vb + (size_t)p * HD);
        }
    }


    // q / 2^e as f16 hi + lo pairs (dims 8 sub .. 8 sub + 7) and the score
    // factors 2^e * scale (q_split)
    half2_t qh[REP][4], ql[REP][4];
    float sscale[REP];
    uint4 kcur = {}, vcur = {};
    if constexpr (DIST) {
        if constexpr (QP) qk_norm_rope<LP>(rw, nw, cs, sn, HD, a.qp.eps);
        if (role < REP) {
            half2_t h[4], lo[4];
            const float f = q_split<LP>(rw, h, lo, a.scale);
            sqp[role][0][sub] = __builtin_bit_cast(uint4, h);
            sqp[role][1][sub] = __builtin_bit_cast(uint4, lo);
            if (sub == 0) ssc[role] = f;
        }
        if constexpr (QP) {
            if (owner && grp == REP) {
                uint32_t kw[4], vw[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    kw[i] = __builtin_bit_cast(uint32_t, half2_t{(_Float16)rw[2 * i], (_Float16)rw[2 * i + 1]});
                    vw[i] = __builtin_bit_cast(uint32_t, half2_t{(_Float16)vnew[2 * i], (_Float16)vnew[2 * i + 1]});
                }
                const uint4 k4 = make_uint4(kw[0], kw[1], kw[2], kw[3]), v4 = make_uint4(vw[0], vw[1], vw[2], vw[3]);
                skv[0][sub] = k4;
                skv[1][sub] = v4;
                const size_t o = ((size_t)kh * a.ctx + (L - 1)) * HD + 8 * sub;
                *reinterpret_cast<uint4 *>(a.qp.kc + o) = k4;
                *reinterpret_cast<uint4 *>(a.qp.vc + o) = v4;
            }
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < REP; r++) {
            const uint4 h = sqp[r][0][sub], lo = sqp[r][1][sub];
            const half2_t *hp = reinterpret_cast<const half2_t *>(&h), *lp = reinterpret_cast<const half2_t *>(&lo);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                qh[r][i] = hp[i];
                ql[r][i] = lp[i];
            }
            sscale[r] = ssc[r];
        }
        if (QP && owner) {
            kcur = skv[0][sub];
            vcur = skv[1][sub];
        }
    } else {
#pragma unroll
        for (int r = 0; r < REP; r++) {
            const float4 x0 = qx[r][0], x1 = qx[r][1];
            float qv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            sscale[r] = q_split<LP>(qv, qh[r], ql[r], a.scale);
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
                uint4 k = kr[i], v = vr[i];
                if constexpr (QP) {
                    // the current position's slot from the row built above
                    // (its cache load may predate the row's store), blended
                    // by an opaque mask: a select lets the compiler move the
                    // f16 unpacking of every slot into its load branch and
                    // wait for each early load before it reads the position
                    uint32_t msk = owner && p == L - 1 ? ~0u : 0u;
                    __asm__("" : "+v"(msk));
                    k.x = (k.x & ~msk) | (kcur.x & msk);
                    k.y = (k.y & ~msk) | (kcur.y & msk);
                    k.z = (k.z & ~msk) | (kcur.z & msk);
                    k.w = (k.w & ~msk) | (kcur.w & msk);
                    v.x = (v.x & ~msk) | (vcur.x & msk);
                    v.y = (v.y & ~msk) | (vcur.y & msk);
                    v.z = (v.z & ~msk) | (vcur.z & msk);
                    v.w = (v.w & ~msk) | (vcur.w & msk);
                }
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
                    if (k0 == 0 && i == 0) {
                        // the lane group's first position (slot 0 is its
                        // smallest): the update below from m = -inf, l = 0,
                        // acc = 0 gives exactly m = s, l = 1, acc = v
                        m[r] = s;
                        l[r] = 1.f;
#pragma unroll
                        for (int e = 0; e < 8; e++) acc[r][e] = vf[e];
                        continue;
                    }
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
            st_part<AG>(pp + HD, M);
            st_part<AG>(pp + HD + 1, den);
        }
    }
    __syncthreads();
    for (uint32_t i = tid; i < REP * HD; i += ATT_THREADS) {
        const uint32_t r = i / HD, d = i % HD;
        float num = 0.f;
#pragma unroll
        for (int g = 0; g < NG; g++) num = fmaf(sw[g][r], sacc[g][r][d], num);
        st_part<AG>(a.part + ((size_t)(h0 + r) * a.splits + sp) * (HD + 4) + d, num);  // relative to the split max
    }
    return true;
}

}  // namespace lrs
