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
template <int HD, int REP, bool QP = false, bool DQ = false>
__global__ __launch_bounds__(ATT_THREADS) void k_attn(AttnArgs a) {
    constexpr int LP = HD / 8;              // lanes per position
    constexpr int NG = ATT_THREADS / LP;    // lane groups per workgroup
    // DIST: lane group g < REP splits query head g alone and shares it
    // through LDS (QP always; DQ: the same for the dense model's q)
    constexpr bool DIST = QP || DQ;
    static_assert(REP * NG <= ATT_THREADS, "one thread per (query head, lane group) in the merge");
    static_assert(!QP || REP < NG, "QP: a lane group per query head and one for k");
    __shared__ float sm[NG][REP], sl[NG][REP], sw[NG][REP];
    __shared__ float sacc[NG][REP][HD];
    // DIST: the query heads' hi / lo pairs and score factors; QP: the current K / V row
    __shared__ uint4 sqp[DIST ? REP : 1][2][LP];
    __shared__ float ssc[DIST ? REP : 1];
    __shared__ uint4 skv[QP ? 2 : 1][LP];
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
    if (sp * ATT_BLOCK >= L) return;  // no position in this split (the combine skips it)
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
// QP needs a lane group per query head plus one for k: REP < 2048 / HD
template <int HD, int REP, bool QP, bool DQ>
static AttnFn rep_fn() {
    if constexpr (QP && REP >= ATT_THREADS / (HD / 8)) return nullptr;
    else return k_attn<HD, REP, QP, DQ>;
}
template <int HD, bool QP = false, bool DQ = false>
static AttnFn pick_rep(uint32_t rep) {
    switch (rep) {
    case 1: return rep_fn<HD, 1, QP, DQ>();
    case 2: return rep_fn<HD, 2, QP, DQ>();
    case 3: return rep_fn<HD, 3, QP, DQ>();
    case 4: return rep_fn<HD, 4, QP, DQ>();
    case 5: return rep_fn<HD, 5, QP, DQ>();
    case 6: return rep_fn<HD, 6, QP, DQ>();
    case 7: return rep_fn<HD, 7, QP, DQ>();
    case 8: return rep_fn<HD, 8, QP, DQ>();
    default: return nullptr;
    }
}
template <int HD>
static AttnFn pick_hd(uint32_t rep, bool qp, bool dq) {
    return qp ? pick_rep<HD, true>(rep) : dq ? pick_rep<HD, false, true>(rep) : pick_rep<HD>(rep);
}

bool attn_qp_supported(uint32_t head_dim, uint32_t rep) {
    return (head_dim == 64 || head_dim == 128 || head_dim == 256) && rep >= 1 && rep <= 8 &&
           rep < ATT_THREADS / (head_dim / 8);
}

hipError_t launch_attention(const float *q, const _Float16 *kc, const _Float16 *vc, float *part,
                            XPack out, const uint32_t *step, uint32_t n_head, uint32_t n_kv,
                            uint32_t head_dim, uint32_t ctx, uint32_t splits, hipStream_t s,
                            const float *gate, uint32_t gstride, bool combine, const QkPrep *qp,
                            bool dq) {
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
    if (qp) {
        // the QK-norm + RoPE inputs
        if (!qp->qg || !qp->kb || !qp->vb || !qp->q_norm || !qp->k_norm || !qp->rope || !qp->kc ||
            !qp->vc || !attn_qp_supported(head_dim, rep))
            return hipErrorInvalidValue;
        a.qp = *qp;
    }
    switch (head_dim) {
    case 64: fn = pick_hd<64>(rep, qp, dq); break;
    case 128: fn = pick_hd<128>(rep, qp, dq); break;
    case 256: fn = pick_hd<256>(rep, qp, dq); break;
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
