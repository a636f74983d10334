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
#include "attn_split_dev.h"

namespace lrs {

template <int HD, int REP, bool QP = false, bool DQ = false>
__global__ __launch_bounds__(ATT_THREADS) void k_attn(AttnArgs a) {
    __shared__ AttnLds<HD, REP, QP, DQ> sh;
    attn_split<HD, REP, QP, DQ, false>(a, blockIdx.x, blockIdx.y, sh);
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
