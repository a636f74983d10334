// Arguments of the matrix-core matvec (mq.hip) shared with its callers.
#pragma once

#include <cstdint>

namespace lrs {

// Activation pack: a vector of n elements as three int8 digits per element
// with one power-of-two scale per 32-element block:
//   x[32b + i] ~= scale_b * (d0 * 65536 + d1 * 256 + d2),  |error| <= scale_b / 2
// where scale_b = 2^(e - 21) and 2^(e-1) <= max |x| of the block < 2^e (22
// significant bits against the block maximum).  Sums of the original f32
// elements ride along for the K-quant min / Q6_K offset terms.
//   dig  [nxb][3][32] int8: digit d of element i at 96 b + 32 d + i
//   meta [nxb] float4 {scale, sum of the 32 elements, sum of 0..15, sum of 16..31}
// With q8 set the pack instead holds the reference forward's Q8_0 rounding of
// the block (quantize_q8_0_avx2, ops.rs:284-340): digits (0, 0, q) with
// q = round-half-even(x / d) in [-128, 127], d = max |x| / 127, and meta.x =
// f16(d) widened (the sums are unused: only Q8_0 weights read such a pack).
struct XPack {
    int8_t *dig;
    float *meta;
    uint32_t q8;
};

// bytes of a pack of nxb blocks (digits, then meta, both 16-aligned)
inline size_t xpack_bytes(uint32_t nxb) { return (size_t)nxb * 96 + (size_t)nxb * 16; }
inline XPack xpack_at(void *base, uint32_t nxb) {
    XPack p;
    p.dig = reinterpret_cast<int8_t *>(base);
    p.meta = reinterpret_cast<float *>(reinterpret_cast<char *>(base) + (size_t)nxb * 96);
    p.q8 = 0;
    return p;
}

enum MqEpilogue : uint32_t {
    MQ_STORE = 0,   // out[row] = s*v (+ bias[row]); optional per-workgroup argmax keys
    MQ_QKV = 1,     // q: out f32; k, v: f16 cache append at pos; bias, adjacent-pair RoPE on q/k
    MQ_RESID = 2,   // x[row] += v; writes the pack of x_new * nw (next op's input)
    MQ_SWIGLU = 3,  // tile pairs (gate, up): a = silu(s g) * (s u); writes the pack of a
};

constexpr int MQ_MAX_SEG = 3;

// One output segment: a tiled weight (or a gate/up pair) and where its rows go.
struct MqSeg {
    const uint8_t *w;   // tiled weight
    const uint8_t *w2;  // second weight of a tile pair (SwiGLU up) or null
    uint32_t rows;      // valid rows (output index range for pairs)
    uint32_t wg0;       // first workgroup (set by the launcher)
    uint32_t kind;      // MQ_QKV: 0 = q, 1 = k, 2 = v
    const float *bias;  // [rows] or null
    float *out;         // f32 destination (STORE, QKV q)
    _Float16 *kv;       // MQ_QKV k / v: this layer's cache [kv_head][ctx][head_dim]
};

struct MqArgs {
    MqSeg seg[MQ_MAX_SEG];
    uint32_t n_seg, n_seg0;  // segments; the first n_seg0 are of the first type
    uint32_t n_in;           // K (elements)
    uint32_t nxb;            // 32-element blocks of the input pack (K padded to units)
    XPack xin;               // input pack
    // fused RMSNorm: sum(x^2) of each 32-element block of the f32 vector x whose
    // rms scales the result ([n_in / 32], written by x's producer), or null
    const float *xsq;
    float eps;
    // MQ_RESID
    float *x;                // residual [rows]
    float *xsq_out;          // sum(x_new^2) of each 32-row block of x, or null
    const float *nw;         // norm weight folded into the output pack (null: 1)
    XPack xout;              // output pack (RESID / SWIGLU)
    // MQ_QKV
    const uint32_t *step;    // device {token, pos}
    const float *freq;       // RoPE frequencies [rope_dim / 2]
    // optional: {cos, sin} of the position's angle for each pair (floats
    // 2i, 2i + 1), written by the token's first kernel with the same
    // expression (then no sincosf here)
    const float *rope;
    uint32_t head_dim, rope_dim, ctx;
    // greedy (MQ_STORE)
    unsigned long long *amax;  // [workgroups] argmax keys of the rows, or null
    // per-group RMS factor of the input (the delta net's gated norm): input
    // block b belongs to group b / gblk and is scaled by
    // 1 / sqrt(sum(gss[g*gblk .. g*gblk + gblk)) / gn + eps); null: none
    const float *gss;
    uint32_t gblk;
    float gn;
    // plain matvec of f32 columns packed in the kernel (k_mqx): column c of
    // the input at xf + c * n_in, its outputs at seg[0].out + c * ostride
    const float *xf;
    uint32_t ostride;
    // MQ_RESID / MQ_SWIGLU split over K across workgroups: xsplit workgroups
    // per 32-output block, each over its own contiguous share of the units;
    // each writes its partial sums to xpart[(block * xsplit + slice) * 32 + i]
    // (SwiGLU: * 64, gate then up) and counts itself in xcnt[block]; the last
    // to arrive adds the partials in slice order, runs the epilogue and sets
    // xcnt[block] back to 0 (so xcnt must start at zero, and does again after
    // every launch)
    // With xfull > 0 only the blocks from xfull on are split (workgroups
    // [0, xfull) take one whole block each, the rest xsplit per block): a
    // block count that is not a multiple of the CUs gets its tail spread.
    uint32_t xsplit, xfull;
    float *xpart;
    uint32_t *xcnt;
    // input pack written in the same launch (k_mq_ao): workgroup w of the
    // matvec waits until the n_wait flags wflag[64 w + i] (producer i sets
    // flag i) are all non-zero, clears them, then stages xin; a wait that
    // runs out of polls sets werr to 1 and goes on
    uint32_t *wflag, *werr;
    uint32_t n_wait;
    uint32_t wait_polls;  // the wait's poll limit (0: the default, about a second)
};

// the attention combine ahead of the o-projection in one launch (k_mq_ao):
// workgroups [0, n_prod) merge query head blockIdx.x's split partials into
// the o input pack, then each raises its flag in every matvec workgroup's
// row of the flag matrix (MqArgs::wflag)
struct AoArgs {
    const float *part;   // [n_head][splits][head_dim + 4]
    const float *gate;   // gated attention: sigmoid gate at gate[h * gstride + d], or null
    uint32_t splits, head_dim, gstride, n_prod, n_cons;
    // split, combine and o in one launch (k_mq_sao): split s of KV head g
    // raises flag s of row h of sflag (64 words per query head h of the
    // group); combine workgroup h waits for its row's live splits
    uint32_t *sflag;
    // the producers raise no flags (a test of the wait's bound: the host sets
    // it together with a small MqArgs::wait_polls, so every wait runs out)
    uint32_t no_signal;
};

// launch shape: TPW tiles per wavefront sharing the activation, TG tile
// groups and KS K-slices of wavefronts per workgroup, P units in flight;
// XS workgroups share one output block over K (MQ_RESID only; 0 or 1: one)
struct MqGeom {
    int tpw, tg, ks, p;
    int xs = 1;
    int xfull = 0;  // with xs > 1: blocks before the split tail (0: every block split)
};

}  // namespace lrs
