// Internal declarations shared by the HIP translation units of liblrs.so.
// gfx950 (CDNA4, wave64) only.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/lrs.h"
#include "tiled.h"
#include "mq_args.h"

namespace lrs {

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------
void set_error(const std::string &msg);
int fail(int code, const std::string &msg);
int hip_fail(hipError_t e, const char *what);

#define LRS_HIP(call)                                          \
    do {                                                       \
        hipError_t e_ = (call);                                \
        if (e_ != hipSuccess) return ::lrs::hip_fail(e_, #call); \
    } while (0)

// ---------------------------------------------------------------------------
// GGUF block geometry (crates/gguf/src/types.rs:30-78)
// ---------------------------------------------------------------------------
constexpr uint32_t T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14;

__host__ __device__ inline int64_t block_elems(uint32_t t) {
    switch (t) {
    case T_F32: case T_F16: return 1;
    case T_Q4_0: case T_Q8_0: return 32;
    case T_Q4_K: case T_Q5_K: case T_Q6_K: return 256;
    default: return -1;
    }
}
__host__ __device__ inline int64_t block_bytes(uint32_t t) {
    switch (t) {
    case T_F32: return 4;
    case T_F16: return 2;
    case T_Q4_0: return 18;
    case T_Q8_0: return 34;
    case T_Q4_K: return 144;
    case T_Q5_K: return 176;
    case T_Q6_K: return 210;
    default: return -1;
    }
}

// ---------------------------------------------------------------------------
// Device layout of a resident weight (n_out rows x nb GGUF blocks per row):
//   Q4_K / Q5_K / Q6_K / Q8_0: the tiled layout of tiled.h (16-row tiles,
//         one contiguous chunk per unit, GGUF bytes only)
//   Q4_0 / F32 / F16: the raw GGUF bytes (dequant / embedding only)
// ---------------------------------------------------------------------------
struct WeightView {
    const uint8_t *q;
    uint32_t type, n_in, n_out, nb;  // nb = GGUF blocks per row
};

// device bytes of a weight's allocation
inline size_t weight_dev_bytes(uint32_t t, uint32_t n_in, uint32_t n_out) {
    if (is_tiled(t)) return tbytes(t, n_in, n_out);
    return (size_t)(n_in / block_elems(t)) * n_out * block_bytes(t);
}

// launch wrappers implemented in the .hip files (all enqueue on `s`)
hipError_t launch_repack_from_gguf(const uint8_t *gguf_dev, WeightView w, uint8_t *q,
                                   hipStream_t s);
hipError_t launch_repack_to_gguf(WeightView w, uint8_t *gguf_dev, hipStream_t s);
hipError_t launch_generate(WeightView w, uint8_t *q, uint64_t seed, int mode, float d_lo,
                           float d_hi, hipStream_t s);
hipError_t launch_dequant(WeightView w, float *out, hipStream_t s);
hipError_t launch_dequant_rows(WeightView w, const uint32_t *rows_dev, uint32_t n_rows,
                               float *out, hipStream_t s);
// matrix-core matvec (mq.hip)
hipError_t launch_xpack(const float *x, const float *nw, uint32_t n, uint32_t nxb, XPack p,
                        hipStream_t s,
                        float *xsq = nullptr);
// gates (MQ_STORE, two Q4_K segments, shape (1, 2, 4, 2) only): one more
// workgroup per value head computes the delta net's gate projections into
// gates->out (the step then reads them; dn_dev.h)
struct DnGateArgs;
hipError_t launch_mq(const MqArgs &a, uint32_t t0, uint32_t t1, MqGeom g, int epi, hipStream_t s,
                     uint32_t *wgs_out = nullptr, uint32_t *keys_per_wg = nullptr,
                     const DnGateArgs *gates = nullptr);
bool mq_gates_supported(uint32_t t0, uint32_t t1, const MqGeom &g);
bool mq_geom_supported(const MqGeom &g);
// the attention combine and the o-projection (RESID) in one launch
bool mq_ao_supported(uint32_t t, uint32_t n_in, uint32_t rows, uint32_t head_dim, uint32_t splits,
                     uint32_t n_head);
hipError_t launch_mq_ao(const MqArgs &a, const AoArgs &c, uint32_t t, hipStream_t s);
struct QkPrep;
// the attention split, its combine and the o-projection in one launch
// (k_mq_sao); c.n_prod = n_head, c.sflag: 64 zeroed words per query head
bool attn_ao_supported(uint32_t t, uint32_t n_in, uint32_t rows, uint32_t head_dim, uint32_t splits,
                       uint32_t n_head, uint32_t n_kv, bool qp, bool dq);
hipError_t launch_attn_ao(const float *q, const _Float16 *kc, const _Float16 *vc, uint32_t n_kv,
                          uint32_t ctx, const QkPrep *qp, bool dq, const MqArgs &a, const AoArgs &c,
                          uint32_t t, hipStream_t s);
MqGeom store_geom(uint32_t t, uint32_t n_in, uint32_t n_out);
// plain-matvec launch shape override (tiles per wave, tile groups, K-slices; all 0 = automatic)
int set_matvec_geom(int tpw, int tg, int ks);
// 32-element pack blocks of a K-long input of a weight of type t (K padded to units)
inline uint32_t pack_blocks(uint32_t t, uint32_t n_in) {
    return is_tiled(t) ? tunits(t, n_in) * tunit_elems(t) / 32 : (n_in + 31) / 32;
}
// reduces argmax keys (amax_key) into step {token, pos, n} and out[n]
hipError_t launch_argmax_finish(const unsigned long long *keys, uint32_t n, uint32_t *step,
                                uint32_t *out, uint32_t out_cap, hipStream_t s);
// y[c] = W x[c] for cols columns: when matvec_packs_in_kernel, up to 8
// columns per launch share each weight load and every workgroup packs its
// input columns itself (`pack` unused, may be null); otherwise the staged
// form below with `pack` (xpack_bytes of the weight)
hipError_t launch_matvec(WeightView w, const float *x, float *y, uint32_t cols, void *pack,
                         hipStream_t s);
bool matvec_packs_in_kernel(WeightView w, uint32_t cols);
// the staged form: each column packed into `pack` by its own launch, then one
// matvec launch per column over that pack (same results)
hipError_t launch_matvec_staged(WeightView w, const float *x, float *y, uint32_t cols, void *pack,
                                hipStream_t s);
// Q8_0 activation quantization (reference CPU forward): GGUF Q8_0 bytes to
// q8 (n / 32 blocks) and / or the matvec pack p (nxb blocks) when non-null
hipError_t launch_q8act(const float *x, uint32_t n, uint32_t nxb, int half_even, uint8_t *q8,
                        XPack p, hipStream_t s);
// Q8_0-rounded pack (p.q8 set) of rmsnorm(x) * w, n a multiple of 256
hipError_t launch_q8norm(const float *x, const float *w, uint32_t n, float eps, XPack p,
                         hipStream_t s);
// launch_matvec with each column rounded to Q8_0 first (Q8_0 weights only)
hipError_t launch_matvec_actq(WeightView w, const float *x, float *y, uint32_t cols, void *pack,
                              int half_even, hipStream_t s);
// Y[M][ldy] = A[M][K] W^T on the matrix cores; A given as bf16 planes
// (prec 1: hi only; 3: hi + lo, three products) from launch_split_bf16
// work: gemm_work_bytes(M, N, K, prec) of scratch for the K-sliced form (null: one slice)
// ks_out: when given, a K split leaves its ks_out slices of [M][N] partials in
// work for the caller to reduce (ks_out 1: y written directly)
hipError_t launch_gemm(WeightView w, const __bf16 *ahi, const __bf16 *alo, float *y, uint32_t M,
                       uint32_t ldy, int prec, hipStream_t s, bool accum = false,
                       float *work = nullptr, uint32_t *ks_out = nullptr);
size_t gemm_work_bytes(uint32_t M, uint32_t N, uint32_t K, int prec);
// several weights over the same A in one launch (their output tiles side by
// side; y[i] [M][ldy[i]]): at most 3, the same n_in, at most two types with
// the first type's weights first and only the pairs the kernel is built for
// (one type; Q4_K or Q5_K then Q6_K); no K split
bool gemm_segs_supported(const WeightView *w, uint32_t nseg);
// output tiles (workgroups without a K split) of an M x N GEMM
uint32_t gemm_out_tiles(uint32_t M, uint32_t N, int prec);
hipError_t launch_gemm_segs(const WeightView *w, float *const *y, const uint32_t *ldy, uint32_t nseg,
                            const __bf16 *ahi, const __bf16 *alo, uint32_t M, int prec,
                            hipStream_t s, bool accum = false, float *work = nullptr,
                            uint32_t *ks_out = nullptr);
// hi = bf16(a), lo = bf16(a - hi) (lo may be null); n a multiple of 4
hipError_t launch_split_bf16(const float *a, size_t n, __bf16 *hi, __bf16 *lo, hipStream_t s);
// batched prompt block (prefill.hip)
// Y = RMSNorm rows of X times w (Y may be null), and, when hi is given, the
// same values as the bf16 planes of launch_split_bf16 ([n][E] hi, then lo)
hipError_t launch_rmsnorm_rows(const float *X, const float *w, float eps, uint32_t E, uint32_t n,
                               float *Y, hipStream_t s, __bf16 *hi = nullptr);
// X += the ks K-slice partials part[z][n][E] (slices in order, as
// k_reduce_ks), then the RMSNorm rows of the new X times w as
// launch_rmsnorm_rows writes them (Y may be null; hi planes)
hipError_t launch_reduce_norm_rows(const float *part, uint32_t ks, float *X, const float *w,
                                   float eps, uint32_t E, uint32_t n, float *Y, __bf16 *hi,
                                   hipStream_t s);
hipError_t launch_qkv_post(const float *qt, const float *kt, const float *vt, const float *bq,
                           const float *bk, const float *bv, const float *freq, float *q,
                           _Float16 *kc, _Float16 *vc, uint32_t n, uint32_t pos0, uint32_t qd,
                           uint32_t kvd, uint32_t hd, uint32_t rope_dim, uint32_t ctx,
                           hipStream_t s);
hipError_t launch_attn_prefill(const float *q, const _Float16 *kc, const _Float16 *vc, float *out,
                               uint32_t n, uint32_t pos0, uint32_t n_head, uint32_t n_kv,
                               uint32_t hd, uint32_t ctx, hipStream_t s);
// silu(G) * U written straight to the bf16 planes of launch_split_bf16 (hi,
// then lo = hi + n); n a multiple of 4
hipError_t launch_swiglu_split(const float *G, const float *U, size_t n, __bf16 *hi,
                               hipStream_t s);
// hybrid (qwen35) mixers (dn.hip)
// QK-norm + RoPE of the hybrid's gated attention run by the split kernel
// (attention.hip, QP): query rows from the projection's q + gate rows, the
// current position's K / V rows from its k / v outputs
struct QkPrep {
    const float *qg, *kb, *vb;    // [n_head][2 HD] q | gate, [n_kv][HD] k, v
    const float *q_norm, *k_norm;  // [HD]
    const float2 *rope;            // [HD / 2] {cos, sin} of pair i at the position ({1, 0} past rope_dim)
    _Float16 *kc, *vc;             // the layer's caches: the current row is written here
    float eps;
};
// the split kernel can do the QK-norm + RoPE for this head shape
bool attn_qp_supported(uint32_t head_dim, uint32_t rep);
struct DnArgs {
    const float *qkv;           // [conv_dim] conv input (RMSNorm already applied by the matvec)
    const float *z;             // [v_heads * D] output gate
    const float *x;             // [n_embd] residual (gate projections)
    const float *attn_norm;     // [n_embd]
    const float *alpha, *beta;  // [v_heads][n_embd]
    const float *a, *dt;        // [v_heads]
    const float *conv_w;        // [conv_dim][d_conv]
    float *win;                 // [d_conv][conv_dim] ring of conv inputs
    float *state;               // [v_heads][D][D]
    const float *norm_w;        // [D]
    float *part;                // [v_heads][D/32] partial sums of squares of o
    XPack out;                  // pack of y [v_heads * D] without the head's RMS factor
    const uint32_t *step;       // {token, pos}
    uint32_t n_embd, k_heads, v_heads, d_conv;
    float eps;
    // {e^g, beta} per value head computed by the projection launch
    // (launch_mq_gates), or null: the step computes them from x, attn_norm,
    // alpha, beta, a and dt
    const float2 *gates;
};
hipError_t launch_dn_step(const DnArgs &a, uint32_t d_state, hipStream_t s);
// delta-net layer of a prompt block of nb tokens at pos0 (after the qkv / z GEMMs)
struct DnBlockArgs {
    const float *hn;            // [nb][n_embd] rmsnorm(x) * attn_norm (gate projections)
    const float *alpha, *beta, *a, *dt, *conv_w, *norm_w;
    const float *cin;           // [nb][conv_dim] conv input (qkv GEMM output)
    const float *z;             // [nb][v_heads * D] output gate (GEMM output)
    float *win, *state;         // the layer's position ring and states
    float *cout;                // [nb][conv_dim] conv + SiLU, q / k L2-normalised
    float2 *gb;                 // [nb][v_heads] {e^g, beta}
    float *o;                   // [nb][v_heads * D] rule output
    float *y;                   // [nb][v_heads * D] gated norm (ssm_out GEMM input)
    uint32_t n_embd, k_heads, v_heads, d_state, d_conv, nb, pos0;
    float eps;
};
hipError_t launch_dn_prefill(const DnBlockArgs &a, hipStream_t s);
hipError_t launch_qk_prep_rows(const float *qg, const float *kb, const float *vb, const float *q_norm,
                               const float *k_norm, const float *freq, float *q, _Float16 *kc,
                               _Float16 *vc, uint32_t nb, uint32_t pos0, uint32_t n_head,
                               uint32_t n_kv, uint32_t head_dim, uint32_t ctx, uint32_t rope_dim,
                               float eps, hipStream_t s);
hipError_t launch_gate_rows(float *att, const float *qg, uint32_t nb, uint32_t qd, uint32_t hd,
                            hipStream_t s);
hipError_t launch_qk_prep(const float *qg, const float *kb, const float *vb, const float *q_norm,
                          const float *k_norm, const float *freq, const uint32_t *step, float *q,
                          _Float16 *kc, _Float16 *vc, uint32_t n_head, uint32_t n_kv,
                          uint32_t head_dim, uint32_t ctx, uint32_t rope_dim, float eps,
                          hipStream_t s);

}  // namespace lrs

struct lrs_ctx {
    int device;
    hipStream_t stream;
    hipEvent_t ev0, ev1;
    int live_graphs = 0;  // lrs_graph objects captured on this context and not destroyed
};

struct lrs_weight {
    lrs_ctx *ctx;
    lrs::WeightView v;
    uint8_t *q;
    size_t q_alloc;
};
