// model.hip — the resident batch-1 decode of a dense Llama/Qwen2 model
// (llama_model::GpuResidentDecode, crates/llama-model/src/gpu.rs:379-455, as
// implemented by llama_vulkan::ResidentForward::{decode, decode_batch, reset},
// resident_forward.rs:5223-5282), restating Model::forward
// (crates/llama-model/src/model.rs:99-266) as a fixed sequence of fused
// launches captured once in a HIP graph:
//
//   embed            x = dequant(token_embd[token])              (ops.rs:11-26)
//   per layer
//     qkv            rmsnorm(x)*attn_norm -> q,k,v (+bias) -> RoPE(q,k) ->
//                    q to f32, k/v appended to the f16 cache at pos
//     attention      split-K GQA over positions 0..pos            (attention.rs)
//     o              x += W_o attn
//     gate/up        rmsnorm(x)*ffn_norm -> silu(gate)*up          (ops.rs:983-988)
//     down           x += W_down act
//   head             rmsnorm(x)*output_norm -> logits            (model.rs:254-265)
//   [argmax]         greedy token, written back as the next step's token
//
// Every matvec reads its activation as a pack (mq_args.h) written by the op
// before it: embed and down write the pack of x * attn_norm (or output_norm
// before the head), o the pack of x * ffn_norm, gate/up the pack of the
// SwiGLU output, attention the pack of its output.  RMSNorm is applied as
// W (x * w) * s, with s = 1/sqrt(mean(x^2) + eps) reduced from x by the
// consuming kernel itself.
//
// The step's token and position live in device memory, so the same graph is
// replayed for every token; a greedy generation loop runs as back-to-back
// graph launches with no host round trip.
#include "dn_dev.h"
#include "lrs_internal.h"
#include "pack_dev.h"
#include "quant_dev.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <strings.h>
#include <vector>

namespace lrs {
uint32_t attn_splits(uint32_t n_kv);
hipError_t launch_attention(const float *q, const _Float16 *kc, const _Float16 *vc, float *part,
                            XPack out, const uint32_t *step, uint32_t n_head, uint32_t n_kv,
                            uint32_t head_dim, uint32_t ctx, uint32_t splits, hipStream_t s,
                            const float *gate = nullptr, uint32_t gstride = 0,
                            bool combine = true, const QkPrep *qp = nullptr, bool dq = false);

// x = dequant(token_embd row step[0])  (TokenEmbd::linha, gpu.rs:297-304),
// and the pack of x * nw for the first layer's q/k/v.  rope (n_pairs > 0):
// {cos, sin} of pos * freq[i] for the position step[1], pair i <
// rope_pairs (the arithmetic of the QK-prep launch's rotation), {1, 0} for
// the other pairs up to n_pairs, for the attention splits that rotate q and
// k themselves
__global__ __launch_bounds__(256) void k_embed(WeightView w, const uint32_t *__restrict__ step,
                                               const float *__restrict__ nw, float *__restrict__ x,
                                               XPack p, float *__restrict__ xsq,
                                               const float *__restrict__ freq, float2 *__restrict__ rope,
                                               uint32_t n_pairs, uint32_t rope_pairs) {
    const uint32_t be = (uint32_t)block_elems(w.type);
    uint32_t tok = step[0];
    if (tok >= w.n_out) tok = w.n_out - 1;  // ids are validated on the host
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;  // n_in is a multiple of 256
    // block types: the GGUF blocks of this workgroup's 256 elements staged
    // in LDS first, one byte per thread (each element then reads its
    // block's bytes from LDS, not 4-17 separate loads from the weights)
    __shared__ uint8_t blk[8 * 210];  // 256 elements: one K-quant block or 8 Q8_0 / Q4_0 blocks
    const bool staged = w.type != T_F16 && w.type != T_F32;
    const uint32_t bb = (uint32_t)block_bytes(w.type);
    const uint32_t b0 = blockIdx.x * blockDim.x / be;  // first block in the row
    if (staged) {
        const uint32_t nbytes = 256 / be * bb;
        for (uint32_t t = threadIdx.x; t < nbytes; t += blockDim.x)
            blk[t] = gbyte(w, tok, b0 + t / bb, t % bb);
        __syncthreads();
    }
    if (i < n_pairs) {
        float sn = 0.f, cs = 1.f;
        if (i < rope_pairs) {
            const float th = (float)step[1] * freq[i];
            sincosf(th, &sn, &cs);
        }
        rope[i] = make_float2(cs, sn);
    }
    float v;
    if (staged) {
        const uint8_t *bp = blk + (threadIdx.x / be) * bb;
        v = deq_block_elem(w.type, threadIdx.x % be, [&](uint32_t o) { return bp[o]; });
    } else {
        const uint64_t e = (uint64_t)tok * w.n_in + i;
        v = deq_elem(w, e / be, (uint32_t)(e % be));
    }
    x[i] = v;
    pack_half(v * nw[i], i >> 5, p);
    const float sq = half_sum(v * v);  // the first RMSNorm's block sums
    if ((i & 31) == 0) xsq[i >> 5] = sq;
}

}  // namespace lrs

using namespace lrs;

struct DevLayer {
    const lrs_weight *q, *k, *v, *o, *gate, *up, *down;
    float *attn_norm, *ffn_norm, *bq, *bk, *bv;  // ffn_norm: post_attention_norm (hybrid)
    _Float16 *kc, *vc;
    // hybrid: gated delta-net mixer (dn) or gated attention with QK-norm
    bool dn = false;
    const lrs_weight *ssm_qkv = nullptr, *ssm_gate = nullptr, *ssm_out = nullptr;
    float *q_norm = nullptr, *k_norm = nullptr;
    float *alpha = nullptr, *beta = nullptr, *ssm_a = nullptr, *ssm_dt = nullptr;
    float *conv = nullptr, *ssm_norm = nullptr;
    float *win = nullptr, *state = nullptr;  // conv input ring [d_conv][conv_dim], S [v][D][D]
    // dense model, Q8_0 weights: which matmul inputs take the reference
    // forward's Q8_0 rounding (weights.rs:113-117) instead of the 22-bit pack
    bool qkv_q8 = false, o_q8 = false, ffn_q8 = false, down_q8 = false;
};

struct lrs_model {
    lrs_ctx *ctx;
    lrs_config cfg;
    std::vector<DevLayer> layers;
    const lrs_weight *embd, *output;
    float *output_norm, *freq;
    // activations: residual, q after RoPE, logits, attention split partials
    float *x, *qbuf, *logits, *pa;
    // sum(x^2) of each 32-element block of x, written with x (embed, the
    // residual epilogues) and read by the fused RMSNorm of the next matvec
    float *xsq = nullptr;
    // partial sums and arrival counts of the matvecs split over K across
    // workgroups (down, o, gate/up): [blocks][8 slices][64], [blocks], for
    // max(n_embd, n_ff) / 32 output blocks
    float *xpart = nullptr;
    uint32_t *xcnt = nullptr;
    uint32_t a_splits;
    // attention combine in the o launch (k_mq_ao; LRS_AO=0 turns it off):
    // the consumers' wait-error word at [32], then the flag matrix from [64]
    // (a row of 64 words per o workgroup, one word per producer); all zero
    // between launches
    bool ao_on = true;
    // the {cos, sin} table of the token's position, written by the embed
    // kernel, head_dim / 2 pairs: read by the hybrid's attention split when
    // it does the QK-norm + RoPE (LRS_QKP=0: a launch of its own), and by the
    // dense model's q/k/v epilogue (rope_qkv; LRS_ROPE_TABLE=0: sincosf
    // there); null when neither uses it
    float2 *rope_cs = nullptr;
    bool rope_qkv = false;
    // the split attention's query heads split into f16 pairs by one lane
    // group each and shared through LDS (LRS_ATTN_DQ=0: every lane group
    // splits every head)
    bool attn_dq = true;
    bool ao_wait_test = false;
    bool sao_on = true;  // attention split + combine + o in one launch (k_mq_sao; LRS_SAO=0: two launches)
    uint32_t *ao_sync = nullptr;
    size_t ao_sync_bytes = 0;
    // packs: x*attn_norm (or x*output_norm), x*ffn_norm, attention output,
    // SwiGLU output
    XPack pk_n, pk_f, pk_a, pk_s;
    // Q8_0-rounded pack of an RMSNorm'd input (q/k/v, gate/up or head input)
    // of Q8_0 weights
    XPack pk_q8 = {};
    bool head_q8 = false;
    uint32_t *step, *gen;  // step = {token, pos, n_generated}
    uint32_t gen_cap;
    // greedy: per-workgroup argmax keys of the head (ops.rs:1035-1045: the
    // first index of the maximum), reduced into step / gen by k_argmax_finish
    unsigned long long *amax;
    uint32_t head_keys = 0;
    // batched prompt blocks (allocated at the first block): residual,
    // normalised rows, q/k/v GEMM outputs, q after RoPE, attention output,
    // gate / up, token ids
    uint32_t pb_cap = 0;
    float *pX = nullptr, *pXN, *pQt, *pKt, *pVt, *pQ, *pATT, *pG, *pU;
    __bf16 *pA16 = nullptr;  // bf16 hi / lo planes of the current GEMM input
    // hybrid blocks: Q + gate rows, conv in / out, output gate, rule output,
    // gated norm, per-(token, head) gates
    float *pQG = nullptr, *pCI = nullptr, *pCO = nullptr, *pZ = nullptr, *pO = nullptr,
          *pY = nullptr;
    float2 *pGB = nullptr;
    float *pWork = nullptr;  // K-slice partials of the split GEMMs
    size_t work_bytes = 0;
    uint32_t *ptok;
    _Float16 *kv;                // all layers' caches
    uint32_t *step_host;         // pinned
    float *logits_host;          // pinned
    uint32_t *gen_host;          // pinned [gen_cap]: generated tokens on their way out
    hipGraphExec_t g_logits = nullptr, g_greedy = nullptr;
    uint32_t len = 0;
    size_t gguf_bytes_per_token = 0;
    std::vector<void *> allocs;
    // hybrid (qwen35) model: config and per-token buffers: Q rows (query +
    // gate per head), k, v, conv input, output gate, per-32-row sums of
    // squares of the delta-net output; recurrent memory (rings +
    // states of every delta-net layer) cleared by reset
    bool hybrid = false;
    lrs_hybrid_config hc = {};
    float *qg = nullptr, *kb = nullptr, *vb = nullptr, *dn_qkv = nullptr, *dn_z = nullptr,
          *dn_part = nullptr;
    // {e^g, beta} per value head from the projection launch (LRS_DN_GATES=0:
    // null, the step computes them)
    float2 *dn_gates = nullptr;
    void *rec = nullptr;
    size_t rec_bytes = 0;
    // weights the model owns (built by lrs_model_load_gguf), freed with it
    std::vector<lrs_weight *> owned;
};

// hands the loader's uploaded weights to the model
void lrs_model_adopt_weights(lrs_model *m, std::vector<lrs_weight *> &ws) {
    m->owned.insert(m->owned.end(), ws.begin(), ws.end());
    ws.clear();
}

namespace {

int dev_alloc(lrs_model *m, size_t bytes, void **p) {
    hipError_t e = hipMalloc(p, bytes ? bytes : 4);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(model)");
    m->allocs.push_back(*p);
    return LRS_OK;
}

int upload_vec(lrs_model *m, const float *host, size_t n, float **dev) {
    if (!host) {
        *dev = nullptr;
        return LRS_OK;
    }
    int rc = dev_alloc(m, n * sizeof(float), (void **)dev);
    if (rc) return rc;
    LRS_HIP(hipMemcpy(*dev, host, n * sizeof(float), hipMemcpyHostToDevice));
    return LRS_OK;
}

bool is_mv_type(uint32_t t) { return t == T_Q8_0 || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K; }

int check_w(const lrs_weight *w, const char *name, uint32_t n_in, uint32_t n_out, bool mv) {
    if (!w) return fail(LRS_E_ARG, std::string("missing weight ") + name);
    if (w->v.n_in != n_in || w->v.n_out != n_out)
        return fail(LRS_E_ARG, std::string(name) + " is " + std::to_string(w->v.n_out) + "x" +
                                   std::to_string(w->v.n_in) + ", expected " +
                                   std::to_string(n_out) + "x" + std::to_string(n_in));
    if (mv && !is_mv_type(w->v.type))
        return fail(LRS_E_UNSUPPORTED, std::string(name) + ": matvec needs Q8_0/Q4_K/Q5_K/Q6_K");
    return LRS_OK;
}

MqSeg mseg(const lrs_weight *w, uint32_t rows) {
    MqSeg s = {};
    s.w = w->v.q;
    s.rows = rows;
    return s;
}

// launch shapes of the decode ops (16-row tiles; see mq.hip)
constexpr MqGeom G_QKV = {1, 1, 4, 3};    // 448 workgroups of 4 K-slices (32B shape)
constexpr MqGeom G_O = {1, 2, 4, 2};      // 2 tiles (one 32-row pack block) x 4 K-slices
constexpr MqGeom G_HEAD = {1, 2, 2, 2};   // 2 tiles per workgroup x 2 K-slices
constexpr MqGeom G_STORE = {1, 2, 4, 2};  // hybrid q/k/v and delta-net projections

// gate+up tile pairs: 4 per workgroup x 2 K-slices while that gives >= 400
// workgroups (27648 rows: 432); else 2 per workgroup x 4 K-slices when all of
// them fit at once (2 workgroups of 8 wavefronts per CU: 13824 rows, 432);
// else 2 per workgroup x 2 K-slices (unsplit with one unit in flight: 544
// workgroups of 4 wavefronts at 5 per CU, 21.9 against 23.0 us for x 4
// K-slices), with a split tail when the block count just passes 512
MqGeom gateup_geom(uint32_t n_ff) {
    const uint32_t t = ttiles(n_ff);
    if (t / 4 >= 400) return MqGeom{2, 4, 2, 2};
    if (t / 2 <= 512) return MqGeom{2, 2, 4, 2};
    // more blocks of 2 tile pairs than twice the 256 CUs: a few CUs would
    // stream a third whole block (17408 rows: 544 blocks, 32 CUs with 3), so
    // the blocks past the last multiple of 256 split over K in 6 workgroups
    // each (21.1 -> 18.4 us at 17408, two units in flight)
    const uint32_t blocks = t / 2, tail = blocks % 256;
    if (tail && tail <= 64) {
        MqGeom g = {2, 2, 2, 2, 6};
        g.xfull = (int)(blocks - tail);
        return g;
    }
    return MqGeom{2, 2, 2, 1};
}
// down (n_embd rows, K = n_ff): one 32-row block per workgroup leaves 96 of
// the 256 CUs idle, and one CU streams ~35-40 GB/s, so wide down projections
// split K over 3 workgroups per block (480 workgroups; the last slice to
// arrive adds the partials and runs the residual + pack epilogue):
//   n_ff >= 24576: 2 tiles x 4 K-slices x 2 units in flight x 3 slices
//     (27648: 22.3 against 23.6 us unsplit at 2 tiles x 6 K-slices x 1 unit);
//   16384..24575: x 4 K-slices x 1 unit x 3 slices (17408: 16.4 against 17.2 us
//     unsplit at x 4 K-slices x 2 units);
//   below: 2 tiles x 6 K-slices x 1 unit, unsplit (13824: 13.6 us; the best
//     split 13.9).
MqGeom down_geom(uint32_t n_ff) {
    if (n_ff >= 24576) return MqGeom{1, 2, 4, 2, 3};
    if (n_ff >= 16384) return MqGeom{1, 2, 4, 1, 3};
    return MqGeom{1, 2, 6, 1};
}

// A launch-shape override from the environment, "tpw,tg,ks,p[,xs[,xfull]]" (the
// LLAMA_RS_MATVEC_GEOM knob of resident_forward.rs:164-176, per op here):
// LRS_GEOM_DOWN, LRS_GEOM_O, LRS_GEOM_GATEUP.  Read when the op is enqueued (graphs: at
// capture); a shape the kernels do not have fails the launch.
MqGeom env_geom(const char *name, MqGeom dflt) {
    const char *v = getenv(name);
    if (!v || !v[0]) return dflt;
    MqGeom g = {0, 0, 0, 0};
    int xs = 1;
    int xfull = 0;
    const int n = sscanf(v, "%d,%d,%d,%d,%d,%d", &g.tpw, &g.tg, &g.ks, &g.p, &xs, &xfull);
    if (n < 4) return dflt;
    g.xs = xs;
    g.xfull = xfull;
    return g;
}

// ---- one fused op of the per-token plan, enqueued on the model stream ----
hipError_t op_embed(lrs_model *m) {
    const lrs_config &c = m->cfg;
    // the rotation table when an attention split rotates q and k itself
    const uint32_t n_pairs = m->rope_cs ? c.head_dim / 2 : 0;
    if (n_pairs > c.n_embd) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_embed, dim3(c.n_embd / 256), dim3(256), 0, m->ctx->stream, m->embd->v,
                       m->step, m->layers[0].attn_norm, m->x, m->pk_n, m->xsq, m->freq, m->rope_cs,
                       n_pairs, c.rope_dim / 2);
    return hipGetLastError();
}

// q, k, v: rmsnorm + matvec + bias + RoPE + f16 KV append.  Segments of two
// weight types share a launch (Q4_K q/k with Q6_K v in the Q4_K_M mix);
// otherwise one launch per type.
hipError_t op_qkv(lrs_model *m, uint32_t l) {
    const lrs_config &c = m->cfg;
    const DevLayer &L = m->layers[l];
    MqArgs a = {};
    a.n_in = c.n_embd;
    a.xin = m->pk_n;
    a.xsq = m->xsq;
    a.eps = c.rms_eps;
    a.step = m->step;
    a.freq = m->freq;
    a.rope = m->rope_qkv ? reinterpret_cast<const float *>(m->rope_cs) : nullptr;
    a.head_dim = c.head_dim;
    a.rope_dim = c.rope_dim;
    a.ctx = c.ctx;
    MqSeg sq = mseg(L.q, L.q->v.n_out);
    sq.kind = 0;
    sq.bias = L.bq;
    sq.out = m->qbuf;
    MqSeg sk = mseg(L.k, L.k->v.n_out);
    sk.kind = 1;
    sk.bias = L.bk;
    sk.kv = L.kc;
    MqSeg sv = mseg(L.v, L.v->v.n_out);
    sv.kind = 2;
    sv.bias = L.bv;
    sv.kv = L.vc;
    if (L.qkv_q8) {
        // Q8_0 segments read rmsnorm(x) * attn_norm rounded to Q8_0 (the norm
        // is inside the pack: no RMS factor on their results)
        hipError_t e = launch_q8norm(m->x, L.attn_norm, c.n_embd, c.rms_eps, m->pk_q8,
                                     m->ctx->stream);
        if (e != hipSuccess) return e;
    }
    const lrs_weight *ws[3] = {L.q, L.k, L.v};
    const MqSeg segs[3] = {sq, sk, sv};
    const uint32_t tq = L.q->v.type, tv = L.v->v.type;
    if (L.k->v.type == tq && tv != tq) {
        a.n_seg = 3;
        a.n_seg0 = 2;
        a.seg[0] = sq;
        a.seg[1] = sk;
        a.seg[2] = sv;
        a.nxb = pack_blocks(tq, c.n_embd);
        hipError_t e = launch_mq(a, tq, tv, G_QKV, MQ_QKV, m->ctx->stream);
        if (e != hipErrorNotSupported) return e;
    }
    bool done[3] = {false, false, false};
    for (int i = 0; i < 3; i++) {
        if (done[i]) continue;
        const uint32_t t = ws[i]->v.type;
        a.n_seg = 0;
        for (int j = i; j < 3; j++) {
            if (!done[j] && ws[j]->v.type == t) {
                a.seg[a.n_seg++] = segs[j];
                done[j] = true;
            }
        }
        a.n_seg0 = a.n_seg;
        a.nxb = pack_blocks(t, c.n_embd);
        const bool q8 = L.qkv_q8 && t == T_Q8_0;
        a.xin = q8 ? m->pk_q8 : m->pk_n;
        a.xsq = q8 ? nullptr : m->xsq;
        hipError_t e = launch_mq(a, t, t, G_QKV, MQ_QKV, m->ctx->stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// whether layer l's attention combine runs in its o launch (k_mq_ao):
// attention layers whose o weight has the kernel and takes the 22-bit pack
// whether layer L's QK-norm + RoPE run in its attention split (the gated
// attention of the hybrid model; LRS_QKP=0 keeps the separate launch)
bool qkp_fused(const lrs_model *m, const DevLayer &L) { return m->hybrid && !L.dn && m->rope_cs; }

bool ao_fused(const lrs_model *m, const DevLayer &L) {
    const lrs_config &c = m->cfg;
    return m->ao_on && m->ao_sync && !L.dn && L.o && !L.o_q8 &&
           mq_ao_supported(L.o->v.type, L.o->v.n_in, c.n_embd, c.head_dim, m->a_splits, c.n_head);
}

// whether layer L's attention split runs in the o launch too (k_mq_sao)
bool sao_fused(const lrs_model *m, const DevLayer &L) {
    const lrs_config &c = m->cfg;
    return m->sao_on && ao_fused(m, L) &&
           attn_ao_supported(L.o->v.type, L.o->v.n_in, c.n_embd, c.head_dim, m->a_splits, c.n_head,
                             c.n_head_kv, qkp_fused(m, L), m->attn_dq);
}

// algorithmic bytes of layer L's attention over a cache of L positions
// (lrs_model_profile): the f16 K/V rows and q read, the partials' pack out;
// with the QK-norm + RoPE in the split (which reads the query rows in place
// of the q buffer), the new k / v rows, the two norm weights, the rotation
// table and the f16 K/V append
size_t attn_bytes(const lrs_model *m, const DevLayer &D, uint32_t len) {
    const lrs_config &c = m->cfg;
    const size_t qd4 = (size_t)c.n_head * c.head_dim * 4, kvd = (size_t)c.n_head_kv * c.head_dim;
    return (size_t)len * kvd * 2 * sizeof(_Float16) + 2 * qd4 +
           (qkp_fused(m, D) ? kvd * 8 + 3 * (size_t)c.head_dim * 4 + kvd * 4 : 0);
}

// QK-norm + RoPE inputs of layer L's split (qkp_fused)
QkPrep qk_prep(const lrs_model *m, const DevLayer &L) {
    QkPrep qp = {};
    qp.qg = m->qg;
    qp.kb = m->kb;
    qp.vb = m->vb;
    qp.q_norm = L.q_norm;
    qp.k_norm = L.k_norm;
    qp.rope = m->rope_cs;
    qp.kc = L.kc;
    qp.vc = L.vc;
    qp.eps = m->cfg.rms_eps;
    return qp;
}

// attention over the f16 cache; hybrid layers gate the output with
// sigmoid(second half of each head's Q rows) before packing it (the combine
// in the o launch when ao_fused)
hipError_t op_attn(lrs_model *m, uint32_t l) {
    const lrs_config &c = m->cfg;
    const DevLayer &L = m->layers[l];
    if (sao_fused(m, L)) return hipSuccess;  // the o launch runs the split
    const float *gate = m->hybrid ? m->qg + c.head_dim : nullptr;
    XPack out = m->pk_a;
    out.q8 = L.o_q8;
    const QkPrep qp = qkp_fused(m, L) ? qk_prep(m, L) : QkPrep{};
    return launch_attention(m->qbuf, L.kc, L.vc, m->pa, out, m->step, c.n_head, c.n_head_kv,
                            c.head_dim, c.ctx, m->a_splits, m->ctx->stream, gate,
                            2 * c.head_dim, !ao_fused(m, L), qkp_fused(m, L) ? &qp : nullptr,
                            m->attn_dq);
}

// x += W_o att (or W_ssm_out y of a delta-net layer); pack of x * ffn_norm
// (post_attention_norm) for gate/up
hipError_t op_o(lrs_model *m, uint32_t l) {
    const lrs_config &c = m->cfg;
    const DevLayer &L = m->layers[l];
    const lrs_weight *wo = L.dn ? L.ssm_out : L.o;
    MqArgs a = {};
    a.n_seg = 1;
    a.seg[0] = mseg(wo, c.n_embd);
    a.n_in = wo->v.n_in;
    a.nxb = pack_blocks(wo->v.type, a.n_in);
    a.xin = m->pk_a;
    a.x = m->x;
    a.xsq_out = m->xsq;
    a.nw = L.ffn_norm;
    a.xout = m->pk_f;
    if (L.dn) {
        // the gated norm's per-head RMS factor, from the step's partial sums
        a.gss = m->dn_part;
        a.gblk = m->hc.dn_state / 32;
        a.gn = (float)m->hc.dn_state;
        a.eps = c.rms_eps;
    }
    a.xpart = m->xpart;
    a.xcnt = m->xcnt;
    if (ao_fused(m, L)) {
        // the attention combine's workgroups (one per query head) ahead of o's
        AoArgs ao = {};
        ao.part = m->pa;
        ao.gate = m->hybrid ? m->qg + c.head_dim : nullptr;
        ao.splits = m->a_splits;
        ao.head_dim = c.head_dim;
        ao.gstride = 2 * c.head_dim;
        ao.n_prod = c.n_head;
        if (m->ao_wait_test) {
            // LRS_AO_WAIT_TEST: no flags are raised and each wait gives up
            // after 16 polls, so the call must report the error
            ao.no_signal = 1;
            a.wait_polls = 16;
        }
        a.werr = m->ao_sync + 32;
        a.wflag = m->ao_sync + 64;
        a.step = m->step;
        if (sao_fused(m, L)) {
            ao.sflag = m->ao_sync + 64 + 64 * (size_t)(c.n_embd / 32);
            const QkPrep qp = qk_prep(m, L);
            return launch_attn_ao(m->qbuf, L.kc, L.vc, c.n_head_kv, c.ctx, qkp_fused(m, L) ? &qp : nullptr,
                                  m->attn_dq, a, ao, wo->v.type, m->ctx->stream);
        }
        return launch_mq_ao(a, ao, wo->v.type, m->ctx->stream);
    }
    return launch_mq(a, wo->v.type, wo->v.type, env_geom("LRS_GEOM_O", G_O), MQ_RESID,
                     m->ctx->stream);
}

// outs[i] = W_i (rmsnorm(x) * attn_norm) for n weights (f32 rows out): one
// launch when they share a type or are Q4_K + Q6_K, else one per type
hipError_t op_store(lrs_model *m, const lrs_weight *const *ws, float *const *outs, int n) {
    const lrs_config &c = m->cfg;
    MqArgs a = {};
    a.n_in = c.n_embd;
    a.xin = m->pk_n;
    a.xsq = m->xsq;
    a.eps = c.rms_eps;
    bool q4 = false, q6 = false, other = false;
    for (int i = 0; i < n; i++) {
        const uint32_t t = ws[i]->v.type;
        q4 |= t == T_Q4_K;
        q6 |= t == T_Q6_K;
        other |= t != T_Q4_K && t != T_Q6_K;
    }
    if (q4 && q6 && !other) {
        a.n_seg = 0;
        for (int pass = 0; pass < 2; pass++)
            for (int i = 0; i < n; i++)
                if ((ws[i]->v.type == T_Q4_K) == (pass == 0)) {
                    MqSeg sg = mseg(ws[i], ws[i]->v.n_out);
                    sg.out = outs[i];
                    a.seg[a.n_seg++] = sg;
                }
        a.n_seg0 = 0;
        for (int i = 0; i < n; i++) a.n_seg0 += ws[i]->v.type == T_Q4_K;
        a.nxb = pack_blocks(T_Q4_K, c.n_embd);
        hipError_t e = launch_mq(a, T_Q4_K, T_Q6_K, G_STORE, MQ_STORE, m->ctx->stream);
        if (e != hipErrorNotSupported) return e;
    }
    bool done[MQ_MAX_SEG] = {false, false, false};
    for (int i = 0; i < n; i++) {
        if (done[i]) continue;
        const uint32_t t = ws[i]->v.type;
        a.n_seg = 0;
        for (int j = i; j < n; j++)
            if (!done[j] && ws[j]->v.type == t) {
                MqSeg sg = mseg(ws[j], ws[j]->v.n_out);
                sg.out = outs[j];
                a.seg[a.n_seg++] = sg;
                done[j] = true;
            }
        a.n_seg0 = a.n_seg;
        a.nxb = pack_blocks(t, c.n_embd);
        hipError_t e = launch_mq(a, t, t, G_STORE, MQ_STORE, m->ctx->stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// hybrid attention layer: Q (query + gate rows), k, v projections
hipError_t op_hattn_proj(lrs_model *m, uint32_t l) {
    const DevLayer &L = m->layers[l];
    const lrs_weight *ws[3] = {L.q, L.k, L.v};
    float *outs[3] = {m->qg, m->kb, m->vb};
    return op_store(m, ws, outs, 3);
}

// QK-norm + RoPE; q to qbuf, k / v to the f16 cache at pos
hipError_t op_qk_prep(lrs_model *m, uint32_t l) {
    const lrs_config &c = m->cfg;
    const DevLayer &L = m->layers[l];
    if (qkp_fused(m, L)) return hipSuccess;  // in the split (op_attn)
    return launch_qk_prep(m->qg, m->kb, m->vb, L.q_norm, L.k_norm, m->freq, m->step, m->qbuf, L.kc,
                          L.vc, c.n_head, c.n_head_kv, c.head_dim, c.ctx, c.rope_dim, c.rms_eps,
                          m->ctx->stream);
}

// delta-net layer: conv input (q | k | v channels) and output gate z
// whether delta-net layer L's gate projections run in its projection launch
// (launch_mq with gates) rather than in every workgroup of the step
bool dn_gates_fused(const lrs_model *m, const DevLayer &L) {
    return m->dn_gates && L.dn && L.ssm_qkv->v.type == L.ssm_gate->v.type &&
           mq_gates_supported(L.ssm_qkv->v.type, L.ssm_gate->v.type, G_STORE) &&
           m->cfg.n_embd % 4 == 0 && m->cfg.n_embd <= 4 * DN_GATE_THREADS * DN_GI;
}

hipError_t op_dn_proj(lrs_model *m, uint32_t l) {
    const DevLayer &L = m->layers[l];
    const lrs_weight *ws[2] = {L.ssm_qkv, L.ssm_gate};
    float *outs[2] = {m->dn_qkv, m->dn_z};
    if (dn_gates_fused(m, L)) {
        // ssm_qkv and ssm_gate (one type) in one launch, then one workgroup
        // per value head for the gate projections
        const lrs_config &c = m->cfg;
        MqArgs a = {};
        a.n_in = c.n_embd;
        a.xin = m->pk_n;
        a.xsq = m->xsq;
        a.eps = c.rms_eps;
        a.n_seg = 2;
        for (int i = 0; i < 2; i++) {
            a.seg[i] = mseg(ws[i], ws[i]->v.n_out);
            a.seg[i].out = outs[i];
        }
        a.nxb = pack_blocks(ws[0]->v.type, c.n_embd);
        DnGateArgs g = {};
        g.x = m->x;
        g.attn_norm = L.attn_norm;
        g.alpha = L.alpha;
        g.beta = L.beta;
        g.a = L.ssm_a;
        g.dt = L.ssm_dt;
        g.out = m->dn_gates;
        g.n_embd = c.n_embd;
        g.v_heads = m->hc.dn_v_heads;
        g.eps = c.rms_eps;
        return launch_mq(a, ws[0]->v.type, ws[1]->v.type, G_STORE, MQ_STORE, m->ctx->stream,
                         nullptr, nullptr, &g);
    }
    return op_store(m, ws, outs, 2);
}

// delta-net step: gates, conv, L2, delta rule, gated norm -> pack of y
hipError_t op_dn_step(lrs_model *m, uint32_t l) {
    const DevLayer &L = m->layers[l];
    DnArgs a = {};
    a.qkv = m->dn_qkv;
    a.z = m->dn_z;
    a.x = m->x;
    a.attn_norm = L.attn_norm;
    a.alpha = L.alpha;
    a.beta = L.beta;
    a.a = L.ssm_a;
    a.dt = L.ssm_dt;
    a.conv_w = L.conv;
    a.win = L.win;
    a.state = L.state;
    a.norm_w = L.ssm_norm;
    a.part = m->dn_part;
    a.out = m->pk_a;
    a.step = m->step;
    a.n_embd = m->cfg.n_embd;
    a.k_heads = m->hc.dn_k_heads;
    a.v_heads = m->hc.dn_v_heads;
    a.d_conv = m->hc.dn_conv;
    a.eps = m->cfg.rms_eps;
    a.gates = dn_gates_fused(m, L) ? m->dn_gates : nullptr;
    return launch_dn_step(a, m->hc.dn_state, m->ctx->stream);
}

// act = silu(gate h) * (up h), h = rmsnorm(x) * ffn_norm; gate and up tiles
// of the same outputs in one wavefront; pack of act for down
hipError_t op_gateup(lrs_model *m, uint32_t l) {
    const lrs_config &c = m->cfg;
    const DevLayer &L = m->layers[l];
    MqArgs a = {};
    a.n_seg = 1;
    a.seg[0] = mseg(L.gate, c.n_ff);
    a.seg[0].w2 = L.up->v.q;
    a.n_in = c.n_embd;
    a.nxb = pack_blocks(L.gate->v.type, c.n_embd);
    a.xin = m->pk_f;
    a.xsq = m->xsq;
    a.eps = c.rms_eps;
    if (L.ffn_q8) {
        hipError_t e = launch_q8norm(m->x, L.ffn_norm, c.n_embd, c.rms_eps, m->pk_q8,
                                     m->ctx->stream);
        if (e != hipSuccess) return e;
        a.xin = m->pk_q8;
        a.xsq = nullptr;
    }
    a.xout = m->pk_s;
    a.xout.q8 = L.down_q8;
    a.xpart = m->xpart;
    a.xcnt = m->xcnt;
    return launch_mq(a, L.gate->v.type, L.gate->v.type, env_geom("LRS_GEOM_GATEUP", gateup_geom(c.n_ff)),
                     MQ_SWIGLU, m->ctx->stream);
}

// x += W_down act; pack of x * (next layer's attn_norm, or output_norm)
hipError_t op_down(lrs_model *m, uint32_t l) {
    const lrs_config &c = m->cfg;
    const DevLayer &L = m->layers[l];
    MqArgs a = {};
    a.n_seg = 1;
    a.seg[0] = mseg(L.down, c.n_embd);
    a.n_in = c.n_ff;
    a.nxb = pack_blocks(L.down->v.type, c.n_ff);
    a.xin = m->pk_s;
    a.x = m->x;
    a.xsq_out = m->xsq;
    a.nw = l + 1 < c.n_layer ? m->layers[l + 1].attn_norm : m->output_norm;
    a.xout = m->pk_n;
    a.xpart = m->xpart;
    a.xcnt = m->xcnt;
    return launch_mq(a, L.down->v.type, L.down->v.type, env_geom("LRS_GEOM_DOWN", down_geom(c.n_ff)),
                     MQ_RESID, m->ctx->stream);
}

// the FFN of layer l: gate/up + SwiGLU, then down + residual
hipError_t op_ffn(lrs_model *m, uint32_t l) {
    hipError_t e = op_gateup(m, l);
    return e != hipSuccess ? e : op_down(m, l);
}

// logits = W_out (rmsnorm(x) * output_norm); greedy: each wavefront of
// outputs also leaves the argmax key of its rows, reduced by op_argmax
hipError_t op_head(lrs_model *m, bool greedy) {
    const lrs_config &c = m->cfg;
    MqArgs a = {};
    a.n_seg = 1;
    a.seg[0] = mseg(m->output, c.vocab);
    a.seg[0].out = m->logits;
    a.n_in = c.n_embd;
    a.nxb = pack_blocks(m->output->v.type, c.n_embd);
    a.xin = m->pk_n;
    a.xsq = m->xsq;
    a.eps = c.rms_eps;
    if (m->head_q8) {
        hipError_t e = launch_q8norm(m->x, m->output_norm, c.n_embd, c.rms_eps, m->pk_q8,
                                     m->ctx->stream);
        if (e != hipSuccess) return e;
        a.xin = m->pk_q8;
        a.xsq = nullptr;
    }
    if (greedy) a.amax = m->amax;
    uint32_t wgs = 0, kpw = 0;
    hipError_t e = launch_mq(a, m->output->v.type, m->output->v.type, G_HEAD, MQ_STORE,
                             m->ctx->stream, &wgs, &kpw);
    m->head_keys = wgs * kpw;
    return e;
}

hipError_t op_argmax(lrs_model *m) {
    return launch_argmax_finish(m->amax, m->head_keys, m->step, m->gen, m->gen_cap,
                                m->ctx->stream);
}

// enqueue one token's forward on the model stream
hipError_t enqueue_forward(lrs_model *m, bool greedy) {
    hipError_t e;
    if ((e = op_embed(m)) != hipSuccess) return e;
    for (uint32_t l = 0; l < m->cfg.n_layer; l++) {
        if (m->layers[l].dn) {
            if ((e = op_dn_proj(m, l)) != hipSuccess || (e = op_dn_step(m, l)) != hipSuccess)
                return e;
        } else if (m->hybrid) {
            if ((e = op_hattn_proj(m, l)) != hipSuccess || (e = op_qk_prep(m, l)) != hipSuccess ||
                (e = op_attn(m, l)) != hipSuccess)
                return e;
        } else if ((e = op_qkv(m, l)) != hipSuccess || (e = op_attn(m, l)) != hipSuccess) {
            return e;
        }
        if ((e = op_o(m, l)) != hipSuccess || (e = op_ffn(m, l)) != hipSuccess) return e;
    }
    if ((e = op_head(m, greedy)) != hipSuccess) return e;
    if (greedy && (e = op_argmax(m)) != hipSuccess) return e;
    return hipSuccess;
}

int capture(lrs_model *m, bool greedy, hipGraphExec_t *out) {
    hipStream_t s = m->ctx->stream;
    hipGraph_t g = nullptr;
    LRS_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    hipError_t e = enqueue_forward(m, greedy);
    hipError_t e2 = hipStreamEndCapture(s, &g);
    if (e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return hip_fail(e, "forward capture");
    }
    if (e2 != hipSuccess) return hip_fail(e2, "hipStreamEndCapture");
    e = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    return LRS_OK;
}

// one token's forward: the captured graph, or the same launches directly
hipError_t run_forward(lrs_model *m, bool greedy) {
    hipGraphExec_t g = greedy ? m->g_greedy : m->g_logits;
    if (g) return hipGraphLaunch(g, m->ctx->stream);
    return enqueue_forward(m, greedy);
}

size_t wbytes(const lrs_weight *w) { return lrs_weight_gguf_bytes(w); }

// RawTensor::matmul_into (weights.rs:109-124): with the reference rounding on,
// a Q8_0 weight multiplies its input rounded to Q8_0 (quantize_q8_0_split);
// otherwise, and for every other type, the f32 input (the 22-bit pack)
void set_q8_flags(lrs_model *m, bool on) {
    for (DevLayer &D : m->layers) {
        if (D.dn || !D.q) continue;  // dense layers only
        D.qkv_q8 = on && (D.q->v.type == T_Q8_0 || D.k->v.type == T_Q8_0 || D.v->v.type == T_Q8_0);
        D.o_q8 = on && D.o->v.type == T_Q8_0;
        D.ffn_q8 = on && D.gate->v.type == T_Q8_0;
        D.down_q8 = on && D.down->v.type == T_Q8_0;
    }
    m->head_q8 = on && !m->hybrid && m->output->v.type == T_Q8_0;
}

// Whether the per-token forward is captured into HIP graphs.  LRS_GRAPH=0
// issues the same launches directly on the stream instead.  So does a
// process running under rocprofv3 kernel tracing or counter collection (it
// exports ROCPROF_KERNEL_TRACE / ROCPROF_COUNTER_COLLECTION to the program):
// a traced run of back-to-back graph launches ended in a host SIGSEGV inside
// the profiler's own code, so traced runs replay the launches directly.
bool env_on(const char *name) {
    const char *v = getenv(name);
    return v && v[0] && strcmp(v, "0") != 0 && strcasecmp(v, "false") != 0;
}
bool use_graphs() {
    const char *ge = getenv("LRS_GRAPH");
    if (ge && ge[0] == '0') return false;
    return !env_on("ROCPROF_KERNEL_TRACE") && !env_on("ROCPROF_COUNTER_COLLECTION");
}

// (re)captures the per-token graphs unless graphs are off
int capture_graphs(lrs_model *m) {
    if (m->g_logits) (void)hipGraphExecDestroy(m->g_logits);
    if (m->g_greedy) (void)hipGraphExecDestroy(m->g_greedy);
    m->g_logits = m->g_greedy = nullptr;
    if (!use_graphs()) return LRS_OK;
    int rc;
    if ((rc = capture(m, false, &m->g_logits)) || (rc = capture(m, true, &m->g_greedy))) return rc;
    return LRS_OK;
}

// allocations shared by the dense and hybrid models, then the graph capture;
// pack_a_elems: elements of the o-projection's input pack beyond n_head*head_dim
int finish_model(lrs_model *m, const float *output_norm, const std::vector<float> &fr,
                 uint32_t pack_a_elems) {
    const lrs_config &c = m->cfg;
    const uint32_t qd = c.n_head * c.head_dim;
    int rc;
    m->gguf_bytes_per_token += wbytes(m->output);
    if ((rc = upload_vec(m, output_norm, c.n_embd, &m->output_norm))) return rc;
    if ((rc = upload_vec(m, fr.data(), fr.size(), &m->freq))) return rc;
    m->gen_cap = 1u << 16;
    m->a_splits = attn_splits(c.n_head_kv);
    {
        // LRS_ATTN_SPLITS: the decode attention's position splits per KV head
        // (tuning knob; at most the default's 256 / n_head_kv, 40)
        const char *v = getenv("LRS_ATTN_SPLITS");
        const int n = v ? atoi(v) : 0;
        if (n > 0 && (uint32_t)n < m->a_splits) m->a_splits = (uint32_t)n;
    }
    if ((rc = dev_alloc(m, (size_t)c.n_head * m->a_splits * (c.head_dim + 4) * sizeof(float),
                        (void **)&m->pa)) ||
        (rc = dev_alloc(m, c.n_embd * sizeof(float), (void **)&m->x)) ||
        (rc = dev_alloc(m, c.n_embd / 32 * sizeof(float), (void **)&m->xsq)) ||
        (rc = dev_alloc(m, qd * sizeof(float), (void **)&m->qbuf)) ||
        (rc = dev_alloc(m, c.vocab * sizeof(float), (void **)&m->logits)) ||
        (rc = dev_alloc(m, 4 * sizeof(uint32_t), (void **)&m->step)) ||
        (rc = dev_alloc(m, m->gen_cap * sizeof(uint32_t), (void **)&m->gen)) ||
        (rc = dev_alloc(m, (size_t)c.vocab * sizeof(unsigned long long), (void **)&m->amax)))
        return rc;
    {
        // activation packs (n_embd, n_ff and the o-projection inputs are
        // multiples of 256)
        void *p = nullptr;
        const uint32_t ne = c.n_embd / 32, nq = (qd > pack_a_elems ? qd : pack_a_elems) / 32,
                       nf = c.n_ff / 32;
        if ((rc = dev_alloc(m, xpack_bytes(ne), &p))) return rc;
        m->pk_n = xpack_at(p, ne);
        if ((rc = dev_alloc(m, xpack_bytes(ne), &p))) return rc;
        m->pk_f = xpack_at(p, ne);
        if ((rc = dev_alloc(m, xpack_bytes(nq), &p))) return rc;
        m->pk_a = xpack_at(p, nq);
        if ((rc = dev_alloc(m, xpack_bytes(nf), &p))) return rc;
        m->pk_s = xpack_at(p, nf);
        if ((rc = dev_alloc(m, xpack_bytes(ne), &p))) return rc;
        m->pk_q8 = xpack_at(p, ne);
        m->pk_q8.q8 = 1;
    }
    if (hipMemset(m->step, 0, 4 * sizeof(uint32_t)) != hipSuccess) return fail(LRS_E_HIP, "memset");
    {
        // the split matvecs' arrival counts start at zero and every launch
        // leaves them at zero (the last slice to arrive resets its block's)
        const size_t nb = (c.n_embd > c.n_ff ? c.n_embd : c.n_ff) / 32;
        if ((rc = dev_alloc(m, nb * 8 * 64 * sizeof(float), (void **)&m->xpart)) ||
            (rc = dev_alloc(m, nb * sizeof(uint32_t), (void **)&m->xcnt)))
            return rc;
        if (hipMemset(m->xcnt, 0, nb * sizeof(uint32_t)) != hipSuccess)
            return fail(LRS_E_HIP, "memset");
        // error word, a row of flags per 32 rows of o's output, then a row
        // per query head (the splits' flags of k_mq_sao)
        const size_t aw = 64 + 64 * (size_t)(c.n_embd / 32) + 64 * (size_t)c.n_head;
        if ((rc = dev_alloc(m, aw * sizeof(uint32_t), (void **)&m->ao_sync))) return rc;
        m->ao_sync_bytes = aw * sizeof(uint32_t);
        if (hipMemset(m->ao_sync, 0, aw * sizeof(uint32_t)) != hipSuccess)
            return fail(LRS_E_HIP, "memset");
        const char *v = getenv("LRS_AO");
        m->ao_on = !(v && (strcmp(v, "0") == 0 || strcasecmp(v, "false") == 0));
        m->ao_wait_test = env_on("LRS_AO_WAIT_TEST");
        const char *vs = getenv("LRS_SAO");
        m->sao_on = !(vs && (strcmp(vs, "0") == 0 || strcasecmp(vs, "false") == 0));
        const char *vd = getenv("LRS_ATTN_DQ");
        m->attn_dq = !(vd && (strcmp(vd, "0") == 0 || strcasecmp(vd, "false") == 0));
        const char *vq = getenv("LRS_QKP");
        const bool qkp_on = !(vq && (strcmp(vq, "0") == 0 || strcasecmp(vq, "false") == 0));
        const char *vr = getenv("LRS_ROPE_TABLE");
        m->rope_qkv = !m->hybrid && !(vr && (strcmp(vr, "0") == 0 || strcasecmp(vr, "false") == 0));
        if ((m->hybrid && qkp_on && attn_qp_supported(c.head_dim, c.n_head / c.n_head_kv)) ||
            m->rope_qkv) {
            const size_t rb = c.head_dim / 2 * sizeof(float2);
            if ((rc = dev_alloc(m, rb, (void **)&m->rope_cs))) return rc;
            if (hipMemset(m->rope_cs, 0, rb) != hipSuccess) return fail(LRS_E_HIP, "memset");
        }
    }
    // 1024 step slots of 4 words (enqueue_tokens), then the wait-error word
    if (hipHostMalloc((void **)&m->step_host, (4 * 1024 + 4) * sizeof(uint32_t), hipHostMallocDefault) !=
            hipSuccess ||
        hipHostMalloc((void **)&m->logits_host, c.vocab * sizeof(float), hipHostMallocDefault) !=
            hipSuccess ||
        hipHostMalloc((void **)&m->gen_host, m->gen_cap * sizeof(uint32_t), hipHostMallocDefault) !=
            hipSuccess)
        return fail(LRS_E_OOM, "pinned host buffers");
    return capture_graphs(m);
}

}  // namespace

extern "C" {

int lrs_model_create(lrs_ctx *ctx, const lrs_config *cfg, const lrs_layer_weights *layers,
                     const lrs_weight *token_embd, const float *output_norm,
                     const lrs_weight *output, lrs_model **out) {
    if (!ctx || !cfg || !layers || !token_embd || !output_norm || !output || !out)
        return fail(LRS_E_ARG, "null argument");
    const lrs_config c = *cfg;
    if (c.n_layer == 0 || c.n_embd == 0 || c.n_head == 0 || c.n_head_kv == 0 || c.vocab == 0 ||
        c.ctx == 0 || c.n_ff == 0)
        return fail(LRS_E_ARG, "empty dimension in config");
    if (c.n_head % c.n_head_kv) return fail(LRS_E_ARG, "n_head must be a multiple of n_head_kv");
    if (c.head_dim != 64 && c.head_dim != 128 && c.head_dim != 256)
        return fail(LRS_E_UNSUPPORTED, "head_dim must be 64, 128 or 256");
    if (c.rope_dim > c.head_dim || (c.rope_dim & 1)) return fail(LRS_E_ARG, "bad rope_dim");
    if (c.n_head / c.n_head_kv > 8) return fail(LRS_E_UNSUPPORTED, "n_head / n_head_kv > 8");
    if (c.n_embd % 256 || c.n_ff % 256 || (c.n_head * c.head_dim) % 256)
        return fail(LRS_E_UNSUPPORTED, "n_embd, n_ff and n_head*head_dim must be multiples of 256");
    const uint32_t qd = c.n_head * c.head_dim, kvd = c.n_head_kv * c.head_dim;
    int rc;
    for (uint32_t l = 0; l < c.n_layer; l++) {
        const lrs_layer_weights &L = layers[l];
        if ((rc = check_w(L.attn_q, "attn_q", c.n_embd, qd, true)) ||
            (rc = check_w(L.attn_k, "attn_k", c.n_embd, kvd, true)) ||
            (rc = check_w(L.attn_v, "attn_v", c.n_embd, kvd, true)) ||
            (rc = check_w(L.attn_output, "attn_output", qd, c.n_embd, true)) ||
            (rc = check_w(L.ffn_gate, "ffn_gate", c.n_embd, c.n_ff, true)) ||
            (rc = check_w(L.ffn_up, "ffn_up", c.n_embd, c.n_ff, true)) ||
            (rc = check_w(L.ffn_down, "ffn_down", c.n_ff, c.n_embd, true)))
            return rc;
        if (L.ffn_gate->v.type != L.ffn_up->v.type)
            return fail(LRS_E_UNSUPPORTED, "ffn_gate and ffn_up must share a type");
        if (!L.attn_norm || !L.ffn_norm) return fail(LRS_E_ARG, "missing norm weights");
        if (L.attn_q->ctx != ctx || L.ffn_down->ctx != ctx)
            return fail(LRS_E_ARG, "weights belong to another context");
    }
    if ((rc = check_w(token_embd, "token_embd", c.n_embd, c.vocab, false))) return rc;
    if ((rc = check_w(output, "output", c.n_embd, c.vocab, true))) return rc;
    if (token_embd->v.type == T_Q4_0 || block_elems(token_embd->v.type) < 0)
        return fail(LRS_E_UNSUPPORTED, "token_embd type");

    LRS_HIP(hipSetDevice(ctx->device));
    lrs_model *m = new lrs_model();
    m->ctx = ctx;
    m->cfg = c;
    m->embd = token_embd;
    m->output = output;
    m->layers.resize(c.n_layer);
    auto bail = [&](int code) {
        lrs_model_destroy(m);
        return code;
    };
    const size_t kv_layer = (size_t)kvd * c.ctx;
    if ((rc = dev_alloc(m, kv_layer * 2 * c.n_layer * sizeof(_Float16), (void **)&m->kv))) return bail(rc);
    if (hipMemset(m->kv, 0, kv_layer * 2 * c.n_layer * sizeof(_Float16)) != hipSuccess)
        return bail(fail(LRS_E_HIP, "kv memset"));
    for (uint32_t l = 0; l < c.n_layer; l++) {
        const lrs_layer_weights &L = layers[l];
        DevLayer &D = m->layers[l];
        D.q = L.attn_q;
        D.k = L.attn_k;
        D.v = L.attn_v;
        D.o = L.attn_output;
        D.gate = L.ffn_gate;
        D.up = L.ffn_up;
        D.down = L.ffn_down;
        D.kc = m->kv + kv_layer * 2 * l;
        D.vc = D.kc + kv_layer;
        if ((rc = upload_vec(m, L.attn_norm, c.n_embd, &D.attn_norm)) ||
            (rc = upload_vec(m, L.ffn_norm, c.n_embd, &D.ffn_norm)) ||
            (rc = upload_vec(m, L.bq, qd, &D.bq)) || (rc = upload_vec(m, L.bk, kvd, &D.bk)) ||
            (rc = upload_vec(m, L.bv, kvd, &D.bv)))
            return bail(rc);
        m->gguf_bytes_per_token += wbytes(L.attn_q) + wbytes(L.attn_k) + wbytes(L.attn_v) +
                                   wbytes(L.attn_output) + wbytes(L.ffn_gate) + wbytes(L.ffn_up) +
                                   wbytes(L.ffn_down);
    }
    // RoPE table freq[i] = base^(-2i/rope_dim), f32 powf (model.rs:339-343)
    std::vector<float> fr(c.rope_dim / 2 + 1, 0.f);
    for (uint32_t i = 0; i < c.rope_dim / 2; i++) {
        float ex = -2.0f * (float)i;
        ex = ex / (float)c.rope_dim;
        fr[i] = powf(c.freq_base, ex);
    }
    if ((rc = finish_model(m, output_norm, fr, 0))) return bail(rc);
    *out = m;
    return LRS_OK;
}

int lrs_hybrid_create(lrs_ctx *ctx, const lrs_hybrid_config *hcfg, const lrs_hybrid_layer *layers,
                      const lrs_weight *token_embd, const float *output_norm,
                      const lrs_weight *output, lrs_model **out) {
    if (!ctx || !hcfg || !layers || !token_embd || !output_norm || !output || !out)
        return fail(LRS_E_ARG, "null argument");
    const lrs_hybrid_config hc = *hcfg;
    const lrs_config c = hc.base;
    if (c.n_layer == 0 || c.n_embd == 0 || c.n_head == 0 || c.n_head_kv == 0 || c.vocab == 0 ||
        c.ctx == 0 || c.n_ff == 0 || hc.full_attn_interval == 0 || hc.dn_k_heads == 0 ||
        hc.dn_v_heads == 0 || hc.dn_conv == 0)
        return fail(LRS_E_ARG, "empty dimension in config");
    if (c.n_head % c.n_head_kv) return fail(LRS_E_ARG, "n_head must be a multiple of n_head_kv");
    if (hc.dn_v_heads % hc.dn_k_heads)
        return fail(LRS_E_ARG, "dn_v_heads must be a multiple of dn_k_heads");
    if (c.head_dim != 64 && c.head_dim != 128 && c.head_dim != 256)
        return fail(LRS_E_UNSUPPORTED, "head_dim must be 64, 128 or 256");
    if (hc.dn_state != 64 && hc.dn_state != 128)
        return fail(LRS_E_UNSUPPORTED, "dn_state must be 64 or 128");
    if (hc.dn_conv > 8) return fail(LRS_E_UNSUPPORTED, "dn_conv above 8");
    if (c.n_embd > 8192) return fail(LRS_E_UNSUPPORTED, "hybrid n_embd above 8192");
    if (c.rope_dim > c.head_dim || (c.rope_dim & 1)) return fail(LRS_E_ARG, "bad rope_dim");
    if (c.n_head / c.n_head_kv > 8) return fail(LRS_E_UNSUPPORTED, "n_head / n_head_kv > 8");
    const uint32_t qd = c.n_head * c.head_dim, kvd = c.n_head_kv * c.head_dim;
    const uint32_t D = hc.dn_state, KD = hc.dn_k_heads * D, VD = hc.dn_v_heads * D;
    const uint32_t CD = 2 * KD + VD;
    if (c.n_embd % 256 || c.n_ff % 256 || qd % 256 || VD % 256)
        return fail(LRS_E_UNSUPPORTED,
                    "n_embd, n_ff, n_head*head_dim and dn_v_heads*dn_state must be multiples of 256");
    int rc;
    uint32_t n_attn = 0, n_dn = 0;
    for (uint32_t l = 0; l < c.n_layer; l++) {
        const lrs_hybrid_layer &L = layers[l];
        const bool full = (l + 1) % hc.full_attn_interval == 0;  // config.rs:25-35
        if ((rc = check_w(L.ffn_gate, "ffn_gate", c.n_embd, c.n_ff, true)) ||
            (rc = check_w(L.ffn_up, "ffn_up", c.n_embd, c.n_ff, true)) ||
            (rc = check_w(L.ffn_down, "ffn_down", c.n_ff, c.n_embd, true)))
            return rc;
        if (L.ffn_gate->v.type != L.ffn_up->v.type)
            return fail(LRS_E_UNSUPPORTED, "ffn_gate and ffn_up must share a type");
        if (!L.attn_norm || !L.post_norm) return fail(LRS_E_ARG, "missing norm weights");
        if (L.ffn_down->ctx != ctx) return fail(LRS_E_ARG, "weights belong to another context");
        if (full) {
            if ((rc = check_w(L.attn_q, "attn_q", c.n_embd, 2 * qd, true)) ||
                (rc = check_w(L.attn_k, "attn_k", c.n_embd, kvd, true)) ||
                (rc = check_w(L.attn_v, "attn_v", c.n_embd, kvd, true)) ||
                (rc = check_w(L.attn_output, "attn_output", qd, c.n_embd, true)))
                return rc;
            if (!L.q_norm || !L.k_norm) return fail(LRS_E_ARG, "missing q_norm / k_norm");
            n_attn++;
        } else {
            if ((rc = check_w(L.ssm_qkv, "ssm_qkv", c.n_embd, CD, true)) ||
                (rc = check_w(L.ssm_gate, "ssm_gate", c.n_embd, VD, true)) ||
                (rc = check_w(L.ssm_out, "ssm_out", VD, c.n_embd, true)))
                return rc;
            if (!L.ssm_alpha || !L.ssm_beta || !L.ssm_a || !L.ssm_dt || !L.ssm_conv || !L.ssm_norm)
                return fail(LRS_E_ARG, "missing delta-net vectors");
            n_dn++;
        }
    }
    if ((rc = check_w(token_embd, "token_embd", c.n_embd, c.vocab, false))) return rc;
    if ((rc = check_w(output, "output", c.n_embd, c.vocab, true))) return rc;
    if (token_embd->v.type == T_Q4_0 || block_elems(token_embd->v.type) < 0)
        return fail(LRS_E_UNSUPPORTED, "token_embd type");

    LRS_HIP(hipSetDevice(ctx->device));
    lrs_model *m = new lrs_model();
    m->ctx = ctx;
    m->cfg = c;
    m->hybrid = true;
    m->hc = hc;
    m->embd = token_embd;
    m->output = output;
    m->layers.resize(c.n_layer);
    auto bail = [&](int code) {
        lrs_model_destroy(m);
        return code;
    };
    const size_t kv_layer = (size_t)kvd * c.ctx;
    const size_t win_f = (size_t)hc.dn_conv * CD, st_f = (size_t)hc.dn_v_heads * D * D;
    m->rec_bytes = (win_f + st_f) * n_dn * sizeof(float);
    if ((rc = dev_alloc(m, kv_layer * 2 * n_attn * sizeof(_Float16), (void **)&m->kv)) ||
        (rc = dev_alloc(m, m->rec_bytes, &m->rec)) ||
        (rc = dev_alloc(m, 2 * (size_t)qd * sizeof(float), (void **)&m->qg)) ||
        (rc = dev_alloc(m, kvd * sizeof(float), (void **)&m->kb)) ||
        (rc = dev_alloc(m, kvd * sizeof(float), (void **)&m->vb)) ||
        (rc = dev_alloc(m, CD * sizeof(float), (void **)&m->dn_qkv)) ||
        (rc = dev_alloc(m, VD * sizeof(float), (void **)&m->dn_z)) ||
        (rc = dev_alloc(m, (size_t)hc.dn_v_heads * (D / 32) * sizeof(float), (void **)&m->dn_part)) ||
        (rc = dev_alloc(m, (size_t)hc.dn_v_heads * sizeof(float2), (void **)&m->dn_gates)))
        return bail(rc);
    {
        const char *v = getenv("LRS_DN_GATES");
        if (v && (strcmp(v, "0") == 0 || strcasecmp(v, "false") == 0)) m->dn_gates = nullptr;
    }
    if (hipMemset(m->kv, 0, kv_layer * 2 * n_attn * sizeof(_Float16)) != hipSuccess ||
        hipMemset(m->rec, 0, m->rec_bytes) != hipSuccess)
        return bail(fail(LRS_E_HIP, "memset"));
    uint32_t ia = 0, id = 0;
    for (uint32_t l = 0; l < c.n_layer; l++) {
        const lrs_hybrid_layer &L = layers[l];
        DevLayer &D_ = m->layers[l];
        D_.gate = L.ffn_gate;
        D_.up = L.ffn_up;
        D_.down = L.ffn_down;
        if ((rc = upload_vec(m, L.attn_norm, c.n_embd, &D_.attn_norm)) ||
            (rc = upload_vec(m, L.post_norm, c.n_embd, &D_.ffn_norm)))
            return bail(rc);
        m->gguf_bytes_per_token += wbytes(L.ffn_gate) + wbytes(L.ffn_up) + wbytes(L.ffn_down);
        if ((l + 1) % hc.full_attn_interval == 0) {
            D_.q = L.attn_q;
            D_.k = L.attn_k;
            D_.v = L.attn_v;
            D_.o = L.attn_output;
            D_.kc = m->kv + kv_layer * 2 * ia++;
            D_.vc = D_.kc + kv_layer;
            if ((rc = upload_vec(m, L.q_norm, c.head_dim, &D_.q_norm)) ||
                (rc = upload_vec(m, L.k_norm, c.head_dim, &D_.k_norm)))
                return bail(rc);
            m->gguf_bytes_per_token += wbytes(L.attn_q) + wbytes(L.attn_k) + wbytes(L.attn_v) +
                                       wbytes(L.attn_output);
        } else {
            D_.dn = true;
            D_.ssm_qkv = L.ssm_qkv;
            D_.ssm_gate = L.ssm_gate;
            D_.ssm_out = L.ssm_out;
            float *r0 = reinterpret_cast<float *>(m->rec) + (win_f + st_f) * id++;
            D_.win = r0;
            D_.state = r0 + win_f;
            if ((rc = upload_vec(m, L.ssm_alpha, (size_t)hc.dn_v_heads * c.n_embd, &D_.alpha)) ||
                (rc = upload_vec(m, L.ssm_beta, (size_t)hc.dn_v_heads * c.n_embd, &D_.beta)) ||
                (rc = upload_vec(m, L.ssm_a, hc.dn_v_heads, &D_.ssm_a)) ||
                (rc = upload_vec(m, L.ssm_dt, hc.dn_v_heads, &D_.ssm_dt)) ||
                (rc = upload_vec(m, L.ssm_conv, (size_t)CD * hc.dn_conv, &D_.conv)) ||
                (rc = upload_vec(m, L.ssm_norm, D, &D_.ssm_norm)))
                return bail(rc);
            m->gguf_bytes_per_token += wbytes(L.ssm_qkv) + wbytes(L.ssm_gate) + wbytes(L.ssm_out) +
                                       2 * (size_t)hc.dn_v_heads * c.n_embd * sizeof(float);
        }
    }
    // freq[i] = 1 / base^(2i/rope_dim) (gpu.rs:540-547)
    std::vector<float> fr(c.rope_dim / 2 + 1, 0.f);
    for (uint32_t i = 0; i < c.rope_dim / 2; i++) {
        const float ex = (float)(2 * i) / (float)c.rope_dim;
        fr[i] = 1.0f / powf(c.freq_base, ex);
    }
    if ((rc = finish_model(m, output_norm, fr, VD))) return bail(rc);
    *out = m;
    return LRS_OK;
}

void lrs_model_destroy(lrs_model *m) {
    if (!m) return;
    (void)hipSetDevice(m->ctx->device);
    (void)hipStreamSynchronize(m->ctx->stream);
    if (m->g_logits) (void)hipGraphExecDestroy(m->g_logits);
    if (m->g_greedy) (void)hipGraphExecDestroy(m->g_greedy);
    for (void *p : m->allocs) (void)hipFree(p);
    if (m->step_host) (void)hipHostFree(m->step_host);
    if (m->logits_host) (void)hipHostFree(m->logits_host);
    if (m->gen_host) (void)hipHostFree(m->gen_host);
    for (lrs_weight *w : m->owned) lrs_weight_free(w);
    delete m;
}

// a hybrid model's recurrent state only moves forward: pos0 must be the
// current length
static int check_continue(lrs_model *m, uint32_t pos0) {
    if (m->hybrid && pos0 != m->len)
        return fail(LRS_E_ARG, "hybrid model: position " + std::to_string(pos0) +
                                   " must continue the sequence at " + std::to_string(m->len) +
                                   " (the recurrent state cannot be rewound; reset first)");
    return LRS_OK;
}

// the wait-error word of the combine + o launches (a matvec workgroup that
// ran out of polls went on without its input): copied out with each call's
// results, checked after the call's synchronisation
static constexpr uint32_t AO_ERR_WORD = 4 * 1024;  // past the step slots of step_host
static hipError_t ao_err_fetch(lrs_model *m, hipStream_t s) {
    m->step_host[AO_ERR_WORD] = 0;
    if (!m->ao_sync) return hipSuccess;
    return hipMemcpyAsync(m->step_host + AO_ERR_WORD, m->ao_sync + 32, sizeof(uint32_t),
                          hipMemcpyDeviceToHost, s);
}
static int ao_err_check(lrs_model *m) {
    if (m->step_host[AO_ERR_WORD] == 0) return LRS_OK;
    // the word and the whole flag matrix back to zero: flags a late producer
    // raised after its consumer gave up must not release the next launch's
    (void)hipMemset(m->ao_sync, 0, m->ao_sync_bytes);
    return fail(LRS_E_HIP, "attention output launch: a workgroup's wait for its input ran out");
}

static int check_step(lrs_model *m, uint32_t token, uint32_t pos) {
    if (token >= m->cfg.vocab)
        return fail(LRS_E_ARG, "token " + std::to_string(token) + " outside the vocabulary");
    if (pos >= m->cfg.ctx)
        return fail(LRS_E_CTX_OVERFLOW, "position " + std::to_string(pos) + " beyond context " +
                                            std::to_string(m->cfg.ctx));
    return LRS_OK;
}

// ---- batched prompt blocks on the matrix cores --------------------------
// Tokens per block of the batched prompt path (batch_size()).
static constexpr uint32_t PREFILL_BLOCK = 512;

// every matmul weight has a GEMM kernel and the attention shape is supported
static bool prefill_capable(const lrs_model *m) {
    // with the reference's Q8_0 input rounding on, Q8_0 weights stay on the
    // token path (the GEMM multiplies the f32 activations)
    const bool q8_ok = std::none_of(m->layers.begin(), m->layers.end(), [](const DevLayer &L) {
        return L.qkv_q8 || L.o_q8 || L.ffn_q8 || L.down_q8;
    });
    auto ok = [q8_ok](const lrs_weight *w) {
        const uint32_t t = w->v.type;
        return (t == T_Q4_K || t == T_Q5_K || t == T_Q6_K || (t == T_Q8_0 && q8_ok)) &&
               w->v.n_in % 256 == 0;
    };
    const lrs_config &c = m->cfg;
    if ((c.head_dim != 64 && c.head_dim != 128 && (c.head_dim != 256 || !m->hybrid)) ||
        c.n_head / c.n_head_kv > 8 || c.n_embd % 4)
        return false;
    for (const DevLayer &L : m->layers) {
        if (!ok(L.gate) || !ok(L.up) || !ok(L.down)) return false;
        if (L.dn ? (!ok(L.ssm_qkv) || !ok(L.ssm_gate) || !ok(L.ssm_out))
                 : (!ok(L.q) || !ok(L.k) || !ok(L.v) || !ok(L.o)))
            return false;
    }
    return true;
}

static int ensure_prefill(lrs_model *m) {
    if (m->pb_cap) return LRS_OK;
    const lrs_config &c = m->cfg;
    const size_t B = PREFILL_BLOCK, qd = (size_t)c.n_head * c.head_dim,
                 kvd = (size_t)c.n_head_kv * c.head_dim;
    int rc;
    if ((rc = dev_alloc(m, B * c.n_embd * 4, (void **)&m->pX)) ||
        (rc = dev_alloc(m, B * c.n_embd * 4, (void **)&m->pXN)) ||
        (rc = dev_alloc(m, B * qd * 4, (void **)&m->pQt)) ||
        (rc = dev_alloc(m, B * kvd * 4, (void **)&m->pKt)) ||
        (rc = dev_alloc(m, B * kvd * 4, (void **)&m->pVt)) ||
        (rc = dev_alloc(m, B * qd * 4, (void **)&m->pQ)) ||
        (rc = dev_alloc(m, B * qd * 4, (void **)&m->pATT)) ||
        (rc = dev_alloc(m, B * c.n_ff * 4, (void **)&m->pG)) ||
        (rc = dev_alloc(m, B * c.n_ff * 4, (void **)&m->pU)) ||
        (rc = dev_alloc(m, B * std::max<size_t>(std::max<size_t>(c.n_embd, qd),
                                                std::max<size_t>(c.n_ff, (size_t)m->hc.dn_v_heads *
                                                                             m->hc.dn_state)) * 4,
                        (void **)&m->pA16)) ||
        // K-sliced GEMMs (few output tiles: o, down, and the narrow k / v):
        // 8 slices of [rows][n_embd] partials
        (rc = dev_alloc(m, m->work_bytes = 8 * B * c.n_embd * 4, (void **)&m->pWork)) ||
        (rc = dev_alloc(m, B * 4, (void **)&m->ptok)))
        return rc;
    if (m->hybrid) {
        const lrs_hybrid_config &hc = m->hc;
        const size_t VD = (size_t)hc.dn_v_heads * hc.dn_state,
                     CD = 2 * (size_t)hc.dn_k_heads * hc.dn_state + VD;
        if ((rc = dev_alloc(m, B * 2 * qd * 4, (void **)&m->pQG)) ||
            (rc = dev_alloc(m, B * CD * 4, (void **)&m->pCI)) ||
            (rc = dev_alloc(m, B * CD * 4, (void **)&m->pCO)) ||
            (rc = dev_alloc(m, B * VD * 4, (void **)&m->pZ)) ||
            (rc = dev_alloc(m, B * VD * 4, (void **)&m->pO)) ||
            (rc = dev_alloc(m, B * VD * 4, (void **)&m->pY)) ||
            (rc = dev_alloc(m, B * hc.dn_v_heads * sizeof(float2), (void **)&m->pGB)))
            return rc;
    }
    m->pb_cap = PREFILL_BLOCK;
    return LRS_OK;
}

// one block of nb tokens at positions pos0.. through every layer (the
// forward of model.rs:99-266 with the matmuls as GEMMs, operands split into
// bf16 hi + lo); leaves the residual rows in pX
static int prefill_block(lrs_model *m, const uint32_t *tokens, uint32_t nb, uint32_t pos0) {
    const lrs_config &c = m->cfg;
    hipStream_t s = m->ctx->stream;
    const uint32_t qd = c.n_head * c.head_dim, kvd = c.n_head_kv * c.head_dim, E = c.n_embd;
    constexpr int P = 3;
    // GEMM inputs as bf16 hi / lo planes: hi at pA16, lo right after the
    // rows x cols hi plane
    __bf16 *const hi = m->pA16;
    auto lo = [&](uint32_t rows, uint32_t cols) { return hi + (size_t)rows * cols; };
    auto split = [&](const float *a, size_t n) { return launch_split_bf16(a, n, hi, hi + n, s); };
    // y (+)= A W^T over the block, split over K across workgroups when the
    // weight has too few output tiles to fill the GPU (the slices' partials
    // must fit the work buffer)
    auto gemm = [&](const lrs_weight *w, uint32_t K, float *y, uint32_t N, bool accum = false) {
        float *work = gemm_work_bytes(nb, N, K, P) <= m->work_bytes ? m->pWork : nullptr;
        return launch_gemm(w->v, hi, lo(nb, K), y, nb, N, P, s, accum, work);
    };
    // weights over the same normalised rows (q / k / v, gate / up, or the
    // delta net's in-projections): one launch over all their output tiles
    // when that alone keeps most CUs busy for the whole K (fewer partly
    // filled rounds of workgroups than one launch each), else one launch
    // each (split over K)
    auto gemm_group = [&](uint32_t n, const lrs_weight *const *w, float *const *y,
                          const uint32_t *N) -> hipError_t {
        WeightView wv[3];
        uint32_t tiles = 0;
        for (uint32_t i = 0; i < n; i++) {
            wv[i] = w[i]->v;
            tiles += gemm_out_tiles(nb, N[i], P);
        }
        if (tiles >= 192 && gemm_segs_supported(wv, n))
            return launch_gemm_segs(wv, y, N, n, hi, lo(nb, E), nb, P, s);
        for (uint32_t i = 0; i < n; i++) {
            const hipError_t e = gemm(w[i], E, y[i], N[i]);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    };
    // pX += A W^T (o, down, the delta net's out-projection), then the
    // RMSNorm rows of pX times nw as GEMM planes (and in f32 into xn): when
    // the GEMM splits over K, its slices' reduce and the norm run as one
    // kernel
    auto gemm_resid_norm = [&](const lrs_weight *w, uint32_t K, const float *nw,
                               float *xn) -> hipError_t {
        float *work = gemm_work_bytes(nb, E, K, P) <= m->work_bytes ? m->pWork : nullptr;
        uint32_t ks = 1;
        const hipError_t e = launch_gemm(w->v, hi, lo(nb, K), m->pX, nb, E, P, s, true, work, &ks);
        if (e != hipSuccess) return e;
        return ks > 1 ? launch_reduce_norm_rows(m->pWork, ks, m->pX, nw, c.rms_eps, E, nb, xn, hi, s)
                      : launch_rmsnorm_rows(m->pX, nw, c.rms_eps, E, nb, xn, s, hi);
    };
    // the normalised rows as GEMM planes, and in f32 for a delta-net block,
    // which reads them for its gates
    auto xn_for = [&](const DevLayer &L) { return m->hybrid && L.dn ? m->pXN : nullptr; };
    // the previous layer's down GEMM already normalised the rows for this one
    bool normed = false;
    // the FFN of layer l: gate / up, SwiGLU, down + residual (+ the next
    // layer's attention norm)
    auto ffn = [&](uint32_t l) -> hipError_t {
        const DevLayer &L = m->layers[l];
        {
            const lrs_weight *const w[2] = {L.gate, L.up};
            float *const y[2] = {m->pG, m->pU};
            const uint32_t N[2] = {c.n_ff, c.n_ff};
            const hipError_t e = gemm_group(2, w, y, N);
            if (e != hipSuccess) return e;
        }
        const hipError_t e = launch_swiglu_split(m->pG, m->pU, (size_t)nb * c.n_ff, hi, s);
        if (e != hipSuccess) return e;
        if (l + 1 == c.n_layer) return gemm(L.down, c.n_ff, m->pX, E, true);
        const DevLayer &N = m->layers[l + 1];
        normed = true;
        return gemm_resid_norm(L.down, c.n_ff, N.attn_norm, xn_for(N));
    };
    LRS_HIP(hipMemcpyAsync(m->ptok, tokens, nb * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    LRS_HIP(launch_dequant_rows(m->embd->v, m->ptok, nb, m->pX, s));
    for (uint32_t l = 0; l < c.n_layer; l++) {
        const DevLayer &L = m->layers[l];
        if (!normed) LRS_HIP(launch_rmsnorm_rows(m->pX, L.attn_norm, c.rms_eps, E, nb, xn_for(L), s, hi));
        normed = false;
        if (m->hybrid) {
            if (L.dn) {
                // gated delta net over the block (plano_delta with n_tok = nb)
                const lrs_hybrid_config &hc = m->hc;
                const uint32_t VD = hc.dn_v_heads * hc.dn_state;
                const uint32_t CD = 2 * hc.dn_k_heads * hc.dn_state + VD;
                {
                    const lrs_weight *const w[2] = {L.ssm_qkv, L.ssm_gate};
                    float *const y[2] = {m->pCI, m->pZ};
                    const uint32_t N[2] = {CD, VD};
                    LRS_HIP(gemm_group(2, w, y, N));
                }
                DnBlockArgs da = {};
                da.hn = m->pXN;
                da.alpha = L.alpha;
                da.beta = L.beta;
                da.a = L.ssm_a;
                da.dt = L.ssm_dt;
                da.conv_w = L.conv;
                da.norm_w = L.ssm_norm;
                da.cin = m->pCI;
                da.z = m->pZ;
                da.win = L.win;
                da.state = L.state;
                da.cout = m->pCO;
                da.gb = m->pGB;
                da.o = m->pO;
                da.y = m->pY;
                da.n_embd = E;
                da.k_heads = hc.dn_k_heads;
                da.v_heads = hc.dn_v_heads;
                da.d_state = hc.dn_state;
                da.d_conv = hc.dn_conv;
                da.nb = nb;
                da.pos0 = pos0;
                da.eps = c.rms_eps;
                LRS_HIP(launch_dn_prefill(da, s));
                LRS_HIP(split(m->pY, (size_t)nb * VD));
                LRS_HIP(gemm_resid_norm(L.ssm_out, VD, L.ffn_norm, nullptr));
            } else {
                // gated attention: Q (+ gate), k, v; QK-norm + RoPE; causal
                // attention over the cache; sigmoid gate; o
                {
                    const lrs_weight *const w[3] = {L.q, L.k, L.v};
                    float *const y[3] = {m->pQG, m->pKt, m->pVt};
                    const uint32_t N[3] = {2 * qd, kvd, kvd};
                    LRS_HIP(gemm_group(3, w, y, N));
                }
                LRS_HIP(launch_qk_prep_rows(m->pQG, m->pKt, m->pVt, L.q_norm, L.k_norm, m->freq, m->pQ,
                                            L.kc, L.vc, nb, pos0, c.n_head, c.n_head_kv, c.head_dim,
                                            c.ctx, c.rope_dim, c.rms_eps, s));
                LRS_HIP(launch_attn_prefill(m->pQ, L.kc, L.vc, m->pATT, nb, pos0, c.n_head, c.n_head_kv,
                                            c.head_dim, c.ctx, s));
                LRS_HIP(launch_gate_rows(m->pATT, m->pQG, nb, qd, c.head_dim, s));
                LRS_HIP(split(m->pATT, (size_t)nb * qd));
                LRS_HIP(gemm_resid_norm(L.o, qd, L.ffn_norm, nullptr));
            }
            LRS_HIP(ffn(l));
            continue;
        }
        {
            const lrs_weight *const w[3] = {L.q, L.k, L.v};
            float *const y[3] = {m->pQt, m->pKt, m->pVt};
            const uint32_t N[3] = {qd, kvd, kvd};
            LRS_HIP(gemm_group(3, w, y, N));
        }
        LRS_HIP(launch_qkv_post(m->pQt, m->pKt, m->pVt, L.bq, L.bk, L.bv, m->freq, m->pQ, L.kc,
                                L.vc, nb, pos0, qd, kvd, c.head_dim, c.rope_dim, c.ctx, s));
        LRS_HIP(launch_attn_prefill(m->pQ, L.kc, L.vc, m->pATT, nb, pos0, c.n_head, c.n_head_kv,
                                    c.head_dim, c.ctx, s));
        LRS_HIP(split(m->pATT, (size_t)nb * qd));
        LRS_HIP(gemm_resid_norm(L.o, qd, L.ffn_norm, nullptr));
        LRS_HIP(ffn(l));
    }
    return LRS_OK;
}

// the prompt in blocks of at most PREFILL_BLOCK tokens; with head, the logits
// of the last token land in m->logits
static int prefill(lrs_model *m, const uint32_t *tokens, uint32_t n, uint32_t pos0, bool head) {
    int rc = ensure_prefill(m);
    if (rc) return rc;
    hipStream_t s = m->ctx->stream;
    uint32_t nb = 0;
    for (uint32_t i = 0; i < n; i += nb) {
        nb = min(m->pb_cap, n - i);
        if ((rc = prefill_block(m, tokens + i, nb, pos0 + i))) return rc;
        // the host token ids of this block must stay valid until it is read
        LRS_HIP(hipStreamSynchronize(s));
    }
    if (!head) return LRS_OK;
    LRS_HIP(hipMemcpyAsync(m->x, m->pX + (size_t)(nb - 1) * m->cfg.n_embd,
                           m->cfg.n_embd * sizeof(float), hipMemcpyDeviceToDevice, s));
    LRS_HIP(launch_xpack(m->x, m->output_norm, m->cfg.n_embd, m->cfg.n_embd / 32, m->pk_n, s,
                         m->xsq));
    LRS_HIP(op_head(m, false));
    return LRS_OK;
}

// enqueues n tokens at pos0.. (logits graph) without waiting; every token's
// {token, pos} goes through its own pinned slot, and the stream is drained
// whenever the slots run out
static constexpr uint32_t STEP_SLOTS = 1024;
static_assert(4 * STEP_SLOTS <= AO_ERR_WORD, "the wait-error word follows the step slots");

static int enqueue_tokens(lrs_model *m, const uint32_t *tokens, uint32_t n, uint32_t pos0) {
    for (uint32_t i = 0; i < n; i++) {
        int rc = check_step(m, tokens[i], pos0 + i);
        if (rc) return rc;
    }
    LRS_HIP(hipSetDevice(m->ctx->device));
    hipStream_t s = m->ctx->stream;
    LRS_HIP(hipStreamSynchronize(s));  // slots of an earlier call are free
    for (uint32_t i = 0; i < n; i++) {
        const uint32_t slot = i % STEP_SLOTS;
        if (i > 0 && slot == 0) LRS_HIP(hipStreamSynchronize(s));
        uint32_t *sh = m->step_host + 4 * slot;
        sh[0] = tokens[i];
        sh[1] = pos0 + i;
        sh[2] = 0;
        LRS_HIP(hipMemcpyAsync(m->step, sh, 3 * sizeof(uint32_t), hipMemcpyHostToDevice, s));
        LRS_HIP(run_forward(m, false));
    }
    return LRS_OK;
}

int lrs_decode(lrs_model *m, uint32_t token, uint32_t pos, float *logits) {
    if (!m || !logits) return fail(LRS_E_ARG, "null argument");
    int rc = check_step(m, token, pos);
    if (rc || (rc = check_continue(m, pos))) return rc;
    LRS_HIP(hipSetDevice(m->ctx->device));
    hipStream_t s = m->ctx->stream;
    m->step_host[0] = token;
    m->step_host[1] = pos;
    m->step_host[2] = 0;
    LRS_HIP(hipMemcpyAsync(m->step, m->step_host, 3 * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    LRS_HIP(run_forward(m, false));
    LRS_HIP(hipMemcpyAsync(m->logits_host, m->logits, m->cfg.vocab * sizeof(float),
                           hipMemcpyDeviceToHost, s));
    LRS_HIP(ao_err_fetch(m, s));
    LRS_HIP(hipStreamSynchronize(s));
    if (int e = ao_err_check(m)) return e;
    memcpy(logits, m->logits_host, m->cfg.vocab * sizeof(float));
    m->len = pos + 1;
    return LRS_OK;
}

uint32_t lrs_batch_size(const lrs_model *m) {
    if (!m) return 0u;
    return prefill_capable(m) ? PREFILL_BLOCK : 1u;
}

int lrs_decode_batch(lrs_model *m, const uint32_t *tokens, uint32_t n, uint32_t pos0, float *logits) {
    if (!m || !tokens || !logits || n == 0) return fail(LRS_E_ARG, "null argument / empty batch");
    // GpuResidentDecode::decode_batch (gpu.rs:392-400): the logits of the last
    // token; several tokens go through the matrix-core GEMMs in blocks when
    // every weight has one, else token by token
    int rc = check_continue(m, pos0);
    if (rc) return rc;
    if (n > 1 && prefill_capable(m)) {
        for (uint32_t i = 0; i < n; i++)
            if ((rc = check_step(m, tokens[i], pos0 + i))) return rc;
        LRS_HIP(hipSetDevice(m->ctx->device));
        LRS_HIP(hipStreamSynchronize(m->ctx->stream));
        if ((rc = prefill(m, tokens, n, pos0, true))) return rc;
    } else if ((rc = enqueue_tokens(m, tokens, n, pos0))) {
        return rc;
    }
    hipStream_t s = m->ctx->stream;
    LRS_HIP(hipMemcpyAsync(m->logits_host, m->logits, m->cfg.vocab * sizeof(float),
                           hipMemcpyDeviceToHost, s));
    LRS_HIP(ao_err_fetch(m, s));
    LRS_HIP(hipStreamSynchronize(s));
    if (int e = ao_err_check(m)) return e;
    memcpy(logits, m->logits_host, m->cfg.vocab * sizeof(float));
    m->len = pos0 + n;
    return LRS_OK;
}

void lrs_reset(lrs_model *m) {
    if (!m) return;
    m->len = 0;
    if (m->rec) {
        // delta-net states and conv windows back to zero (the KV cache needs
        // no clearing: attention reads positions 0..pos only)
        (void)hipSetDevice(m->ctx->device);
        (void)hipMemsetAsync(m->rec, 0, m->rec_bytes, m->ctx->stream);
        (void)hipStreamSynchronize(m->ctx->stream);
    }
}

uint32_t lrs_model_len(const lrs_model *m) { return m ? m->len : 0; }

int lrs_model_set_q8_rounding(lrs_model *m, int on) {
    if (!m) return fail(LRS_E_ARG, "null model");
    if (m->hybrid) return fail(LRS_E_UNSUPPORTED, "the Q8_0 input rounding applies to dense models");
    LRS_HIP(hipSetDevice(m->ctx->device));
    LRS_HIP(hipStreamSynchronize(m->ctx->stream));
    set_q8_flags(m, on != 0);
    return capture_graphs(m);
}

int lrs_decode_greedy(lrs_model *m, uint32_t token, uint32_t pos, uint32_t *next) {
    if (!m || !next) return fail(LRS_E_ARG, "null argument");
    int rc = check_step(m, token, pos);
    if (rc || (rc = check_continue(m, pos))) return rc;
    LRS_HIP(hipSetDevice(m->ctx->device));
    hipStream_t s = m->ctx->stream;
    m->step_host[0] = token;
    m->step_host[1] = pos;
    m->step_host[2] = 0;
    LRS_HIP(hipMemcpyAsync(m->step, m->step_host, 3 * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    LRS_HIP(run_forward(m, true));
    LRS_HIP(hipMemcpyAsync(m->step_host + 4, m->step, sizeof(uint32_t), hipMemcpyDeviceToHost, s));
    LRS_HIP(ao_err_fetch(m, s));
    LRS_HIP(hipStreamSynchronize(s));
    if (int e = ao_err_check(m)) return e;
    *next = m->step_host[4];
    m->len = pos + 1;
    return LRS_OK;
}

int lrs_generate_greedy(lrs_model *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t pos0,
                        uint32_t n_gen, uint32_t *out_tokens) {
    if (!m || !prompt || !out_tokens || n_prompt == 0 || n_gen == 0)
        return fail(LRS_E_ARG, "null argument / empty prompt or generation");
    // the last generated token is not fed back, so it needs no cache slot
    if ((size_t)pos0 + n_prompt + n_gen - 1 > m->cfg.ctx)
        return fail(LRS_E_CTX_OVERFLOW, "prompt + generation exceed the context");
    if (n_gen > m->gen_cap) return fail(LRS_E_ARG, "too many tokens for one call");
    for (uint32_t i = 0; i < n_prompt; i++)
        if (prompt[i] >= m->cfg.vocab) return fail(LRS_E_ARG, "prompt token outside the vocabulary");
    if (int rc0 = check_continue(m, pos0)) return rc0;
    LRS_HIP(hipSetDevice(m->ctx->device));
    hipStream_t s = m->ctx->stream;
    // prefill: tokens 0..n_prompt-2, then the last prompt token starts the
    // greedy chain (its argmax is the first generated token)
    int rc = LRS_OK;
    if (n_prompt > 2 && prefill_capable(m)) {
        if ((rc = prefill(m, prompt, n_prompt - 1, pos0, false))) return rc;
    } else if (n_prompt > 1 && (rc = enqueue_tokens(m, prompt, n_prompt - 1, pos0))) {
        return rc;
    }
    LRS_HIP(hipStreamSynchronize(s));
    m->step_host[0] = prompt[n_prompt - 1];
    m->step_host[1] = pos0 + n_prompt - 1;
    m->step_host[2] = 0;
    LRS_HIP(hipMemcpyAsync(m->step, m->step_host, 3 * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    for (uint32_t i = 0; i < n_gen; i++) LRS_HIP(run_forward(m, true));
    // through the pinned buffer: the caller's memory is pageable
    LRS_HIP(hipMemcpyAsync(m->gen_host, m->gen, n_gen * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
    LRS_HIP(ao_err_fetch(m, s));
    LRS_HIP(hipStreamSynchronize(s));
    if (int e = ao_err_check(m)) return e;
    memcpy(out_tokens, m->gen_host, n_gen * sizeof(uint32_t));
    m->len = pos0 + n_prompt + n_gen - 1;
    return LRS_OK;
}

int lrs_model_profile(lrs_model *m, uint32_t op, uint32_t iters, float *avg_us, size_t *bytes) {
    if (!m || !avg_us || iters == 0) return fail(LRS_E_ARG, "null argument");
    const lrs_config &c = m->cfg;
    if (op > LRS_OP_MATVECS) return fail(LRS_E_ARG, "unknown op");
    if (op == LRS_OP_MATVECS && m->hybrid) return fail(LRS_E_ARG, "op needs a dense model");
    const bool dn_op = op == LRS_OP_DN_PROJ || op == LRS_OP_DN_STEP || op == LRS_OP_DN_OUT;
    const bool attn_op = op == LRS_OP_QKV || op == LRS_OP_ATTN || op == LRS_OP_O ||
                         op == LRS_OP_QK_PREP;
    if ((dn_op || op == LRS_OP_QK_PREP) && !m->hybrid)
        return fail(LRS_E_ARG, "op needs a hybrid model");
    // the layers the op runs on (all, or those of its mixer kind)
    std::vector<uint32_t> ls;
    for (uint32_t l = 0; l < c.n_layer; l++)
        if ((!dn_op && !attn_op) || (dn_op == m->layers[l].dn)) ls.push_back(l);
    if (ls.empty()) return fail(LRS_E_ARG, "no layer of this kind");
    LRS_HIP(hipSetDevice(m->ctx->device));
    hipStream_t s = m->ctx->stream;
    const bool per_layer = op != LRS_OP_HEAD;
    size_t b = 0;
    const uint32_t kvd = c.n_head_kv * c.head_dim;
    const uint32_t L = m->len ? m->len : 1;  // attention reads this many positions
    // algorithmic bytes: GGUF weight bytes + f16 K/V + f32 vectors read or
    // written once (scratch such as attention partials is not counted)
    const size_t E4 = (size_t)c.n_embd * 4, qd4 = (size_t)c.n_head * c.head_dim * 4;
    const lrs_hybrid_config &hc = m->hc;
    const size_t dnD = hc.dn_state, VD4 = (size_t)hc.dn_v_heads * dnD * 4,
                 CD4 = (size_t)(2 * hc.dn_k_heads + hc.dn_v_heads) * dnD * 4;
    if (per_layer) {
        const DevLayer &D = m->layers[ls[0]];
        switch (op) {
        case LRS_OP_QKV:
            if (m->hybrid)  // Q (query + gate) / k / v rows out as f32
                b = wbytes(D.q) + wbytes(D.k) + wbytes(D.v) + 2 * E4 + 2 * qd4 + (size_t)kvd * 8;
            else
                b = wbytes(D.q) + wbytes(D.k) + wbytes(D.v) + 2 * E4 + qd4 + (size_t)kvd * 2 * 2 +
                    (D.bq ? qd4 + (size_t)kvd * 8 : 0);
            break;
        case LRS_OP_QK_PREP:
            // nothing of its own when the attention split does it
            if (qkp_fused(m, D)) {
                *avg_us = 0.f;
                if (bytes) *bytes = 0;
                return LRS_OK;
            }
            b = 2 * qd4 + (size_t)kvd * 8 + qd4 + (size_t)kvd * 4;
            break;
        case LRS_OP_DN_PROJ:
            // plus the f32 gate rows when the launch computes the gates
            b = wbytes(D.ssm_qkv) + wbytes(D.ssm_gate) + 2 * E4 + CD4 + VD4 +
                (dn_gates_fused(m, D) ? 2 * (size_t)hc.dn_v_heads * E4 : 0);
            break;
        case LRS_OP_DN_STEP:
            // state read + written, f32 gate rows (unless the projection
            // launch read them), conv weights and window, inputs, the y pack
            // (3.5 B per element)
            b = 2 * (size_t)hc.dn_v_heads * dnD * dnD * 4 +
                (dn_gates_fused(m, D) ? 0 : 2 * (size_t)hc.dn_v_heads * E4) + CD4 * hc.dn_conv +
                CD4 * hc.dn_conv + CD4 + VD4 + 2 * E4 + VD4 / 4 * 7 / 2;
            break;
        case LRS_OP_DN_OUT: b = wbytes(D.ssm_out) + VD4 + 2 * E4; break;
        case LRS_OP_ATTN:
            // nothing of its own when the o launch runs the split
            if (sao_fused(m, D)) {
                *avg_us = 0.f;
                if (bytes) *bytes = 0;
                return LRS_OK;
            }
            b = attn_bytes(m, D, L);
            break;
        case LRS_OP_O: b = wbytes(D.o) + qd4 + 2 * E4 + (sao_fused(m, D) ? attn_bytes(m, D, L) : 0); break;
        case LRS_OP_GATEUP: b = wbytes(D.gate) + wbytes(D.up) + 2 * E4 + (size_t)c.n_ff * 4; break;
        case LRS_OP_DOWN: b = wbytes(D.down) + (size_t)c.n_ff * 4 + 2 * E4; break;
        case LRS_OP_FFN: b = wbytes(D.gate) + wbytes(D.up) + wbytes(D.down) + 3 * E4; break;
        case LRS_OP_MATVECS:
            // q/k/v (norm input + residual for the RMS sum, q out, K/V rows
            // appended), o (input, residual read + written), the FFN
            b = wbytes(D.q) + wbytes(D.k) + wbytes(D.v) + 2 * E4 + qd4 + (size_t)kvd * 2 * 2 +
                (D.bq ? qd4 + (size_t)kvd * 8 : 0) + wbytes(D.o) + qd4 + 2 * E4 + wbytes(D.gate) +
                wbytes(D.up) + wbytes(D.down) + 3 * E4;
            break;
        }
    } else {
        b = wbytes(m->output) + 2 * E4 + (size_t)c.vocab * 4;
    }
    // the step buffer must hold a valid position: the last decoded one
    m->step_host[0] = 0;
    m->step_host[1] = L - 1;
    m->step_host[2] = 0;
    LRS_HIP(hipMemcpyAsync(m->step, m->step_host, 3 * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    auto one = [&](uint32_t i) -> hipError_t {
        const uint32_t l = ls[i % ls.size()];
        switch (op) {
        case LRS_OP_QKV: return m->hybrid ? op_hattn_proj(m, l) : op_qkv(m, l);
        case LRS_OP_ATTN: return op_attn(m, l);
        case LRS_OP_O: case LRS_OP_DN_OUT: return op_o(m, l);
        case LRS_OP_GATEUP: return op_gateup(m, l);
        case LRS_OP_DOWN: return op_down(m, l);
        case LRS_OP_FFN: return op_ffn(m, l);
        case LRS_OP_MATVECS: {
            hipError_t e;
            if ((e = op_qkv(m, l)) != hipSuccess || (e = op_o(m, l)) != hipSuccess) return e;
            return op_ffn(m, l);
        }
        case LRS_OP_QK_PREP: return op_qk_prep(m, l);
        case LRS_OP_DN_PROJ: return op_dn_proj(m, l);
        case LRS_OP_DN_STEP: return op_dn_step(m, l);
        default: return op_head(m, false);
        }
    };
    for (uint32_t i = 0; i < ls.size() && i < iters; i++) LRS_HIP(one(i));  // warm
    LRS_HIP(hipEventRecord(m->ctx->ev0, s));
    for (uint32_t i = 0; i < iters; i++) LRS_HIP(one(i));
    LRS_HIP(hipEventRecord(m->ctx->ev1, s));
    LRS_HIP(ao_err_fetch(m, s));
    LRS_HIP(hipEventSynchronize(m->ctx->ev1));
    LRS_HIP(hipStreamSynchronize(s));
    if (int e = ao_err_check(m)) return e;
    float ms = 0.f;
    LRS_HIP(hipEventElapsedTime(&ms, m->ctx->ev0, m->ctx->ev1));
    *avg_us = ms * 1000.f / (float)iters;
    if (bytes) *bytes = b;
    return LRS_OK;
}

size_t lrs_model_bytes_per_token(const lrs_model *m) { return m ? m->gguf_bytes_per_token : 0; }

}  // extern "C"
