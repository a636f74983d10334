/*
 * lrs_oracle — CPU restatement of llama.rs's reference CPU path for the batch-1
 * dequant x matvec decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product (llama.rs_amd/liblrs.so) never links, loads or falls back to it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the llama.rs repository root).  Floating-point order follows the Rust code:
 * Rust never contracts a*b+c into an FMA and f32 `Iterator::sum` is a
 * sequential left fold, so this file is compiled with -ffp-contract=off and
 * every reduction is a plain left-to-right loop.
 *
 * Pinning (see tests/test_oracle.py):
 *   f16<->f32          exhaustive vs numpy float16 (independent implementation)
 *   Q8_0/Q4_0/Q4_K/Q6_K dequant   reference known answers (dequant.rs:269-469)
 *                                 + an independent numpy restatement, brute force
 *   Q5_K dequant       llama.cpp gguf-py golden block (dequant.rs:472-548)
 *   matvec             f64 dot, one-hot columns, batched-column invariance
 *   rmsnorm/rope/swiglu/softmax/argmax/attention  reference known answers
 *                                 (ops.rs:1065-1164, attention.rs:174-200)
 *   forward            closed-form reductions (tests/test_oracle_model_pins.py:
 *                      zeroed mixers, one cached position, W_v = 0, FFN-only
 *                      layer, the int8-activation head) and a numpy float64
 *                      restatement of model.rs:99-266 (no reference golden
 *                      logits exist)
 *   delta-net ops      reference known answers (delta_net.rs:133-255) and a
 *                      numpy restatement
 *   hybrid forward     closed forms in tests/test_oracle_model_pins.py: the
 *                      delta rule over two tokens from a zero state; the gated
 *                      attention with one cached position (gate = rows
 *                      [HD, 2HD) of each head's Q block); QK-norm scale
 *                      invariance per head; partial RoPE leaving dims >=
 *                      rope_dim alone; adjacent-pair scores expanded by hand
 *                      at the closed-form frequencies 1 and base^(-1/2); a
 *                      delta-net layer followed by an attention layer
 */
#ifndef LRS_ORACLE_H
#define LRS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type ids: crates/gguf/src/types.rs:84-107 */
enum {
    LRSO_F32 = 0,
    LRSO_F16 = 1,
    LRSO_Q4_0 = 2,
    LRSO_Q8_0 = 8,
    LRSO_Q4_K = 12,
    LRSO_Q5_K = 13,
    LRSO_Q6_K = 14,
};

/* elements / bytes per block: types.rs:30-78.  <0 for unsupported ids. */
int64_t lrso_block_size(uint32_t type);
int64_t lrso_type_size(uint32_t type);

/* IEEE binary16 widening (half 2.7.1 `to_f32`) and round-to-nearest-even
 * narrowing (`half::f16::from_f32`). */
float lrso_f16_to_f32(uint16_t h);
uint16_t lrso_f32_to_f16(float f);

/* ggml_cpu::dequant_to_f32 (crates/ggml-cpu/src/dequant.rs:10-258).
 * Returns the element count, or -1 on a size error / -2 on unsupported type. */
int64_t lrso_dequant(uint32_t type, const uint8_t *bytes, size_t len, float *out);

/* RawTensor::matmul_into for non-Q8_0 types (weights.rs:109-124) == dequant +
 * ops::matmul (ops.rs:78-101): y[c*n_out+j] = sequential f32 fold over i of
 * deq(W[j,i]) * x[c*n_in+i].  Q8_0 is handled the same way here (dequant + f32
 * dot, the config-1 oracle of integration.rs:383-402).  Rows are dequantized
 * one at a time (same per-element arithmetic as the cached f32 tensor).
 * n_threads <= 1 runs serially; rows are split in chunks of 32 (ops.rs:76).
 * Returns 0, or <0 on bad sizes. */
int lrso_matvec(uint32_t type, const uint8_t *w, size_t w_len, uint32_t n_in,
                uint32_t n_out, const float *x, float *y, uint32_t cols,
                int n_threads);
/* Q8_0 activation quantization (ops.rs:284-368; half_even: the AVX2 path,
 * else the scalar path) into n/32 GGUF Q8_0 blocks, and the int8-activation
 * Q8_0 matvec of one column (ops.rs:704-724, 728-886). */
int lrso_quantize_q8_0(const float *x, uint32_t n, int half_even, uint8_t *out);
int lrso_matvec_q8_0_actq(const uint8_t *w, size_t w_len, uint32_t n_in, uint32_t n_out,
                          const float *x, int half_even, float *y);
/* the same over n_threads threads (rows in chunks of 32) */
int lrso_matvec_q8_0_actq_mt(const uint8_t *w, size_t w_len, uint32_t n_in, uint32_t n_out,
                             const float *x, int half_even, float *y, int n_threads);

/* ---- deterministic synthetic blocks (counter-based, identical on GPU) ---- */
uint64_t lrso_hash(uint64_t seed, uint64_t block, uint32_t j);
/* mode 0: the BASELINE distributions (random scale bytes).
 * mode 1: "centred" K-quants (Q4_K/Q5_K mins equal their scales and
 *         dmin = f16(7.5*d) / f16(15.5*d), so weights are roughly zero-mean).
 * d_lo/d_hi: range of the f16 super-block scales (BASELINE: 1e-3..1e-2). */
int lrso_gen_blocks(uint32_t type, uint64_t seed, uint64_t block0,
                    uint64_t n_blocks, int mode, float d_lo, float d_hi,
                    uint8_t *out);
/* uniform f32 in [lo,hi) from the hash stream (element i uses block=i, j=0) */
void lrso_gen_uniform(uint64_t seed, uint64_t n, float lo, float hi, float *out);
/* N(0,1) f32 via Box-Muller in double precision (host-only). */
void lrso_gen_normal(uint64_t seed, uint64_t n, float *out);

/* ---- per-op restatements ---- */
/* ops.rs:56-66 */
void lrso_rmsnorm_scale(const float *x, const float *w, uint32_t n_tok,
                        uint32_t dim, float eps, float *out);
/* model.rs:339-343 */
void lrso_freq_table(float freq_base, uint32_t rope_dim, float *out);
/* ops.rs:952-975 (in place) */
void lrso_rope_norm(float *x, uint32_t n_tok, uint32_t n_head, uint32_t head_dim,
                    uint32_t rope_dim, const float *freq, uint32_t pos0);
/* ops.rs:978-988 */
void lrso_swiglu(const float *g, const float *u, uint32_t n, float *out);
/* ops.rs:991-1003 (in place) */
void lrso_softmax(float *z, uint32_t n);
/* ops.rs:1035-1045 */
uint32_t lrso_argmax(const float *v, uint32_t n);
/* attention.rs:76-166: q [n_tok*n_head*hd], k/v caches [(pos0+n_tok)*kv_dim] */
void lrso_attention(const float *q, const float *k_cache, const float *v_cache,
                    uint32_t n_tok, uint32_t pos0, uint32_t n_head,
                    uint32_t n_head_kv, uint32_t head_dim, float *out);

/* ---- dense Llama/Qwen2 model forward (model.rs:99-266) ---- */
typedef struct {
    uint32_t n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, vocab;
    uint32_t rope_dim, ctx;
    float rms_eps, freq_base;
} lrso_config;

typedef struct {
    uint32_t type;          /* GGUF type id */
    const uint8_t *bytes;   /* borrowed for the model's lifetime */
    size_t len;
} lrso_tensor;

typedef struct {
    lrso_tensor attn_norm, attn_q, attn_k, attn_v, attn_output;
    lrso_tensor ffn_norm, ffn_gate, ffn_up, ffn_down;
    lrso_tensor bq, bk, bv; /* optional F32 biases: bytes == NULL when absent */
} lrso_layer;

typedef struct lrso_model lrso_model;

/* kv_f16 != 0 rounds K/V through binary16 on append (the GPU cache format,
 * integration.rs:872-893 does the same in its CPU reference). */
lrso_model *lrso_model_create(const lrso_config *cfg, const lrso_tensor *token_embd,
                              const lrso_layer *layers, const lrso_tensor *output_norm,
                              const lrso_tensor *output, int kv_f16, int n_threads);
/* Model::forward: processes tokens at positions len..len+n_tok, appends to the
 * cache and writes the last token's logits [vocab].  0 / <0 on error
 * (-3 = context overflow, attention.rs:36-40). */
int lrso_model_forward(lrso_model *m, const uint32_t *tokens, uint32_t n_tok,
                       float *logits);
/* Same forward but stops after `n_layers_run` layers and skips the head; used
 * to time a bounded sample of a large model for the CPU baseline. */
int lrso_model_forward_partial(lrso_model *m, const uint32_t *tokens, uint32_t n_tok,
                               uint32_t n_layers_run);
/* on (the default): Q8_0 weights take the reference forward's int8-activation
 * path (weights.rs:113-117); off: dequant + f32 matmul like the K-quants */
void lrso_model_set_q8_actq(lrso_model *m, int on);
uint32_t lrso_model_len(const lrso_model *m);
void lrso_model_reset(lrso_model *m);
void lrso_model_destroy(lrso_model *m);

/* ---- gated delta-net primitives (crates/llama-model/src/delta_net.rs) ---- */
float lrso_softplus(float x);                       /* delta_net.rs:13-20 */
float lrso_sigmoid(float x);                        /* delta_net.rs:22-25 */
void lrso_l2_norm_rows(float *x, uint32_t n_rows, uint32_t dim, float eps);
/* causal depthwise conv over one token with a [channel][d_conv-1] state
 * window (no activation; the caller applies SiLU): delta_net.rs:51-78 */
void lrso_conv1d_step(float *state, const float *x, const float *w,
                      uint32_t channels, uint32_t d_conv, float *out);
/* one gated delta-rule step for one head with a d x d state stored transposed
 * (state[j*d+i] = S[i][j]): delta_net.rs:90-131 */
void lrso_delta_net_step(float *state, const float *q, const float *k,
                         const float *v, float g, float beta, uint32_t d,
                         float *out);
float lrso_silu(float x);                           /* delta_net.rs:27-30 */

/* ---- hybrid attention + gated delta-net model (qwen35) ----
 * The reference has no CPU forward for this architecture (runner.rs:164); this
 * restates the GPU plan's op order (resident_forward.rs:3826-4103 with
 * plano_delta :2252-2470) with the CPU primitives of delta_net.rs and ops.rs
 * and the shader formulas of dn_gates.comp, dn_norm.comp, dn_l2_qk.comp,
 * dn_conv.comp, delta_net.comp and gate_quant.comp.  No reference logits
 * exist for it; both mixers are pinned by closed forms (see the top of this
 * header) and the whole by a float64 numpy restatement (tests/npref.py). */
typedef struct {
    lrso_config base;            /* full-attention layers use n_head, n_head_kv, head_dim */
    uint32_t full_attn_interval; /* layer l is full attention iff (l+1) % interval == 0 */
    uint32_t dn_k_heads, dn_v_heads, dn_state, dn_conv;
} lrso_hybrid_config;
typedef struct {
    lrso_tensor attn_norm, post_norm, ffn_gate, ffn_up, ffn_down;
    /* full attention: attn_q is [n_head * 2 * head_dim] rows, query then gate
     * per head; q_norm / k_norm F32 [head_dim] */
    lrso_tensor attn_q, attn_k, attn_v, attn_output, q_norm, k_norm;
    /* delta net: ssm_qkv [conv_dim = 2*k_heads*state + v_heads*state] rows
     * (q | k | v channels), ssm_gate (z) [v_heads*state], ssm_out [n_embd] */
    lrso_tensor ssm_qkv, ssm_gate, ssm_out;
    lrso_tensor ssm_alpha, ssm_beta; /* F32 [v_heads][n_embd] */
    lrso_tensor ssm_a, ssm_dt;       /* F32 [v_heads] (ssm_a < 0) */
    lrso_tensor ssm_conv;            /* F32 [conv_dim][dn_conv] */
    lrso_tensor ssm_norm;            /* F32 [dn_state] */
} lrso_hybrid_layer;
typedef struct lrso_hybrid lrso_hybrid;
lrso_hybrid *lrso_hybrid_create(const lrso_hybrid_config *cfg, const lrso_tensor *token_embd,
                                const lrso_hybrid_layer *layers,
                                const lrso_tensor *output_norm, const lrso_tensor *output,
                                int kv_f16, int n_threads);
/* tokens at positions len..len+n_tok-1, one at a time (the recurrence is
 * sequential); last token's logits [vocab].  -3 on context overflow. */
int lrso_hybrid_forward(lrso_hybrid *m, const uint32_t *tokens, uint32_t n_tok, float *logits);
uint32_t lrso_hybrid_len(const lrso_hybrid *m);
/* length 0, recurrent states and conv windows cleared */
void lrso_hybrid_reset(lrso_hybrid *m);
void lrso_hybrid_destroy(lrso_hybrid *m);

#ifdef __cplusplus
}
#endif
#endif
