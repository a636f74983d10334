/*
 * lrs.h — C ABI of the MI355X (gfx950) batch-1 decode hot path of llama.rs.
 *
 * This is the drop-in boundary: a thin Rust `extern "C"` crate implements the
 * reference's `llama_model::GpuMatmul` and `llama_model::GpuResidentDecode`
 * traits on top of these calls, one trait method per call.  All arguments are plain
 * pointers and sizes; no HIP or torch type crosses the boundary.
 *
 * Conventions (mirroring the reference's error and ownership rules):
 *  - Every call returns LRS_OK (0) or a negative LRS_E_* code; the message is
 *    in lrs_last_error() (thread-local), which the Rust shim maps to
 *    ModelError::Gpu(String) (crates/llama-model/src/error.rs:26-27).
 *  - Weight bytes are borrowed only for the duration of the upload call and
 *    copied to device memory; the caller may drop them afterwards
 *    (crates/llama-vulkan/src/resident_forward.rs:1298-1299).
 *  - Calls are synchronous unless named *_dev (those enqueue on the context's
 *    stream and return at once) and are not re-entrant per context/model
 *    (the reference backend is !Sync, resident_forward.rs:797, 835-854).
 *  - GGUF type ids are those of crates/gguf/src/types.rs:84-107:
 *    F32=0 F16=1 Q8_0=8 Q4_K=12 Q5_K=13 Q6_K=14.
 */
#ifndef LRS_H
#define LRS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LRS_OK 0
#define LRS_E_ARG (-1)          /* bad argument / shape (gpu.rs:149-164 checks) */
#define LRS_E_HIP (-2)          /* HIP runtime error; also a model call whose launch's bounded
                                   wait between its workgroups ran out (outputs not valid) */
#define LRS_E_OOM (-3)          /* device allocation failed */
#define LRS_E_CTX_OVERFLOW (-4) /* KV cache full (attention.rs:36-40) */
#define LRS_E_UNSUPPORTED (-5)  /* type / shape not supported */

#define LRS_TYPE_F32 0u
#define LRS_TYPE_F16 1u
#define LRS_TYPE_Q8_0 8u
#define LRS_TYPE_Q4_K 12u
#define LRS_TYPE_Q5_K 13u
#define LRS_TYPE_Q6_K 14u

typedef struct lrs_ctx lrs_ctx;
typedef struct lrs_weight lrs_weight;
typedef struct lrs_model lrs_model;

/* Message of the last failed call on this thread ("" if none).
 * Replaces the String inside ModelError::Gpu (error.rs:26-27). */
const char *lrs_last_error(void);

/* Library version string, e.g. "lrs 0.1 gfx950". */
const char *lrs_version(void);

/* ------------------------------------------------------------------------ */
/* context                                                                  */
/* ------------------------------------------------------------------------ */
/* Opens a device and a stream.  device >= 0 opens that device only.
 * device = -1 picks the device with the most free HBM, like pick_device
 * (resident_forward.rs:1119-1133); to compare them it makes every visible
 * device current once, so callers that must not touch other GPUs pass an
 * index.  Replaces VulkanContext::new + VulkanDevice::create (device.rs). */
int lrs_ctx_create(int device, lrs_ctx **out);
void lrs_ctx_destroy(lrs_ctx *ctx);
/* Blocks until all work enqueued on the context's stream has finished. */
int lrs_ctx_sync(lrs_ctx *ctx);
/* Free / total HBM of the context's device, bytes. */
int lrs_ctx_mem_info(lrs_ctx *ctx, size_t *free_bytes, size_t *total_bytes);

/* ------------------------------------------------------------------------ */
/* weights (QTensor / GpuRawWeights, crates/llama-model/src/gpu.rs:13-17,    */
/* 128-248; upload = Uploader::tensor, llama-vulkan/src/tensor.rs:555-598)   */
/* ------------------------------------------------------------------------ */
/* Copies an n_out x n_in GGUF tensor (row-major blocks, len bytes) to HBM,
 * repacking it to the device layout.  Types: Q8_0, Q4_K, Q5_K, Q6_K, F32, F16.
 * Fails with LRS_E_ARG when n_in is not a multiple of the block size or len
 * != n_out * n_in / block * type_size (gpu.rs:149-164). */
int lrs_weight_upload(lrs_ctx *ctx, uint32_t ggml_type, const void *bytes, size_t len,
                      uint32_t n_in, uint32_t n_out, lrs_weight **out);
/* Fills an n_out x n_in tensor on the device with the library's seeded
 * synthetic blocks (counter-based hash of (seed, block, byte); mode 0 = the
 * benchmark distributions, 1 = zero-mean K-quants; f16 scales uniform in
 * [d_lo, d_hi)).  Used for random-init models too large to build on the host.
 * No reference counterpart: the reference loads weights from GGUF files. */
int lrs_weight_generate(lrs_ctx *ctx, uint32_t ggml_type, uint64_t seed, int mode,
                        float d_lo, float d_hi, uint32_t n_in, uint32_t n_out,
                        lrs_weight **out);
/* Copies a weight back to the host in GGUF byte layout (len must equal the
 * GGUF size).  For round-trip checks. */
int lrs_weight_download(lrs_ctx *ctx, const lrs_weight *w, void *dst, size_t len);
/* GGUF bytes of the tensor (the algorithmic bytes one matvec reads). */
size_t lrs_weight_gguf_bytes(const lrs_weight *w);
void lrs_weight_free(lrs_weight *w);

/* ------------------------------------------------------------------------ */
/* kernel level                                                             */
/* ------------------------------------------------------------------------ */
/* ggml_cpu::dequant_to_f32 on the GPU (crates/ggml-cpu/src/dequant.rs:10-21),
 * bit-exact: host GGUF bytes in, host f32 out (len/type_size*block floats). */
int lrs_dequant_f32(lrs_ctx *ctx, uint32_t ggml_type, const void *bytes, size_t len,
                    float *out);
/* Dequantizes a resident weight to a device f32 buffer [n_out*n_in]. */
int lrs_weight_dequant_dev(lrs_ctx *ctx, const lrs_weight *w, float *out_dev);

/* y = W x for `cols` columns: x [cols*n_in] host f32, y [cols*n_out] host f32.
 * GpuMatmul::matvec_q8_0 (crates/llama-model/src/gpu.rs:1057-1065) generalised
 * to every resident type, and matmul::dispatch_{q8_0,q4_k,q5_k,q6_k}_matvec
 * (crates/llama-vulkan/src/matmul.rs:36-430).  The activation keeps 22
 * significant bits per 32-element block (three exact int8 digits on the
 * matrix cores; the reference rounds it to 8 bits).  Up to 8 columns (Q8_0)
 * or 4 (K-quants) share each weight load, as the reference's COLS
 * specialisation (shaders/q5_k_matvec.comp:43-47, q8_0_matvec.comp:8-10)
 * does; each column's result is bit-identical to a one-column call.
 * Blocking. */
int lrs_matvec_f32(lrs_ctx *ctx, const lrs_weight *w, const float *x, float *y,
                   uint32_t cols);
/* Same on device buffers, enqueued on the context stream (async).  Q8_0
 * weights, several columns and inputs of up to 4096 elements are packed by
 * the matvec launch itself (no scratch); wider single K-quant columns take a
 * pack launch into the context scratch first. */
int lrs_matvec_dev(lrs_ctx *ctx, const lrs_weight *w, const float *x_dev, float *y_dev,
                   uint32_t cols);

/* lrs_matvec_dev that allocates nothing: no counterpart in the reference; for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The input pack
 * lives in a static device array of the library (160 KiB, one copy per GPU,
 * held until the process ends) instead of the context scratch, so n_in is
 * limited to LRS_NOALLOC_MAX_N_IN (LRS_E_ARG beyond).  Every call on one GPU
 * shares that array: calls on the same stream are ordered, calls that
 * overlap on one GPU (other streams or contexts) race.  Async on the context
 * stream; results equal lrs_matvec_dev's. */
#define LRS_NOALLOC_MAX_N_IN 46592u
int lrs_matvec_dev_noalloc(lrs_ctx *ctx, const lrs_weight *w, const float *x_dev, float *y_dev,
                           uint32_t cols);

/* The int8-activation path the reference's CPU Model::forward takes for Q8_0
 * weights (crates/llama-model/src/ops.rs), on device buffers, enqueued on
 * the context stream (async).
 * lrs_quantize_q8_0_dev: x [n] f32 -> n/32 GGUF Q8_0 blocks (34 bytes each,
 * f16 d then 32 int8) at q8_dev, bit-exact with quantize_q8_0 (ops.rs:343-368,
 * round half away from zero: half_even = 0) or quantize_q8_0_avx2
 * (ops.rs:284-340, round half to even: half_even = 1); n a multiple of 32.
 * lrs_matvec_q8_0_actq_dev: y = W x for `cols` columns with each column
 * rounded as above first, matmul_q8_0_actq (ops.rs:728-886) with the block
 * dot of q8_0_q8_0_dot_scalar (ops.rs:704-724): exact int32 block sums
 * times dw * dx, summed in f32 (order differs: within 1e-4 relative L2).
 * Q8_0 weights only (LRS_E_UNSUPPORTED otherwise). */
int lrs_quantize_q8_0_dev(lrs_ctx *ctx, const float *x_dev, uint32_t n, int half_even,
                          uint8_t *q8_dev);
int lrs_matvec_q8_0_actq_dev(lrs_ctx *ctx, const lrs_weight *w, const float *x_dev,
                             float *y_dev, uint32_t cols, int half_even);

/* Batched prefill GEMM on the matrix cores: y [m * n_out] = a [m * n_in] W^T,
 * device f32 buffers, enqueued on the context stream (async).  Replaces the
 * prefill matmul matmul::dispatch_mul_mm_q4k / shaders/mul_mm.comp
 * (crates/llama-vulkan/src/matmul.rs:433-465), which quantizes a to int8:
 * here a and dequant(W) go to v_mfma_f32_32x32x16_bf16 as bf16 with f32
 * accumulation.  precision 1: each operand rounded to bf16 once;
 * precision 3: each split into bf16 hi + lo and three products summed
 * (~2^-16 relative, for prefill that must match the f32 forward).
 * Weights: Q4_K, Q5_K, Q6_K, Q8_0; n_in a multiple of 256. */
int lrs_gemm_dev(lrs_ctx *ctx, const lrs_weight *w, const float *a_dev, float *y_dev, uint32_t m,
                 int precision);
/* lrs_gemm_dev for n_w (1..3) weights over the same a, as one launch over
 * all their output tiles: y_dev[i] [m * n_out(w[i])] = a W[i]^T.  No
 * reference counterpart (the reference dispatches one GEMM per weight); it
 * is the form a prompt block uses for q / k / v.  The weights share n_in;
 * at most two types, the first type's weights first, and the mixes Q4_K or
 * Q5_K followed by Q6_K (else LRS_E_UNSUPPORTED).  Each output equals the
 * single-weight GEMM without a split over K. */
int lrs_gemm_group_dev(lrs_ctx *ctx, const lrs_weight *const *w, uint32_t n_w, const float *a_dev,
                       float *const *y_dev, uint32_t m, int precision);

/* Matvec launch shape override: tiles of 16 rows per wavefront, tile groups
 * per workgroup, K-slices per workgroup; one of the instantiated shapes
 * (1,1,4) (1,2,4) (1,2,2) (2,4,2) (2,2,4) (1,2,6), or all 0 = automatic.
 * Replaces the LLAMA_RS_MATVEC_GEOM knob (resident_forward.rs:164-176). */
int lrs_matvec_set_geom(int tiles_per_wave, int tile_groups, int k_slices);

/* device memory + timing helpers for callers that keep buffers resident */
int lrs_dev_alloc(lrs_ctx *ctx, size_t bytes, void **dptr);
int lrs_dev_free(lrs_ctx *ctx, void *dptr);
int lrs_copy_h2d(lrs_ctx *ctx, void *dst_dev, const void *src, size_t bytes);
int lrs_copy_d2h(lrs_ctx *ctx, void *dst, const void *src_dev, size_t bytes);
/* Graph capture of the asynchronous entry points (lrs_matvec_dev,
 * lrs_gemm_dev, copies): between lrs_capture_begin and lrs_capture_end the
 * calls on the context stream are recorded into a HIP graph instead of run;
 * lrs_graph_launch replays it on the context stream (async).  The
 * resolve-once pattern of the reference's recorded command buffers
 * (resident_forward.rs build_plan, :3678-3762) for kernel-level callers.
 * Blocking calls, and a first call whose context scratch must grow, fail
 * inside a capture: make one uncaptured call of the same shape first.
 * A graph records the address of the context's scratch buffer, so while any
 * graph of the context is alive a call that would grow the scratch fails with
 * LRS_E_ARG and leaves the buffer in place (make the largest call before
 * capturing, or destroy the graphs first).  Graphs must be destroyed before
 * their context. */
typedef struct lrs_graph lrs_graph;
int lrs_capture_begin(lrs_ctx *ctx);
int lrs_capture_end(lrs_ctx *ctx, lrs_graph **out);
int lrs_graph_launch(lrs_graph *g);
void lrs_graph_destroy(lrs_graph *g);

/* HIP events on the context stream: start, then stop returns elapsed ms. */
int lrs_timer_start(lrs_ctx *ctx);
int lrs_timer_stop(lrs_ctx *ctx, float *ms);

/* ------------------------------------------------------------------------ */
/* model level: llama_model::GpuResidentDecode                              */
/* (crates/llama-model/src/gpu.rs:379-455) as implemented by                 */
/* llama_vulkan::ResidentForward (resident_forward.rs:5223-5282)             */
/* ------------------------------------------------------------------------ */
/* The LlamaConfig fields the dense forward uses (config.rs:51-187). */
typedef struct {
    uint32_t n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, vocab;
    uint32_t rope_dim; /* RoPE on the first rope_dim dims of a head (adjacent pairs) */
    uint32_t ctx;      /* KV-cache positions (--ctx, args.rs:38-42) */
    float rms_eps, freq_base;
} lrs_config;

/* One decoder layer (LayerWeights, weights.rs; GpuRawWeights, gpu.rs:128-248).
 * Weights are resident handles from lrs_weight_upload/generate on the same
 * context and must outlive the model; norm/bias vectors are host f32 and are
 * copied.  Biases (Qwen2 q/k/v) may be NULL. */
typedef struct {
    const lrs_weight *attn_q, *attn_k, *attn_v, *attn_output;
    const lrs_weight *ffn_gate, *ffn_up, *ffn_down;
    const float *attn_norm, *ffn_norm; /* [n_embd] */
    const float *bq, *bk, *bv;         /* [n_head*head_dim], [n_head_kv*head_dim] x2 */
} lrs_layer_weights;

/* ResidentForward::new (resident_forward.rs:1302-1311): builds the f16 KV
 * cache and captures the per-token forward as HIP graphs.  token_embd may be
 * any dequantizable type (the row of each token is dequantized on the GPU,
 * TokenEmbd::linha gpu.rs:297-304); matvec weights Q8_0/Q4_K/Q5_K/Q6_K.
 * With the environment variable LRS_GRAPH=0 no graph is captured and every
 * token issues the same kernel launches directly; the same holds when
 * ROCPROF_KERNEL_TRACE or ROCPROF_COUNTER_COLLECTION is set (rocprofv3 sets
 * them for the program it traces). */
int lrs_model_create(lrs_ctx *ctx, const lrs_config *cfg, const lrs_layer_weights *layers,
                     const lrs_weight *token_embd, const float *output_norm,
                     const lrs_weight *output, lrs_model **out);

/* Hybrid attention + gated delta-net model (qwen35; LlamaConfig::delta_net,
 * config.rs:10-46, 126-141): layer l is gated full attention when
 * (l + 1) % full_attn_interval == 0 and a gated delta net otherwise
 * (LlamaConfig::eh_linear).  Replaces ResidentForward::new for this
 * architecture (resident_forward.rs:1302-1311; plan of the layer loop
 * :3826-4103 and plano_delta :2252-2470).  The full-attention layers use
 * base.n_head / n_head_kv / head_dim and RoPE of the first base.rope_dim dims
 * with freq[i] = 1 / freq_base^(2i/rope_dim) (gpu.rs:540-547).  Delta-net
 * layers: dn_v_heads value heads of dn_state x dn_state f32 state reading key
 * head h % dn_k_heads; conv over the last dn_conv inputs.  dn_state 64 or 128
 * (the key and value head width, ssm.state_size). */
typedef struct {
    lrs_config base;
    uint32_t full_attn_interval;
    uint32_t dn_k_heads, dn_v_heads, dn_state, dn_conv;
} lrs_hybrid_config;

/* One hybrid layer.  Every layer: FFN weights, attn_norm (input norm) and
 * post_norm (post_attention_norm, before the FFN).  Full-attention layers:
 * attn_q has 2*n_head*head_dim rows (per head the query, then its output
 * gate), q_norm / k_norm [head_dim] (per-head RMSNorm before RoPE).  Delta-net
 * layers: ssm_qkv [conv_dim = (2*k_heads + v_heads)*dn_state rows: q | k | v
 * channels], ssm_gate (z) [v_heads*dn_state], ssm_out [n_embd x v_heads*dn_state];
 * host f32: ssm_alpha / ssm_beta [v_heads][n_embd], ssm_a (negative) and
 * ssm_dt [v_heads], ssm_conv [conv_dim][dn_conv], ssm_norm [dn_state].
 * Unused members of the other layer kind may be NULL. */
typedef struct {
    const lrs_weight *ffn_gate, *ffn_up, *ffn_down;
    const float *attn_norm, *post_norm;
    const lrs_weight *attn_q, *attn_k, *attn_v, *attn_output;
    const float *q_norm, *k_norm;
    const lrs_weight *ssm_qkv, *ssm_gate, *ssm_out;
    const float *ssm_alpha, *ssm_beta, *ssm_a, *ssm_dt, *ssm_conv, *ssm_norm;
} lrs_hybrid_layer;

/* Builds a hybrid model: the same decode / decode_batch / greedy / reset
 * entry points apply.  Its recurrent state cannot be rewound: every decode
 * must continue at the current length (pos == lrs_model_len) and
 * lrs_reset clears the states and conv windows.  batch_size() is 512 when
 * every matmul weight is Q4_K, Q5_K, Q6_K or Q8_0 (prompt blocks: GEMM projections and
 * block delta-net kernels), else 1. */
int lrs_hybrid_create(lrs_ctx *ctx, const lrs_hybrid_config *cfg, const lrs_hybrid_layer *layers,
                      const lrs_weight *token_embd, const float *output_norm,
                      const lrs_weight *output, lrs_model **out);
void lrs_model_destroy(lrs_model *m);
/* GpuResidentDecode::decode: token at position pos (KV written at slot pos,
 * attends 0..pos), logits [vocab] into caller memory; the cache length
 * becomes pos+1.  LRS_E_CTX_OVERFLOW when pos >= ctx. */
int lrs_decode(lrs_model *m, uint32_t token, uint32_t pos, float *logits);
/* GpuResidentDecode::decode_batch: tokens at pos0..pos0+n-1, logits of the
 * last one (gpu.rs:392-400). */
int lrs_decode_batch(lrs_model *m, const uint32_t *tokens, uint32_t n, uint32_t pos0,
                     float *logits);
/* GpuResidentDecode::batch_size (tokens per decode_batch block). */
uint32_t lrs_batch_size(const lrs_model *m);
/* Numerics of Q8_0 weights in a dense model.  Off (the default): every
 * weight, Q8_0 included, multiplies the f32 activation (kept to 22 bits per
 * 32-element block), i.e. dequant + f32 matmul, within 1e-3 of that forward.
 * On: a Q8_0 weight multiplies its input rounded like the reference CPU
 * forward does (RawTensor::matmul_into, crates/llama-model/src/weights.rs:
 * 109-124: quantize_q8_0_split with the AVX2 quantizer, ops.rs:284-340, then
 * exact int8 block dots, matmul_q8_0_actq ops.rs:728-886).  That rounding is
 * discontinuous: logits follow the reference to ~1e-7 until an activation
 * lands on the other side of a rounding boundary because of f32 summation
 * order, after which they can differ by ~1e-2.  Re-captures the token graphs. */
int lrs_model_set_q8_rounding(lrs_model *m, int on);
/* GpuResidentDecode::reset: cache length back to 0. */
void lrs_reset(lrs_model *m);
/* Current cache length (ResidentState::len). */
uint32_t lrs_model_len(const lrs_model *m);
/* decode + greedy sampling on the device (Sampler::sample with temperature 0,
 * llama-sampling/src/sampler.rs:25-27, = ops::argmax ops.rs:1035-1045):
 * writes the next token id instead of the logits. */
int lrs_decode_greedy(lrs_model *m, uint32_t token, uint32_t pos, uint32_t *next);
/* The greedy loop of gerar_streaming_residente (gpu.rs:609-666) without a
 * tokenizer: prompt at positions pos0.., then n_gen greedy tokens generated
 * on the device with no host round trip per token (out_tokens[n_gen]). */
int lrs_generate_greedy(lrs_model *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t pos0,
                        uint32_t n_gen, uint32_t *out_tokens);
/* Per-op timing of the decode plan (the LLAMA_RS_PROFILE timestamps of
 * resident_forward.rs:3141-3149, 4556-4745): launches `op` for layers
 * 0,1,2,.. in turn `iters` times on the model stream, outside the graph, and
 * returns the mean duration per launch (HIP events) and the algorithmic bytes
 * of one launch: GGUF weight bytes, f16 K/V read or appended and the f32
 * vectors read or written once.  Attention reads the current cache length. */
#define LRS_OP_QKV 0u
#define LRS_OP_ATTN 1u
#define LRS_OP_O 2u
#define LRS_OP_GATEUP 3u
#define LRS_OP_DOWN 4u
#define LRS_OP_HEAD 5u
/* hybrid models: delta-net projections (qkv + z), the delta-net step, its
 * output projection, and the QK-norm + RoPE of the attention layers;
 * LRS_OP_QKV / ATTN / O then time the attention layers' ops.  The
 * attention split kernel does the QK-norm + RoPE by default (then
 * LRS_OP_QK_PREP reports 0 us and 0 bytes and LRS_OP_ATTN includes it);
 * LRS_QKP=0 at model creation gives it a launch of its own.  Likewise the
 * o launch runs the attention split and combine by default: LRS_OP_ATTN
 * then reports 0 us and 0 bytes and LRS_OP_O includes both (LRS_SAO=0 at
 * model creation keeps the split launch). */
#define LRS_OP_DN_PROJ 6u
#define LRS_OP_DN_STEP 7u
#define LRS_OP_DN_OUT 8u
#define LRS_OP_QK_PREP 9u
/* the whole FFN of a layer: gate/up + SwiGLU, then down + residual */
#define LRS_OP_FFN 10u
/* dense models: every matvec of a layer as the token plan launches them
 * (q/k/v, o, gate/up, down with their fused norms and epilogues), without
 * the attention between q/k/v and o */
#define LRS_OP_MATVECS 11u
int lrs_model_profile(lrs_model *m, uint32_t op, uint32_t iters, float *avg_us, size_t *bytes);
/* GGUF bytes of every weight matrix one decoded token streams. */
size_t lrs_model_bytes_per_token(const lrs_model *m);

/* ------------------------------------------------------------------------ */
/* GGUF files: gguf::GgufFile (crates/gguf/src/file.rs, parse.rs)            */
/* ------------------------------------------------------------------------ */
/* Maps and parses a GGUF v3 file: metadata, tensor infos, data section at
 * general.alignment (default 32) (GgufFile::parse, parse.rs:64-126). */
typedef struct lrs_gguf lrs_gguf;
int lrs_gguf_open(const char *path, lrs_gguf **out);
void lrs_gguf_close(lrs_gguf *g);
uint32_t lrs_gguf_version(const lrs_gguf *g);
uint64_t lrs_gguf_n_tensors(const lrs_gguf *g);
/* typed metadata reads (MetadataValue::as_u32 / as_f32, types.rs) */
int lrs_gguf_get_u32(const lrs_gguf *g, const char *key, uint32_t *v);
int lrs_gguf_get_f32(const lrs_gguf *g, const char *key, float *v);
int lrs_gguf_get_str(const lrs_gguf *g, const char *key, const char **s);
int lrs_gguf_array_len(const lrs_gguf *g, const char *key, uint64_t *n);
/* GgufFile::tensor_data (file.rs:47-75): type, dims (up to 4; dims[0] is
 * the row length), and the bytes inside the mapping, bounds-checked */
int lrs_gguf_tensor(const lrs_gguf *g, const char *name, uint32_t *ggml_type, uint64_t *dims,
                    uint32_t *n_dims, const void **data, size_t *len);
/* LlamaConfig::from_gguf (config.rs:81-187) + GpuRawWeights::from_gguf /
 * GpuAuxWeights::from_gguf (gpu.rs:128-600) + ResidentForward::new: uploads
 * every weight of the file and builds the dense (llama / qwen2) or hybrid
 * (qwen35: *.ssm.conv_kernel present) model, which owns those weights.
 * ctx_len 0 keeps the file's context_length.  The file may be closed
 * afterwards. */
int lrs_model_load_gguf(lrs_ctx *ctx, const lrs_gguf *g, uint32_t ctx_len, lrs_model **out);

#ifdef __cplusplus
}
#endif
#endif
