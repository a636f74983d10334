// Internal declarations shared by the HIP translation units of liblrs.so.
// gfx950 (CDNA4, wave64) only.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/lrs.h"
#include "mv_args.h"

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
// Device layout of a resident weight (n_out rows x nb blocks per row):
//   Q4_K  q = GGUF blocks as-is (144 B, 16-B aligned), d unused
//   Q5_K  q = GGUF blocks as-is (176 B), d unused
//   Q6_K  q = per block [ql 128 | qh 64 | scales 16] = 208 B (16-B aligned),
//         d = f16 super-block scale array [n_out*nb]
//   Q8_0  q = per block qs[32] (32 B), d = f16 scale array [n_out*nb]
//   Q4_0 / F32 / F16: q = the raw GGUF bytes (dequant only, no matvec)
// Every byte read by a matvec is a GGUF byte: no padding is streamed.
// ---------------------------------------------------------------------------
constexpr uint32_t Q6_QBYTES = 208;
constexpr uint32_t Q8_QBYTES = 32;

struct WeightView {
    const uint8_t *q;
    const uint16_t *d;
    uint32_t type, n_in, n_out, nb;  // nb = blocks per row
};

__host__ __device__ inline size_t q_bytes_per_block(uint32_t t) {
    switch (t) {
    case T_Q6_K: return Q6_QBYTES;
    case T_Q8_0: return Q8_QBYTES;
    default: return (size_t)block_bytes(t);
    }
}
__host__ __device__ inline bool has_d_array(uint32_t t) { return t == T_Q6_K || t == T_Q8_0; }

// launch wrappers implemented in the .hip files (all enqueue on `s`)
hipError_t launch_repack_from_gguf(const uint8_t *gguf_dev, WeightView w, uint8_t *q,
                                   uint16_t *d, hipStream_t s);
hipError_t launch_repack_to_gguf(WeightView w, uint8_t *gguf_dev, hipStream_t s);
hipError_t launch_generate(WeightView w, uint8_t *q, uint16_t *d, uint64_t seed, int mode,
                           float d_lo, float d_hi, hipStream_t s);
hipError_t launch_dequant(WeightView w, float *out, hipStream_t s);
hipError_t launch_dequant_rows(WeightView w, const uint32_t *rows_dev, uint32_t n_rows,
                               float *out, hipStream_t s);
int set_matvec_geom(int lpr, int r, int waves);
MvGeom choose_geom(uint32_t t, uint32_t n_in, uint32_t rows, bool pairs);
hipError_t launch_mv(const MvArgs &args, MvGeom gm, uint32_t type, hipStream_t s,
                     uint32_t *blocks_out = nullptr);
// two weight types in one launch (Q4_K q/k + Q6_K v); hipErrorNotSupported otherwise
hipError_t launch_mv2(const MvArgs &args, uint32_t t0, MvGeom g0, uint32_t t1, MvGeom g1,
                      hipStream_t s);
// reduces the per-block argmax keys of a launch with MvArgs::amax into step / out
hipError_t launch_argmax_finish(const unsigned long long *keys, uint32_t n, uint32_t *step,
                                uint32_t *out, uint32_t out_cap, hipStream_t s);
hipError_t launch_matvec(WeightView w, const float *x, float *y, uint32_t cols,
                         const float *bias, hipStream_t s);
// Y[M][ldy] = A[M][K] W^T on the matrix cores (prec 1: bf16, 3: bf16 hi/lo split)
hipError_t launch_gemm(WeightView w, const float *a, float *y, uint32_t M, uint32_t ldy, int prec,
                       hipStream_t s, bool accum = false);
// batched prompt block (prefill.hip)
hipError_t launch_rmsnorm_rows(const float *X, const float *w, float eps, uint32_t E, uint32_t n,
                               float *Y, hipStream_t s);
hipError_t launch_qkv_post(const float *qt, const float *kt, const float *vt, const float *bq,
                           const float *bk, const float *bv, const float *freq, float *q,
                           _Float16 *kc, _Float16 *vc, uint32_t n, uint32_t pos0, uint32_t qd,
                           uint32_t kvd, uint32_t hd, uint32_t rope_dim, uint32_t ctx,
                           hipStream_t s);
hipError_t launch_attn_prefill(const float *q, const _Float16 *kc, const _Float16 *vc, float *out,
                               uint32_t n, uint32_t pos0, uint32_t n_head, uint32_t n_kv,
                               uint32_t hd, uint32_t ctx, hipStream_t s);
hipError_t launch_swiglu_rows(float *G, const float *U, size_t n, hipStream_t s);

}  // namespace lrs

struct lrs_ctx {
    int device;
    hipStream_t stream;
    hipEvent_t ev0, ev1;
};

struct lrs_weight {
    lrs_ctx *ctx;
    lrs::WeightView v;
    uint8_t *q;
    uint16_t *d;
    size_t q_alloc, d_alloc;
};
