// Arguments of the fused matvec kernel (matvec.hip) shared with its callers.
#pragma once

#include <cstdint>

namespace lrs {

constexpr int MV_MAX_SEG = 3;

enum MvEpilogue : uint32_t {
    EPI_STORE = 0,   // out[row] = v (+ bias)
    EPI_ACCUM = 1,   // out[row] += v (+ bias): residual add (model.rs:228-233, 249-252)
    EPI_SWIGLU = 2,  // dual rows (gate, up): out[j] = silu(gate_j) * up_j (ops.rs:983-988)
    EPI_KV = 3,      // f16 KV-cache append at slot pos (+ bias, + RoPE)
};

// One output segment: a weight (or a gate/up pair when dual) and where its
// rows go.  All segments of a launch share the activation and its length.
struct MvSeg {
    const uint8_t *q0, *q1;    // q-part of the weight for even / odd logical rows
    const uint16_t *d0, *d1;   // f16 scale arrays (Q6_K / Q8_0), else null
    uint32_t rows;             // logical rows
    uint32_t dual;             // 1: logical row r is row r>>1 of (r&1 ? q1 : q0)
    uint32_t block0;           // first workgroup of the segment (set by launch_mv)
    uint32_t rope;             // 1: rotate adjacent row pairs (Q and K)
    uint32_t epi;              // MvEpilogue
    const float *bias;         // [rows] or null
    float *out;                // f32 destination (STORE / ACCUM / SWIGLU)
    _Float16 *kv;              // f16 cache of this layer, [kv_head][ctx][head_dim]
};

struct MvArgs {
    MvSeg seg[MV_MAX_SEG];
    uint32_t n_seg;
    uint32_t n_in, nb;         // activation length, blocks per weight row
    const float *x;            // activation [cols][n_in]
    const float *norm_w;       // RMSNorm weight [n_in] or null (no norm)
    float eps;
    uint32_t cols, y_stride;   // columns (consecutive tokens); output column stride
    const uint32_t *step;      // device [token, pos] or null (pos 0)
    const float *freq;         // RoPE frequency table [rope_dim/2]
    uint32_t head_dim, rope_dim, ctx;
    uint32_t tile;             // K-tile staged in LDS (set by launch_mv)
    uint32_t n_seg0;           // two-type launches: segments of the first type
    unsigned long long *amax;  // [blocks] per-block argmax keys of the output, or null
    uint32_t amax_cap;         // entries of amax
};

struct MvGeom {
    int lpr, r, waves;
};

// the activation is staged in LDS in K-tiles of at most this many elements
constexpr uint32_t MV_TILE = 8192;

}  // namespace lrs
