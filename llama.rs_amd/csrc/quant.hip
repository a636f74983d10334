// quant.hip — device-layout repack, seeded synthetic blocks and bit-exact
// dequant for the GGUF block types on the decode path (gfx950).
//
// Dequant follows ggml_cpu::dequant_to_f32 (crates/ggml-cpu/src/dequant.rs:
// 58-258) element by element with the same f32 operation order; the library
// is compiled with -ffp-contract=off, so d1*q - m1 rounds twice as in Rust.
#include "lrs_internal.h"
#include "quant_dev.h"

namespace lrs {

static unsigned grid_for(uint64_t n, unsigned bs) {
    uint64_t g = (n + bs - 1) / bs;
    if (g > 65536u * 4u) g = 65536u * 4u;
    if (g == 0) g = 1;
    return (unsigned)g;
}

// ---------------------------------------------------------------------------
// GGUF row-major blocks <-> device layout (tiled.h for the matvec types, the
// GGUF bytes as they are for the others).  One thread per device word; every
// padding byte is written as zero.
// ---------------------------------------------------------------------------
__global__ void k_repack_from_gguf(const uint8_t *__restrict__ g, WeightView w, size_t dev_bytes,
                                   uint8_t *__restrict__ q) {
    const uint32_t bb = (uint32_t)block_bytes(w.type);
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < dev_bytes / 4;
         i += (size_t)gridDim.x * blockDim.x) {
        uint32_t v = 0;
        for (int k = 0; k < 4; k++) {
            uint32_t row, blk, o;
            if (tinv(w.type, w.n_in, w.n_out, 4 * i + k, row, blk, o))
                v |= (uint32_t)g[((size_t)row * w.nb + blk) * bb + o] << (8 * k);
        }
        reinterpret_cast<uint32_t *>(q)[i] = v;
    }
}

__global__ void k_repack_to_gguf(WeightView w, size_t dev_bytes, uint8_t *__restrict__ g) {
    const uint32_t bb = (uint32_t)block_bytes(w.type);
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < dev_bytes;
         i += (size_t)gridDim.x * blockDim.x) {
        uint32_t row, blk, o;
        if (tinv(w.type, w.n_in, w.n_out, i, row, blk, o)) g[((size_t)row * w.nb + blk) * bb + o] = w.q[i];
    }
}

hipError_t launch_repack_from_gguf(const uint8_t *gguf_dev, WeightView w, uint8_t *q, hipStream_t s) {
    const size_t db = weight_dev_bytes(w.type, w.n_in, w.n_out);
    if (!is_tiled(w.type)) return hipMemcpyAsync(q, gguf_dev, db, hipMemcpyDeviceToDevice, s);
    hipLaunchKernelGGL(k_repack_from_gguf, dim3(grid_for(db / 4, 256)), dim3(256), 0, s, gguf_dev, w, db, q);
    return hipGetLastError();
}

hipError_t launch_repack_to_gguf(WeightView w, uint8_t *gguf_dev, hipStream_t s) {
    const size_t db = weight_dev_bytes(w.type, w.n_in, w.n_out);
    if (!is_tiled(w.type)) return hipMemcpyAsync(gguf_dev, w.q, db, hipMemcpyDeviceToDevice, s);
    hipLaunchKernelGGL(k_repack_to_gguf, dim3(grid_for(db, 256)), dim3(256), 0, s, w, db, gguf_dev);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// seeded synthetic blocks: the same counter-based hash and field rules as the
// host generator, so any block can be regenerated bit-identically on the CPU
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t hsh(uint64_t seed, uint64_t blk, uint32_t j) {
    return mix64(seed * 0x9E3779B97F4A7C15ULL + blk * 0xD1B54A32D192ED03ULL +
                 (uint64_t)j * 0x8CB92BA72F3D8DD7ULL + 0x2545F4914F6CDD1DULL);
}
__device__ __forceinline__ float h_unif(uint64_t h, float lo, float hi) {
    float u = __fmul_rn((float)(uint32_t)(h >> 40), 1.0f / 16777216.0f);
    float span = __fsub_rn(hi, lo);
    return __fadd_rn(lo, __fmul_rn(span, u));
}
// binary16 round-to-nearest-even narrowing, integer-only
__device__ __forceinline__ uint16_t f2h_rne(float f) {
    uint32_t x = __float_as_uint(f);
    uint32_t sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xFFu, man = x & 0x7FFFFFu;
    if (exp == 0xFF) return (uint16_t)(sign | (man ? (0x7E00u | (man >> 13)) : 0x7C00u));
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u, sh = (uint32_t)(14 - e);
        uint32_t q = m >> sh, rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13), rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}
__device__ __forceinline__ uint8_t hbyte(uint64_t h) { return (uint8_t)(h >> 56); }

__device__ uint16_t gen_d16(uint32_t t, uint64_t seed, uint64_t blk, int mode, float lo, float hi,
                            bool is_min) {
    if (t == T_Q6_K) return f2h_rne(h_unif(hsh(seed, blk, 208), lo, hi));
    if (!is_min) return f2h_rne(h_unif(hsh(seed, blk, 0), lo, hi));
    if (mode == 1) {
        float d = h2f(f2h_rne(h_unif(hsh(seed, blk, 0), lo, hi)));
        return f2h_rne(__fmul_rn(d, t == T_Q4_K ? 7.5f : 15.5f));
    }
    return f2h_rne(h_unif(hsh(seed, blk, 1), lo, hi));
}

// GGUF byte `o` of synthetic block `blk`
__device__ uint8_t gen_byte(uint32_t t, uint64_t seed, uint64_t blk, uint32_t o, int mode,
                            float lo, float hi) {
    switch (t) {
    case T_Q8_0: {
        if (o < 2) {
            uint16_t v = gen_d16(t, seed, blk, mode, lo, hi, false);
            return (uint8_t)(o == 0 ? (v & 0xFF) : (v >> 8));
        }
        uint64_t h = hsh(seed, blk, o - 1);
        int q = (int)(((h >> 32) * 255ULL) >> 32) - 127;
        return (uint8_t)(int8_t)q;
    }
    case T_Q4_K:
    case T_Q5_K: {
        if (o < 4) {
            uint16_t v = gen_d16(t, seed, blk, mode, lo, hi, o >= 2);
            return (uint8_t)((o & 1) ? (v >> 8) : (v & 0xFF));
        }
        if (o < 16 && mode == 1) {
            // packed 6-bit scales with mins equal to scales
            uint32_t k = o - 4;  // 0..11
            auto sc = [&](uint32_t j) { return (uint32_t)(hbyte(hsh(seed, blk, 4 + j)) & 63); };
            if (k < 4) return (uint8_t)((sc(k) & 63) | ((sc(k + 4) >> 4) << 6));
            if (k < 8) return (uint8_t)((sc(k - 4) & 63) | ((sc(k) >> 4) << 6));
            uint32_t j = k - 8;
            return (uint8_t)((sc(j + 4) & 15) | ((sc(j + 4) & 15) << 4));
        }
        return hbyte(hsh(seed, blk, o));
    }
    case T_Q6_K: {
        if (o < 192) return hbyte(hsh(seed, blk, o));
        if (o < 208) return (uint8_t)(int8_t)((int)(hsh(seed, blk, o) >> 57) - 64);
        uint16_t v = gen_d16(t, seed, blk, mode, lo, hi, false);
        return (uint8_t)(o == 208 ? (v & 0xFF) : (v >> 8));
    }
    default:
        return 0;
    }
}

// synthetic weight straight into the device layout: one thread per device
// word, each byte the generator byte of its GGUF (block, offset); the block
// index is the GGUF row-major one (row * nb + block), as on the host
__global__ void k_generate(WeightView w, size_t dev_bytes, uint64_t seed, int mode, float lo, float hi,
                           uint8_t *__restrict__ q) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < dev_bytes / 4;
         i += (size_t)gridDim.x * blockDim.x) {
        uint32_t v = 0;
        for (int k = 0; k < 4; k++) {
            uint32_t row, blk, o;
            if (tinv(w.type, w.n_in, w.n_out, 4 * i + k, row, blk, o))
                v |= (uint32_t)gen_byte(w.type, seed, (uint64_t)row * w.nb + blk, o, mode, lo, hi) << (8 * k);
        }
        reinterpret_cast<uint32_t *>(q)[i] = v;
    }
}

hipError_t launch_generate(WeightView w, uint8_t *q, uint64_t seed, int mode, float d_lo, float d_hi,
                           hipStream_t s) {
    if (!is_tiled(w.type)) return hipErrorInvalidValue;
    const size_t db = weight_dev_bytes(w.type, w.n_in, w.n_out);
    hipLaunchKernelGGL(k_generate, dim3(grid_for(db / 4, 256)), dim3(256), 0, s, w, db, seed, mode,
                       d_lo, d_hi, q);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// dequant (bit-exact with dequant.rs)
// ---------------------------------------------------------------------------
__global__ void k_dequant(WeightView w, float *__restrict__ out) {
    const uint32_t be = (uint32_t)block_elems(w.type);
    const uint64_t n = (uint64_t)w.n_out * w.n_in;
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = deq_elem(w, i / be, (uint32_t)(i % be));
}

// rows_dev[r] selects a row; out is [n_rows * n_in] (embedding lookup,
// ops.rs:11-26 on the dequantized table, done one row at a time)
__global__ void k_dequant_rows(WeightView w, const uint32_t *__restrict__ rows, uint32_t n_rows,
                               float *__restrict__ out) {
    const uint32_t be = (uint32_t)block_elems(w.type);
    const uint64_t n = (uint64_t)n_rows * w.n_in;
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        uint32_t r = (uint32_t)(i / w.n_in), c = (uint32_t)(i % w.n_in);
        uint32_t row = rows[r];
        if (row >= w.n_out) row = w.n_out - 1;  // ids are validated on the host
        uint64_t e = (uint64_t)row * w.n_in + c;
        out[i] = deq_elem(w, e / be, (uint32_t)(e % be));
    }
}

hipError_t launch_dequant(WeightView w, float *out, hipStream_t s) {
    uint64_t n = (uint64_t)w.n_out * w.n_in;
    hipLaunchKernelGGL(k_dequant, dim3(grid_for(n, 256)), dim3(256), 0, s, w, out);
    return hipGetLastError();
}

hipError_t launch_dequant_rows(WeightView w, const uint32_t *rows_dev, uint32_t n_rows, float *out,
                               hipStream_t s) {
    uint64_t n = (uint64_t)n_rows * w.n_in;
    hipLaunchKernelGGL(k_dequant_rows, dim3(grid_for(n, 256)), dim3(256), 0, s, w, rows_dev,
                       n_rows, out);
    return hipGetLastError();
}

}  // namespace lrs
