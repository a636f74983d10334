// Tiled device layout of the matvec weights (Q4_K, Q5_K, Q6_K, Q8_0).
//
// The GGUF tensor is row-major: row r is n_in/block consecutive blocks
// (crates/llama-model/src/gpu.rs:158).  On the device the rows are grouped in
// tiles of 16 and the K dimension in "units" (a K-quant super-block of 256
// elements, or two Q8_0 blocks = 64 elements).  The bytes of one unit of the 16
// rows of a tile form one contiguous chunk, cut into 16-byte pieces ordered so
// that lane n + 16 g of a wavefront (row n of the tile, lane group g) reads
// piece (g, n): one load instruction of a wavefront reads 1 KB contiguous.
// Only GGUF bytes are stored (plus zero rows / zero Q8_0 blocks that pad the
// shape to whole tiles and units), so a matvec streams exactly the GGUF bytes.
//
//   Q4_K  chunk 2304 B = [hdr n: d,dmin,scales (16 B) x16]
//                        [qs bytes 16g..16g+15 of half 0 (g,n)] [same, half 1]
//   Q5_K  chunk 2816 B = [hdr x16] [qh bytes 16h..16h+15 (h,n), h=0,1]
//                        [qs half 0 (g,n)] [qs half 1 (g,n)]
//   Q6_K  chunk 3360 B = [scales (16 B) x16] [ql A (g,n)] [ql B (g,n)] [qh (g,n)]
//                        [d (2 B) x16]; lane group g = (half g>>1, is g&1):
//                        ql A = ql[64 half + 16 is ..+16), ql B = ql[64 half +
//                        32 + 16 is ..+16), qh = qh[32 half + 16 is ..+16)
//   Q8_0  chunk 1088 B = [qs (g,n): block 2u + (g>>1), bytes 16(g&1)..+16]
//                        [d (2 B) of (n, block 2u + b) at 1024 + 4n + 2b]
#pragma once

#include <cstddef>
#include <cstdint>

namespace lrs {

constexpr uint32_t TILE_ROWS = 16;

__host__ __device__ inline bool is_tiled(uint32_t t) { return t == 8 || t == 12 || t == 13 || t == 14; }

// bytes of one unit chunk (16 rows)
__host__ __device__ constexpr uint32_t tchunk_bytes(uint32_t t) {
    switch (t) {
    case 12: return 2304;
    case 13: return 2816;
    case 14: return 3360;
    case 8: return 1088;
    default: return 0;
    }
}
// elements of one unit
__host__ __device__ constexpr uint32_t tunit_elems(uint32_t t) { return t == 8 ? 64u : 256u; }

// units per row (Q8_0: blocks rounded up to pairs)
__host__ __device__ inline uint32_t tunits(uint32_t t, uint32_t n_in) {
    const uint32_t ue = tunit_elems(t);
    return (n_in + ue - 1) / ue;
}
__host__ __device__ inline uint32_t ttiles(uint32_t n_out) { return (n_out + TILE_ROWS - 1) / TILE_ROWS; }
__host__ __device__ inline size_t tbytes(uint32_t t, uint32_t n_in, uint32_t n_out) {
    return (size_t)ttiles(n_out) * tunits(t, n_in) * tchunk_bytes(t);
}

// device byte offset (from the tensor start) of GGUF byte `o` of GGUF block
// `blk` of row `row`
__host__ __device__ inline size_t toff(uint32_t t, uint32_t n_in, uint32_t row, uint32_t blk, uint32_t o) {
    const uint32_t units = tunits(t, n_in), n = row % TILE_ROWS;
    const size_t tile0 = (size_t)(row / TILE_ROWS) * units * tchunk_bytes(t);
    uint32_t u, off;
    switch (t) {
    case 12: {  // Q4_K
        u = blk;
        if (o < 16) {
            off = 16 * n + o;
        } else {
            const uint32_t j = o - 16, p = j >> 6, g = (j & 63) >> 4;
            off = 256 + 1024 * p + 16 * (16 * g + n) + (j & 15);
        }
        break;
    }
    case 13: {  // Q5_K
        u = blk;
        if (o < 16) {
            off = 16 * n + o;
        } else if (o < 48) {
            const uint32_t j = o - 16;
            off = 256 + 16 * (16 * (j >> 4) + n) + (j & 15);
        } else {
            const uint32_t j = o - 48, p = j >> 6, g = (j & 63) >> 4;
            off = 768 + 1024 * p + 16 * (16 * g + n) + (j & 15);
        }
        break;
    }
    case 14: {  // Q6_K: ql[128] qh[64] scales[16] d[2]
        u = blk;
        if (o < 128) {
            const uint32_t half = o >> 6, r = o & 63, part = r >> 5, is = (r & 31) >> 4;
            const uint32_t g = 2 * half + is;
            off = 256 + 1024 * part + 16 * (16 * g + n) + (r & 15);
        } else if (o < 192) {
            const uint32_t j = o - 128, half = j >> 5, r = j & 31, is = r >> 4;
            const uint32_t g = 2 * half + is;
            off = 2304 + 16 * (16 * g + n) + (r & 15);
        } else if (o < 208) {
            off = 16 * n + (o - 192);
        } else {
            off = 3328 + 2 * n + (o - 208);
        }
        break;
    }
    default: {  // Q8_0: d[2] qs[32]
        u = blk >> 1;
        const uint32_t b = blk & 1;
        if (o < 2) {
            off = 1024 + 4 * n + 2 * b + o;
        } else {
            const uint32_t j = o - 2, g = 2 * b + (j >> 4);
            off = 16 * (16 * g + n) + (j & 15);
        }
        break;
    }
    }
    return tile0 + (size_t)u * tchunk_bytes(t) + off;
}

// inverse of toff: the GGUF (row, block, byte) held by device byte `off`;
// false for padding bytes (rows past n_out, the odd Q8_0 block past n_in)
__host__ __device__ inline bool tinv(uint32_t t, uint32_t n_in, uint32_t n_out, size_t off,
                                     uint32_t &row, uint32_t &blk, uint32_t &o) {
    const uint32_t cb = tchunk_bytes(t);
    const size_t tstride = (size_t)tunits(t, n_in) * cb;
    const uint32_t tile = (uint32_t)(off / tstride);
    const size_t rem = off - (size_t)tile * tstride;
    const uint32_t u = (uint32_t)(rem / cb), x = (uint32_t)(rem - (size_t)u * cb);
    uint32_t n = 0, b = 0;
    switch (t) {
    case 12:  // Q4_K
        if (x < 256) {
            n = x >> 4;
            o = x & 15;
        } else {
            const uint32_t j = x - 256, p = j >> 10, r = j & 1023, pc = r >> 4;
            n = pc & 15;
            o = 16 + 64 * p + 16 * (pc >> 4) + (r & 15);
        }
        break;
    case 13:  // Q5_K
        if (x < 256) {
            n = x >> 4;
            o = x & 15;
        } else if (x < 768) {
            const uint32_t j = x - 256, pc = j >> 4;
            n = pc & 15;
            o = 16 + 16 * (pc >> 4) + (j & 15);
        } else {
            const uint32_t j = x - 768, p = j >> 10, r = j & 1023, pc = r >> 4;
            n = pc & 15;
            o = 48 + 64 * p + 16 * (pc >> 4) + (r & 15);
        }
        break;
    case 14:  // Q6_K
        if (x < 256) {
            n = x >> 4;
            o = 192 + (x & 15);
        } else if (x < 3328) {
            const uint32_t j = x - 256, part = j >> 10, r = j & 1023, pc = r >> 4;
            const uint32_t g = pc >> 4, half = g >> 1, is = g & 1, bb = r & 15;
            n = pc & 15;
            o = part == 0 ? 64 * half + 16 * is + bb
                : part == 1 ? 64 * half + 32 + 16 * is + bb
                            : 128 + 32 * half + 16 * is + bb;
        } else {
            const uint32_t j = x - 3328;
            n = j >> 1;
            o = 208 + (j & 1);
        }
        break;
    default:  // Q8_0
        if (x < 1024) {
            const uint32_t pc = x >> 4, g = pc >> 4;
            n = pc & 15;
            b = g >> 1;
            o = 2 + 16 * (g & 1) + (x & 15);
        } else {
            const uint32_t j = x - 1024;
            n = j >> 2;
            b = (j >> 1) & 1;
            o = j & 1;
        }
        break;
    }
    row = tile * TILE_ROWS + n;
    blk = t == 8 ? 2 * u + b : u;
    const uint32_t nb = n_in / (t == 8 ? 32u : 256u);
    return row < n_out && blk < nb;
}

}  // namespace lrs
