// formats.h -- GGUF block formats, format codes and the private device layout.
//
// Format codes are the reference's (src/smol_engine.py:46-47):
//   0 Q8_0, 3 Q5_K, 4 Q6_K, 5 Q4_K, 7 F16, 9 F32.
// GGUF stores a weight matrix W[n_out x n_in] row-major with n_in fastest;
// a row is n_in / block_values blocks (src/m6_engine.c:40-54).
//
// The device copy of a matrix is private to this library and is stored
// "structure of arrays" per matrix so every lane load is a 16-byte aligned
// vector load (Q6_K and Q8_0 blocks are 210 and 34 bytes, not multiples of
// 16).  The repack only moves bytes; no value is re-encoded.
#pragma once
#include <stddef.h>
#include <stdint.h>

#if defined(__HIPCC__)
#define DRACO_HD __host__ __device__
#else
#define DRACO_HD
#endif

enum {
    DRACO_Q8_0 = 0,
    DRACO_Q5_K = 3,
    DRACO_Q6_K = 4,
    DRACO_Q4_K = 5,
    DRACO_F16 = 7,
    DRACO_F32 = 9,
};

#define Q8K_BLOCK_BYTES 292  // { float d; int8 qs[256]; int16 bsums[16]; }

DRACO_HD static inline size_t draco_row_bytes(int code, int n_in) {
    switch (code) {
    case DRACO_Q8_0: return (size_t)(n_in / 32) * 34;
    case DRACO_Q5_K: return (size_t)(n_in / 256) * 176;
    case DRACO_Q6_K: return (size_t)(n_in / 256) * 210;
    case DRACO_Q4_K: return (size_t)(n_in / 256) * 144;
    case DRACO_F16: return (size_t)n_in * 2;
    case DRACO_F32: return (size_t)n_in * 4;
    default: return 0;
    }
}

DRACO_HD static inline int draco_block_values(int code) {
    switch (code) {
    case DRACO_Q8_0: return 32;
    case DRACO_Q5_K:
    case DRACO_Q6_K:
    case DRACO_Q4_K: return 256;
    case DRACO_F16:
    case DRACO_F32: return 1;
    default: return 0;
    }
}

// Private device layout of one matrix.
//
// Q4_K, Q5_K and Q6_K use a tile layout built for the int8 MFMA GEMV: rows are
// grouped in tiles of 16, and for every (tile, super-block) "item" the 16
// rows' blocks are stored together, ordered so that lane l = j + 16*g of a
// wave (row j of the tile, lane group g = 0..3) finds each of its operands as
// one aligned vector at 16*l (or 4*l).  Items are stored tile-major:
// item (t, b) at (t*nb + b) * item_bytes.  Rows past n_out in the last tile
// are zero (d = 0, so they contribute nothing and are never stored).
//
//   Q4_K item, 2304 B:
//     [   0,1024) lane l: qs[(g>>1)*32 + (g&1)*16 + e] of row j, e = 0..15
//     [1024,2048) lane l: qs[64 + (g>>1)*32 + (g&1)*16 + e] of row j
//     [2048,2304) row j: the 16-byte header (d, dmin, scales[12])
//     Every qs byte is stored XOR 0x80: the low nibble is unchanged and the
//     high nibble u reads as the signed byte 16*(u-8) after one AND.
//   Q6_K item, 3360 B (g2 = g>>1, c = g&1):
//     [   0,1024) lane l: ql[64*g2 + 16*c + e]
//     [1024,2048) lane l: ql[64*g2 + 32 + 16*c + e]
//     [2048,3072) lane l: qh[32*g2 + 16*c + e]
//     [3072,3328) lane l: sc[8*g2 + c + 2*r], r = 0..3 (4 bytes)
//     [3328,3360) row j: d (f16)
//
//   Q5_K item, 2816 B (the Q4_K item's qs and header, then the high bits):
//     [   0,1024) lane l: qs[(g>>1)*32 + (g&1)*16 + e] of row j (not XORed)
//     [1024,2048) lane l: qs[64 + (g>>1)*32 + (g&1)*16 + e] of row j
//     [2048,2304) row j: the 16-byte header (d, dmin, scales[12])
//     [2304,2816) 16 bytes per (row j, half c): qh[16*c + e], e = 0..15, at
//                 2304 + 16*(j + 16*c); lane l reads the half c = g&1
//     (bit s of qh[k] is the fifth bit of value 32*s + k)
//   Q8_0 : structure of arrays, [0] qs n_out*nb*32, [1] d n_out*nb*2 (f16)
//   F16/F32 : [0] the GGUF rows unchanged
// The repack only moves bytes (and flips the Q4_K bit 7); it is a bijection
// (draco_unpack inverts it).
struct DracoLayout {
    int code, n_out, n_in, nb;
    int ntiles;  // Q4_K / Q6_K: 16-row tiles
    size_t off[4];
    size_t bytes;
};

#define DRACO_Q4T_ITEM 2304
#define DRACO_Q6T_ITEM 3360
#define DRACO_Q5T_ITEM 2816

// Byte offsets inside the tile layouts (row r, super-block b, byte index i of
// the GGUF field).
DRACO_HD static inline size_t draco_item(int nb, int r, int b, int item_bytes) {
    return ((size_t)(r >> 4) * nb + b) * (size_t)item_bytes;
}
DRACO_HD static inline size_t draco_q4t_qs(int nb, int r, int b, int i) {  // i in [0,128)
    const int j2 = i >> 5, k = i & 31, g = ((j2 & 1) << 1) | (k >> 4);
    return draco_item(nb, r, b, DRACO_Q4T_ITEM) + (size_t)(j2 >> 1) * 1024 + 16 * ((r & 15) + 16 * g) + (k & 15);
}
DRACO_HD static inline size_t draco_q4t_hdr(int nb, int r, int b) {
    return draco_item(nb, r, b, DRACO_Q4T_ITEM) + 2048 + 16 * (r & 15);
}
DRACO_HD static inline size_t draco_q5t_qs(int nb, int r, int b, int i) {  // i in [0,128)
    const int j2 = i >> 5, k = i & 31, g = ((j2 & 1) << 1) | (k >> 4);
    return draco_item(nb, r, b, DRACO_Q5T_ITEM) + (size_t)(j2 >> 1) * 1024 + 16 * ((r & 15) + 16 * g) + (k & 15);
}
DRACO_HD static inline size_t draco_q5t_hdr(int nb, int r, int b) {
    return draco_item(nb, r, b, DRACO_Q5T_ITEM) + 2048 + 16 * (r & 15);
}
DRACO_HD static inline size_t draco_q5t_qh(int nb, int r, int b, int i) {  // i in [0,32)
    return draco_item(nb, r, b, DRACO_Q5T_ITEM) + 2304 + 16 * ((r & 15) + 16 * (i >> 4)) + (i & 15);
}
DRACO_HD static inline size_t draco_q6t_ql(int nb, int r, int b, int i) {  // i in [0,128)
    const int g2 = i >> 6, h = (i >> 5) & 1, c = (i >> 4) & 1, g = 2 * g2 + c;
    return draco_item(nb, r, b, DRACO_Q6T_ITEM) + (size_t)h * 1024 + 16 * ((r & 15) + 16 * g) + (i & 15);
}
DRACO_HD static inline size_t draco_q6t_qh(int nb, int r, int b, int i) {  // i in [0,64)
    const int g2 = i >> 5, c = (i >> 4) & 1, g = 2 * g2 + c;
    return draco_item(nb, r, b, DRACO_Q6T_ITEM) + 2048 + 16 * ((r & 15) + 16 * g) + (i & 15);
}
DRACO_HD static inline size_t draco_q6t_sc(int nb, int r, int b, int i) {  // i in [0,16)
    const int g2 = i >> 3, c = i & 1, rr = (i & 7) >> 1, g = 2 * g2 + c;
    return draco_item(nb, r, b, DRACO_Q6T_ITEM) + 3072 + 4 * ((r & 15) + 16 * g) + rr;
}
DRACO_HD static inline size_t draco_q6t_d(int nb, int r, int b) {
    return draco_item(nb, r, b, DRACO_Q6T_ITEM) + 3328 + 2 * (r & 15);
}

static inline size_t draco_align256(size_t v) { return (v + 255) & ~(size_t)255; }

static inline int draco_layout(int code, int n_out, int n_in, DracoLayout* L) {
    const int bv = draco_block_values(code);
    if (bv == 0 || n_in <= 0 || n_out <= 0 || n_in % bv) return -1;
    L->code = code;
    L->n_out = n_out;
    L->n_in = n_in;
    L->nb = n_in / bv;
    L->ntiles = (n_out + 15) / 16;
    const size_t nbl = (size_t)n_out * L->nb;
    size_t o = 0;
    for (int i = 0; i < 4; i++) L->off[i] = 0;
    switch (code) {
    case DRACO_Q4_K:
        o = draco_align256((size_t)L->ntiles * L->nb * DRACO_Q4T_ITEM);
        break;
    case DRACO_Q6_K:
        o = draco_align256((size_t)L->ntiles * L->nb * DRACO_Q6T_ITEM);
        break;
    case DRACO_Q5_K:
        o = draco_align256((size_t)L->ntiles * L->nb * DRACO_Q5T_ITEM);
        break;
    case DRACO_Q8_0:
        L->off[0] = o; o = draco_align256(o + nbl * 32);
        L->off[1] = o; o = draco_align256(o + nbl * 2);
        break;
    case DRACO_F16:
    case DRACO_F32:
        L->off[0] = 0; o = draco_align256(draco_row_bytes(code, n_in) * n_out);
        break;
    default:
        return -1;
    }
    L->bytes = o;
    return 0;
}
