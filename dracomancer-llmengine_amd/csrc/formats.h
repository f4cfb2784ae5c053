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

// Private device layout of one matrix: up to four regions, each 256-byte
// aligned, addressed as base + off[i].  Per format (nb = blocks per row):
//   Q4_K : [0] qs  n_out*nb*128   [1] head n_out*nb*16 (d, dmin, scales[12])
//   Q6_K : [0] ql  n_out*nb*128   [1] qh   n_out*nb*64   [2] sc n_out*nb*16
//          [3] d   n_out*nb*2  (f16)
//   Q8_0 : [0] qs  n_out*nb*32    [1] d    n_out*nb*2  (f16)
//   F16/F32 : [0] the GGUF rows unchanged
struct DracoLayout {
    int code, n_out, n_in, nb;
    size_t off[4];
    size_t bytes;
};

static inline size_t draco_align256(size_t v) { return (v + 255) & ~(size_t)255; }

static inline int draco_layout(int code, int n_out, int n_in, DracoLayout* L) {
    const int bv = draco_block_values(code);
    if (bv == 0 || n_in <= 0 || n_out <= 0 || n_in % bv) return -1;
    L->code = code;
    L->n_out = n_out;
    L->n_in = n_in;
    L->nb = n_in / bv;
    const size_t nbl = (size_t)n_out * L->nb;
    size_t o = 0;
    for (int i = 0; i < 4; i++) L->off[i] = 0;
    switch (code) {
    case DRACO_Q4_K:
        L->off[0] = o; o = draco_align256(o + nbl * 128);
        L->off[1] = o; o = draco_align256(o + nbl * 16);
        break;
    case DRACO_Q6_K:
        L->off[0] = o; o = draco_align256(o + nbl * 128);
        L->off[1] = o; o = draco_align256(o + nbl * 64);
        L->off[2] = o; o = draco_align256(o + nbl * 16);
        L->off[3] = o; o = draco_align256(o + nbl * 2);
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
