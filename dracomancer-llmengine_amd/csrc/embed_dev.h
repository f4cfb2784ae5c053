// embed_dev.h -- one value of an embedding row, decoded on the device.
#pragma once
#include <hip/hip_runtime.h>

#include "dev_common.h"
#include "formats.h"

// Value p of row `tok` of a private-layout matrix; bit-identical to the host
// decoders: (d*sc)*q for Q6_K, d*sc*q - dmin*m for Q4_K, (q*d)*sc - dmin*m
// for Q5_K, q*d for Q8_0.
__device__ __forceinline__ float embed_value(const uint8_t* __restrict__ base, const DracoLayout& L, int tok, int p) {
#pragma clang fp contract(off)  // each product rounded on its own, as the host decoders
    // a row outside the matrix reads row 0 (host entry points reject such ids;
    // this keeps a device-produced index from addressing past the weights)
    if ((unsigned)tok >= (unsigned)L.n_out) tok = 0;
    const int n_in = L.n_in, nb = L.nb;
    const size_t blk = (size_t)tok * nb + p / draco_block_values(L.code);
    float val = 0.f;
    if (L.code == DRACO_Q8_0) {
        const int8_t q = (int8_t)base[L.off[0] + blk * 32 + (p & 31)];
        const float d = h2f(*reinterpret_cast<const uint16_t*>(base + L.off[1] + blk * 2));
        val = (float)q * d;
    } else if (L.code == DRACO_Q6_K) {
        // value i of the block: ql[64*(i>>7) + (i&63)] nibble (i>>6)&1, qh[32*(i>>7) + (i&31)]
        // bits 2*((i>>5)&3), scale i>>4 (src/m5_kern_scalar.c:115-142)
        const int i = p & 255, b = p >> 8;
        const uint8_t lb = base[draco_q6t_ql(nb, tok, b, (i >> 7) * 64 + (i & 63))];
        const int lo4 = ((i >> 6) & 1) ? (lb >> 4) : (lb & 0xF);
        const int hi2 = (base[draco_q6t_qh(nb, tok, b, (i >> 7) * 32 + (i & 31))] >> (((i >> 5) & 3) * 2)) & 3;
        const int8_t sc = (int8_t)base[draco_q6t_sc(nb, tok, b, i >> 4)];
        const float d = h2f(*reinterpret_cast<const uint16_t*>(base + draco_q6t_d(nb, tok, b)));
        val = (d * (float)sc) * (float)((lo4 | (hi2 << 4)) - 32);
    } else if (L.code == DRACO_Q4_K) {
        const int i = p & 255, j = i >> 5, b = p >> 8;
        const uint8_t* hd = base + draco_q4t_hdr(nb, tok, b);
        const float d = h2f(*reinterpret_cast<const uint16_t*>(hd)), dmin = h2f(*reinterpret_cast<const uint16_t*>(hd + 2));
        const uint8_t* s = hd + 4;
        int sc, m;
        if (j < 4) {
            sc = s[j] & 63;
            m = s[j + 4] & 63;
        } else {
            sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
            m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        }
        const uint8_t qb = base[draco_q4t_qs(nb, tok, b, (j >> 1) * 32 + (i & 31))] ^ 0x80;
        const int q = (j & 1) ? (qb >> 4) : (qb & 0xF);
        val = (d * (float)sc) * (float)q - dmin * (float)m;
    } else if (L.code == DRACO_Q5_K) {
        // the row decoder's order, (q*d)*sc - dmin*m (src/m5/m5_gemm.c:212-231)
        const int i = p & 255, j = i >> 5, b = p >> 8;
        const uint8_t* hd = base + draco_q5t_hdr(nb, tok, b);
        const float d = h2f(*reinterpret_cast<const uint16_t*>(hd)), dmin = h2f(*reinterpret_cast<const uint16_t*>(hd + 2));
        const uint8_t* s = hd + 4;
        int sc, m;
        if (j < 4) {
            sc = s[j] & 63;
            m = s[j + 4] & 63;
        } else {
            sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
            m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        }
        const uint8_t qb = base[draco_q5t_qs(nb, tok, b, (j >> 1) * 32 + (i & 31))];
        const int nib = (j & 1) ? (qb >> 4) : (qb & 0xF);
        const int top = (base[draco_q5t_qh(nb, tok, b, i & 31)] >> j) & 1;
        val = (float)(nib | (top << 4)) * d * (float)sc - dmin * (float)m;
    } else if (L.code == DRACO_F32) {
        val = reinterpret_cast<const float*>(base)[(size_t)tok * n_in + p];
    } else if (L.code == DRACO_F16) {
        val = h2f(reinterpret_cast<const uint16_t*>(base)[(size_t)tok * n_in + p]);
    }
    return val;
}
