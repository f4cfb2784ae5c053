// host_quant.cpp -- host-side byte work: GGUF block encoders for the synthetic
// models, the one-time repack into the private device layout, and the rope
// angle table.  Pure CPU code (no HIP calls), so it is testable without a GPU.
//
// The encoders write valid GGUF Q8_0 / Q4_K / Q5_K / Q6_K blocks (layouts as
// read by src/m5_kern_scalar.c:58-142).  Any valid encoder is acceptable for the
// benchmark configurations: the GPU path and the CPU oracle consume the same
// bytes.  Rounding is round-half-even everywhere (rintf), so the bytes are
// reproducible on every IEEE host.
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <string.h>

#include "formats.h"

static inline float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t ex = (h >> 10) & 0x1Fu, mant = h & 0x3FFu;
    uint32_t bits;
    if (ex == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            float v = (float)mant * 5.9604644775390625e-8f;
            uint32_t vb;
            memcpy(&vb, &v, 4);
            bits = sign | vb;
        }
    } else if (ex == 31) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((ex + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// float -> IEEE half, round to nearest even (finite inputs well inside range).
static inline uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int32_t ex = (int32_t)((x >> 23) & 0xFF) - 127 + 15;
    uint32_t mant = x & 0x7FFFFFu;
    if (((x >> 23) & 0xFF) == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0u));
    if (ex >= 31) return (uint16_t)(sign | 0x7C00u);
    if (ex <= 0) {
        if (ex < -10) return (uint16_t)sign;
        mant |= 0x800000u;
        const int shift = 14 - ex;  // 1 - ex + 13
        uint32_t h = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)ex << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;  // carry may roll into the exponent: still RNE
    return (uint16_t)(sign | h);
}

static inline float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

// ---- Q8_0: [d f16][32 x int8] ----
static void enc_q8_0(const float* x, uint8_t* blk) {
    float amax = 0.f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
    const uint16_t hd = f32_to_f16(amax / 127.f);
    const float d = f16_to_f32(hd);
    memcpy(blk, &hd, 2);
    for (int i = 0; i < 32; i++) {
        const float q = d > 0.f ? clampf(rintf(x[i] / d), -127.f, 127.f) : 0.f;
        blk[2 + i] = (uint8_t)(int8_t)q;
    }
}

// ---- Q4_K: [d f16][dmin f16][scales 12][qs 128]; w = d*sc_j*q - dmin*m_j ----
static void enc_q4_k(const float* x, uint8_t* blk) {
    float scale[8], minv[8];
    for (int j = 0; j < 8; j++) {
        float lo = 0.f, hi = -INFINITY;
        for (int k = 0; k < 32; k++) {
            lo = fminf(lo, x[j * 32 + k]);
            hi = fmaxf(hi, x[j * 32 + k]);
        }
        if (hi < lo) hi = lo;
        scale[j] = (hi - lo) / 15.f;
        minv[j] = -lo;
    }
    float ms = 0.f, mm = 0.f;
    for (int j = 0; j < 8; j++) {
        ms = fmaxf(ms, scale[j]);
        mm = fmaxf(mm, minv[j]);
    }
    const uint16_t hd = f32_to_f16(ms / 63.f), hm = f32_to_f16(mm / 63.f);
    const float d = f16_to_f32(hd), dmin = f16_to_f32(hm);
    int sc[8], mn[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = d > 0.f ? (int)clampf(rintf(scale[j] / d), 0.f, 63.f) : 0;
        mn[j] = dmin > 0.f ? (int)clampf(rintf(minv[j] / dmin), 0.f, 63.f) : 0;
    }
    memcpy(blk, &hd, 2);
    memcpy(blk + 2, &hm, 2);
    uint8_t* s = blk + 4;
    for (int i = 0; i < 4; i++) {
        s[i] = (uint8_t)(sc[i] | ((sc[4 + i] >> 4) << 6));
        s[4 + i] = (uint8_t)(mn[i] | ((mn[4 + i] >> 4) << 6));
        s[8 + i] = (uint8_t)((sc[4 + i] & 0xF) | ((mn[4 + i] & 0xF) << 4));
    }
    uint8_t* qs = blk + 16;
    memset(qs, 0, 128);
    for (int j = 0; j < 8; j++) {
        const float S = d * (float)sc[j], M = dmin * (float)mn[j];
        for (int k = 0; k < 32; k++) {
            const int q = S > 0.f ? (int)clampf(rintf((x[j * 32 + k] + M) / S), 0.f, 15.f) : 0;
            qs[(j >> 1) * 32 + k] |= (uint8_t)(q << ((j & 1) * 4));
        }
    }
}

// ---- Q5_K: [d f16][dmin f16][scales 12][qh 32][qs 128]; w = d*sc_j*q - dmin*m_j,
// q = nibble | (bit j of qh[k]) << 4 for value 32 j + k ----
static void enc_q5_k(const float* x, uint8_t* blk) {
    float scale[8], minv[8];
    for (int j = 0; j < 8; j++) {
        float lo = 0.f, hi = -INFINITY;
        for (int k = 0; k < 32; k++) {
            lo = fminf(lo, x[j * 32 + k]);
            hi = fmaxf(hi, x[j * 32 + k]);
        }
        if (hi < lo) hi = lo;
        scale[j] = (hi - lo) / 31.f;
        minv[j] = -lo;
    }
    float ms = 0.f, mm = 0.f;
    for (int j = 0; j < 8; j++) {
        ms = fmaxf(ms, scale[j]);
        mm = fmaxf(mm, minv[j]);
    }
    const uint16_t hd = f32_to_f16(ms / 63.f), hm = f32_to_f16(mm / 63.f);
    const float d = f16_to_f32(hd), dmin = f16_to_f32(hm);
    int sc[8], mn[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = d > 0.f ? (int)clampf(rintf(scale[j] / d), 0.f, 63.f) : 0;
        mn[j] = dmin > 0.f ? (int)clampf(rintf(minv[j] / dmin), 0.f, 63.f) : 0;
    }
    memcpy(blk, &hd, 2);
    memcpy(blk + 2, &hm, 2);
    uint8_t* s = blk + 4;
    for (int i = 0; i < 4; i++) {
        s[i] = (uint8_t)(sc[i] | ((sc[4 + i] >> 4) << 6));
        s[4 + i] = (uint8_t)(mn[i] | ((mn[4 + i] >> 4) << 6));
        s[8 + i] = (uint8_t)((sc[4 + i] & 0xF) | ((mn[4 + i] & 0xF) << 4));
    }
    uint8_t* qh = blk + 16;
    uint8_t* qs = blk + 48;
    memset(qh, 0, 32 + 128);
    for (int j = 0; j < 8; j++) {
        const float S = d * (float)sc[j], M = dmin * (float)mn[j];
        for (int k = 0; k < 32; k++) {
            const int q = S > 0.f ? (int)clampf(rintf((x[j * 32 + k] + M) / S), 0.f, 31.f) : 0;
            qs[(j >> 1) * 32 + k] |= (uint8_t)((q & 15) << ((j & 1) * 4));
            qh[k] |= (uint8_t)((q >> 4) << j);
        }
    }
}

// ---- Q6_K: [ql 128][qh 64][sc 16 x int8][d f16]; w = d*sc_g*(q-32) ----
static void enc_q6_k(const float* x, uint8_t* blk) {
    float gs[16];
    for (int g = 0; g < 16; g++) {
        float amax = 0.f;
        for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(x[g * 16 + i]));
        gs[g] = amax / 31.f;
    }
    float mg = 0.f;
    for (int g = 0; g < 16; g++) mg = fmaxf(mg, gs[g]);
    const uint16_t hd = f32_to_f16(mg / 127.f);
    const float d = f16_to_f32(hd);
    uint8_t* ql = blk;
    uint8_t* qh = blk + 128;
    int8_t* sc = (int8_t*)(blk + 192);
    memset(blk, 0, 210);
    for (int g = 0; g < 16; g++) sc[g] = (int8_t)(d > 0.f ? clampf(rintf(gs[g] / d), -128.f, 127.f) : 0.f);
    for (int p = 0; p < 256; p++) {
        const float S = d * (float)sc[p >> 4];
        const int q = (S > 0.f ? (int)clampf(rintf(x[p] / S), -32.f, 31.f) : 0) + 32;
        const int half = p >> 7, rr = (p >> 5) & 3, l = p & 31;
        ql[half * 64 + (rr & 1) * 32 + l] |= (uint8_t)((q & 0xF) << ((rr >> 1) * 4));
        qh[half * 32 + l] |= (uint8_t)(((q >> 4) & 3) << (2 * rr));
    }
    memcpy(blk + 208, &hd, 2);
}

extern "C" {

float draco_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
uint16_t draco_f32_to_f16(float f) { return f32_to_f16(f); }

// Encode n_rows x n_in floats into GGUF rows of format `code`.
int draco_quantize(int code, const float* x, int n_rows, int n_in, uint8_t* out) {
    const int bv = draco_block_values(code);
    if (bv <= 1 || n_in % bv) return -1;
    const size_t rb = draco_row_bytes(code, n_in);
    const int nb = n_in / bv;
    const int64_t total = (int64_t)n_rows * nb;
    const int bb = (int)draco_row_bytes(code, bv);
    if (code != DRACO_Q8_0 && code != DRACO_Q4_K && code != DRACO_Q5_K && code != DRACO_Q6_K) return -1;
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < total; i++) {
        const int64_t r = i / nb, b = i % nb;
        const float* src = x + r * (int64_t)n_in + b * bv;
        uint8_t* dst = out + r * (int64_t)rb + b * bb;
        if (code == DRACO_Q8_0) enc_q8_0(src, dst);
        else if (code == DRACO_Q4_K) enc_q4_k(src, dst);
        else if (code == DRACO_Q5_K) enc_q5_k(src, dst);
        else enc_q6_k(src, dst);
    }
    return 0;
}

// Layout query: fills off[4] and returns the total device bytes (0 = unsupported).
size_t draco_layout_query(int code, int n_out, int n_in, size_t* off4) {
    DracoLayout L;
    if (draco_layout(code, n_out, n_in, &L)) return 0;
    if (off4) for (int i = 0; i < 4; i++) off4[i] = L.off[i];
    return L.bytes;
}

// GGUF rows -> private layout (dst must hold draco_layout_query bytes).
int draco_repack(int code, const uint8_t* src, int n_out, int n_in, uint8_t* dst) {
    DracoLayout L;
    if (draco_layout(code, n_out, n_in, &L)) return -1;
    const int nb = L.nb;
    const size_t rb = draco_row_bytes(code, n_in);
    if (code == DRACO_F16 || code == DRACO_F32) {
        memcpy(dst, src, rb * (size_t)n_out);
        return 0;
    }
    if (code != DRACO_Q4_K && code != DRACO_Q5_K && code != DRACO_Q6_K && code != DRACO_Q8_0) return -1;
    if (code != DRACO_Q8_0) memset(dst, 0, L.bytes);  // padding rows of the last tile
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < n_out; r++) {
        for (int b = 0; b < nb; b++) {
            if (code == DRACO_Q4_K) {
                const uint8_t* blk = src + (size_t)r * rb + (size_t)b * 144;
                memcpy(dst + draco_q4t_hdr(nb, r, b), blk, 16);
                for (int i = 0; i < 128; i += 16)  // 16-byte runs stay contiguous
                    for (int e = 0; e < 16; e++) dst[draco_q4t_qs(nb, r, b, i) + e] = blk[16 + i + e] ^ 0x80;
            } else if (code == DRACO_Q5_K) {
                const uint8_t* blk = src + (size_t)r * rb + (size_t)b * 176;
                memcpy(dst + draco_q5t_hdr(nb, r, b), blk, 16);
                for (int i = 0; i < 32; i += 16) memcpy(dst + draco_q5t_qh(nb, r, b, i), blk + 16 + i, 16);
                for (int i = 0; i < 128; i += 16) memcpy(dst + draco_q5t_qs(nb, r, b, i), blk + 48 + i, 16);
            } else if (code == DRACO_Q6_K) {
                const uint8_t* blk = src + (size_t)r * rb + (size_t)b * 210;
                for (int i = 0; i < 128; i += 16) memcpy(dst + draco_q6t_ql(nb, r, b, i), blk + i, 16);
                for (int i = 0; i < 64; i += 16) memcpy(dst + draco_q6t_qh(nb, r, b, i), blk + 128 + i, 16);
                for (int i = 0; i < 16; i++) dst[draco_q6t_sc(nb, r, b, i)] = blk[192 + i];
                memcpy(dst + draco_q6t_d(nb, r, b), blk + 208, 2);
            } else {
                const size_t i = (size_t)r * nb + b;
                const uint8_t* blk = src + (size_t)r * rb + (size_t)b * 34;
                memcpy(dst + L.off[0] + i * 32, blk + 2, 32);
                memcpy(dst + L.off[1] + i * 2, blk, 2);
            }
        }
    }
    return 0;
}

// Inverse of draco_repack (used by tests to prove the repack is a bijection).
int draco_unpack(int code, const uint8_t* src, int n_out, int n_in, uint8_t* dst) {
    DracoLayout L;
    if (draco_layout(code, n_out, n_in, &L)) return -1;
    const int nb = L.nb;
    const size_t rb = draco_row_bytes(code, n_in);
    if (code == DRACO_F16 || code == DRACO_F32) {
        memcpy(dst, src, rb * (size_t)n_out);
        return 0;
    }
    for (int r = 0; r < n_out; r++)
        for (int b = 0; b < nb; b++) {
            if (code == DRACO_Q4_K) {
                uint8_t* blk = dst + (size_t)r * rb + (size_t)b * 144;
                memcpy(blk, src + draco_q4t_hdr(nb, r, b), 16);
                for (int i = 0; i < 128; i++) blk[16 + i] = src[draco_q4t_qs(nb, r, b, i)] ^ 0x80;
            } else if (code == DRACO_Q5_K) {
                uint8_t* blk = dst + (size_t)r * rb + (size_t)b * 176;
                memcpy(blk, src + draco_q5t_hdr(nb, r, b), 16);
                for (int i = 0; i < 32; i++) blk[16 + i] = src[draco_q5t_qh(nb, r, b, i)];
                for (int i = 0; i < 128; i++) blk[48 + i] = src[draco_q5t_qs(nb, r, b, i)];
            } else if (code == DRACO_Q6_K) {
                uint8_t* blk = dst + (size_t)r * rb + (size_t)b * 210;
                for (int i = 0; i < 128; i++) blk[i] = src[draco_q6t_ql(nb, r, b, i)];
                for (int i = 0; i < 64; i++) blk[128 + i] = src[draco_q6t_qh(nb, r, b, i)];
                for (int i = 0; i < 16; i++) blk[192 + i] = src[draco_q6t_sc(nb, r, b, i)];
                memcpy(blk + 208, src + draco_q6t_d(nb, r, b), 2);
            } else {
                const size_t i = (size_t)r * nb + b;
                uint8_t* blk = dst + (size_t)r * rb + (size_t)b * 34;
                memcpy(blk + 2, src + L.off[0] + i * 32, 32);
                memcpy(blk, src + L.off[1] + i * 2, 2);
            }
        }
    return 0;
}

// Rope angle table, computed with the same libm calls and operation order as
// the reference's consecutive-pair rope (src/m6_engine.c:134-143):
//   theta = (float)pos * powf(base, -2.0f*(float)i/(float)rot)
//   tab[(pos*half + i)*2 + 0] = cosf(theta), [..+1] = sinf(theta)
void draco_rope_table(int max_t, int rot, float base, float* tab) {
    const int half = rot / 2;
    for (int pos = 0; pos < max_t; pos++)
        for (int i = 0; i < half; i++) {
            const float theta = (float)pos * powf(base, -2.0f * (float)i / (float)rot);
            tab[((size_t)pos * half + i) * 2 + 0] = cosf(theta);
            tab[((size_t)pos * half + i) * 2 + 1] = sinf(theta);
        }
}

}  // extern "C"
