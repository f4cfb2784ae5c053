// tile_frag.h -- one wave's operands of a (tile, super-block) item of the
// Q4_K / Q6_K tile layout (formats.h), shared by the fp32-activation GEMV
// (gemv.hip) and the Q8_K-activation GEMV (q8k.hip).
//
// Lane l = j + 16*g (row j of the 16-row tile, lane group g = 0..3).
#pragma once
#include <hip/hip_runtime.h>

#include "dev_common.h"
#include "formats.h"

typedef int v4i __attribute__((ext_vector_type(4)));

struct Frag {
    uint4 a, b, c;   // Q4_K / Q5_K: qs r=0, qs r=1, header.  Q6_K: ql A, ql B, qh
    uint4 h;         // Q5_K: 16 qh bytes (the fifth bits)
    uint32_t sc, d;  // Q6_K: 4 scales, d
};

__device__ __forceinline__ void load_q4(const uint8_t* item, int lane, Frag& f) {
    f.a = ldnt4(item + 16 * lane);
    f.b = ldnt4(item + 1024 + 16 * lane);
    f.c = ldnt4(item + 2048 + 16 * (lane & 15));
    f.sc = 0u;
    f.d = 0u;
}

__device__ __forceinline__ void load_q5(const uint8_t* item, int lane, Frag& f) {
    f.a = ldnt4(item + 16 * lane);
    f.b = ldnt4(item + 1024 + 16 * lane);
    f.c = ldnt4(item + 2048 + 16 * (lane & 15));
    f.h = ldnt4(item + 2304 + 16 * ((lane & 15) + 16 * ((lane >> 4) & 1)));
    f.sc = 0u;
    f.d = 0u;
}

__device__ __forceinline__ void load_q6(const uint8_t* item, int lane, Frag& f) {
    f.a = ldnt4(item + 16 * lane);
    f.b = ldnt4(item + 1024 + 16 * lane);
    f.c = ldnt4(item + 2048 + 16 * lane);
    f.sc = *gptr<uint32_t>(item + 3072 + 4 * lane);
    f.d = *gptr<uint16_t>(item + 3328 + 2 * (lane & 15));
}

// The same items through buffer loads: the item's address is one SGPR
// descriptor (range = the item's bytes), each lane's offset a fixed VGPR, so
// a loop that walks items forms no per-item VGPR address.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t item_rsrc(const uint8_t* item, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(item), (short)0, bytes, 0x00020000);
}

__device__ __forceinline__ uint4 bufnt4(__amdgpu_buffer_rsrc_t r, int off) {
    const v4u32 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);  // aux 2: non-temporal
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void load_q4b(const uint8_t* item, int lane, Frag& f) {
    const __amdgpu_buffer_rsrc_t r = item_rsrc(item, DRACO_Q4T_ITEM);
    f.a = bufnt4(r, 16 * lane);
    f.b = bufnt4(r, 1024 + 16 * lane);
    f.c = bufnt4(r, 2048 + 16 * (lane & 15));
    f.sc = 0u;
    f.d = 0u;
}

__device__ __forceinline__ void load_q6b(const uint8_t* item, int lane, Frag& f) {
    const __amdgpu_buffer_rsrc_t r = item_rsrc(item, DRACO_Q6T_ITEM);
    f.a = bufnt4(r, 16 * lane);
    f.b = bufnt4(r, 1024 + 16 * lane);
    f.c = bufnt4(r, 2048 + 16 * lane);
    f.sc = __builtin_amdgcn_raw_buffer_load_b32(r, 3072 + 4 * lane, 0, 0);
    f.d = __builtin_amdgcn_raw_buffer_load_b16(r, 3328 + 2 * (lane & 15), 0, 0);
}

// Either format with the same five loads and no branch (a launch that mixes
// Q4_K and Q6_K tiles): the descriptor's range is the item's bytes, so for a
// Q4_K item the two Q6_K-only loads fall past the range and read zero
// without touching memory.
__device__ __forceinline__ void load_q46b(const uint8_t* item, bool q4, int lane, Frag& f) {
    const __amdgpu_buffer_rsrc_t r = item_rsrc(item, q4 ? DRACO_Q4T_ITEM : DRACO_Q6T_ITEM);
    f.a = bufnt4(r, 16 * lane);
    f.b = bufnt4(r, 1024 + 16 * lane);
    f.c = bufnt4(r, 2048 + 16 * (q4 ? lane & 15 : lane));
    f.sc = __builtin_amdgcn_raw_buffer_load_b32(r, 3072 + 4 * lane, 0, 0);
    f.d = __builtin_amdgcn_raw_buffer_load_b16(r, 3328 + 2 * (lane & 15), 0, 0);
}

__device__ __forceinline__ float fold(const v4i C) {
    const int i0 = (C[0] << 7) + C[1], i1 = (C[2] << 7) + C[3];
    return fmaf((float)i1, 6.103515625e-05f, (float)i0);
}

// A operand of one int8 MFMA: 16 bytes at p, or zeros for lanes that hold
// no activation row (p == nullptr is never passed: callers point those lanes
// at a zeroed LDS region instead, so the load is unconditional).
__device__ __forceinline__ v4i lds_v4i(const int8_t* p) { return *reinterpret_cast<const v4i*>(p); }

// One Q4_K item: 16 rows x 256 values.  xa: this lane's A address for the
// item's first group (or the zero region), xsm + gi: its (scale, sum) pairs.
// Returns (d * sum_g sc*(x.q), dmin * sum_g m*(sum x)).
__device__ __forceinline__ float2 dot_q4(const Frag& f, const int8_t* xa, const float2* xsm, int gi, int g) {
    const int gh = g >> 1;
    float sD = 0.f, sM = 0.f;
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const uint4 q = r ? f.b : f.a;
#pragma unroll
        for (int nib = 0; nib < 2; nib++) {
            const uint32_t m = nib ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
            const v4i B = {(int)(q.x & m), (int)(q.y & m), (int)(q.z & m), (int)(q.w & m)};
            const int go = 8 * r + 2 * nib;  // group offset of this MFMA (lane adds 4*gh + (g&1))
            const v4i A = *reinterpret_cast<const v4i*>(xa + go * 64);
            const v4i C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, (v4i){0, 0, 0, 0}, 0, 0, 0);
            const float fv = fold(C);
            const float2 sm = xsm[gi + go];
            // six-bit scale/min of sub-block 4r + 2gh + nib (src/m5_kern_scalar.c:39-46)
            const int s0 = 2 * gh + nib;
            int sc, mn;
            if (r == 0) {
                sc = (f.c.y >> (8 * s0)) & 63;
                mn = (f.c.z >> (8 * s0)) & 63;
            } else {
                sc = ((f.c.w >> (8 * s0)) & 15) | (((f.c.y >> (8 * s0 + 6)) & 3) << 4);
                mn = ((f.c.w >> (8 * s0 + 4)) & 15) | (((f.c.z >> (8 * s0 + 6)) & 3) << 4);
            }
            const float scf = (float)sc;
            if (nib) {
                sD = fmaf(scf, fv * (sm.x * 0.0625f), sD);
                sD = fmaf(8.f * scf, sm.y, sD);
            } else {
                sD = fmaf(scf, fv * sm.x, sD);
            }
            sM = fmaf((float)mn, sm.y, sM);
        }
    }
    return make_float2(h2f((uint16_t)(f.c.x & 0xFFFF)) * sD, h2f((uint16_t)(f.c.x >> 16)) * sM);
}

// One Q5_K item: the Q4_K item's groups, each B byte the 5-bit quant
// nibble | (fifth bit << 4) in [0, 31] (src/m5_kern_scalar.c:91-114: bit s of
// qh[k] tops value 32*s + k), so a group's dot is (x.q5) and the weights
// regroup as d*sc_s*(x.q5) - dmin*m_s*(sum x), as for Q4_K.
// Returns (d * sum_g sc*(x.q), dmin * sum_g m*(sum x)).
__device__ __forceinline__ float2 dot_q5(const Frag& f, const int8_t* xa, const float2* xsm, int gi, int g) {
    const int gh = g >> 1;
    const uint32_t H4[4] = {f.h.x, f.h.y, f.h.z, f.h.w};
    float sD = 0.f, sM = 0.f;
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const uint4 q = r ? f.b : f.a;
        const uint32_t Q4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int nib = 0; nib < 2; nib++) {
            const int s = 4 * r + 2 * gh + nib;  // sub-block of this lane's values
            v4i B;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const uint32_t lo = nib ? (Q4[w] >> 4) & 0x0F0F0F0Fu : Q4[w] & 0x0F0F0F0Fu;
                B[w] = (int)(lo | (((H4[w] >> s) & 0x01010101u) << 4));
            }
            const int go = 8 * r + 2 * nib;
            const v4i A = *reinterpret_cast<const v4i*>(xa + go * 64);
            const v4i C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, (v4i){0, 0, 0, 0}, 0, 0, 0);
            const float fv = fold(C);
            const float2 sm = xsm[gi + go];
            const int s0 = 2 * gh + nib;
            int sc, mn;
            if (r == 0) {
                sc = (f.c.y >> (8 * s0)) & 63;
                mn = (f.c.z >> (8 * s0)) & 63;
            } else {
                sc = ((f.c.w >> (8 * s0)) & 15) | (((f.c.y >> (8 * s0 + 6)) & 3) << 4);
                mn = ((f.c.w >> (8 * s0 + 4)) & 15) | (((f.c.z >> (8 * s0 + 6)) & 3) << 4);
            }
            sD = fmaf((float)sc, fv * sm.x, sD);
            sM = fmaf((float)mn, sm.y, sM);
        }
    }
    return make_float2(h2f((uint16_t)(f.c.x & 0xFFFF)) * sD, h2f((uint16_t)(f.c.x >> 16)) * sM);
}

// One Q6_K item.  Fragment r (0..3) holds values 128*g2 + 32*r + 16*c + e
// (g2 = g>>1, c = g&1), i.e. group 8*g2 + 2*r + c, with the GGUF bit map of
// src/m5_kern_scalar.c:115-142: low nibble of ql A (r=0) / ql B (r=1), high
// nibble of ql A (r=2) / ql B (r=3), and qh bits 2r.
__device__ __forceinline__ float dot_q6(const Frag& f, const int8_t* xa, const float2* xsm, int gi) {
    const uint32_t A4[4] = {f.a.x, f.a.y, f.a.z, f.a.w};
    const uint32_t B4[4] = {f.b.x, f.b.y, f.b.z, f.b.w};
    const uint32_t H4[4] = {f.c.x, f.c.y, f.c.z, f.c.w};
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        v4i Bv;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            uint32_t v;
            if (r == 0) v = (A4[w] & 0x0F0F0F0Fu) | ((H4[w] << 4) & 0x30303030u);
            else if (r == 1) v = (B4[w] & 0x0F0F0F0Fu) | ((H4[w] << 2) & 0x30303030u);
            else if (r == 2) v = ((A4[w] >> 4) & 0x0F0F0F0Fu) | (H4[w] & 0x30303030u);
            else v = ((B4[w] >> 4) & 0x0F0F0F0Fu) | ((H4[w] >> 2) & 0x30303030u);
            Bv[w] = (int)v;
        }
        const v4i A = *reinterpret_cast<const v4i*>(xa + r * 128);
        const v4i C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, Bv, (v4i){0, 0, 0, 0}, 0, 0, 0);
        const float2 sm = xsm[gi + 2 * r];
        const float scf = (float)(int)(int8_t)(f.sc >> (8 * r));
        s = fmaf(scf, fmaf(-32.f, sm.y, fold(C) * sm.x), s);
    }
    return h2f((uint16_t)f.d) * s;
}


// Exact int8 digits of x for the MFMA GEMVs.  Values 4*i4 .. 4*i4+3 (v) of a
// vector go to the LDS layout xd[group][4 digits][16 values] and
// xsm[group] = (2^(k-7), sum of the group's values), where group = i4 / 4 and
// k = ilogb(max |x| of the group) - 5 (clamped at -100).  X = rint(x*2^(21-k))
// = d0*2^21 + d1*2^14 + d2*2^7 + d3, |X| < 2^27, d0 signed, d1..d3 in [0,127].
// The four threads of a group (consecutive lanes, i4 % 4 = 0..3) must call it
// together: the group maximum and sum use DPP quad moves.
__device__ __forceinline__ void digits4(float4 v, int i4, int8_t* xd, float2* xsm) {
    float am = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    float sum = (v.x + v.y) + (v.z + v.w);
    am = group_max<4>(am);
    sum = group_sum<4>(sum);
    const int k = am > 0.f ? max(ilogbf(am) - 5, -100) : 0;
    const float up = __builtin_bit_cast(float, (uint32_t)(127 + 21 - k) << 23);  // 2^(21-k)
    const uint32_t X0 = (uint32_t)(int)rintf(v.x * up), X1 = (uint32_t)(int)rintf(v.y * up);
    const uint32_t X2 = (uint32_t)(int)rintf(v.z * up), X3 = (uint32_t)(int)rintf(v.w * up);
    const int grp = i4 >> 2, qq = i4 & 3;
#pragma unroll
    for (int dg = 0; dg < 4; dg++) {
        const int sh = 21 - 7 * dg, wd = dg ? 7 : 8;
        const uint32_t o = __builtin_amdgcn_ubfe(X0, sh, wd) | (__builtin_amdgcn_ubfe(X1, sh, wd) << 8) |
                           (__builtin_amdgcn_ubfe(X2, sh, wd) << 16) | (__builtin_amdgcn_ubfe(X3, sh, wd) << 24);
        *reinterpret_cast<uint32_t*>(xd + (grp * 4 + dg) * 16 + 4 * qq) = o;
    }
    if (qq == 0) xsm[grp] = make_float2(__builtin_bit_cast(float, (uint32_t)(127 + k - 7) << 23), sum);
}
