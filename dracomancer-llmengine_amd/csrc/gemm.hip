// gemm.hip -- chunked-prefill GEMM  Y[T x n_out] = X[T x n_in] . W^T  (gfx950).
//
// Reference semantics: m5_gemm (src/m5/m5_gemm.c:249-272: dequantized row
// times every token, fp32) and m5_gemm_auto (src/m5/m5_gemm_fused.c:231-241).
// Weights are the Q4_K / Q6_K tile layout shared with the decode GEMV
// (formats.h).
//
// x is first turned into exact int8 digits (k_gemm_digits): per token and
// 256-value super-block, k = ilogb(max|x|) - 5 and X = rint(x*2^(21-k)) =
// d0*2^21 + d1*2^14 + d2*2^7 + d3 (d0 signed, d1..d3 in [0,127]); the
// representation error is below 2^(k-22), under half an fp32 ulp of the
// super-block maximum.  The product then runs on v_mfma_i32_32x32x32_i8:
//   A (32 x 32): rows m = 4*token + digit for 8 tokens, K = 32 values;
//   B (32 x 32): 32 weight rows (two 16-row tiles) x the same 32 values,
//                lane (n, u) loading its 16 quant bytes straight from the
//                tile layout (row n, values 16u..16u+15);
//   C (32 x 32): lane (n, u) receives, for row n, the 4 digit dots of
//                tokens 2q+u (q = 0..3), exact int32.
// Q4_K: one MFMA per 32-value sub-block; the lane accumulates sc*C (x16 for
// low nibbles; high nibbles are stored as 16*(q-8), formats.h) in int32 over
// the super-block and folds the 4 digits to fp32 once:
//   y += d*2^k*fold/16 + sum_sb (8*d*sc_sb*[sb odd] - dmin*m_sb) * xsum_sb
// (fold = sum over digits of acc_digit * 2^(-7*digit), in units of X / 2^21)
// where xsum_sb is the fp32 sum of the token's 32 values in sub-block sb.
// Q6_K: scales change every 16 values, so A is block-diagonal over the two
// 16-value halves of a 32-value chunk (rows m = 16*h + 4*token + digit, 4
// tokens); each half's C is scaled by its own sc and the -32 offset uses the
// 16-value sums.
// Every product of quant and digit is exact; the order of the fp32 sums over
// super-blocks differs from the reference's row dot, so results agree to fp32
// rounding (~1e-7 relative), not bitwise.
#include <hip/hip_runtime.h>

#include "dev_common.h"
#include "formats.h"
#include "gemm.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------- digits --
// One block of 64 threads per (token, super-block); thread i owns values
// 4i..4i+3.  Outputs (T padded to a multiple of 8 with zero tokens):
//   xdig[T/8][n_in/32][64 lanes][16]  lane = (4*(t%8) + digit) + 32*u holds the
//                                     digit of values 16u..16u+15 of a 32-chunk
//   xsc[T/8][nb][2][4]                2^k of token 2q+u at [u][q]
//   xs32[T/8][n_in/32][2][4]          sum of the 32 values, same token order
//   xs16[T/8][n_in/16][2][4]          sum of the 16 values (Q6_K offset)
__global__ __launch_bounds__(64) void k_gemm_digits(const float* __restrict__ X, int T, int n_in,
                                                    int8_t* __restrict__ xdig, float* __restrict__ xsc,
                                                    float* __restrict__ xs32, float* __restrict__ xs16) {
    const int b = blockIdx.x, t = blockIdx.y, i = threadIdx.x;
    const int nb = n_in >> 8, nc = n_in >> 5, ng = n_in >> 4;
    const int oc = t >> 3, tt = t & 7, u8 = tt & 1, q8 = tt >> 1;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t < T) v = ld4(X + (size_t)t * n_in + (size_t)b * 256 + 4 * i);
    float am = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    am = wave_max(am);
    const int k = am > 0.f ? max(ilogbf(am) - 5, -100) : 0;
    const float up = __builtin_bit_cast(float, (uint32_t)(127 + 21 - k) << 23);  // 2^(21-k)
    const uint32_t X0 = (uint32_t)(int)rintf(v.x * up), X1 = (uint32_t)(int)rintf(v.y * up);
    const uint32_t X2 = (uint32_t)(int)rintf(v.z * up), X3 = (uint32_t)(int)rintf(v.w * up);
    // position: value p = 4i .. 4i+3 of the super-block; chunk c = b*8 + p/32
    const int p = 4 * i, c = b * 8 + (p >> 5), kk = p & 31, u = kk >> 4, e = kk & 15;
#pragma unroll
    for (int dg = 0; dg < 4; dg++) {
        const int sh = 21 - 7 * dg, wd = dg ? 7 : 8;
        const uint32_t o = __builtin_amdgcn_ubfe(X0, sh, wd) | (__builtin_amdgcn_ubfe(X1, sh, wd) << 8) |
                           (__builtin_amdgcn_ubfe(X2, sh, wd) << 16) | (__builtin_amdgcn_ubfe(X3, sh, wd) << 24);
        const int lane = (4 * tt + dg) + 32 * u;
        *reinterpret_cast<uint32_t*>(xdig + (((size_t)oc * nc + c) * 64 + lane) * 16 + e) = o;
    }
    // 16- and 32-value sums (4 and 8 consecutive threads)
    float s = (v.x + v.y) + (v.z + v.w);
    s = group_sum<4>(s);
    if ((i & 3) == 0) xs16[(((size_t)oc * ng + b * 16 + (i >> 2)) * 2 + u8) * 4 + q8] = s;
    s += dpp<DPP_MIRROR8>(s);  // the other 4 lanes of the 8, uniform after the step above
    if ((i & 7) == 0) xs32[(((size_t)oc * nc + c) * 2 + u8) * 4 + q8] = s;
    // the digit fold gives X / 2^21, and x = (X / 2^21) * 2^k
    if (i == 0) xsc[(((size_t)oc * nb + b) * 2 + u8) * 4 + q8] = __builtin_bit_cast(float, (uint32_t)(127 + k) << 23);
}

__device__ __forceinline__ float fold4(int a0, int a1, int a2, int a3) {
    return fmaf((float)a3, 4.76837158203125e-07f, fmaf((float)a2, 6.103515625e-05f, fmaf((float)a1, 0.0078125f, (float)a0)));
}

// ------------------------------------------------------------------ Q4_K --
// Block: NW waves, wave w = token octet (blockIdx.y*NW + w); the block walks
// RP row-pairs (32 rows each) from blockIdx.x*RP.
template <int NW, int RP>
__global__ __launch_bounds__(64 * NW) void k_gemm_q4(const GemmArgs a) {
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 31, u = lane >> 5;
    // grouped launch: blockIdx.z selects the group (weights, token octets)
    const GemmGroup* gp = a.groups ? a.groups + blockIdx.z : nullptr;
    const uint8_t* Wb = gp ? gp->W : a.W;
    const int oi = blockIdx.y * NW + w;
    const int n_oct = gp ? gp->n_oct : (a.T + 7) >> 3;
    if (oi >= n_oct) return;                             // uniform per wave; no barriers below
    const int oc = (gp ? gp->oct0 : 0) + oi;             // token octet in the digit buffer
    const int nb = a.n_in >> 8, nc = a.n_in >> 5;
    const int p0 = blockIdx.x * RP;
    float y[RP][4];
#pragma unroll
    for (int p = 0; p < RP; p++)
#pragma unroll
        for (int q = 0; q < 4; q++) y[p][q] = 0.f;
    for (int b = 0; b < nb; b++) {
        // A: this octet's 8 chunks of super-block b
        v4i A[8];
#pragma unroll
        for (int sb = 0; sb < 8; sb++)
            A[sb] = *reinterpret_cast<const v4i*>(a.xdig + (((size_t)oc * nc + b * 8 + sb) * 64 + lane) * 16);
        const float4 xs = *reinterpret_cast<const float4*>(a.xsc + (((size_t)oc * nb + b) * 2 + u) * 4);
        float4 s32[8];
#pragma unroll
        for (int sb = 0; sb < 8; sb++)
            s32[sb] = *reinterpret_cast<const float4*>(a.xs32 + (((size_t)oc * nc + b * 8 + sb) * 2 + u) * 4);
#pragma unroll
        for (int p = 0; p < RP; p++) {
            const int tile = 2 * (p0 + p) + (n >> 4), j = n & 15;
            if (2 * (p0 + p) >= a.L.ntiles) break;       // uniform
            const int tl = tile < a.L.ntiles ? tile : a.L.ntiles - 1;
            const uint8_t* item = Wb + ((size_t)tl * nb + b) * DRACO_Q4T_ITEM;
            uint4 q[2][2];
#pragma unroll
            for (int r = 0; r < 2; r++)
#pragma unroll
                for (int gh = 0; gh < 2; gh++) q[r][gh] = ldu4(item + r * 1024 + 16 * (j + 16 * (2 * gh + u)));
            const uint4 h = ldu4(item + 2048 + 16 * j);
            int acc[16];
#pragma unroll
            for (int i = 0; i < 16; i++) acc[i] = 0;
            float coef[8];
            const float d = h2f((uint16_t)(h.x & 0xFFFF)), dmin = h2f((uint16_t)(h.x >> 16));
#pragma unroll
            for (int sb = 0; sb < 8; sb++) {
                const int r = sb >> 2, gh = (sb >> 1) & 1, nib = sb & 1;
                // six-bit scale and min of sub-block sb (src/m5_kern_scalar.c:39-46)
                int sc, mn;
                if (sb < 4) {
                    sc = (h.y >> (8 * sb)) & 63;
                    mn = (h.z >> (8 * sb)) & 63;
                } else {
                    const int s0 = sb - 4;
                    sc = ((h.w >> (8 * s0)) & 15) | (((h.y >> (8 * s0 + 6)) & 3) << 4);
                    mn = ((h.w >> (8 * s0 + 4)) & 15) | (((h.z >> (8 * s0 + 6)) & 3) << 4);
                }
                coef[sb] = (nib ? 8.f * d * (float)sc : 0.f) - dmin * (float)mn;
                const uint32_t m = nib ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
                const uint4 qq = q[r][gh];
                const v4i B = {(int)(qq.x & m), (int)(qq.y & m), (int)(qq.z & m), (int)(qq.w & m)};
                const v16i C = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[sb], B, (v16i){}, 0, 0, 0);
                const int scm = nib ? sc : 16 * sc;
#pragma unroll
                for (int i = 0; i < 16; i++) acc[i] += __mul24(scm, C[i]);  // |scm| < 2^10, |C| < 2^20: exact
            }
#pragma unroll
            for (int qt = 0; qt < 4; qt++) {
                const float f = fold4(acc[4 * qt], acc[4 * qt + 1], acc[4 * qt + 2], acc[4 * qt + 3]);
                const float xsq = qt == 0 ? xs.x : (qt == 1 ? xs.y : (qt == 2 ? xs.z : xs.w));
                float t = (d * xsq) * (f * 0.0625f);
#pragma unroll
                for (int sb = 0; sb < 8; sb++) {
                    const float4 sv = s32[sb];
                    const float sq = qt == 0 ? sv.x : (qt == 1 ? sv.y : (qt == 2 ? sv.z : sv.w));
                    t = fmaf(coef[sb], sq, t);
                }
                y[p][qt] += t;
            }
        }
    }
#pragma unroll
    for (int p = 0; p < RP; p++) {
        const int row = 32 * (p0 + p) + n;
        if (row >= a.L.n_out) continue;
#pragma unroll
        for (int qt = 0; qt < 4; qt++) {
            const int tok = 8 * oc + 2 * qt + u;
            if (tok < a.T) a.Y[(size_t)tok * a.ldy + row] = y[p][qt];
        }
    }
}

// ------------------------------------------------------------------ Q6_K --
// A rows m = 16*h + 4*t4 + digit: half h of a 32-value chunk, token 4*qs + t4
// of the octet (qs = token quad 0/1).  Lane (n, u) with u == h supplies the
// digits; the others supply zeros.  C element i of lane (n, u): m = 8*(i/4) +
// 4u + i%4 -> h = i/8, t4 = 2*((i/4)&1) + u, digit i%4.
template <int NW, int RP>
__global__ __launch_bounds__(64 * NW) void k_gemm_q6(const GemmArgs a) {
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 31, u = lane >> 5;
    // grouped launch: blockIdx.z selects the group (weights, token octets)
    const GemmGroup* gp = a.groups ? a.groups + blockIdx.z : nullptr;
    const uint8_t* Wb = gp ? gp->W : a.W;
    const int oi = blockIdx.y * NW + w;
    const int n_oct = gp ? gp->n_oct : (a.T + 7) >> 3;
    if (oi >= n_oct) return;                             // uniform per wave; no barriers below
    const int oc = (gp ? gp->oct0 : 0) + oi;             // token octet in the digit buffer
    const int nb = a.n_in >> 8, nc = a.n_in >> 5, ng = a.n_in >> 4;
    const int p0 = blockIdx.x * RP;
    // A-row role of this lane: m = lane & 31 = 16h + 4t4 + dg
    const int hA = (lane & 31) >> 4, t4A = (lane >> 2) & 3, dgA = lane & 3;
    const bool asup = hA == u;
    float y[RP][2][4];  // [p][token quad][token 2*(i/4&1)+u ... ] -> [p][qs][t4 pair]
#pragma unroll
    for (int p = 0; p < RP; p++)
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int q = 0; q < 4; q++) y[p][s][q] = 0.f;
    for (int b = 0; b < nb; b++) {
        // token scales of this octet's parity-u tokens (2^k per token, k per super-block)
        const float4 xs = *reinterpret_cast<const float4*>(a.xsc + (((size_t)oc * nb + b) * 2 + u) * 4);
#pragma unroll
        for (int p = 0; p < RP; p++) {
            if (2 * (p0 + p) >= a.L.ntiles) break;
            const int tile = 2 * (p0 + p) + (n >> 4), j = n & 15;
            const int tl = tile < a.L.ntiles ? tile : a.L.ntiles - 1;
            const uint8_t* item = Wb + ((size_t)tl * nb + b) * DRACO_Q6T_ITEM;
            const float d = h2f(*gptr<uint16_t>(item + 3328 + 2 * j));
            // per super-block: int32 sums of sc * C over the 8 chunks (exact), and the
            // fp32 sums of sc * (16-value sums) for the -32 offset
            int acc[2][16];
            float off[2][2];
#pragma unroll
            for (int qs = 0; qs < 2; qs++) {
#pragma unroll
                for (int i = 0; i < 16; i++) acc[qs][i] = 0;
                off[qs][0] = off[qs][1] = 0.f;
            }
#pragma unroll 1
            for (int g2 = 0; g2 < 2; g2++) {
                const int ls = j + 16 * (2 * g2 + u);  // tile-layout lane slot of (row j, group pair g2, half u)
                const uint4 qa = ldu4(item + 16 * ls), qb = ldu4(item + 1024 + 16 * ls), qh = ldu4(item + 2048 + 16 * ls);
                const uint32_t sc4 = *gptr<uint32_t>(item + 3072 + 4 * ls);
                // every activation operand of the four 32-value chunks of this group pair,
                // loaded before the first MFMA (one memory round trip per group pair)
                v4i A[4][2];
                float4 s16[4][2];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int c = b * 8 + 4 * g2 + r;  // 32-value chunk: values 128*g2 + 32r .. +31
#pragma unroll
                    for (int qs = 0; qs < 2; qs++) {
                        // A: digits of token 4*qs + t4A, half hA, from the octet layout
                        const int mo = 4 * (4 * qs + t4A) + dgA;  // octet A-row (4*token + digit)
                        const v4i av = *reinterpret_cast<const v4i*>(a.xdig + (((size_t)oc * nc + c) * 64 + mo + 32 * hA) * 16);
                        A[r][qs] = asup ? av : (v4i){0, 0, 0, 0};
                    }
#pragma unroll
                    for (int h = 0; h < 2; h++)
                        s16[r][h] = *reinterpret_cast<const float4*>(a.xs16 + (((size_t)oc * ng + 2 * c + h) * 2 + u) * 4);
                }
                // this lane's scale for chunk r is that of group 8*g2 + 2r + u; the other half's comes from lane^32
                const uint32_t sc4o = lane_xor32(sc4);
                const uint32_t A4[4] = {qa.x, qa.y, qa.z, qa.w}, B4[4] = {qb.x, qb.y, qb.z, qb.w};
                const uint32_t H4[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    v4i Bv;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        uint32_t vv;
                        if (r == 0) vv = (A4[q] & 0x0F0F0F0Fu) | ((H4[q] << 4) & 0x30303030u);
                        else if (r == 1) vv = (B4[q] & 0x0F0F0F0Fu) | ((H4[q] << 2) & 0x30303030u);
                        else if (r == 2) vv = ((A4[q] >> 4) & 0x0F0F0F0Fu) | (H4[q] & 0x30303030u);
                        else vv = ((B4[q] >> 4) & 0x0F0F0F0Fu) | ((H4[q] >> 2) & 0x30303030u);
                        Bv[q] = (int)vv;
                    }
                    // group of half h: 16-value group 2c + h
                    const int sc_u = (int)(int8_t)(sc4 >> (8 * r));    // half u
                    const int sc_o = (int)(int8_t)(sc4o >> (8 * r));   // half 1-u
                    const int sc0 = u == 0 ? sc_u : sc_o, sc1 = u == 1 ? sc_u : sc_o;  // halves 0, 1
#pragma unroll
                    for (int qs = 0; qs < 2; qs++) {
                        const v16i C = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[r][qs], Bv, (v16i){}, 0, 0, 0);
                        // C[i]: h = i/8, t4 = 2*((i/4)&1) + u, digit i%4
#pragma unroll
                        for (int i = 0; i < 16; i++) acc[qs][i] += __mul24(i < 8 ? sc0 : sc1, C[i]);  // exact: < 2^27
#pragma unroll
                        for (int tq = 0; tq < 2; tq++) {
                            const int tq2 = 2 * qs + tq;  // token 4*qs + 2*tq + u = 2*tq2 + u
                            const float4 v0 = s16[r][0], v1 = s16[r][1];
                            const float sv0 = tq2 == 0 ? v0.x : (tq2 == 1 ? v0.y : (tq2 == 2 ? v0.z : v0.w));
                            const float sv1 = tq2 == 0 ? v1.x : (tq2 == 1 ? v1.y : (tq2 == 2 ? v1.z : v1.w));
                            off[qs][tq] = fmaf((float)sc1, sv1, fmaf((float)sc0, sv0, off[qs][tq]));
                        }
                    }
                }
            }
            // fold once per super-block: both halves' digit sums, then the token scale
#pragma unroll
            for (int qs = 0; qs < 2; qs++)
#pragma unroll
                for (int tq = 0; tq < 2; tq++) {
                    const int tq2 = 2 * qs + tq;
                    const float xsq = tq2 == 0 ? xs.x : (tq2 == 1 ? xs.y : (tq2 == 2 ? xs.z : xs.w));
                    const int i0 = 4 * tq;
                    const float f = fold4(acc[qs][i0] + acc[qs][i0 + 8], acc[qs][i0 + 1] + acc[qs][i0 + 9],
                                          acc[qs][i0 + 2] + acc[qs][i0 + 10], acc[qs][i0 + 3] + acc[qs][i0 + 11]);
                    y[p][qs][tq] = fmaf(d, fmaf(-32.f, off[qs][tq], f * xsq), y[p][qs][tq]);
                }
        }
    }
#pragma unroll
    for (int p = 0; p < RP; p++) {
        const int row = 32 * (p0 + p) + n;
        if (row >= a.L.n_out) continue;
#pragma unroll
        for (int qs = 0; qs < 2; qs++)
#pragma unroll
            for (int tq = 0; tq < 2; tq++) {
                const int tok = 8 * oc + 4 * qs + 2 * tq + u;
                if (tok < a.T) a.Y[(size_t)tok * a.ldy + row] = y[p][qs][tq];
            }
    }
}

}  // namespace

size_t draco_gemm_digit_bytes(int T, int n_in) {
    const size_t oct = (size_t)(T + 7) / 8;
    const size_t dig = oct * ((size_t)n_in / 32) * 1024 + oct * ((size_t)n_in / 256) * 32 +
                       oct * ((size_t)n_in / 32) * 32 + oct * ((size_t)n_in / 16) * 32 + 256;
    // the buffer also holds the f16 GEMM's activation operands (draco_enqueue_gemm)
    const size_t xh = draco_gemmh_x_bytes(T, n_in);
    return dig > xh ? dig : xh;
}

int draco_gemm_digits_launch(const float* X, int T, int n_in, uint8_t* buf, GemmArgs& a, hipStream_t st) {
    if (T < 1 || n_in % 256) return -1;
    const size_t oct = (size_t)(T + 7) / 8;
    a.xdig = reinterpret_cast<int8_t*>(buf);
    a.xsc = reinterpret_cast<float*>(buf + oct * ((size_t)n_in / 32) * 1024);
    a.xs32 = a.xsc + oct * ((size_t)n_in / 256) * 8;
    a.xs16 = a.xs32 + oct * ((size_t)n_in / 32) * 8;
    a.T = T;
    a.n_in = n_in;
    int8_t* xdig = reinterpret_cast<int8_t*>(buf);
    float* xsc = reinterpret_cast<float*>(buf + oct * ((size_t)n_in / 32) * 1024);
    float* xs32 = xsc + oct * ((size_t)n_in / 256) * 8;
    float* xs16 = xs32 + oct * ((size_t)n_in / 32) * 8;
    hipLaunchKernelGGL(k_gemm_digits, dim3(n_in / 256, (unsigned)(oct * 8)), dim3(64), 0, st, X, T, n_in, xdig, xsc,
                       xs32, xs16);
    return 0;
}

int draco_gemm_grouped_launch(GemmArgs& a, hipStream_t st) {
    constexpr int NW = 4, RP = 1;
    const int code = a.L.code;
    if (!a.groups || a.n_groups < 1 || a.max_oct < 1 || a.n_in != a.L.n_in) return -1;
    const int pairs = (a.L.n_out + 31) / 32;
    const dim3 grid((pairs + RP - 1) / RP, (a.max_oct + NW - 1) / NW, a.n_groups);
    if (code == DRACO_Q4_K) hipLaunchKernelGGL((k_gemm_q4<NW, RP>), grid, dim3(64 * NW), 0, st, a);
    else if (code == DRACO_Q6_K) hipLaunchKernelGGL((k_gemm_q6<NW, RP>), grid, dim3(64 * NW), 0, st, a);
    else return -1;
    return 0;
}

int draco_gemm_launch(GemmArgs& a, hipStream_t st) {
    constexpr int NW = 4, RP = 1;
    const int code = a.L.code;
    if (a.n_in != a.L.n_in || a.T < 1) return -1;
    const int pairs = (a.L.n_out + 31) / 32;
    const int oct = (a.T + 7) / 8;
    const dim3 grid((pairs + RP - 1) / RP, (oct + NW - 1) / NW);
    if (code == DRACO_Q4_K) hipLaunchKernelGGL((k_gemm_q4<NW, RP>), grid, dim3(64 * NW), 0, st, a);
    else if (code == DRACO_Q6_K) hipLaunchKernelGGL((k_gemm_q6<NW, RP>), grid, dim3(64 * NW), 0, st, a);
    else return -1;
    return 0;
}
