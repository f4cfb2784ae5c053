// gemmh.hip -- chunked-prefill GEMM on f16 MFMA (gfx950): Y[t][n] = x_t . W_n
// for Q4_K / Q6_K weights in the 16-row tile layout (formats.h).
//
// Exactness.  The weights enter the MFMA as f16 integers that carry their
// sub-block scale: Q4_K sc*q (<= 63*15 = 945), Q6_K sh*(q-32) and sl*(q-32)
// with sc = 8*sh + sl, sl in [0,7] (|values| <= 512); every one is an exact
// f16.  Per (token, 256-value super-block) the activations are scaled by
// 2^-e (e = ilogb(max|x|) - 14, so |x'| < 2^15) and split into two f16
// (hi = f16(x'), lo = f16(x' - hi)); x' - hi - lo is below 2^-22 |x'|.
// Every f16 x f16 product is exact in the MFMA's fp32 accumulation, so the
// result differs from the reference's fp32 row dot only by fp32 summation
// order and that 2^-22 representation step.  Per super-block and row:
//   Q4_K: y += 2^e * (d * sum_k (sc*q)_k x'_k - 32 * dmin * sum_sb m_sb S'_sb)
//         with S'_sb = 2^-5 * (sum of the sub-block's x'), itself on the MFMA
//         (K = 8 sub-blocks, hi/lo);
//   Q6_K: y += 2^e * d * (8 * sum (sh*(q-32)) x' + sum (sl*(q-32)) x').
//
// Operand order.  v_mfma_f32_32x32x16_f16: A lane l = row (token) l%32,
// K 8*(l/32)..+7; B lane l = column (weight row) l%32, same K; C lane l =
// column l%32, rows 8*(i/4) + 4*(l/32) + i%4.  The K order inside a
// super-block is the one the tile layout hands each lane: K-step s (0..15),
// lane half u supplies the 8 values 16*G + 8*(s&1) + i of group
// G = 8*(s>>3) + 2*((s>>1)&3) + u -- for Q4_K the low (s>>1 even) or high
// nibbles of quant vector (r = s>>3, gh = (s>>2)&1), for Q6_K fragment
// (s>>1)&3 of lane slot s>>3.  k_gemmh_x writes the activations in the same
// order, so one activation buffer serves both formats.
//
// Blocking.  Block = 4 waves on 32 tokens x 4*RW row tiles of 32 rows; the
// activation operands of one super-block (34944 B: 16 K-steps x hi/lo x 1 KB,
// the min-term operands, the 32 token scales) are staged in LDS, double
// buffered, and read by all four waves; each wave reads a K-step's A once and
// runs it against its RW row tiles (independent accumulator chains).  Weights stream from global memory (non-temporal loads).
// Tall-K products split K across blockIdx.z and a reduce kernel sums the
// partials in a fixed order.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "dev_common.h"
#include "formats.h"
#include "gemm.h"

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int XH_A = 16 * 2 * 64 * 16;          // A operands of one super-block (bytes)
constexpr int XH_M = 2 * 64 * 16;               // min-term A operands
constexpr int XH_SB = XH_A + XH_M + 32 * 4;     // + 32 token scales = 34944 B per (token tile, super-block)
constexpr int XH_V4 = XH_SB / 16;               // 2184 uint4 per super-block

// ------------------------------------------------------------ activations --
// Block (b, tt), 256 threads: thread (m = tid/8, sb = tid%8) owns the 32
// values of sub-block sb of token 32*tt + m in super-block b.
__global__ __launch_bounds__(256) void k_gemmh_x(const float* __restrict__ X, int T, int n_in,
                                                 uint8_t* __restrict__ xh) {
    const int b = blockIdx.x, tt = blockIdx.y, tid = threadIdx.x;
    const int m = tid >> 3, sb = tid & 7, t = 32 * tt + m, nb = n_in >> 8;
    float v[32];
    const float* src = X + (size_t)t * n_in + (size_t)b * 256 + 32 * sb;
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
        const float4 q = t < T ? ld4(src + i) : make_float4(0.f, 0.f, 0.f, 0.f);
        v[i] = q.x; v[i + 1] = q.y; v[i + 2] = q.z; v[i + 3] = q.w;
    }
    float am = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) am = fmaxf(am, fabsf(v[i]));
    am = group_max<8>(am);  // the token's 8 threads are consecutive lanes
    const int e = am > 0.f ? max(ilogbf(am) - 14, -100) : 0;
    const float sdown = __builtin_bit_cast(float, (uint32_t)(127 - e) << 23);  // 2^-e (e in [-100, 113])
    uint8_t* base = xh + ((size_t)tt * nb + b) * XH_SB;
    float ssum = 0.f;
#pragma unroll
    for (int gg = 0; gg < 2; gg++) {           // the two 16-value groups of this sub-block
        const int G = 2 * sb + gg, u = G & 1;
        const int lane = m + 32 * u;
#pragma unroll
        for (int bh = 0; bh < 2; bh++) {
            const int s = 8 * (G >> 3) + 2 * ((G >> 1) & 3) + bh;
            v8h hi, lo;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float xs = v[16 * gg + 8 * bh + i] * sdown;
                ssum += xs;
                const _Float16 h = (_Float16)xs;
                hi[i] = h;
                lo[i] = (_Float16)(xs - (float)h);
            }
            *reinterpret_cast<v8h*>(base + ((size_t)(2 * s) * 64 + lane) * 16) = hi;
            *reinterpret_cast<v8h*>(base + ((size_t)(2 * s + 1) * 64 + lane) * 16) = lo;
        }
    }
    // min-term operand: lane m (u = 0) holds S'_sb for sb = 0..7 in its 8 K slots;
    // lanes m + 32 (u = 1) hold zeros
    const float s5 = ssum * 0.03125f;
    const _Float16 sh = (_Float16)s5;
    const _Float16 sl = (_Float16)(s5 - (float)sh);
    _Float16* mh = reinterpret_cast<_Float16*>(base + XH_A);
    _Float16* ml = reinterpret_cast<_Float16*>(base + XH_A + 64 * 16);
    mh[m * 8 + sb] = sh;
    ml[m * 8 + sb] = sl;
    mh[(m + 32) * 8 + sb] = (_Float16)0.f;
    ml[(m + 32) * 8 + sb] = (_Float16)0.f;
    if (sb == 0) reinterpret_cast<float*>(base + XH_A + XH_M)[m] = __builtin_bit_cast(float, (uint32_t)(127 + e) << 23);
}

// f16 pairs of (bytes n0, n1) and (n2, n3) of w (each < 64) times c, exactly:
// the pair (1024 + n) is built by a byte permute, then fma((1024 + n), c, -1024 c)
// rounds once to the exact n*c (|n*c| <= 2048 by the callers' ranges)
__device__ __forceinline__ void nib2h(uint32_t w, v2h c2, v2h off2, uint32_t& p01, uint32_t& p23) {
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u);
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u);
    const v2h ha = __builtin_bit_cast(v2h, a), hb = __builtin_bit_cast(v2h, b);
    p01 = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(ha, c2, off2));
    p23 = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(hb, c2, off2));
}

__device__ __forceinline__ v8h pack8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(v8h, (v4u){a, b, c, d});
}

__device__ __forceinline__ v8h lds8(const uint8_t* p) { return *reinterpret_cast<const v8h*>(p); }

// stage super-block b's activation block into LDS (all 256 threads)
__device__ __forceinline__ void stage_load(const uint8_t* src, uint4 (&r)[9], int tid) {
#pragma unroll
    for (int k = 0; k < 9; k++) {
        const int i = tid + 256 * k;
        r[k] = i < XH_V4 ? *reinterpret_cast<const uint4*>(src + (size_t)i * 16) : make_uint4(0, 0, 0, 0);
    }
}
__device__ __forceinline__ void stage_store(uint8_t* dst, const uint4 (&r)[9], int tid) {
#pragma unroll
    for (int k = 0; k < 9; k++) {
        const int i = tid + 256 * k;
        if (i < XH_V4) *reinterpret_cast<uint4*>(dst + (size_t)i * 16) = r[k];
    }
}

// ------------------------------------------------------------------ GEMM --
// Raw weight registers of one (32-row tile, super-block) for lane (n, u).
template <int FM>
struct WFrag;
template <>
struct WFrag<1> {  // Q4_K: quant vectors (r, gh) = (v>>1, v&1), the row header
    uint4 qv[4], h;
};
template <>
struct WFrag<2> {  // Q6_K: ql A, ql B, qh and 4 scales of lane slots g2 = 0, 1; d
    uint4 qa[2], qb[2], qh[2];
    uint32_t sc4[2];
    uint32_t d;
};

__device__ __forceinline__ void wload(const uint8_t* item, int j, int u, WFrag<1>& f) {
#pragma unroll
    for (int v = 0; v < 4; v++) f.qv[v] = ldnt4(item + (v >> 1) * 1024 + 16 * (j + 16 * (2 * (v & 1) + u)));
    f.h = ldnt4(item + 2048 + 16 * j);
}
__device__ __forceinline__ void wload(const uint8_t* item, int j, int u, WFrag<2>& f) {
#pragma unroll
    for (int g2 = 0; g2 < 2; g2++) {
        const int ls = j + 16 * (2 * g2 + u);
        f.qa[g2] = ldnt4(item + 16 * ls);
        f.qb[g2] = ldnt4(item + 1024 + 16 * ls);
        f.qh[g2] = ldnt4(item + 2048 + 16 * ls);
        f.sc4[g2] = *reinterpret_cast<const uint32_t*>(item + 3072 + 4 * ls);
    }
    f.d = *reinterpret_cast<const uint16_t*>(item + 3328 + 2 * j);
}

// RW (32-row tile, super-block) items against the staged activations `cur`:
// each K-step reads its A operands (hi, lo) from LDS once and runs them
// against every tile's B, so the LDS traffic per MFMA falls with RW and the
// RW accumulator chains are independent.  Returns each tile's contribution
// before the token scale, per C element.
template <int RW>
__device__ __forceinline__ void tiles_q4(const WFrag<1> (&f)[RW], const uint8_t* cur, int lane, int u,
                                         float (&part)[RW][16]) {
    v16f P[RW], Q[RW];
    int sc[RW][8];
    v8h Bm[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) {
        P[r] = (v16f){};
        Q[r] = (v16f){};
        // 6-bit scales and mins of the 8 sub-blocks (src/m5_kern_scalar.c:39-46)
#pragma unroll
        for (int s8 = 0; s8 < 8; s8++) {
            int mn;
            if (s8 < 4) {
                sc[r][s8] = (f[r].h.y >> (8 * s8)) & 63;
                mn = (f[r].h.z >> (8 * s8)) & 63;
            } else {
                const int s0 = s8 - 4;
                sc[r][s8] = ((f[r].h.w >> (8 * s0)) & 15) | (((f[r].h.y >> (8 * s0 + 6)) & 3) << 4);
                mn = ((f[r].h.w >> (8 * s0 + 4)) & 15) | (((f[r].h.z >> (8 * s0 + 6)) & 3) << 4);
            }
            // min term: B lane (n, 0) = m_0..m_7 of row n, lanes (n, 1) zero
            Bm[r][s8] = u ? (_Float16)0.f : (_Float16)mn;
        }
    }
#pragma unroll
    for (int s = 0; s < 16; s++) {
        const int v = s >> 2, nib = (s >> 1) & 1, bh = s & 1;
        const int sbk = 4 * (s >> 3) + ((s >> 1) & 3);  // sub-block of this K-step
        const v8h Ahi = lds8(cur + ((size_t)(2 * s) * 64 + lane) * 16);
        const v8h Alo = lds8(cur + ((size_t)(2 * s + 1) * 64 + lane) * 16);
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const uint4 q = f[r].qv[v];
            uint32_t w0 = bh ? q.z : q.x, w1 = bh ? q.w : q.y;
            if (nib) {
                w0 = ((w0 >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;  // stored XOR 0x80: high nibble u ^ 8
                w1 = ((w1 >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;
            } else {
                w0 &= 0x0F0F0F0Fu;
                w1 &= 0x0F0F0F0Fu;
            }
            const _Float16 c = (_Float16)sc[r][sbk], o = (_Float16)(-1024.f * (float)sc[r][sbk]);
            uint32_t p0, p1, p2, p3;
            nib2h(w0, (v2h){c, c}, (v2h){o, o}, p0, p1);
            nib2h(w1, (v2h){c, c}, (v2h){o, o}, p2, p3);
            const v8h B = pack8(p0, p1, p2, p3);
            P[r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(Ahi, B, P[r], 0, 0, 0);
            P[r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(Alo, B, P[r], 0, 0, 0);
        }
    }
    const v8h Mhi = lds8(cur + XH_A + (size_t)lane * 16), Mlo = lds8(cur + XH_A + 1024 + (size_t)lane * 16);
#pragma unroll
    for (int r = 0; r < RW; r++) {
        Q[r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(Mhi, Bm[r], Q[r], 0, 0, 0);
        Q[r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(Mlo, Bm[r], Q[r], 0, 0, 0);
        const float dd = h2f((uint16_t)(f[r].h.x & 0xFFFF)), dm32 = -32.f * h2f((uint16_t)(f[r].h.x >> 16));
#pragma unroll
        for (int i = 0; i < 16; i++) part[r][i] = fmaf(dd, P[r][i], dm32 * Q[r][i]);
    }
}

template <int RW>
__device__ __forceinline__ void tiles_q6(const WFrag<2> (&f)[RW], const uint8_t* cur, int lane,
                                         float (&part)[RW][16]) {
    v16f P[RW], Q[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) {
        P[r] = (v16f){};
        Q[r] = (v16f){};
    }
#pragma unroll
    for (int s = 0; s < 16; s++) {
        const int g2 = s >> 3, r6 = (s >> 1) & 3, bh = s & 1;
        const v8h Ahi = lds8(cur + ((size_t)(2 * s) * 64 + lane) * 16);
        const v8h Alo = lds8(cur + ((size_t)(2 * s + 1) * 64 + lane) * 16);
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const uint4 A4 = f[r].qa[g2], B4 = f[r].qb[g2], H4 = f[r].qh[g2];
            uint32_t wq[2];
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int qd = 2 * bh + k;  // dword of the 16-byte vectors
                const uint32_t av = qd == 0 ? A4.x : (qd == 1 ? A4.y : (qd == 2 ? A4.z : A4.w));
                const uint32_t bv = qd == 0 ? B4.x : (qd == 1 ? B4.y : (qd == 2 ? B4.z : B4.w));
                const uint32_t hv = qd == 0 ? H4.x : (qd == 1 ? H4.y : (qd == 2 ? H4.z : H4.w));
                // the GGUF 6-bit map of src/m5_kern_scalar.c:115-142 (as the GEMV's dot_q6)
                if (r6 == 0) wq[k] = (av & 0x0F0F0F0Fu) | ((hv << 4) & 0x30303030u);
                else if (r6 == 1) wq[k] = (bv & 0x0F0F0F0Fu) | ((hv << 2) & 0x30303030u);
                else if (r6 == 2) wq[k] = ((av >> 4) & 0x0F0F0F0Fu) | (hv & 0x30303030u);
                else wq[k] = ((bv >> 4) & 0x0F0F0F0Fu) | ((hv >> 2) & 0x30303030u);
            }
            const int scv = (int)(int8_t)(f[r].sc4[g2] >> (8 * r6));
            const int shv = scv >> 3, slv = scv & 7;  // sc = 8*sh + sl
            const _Float16 ch = (_Float16)shv, cl = (_Float16)slv;
            const _Float16 oh = (_Float16)(-1056.f * (float)shv), ol = (_Float16)(-1056.f * (float)slv);
            uint32_t p0, p1, p2, p3;
            nib2h(wq[0], (v2h){ch, ch}, (v2h){oh, oh}, p0, p1);
            nib2h(wq[1], (v2h){ch, ch}, (v2h){oh, oh}, p2, p3);
            const v8h Bh = pack8(p0, p1, p2, p3);
            nib2h(wq[0], (v2h){cl, cl}, (v2h){ol, ol}, p0, p1);
            nib2h(wq[1], (v2h){cl, cl}, (v2h){ol, ol}, p2, p3);
            const v8h Bl = pack8(p0, p1, p2, p3);
            P[r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(Ahi, Bh, P[r], 0, 0, 0);
            P[r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(Alo, Bh, P[r], 0, 0, 0);
            Q[r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(Ahi, Bl, Q[r], 0, 0, 0);
            Q[r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(Alo, Bl, Q[r], 0, 0, 0);
        }
    }
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const float dd = h2f((uint16_t)f[r].d);
#pragma unroll
        for (int i = 0; i < 16; i++) part[r][i] = dd * fmaf(8.f, P[r][i], Q[r][i]);
    }
}

// FM 1 = Q4_K, 2 = Q6_K.  Grid (row blocks of 4*RW*32 rows, token tiles, K
// splits).  The next super-block's weights are loaded into registers while
// the current one is computed, as are its activations (then written to the
// other LDS buffer).
template <int FM, int RW>
__global__ __launch_bounds__(256) void k_gemmh(const GemmHArgs a) {
    extern __shared__ __align__(16) uint8_t sm[];  // [2][XH_SB]
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 31, u = lane >> 5, j = n & 15;
    const int tt = blockIdx.y, nb = a.n_in >> 8;
    const int per = (nb + gridDim.z - 1) / gridDim.z;
    const int b0 = blockIdx.z * per, b1 = min(nb, b0 + per);
    const int rt0 = (4 * blockIdx.x + w) * RW;  // this wave's first 32-row tile
    constexpr size_t IB = FM == 1 ? DRACO_Q4T_ITEM : DRACO_Q6T_ITEM;
    const uint8_t* xsrc = a.xh + (size_t)tt * nb * XH_SB;
    float y[RW][16];
    const uint8_t* wrow[RW];  // item 0 of each row tile (tile index clamped in bounds)
#pragma unroll
    for (int r = 0; r < RW; r++) {
#pragma unroll
        for (int i = 0; i < 16; i++) y[r][i] = 0.f;
        const int tile = min(2 * (rt0 + r) + (n >> 4), a.L.ntiles - 1);
        wrow[r] = a.W + (size_t)tile * nb * IB;
    }
    if (b0 >= b1) return;  // uniform per block (empty K split)

    WFrag<FM> wc[RW], wn[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) wload(wrow[r] + (size_t)b0 * IB, j, u, wc[r]);
    uint4 stg[9];
    stage_load(xsrc + (size_t)b0 * XH_SB, stg, tid);
    stage_store(sm, stg, tid);
    __syncthreads();
    for (int b = b0; b < b1; b++) {
        const uint8_t* cur = sm + (size_t)((b - b0) & 1) * XH_SB;
        uint8_t* nxt = sm + (size_t)((b - b0 + 1) & 1) * XH_SB;
        const int bn = b + 1 < b1 ? b + 1 : b;  // the last step reloads its own (cached) data
        stage_load(xsrc + (size_t)bn * XH_SB, stg, tid);
#pragma unroll
        for (int r = 0; r < RW; r++) wload(wrow[r] + (size_t)bn * IB, j, u, wn[r]);
        float4 ts4[4];  // token scales of this lane's C rows 8q + 4u .. +3
#pragma unroll
        for (int q = 0; q < 4; q++) ts4[q] = *reinterpret_cast<const float4*>(cur + XH_A + XH_M + 4 * (8 * q + 4 * u));
        if (32 * rt0 < a.L.n_out) {  // uniform per wave; no barrier inside.  Tiles past n_out
                                     // (clamped loads) are computed and not stored.
            float part[RW][16];
            if constexpr (FM == 1) tiles_q4<RW>(wc, cur, lane, u, part);
            else tiles_q6<RW>(wc, cur, lane, part);
#pragma unroll
            for (int r = 0; r < RW; r++)
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float4 t4 = ts4[i >> 2];
                    const float tsc = (i & 3) == 0 ? t4.x : ((i & 3) == 1 ? t4.y : ((i & 3) == 2 ? t4.z : t4.w));
                    y[r][i] = fmaf(tsc, part[r][i], y[r][i]);
                }
        }
#pragma unroll
        for (int r = 0; r < RW; r++) wc[r] = wn[r];
        if (b + 1 < b1) stage_store(nxt, stg, tid);
        __syncthreads();
    }
    float* out = gridDim.z > 1 ? a.part + (size_t)blockIdx.z * a.T * a.ldy : a.Y;
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const int row = 32 * (rt0 + r) + n;
        if (row >= a.L.n_out) continue;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int t = 32 * tt + 8 * (i >> 2) + 4 * u + (i & 3);
            if (t < a.T) out[(size_t)t * a.ldy + row] = y[r][i];
        }
    }
}

// Y[t][row] = sum_z part[z][t][row] (z in order)
__global__ __launch_bounds__(256) void k_gemmh_reduce(const float* __restrict__ part, float* __restrict__ Y, int T,
                                                      int n_out, int ldy, int nz) {
    const size_t n = (size_t)T * n_out;
    for (size_t i = blockIdx.x * (size_t)256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const int t = (int)(i / n_out), row = (int)(i % n_out);
        float s = 0.f;
        for (int z = 0; z < nz; z++) s += part[((size_t)z * T + t) * ldy + row];
        Y[(size_t)t * ldy + row] = s;
    }
}

template <int FM, int RW>
void launch_h(const GemmHArgs& a, dim3 grid, hipStream_t st) {
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemmh<FM, RW>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 2 * XH_SB);
        attr = true;
    }
    hipLaunchKernelGGL((k_gemmh<FM, RW>), grid, dim3(256), 2 * XH_SB, st, a);
}

}  // namespace

size_t draco_gemmh_x_bytes(int T, int n_in) { return (size_t)((T + 31) / 32) * (n_in / 256) * XH_SB + 256; }

int draco_gemmh_x_launch(const float* X, int T, int n_in, uint8_t* buf, hipStream_t st) {
    if (T < 1 || n_in % 256) return -1;
    hipLaunchKernelGGL(k_gemmh_x, dim3(n_in / 256, (T + 31) / 32), dim3(256), 0, st, X, T, n_in, buf);
    return 0;
}

// Row blocks of 256 rows (two tiles per wave, sharing each A read) for
// products of at least 64 row tiles over at least 4 token tiles, else 128
// rows; K split so that about 256 blocks run, each over at least 2
// super-blocks.  Measured on the configs[2] chunk (256 tokens): q / o 17.0 ->
// 15.4 us, down 55.5 -> 51 us with two tiles per wave; k / v (16 row tiles)
// slower with them, and so was the configs[4] prefill's 64-token chunk
// (9610 -> 9385 tok/s).  part: kspl * T * ldy floats (draco_gemmh_part_floats).
static void plan(const DracoLayout& L, int T, int& rw, int& kspl) {
    const int nb = L.n_in / 256, tiles32 = (L.n_out + 31) / 32, ntt = (T + 31) / 32;
    rw = tiles32 >= 64 && ntt >= 4 ? 2 : 1;
    const int blocks = ((tiles32 + 4 * rw - 1) / (4 * rw)) * ntt;
    kspl = 1;
    while (blocks * kspl * 2 <= 256 && nb / (kspl * 2) >= 2) kspl *= 2;
}

size_t draco_gemmh_part_floats(const DracoLayout& L, int T, int ldy) {
    int rw, kspl;
    plan(L, T, rw, kspl);
    return kspl > 1 ? (size_t)kspl * T * ldy : 0;
}

int draco_gemmh_launch(GemmHArgs& a, hipStream_t st) {
    if (a.L.code != DRACO_Q4_K && a.L.code != DRACO_Q6_K) return -1;
    if (a.n_in != a.L.n_in || a.T < 1 || a.n_in % 256) return -1;
    int rw, kspl;
    plan(a.L, a.T, rw, kspl);
    if (kspl > 1 && !a.part) return -1;
    const int tiles32 = (a.L.n_out + 31) / 32;
    const dim3 grid((tiles32 + 4 * rw - 1) / (4 * rw), (a.T + 31) / 32, kspl);
    if (a.L.code == DRACO_Q4_K) {
        if (rw == 2) launch_h<1, 2>(a, grid, st);
        else launch_h<1, 1>(a, grid, st);
    } else {
        if (rw == 2) launch_h<2, 2>(a, grid, st);
        else launch_h<2, 1>(a, grid, st);
    }
    if (kspl > 1) {
        const size_t n = (size_t)a.T * a.L.n_out;
        const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
        hipLaunchKernelGGL(k_gemmh_reduce, dim3(blocks), dim3(256), 0, st, a.part, a.Y, a.T, a.L.n_out, a.ldy, kspl);
    }
    return 0;
}
