// q8k.hip -- Q8_K activation quantizer and the Q4_K / Q6_K x Q8_K GEMV (gfx950).
//
// Q8_K block (256 values, 292 bytes): { float d; int8 qs[256]; int16 bsums[16] }.
// Quantizer semantics (llama.cpp b10819 quantize_row_q8_K_ref, restated in
// the oracle's or_quantize_q8k): m = the x of largest |x| (first index on
// ties), iscale = -127/m, q = min(127, round-half-even(iscale*x)),
// d = 1/iscale, bsums[i] = sum of q[16i..16i+15]; an all-zero block has d = 0.
// The GPU computes the same IEEE operations (correctly rounded division,
// unfused product), so the bytes are identical.
//
// GEMV: y[v][r] = sum_b (d8[v][b]*d) * isc - (d8[v][b]*dmin) * imn with the
// integer super-block sums of the oracle's or_q8k_block_isums:
//   Q4_K: isc = sum_j sc_j * sum_{k in j} q4*q8,  imn = sum_j m_j * (bsum_2j + bsum_2j+1)
//   Q6_K: isc = sum_g sc_g * sum_{k in g} (q6-32)*q8,  imn = 0
// The int8 MFMA (v_mfma_i32_16x16x64_i8) computes the per-16 group dots
// exactly: B holds the weight quants of 16 rows as in gemv.hip, A the q8
// bytes (block-diagonal: lane group g's 16 K values against A rows 4g..4g+3,
// which hold up to 4 activation vectors).  The Q4_K high nibble is stored as
// the signed byte 16*(u-8), so its dot is (C + 128*bsum) >> 4 (exact); the
// Q6_K dot is C - 32*bsum.  Integer sums are exact in any order; only the
// final fp32 combination over super-blocks is ordered differently from the
// oracle (a wave tree instead of a sequential loop).
#include <hip/hip_runtime.h>

#include <mutex>

#include "formats.h"
#include "q8k.h"
#include "tile_frag.h"

namespace {

// ------------------------------------------------------------ quantizer --
// grid (n/256, nvec), 256 threads: thread t owns value t of the block.
// IMG: the values go to the GEMV image (q8k.h) instead of the block.
template <bool IMG>
__global__ __launch_bounds__(256) void k_q8k_quantize(const float* __restrict__ x, int n, uint8_t* __restrict__ out) {
    __shared__ float wv[4];
    __shared__ int wi[4];
    __shared__ float mxs;
    const int b = blockIdx.x, v = blockIdx.y, t = threadIdx.x, lane = t & 63, w = t >> 6;
    const float xv = x[(size_t)v * n + (size_t)b * 256 + t];
    // first index of the largest |x|
    float ax = fabsf(xv);
    int idx = t;
    group_argmax<64>(ax, idx);
    if (lane == 0) {
        wv[w] = ax;
        wi[w] = idx;
    }
    __syncthreads();
    if (t == 0) {
        float ba = wv[0];
        int bi = wi[0];
        for (int k = 1; k < 4; k++)
            if (wv[k] > ba || (wv[k] == ba && wi[k] < bi)) {
                ba = wv[k];
                bi = wi[k];
            }
        mxs = ba > 0.f ? x[(size_t)v * n + (size_t)b * 256 + bi] : 0.f;
    }
    __syncthreads();
    const float mx = mxs;
    int q = 0;
    float d = 0.f;
    if (mx != 0.f) {
        const float iscale = -127.f / mx;
        q = (int)rintf(iscale * xv);
        q = q < 127 ? q : 127;
        d = 1.f / iscale;
    }
    const int s = group_reduce<16>(q, OpAdd{});
    if (IMG) {
        const int nv = gridDim.y;
        out[(size_t)v * n + (size_t)b * 256 + t] = (uint8_t)(int8_t)q;
        // group sums as f16 (|s| <= 16 * 127 < 2^11: exact), [block][vector][16]
        _Float16* bs = reinterpret_cast<_Float16*>(out + (size_t)nv * n);
        if ((t & 15) == 0) bs[((size_t)b * nv + v) * 16 + (t >> 4)] = (_Float16)s;
        float* dd = reinterpret_cast<float*>(bs + (size_t)(n / 16) * nv);
        if (t == 0) dd[(size_t)b * nv + v] = d;
        return;
    }
    uint8_t* blk = out + ((size_t)v * (n / 256) + b) * Q8K_BLOCK_BYTES;
    blk[4 + t] = (uint8_t)(int8_t)q;
    if ((t & 15) == 0) *reinterpret_cast<int16_t*>(blk + 260 + 2 * (t >> 4)) = (int16_t)s;
    if (t == 0) *reinterpret_cast<float*>(blk) = d;
}

// ----------------------------------------------------------------- GEMV --
// FM: 1 = Q4_K, 2 = Q6_K.  NB: activation vectors (1, 4 or 8).  ISUMS: also
// write each (row, super-block)'s integer sums (NB == 1).  IMG: xq is the
// GEMV image (q8 [NB][n_in], bsums [nb][NB][16] f16, d [nb][NB]), which is
// the LDS layout itself, so the prologue is a flat 16-byte copy; otherwise
// the prologue scatters the Q8_K blocks into that layout.  QX (NB == 1):
// a.xf is the fp32 vector and the prologue quantizes it into the image
// itself, with k_q8k_quantize's operations (so the bytes are the same):
// 32 threads per super-block, 8 consecutive values each; the first index of
// the largest |x| by am_merge within the thread and across the 32 lanes, the
// signed maximum from its lane by a sum of one non-zero term, the group sums
// of 16 values over two lanes.  One launch instead of two (the quantizer's
// launch and its dependency).
//
// Per item (16 rows x one super-block) and lane (row j, lane group g) the
// int8 MFMAs give the exact group dots C of the lane's four groups with every
// vector; a lane adds c * C per (group, vector) into I, where c is a small
// integer of the group's scale.  The terms that couple a weight scale with
// an activation group sum -- the Q4_K mins, the Q4_K high nibble's bias
// (the stored byte is 16(u - 8), so its C is 16 t - 128 bsum) and the Q6_K
// offset (C - 32 bsum) -- are one f16 MFMA each per super-block over the 16
// group sums of every vector (coefficients and sums are integers below 2^11,
// every partial sum below 2^24: exact in the fp32 accumulator):
//   Q4_K: 16 isc = I + 16 Tb, Tb = sum_{hi groups} 8 sc bsum, imn = Tm = sum m bsum
//         y += d8 (dw (I / 16 + Tb) - dmin Tm)
//   Q6_K: isc = I - 32 Tb, Tb = sum_g sc bsum,  y += d8 dw (I - 32 Tb)
// which are the oracle's or_q8k_block_isums regrouped (exact integers).  The
// f16 MFMA leaves vector 4g' + i's T in lane (j, g') element i; those are
// added to the row sums once per tile.
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t pk_h2(float a, float b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
}

template <int NW, int FM, int NB, bool ISUMS, bool IMG, bool QX = false>
__global__ __launch_bounds__(64 * NW) void k_dq8(const Q8Launch a) {
    static_assert(!QX || (NB == 1 && !IMG && !ISUMS), "the in-block quantizer serves one vector");
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int NT = 64 * NW, NH = NB >= 4 ? NB / 4 : 1;
    const int n_in = a.n_in, nb = n_in >> 8;
    const size_t img = (size_t)NB * nb * Q8K_BLOCK_BYTES;                   // image bytes
    int8_t* q8 = reinterpret_cast<int8_t*>(smem);                           // [NB][n_in]
    uint16_t* bsf = reinterpret_cast<uint16_t*>(q8 + (size_t)NB * n_in);    // [nb][NB][16] f16
    float* d8 = reinterpret_cast<float*>(bsf + (size_t)nb * NB * 16);      // [nb][NB]
    int8_t* zero = reinterpret_cast<int8_t*>(smem + ((img + 15) & ~(size_t)15));  // 1 KB of zeros
    float* red = reinterpret_cast<float*>(zero + 1024);                     // [NB][NW][16]

    const int tid = threadIdx.x, lane = tid & 63, j = lane & 15, g = lane >> 4, gh = g >> 1;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int bx = blockIdx.x, G = gridDim.x;
    const int total = a.n_tiles;
    const int ipt = (nb + NW - 1) / NW;
    const int my_tiles = bx < total ? (total - bx + G - 1) / G : 0;
    const int n_items = my_tiles * ipt;
    constexpr size_t IB = FM == 1 ? DRACO_Q4T_ITEM : DRACO_Q6T_ITEM;

    auto load = [&](int T, int b, Frag& f) {
        const uint8_t* p = a.base + ((size_t)(T + a.tile0) * nb + b) * IB;
        if (FM == 1) load_q4(p, lane, f);
        else load_q6(p, lane, f);
    };
    Frag P0, P1;
    int ct = bx, cb = w, cp = 0;
    load(ct < total ? ct : total - 1, cb < nb ? cb : nb - 1, P0);

    // prologue: Q8_K blocks -> LDS (q8 bytes, f16 bsums, d)
    for (int i = tid; i < 256; i += NT) reinterpret_cast<uint32_t*>(zero)[i] = 0u;
    if (IMG) {
        const int n16 = (int)((img + 15) >> 4);
        const uint4* src = reinterpret_cast<const uint4*>(a.xq);
        uint4* dst = reinterpret_cast<uint4*>(smem);
        for (int i = tid; i < n16; i += NT) dst[i] = src[i];
    }
    if constexpr (QX) {
        constexpr int SPP = NT / 32;                 // super-blocks per pass
        constexpr int MP = (64 + SPP - 1) / SPP;     // passes for rows of up to 64 super-blocks (16384 values)
        const int l32 = tid & 31;
        // every pass's x requested before the first wait (clamped super-block)
        float4 u[2 * MP];
#pragma unroll
        for (int p = 0; p < MP; p++) {
            if (p * SPP >= nb) break;  // uniform
            const int b = p * SPP + tid / 32, bc = b < nb ? b : nb - 1;
            const float* xp = a.xf + (size_t)bc * 256 + l32 * 8;
            u[2 * p] = ld4(xp);
            u[2 * p + 1] = ld4(xp + 4);
        }
#pragma unroll
        for (int p = 0; p < MP; p++) {
            if (p * SPP >= nb) break;
            const int b = p * SPP + tid / 32;  // whole half-waves past the end compute and discard
            const float4 u0 = u[2 * p], u1 = u[2 * p + 1];
            const float xv[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
            float ax = fabsf(xv[0]);
            int idx = l32 * 8;
#pragma unroll
            for (int k = 1; k < 8; k++) am_merge(ax, idx, fabsf(xv[k]), l32 * 8 + k);
            group_argmax<32>(ax, idx);
            float own = 0.f;  // the signed maximum, from the lane that holds it
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (idx == l32 * 8 + k) own = xv[k];
            const float sown = group_sum<32>(own);  // every lane of the group active
            const float mx = ax > 0.f ? sown : 0.f;
            int q[8];
            float d = 0.f;
#pragma unroll
            for (int k = 0; k < 8; k++) q[k] = 0;
            if (mx != 0.f) {
                const float iscale = -127.f / mx;
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const int qq = (int)rintf(iscale * xv[k]);
                    q[k] = qq < 127 ? qq : 127;
                }
                d = 1.f / iscale;
            }
            int part = 0;
#pragma unroll
            for (int k = 0; k < 8; k++) part += q[k];
            const int gs = part + dpp<DPP_XOR1>(part);  // the 16 values of lanes 2m, 2m + 1
            if (b < nb) {
                uint32_t p0 = 0, p1 = 0;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    p0 |= (uint32_t)(uint8_t)(int8_t)q[k] << (8 * k);
                    p1 |= (uint32_t)(uint8_t)(int8_t)q[4 + k] << (8 * k);
                }
                *reinterpret_cast<uint2*>(q8 + (size_t)b * 256 + l32 * 8) = make_uint2(p0, p1);
                if ((l32 & 1) == 0) bsf[(size_t)b * 16 + (l32 >> 1)] = __builtin_bit_cast(uint16_t, (_Float16)gs);
                if (l32 == 0) d8[b] = d;
            }
        }
    }
    const int ndw = (IMG || QX) ? 0 : NB * nb * (Q8K_BLOCK_BYTES / 4);
    for (int i = tid; i < ndw; i += NT) {
        const int blk = i / (Q8K_BLOCK_BYTES / 4), k = i % (Q8K_BLOCK_BYTES / 4);
        const int v = blk / nb, b = blk % nb;
        const uint32_t val = reinterpret_cast<const uint32_t*>(a.xq)[i];
        if (k == 0) {
            d8[b * NB + v] = __builtin_bit_cast(float, val);
        } else if (k <= 64) {
            *reinterpret_cast<uint32_t*>(q8 + (size_t)v * n_in + b * 256 + 4 * (k - 1)) = val;
        } else {
            const int gi = 2 * (k - 65);  // groups gi, gi + 1 of super-block b
            *reinterpret_cast<uint32_t*>(bsf + ((size_t)b * NB + v) * 16 + gi) =
                pk_h2((float)(int16_t)(val & 0xFFFF), (float)(int16_t)(val >> 16));
        }
    }
    lds_barrier();

    // int8 A rows.  Q6_K: lane (j, g) supplies vector (4h + (j&3)) for group
    // slot g when (j>>2) == g.  Q4_K: the two groups of a sub-block (one
    // scale) share a 32-value K slot: row 8k + v is vector v over slot k
    // (lane groups 2k, 2k + 1), so one MFMA serves 8 vectors and lane (j, g)
    // receives vectors 4(g&1) + i of the sub-block of its own slot g >> 1.
    const bool arow = FM == 1 ? ((j >> 3) == gh && (j & 7) < NB) : ((j >> 2) == g && (NB > 1 || (j & 3) == 0));
    const int av = FM == 1 ? (j & 7) : (NB > 1 ? (j & 3) : 0);
    // f16 A rows: lane (j, g) supplies vector j's group sums (vectors past NB: zeros)
    const bool brow = j < NB;
    // Q4_K: a lane accumulates its 4 vectors 4(g&1) + i (NV = min(NB, 4) of them)
    constexpr int NV = FM == 1 ? (NB < 4 ? NB : 4) : NB;
    const int vb = FM == 1 && NB > 4 ? 4 * (g & 1) : 0;  // first vector of a Q4_K lane
    float yacc[NV], yT[4];
#pragma unroll
    for (int v = 0; v < NV; v++) yacc[v] = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) yT[i] = 0.f;

    auto step = [&](int i, Frag& cur, Frag& nxt) {
        int nt = ct, nbk = cb + NW, np = cp + 1;
        if (np == ipt) {
            np = 0;
            nbk = w;
            nt = ct + G;
        }
        // a padding item (or the end) reloads this wave's first item of the
        // current tile, already fetched, so it costs no HBM traffic
        const bool real = i + 1 < n_items && nbk < nb;
        load(real ? nt : ct, real ? nbk : (w < nb ? w : nb - 1), nxt);
        if (cb < nb) {
            int I[NV];
#pragma unroll
            for (int v = 0; v < NV; v++) I[v] = 0;
            int scs[4], mns[4];
            // Q4_K A base of this item (fragment offsets are immediates; lanes
            // without a row read the zero page)
            const int8_t* ab = arow ? q8 + (size_t)av * n_in + cb * 256 + (4 * gh + (g & 1)) * 16 : zero;
            // one fragment = one group slot per lane; FM 1: 4 fragments (r, nib), FM 2: 4 (r)
#pragma unroll
            for (int fr = 0; fr < 4; fr++) {
                v4i B;
                int grp, cf;
                if (FM == 1) {
                    const int r = fr >> 1, nib = fr & 1;
                    const uint4 q = r ? cur.b : cur.a;
                    const uint32_t m = nib ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
                    B = (v4i){(int)(q.x & m), (int)(q.y & m), (int)(q.z & m), (int)(q.w & m)};
                    grp = 8 * r + 4 * gh + 2 * nib + (g & 1);
                    const int s0 = 2 * gh + nib;  // six-bit scale/min of sub-block 4r + s0
                    int sc, mn;
                    if (r == 0) {
                        sc = (cur.c.y >> (8 * s0)) & 63;
                        mn = (cur.c.z >> (8 * s0)) & 63;
                    } else {
                        sc = ((cur.c.w >> (8 * s0)) & 15) | (((cur.c.y >> (8 * s0 + 6)) & 3) << 4);
                        mn = ((cur.c.w >> (8 * s0 + 4)) & 15) | (((cur.c.z >> (8 * s0 + 6)) & 3) << 4);
                    }
                    scs[fr] = sc;
                    mns[fr] = mn;
                    cf = nib ? sc : 16 * sc;
                } else {
                    const int r = fr;
                    const uint32_t A4[4] = {cur.a.x, cur.a.y, cur.a.z, cur.a.w};
                    const uint32_t B4[4] = {cur.b.x, cur.b.y, cur.b.z, cur.b.w};
                    const uint32_t H4[4] = {cur.c.x, cur.c.y, cur.c.z, cur.c.w};
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        uint32_t vv;
                        if (r == 0) vv = (A4[q] & 0x0F0F0F0Fu) | ((H4[q] << 4) & 0x30303030u);
                        else if (r == 1) vv = (B4[q] & 0x0F0F0F0Fu) | ((H4[q] << 2) & 0x30303030u);
                        else if (r == 2) vv = ((A4[q] >> 4) & 0x0F0F0F0Fu) | (H4[q] & 0x30303030u);
                        else vv = ((B4[q] >> 4) & 0x0F0F0F0Fu) | ((H4[q] >> 2) & 0x30303030u);
                        B[q] = (int)vv;
                    }
                    grp = 8 * gh + 2 * r + (g & 1);
                    cf = (int)(int8_t)(cur.sc >> (8 * r));
                    scs[fr] = cf;
                    mns[fr] = 0;
                }
                // |C| < 2^19 and |cf| <= 1008: the full-rate 24-bit multiply is exact
                // (a 32-bit v_mul_lo is quarter rate)
                if (FM == 1) {
                    const int r = fr >> 1, nib = fr & 1;
                    const v4i C = __builtin_amdgcn_mfma_i32_16x16x64_i8(lds_v4i(ab + (8 * r + 2 * nib) * 16), B,
                                                                       (v4i){0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                    for (int vv = 0; vv < NV; vv++) I[vv] += __mul24(cf, C[vv]);
                } else {
                    const int gg = cb * 16 + grp;  // this lane's group in the row
#pragma unroll
                    for (int h = 0; h < NH; h++) {
                        const int8_t* ap = arow ? q8 + (size_t)(4 * h + av) * n_in + gg * 16 : zero;
                        const v4i C = __builtin_amdgcn_mfma_i32_16x16x64_i8(lds_v4i(ap), B, (v4i){0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                        for (int vv = 0; vv < (NB > 1 ? 4 : 1); vv++)
                            I[NB > 1 ? 4 * h + vv : 0] += __mul24(cf, C[vv]);
                    }
                }
            }
            // group-sum terms: lane (j, g) holds the scales of its fragments' groups
            const uint16_t* bsb = bsf + ((size_t)cb * NB + (brow ? j : 0)) * 16;
            v4f Tb, Tm = (v4f){0.f, 0.f, 0.f, 0.f};
            if (FM == 1) {
                // Tm: K slot 4g + e = group of the lane's sub-blocks (g 0: groups 0-3,
                // 1: 8-11, 2: 4-7, 3: 12-15); slots of g's pair share their scales
                const int gm = ((g & 1) ? 8 : 0) + 4 * gh;
                const int mlo = (g & 1) ? mns[2] : mns[0], mhi = (g & 1) ? mns[3] : mns[1];
                const uint2 bm = brow ? *reinterpret_cast<const uint2*>(bsb + gm) : make_uint2(0u, 0u);
                const uint32_t cm0 = pk_h2((float)mlo, (float)mlo), cm1 = pk_h2((float)mhi, (float)mhi);
                Tm = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(v4h, bm),
                                                             __builtin_bit_cast(v4h, make_uint2(cm0, cm1)), Tm, 0, 0, 0);
                // Tb: lanes of g 0 / 2 supply the high-nibble groups {2,3,10,11} + 4gh
                // with coefficient 8 sc; lanes of g 1 / 3 supply zeros
                const bool bl = (g & 1) == 0 && brow;
                const uint32_t b0 = bl ? *reinterpret_cast<const uint32_t*>(bsb + 4 * gh + 2) : 0u;
                const uint32_t b1 = bl ? *reinterpret_cast<const uint32_t*>(bsb + 4 * gh + 10) : 0u;
                const float c1 = (g & 1) ? 0.f : (float)(8 * scs[1]), c3 = (g & 1) ? 0.f : (float)(8 * scs[3]);
                Tb = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(v4h, make_uint2(b0, b1)),
                                                             __builtin_bit_cast(v4h, make_uint2(pk_h2(c1, c1), pk_h2(c3, c3))),
                                                             (v4f){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            } else {
                // Tb: K slot 4g + r = group 8gh + 2r + (g & 1), coefficient sc_r
                const uint4 bq = brow ? *reinterpret_cast<const uint4*>(bsb + 8 * gh) : make_uint4(0u, 0u, 0u, 0u);
                const uint32_t sel = (g & 1) ? 0x07060302u : 0x05040100u;  // odd / even halves of each dword pair
                const uint32_t a0 = __builtin_amdgcn_perm(bq.y, bq.x, sel), a1 = __builtin_amdgcn_perm(bq.w, bq.z, sel);
                Tb = __builtin_amdgcn_mfma_f32_16x16x16f16(
                    __builtin_bit_cast(v4h, make_uint2(a0, a1)),
                    __builtin_bit_cast(v4h, make_uint2(pk_h2((float)scs[0], (float)scs[1]), pk_h2((float)scs[2], (float)scs[3]))),
                    (v4f){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            }
            const float dw = FM == 1 ? h2f((uint16_t)(cur.c.x & 0xFFFF)) : h2f((uint16_t)cur.d);
            const float dm = FM == 1 ? h2f((uint16_t)(cur.c.x >> 16)) : 0.f;
            const float ds = FM == 1 ? dw * 0.0625f : dw;
#pragma unroll
            for (int v = 0; v < NV; v++) yacc[v] = fmaf(d8[cb * NB + vb + v] * ds, (float)I[v], yacc[v]);
            // T of vector 4g + i (lanes g >= NB / 4 hold zero rows)
            if (4 * g < NB) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    if (4 * g + e >= NB) break;
                    const float dx = d8[cb * NB + 4 * g + e];
                    const float t = FM == 1 ? dw * Tb[e] - dm * Tm[e] : -32.f * dw * Tb[e];
                    yT[e] = fmaf(dx, t, yT[e]);
                }
            }
            if (ISUMS) {
                // NB == 1: vector 0's T sits in the lanes of g 0
                int s = rows_sum_i(I[0]);
                const int row = (ct + a.tile0) * 16 + j;
                if (g == 0 && row >= a.row0 && row < a.row1) {
                    const int tb = (int)Tb[0], tm = (int)Tm[0];
                    a.isc[(size_t)row * nb + cb] = FM == 1 ? (s + 16 * tb) / 16 : s - 32 * tb;
                    a.imn[(size_t)row * nb + cb] = FM == 1 ? tm : 0;
                }
            }
        }
        if (cp == ipt - 1) {  // tile done
            if constexpr (FM == 1) {
                // lane (j, g) holds vectors 4(g&1) + i (its T terms too when g < 2);
                // lanes g and g ^ 2 hold the same vectors: one permlane32 swap per
                // pair of them leaves the lower lanes vectors vb + k, the upper
                // lanes vb + 2 + k, each summed over both lanes
                float h[4];
#pragma unroll
                for (int i = 0; i < 4; i++) h[i] = (i < NV ? yacc[i < NV ? i : 0] : 0.f) + (g < 2 ? yT[i] : 0.f);
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    const int b0 = __builtin_bit_cast(int, h[k]), b1 = __builtin_bit_cast(int, h[2 + k]);
                    const auto p = __builtin_amdgcn_permlane32_swap(b0, b1, false, false);
                    const float t = __builtin_bit_cast(float, (int)p[0]) + __builtin_bit_cast(float, (int)p[1]);
                    const int v = 4 * (g & 1) + (g >= 2 ? 2 : 0) + k;  // lanes of odd g hold vectors 4-7
                    if (v < NB) red[(v * NW + w) * 16 + j] = t;
                }
            } else {
#pragma unroll
                for (int v = 0; v < NB; v++) {
                    float s = (g == (v >> 2) ? yT[v & 3] : 0.f) + yacc[v];
                    s = rows_sum(s);
                    if (lane < 16) red[(v * NW + w) * 16 + j] = s;
                }
            }
#pragma unroll
            for (int v = 0; v < NV; v++) yacc[v] = 0.f;
#pragma unroll
            for (int e = 0; e < 4; e++) yT[e] = 0.f;
            lds_barrier();
            for (int o = tid; o < 16 * NB; o += NT) {
                const int v = o >> 4, jj = o & 15;
                float s = 0.f;
#pragma unroll
                for (int q = 0; q < NW; q++) s += red[(v * NW + q) * 16 + jj];
                const int row = (ct + a.tile0) * 16 + jj;
                if (row >= a.row0 && row < a.row1) a.y[(size_t)v * a.y_stride + row] = s;
            }
            lds_barrier();
        }
        ct = nt;
        cb = nbk;
        cp = np;
    };
    for (int i = 0; i < n_items; i += 2) {
        step(i, P0, P1);
        if (i + 1 >= n_items) break;
        step(i + 1, P1, P0);
    }
}

int cu_count() {
    static int n = 0;
    static std::once_flag once;
    std::call_once(once, [] {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
    });
    return n;
}

template <int NW, int FM, int NB, bool IS, bool IMG, bool QX = false>
void launch_dq8i(const Q8Launch& a, int grid, size_t lds, hipStream_t st) {
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_dq8<NW, FM, NB, IS, IMG, QX>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    });
    hipLaunchKernelGGL((k_dq8<NW, FM, NB, IS, IMG, QX>), dim3(grid), dim3(64 * NW), lds, st, a);
}

template <int NW, int FM, int NB, bool IS>
void launch_dq8(const Q8Launch& a, int grid, size_t lds, hipStream_t st) {
    if constexpr (NB == 1 && !IS) {
        if (a.xf) return launch_dq8i<NW, FM, 1, false, false, true>(a, grid, lds, st);
    }
    if (a.img && !IS) launch_dq8i<NW, FM, NB, false, true>(a, grid, lds, st);
    else launch_dq8i<NW, FM, NB, IS, false>(a, grid, lds, st);
}

template <int NW, int FM>
int launch_nb(const Q8Launch& a, int nb_vec, bool isums, int grid, size_t lds, hipStream_t st) {
    if (isums) {
        if (nb_vec != 1) return -1;
        launch_dq8<NW, FM, 1, true>(a, grid, lds, st);
    } else if (nb_vec == 1) {
        launch_dq8<NW, FM, 1, false>(a, grid, lds, st);
    } else if (nb_vec <= 4) {
        launch_dq8<NW, FM, 4, false>(a, grid, lds, st);
    } else if (nb_vec <= 8) {
        launch_dq8<NW, FM, 8, false>(a, grid, lds, st);
    } else {
        return -1;
    }
    return 0;
}

}  // namespace

int draco_q8k_quantize_launch(const float* x, int n, int nvec, uint8_t* out, hipStream_t st, bool image) {
    if (n <= 0 || n % 256 || nvec < 1) return -1;
    if (image) hipLaunchKernelGGL(k_q8k_quantize<true>, dim3(n / 256, nvec), dim3(256), 0, st, x, n, out);
    else hipLaunchKernelGGL(k_q8k_quantize<false>, dim3(n / 256, nvec), dim3(256), 0, st, x, n, out);
    return 0;
}

namespace {

// Waves per block and LDS bytes of a Q8_K GEMV over rows n_in wide for nvec
// vectors; -1 when no instance serves the request.
int q8k_shape(int code, int n_in, int nvec, bool img, bool isums, int* nw_out, size_t* lds_out) {
    if (code != DRACO_Q4_K && code != DRACO_Q6_K) return -1;
    // vectors beyond nvec would be read from the caller's buffer: only the
    // instance counts 1, 4 and 8 are served
    if (n_in <= 0 || n_in % 256 || (nvec != 1 && nvec != 4 && nvec != 8)) return -1;
    if (img && isums) return -1;
    const int nb = n_in / 256;
    // 16 waves for long rows unless that leaves padding items (a padding item
    // re-reads its wave's first item, which the non-temporal weight loads may
    // already have evicted: 56 super-blocks over 16 waves fetched 11% more
    // than the matrix); 8 waves divide 56
    const int nw = nb >= 32 && nb % 16 == 0 ? 16 : (nb >= 8 ? 8 : 4);
    const size_t image = (size_t)nvec * nb * Q8K_BLOCK_BYTES;  // = nvec * n_in + n_in / 16 * nvec * 2 + nb * nvec * 4
    const size_t lds = ((image + 15) & ~(size_t)15) + 1024 + (size_t)nvec * nw * 16 * 4;
    if (lds > 160 * 1024) return -1;
    *nw_out = nw;
    *lds_out = lds;
    return 0;
}

}  // namespace

int draco_gemv_q8k_shape_ok(int code, int n_in, int nvec, bool img, bool isums) {
    int nw;
    size_t lds;
    return q8k_shape(code, n_in, nvec, img, isums, &nw, &lds) == 0;
}

int draco_gemv_q8k_fused_ok(int code, int n_in) {
    int nw;
    size_t lds;
    return q8k_shape(code, n_in, 1, false, false, &nw, &lds) == 0 && n_in / 256 <= 2 * nw;
}

int draco_gemv_q8k_launch(Q8Launch& a, int nvec, bool isums, hipStream_t st) {
    const int code = a.L.code;
    const int n_in = a.n_in;
    int nw;
    size_t lds;
    if (n_in != a.L.n_in || q8k_shape(code, n_in, nvec, a.img, isums, &nw, &lds)) return -1;
    // the in-block quantizer: one vector, plain GEMV, one pass of the block's
    // half-waves over the row's super-blocks
    if (a.xf && (nvec != 1 || isums || a.img || n_in / 256 > 2 * nw)) return -1;
    if (a.row1 <= 0) a.row1 = a.L.n_out;
    if (a.row0 < 0 || a.row1 > a.L.n_out || a.row0 >= a.row1) return -1;
    a.tile0 = a.row0 / 16;
    a.n_tiles = (a.row1 + 15) / 16 - a.tile0;
    const int cap = cu_count() * (nw == 4 ? 4 : (nw == 8 ? 2 : 1));
    const int grid = a.n_tiles < cap ? a.n_tiles : cap;
    const int fm = code == DRACO_Q4_K ? 1 : 2;
    if (nw == 4) return fm == 1 ? launch_nb<4, 1>(a, nvec, isums, grid, lds, st) : launch_nb<4, 2>(a, nvec, isums, grid, lds, st);
    if (nw == 8) return fm == 1 ? launch_nb<8, 1>(a, nvec, isums, grid, lds, st) : launch_nb<8, 2>(a, nvec, isums, grid, lds, st);
    return fm == 1 ? launch_nb<16, 1>(a, nvec, isums, grid, lds, st) : launch_nb<16, 2>(a, nvec, isums, grid, lds, st);
}
