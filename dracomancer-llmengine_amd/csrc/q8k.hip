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
        int16_t* bs = reinterpret_cast<int16_t*>(out + (size_t)nv * n);
        if ((t & 15) == 0) bs[(size_t)(b * 16 + (t >> 4)) * nv + v] = (int16_t)s;
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
// GEMV image (q8 [NB][n_in], bsums [ng][NB], d [nb][NB]), which is the LDS
// layout itself, so the prologue is a flat 16-byte copy; otherwise the
// prologue scatters the Q8_K blocks into that layout.
template <int NW, int FM, int NB, bool ISUMS, bool IMG>
__global__ __launch_bounds__(64 * NW) void k_dq8(const Q8Launch a) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int NT = 64 * NW, NH = NB >= 4 ? NB / 4 : 1;
    const int n_in = a.n_in, nb = n_in >> 8, ng = n_in >> 4;
    const size_t img = (size_t)NB * nb * Q8K_BLOCK_BYTES;                   // image bytes
    int8_t* q8 = reinterpret_cast<int8_t*>(smem);                           // [NB][n_in]
    int16_t* bsum = reinterpret_cast<int16_t*>(q8 + (size_t)NB * n_in);     // [ng][NB]
    float* d8 = reinterpret_cast<float*>(bsum + (size_t)ng * NB);         // [nb][NB] (ng % 16 == 0: aligned)
    int8_t* zero = reinterpret_cast<int8_t*>(smem + ((img + 15) & ~(size_t)15));  // 1 KB of zeros
    float* red = reinterpret_cast<float*>(zero + 1024);                     // [NB][NW][16]

    const int tid = threadIdx.x, lane = tid & 63, j = lane & 15, g = lane >> 4;
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

    // prologue: Q8_K blocks -> LDS (q8 bytes, bsums, d)
    for (int i = tid; i < 256; i += NT) reinterpret_cast<uint32_t*>(zero)[i] = 0u;
    if (IMG) {
        const int n16 = (int)((img + 15) >> 4);
        const uint4* src = reinterpret_cast<const uint4*>(a.xq);
        uint4* dst = reinterpret_cast<uint4*>(smem);
        for (int i = tid; i < n16; i += NT) dst[i] = src[i];
    }
    const int ndw = IMG ? 0 : NB * nb * (Q8K_BLOCK_BYTES / 4);
    for (int i = tid; i < ndw; i += NT) {
        const int blk = i / (Q8K_BLOCK_BYTES / 4), k = i % (Q8K_BLOCK_BYTES / 4);
        const int v = blk / nb, b = blk % nb;
        const uint32_t val = reinterpret_cast<const uint32_t*>(a.xq)[i];
        if (k == 0) {
            d8[b * NB + v] = __builtin_bit_cast(float, val);
        } else if (k <= 64) {
            *reinterpret_cast<uint32_t*>(q8 + (size_t)v * n_in + b * 256 + 4 * (k - 1)) = val;
        } else {
            const int gi = b * 16 + 2 * (k - 65);
            bsum[(size_t)gi * NB + v] = (int16_t)(val & 0xFFFF);
            bsum[(size_t)(gi + 1) * NB + v] = (int16_t)(val >> 16);
        }
    }
    lds_barrier();

    // A rows: lane (j, g) supplies vector (4h + (j&3)) for group slot g when (j>>2) == g
    const bool arow = (j >> 2) == g && (NB > 1 || (j & 3) == 0);
    const int av = NB > 1 ? (j & 3) : 0;
    float yacc[NB];
#pragma unroll
    for (int v = 0; v < NB; v++) yacc[v] = 0.f;

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
            int isc[NB], imn[NB];
#pragma unroll
            for (int v = 0; v < NB; v++) isc[v] = imn[v] = 0;
            // one fragment = one group slot per lane; FM 1: 4 fragments (r, nib), FM 2: 4 (r)
#pragma unroll
            for (int fr = 0; fr < 4; fr++) {
                v4i B;
                int grp, sc, mn = 0;
                if (FM == 1) {
                    const int r = fr >> 1, nib = fr & 1, gh = g >> 1;
                    const uint4 q = r ? cur.b : cur.a;
                    const uint32_t m = nib ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
                    B = (v4i){(int)(q.x & m), (int)(q.y & m), (int)(q.z & m), (int)(q.w & m)};
                    grp = 8 * r + 4 * gh + 2 * nib + (g & 1);
                    const int s0 = 2 * gh + nib;
                    if (r == 0) {
                        sc = (cur.c.y >> (8 * s0)) & 63;
                        mn = (cur.c.z >> (8 * s0)) & 63;
                    } else {
                        sc = ((cur.c.w >> (8 * s0)) & 15) | (((cur.c.y >> (8 * s0 + 6)) & 3) << 4);
                        mn = ((cur.c.w >> (8 * s0 + 4)) & 15) | (((cur.c.z >> (8 * s0 + 6)) & 3) << 4);
                    }
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
                    grp = 8 * (g >> 1) + 2 * r + (g & 1);
                    sc = (int)(int8_t)(cur.sc >> (8 * r));
                }
                const int gg = cb * 16 + grp;  // this lane's group in the row
                // bsums of this group for the lane's output vectors
                int bs[NB];
#pragma unroll
                for (int v = 0; v < NB; v++) bs[v] = bsum[(size_t)gg * NB + v];
#pragma unroll
                for (int h = 0; h < NH; h++) {
                    const int8_t* ap = arow ? q8 + (size_t)(4 * h + av) * n_in + gg * 16 : zero;
                    const v4i C = __builtin_amdgcn_mfma_i32_16x16x64_i8(lds_v4i(ap), B, (v4i){0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                    for (int vv = 0; vv < (NB > 1 ? 4 : 1); vv++) {
                        const int v = NB > 1 ? 4 * h + vv : 0;
                        int t;
                        if (FM == 1) t = (fr & 1) ? (C[vv] + 128 * bs[v]) >> 4 : C[vv];
                        else t = C[vv] - 32 * bs[v];
                        isc[v] += sc * t;
                        if (FM == 1) imn[v] += mn * bs[v];
                    }
                }
            }
            const float dw = FM == 1 ? h2f((uint16_t)(cur.c.x & 0xFFFF)) : h2f((uint16_t)cur.d);
            const float dm = FM == 1 ? h2f((uint16_t)(cur.c.x >> 16)) : 0.f;
#pragma unroll
            for (int v = 0; v < NB; v++) {
                const float dx = d8[cb * NB + v];
                yacc[v] += (dx * dw) * (float)isc[v] - (dx * dm) * (float)imn[v];
            }
            if (ISUMS) {
                int s = isc[0], m = imn[0];
                s = rows_sum_i(s);
                m = rows_sum_i(m);
                const int row = (ct + a.tile0) * 16 + j;
                if (g == 0 && row >= a.row0 && row < a.row1) {
                    a.isc[(size_t)row * nb + cb] = s;
                    a.imn[(size_t)row * nb + cb] = m;
                }
            }
        }
        if (cp == ipt - 1) {  // tile done
#pragma unroll
            for (int v = 0; v < NB; v++) {
                float s = yacc[v];
                s = rows_sum(s);
                if (lane < 16) red[(v * NW + w) * 16 + j] = s;
                yacc[v] = 0.f;
            }
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

template <int NW, int FM, int NB, bool IS, bool IMG>
void launch_dq8i(const Q8Launch& a, int grid, size_t lds, hipStream_t st) {
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_dq8<NW, FM, NB, IS, IMG>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    });
    hipLaunchKernelGGL((k_dq8<NW, FM, NB, IS, IMG>), dim3(grid), dim3(64 * NW), lds, st, a);
}

template <int NW, int FM, int NB, bool IS>
void launch_dq8(const Q8Launch& a, int grid, size_t lds, hipStream_t st) {
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

int draco_gemv_q8k_launch(Q8Launch& a, int nvec, bool isums, hipStream_t st) {
    const int code = a.L.code;
    if (code != DRACO_Q4_K && code != DRACO_Q6_K) return -1;
    const int n_in = a.n_in;
    if (n_in != a.L.n_in || n_in % 256 || nvec < 1 || nvec > 8) return -1;
    if (a.row1 <= 0) a.row1 = a.L.n_out;
    if (a.row0 < 0 || a.row1 > a.L.n_out || a.row0 >= a.row1) return -1;
    a.tile0 = a.row0 / 16;
    a.n_tiles = (a.row1 + 15) / 16 - a.tile0;
    const int nb = n_in / 256, ng = n_in / 16;
    const int NBp = nvec == 1 ? 1 : (nvec <= 4 ? 4 : 8);
    if (NBp != nvec) {
        // vectors beyond nvec are read from the caller's buffer: require the padded count
        return -1;
    }
    if (a.img && isums) return -1;
    const int nw = nb >= 32 ? 16 : (nb >= 8 ? 8 : 4);
    const size_t img = (size_t)NBp * nb * Q8K_BLOCK_BYTES;  // = NBp * n_in + ng * NBp * 2 + nb * NBp * 4
    const size_t lds = ((img + 15) & ~(size_t)15) + 1024 + (size_t)NBp * nw * 16 * 4;
    (void)ng;
    if (lds > 160 * 1024) return -1;
    const int cap = cu_count() * (nw == 4 ? 4 : (nw == 8 ? 2 : 1));
    const int grid = a.n_tiles < cap ? a.n_tiles : cap;
    const int fm = code == DRACO_Q4_K ? 1 : 2;
    if (nw == 4) return fm == 1 ? launch_nb<4, 1>(a, nvec, isums, grid, lds, st) : launch_nb<4, 2>(a, nvec, isums, grid, lds, st);
    if (nw == 8) return fm == 1 ? launch_nb<8, 1>(a, nvec, isums, grid, lds, st) : launch_nb<8, 2>(a, nvec, isums, grid, lds, st);
    return fm == 1 ? launch_nb<16, 1>(a, nvec, isums, grid, lds, st) : launch_nb<16, 2>(a, nvec, isums, grid, lds, st);
}
