// gemv.hip -- GEMV over block-quantized weights with fp32 activations (gfx950).
//
//   y[r] = sum_k W[r][k] * x[k]
//
// Reference semantics: dot_row / m5_gemv_range, src/m5_kern_scalar.c:48-165
// (decoded weight w = d*sc*q - dmin*m for Q4_K, d*sc*(q-32) for Q6_K, d*q
// for Q8_0).  Summation orders differ from the reference's sequential loop,
// so results agree to fp32 rounding, not bitwise.
//
// Q4_K / Q6_K (k_dq): int8 MFMA on exact integer digits of x.
//   x is cut into groups of 16 values.  Group G gets a power-of-two scale
//   2^k, k = ilogb(max|x_G|) - 5, so |x|/2^k < 64, and X = rint(x*2^(21-k))
//   is an integer below 2^27 in magnitude: X = d0*2^21 + d1*2^14 + d2*2^7 + d3
//   with d0 in [-64,63] and d1..d3 in [0,127] -- four int8 digits, and
//   |x - X*2^(k-21)| <= 2^(k-22), below half an fp32 ulp of the group maximum.
//   One v_mfma_i32_16x16x64_i8 multiplies 16 weight rows (B: the raw 4- or
//   6-bit quants, lane (j, g) holding 16 K values of row j) by the digits
//   (A: block-diagonal, digit rows 4g..4g+3 non-zero only against lane group
//   g's K values).  Lane (j, g) receives the four exact int32 digit dots of
//   its (row, group); they fold to fp32 as (128*C0 + C1) + (128*C2 + C3)*2^-14
//   times 2^(k-7), and the block scales apply per group:
//     Q4_K: d*sc_j*(x.q) - dmin*m_j*(sum x)
//     Q6_K: d*sc*(x.q - 32*(sum x))
//   which is the reference's per-weight expression regrouped.
//   The device layout is the 16-row tile layout of formats.h, so each of a
//   lane's weight loads is one aligned 16-byte vector and every wave load
//   instruction reads 1 KB contiguously.  The Q4_K high nibble is read with
//   one AND thanks to the XOR 0x80 applied at repack: the byte then holds
//   16*(u-8), so x.u = C/16 + 8*(sum x).
//
//   Mapping: a block of NW waves owns one 16-row tile at a time (tiles of all
//   segments are numbered consecutively and visited grid-stride); wave w takes
//   super-blocks w, w+NW, ... of the tile; every wave runs the same number of
//   items per tile (padding items are skipped) so the per-tile reduction
//   barrier is uniform.  The next item's weights are loaded before the current
//   one is computed (two register buffers), and the first item's loads are in
//   flight while the prologue (RMSNorm + digits into LDS) runs.
//
// Q8_0 (k_seg): one wave owns SEG_R rows; fp32 VALU dot per 32-value block.
#include <hip/hip_runtime.h>

#include <mutex>

#include "dev_common.h"
#include "embed_dev.h"
#include "formats.h"
#include "gemv.h"
#include "tile_frag.h"

namespace {

constexpr int SEG_R = 2;                  // rows per wave in k_seg (Q8_0; 1 for wide rows without rope or norm)
constexpr int XP_MAXV = 4;                // float4s of x per thread held by the prologue

// ------------------------------------------------------- kernel arguments --
// What the kernels read of a SegLaunch, packed.  The launch cost on MI355X
// grows with the kernel-argument size (80 bytes of padding measured at +0.2 to
// +0.4 us per launch, same kernel code), so the host request -- four full
// layouts and fields only the host or the finalize launch needs -- is not
// passed as is.
// Field order: the kernels receive the first 14 dwords of the argument
// block in SGPRs (kernel-argument preloading), so what the prologue's first
// loads need comes first -- x, the norm weight, the pending accumulator, the
// row width and tile count, then segment 0's weight base, first tile and tile
// offset -- and those loads need no scalar load of an argument.
struct SegK {
    const uint8_t* base;  // K-quant tiles; Q8_0: the quants (layout off[0])
    int first;            // first global tile (K-quants) or first grid block (Q8_0)
    int tile0;
    int code, n_out;
    const uint8_t* aux;   // Q8_0: the fp16 scales (layout off[1])
    float* y;
    const float* yadd;
    int nb, epi;
    int row0, row1;
};

struct SegKArgs {
    const float* x;
    const float* norm_w;
    float* am_val;
    int n_in, total_tiles;
    int rot;  // also the split-K launches' tile count per half
    int nseg;
    SegK seg[SEG_MAX];
    float* xn_out;
    const float* rope_tab;
    const int* state;
    float* kc;
    float* vc;
    int* am_idx;
    int do_norm;
    float eps;
    int layer, head_dim, kv_dim;
    // row dots (SegLaunch.gdot_*): launches that carry them have no rope or
    // KV epilogue and no GNORM prologue, so their rows ride in rope_tab (w0)
    // and kc (w1) and the dots go to vc (the argument block stays 368 bytes)
    int gdot;
};

SegKArgs seg_kargs(const SegLaunch& a, bool q80) {
    SegKArgs k = {};
    for (int i = 0; i < SEG_MAX; i++) {
        const SegDesc& d = a.seg[i];
        SegK& o = k.seg[i];
        o.base = q80 && d.base ? d.base + d.L.off[0] : d.base;
        o.aux = q80 && d.base ? d.base + d.L.off[1] : nullptr;
        o.y = d.y;
        o.yadd = d.yadd;
        o.code = d.L.code;
        o.n_out = d.L.n_out;
        o.nb = d.L.nb;
        o.epi = d.epi;
        o.row0 = d.row0;
        o.row1 = d.row1;
        o.first = q80 ? d.first_block : d.first_tile;
        o.tile0 = d.tile0;
    }
    k.x = a.x;
    k.norm_w = a.norm_w;
    k.xn_out = a.xn_out;
    k.rope_tab = a.rope_tab;
    k.state = a.state;
    k.kc = a.kc;
    k.vc = a.vc;
    k.am_val = a.am_val;
    k.am_idx = a.am_idx;
    k.nseg = a.nseg;
    k.total_tiles = a.total_tiles;
    k.n_in = a.n_in;
    k.do_norm = a.do_norm;
    k.eps = a.eps;
    k.layer = a.layer;
    k.head_dim = a.head_dim;
    k.rot = a.rot;
    k.kv_dim = a.kv_dim;
    if (!q80 && a.gdot_done) {
        k.rope_tab = a.gdot_w0;
        k.kc = const_cast<float*>(a.gdot_w1);
        k.vc = a.gdot_out;
        k.gdot = a.gdot_n;
    }
    return k;
}

// ------------------------------------------------------------------ k_dq --
// Segment of global tile T.  Segment first tiles ascend; unused slots (and
// the "up" half of a SwiGLU pair) hold 1 << 30, so three comparisons against
// kernel-argument values (loaded once, kept in SGPRs) replace a loop.
__device__ __forceinline__ int seg_of_tile(const SegKArgs& a, int T) {
    return (T >= a.seg[1].first) + (T >= a.seg[2].first);  // k_dq launches have at most 3 segments
}

// Fields of segment si picked with selects over compile-time indices (no
// dynamic indexing into the kernel arguments, which costs a scalar load).
template <class F>
__device__ __forceinline__ auto seg_pick(const SegKArgs& a, int si, F f) -> decltype(f(a.seg[0])) {
    auto r = f(a.seg[0]);
    if (si == 1) r = f(a.seg[1]);
    if (si == 2) r = f(a.seg[2]);
    if (si == 3) r = f(a.seg[3]);
    return r;
}

// k_dq's pick: at most 3 segments (seg_launch_dq refuses more), so the
// fields of a fourth are never loaded
template <class F>
__device__ __forceinline__ auto seg_pick3(const SegKArgs& a, int si, F f) -> decltype(f(a.seg[0])) {
    auto r = f(a.seg[0]);
    if (si == 1) r = f(a.seg[1]);
    if (si == 2) r = f(a.seg[2]);
    return r;
}

// FM: 1 = Q4_K segments only, 2 = Q6_K only, 3 = both (per-tile switch),
// 4 = Q5_K only (Q5_K never shares a launch with the other formats).
// MULTI: more than one segment (a SwiGLU pair counts as one); without it the
// segment of every tile is 0 at compile time and its selection code is gone.
// EPI: the epilogue when it is fixed for the launch (single segment), or
// EPI_RT to read it from the tile's segment; EPI_QKV: the llama q/k/v launch
// (segments 0, 1, 2 = rope q, rope k + KV append, V append).  NORM: the
// launch's do_norm: 1 the RMSNorm prologue; 2 the GDN gated rms of 128-wide
// groups (x, already gated by the scan, scaled per group by rsqrt(sum of
// its 16 partial sums of squares / 128 + eps); see GNORM below); 3 the
// RMSNorm of a pending residual x + p0 + p1 (PRES below); 4 the same with
// the fused attention-merge + o projection's accumulator (PRES8 below: x +
// acc * 2^-32, acc int64 fixed point), one float4 of x per thread.
// KS: split-K launch (one EPI_STORE segment, no prologue norm): tiles
// [0, a.rot) multiply the first half of every row's super-blocks and store
// to y, tiles [a.rot, 2 a.rot) the second half and store to y + a.kv_dim.
// Per-wave timeline of the roofline launch (k_dq<8, 1, false, false, 0, 0,
// ...>: one Q4_K segment, fp32 x, no prologue norm), compiled only with
// -DDRACO_TIMELINE (build.py --timeline, timeline.py): lane 0 of each wave
// stores s_memrealtime stamps (100 MHz) at the wave's start, x digitised in
// LDS, after each of its first four items (the second and fourth end a tile,
// with its reduction and store) and the end, plus its XCC id, into g_tl.
// Product builds compile none of it.
#ifdef DRACO_TIMELINE
constexpr bool TL_BUILD = true;
__device__ unsigned long long g_tl[1024 * 16 * 8];
#else
constexpr bool TL_BUILD = false;
#endif
constexpr int EPI_RT = -1, EPI_QKV = -2;
// GD: the launch carries row dots (a.gdot, RMSNorm prologues only).
// The prologue's arguments come first, as scalars (agrid = the launch's
// grid size): the dispatcher preloads the first 14 argument dwords into
// SGPRs (a struct argument is never preloaded), so the first x and weight
// loads wait for no argument load.
template <int NW, int FM, bool DUAL, bool MULTI, int EPI, int NORM, bool IPT1, bool KS = false, bool GD = false>
__global__ __launch_bounds__(64 * NW) void k_dq(const float* __restrict__ ax, const float* __restrict__ anw,
                                                 float* __restrict__ aacc, int an_in, int atotal, int arot,
                                                 int agrid, const uint8_t* __restrict__ abase0, int afirst0,
                                                 int atile00, const SegKArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int NT = 64 * NW;
    const int n_in = an_in, nb = n_in >> 8, ng = n_in >> 4, n4 = n_in >> 2;
    int8_t* xd = reinterpret_cast<int8_t*>(smem);                           // [ng][4 digits][16]
    int8_t* zero = xd + (size_t)ng * 64;                                    // 1 KB of zeros
    float2* xsm = reinterpret_cast<float2*>(smem + (size_t)ng * 64 + 1024);  // [ng] (2^(k-7), sum x)
    float* red = reinterpret_cast<float*>(xsm + ng);                        // [2][NW][16]

    const int tid = threadIdx.x, lane = tid & 63, j = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    constexpr bool TSON = TL_BUILD && NW == 8 && FM == 1 && !DUAL && !MULTI && NORM == 0 && !KS && !GD && EPI == 0 &&
                          !IPT1;
    unsigned long long ts0 = 0, ts1 = 0, ts2 = 0, ts3 = 0, ts4 = 0, ts5 = 0;
    if (TSON) ts0 = __builtin_amdgcn_s_memrealtime();
    const int bx = blockIdx.x, G = agrid;
    const int total = atotal;
    const int ipt = IPT1 ? 1 : (KS ? (nb >> 1) / NW : (nb + NW - 1) / NW);  // IPT1: one item per wave and tile
    // KS: the half of tile T (0 or 1) and its first super-block
    auto khalf = [&](int T) { return KS && T >= arot ? 1 : 0; };
    auto kfirst = [&](int T) { return KS ? khalf(T) * (nb >> 1) : 0; };
    const int my_tiles = bx < total ? (total - bx + G - 1) / G : 0;
    const int n_items = my_tiles * ipt;

    // Item 0 of tile T (wave-uniform): base pointer(s) and format.  Items of
    // a tile are contiguous, super-block b at + b * item bytes.
    struct TileRef {
        const uint8_t* p;
        const uint8_t* p2;
        bool q4;
    };
    auto tile_ref = [&](int T) {
        if (KS) T -= khalf(T) * arot;
        const int si = MULTI ? seg_of_tile(a, T) : 0;
        const bool q4 = FM == 3 ? seg_pick3(a, si, [](const SegK& d) { return d.code; }) == DRACO_Q4_K : FM == 1;
        const size_t ib = FM == 4 ? DRACO_Q5T_ITEM : (q4 ? DRACO_Q4T_ITEM : DRACO_Q6T_ITEM);
        // segment 0's fields from the preloaded arguments
        const int tl = T - (si == 0 ? afirst0 : seg_pick3(a, si, [](const SegK& d) { return d.first; })) +
                       (si == 0 ? atile00 : seg_pick3(a, si, [](const SegK& d) { return d.tile0; }));
        const size_t off = (size_t)tl * nb * ib;
        TileRef r;
        r.p = (si == 0 ? abase0 : seg_pick3(a, si, [](const SegK& d) { return d.base; })) + off;
        r.p2 = DUAL ? seg_pick3(a, si + 1, [](const SegK& d) { return d.base; }) + off : r.p;
        r.q4 = q4;
        return r;
    };
    // Buffer loads for the K-quant items: with global loads the compiler
    // formed each item's 64-bit VGPR address in the loop and waited for every
    // load in flight (vmcnt(0)) before issuing the next item's, and a launch
    // mixing Q4_K and Q6_K tiles loaded under a per-tile branch, which
    // forced the same full waits (configs[2] decode 2438 -> 2520 tok/s,
    // configs[4] 1062 -> 1084 same-box).
    auto load_at = [&](const uint8_t* p, const uint8_t* p2, bool q4, Frag& f, Frag& f2) {
        if (FM == 4) load_q5(p, lane, f);
        else if (FM == 3) load_q46b(p, q4, lane, f);
        else if (q4) load_q4b(p, lane, f);
        else load_q6b(p, lane, f);
        if (DUAL) {
            if (FM == 4) load_q5(p2, lane, f2);
            else if (FM == 3) load_q46b(p2, q4, lane, f2);
            else if (q4) load_q4b(p2, lane, f2);
            else load_q6b(p2, lane, f2);
        }
    };

    // ---- prologue part 1: x (and norm weight) loads, then the first item's weights
    constexpr bool RMS = NORM == 1 || NORM == 3 || NORM == 4;  // the RMSNorm prologue
    constexpr int XPV = NORM == 4 ? 1 : XP_MAXV;               // float4s of x per thread
    float4 xv[XPV], wv[XPV];
    // NORM 4 (PRES8): the pending residual's int64 fixed-point accumulator at
    // aacc ([n_in] sums of round(2^32 p), then a flag at [n_in], set when
    // a contribution was not finite)
    longlong2 pq[NORM == 4 ? 2 : 1];
    long long pflag = 0;
    // NORM 2 (GNORM): the group partials [n_in / 128][64] (16 used), passed in
    // the preloaded aacc slot (the launch's a.kc; GNORM launches have no
    // accumulator)
    // NORM 3 (PRES): the pending residual's two split-K partials at aacc
    // ([2][n_in]); x = (x + p0) + p1, written to a.xn_out by block 0
    float4 pv0[NORM == 2 || NORM == 3 ? XP_MAXV : 1], pv1[NORM == 2 || NORM == 3 ? XP_MAXV : 1],
        pv2[NORM == 2 ? XP_MAXV : 1], pv3[NORM == 2 ? XP_MAXV : 1];
    // KS with one tile per block: the block multiplies one half of x only,
    // so only that half is loaded and digitised (chunks q of NT float4s;
    // chunk q holds super-blocks [q NW, q NW + NW), and NW divides the half)
    const bool kown = KS && G == total;
    const int kq_n = kown ? (nb >> 1) / NW : XPV, kq_lo = kown ? khalf(bx) * kq_n : 0;
#pragma unroll
    for (int q = 0; q < XPV; q++) {
        const int i4 = tid + q * NT;
        if (i4 < n4 && q >= kq_lo && q < kq_lo + kq_n) {
            xv[q] = ld4(ax + 4 * i4);
            if (RMS && anw) wv[q] = ld4(anw + 4 * i4);
            if constexpr (NORM == 4) {
                const longlong2* A = reinterpret_cast<const longlong2*>(aacc) + 2 * i4;
                pq[0] = A[0];
                pq[1] = A[1];
                pflag = reinterpret_cast<const long long*>(aacc)[n_in];
            }
            if constexpr (NORM == 3) {
                pv0[q] = ld4(aacc + 4 * i4);
                pv1[q] = ld4(aacc + n_in + 4 * i4);
            }
            if constexpr (NORM == 2) {
                const float* pp = aacc + ((4 * i4) >> 7) * 64;
                pv0[q] = ld4(pp);
                pv1[q] = ld4(pp + 4);
                pv2[q] = ld4(pp + 8);
                pv3[q] = ld4(pp + 12);
            }
        }
    }
    // row dots (GD): block G - 2 a.gdot + r dots row r of [w0; w1] with the
    // normalised x, up to 2 float4 per thread.  Every block loads (the other
    // blocks re-read row 0, an L2 hit): a load under a block-dependent
    // branch leaves the wait-count analysis no choice but to wait for it
    // before the first weights are used.
    static_assert(!GD || NORM == 1 || NORM == 3, "row dots ride on the RMSNorm prologue");
    static_assert(NORM != 4 || !KS, "PRES8 launches are not split-K");
    const int gr = GD ? bx - (G - 2 * a.gdot) : -1;
    float4 gv[2];
    if constexpr (GD) {
        const int r = gr >= 0 ? gr : 0;
        const float* row = r < a.gdot ? a.rope_tab + (size_t)r * n_in : a.kc + (size_t)(r - a.gdot) * n_in;
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int i4 = tid + q * NT;
            if (i4 < n4) gv[q] = ld4(row + 4 * i4);
        }
    }
    Frag P0, P1, Q0, Q1;
    // Load cursor (one item ahead of the compute cursor).  Loads are issued
    // unconditionally: a padding item or a load past the wave's last item
    // re-reads the last real item it loaded (already fetched or in flight,
    // so no HBM traffic) -- a skipped load would leave the wait-count
    // analysis no choice but vmcnt(0) before every use.
    int lt = bx < total ? bx : total - 1, lb = w + kfirst(lt), lp = 0, li = 0;
    TileRef lref = tile_ref(lt);
    const size_t lib = FM == 4 ? DRACO_Q5T_ITEM : (lref.q4 ? DRACO_Q4T_ITEM : DRACO_Q6T_ITEM);
    const uint8_t* lastp = lref.p + (size_t)(w < nb ? w : nb - 1) * lib;
    const uint8_t* lastp2 = lref.p2 + (size_t)(w < nb ? w : nb - 1) * lib;
    bool lastq4 = lref.q4;
    auto load_next = [&](Frag& f, Frag& f2) {
        if (li < n_items && lb < nb) {
            const size_t ib = FM == 4 ? DRACO_Q5T_ITEM : (lref.q4 ? DRACO_Q4T_ITEM : DRACO_Q6T_ITEM);
            lastp = lref.p + (size_t)lb * ib;
            lastp2 = lref.p2 + (size_t)lb * ib;
            lastq4 = lref.q4;
        }
        load_at(lastp, lastp2, lastq4, f, f2);
        li++;
        lp++;
        lb += NW;
        if (lp == ipt) {
            lp = 0;
            lt += G;
            lb = w + kfirst(lt);
            if (li < n_items) lref = tile_ref(lt);
        }
    };
    load_next(P0, Q0);
    // the zero page: written by the block before its barrier, or without the
    // barrier (no RMSNorm) by every wave for itself (identical values)
    if (RMS)
        for (int i = tid; i < 256; i += NT) reinterpret_cast<uint32_t*>(zero)[i] = 0u;
    else
        for (int i = lane; i < 256; i += 64) reinterpret_cast<uint32_t*>(zero)[i] = 0u;

    // ---- prologue part 2: digits into LDS, with the RMSNorm of
    // src/m6_engine.c:31-37 split in two: the digits are those of x*w, and
    // the scalar 1/rms (sum of squares reduced across waves through the same
    // barrier) multiplies each finished row dot in the epilogue.  One barrier
    // instead of two; the result differs from dotting (x*inv)*w only by fp32
    // rounding.
    float* ssp = red + 2 * NW * 16;  // [NW] per-wave sums of squares
    float* gsp = ssp + NW;           // [NW] per-wave row-dot partials
    float ss = 0.f, gp = 0.f;
#pragma unroll
    for (int q = 0; q < XPV; q++) {
        const int i4 = tid + q * NT;
        if (i4 >= n4) break;
        if (q < kq_lo || q >= kq_lo + kq_n) continue;
        float4 v = xv[q];
        if constexpr (NORM == 4) {
            constexpr float S = 2.3283064365386963e-10f;  // 2^-32
            if (pflag) {
                v.x = v.y = v.z = v.w = __builtin_nanf("");
            } else {
                v.x += (float)pq[0].x * S; v.y += (float)pq[0].y * S;
                v.z += (float)pq[1].x * S; v.w += (float)pq[1].y * S;
            }
            xv[q] = v;
            if (a.xn_out && bx == 0) *reinterpret_cast<float4*>(a.xn_out + 4 * i4) = v;
        }
        if constexpr (NORM == 3) {
            const float4 p = pv0[q], p2 = pv1[q];
            v.x = (v.x + p.x) + p2.x; v.y = (v.y + p.y) + p2.y; v.z = (v.z + p.z) + p2.z; v.w = (v.w + p.w) + p2.w;
            xv[q] = v;
            if (a.xn_out && bx == 0) *reinterpret_cast<float4*>(a.xn_out + 4 * i4) = v;
        }
        if constexpr (NORM == 2) {
            // GNORM (src/m6_layer.c:320-331): the group's 16 partial sums in
            // order (as k_gdn_gnorm), x = (o * norm_w * silu(z)) * rsqrt(.)
            const float4 p0 = pv0[q], p1 = pv1[q], p2 = pv2[q], p3 = pv3[q];
            float ms2 = 0.f;
            ms2 += p0.x; ms2 += p0.y; ms2 += p0.z; ms2 += p0.w;
            ms2 += p1.x; ms2 += p1.y; ms2 += p1.z; ms2 += p1.w;
            ms2 += p2.x; ms2 += p2.y; ms2 += p2.z; ms2 += p2.w;
            ms2 += p3.x; ms2 += p3.y; ms2 += p3.z; ms2 += p3.w;
            const float inv2 = 1.f / sqrtf(ms2 / 128.f + a.eps);
            v.x *= inv2; v.y *= inv2; v.z *= inv2; v.w *= inv2;
        }
        if (RMS) {
            ss = fmaf(v.x, v.x, ss);
            ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss);
            ss = fmaf(v.w, v.w, ss);
            if (anw) {
                const float4 nw = wv[q];
                v.x *= nw.x; v.y *= nw.y; v.z *= nw.z; v.w *= nw.w;
            }
            if (GD && q < 2) {
                const float4 r = gv[q < 2 ? q : 0];
                gp = fmaf(v.x, r.x, gp);
                gp = fmaf(v.y, r.y, gp);
                gp = fmaf(v.z, r.z, gp);
                gp = fmaf(v.w, r.w, gp);
            }
        }
        digits4(v, i4, xd, xsm);
    }
    if (TSON) ts1 = __builtin_amdgcn_s_memrealtime();
    if (RMS) {
        ss = wave_sum(ss);
        if (GD && gr >= 0) gp = wave_sum(gp);
        if (lane == 0) {
            ssp[w] = ss;
            if (GD) gsp[w] = gp;
        }
        lds_barrier();
    } else {
        // Wave w digitizes exactly the super-blocks it multiplies (float4 i4 =
        // tid + q * NT lies in super-block w + q * NW, and its items are
        // w, w + NW, ...), so without the RMSNorm no wave reads another
        // wave's LDS before the first tile reduction: its own writes are
        // ordered before its reads and the block barrier is skipped
        // (decode 1995 -> 2009 tok/s same-box; deferring 1/rms past the
        // barrier in the RMSNorm instances was slower, 2004 -> 1983).
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    }
    float inv = 1.f;
    if (RMS) {
        float tot = 0.f;
#pragma unroll
        for (int i = 0; i < NW; i++) tot += ssp[i];
        inv = 1.f / sqrtf(tot / (float)n_in + a.eps);
        if (GD && gr >= 0 && tid == 0) {
            float d = 0.f;
#pragma unroll
            for (int i = 0; i < NW; i++) d += gsp[i];
            a.vc[gr] = d * inv;
        }
        if (NORM == 1 && a.xn_out && bx == 0) {
#pragma unroll
            for (int q = 0; q < XPV; q++) {
                const int i4 = tid + q * NT;
                if (i4 >= n4) break;
                float4 v = xv[q];
                if (anw) {
                    const float4 nw = wv[q];
                    v.x = v.x * inv * nw.x; v.y = v.y * inv * nw.y; v.z = v.z * inv * nw.z; v.w = v.w * inv * nw.w;
                } else {
                    v.x *= inv; v.y *= inv; v.z *= inv; v.w *= inv;
                }
                *reinterpret_cast<float4*>(a.xn_out + 4 * i4) = v;
            }
        }
    }

    // this lane's A row: digit (j&3) of its group, non-zero only when (j>>2) == g
    const bool adig = (j >> 2) == g;
    const int gl4 = 4 * (g >> 1) + (g & 1), gl6 = 8 * (g >> 1) + (g & 1);
    float am_v = -INFINITY;
    int am_i = 0x7fffffff;
    float aD = 0.f, aM = 0.f, aD2 = 0.f, aM2 = 0.f;
    const int pos = a.state ? a.state[0] : 0;
    const int kv_row = a.state ? a.state[1 + a.layer] : 0;
    // compute cursor and the current tile's epilogue context (set at tile start)
    int ct = bx, cb = w + kfirst(bx), cp = 0;
    int c_epi = EPI_STORE, c_row = 0, c_r0 = 0, c_r1 = 0;
    float* c_y = nullptr;
    bool cq4 = FM != 2;
    float ep0 = 0.f, ep1 = 0.f;  // epilogue inputs, loaded at tile start (off the tile-end critical path)
    constexpr bool RB2 = !DUAL && !MULTI && EPI == EPI_STORE && !IPT1 && !KS;
    int rpar = 0;  // RB2: the half of red this tile's partials use

    auto step = [&](Frag& cur, Frag& nxt, Frag& cur2, Frag& nxt2) {
        if (cp == 0) {
            const int si = MULTI ? seg_of_tile(a, ct) : 0;
            if constexpr (EPI == EPI_QKV) c_epi = si == 0 ? EPI_ROPE_Q : (si == 1 ? EPI_ROPE_K : EPI_V_APPEND);
            else c_epi = EPI != EPI_RT ? EPI : seg_pick3(a, si, [](const SegK& d) { return d.epi; });
            c_row = (ct - khalf(ct) * arot - seg_pick3(a, si, [](const SegK& d) { return d.first; }) +
                     seg_pick3(a, si, [](const SegK& d) { return d.tile0; })) * 16;
            c_r0 = seg_pick3(a, si, [](const SegK& d) { return d.row0; });
            c_r1 = seg_pick3(a, si, [](const SegK& d) { return d.row1; });
            c_y = seg_pick3(a, si, [](const SegK& d) { return d.y; }) + (KS ? (size_t)khalf(ct) * a.kv_dim : 0);
            if (FM == 3) cq4 = seg_pick3(a, si, [](const SegK& d) { return d.code; }) == DRACO_Q4_K;
            if (tid < 16) {
                const int n_out = seg_pick3(a, si, [](const SegK& d) { return d.n_out; });
                const int row = c_row + tid;
                const int rr = row < n_out ? row : n_out - 1;
                const float* src = nullptr;
                if (c_epi == EPI_RESID) {
                    src = seg_pick3(a, si, [](const SegK& d) { return d.yadd; }) + rr;
                } else if ((c_epi == EPI_ROPE_Q || c_epi == EPI_ROPE_K) && rr % a.head_dim < arot) {
                    src = a.rope_tab + ((size_t)pos * (arot / 2) + (rr % a.head_dim) / 2) * 2;
                }
                const float2 e =
                    src ? make_float2(src[0], c_epi == EPI_RESID ? 0.f : src[1]) : make_float2(0.f, 0.f);
                ep0 = e.x;
                ep1 = e.y;
            }
        }
        load_next(nxt, nxt2);
        if (cb < nb) {
            float cD, cM, cD2 = 0.f, cM2 = 0.f;
            if constexpr (FM == 4) {
                const int8_t* xa = adig ? xd + (size_t)cb * 1024 + (gl4 * 4 + (j & 3)) * 16 : zero;
                const float2 r = dot_q5(cur, xa, xsm, cb * 16 + gl4, g);
                cD = r.x;
                cM = r.y;
                if (DUAL) {
                    const float2 r2 = dot_q5(cur2, xa, xsm, cb * 16 + gl4, g);
                    cD2 = r2.x;
                    cM2 = r2.y;
                }
            } else if (cq4) {
                const int8_t* xa = adig ? xd + (size_t)cb * 1024 + (gl4 * 4 + (j & 3)) * 16 : zero;
                const float2 r = dot_q4(cur, xa, xsm, cb * 16 + gl4, g);
                cD = r.x;
                cM = r.y;
                if (DUAL) {
                    const float2 r2 = dot_q4(cur2, xa, xsm, cb * 16 + gl4, g);
                    cD2 = r2.x;
                    cM2 = r2.y;
                }
            } else {
                const int8_t* xa = adig ? xd + (size_t)cb * 1024 + (gl6 * 4 + (j & 3)) * 16 : zero;
                cD = dot_q6(cur, xa, xsm, cb * 16 + gl6);
                cM = 0.f;
                if (DUAL) cD2 = dot_q6(cur2, xa, xsm, cb * 16 + gl6);
            }
            aD += cD;
            aM += cM;
            if (DUAL) {
                aD2 += cD2;
                aM2 += cM2;
            }
        }
        if (cp == ipt - 1) {  // tile done: reduce lanes (g) and waves, run the epilogue
            float acc = aD - aM, acc2 = aD2 - aM2;
            acc = rows_sum(acc);
            if (DUAL) acc2 = rows_sum(acc2);
            // RB2 (plain GEMV launches -- one store segment, several items per
            // wave, no split-K: the drop-in GEMV calls): the tiles alternate
            // between the two halves of red, so
            // the next tile's partials never overwrite the half wave 0 is
            // still summing: tile k + 2 reuses tile k's half only after tile
            // k + 1's barrier, which wave 0 reaches once tile k's epilogue is
            // done -- and the barrier after the epilogue goes (the 14336x4096
            // launch 7.7-8.1 -> 7.5-7.8 us same-box; configs[2]'s decode launches
            // measured 0.25-0.3% slower with it and keep the barrier)
            float* rb = RB2 ? red + rpar * NW * 16 : red;
            if (lane < 16) {
                rb[w * 16 + j] = acc;
                if (DUAL) red[(NW + w) * 16 + j] = acc2;
            }
            lds_barrier();
            if (tid < 16) {
                float v = 0.f, v2 = 0.f;
#pragma unroll
                for (int q = 0; q < NW; q++) {
                    v += rb[q * 16 + tid];
                    if (DUAL) v2 += red[(NW + q) * 16 + tid];
                }
                if (RMS) {
                    v *= inv;
                    v2 *= inv;
                }
                const int row = c_row + tid;
                const bool ok = row >= c_r0 && row < c_r1;
                switch (c_epi) {
                case EPI_STORE:
                    if (ok) c_y[row] = v;
                    break;
                case EPI_RESID:
                    if (ok) c_y[row] = ep0 + v;
                    break;
                case EPI_SWIGLU:
                    if (ok) c_y[row] = (v / (1.f + expf(-v))) * v2;
                    break;
                case EPI_ROPE_Q:
                case EPI_ROPE_K: {
                    // pairs (2i, 2i+1) of a head, src/m6_engine.c:134-143
                    const float pv = dpp<DPP_XOR1>(v);
                    float o = v;
                    if (row % a.head_dim < arot) {
                        const float c = ep0, sn = ep1;
                        o = (row & 1) ? pv * sn + v * c : v * c - pv * sn;
                    }
                    if (ok) {
                        if (c_epi == EPI_ROPE_Q) c_y[row] = o;
                        else a.kc[(size_t)kv_row * a.kv_dim + row] = o;
                    }
                    break;
                }
                case EPI_V_APPEND:
                    if (ok) a.vc[(size_t)kv_row * a.kv_dim + row] = v;
                    break;
                case EPI_ARGMAX: {
                    if (ok) c_y[row] = v;
                    float bv = ok ? v : -INFINITY;
                    int bi = ok ? row : 0x7fffffff;
                    group_argmax<16>(bv, bi);
                    am_merge(am_v, am_i, bv, bi);
                    break;
                }
                default:
                    break;
                }
            }
            if (!RB2) lds_barrier();
            rpar ^= 1;
            aD = aM = aD2 = aM2 = 0.f;
        }
        cp++;
        cb += NW;
        if (cp == ipt) {
            cp = 0;
            ct += G;
            cb = w + kfirst(ct);
        }
    };
    for (int i = 0; i < n_items; i += 2) {
        step(P0, P1, Q0, Q1);
        if (TSON) {
            const unsigned long long now = __builtin_amdgcn_s_memrealtime();
            if (i == 0) ts2 = now;
            if (i == 2) ts4 = now;
        }
        if (i + 1 >= n_items) break;
        step(P1, P0, Q1, Q0);
        if (TSON) {
            const unsigned long long now = __builtin_amdgcn_s_memrealtime();
            if (i == 0) ts3 = now;
            if (i == 2) ts5 = now;
        }
    }
    if ((EPI >= 0 ? EPI : (EPI == EPI_QKV ? EPI_ROPE_Q : a.seg[0].epi)) == EPI_ARGMAX && tid == 0) {
        aacc[bx] = am_v;
        a.am_idx[bx] = am_i;
    }
#ifdef DRACO_TIMELINE
    if (TSON) {
        const unsigned long long ts6 = __builtin_amdgcn_s_memrealtime();
        unsigned xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        if (lane == 0 && bx < 1024) {
            unsigned long long* o = g_tl + ((size_t)bx * NW + w) * 8;
            o[0] = ts0; o[1] = ts1; o[2] = ts2; o[3] = ts3; o[4] = ts4; o[5] = ts5; o[6] = ts6; o[7] = xcc;
        }
    }
#else
    (void)ts0; (void)ts1; (void)ts2; (void)ts3; (void)ts4; (void)ts5;
#endif
}

// ------------------------------------------------------------------ Q8_0 --
struct FQ80 {
    static constexpr int UPB = 1, NX = 32, NS = 1;
    __device__ static void xslice(const float* x, int u, float* xv, float* sx) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 a = ld4(x + u * 32 + 4 * i);
            xv[4 * i] = a.x; xv[4 * i + 1] = a.y; xv[4 * i + 2] = a.z; xv[4 * i + 3] = a.w;
        }
        sx[0] = 0.f;
    }
    struct W {  // one block's quants and scale
        uint4 q0, q1;
        uint16_t d;
    };
    __device__ static W load(const SegK& sg, int row, int u) {
        const size_t blk = (size_t)row * sg.nb + u;
        W w;
        w.q0 = ldnt4(sg.base + blk * 32);
        w.q1 = ldnt4(sg.base + blk * 32 + 16);
        w.d = *reinterpret_cast<const uint16_t*>(sg.aux + blk * 2);
        return w;
    }
    __device__ static float dotw(const W& w, const float* xv, const float* sx) {
        (void)sx;
        const uint32_t Q[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        float s = 0.f;
#pragma unroll
        for (int dw = 0; dw < 8; dw++)
#pragma unroll
            for (int k = 0; k < 4; k++) s = fmaf(sbyte_f(Q[dw], k), xv[4 * dw + k], s);
        return h2f(w.d) * s;
    }
};

// Fused segment kernel for Q8_0 (one instantiation per dual mode, preload
// depth NP, RMSNorm prologue and rows per wave R).  A wave owns R rows (2:
// the rope epilogue's pairs, and short rows fill the wave; 1 for rows wider
// than 32 blocks without rope, so each wave runs half the passes); its lanes cover (row, block)
// pairs p = i * U + u (U blocks per row) in passes of 64, so rows of fewer
// than 64 blocks still occupy every lane (SmolLM2's 960-wide rows are 30
// blocks: two rows per pass instead of 30 of 64 lanes).  Each lane adds its
// pair's dot to its row's accumulator in pass order, and the wave sums the
// lanes.  Latency: the weights of the first NP passes are requested first
// (pairs past the end re-read the last real pair, rows past the end the last
// row, so every load is unconditional and in bounds), then x with all of a
// thread's float4s in flight together, staged in LDS (RMS-normalised when
// do_norm) behind LDS-only barriers; one memory round trip before the first
// dot.  Passes beyond NP load one pass ahead.
// PEND (with NORM; rows of at most 4096 values): the input is x plus a
// pending residual held as 64-bit fixed point at a.am_val ([n_in] sums of
// round(2^32 p), then a flag at [n_in], set when a contribution was not
// finite: the input is then NaN), the fused attention merge + o projection's
// output; block 0 stores the sum (not normalised) to a.xn_out.
// The prologue's arguments come first, as scalars the dispatcher preloads
// into SGPRs (x, norm weight, pending accumulator, width, the first blocks
// of segments 1 and 2, segment 0's quants / scales / rows); the block's
// segment (at most 3) is picked branch-free from the preloaded first blocks
// (unused slots start at block 1 << 30), segment 0's blocks read no further
// argument before their first loads, and the other segments' fields go out
// together instead of one load per segment.
template <class F, bool DUAL, int NP, bool NORM, int R, bool PEND = false>
__global__ __launch_bounds__(256) void k_seg(const float* __restrict__ ax, const float* __restrict__ anw,
                                             float* __restrict__ aacc, int an_in, int afirst1,
                                             const uint8_t* __restrict__ abase0, const uint8_t* __restrict__ aaux0,
                                             int an_out0, int afirst2, const SegKArgs a) {
    extern __shared__ float xsh[];  // the block's x, n_in floats (normalised when do_norm)
    __shared__ float red[4];
    __shared__ float amv[4 * R];
    __shared__ int ami[4 * R];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int bx = blockIdx.x;
    // Q8_0 launches have at most 3 segments; a dual launch is one pair (segments 0 and 1)
    const int si = DUAL ? 0 : (bx >= afirst1) + (bx >= afirst2);
    SegK s, s2;
    if (si == 0) {  // wave-uniform: segment 0's blocks use the preloaded fields only
        s.base = abase0;
        s.aux = aaux0;
        s.n_out = an_out0;
        s.first = 0;
    } else {
        s.base = seg_pick(a, si, [](const SegK& d) { return d.base; });
        s.aux = seg_pick(a, si, [](const SegK& d) { return d.aux; });
        s.n_out = seg_pick(a, si, [](const SegK& d) { return d.n_out; });
        s.first = si == 1 ? afirst1 : afirst2;
    }
    s.nb = an_in / F::NX;  // the epilogue's fields are picked where they are used
    if (DUAL) {
        s2.base = a.seg[1].base;
        s2.aux = a.seg[1].aux;
        s2.nb = s.nb;
    } else {
        s2 = s;
    }
    const int r0 = (bx - s.first) * (4 * R) + wv * R;
    const int n_out = s.n_out, U = s.nb * F::UPB, npair = R * U, passes = (npair + 63) / 64;
    // pass k of this lane: row index i within the wave's rows, block u; live
    // when the pair exists and its row is in range
    auto pair = [&](int k, int& i, int& u) {
        const int p0 = lane + 64 * k;
        const int p = p0 < npair ? p0 : npair - 1;
        i = p / U;
        u = p - i * U;
        return p0 < npair && r0 + i < n_out;
    };
    auto row_of = [&](int i) { return r0 + i < n_out ? r0 + i : n_out - 1; };
    typename F::W wa[NP], wb[NP];

    // prologue: x into LDS, every block the same way.  With the RMSNorm the
    // block stages x * w and reduces the sum of squares of x through the same
    // LDS-only barrier; 1/rms multiplies every finished row dot (one barrier
    // instead of two; the result differs from dotting (x / rms) * w by fp32
    // rounding only).  The first XB float4s of every thread (n_in <= 4096)
    // are requested together and unconditionally (clamped index; a null norm
    // weight re-reads x), so the wait for them does not wait for the
    // weights; longer rows take further batches.
    const int n4 = an_in >> 2;
    constexpr int XB = 4;  // float4s per thread per batch
    const float* nwp = anw ? anw : ax;
    float4 xv[XB], nv[XB];
    longlong2 pa[PEND ? XB : 1], pb[PEND ? XB : 1];
    long long pflag = 0;
    if constexpr (PEND) pflag = load_flag(reinterpret_cast<const long long*>(aacc) + an_in);
#pragma unroll
    for (int q = 0; q < XB; q++) {
        const int i4 = tid + q * 256, ic = i4 < n4 ? i4 : n4 - 1;
        xv[q] = ld4(ax + 4 * ic);
        if (NORM) nv[q] = ld4(nwp + 4 * ic);
        if constexpr (PEND) {
            const longlong2* A = reinterpret_cast<const longlong2*>(aacc) + 2 * ic;
            pa[q] = A[0];
            pb[q] = A[1];
        }
    }
    // the weights after x, so x (needed first) returns first
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < NP; k++) {
        int i, u;
        pair(k, i, u);
        wa[k] = F::load(s, row_of(i), u);
    }
    if (DUAL) {
        // the pair's second half reads its pointers from the struct argument:
        // its loads follow the first half's and x's, which need no argument
        // load (the barrier only where the assembly shows it costs no register
        // copies of loads in flight: the pending-input prologue)
        if constexpr (PEND) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < NP; k++) {
            int i, u;
            pair(k, i, u);
            wb[k] = F::load(s2, row_of(i), u);
        }
    }
    if constexpr (PEND) {
#pragma unroll
        for (int q = 0; q < XB; q++) {
            const float4 v = fx_pending(xv[q], pa[q], pb[q], pflag != 0);
            xv[q] = v;
            if (a.xn_out && blockIdx.x == 0 && tid + q * 256 < n4)
                *reinterpret_cast<float4*>(a.xn_out + 4 * (tid + q * 256)) = v;
        }
    }
    float ss = 0.f;
    auto stage = [&](int i4, float4 v, const float4 w) {
        if (NORM) {
            ss = fmaf(v.x, v.x, ss);
            ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss);
            ss = fmaf(v.w, v.w, ss);
            if (anw) {
                v.x *= w.x; v.y *= w.y; v.z *= w.z; v.w *= w.w;
            }
        }
        *reinterpret_cast<float4*>(xsh + 4 * i4) = v;
    };
#pragma unroll
    for (int q = 0; q < XB; q++)
        if (tid + q * 256 < n4) stage(tid + q * 256, xv[q], nv[q]);
    for (int i4 = tid + XB * 256; i4 < n4; i4 += 256) stage(i4, ld4(ax + 4 * i4), NORM ? ld4(nwp + 4 * i4) : xv[0]);
    float inv = 1.f;
    if (NORM) {
        ss = wave_sum(ss);
        if (lane == 0) red[wv] = ss;
    }
    lds_barrier();  // LDS only: the weight loads above stay in flight
    if (NORM) {
        const float tot = (red[0] + red[1]) + (red[2] + red[3]);
        inv = 1.f / sqrtf(tot / (float)an_in + a.eps);
        if (!PEND && a.xn_out && blockIdx.x == 0) {  // the normalised x, (x / rms) * w as the reference
            auto put = [&](int i4, float4 v, const float4 w) {
                if (anw) {
                    v.x = v.x * inv * w.x; v.y = v.y * inv * w.y; v.z = v.z * inv * w.z; v.w = v.w * inv * w.w;
                } else {
                    v.x *= inv; v.y *= inv; v.z *= inv; v.w *= inv;
                }
                *reinterpret_cast<float4*>(a.xn_out + 4 * i4) = v;
            };
#pragma unroll
            for (int q = 0; q < XB; q++)
                if (tid + q * 256 < n4) put(tid + q * 256, xv[q], nv[q]);
            for (int i4 = tid + XB * 256; i4 < n4; i4 += 256) put(i4, ld4(ax + 4 * i4), ld4(nwp + 4 * i4));
        }
    }

    float acc[2 * R];
#pragma unroll
    for (int i = 0; i < 2 * R; i++) acc[i] = 0.f;
    auto dot_pass = [&](int k, const typename F::W& w, const typename F::W& w2) {
        int i, u;
        const bool live = pair(k, i, u);
        float xv[F::NX], sx[F::NS];
        F::xslice(xsh, u, xv, sx);
        const float d = F::dotw(w, xv, sx);
        const float d2 = DUAL ? F::dotw(w2, xv, sx) : 0.f;
#pragma unroll
        for (int r = 0; r < R; r++)
            if (live && r == i) {
                acc[r] += d;
                if (DUAL) acc[R + r] += d2;
            }
    };
#pragma unroll
    for (int k = 0; k < NP; k++)
        if (k < passes) dot_pass(k, wa[k], wb[k]);
    if (passes > NP) {
        typename F::W c = wa[0], c2 = wb[0];
        {
            int i, u;
            pair(NP, i, u);
            c = F::load(s, row_of(i), u);
            if (DUAL) c2 = F::load(s2, row_of(i), u);
        }
        for (int k = NP; k < passes; k++) {
            int i, u;
            pair(k + 1, i, u);  // clamped: past the last pass it re-reads a real pair
            const typename F::W n = F::load(s, row_of(i), u);
            const typename F::W n2 = DUAL ? F::load(s2, row_of(i), u) : n;
            dot_pass(k, c, c2);
            c = n;
            c2 = n2;
        }
    }
#pragma unroll
    for (int i = 0; i < (DUAL ? 2 : 1) * R; i++) acc[i] = wave_sum(acc[i]) * inv;

    s.epi = seg_pick(a, si, [](const SegK& d) { return d.epi; });
    s.y = seg_pick(a, si, [](const SegK& d) { return d.y; });
    s.yadd = seg_pick(a, si, [](const SegK& d) { return d.yadd; });
    switch (s.epi) {
    case EPI_STORE:
    case EPI_ARGMAX:
        if (lane == 0)
            for (int i = 0; i < R; i++)
                if (r0 + i < n_out) s.y[r0 + i] = acc[i];
        break;
    case EPI_RESID:
        if (lane == 0)
            for (int i = 0; i < R; i++)
                if (r0 + i < n_out) s.y[r0 + i] = s.yadd[r0 + i] + acc[i];
        break;
    case EPI_SWIGLU:
        if (lane == 0)
            for (int i = 0; i < R; i++)
                if (r0 + i < n_out) {
                    const float g = acc[i];
                    s.y[r0 + i] = (g / (1.f + expf(-g))) * acc[R + i];
                }
        break;
    case EPI_ROPE_Q:
    case EPI_ROPE_K:
        if (lane == 0) {
            // rows r0, r0+1 are one consecutive pair of a head (src/m6_engine.c:134-143)
            const int d = r0 % a.head_dim;
            float o0 = acc[0], o1 = acc[1];
            if (d < a.rot) {
                const int pos = a.state[0];
                const float* ang = a.rope_tab + ((size_t)pos * (a.rot / 2) + d / 2) * 2;
                const float c = ang[0], sn = ang[1];
                const float x0 = acc[0], x1 = acc[1];
                o0 = x0 * c - x1 * sn;
                o1 = x0 * sn + x1 * c;
            }
            if (s.epi == EPI_ROPE_Q) {
                if (r0 < n_out) s.y[r0] = o0;
                if (r0 + 1 < n_out) s.y[r0 + 1] = o1;
            } else {
                float* dst = a.kc + (size_t)a.state[1 + a.layer] * a.kv_dim;
                if (r0 < n_out) dst[r0] = o0;
                if (r0 + 1 < n_out) dst[r0 + 1] = o1;
            }
        }
        break;
    case EPI_V_APPEND:
        if (lane == 0) {
            float* dst = a.vc + (size_t)a.state[1 + a.layer] * a.kv_dim;
            for (int i = 0; i < R; i++)
                if (r0 + i < n_out) dst[r0 + i] = acc[i];
        }
        break;
    default:
        break;
    }

    if (s.epi != EPI_ARGMAX) return;
    // per-block argmax partial; k_argmax_finalize (next launch) reduces them
    if (lane == 0)
        for (int i = 0; i < R; i++) {
            amv[wv * R + i] = (r0 + i < n_out) ? acc[i] : -INFINITY;
            ami[wv * R + i] = (r0 + i < n_out) ? r0 + i : 0x7fffffff;
        }
    __syncthreads();
    if (tid == 0) {
        float v = amv[0];
        int idx = ami[0];
        for (int i = 1; i < 4 * R; i++) am_merge(v, idx, amv[i], ami[i]);
        const int bi = (int)blockIdx.x - s.first;
        aacc[bi] = v;
        a.am_idx[bi] = idx;
    }
}

// Persistent Q8_0 GEMV for long single-segment launches (the vocabulary
// head, store or argmax epilogue).  k_seg gives every block 8 rows, so the
// head's 6144 blocks each repeat the x prologue for 2 KB of weights per wave;
// here a block stages x (RMS-normalised when NORM) in LDS once and then takes
// row groups gi = blockIdx.x, + gridDim.x, ... of 4 waves x RPW rows.  A
// wave's lanes cover the (row, block) pairs p = lane + 64 k of its RPW rows
// (PASSES passes); the next group's weights are requested before the current
// group is dotted (loads clamped to real pairs, so they are unconditional and
// in bounds).  Row dots, the 1/rms scaling and the argmax merge are k_seg's.
template <int RPW, int PASSES, bool NORM>
__global__ __launch_bounds__(256) void k_seg_rows(const float* __restrict__ ax, const float* __restrict__ anw,
                                                  int an_in, int an_out0, const uint8_t* __restrict__ abase0,
                                                  const uint8_t* __restrict__ aaux0, float* __restrict__ ay0,
                                                  int aepi0, const SegKArgs a) {
    using F = FQ80;
    extern __shared__ float xsh[];
    __shared__ float red[4];
    __shared__ float amv[4];
    __shared__ int ami[4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    SegK s;  // the one segment, from the preloaded arguments
    s.base = abase0;
    s.aux = aaux0;
    s.n_out = an_out0;
    s.nb = an_in / F::NX;
    s.epi = aepi0;
    s.y = ay0;
    const int n_out = s.n_out, U = s.nb, npair = RPW * U;
    const int n_groups = (n_out + 4 * RPW - 1) / (4 * RPW);
    const bool argmax = s.epi == EPI_ARGMAX;
    auto load_group = [&](int gi, typename F::W (&w)[PASSES]) {
        const int r0 = gi * 4 * RPW + wv * RPW;
#pragma unroll
        for (int k = 0; k < PASSES; k++) {
            const int p0 = lane + 64 * k, p = p0 < npair ? p0 : npair - 1;
            const int i = p / U, u = p - i * U;
            w[k] = F::load(s, r0 + i < n_out ? r0 + i : n_out - 1, u);
        }
    };
    int gi = blockIdx.x;
    typename F::W cur[PASSES], nxt[PASSES];

    // prologue as k_seg's: x (times the norm weight) into LDS with the sum of
    // squares through one LDS-only barrier; x requested before the first
    // group's weights, so it returns first
    const int n4 = an_in >> 2;
    constexpr int XB = 4;
    const float* nwp = anw ? anw : ax;
    float4 xv[XB], nv[XB];
#pragma unroll
    for (int q = 0; q < XB; q++) {
        const int i4 = tid + q * 256, ic = i4 < n4 ? i4 : n4 - 1;
        xv[q] = ld4(ax + 4 * ic);
        if (NORM) nv[q] = ld4(nwp + 4 * ic);
    }
    __builtin_amdgcn_sched_barrier(0);
    load_group(gi < n_groups ? gi : n_groups - 1, cur);
    float ss = 0.f;
    auto stage = [&](int i4, float4 v, const float4 w) {
        if (NORM) {
            ss = fmaf(v.x, v.x, ss);
            ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss);
            ss = fmaf(v.w, v.w, ss);
            if (anw) {
                v.x *= w.x; v.y *= w.y; v.z *= w.z; v.w *= w.w;
            }
        }
        *reinterpret_cast<float4*>(xsh + 4 * i4) = v;
    };
#pragma unroll
    for (int q = 0; q < XB; q++)
        if (tid + q * 256 < n4) stage(tid + q * 256, xv[q], nv[q]);
    for (int i4 = tid + XB * 256; i4 < n4; i4 += 256) stage(i4, ld4(ax + 4 * i4), NORM ? ld4(nwp + 4 * i4) : xv[0]);
    float inv = 1.f;
    if (NORM) {
        ss = wave_sum(ss);
        if (lane == 0) red[wv] = ss;
    }
    lds_barrier();  // LDS only: the weight loads above stay in flight
    if (NORM) {
        const float tot = (red[0] + red[1]) + (red[2] + red[3]);
        inv = 1.f / sqrtf(tot / (float)an_in + a.eps);
        if (a.xn_out && blockIdx.x == 0) {  // the normalised x, (x / rms) * w as the reference
            for (int i4 = tid; i4 < n4; i4 += 256) {
                float4 v = ld4(ax + 4 * i4);
                if (anw) {
                    const float4 w = ld4(anw + 4 * i4);
                    v.x = v.x * inv * w.x; v.y = v.y * inv * w.y; v.z = v.z * inv * w.z; v.w = v.w * inv * w.w;
                } else {
                    v.x *= inv; v.y *= inv; v.z *= inv; v.w *= inv;
                }
                *reinterpret_cast<float4*>(a.xn_out + 4 * i4) = v;
            }
        }
    }

    float am_v = -INFINITY;
    int am_i = 0x7fffffff;
    for (; gi < n_groups; gi += gridDim.x) {
        const int gn = gi + (int)gridDim.x < n_groups ? gi + (int)gridDim.x : n_groups - 1;
        load_group(gn, nxt);  // the last group re-requests itself: in bounds, unused
        const int r0 = gi * 4 * RPW + wv * RPW;
        float acc[RPW];
#pragma unroll
        for (int r = 0; r < RPW; r++) acc[r] = 0.f;
#pragma unroll
        for (int k = 0; k < PASSES; k++) {
            const int p0 = lane + 64 * k, p = p0 < npair ? p0 : npair - 1;
            const int i = p / U, u = p - i * U;
            float xs[F::NX], sx[F::NS];
            F::xslice(xsh, u, xs, sx);
            const float d = F::dotw(cur[k], xs, sx);
#pragma unroll
            for (int r = 0; r < RPW; r++)
                if (p0 < npair && r == i) acc[r] += d;
        }
#pragma unroll
        for (int r = 0; r < RPW; r++) acc[r] = wave_sum(acc[r]) * inv;
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < RPW; r++)
                if (r0 + r < n_out) {
                    s.y[r0 + r] = acc[r];
                    am_merge(am_v, am_i, acc[r], r0 + r);
                }
        }
#pragma unroll
        for (int k = 0; k < PASSES; k++) cur[k] = nxt[k];
    }
    if (!argmax) return;
    if (lane == 0) {
        amv[wv] = am_v;
        ami[wv] = am_i;
    }
    __syncthreads();
    if (tid == 0) {
        float v = amv[0];
        int idx = ami[0];
        for (int i = 1; i < 4; i++) am_merge(v, idx, amv[i], ami[i]);
        a.am_val[blockIdx.x] = v;
        a.am_idx[blockIdx.x] = idx;
    }
}

// Reduce the head's per-block argmax partials (np.argmax semantics: first
// index of the maximum), write tokens[*cursor + 1] and advance the token
// state.  With emb_out set, also decode the new token's embedding row into
// emb_out (the next token's input), so generation needs no embedding launch.
// Runs after the head GEMV in stream order: one block, or with emb_out one
// block per 256 embedding values (at most 64).
__global__ __launch_bounds__(256) void k_argmax_finalize(const float* __restrict__ pv, const int* __restrict__ pi,
                                                         int nb, int* __restrict__ tokens, int* cursor,
                                                         int* state, int n_layer, const uint8_t* __restrict__ emb,
                                                         DracoLayout emb_L, float* __restrict__ emb_out) {
    __shared__ float sv[4];
    __shared__ int si[4];
    __shared__ int tok_s;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const bool lead = blockIdx.x == 0;
    // position and per-layer lengths advance in parallel, one entry per
    // thread (nothing in this launch reads them)
    if (state && lead)
        for (int i = tid; i <= n_layer; i += 256) state[i] += 1;
    const int cur = (lead && tid == 0 && cursor) ? cursor[0] : -1;
    // every block reduces the same partials in the same order (same winner);
    // block 0 records the token, every block decodes its slice of the next
    // token's embedding row
    float v = -INFINITY;
    int idx = 0x7fffffff;
    // the partials in batches of 8 per thread, each batch's loads issued
    // together (clamped index; the merge is order-independent: larger value,
    // then lower index)
    constexpr int MB = 8;
    for (int i0 = tid; i0 < nb; i0 += 256 * MB) {
        float bv[MB];
        int bi[MB];
#pragma unroll
        for (int k = 0; k < MB; k++) {
            const int i = i0 + 256 * k, ic = i < nb ? i : nb - 1;
            bv[k] = pv[ic];
            bi[k] = pi[ic];
        }
#pragma unroll
        for (int k = 0; k < MB; k++)
            if (i0 + 256 * k < nb) am_merge(v, idx, bv[k], bi[k]);
    }
    group_argmax<64>(v, idx);
    if (lane == 0) {
        sv[wv] = v;
        si[wv] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; w++) am_merge(v, idx, sv[w], si[w]);
        // no partial at all: token 0, never an out-of-range row (every real
        // value, -inf and NaN included, beats the padding's index)
        if (idx == 0x7fffffff) idx = 0;
        if (lead) {
            tokens[cur + 1] = idx;
            if (cursor) cursor[0] = cur + 1;
        }
        tok_s = idx;
    }
    if (!emb_out) return;
    __syncthreads();
    const int tok = tok_s;
    for (int p = blockIdx.x * 256 + tid; p < emb_L.n_in; p += gridDim.x * 256) emb_out[p] = embed_value(emb, emb_L, tok, p);
}

unsigned finalize_blocks(const float* emb_out, int n_in) {
    return emb_out ? (unsigned)((n_in + 255) / 256 < 64 ? (n_in + 255) / 256 : 64) : 1u;
}

// ------------------------------------------------------------ F32 / F16 --
template <int R, bool HALF>
__global__ __launch_bounds__(256) void k_gemv_plain(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                    float* __restrict__ y, const float* __restrict__ yadd,
                                                    int row0, int row1, int n_in) {
    const int lane = threadIdx.x & 63;
    const int r0 = row0 + (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * R;
    if (r0 >= row1) return;
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; i++) acc[i] = 0.f;
    for (int k = lane; k < n_in; k += 64) {
        const float xv = x[k];
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int r = r0 + i;
            if (r < row1) {
                float wv;
                if (HALF) wv = h2f(reinterpret_cast<const uint16_t*>(w)[(size_t)r * n_in + k]);
                else wv = reinterpret_cast<const float*>(w)[(size_t)r * n_in + k];
                acc[i] = fmaf(wv, xv, acc[i]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < R; i++) {
        const float s = wave_sum(acc[i]);
        const int r = r0 + i;
        if (lane == 0 && r < row1) y[r] = (yadd ? yadd[r] : 0.f) + s;
    }
}

}  // namespace

namespace {

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

size_t dq_lds_bytes(int n_in, int nw) { return (size_t)(n_in / 16) * 72 + 1024 + (size_t)2 * nw * 16 * 4 + (size_t)nw * 8; }

template <int NW, int FM, bool DUAL, bool MULTI, int EPI, int NORM, bool IPT1, bool KS = false, bool GD = false>
void launch_dq1(SegLaunch& a, int grid, hipStream_t st) {
    static std::once_flag once;
    std::call_once(once, [] {
        // allow LDS beyond 64 KB for long rows (n_in up to 16384 needs ~74 KB)
        (void)hipFuncSetAttribute(
            reinterpret_cast<const void*>(&k_dq<NW, FM, DUAL, MULTI, EPI, NORM, IPT1, KS, GD>),
            hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    });
    const SegKArgs k = seg_kargs(a, false);
    hipLaunchKernelGGL((k_dq<NW, FM, DUAL, MULTI, EPI, NORM, IPT1, KS, GD>), dim3(grid), dim3(64 * NW),
                       dq_lds_bytes(a.n_in, NW), st, k.x, k.norm_w, NORM == 2 ? k.kc : k.am_val, k.n_in,
                       k.total_tiles, k.rot, grid,
                       k.seg[0].base, k.seg[0].first, k.seg[0].tile0, k);
}

// launches carrying row dots: 8 waves, several store / residual segments
template <int FM, int NORM>
void launch_dq_gd1(SegLaunch& a, int grid, hipStream_t st) {
    if ((a.n_in >> 8) <= 8) launch_dq1<8, FM, false, true, EPI_RT, NORM, true, false, true>(a, grid, st);
    else launch_dq1<8, FM, false, true, EPI_RT, NORM, false, false, true>(a, grid, st);
}

template <int NORM>
void launch_dq_gd(SegLaunch& a, int fm, int grid, hipStream_t st) {
    if (fm == 1) launch_dq_gd1<1, NORM>(a, grid, st);
    else if (fm == 2) launch_dq_gd1<2, NORM>(a, grid, st);
    else launch_dq_gd1<3, NORM>(a, grid, st);
}

template <int NW, int FM, bool DUAL, bool MULTI, int EPI, int NORM>
void launch_dq(SegLaunch& a, int grid, hipStream_t st) {
    if ((a.n_in >> 8) <= NW) launch_dq1<NW, FM, DUAL, MULTI, EPI, NORM, true>(a, grid, st);
    else launch_dq1<NW, FM, DUAL, MULTI, EPI, NORM, false>(a, grid, st);
}

// single-segment launches get their epilogue at compile time (a SwiGLU pair
// is always one); the rest read it per tile
template <int NW, int FM, bool DUAL, int NORM>
void launch_dq_e(SegLaunch& a, bool multi, int grid, hipStream_t st) {
    if constexpr (DUAL) {
        launch_dq<NW, FM, true, false, EPI_SWIGLU, NORM>(a, grid, st);  // dual launches have exactly one pair
    } else {
        if (multi) launch_dq<NW, FM, false, true, EPI_RT, NORM>(a, grid, st);
        else if (a.seg[0].epi == EPI_STORE) launch_dq<NW, FM, false, false, EPI_STORE, NORM>(a, grid, st);
        else if (a.seg[0].epi == EPI_RESID) launch_dq<NW, FM, false, false, EPI_RESID, NORM>(a, grid, st);
        else if (a.seg[0].epi == EPI_ARGMAX) launch_dq<NW, FM, false, false, EPI_ARGMAX, NORM>(a, grid, st);
        else launch_dq<NW, FM, false, false, EPI_RT, NORM>(a, grid, st);
    }
}

template <int NW, int FM, bool DUAL>
void launch_dq_m(SegLaunch& a, bool multi, int grid, hipStream_t st) {
    if (a.do_norm == 2) {  // GNORM: one residual segment (checked by seg_launch_dq)
        if constexpr (!DUAL) launch_dq<NW, FM, false, false, EPI_RESID, 2>(a, grid, st);
    } else if (a.do_norm == 3) {  // PRES: per-tile epilogues, or the SwiGLU pair
        if constexpr (DUAL) launch_dq<NW, FM, true, false, EPI_SWIGLU, 3>(a, grid, st);
        else launch_dq<NW, FM, false, true, EPI_RT, 3>(a, grid, st);
    } else if (a.do_norm == 4) {  // PRES8: the SwiGLU pair (checked by draco_dq_shape)
        if constexpr (DUAL) launch_dq<NW, FM, true, false, EPI_SWIGLU, 4>(a, grid, st);
    } else if (a.do_norm) {
        launch_dq_e<NW, FM, DUAL, 1>(a, multi, grid, st);
    } else {
        launch_dq_e<NW, FM, DUAL, 0>(a, multi, grid, st);
    }
}

template <int NW>
void launch_dq_nw(SegLaunch& a, int fm, bool dual, int grid, hipStream_t st) {
    const bool multi = a.nseg > (dual ? 2 : 1);
    if (dual) {
        if (fm == 1) launch_dq_m<NW, 1, true>(a, multi, grid, st);
        else launch_dq_m<NW, 2, true>(a, multi, grid, st);
    } else if (fm == 1) {
        launch_dq_m<NW, 1, false>(a, multi, grid, st);
    } else if (fm == 2) {
        launch_dq_m<NW, 2, false>(a, multi, grid, st);
    } else {
        const bool qkv = a.nseg == 3 && a.seg[0].epi == EPI_ROPE_Q && a.seg[1].epi == EPI_ROPE_K &&
                         a.seg[2].epi == EPI_V_APPEND;
        if (qkv && a.do_norm == 3) launch_dq<NW, 3, false, true, EPI_QKV, 3>(a, grid, st);
        else if (a.do_norm == 3) launch_dq<NW, 3, false, true, EPI_RT, 3>(a, grid, st);
        else if (qkv && a.do_norm) launch_dq<NW, 3, false, true, EPI_QKV, 1>(a, grid, st);
        else if (a.do_norm) launch_dq<NW, 3, false, true, EPI_RT, 1>(a, grid, st);
        else launch_dq<NW, 3, false, true, EPI_RT, 0>(a, grid, st);
    }
}

// Q5_K launches: the SwiGLU pair or per-tile epilogues read at run time, the
// RMSNorm prologue or none (a smaller instance set than Q4_K / Q6_K's)
template <int NW>
void launch_dq_q5(SegLaunch& a, bool dual, int grid, hipStream_t st) {
    if (dual) {
        if (a.do_norm) launch_dq<NW, 4, true, false, EPI_SWIGLU, 1>(a, grid, st);
        else launch_dq<NW, 4, true, false, EPI_SWIGLU, 0>(a, grid, st);
    } else if (a.do_norm) {
        launch_dq<NW, 4, false, true, EPI_RT, 1>(a, grid, st);
    } else {
        launch_dq<NW, 4, false, true, EPI_RT, 0>(a, grid, st);
    }
}

// Q4_K / Q5_K / Q6_K segments: tile bookkeeping, instance choice, persistent grid.
int seg_launch_dq(SegLaunch& a, hipStream_t st) {
    const int n_in = a.n_in;
    if (n_in % 256 || n_in > 16384) return -1;
    const int nb = n_in / 256;
    int tiles = 0, fm = 0;
    bool dual = false;
    for (int i = 0; i < a.nseg; i++) {
        SegDesc& s = a.seg[i];
        if (s.row1 <= 0) s.row1 = s.L.n_out;
        if (s.row0 < 0 || s.row1 > s.L.n_out || s.row0 >= s.row1) return -1;
        fm |= s.L.code == DRACO_Q4_K ? 1 : (s.L.code == DRACO_Q6_K ? 2 : 4);
        s.tile0 = s.row0 / 16;
        s.first_tile = tiles;
        s.n_tiles = (s.row1 + 15) / 16 - s.tile0;
        if (s.epi == EPI_SWIGLU) {
            if (i + 1 >= a.nseg) return -1;
            SegDesc& u = a.seg[i + 1];
            if (u.L.code != s.L.code || u.L.n_out != s.L.n_out || u.L.n_in != n_in) return -1;
            u.row0 = s.row0;
            u.row1 = s.row1;
            u.tile0 = s.tile0;
            u.first_tile = 1 << 30;  // never selected: computed with its gate
            u.n_tiles = 0;
            dual = true;
            tiles += s.n_tiles;
            i++;
            continue;
        }
        if ((s.epi == EPI_ROPE_Q || s.epi == EPI_ROPE_K) && (a.head_dim & 1)) return -1;
        if (s.epi == EPI_ARGMAX && a.nseg != 1) return -1;
        tiles += s.n_tiles;
    }
    if (dual && (a.nseg != 2 || fm == 3)) return -1;
    // Q5_K: launches of Q5_K segments only, with the RMSNorm prologue or none
    // (its layers never take a split-K half, a pending residual or row dots)
    if ((fm & 4) && (fm != 4 || a.ksplit || a.do_norm > 1)) return -1;
    // GNORM prologue: one residual segment (a store segment when split-K) over whole 128-wide groups
    if (a.do_norm == 2 && (a.nseg != 1 || a.seg[0].epi != (a.ksplit ? EPI_STORE : EPI_RESID) || n_in % 128 || !a.kc))
        return -1;
    // PRES prologues: the partials of the pending residual
    if ((a.do_norm == 3 || a.do_norm == 4) && !a.am_val) return -1;
    // split-K: one whole-matrix store segment (the row widths and prologues
    // it serves are draco_dq_shape's to decide)
    if (a.ksplit) {
        const SegDesc& s0 = a.seg[0];
        if (a.nseg != 1 || s0.epi != EPI_STORE || s0.row0 != 0 || s0.row1 != s0.L.n_out) return -1;
    }
    // row dots: store / residual segments only, on a normalising launch
    int gd_n = 0;
    if (a.gdot_n > 0 && fm != 4 && !a.ksplit && !dual && a.nseg >= 2 && (a.do_norm == 1 || a.do_norm == 3) && a.gdot_w0 &&
        a.gdot_w1 && a.gdot_out) {
        bool ok = true;
        for (int i = 0; i < a.nseg; i++) ok = ok && (a.seg[i].epi == EPI_STORE || a.seg[i].epi == EPI_RESID);
        gd_n = ok ? a.gdot_n : 0;
    }
    DqShape sh;
    if (draco_dq_shape(n_in, tiles, dual, a.ksplit, a.do_norm, gd_n, cu_count(), sh)) return -1;
    for (int i = a.nseg; i < SEG_MAX; i++) {  // unused slots: never selected by seg_of_tile
        a.seg[i] = a.seg[a.nseg - 1];
        a.seg[i].first_tile = 1 << 30;
        a.seg[i].n_tiles = 0;
    }
    a.total_tiles = tiles;
    const int grid = sh.grid;
    if (a.nseg > 3) return -1;  // k_dq picks among 3 segments
    a.gdot_done = sh.gd;
    if (sh.ks) {
        // tiles [0, tiles) take each row's first half, [tiles, 2 tiles) the second
        a.rot = tiles;
        a.kv_dim = a.seg[0].L.n_out;
        a.total_tiles = 2 * tiles;
        if (sh.nw == 4) {
            if (fm == 1) launch_dq1<4, 1, false, false, EPI_STORE, 0, false, true>(a, grid, st);
            else launch_dq1<4, 2, false, false, EPI_STORE, 0, false, true>(a, grid, st);
        } else if (a.do_norm == 2) {
            if (fm == 1) launch_dq1<8, 1, false, false, EPI_STORE, 2, false, true>(a, grid, st);
            else launch_dq1<8, 2, false, false, EPI_STORE, 2, false, true>(a, grid, st);
        } else if (fm == 1) {
            launch_dq1<8, 1, false, false, EPI_STORE, 0, false, true>(a, grid, st);
        } else {
            launch_dq1<8, 2, false, false, EPI_STORE, 0, false, true>(a, grid, st);
        }
        return 0;
    }
    const int nw = sh.nw;
    if (grid <= 0) return 0;
    if (a.gdot_done) {
        if (a.do_norm == 3) launch_dq_gd<3>(a, fm, grid, st);
        else launch_dq_gd<1>(a, fm, grid, st);
        return 0;
    }
    if (fm == 4) {
        if (nw == 4) launch_dq_q5<4>(a, dual, grid, st);
        else if (nw == 8) launch_dq_q5<8>(a, dual, grid, st);
        else launch_dq_q5<16>(a, dual, grid, st);
    } else if (nw == 4) {
        launch_dq_nw<4>(a, fm, dual, grid, st);
    } else if (nw == 8) {
        launch_dq_nw<8>(a, fm, dual, grid, st);
    } else {
        launch_dq_nw<16>(a, fm, dual, grid, st);
    }
    if (a.seg[0].epi == EPI_ARGMAX)
        hipLaunchKernelGGL(k_argmax_finalize, dim3(finalize_blocks(a.emb_out, a.emb_L.n_in)), dim3(256), 0, st, a.am_val, a.am_idx, grid, a.tokens,
                           const_cast<int*>(a.cursor), a.advance_state, a.advance_layers, a.emb, a.emb_L,
                           a.emb_out);
    return 0;
}

template <bool DUAL, int NP, bool NORM, int R = SEG_R, bool PEND = false>
void launch_seg1(dim3 g, size_t shm, hipStream_t st, const SegKArgs& k) {
    static std::once_flag once;
    std::call_once(once, [] {
        // 128 KB of x (the kernel's static LDS and this stay below the CU's 160 KB)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_seg<FQ80, DUAL, NP, NORM, R, PEND>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024);
    });
    hipLaunchKernelGGL((k_seg<FQ80, DUAL, NP, NORM, R, PEND>), g, dim3(256), shm, st, k.x, k.norm_w, k.am_val, k.n_in,
                       k.seg[1].first, k.seg[0].base, k.seg[0].aux, k.seg[0].n_out, k.seg[2].first, k);
}

template <bool DUAL, int NP>
void launch_seg(dim3 g, size_t shm, hipStream_t st, const SegKArgs& k) {
    if (k.do_norm == 4) {  // the pending residual's fixed-point accumulator (SwiGLU pairs only)
        if constexpr (DUAL) launch_seg1<true, NP, true, SEG_R, true>(g, shm, st, k);
    } else if (k.do_norm) {
        launch_seg1<DUAL, NP, true>(g, shm, st, k);
    } else {
        launch_seg1<DUAL, NP, false>(g, shm, st, k);
    }
}

int g_seg_rows = 2;  // blocks per CU of the persistent Q8_0 head kernel; 0: k_seg

// Q8_0 segments (k_seg).
int seg_launch_q8(SegLaunch& a, hipStream_t st) {
    // one row per wave for rows wider than 32 blocks when no segment needs
    // the rope epilogue's row pairs and x is not normalised (the o and down
    // projections): twice the waves, half the passes each
    bool pairs = a.do_norm != 0;
    for (int i = 0; i < a.nseg; i++)
        pairs = pairs || a.seg[i].epi == EPI_SWIGLU || a.seg[i].epi == EPI_ROPE_Q || a.seg[i].epi == EPI_ROPE_K;
    const int R = !pairs && a.n_in > 1024 ? 1 : SEG_R;
    int blocks = 0;
    for (int i = 0; i < a.nseg; i++) {
        SegDesc& s = a.seg[i];
        if (s.row1 <= 0) s.row1 = s.L.n_out;
        if (s.row0 != 0 || s.row1 != s.L.n_out) return -1;  // row ranges go through draco_gemv_launch
        s.first_block = blocks;
        s.n_blocks = (s.L.n_out + 4 * R - 1) / (4 * R);
        if (s.epi == EPI_SWIGLU) {
            if (i + 1 >= a.nseg) return -1;
            const SegDesc& u = a.seg[i + 1];
            if (u.L.code != s.L.code || u.L.n_out != s.L.n_out) return -1;
            blocks += s.n_blocks;
            a.seg[i + 1].first_block = 1 << 30;  // never selected: computed with its gate
            a.seg[i + 1].n_blocks = 0;
            i++;
            continue;
        }
        if ((s.epi == EPI_ROPE_Q || s.epi == EPI_ROPE_K) && ((s.L.n_out & 1) || (a.head_dim & 1))) return -1;
        blocks += s.n_blocks;
    }
    bool dual = false;
    for (int i = 0; i < a.nseg; i++) dual = dual || a.seg[i].epi == EPI_SWIGLU;
    if (dual && a.nseg != 2) return -1;
    if (a.nseg > 3) return -1;  // k_seg picks among 3 segments
    for (int i = a.nseg; i < SEG_MAX; i++) a.seg[i].first_block = 1 << 30;  // never selected
    // the fixed-point pending residual: a SwiGLU pair whose rows fit one
    // batch of the prologue (4 float4s per thread), with its accumulator
    if (a.do_norm == 4 && (!dual || a.n_in > 4096 || !a.am_val)) return -1;
    if (a.do_norm == 2 || a.do_norm == 3) return -1;
    // x is staged in LDS: up to 32768 floats (128 KB, above the default 64 KB)
    if (a.n_in % 32 || a.n_in > 32768) return -1;
    const size_t shm = sizeof(float) * (size_t)a.n_in;
    const dim3 g(blocks), b(256);
    const SegKArgs k = seg_kargs(a, true);
    // passes of 64 (row, block) pairs per wave; the first NP preloaded
    const int passes = (R * (a.n_in / 32) + 63) / 64;
    // long single-segment launches (the head): the persistent row-group kernel
    const int n_out0 = a.seg[0].L.n_out;
    if (g_seg_rows > 0 && a.nseg == 1 && (a.seg[0].epi == EPI_STORE || a.seg[0].epi == EPI_ARGMAX) &&
        n_out0 >= 16384 && a.n_in <= 4096 && a.do_norm <= 1) {
        constexpr int RPW = 8;
        const int npair = RPW * (a.n_in / 32);
        const int n_groups = (n_out0 + 4 * RPW - 1) / (4 * RPW);
        const int grid = n_groups < 256 * g_seg_rows ? n_groups : 256 * g_seg_rows;
        const dim3 gr(grid);
        auto go = [&](void (*kern)(const float*, const float*, int, int, const uint8_t*, const uint8_t*, float*, int,
                                   SegKArgs)) {
            hipLaunchKernelGGL(kern, gr, dim3(256), shm, st, k.x, k.norm_w, k.n_in, k.seg[0].n_out, k.seg[0].base,
                               k.seg[0].aux, k.seg[0].y, k.seg[0].epi, k);
        };
        if (npair <= 128) {
            if (a.do_norm) go(k_seg_rows<RPW, 2, true>); else go(k_seg_rows<RPW, 2, false>);
        } else if (npair <= 256) {
            if (a.do_norm) go(k_seg_rows<RPW, 4, true>); else go(k_seg_rows<RPW, 4, false>);
        } else if (npair <= 512) {
            if (a.do_norm) go(k_seg_rows<RPW, 8, true>); else go(k_seg_rows<RPW, 8, false>);
        } else {
            goto plain;
        }
        if (a.seg[0].epi == EPI_ARGMAX)
            hipLaunchKernelGGL(k_argmax_finalize, dim3(finalize_blocks(a.emb_out, a.emb_L.n_in)), dim3(256), 0, st,
                               a.am_val, a.am_idx, grid, a.tokens, const_cast<int*>(a.cursor), a.advance_state,
                               a.advance_layers, a.emb, a.emb_L, a.emb_out);
        return 0;
    }
plain:
    if (R == 1) {
        if (passes <= 1) launch_seg1<false, 1, false, 1>(g, shm, st, k);
        else if (passes <= 2) launch_seg1<false, 2, false, 1>(g, shm, st, k);
        else launch_seg1<false, 4, false, 1>(g, shm, st, k);
    } else if (dual) {
        if (passes <= 1) launch_seg<true, 1>(g, shm, st, k);
        else launch_seg<true, 2>(g, shm, st, k);
    } else {
        if (passes <= 1) launch_seg<false, 1>(g, shm, st, k);
        else if (passes <= 2) launch_seg<false, 2>(g, shm, st, k);
        else launch_seg<false, 4>(g, shm, st, k);
    }
    if (a.seg[0].epi == EPI_ARGMAX)
        hipLaunchKernelGGL(k_argmax_finalize, dim3(finalize_blocks(a.emb_out, a.emb_L.n_in)), dim3(256), 0, st, a.am_val, a.am_idx, a.seg[0].n_blocks,
                           a.tokens, const_cast<int*>(a.cursor), a.advance_state, a.advance_layers, a.emb, a.emb_L,
                           a.emb_out);
    return 0;
}

}  // namespace

#ifdef DRACO_TIMELINE
// Timeline builds only: copy out / clear the stamps of the last roofline launch.
extern "C" int draco_timeline_read(unsigned long long* host) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_tl), sizeof(unsigned long long) * 1024 * 16 * 8) == hipSuccess
               ? 0 : -1;
}
extern "C" int draco_timeline_clear() {
    static unsigned long long z[1024 * 16 * 8];
    return hipMemcpyToSymbol(HIP_SYMBOL(g_tl), z, sizeof(z)) == hipSuccess ? 0 : -1;
}
#endif

extern "C" int draco_set_seg_rows(int n) {
    const int old = g_seg_rows;
    if (n >= 0 && n <= 8) g_seg_rows = n;
    return old;
}

int draco_dq_ksplit_waves(int n_in, int do_norm) {
    if (n_in <= 0 || n_in % 512) return 0;
    const int nb = n_in / 256, half = nb / 2;
    if (nb < 8 || nb > 32) return 0;
    // the split-K instances: 8 waves (prologue none or GNORM), 4 waves (none).
    // A half splits into whole items per wave, and with one tile per block
    // (kown) chunk q of the prologue holds super-blocks [q nw, q nw + nw), so
    // the second half's last chunk nb / nw - 1 must lie below XP_MAXV.
    if (half % 8 == 0 && nb <= XP_MAXV * 8) return 8;
    if (do_norm == 0 && half % 4 == 0 && nb <= XP_MAXV * 4) return 4;
    return 0;
}

int draco_dq_shape(int n_in, int tiles, bool dual, int ksplit, int do_norm, int gd_n, int cus, DqShape& s) {
    s = DqShape{};
    // the PRES8 prologue (do_norm 4) holds one float4 of x per thread
    const int xp = do_norm == 4 ? 1 : XP_MAXV;
    s.xp_max = xp;
    if (do_norm == 4 && (ksplit || !dual)) return -1;
    if (n_in <= 0 || n_in % 256 || n_in > 16384 || tiles <= 0 || cus <= 0) return -1;
    const int nb = n_in / 256;
    if (ksplit) {
        if (ksplit != 2 || dual || (do_norm != 0 && do_norm != 2)) return -1;
        const int nw = draco_dq_ksplit_waves(n_in, do_norm);
        if (!nw) return -1;
        const int cap = cus * (16 / nw);  // 4-wave blocks: four per CU; 8-wave: two
        s.nw = nw;
        s.ks = 1;
        s.grid = 2 * tiles < cap ? 2 * tiles : cap;
    } else {
        // waves per block: enough to split a row's super-blocks, and enough
        // threads for the prologue's XP_MAXV float4s per thread (8 waves up
        // to 63 super-blocks per row: measured faster than 16 for the decode
        // down projection, n_in 8192)
        int nw = nb >= 64 ? 16 : (nb >= 8 ? 8 : 4);
        while (n_in > xp * 4 * 64 * nw) nw *= 2;
        if (nw > 16) return -1;
        const int cap = cus * (16 / nw);
        int grid = tiles < cap ? tiles : cap;
        // One item per wave and one tile per block (a row of at most NW
        // super-blocks, at least two tiles per CU): blocks of two tiles
        // instead, one per CU, so every wave keeps its second item's loads in
        // flight while it computes the first, and half the blocks repeat the
        // x prologue.  Measured on the configs[2] decode (the gate/up SwiGLU
        // launch, 512 tiles): 2008 -> 2108 tok/s; an 8192x2048 Q4_K GEMV
        // 4.07 -> 3.83 us.  Launches with fewer tiles than that keep one per
        // block (halving the qkv or wo grid was slower: 2108 -> 1917 / 1821
        // tok/s).
        if (nb <= nw && tiles >= 2 * cus && tiles <= cap) grid = (tiles + 1) / 2;
        s.nw = nw;
        s.grid = grid;
        s.ipt1 = nb <= nw;
        // row dots: the 8-wave instances, two float4 of the row per thread,
        // 2 gd_n blocks at the end of the grid
        if (gd_n > 0 && !dual && nw == 8 && (do_norm == 1 || do_norm == 3) && grid >= 2 * gd_n &&
            n_in <= 2 * 4 * 64 * nw)
            s.gd = 1;
    }
    if (dq_lds_bytes(n_in, s.nw) > 160 * 1024) return -1;
    return 0;
}

int draco_seg_launch(SegLaunch& a, hipStream_t st) {
    if (a.nseg < 1 || a.nseg > SEG_MAX) return -1;
    bool kq = false, q8 = false;
    for (int i = 0; i < a.nseg; i++) {
        const int c = a.seg[i].L.code;
        if (a.seg[i].L.n_in != a.n_in) return -1;
        if (c == DRACO_Q4_K || c == DRACO_Q6_K || c == DRACO_Q5_K) kq = true;
        else if (c == DRACO_Q8_0) q8 = true;
        else return -1;
    }
    if (kq && q8) return -1;
    if (a.do_norm == 2 && !kq) return -1;  // the GNORM prologue is k_dq's only
    return kq ? seg_launch_dq(a, st) : seg_launch_q8(a, st);
}

int draco_gemv_launch(const DracoMat& m, const float* x, float* y, const float* yadd, int row0, int row1,
                      hipStream_t st) {
    if (row0 < 0 || row1 > m.L.n_out || row0 > row1) return -1;
    if (row0 == row1) return 0;
    const int code = m.L.code;
    if (code == DRACO_Q4_K || code == DRACO_Q6_K || code == DRACO_Q5_K) {
        SegLaunch a = {};
        a.nseg = 1;
        a.n_in = m.L.n_in;
        a.x = x;
        SegDesc& s = a.seg[0];
        s.base = m.dev;
        s.L = m.L;
        s.row0 = row0;
        s.row1 = row1;
        s.y = y;
        s.yadd = yadd;
        s.epi = yadd ? EPI_RESID : EPI_STORE;
        return draco_seg_launch(a, st);
    }
    if (code == DRACO_Q8_0) {
        // a row range is a segment over rows [row0, row1): offset the region bases by row0 rows
        SegLaunch a = {};
        a.nseg = 1;
        a.n_in = m.L.n_in;
        a.x = x;
        SegDesc& s = a.seg[0];
        s.L = m.L;
        s.L.n_out = row1 - row0;
        s.base = m.dev;
        const size_t nb = (size_t)m.L.nb;
        s.L.off[0] += 32 * nb * (size_t)row0;
        s.L.off[1] += 2 * nb * (size_t)row0;
        s.y = y + row0;
        s.yadd = yadd ? yadd + row0 : nullptr;
        s.epi = yadd ? EPI_RESID : EPI_STORE;
        return draco_seg_launch(a, st);
    }
    const int R = 1;
    const int waves = row1 - row0;
    const dim3 grid((waves + 3) / 4), block(256);
    if (code == DRACO_F32)
        hipLaunchKernelGGL((k_gemv_plain<R, false>), grid, block, 0, st, m.dev, x, y, yadd, row0, row1, m.L.n_in);
    else if (code == DRACO_F16)
        hipLaunchKernelGGL((k_gemv_plain<R, true>), grid, block, 0, st, m.dev, x, y, yadd, row0, row1, m.L.n_in);
    else
        return -1;
    return 0;
}

int draco_gemv_supported(int code) {
    return code == DRACO_Q4_K || code == DRACO_Q5_K || code == DRACO_Q6_K || code == DRACO_Q8_0 ||
           code == DRACO_F32 || code == DRACO_F16;
}

// Host-side launch planning, exported so tests can enumerate shapes without a
// GPU: out = {nw, grid, ipt1, ks, gd, xp_max}.  Returns draco_dq_shape's code.
extern "C" int draco_dq_plan(int n_in, int tiles, int dual, int ksplit, int do_norm, int gd_n, int cus, int* out) {
    DqShape s;
    const int rc = draco_dq_shape(n_in, tiles, dual != 0, ksplit, do_norm, gd_n, cus, s);
    if (out) {
        out[0] = s.nw;
        out[1] = s.grid;
        out[2] = s.ipt1;
        out[3] = s.ks;
        out[4] = s.gd;
        out[5] = s.xp_max;
    }
    return rc;
}
