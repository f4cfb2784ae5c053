// gdn.hip -- Gated-DeltaNet recurrent scan (gfx950).
//
// Reference: m6_gdn_scan, src/m6_gdn_scan.c:18-93 (the same step as
// m6_gdn_attn, src/m6_layer.c:262-331).  Per token t and V head h (q/k head
// j = h % NHQ, head size 128):
//   c = silu(w0*tail0 + w1*tail1 + w2*tail2 + w3*qkv_t)   per channel, tail shifts
//   q_j, k_j l2-normalised (1 / max(|.|, 1e-6))
//   S *= g;  sk = S^T k;  d = (v - sk) * b;  S += k (x) d;  o = S^T q
//   on = (o/sqrt(128)) * rsqrt(mean(o^2)+1e-6) * ssm_norm * silu(z)
// S is [k][v] (row k), 128 x 128 fp32 per V head.
//
// Mapping: the 128 columns of a V head's state are split over NSPL blocks
// of NW waves (grid n_vh x NSPL); every block keeps its columns of the state
// in registers for the whole scan.  Wave w of split sp owns CPW = 128 /
// (NSPL NW) columns, v = CPW (sp NW + w) + v_lo; lane (v_lo = lane / KQ,
// kq = lane % KQ, KQ = 64 / CPW) holds rows RPL kq .. RPL kq + RPL - 1 of
// column v (RPL = 128 / KQ).  Each lane applies the reference's per-element
// operations in k order within its chunk (decay, multiply, add, unfused); the
// KQ chunks of a column combine with DPP moves, so the delta rule needs no
// LDS and no barrier.  The conv runs on the block's threads, channel c =
// tid + r * threads (q and k of head j in every block: the l2 norms need
// them whole; v only for the block's columns), the tails in registers; only
// the block that owns a channel writes its tail back (q/k channels: the last
// block of the head's readers to count itself in g_qk_cnt).  The l2 norms reduce across the block's waves
// through LDS.  The gated rms needs all 128 columns of a head: with one
// block per head (NW = 8) it is finished in the block; split across blocks,
// each wave writes its columns' o / sqrt(128) to ON and the sum of their
// squares to a partial buffer, and k_gdn_gnorm applies the rms, the norm
// weight and the gate in place.  Results agree with the reference to fp32
// rounding: the per-column sums are split in KQ chunks and the l2 / rms
// sums use a tree.
//
// The split spreads each head's 64 KB of state over NSPL CUs (the state load
// and store at the ends of a launch run NSPL-wide) and gives a long scan one
// in-block barrier per token fewer with fewer waves behind each (the rms
// needs none when split); the defaults below are the measured best.
#include <hip/hip_runtime.h>

#include "dev_common.h"
#include "gdn.h"

namespace {

constexpr int SV = 128;
constexpr float EPS = 1e-6f;

// The q / k channels of a q/k head's conv are read by every block (wave) of
// each V head that uses the head and updated once.  The last reader writes
// the new tails: each reader adds 1 to its head's counter here once its tail
// loads have returned; the one that brings it to the number of readers
// writes the tails and puts the counter back to 0 for the next launch.  A
// fixed writer could overwrite a tail before a reader's queued load of it
// had been served (the readers of a head run on the same XCD, so such a load
// would hit the new value in L2).
// One counter per q/k head, 4 KB apart: atomics on one line serialise.
constexpr int QK_CNT_STRIDE = 1024;
constexpr int QK_CNT_MAX = 64;  // q/k heads
__device__ unsigned g_qk_cnt[QK_CNT_MAX * QK_CNT_STRIDE];

__device__ __forceinline__ float silu(float a) { return a / (1.f + expf(-a)); }

// Decode-step gates of V head h (src/m6_layer.c:237-256): every thread
// gets beta and the decay exp(alpha).  xn = h1 * rms^-1 * attn_norm: the
// block reduces the sum of squares of h1 and the two dots of (h1 * attn_norm)
// with its head's beta / alpha rows through one barrier, and applies rms^-1
// to the dots (the reference scales each element first; the results differ
// by fp32 rounding).  h1 and attn_norm are L2-resident after the first
// block; the rows are contiguous [n_vh][H].  issue() requests every operand
// (up to 8 float4 per array and thread, so blocks of 128 threads and more
// hold them in registers) ahead of the kernel's state loads; finish() reduces.
template <int NW>
struct GdnGates {
    static constexpr int NT = 64 * NW;
    static constexpr int NV = (4096 + 4 * NT - 1) / (4 * NT);  // float4 per thread covering H <= 4096
    static constexpr int NR = NV <= 8 ? NV : 1;
    float4 hv[NR], nv[NR], bv[NR], av[NR];

    __device__ __forceinline__ void load(const GdnArgs& a, int h, int tid, int k, int slot) {
        const int i = 4 * tid + 4 * NT * k;  // clamped, unconditional loads; masked in finish()
        const int ic = i < a.H ? i : 0;
        hv[slot] = ld4(a.h1 + ic);
        nv[slot] = ld4(a.attn_norm + ic);
        bv[slot] = ld4(a.bw + (size_t)h * a.H + ic);
        av[slot] = ld4(a.aw + (size_t)h * a.H + ic);
    }
    __device__ __forceinline__ void issue(const GdnArgs& a, int h, int tid) {
        if constexpr (NR == NV) {
#pragma unroll
            for (int k = 0; k < NV; k++) load(a, h, tid, k, k);
        }
    }
    __device__ __forceinline__ void finish(const GdnArgs& a, int h, int tid, float* beta, float* gdec) {
        __shared__ float pre[3][NW];
        const int lane = tid & 63, w = tid >> 6;
        float ss = 0.f, pb = 0.f, pa = 0.f;
        auto acc = [&](int k, int slot) {
            if (4 * tid + 4 * NT * k < a.H) {
                const float4 x = hv[slot], n = nv[slot], b = bv[slot], al = av[slot];
                ss += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
                const float x0 = x.x * n.x, x1 = x.y * n.y, x2 = x.z * n.z, x3 = x.w * n.w;
                pb += b.x * x0 + b.y * x1 + b.z * x2 + b.w * x3;
                pa += al.x * x0 + al.y * x1 + al.z * x2 + al.w * x3;
            }
        };
        if constexpr (NR == NV) {
#pragma unroll
            for (int k = 0; k < NV; k++) acc(k, k);
        } else {
            for (int k = 0; k < NV; k++) {
                load(a, h, tid, k, 0);
                acc(k, 0);
            }
        }
        ss = wave_sum(ss);
        pb = wave_sum(pb);
        pa = wave_sum(pa);
        if (lane == 0) {
            pre[0][w] = ss;
            pre[1][w] = pb;
            pre[2][w] = pa;
        }
        lds_barrier();
        float tot = 0.f, bacc = 0.f, aacc = 0.f;
#pragma unroll
        for (int q = 0; q < NW; q++) {
            tot += pre[0][q];
            bacc += pre[1][q];
            aacc += pre[2][q];
        }
        const float inv = 1.f / sqrtf(tot / (float)a.H + EPS);
        gates_of(a, h, bacc * inv, aacc * inv, beta, gdec);
    }
    // beta = sigmoid(xn.bw), decay = exp(softplus(xn.aw + dt) * a) from the two dots
    static __device__ __forceinline__ void gates_of(const GdnArgs& a, int h, float db, float da, float* beta,
                                                    float* gdec) {
        *beta = 1.f / (1.f + expf(-db));
        const float avv = da + a.ssm_dt[h];
        const float sp = avv > 0.f ? avv + log1pf(expf(-avv)) : log1pf(expf(avv));
        *gdec = expf(sp * a.ssm_a[h]);
    }
};

// NW waves per block, NSPL blocks per V head: a wave owns CPW = 128 /
// (NSPL * NW) columns, KQ = 64 / CPW lanes share a column and each lane
// holds RPL = 128 / KQ of its rows.
template <bool DEC, int NW, int NSPL>
__global__ __launch_bounds__(64 * NW) void k_gdn_scan(const GdnArgs a) {
    constexpr int NT = 64 * NW, NC = SV / NSPL;  // threads, columns per block
    constexpr int CPW = NC / NW, KQ = 64 / CPW, RPL = SV / KQ;
    static_assert(CPW * NW * NSPL == SV && KQ * CPW == 64 && NSPL * NW <= GDN_PSS_STRIDE, "scan shape");
    constexpr int CH = 2 * SV + NC;                            // conv channels of a block
    constexpr int R = (CH + NT - 1) / NT;                      // channels per thread
    __shared__ float cq[SV], ck[SV], cv[NC];  // conv outputs of this token (q, k normalised in place)
    __shared__ float red[2][NW];
    __shared__ float ored[NW];
    const int h = blockIdx.x, sp = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int NHQ = a.nhq, n_qkv = a.n_qkv, n_vh = a.n_vh, T = a.T;
    const int j = h % NHQ;
    const int col0 = sp * NC;  // this block's first column of the head
    // decode: the gates' operands are requested first, then the conv inputs
    // and the state, so the gate arithmetic runs while the state arrives
    GdnGates<NW> gates;
    float gdb = 0.f, gda = 0.f;  // the gates' dots when the in-projection formed them
    if constexpr (DEC) {
        if (a.glog) {
            gdb = a.glog[h];
            gda = a.glog[n_vh + h];
        } else {
            gates.issue(a, h, tid);
        }
    }
    // conv channels of this thread: local c = tid + r * NT; 0..127 q_j,
    // 128..255 k_j, 256.. v_h columns col0 ..
    int ch[R];
    bool own[R];
    float w0[R], w1[R], w2[R], w3[R], t0[R], t1[R], t2[R], xin[R];
    // Every load of the prologue is unconditional (a thread past the block's
    // channels reads channel j * 128 and discards it; the launchers never
    // start a scan of 0 tokens), so the conv inputs and the state below are
    // all in flight before the first wait.
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int c = tid + r * NT;
        int cc = j * SV;
        if (c < SV) cc = j * SV + c;
        else if (c < 2 * SV) cc = NHQ * SV + j * SV + (c - SV);
        else if (c < CH) cc = 2 * NHQ * SV + h * SV + col0 + (c - 2 * SV);
        const bool live = c < CH;
        ch[r] = live ? cc : -1;
        own[r] = c >= 2 * SV;  // q / k channels: the head's last reader block (below)
        const float4 cw = ld4(a.conv + (size_t)cc * 4);
        const float ta = a.tail[(size_t)cc * 3], tb = a.tail[(size_t)cc * 3 + 1], tc = a.tail[(size_t)cc * 3 + 2];
        const float xi = a.QKV[cc];
        w0[r] = live ? cw.x : 0.f;
        w1[r] = live ? cw.y : 0.f;
        w2[r] = live ? cw.z : 0.f;
        w3[r] = live ? cw.w : 0.f;
        t0[r] = live ? ta : 0.f;
        t1[r] = live ? tb : 0.f;
        t2[r] = live ? tc : 0.f;
        xin[r] = live ? xi : 0.f;
    }
    // state slice
    const int vl = lane / KQ, kq = lane % KQ, vloc = CPW * w + vl, v = col0 + vloc;
    float* Sh = a.S + (size_t)h * SV * SV;
    const float nw = a.ssm_norm[v];
    // per-token inputs, prefetched one token ahead
    float zin = a.Z[(size_t)h * SV + v];
    float s[RPL];
#pragma unroll
    for (int i = 0; i < RPL; i++) s[i] = Sh[(size_t)(RPL * kq + i) * SV + v];
    const float scale = 1.f / sqrtf((float)SV);

    __shared__ unsigned qk_prev;
    unsigned prev = 0;  // thread 0's: the block's count as a reader of its q / k head's tails (below)
    float gin = 0.f, bin = 0.f;
    if constexpr (DEC) {
        if (a.glog) GdnGates<NW>::gates_of(a, h, gdb, gda, &bin, &gin);
        else gates.finish(a, h, tid, &bin, &gin);
    } else {
        gin = a.G[h];
        bin = a.B[h];
    }
    for (int t = 0; t < T; t++) {
        const float z = zin, g = gin, b = bin;
        float x[R];
#pragma unroll
        for (int r = 0; r < R; r++) x[r] = xin[r];
        if (!DEC && t + 1 < T) {
#pragma unroll
            for (int r = 0; r < R; r++)
                if (ch[r] >= 0) xin[r] = a.QKV[(size_t)(t + 1) * n_qkv + ch[r]];
            zin = a.Z[(size_t)(t + 1) * n_vh * SV + (size_t)h * SV + v];
            gin = a.G[(size_t)(t + 1) * n_vh + h];
            bin = a.B[(size_t)(t + 1) * n_vh + h];
        }
        // (1) conv + silu (src/m6_gdn_scan.c:30-38); (2) squares for the l2 norms
        float c[R];
        float sqq = 0.f, sqk = 0.f;
#pragma unroll
        for (int r = 0; r < R; r++) {
            c[r] = 0.f;
            if (ch[r] >= 0) {
                const float acc = w0[r] * t0[r] + w1[r] * t1[r] + w2[r] * t2[r] + w3[r] * x[r];
                c[r] = silu(acc);
                t0[r] = t1[r];
                t1[r] = t2[r];
                t2[r] = x[r];
            }
            const int cl = tid + r * NT;
            if (cl < SV) sqq += c[r] * c[r];
            else if (cl < 2 * SV) sqk += c[r] * c[r];
        }
        sqq = wave_sum(sqq);
        sqk = wave_sum(sqk);
        if (lane == 0) {
            red[0][w] = sqq;
            red[1][w] = sqk;
        }
        lds_barrier();
        // every wave has used its tails in the first token's conv (their loads
        // have returned): count the block as a reader of its q / k head's
        // tails; the result is read after the token loop, so the atomic's
        // round trip overlaps the scan
        if (t == 0 && tid == 0)
            prev = __hip_atomic_fetch_add(&g_qk_cnt[j * QK_CNT_STRIDE], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        float nq = 0.f, nk = 0.f;
#pragma unroll
        for (int q = 0; q < NW; q++) {
            nq += red[0][q];
            nk += red[1][q];
        }
        const float rq = sqrtf(nq), rk = sqrtf(nk);
        const float iq = 1.f / (rq > EPS ? rq : EPS), ik = 1.f / (rk > EPS ? rk : EPS);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int cl = tid + r * NT;
            if (cl < SV) cq[cl] = c[r] * iq;
            else if (cl < 2 * SV) ck[cl - SV] = c[r] * ik;
            else if (cl < CH) cv[cl - 2 * SV] = c[r];
        }
        lds_barrier();
        // (3) delta rule on this lane's 32 rows of column v
        float sk = 0.f;
#pragma unroll
        for (int i = 0; i < RPL; i++) {
            s[i] = s[i] * g;
            sk = sk + s[i] * ck[RPL * kq + i];
        }
        sk = group_sum<KQ>(sk);
        const float d = (cv[vloc] - sk) * b;
        float o = 0.f;
#pragma unroll
        for (int i = 0; i < RPL; i++) {
            s[i] = s[i] + ck[RPL * kq + i] * d;
            o = o + s[i] * cq[RPL * kq + i];
        }
        o = group_sum<KQ>(o);
        // (4) gated rms over the 128 columns
        o = o * scale;
        float o2 = kq == 0 ? o * o : 0.f;
        o2 = wave_sum(o2);
        if constexpr (NSPL == 1) {
            if (lane == 0) ored[w] = o2;
            lds_barrier();
            float ms2 = 0.f;
#pragma unroll
            for (int q = 0; q < NW; q++) ms2 += ored[q];
            const float inv2 = 1.f / sqrtf(ms2 / SV + EPS);
            if (kq == 0) a.ON[(size_t)t * n_vh * SV + (size_t)h * SV + v] = o * inv2 * nw * silu(z);
        } else {
            // o / sqrt(128) and this wave's sum of squares; k_gdn_gnorm finishes
            // (deferred: o * ssm_norm * silu(z), and the consumer applies the rms)
            if (kq == 0) a.ON[(size_t)t * n_vh * SV + (size_t)h * SV + v] = a.defer_gnorm ? o * nw * silu(z) : o;
            if (lane == 0) a.PSS[((size_t)t * n_vh + h) * GDN_PSS_STRIDE + sp * NW + w] = o2;
        }
        lds_barrier();  // cq/ck/cv/red/ored are rewritten by the next token
    }
#pragma unroll
    for (int i = 0; i < RPL; i++) Sh[(size_t)(RPL * kq + i) * SV + v] = s[i];
    if (tid == 0) qk_prev = prev;
    lds_barrier();
    const bool last = qk_prev + 1 == (unsigned)(NSPL * ((n_vh - 1 - j) / NHQ + 1));
    if (last && tid == 0) __hip_atomic_store(&g_qk_cnt[j * QK_CNT_STRIDE], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int r = 0; r < R; r++)
        if (ch[r] >= 0 && (own[r] || last)) {
            a.tail[(size_t)ch[r] * 3] = t0[r];
            a.tail[(size_t)ch[r] * 3 + 1] = t1[r];
            a.tail[(size_t)ch[r] * 3 + 2] = t2[r];
        }
}

// Decode step (T = 1) with the gates' dots from the in-projection (a.glog),
// without block barriers: 16 waves per V head (blockIdx.y * NW + w = wg),
// wave wg owning columns 8 wg .. 8 wg + 7 in k_gdn_scan's lane layout (KQ = 8
// lanes per column, 16 rows per lane), and every wave recomputing the conv +
// silu + l2 norms of its q / k head's 256 channels itself (lane l: channels
// l and l + 64 of q and of k; lanes 0-7 also its v column l's channel), so
// no wave waits for another.  The normalised q / k pass between the lanes of
// a wave through the wave's own LDS rows.  The per-element operations are
// k_gdn_scan's; the l2 norms' sums of squares reduce in another tree order
// (fp32 rounding).  Outputs as k_gdn_scan's split form: ON and the 16
// per-wave sums of squares in PSS.  Tails: a v channel's by its wave, the
// q / k channels' by the head's last reader (g_qk_cnt).
// The prologue's operands come first as scalars the dispatcher preloads into
// SGPRs (a struct argument is never preloaded).
template <int NW>
__global__ __launch_bounds__(64 * NW) void k_gdn_dec(float* __restrict__ pS, const float* __restrict__ pconv,
                                                     float* __restrict__ ptail, const float* __restrict__ pqkv,
                                                     const float* __restrict__ pglog, int pnhq, int pnvh,
                                                     const float* __restrict__ pZ, const GdnArgs a) {
    constexpr int CPW = 8, KQ = 8, RPL = SV / KQ;
    __shared__ float qk[NW][2 * SV];
    __shared__ float cvs[NW][CPW];
    const int h = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int wg = blockIdx.y * NW + w;
    const int NHQ = pnhq, n_vh = pnvh;
    const int j = h % NHQ;
    // every load first: gates' dots, conv weights / tails / inputs of the 5
    // channels, z, norm weight and the state slice
    const float gdb = pglog[h], gda = pglog[n_vh + h];
    int ch[5];
    ch[0] = j * SV + lane;
    ch[1] = ch[0] + 64;
    ch[2] = NHQ * SV + j * SV + lane;
    ch[3] = ch[2] + 64;
    ch[4] = 2 * NHQ * SV + h * SV + CPW * wg + (lane & (CPW - 1));
    float w0[5], w1[5], w2[5], w3[5], t0[5], t1[5], t2[5], xi[5];
#pragma unroll
    for (int r = 0; r < 5; r++) {
        const float4 cw = ld4(pconv + (size_t)ch[r] * 4);
        w0[r] = cw.x;
        w1[r] = cw.y;
        w2[r] = cw.z;
        w3[r] = cw.w;
        t0[r] = ptail[(size_t)ch[r] * 3];
        t1[r] = ptail[(size_t)ch[r] * 3 + 1];
        t2[r] = ptail[(size_t)ch[r] * 3 + 2];
        xi[r] = pqkv[ch[r]];
    }
    const int vl = lane / KQ, kq = lane % KQ, v = CPW * wg + vl;
    float* Sh = pS + (size_t)h * SV * SV;
    const float nw = a.ssm_norm[v];
    const float z = pZ[(size_t)h * SV + v];
    float s[RPL];
#pragma unroll
    for (int i = 0; i < RPL; i++) s[i] = Sh[(size_t)(RPL * kq + i) * SV + v];
    float b, g;
    GdnGates<NW>::gates_of(a, h, gdb, gda, &b, &g);
    // (1) conv + silu (src/m6_gdn_scan.c:30-38), (2) the l2 norms of q and k
    float c[5];
#pragma unroll
    for (int r = 0; r < 5; r++) {
        const float acc = w0[r] * t0[r] + w1[r] * t1[r] + w2[r] * t2[r] + w3[r] * xi[r];
        c[r] = silu(acc);
    }
    // Count the wave as a reader of its q / k head's tails once every load
    // above has returned: the empty asm statements read every loaded value,
    // so the compiler waits for all of them here (they are all needed from
    // here on) and no wait after the atomic is for anything but the atomic,
    // whose result is read at the end: its round trip overlaps the step.
    // (gdn.hip is built without the atomic optimizer, whose wave-level
    // rewrite waits for the result where the atomic is.)
#pragma unroll
    for (int r = 0; r < 5; r++)
        asm volatile("" ::"v"(w0[r]), "v"(w1[r]), "v"(w2[r]), "v"(w3[r]), "v"(t0[r]), "v"(t1[r]), "v"(t2[r]),
                     "v"(xi[r]));
#pragma unroll
    for (int i = 0; i < RPL; i += 4) asm volatile("" ::"v"(s[i]), "v"(s[i + 1]), "v"(s[i + 2]), "v"(s[i + 3]));
    asm volatile("" ::"v"(z), "v"(nw) : "memory");
    unsigned prev = 0;  // lane 0's
    if (lane == 0) prev = __hip_atomic_fetch_add(&g_qk_cnt[j * QK_CNT_STRIDE], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const float sqq = wave_sum(c[0] * c[0] + c[1] * c[1]);
    const float sqk = wave_sum(c[2] * c[2] + c[3] * c[3]);
    const float rq = sqrtf(sqq), rk = sqrtf(sqk);
    const float iq = 1.f / (rq > EPS ? rq : EPS), ik = 1.f / (rk > EPS ? rk : EPS);
    float* cq = qk[w];
    float* ck = qk[w] + SV;
    cq[lane] = c[0] * iq;
    cq[lane + 64] = c[1] * iq;
    ck[lane] = c[2] * ik;
    ck[lane + 64] = c[3] * ik;
    if (lane < CPW) cvs[w][lane] = c[4];
    // the wave's own LDS rows: its writes ordered before its reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    // (3) delta rule on this lane's 16 rows of column v
    float sk = 0.f;
#pragma unroll
    for (int i = 0; i < RPL; i++) {
        s[i] = s[i] * g;
        sk = sk + s[i] * ck[RPL * kq + i];
    }
    sk = group_sum<KQ>(sk);
    const float d = (cvs[w][vl] - sk) * b;
    float o = 0.f;
#pragma unroll
    for (int i = 0; i < RPL; i++) {
        s[i] = s[i] + ck[RPL * kq + i] * d;
        o = o + s[i] * cq[RPL * kq + i];
    }
    o = group_sum<KQ>(o);
    // (4) o / sqrt(128) and the wave's sum of squares for the gated rms
    o = o * (1.f / sqrtf((float)SV));
    const float o2 = wave_sum(kq == 0 ? o * o : 0.f);
    if (kq == 0) a.ON[(size_t)h * SV + v] = a.defer_gnorm ? o * nw * silu(z) : o;
    if (lane == 0) a.PSS[(size_t)h * GDN_PSS_STRIDE + wg] = o2;
#pragma unroll
    for (int i = 0; i < RPL; i++) Sh[(size_t)(RPL * kq + i) * SV + v] = s[i];
    // the last of the head's 16 * (V heads using it) reader waves writes the q / k tails
    const bool own_qk = __builtin_amdgcn_readfirstlane(prev) + 1 == 16u * (unsigned)((n_vh - 1 - j) / NHQ + 1);
    if (own_qk && lane == 0) __hip_atomic_store(&g_qk_cnt[j * QK_CNT_STRIDE], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int r = 0; r < 5; r++)
        if (r == 4 ? lane < CPW : own_qk) {
            ptail[(size_t)ch[r] * 3] = t1[r];
            ptail[(size_t)ch[r] * 3 + 1] = t2[r];
            ptail[(size_t)ch[r] * 3 + 2] = xi[r];
        }
}

// The gated rms of split scans, in place: for token t and V head h,
// ON[t][h][v] = o * rsqrt(sum of the NP wave partials / 128 + eps) *
// ssm_norm[v] * silu(Z[t][h][v]), the reference's order (src/m6_layer.c:
// 320-331).  Block (t, h), 128 threads.
template <int NP>
__global__ __launch_bounds__(128) void k_gdn_gnorm(const GdnArgs a) {
    const int t = blockIdx.x, h = blockIdx.y, v = threadIdx.x;
    const float* ps = a.PSS + ((size_t)t * a.n_vh + h) * GDN_PSS_STRIDE;
    float ms2 = 0.f;
#pragma unroll
    for (int q = 0; q < NP; q++) ms2 += ps[q];
    const float inv2 = 1.f / sqrtf(ms2 / SV + EPS);
    const size_t i = (size_t)t * a.n_vh * SV + (size_t)h * SV + v;
    a.ON[i] = a.ON[i] * inv2 * a.ssm_norm[v] * silu(a.Z[i]);
}

// A split decode step leaves NSPL * NW = 16 partials (the ssm_out GEMV's
// GNORM prologue reads 16); scans of several tokens use 8 waves per block.
// k_gdn_dec's waves per block (1 or 2; 0: k_gdn_scan<true, 2, 8>)
int g_dec_waves = 2;

template <bool DEC>
int launch_scan(const GdnArgs& a, int nspl, hipStream_t st) {
    if (nspl > 1 && !a.PSS) return -1;
    const dim3 g(a.n_vh, nspl);
    int np = 16;
    if (DEC && nspl == 8 && a.glog && g_dec_waves) {
        // the barrier-free decode step: 16 waves per V head in blocks of 1 or 2
        if (g_dec_waves == 1)
            hipLaunchKernelGGL(k_gdn_dec<1>, dim3(a.n_vh, 16), dim3(64), 0, st, a.S, a.conv, a.tail, a.QKV, a.glog,
                               a.nhq, a.n_vh, a.Z, a);
        else
            hipLaunchKernelGGL(k_gdn_dec<2>, dim3(a.n_vh, 8), dim3(128), 0, st, a.S, a.conv, a.tail, a.QKV, a.glog,
                               a.nhq, a.n_vh, a.Z, a);
    } else if (DEC || nspl == 1) {
        switch (nspl) {
        case 1: hipLaunchKernelGGL((k_gdn_scan<DEC, 8, 1>), g, dim3(512), 0, st, a); return 0;
        case 2: hipLaunchKernelGGL((k_gdn_scan<DEC, 8, 2>), g, dim3(512), 0, st, a); break;
        case 4: hipLaunchKernelGGL((k_gdn_scan<DEC, 4, 4>), g, dim3(256), 0, st, a); break;
        case 8: hipLaunchKernelGGL((k_gdn_scan<DEC, 2, 8>), g, dim3(128), 0, st, a); break;
        default: return -1;
        }
    } else {
        switch (nspl) {
        case 2: hipLaunchKernelGGL((k_gdn_scan<DEC, 8, 2>), g, dim3(512), 0, st, a); np = 16; break;
        case 4: hipLaunchKernelGGL((k_gdn_scan<DEC, 8, 4>), g, dim3(512), 0, st, a); np = 32; break;
        case 8: hipLaunchKernelGGL((k_gdn_scan<DEC, 8, 8>), g, dim3(512), 0, st, a); np = 64; break;
        default: return -1;
        }
    }
    if (a.defer_gnorm) return np == 16 ? 0 : -1;
    const dim3 gg(a.T, a.n_vh);
    if (np == 16) hipLaunchKernelGGL(k_gdn_gnorm<16>, gg, dim3(SV), 0, st, a);
    else if (np == 32) hipLaunchKernelGGL(k_gdn_gnorm<32>, gg, dim3(SV), 0, st, a);
    else hipLaunchKernelGGL(k_gdn_gnorm<64>, gg, dim3(SV), 0, st, a);
    return 0;
}

// Measured on MI355X (configs[4] heads, 32 V heads, graph-replayed): the
// decode step with its gates (kernel alone) takes 8.3 us in one block of 8
// waves per head, split 4 ways 6.2 us in blocks of 2 waves, 5.8 in blocks of
// 4 (7.3 of 8), split 8 ways 5.9 in blocks of 4; the split's gated rms then
// costs 0.5 us in the ssm_out GEMV's prologue (a k_gdn_gnorm launch would
// cost more than the split saves): the 48-layer configs[4] stack decodes at
// 974 tok/s split 4 (2-wave blocks) against 922 unsplit, 964 split 4 in
// 4-wave blocks and 998 split 8 in 2-wave blocks (same box, +-2%).  A 64-token scan (the kernel
// alone) takes 1.43 us/token in 2 blocks of 4 waves per head, 1.09 in 8
// blocks of 4 waves, 1.17 / 1.00 / 0.96 in 2 / 4 / 8 blocks of 8 waves
// (more lanes per column: shorter per-lane chains, every wave busy on its
// SIMD) and 1.39 / 1.27 in 2 / 4 blocks of 16 waves.
int g_split_dec = 8;
int g_split_scan = 8;

}  // namespace

int draco_gdn_split(bool decode) { return decode ? g_split_dec : g_split_scan; }

// Blocks per V head of the GDN decode step and of multi-token scans (1, 2, 4
// or 8; a negative argument keeps the setting).  Returns the previous values
// as decode * 16 + scan.
// Waves per block of the barrier-free GDN decode step (1 or 2), or 0 for
// the split scan kernel's decode form; other values only query.  Returns the
// previous value.
extern "C" int draco_set_gdn_dec(int waves) {
    const int old = g_dec_waves;
    if (waves >= 0 && waves <= 2) g_dec_waves = waves;
    return old;
}

extern "C" int draco_set_gdn_split(int decode_split, int scan_split) {
    const int old = g_split_dec * 16 + g_split_scan;
    auto ok = [](int n) { return n == 1 || n == 2 || n == 4 || n == 8; };
    if (ok(decode_split)) g_split_dec = decode_split;
    if (ok(scan_split)) g_split_scan = scan_split;
    return old;
}

int draco_gdn_scan_launch(const GdnArgs& a, hipStream_t st) {
    if (a.n_vh < 1 || a.nhq < 1 || a.nhq > QK_CNT_MAX || a.n_qkv != a.n_vh * SV + 2 * a.nhq * SV || a.T < 0)
        return -1;
    if (a.T == 0) return 0;
    return launch_scan<false>(a, a.nspl < 1 ? 1 : a.nspl, st);
}

int draco_gdn_step_launch(const GdnArgs& a, hipStream_t st) {
    if (a.n_vh < 1 || a.nhq < 1 || a.nhq > QK_CNT_MAX || a.n_qkv != a.n_vh * SV + 2 * a.nhq * SV || a.T != 1)
        return -1;
    if (a.H < 4 || a.H > 4096 || a.H % 4 || !a.h1 || !a.attn_norm || !a.bw || !a.aw || !a.ssm_a || !a.ssm_dt)
        return -1;
    return launch_scan<true>(a, a.nspl < 1 ? 1 : a.nspl, st);
}
