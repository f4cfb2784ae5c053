// decode.hip -- the non-GEMV kernels of one llama decode token (gfx950).
//
// Reference semantics (src/m6_engine.c):
//   rms_norm            :31-37    out = x * (1/sqrtf(mean(x^2)+eps)) * w
//   consecutive-pair rope :134-143 (angles from a host table built with the
//                        same libm calls, so they are bit-identical)
//   KV append            :477-481  row T of the caches, after rope
//   attention            :482-505  per q head h (kv head h/rep): softmax over
//                        rows 0..T of (q.k_t)*scale, weighted sum of v_t
//   SwiGLU               :289-302  g = g/(1+expf(-g)) * u
//
// Device "token state": st[0] = position, st[1 + l] = tlen of layer l before
// this token.  Kernels read T and pos from it, so a captured graph of a
// token can be replayed for every position (k_advance bumps it).
#include <hip/hip_runtime.h>
#include <math.h>

#include "decode.h"
#include "dev_common.h"
#include "embed_dev.h"
#include "tile_frag.h"

namespace {

// ------------------------------------------------------------- RMSNorm --
// One block of 1024 threads; deterministic tree sum.
// Any h: two passes over x.
__global__ __launch_bounds__(1024) void k_rmsnorm_loop(const float* __restrict__ x, const float* __restrict__ w,
                                                       float* __restrict__ out, int h, float eps) {
    __shared__ float red[16];
    float s = 0.f;
    for (int i = threadIdx.x; i < h; i += blockDim.x) s = fmaf(x[i], x[i], s);
    s = wave_sum(s);
    const int wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wv] = s;
    __syncthreads();
    float tot = 0.f;
    for (int i = 0; i < nw; i++) tot += red[i];
    const float inv = 1.f / sqrtf(tot / (float)h + eps);
    for (int i = threadIdx.x; i < h; i += blockDim.x) out[i] = w ? x[i] * inv * w[i] : x[i] * inv;
}

// h <= RMS_PER_THREAD * blockDim.x: x and w are read once, held in registers.
constexpr int RMS_PER_THREAD = 8;
__global__ __launch_bounds__(1024) void k_rmsnorm(const float* __restrict__ x, const float* __restrict__ w,
                                                  float* __restrict__ out, int h, float eps) {
    __shared__ float red[16];
    float v[RMS_PER_THREAD], wv8[RMS_PER_THREAD];
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < RMS_PER_THREAD; k++) {
        const int i = threadIdx.x + k * blockDim.x;
        v[k] = i < h ? x[i] : 0.f;
        wv8[k] = (w && i < h) ? w[i] : 1.f;
        s = fmaf(v[k], v[k], s);
    }
    s = wave_sum(s);
    const int wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wv] = s;
    __syncthreads();
    float tot = 0.f;
    for (int i = 0; i < nw; i++) tot += red[i];
    const float inv = 1.f / sqrtf(tot / (float)h + eps);
#pragma unroll
    for (int k = 0; k < RMS_PER_THREAD; k++) {
        const int i = threadIdx.x + k * blockDim.x;
        if (i < h) out[i] = w ? v[k] * inv * wv8[k] : v[k] * inv;
    }
}

// ---------------------------------------------------- rope + KV append --
// q: [NH][HD], k,v: [NKV][HD]; rope on the first `rot` dims of every head.
__global__ __launch_bounds__(256) void k_rope_append(float* __restrict__ q, const float* __restrict__ k,
                                                     const float* __restrict__ v, float* __restrict__ kc,
                                                     float* __restrict__ vc, const float* __restrict__ tab,
                                                     const int* __restrict__ st, int layer, int NH, int NKV,
                                                     int HD, int rot) {
    const int pos = st[0];
    const int T = st[1 + layer];
    const int half = rot / 2;
    const int KD = NKV * HD;
    const float* ang = tab + (size_t)pos * half * 2;
    const int n_q = NH * HD, n_k = KD;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n_q + 2 * n_k; i += gridDim.x * blockDim.x) {
        if (i < n_q) {  // q: rotate pairs in place (one thread per pair, even index)
            const int d = i % HD;
            if (d < rot && (d & 1) == 0) {
                const float c = ang[d], s = ang[d + 1];  // pair index d/2 -> tab[(d/2)*2 + {0,1}]
                const float a = q[i], b = q[i + 1];
                q[i] = a * c - b * s;
                q[i + 1] = a * s + b * c;
            }
        } else if (i < n_q + n_k) {
            const int j = i - n_q, d = j % HD;
            float* dst = kc + (size_t)T * KD;
            if (d < rot) {
                if ((d & 1) == 0) {
                    const float c = ang[d], s = ang[d + 1];
                    const float a = k[j], b = k[j + 1];
                    dst[j] = a * c - b * s;
                    dst[j + 1] = a * s + b * c;
                }
            } else {
                dst[j] = k[j];
            }
        } else {
            const int j = i - n_q - n_k;
            vc[(size_t)T * KD + j] = v[j];
        }
    }
}

// ----------------------------------------------------------- attention --
// Split-T decode attention.  Block (g, s) handles kv head g and rows
// [t0, t1) of 0..T for the `rep` q heads that share it (GQA: q head h reads
// kv head h/rep, src/m6_engine.c:484); wave j of the block is q head
// g*rep + j.  A pass covers TPP = 64/LPT rows: LPT = HD/32 lanes share a row
// (32 head dims each), so a lane's K slice is 8 float4 loads; lane d also
// loads V[t][d] (and V[t][d+64] when HD = 128) for the pass's rows.  All of a
// pass's K and V loads are issued before the first FMA; scores reduce over
// the row's lanes with DPP moves, the softmax over the wave, and P.V uses
// readlane broadcasts -- no LDS and no barrier.  Passes are merged with the
// online-softmax rescale.  Each (q head, split) writes an unnormalised
// partial (o[HD], m, l); k_attn_combine merges the splits:
//   out[h] = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M),  M = max_s m_s
// which equals the reference's single-pass softmax up to fp32 rounding.
template <int HD>
__global__ __launch_bounds__(1024) void k_attn_part(const float* __restrict__ q, const float* __restrict__ kc,
                                                    const float* __restrict__ vc, float* __restrict__ part,
                                                    const int* __restrict__ st, int layer, int NH, int NKV,
                                                    int nsplit, float scale) {
    constexpr int LPT = HD / 32, TPP = 64 / LPT, DV = HD / 64;
    const int g = blockIdx.x, s = blockIdx.y;
    const int lane = threadIdx.x & 63, j = threadIdx.x >> 6;
    const int rep = NH / NKV, KD = NKV * HD;
    const int h = g * rep + j;
    const int Tn = st[1 + layer] + 1;
    const int chunk = (Tn + nsplit - 1) / nsplit;
    const int t0 = s * chunk, t1 = min(Tn, t0 + chunk);
    const int tt = lane / LPT, pt = lane % LPT;
    float4 qv[8];
#pragma unroll
    for (int i = 0; i < 8; i++) qv[i] = ld4(q + (size_t)h * HD + 32 * pt + 4 * i);
    float m_run = -INFINITY, l_run = 0.f, o[DV];
#pragma unroll
    for (int e = 0; e < DV; e++) o[e] = 0.f;
    for (int pb = t0; pb < t1; pb += TPP) {
        const int t = pb + tt;
        const bool valid = t < t1;
        const int tr = valid ? t : t0;  // clamped row: loads stay in bounds
        float4 kv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) kv[i] = ld4(kc + (size_t)tr * KD + g * HD + 32 * pt + 4 * i);
        float vv[TPP][DV];
#pragma unroll
        for (int r = 0; r < TPP; r++) {
            const int trr = pb + r < t1 ? pb + r : t0;
#pragma unroll
            for (int e = 0; e < DV; e++) vv[r][e] = vc[(size_t)trr * KD + g * HD + lane + 64 * e];
        }
        // every K and V request of the pass leaves before the first wait (the
        // scheduler would otherwise start the scores between them, and the
        // wait for the first K rows would hold back the remaining V requests)
        __builtin_amdgcn_sched_barrier(0);
        float sc = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            sc = fmaf(qv[i].x, kv[i].x, sc);
            sc = fmaf(qv[i].y, kv[i].y, sc);
            sc = fmaf(qv[i].z, kv[i].z, sc);
            sc = fmaf(qv[i].w, kv[i].w, sc);
        }
        sc = group_sum<LPT>(sc);
        sc = valid ? sc * scale : -INFINITY;
        const float m_new = fmaxf(m_run, wave_max(sc));
        const float corr = m_run > -INFINITY ? expf(m_run - m_new) : 0.f;
        const float p = valid ? expf(sc - m_new) : 0.f;
        l_run = l_run * corr + wave_sum(pt == 0 ? p : 0.f);
#pragma unroll
        for (int e = 0; e < DV; e++) {
            float acc = o[e] * corr;
#pragma unroll
            for (int r = 0; r < TPP; r++)
                acc = fmaf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), r * LPT)),
                           vv[r][e], acc);
            o[e] = acc;
        }
        m_run = m_new;
    }
    float* pp = part + ((size_t)h * nsplit + s) * (HD + 2);
#pragma unroll
    for (int e = 0; e < DV; e++) pp[lane + 64 * e] = o[e];
    if (lane == 0) {
        pp[HD] = m_run;
        pp[HD + 1] = l_run;
    }
}

// Any head dim (even, up to 512) and any GQA ratio: block h is q head h
// (kv head h / rep, src/m6_engine.c:482-505), 256 threads over the whole row
// range.  Rows go in sub-chunks of ATT_ANY_CH: wave w scores rows w, w + 4,
// ... (lanes stride the head dims, then a wave sum) into LDS; the
// sub-chunk's maximum rescales the running (m, l) and output (online
// softmax); thread d accumulates p V[t][d] for dims d and d + 256.  It
// writes the normalised output (times the optional gate) directly: this is
// the fallback for shapes the tuned kernels above and below do not serve.
constexpr int ATT_ANY_CH = 64;

__global__ __launch_bounds__(256) void k_attn_any(const float* __restrict__ q, const float* __restrict__ kc,
                                                  const float* __restrict__ vc, float* __restrict__ out,
                                                  const int* __restrict__ st, int layer, int NH, int NKV, int HD,
                                                  float scale, const float* __restrict__ gate, int gstride) {
    __shared__ float qs[512];
    __shared__ float sc[ATT_ANY_CH];
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int rep = NH / NKV, g = h / rep, KD = NKV * HD;
    const int Tn = st[1 + layer] + 1;
    for (int d = tid; d < HD; d += 256) qs[d] = q[(size_t)h * HD + d];
    __syncthreads();
    float m_run = -INFINITY, l_run = 0.f, o0 = 0.f, o1 = 0.f;
    for (int c0 = 0; c0 < Tn; c0 += ATT_ANY_CH) {
        const int nr = min(ATT_ANY_CH, Tn - c0);
        for (int r = w; r < nr; r += 4) {
            const float* kr = kc + (size_t)(c0 + r) * KD + (size_t)g * HD;
            float acc = 0.f;
            for (int d = lane; d < HD; d += 64) acc = fmaf(qs[d], kr[d], acc);
            acc = wave_sum(acc);
            if (lane == 0) sc[r] = acc * scale;
        }
        __syncthreads();
        float cm = -INFINITY;
        for (int r = 0; r < nr; r++) cm = fmaxf(cm, sc[r]);
        const float mn = fmaxf(m_run, cm);
        const float corr = m_run > -INFINITY ? expf(m_run - mn) : 0.f;
        float ls = 0.f;
        o0 *= corr;
        o1 *= corr;
        for (int r = 0; r < nr; r++) {
            const float p = expf(sc[r] - mn);
            ls += p;
            const float* vr = vc + (size_t)(c0 + r) * KD + (size_t)g * HD;
            if (tid < HD) o0 = fmaf(p, vr[tid], o0);
            if (tid + 256 < HD) o1 = fmaf(p, vr[tid + 256], o1);
        }
        l_run = l_run * corr + ls;
        m_run = mn;
        __syncthreads();  // sc is rewritten by the next sub-chunk
    }
    const float il = 1.f / l_run;
    for (int k = 0; k < 2; k++) {
        const int d = tid + 256 * k;
        if (d >= HD) break;
        float r = (k ? o1 : o0) * il;
        if (gate) r *= 1.f / (1.f + expf(-gate[(size_t)h * gstride + d]));
        out[(size_t)h * HD + d] = r;
    }
}

// Group-shared split-T decode attention.  Block (g, s) handles kv head g
// and rows [t0, t1) for all REP q heads of the group, so every K / V element
// is read from memory once per block (the per-head kernel above reads it once
// per q head).  Rows are processed in sub-chunks of GQ_CH:
//   scores  wave w takes rows w, w + 4, ...; a lane holds DPL = HD/64 dims of
//           K and of each group q head, forms REP partial dots and reduces
//           them with a reduce-scatter (each halving lane-exchange stage leaves a
//           lane half of the heads), so a row costs REP - 1 + 6 - log2(REP)
//           exchanges instead of 6 * REP; scores go to LDS as [row][head]
//   softmax per head over the sub-chunk, merged into a running (m, l) with
//           the online rescale
//   P.V     thread (d, head group) owns HPT = REP*HD/256 outputs of dim d,
//           rescales them and accumulates p[row][head] * V[row][d]
// Each (q head, split) writes (o[HD], m, l) for k_attn_merge.
constexpr int GQ_CH = 32;

template <int HD, int REP, int NWV>
__global__ __launch_bounds__(64 * NWV) void k_attn_gqa(const float* __restrict__ q, const float* __restrict__ kc,
                                                       const float* __restrict__ vc, float* __restrict__ part,
                                                       const int* __restrict__ st, int layer, int NKV, int nsplit,
                                                       float scale) {
    // NWV waves: scores take rows w, w + NWV, ...; for P.V the threads past
    // the first 256 take further row ranges (RQ of them), whose sums meet in
    // LDS after the last sub-chunk
    constexpr int DPL = HD / 64, HPT = REP * HD / 256, RPW = GQ_CH / NWV, RQ = NWV / 4, RPQ = GQ_CH / RQ;
    static_assert(NWV == 4 || NWV == 8 || NWV == 16, "4, 8 or 16 waves");
    __shared__ float sc[GQ_CH * REP];
    __shared__ float mrun[REP], lrun[REP], corr[REP];
    __shared__ float ored[RQ > 1 ? (RQ - 1) * 256 * HPT : 1];
    const int g = blockIdx.x, s = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int KD = NKV * HD;
    const int Tn = st[1 + layer] + 1;
    const int chunk = (Tn + nsplit - 1) / nsplit;
    const int t0 = s * chunk, t1 = min(Tn, t0 + chunk);
    float qv[REP][DPL];
#pragma unroll
    for (int h = 0; h < REP; h++)
#pragma unroll
        for (int e = 0; e < DPL; e++) qv[h][e] = q[(size_t)(g * REP + h) * HD + DPL * lane + e];
    const int tb = tid & 255, rq = tid >> 8, d = tb % HD, hg = tb / HD;
    float o[HPT];
#pragma unroll
    for (int i = 0; i < HPT; i++) o[i] = 0.f;
    if (tid < REP) {
        mrun[tid] = -INFINITY;
        lrun[tid] = 0.f;
    }
    const float* kg = kc + (size_t)g * HD + DPL * lane;
    const float* vg = vc + (size_t)g * HD + d;
    for (int c0 = t0; c0 < t1; c0 += GQ_CH) {
        const int nr = min(GQ_CH, t1 - c0);
        // all loads of the sub-chunk first: K for this wave's rows, V for this
        // thread's dim over its row range
        float kx[RPW][DPL];
#pragma unroll
        for (int i = 0; i < RPW; i++) {
            const int t = min(c0 + w + NWV * i, t1 - 1);
#pragma unroll
            for (int e = 0; e < DPL; e++) kx[i][e] = kg[(size_t)t * KD + e];
        }
        float vv[RPQ];
#pragma unroll
        for (int r = 0; r < RPQ; r++) vv[r] = vg[(size_t)min(c0 + rq * RPQ + r, t1 - 1) * KD];
        __builtin_amdgcn_sched_barrier(0);  // every request of the sub-chunk before the first wait
        // reduce-scatter over the heads: each stage halves the heads a lane
        // holds and pairs it (lane_flip) with a lane keeping the other half;
        // the exchanges are DPP / permlane moves, no LDS traffic
        float pd[RPW][REP];
#pragma unroll
        for (int i = 0; i < RPW; i++)
#pragma unroll
            for (int h = 0; h < REP; h++) {
                float a = 0.f;
#pragma unroll
                for (int e = 0; e < DPL; e++) a = fmaf(qv[h][e], kx[i][e], a);
                pd[i][h] = a;
            }
        int hs = 0;
#pragma unroll
        for (int n = REP, m = 32; n > 1; n >>= 1, m >>= 1) {
            const bool up = (lane & m) != 0;
            hs += up ? n / 2 : 0;
#pragma unroll
            for (int i = 0; i < RPW; i++)
#pragma unroll
                for (int k = 0; k < n / 2; k++) {
                    const float send = up ? pd[i][k] : pd[i][k + n / 2];
                    const float keep = up ? pd[i][k + n / 2] : pd[i][k];
                    pd[i][k] = keep + lane_flip(send, m);
                }
        }
#pragma unroll
        for (int i = 0; i < RPW; i++) pd[i][0] = group_sum<64 / REP>(pd[i][0]);
#pragma unroll
        for (int i = 0; i < RPW; i++) {
            const int r = w + NWV * i;
            if ((lane & (64 / REP - 1)) == 0) sc[r * REP + hs] = r < nr ? pd[i][0] * scale : -INFINITY;
        }
        lds_barrier();
        // softmax: wave w takes heads 2w (lanes 0-31) and 2w+1 (lanes 32-63), then + 2 NWV
        for (int h = 2 * w + (lane >> 5); h < REP; h += 2 * NWV) {
            const int r = lane & 31;
            const float sv = sc[r * REP + h];
            const float cm = group_max<32>(sv);
            const float mo = mrun[h];
            const float mn = fmaxf(mo, cm);
            const float cr = mo == -INFINITY ? 0.f : expf(mo - mn);
            const float p = sv == -INFINITY ? 0.f : expf(sv - mn);
            const float ps = group_sum<32>(p);
            sc[r * REP + h] = p;
            if (r == 0) {
                mrun[h] = mn;
                lrun[h] = lrun[h] * cr + ps;
                corr[h] = cr;
            }
        }
        lds_barrier();
#pragma unroll
        for (int i = 0; i < HPT; i++) o[i] *= corr[hg * HPT + i];
#pragma unroll
        for (int r = 0; r < RPQ; r++) {
#pragma unroll
            for (int i = 0; i < HPT; i++) o[i] = fmaf(sc[(rq * RPQ + r) * REP + hg * HPT + i], vv[r], o[i]);
        }
        lds_barrier();  // sc / corr / mrun are rewritten by the next sub-chunk
    }
    if (RQ > 1) {
        if (rq > 0) {
#pragma unroll
            for (int i = 0; i < HPT; i++) ored[((rq - 1) * HPT + i) * 256 + tb] = o[i];
        }
        lds_barrier();
        if (rq > 0) return;
#pragma unroll
        for (int j = 0; j < RQ - 1; j++)
#pragma unroll
            for (int i = 0; i < HPT; i++) o[i] += ored[(j * HPT + i) * 256 + tb];
    }
#pragma unroll
    for (int i = 0; i < HPT; i++) part[((size_t)(g * REP + hg * HPT + i) * nsplit + s) * (HD + 2) + d] = o[i];
    if (tid < REP) {
        float* pp = part + ((size_t)(g * REP + tid) * nsplit + s) * (HD + 2);
        pp[HD] = mrun[tid];
        pp[HD + 1] = lrun[tid];
    }
}

// Merge the splits of one q head:
//   out[h] = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M),  M = max_s m_s
// Block (h, d0) of 4 waves covers head dims d0*64 .. d0*64+63; wave q sums the
// splits q, q+4, ... for its lane's dim and the four partial sums meet in
// LDS.  The partial loads of the first batch are issued before the split
// statistics are reduced, so the kernel costs about one memory round trip;
// loads are unconditional (indices clamped, weights of padding splits 0).
constexpr int MERGE_MAXS = 256;
constexpr int MERGE_BATCH = 32;

__global__ __launch_bounds__(256) void k_attn_merge(const float* __restrict__ part, float* __restrict__ out,
                                                    int nsplit, int HD, const float* __restrict__ gate,
                                                    int gstride) {
    __shared__ float wsh[MERGE_MAXS + 4 * MERGE_BATCH];
    __shared__ float red[2][4];
    __shared__ float accs[4][64];
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, q = tid >> 6;
    const int d = blockIdx.y * 64 + lane;
    const float* ph = part + (size_t)h * nsplit * (HD + 2);
    float pv[MERGE_BATCH];
#pragma unroll
    for (int j = 0; j < MERGE_BATCH; j++) pv[j] = ph[(size_t)min(q + 4 * j, nsplit - 1) * (HD + 2) + d];
    // split statistics: thread k holds split k's (m, l) (nsplit <= 256),
    // requested with the partials above
    const int kc = min(tid, nsplit - 1);
    const float mk0 = ph[(size_t)kc * (HD + 2) + HD], lk0 = ph[(size_t)kc * (HD + 2) + HD + 1];
    const bool ks = tid < nsplit;
    float mloc = ks ? mk0 : -INFINITY;
    mloc = wave_max(mloc);
    if (lane == 0) red[0][q] = mloc;
    lds_barrier();
    const float M = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    const float wk = !ks || mk0 == -INFINITY ? 0.f : expf(mk0 - M);
    float lsum = ks ? lk0 * wk : 0.f;
    wsh[tid] = wk;
    if (tid < 4 * MERGE_BATCH) wsh[MERGE_MAXS + tid] = 0.f;  // padding splits of the last batch
    lsum = wave_sum(lsum);
    if (lane == 0) red[1][q] = lsum;
    lds_barrier();
    const float L = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < MERGE_BATCH; j++) acc = fmaf(pv[j], wsh[q + 4 * j], acc);
    for (int k0 = 4 * MERGE_BATCH; k0 < nsplit; k0 += 4 * MERGE_BATCH) {
#pragma unroll
        for (int j = 0; j < MERGE_BATCH; j++) pv[j] = ph[(size_t)min(k0 + q + 4 * j, nsplit - 1) * (HD + 2) + d];
#pragma unroll
        for (int j = 0; j < MERGE_BATCH; j++) acc = fmaf(pv[j], wsh[k0 + q + 4 * j], acc);
    }
    accs[q][lane] = acc;
    lds_barrier();
    if (q == 0) {
        float r = ((accs[0][lane] + accs[1][lane]) + (accs[2][lane] + accs[3][lane])) * (1.f / L);
        if (gate) r *= 1.f / (1.f + expf(-gate[(size_t)h * gstride + d]));
        out[(size_t)h * HD + d] = r;
    }
}

// Merge the splits of one q head (block), one thread per head dim.  Lane k
// of each wave holds split k's (m, l); the weights exp(m_k - M) are
// broadcast with readlane, and all of a lane's partial loads are issued
// before the first FMA, so the kernel costs two dependent L2 round trips.
// With `gate` set the result is multiplied by sigmoid(gate[h * gstride + d])
// (qwen35 full attention, src/m6_layer.c:500-505).
// Block b merges q head h = (b % NKV) rep + b / NKV.  Blocks are dispatched
// round-robin over the XCDs, and k_attn_part's block (g, s) is linear block
// g + NKV s, so with NKV = 8 every split of kv head g ran on XCD g; this
// order puts the merges of g's q heads on XCD g too, where the partials are
// still in L2.
template <int MAXS>
__global__ __launch_bounds__(256) void k_attn_combine(const float* __restrict__ part, float* __restrict__ out,
                                                      int nsplit, int HD, const float* __restrict__ gate,
                                                      int gstride, int NKV) {
    const int b = blockIdx.x, rep = gridDim.x / NKV;
    const int h = (b % NKV) * rep + b / NKV, tid = threadIdx.x, lane = tid & 63;
    const float* ph = part + (size_t)h * nsplit * (HD + 2);
    // every load unconditional (clamped split index), so all of them are in
    // flight together: one memory round trip
    const int kl = min(lane, nsplit - 1);
    const float m0 = ph[kl * (HD + 2) + HD], l0 = ph[kl * (HD + 2) + HD + 1];
    float pv[MAXS];
#pragma unroll
    for (int k = 0; k < MAXS; k++) pv[k] = ph[min(k, nsplit - 1) * (HD + 2) + tid];
    const float m = lane < nsplit ? m0 : -INFINITY;
    const float lk = lane < nsplit ? l0 : 0.f;
    const float M = wave_max(m);
    const float wk = m > -INFINITY ? expf(m - M) : 0.f;
    const float L = wave_sum(lk * wk);
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < MAXS; k++) {  // lanes k >= nsplit carry weight 0
        acc = fmaf(pv[k], __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wk), k)), acc);
    }
    // the block is HD threads (no guard: a store under a thread test would let
    // the compiler sink the partial loads below the statistics' reductions)
    float r = acc * (1.f / L);
    if (gate) r *= 1.f / (1.f + expf(-gate[(size_t)h * gstride + tid]));
    out[(size_t)h * HD + tid] = r;
}

// The split merge fused with the o projection (Q4_K / Q6_K tile layout):
// input super-block c of the o rows is chunk c, the 256 attention outputs
// 256 c .. 256 c + 255 (q heads 4c .. 4c+3 at head dim 64, 2c, 2c+1 at 128,
// c at 256).  Block b takes chunk c = b % NC and row tiles 4 (b / NC) .. +3.
// Wave w first requests its tile's item c (the weights stream while the
// merge runs), then merges outputs 256 c + 64 w .. + 63 (one head's 64 dims,
// or a quarter / half of one, with that head's split statistics) as
// k_attn_combine does (statistics and partials in one round trip); wave 0
// digitises the 256 merged values (as k_dq's prologue) and every wave
// multiplies its tile.
// The chunks' contributions W[row, 256c .. 256c + 255] . att[256c ..] meet
// in acc[row] as 64-bit fixed point (round(v * 2^32), agent-scope atomic
// adds): integer addition is associative, so the sum is the same bit for
// bit whatever order the blocks arrive in, and the consumer (the gate/up
// launch's PRES8 prologue) reads one vector instead of NC.  A non-finite or
// out-of-range contribution sets acc[n_out] instead, which makes the
// consumer's input NaN, as the reference's fp32 sum would be.  The grid also
// clears zacc[0 .. zn) (the previous fused layer's accumulator, consumed
// before this launch).  With NC = 8 kv groups of 4 heads block b
// runs on XCD b mod 8, the XCD that ran the splits of kv head c (k_attn_part's
// block (c, s) is linear block c + 8 s).
template <int FM, int MAXS, int HD>
__global__ __launch_bounds__(256) void k_attn_o(const float* __restrict__ part, int nsplit,
                                                const uint8_t* __restrict__ wo, int nb, int n_out, int NC,
                                                unsigned long long* __restrict__ acc,
                                                unsigned long long* __restrict__ zacc, int zn) {
    static_assert(HD == 64 || HD == 128 || HD == 256, "chunk = whole heads or parts of one");
    constexpr size_t IB = FM == 1 ? DRACO_Q4T_ITEM : DRACO_Q6T_ITEM;
    __shared__ __align__(16) float att[256];
    __shared__ __align__(16) int8_t xd[1024];
    __shared__ __align__(16) int8_t zero[1024];
    __shared__ float2 xsm[16];
    const int b = blockIdx.x, c = b % NC, rr = b / NC;
    const int tid = threadIdx.x, lane = tid & 63, j = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: the item's descriptor in SGPRs
    const int ntiles = (n_out + 15) >> 4;
    const int T = rr * 4 + w, Tc = T < ntiles ? T : ntiles - 1;
    // merge outputs 256 c + 64 w + lane: head (256 c + 64 w) / HD, dim
    // (64 w) % HD + lane; every load unconditional (clamped split index)
    const int hh = (256 * c + 64 * w) / HD, dd = (64 * w) % HD + lane;
    const float* ph = part + (size_t)hh * nsplit * (HD + 2);
    const int kl = min(lane, nsplit - 1);
    const float m0 = ph[kl * (HD + 2) + HD], l0 = ph[kl * (HD + 2) + HD + 1];
    float pv[MAXS];
#pragma unroll
    for (int k = 0; k < MAXS; k++) pv[k] = ph[min(k, nsplit - 1) * (HD + 2) + dd];
    // the o item after the partials: the merge needs them first, the dot
    // this (requested before the first wait all the same)
    __builtin_amdgcn_sched_barrier(0);
    Frag f;
    const uint8_t* item = wo + ((size_t)Tc * nb + c) * IB;
    if (FM == 1) load_q4b(item, lane, f);
    else load_q6b(item, lane, f);
    reinterpret_cast<uint32_t*>(zero)[tid] = 0u;
    for (int i = b * 256 + tid; i < zn; i += gridDim.x * 256) zacc[i] = 0ull;
    const float m = lane < nsplit ? m0 : -INFINITY;
    const float lk = lane < nsplit ? l0 : 0.f;
    const float M = wave_max(m);
    const float wk = m > -INFINITY ? expf(m - M) : 0.f;
    const float L = wave_sum(lk * wk);
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < MAXS; k++)  // lanes k >= nsplit carry weight 0
        s = fmaf(pv[k], __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wk), k)), s);
    att[w * 64 + lane] = s * (1.f / L);
    lds_barrier();
    if (w == 0) digits4(reinterpret_cast<const float4*>(att)[lane], lane, xd, xsm);
    lds_barrier();
    const bool adig = (j >> 2) == g;
    float v;
    if (FM == 1) {
        const int gl4 = 4 * (g >> 1) + (g & 1);
        const float2 r = dot_q4(f, adig ? xd + (gl4 * 4 + (j & 3)) * 16 : zero, xsm, gl4, g);
        v = r.x - r.y;
    } else {
        const int gl6 = 8 * (g >> 1) + (g & 1);
        v = dot_q6(f, adig ? xd + (gl6 * 4 + (j & 3)) * 16 : zero, xsm, gl6);
    }
    v = rows_sum(v);
    const int row = T * 16 + j;
    if (lane < 16 && T < ntiles && row < n_out) {
        const float sv = v * 4294967296.f;  // 2^32
        if (fabsf(sv) < 9.0e18f) {          // |round(sv)| < 2^63, and not NaN
            atomicAdd(acc + row, (unsigned long long)(long long)rintf(sv));
        } else {
            atomicOr(acc + n_out, 1ull);
        }
    }
}

// The same fusion for a Q8_0 o projection (head dim 64, REP q heads per kv
// head, REP <= 4).  Chunk c is kv group c: q heads c REP .. c REP + REP - 1,
// the 2 REP blocks [2 c REP, 2 c REP + 2 REP) of every o row.  Block b takes
// chunk c = b % NC and rows 32 (b / NC) .. + 31; wave w < REP merges the
// splits of head c REP + w (k_attn_combine's single memory round trip) into
// LDS, while every wave's lanes (r, k) = (lane >> 3, lane & 7) already hold
// row 32 (b / NC) + 8 w + r's block 2 c REP + k (k < 2 REP; the other lanes
// re-read a real block and contribute nothing), requested first.  Each lane
// dots its 32 quants with the 32 merged values of its block, the 8 lanes of
// a row sum, and the row's contribution meets the other chunks' in acc[row]
// as 64-bit fixed point (as k_attn_o: order-independent integer sums, a
// flag at acc[n_out] for a non-finite or out-of-range value).  The merged
// values sit in LDS with a 36-float stride per 32-value block, so the 8
// blocks a row's lanes read fall in different banks.
template <int MAXS, int REP>
__global__ __launch_bounds__(256) void k_attn_o8(const float* __restrict__ part, int nsplit,
                                                 const uint8_t* __restrict__ qs, const uint8_t* __restrict__ ds,
                                                 int nb, int n_out, int NC, unsigned long long* __restrict__ acc,
                                                 unsigned long long* __restrict__ zacc, int zn) {
    constexpr int HD = 64, KB = 2 * REP;  // blocks of the chunk
    __shared__ __align__(16) float att[8 * 36];
    const int b = blockIdx.x, c = b % NC, rb = b / NC;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane >> 3, k = lane & 7;
    const int row = rb * 32 + w * 8 + r, rc = row < n_out ? row : n_out - 1;
    const int kc = k < KB ? k : KB - 1;
    const size_t blk = (size_t)rc * nb + (size_t)c * KB + kc;
    const uint4 q0 = ldnt4(qs + blk * 32), q1 = ldnt4(qs + blk * 32 + 16);
    const uint16_t dh = *reinterpret_cast<const uint16_t*>(ds + blk * 2);
    // merge head c REP + w (waves w < REP): every load unconditional
    const int hw = w < REP ? w : REP - 1;
    const float* ph = part + (size_t)(c * REP + hw) * nsplit * (HD + 2);
    const int kl = min(lane, nsplit - 1);
    const float m0 = ph[kl * (HD + 2) + HD], l0 = ph[kl * (HD + 2) + HD + 1];
    float pv[MAXS];
#pragma unroll
    for (int s = 0; s < MAXS; s++) pv[s] = ph[min(s, nsplit - 1) * (HD + 2) + lane];
    for (int i = b * 256 + tid; i < zn; i += gridDim.x * 256) zacc[i] = 0ull;
    const float m = lane < nsplit ? m0 : -INFINITY;
    const float lk = lane < nsplit ? l0 : 0.f;
    const float M = wave_max(m);
    const float wk = m > -INFINITY ? expf(m - M) : 0.f;
    const float L = wave_sum(lk * wk);
    float sacc = 0.f;
#pragma unroll
    for (int s = 0; s < MAXS; s++)  // lanes s >= nsplit carry weight 0
        sacc = fmaf(pv[s], __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wk), s)), sacc);
    // head w's dims 0..31 are chunk block 2w, 32..63 block 2w + 1
    if (w < REP) att[(2 * w + (lane >> 5)) * 36 + (lane & 31)] = sacc * (1.f / L);
    lds_barrier();
    const float* xa = att + kc * 36;
    const uint32_t Q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    float d = 0.f;
#pragma unroll
    for (int dw = 0; dw < 8; dw++) {
        const float4 x4 = *reinterpret_cast<const float4*>(xa + 4 * dw);
        d = fmaf(sbyte_f(Q[dw], 0), x4.x, d);
        d = fmaf(sbyte_f(Q[dw], 1), x4.y, d);
        d = fmaf(sbyte_f(Q[dw], 2), x4.z, d);
        d = fmaf(sbyte_f(Q[dw], 3), x4.w, d);
    }
    float v = k < KB ? h2f(dh) * d : 0.f;
    v = group_sum<8>(v);
    if (k == 0 && row < n_out) {
        const float sv = v * 4294967296.f;  // 2^32
        if (fabsf(sv) < 9.0e18f) {          // |round(sv)| < 2^63, and not NaN
            atomicAdd(acc + row, (unsigned long long)(long long)rintf(sv));
        } else {
            atomicOr(acc + n_out, 1ull);
        }
    }
}

// Short caches (at most ATT_SHORT_T rows in this call): the whole attention of
// kv group c runs inside every o-projection block of chunk c, with no splits
// and no merge, and the Q8_0 o projection follows as in k_attn_o8 (one launch
// instead of the split attention and k_attn_o8).  Each of the NKV chunks is
// recomputed by its ceil(n_out / 32) row groups from L2-resident K / V rows
// (the row groups of one chunk read the same rows).  Block b: chunk c = b % NC,
// rows 32 (b / NC) .. + 31.  All loads are requested first: the o rows'
// quants (lane (r, k) as k_attn_o8), the group's q (into LDS), K row t =
// 32 w + lane / 2 for lane pair half lane & 1 (32 dims, 8 float4), V rows
// t = w + 4 i (i < 32) at dim lane, every row index clamped below tcap.
// Then: scores of the REP heads for the wave's K rows (a 2-lane sum; rows at
// or past the cache length are -inf), softmax per head over the rows by wave
// h (max, exp, sum; the probabilities unnormalised in LDS), P.V of each
// wave's V rows for every head, the 4 waves' sums added in LDS and divided
// by the head's sum.  Results agree with the split form to fp32 rounding.
constexpr int ATT_SHORT_T = 128;

// Every argument the first loads need comes within the 14 dwords the
// dispatcher preloads into SGPRs: ncn packs NC (bits 0-7) and n_out (from
// bit 8), tn points at the layer's cache length (state + 1 + layer), and the
// row stride in blocks is NC * KB (the o projection's n_in is NC * REP * 64).
template <int REP>
__global__ __launch_bounds__(256) void k_attn_o8s(const uint8_t* __restrict__ qs, const uint8_t* __restrict__ ds,
                                                  int ncn, const float* __restrict__ q, const float* __restrict__ kc,
                                                  const float* __restrict__ vc, int tcap, const int* __restrict__ tn,
                                                  float scale, unsigned long long* __restrict__ acc,
                                                  unsigned long long* __restrict__ zacc, int zn) {
    constexpr int HD = 64, KB = 2 * REP;
    const int NC = ncn & 255, n_out = ncn >> 8, nb = NC * KB;
    __shared__ __align__(16) float qsh[REP * HD];
    __shared__ float psh[REP][ATT_SHORT_T];
    __shared__ float lsh[REP];
    __shared__ __align__(16) float osh[4][REP][HD];
    __shared__ __align__(16) float att[8 * 36];
    const int b = blockIdx.x, c = b % NC, rb = b / NC;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane >> 3, k = lane & 7;
    const int KD = NC * HD;  // NC = NKV: one chunk per kv group
    // the group's q (REP heads of 64): one float4 per thread of the first REP * 16
    const int qi = tid < REP * 16 ? tid : 0;
    const float4 qv4 = ld4(q + (size_t)c * REP * HD + 4 * qi);
    // K: row tk = 32 w + lane / 2, dims 32 (lane & 1) .. + 31
    const int tk = 32 * w + (lane >> 1), half = lane & 1;
    const int tkc = tk < tcap ? tk : tcap - 1;
    float4 kx[8];
#pragma unroll
    for (int i = 0; i < 8; i++) kx[i] = ld4(kc + (size_t)tkc * KD + c * HD + 32 * half + 4 * i);
    // V: rows w + 4 i at dim lane
    float vv[ATT_SHORT_T / 4];
#pragma unroll
    for (int i = 0; i < ATT_SHORT_T / 4; i++) {
        const int t = w + 4 * i, tc = t < tcap ? t : tcap - 1;
        vv[i] = vc[(size_t)tc * KD + c * HD + lane];
    }
    const int Tn = *tn + 1;
    // o rows' quants (as k_attn_o8), requested last: the scores need q and
    // K first, the o dot these
    const int row = rb * 32 + w * 8 + r, rc = row < n_out ? row : n_out - 1;
    const int kcb = k < KB ? k : KB - 1;
    const size_t blk = (size_t)rc * nb + (size_t)c * KB + kcb;
    const uint4 q0 = ldnt4(qs + blk * 32), q1 = ldnt4(qs + blk * 32 + 16);
    const uint16_t dh = *reinterpret_cast<const uint16_t*>(ds + blk * 2);
    __builtin_amdgcn_sched_barrier(0);  // every request before the first wait
    for (int i = b * 256 + tid; i < zn; i += gridDim.x * 256) zacc[i] = 0ull;
    if (tid < REP * 16) reinterpret_cast<float4*>(qsh)[tid] = qv4;
    lds_barrier();
    // scores of the wave's K rows for the REP heads
    const bool kval = tk < Tn;
#pragma unroll
    for (int h = 0; h < REP; h++) {
        const float4* qh = reinterpret_cast<const float4*>(qsh + h * HD + 32 * half);
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 a = qh[i];
            s = fmaf(a.x, kx[i].x, s);
            s = fmaf(a.y, kx[i].y, s);
            s = fmaf(a.z, kx[i].z, s);
            s = fmaf(a.w, kx[i].w, s);
        }
        s = group_sum<2>(s);
        if (half == 0) psh[h][tk] = kval ? s * scale : -INFINITY;
    }
    lds_barrier();
    // softmax of head h over the rows (wave h; lanes hold rows lane, lane + 64)
    if (w < REP) {
        const float s0 = psh[w][lane], s1 = psh[w][lane + 64];
        const float m = wave_max(fmaxf(s0, s1));
        const float p0 = s0 == -INFINITY ? 0.f : expf(s0 - m), p1 = s1 == -INFINITY ? 0.f : expf(s1 - m);
        const float l = wave_sum(p0 + p1);
        psh[w][lane] = p0;
        psh[w][lane + 64] = p1;
        if (lane == 0) lsh[w] = l;
    }
    lds_barrier();
    // P.V over the wave's V rows, every head
    float o[REP];
#pragma unroll
    for (int h = 0; h < REP; h++) o[h] = 0.f;
#pragma unroll
    for (int i = 0; i < ATT_SHORT_T / 4; i++) {
        const int t = w + 4 * i;
        const float v = t < Tn ? vv[i] : 0.f;  // rows past the length may hold anything
#pragma unroll
        for (int h = 0; h < REP; h++) o[h] = fmaf(psh[h][t], v, o[h]);
    }
#pragma unroll
    for (int h = 0; h < REP; h++) osh[w][h][lane] = o[h];
    lds_barrier();
    if (w < REP) {
        const float sum = (osh[0][w][lane] + osh[1][w][lane]) + (osh[2][w][lane] + osh[3][w][lane]);
        att[(2 * w + (lane >> 5)) * 36 + (lane & 31)] = sum * (1.f / lsh[w]);
    }
    lds_barrier();
    // the o projection of the chunk (as k_attn_o8)
    const float* xa = att + kcb * 36;
    const uint32_t Q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    float d = 0.f;
#pragma unroll
    for (int dw = 0; dw < 8; dw++) {
        const float4 x4 = *reinterpret_cast<const float4*>(xa + 4 * dw);
        d = fmaf(sbyte_f(Q[dw], 0), x4.x, d);
        d = fmaf(sbyte_f(Q[dw], 1), x4.y, d);
        d = fmaf(sbyte_f(Q[dw], 2), x4.z, d);
        d = fmaf(sbyte_f(Q[dw], 3), x4.w, d);
    }
    float v = k < KB ? h2f(dh) * d : 0.f;
    v = group_sum<8>(v);
    if (k == 0 && row < n_out) {
        const float sv = v * 4294967296.f;  // 2^32
        if (fabsf(sv) < 9.0e18f) {
            atomicAdd(acc + row, (unsigned long long)(long long)rintf(sv));
        } else {
            atomicOr(acc + n_out, 1ull);
        }
    }
}

// qwen35 full attention, per-head RMSNorm over 256 dims and rope on the pairs
// (t, t + 32), t < 32 (src/m6_layer.c:427-457).  Blocks 0..NH-1 normalise q
// head b from QG[b * 512 .. + 256] into Qr[b * 256] as (x * r) * q_norm; blocks
// NH, NH + 1 normalise k head kv from kin[kv * 256] into kout[kv * 256] as
// x * (r * k_norm), the two association orders of the reference.  cs holds
// [32][cos, sin] of pos0 * rope_inv[t].  Rope partners t and t + 32 are lanes
// of wave 0 and swap values with one permlane32 swap.
__global__ __launch_bounds__(256) void k_fa_prep(const float* __restrict__ QG, float* __restrict__ Qr,
                                                 const float* __restrict__ kin, float* __restrict__ kout,
                                                 const float* __restrict__ qn, const float* __restrict__ kn,
                                                 const float* __restrict__ cs, int NH) {
    __shared__ float red[4];
    const int b = blockIdx.x, t = threadIdx.x, lane = t & 63, w = t >> 6;
    const bool isq = b < NH;
    const float x = isq ? QG[(size_t)b * 512 + t] : kin[(b - NH) * 256 + t];
    const float s = wave_sum(x * x);
    if (lane == 0) red[w] = s;
    __syncthreads();
    const float n2 = (red[0] + red[1]) + (red[2] + red[3]);
    const float r = 1.f / sqrtf(n2 / 256.f + 1e-6f);
    float y = isq ? x * r * qn[t] : x * (r * kn[t]);
    if (w == 0) {
        const float o = lane_xor32(y);
        const float c = cs[2 * (lane & 31)], sn = cs[2 * (lane & 31) + 1];
        y = lane < 32 ? y * c - o * sn : o * sn + y * c;
    }
    (isq ? Qr + (size_t)b * 256 : kout + (b - NH) * 256)[t] = y;
}

// The same head norms and rope for T tokens whose positions and cache rows
// come from the device (graph-replayable): token t sits at position
// p = (state ? state[0] : pos0) + t and cache row r = (state ? state[1] : row0)
// + t.  Block (b, t): b < NH normalises + ropes q head b of QG[t] (row
// stride qg_stride) into Qr[t]; b = NH + g normalises + ropes k head g of
// kin[t] into kc row r and copies v head g of vin[t] into vc row r.  The
// rope's cos / sin come from cs_tab row p (64 floats: the reference's
// (float)pos * rope_inv[t] angle, computed on the host).
// The operands of the first loads lead the arguments (the first 14 dwords
// arrive in SGPRs); the head's value, its norm weight and the v value are
// requested before the position is read from the state, whose rope row
// follows (the one dependent load).
__global__ __launch_bounds__(256) void k_fa_prep_rows(const float* __restrict__ QG, const float* __restrict__ kin,
                                                      const float* __restrict__ vin, const float* __restrict__ qn,
                                                      const float* __restrict__ kn, const int* __restrict__ state,
                                                      int qg_stride, int NH, const float* __restrict__ cs_tab,
                                                      float* __restrict__ Qr, float* __restrict__ kc,
                                                      float* __restrict__ vc, int pos0, int row0) {
    __shared__ float red[4];
    const int b = blockIdx.x, tok = blockIdx.y, t = threadIdx.x, lane = t & 63, w = t >> 6;
    const bool isq = b < NH;
    const int g = b - NH;
    const float* xp = isq ? QG + (size_t)tok * qg_stride + (size_t)b * 512 : kin + (size_t)tok * 512 + g * 256;
    const float* vp = vin + (size_t)tok * 512 + (isq ? 0 : g * 256);
    const float x = xp[t], nwt = (isq ? qn : kn)[t], vv = vp[t];
    // state[0..1] in one 8-byte load (the device state array is 8-byte aligned)
    const int2 pr = state ? *reinterpret_cast<const int2*>(state) : make_int2(pos0, row0);
    const int pos = pr.x + tok, row = pr.y + tok;
    const float* cs = cs_tab + (size_t)pos * 64;
    const float c = cs[2 * (lane & 31)], sn = cs[2 * (lane & 31) + 1];
    if (!isq) vc[(size_t)row * 512 + g * 256 + t] = vv;
    const float s = wave_sum(x * x);
    if (lane == 0) red[w] = s;
    lds_barrier();
    const float n2 = (red[0] + red[1]) + (red[2] + red[3]);
    const float r = 1.f / sqrtf(n2 / 256.f + 1e-6f);
    float y = isq ? x * r * nwt : x * (r * nwt);
    if (w == 0) {
        const float o = lane_xor32(y);
        y = lane < 32 ? y * c - o * sn : o * sn + y * c;
    }
    if (isq) Qr[(size_t)tok * NH * 256 + (size_t)b * 256 + t] = y;
    else kc[(size_t)row * 512 + g * 256 + t] = y;
}

// -------------------------------------------------------------- SwiGLU --
__global__ __launch_bounds__(256) void k_swiglu(float* __restrict__ g, const float* __restrict__ u, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const float gv = g[i];
        g[i] = (gv / (1.f + expf(-gv))) * u[i];
    }
}

// out[i] = y[i] * sigmoid(g[0]): the shared expert's scalar gate
// (src/m6_engine.c:1125-1126)
__global__ __launch_bounds__(256) void k_sigmoid_scale(const float* __restrict__ y, const float* __restrict__ g,
                                                       float* __restrict__ out, int n) {
    const float s = 1.0f / (1.0f + expf(-g[0]));
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) out[i] = y[i] * s;
}

// out[i] = y[i] * sigmoid(x . g) for a one-row fp32 / fp16 gate g of n
// values (n % 4 == 0): every block forms the dot (tree sum, 4 wave sums in
// order) and scales its slice; block 0 also stores the dot in gdot[0].
__global__ __launch_bounds__(256) void k_gate_scale(const float* __restrict__ x, const void* __restrict__ g,
                                                    int f16, const float* __restrict__ y, float* __restrict__ out,
                                                    float* __restrict__ gdot, int n) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    __shared__ float red[4];
    const int tid = threadIdx.x;
    float acc = 0.f;
    for (int i = tid * 4; i < n; i += 1024) {
        const float4 a = ld4(x + i);
        float4 b;
        if (f16) {
            const h4 v = *reinterpret_cast<const h4*>(reinterpret_cast<const _Float16*>(g) + i);
            b = make_float4((float)v.x, (float)v.y, (float)v.z, (float)v.w);
        } else {
            b = ld4(reinterpret_cast<const float*>(g) + i);
        }
        acc = fmaf(a.x, b.x, acc);
        acc = fmaf(a.y, b.y, acc);
        acc = fmaf(a.z, b.z, acc);
        acc = fmaf(a.w, b.w, acc);
    }
    acc = wave_sum(acc);
    if ((tid & 63) == 0) red[tid >> 6] = acc;
    lds_barrier();
    const float d = (red[0] + red[1]) + (red[2] + red[3]);
    const float sgm = 1.0f / (1.0f + expf(-d));
    if (blockIdx.x == 0 && tid == 0) gdot[0] = d;
    for (int i = blockIdx.x * 256 + tid; i < n; i += gridDim.x * 256) out[i] = y[i] * sgm;
}

// ---------------------------------------------------------- embedding --
// Dequantize row `tok` of a private-layout matrix into out[n_in]
// (embed_value, embed_dev.h).
__global__ __launch_bounds__(256) void k_embed(const uint8_t* __restrict__ base, DracoLayout L,
                                               const int* __restrict__ ids, const int* __restrict__ cursor,
                                               float* __restrict__ out) {
    const int tok = ids[cursor ? cursor[0] : 0];
    for (int p = blockIdx.x * blockDim.x + threadIdx.x; p < L.n_in; p += gridDim.x * blockDim.x)
        out[p] = embed_value(base, L, tok, p);
}

// -------------------------------------------------------------- argmax --
// First index of the maximum (np.argmax semantics).  Stage 1: per-block
// (value, index); stage 2: one block reduces the partials.
__global__ __launch_bounds__(256) void k_argmax_part(const float* __restrict__ x, int n, float* __restrict__ pv,
                                                     int* __restrict__ pi) {
    float v = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) am_merge(v, idx, x[i], i);
    group_argmax<64>(v, idx);
    __shared__ float sv[4];
    __shared__ int si[4];
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = v;
        si[threadIdx.x >> 6] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) am_merge(v, idx, sv[w], si[w]);
        pv[blockIdx.x] = v;
        pi[blockIdx.x] = idx;
    }
}

__global__ __launch_bounds__(64) void k_argmax_final(const float* __restrict__ pv, const int* __restrict__ pi,
                                                     int nb, int* __restrict__ out, const int* __restrict__ slotp,
                                                     int slot) {
    float v = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = threadIdx.x; i < nb; i += 64) am_merge(v, idx, pv[i], pi[i]);
    group_argmax<64>(v, idx);
    // no partial at all: token 0, never an out-of-range row
    if (threadIdx.x == 0) out[slotp ? slotp[0] + 1 : slot] = idx == 0x7fffffff ? 0 : idx;
}

// ------------------------------------------------------ token advance --
// After a token: pos += 1, every layer's tlen += 1, next token slot.
__global__ void k_advance(int* st, int n_layer, int* tok_cursor) {
    if (threadIdx.x == 0) {
        st[0] += 1;
        for (int l = 0; l < n_layer; l++) st[1 + l] += 1;
        if (tok_cursor) tok_cursor[0] += 1;
    }
}

// copy token ids[cursor] -> cur (used by the graph: embed reads cur)
__global__ void k_pick_token(const int* ids, const int* cursor, int* cur) {
    if (threadIdx.x == 0) cur[0] = ids[cursor[0]];
}

}  // namespace

// ------------------------------------------------------------ launchers --
void dk_rmsnorm(const float* x, const float* w, float* out, int h, float eps, hipStream_t st) {
    // one block; enough threads that each holds at most RMS_PER_THREAD values
    if (h > 1024 * RMS_PER_THREAD) {
        hipLaunchKernelGGL(k_rmsnorm_loop, dim3(1), dim3(1024), 0, st, x, w, out, h, eps);
        return;
    }
    int nt = 64;
    while (nt < 1024 && nt * RMS_PER_THREAD < h) nt *= 2;
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(nt), 0, st, x, w, out, h, eps);
}

void dk_rope_append(float* q, const float* k, const float* v, float* kc, float* vc, const float* tab,
                    const int* state, int layer, int NH, int NKV, int HD, int rot, hipStream_t st) {
    const int n = NH * HD + 2 * NKV * HD;
    const int blocks = (n + 255) / 256;
    hipLaunchKernelGGL(k_rope_append, dim3(blocks), dim3(256), 0, st, q, k, v, kc, vc, tab, state, layer, NH,
                       NKV, HD, rot);
}

// Waves per block of k_attn_gqa.  8 measured best on MI355X: configs[3]
// (head dim 128, 8 q heads per kv head, 16 splits) 595 -> 601 tok/s against
// 4 waves, configs[4] (head dim 256, 130 splits) within its spread; 16 no
// better than 4.
static int g_gqa_waves = 8;
extern "C" int draco_set_gqa_waves(int n) {
    const int old = g_gqa_waves;
    if (n == 4 || n == 8 || n == 16) g_gqa_waves = n;
    return old;
}

int dk_attention(const float* q, const float* kc, const float* vc, float* part, unsigned* count, float* out,
                 const int* state, int layer, int NH, int NKV, int HD, int max_t, float scale, hipStream_t st,
                 const float* gate, int gstride) {
    (void)count;
    if (NKV < 1 || NH < NKV || NH % NKV || HD < 2 || HD > 512 || (HD & 1)) return -1;
    const int rep = NH / NKV;
    if (!attn_grouped(NH, NKV, HD) && !attn_per_head(NH, NKV, HD)) {
        hipLaunchKernelGGL(k_attn_any, dim3(NH), dim3(256), 0, st, q, kc, vc, out, state, layer, NH, NKV, HD, scale,
                           gate, gstride);
        return 0;
    }
    const int nsplit = attn_nsplit(max_t, NH, NKV, HD);
    if (attn_grouped(NH, NKV, HD)) {
        const dim3 grid(NKV, nsplit);
#define GQA_CASE(H_, R_)                                                                                  \
    if (HD == H_ && rep == R_) {                                                                          \
        if (g_gqa_waves == 16)                                                                            \
            hipLaunchKernelGGL((k_attn_gqa<H_, R_, 16>), grid, dim3(1024), 0, st, q, kc, vc, part, state, \
                               layer, NKV, nsplit, scale);                                                \
        else if (g_gqa_waves == 8)                                                                        \
            hipLaunchKernelGGL((k_attn_gqa<H_, R_, 8>), grid, dim3(512), 0, st, q, kc, vc, part, state,   \
                               layer, NKV, nsplit, scale);                                                \
        else                                                                                              \
            hipLaunchKernelGGL((k_attn_gqa<H_, R_, 4>), grid, dim3(256), 0, st, q, kc, vc, part, state,   \
                               layer, NKV, nsplit, scale);                                                \
    } else
        // the shapes attn_grouped sends here: head dim 128 with GQA <= 8
        // (llama attention) and head dim 256 with GQA <= 16 (qwen35 full
        // attention)
        GQA_CASE(128, 2) GQA_CASE(128, 4) GQA_CASE(128, 8)
        GQA_CASE(256, 2) GQA_CASE(256, 4) GQA_CASE(256, 8) GQA_CASE(256, 16) return -1;
#undef GQA_CASE
        hipLaunchKernelGGL(k_attn_merge, dim3(NH, HD / 64), dim3(256), 0, st, part, out, nsplit, HD, gate, gstride);
        return 0;
    }
    const dim3 grid(NKV, nsplit), block(64 * rep);
    if (HD == 64)
        hipLaunchKernelGGL(k_attn_part<64>, grid, block, 0, st, q, kc, vc, part, state, layer, NH, NKV, nsplit, scale);
    else if (HD == 128)
        hipLaunchKernelGGL(k_attn_part<128>, grid, block, 0, st, q, kc, vc, part, state, layer, NH, NKV, nsplit,
                           scale);
    else if (HD == 256)
        hipLaunchKernelGGL(k_attn_part<256>, grid, block, 0, st, q, kc, vc, part, state, layer, NH, NKV, nsplit,
                           scale);
    else
        return -1;
    const dim3 cg(NH), cb(HD);
    if (nsplit <= 16)
        hipLaunchKernelGGL(k_attn_combine<16>, cg, cb, 0, st, part, out, nsplit, HD, gate, gstride, NKV);
    else if (nsplit <= 32)
        hipLaunchKernelGGL(k_attn_combine<32>, cg, cb, 0, st, part, out, nsplit, HD, gate, gstride, NKV);
    else
        hipLaunchKernelGGL(k_attn_combine<64>, cg, cb, 0, st, part, out, nsplit, HD, gate, gstride, NKV);
    return 0;
}

int dk_attention_parts(const float* q, const float* kc, const float* vc, float* part, const int* state, int layer,
                       int NH, int NKV, int HD, int max_t, float scale, hipStream_t st) {
    const int nsplit = attn_nsplit(max_t, NH, NKV, HD);
    if (attn_grouped(NH, NKV, HD)) {
        const int rep = NH / NKV;
        const dim3 grid(NKV, nsplit);
#define GQA_CASE(H_, R_)                                                                                  \
    if (HD == H_ && rep == R_) {                                                                          \
        if (g_gqa_waves == 16)                                                                            \
            hipLaunchKernelGGL((k_attn_gqa<H_, R_, 16>), grid, dim3(1024), 0, st, q, kc, vc, part, state, \
                               layer, NKV, nsplit, scale);                                                \
        else if (g_gqa_waves == 8)                                                                        \
            hipLaunchKernelGGL((k_attn_gqa<H_, R_, 8>), grid, dim3(512), 0, st, q, kc, vc, part, state,   \
                               layer, NKV, nsplit, scale);                                                \
        else                                                                                              \
            hipLaunchKernelGGL((k_attn_gqa<H_, R_, 4>), grid, dim3(256), 0, st, q, kc, vc, part, state,   \
                               layer, NKV, nsplit, scale);                                                \
    } else
        GQA_CASE(128, 2) GQA_CASE(128, 4) GQA_CASE(128, 8)
        GQA_CASE(256, 2) GQA_CASE(256, 4) GQA_CASE(256, 8) GQA_CASE(256, 16) return -1;
#undef GQA_CASE
        return 0;
    }
    if (!attn_per_head(NH, NKV, HD)) return -1;
    const dim3 grid(NKV, nsplit), block(64 * (NH / NKV));
    if (HD == 64)
        hipLaunchKernelGGL(k_attn_part<64>, grid, block, 0, st, q, kc, vc, part, state, layer, NH, NKV, nsplit, scale);
    else if (HD == 128)
        hipLaunchKernelGGL(k_attn_part<128>, grid, block, 0, st, q, kc, vc, part, state, layer, NH, NKV, nsplit,
                           scale);
    else if (HD == 256)
        hipLaunchKernelGGL(k_attn_part<256>, grid, block, 0, st, q, kc, vc, part, state, layer, NH, NKV, nsplit,
                           scale);
    else
        return -1;
    return 0;
}

int dk_attn_o(const float* part, int NH, int NKV, int HD, int max_t, const DracoMat& wo, unsigned long long* acc,
              unsigned long long* zacc, int zn, hipStream_t st) {
    const int nsplit = attn_nsplit(max_t, NH, NKV, HD);
    if (wo.L.code == DRACO_Q8_0) {
        // chunks = kv groups of REP q heads, 2 REP blocks of every o row
        const int REP = NKV > 0 && NH % NKV == 0 ? NH / NKV : 0;
        if (HD != 64 || REP < 1 || REP > 4 || wo.L.n_in != NH * 64 || wo.L.nb != 2 * NH || nsplit > 64) return -1;
        const dim3 grid(NKV * ((wo.L.n_out + 31) / 32)), block(256);
        const uint8_t* qs = wo.dev + wo.L.off[0];
        const uint8_t* ds = wo.dev + wo.L.off[1];
#define AO8_CASE(S_, R_)                                                                                        \
    hipLaunchKernelGGL((k_attn_o8<S_, R_>), grid, block, 0, st, part, nsplit, qs, ds, wo.L.nb, wo.L.n_out, NKV, acc, \
                       zacc, zn)
#define AO8_REP(S_)            \
    if (REP == 1) AO8_CASE(S_, 1); \
    else if (REP == 2) AO8_CASE(S_, 2); \
    else if (REP == 3) AO8_CASE(S_, 3); \
    else AO8_CASE(S_, 4);
        if (nsplit <= 16) {
            AO8_REP(16)
        } else if (nsplit <= 32) {
            AO8_REP(32)
        } else {
            AO8_REP(64)
        }
#undef AO8_REP
#undef AO8_CASE
        return 0;
    }
    // K-quants: one chunk per o input super-block (256 attention outputs)
    if (HD != 64 && HD != 128 && HD != 256) return -1;
    const int NC = NH * HD / 256;
    if ((NH * HD) % 256 || wo.L.n_in != NH * HD || wo.L.nb != NC || nsplit > 64 ||
        (wo.L.code != DRACO_Q4_K && wo.L.code != DRACO_Q6_K))
        return -1;
    const int ntiles = (wo.L.n_out + 15) / 16;
    const dim3 grid(NC * ((ntiles + 3) / 4)), block(256);
    const bool q4 = wo.L.code == DRACO_Q4_K;
#define AO_CASE(S_, H_)                                                                                          \
    if (q4) hipLaunchKernelGGL((k_attn_o<1, S_, H_>), grid, block, 0, st, part, nsplit, wo.dev, wo.L.nb, wo.L.n_out, \
                               NC, acc, zacc, zn);                                                               \
    else hipLaunchKernelGGL((k_attn_o<2, S_, H_>), grid, block, 0, st, part, nsplit, wo.dev, wo.L.nb, wo.L.n_out, \
                            NC, acc, zacc, zn);
#define AO_HD(S_)                \
    if (HD == 64) {              \
        AO_CASE(S_, 64)          \
    } else if (HD == 128) {      \
        AO_CASE(S_, 128)         \
    } else {                     \
        AO_CASE(S_, 256)         \
    }
    if (nsplit <= 16) {
        AO_HD(16)
    } else if (nsplit <= 32) {
        AO_HD(32)
    } else {
        AO_HD(64)
    }
#undef AO_HD
#undef AO_CASE
    return 0;
}

int dk_attn_o8_short(const float* q, const float* kc, const float* vc, const int* state, int layer, int NH, int NKV,
                     int HD, float scale, int tcap, const DracoMat& wo, unsigned long long* acc,
                     unsigned long long* zacc, int zn, hipStream_t st) {
    const int REP = NKV > 0 && NH % NKV == 0 ? NH / NKV : 0;
    if (HD != 64 || REP < 1 || REP > 4 || tcap < 1 || tcap > ATT_SHORT_T || wo.L.code != DRACO_Q8_0 ||
        wo.L.n_in != NH * 64 || wo.L.nb != 2 * NH || NKV > 255 || wo.L.n_out >= (1 << 23))
        return -1;
    const dim3 grid(NKV * ((wo.L.n_out + 31) / 32)), block(256);
    const uint8_t* qs = wo.dev + wo.L.off[0];
    const uint8_t* ds = wo.dev + wo.L.off[1];
#define AOS_CASE(R_)                                                                                            \
    hipLaunchKernelGGL((k_attn_o8s<R_>), grid, block, 0, st, qs, ds, NKV | (wo.L.n_out << 8), q, kc, vc, tcap, \
                       state + 1 + layer, scale, acc, zacc, zn)
    if (REP == 1) AOS_CASE(1);
    else if (REP == 2) AOS_CASE(2);
    else if (REP == 3) AOS_CASE(3);
    else AOS_CASE(4);
#undef AOS_CASE
    return 0;
}

void dk_fa_prep(const float* QG, float* Qr, const float* kin, float* kout, const float* qn, const float* kn,
                const float* cs, int NH, hipStream_t st) {
    hipLaunchKernelGGL(k_fa_prep, dim3(NH + 2), dim3(256), 0, st, QG, Qr, kin, kout, qn, kn, cs, NH);
}

void dk_fa_prep_rows(const float* QG, int qg_stride, float* Qr, const float* kin, const float* vin, float* kc,
                     float* vc, const float* qn, const float* kn, const float* cs_tab, const int* state, int pos0,
                     int row0, int NH, int T, hipStream_t st) {
    hipLaunchKernelGGL(k_fa_prep_rows, dim3(NH + 2, T), dim3(256), 0, st, QG, kin, vin, qn, kn, state, qg_stride, NH,
                       cs_tab, Qr, kc, vc, pos0, row0);
}

void dk_swiglu(float* g, const float* u, int n, hipStream_t st) {
    const int blocks = (n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024;
    hipLaunchKernelGGL(k_swiglu, dim3(blocks), dim3(256), 0, st, g, u, n);
}

void dk_sigmoid_scale(const float* y, const float* g, float* out, int n, hipStream_t st) {
    const int blocks = (n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024;
    hipLaunchKernelGGL(k_sigmoid_scale, dim3(blocks), dim3(256), 0, st, y, g, out, n);
}

int dk_gate_scale(const float* x, const DracoMat& g, const float* y, float* out, float* gdot, int n, hipStream_t st) {
    if ((g.L.code != DRACO_F32 && g.L.code != DRACO_F16) || g.L.n_out != 1 || g.L.n_in != n || n % 4) return -1;
    const int blocks = (n + 255) / 256 < 64 ? (n + 255) / 256 : 64;
    hipLaunchKernelGGL(k_gate_scale, dim3(blocks), dim3(256), 0, st, x, (const void*)g.dev, g.L.code == DRACO_F16 ? 1 : 0,
                       y, out, gdot, n);
    return 0;
}

void dk_embed(const DracoMat& m, const int* ids, const int* cursor, float* out, hipStream_t st) {
    const int blocks = (m.L.n_in + 255) / 256;
    hipLaunchKernelGGL(k_embed, dim3(blocks), dim3(256), 0, st, m.dev, m.L, ids, cursor, out);
}

void dk_argmax(const float* x, int n, float* pv, int* pi, int* out, const int* slotp, int slot, hipStream_t st) {
    hipLaunchKernelGGL(k_argmax_part, dim3(ARGMAX_BLOCKS), dim3(256), 0, st, x, n, pv, pi);
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(64), 0, st, pv, pi, ARGMAX_BLOCKS, out, slotp, slot);
}

void dk_advance(int* state, int n_layer, int* tok_cursor, hipStream_t st) {
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(64), 0, st, state, n_layer, tok_cursor);
}

void dk_pick_token(const int* ids, const int* cursor, int* cur, hipStream_t st) {
    hipLaunchKernelGGL(k_pick_token, dim3(1), dim3(64), 0, st, ids, cursor, cur);
}
