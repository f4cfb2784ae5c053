// prefill.hip -- chunked prefill of the llama family (gfx950): the T tokens
// of a chunk go through each layer together, with the weight products on the
// f16-MFMA GEMM (gemmh.hip) and these row-parallel kernels around them:
//
//   k_pf_embed          X[t] = embedding row ids[t]
//   k_pf_rms            Xn[t] = RMSNorm(X[t]) * w            (src/m6_engine.c:31-37)
//   k_pf_add_rms        X[t] += Y[t], then the RMSNorm of the sum
//   k_pf_rope_append    rope on Q[t] and K[t] at position pos0 + t, K/V rows
//                       appended at cache row row0 + t       (src/m6_engine.c:456-481)
//   k_pf_attn, k_pf_merge
//                       causal attention: token t attends cache rows
//                       [0, row0 + t]                        (src/m6_engine.c:482-505)
//   k_pf_add            X += Y (residual)
//
// The result equals running the tokens one by one through m6_forward_token
// up to fp32 rounding (summation orders differ; the softmax is the split
// online form, exact in exact arithmetic).
#include <hip/hip_runtime.h>

#include "dev_common.h"
#include "embed_dev.h"
#include "formats.h"
#include "prefill.h"

namespace {

__global__ __launch_bounds__(256) void k_pf_embed(const uint8_t* __restrict__ base, DracoLayout L,
                                                  const int* __restrict__ ids, float* __restrict__ X) {
    const int t = blockIdx.y, p = blockIdx.x * 256 + threadIdx.x;
    if (p < L.n_in) X[(size_t)t * L.n_in + p] = embed_value(base, L, ids[t], p);
}

// one block of 256 threads per token row; x held in registers (h <= 256 * PF_RMS_PT)
constexpr int PF_RMS_PT = 16;
__global__ __launch_bounds__(256) void k_pf_rms(const float* __restrict__ X, const float* __restrict__ w,
                                                float* __restrict__ Xn, int h, float eps) {
    __shared__ float red[4];
    const float* x = X + (size_t)blockIdx.x * h;
    float* o = Xn + (size_t)blockIdx.x * h;
    // every load (the row and its norm weights, clamped index) before the
    // first wait; a null weight re-reads the row
    const float* wp = w ? w : x;
    float v[PF_RMS_PT], wv[PF_RMS_PT];
#pragma unroll
    for (int k = 0; k < PF_RMS_PT; k++) {
        const int i = threadIdx.x + 256 * k, ic = i < h ? i : h - 1;
        v[k] = x[ic];
        wv[k] = wp[ic];
    }
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < PF_RMS_PT; k++) {
        if (threadIdx.x + 256 * k >= h) v[k] = 0.f;
        s = fmaf(v[k], v[k], s);
    }
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    lds_barrier();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.f / sqrtf(tot / (float)h + eps);
#pragma unroll
    for (int k = 0; k < PF_RMS_PT; k++) {
        const int i = threadIdx.x + 256 * k;
        if (i < h) o[i] = w ? v[k] * inv * wv[k] : v[k] * inv;
    }
}

// X[t] += Y[t] (the residual), then Xn[t] = (X[t] * inv_rms) * w: one block
// per token row, the sum held in registers between the two steps
__global__ __launch_bounds__(256) void k_pf_add_rms(float* __restrict__ X, const float* __restrict__ Y,
                                                    const float* __restrict__ w, float* __restrict__ Xn, int h,
                                                    float eps) {
    __shared__ float red[4];
    float* x = X + (size_t)blockIdx.x * h;
    const float* y = Y + (size_t)blockIdx.x * h;
    float* o = Xn + (size_t)blockIdx.x * h;
    // every load (row, residual, norm weights; clamped index) before the
    // first wait and the first store; a null weight re-reads the row
    const float* wp = w ? w : x;
    float v[PF_RMS_PT], yv[PF_RMS_PT], wv[PF_RMS_PT];
#pragma unroll
    for (int k = 0; k < PF_RMS_PT; k++) {
        const int i = threadIdx.x + 256 * k, ic = i < h ? i : h - 1;
        v[k] = x[ic];
        yv[k] = y[ic];
        wv[k] = wp[ic];
    }
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < PF_RMS_PT; k++) {
        const int i = threadIdx.x + 256 * k;
        v[k] = i < h ? v[k] + yv[k] : 0.f;
        if (i < h) x[i] = v[k];
        s = fmaf(v[k], v[k], s);
    }
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    lds_barrier();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.f / sqrtf(tot / (float)h + eps);
#pragma unroll
    for (int k = 0; k < PF_RMS_PT; k++) {
        const int i = threadIdx.x + 256 * k;
        if (i < h) o[i] = w ? v[k] * inv * wv[k] : v[k] * inv;
    }
}

// Q [T][NH*HD] rotated in place; K [T][KD] rotated into kc row row0 + t; V
// [T][KD] copied into vc row row0 + t.  One thread per even index of a pair
// (pairs (2i, 2i+1) of a head, the GGML "normal" rope, src/m6_engine.c:134-143).
__global__ __launch_bounds__(256) void k_pf_rope_append(float* __restrict__ Q, const float* __restrict__ K,
                                                        const float* __restrict__ V, float* __restrict__ kc,
                                                        float* __restrict__ vc, const float* __restrict__ tab,
                                                        int pos0, int row0, int NH, int NKV, int HD, int rot) {
    const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    const int QD = NH * HD, KD = NKV * HD, half = rot / 2;
    const float* ang = tab + (size_t)(pos0 + t) * half * 2;
    if (i < QD) {
        const int d = i % HD;
        float* q = Q + (size_t)t * QD;
        if (d < rot && (d & 1) == 0) {
            const float c = ang[d], s = ang[d + 1];
            const float a = q[i], b = q[i + 1];
            q[i] = a * c - b * s;
            q[i + 1] = a * s + b * c;
        }
    } else if (i < QD + KD) {
        const int j = i - QD, d = j % HD;
        const float* k = K + (size_t)t * KD;
        float* dst = kc + (size_t)(row0 + t) * KD;
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
    } else if (i < QD + 2 * KD) {
        const int j = i - QD - KD;
        vc[(size_t)(row0 + t) * KD + j] = V[(size_t)t * KD + j];
    }
}

// Causal attention of a chunk, split over the key rows.  Block (g, qt, s):
// kv head g, queries qt*64 .. qt*64+63 of the chunk (lane = query), key split
// s of rows [0, row0 + last query of the tile].  Wave j is q head g*rep + j;
// the rep waves share the K / V rows, staged in LDS 64 rows at a time and
// read by every lane at the same address (broadcast).  Keys go in groups of
// 16: scores, one online-softmax rescale, then P.V.  Writes the unnormalised
// (o[HD], m, l) of (head, query, split) for k_pf_merge.
constexpr int PF_QT = 64, PF_KT = 64, PF_KG = 16;

// K and V rows [kb, kb + nr) of kv head g into LDS (row-major, HD wide):
// each thread requests up to 4 float4s of each array together (clamped
// index; the stores skip the clamped ones), so a tile costs one memory round
// trip per 4 float4s per thread instead of one per float4.
template <int HD>
__device__ __forceinline__ void stage_kv(float* Ks, float* Vs, const float* __restrict__ kc,
                                         const float* __restrict__ vc, int kb, int nr, int KD, int g) {
    constexpr int SB = 4;
    const int n = nr * (HD / 4), nt = blockDim.x, tid = threadIdx.x;
    for (int b0 = 0; b0 < n; b0 += SB * nt) {
        float4 kv[SB], vv[SB];
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const int i = b0 + tid + u * nt, ic = i < n ? i : n - 1;
            const int r = ic / (HD / 4), c = 4 * (ic % (HD / 4));
            kv[u] = ld4(kc + (size_t)(kb + r) * KD + g * HD + c);
            vv[u] = ld4(vc + (size_t)(kb + r) * KD + g * HD + c);
        }
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const int i = b0 + tid + u * nt;
            if (i < n) {
                const int r = i / (HD / 4), c = 4 * (i % (HD / 4));
                *reinterpret_cast<float4*>(Ks + r * HD + c) = kv[u];
                *reinterpret_cast<float4*>(Vs + r * HD + c) = vv[u];
            }
        }
    }
}

template <int HD>
__global__ __launch_bounds__(512) void k_pf_attn(const float* __restrict__ Q, const float* __restrict__ kc,
                                                 const float* __restrict__ vc, float* __restrict__ part, int row0,
                                                 int T, int NH, int NKV, int nspl, float scale) {
    extern __shared__ __align__(16) float sm[];
    float* Ks = sm;
    float* Vs = sm + PF_KT * HD;
    const int g = blockIdx.x, qt = blockIdx.y, s = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, j = tid >> 6;
    const int rep = NH / NKV, h = g * rep + j, KD = NKV * HD, QD = NH * HD;
    const int t = qt * PF_QT + lane, qrow = row0 + t;
    const bool live = t < T;
    const int kend = row0 + min(T, (qt + 1) * PF_QT);
    const int chunk = (kend + nspl - 1) / nspl;
    const int k0 = min(kend, s * chunk), k1 = min(kend, k0 + chunk);
    float q[HD], o[HD];
    const int tq = live ? t : 0;  // a query past the chunk reads row 0 and discards it
#pragma unroll
    for (int d = 0; d < HD; d += 4) {
        const float4 v = ld4(Q + (size_t)tq * QD + h * HD + d);
        q[d] = live ? v.x : 0.f; q[d + 1] = live ? v.y : 0.f; q[d + 2] = live ? v.z : 0.f; q[d + 3] = live ? v.w : 0.f;
        o[d] = o[d + 1] = o[d + 2] = o[d + 3] = 0.f;
    }
    float m = -INFINITY, l = 0.f;
    for (int kb = k0; kb < k1; kb += PF_KT) {
        const int nr = min(PF_KT, k1 - kb);
        stage_kv<HD>(Ks, Vs, kc, vc, kb, nr, KD, g);
        __syncthreads();
        for (int c0 = 0; c0 < nr; c0 += PF_KG) {
            const int ng = min(PF_KG, nr - c0);
            float sc[PF_KG];
            float cm = -INFINITY;
#pragma unroll
            for (int jj = 0; jj < PF_KG; jj++) {
                sc[jj] = -INFINITY;
                if (jj < ng) {
                    const float* kr = Ks + (c0 + jj) * HD;
                    float acc = 0.f;
#pragma unroll
                    for (int d = 0; d < HD; d += 4) {
                        const float4 kv = *reinterpret_cast<const float4*>(kr + d);
                        acc = fmaf(q[d], kv.x, acc);
                        acc = fmaf(q[d + 1], kv.y, acc);
                        acc = fmaf(q[d + 2], kv.z, acc);
                        acc = fmaf(q[d + 3], kv.w, acc);
                    }
                    if (live && kb + c0 + jj <= qrow) sc[jj] = acc * scale;
                    cm = fmaxf(cm, sc[jj]);
                }
            }
            const float mn = fmaxf(m, cm);
            if (mn > -INFINITY) {
                const float corr = m > -INFINITY ? expf(m - mn) : 0.f;
                l *= corr;
#pragma unroll
                for (int d = 0; d < HD; d++) o[d] *= corr;
#pragma unroll
                for (int jj = 0; jj < PF_KG; jj++) {
                    if (jj < ng) {
                        const float p = sc[jj] > -INFINITY ? expf(sc[jj] - mn) : 0.f;
                        l += p;
                        const float* vr = Vs + (c0 + jj) * HD;
#pragma unroll
                        for (int d = 0; d < HD; d += 4) {
                            const float4 vv = *reinterpret_cast<const float4*>(vr + d);
                            o[d] = fmaf(p, vv.x, o[d]);
                            o[d + 1] = fmaf(p, vv.y, o[d + 1]);
                            o[d + 2] = fmaf(p, vv.z, o[d + 2]);
                            o[d + 3] = fmaf(p, vv.w, o[d + 3]);
                        }
                    }
                }
                m = mn;
            }
        }
        __syncthreads();
    }
    if (!live) return;
    float* pp = part + (((size_t)h * T + t) * nspl + s) * (HD + 2);
#pragma unroll
    for (int d = 0; d < HD; d++) pp[d] = o[d];
    pp[HD] = m;
    pp[HD + 1] = l;
}

// The split merge of one (query, head, dim): M = max_s m_s, then num / den
// with den = sum_s l_s e^(m_s - M), num = sum_s o_s[d] e^(m_s - M) in split
// order.  Loads go in batches of 16 splits, all of a batch requested together
// (clamped split index; the merge skips the clamped ones), instead of one
// dependent round trip per split.
__device__ __forceinline__ float pf_merge_one(const float* __restrict__ pp, int HD, int nspl, int d) {
    constexpr int MB = 16;
    float M = -INFINITY;
    for (int s0 = 0; s0 < nspl; s0 += MB) {
        float mv[MB];
#pragma unroll
        for (int k = 0; k < MB; k++) mv[k] = pp[(size_t)min(s0 + k, nspl - 1) * (HD + 2) + HD];
#pragma unroll
        for (int k = 0; k < MB; k++)
            if (s0 + k < nspl) M = fmaxf(M, mv[k]);
    }
    float num = 0.f, den = 0.f;
    for (int s0 = 0; s0 < nspl; s0 += MB) {
        float mv[MB], lv[MB], ov[MB];
#pragma unroll
        for (int k = 0; k < MB; k++) {
            const float* q = pp + (size_t)min(s0 + k, nspl - 1) * (HD + 2);
            mv[k] = q[HD];
            lv[k] = q[HD + 1];
            ov[k] = q[d];
        }
#pragma unroll
        for (int k = 0; k < MB; k++) {
            if (s0 + k >= nspl || mv[k] == -INFINITY) continue;
            const float e = expf(mv[k] - M);
            den = fmaf(lv[k], e, den);
            num = fmaf(ov[k], e, num);
        }
    }
    return num / den;
}

// out[t][h*HD + d] = sum_s o_s[d] e^(m_s - M) / sum_s l_s e^(m_s - M)
__global__ __launch_bounds__(256) void k_pf_merge(const float* __restrict__ part, float* __restrict__ O, int T,
                                                  int NH, int HD, int nspl) {
    const int t = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
    if (d >= HD) return;
    const float* pp = part + ((size_t)h * T + t) * nspl * (HD + 2);
    O[(size_t)t * NH * HD + h * HD + d] = pf_merge_one(pp, HD, nspl, d);
}

// Causal chunk attention at head dim 256 (qwen35 full attention, the chunked
// form of src/m6_layer.c:455-500 that src/qwen35_prefill.py:137-168 runs).
// Block (g, qt, s): kv head g, queries qt*8 .. qt*8+7 of the chunk, key split
// s; wave j = q head g*rep + j.  Eight lanes share a query: lane = 8*query +
// k holds the dims 4*(k + 8*i) .. +3 (i < 8) of q and of the output, so the
// eight lanes of a query read one 128-byte run of a staged K / V row
// (conflict-free) and a score is the sum over those eight lanes.  K / V rows
// are staged in LDS 32 at a time; keys go in groups of 16 (scores, one
// online-softmax rescale, P.V).  Writes (o[256], m, l) per (head, query,
// split) for k_pf_merge256.
constexpr int PF256_QT = 8, PF256_KT = 32;

__global__ __launch_bounds__(1024) void k_pf_attn256(const float* __restrict__ Q, const float* __restrict__ kc,
                                                     const float* __restrict__ vc, float* __restrict__ part,
                                                     int row0, int T, int NH, int NKV, int nspl, float scale) {
    constexpr int HD = 256;
    __shared__ __align__(16) float Ks[PF256_KT * HD];
    __shared__ __align__(16) float Vs[PF256_KT * HD];
    const int g = blockIdx.x, qt = blockIdx.y, s = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, j = tid >> 6, k = lane & 7;
    const int rep = NH / NKV, h = g * rep + j, KD = NKV * HD, QD = NH * HD;
    const int t = qt * PF256_QT + (lane >> 3), qrow = row0 + t;
    const bool live = t < T;
    const int kend = row0 + min(T, (qt + 1) * PF256_QT);
    const int chunk = (kend + nspl - 1) / nspl;
    const int k0 = min(kend, s * chunk), k1 = min(kend, k0 + chunk);
    float q[32], o[32];
    const int tq = live ? t : 0;  // a query past the chunk reads row 0 and discards it
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 v = ld4(Q + (size_t)tq * QD + h * HD + 4 * (k + 8 * i));
        q[4 * i] = live ? v.x : 0.f; q[4 * i + 1] = live ? v.y : 0.f;
        q[4 * i + 2] = live ? v.z : 0.f; q[4 * i + 3] = live ? v.w : 0.f;
        o[4 * i] = o[4 * i + 1] = o[4 * i + 2] = o[4 * i + 3] = 0.f;
    }
    float m = -INFINITY, l = 0.f;
    for (int kb = k0; kb < k1; kb += PF256_KT) {
        const int nr = min(PF256_KT, k1 - kb);
        stage_kv<HD>(Ks, Vs, kc, vc, kb, nr, KD, g);
        __syncthreads();
        for (int c0 = 0; c0 < nr; c0 += 16) {
            const int ng = min(16, nr - c0);
            float sc[16];
            float cm = -INFINITY;
#pragma unroll
            for (int jj = 0; jj < 16; jj++) {
                float acc = 0.f;
                if (jj < ng) {
                    const float* kr = Ks + (c0 + jj) * HD;
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        const float4 kv = *reinterpret_cast<const float4*>(kr + 4 * (k + 8 * i));
                        acc = fmaf(q[4 * i], kv.x, acc);
                        acc = fmaf(q[4 * i + 1], kv.y, acc);
                        acc = fmaf(q[4 * i + 2], kv.z, acc);
                        acc = fmaf(q[4 * i + 3], kv.w, acc);
                    }
                }
                acc = group_sum<8>(acc);
                sc[jj] = (jj < ng && live && kb + c0 + jj <= qrow) ? acc * scale : -INFINITY;
                cm = fmaxf(cm, sc[jj]);
            }
            const float mn = fmaxf(m, cm);
            if (mn > -INFINITY) {
                const float corr = m > -INFINITY ? expf(m - mn) : 0.f;
                l *= corr;
#pragma unroll
                for (int d = 0; d < 32; d++) o[d] *= corr;
#pragma unroll
                for (int jj = 0; jj < 16; jj++) {
                    if (jj < ng) {
                        const float p = sc[jj] > -INFINITY ? expf(sc[jj] - mn) : 0.f;
                        l += p;
                        const float* vr = Vs + (c0 + jj) * HD;
#pragma unroll
                        for (int i = 0; i < 8; i++) {
                            const float4 vv = *reinterpret_cast<const float4*>(vr + 4 * (k + 8 * i));
                            o[4 * i] = fmaf(p, vv.x, o[4 * i]);
                            o[4 * i + 1] = fmaf(p, vv.y, o[4 * i + 1]);
                            o[4 * i + 2] = fmaf(p, vv.z, o[4 * i + 2]);
                            o[4 * i + 3] = fmaf(p, vv.w, o[4 * i + 3]);
                        }
                    }
                }
                m = mn;
            }
        }
        __syncthreads();
    }
    if (!live) return;
    float* pp = part + (((size_t)h * T + t) * nspl + s) * (HD + 2);
#pragma unroll
    for (int i = 0; i < 8; i++)
        *reinterpret_cast<float4*>(pp + 4 * (k + 8 * i)) = make_float4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
    if (k == 0) {
        pp[HD] = m;
        pp[HD + 1] = l;
    }
}

// k_pf_merge with the qwen35 output gate: O[t][h*HD + d] *= sigmoid(gate
// row t, h*gstride_h + d) (the reference's attn * sigmoid(q gate half),
// src/qwen35_prefill.py:164-166 / src/m6_layer.c:497).
__global__ __launch_bounds__(256) void k_pf_merge_gate(const float* __restrict__ part, float* __restrict__ O, int T,
                                                       int NH, int HD, int nspl, const float* __restrict__ gate,
                                                       int g_row, int g_head) {
    const int t = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
    if (d >= HD) return;
    const float* pp = part + ((size_t)h * T + t) * nspl * (HD + 2);
    const float gv = gate[(size_t)t * g_row + (size_t)h * g_head + d];
    O[(size_t)t * NH * HD + h * HD + d] = pf_merge_one(pp, HD, nspl, d) * (1.f / (1.f + expf(-gv)));
}

// GDN gates of a chunk (src/qwen35_prefill.py:118-123): for token t and V
// head e, B = sigmoid(Xn[t] . bw[e]) and G = exp(softplus(Xn[t] . aw[e] +
// dt[e]) * a[e]); bw / aw stored [n_vh][H].  Block (t, e), 256 threads.
__global__ __launch_bounds__(256) void k_pf_gdn_gates(const float* __restrict__ Xn, int H,
                                                      const float* __restrict__ bw, const float* __restrict__ aw,
                                                      const float* __restrict__ dt, const float* __restrict__ sa,
                                                      float* __restrict__ B, float* __restrict__ G, int n_vh) {
    __shared__ float red[2][4];
    const int t = blockIdx.x, e = blockIdx.y, tid = threadIdx.x;
    const float* x = Xn + (size_t)t * H;
    float sb = 0.f, sa_ = 0.f;
    for (int i = tid * 4; i < H; i += 1024) {
        const float4 xv = ld4(x + i), bv = ld4(bw + (size_t)e * H + i), av = ld4(aw + (size_t)e * H + i);
        sb = fmaf(xv.x, bv.x, sb); sb = fmaf(xv.y, bv.y, sb); sb = fmaf(xv.z, bv.z, sb); sb = fmaf(xv.w, bv.w, sb);
        sa_ = fmaf(xv.x, av.x, sa_); sa_ = fmaf(xv.y, av.y, sa_); sa_ = fmaf(xv.z, av.z, sa_); sa_ = fmaf(xv.w, av.w, sa_);
    }
    sb = wave_sum(sb);
    sa_ = wave_sum(sa_);
    if ((tid & 63) == 0) {
        red[0][tid >> 6] = sb;
        red[1][tid >> 6] = sa_;
    }
    __syncthreads();
    if (tid == 0) {
        const float b = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
        const float a = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]) + dt[e];
        const float sp = a > 0.f ? a + log1pf(expf(-a)) : log1pf(expf(a));  // softplus, src/m6_layer.c:253
        B[(size_t)t * n_vh + e] = 1.f / (1.f + expf(-b));
        G[(size_t)t * n_vh + e] = expf(sp * sa[e]);
    }
}

__global__ __launch_bounds__(256) void k_pf_add(float* __restrict__ X, const float* __restrict__ Y, size_t n) {
    for (size_t i = blockIdx.x * (size_t)256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) X[i] += Y[i];
}

}  // namespace

int pf_attn_nsplit(int row0, int T) {
    // about 64 key rows per split at the tile holding the chunk's last query
    const int n = (row0 + T + 63) / 64;
    return n < 1 ? 1 : (n > 64 ? 64 : n);
}

size_t pf_part_floats(int NH, int T, int HD, int nspl) { return (size_t)NH * T * nspl * (HD + 2); }

int pf_embed(const uint8_t* base, const DracoLayout& L, const int* ids, int T, float* X, hipStream_t st) {
    if (T < 1) return -1;
    hipLaunchKernelGGL(k_pf_embed, dim3((L.n_in + 255) / 256, T), dim3(256), 0, st, base, L, ids, X);
    return 0;
}

int pf_rms(const float* X, const float* w, float* Xn, int T, int h, float eps, hipStream_t st) {
    if (T < 1 || h > 256 * PF_RMS_PT) return -1;
    hipLaunchKernelGGL(k_pf_rms, dim3(T), dim3(256), 0, st, X, w, Xn, h, eps);
    return 0;
}

int pf_add_rms(float* X, const float* Y, const float* w, float* Xn, int T, int h, float eps, hipStream_t st) {
    if (T < 1 || h > 256 * PF_RMS_PT) return -1;
    hipLaunchKernelGGL(k_pf_add_rms, dim3(T), dim3(256), 0, st, X, Y, w, Xn, h, eps);
    return 0;
}

int pf_rope_append(float* Q, const float* K, const float* V, float* kc, float* vc, const float* tab, int pos0,
                   int row0, int T, int NH, int NKV, int HD, int rot, hipStream_t st) {
    if (T < 1 || (rot & 1) || rot > HD) return -1;
    const int n = NH * HD + 2 * NKV * HD;
    hipLaunchKernelGGL(k_pf_rope_append, dim3((n + 255) / 256, T), dim3(256), 0, st, Q, K, V, kc, vc, tab, pos0,
                       row0, NH, NKV, HD, rot);
    return 0;
}

int pf_attention(const float* Q, const float* kc, const float* vc, float* part, float* O, int row0, int T, int NH,
                 int NKV, int HD, float scale, hipStream_t st) {
    if (T < 1 || !pf_attention_ok(NH, NKV, HD)) return -1;
    const int nspl = pf_attn_nsplit(row0, T);
    const dim3 grid(NKV, (T + PF_QT - 1) / PF_QT, nspl), block(64 * (NH / NKV));
    const size_t lds = sizeof(float) * 2 * PF_KT * HD;
    if (HD == 64) {
        hipLaunchKernelGGL(k_pf_attn<64>, grid, block, lds, st, Q, kc, vc, part, row0, T, NH, NKV, nspl, scale);
    } else {
        static bool attr = false;
        if (!attr) {
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_pf_attn<128>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024);
            attr = true;
        }
        hipLaunchKernelGGL(k_pf_attn<128>, grid, block, lds, st, Q, kc, vc, part, row0, T, NH, NKV, nspl, scale);
    }
    hipLaunchKernelGGL(k_pf_merge, dim3(T, NH), dim3(HD), 0, st, part, O, T, NH, HD, nspl);
    return 0;
}

int pf_attention256(const float* Q, const float* kc, const float* vc, float* part, float* O, int row0, int T, int NH,
                    int NKV, float scale, const float* gate, int g_row, int g_head, hipStream_t st) {
    if (T < 1 || NKV < 1 || NH % NKV || NH / NKV > 16 || !gate) return -1;
    const int nspl = pf_attn_nsplit(row0, T);
    const dim3 grid(NKV, (T + PF256_QT - 1) / PF256_QT, nspl), block(64 * (NH / NKV));
    hipLaunchKernelGGL(k_pf_attn256, grid, block, 0, st, Q, kc, vc, part, row0, T, NH, NKV, nspl, scale);
    hipLaunchKernelGGL(k_pf_merge_gate, dim3(T, NH), dim3(256), 0, st, part, O, T, NH, 256, nspl, gate, g_row, g_head);
    return 0;
}

int pf_gdn_gates(const float* Xn, int T, int H, const float* bw, const float* aw, const float* dt, const float* sa,
                 float* B, float* G, int n_vh, hipStream_t st) {
    if (T < 1 || H % 4 || n_vh < 1) return -1;
    hipLaunchKernelGGL(k_pf_gdn_gates, dim3(T, n_vh), dim3(256), 0, st, Xn, H, bw, aw, dt, sa, B, G, n_vh);
    return 0;
}

int pf_add(float* X, const float* Y, size_t n, hipStream_t st) {
    const size_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(k_pf_add, dim3(blocks < 2048 ? (unsigned)blocks : 2048u), dim3(256), 0, st, X, Y, n);
    return 0;
}
