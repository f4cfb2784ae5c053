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
// Mapping: one block of 8 waves per V head for the whole scan; the state
// lives in registers.  Wave w owns columns v = 16w .. 16w+15; lane
// (v_lo = lane>>2, kq = lane&3) holds S[32kq .. 32kq+31][16w + v_lo].  Each
// lane applies the reference's per-element operations in k order within its
// chunk (decay, multiply, add, unfused); the four chunks of a column combine
// with DPP moves, so the delta rule needs no LDS and no barrier.  The conv
// runs on threads 0..383 (one channel each: q, k of head j and v of head h,
// tail in registers); only the block that owns a channel writes its tail back
// (q/k channels: the block with h < NHQ).  l2 norms and the gated rms reduce
// across waves through LDS.  Results agree with the reference to fp32
// rounding: the per-column sums are split in four chunks and the l2 / rms sums
// use a tree.
#include <hip/hip_runtime.h>

#include "dev_common.h"
#include "gdn.h"

namespace {

constexpr int SV = 128;
constexpr float EPS = 1e-6f;

__device__ __forceinline__ float silu(float a) { return a / (1.f + expf(-a)); }

// Decode-step gates of V head h (src/m6_layer.c:237-256): every thread
// returns beta and the decay exp(alpha).  xn = h1 * rms^-1 * attn_norm is
// recomputed by each block (H floats, L2-resident after the first block);
// the beta / alpha rows are contiguous [n_vh][H], read once per block.
__device__ __forceinline__ void gdn_gates(const GdnArgs& a, int h, int tid, float* beta, float* gdec) {
    __shared__ float pre[3][8];
    const int lane = tid & 63, w = tid >> 6;
    float4 hv[2], nv[2], bv[2], av[2];
#pragma unroll
    for (int k = 0; k < 2; k++) {  // clamped, unconditional loads; masked below
        const int i = 4 * tid + 2048 * k;
        const int ic = i < a.H ? i : 0;
        hv[k] = ld4(a.h1 + ic);
        nv[k] = ld4(a.attn_norm + ic);
        bv[k] = ld4(a.bw + (size_t)h * a.H + ic);
        av[k] = ld4(a.aw + (size_t)h * a.H + ic);
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 2; k++)
        if (4 * tid + 2048 * k < a.H) ss += hv[k].x * hv[k].x + hv[k].y * hv[k].y + hv[k].z * hv[k].z + hv[k].w * hv[k].w;
    ss = wave_sum(ss);
    if (lane == 0) pre[0][w] = ss;
    lds_barrier();
    float tot = 0.f;
#pragma unroll
    for (int q = 0; q < 8; q++) tot += pre[0][q];
    const float inv = 1.f / sqrtf(tot / (float)a.H + EPS);
    float pb = 0.f, pa = 0.f;
#pragma unroll
    for (int k = 0; k < 2; k++) {
        if (4 * tid + 2048 * k < a.H) {
            const float x0 = hv[k].x * inv * nv[k].x, x1 = hv[k].y * inv * nv[k].y;
            const float x2 = hv[k].z * inv * nv[k].z, x3 = hv[k].w * inv * nv[k].w;
            pb += bv[k].x * x0 + bv[k].y * x1 + bv[k].z * x2 + bv[k].w * x3;
            pa += av[k].x * x0 + av[k].y * x1 + av[k].z * x2 + av[k].w * x3;
        }
    }
    pb = wave_sum(pb);
    pa = wave_sum(pa);
    if (lane == 0) {
        pre[1][w] = pb;
        pre[2][w] = pa;
    }
    lds_barrier();
    float bacc = 0.f, aacc = 0.f;
#pragma unroll
    for (int q = 0; q < 8; q++) {
        bacc += pre[1][q];
        aacc += pre[2][q];
    }
    *beta = 1.f / (1.f + expf(-bacc));
    const float avv = aacc + a.ssm_dt[h];
    const float sp = avv > 0.f ? avv + log1pf(expf(-avv)) : log1pf(expf(avv));
    *gdec = expf(sp * a.ssm_a[h]);
}

template <bool DEC>
__global__ __launch_bounds__(512) void k_gdn_scan(const GdnArgs a) {
    __shared__ float cq[SV], ck[SV], cv[SV];   // conv outputs of this token (q, k normalised in place)
    __shared__ float red[2][8];
    __shared__ float ored[8];
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int NHQ = a.nhq, n_qkv = a.n_qkv, n_vh = a.n_vh, T = a.T;
    const int j = h % NHQ;
    // conv channel of this thread: 0..127 q_j, 128..255 k_j, 256..383 v_h
    int ch = -1;
    if (tid < SV) ch = j * SV + tid;
    else if (tid < 2 * SV) ch = NHQ * SV + j * SV + (tid - SV);
    else if (tid < 3 * SV) ch = 2 * NHQ * SV + h * SV + (tid - 2 * SV);
    const bool owner = tid >= 2 * SV ? true : (h < NHQ);
    float w0 = 0.f, w1 = 0.f, w2 = 0.f, w3 = 0.f, t0 = 0.f, t1 = 0.f, t2 = 0.f;
    if (ch >= 0) {
        const float4 cw = ld4(a.conv + (size_t)ch * 4);
        w0 = cw.x; w1 = cw.y; w2 = cw.z; w3 = cw.w;
        t0 = a.tail[(size_t)ch * 3];
        t1 = a.tail[(size_t)ch * 3 + 1];
        t2 = a.tail[(size_t)ch * 3 + 2];
    }
    // state slice
    const int vl = lane >> 2, kq = lane & 3, v = 16 * w + vl;
    float* Sh = a.S + (size_t)h * SV * SV;
    float s[32];
#pragma unroll
    for (int i = 0; i < 32; i++) s[i] = Sh[(size_t)(32 * kq + i) * SV + v];
    const float nw = a.ssm_norm[v];
    const float scale = 1.f / sqrtf((float)SV);

    // per-token inputs, prefetched one token ahead
    float xin = ch >= 0 && T > 0 ? a.QKV[ch] : 0.f;
    float zin = T > 0 ? a.Z[(size_t)h * SV + v] : 0.f;
    float gin = 0.f, bin = 0.f;
    if constexpr (DEC) {
        gdn_gates(a, h, tid, &bin, &gin);
    } else {
        gin = T > 0 ? a.G[h] : 0.f;
        bin = T > 0 ? a.B[h] : 0.f;
    }
    for (int t = 0; t < T; t++) {
        const float x = xin, z = zin, g = gin, b = bin;
        if (!DEC && t + 1 < T) {
            xin = ch >= 0 ? a.QKV[(size_t)(t + 1) * n_qkv + ch] : 0.f;
            zin = a.Z[(size_t)(t + 1) * n_vh * SV + (size_t)h * SV + v];
            gin = a.G[(size_t)(t + 1) * n_vh + h];
            bin = a.B[(size_t)(t + 1) * n_vh + h];
        }
        // (1) conv + silu (src/m6_gdn_scan.c:30-38)
        float c = 0.f;
        if (ch >= 0) {
            const float acc = w0 * t0 + w1 * t1 + w2 * t2 + w3 * x;
            c = silu(acc);
            t0 = t1;
            t1 = t2;
            t2 = x;
        }
        // (2) l2 norms of q (waves 0,1) and k (waves 2,3)
        float sq = tid < 2 * SV ? c * c : 0.f;
        sq = wave_sum(sq);
        if (lane == 0 && w < 4) red[w >> 1][w & 1] = sq;
        lds_barrier();
        if (tid < 2 * SV) {
            const float n2 = red[w >> 1][0] + red[w >> 1][1];
            const float nr = sqrtf(n2);
            const float inv = 1.f / (nr > EPS ? nr : EPS);
            if (tid < SV) cq[tid] = c * inv;
            else ck[tid - SV] = c * inv;
        } else if (tid < 3 * SV) {
            cv[tid - 2 * SV] = c;
        }
        lds_barrier();
        // (3) delta rule on this lane's 32 rows of column v
        float sk = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            s[i] = s[i] * g;
            sk = sk + s[i] * ck[32 * kq + i];
        }
        sk = group_sum<4>(sk);
        const float d = (cv[v] - sk) * b;
        float o = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            s[i] = s[i] + ck[32 * kq + i] * d;
            o = o + s[i] * cq[32 * kq + i];
        }
        o = group_sum<4>(o);
        // (4) gated rms over the 128 columns
        o = o * scale;
        float o2 = kq == 0 ? o * o : 0.f;
        o2 = wave_sum(o2);
        if (lane == 0) ored[w] = o2;
        lds_barrier();
        float ms2 = 0.f;
#pragma unroll
        for (int q = 0; q < 8; q++) ms2 += ored[q];
        const float inv2 = 1.f / sqrtf(ms2 / SV + EPS);
        if (kq == 0) a.ON[(size_t)t * n_vh * SV + (size_t)h * SV + v] = o * inv2 * nw * silu(z);
        lds_barrier();  // cq/ck/cv/red/ored are rewritten by the next token
    }
#pragma unroll
    for (int i = 0; i < 32; i++) Sh[(size_t)(32 * kq + i) * SV + v] = s[i];
    if (ch >= 0 && owner) {
        a.tail[(size_t)ch * 3] = t0;
        a.tail[(size_t)ch * 3 + 1] = t1;
        a.tail[(size_t)ch * 3 + 2] = t2;
    }
}

}  // namespace

int draco_gdn_scan_launch(const GdnArgs& a, hipStream_t st) {
    if (a.n_vh < 1 || a.nhq < 1 || a.n_qkv != a.n_vh * SV + 2 * a.nhq * SV || a.T < 0) return -1;
    if (a.T == 0) return 0;
    hipLaunchKernelGGL(k_gdn_scan<false>, dim3(a.n_vh), dim3(512), 0, st, a);
    return 0;
}

int draco_gdn_step_launch(const GdnArgs& a, hipStream_t st) {
    if (a.n_vh < 1 || a.nhq < 1 || a.n_qkv != a.n_vh * SV + 2 * a.nhq * SV || a.T != 1) return -1;
    if (a.H < 4 || a.H > 4096 || a.H % 4 || !a.h1 || !a.attn_norm || !a.bw || !a.aw || !a.ssm_a || !a.ssm_dt)
        return -1;
    hipLaunchKernelGGL(k_gdn_scan<true>, dim3(a.n_vh), dim3(512), 0, st, a);
    return 0;
}
