// abi_qwen.cpp -- qwen35 hybrid-layer decode ops: m6_gdn_attn (Gated-DeltaNet
// layer) and m6_full_attn (gated full attention), src/m6_layer.c:189-518.
//
// Host pointers in and out, as in the reference: the recurrent state (ssm,
// tail) and the cached K / V rows are the caller's arrays.  Each call uploads
// them, runs the layer on the device and downloads every output the reference
// writes (the state in place, kr_new / v_new for the caller's cache append).
// Weights and fp32 parameter arrays are registered by host address and stay
// resident.  The reference's scratch arguments (buf, scores) are accepted and
// not used.
//
// Device work per GDN token (5 launches):
//   k_dq      qkv + gate projections, attention RMSNorm in the prologue
//   k_gdn     per V head: beta / decay from xn, conv + silu, l2 norms, delta
//             rule on the register-resident state, gated rms   -> on
//   k_dq      ssm_out projection + residual                     -> x2_out
//   k_rmsnorm post-attention norm                               -> x2n
// Device work per full-attention token (6 launches):
//   k_dq        q+gate, k, v projections (v straight into cache row Told)
//   k_fa_prep   q / k head RMSNorm + rope (k into cache row Told)
//   k_attn_part split-T attention over Told + 1 rows, then k_attn_combine
//               with the sigmoid gate
//   k_dq        o projection + residual; k_rmsnorm               -> x2n
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "decode.h"
#include "gdn.h"
#include "gemv.h"
#include "runtime.h"

using namespace draco;

// Field for field the reference's descriptors (src/m6_layer.c:189-202,
// :375-387; ctypes twins src/qwen35_engine.py:137-157).
typedef struct {
    const float* attn_norm;
    const uint8_t* qkv_buf;
    int qkv_code;
    const uint8_t* gate_buf;
    int gate_code;
    const float* beta_wt;
    const float* alpha_wt;
    const float* ssm_a;
    const float* ssm_dt;
    const float* conv;
    const float* ssm_norm;
    const uint8_t* ssm_out_buf;
    int ssm_out_code;
    const float* post_norm;
    int n_qkv;
    int n_vh;
    int d_in;
} GdnW;

typedef struct {
    const float* attn_norm;
    const uint8_t* q_buf;
    int q_code;
    const uint8_t* k_buf;
    int k_code;
    const uint8_t* v_buf;
    int v_code;
    const float* q_norm;
    const float* k_norm;
    const uint8_t* o_buf;
    int o_code;
    const float* post_norm;
    const float* rope_inv;
    int nh;
} FullW;

namespace {

constexpr int QH = 2048;      // hidden width fixed by the reference ops (src/m6_layer.c:11-13)
constexpr int QNKH = 16;      // GDN q/k heads
constexpr int QSV = 128;      // GDN head width
constexpr int FHD = 256;      // full-attention head dim
constexpr int FNKV = 2;       // full-attention KV heads
constexpr float QEPS = 1e-6f;

int report(int rc, const char* where) {
    fprintf(stderr, "[draco_hip] %s failed (rc=%d): %s\n", where, rc, last_error());
    return rc;
}

struct Proj {
    const DracoMat* m;
    float* y;
    const float* yadd;  // nullable: y = yadd + W.x
};

// Post-projection RMSNorm request: out = RMSNorm(y) * w (eps QEPS), one
// k_rmsnorm launch after the projection.  (A last-block-done finisher inside
// the GEMV was measured slower on MI355X: the agent-scope release each block
// needs before counting itself writes back its XCD's L2.)
struct PostNorm {
    const float* w;
    float* out;
};

// GEMVs of several matrices sharing the input x (n_in wide), with x
// RMS-normalised by norm_w in the kernels' prologue when norm_w is set.
// Q4_K / Q6_K matrices share one launch, Q8_0 matrices another; any other
// format runs through the plain GEMV on an explicitly normalised copy in xn.
// With `post` (one matrix only) the output's RMSNorm is produced too.
int enqueue_proj(const Proj* p, int n, const float* x, int n_in, const float* norm_w, float* xn,
                 hipStream_t st, const PostNorm* post = nullptr) {
    if (post && n != 1) return fail(-1, "enqueue_proj: post-norm needs one matrix");
    bool done[SEG_MAX] = {};
    if (n > SEG_MAX) return fail(-1, "enqueue_proj: %d matrices", n);
    auto fam = [](int c) { return c == DRACO_Q8_0 ? 0 : (c == DRACO_Q4_K || c == DRACO_Q6_K ? 1 : 2); };
    bool plain_x_ready = false;
    for (int i = 0; i < n; i++) {
        if (done[i]) continue;
        const int f = fam(p[i].m->L.code);
        if (f == 2) {
            const float* xin = x;
            if (norm_w) {
                if (!plain_x_ready) dk_rmsnorm(x, norm_w, xn, n_in, QEPS, st);
                plain_x_ready = true;
                xin = xn;
            }
            if (draco_gemv_launch(*p[i].m, xin, p[i].y, p[i].yadd, 0, p[i].m->L.n_out, st))
                return fail(-1, "plain GEMV launch rejected (code %d)", p[i].m->L.code);
            if (post) dk_rmsnorm(p[i].y, post->w, post->out, p[i].m->L.n_out, QEPS, st);
            done[i] = true;
            continue;
        }
        SegLaunch s = {};
        s.n_in = n_in;
        s.x = x;
        s.do_norm = norm_w ? 1 : 0;
        s.norm_w = norm_w;
        s.eps = QEPS;
        for (int j = i; j < n; j++) {
            if (done[j] || fam(p[j].m->L.code) != f) continue;
            SegDesc d = {};
            d.base = p[j].m->dev;
            d.L = p[j].m->L;
            d.epi = p[j].yadd ? EPI_RESID : EPI_STORE;
            d.y = p[j].y;
            d.yadd = p[j].yadd;
            s.seg[s.nseg++] = d;
            done[j] = true;
        }
        if (draco_seg_launch(s, st)) return fail(-1, "segment GEMV launch rejected");
        if (post) dk_rmsnorm(p[i].y, post->w, post->out, p[i].m->L.n_out, QEPS, st);
    }
    return 0;
}

// ------------------------------------------------------------------ GDN --
struct GdnDev {
    const DracoMat *qkv, *gate, *out;
    const float *attn_norm, *bw, *aw, *ssm_a, *ssm_dt, *conv, *ssm_norm, *post_norm;
    int n_qkv, n_vh, d_in;
};

struct GdnBufs {
    float *h1, *qkv, *z, *on, *x2o, *x2n, *xn, *S, *tail;
};

int gdn_resolve(const GdnW* w, GdnDev& g) {
    if (!w) return fail(-1, "m6_gdn_attn: null descriptor");
    g.n_qkv = w->n_qkv;
    g.n_vh = w->n_vh;
    g.d_in = w->d_in;
    if (g.n_vh < 1 || g.n_vh > 64 || g.n_qkv != 2 * QNKH * QSV + g.n_vh * QSV || g.d_in != g.n_vh * QSV)
        return fail(-1, "m6_gdn_attn: n_qkv %d / n_vh %d / d_in %d is not the 16-head 128-wide split", g.n_qkv,
                    g.n_vh, g.d_in);
    g.qkv = get_mat(w->qkv_buf, w->qkv_code, g.n_qkv, QH);
    g.gate = get_mat(w->gate_buf, w->gate_code, g.n_vh * QSV, QH);
    g.out = get_mat(w->ssm_out_buf, w->ssm_out_code, QH, g.d_in);
    if (!g.qkv || !g.gate || !g.out) return -1;
    g.attn_norm = get_vec(w->attn_norm, QH);
    g.bw = get_vec(w->beta_wt, (size_t)QH * g.n_vh, g.n_vh);
    g.aw = get_vec(w->alpha_wt, (size_t)QH * g.n_vh, g.n_vh);
    g.ssm_a = get_vec(w->ssm_a, g.n_vh);
    g.ssm_dt = get_vec(w->ssm_dt, g.n_vh);
    g.conv = get_vec(w->conv, (size_t)g.n_qkv * 4);
    g.ssm_norm = get_vec(w->ssm_norm, QSV);
    g.post_norm = get_vec(w->post_norm, QH);
    if (!g.attn_norm || !g.bw || !g.aw || !g.ssm_a || !g.ssm_dt || !g.conv || !g.ssm_norm || !g.post_norm)
        return -2;
    return 0;
}

int gdn_bufs(const GdnDev& g, int slot, GdnBufs& b) {
    const size_t ns = (size_t)g.n_vh * QSV * QSV, nt = (size_t)g.n_qkv * 3;
    const size_t n = 5 * (size_t)QH + g.n_qkv + 2 * (size_t)g.d_in + ns + nt + 16 * 64;  // + carve slack
    float* p = (float*)scratch(slot, sizeof(float) * n);
    if (!p) return -2;
    auto take = [&](size_t k) {  // 256-byte aligned carve
        float* r = p;
        p += (k + 63) & ~(size_t)63;
        return r;
    };
    b.h1 = take(QH);
    b.x2o = take(QH);
    b.x2n = take(QH);
    b.xn = take(QH);
    b.qkv = take(g.n_qkv);
    b.z = take(g.d_in);
    b.on = take(g.d_in);
    b.S = take(ns);
    b.tail = take(nt);
    return 0;
}

int enqueue_gdn(const GdnDev& g, const GdnBufs& b, hipStream_t st) {
    const Proj in[2] = {{g.qkv, b.qkv, nullptr}, {g.gate, b.z, nullptr}};
    if (int rc = enqueue_proj(in, 2, b.h1, QH, g.attn_norm, b.xn, st)) return rc;
    GdnArgs a = {};
    a.QKV = b.qkv;
    a.Z = b.z;
    a.conv = g.conv;
    a.ssm_norm = g.ssm_norm;
    a.tail = b.tail;
    a.S = b.S;
    a.ON = b.on;
    a.T = 1;
    a.n_qkv = g.n_qkv;
    a.n_vh = g.n_vh;
    a.nhq = QNKH;
    a.h1 = b.h1;
    a.attn_norm = g.attn_norm;
    a.bw = g.bw;
    a.aw = g.aw;
    a.ssm_a = g.ssm_a;
    a.ssm_dt = g.ssm_dt;
    a.H = QH;
    if (draco_gdn_step_launch(a, st)) return fail(-1, "gdn step launch rejected");
    const Proj out[1] = {{g.out, b.x2o, b.h1}};
    const PostNorm pn = {g.post_norm, b.x2n};
    return enqueue_proj(out, 1, b.on, g.d_in, nullptr, b.xn, st, &pn);
}

int gdn_host(const float* h1, const GdnW* w, float* ssm, float* tail, float* x2n, float* x2_out) {
    if (int rc = ensure_init()) return rc;
    GdnDev g;
    if (int rc = gdn_resolve(w, g)) return rc;
    GdnBufs b;
    if (gdn_bufs(g, 20, b)) return -2;
    hipStream_t st = stream();
    const size_t ns = (size_t)g.n_vh * QSV * QSV, nt = (size_t)g.n_qkv * 3;
    DRACO_HIP(hipMemcpyAsync(b.h1, h1, sizeof(float) * QH, hipMemcpyHostToDevice, st));
    DRACO_HIP(hipMemcpyAsync(b.S, ssm, sizeof(float) * ns, hipMemcpyHostToDevice, st));
    DRACO_HIP(hipMemcpyAsync(b.tail, tail, sizeof(float) * nt, hipMemcpyHostToDevice, st));
    if (int rc = enqueue_gdn(g, b, st)) return rc;
    DRACO_HIP(hipGetLastError());
    DRACO_HIP(hipMemcpyAsync(x2n, b.x2n, sizeof(float) * QH, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipMemcpyAsync(x2_out, b.x2o, sizeof(float) * QH, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipMemcpyAsync(ssm, b.S, sizeof(float) * ns, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipMemcpyAsync(tail, b.tail, sizeof(float) * nt, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipStreamSynchronize(st));
    return 0;
}

// --------------------------------------------------------- full attention --
struct FullDev {
    const DracoMat *q, *k, *v, *o;
    const float *attn_norm, *q_norm, *k_norm, *post_norm;
    int nh;
};

struct FullBufs {
    float *h1, *QG, *Qr, *kraw, *kc, *vc, *ao, *part, *cs, *x2o, *x2n, *xn;
    int* state;
};

int full_resolve(const FullW* w, FullDev& f) {
    if (!w) return fail(-1, "m6_full_attn: null descriptor");
    f.nh = w->nh;
    if (f.nh < FNKV || f.nh % FNKV || f.nh / FNKV > 16)
        return fail(-1, "m6_full_attn: nh %d (needs an even count of at most 32)", f.nh);
    f.q = get_mat(w->q_buf, w->q_code, f.nh * 2 * FHD, QH);
    f.k = get_mat(w->k_buf, w->k_code, FNKV * FHD, QH);
    f.v = get_mat(w->v_buf, w->v_code, FNKV * FHD, QH);
    f.o = get_mat(w->o_buf, w->o_code, QH, f.nh * FHD);
    if (!f.q || !f.k || !f.v || !f.o) return -1;
    f.attn_norm = get_vec(w->attn_norm, QH);
    f.q_norm = get_vec(w->q_norm, FHD);
    f.k_norm = get_vec(w->k_norm, FHD);
    f.post_norm = get_vec(w->post_norm, QH);
    if (!f.attn_norm || !f.q_norm || !f.k_norm || !f.post_norm) return -2;
    return 0;
}

// buffers for caches of up to max_t rows
int full_bufs(const FullDev& f, int max_t, int slot, FullBufs& b) {
    const int nsplit = attn_nsplit(max_t, f.nh, FNKV, FHD);
    const size_t kv = (size_t)max_t * FNKV * FHD;
    const size_t part = (size_t)f.nh * nsplit * (FHD + 2);
    const size_t n = 5 * (size_t)QH + (size_t)f.nh * 2 * FHD + 2 * (size_t)f.nh * FHD + FNKV * FHD + 2 * kv +
                     part + 64 + 64 + 16 * 64;
    float* p = (float*)scratch(slot, sizeof(float) * n);
    if (!p) return -2;
    auto take = [&](size_t k) {
        float* r = p;
        p += (k + 63) & ~(size_t)63;
        return r;
    };
    b.h1 = take(QH);
    b.x2o = take(QH);
    b.x2n = take(QH);
    b.xn = take(QH);
    b.QG = take((size_t)f.nh * 2 * FHD);
    b.Qr = take((size_t)f.nh * FHD);
    b.ao = take((size_t)f.nh * FHD);
    b.kraw = take(FNKV * FHD);
    b.kc = take(kv);
    b.vc = take(kv);
    b.part = take(part);
    b.cs = take(64);
    b.state = (int*)take(64);
    return 0;
}

// rope table of one position, computed as the reference does in fp32
// (src/m6_layer.c:434-440): ang = (float)pos0 * rope_inv[t]
void rope_cs(const float* rope_inv, int pos0, float* cs) {
    for (int t = 0; t < 32; t++) {
        const float ang = (float)pos0 * rope_inv[t];
        cs[2 * t] = cosf(ang);
        cs[2 * t + 1] = sinf(ang);
    }
}

// state[0] = pos0, state[1] = Told must already be on the device, with cache
// rows [0, Told) in b.kc / b.vc; row Told is written here.
int enqueue_full(const FullDev& f, const FullBufs& b, int told, hipStream_t st) {
    const size_t row = (size_t)told * FNKV * FHD;
    const Proj in[3] = {{f.q, b.QG, nullptr}, {f.k, b.kraw, nullptr}, {f.v, b.vc + row, nullptr}};
    if (int rc = enqueue_proj(in, 3, b.h1, QH, f.attn_norm, b.xn, st)) return rc;
    dk_fa_prep(b.QG, b.Qr, b.kraw, b.kc + row, f.q_norm, f.k_norm, b.cs, f.nh, st);
    if (dk_attention(b.Qr, b.kc, b.vc, b.part, nullptr, b.ao, b.state, 0, f.nh, FNKV, FHD, told + 1,
                     1.f / sqrtf((float)FHD), st, b.QG + FHD, 2 * FHD))
        return fail(-1, "attention launch rejected");
    const Proj out[1] = {{f.o, b.x2o, b.h1}};
    const PostNorm pn = {f.post_norm, b.x2n};
    return enqueue_proj(out, 1, b.ao, f.nh * FHD, nullptr, b.xn, st, &pn);
}

int full_host(const float* h1, const FullW* w, const float* Kr, const float* Vc, int told, int pos0, float* x2n,
              float* x2_out, float* kr_new, float* v_new) {
    if (told < 0) return fail(-1, "m6_full_attn: Told %d", told);
    if (int rc = ensure_init()) return rc;
    FullDev f;
    if (int rc = full_resolve(w, f)) return rc;
    FullBufs b;
    if (full_bufs(f, told + 1, 21, b)) return -2;
    float* hs = (float*)pinned(5, sizeof(float) * 128);
    if (!hs) return -2;
    rope_cs(w->rope_inv, pos0, hs);
    int* hi = (int*)(hs + 64);
    hi[0] = pos0;
    hi[1] = told;
    hipStream_t st = stream();
    const size_t rowf = (size_t)FNKV * FHD;
    DRACO_HIP(hipMemcpyAsync(b.h1, h1, sizeof(float) * QH, hipMemcpyHostToDevice, st));
    DRACO_HIP(hipMemcpyAsync(b.cs, hs, sizeof(float) * 64, hipMemcpyHostToDevice, st));
    DRACO_HIP(hipMemcpyAsync(b.state, hi, sizeof(int) * 2, hipMemcpyHostToDevice, st));
    if (told > 0) {
        DRACO_HIP(hipMemcpyAsync(b.kc, Kr, sizeof(float) * rowf * told, hipMemcpyHostToDevice, st));
        DRACO_HIP(hipMemcpyAsync(b.vc, Vc, sizeof(float) * rowf * told, hipMemcpyHostToDevice, st));
    }
    if (int rc = enqueue_full(f, b, told, st)) return rc;
    DRACO_HIP(hipGetLastError());
    DRACO_HIP(hipMemcpyAsync(x2n, b.x2n, sizeof(float) * QH, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipMemcpyAsync(x2_out, b.x2o, sizeof(float) * QH, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipMemcpyAsync(kr_new, b.kc + rowf * told, sizeof(float) * rowf, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipMemcpyAsync(v_new, b.vc + rowf * told, sizeof(float) * rowf, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipStreamSynchronize(st));
    return 0;
}

// graph-replayed timing of `iters` launches sequences recorded by `enq`
template <class F>
int time_graph(int iters, F enq, float* us) {
    hipStream_t st = stream();
    hipGraph_t graph;
    hipGraphExec_t exec;
    DRACO_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
    for (int i = 0; i < iters; i++)
        if (int rc = enq()) {
            hipStreamEndCapture(st, &graph);
            return rc;
        }
    DRACO_HIP(hipStreamEndCapture(st, &graph));
    DRACO_HIP(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    hipEvent_t e0, e1;
    DRACO_HIP(hipEventCreate(&e0));
    DRACO_HIP(hipEventCreate(&e1));
    DRACO_HIP(hipGraphLaunch(exec, st));
    DRACO_HIP(hipEventRecord(e0, st));
    DRACO_HIP(hipGraphLaunch(exec, st));
    DRACO_HIP(hipEventRecord(e1, st));
    DRACO_HIP(hipStreamSynchronize(st));
    float ms = 0.f;
    DRACO_HIP(hipEventElapsedTime(&ms, e0, e1));
    *us = ms * 1000.f / iters;
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    hipGraphExecDestroy(exec);
    hipGraphDestroy(graph);
    return 0;
}

}  // namespace

extern "C" {

// src/m6_layer.c:205-364
void m6_gdn_attn(const float* h1, const GdnW* w, float* ssm, float* tail, float* buf, float* x2n,
                 float* x2_out) {
    (void)buf;
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = gdn_host(h1, w, ssm, tail, x2n, x2_out)) report(rc, "m6_gdn_attn");
}

// src/m6_layer.c:389-518
void m6_full_attn(const float* h1, const FullW* w, const float* Kr, const float* Vc, int Told, int pos0,
                  float* buf, float* scores, float* x2n, float* x2_out, float* kr_new, float* v_new) {
    (void)buf;
    (void)scores;
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = full_host(h1, w, Kr, Vc, Told, pos0, x2n, x2_out, kr_new, v_new)) report(rc, "m6_full_attn");
}

// Device-resident timing of one qwen35 layer op (no reference counterpart).
// kind 0: m6_gdn_attn with descriptor w (GdnW*), state taken from ssm/tail
// (not modified); kind 1: m6_full_attn (FullW*) at cache length told (cache
// rows uploaded from Kr/Vc, not modified).  The state advances across the
// replayed steps exactly as in a decode loop (GDN state updated in place;
// full attention re-attends the same told rows).  out[0] us per op from a
// graph replay of `iters` ops, out[1] weight bytes per op (device layout),
// out[2] algorithmic HBM bytes per op (weights + state / KV traffic).
int draco_bench_qwen_op(int kind, const void* w, const float* h1, const float* ssm_or_kr,
                        const float* tail_or_vc, int told, int iters, float* out) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (iters < 1 || !out) return fail(-1, "bench qwen: bad arguments");
    if (int rc = ensure_init()) return rc;
    hipStream_t st = stream();
    if (kind == 0) {
        GdnDev gd;
        if (int rc = gdn_resolve((const GdnW*)w, gd)) return rc;
        GdnBufs b;
        if (gdn_bufs(gd, 22, b)) return -2;
        const size_t ns = (size_t)gd.n_vh * QSV * QSV, nt = (size_t)gd.n_qkv * 3;
        DRACO_HIP(hipMemcpy(b.h1, h1, sizeof(float) * QH, hipMemcpyHostToDevice));
        DRACO_HIP(hipMemcpy(b.S, ssm_or_kr, sizeof(float) * ns, hipMemcpyHostToDevice));
        DRACO_HIP(hipMemcpy(b.tail, tail_or_vc, sizeof(float) * nt, hipMemcpyHostToDevice));
        if (int rc = time_graph(iters, [&] { return enqueue_gdn(gd, b, st); }, &out[0])) return rc;
        const double wb = (double)gd.qkv->L.bytes + gd.gate->L.bytes + gd.out->L.bytes;
        out[1] = (float)wb;
        // + beta/alpha rows, state read + write, conv taps, tail r/w, activations
        out[2] = (float)(wb + 2.0 * QH * gd.n_vh * 4 + 2.0 * ns * 4 + gd.n_qkv * 4.0 * 4 + 2.0 * nt * 4);
        return 0;
    }
    if (kind == 1) {
        FullDev fd;
        if (told < 0) return fail(-1, "bench qwen: told %d", told);
        if (int rc = full_resolve((const FullW*)w, fd)) return rc;
        FullBufs b;
        if (full_bufs(fd, told + 1, 23, b)) return -2;
        const FullW* fw = (const FullW*)w;
        float cs[64];
        rope_cs(fw->rope_inv, told, cs);
        const int hi[2] = {told, told};
        const size_t rowf = (size_t)FNKV * FHD;
        DRACO_HIP(hipMemcpy(b.h1, h1, sizeof(float) * QH, hipMemcpyHostToDevice));
        DRACO_HIP(hipMemcpy(b.cs, cs, sizeof(cs), hipMemcpyHostToDevice));
        DRACO_HIP(hipMemcpy(b.state, hi, sizeof(hi), hipMemcpyHostToDevice));
        if (told > 0) {
            DRACO_HIP(hipMemcpy(b.kc, ssm_or_kr, sizeof(float) * rowf * told, hipMemcpyHostToDevice));
            DRACO_HIP(hipMemcpy(b.vc, tail_or_vc, sizeof(float) * rowf * told, hipMemcpyHostToDevice));
        }
        if (int rc = time_graph(iters, [&] { return enqueue_full(fd, b, told, st); }, &out[0])) return rc;
        const double wb = (double)fd.q->L.bytes + fd.k->L.bytes + fd.v->L.bytes + fd.o->L.bytes;
        out[1] = (float)wb;
        out[2] = (float)(wb + 2.0 * (told + 1) * rowf * 4);
        return 0;
    }
    return fail(-1, "bench qwen: kind %d", kind);
}

}  // extern "C"
