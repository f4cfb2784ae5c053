// abi_qwen.cpp -- qwen35 hybrid-layer decode ops: m6_gdn_attn (Gated-DeltaNet
// layer) and m6_full_attn (gated full attention), src/m6_layer.c:189-518.
//
// Host pointers in and out, as in the reference.  The recurrent state (ssm,
// tail) and the cached K / V rows stay in device mirrors of the caller's
// arrays between calls (the residency rules are next to gdn_host below), so
// a call moves h1 in and the outputs out.  Weights and fp32 parameter arrays
// are registered by host address and stay resident.  The reference's scratch
// arguments (buf, scores) are accepted and not used.
//
// Device work per GDN token (4 launches):
//   k_dq      qkv + gate projections, attention RMSNorm in the prologue
//   k_gdn     per V head: beta / decay from xn, conv + silu, l2 norms, delta
//             rule on the register-resident state, gated rms   -> on
//   k_dq      ssm_out projection + residual                     -> x2_out
//   k_rmsnorm post-attention norm                               -> x2n
// Device work per full-attention token (6 launches):
//   k_dq        q+gate, k, v projections (v straight into cache row Told)
//   k_fa_prep   q / k head RMSNorm + rope (k into cache row Told)
//   k_attn_gqa  split-T attention over Told + 1 rows, each K / V row read
//               once per GQA group; k_attn_merge merges the splits and
//               applies the sigmoid gate
//   k_dq        o projection + residual; k_rmsnorm               -> x2n
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <vector>

#include "decode.h"
#include "gdn.h"
#include "gemm.h"
#include "gemv.h"
#include "moe.h"
#include "prefill.h"
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

// the dense FFN op's parameters (src/m6_engine.c:270-273), as in abi_m6.cpp
typedef struct {
    const uint8_t *g, *u, *d;
    int cg, cu, cd, n_ff, h;
} M6DenseP;

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
// With `pend` (a pending residual, x + pend[0..n_in) + pend[n_in..2 n_in))
// every matrix must be a K-quant (one launch): its prologue forms the sum,
// normalises it and stores it to pend_sum.
// With `gd` the K-quant launch also dots gd->n rows of gd->w0 and of gd->w1
// ([n][n_in] fp32) with the normalised x into gd->out[0 .. 2n), when it can;
// gd->done says whether it did.
struct GateDots {
    const float* w0;
    const float* w1;
    int n;
    float* out;
    bool done;
};

int enqueue_proj(const Proj* p, int n, const float* x, int n_in, const float* norm_w, float* xn,
                 hipStream_t st, const PostNorm* post = nullptr, const float* pend = nullptr,
                 float* pend_sum = nullptr, GateDots* gd = nullptr) {
    if (gd) gd->done = false;
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
        if (pend) {
            if (f != 1 || !norm_w || !pend_sum) return fail(-1, "enqueue_proj: a pending residual needs K-quants");
            s.do_norm = 3;
            s.am_val = const_cast<float*>(pend);
            s.xn_out = pend_sum;
        }
        if (gd && f == 1 && norm_w && gd->out) {
            s.gdot_w0 = gd->w0;
            s.gdot_w1 = gd->w1;
            s.gdot_out = gd->out;
            s.gdot_n = gd->n;
        }
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
        if (gd && s.gdot_done) gd->done = true;
        if (pend) {
            for (int j = 0; j < n; j++)
                if (!done[j]) return fail(-1, "enqueue_proj: a pending residual needs one launch");
        }
        if (post) dk_rmsnorm(p[i].y, post->w, post->out, p[i].m->L.n_out, QEPS, st);
    }
    return 0;
}

// A split-K projection of x (n_in wide) into the two partials pd[0..n_out) and
// pd[n_out..2 n_out) (SegLaunch.ksplit), optionally with the GDN gated-rms
// prologue (gnorm_pss: its partial sums of squares).
int enqueue_proj_ks(const DracoMat* m, const float* x, int n_in, float* pd, const float* gnorm_pss,
                    hipStream_t st) {
    SegLaunch s = {};
    s.nseg = 1;
    s.n_in = n_in;
    s.x = x;
    s.ksplit = 2;
    if (gnorm_pss) {
        s.do_norm = 2;
        s.eps = QEPS;
        s.kc = const_cast<float*>(gnorm_pss);
    }
    SegDesc& d = s.seg[0];
    d.base = m->dev;
    d.L = m->L;
    d.row0 = 0;
    d.row1 = m->L.n_out;
    d.y = pd;
    d.epi = EPI_STORE;
    if (draco_seg_launch(s, st)) return fail(-1, "split-K projection launch rejected");
    return 0;
}

// Whether a projection can run split-K (rows of 16 or 32 super-blocks, at
// most 128 row tiles: the launches that leave CUs idle otherwise).
bool ks_ok(const DracoMat* m) {
    const int nb = m->L.n_in / 256;
    return (m->L.code == DRACO_Q4_K || m->L.code == DRACO_Q6_K) && m->L.n_in % 256 == 0 && (nb == 16 || nb == 32) &&
           draco_dq_ksplit_waves(m->L.n_in, 2) && (m->L.n_out + 15) / 16 <= 128;
}

// ------------------------------------------------------------------ GDN --
struct GdnDev {
    const DracoMat *qkv, *gate, *out;
    const float *attn_norm, *bw, *aw, *ssm_a, *ssm_dt, *conv, *ssm_norm, *post_norm;
    int n_qkv, n_vh, d_in;
};

struct GdnBufs {
    float *h1, *qkv, *z, *on, *x2o, *x2n, *xn, *S, *tail, *pss;
    // the stack's pending residual: the layer input is h1 + pend[0..H) +
    // pend[H..2H), formed into pend_sum by the in-projection (then the
    // layer's input for the scan's gates and the residual); with ks_out the
    // ssm_out projection runs split-K into ks_out instead of adding its
    // residual into x2o
    const float* pend;
    float *pend_sum, *ks_out;
    // nullable: [2 n_vh] for the gates' dots formed by the in-projection
    float* glog;
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
    const size_t n = 5 * (size_t)QH + g.n_qkv + 2 * (size_t)g.d_in + ns + nt + (size_t)g.n_vh * GDN_PSS_STRIDE +
                     2 * (size_t)g.n_vh + 16 * 64;  // + carve slack
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
    b.pss = take((size_t)g.n_vh * GDN_PSS_STRIDE);
    b.glog = take(2 * (size_t)g.n_vh);
    b.pend = nullptr;
    b.pend_sum = nullptr;
    b.ks_out = nullptr;
    return 0;
}

// post_norm false: x2n is not produced (a stack whose FFN normalises x2_out
// itself, or has none)
int enqueue_gdn(const GdnDev& g, const GdnBufs& b, hipStream_t st, bool post_norm = true) {
    const Proj in[2] = {{g.qkv, b.qkv, nullptr}, {g.gate, b.z, nullptr}};
    // the gates' dots (xn.beta_wt, xn.alpha_wt rows) ride on the in-projection
    // when it is one K-quant launch with blocks to spare
    GateDots gd = {g.bw, g.aw, g.n_vh, b.glog, false};
    if (int rc = enqueue_proj(in, 2, b.h1, QH, g.attn_norm, b.xn, st, nullptr, b.pend, b.pend_sum,
                              b.glog ? &gd : nullptr))
        return rc;
    const float* h1 = b.pend ? b.pend_sum : b.h1;
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
    a.h1 = h1;
    a.attn_norm = g.attn_norm;
    a.bw = g.bw;
    a.aw = g.aw;
    a.ssm_a = g.ssm_a;
    a.ssm_dt = g.ssm_dt;
    a.H = QH;
    a.glog = b.glog && gd.done ? b.glog : nullptr;
    a.PSS = b.pss;
    // split over several blocks per V head only when the ssm_out GEMV can
    // take the gated rms into its prologue (Q4_K / Q6_K): the split's extra
    // k_gdn_gnorm launch costs more than the split saves
    const bool kq = g.out->L.code == DRACO_Q4_K || g.out->L.code == DRACO_Q6_K;
    a.nspl = kq ? draco_gdn_split(true) : 1;
    a.defer_gnorm = a.nspl > 1;
    if (draco_gdn_step_launch(a, st)) return fail(-1, "gdn step launch rejected");
    if (b.ks_out && !a.defer_gnorm) return fail(-1, "gdn: split-K ssm_out needs the gated-rms prologue");
    if (b.ks_out) return enqueue_proj_ks(g.out, b.on, g.d_in, b.ks_out, b.pss, st);
    if (a.defer_gnorm) {
        SegLaunch s = {};
        s.nseg = 1;
        s.n_in = g.d_in;
        s.x = b.on;
        s.do_norm = 2;
        s.eps = QEPS;
        s.kc = b.pss;
        SegDesc& d = s.seg[0];
        d.base = g.out->dev;
        d.L = g.out->L;
        d.epi = EPI_RESID;
        d.y = b.x2o;
        d.yadd = h1;
        if (draco_seg_launch(s, st)) return fail(-1, "gdn ssm_out launch rejected");
        if (post_norm) dk_rmsnorm(b.x2o, g.post_norm, b.x2n, QH, QEPS, st);
        return 0;
    }
    const Proj out[1] = {{g.out, b.x2o, h1}};
    const PostNorm pn = {g.post_norm, b.x2n};
    return enqueue_proj(out, 1, b.on, g.d_in, nullptr, b.xn, st, post_norm ? &pn : nullptr);
}

// ---- state residency of the per-layer ops ----
// m6_gdn_attn and m6_full_attn keep the caller's state arrays on the device:
// the GDN recurrent state and conv tail and the full-attention K / V rows
// live in mirrors keyed by the arrays' host addresses (the same mirrors the
// qwen stack entry points use), so a call moves h1 in and x2n / x2_out
// (+ kr_new / v_new) out.  The caller's arrays are not kept current
// (draco_array_pull copies a mirror back, draco_array_push forces an
// upload).  A write of the caller's own is detected:
//  - GDN: after every call the first QSAMP floats of the device state are
//    written into the caller's ssm.  If at the next call they are not there
//    bit for bit (a reset that zeroed the arrays, a restored snapshot), the
//    state and tail are uploaded from the caller's arrays.
//  - full attention: the caller appends kr_new / v_new to its own rows (the
//    reference's driver, src/qwen35_engine.py:317-323), so its rows equal
//    the device's.  The first float of every row the device holds is kept
//    here; up to 17 rows of [0, Told) are compared per call, and a mismatch
//    uploads rows [0, Told).  Rows the device never held are uploaded too.
constexpr int QSAMP = 128;

struct OpState {
    const void* dev = nullptr;     // the mirror these records describe
    std::vector<uint32_t> samp;    // GDN: written-back state floats
    int rows = 0;                  // full attention: leading rows the device holds
    int cap = 0;                   // full attention: rows the mirrors were sized for
    std::vector<uint32_t> shk, shv;  // full attention: first float of each held row
};

std::map<const void*, OpState>& op_states() {
    static auto* m = new std::map<const void*, OpState>();
    return *m;
}

uint32_t fbits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

int gdn_host(const float* h1, const GdnW* w, float* ssm, float* tail, float* x2n, float* x2_out) {
    if (int rc = ensure_init()) return rc;
    GdnDev g;
    if (int rc = gdn_resolve(w, g)) return rc;
    GdnBufs b;
    if (gdn_bufs(g, 20, b)) return -2;
    hipStream_t st = stream();
    const size_t ns = (size_t)g.n_vh * QSV * QSV, nt = (size_t)g.n_qkv * 3;
    bool fs = false, ft = false;
    b.S = (float*)get_mirror(ssm, sizeof(float) * ns, &fs);
    b.tail = (float*)get_mirror(tail, sizeof(float) * nt, &ft);
    if (!b.S || !b.tail) return -2;
    OpState& os = op_states()[ssm];
    bool upload = fs || ft || os.dev != b.S || os.samp.size() != QSAMP;
    for (int i = 0; !upload && i < QSAMP; i++) upload = fbits(ssm[i]) != os.samp[i];
    if (upload) {
        DRACO_HIP(hipMemcpyAsync(b.S, ssm, sizeof(float) * ns, hipMemcpyHostToDevice, st));
        DRACO_HIP(hipMemcpyAsync(b.tail, tail, sizeof(float) * nt, hipMemcpyHostToDevice, st));
    }
    // pinned staging: h1 in; x2_out, x2n (adjacent on the device) and the
    // state sample out
    float* hp = (float*)pinned(5, sizeof(float) * (3 * QH + QSAMP));
    if (!hp) return -2;
    memcpy(hp, h1, sizeof(float) * QH);
    DRACO_HIP(hipMemcpyAsync(b.h1, hp, sizeof(float) * QH, hipMemcpyHostToDevice, st));
    if (int rc = enqueue_gdn(g, b, st)) return rc;
    DRACO_HIP(hipGetLastError());
    float* ho = hp + QH;
    DRACO_HIP(hipMemcpyAsync(ho, b.x2o, sizeof(float) * 2 * QH, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipMemcpyAsync(ho + 2 * QH, b.S, sizeof(float) * QSAMP, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipStreamSynchronize(st));
    memcpy(x2_out, ho, sizeof(float) * QH);
    memcpy(x2n, ho + QH, sizeof(float) * QH);
    memcpy(ssm, ho + 2 * QH, sizeof(float) * QSAMP);
    os.dev = b.S;
    os.samp.resize(QSAMP);
    for (int i = 0; i < QSAMP; i++) os.samp[i] = fbits(ho[2 * QH + i]);
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

// buffers for caches of up to max_t rows (with cache false, kc / vc are left
// null: the caller's mirrors hold the rows)
int full_bufs(const FullDev& f, int max_t, int slot, FullBufs& b, bool cache = true) {
    const int nsplit = attn_nsplit(max_t, f.nh, FNKV, FHD);
    const size_t kv = cache ? (size_t)max_t * FNKV * FHD : 0;
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
    // h1, cs, state adjacent (one upload), then x2_out, x2n adjacent (one
    // download)
    b.h1 = take(QH);
    b.cs = take(64);
    b.state = (int*)take(64);
    b.x2o = take(QH);
    b.x2n = take(QH);
    b.xn = take(QH);
    b.QG = take((size_t)f.nh * 2 * FHD);
    b.Qr = take((size_t)f.nh * FHD);
    b.ao = take((size_t)f.nh * FHD);
    b.kraw = take(FNKV * FHD);
    b.kc = cache ? take(kv) : nullptr;
    b.vc = cache ? take(kv) : nullptr;
    b.part = take(part);
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
    if (full_bufs(f, told + 1, 21, b, false)) return -2;
    hipStream_t st = stream();
    const size_t rowf = (size_t)FNKV * FHD, rowb = sizeof(float) * rowf;
    // K / V mirrors of at least told + 1 rows, grown by doubling (the held
    // rows move with them)
    OpState& os = op_states()[Kr];
    if (!os.dev) os.cap = os.rows = 0;
    const int need = told + 1;
    const bool grow = need > os.cap;
    if (grow) os.cap = std::max(std::max(need, 2 * os.cap), 256);
    const size_t keep = rowb * (size_t)std::min(os.rows, told);
    bool fk = false, fv = false;
    b.kc = (float*)grow_mirror(Kr, rowb * os.cap, keep, &fk);
    b.vc = (float*)grow_mirror(Vc, rowb * os.cap, keep, &fv);
    if (!b.kc || !b.vc) return -2;
    if (fk || fv || (b.kc != os.dev && !(grow && os.dev))) os.rows = 0;
    os.dev = b.kc;
    if (os.shk.size() < (size_t)os.cap) {
        os.shk.resize(os.cap);
        os.shv.resize(os.cap);
    }
    int held = std::min(os.rows, told);
    for (int i = 0; held > 0 && i <= 16; i++) {
        const int r = i == 16 ? held - 1 : (int)((int64_t)i * held / 16);
        if (fbits(Kr[(size_t)r * rowf]) != os.shk[r] || fbits(Vc[(size_t)r * rowf]) != os.shv[r]) held = 0;
    }
    if (held < told) {
        const size_t n = rowb * (size_t)(told - held);
        DRACO_HIP(hipMemcpyAsync(b.kc + (size_t)held * rowf, Kr + (size_t)held * rowf, n, hipMemcpyHostToDevice, st));
        DRACO_HIP(hipMemcpyAsync(b.vc + (size_t)held * rowf, Vc + (size_t)held * rowf, n, hipMemcpyHostToDevice, st));
        for (int r = held; r < told; r++) {
            os.shk[r] = fbits(Kr[(size_t)r * rowf]);
            os.shv[r] = fbits(Vc[(size_t)r * rowf]);
        }
    }
    // pinned staging: h1, rope cos / sin, [pos0, told] in (adjacent on the
    // device); x2_out and x2n (adjacent), kr_new, v_new out
    float* hp = (float*)pinned(5, sizeof(float) * (QH + 128 + 2 * QH + 2 * rowf));
    if (!hp) return -2;
    memcpy(hp, h1, sizeof(float) * QH);
    rope_cs(w->rope_inv, pos0, hp + QH);
    int* hi = (int*)(hp + QH + 64);
    hi[0] = pos0;
    hi[1] = told;
    DRACO_HIP(hipMemcpyAsync(b.h1, hp, sizeof(float) * (QH + 64 + 2), hipMemcpyHostToDevice, st));
    if (int rc = enqueue_full(f, b, told, st)) return rc;
    DRACO_HIP(hipGetLastError());
    float* ho = hp + QH + 128;
    DRACO_HIP(hipMemcpyAsync(ho, b.x2o, sizeof(float) * 2 * QH, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipMemcpyAsync(ho + 2 * QH, b.kc + rowf * told, rowb, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipMemcpyAsync(ho + 2 * QH + rowf, b.vc + rowf * told, rowb, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipStreamSynchronize(st));
    memcpy(x2_out, ho, sizeof(float) * QH);
    memcpy(x2n, ho + QH, sizeof(float) * QH);
    memcpy(kr_new, ho + 2 * QH, rowb);
    memcpy(v_new, ho + 2 * QH + rowf, rowb);
    os.shk[told] = fbits(kr_new[0]);
    os.shv[told] = fbits(v_new[0]);
    os.rows = told + 1;
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

// ================================================ the hybrid stack ======
// One qwen35 token as the reference's driver composes it per layer
// (src/qwen35_engine.py:310-327): the layer op (m6_gdn_attn or m6_full_attn)
// leaves x2_out = x + attn and x2n = RMSNorm(x2_out) * post_norm; the FFN of
// x2n (none, dense m6_dense_op, or MoE m6_granite_moe) is added to x2_out.
// Here every layer's state lives on the device: the recurrent state and
// conv tail of a GDN layer, the K / V rows of a full-attention layer (device
// mirrors of the caller's arrays, keyed by their host addresses; the state
// hooks move them), so a token moves no state over PCIe.

constexpr int QFFN_NONE = 0, QFFN_DENSE = 1, QFFN_MOE = 2;
constexpr int QCHUNK_MAX = 256;

struct QStackLayer {
    int kind = 0;
    const void* w = nullptr;
    float* state0 = nullptr;  // host: GDN ssm / full Kr
    float* state1 = nullptr;  // host: GDN tail / full Vc
    int max_t = 0;
    int ffn_kind = 0;
    const void* ffn = nullptr;
};

struct QLayer {
    QStackLayer desc;
    GdnW gw = {};
    FullW fw = {};
    M6DenseP dp = {};
    DracoMoeP mp = {};
    GdnDev g = {};
    FullDev f = {};
    float *S = nullptr, *tail = nullptr;  // GDN device state
    float *kc = nullptr, *vc = nullptr;   // full-attention device cache rows
    const float* cs = nullptr;            // full attention: rope cos / sin table [max_t][64]
    const DracoMat *fg = nullptr, *fu = nullptr, *fd = nullptr;  // dense FFN
    int FF = 0;
    MoeLayer* moe = nullptr;
};

struct QStack {
    uint64_t epoch = 0;
    std::vector<QStackLayer> descs;
    std::vector<QLayer> L;
    int n_layer = 0, max_qkv = 0, max_din = 0, max_nh = 0, max_t = 0, max_ff = 0, max_vh = 0;
    // one token
    float *x = nullptr, *x2n = nullptr, *xn = nullptr, *qkv = nullptr, *z = nullptr, *on = nullptr, *QG = nullptr,
          *Qr = nullptr, *kraw = nullptr, *vraw = nullptr, *ao = nullptr, *part = nullptr, *fg = nullptr,
          *fu = nullptr, *xe = nullptr, *pss = nullptr;
    float *xs = nullptr, *pd = nullptr;  // pending residual: its materialised sum and the split-K partials [2][H]
    float* glog = nullptr;               // GDN gates' dots [2][max_vh]
    int* state = nullptr;   // device [pos, told]
    int* hstate = nullptr;  // pinned
    // a prefill chunk of up to pf_cap tokens
    int pf_cap = 0;
    float *X = nullptr, *Xn = nullptr, *QKV = nullptr, *Z = nullptr, *B = nullptr, *G = nullptr, *ON = nullptr,
          *Y = nullptr, *PQG = nullptr, *PQr = nullptr, *PK = nullptr, *PV = nullptr, *AO = nullptr, *Ppart = nullptr,
          *PG = nullptr, *PU = nullptr, *PPSS = nullptr;
    uint8_t* dig = nullptr;
    int* ids = nullptr;
    std::vector<void*> allocs, pf_allocs;
};

std::map<const void*, QStack*>& qstacks() {
    static auto* m = new std::map<const void*, QStack*>();
    return *m;
}

// rope cos / sin of positions [0, rows) for one rope_inv table, computed as
// the reference does per token ((float)pos * rope_inv[t], cosf / sinf,
// src/m6_layer.c:434-440); device copy cached per (host table, rows)
const float* rope_rows(const float* rope_inv, int rows) {
    struct Tab {
        float* dev = nullptr;
        int rows = 0;
        std::vector<float> inv;
    };
    static auto* tabs = new std::map<const float*, Tab>();
    Tab& t = (*tabs)[rope_inv];
    const bool same = t.inv.size() == 32 && memcmp(t.inv.data(), rope_inv, sizeof(float) * 32) == 0;
    if (t.dev && same && t.rows >= rows) return t.dev;
    std::vector<float> h((size_t)rows * 64);
    for (int p = 0; p < rows; p++) rope_cs(rope_inv, p, h.data() + (size_t)p * 64);
    if (t.dev) {
        hipStreamSynchronize(stream());
        hipFree(t.dev);
        t.dev = nullptr;
    }
    if (hipMalloc(&t.dev, sizeof(float) * h.size()) != hipSuccess ||
        hipMemcpy(t.dev, h.data(), sizeof(float) * h.size(), hipMemcpyHostToDevice) != hipSuccess) {
        fail(-2, "qwen stack: rope table upload failed");
        t = Tab();
        return nullptr;
    }
    t.rows = rows;
    t.inv.assign(rope_inv, rope_inv + 32);
    return t.dev;
}

// device state of one layer: a mirror of the caller's array, uploaded when
// the mirror is new (the caller's array holds the state to start from)
float* state_mirror(float* host, size_t floats) {
    bool fresh = false;
    float* d = (float*)get_mirror(host, sizeof(float) * floats, &fresh);
    if (d && fresh && hipMemcpy(d, host, sizeof(float) * floats, hipMemcpyHostToDevice) != hipSuccess) {
        fail(-2, "qwen stack: state upload failed");
        return nullptr;
    }
    return d;
}

size_t gdn_state_floats(const GdnDev& g) { return (size_t)g.n_vh * QSV * QSV; }
size_t gdn_tail_floats(const GdnDev& g) { return (size_t)g.n_qkv * 3; }
size_t full_cache_floats(int max_t) { return (size_t)max_t * FNKV * FHD; }

int qstack_alloc(std::vector<void*>& keep, float** p, size_t floats) {
    if (hipMalloc(p, sizeof(float) * (floats + 64)) != hipSuccess) return fail(-2, "qwen stack: allocation failed");
    keep.push_back(*p);
    return 0;
}

// Frees a stack's device buffers and pinned state (its mirrors stay
// registered: they hold the caller's state).
void release_qstack(QStack* s) {
    if (!s) return;
    hipStreamSynchronize(stream());
    for (void* p : s->allocs) hipFree(p);
    for (void* p : s->pf_allocs) hipFree(p);
    if (s->hstate) hipHostFree(s->hstate);
    delete s;
}

QStack* build_qstack(const QStackLayer* layers, int n_layer, int h) {
    if (h != QH) {
        fail(-1, "qwen stack: hidden %d (the qwen35 ops fix it at %d)", h, QH);
        return nullptr;
    }
    if (n_layer < 1) {
        fail(-1, "qwen stack: no layers");
        return nullptr;
    }
    QStack*& slot = qstacks()[layers];
    if (slot && slot->epoch == epoch() && slot->n_layer == n_layer &&
        memcmp(slot->descs.data(), layers, sizeof(QStackLayer) * n_layer) == 0) {
        bool same = true;
        for (int l = 0; same && l < n_layer; l++) {
            const QLayer& q = slot->L[l];
            same = q.desc.kind == 0 ? memcmp(&q.gw, q.desc.w, sizeof(GdnW)) == 0
                                    : memcmp(&q.fw, q.desc.w, sizeof(FullW)) == 0;
            if (same && q.desc.ffn_kind == QFFN_DENSE) same = memcmp(&q.dp, q.desc.ffn, sizeof(M6DenseP)) == 0;
            if (same && q.desc.ffn_kind == QFFN_MOE)
                same = memcmp(&q.mp, q.desc.ffn, sizeof(DracoMoeP)) == 0 &&
                       draco_moe_layer((const DracoMoeP*)q.desc.ffn) == q.moe;
        }
        if (same && slot->epoch == epoch()) return slot;
    }
    if (slot) {  // rebuild: release the old token buffers (mirrors stay registered)
        release_qstack(slot);
        slot = nullptr;
    }
    // a stack that fails part-way is released on the way out
    struct Building {
        QStack* s;
        ~Building() { release_qstack(s); }
    } building{new QStack()};
    QStack* s = building.s;
    s->descs.assign(layers, layers + n_layer);
    s->L.resize(n_layer);
    s->n_layer = n_layer;
    for (int l = 0; l < n_layer; l++) {
        QLayer& q = s->L[l];
        q.desc = layers[l];
        if (q.desc.kind == 0) {
            q.gw = *(const GdnW*)q.desc.w;
            if (gdn_resolve(&q.gw, q.g)) return nullptr;
            q.S = state_mirror(q.desc.state0, gdn_state_floats(q.g));
            q.tail = state_mirror(q.desc.state1, gdn_tail_floats(q.g));
            if (!q.S || !q.tail) return nullptr;
            s->max_qkv = std::max(s->max_qkv, q.g.n_qkv);
            s->max_din = std::max(s->max_din, q.g.d_in);
            s->max_vh = std::max(s->max_vh, q.g.n_vh);
        } else if (q.desc.kind == 1) {
            q.fw = *(const FullW*)q.desc.w;
            if (full_resolve(&q.fw, q.f)) return nullptr;
            if (q.desc.max_t < 1) {
                fail(-1, "qwen stack: layer %d: full attention needs max_t >= 1", l);
                return nullptr;
            }
            q.kc = state_mirror(q.desc.state0, full_cache_floats(q.desc.max_t));
            q.vc = state_mirror(q.desc.state1, full_cache_floats(q.desc.max_t));
            q.cs = rope_rows(q.fw.rope_inv, q.desc.max_t);
            if (!q.kc || !q.vc || !q.cs) return nullptr;
            s->max_nh = std::max(s->max_nh, q.f.nh);
            s->max_t = std::max(s->max_t, q.desc.max_t);
        } else {
            fail(-1, "qwen stack: layer %d kind %d (0 GDN, 1 full attention)", l, q.desc.kind);
            return nullptr;
        }
        if (q.desc.ffn_kind == QFFN_DENSE) {
            q.dp = *(const M6DenseP*)q.desc.ffn;
            if (q.dp.h != QH) {
                fail(-1, "qwen stack: layer %d dense FFN width %d", l, q.dp.h);
                return nullptr;
            }
            q.FF = q.dp.n_ff;
            q.fg = get_mat(q.dp.g, q.dp.cg, q.FF, QH);
            q.fu = get_mat(q.dp.u, q.dp.cu, q.FF, QH);
            q.fd = get_mat(q.dp.d, q.dp.cd, QH, q.FF);
            if (!q.fg || !q.fu || !q.fd) return nullptr;
            s->max_ff = std::max(s->max_ff, q.FF);
        } else if (q.desc.ffn_kind == QFFN_MOE) {
            q.mp = *(const DracoMoeP*)q.desc.ffn;
            if (q.mp.n_in != QH || q.mp.n_out != QH) {
                fail(-1, "qwen stack: layer %d MoE width %d/%d", l, q.mp.n_in, q.mp.n_out);
                return nullptr;
            }
            q.moe = draco_moe_layer((const DracoMoeP*)q.desc.ffn);
            if (!q.moe) return nullptr;
        } else if (q.desc.ffn_kind != QFFN_NONE) {
            fail(-1, "qwen stack: layer %d FFN kind %d (0 none, 1 dense, 2 MoE)", l, q.desc.ffn_kind);
            return nullptr;
        }
    }
    const int nsplit = s->max_nh ? attn_nsplit(s->max_t, s->max_nh, FNKV, FHD) : 1;
    auto& k = s->allocs;
    if (qstack_alloc(k, &s->x, QH) || qstack_alloc(k, &s->x2n, QH) || qstack_alloc(k, &s->xn, QH) ||
        qstack_alloc(k, &s->xe, QH) || qstack_alloc(k, &s->qkv, std::max(s->max_qkv, 1)) ||
        qstack_alloc(k, &s->z, std::max(s->max_din, 1)) || qstack_alloc(k, &s->on, std::max(s->max_din, 1)) ||
        qstack_alloc(k, &s->QG, (size_t)std::max(s->max_nh, 1) * 2 * FHD) ||
        qstack_alloc(k, &s->Qr, (size_t)std::max(s->max_nh, 1) * FHD) ||
        qstack_alloc(k, &s->ao, (size_t)std::max(s->max_nh, 1) * FHD) || qstack_alloc(k, &s->kraw, FNKV * FHD) ||
        qstack_alloc(k, &s->vraw, FNKV * FHD) ||
        qstack_alloc(k, &s->part, (size_t)std::max(s->max_nh, 1) * nsplit * (FHD + 2)) ||
        qstack_alloc(k, &s->fg, std::max(s->max_ff, 1)) || qstack_alloc(k, &s->fu, std::max(s->max_ff, 1)) ||
        qstack_alloc(k, &s->pss, (size_t)std::max(s->max_vh, 1) * GDN_PSS_STRIDE) ||
        qstack_alloc(k, &s->xs, QH) || qstack_alloc(k, &s->pd, 2 * QH) ||
        qstack_alloc(k, &s->glog, 2 * (size_t)std::max(s->max_vh, 1)))
        return nullptr;
    if (hipMalloc(&s->state, sizeof(int) * 16) != hipSuccess) {
        s->state = nullptr;
        fail(-2, "qwen stack: state allocation failed");
        return nullptr;
    }
    k.push_back(s->state);
    if (hipHostMalloc(&s->hstate, sizeof(int) * 16, hipHostMallocDefault) != hipSuccess) {
        s->hstate = nullptr;
        fail(-2, "qwen stack: state allocation failed");
        return nullptr;
    }
    s->epoch = epoch();
    building.s = nullptr;
    slot = s;
    return s;
}

// prefill chunk buffers for up to cap tokens
int qstack_pf(QStack* s, int cap) {
    if (s->pf_cap >= cap) return 0;
    hipStreamSynchronize(stream());
    for (void* p : s->pf_allocs) hipFree(p);
    s->pf_allocs.clear();
    const size_t c = (size_t)cap;
    const int nh = std::max(s->max_nh, 1);
    auto& k = s->pf_allocs;
    const int win = std::max(std::max(QH, std::max(s->max_din, nh * FHD)), s->max_ff);
    const size_t nspl = pf_attn_nsplit(s->max_t, cap);
    if (qstack_alloc(k, &s->X, c * QH) || qstack_alloc(k, &s->Xn, c * QH) ||
        qstack_alloc(k, &s->QKV, c * std::max(s->max_qkv, 1)) || qstack_alloc(k, &s->Z, c * std::max(s->max_din, 1)) ||
        qstack_alloc(k, &s->B, c * std::max(s->max_vh, 1)) || qstack_alloc(k, &s->G, c * std::max(s->max_vh, 1)) ||
        qstack_alloc(k, &s->ON, c * std::max(s->max_din, 1)) || qstack_alloc(k, &s->Y, c * QH) ||
        qstack_alloc(k, &s->PQG, c * nh * 2 * FHD) || qstack_alloc(k, &s->PQr, c * nh * FHD) ||
        qstack_alloc(k, &s->PK, c * FNKV * FHD) || qstack_alloc(k, &s->PV, c * FNKV * FHD) ||
        qstack_alloc(k, &s->AO, c * nh * FHD) || qstack_alloc(k, &s->Ppart, pf_part_floats(nh, cap, FHD, nspl)) ||
        qstack_alloc(k, &s->PG, c * std::max(s->max_ff, 1)) || qstack_alloc(k, &s->PU, c * std::max(s->max_ff, 1)) ||
        qstack_alloc(k, &s->PPSS, c * std::max(s->max_vh, 1) * GDN_PSS_STRIDE))
        return -2;
    if (hipMalloc(&s->dig, draco_gemm_digit_bytes(cap, ((win + 255) / 256) * 256)) != hipSuccess ||
        hipMalloc(&s->ids, sizeof(int) * c) != hipSuccess)
        return fail(-2, "qwen stack: prefill allocation failed");
    k.push_back(s->dig);
    k.push_back(s->ids);
    s->pf_cap = cap;
    return 0;
}

// the FFN of one token: x += FFN(x2n), x2n = RMSNorm(x2_out) * post_norm
// formed by the FFN's own first launch (x holds x2_out): the MoE's norm
// launch, or the gate/up GEMV's RMSNorm prologue
int enqueue_qffn(QStack* s, QLayer& q, hipStream_t st) {
    if (q.desc.ffn_kind == QFFN_NONE) return 0;
    const float* pn = q.desc.kind == 0 ? q.g.post_norm : q.f.post_norm;
    if (q.desc.ffn_kind == QFFN_MOE) return draco_moe_layer_enqueue(q.moe, s->x, pn, QEPS, s->x, s->x, st);
    const Proj gu[2] = {{q.fg, s->fg, nullptr}, {q.fu, s->fu, nullptr}};
    if (int rc = enqueue_proj(gu, 2, s->x, QH, pn, s->xn, st)) return rc;
    dk_swiglu(s->fg, s->fu, q.FF, st);
    const Proj dn[1] = {{q.fd, s->x, s->x}};
    return enqueue_proj(dn, 1, s->fg, q.FF, nullptr, s->xn, st);
}

// Whether layer l's output projection runs split-K, leaving its residual add
// to layer l + 1's in-projection: a layer without FFN (its projection's
// output is the layer output) followed by a layer whose in-projection is all
// K-quants; GDN layers only on the gated-rms prologue path.
bool qks(const QStack* s, int l) {
    if (l + 1 >= s->n_layer) return false;
    const QLayer& q = s->L[l];
    if (q.desc.ffn_kind != QFFN_NONE) return false;
    auto kq = [](const DracoMat* m) { return m->L.code == DRACO_Q4_K || m->L.code == DRACO_Q6_K; };
    if (q.desc.kind == 0) {
        if (!ks_ok(q.g.out) || draco_gdn_split(true) <= 1) return false;
    } else if (!ks_ok(q.f.o)) {
        return false;
    }
    const QLayer& n = s->L[l + 1];
    if (n.desc.kind == 0) return kq(n.g.qkv) && kq(n.g.gate);
    return kq(n.f.q) && kq(n.f.k) && kq(n.f.v);
}

// one token through every layer: x (device) in place, or, with xin, layer 0
// reads its input from xin and every layer leaves its output in x; position
// and told from s->state ([pos, told], told = pos as the reference's driver
// passes them).  After a split-K output projection (qks) the layer output is
// pending: base + the partials in s->pd, which the next layer's in-projection
// forms into the other of s->x / s->xs (its input from then on).
int enqueue_qtoken(QStack* s, hipStream_t st, float* xin = nullptr) {
    float* base = s->x;   // the current layer's materialised input (or pending base)
    bool pending = false;
    for (int l = 0; l < s->n_layer; l++) {
        QLayer& q = s->L[l];
        float* x0 = (l == 0 && xin) ? xin : base;
        float* alt = base == s->x ? s->xs : s->x;  // where a pending sum is formed
        const bool ks = qks(s, l);
        float* in = pending ? alt : x0;  // this layer's input once formed
        if (q.desc.kind == 0) {
            GdnBufs b = {};
            b.h1 = x0;
            b.qkv = s->qkv;
            b.z = s->z;
            b.on = s->on;
            b.x2o = s->x;  // in place (or from the formed input): the ssm_out projection adds its residual row by row
            b.x2n = s->x2n;
            b.xn = s->xn;
            b.S = q.S;
            b.tail = q.tail;
            b.pss = s->pss;
            b.glog = s->glog;
            b.pend = pending ? s->pd : nullptr;
            b.pend_sum = pending ? alt : nullptr;
            b.ks_out = ks ? s->pd : nullptr;
            if (int rc = enqueue_gdn(q.g, b, st, false)) return rc;
        } else {
            const FullDev& f = q.f;
            const Proj in3[3] = {{f.q, s->QG, nullptr}, {f.k, s->kraw, nullptr}, {f.v, s->vraw, nullptr}};
            if (int rc = enqueue_proj(in3, 3, x0, QH, f.attn_norm, s->xn, st, nullptr, pending ? s->pd : nullptr,
                                      pending ? alt : nullptr))
                return rc;
            dk_fa_prep_rows(s->QG, f.nh * 2 * FHD, s->Qr, s->kraw, s->vraw, q.kc, q.vc, f.q_norm, f.k_norm, q.cs,
                            s->state, 0, 0, f.nh, 1, st);
            if (dk_attention(s->Qr, q.kc, q.vc, s->part, nullptr, s->ao, s->state, 0, f.nh, FNKV, FHD, q.desc.max_t,
                             1.f / sqrtf((float)FHD), st, s->QG + FHD, 2 * FHD))
                return fail(-1, "qwen stack: attention launch rejected");
            if (ks) {
                if (int rc = enqueue_proj_ks(f.o, s->ao, f.nh * FHD, s->pd, nullptr, st)) return rc;
            } else {
                const Proj out[1] = {{f.o, s->x, in}};
                if (int rc = enqueue_proj(out, 1, s->ao, f.nh * FHD, nullptr, s->xn, st)) return rc;
            }
        }
        if (ks) {
            // the layer output is in + the partials: the next layer forms it
            base = in;
            pending = true;
            continue;
        }
        base = s->x;
        pending = false;
        if (int rc = enqueue_qffn(s, q, st)) return rc;
    }
    return 0;
}

int qstack_positions(QStack* s, int pos0, int n) {
    if (pos0 < 0) return fail(-1, "qwen stack: negative position %d", pos0);
    for (int l = 0; l < s->n_layer; l++)
        if (s->L[l].desc.kind == 1 && pos0 + n > s->L[l].desc.max_t)
            return fail(-1, "qwen stack: layer %d: position %d + %d tokens exceeds max_t %d", l, pos0, n,
                        s->L[l].desc.max_t);
    return 0;
}

// T tokens whose hidden rows are in s->X (positions pos0 .. pos0 + T - 1)
// through every layer: the chunked form the reference runs in
// src/qwen35_prefill.py:209-239 (_gdn :110-135, _full :137-168), with the
// projections as f16-MFMA GEMMs over the chunk and the scan token-serial
int enqueue_qchunk(QStack* s, int T, int pos0, hipStream_t st) {
    auto kq = [](const DracoMat* m) { return m->L.code == DRACO_Q4_K || m->L.code == DRACO_Q6_K; };
    for (int l = 0; l < s->n_layer; l++) {
        QLayer& q = s->L[l];
        if (q.desc.kind == 0) {
            const GdnDev& g = q.g;
            if (pf_rms(s->X, g.attn_norm, s->Xn, T, QH, QEPS, st)) return fail(-1, "qwen prefill: rms rejected");
            if (draco_enqueue_gemm(*g.qkv, s->Xn, T, s->QKV, s->dig, false, st)) return -1;
            if (draco_enqueue_gemm(*g.gate, s->Xn, T, s->Z, s->dig, kq(g.qkv), st)) return -1;
            if (pf_gdn_gates(s->Xn, T, QH, g.bw, g.aw, g.ssm_dt, g.ssm_a, s->B, s->G, g.n_vh, st))
                return fail(-1, "qwen prefill: gates rejected");
            GdnArgs a = {};
            a.QKV = s->QKV;
            a.Z = s->Z;
            a.B = s->B;
            a.G = s->G;
            a.conv = g.conv;
            a.ssm_norm = g.ssm_norm;
            a.tail = q.tail;
            a.S = q.S;
            a.ON = s->ON;
            a.T = T;
            a.n_qkv = g.n_qkv;
            a.n_vh = g.n_vh;
            a.nhq = QNKH;
            a.nspl = T == 1 ? 1 : draco_gdn_split(false);
            a.PSS = s->PPSS;
            if (draco_gdn_scan_launch(a, st)) return fail(-1, "qwen prefill: scan rejected");
            if (draco_enqueue_gemm(*g.out, s->ON, T, s->Y, s->dig, false, st)) return -1;
            if (pf_add_rms(s->X, s->Y, g.post_norm, s->Xn, T, QH, QEPS, st)) return fail(-1, "qwen prefill: rms");
        } else {
            const FullDev& f = q.f;
            if (pf_rms(s->X, f.attn_norm, s->Xn, T, QH, QEPS, st)) return fail(-1, "qwen prefill: rms rejected");
            if (draco_enqueue_gemm(*f.q, s->Xn, T, s->PQG, s->dig, false, st)) return -1;
            if (draco_enqueue_gemm(*f.k, s->Xn, T, s->PK, s->dig, kq(f.q), st)) return -1;
            if (draco_enqueue_gemm(*f.v, s->Xn, T, s->PV, s->dig, kq(f.q) || kq(f.k), st)) return -1;
            dk_fa_prep_rows(s->PQG, f.nh * 2 * FHD, s->PQr, s->PK, s->PV, q.kc, q.vc, f.q_norm, f.k_norm, q.cs,
                            nullptr, pos0, pos0, f.nh, T, st);
            if (pf_attention256(s->PQr, q.kc, q.vc, s->Ppart, s->AO, pos0, T, f.nh, FNKV, 1.f / sqrtf((float)FHD),
                                s->PQG + FHD, f.nh * 2 * FHD, 2 * FHD, st))
                return fail(-1, "qwen prefill: attention rejected");
            if (draco_enqueue_gemm(*f.o, s->AO, T, s->Y, s->dig, false, st)) return -1;
            if (pf_add_rms(s->X, s->Y, f.post_norm, s->Xn, T, QH, QEPS, st)) return fail(-1, "qwen prefill: rms");
        }
        // FFN of the chunk (input Xn = x2n rows, residual into X)
        if (q.desc.ffn_kind == QFFN_DENSE) {
            if (draco_enqueue_gemm(*q.fg, s->Xn, T, s->PG, s->dig, false, st)) return -1;
            if (draco_enqueue_gemm(*q.fu, s->Xn, T, s->PU, s->dig, kq(q.fg), st)) return -1;
            dk_swiglu(s->PG, s->PU, T * q.FF, st);
            if (draco_enqueue_gemm(*q.fd, s->PG, T, s->Y, s->dig, false, st)) return -1;
            pf_add(s->X, s->Y, (size_t)T * QH, st);
        } else if (q.desc.ffn_kind == QFFN_MOE) {
            return fail(-1, "qwen prefill: MoE FFN layers are fed token by token");
        }
    }
    return 0;
}

bool qstack_has_moe(const QStack* s) {
    for (const QLayer& q : s->L)
        if (q.desc.ffn_kind == QFFN_MOE) return true;
    return false;
}

int g_qwen_chunk = 64;

// ids (device) [0, n) at positions pos0 .. through the chunked prefill;
// leaves the last token's hidden row in s->X row (returned T - 1)
int enqueue_qprefill(QStack* s, const DracoMat* em, const int* ids, int n, int pos0, hipStream_t st) {
    const int C = g_qwen_chunk;
    if (C < 1 || n < 1) return 0;
    if (qstack_pf(s, C)) return 0;
    int last = 0;
    for (int c0 = 0; c0 < n; c0 += C) {
        const int T = std::min(C, n - c0);
        if (pf_embed(em->dev, em->L, ids + c0, T, s->X, st)) return 0;
        if (enqueue_qchunk(s, T, pos0 + c0, st)) return 0;
        last = T;
    }
    return last;
}

}  // namespace

bool draco_gdn_state_current(const float* ssm, const float* tail, size_t ns, size_t nt, float** dS, float** dT) {
    *dS = *dT = nullptr;
    auto it = op_states().find(ssm);
    if (it == op_states().end()) return false;
    OpState& os = it->second;
    bool ok = os.samp.size() == QSAMP && ns >= QSAMP;
    for (int i = 0; ok && i < QSAMP; i++) ok = fbits(ssm[i]) == os.samp[i];
    bool fs = true, ft = true;
    float* s = ok ? (float*)get_mirror(ssm, sizeof(float) * ns, &fs) : nullptr;
    float* t = ok ? (float*)get_mirror(tail, sizeof(float) * nt, &ft) : nullptr;
    if (!s || !t || fs || ft || s != os.dev) {
        op_states().erase(it);
        return false;
    }
    *dS = s;
    *dT = t;
    return true;
}

void draco_gdn_state_written(const float* ssm, const float* dS) {
    OpState& os = op_states()[ssm];
    os.dev = dS;
    os.samp.resize(QSAMP);
    for (int i = 0; i < QSAMP; i++) os.samp[i] = fbits(ssm[i]);
}

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

// ---- the qwen35 hybrid stack (no reference counterpart as one call: the
// reference's driver composes the per-layer ops in Python,
// src/qwen35_engine.py:310-327 for a token, src/qwen35_prefill.py:209-239 for
// a chunk) ----

// One token through every layer (x[h] host, in / out: the X the reference's
// forward leaves before its head), at position pos (= the full-attention
// layers' Told, as the reference passes them).  Layer state stays on the
// device (draco_qwen_state_pull / push move it).
int draco_qwen_forward(float* x, int h, int pos, const void* layers, int n_layer) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = ensure_init()) return report(rc, "draco_qwen_forward");
    QStack* s = build_qstack((const QStackLayer*)layers, n_layer, h);
    if (!s) return report(-1, "draco_qwen_forward");
    if (int rc = qstack_positions(s, pos, 1)) return report(rc, "draco_qwen_forward");
    hipStream_t st = stream();
    s->hstate[0] = pos;
    s->hstate[1] = pos;
    if (hipMemcpyAsync(s->state, s->hstate, sizeof(int) * 2, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(s->x, x, sizeof(float) * QH, hipMemcpyHostToDevice, st) != hipSuccess)
        return report(fail(-2, "upload failed"), "draco_qwen_forward");
    if (int rc = enqueue_qtoken(s, st)) return report(rc, "draco_qwen_forward");
    if (hipMemcpyAsync(x, s->x, sizeof(float) * QH, hipMemcpyDeviceToHost, st) != hipSuccess)
        return report(fail(-2, "download failed"), "draco_qwen_forward");
    hipError_t e = hipStreamSynchronize(st);
    if (e != hipSuccess) return report(fail(-2, "draco_qwen_forward: %s", hipGetErrorString(e)), "draco_qwen_forward");
    return 0;
}

// The forward_chunk contract for the stack (src/qwen35_prefill.py:209-239):
// ids[0..n) at positions pos0 .. pos0 + n - 1 in chunks of the qwen chunk
// size; afterwards the state is that of n token-serial forwards.  out_x (h
// floats, host, nullable) = the last token's hidden row.
int draco_qwen_prefill(const void* layers, int n_layer, int h, const uint8_t* emb_w, int emb_code, int vocab,
                       const int* ids, int n, int pos0, float* out_x) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = ensure_init()) return report(rc, "draco_qwen_prefill");
    if (n < 1) return report(fail(-1, "need n >= 1"), "draco_qwen_prefill");
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= vocab) return report(fail(-1, "token id %d out of range", ids[i]), "draco_qwen_prefill");
    QStack* s = build_qstack((const QStackLayer*)layers, n_layer, h);
    if (!s) return report(-1, "draco_qwen_prefill");
    if (qstack_has_moe(s)) return report(fail(-1, "MoE FFN layers are fed token by token"), "draco_qwen_prefill");
    const DracoMat* em = get_mat(emb_w, emb_code, vocab, h);
    if (!em) return report(-1, "draco_qwen_prefill");
    if (int rc = qstack_positions(s, pos0, n)) return report(rc, "draco_qwen_prefill");
    hipStream_t st = stream();
    int* dids = (int*)scratch(5, sizeof(int) * ((size_t)n + 64));
    if (!dids) return report(-2, "draco_qwen_prefill");
    DRACO_HIP(hipMemcpyAsync(dids, ids, sizeof(int) * n, hipMemcpyHostToDevice, st));
    const int last = enqueue_qprefill(s, em, dids, n, pos0, st);
    if (last <= 0) return report(-1, "draco_qwen_prefill");
    if (out_x) DRACO_HIP(hipMemcpyAsync(out_x, s->X + (size_t)(last - 1) * QH, sizeof(float) * QH, hipMemcpyDeviceToHost, st));
    hipError_t e = hipStreamSynchronize(st);
    if (e != hipSuccess) return report(fail(-2, "draco_qwen_prefill: %s", hipGetErrorString(e)), "draco_qwen_prefill");
    return 0;
}

// Tokens per chunk of draco_qwen_prefill and of draco_qwen_generate's prompt
// (default 64, at most 256; 0 = the prompt goes token by token).  Returns the
// previous value; n < 0 only queries.
int draco_set_qwen_chunk(int n) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    const int old = g_qwen_chunk;
    if (n >= 0) g_qwen_chunk = n > QCHUNK_MAX ? QCHUNK_MAX : n;
    return old;
}

// Greedy generation on the device from position pos0: prompt[0..n_prompt-1)
// through the chunked prefill (token-serial decode steps when the chunk size
// is 0 or a layer has a MoE FFN), the last prompt token through the first
// decode step, then n_gen tokens by argmax (first index on ties).  With
// use_graph the token step is captured once and replayed.  out_hidden[h] = x
// after the last forward (nullable); stats[0] = decode ms, stats[1] = prefill
// ms (nullable).
int draco_qwen_generate(const void* layers, int n_layer, int h, float eps, const float* final_norm,
                        const uint8_t* head_w, int head_code, int vocab, const uint8_t* emb_w, int emb_code, int pos0,
                        const int* prompt, int n_prompt, int n_gen, int use_graph, int* out_tokens, float* out_hidden,
                        float* stats) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = ensure_init()) return report(rc, "draco_qwen_generate");
    if (n_prompt < 1 || n_gen < 1) return report(fail(-1, "need n_prompt >= 1 and n_gen >= 1"), "draco_qwen_generate");
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= vocab)
            return report(fail(-1, "prompt token id %d out of range", prompt[i]), "draco_qwen_generate");
    QStack* s = build_qstack((const QStackLayer*)layers, n_layer, h);
    if (!s) return report(-1, "draco_qwen_generate");
    const DracoMat* hm = get_mat(head_w, head_code, vocab, h);
    const DracoMat* em = get_mat(emb_w, emb_code, vocab, h);
    const float* nw = final_norm ? get_vec(final_norm, (size_t)h) : nullptr;
    if (!hm || !em || (final_norm && !nw)) return report(-1, "draco_qwen_generate");
    // get_mat / get_vec may have moved the epoch: the stack's cached pointers must be current
    s = build_qstack((const QStackLayer*)layers, n_layer, h);
    if (!s) return report(-1, "draco_qwen_generate");
    const int steps = n_prompt + n_gen - 1;
    if (int rc = qstack_positions(s, pos0, steps)) return report(rc, "draco_qwen_generate");
    hipStream_t st = stream();
    const int ntok = n_prompt + n_gen;
    int* dtok = (int*)scratch(5, sizeof(int) * (ntok + 64));
    const int hblocks = (vocab + 7) / 8;
    float* dred = (float*)scratch(7, (sizeof(float) + sizeof(int)) * ((size_t)hblocks + 64) + 256);
    float* dlog = (float*)scratch(6, sizeof(float) * (size_t)vocab);
    if (!dtok || !dred || !dlog) return report(-2, "draco_qwen_generate");
    int* cursor = dtok + ntok + 8;
    int* dri = (int*)(dred + hblocks + 32);
    const bool fused_head = hm->L.code == DRACO_Q4_K || hm->L.code == DRACO_Q5_K || hm->L.code == DRACO_Q6_K ||
                            hm->L.code == DRACO_Q8_0;
    const int n_chunked = (g_qwen_chunk > 0 && n_prompt - 1 >= 2 && !qstack_has_moe(s)) ? n_prompt - 1 : 0;
    if (n_chunked && qstack_pf(s, g_qwen_chunk)) return report(-2, "draco_qwen_generate (prefill buffers)");
    std::vector<int> ht(ntok + 64, 0);
    for (int i = 0; i < n_prompt; i++) ht[i] = prompt[i];
    ht[ntok + 8] = n_chunked;
    DRACO_HIP(hipMemcpyAsync(dtok, ht.data(), sizeof(int) * (ntok + 64), hipMemcpyHostToDevice, st));
    auto step = [&](bool decode) -> int {
        const bool emb_ready = decode && fused_head;
        if (!emb_ready) dk_embed(*em, dtok, cursor, s->x, st);
        if (int rc = enqueue_qtoken(s, st, emb_ready ? s->xe : nullptr)) return rc;
        if (!decode) {
            dk_advance(s->state, 1, cursor, st);
            return 0;
        }
        if (fused_head) {
            SegLaunch sl = {};
            sl.nseg = 1;
            sl.n_in = h;
            sl.x = s->x;
            sl.do_norm = 1;
            sl.norm_w = nw;
            sl.eps = eps;
            SegDesc d = {};
            d.base = hm->dev;
            d.L = hm->L;
            d.epi = EPI_ARGMAX;
            d.y = dlog;
            sl.seg[0] = d;
            sl.am_val = dred;
            sl.am_idx = dri;
            sl.tokens = dtok;
            sl.cursor = cursor;
            sl.advance_state = s->state;
            sl.advance_layers = 1;
            sl.emb = em->dev;
            sl.emb_L = em->L;
            sl.emb_out = s->xe;
            if (draco_seg_launch(sl, st)) return fail(-1, "head launch rejected");
            return 0;
        }
        dk_rmsnorm(s->x, nw, s->xn, h, eps, st);
        if (draco_gemv_launch(*hm, s->xn, dlog, nullptr, 0, vocab, st)) return fail(-1, "head gemv");
        dk_argmax(dlog, vocab, dred, dri, dtok, cursor, 0, st);
        dk_advance(s->state, 1, cursor, st);
        return 0;
    };
    struct Guard {
        hipStream_t st;
        hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
        hipGraphExec_t gx[2] = {nullptr, nullptr};
        hipGraph_t gg[2] = {nullptr, nullptr};
        ~Guard() {
            hipStreamSynchronize(st);
            for (int k = 0; k < 2; k++) {
                if (gx[k]) hipGraphExecDestroy(gx[k]);
                if (gg[k]) hipGraphDestroy(gg[k]);
            }
            for (hipEvent_t e : ev)
                if (e) hipEventDestroy(e);
        }
    } G{st};
    for (hipEvent_t& e : G.ev) DRACO_HIP(hipEventCreate(&e));
    if (use_graph) {
        for (int k = 0; k < 2; k++) {
            if (k == 0 && n_chunked == n_prompt - 1) continue;  // no token-serial prompt step to capture
            DRACO_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
            const int rc = step(k == 1);
            hipGraph_t gr = nullptr;
            const hipError_t ce = hipStreamEndCapture(st, &gr);
            G.gg[k] = gr;
            if (rc) return report(rc, "draco_qwen_generate");
            if (ce != hipSuccess) return report(fail(-2, "graph capture: %s", hipGetErrorString(ce)), "draco_qwen_generate");
            DRACO_HIP(hipGraphInstantiate(&G.gx[k], gr, nullptr, nullptr, 0));
        }
    }
    DRACO_HIP(hipEventRecord(G.ev[0], st));
    if (n_chunked && enqueue_qprefill(s, em, dtok, n_chunked, pos0, st) <= 0)
        return report(-1, "draco_qwen_generate (chunked prefill)");
    s->hstate[0] = pos0 + n_chunked;
    s->hstate[1] = pos0 + n_chunked;
    DRACO_HIP(hipMemcpyAsync(s->state, s->hstate, sizeof(int) * 2, hipMemcpyHostToDevice, st));
    for (int i = n_chunked; i < n_prompt - 1; i++) {
        if (use_graph) DRACO_HIP(hipGraphLaunch(G.gx[0], st));
        else if (int rc = step(false)) return report(rc, "draco_qwen_generate");
    }
    if (fused_head) dk_embed(*em, dtok, cursor, s->xe, st);
    DRACO_HIP(hipEventRecord(G.ev[1], st));
    for (int i = 0; i < n_gen; i++) {
        if (use_graph) DRACO_HIP(hipGraphLaunch(G.gx[1], st));
        else if (int rc = step(true)) return report(rc, "draco_qwen_generate");
    }
    DRACO_HIP(hipEventRecord(G.ev[2], st));
    DRACO_HIP(hipMemcpyAsync(ht.data(), dtok, sizeof(int) * ntok, hipMemcpyDeviceToHost, st));
    if (out_hidden) DRACO_HIP(hipMemcpyAsync(out_hidden, s->x, sizeof(float) * h, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipStreamSynchronize(st));
    float ms_pre = 0.f, ms_dec = 0.f;
    hipEventElapsedTime(&ms_pre, G.ev[0], G.ev[1]);
    hipEventElapsedTime(&ms_dec, G.ev[1], G.ev[2]);
    if (stats) {
        stats[0] = ms_dec;
        stats[1] = ms_pre;
    }
    for (int i = 0; i < n_gen; i++) out_tokens[i] = ht[n_prompt + i];
    return 0;
}

// One state array's device mirror -> the caller's array (its first `bytes`):
// a GDN ssm or tail, or the leading rows of a full-attention Kr / Vc, as the
// per-layer ops left them.
int draco_array_pull(void* host, size_t bytes) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    return mirror_pull(host, bytes);
}

// The caller's array (its first `bytes`) -> its device mirror, e.g. after
// restoring a snapshot into it; the per-layer ops re-read it on their next
// call.
int draco_array_push(const void* host, size_t bytes) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = ensure_init()) return rc;
    op_states().erase(host);
    return mirror_push(host, bytes);
}

// Device state of every layer -> the caller's arrays (GDN ssm and tail in
// full; full-attention Kr / Vc rows [0, rows)), e.g. before a snapshot.
int draco_qwen_state_pull(const void* layers_v, int n_layer, int rows) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    const QStackLayer* layers = (const QStackLayer*)layers_v;
    for (int l = 0; l < n_layer; l++) {
        const QStackLayer& d = layers[l];
        if (d.kind == 0) {
            const GdnW* w = (const GdnW*)d.w;
            if (int rc = mirror_pull(d.state0, sizeof(float) * (size_t)w->n_vh * QSV * QSV)) return rc;
            if (int rc = mirror_pull(d.state1, sizeof(float) * (size_t)w->n_qkv * 3)) return rc;
        } else if (rows > 0) {
            const size_t b = sizeof(float) * full_cache_floats(std::min(rows, d.max_t));
            if (int rc = mirror_pull(d.state0, b)) return rc;
            if (int rc = mirror_pull(d.state1, b)) return rc;
        }
    }
    return 0;
}

// The caller's arrays -> device state of every layer (after a reset that
// zeroed them, or a restored snapshot): GDN ssm and tail in full,
// full-attention rows [0, rows).
int draco_qwen_state_push(const void* layers_v, int n_layer, int rows) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = ensure_init()) return rc;
    const QStackLayer* layers = (const QStackLayer*)layers_v;
    for (int l = 0; l < n_layer; l++) {
        const QStackLayer& d = layers[l];
        if (d.kind == 0) {
            const GdnW* w = (const GdnW*)d.w;
            if (int rc = mirror_push(d.state0, sizeof(float) * (size_t)w->n_vh * QSV * QSV)) return rc;
            if (int rc = mirror_push(d.state1, sizeof(float) * (size_t)w->n_qkv * 3)) return rc;
        } else if (rows > 0) {
            const size_t b = sizeof(float) * full_cache_floats(std::min(rows, d.max_t));
            if (int rc = mirror_push(d.state0, b)) return rc;
            if (int rc = mirror_push(d.state1, b)) return rc;
        }
    }
    return 0;
}

}  // extern "C"
