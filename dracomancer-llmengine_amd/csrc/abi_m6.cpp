// abi_m6.cpp -- the layer-engine ABI (drop-in for m6_engine.so's llama path).
//
// Reference: src/m6_engine.c:18-83 (descriptors, m6_forward_token),
// :270-303 (M6DenseP, m6_dense_op), :373-391 (m6_head_op), :396-517
// (M6LlamaAttnP, llama_attn_core, m6_llama_attn_op).  Struct layouts are the
// reference's, field for field: Python callers allocate them through ctypes
// (src/smol_engine.py:97-115).
//
// m6_forward_token recognises descriptors whose op pointers are this
// library's own m6_llama_attn_op / m6_dense_op (Python takes them from the
// same .so, src/smol_engine.py:117-118) and runs the whole token on the
// device: weights resident (registry keyed by host address), KV caches as
// device mirrors of the caller's kcache/vcache arrays, one host->device copy
// of x in and one copy out.  The caller's tlen counters advance exactly as
// the reference's do (src/m6_engine.c:510).
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <unordered_map>
#include <vector>

#include "decode.h"
#include "gemm.h"
#include "moe.h"
#include "prefill.h"
#include "runtime.h"

extern "C" {
typedef void (*m6_attn_op)(const float* xn, void* p, int pos, float* out);
typedef void (*m6_ffn_op)(const float* xn, void* p, float* out);

typedef struct {
    const float* attn_norm;
    const float* ffn_norm;
    m6_attn_op attn;
    void* attn_p;
    m6_ffn_op ffn;
    void* ffn_p;
} M6LayerDesc;

typedef struct {
    const uint8_t *wq, *wk, *wv, *wo;
    int cq, ck, cv, co;
    int n_head, n_kv, head_dim, hidden, rot;
    float rope_base;
    float* kcache;
    float* vcache;
    int* tlen;
    int max_t;
    float* work;
} M6LlamaAttnP;

typedef struct {
    const uint8_t *g, *u, *d;
    int cg, cu, cd, n_ff, h;
} M6DenseP;

void m6_llama_attn_op(const float* xn, void* p, int pos, float* out);
void m6_dense_op(const float* xn, void* p, float* out);
void draco_moe_ffn_op(const float* xn, void* p, float* out);  // abi_moe.cpp
}

using namespace draco;

namespace {

struct DevAttn {
    uint64_t epoch = 0;
    M6LlamaAttnP snap;
    const DracoMat *wq, *wk, *wv, *wo;
    float *kc, *vc;
    int NH, NKV, HD, H, rot, max_t;
    float base, scale;
};

struct DevFfn {
    uint64_t epoch = 0;
    M6DenseP snap;
    const DracoMat *g, *u, *d;
    int FF, H;
};

struct Work {
    float *x = nullptr, *xn = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr,
          *part = nullptr, *g = nullptr, *u = nullptr;
    float* xe = nullptr;      // next token's embedding, written by the head's argmax (generation)
    // a pending residual after a split-K down projection: the layer output is
    // x + pd[0..H) + pd[H..2H), materialised into xs by the next q/k/v launch
    float *pd = nullptr, *xs = nullptr;
    // a MoE layer after a split-K o projection: its input (the layer input +
    // the partials in pd), materialised by the router launch
    float* xm = nullptr;
    unsigned* cnt = nullptr;  // attention merge counters (one per kv head), zero at rest
    size_t cap_h = 0, cap_xn = 0, cap_xe = 0, cap_q = 0, cap_k = 0, cap_part = 0, cap_ff = 0, cap_pd = 0,
           cap_xs = 0, cap_xm = 0;
};

// Chunked-prefill buffers, token-major, for up to `cap` tokens per chunk.
struct PfBufs {
    float *X = nullptr, *Xn = nullptr, *Q = nullptr, *K = nullptr, *V = nullptr, *O = nullptr, *G = nullptr,
          *U = nullptr, *Y = nullptr, *part = nullptr;
    uint8_t* dig = nullptr;
    int* ids = nullptr;
    int cap = 0, H = 0, QD = 0, KD = 0, FF = 0;
    size_t part_n = 0, dig_n = 0;
};

struct DevModel {
    uint64_t epoch = 0;
    PfBufs pf;
    std::vector<M6LayerDesc> descs;
    std::vector<DevAttn*> attn;
    std::vector<DevFfn*> ffn;          // dense FFN layers (m6_dense_op), else null
    std::vector<MoeLayer*> moe;        // MoE FFN layers (draco_moe_ffn_op), else null
    std::vector<DracoMoeP> moe_snap;   // their parameter structs when built
    std::vector<const float*> anorm, fnorm;
    int h = 0, n_layer = 0;
    Work w;
    int* state = nullptr;   // device [1 + n_layer]
    int* hstate = nullptr;  // pinned host mirror of state
    int state_cap = 0;      // ints allocated in state / hstate
    // layers whose attention merge rides on the o projection (fused_o), each
    // with the previous such layer (cyclically: the accumulator it clears),
    // and their int64 accumulators ([n_layer][oacc_stride])
    std::vector<char> fo;
    std::vector<int> fo_prev;
    unsigned long long* oacc = nullptr;
    size_t oacc_stride = 0, oacc_n = 0;
    // the longest cache (rows) a layer reaches in the current call
    int call_rows = 0;
};

struct RopeTab {
    float* dev = nullptr;
    int cap = 0;
};

std::unordered_map<const void*, DevAttn*>& attn_cache() {
    static auto* m = new std::unordered_map<const void*, DevAttn*>();
    return *m;
}
std::unordered_map<const void*, DevFfn*>& ffn_cache() {
    static auto* m = new std::unordered_map<const void*, DevFfn*>();
    return *m;
}
std::unordered_map<const void*, DevModel*>& model_cache() {
    static auto* m = new std::unordered_map<const void*, DevModel*>();
    return *m;
}
std::map<std::pair<int, float>, RopeTab>& rope_cache() {
    static auto* m = new std::map<std::pair<int, float>, RopeTab>();
    return *m;
}
extern "C" void draco_rope_table(int max_t, int rot, float base, float* tab);

int report(int rc, const char* where) {
    fprintf(stderr, "[draco_hip] %s failed (rc=%d): %s\n", where, rc, last_error());
    return rc;
}

// device copy of a norm weight vector: registered like any fp32 parameter
// array (get_vec), so a different array at a recycled host address, or one of
// a different length, is re-uploaded rather than served from the old copy
const float* norm_dev(const float* host, int h) {
    if (!host) return nullptr;
    return get_vec(host, (size_t)h);
}

// rope angle table covering positions [0, need)
const float* rope_dev(int rot, float base, int need) {
    RopeTab& t = rope_cache()[{rot, base}];
    if (t.cap >= need) return t.dev;
    int cap = need < 1024 ? 1024 : need;
    std::vector<float> h((size_t)cap * rot);
    draco_rope_table(cap, rot, base, h.data());
    if (t.dev) {
        hipStreamSynchronize(stream());
        hipFree(t.dev);
    }
    if (hipMalloc(&t.dev, sizeof(float) * h.size()) != hipSuccess) {
        t = RopeTab();
        fail(-2, "hipMalloc rope table failed");
        return nullptr;
    }
    if (hipMemcpy(t.dev, h.data(), sizeof(float) * h.size(), hipMemcpyHostToDevice) != hipSuccess) {
        fail(-2, "rope table upload failed");
        return nullptr;
    }
    t.cap = cap;
    return t.dev;
}

DevAttn* get_attn(const M6LlamaAttnP* p) {
    auto& c = attn_cache();
    auto it = c.find(p);
    if (it != c.end() && it->second->epoch == epoch() && memcmp(&it->second->snap, p, sizeof(*p)) == 0)
        return it->second;
    const int NH = p->n_head, NKV = p->n_kv, HD = p->head_dim, H = p->hidden;
    // src/m6_engine.c:425-511 takes any GQA ratio and head dim; the device
    // attention serves every even head dim up to 512 (decode.h)
    if (NH <= 0 || NKV <= 0 || NH % NKV || HD < 2 || HD > 512 || (HD & 1) || p->rot < 0 || p->rot > HD ||
        (p->rot & 1) || p->max_t <= 0) {
        fail(-1, "m6_llama_attn_op: unsupported shape NH=%d NKV=%d HD=%d rot=%d", NH, NKV, HD, p->rot);
        return nullptr;
    }
    DevAttn* a = (it != c.end()) ? it->second : new DevAttn();
    a->snap = *p;
    a->NH = NH; a->NKV = NKV; a->HD = HD; a->H = H; a->rot = p->rot; a->max_t = p->max_t;
    a->base = p->rope_base;
    a->scale = 1.0f / sqrtf((float)HD);
    const int QD = NH * HD, KD = NKV * HD;
    a->wq = get_mat(p->wq, p->cq, QD, H);
    a->wk = get_mat(p->wk, p->ck, KD, H);
    a->wv = get_mat(p->wv, p->cv, KD, H);
    a->wo = get_mat(p->wo, p->co, H, QD);
    if (!a->wq || !a->wk || !a->wv || !a->wo) return nullptr;
    const size_t kvb = sizeof(float) * (size_t)p->max_t * KD;
    bool fk = false, fv = false;
    a->kc = (float*)get_mirror(p->kcache, kvb, &fk);
    a->vc = (float*)get_mirror(p->vcache, kvb, &fv);
    if (!a->kc || !a->vc) return nullptr;
    const int T = p->tlen ? *p->tlen : 0;
    if ((fk || fv) && T > 0) {  // state the caller already holds (CPU prefill, restored snapshot)
        const size_t b = sizeof(float) * (size_t)T * KD;
        if (hipMemcpy(a->kc, p->kcache, b, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(a->vc, p->vcache, b, hipMemcpyHostToDevice) != hipSuccess) {
            fail(-2, "KV mirror upload failed");
            return nullptr;
        }
    }
    if (!rope_dev(a->rot, a->base, a->max_t)) return nullptr;
    a->epoch = epoch();
    c[p] = a;
    return a;
}

DevFfn* get_ffn(const M6DenseP* p) {
    auto& c = ffn_cache();
    auto it = c.find(p);
    if (it != c.end() && it->second->epoch == epoch() && memcmp(&it->second->snap, p, sizeof(*p)) == 0)
        return it->second;
    DevFfn* f = (it != c.end()) ? it->second : new DevFfn();
    f->snap = *p;
    f->FF = p->n_ff;
    f->H = p->h;
    f->g = get_mat(p->g, p->cg, p->n_ff, p->h);
    f->u = get_mat(p->u, p->cu, p->n_ff, p->h);
    f->d = get_mat(p->d, p->cd, p->h, p->n_ff);
    if (!f->g || !f->u || !f->d) return nullptr;
    f->epoch = epoch();
    c[p] = f;
    return f;
}

int grow(float** p, size_t* cap, size_t n) {
    if (*cap >= n) return 0;
    if (*p) {
        hipStreamSynchronize(stream());
        hipFree(*p);
    }
    DRACO_HIP(hipMalloc(p, sizeof(float) * n));
    *cap = n;
    return 0;
}

int ensure_work(Work& w, int H, int QD, int KD, int NH, int HD, int max_t, int FF) {
    const size_t part = (size_t)NH * attn_nsplit(max_t, NH, KD / HD, HD) * (HD + 2);
    if (!w.cnt) {
        DRACO_HIP(hipMalloc(&w.cnt, sizeof(unsigned) * 256));
        DRACO_HIP(hipMemset(w.cnt, 0, sizeof(unsigned) * 256));
        DRACO_HIP(hipDeviceSynchronize());
    }
    if (grow(&w.x, &w.cap_h, H + 64)) return -2;
    if (grow(&w.xn, &w.cap_xn, H + 64)) return -2;
    if (grow(&w.xe, &w.cap_xe, H + 64)) return -2;
    if (grow(&w.pd, &w.cap_pd, 2 * (size_t)H + 64)) return -2;
    if (grow(&w.xs, &w.cap_xs, H + 64)) return -2;
    if (grow(&w.xm, &w.cap_xm, H + 64)) return -2;
    if (w.cap_q < (size_t)QD) {
        size_t c = w.cap_q;
        if (grow(&w.q, &c, QD)) return -2;
        size_t c2 = w.cap_q;
        if (grow(&w.att, &c2, QD)) return -2;
        w.cap_q = QD;
    }
    if (w.cap_k < (size_t)KD) {
        size_t c = w.cap_k;
        if (grow(&w.k, &c, KD)) return -2;
        size_t c2 = w.cap_k;
        if (grow(&w.v, &c2, KD)) return -2;
        w.cap_k = KD;
    }
    if (grow(&w.part, &w.cap_part, part)) return -2;
    if (w.cap_ff < (size_t)FF) {
        size_t c = w.cap_ff;
        if (grow(&w.g, &c, FF)) return -2;
        size_t c2 = w.cap_ff;
        if (grow(&w.u, &c2, FF)) return -2;
        w.cap_ff = FF;
    }
    return 0;
}

DevModel* build_model(const M6LayerDesc* layers, int n_layer, int h);

DevModel* resolve_model(const M6LayerDesc* layers, int n_layer, int h) {
    // building may evict (a replaced weight bumps the epoch): retry until a
    // build completes within one epoch
    for (int tries = 0; tries < 3; tries++) {
        const uint64_t e0 = epoch();
        DevModel* m = build_model(layers, n_layer, h);
        if (!m || m->epoch == epoch()) return m;
        (void)e0;
    }
    fail(-2, "model residency kept changing while building");
    return nullptr;
}

DevModel* build_model(const M6LayerDesc* layers, int n_layer, int h) {
    auto& c = model_cache();
    auto it = c.find(layers);
    if (it != c.end()) {
        DevModel* m = it->second;
        bool ok = m->epoch == epoch() && m->n_layer == n_layer && m->h == h &&
                  memcmp(m->descs.data(), layers, sizeof(M6LayerDesc) * n_layer) == 0;
        for (int l = 0; ok && l < n_layer; l++) {
            ok = memcmp(&m->attn[l]->snap, layers[l].attn_p, sizeof(M6LlamaAttnP)) == 0 &&
                 attn_cache().count(layers[l].attn_p) && attn_cache().at(layers[l].attn_p) == m->attn[l];
            if (ok && m->moe[l])  // MoE layer: the op's parameter struct unchanged, its experts current
                ok = memcmp(&m->moe_snap[l], layers[l].ffn_p, sizeof(DracoMoeP)) == 0 &&
                     draco_moe_layer((const DracoMoeP*)layers[l].ffn_p) == m->moe[l];
            else if (ok)
                ok = memcmp(&m->ffn[l]->snap, layers[l].ffn_p, sizeof(M6DenseP)) == 0 &&
                     ffn_cache().count(layers[l].ffn_p) && ffn_cache().at(layers[l].ffn_p) == m->ffn[l];
        }
        if (ok && m->epoch == epoch()) return m;
    }
    DevModel* m = (it != c.end()) ? it->second : new DevModel();
    m->descs.assign(layers, layers + n_layer);
    m->attn.assign(n_layer, nullptr);
    m->ffn.assign(n_layer, nullptr);
    m->moe.assign(n_layer, nullptr);
    m->moe_snap.assign(n_layer, DracoMoeP{});
    m->anorm.assign(n_layer, nullptr);
    m->fnorm.assign(n_layer, nullptr);
    m->h = h;
    m->n_layer = n_layer;
    for (int l = 0; l < n_layer; l++) {
        const M6LayerDesc& L = layers[l];
        const bool dense = (void*)L.ffn == (void*)&m6_dense_op;
        const bool moe = (void*)L.ffn == (void*)&draco_moe_ffn_op;
        if ((void*)L.attn != (void*)&m6_llama_attn_op || (!dense && !moe)) {
            fail(-1, "m6_forward_token: layer %d uses an op not served by this library", l);
            return nullptr;
        }
        DevAttn* a = get_attn((const M6LlamaAttnP*)L.attn_p);
        if (!a) return nullptr;
        int FF = 1;
        if (dense) {
            DevFfn* f = get_ffn((const M6DenseP*)L.ffn_p);
            if (!f) return nullptr;
            if (f->H != h) {
                fail(-1, "m6_forward_token: layer %d hidden size mismatch", l);
                return nullptr;
            }
            m->ffn[l] = f;
            FF = f->FF;
        } else {
            const DracoMoeP* mp = (const DracoMoeP*)L.ffn_p;
            if (mp->n_in != h || mp->n_out != h) {
                fail(-1, "m6_forward_token: layer %d MoE width %d/%d != hidden %d", l, mp->n_in, mp->n_out, h);
                return nullptr;
            }
            m->moe[l] = draco_moe_layer(mp);
            if (!m->moe[l]) return nullptr;
            m->moe_snap[l] = *mp;
        }
        if (a->H != h) {
            fail(-1, "m6_forward_token: layer %d hidden size mismatch", l);
            return nullptr;
        }
        m->attn[l] = a;
        m->anorm[l] = norm_dev(L.attn_norm, h);
        m->fnorm[l] = norm_dev(L.ffn_norm, h);
        if ((L.attn_norm && !m->anorm[l]) || (L.ffn_norm && !m->fnorm[l])) return nullptr;
        if (ensure_work(m->w, h, a->NH * a->HD, a->NKV * a->HD, a->NH, a->HD, a->max_t, FF)) return nullptr;
    }
    m->epoch = epoch();
    // [pos, tlen of each layer]; a later model at the same descriptor address
    // may have more layers, so the buffers grow with n_layer
    if (m->state_cap < 1 + n_layer + 8) {
        if (m->state) {
            hipStreamSynchronize(stream());
            hipFree(m->state);
            hipHostFree(m->hstate);
            m->state = nullptr;
            m->hstate = nullptr;
            m->state_cap = 0;
        }
        const int cap = 1 + n_layer + 8;
        if (hipMalloc(&m->state, sizeof(int) * cap) != hipSuccess ||
            hipHostMalloc(&m->hstate, sizeof(int) * cap, hipHostMallocDefault) != hipSuccess) {
            fail(-2, "state allocation failed");
            return nullptr;
        }
        m->state_cap = cap;
    }
    c[layers] = m;
    return m;
}

SegDesc seg_of(const DracoMat* m, int epi, float* y, const float* yadd) {
    SegDesc d = {};
    d.base = m->dev;
    d.L = m->L;
    d.epi = epi;
    d.y = y;
    d.yadd = yadd;
    return d;
}

// q/k/v projections of one attention op from input x (RMS-normalised in the
// prologue when norm != 0), with rope on q/k and the KV append at row T as
// epilogues (src/m6_engine.c:447-481).
int enqueue_qkv(DevAttn* a, Work& w, const float* x, int norm, const float* norm_w, float eps,
                const int* state, int layer, hipStream_t st, bool pending = false) {
    const SegDesc all[3] = {seg_of(a->wq, EPI_ROPE_Q, w.q, nullptr), seg_of(a->wk, EPI_ROPE_K, nullptr, nullptr),
                            seg_of(a->wv, EPI_V_APPEND, nullptr, nullptr)};
    bool done[3] = {false, false, false};
    for (int i = 0; i < 3; i++) {
        if (done[i]) continue;
        SegLaunch s = {};
        s.n_in = a->H;
        s.x = x;
        s.do_norm = norm;
        s.norm_w = norm_w;
        s.eps = eps;
        if (pending) {  // x + the split-K partials, normalised; the sum kept in w.xs
            s.do_norm = 3;
            s.am_val = w.pd;
            s.xn_out = w.xs;
        }
        // every not-yet-issued segment of the same kernel family (Q4_K/Q6_K
        // share one; Q5_K launches hold Q5_K segments only)
        auto fam = [](int c) { return c == DRACO_Q8_0 ? 0 : (c == DRACO_Q5_K ? 2 : 1); };
        for (int j = i; j < 3; j++)
            if (!done[j] && fam(all[j].L.code) == fam(all[i].L.code)) {
                s.seg[s.nseg++] = all[j];
                done[j] = true;
            }
        s.rope_tab = rope_cache()[{a->rot, a->base}].dev;
        s.state = state;
        s.layer = layer;
        s.head_dim = a->HD;
        s.rot = a->rot;
        s.kv_dim = a->NKV * a->HD;
        s.kc = a->kc;
        s.vc = a->vc;
        if (draco_seg_launch(s, st)) return fail(-1, "qkv launch rejected");
    }
    return 0;
}

// gate/up + SwiGLU into w.g (src/m6_engine.c:289-302), input normalised in the
// prologue when norm != 0
// With pend (a pending residual: the input is x + pend[0..H) + pend[H..2H),
// the o projection's split-K partials) the gate/up launch forms the input in
// its RMSNorm prologue and stores it to pend_sum (one launch, same formats).
int enqueue_gateup(DevFfn* f, Work& w, const float* x, int norm, const float* norm_w, float eps,
                   hipStream_t st, const float* pend = nullptr, float* pend_sum = nullptr, int npend = 2) {
    if (pend && (f->g->L.code != f->u->L.code || !norm || !pend_sum))
        return fail(-1, "gate/up: a pending residual needs one launch with the RMSNorm prologue");
    if (f->g->L.code == f->u->L.code) {
        SegLaunch s = {};
        s.nseg = 2;
        s.n_in = f->H;
        s.x = x;
        s.do_norm = pend ? (npend == 8 ? 4 : 3) : norm;
        s.norm_w = norm_w;
        s.eps = eps;
        if (pend) {
            s.am_val = const_cast<float*>(pend);
            s.xn_out = pend_sum;
        }
        s.seg[0] = seg_of(f->g, EPI_SWIGLU, w.g, nullptr);
        s.seg[1] = seg_of(f->u, EPI_STORE, nullptr, nullptr);
        if (draco_seg_launch(s, st)) return fail(-1, "gate/up launch rejected");
        return 0;
    }
    // mixed formats: two launches + the elementwise SwiGLU
    const float* xin = x;
    if (norm) {
        dk_rmsnorm(x, norm_w, w.xn, f->H, eps, st);
        xin = w.xn;
    }
    if (draco_gemv_launch(*f->g, xin, w.g, nullptr, 0, f->FF, st)) return fail(-1, "gemv gate");
    if (draco_gemv_launch(*f->u, xin, w.u, nullptr, 0, f->FF, st)) return fail(-1, "gemv up");
    dk_swiglu(w.g, w.u, f->FF, st);
    return 0;
}

// The shared expert after its gate/up (activation in w.g, input in w.xn):
// down product into w.x, then w.q = w.x * sigmoid(gate row . x) with the gate
// logit in w.k[0].  An F32 / F16 gate row is dotted inside the scaling
// kernel; any other format takes a one-row GEMV first.
int enqueue_shexp_tail(const DracoMat& gi, const DracoMat& down, Work& w, int h, hipStream_t st) {
    if (draco_gemv_launch(down, w.g, w.x, nullptr, 0, h, st)) return -1;
    if (gi.L.code == DRACO_F32 || gi.L.code == DRACO_F16) return dk_gate_scale(w.xn, gi, w.x, w.q, w.k, h, st);
    if (draco_gemv_launch(gi, w.xn, w.k, nullptr, 0, 1, st)) return -1;
    dk_sigmoid_scale(w.x, w.k, w.q, h, st);
    return 0;
}

// Whether layer l's dense down projection runs split-K, leaving its residual
// add to the next layer's q/k/v launch: a short wide matrix (half the CUs or
// fewer with one tile each, 16 or 32 super-blocks per row) followed by a
// layer whose q/k/v are all K-quants (the launch that takes the pending sum).
// A 2048x8192 Q6_K GEMV takes 5.73 us, the same bytes as 4096x4096 4.59 us.
bool ksplit_down(const DevModel* m, int l) {
    if (l + 1 >= m->n_layer || !m->ffn[l] || m->moe[l]) return false;
    const DracoMat& d = *m->ffn[l]->d;
    const int nb = d.L.n_in / 256;
    if ((d.L.code != DRACO_Q4_K && d.L.code != DRACO_Q6_K) || d.L.n_in % 256 || (nb != 16 && nb != 32) ||
        !draco_dq_ksplit_waves(d.L.n_in, 0) || (d.L.n_out + 15) / 16 > 128)
        return false;
    const DevAttn* n = m->attn[l + 1];
    auto kq = [](const DracoMat* x) { return x->L.code == DRACO_Q4_K || x->L.code == DRACO_Q6_K; };
    return kq(n->wq) && kq(n->wk) && kq(n->wv);
}

// Whether layer l's o projection runs split-K, leaving its residual add to
// the MoE router launch (k_moe_logits with a pending residual): a MoE layer
// whose router takes the RMSNorm prologue and an o projection of 16 or 32
// super-blocks per row and at most 128 tiles (configs[3]: 2048x4096 Q6_K).
bool ksplit_o(const DevModel* m, int l) {
    if (!m->moe[l] || !draco_moe_layer_pend_ok(m->moe[l], m->fnorm[l])) return false;
    const DracoMat& o = *m->attn[l]->wo;
    const int nb = o.L.n_in / 256;
    return (o.L.code == DRACO_Q4_K || o.L.code == DRACO_Q6_K) && o.L.n_in % 256 == 0 && (nb == 16 || nb == 32) &&
           draco_dq_ksplit_waves(o.L.n_in, 0) && (o.L.n_out + 15) / 16 <= 128;
}

// Whether dense layer l's o projection runs split-K, leaving its residual
// add to the gate/up launch (which forms the input plus the partials in its
// RMSNorm prologue and stores it to w.xm): an o projection whose rows a
// split-K instance covers (draco_dq_ksplit_waves: 8, 16 or 32 super-blocks)
// and at most 128 tiles, and a gate/up pair of one K-quant format
// (configs[2]: 2048x2048 Q4_K, the 4-wave split-K launch).
bool ksplit_o_dense(const DevModel* m, int l) {
    const DevFfn* f = m->ffn[l];
    if (!f || m->moe[l] || f->g->L.code != f->u->L.code) return false;
    auto kq = [](const DracoMat* x) { return x->L.code == DRACO_Q4_K || x->L.code == DRACO_Q6_K; };
    const DracoMat& o = *m->attn[l]->wo;
    return kq(f->g) && kq(&o) && draco_dq_ksplit_waves(o.L.n_in, 0) && (o.L.n_out + 15) / 16 <= 128;
}

// The attention split merge fused with the o projection (dk_attn_o), on by
// default; draco_set_attn_o_fusion switches it.
int g_attn_o_fusion = 1;
// With it, Q8_0 layers whose caches stay within DK_ATT_SHORT_T rows in a call
// run the whole attention inside the o projection (dk_attn_o8_short); on by
// default, draco_set_attn_short switches it.
int g_attn_short = 1;

// Whether dense layer l's attention split merge rides on its o projection
// (dk_attn_o: one launch fewer per layer) and the o projection's chunk sums
// on the gate/up launch (its pending-residual prologue forms the FFN input
// into w.xm): the per-head attention kernel at head dim 64, and either a
// K-quant o projection of 32 q heads (eight 256-wide input chunks of four
// heads: configs[2]) with a gate/up pair of one K-quant format whose rows the
// PRES8 prologue covers, or a Q8_0 o projection of at most 4 q heads per kv
// head (one chunk per kv group: configs[0]) with a Q8_0 gate/up pair.
bool fused_o_shape(const DevModel* m, int l) {
    if (!g_attn_o_fusion) return false;
    const DevFfn* f = m->ffn[l];
    const DevAttn* a = m->attn[l];
    auto kq = [](const DracoMat* x) { return x->L.code == DRACO_Q4_K || x->L.code == DRACO_Q6_K; };
    if (m->moe[l]) {
        // MoE layers: a K-quant o projection of whole 256-wide
        // chunks at head dim 64 / 128 / 256, the grouped or per-head
        // attention kernel, and a router whose RMSNorm prologue can form the
        // pending input
        const int HD = a->HD;
        return kq(a->wo) && (HD == 64 || HD == 128 || HD == 256) && (a->NH * HD) % 256 == 0 &&
               a->wo->L.n_in == a->NH * HD && (attn_grouped(a->NH, a->NKV, HD) || attn_per_head(a->NH, a->NKV, HD)) &&
               attn_nsplit(a->max_t, a->NH, a->NKV, HD) <= 64 && draco_moe_layer_pend_ok(m->moe[l], m->fnorm[l]);
    }
    if (!f || f->g->L.code != f->u->L.code) return false;
    if (a->HD != 64 || !attn_per_head(a->NH, a->NKV, a->HD) || attn_grouped(a->NH, a->NKV, a->HD) ||
        attn_nsplit(a->max_t, a->NH, a->NKV, a->HD) > 64 || a->wo->L.n_in != a->NH * 64)
        return false;
    // Q8_0: chunks of one kv group of at most 4 heads, a Q8_0
    // gate/up pair whose rows one prologue batch holds (k_seg PEND)
    if (a->wo->L.code == DRACO_Q8_0)
        return f->g->L.code == DRACO_Q8_0 && a->NH / a->NKV <= 4 && f->H <= 4096;
    if (!kq(f->g) || !kq(a->wo) || a->NH != 32 || a->wo->L.n_in != 2048) return false;
    DqShape sh;
    return draco_dq_shape(f->H, (f->FF + 15) / 16, true, 0, 4, 0, 256, sh) == 0;
}

// The fused layers of a model for this call, and their accumulators, all
// cleared on the stream (before any capture): each fused layer's launch
// clears the previous fused layer's accumulator (its consumer, the gate/up
// launch, ran before), so every accumulator is zero when its layer starts,
// call after call; fewer than two fused layers run unfused (a layer cannot
// clear its own).  Called by every entry point before it enqueues layers.
int plan_fusion(DevModel* m, hipStream_t st, int n_steps) {
    const int L = m->n_layer;
    m->call_rows = 0;
    for (int l = 0; l < L; l++) m->call_rows = std::max(m->call_rows, *m->attn[l]->snap.tlen + n_steps);
    m->fo.assign(L, 0);
    m->fo_prev.assign(L, -1);
    std::vector<int> ls;
    for (int l = 0; l < L; l++)
        if (fused_o_shape(m, l)) ls.push_back(l);
    if (ls.size() < 2) return 0;
    for (size_t i = 0; i < ls.size(); i++) {
        m->fo[ls[i]] = 1;
        m->fo_prev[ls[i]] = ls[(i + ls.size() - 1) % ls.size()];
    }
    const size_t stride = ((size_t)m->h + 1 + 63) / 64 * 64;
    const size_t n = stride * L;
    if (m->oacc_n < n) {
        if (m->oacc) {
            DRACO_HIP(hipStreamSynchronize(st));
            DRACO_HIP(hipFree(m->oacc));
            m->oacc = nullptr;
        }
        DRACO_HIP(hipMalloc(&m->oacc, sizeof(unsigned long long) * n));
        m->oacc_n = n;
    }
    m->oacc_stride = stride;
    DRACO_HIP(hipMemsetAsync(m->oacc, 0, sizeof(unsigned long long) * n, st));
    return 0;
}

bool fused_o(const DevModel* m, int l) { return l >= 0 && l < (int)m->fo.size() && m->fo[l]; }

// Whether MoE layer l's expert down launch leaves its two halves' sums
// pending (split_out into w.pd), for layer l + 1's q/k/v launch to form
// w.xm + half 0 + half 1: the MoE input is materialised in w.xm (a fused or
// split-K o projection whose router stored it), the next layer's q/k/v are
// all K-quants (the launch that takes the pending sum) and the down launch
// serves the halves (an even number of experts, at most 16).  A 2048x768
// down of 8 experts runs 256 blocks of 4 waves instead of 128 of 8.
// draco_set_moe_split switches it (on by default).
int g_moe_split = 1;
bool moe_split(const DevModel* m, int l) {
    if (!g_moe_split || l + 1 >= m->n_layer || !m->moe[l] || !draco_moe_layer_split_ok(m->moe[l])) return false;
    if (!fused_o(m, l) && !ksplit_o(m, l)) return false;
    const DevAttn* n = m->attn[l + 1];
    auto kq = [](const DracoMat* x) { return x->L.code == DRACO_Q4_K || x->L.code == DRACO_Q6_K; };
    return kq(n->wq) && kq(n->wk) && kq(n->wv);
}

// enqueue one llama layer on the device (x in w.x, updated in place; with
// xin set the layer reads its input from xin and leaves its output in w.x):
// qkv(+norm,+rope,+append), attention, merge, wo(+residual),
// gate/up(+norm,+SwiGLU), down(+residual).  After a split-K down the output
// is pending (w.x + the partials in w.pd) and the next layer's qkv launch
// forms it (into w.xs), which wo then takes as its residual.  After a
// split-K o projection (ksplit_o_dense) the gate/up launch forms the FFN
// input into w.xm, the down projection's residual: the layer output is then
// w.xm + the down's partials when the down is split-K too.
int enqueue_layer(DevModel* m, int l, float eps, hipStream_t st, const float* xin = nullptr) {
    DevAttn* a = m->attn[l];
    DevFfn* f = m->ffn[l];
    Work& w = m->w;
    const int H = m->h;
    const float* x0 = xin ? xin : w.x;
    const bool pending = !xin && l > 0 && (ksplit_down(m, l - 1) || moe_split(m, l - 1));
    // a pending input's materialised part: w.xm after a split-K or fused o
    // projection (the previous layer's FFN input; for a split MoE layer
    // always, moe_split requires it)
    const float* xq =
        pending && (fused_o(m, l - 1) || ksplit_o_dense(m, l - 1) || moe_split(m, l - 1)) ? w.xm : x0;
    if (int rc = enqueue_qkv(a, w, xq, 1, m->anorm[l], eps, m->state, l, st, pending)) return rc;
    const float* base = pending ? w.xs : x0;  // this layer's input
    const bool fo = fused_o(m, l);
    if (fo) {
        // split partials, then their merge + the o projection into the int64
        // accumulator, which the next launch adds to the input (into w.xm);
        // Q8_0 layers with short caches run the whole attention inside the
        // o projection's blocks (one launch)
        unsigned long long* acc = m->oacc + (size_t)l * m->oacc_stride;
        unsigned long long* zacc = m->oacc + (size_t)m->fo_prev[l] * m->oacc_stride;
        if (g_attn_short && a->wo->L.code == DRACO_Q8_0 && m->call_rows <= DK_ATT_SHORT_T) {
            if (dk_attn_o8_short(w.q, a->kc, a->vc, m->state, l, a->NH, a->NKV, a->HD, a->scale,
                                 std::min(m->call_rows, a->max_t), *a->wo, acc, zacc, (int)m->oacc_stride, st))
                return fail(-1, "short attention o launch");
        } else {
            if (dk_attention_parts(w.q, a->kc, a->vc, w.part, m->state, l, a->NH, a->NKV, a->HD, a->max_t, a->scale,
                                   st))
                return fail(-1, "attention launch");
            if (dk_attn_o(w.part, a->NH, a->NKV, a->HD, a->max_t, *a->wo, acc, zacc, (int)m->oacc_stride, st))
                return fail(-1, "attention o launch");
        }
        if (m->moe[l])  // the router forms base + the o projection into w.xm (its norm input, the down's residual)
            return draco_moe_layer_enqueue(m->moe[l], base, m->fnorm[l], eps, w.x, nullptr, st,
                                           reinterpret_cast<const float*>(acc), w.xm, true,
                                           moe_split(m, l) ? w.pd : nullptr);
        if (int rc = enqueue_gateup(f, w, base, 1, m->fnorm[l], eps, st, reinterpret_cast<const float*>(acc), w.xm, 8))
            return rc;
    } else if (dk_attention(w.q, a->kc, a->vc, w.part, w.cnt, w.att, m->state, l, a->NH, a->NKV, a->HD, a->max_t,
                            a->scale, st)) {
        return fail(-1, "attention launch");
    }
    if (m->moe[l] && ksplit_o(m, l)) {
        // o split-K into w.pd; the router forms base + the partials into w.xm
        // (its RMSNorm input and the down launch's residual)
        SegLaunch s = {};
        s.nseg = 1;
        s.n_in = a->wo->L.n_in;
        s.x = w.att;
        s.ksplit = 2;
        SegDesc& d = s.seg[0];
        d.base = a->wo->dev;
        d.L = a->wo->L;
        d.row0 = 0;
        d.row1 = H;
        d.y = w.pd;
        d.epi = EPI_STORE;
        if (draco_seg_launch(s, st)) return fail(-1, "gemv o (split-K)");
        // (the o partials in w.pd are consumed by the router before the
        // down launch writes its halves there)
        return draco_moe_layer_enqueue(m->moe[l], base, m->fnorm[l], eps, w.x, nullptr, st, w.pd, w.xm, false,
                                       moe_split(m, l) ? w.pd : nullptr);
    }
    const bool kso = !fo && !m->moe[l] && ksplit_o_dense(m, l);
    if (fo) {
        // (launched above)
    } else if (kso) {
        // o split-K into w.pd (free: this layer's qkv consumed the down's)
        SegLaunch s = {};
        s.nseg = 1;
        s.n_in = a->wo->L.n_in;
        s.x = w.att;
        s.ksplit = 2;
        SegDesc& d = s.seg[0];
        d.base = a->wo->dev;
        d.L = a->wo->L;
        d.row0 = 0;
        d.row1 = H;
        d.y = w.pd;
        d.epi = EPI_STORE;
        if (draco_seg_launch(s, st)) return fail(-1, "gemv o (split-K)");
        if (int rc = enqueue_gateup(f, w, base, 1, m->fnorm[l], eps, st, w.pd, w.xm)) return rc;
    } else {
        if (draco_gemv_launch(*a->wo, w.att, w.x, base, 0, H, st)) return fail(-1, "gemv o");
        if (m->moe[l])  // RMSNorm, router, routed gate/up + SwiGLU, down + weighted combine + residual
            return draco_moe_layer_enqueue(m->moe[l], w.x, m->fnorm[l], eps, w.x, w.x, st);
        if (int rc = enqueue_gateup(f, w, w.x, 1, m->fnorm[l], eps, st)) return rc;
    }
    const float* mid = (kso || fo) ? w.xm : w.x;  // the FFN's input, the down's residual
    if (ksplit_down(m, l)) {
        SegLaunch s = {};
        s.nseg = 1;
        s.n_in = f->d->L.n_in;
        s.x = w.g;
        s.ksplit = 2;
        SegDesc& d = s.seg[0];
        d.base = f->d->dev;
        d.L = f->d->L;
        d.row0 = 0;
        d.row1 = H;
        d.y = w.pd;
        d.epi = EPI_STORE;
        if (draco_seg_launch(s, st)) return fail(-1, "gemv down (split-K)");
        return 0;
    }
    if (draco_gemv_launch(*f->d, w.g, w.x, mid, 0, H, st)) return fail(-1, "gemv down");
    return 0;
}

bool has_moe(const DevModel* m) {
    for (const MoeLayer* p : m->moe)
        if (p) return true;
    return false;
}

// Whether the model's tokens can go through the batched (chunked) prefill:
// dense FFNs and attention shapes its kernel serves; other models feed
// their prompts through token-serial decode steps.
bool chunk_ok(const DevModel* m) {
    if (has_moe(m)) return false;
    for (int l = 0; l < m->n_layer; l++)
        if (!pf_attention_ok(m->attn[l]->NH, m->attn[l]->NKV, m->attn[l]->HD)) return false;
    return true;
}

// ---- chunked prefill (configs of the reference's forward_chunk,
// src/qwen35_prefill.py:209-239, for the llama family) ----

int g_prefill_chunk = 256;  // tokens per chunk; 0 = token-serial prefill

int ensure_pf(DevModel* m, int cap) {
    PfBufs& b = m->pf;
    int QD = 0, KD = 0, FF = 0, NH = 0, HD = 0, max_t = 0;
    for (int l = 0; l < m->n_layer; l++) {
        const DevAttn* a = m->attn[l];
        QD = std::max(QD, a->NH * a->HD);
        KD = std::max(KD, a->NKV * a->HD);
        NH = std::max(NH, a->NH);
        HD = std::max(HD, a->HD);
        max_t = std::max(max_t, a->max_t);
        if (m->ffn[l]) FF = std::max(FF, m->ffn[l]->FF);
    }
    const size_t part_n = pf_part_floats(NH, cap, HD, pf_attn_nsplit(max_t, cap));
    const int win = std::max(std::max(m->h, QD), FF);
    const size_t dig_n = draco_gemm_digit_bytes(cap, ((win + 255) / 256) * 256);
    if (b.cap >= cap && b.H == m->h && b.QD >= QD && b.KD >= KD && b.FF >= FF && b.part_n >= part_n && b.dig_n >= dig_n)
        return 0;
    DRACO_HIP(hipStreamSynchronize(stream()));
    float** fl[] = {&b.X, &b.Xn, &b.Q, &b.K, &b.V, &b.O, &b.G, &b.U, &b.Y, &b.part};
    for (float** f : fl)
        if (*f) {
            DRACO_HIP(hipFree(*f));
            *f = nullptr;
        }
    if (b.dig) DRACO_HIP(hipFree(b.dig));
    if (b.ids) DRACO_HIP(hipFree(b.ids));
    b = PfBufs();
    const size_t c = (size_t)cap;
    DRACO_HIP(hipMalloc(&b.X, sizeof(float) * c * m->h));
    DRACO_HIP(hipMalloc(&b.Xn, sizeof(float) * c * m->h));
    DRACO_HIP(hipMalloc(&b.Q, sizeof(float) * c * QD));
    DRACO_HIP(hipMalloc(&b.K, sizeof(float) * c * KD));
    DRACO_HIP(hipMalloc(&b.V, sizeof(float) * c * KD));
    DRACO_HIP(hipMalloc(&b.O, sizeof(float) * c * QD));
    DRACO_HIP(hipMalloc(&b.G, sizeof(float) * c * FF));
    DRACO_HIP(hipMalloc(&b.U, sizeof(float) * c * FF));
    DRACO_HIP(hipMalloc(&b.Y, sizeof(float) * c * m->h));
    DRACO_HIP(hipMalloc(&b.part, sizeof(float) * part_n));
    DRACO_HIP(hipMalloc(&b.dig, dig_n));
    DRACO_HIP(hipMalloc(&b.ids, sizeof(int) * c));
    b.cap = cap;
    b.H = m->h;
    b.QD = QD;
    b.KD = KD;
    b.FF = FF;
    b.part_n = part_n;
    b.dig_n = dig_n;
    return 0;
}

// Layer l for the T tokens whose hidden rows are in pf.X: the same steps as
// enqueue_layer (src/m6_engine.c:61-83 with llama_attn_core and
// m6_dense_op), token rows batched.  Token t sits at rope position pos0 + t
// and cache row row0 + t.
int enqueue_prefill_layer(DevModel* m, int l, int T, int pos0, int row0, float eps, hipStream_t st, bool xn_ready) {
    PfBufs& b = m->pf;
    DevAttn* a = m->attn[l];
    DevFfn* f = m->ffn[l];
    const int H = m->h;
    const float* tab = rope_dev(a->rot, a->base, pos0 + T);
    if (!tab) return -2;
    if (!xn_ready && pf_rms(b.X, m->anorm[l], b.Xn, T, H, eps, st)) return fail(-1, "prefill: rms rejected");
    // the digits of Xn are written by the first K-quant product and reused by the others
    auto kquant = [](const DracoMat* x) { return x->L.code == DRACO_Q4_K || x->L.code == DRACO_Q6_K; };
    if (draco_enqueue_gemm(*a->wq, b.Xn, T, b.Q, b.dig, false, st)) return -1;
    if (draco_enqueue_gemm(*a->wk, b.Xn, T, b.K, b.dig, kquant(a->wq), st)) return -1;
    if (draco_enqueue_gemm(*a->wv, b.Xn, T, b.V, b.dig, kquant(a->wq) || kquant(a->wk), st)) return -1;
    if (pf_rope_append(b.Q, b.K, b.V, a->kc, a->vc, tab, pos0, row0, T, a->NH, a->NKV, a->HD, a->rot, st))
        return fail(-1, "prefill: rope rejected");
    if (pf_attention(b.Q, a->kc, a->vc, b.part, b.O, row0, T, a->NH, a->NKV, a->HD, a->scale, st))
        return fail(-1, "prefill: attention shape NH=%d NKV=%d HD=%d not served", a->NH, a->NKV, a->HD);
    if (draco_enqueue_gemm(*a->wo, b.O, T, b.Y, b.dig, false, st)) return -1;
    if (pf_add_rms(b.X, b.Y, m->fnorm[l], b.Xn, T, H, eps, st)) return fail(-1, "prefill: rms rejected");
    if (draco_enqueue_gemm(*f->g, b.Xn, T, b.G, b.dig, false, st)) return -1;
    if (draco_enqueue_gemm(*f->u, b.Xn, T, b.U, b.dig, kquant(f->g), st)) return -1;
    dk_swiglu(b.G, b.U, T * f->FF, st);
    if (draco_enqueue_gemm(*f->d, b.G, T, b.Y, b.dig, false, st)) return -1;
    // the residual; fused with the next layer's input RMSNorm when there is one
    if (l + 1 < m->n_layer) {
        if (pf_add_rms(b.X, b.Y, m->anorm[l + 1], b.Xn, T, H, eps, st)) return fail(-1, "prefill: rms rejected");
    } else {
        pf_add(b.X, b.Y, (size_t)T * H, st);
    }
    return 0;
}

// Tokens ids[0..n) (device) through every layer in chunks of g_prefill_chunk:
// token i at position pos0 + i and cache row tlen_l + i of layer l (the
// host tlen counters are not advanced here).  The last token's hidden state
// is left in pf.X row (last chunk's T - 1); returns that T (0 on error).
int enqueue_prefill(DevModel* m, const DracoMat* em, const int* ids, int n, int pos0, float eps, hipStream_t st) {
    if (!chunk_ok(m)) {
        fail(-1, "chunked prefill: MoE layers and attention shapes outside the batched kernel go token by token");
        return 0;
    }
    const int C = g_prefill_chunk;
    if (C < 1 || n < 1) return 0;
    if (ensure_pf(m, C)) return 0;
    int last = 0;
    for (int c0 = 0; c0 < n; c0 += C) {
        const int T = std::min(C, n - c0);
        if (pf_embed(em->dev, em->L, ids + c0, T, m->pf.X, st)) return 0;
        for (int l = 0; l < m->n_layer; l++)
            if (enqueue_prefill_layer(m, l, T, pos0 + c0, *m->attn[l]->snap.tlen + c0, eps, st, l > 0)) return 0;
        last = T;
    }
    return last;
}

int check_positions(DevModel* m, int pos, int n_steps) {
    for (int l = 0; l < m->n_layer; l++) {
        const int T = *m->attn[l]->snap.tlen;
        if (T < 0 || T + n_steps > m->attn[l]->max_t)
            return fail(-1, "layer %d: tlen %d + %d steps exceeds max_t %d", l, T, n_steps, m->attn[l]->max_t);
    }
    if (pos < 0) return fail(-1, "negative position %d", pos);
    for (int l = 0; l < m->n_layer; l++)
        if (!rope_dev(m->attn[l]->rot, m->attn[l]->base, pos + n_steps)) return -2;
    return 0;
}

// device state = [pos, tlen_l + add for each layer]
int upload_state(DevModel* m, int pos, hipStream_t st, int add = 0) {
    m->hstate[0] = pos;
    for (int l = 0; l < m->n_layer; l++) m->hstate[1 + l] = *m->attn[l]->snap.tlen + add;
    DRACO_HIP(hipMemcpyAsync(m->state, m->hstate, sizeof(int) * (1 + m->n_layer), hipMemcpyHostToDevice, st));
    return 0;
}

// state layout of a single directly-called op: [pos, tlen]
int* op_state() {
    static int* d = nullptr;
    if (!d && hipMalloc(&d, sizeof(int) * 8) != hipSuccess) return nullptr;
    return d;
}

}  // namespace

extern "C" {

// src/m6_engine.c:31-37
void m6_rms_norm(const float* x, const float* w, int h, float eps, float* out) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = ensure_init()) { report(rc, "m6_rms_norm"); return; }
    hipStream_t st = stream();
    float* dx = (float*)scratch(2, sizeof(float) * h * 3);
    if (!dx) { report(-2, "m6_rms_norm"); return; }
    float* dw = dx + h;
    float* dout = dx + 2 * h;
    hipMemcpyAsync(dx, x, sizeof(float) * h, hipMemcpyHostToDevice, st);
    if (w) hipMemcpyAsync(dw, w, sizeof(float) * h, hipMemcpyHostToDevice, st);
    dk_rmsnorm(dx, w ? dw : nullptr, dout, h, eps, st);
    hipMemcpyAsync(out, dout, sizeof(float) * h, hipMemcpyDeviceToHost, st);
    hipError_t e = hipStreamSynchronize(st);
    if (e != hipSuccess) report(fail(-2, "m6_rms_norm: %s", hipGetErrorString(e)), "m6_rms_norm");
}

// src/m6_engine.c:40-54 (same table, including codes this library does not compute)
size_t m6_rowbytes(int code, int n_in) {
    switch (code) {
    case 0: return (size_t)(n_in / 32) * 34;
    case 1: return (size_t)(n_in / 32) * 18;
    case 2: return (size_t)(n_in / 256) * 110;
    case 3: return (size_t)(n_in / 256) * 176;
    case 4: return (size_t)(n_in / 256) * 210;
    case 5: return (size_t)(n_in / 256) * 144;
    case 6: return (size_t)(n_in / 256) * 136;
    case 7: return (size_t)n_in * 2;
    case 8: return (size_t)(n_in / 32) * 22;
    case 9: return (size_t)n_in * 4;
    default: return 0;
    }
}

const char* m6_engine_version(void) { return "m6_engine/1 draco_hip gfx950"; }

// src/m6_layer.c:123-140.  The HIP library serves every format itself, so the
// kernel-slot paths are accepted and ignored (0 = ok, as the reference).
int m6_init_dl(const char* p012, const char* p3, const char* p4, const char* p56, const char* ps) {
    (void)p012; (void)p3; (void)p4; (void)p56; (void)ps;
    return 0;
}

// src/m6_layer.c:94-100 (Q5_0 slot).  Accepted; code 8 GEMVs fail loudly (-1).
int m6_init_extra_dl(const char* p50) {
    (void)p50;
    return 0;
}

// src/m6_layer.c:108-120, the opt-in IQ3_S integer kernel slot
// (src/qwen35_engine.py:103-108 binds it when DRACO_IQ3_FAST=1).  IQ3_S is
// not carried by this library: returns 1 ("could not load"), which the
// driver reports before going on without the fast path.
int m6_init_iq3_dl(const char* p12) {
    (void)p12;
    fail(-1, "m6_init_iq3_dl: IQ3_S is not carried by this library");
    return 1;
}

// src/m6_engine.c:61-83
int m6_forward_token(float* x, int h, float eps, int pos, const M6LayerDesc* layers, int n_layer,
                     float* scratch) {
    (void)scratch;
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = ensure_init()) return report(rc, "m6_forward_token");
    DevModel* m = resolve_model(layers, n_layer, h);
    if (!m) return report(-1, "m6_forward_token");
    if (int rc = plan_fusion(m, stream(), 1)) return report(rc, "m6_forward_token");
    if (int rc = check_positions(m, pos, 1)) return report(rc, "m6_forward_token");
    hipStream_t st = stream();
    if (int rc = upload_state(m, pos, st)) return report(rc, "m6_forward_token");
    if (hipMemcpyAsync(m->w.x, x, sizeof(float) * h, hipMemcpyHostToDevice, st) != hipSuccess)
        return report(fail(-2, "x upload"), "m6_forward_token");
    for (int l = 0; l < n_layer; l++)
        if (int rc = enqueue_layer(m, l, eps, st)) return report(rc, "m6_forward_token");
    hipMemcpyAsync(x, m->w.x, sizeof(float) * h, hipMemcpyDeviceToHost, st);
    hipError_t e = hipStreamSynchronize(st);
    if (e != hipSuccess) return report(fail(-2, "m6_forward_token: %s", hipGetErrorString(e)), "m6_forward_token");
    for (int l = 0; l < n_layer; l++) *m->attn[l]->snap.tlen += 1;
    return 0;
}

// src/m6_engine.c:373-391 (scratch receives the normalised x, as there)
int m6_head_op(const float* x, const float* final_norm, int h, float eps, const uint8_t* head_w, int code,
               int vocab, float* logits, float* scratch) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = ensure_init()) return report(rc, "m6_head_op");
    const DracoMat* hm = get_mat(head_w, code, vocab, h);
    if (!hm) return report(-1, "m6_head_op");
    const float* nw = norm_dev(final_norm, h);
    if (final_norm && !nw) return report(-2, "m6_head_op");
    hipStream_t st = stream();
    float* dx = (float*)draco::scratch(3, sizeof(float) * (2 * (size_t)h + 64));
    float* dl = (float*)draco::scratch(4, sizeof(float) * (size_t)vocab);
    if (!dx || !dl) return report(-2, "m6_head_op");
    float* dxn = dx + h + 32;
    hipMemcpyAsync(dx, x, sizeof(float) * h, hipMemcpyHostToDevice, st);
    if (hm->L.code == DRACO_Q4_K || hm->L.code == DRACO_Q6_K || hm->L.code == DRACO_Q8_0) {
        SegLaunch sl = {};
        sl.nseg = 1;
        sl.n_in = h;
        sl.x = dx;
        sl.do_norm = 1;
        sl.norm_w = nw;
        sl.eps = eps;
        sl.xn_out = dxn;
        sl.seg[0] = seg_of(hm, EPI_STORE, dl, nullptr);
        if (draco_seg_launch(sl, st)) return report(fail(-1, "head launch rejected"), "m6_head_op");
    } else {
        dk_rmsnorm(dx, nw, dxn, h, eps, st);
        draco_gemv_launch(*hm, dxn, dl, nullptr, 0, vocab, st);
    }
    hipMemcpyAsync(logits, dl, sizeof(float) * vocab, hipMemcpyDeviceToHost, st);
    if (scratch) hipMemcpyAsync(scratch, dxn, sizeof(float) * h, hipMemcpyDeviceToHost, st);
    hipError_t e = hipStreamSynchronize(st);
    if (e != hipSuccess) return report(fail(-2, "m6_head_op: %s", hipGetErrorString(e)), "m6_head_op");
    return 0;
}

// src/m6_engine.c:514-517 called directly (host xn in, host out).
void m6_llama_attn_op(const float* xn, void* pv, int pos, float* out) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = ensure_init()) { report(rc, "m6_llama_attn_op"); return; }
    const M6LlamaAttnP* p = (const M6LlamaAttnP*)pv;
    DevAttn* a = get_attn(p);
    if (!a) { report(-1, "m6_llama_attn_op"); return; }
    const int T = *p->tlen;
    if (T < 0 || T >= a->max_t || pos < 0) { report(fail(-1, "tlen %d / pos %d out of range", T, pos), "m6_llama_attn_op"); return; }
    if (!rope_dev(a->rot, a->base, pos + 1)) { report(-2, "m6_llama_attn_op"); return; }
    static Work w;
    if (ensure_work(w, a->H, a->NH * a->HD, a->NKV * a->HD, a->NH, a->HD, a->max_t, 1)) { report(-2, "m6_llama_attn_op"); return; }
    int* ds = op_state();
    static int* hs = nullptr;
    if (!hs) hipHostMalloc(&hs, sizeof(int) * 8, hipHostMallocDefault);
    hipStream_t st = stream();
    hs[0] = pos;
    hs[1] = T;
    hipMemcpyAsync(ds, hs, sizeof(int) * 2, hipMemcpyHostToDevice, st);
    hipMemcpyAsync(w.xn, xn, sizeof(float) * a->H, hipMemcpyHostToDevice, st);
    if (enqueue_qkv(a, w, w.xn, 0, nullptr, 0.f, ds, 0, st)) { report(-1, "m6_llama_attn_op"); return; }
    dk_attention(w.q, a->kc, a->vc, w.part, w.cnt, w.att, ds, 0, a->NH, a->NKV, a->HD, a->max_t, a->scale, st);
    draco_gemv_launch(*a->wo, w.att, w.x, nullptr, 0, a->H, st);
    hipMemcpyAsync(out, w.x, sizeof(float) * a->H, hipMemcpyDeviceToHost, st);
    hipError_t e = hipStreamSynchronize(st);
    if (e != hipSuccess) { report(fail(-2, "m6_llama_attn_op: %s", hipGetErrorString(e)), "m6_llama_attn_op"); return; }
    *p->tlen = T + 1;
}

// src/m6_engine.c:275-303 called directly.
void m6_dense_op(const float* xn, void* pv, float* out) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = ensure_init()) { report(rc, "m6_dense_op"); return; }
    DevFfn* f = get_ffn((const M6DenseP*)pv);
    if (!f) { report(-1, "m6_dense_op"); return; }
    static Work w;
    if (ensure_work(w, f->H, 1, 1, 1, 64, 64, f->FF)) { report(-2, "m6_dense_op"); return; }
    hipStream_t st = stream();
    hipMemcpyAsync(w.xn, xn, sizeof(float) * f->H, hipMemcpyHostToDevice, st);
    if (enqueue_gateup(f, w, w.xn, 0, nullptr, 0.f, st)) { report(-1, "m6_dense_op"); return; }
    draco_gemv_launch(*f->d, w.g, w.x, nullptr, 0, f->H, st);
    hipMemcpyAsync(out, w.x, sizeof(float) * f->H, hipMemcpyDeviceToHost, st);
    hipError_t e = hipStreamSynchronize(st);
    if (e != hipSuccess) report(fail(-2, "m6_dense_op: %s", hipGetErrorString(e)), "m6_dense_op");
}

// qwen35moe shared expert, src/m6_engine.c:1111-1127: out = down(SwiGLU(gate
// x, up x)) * sigmoid(gate_inp_shexp . x); shp/shc = {gate, up, down,
// gate_inp} (gate/up shi x h, down h x shi, gate_inp 1 x h).  Like the
// reference it returns nothing; on return out[h] holds the gated output,
// shg[h] the ungated down product, sg[0] the gate logit and sh[0, shi) the
// SwiGLU activation (sh[shi, 2 shi) is scratch and is not written).
void m6_granite_shexp(const float* x, const uint64_t* shp, const int* shc, float* sg, float* sh, float* shg,
                      float* out, int shi, int h) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = ensure_init()) { report(rc, "m6_granite_shexp"); return; }
    if (shi <= 0 || h <= 0) { report(fail(-1, "m6_granite_shexp: shape shi %d h %d", shi, h), "m6_granite_shexp"); return; }
    // the gate/up/down triple resolves through the dense-op cache, keyed by a
    // descriptor that is refreshed per call (re-resolved only when it changes)
    static M6DenseP key;
    key.g = (const uint8_t*)(uintptr_t)shp[0];
    key.u = (const uint8_t*)(uintptr_t)shp[1];
    key.d = (const uint8_t*)(uintptr_t)shp[2];
    key.cg = shc[0];
    key.cu = shc[1];
    key.cd = shc[2];
    key.n_ff = shi;
    key.h = h;
    DevFfn* f = get_ffn(&key);
    const DracoMat* gi = get_mat((const void*)(uintptr_t)shp[3], shc[3], 1, h);
    if (!f || !gi) { report(-1, "m6_granite_shexp"); return; }
    static Work w;
    if (ensure_work(w, h, h, 1, 1, 64, 64, shi)) { report(-2, "m6_granite_shexp"); return; }
    hipStream_t st = stream();
    hipMemcpyAsync(w.xn, x, sizeof(float) * h, hipMemcpyHostToDevice, st);
    if (enqueue_gateup(f, w, w.xn, 0, nullptr, 0.f, st) || enqueue_shexp_tail(*gi, *f->d, w, h, st)) {
        report(-1, "m6_granite_shexp");
        return;
    }
    hipMemcpyAsync(out, w.q, sizeof(float) * h, hipMemcpyDeviceToHost, st);
    hipMemcpyAsync(shg, w.x, sizeof(float) * h, hipMemcpyDeviceToHost, st);
    hipMemcpyAsync(sg, w.k, sizeof(float), hipMemcpyDeviceToHost, st);
    hipMemcpyAsync(sh, w.g, sizeof(float) * shi, hipMemcpyDeviceToHost, st);
    hipError_t e = hipStreamSynchronize(st);
    if (e != hipSuccess) report(fail(-2, "m6_granite_shexp: %s", hipGetErrorString(e)), "m6_granite_shexp");
}

// Graph-replayed timing of m6_granite_shexp's device work (gate/up + SwiGLU,
// down, gate row + sigmoid scale) with x resident, the four weights rotated
// over n_copies device copies so that the replay streams from HBM once
// n_copies x the weight bytes exceeds the 256 MB MALL: out[0] = us per call,
// out[1] = weight bytes per call.
int draco_bench_shexp(const float* x, const uint64_t* shp, const int* shc, int shi, int h, int n_copies, int iters,
                      float* out) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = ensure_init()) return rc;
    if (shi <= 0 || h <= 0 || n_copies < 1 || iters < 1) return fail(-1, "bench shexp: bad arguments");
    static M6DenseP key;
    key = M6DenseP{(const uint8_t*)(uintptr_t)shp[0], (const uint8_t*)(uintptr_t)shp[1],
                   (const uint8_t*)(uintptr_t)shp[2], shc[0], shc[1], shc[2], shi, h};
    DevFfn* f = get_ffn(&key);
    const DracoMat* gi = get_mat((const void*)(uintptr_t)shp[3], shc[3], 1, h);
    if (!f || !gi) return -1;
    static Work w;
    if (ensure_work(w, h, h, 1, 1, 64, 64, shi)) return -2;
    hipStream_t st = stream();
    const DracoMat* src[4] = {f->g, f->u, f->d, gi};
    std::vector<DracoMat> cp(4 * (size_t)n_copies);
    for (int c = 0; c < n_copies; c++)
        for (int k = 0; k < 4; k++) {
            DracoMat& m = cp[4 * (size_t)c + k];
            m = *src[k];
            DRACO_HIP(hipMalloc(&m.dev, m.L.bytes));
            DRACO_HIP(hipMemcpyAsync(m.dev, src[k]->dev, m.L.bytes, hipMemcpyDeviceToDevice, st));
        }
    std::vector<DevFfn> fs(n_copies);
    for (int c = 0; c < n_copies; c++) {
        fs[c].g = &cp[4 * (size_t)c];
        fs[c].u = &cp[4 * (size_t)c + 1];
        fs[c].d = &cp[4 * (size_t)c + 2];
        fs[c].FF = shi;
        fs[c].H = h;
    }
    DRACO_HIP(hipMemcpyAsync(w.xn, x, sizeof(float) * h, hipMemcpyHostToDevice, st));
    auto enq = [&](int c) {
        if (enqueue_gateup(&fs[c], w, w.xn, 0, nullptr, 0.f, st) ||
            enqueue_shexp_tail(cp[4 * (size_t)c + 3], cp[4 * (size_t)c + 2], w, h, st))
            return -1;
        return 0;
    };
    int rc = enq(0);
    DRACO_HIP(hipStreamSynchronize(st));
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (!rc) {
        DRACO_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
        for (int i = 0; i < iters && !rc; i++) rc = enq(i % n_copies);
        DRACO_HIP(hipStreamEndCapture(st, &graph));
    }
    if (!rc) {
        DRACO_HIP(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
        DRACO_HIP(hipEventCreate(&e0));
        DRACO_HIP(hipEventCreate(&e1));
        DRACO_HIP(hipGraphLaunch(exec, st));
        DRACO_HIP(hipEventRecord(e0, st));
        DRACO_HIP(hipGraphLaunch(exec, st));
        DRACO_HIP(hipEventRecord(e1, st));
        DRACO_HIP(hipStreamSynchronize(st));
        float ms = 0;
        DRACO_HIP(hipEventElapsedTime(&ms, e0, e1));
        out[0] = ms * 1000.f / iters;
        const double gu = (double)(draco_row_bytes(shc[0], h) + draco_row_bytes(shc[1], h)) * shi;
        out[1] = (float)(gu + (double)draco_row_bytes(shc[2], shi) * h + (double)draco_row_bytes(shc[3], h));
        hipEventDestroy(e0);
        hipEventDestroy(e1);
        hipGraphExecDestroy(exec);
    }
    if (graph) hipGraphDestroy(graph);
    for (auto& m : cp) hipFree(m.dev);
    return rc ? fail(-1, "bench shexp: launch rejected") : 0;
}

// ---- state sync hooks (no reference counterpart; the reference's state is
// the host arrays themselves, src/draco_engine_server.py:907-922) ----

// Copy every layer's device KV mirror into the caller's kcache/vcache arrays
// (rows [0, tlen)), e.g. before snapshotting STATES.
int draco_state_pull(const void* layers_v, int n_layer) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    const M6LayerDesc* layers = (const M6LayerDesc*)layers_v;
    for (int l = 0; l < n_layer; l++) {
        const M6LlamaAttnP* p = (const M6LlamaAttnP*)layers[l].attn_p;
        const size_t b = sizeof(float) * (size_t)(*p->tlen) * p->n_kv * p->head_dim;
        if (b == 0) continue;
        if (int rc = mirror_pull(p->kcache, b)) return rc;
        if (int rc = mirror_pull(p->vcache, b)) return rc;
    }
    return 0;
}

// Upload the caller's kcache/vcache arrays into the device mirrors (rows
// [0, tlen)), e.g. after restoring a snapshot into them.
int draco_state_push(const void* layers_v, int n_layer) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = ensure_init()) return rc;
    const M6LayerDesc* layers = (const M6LayerDesc*)layers_v;
    for (int l = 0; l < n_layer; l++) {
        const M6LlamaAttnP* p = (const M6LlamaAttnP*)layers[l].attn_p;
        DevAttn* a = get_attn(p);
        if (!a) return -1;
        const size_t b = sizeof(float) * (size_t)(*p->tlen) * p->n_kv * p->head_dim;
        if (b == 0) continue;
        DRACO_HIP(hipMemcpy(a->kc, p->kcache, b, hipMemcpyHostToDevice));
        DRACO_HIP(hipMemcpy(a->vc, p->vcache, b, hipMemcpyHostToDevice));
    }
    return 0;
}

// ---- device-resident greedy generation (no reference counterpart: the
// reference's loop is Python, src/smol_engine.py:203-213; this runs the same
// steps without leaving the device) ----
//
// Feeds prompt[0..n_prompt) from the current tlen, then generates n_gen
// tokens greedily (argmax, first index on ties).  Positions are tlen-based:
// token i is at position tlen0 + i.  prompt[0..n_prompt-1) goes through the
// chunked prefill (draco_set_prefill_chunk; token-serial decode steps when it
// is 0), the last prompt token through the first decode step.  With use_graph
// != 0 the token-serial prefill step and the decode step are captured as HIP
// graphs and replayed.  stats[0] = decode ms (n_gen steps), stats[1] =
// prefill ms (the n_prompt - 1 tokens before the first decode step).
int draco_llama_generate(const void* layers_v, int n_layer, int h, float eps, const float* final_norm,
                         const uint8_t* head_w, int head_code, int vocab, const uint8_t* emb_w, int emb_code,
                         const int* prompt, int n_prompt, int n_gen, int use_graph, int* out_tokens,
                         float* out_hidden, float* stats) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = ensure_init()) return report(rc, "draco_llama_generate");
    const M6LayerDesc* layers = (const M6LayerDesc*)layers_v;
    if (n_prompt < 1 || n_gen < 1) return report(fail(-1, "need n_prompt >= 1 and n_gen >= 1"), "draco_llama_generate");
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= vocab)
            return report(fail(-1, "prompt token id %d out of range", prompt[i]), "draco_llama_generate");
    DevModel* m = resolve_model(layers, n_layer, h);
    if (!m) return report(-1, "draco_llama_generate");
    if (int rc = plan_fusion(m, stream(), n_prompt + n_gen)) return report(rc, "draco_llama_generate");
    const DracoMat* hm = get_mat(head_w, head_code, vocab, h);
    const DracoMat* em = get_mat(emb_w, emb_code, vocab, h);
    const float* nw = norm_dev(final_norm, h);
    if (!hm || !em || (final_norm && !nw)) return report(-1, "draco_llama_generate");
    const int steps = n_prompt + n_gen - 1;
    const int pos0 = *m->attn[0]->snap.tlen;
    if (int rc = check_positions(m, pos0, steps)) return report(rc, "draco_llama_generate");
    hipStream_t st = stream();
    const int ntok = n_prompt + n_gen;
    int* dtok = (int*)scratch(5, sizeof(int) * (ntok + 64));
    float* dlog = (float*)scratch(6, sizeof(float) * (size_t)vocab);
    // head argmax partials: one (value, index) per head block (8 rows per block) + a counter
    const int hblocks = (vocab + 7) / 8;
    float* dred = (float*)scratch(7, (sizeof(float) + sizeof(int)) * ((size_t)hblocks + 64) + 256);
    if (!dtok || !dlog || !dred) return report(-2, "draco_llama_generate");
    int* cursor = dtok + ntok + 8;   // index of the token being fed
    int* cur = dtok + ntok + 16;     // its id
    int* dri = (int*)(dred + hblocks + 32);
    const bool fused_head = hm->L.code == DRACO_Q4_K || hm->L.code == DRACO_Q5_K || hm->L.code == DRACO_Q6_K ||
                            hm->L.code == DRACO_Q8_0;
    std::vector<int> ht(ntok + 64, 0);
    for (int i = 0; i < n_prompt; i++) ht[i] = prompt[i];
    // prompt[0 .. n_prompt - 1) goes through the chunked prefill when enabled
    // (the last prompt token goes through the first decode step, which also
    // runs the head); the token cursor then starts past those tokens
    // (MoE models and attention shapes outside the batched prefill kernel
    // feed the prompt through token-serial decode steps)
    const int n_chunked = (g_prefill_chunk > 0 && n_prompt - 1 >= 2 && chunk_ok(m)) ? n_prompt - 1 : 0;
    if (n_chunked && ensure_pf(m, g_prefill_chunk)) return report(-2, "draco_llama_generate (prefill buffers)");
    ht[ntok + 8] = n_chunked;
    DRACO_HIP(hipMemcpyAsync(dtok, ht.data(), sizeof(int) * (ntok + 64), hipMemcpyHostToDevice, st));
    (void)cur;
    // With the fused head, a decode step's input embedding was decoded by the
    // previous step's argmax into w.xe (the first one by an embedding launch
    // after the prompt), and layer 0 reads it from there.
    auto step = [&](bool decode) -> int {
        const bool emb_ready = decode && fused_head;
        if (!emb_ready) dk_embed(*em, dtok, cursor, m->w.x, st);
        for (int l = 0; l < n_layer; l++)
            if (int rc = enqueue_layer(m, l, eps, st, (emb_ready && l == 0) ? m->w.xe : nullptr)) return rc;
        if (!decode) {
            dk_advance(m->state, n_layer, cursor, st);
            return 0;
        }
        if (fused_head) {
            // final RMSNorm + vocab GEMV + argmax (-> token cursor+1) + state advance
            SegLaunch sl = {};
            sl.nseg = 1;
            sl.n_in = h;
            sl.x = m->w.x;
            sl.do_norm = 1;
            sl.norm_w = nw;
            sl.eps = eps;
            sl.seg[0] = seg_of(hm, EPI_ARGMAX, dlog, nullptr);
            sl.am_val = dred;
            sl.am_idx = dri;
            sl.tokens = dtok;
            sl.cursor = cursor;
            sl.advance_state = m->state;
            sl.advance_layers = n_layer;
            sl.emb = em->dev;
            sl.emb_L = em->L;
            sl.emb_out = m->w.xe;
            if (draco_seg_launch(sl, st)) return fail(-1, "head launch rejected");
            return 0;
        }
        dk_rmsnorm(m->w.x, nw, m->w.xn, h, eps, st);
        if (draco_gemv_launch(*hm, m->w.xn, dlog, nullptr, 0, vocab, st)) return fail(-1, "head gemv");
        dk_argmax(dlog, vocab, dred, dri, dtok, cursor, 0, st);
        dk_advance(m->state, n_layer, cursor, st);
        return 0;
    };
    constexpr int GEN_STEPS = 16;
    // events and graphs are released on every return path (the guard's
    // destructor waits for the stream first, so no replay is still running)
    struct Guard {
        hipStream_t st;
        hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
        hipGraphExec_t gx[3] = {nullptr, nullptr, nullptr};
        hipGraph_t gg[3] = {nullptr, nullptr, nullptr};
        ~Guard() {
            hipStreamSynchronize(st);
            for (int k = 0; k < 3; k++) {
                if (gx[k]) hipGraphExecDestroy(gx[k]);
                if (gg[k]) hipGraphDestroy(gg[k]);
            }
            for (hipEvent_t e : ev)
                if (e) hipEventDestroy(e);
        }
    } G{st};
    for (hipEvent_t& e : G.ev) DRACO_HIP(hipEventCreate(&e));
    hipEvent_t e0 = G.ev[0], e1 = G.ev[1], e2 = G.ev[2];
    hipGraphExec_t* gx = G.gx;
    if (use_graph) {
        for (int k = 0; k < 2; k++) {
            DRACO_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
            int rc = step(k == 1);
            hipGraph_t gr = nullptr;
            hipError_t ce = hipStreamEndCapture(st, &gr);
            G.gg[k] = gr;
            if (rc) return report(rc, "draco_llama_generate");
            if (ce != hipSuccess) return report(fail(-2, "graph capture: %s", hipGetErrorString(ce)), "draco_llama_generate");
            DRACO_HIP(hipGraphInstantiate(&gx[k], gr, nullptr, nullptr, 0));
        }
        // GEN_STEPS generated tokens in one graph (the state advances on the
        // device, so consecutive steps capture as they run): one graph launch
        // per GEN_STEPS tokens instead of per token (configs[2], 98 kernels a
        // step: 2,219 -> 2,243 tok/s same-box).  Steps of more kernels keep one
        // graph per token: configs[0] (194 a step) and configs[3] were 0.1-0.2%
        // slower with 16-step graphs.
        size_t step_nodes = 0;
        DRACO_HIP(hipGraphGetNodes(G.gg[1], nullptr, &step_nodes));
        if (n_gen >= GEN_STEPS && step_nodes * GEN_STEPS <= 2048) {
            DRACO_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
            int rc = 0;
            for (int k = 0; k < GEN_STEPS && !rc; k++) rc = step(true);
            hipGraph_t gr = nullptr;
            hipError_t ce = hipStreamEndCapture(st, &gr);
            G.gg[2] = gr;
            if (rc) return report(rc, "draco_llama_generate");
            if (ce != hipSuccess) return report(fail(-2, "graph capture: %s", hipGetErrorString(ce)), "draco_llama_generate");
            DRACO_HIP(hipGraphInstantiate(&gx[2], gr, nullptr, nullptr, 0));
        }
    }
    DRACO_HIP(hipEventRecord(e0, st));
    if (n_chunked && enqueue_prefill(m, em, dtok, n_chunked, pos0, eps, st) <= 0)
        return report(-1, "draco_llama_generate (chunked prefill)");
    if (int rc = upload_state(m, pos0 + n_chunked, st, n_chunked)) return report(rc, "draco_llama_generate");
    for (int i = n_chunked; i < n_prompt - 1; i++) {
        if (use_graph) DRACO_HIP(hipGraphLaunch(gx[0], st));
        else if (int rc = step(false)) return report(rc, "draco_llama_generate");
    }
    if (fused_head) dk_embed(*em, dtok, cursor, m->w.xe, st);
    DRACO_HIP(hipEventRecord(e1, st));
    for (int i = 0; i < n_gen; i++) {
        if (use_graph && gx[2] && i + GEN_STEPS <= n_gen) {
            DRACO_HIP(hipGraphLaunch(gx[2], st));
            i += GEN_STEPS - 1;
            continue;
        }
        if (use_graph) DRACO_HIP(hipGraphLaunch(gx[1], st));
        else if (int rc = step(true)) return report(rc, "draco_llama_generate");
    }
    DRACO_HIP(hipEventRecord(e2, st));
    DRACO_HIP(hipMemcpyAsync(ht.data(), dtok, sizeof(int) * ntok, hipMemcpyDeviceToHost, st));
    if (out_hidden) DRACO_HIP(hipMemcpyAsync(out_hidden, m->w.x, sizeof(float) * h, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipStreamSynchronize(st));
    float ms_pre = 0, ms_dec = 0;
    hipEventElapsedTime(&ms_pre, e0, e1);
    hipEventElapsedTime(&ms_dec, e1, e2);
    if (stats) {
        stats[0] = ms_dec;
        stats[1] = ms_pre;
    }
    for (int i = 0; i < n_gen; i++) out_tokens[i] = ht[n_prompt + i];
    for (int l = 0; l < n_layer; l++) *m->attn[l]->snap.tlen += steps;
    // the attn snapshots hold the tlen pointer, not its value: still valid
    return 0;
}


// ---- chunked prefill of the llama family (the reference's forward_chunk
// contract, src/qwen35_prefill.py:209-210 and src/draco_engine_server.py:836-842:
// the engine state afterwards equals that of forward(ids[i], pos + i) run
// token by token) ----

// The fused attention merge + o projection of the llama decode layers (1 =
// on, the default; 0 = the split merge and the o projection as two launches).
// Returns the previous setting; on < 0 only queries.  Captured decode graphs
// are per call, so a change applies to the next call.
int draco_set_attn_short(int on) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    const int old = g_attn_short;
    if (on >= 0) g_attn_short = on ? 1 : 0;
    return old;
}

int draco_set_moe_split(int on) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    const int old = g_moe_split;
    if (on >= 0) g_moe_split = on ? 1 : 0;
    return old;
}

int draco_set_attn_o_fusion(int on) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    const int old = g_attn_o_fusion;
    if (on >= 0) g_attn_o_fusion = on ? 1 : 0;
    return old;
}

// Tokens per chunk of the chunked prefill (draco_llama_prefill and the
// prompt of draco_llama_generate); 0 makes draco_llama_generate feed its
// prompt token by token.  Returns the previous value; n < 0 only queries.
int draco_set_prefill_chunk(int n) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    const int old = g_prefill_chunk;
    if (n >= 0) g_prefill_chunk = n > 4096 ? 4096 : n;
    return old;
}

// ids[0..n) (host) at positions pos .. pos + n - 1: the KV rows of every layer
// are appended at rows tlen .. tlen + n - 1 (device mirrors) and every tlen
// advances by n, as n calls of m6_forward_token would leave them; out_x (h
// floats, host) receives the last token's hidden state after the last layer.
int draco_llama_prefill(const void* layers_v, int n_layer, int h, float eps, const uint8_t* emb_w, int emb_code,
                        int vocab, const int* ids, int n, int pos, float* out_x) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = ensure_init()) return report(rc, "draco_llama_prefill");
    const M6LayerDesc* layers = (const M6LayerDesc*)layers_v;
    if (n < 1 || pos < 0) return report(fail(-1, "need n >= 1 and pos >= 0"), "draco_llama_prefill");
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= vocab) return report(fail(-1, "token id %d out of range", ids[i]), "draco_llama_prefill");
    DevModel* m = resolve_model(layers, n_layer, h);
    if (!m) return report(-1, "draco_llama_prefill");
    if (int rc = plan_fusion(m, stream(), n)) return report(rc, "draco_llama_prefill");
    const DracoMat* em = get_mat(emb_w, emb_code, vocab, h);
    if (!em) return report(-1, "draco_llama_prefill");
    for (int l = 0; l < n_layer; l++) {
        const int T = *m->attn[l]->snap.tlen;
        if (T < 0 || T + n > m->attn[l]->max_t)
            return report(fail(-1, "layer %d: tlen %d + %d tokens exceeds max_t %d", l, T, n, m->attn[l]->max_t),
                          "draco_llama_prefill");
    }
    const int C = g_prefill_chunk > 0 ? g_prefill_chunk : 256;
    const int saved = g_prefill_chunk;
    g_prefill_chunk = C;
    hipStream_t st = stream();
    int* dids = (int*)scratch(5, sizeof(int) * ((size_t)n + 64));
    if (!dids) {
        g_prefill_chunk = saved;
        return report(-2, "draco_llama_prefill");
    }
    DRACO_HIP(hipMemcpyAsync(dids, ids, sizeof(int) * n, hipMemcpyHostToDevice, st));
    if (!chunk_ok(m)) {
        // token by token through the decode layers (the state of n
        // m6_forward_token calls): embedding of ids[cursor], every layer,
        // then the cursor and every tlen advance
        g_prefill_chunk = saved;
        int* cursor = dids + n + 8;
        const int zero = 0;
        DRACO_HIP(hipMemcpyAsync(cursor, &zero, sizeof(int), hipMemcpyHostToDevice, st));
        if (int rc = check_positions(m, pos, n)) return report(rc, "draco_llama_prefill");
        if (int rc = upload_state(m, pos, st)) return report(rc, "draco_llama_prefill");
        for (int i = 0; i < n; i++) {
            dk_embed(*em, dids, cursor, m->w.x, st);
            for (int l = 0; l < n_layer; l++)
                if (int rc = enqueue_layer(m, l, eps, st)) return report(rc, "draco_llama_prefill");
            dk_advance(m->state, n_layer, cursor, st);
        }
        if (out_x) DRACO_HIP(hipMemcpyAsync(out_x, m->w.x, sizeof(float) * h, hipMemcpyDeviceToHost, st));
    } else {
        const int last = enqueue_prefill(m, em, dids, n, pos, eps, st);
        g_prefill_chunk = saved;
        if (last <= 0) return report(-1, "draco_llama_prefill");
        if (out_x)
            DRACO_HIP(hipMemcpyAsync(out_x, m->pf.X + (size_t)(last - 1) * h, sizeof(float) * h,
                                     hipMemcpyDeviceToHost, st));
    }
    hipError_t e = hipStreamSynchronize(st);
    if (e != hipSuccess) return report(fail(-2, "draco_llama_prefill: %s", hipGetErrorString(e)), "draco_llama_prefill");
    for (int l = 0; l < n_layer; l++) *m->attn[l]->snap.tlen += n;
    return 0;
}

}  // extern "C"
