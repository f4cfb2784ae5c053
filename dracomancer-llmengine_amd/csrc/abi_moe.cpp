// abi_moe.cpp -- MoE entry points.
//
// m6_granite_moe: src/m6_layer.c:771-802 (called per layer by the qwen35
// driver, src/qwen35_engine.py:294-307).  m5_gemvn_q4k / m5_gemvn_q6k:
// src/m5/m5_batch8_k.c:80-183 (called by src/k2_engine.py:461-560).  All
// pointers are caller-owned HOST pointers, as in the reference; expert
// matrices are registered (uploaded once, kept resident) by host address.
#include <stdio.h>
#include <string.h>

#include <map>
#include <vector>

#include "decode.h"
#include "gemm.h"
#include "moe.h"
#include "runtime.h"

using namespace draco;

namespace {

int fm_of(int code) { return code == DRACO_Q4_K ? 1 : (code == DRACO_Q6_K ? 2 : 0); }

// device pointer tables for one expert set, rebuilt when the registry epoch moves
struct ExpertSet {
    uint64_t epoch = 0;
    std::vector<uint64_t> host_ptrs;  // the caller's table when the set was built
    std::vector<int> host_codes;
    const uint8_t** dev = nullptr;  // [3][n_exp]
    int n_exp = 0;
    int fm_gu = 0, fm_d = 0;
    const DracoMat* router = nullptr;
};

std::map<const void*, ExpertSet>& sets() {
    static std::map<const void*, ExpertSet> m;
    return m;
}

ExpertSet* expert_set(const uint64_t* ptrs, const int* codes, const float* gate_inp, int n_exp, int inter,
                      int n_in, int n_out, hipStream_t st) {
    ExpertSet& s = sets()[ptrs];
    // the table address alone does not identify the set: a new table can
    // reuse a freed one's address, so its contents must match too
    const bool same_table = s.n_exp == n_exp && s.host_ptrs.size() == 3 * (size_t)n_exp &&
                            memcmp(s.host_ptrs.data(), ptrs, sizeof(uint64_t) * 3 * (size_t)n_exp) == 0 &&
                            memcmp(s.host_codes.data(), codes, sizeof(int) * 3 * (size_t)n_exp) == 0;
    if (s.dev && s.epoch == epoch() && same_table) {
        // the same pointers can now hold other bytes (new expert buffers at
        // freed addresses): every expert goes through the registry's
        // fingerprint check; a replaced matrix moves the epoch and the table
        // is rebuilt below
        for (int e = 0; e < n_exp; e++)
            if (!get_mat((const void*)(uintptr_t)ptrs[3 * e], codes[3 * e], inter, n_in) ||
                !get_mat((const void*)(uintptr_t)ptrs[3 * e + 1], codes[3 * e + 1], inter, n_in) ||
                !get_mat((const void*)(uintptr_t)ptrs[3 * e + 2], codes[3 * e + 2], n_out, inter))
                return nullptr;
        if (s.epoch == epoch()) {
            s.router = get_mat(gate_inp, DRACO_F32, n_exp, n_in);
            if (s.router && s.epoch == epoch()) return &s;
            if (!s.router) return nullptr;
        }
    }
    const int fg = fm_of(codes[0]), fd = fm_of(codes[2]);
    if (!fg || !fd) {
        fail(-1, "m6_granite_moe: expert formats %d/%d not served (Q4_K, Q6_K)", codes[0], codes[2]);
        return nullptr;
    }
    std::vector<const uint8_t*> tab(3 * (size_t)n_exp);
    for (int e = 0; e < n_exp; e++) {
        if (codes[3 * e] != codes[0] || codes[3 * e + 1] != codes[0] || codes[3 * e + 2] != codes[2]) {
            fail(-1, "m6_granite_moe: mixed expert formats");
            return nullptr;
        }
        const DracoMat* g = get_mat((const void*)(uintptr_t)ptrs[3 * e], codes[3 * e], inter, n_in);
        const DracoMat* u = get_mat((const void*)(uintptr_t)ptrs[3 * e + 1], codes[3 * e + 1], inter, n_in);
        const DracoMat* d = get_mat((const void*)(uintptr_t)ptrs[3 * e + 2], codes[3 * e + 2], n_out, inter);
        if (!g || !u || !d) return nullptr;
        tab[e] = g->dev;
        tab[n_exp + e] = u->dev;
        tab[2 * (size_t)n_exp + e] = d->dev;
    }
    if (s.dev && s.n_exp != n_exp) {
        hipFree(s.dev);
        s.dev = nullptr;
    }
    if (!s.dev && hipMalloc(&s.dev, sizeof(void*) * 3 * (size_t)n_exp) != hipSuccess) {
        fail(-2, "m6_granite_moe: table allocation failed");
        return nullptr;
    }
    if (hipMemcpyAsync(s.dev, tab.data(), sizeof(void*) * tab.size(), hipMemcpyHostToDevice, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess) {
        fail(-2, "m6_granite_moe: table upload failed");
        return nullptr;
    }
    s.n_exp = n_exp;
    s.host_ptrs.assign(ptrs, ptrs + 3 * (size_t)n_exp);
    s.host_codes.assign(codes, codes + 3 * (size_t)n_exp);
    s.fm_gu = fg;
    s.fm_d = fd;
    s.router = get_mat(gate_inp, DRACO_F32, n_exp, n_in);
    if (!s.router) return nullptr;
    s.epoch = epoch();  // after every get_mat: a replacement above bumps it
    return &s;
}

struct MoeWork {
    float *x, *logits, *act, *out, *selw;
    int* sel;
    const uint8_t** seld;
};

int moe_work(MoeWork& w, int n_in, int n_exp, int n_used, int inter, int n_out) {
    w.x = (float*)scratch(0, sizeof(float) * (size_t)n_in);
    w.out = (float*)scratch(1, sizeof(float) * (size_t)n_out);
    char* p = (char*)scratch(4, sizeof(float) * ((size_t)n_exp + (size_t)n_used * inter + 2 * MOE_USED_MAX) +
                                    sizeof(void*) * MOE_USED_MAX + 256);
    if (!w.x || !w.out || !p) return -2;
    w.seld = (const uint8_t**)p;
    w.logits = (float*)(p + sizeof(void*) * MOE_USED_MAX);
    w.selw = w.logits + n_exp;
    w.sel = (int*)(w.selw + MOE_USED_MAX);
    w.act = (float*)(w.sel + MOE_USED_MAX);
    return 0;
}

// enqueue router + routed gate/up + down/combine (x, out device pointers)
// norm_w set: x is the layer input, normalised by the router launch into xn
// (RMSNorm with norm_w, eps), which the expert launches read
int enqueue_moe(ExpertSet* s, const float* x, float* out, const float* resid, MoeWork& w, int n_exp, int n_used,
                int inter, int n_in, int n_out, hipStream_t st, const float* norm_w = nullptr, float eps = 0.f,
                float* xn = nullptr, const float* pend = nullptr, float* xs = nullptr, bool pend_fx = false,
                float* split_out = nullptr) {
    if (draco_moe_logits_launch(x, (const float*)s->router->dev, n_exp, n_in, w.logits, st, norm_w, eps, xn, pend,
                                xs, pend_fx))
        return fail(-1, "moe router launch rejected");
    if (pend) resid = xs;  // the formed input is the residual
    MoeArgs a = {};
    a.x = norm_w ? xn : x;
    a.n_in = n_in;
    a.n_out_e = inter;
    a.n_slots = n_used;
    a.logits = w.logits;
    a.n_exp = n_exp;
    a.base0 = s->dev;
    a.base1 = s->dev + n_exp;
    a.base2 = s->dev + 2 * (size_t)n_exp;
    a.sel = w.sel;
    a.selw = w.selw;
    a.seld = w.seld;
    a.act = w.act;
    if (draco_moe_grp_launch(a, s->fm_gu, true, false, true, st)) return fail(-1, "moe gate/up launch rejected");
    a.inter = inter;
    a.n_out = n_out;
    a.out = split_out ? split_out : out;
    a.resid = split_out ? nullptr : resid;
    a.split = split_out ? 1 : 0;
    if (draco_moe_down_launch(a, s->fm_d, st)) return fail(-1, "moe down launch rejected");
    return 0;
}

int check_moe(int n_exp, int n_used, int inter, int n_in, int n_out) {
    if (n_exp < 1 || n_exp > MOE_EXP_MAX || n_used < 1 || n_used > n_exp || n_used > MOE_USED_MAX)
        return fail(-1, "m6_granite_moe: n_exp %d / n_used %d not served", n_exp, n_used);
    if (inter % 256 || n_in % 256 || n_out % 16)
        return fail(-1, "m6_granite_moe: shape inter %d n_in %d n_out %d not served", inter, n_in, n_out);
    return 0;
}

int granite_moe(const float* x0, const uint64_t* ptrs, const int* codes, const float* gate_inp, int n_exp,
                int n_used, int inter, int n_in, int n_out, float* out) {
    if (int rc = check_moe(n_exp, n_used, inter, n_in, n_out)) return rc;
    if (int rc = ensure_init()) return rc;
    hipStream_t st = stream();
    ExpertSet* s = expert_set(ptrs, codes, gate_inp, n_exp, inter, n_in, n_out, st);
    if (!s) return -2;
    MoeWork w;
    if (moe_work(w, n_in, n_exp, n_used, inter, n_out)) return -2;
    DRACO_HIP(hipMemcpyAsync(w.x, x0, sizeof(float) * (size_t)n_in, hipMemcpyHostToDevice, st));
    if (int rc = enqueue_moe(s, w.x, w.out, nullptr, w, n_exp, n_used, inter, n_in, n_out, st)) return rc;
    DRACO_HIP(hipGetLastError());
    DRACO_HIP(hipMemcpyAsync(out, w.out, sizeof(float) * (size_t)n_out, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipStreamSynchronize(st));
    return 0;
}

int gemvn(int code, const float* x, long x_stride, const uint8_t* W, const int* idx, long per, int n_out_e,
          int n_in, int n_exp, float* y) {
    const int nb = n_in / 256;
    if (nb <= 0 || n_in % 256 || nb > 256) return -1;  // the reference's own checks
    if (n_exp < 1 || n_out_e < 1) return 0;
    if (n_out_e % 16) return fail(-1, "m5_gemvn: n_out_e %d not a multiple of 16", n_out_e);
    if (int rc = ensure_init()) return rc;
    hipStream_t st = stream();
    const size_t xf = x_stride ? (size_t)(n_exp - 1) * x_stride + n_in : (size_t)n_in;
    float* dx = (float*)scratch(0, sizeof(float) * xf);
    float* dy = (float*)scratch(1, sizeof(float) * (size_t)n_exp * n_out_e);
    const uint8_t** db = (const uint8_t**)scratch(5, sizeof(void*) * (size_t)n_exp);
    if (!dx || !dy || !db) return -2;
    std::vector<const uint8_t*> tab(n_exp);
    for (int e = 0; e < n_exp; e++) {
        const DracoMat* m = get_mat(W + (int64_t)idx[e] * per, code, n_out_e, n_in);
        if (!m) return -2;
        tab[e] = m->dev;
    }
    DRACO_HIP(hipMemcpyAsync(db, tab.data(), sizeof(void*) * n_exp, hipMemcpyHostToDevice, st));
    DRACO_HIP(hipMemcpyAsync(dx, x, sizeof(float) * xf, hipMemcpyHostToDevice, st));
    // per-slot x: as many slots per launch as the prologue holds
    const int per_launch = x_stride ? draco_moe_xper_slots(n_in) : MOE_USED_MAX;
    if (per_launch < 1) return fail(-1, "m5_gemvn: n_in %d too long for per-expert x", n_in);
    for (int e0 = 0; e0 < n_exp; e0 += per_launch) {
        const int ns = n_exp - e0 < per_launch ? n_exp - e0 : per_launch;
        MoeArgs a = {};
        a.x = dx + (size_t)e0 * x_stride;
        a.x_stride = x_stride;
        a.n_in = n_in;
        a.n_out_e = n_out_e;
        a.n_slots = ns;
        a.base0 = db + e0;
        a.y = dy + (size_t)e0 * n_out_e;
        if (draco_moe_grp_launch(a, fm_of(code), false, x_stride != 0, false, st))
            return fail(-1, "m5_gemvn launch rejected");
    }
    DRACO_HIP(hipGetLastError());
    DRACO_HIP(hipMemcpyAsync(y, dy, sizeof(float) * (size_t)n_exp * n_out_e, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipStreamSynchronize(st));
    return 0;
}

// ---- token-batched MoE (prefill), src/m6_moe_tok.c:44-161 -----------------
int moe_tok(const float* X, const int* order, const float* wtop, const uint64_t* ep, const int* ec, int T,
            int n_used, int inter, int n_in, int n_out, int n_exp, float* out) {
    if (T < 1 || n_used < 1 || n_exp < 1 || n_exp > MOE_EXP_MAX)
        return fail(-1, "m6_moe_tok: T %d n_used %d n_exp %d not served", T, n_used, n_exp);
    if (inter % 256 || n_in % 256 || n_out % 16)
        return fail(-1, "m6_moe_tok: shape inter %d n_in %d n_out %d not served", inter, n_in, n_out);
    // expert grouping (the reference's off/ilist/slot, segments padded to 8 tokens)
    std::vector<int> cnt(n_exp, 0);
    for (int i = 0; i < T * n_used; i++)
        if (order[i] >= 0 && order[i] < n_exp) cnt[order[i]]++;
    std::vector<int> oct0(n_exp, 0), active;
    int n_oct = 0, max_oct = 0;
    int cg = -1, cu = -1, cd = -1;
    for (int e = 0; e < n_exp; e++) {
        if (!cnt[e]) continue;
        active.push_back(e);
        oct0[e] = n_oct;
        const int o = (cnt[e] + 7) / 8;
        n_oct += o;
        max_oct = o > max_oct ? o : max_oct;
        if (cg < 0) {
            cg = ec[3 * e];
            cu = ec[3 * e + 1];
            cd = ec[3 * e + 2];
        }
        if (ec[3 * e] != cg || ec[3 * e + 1] != cu || ec[3 * e + 2] != cd)
            return fail(-1, "m6_moe_tok: mixed expert formats");
    }
    if (active.empty()) {
        memset(out, 0, sizeof(float) * (size_t)T * n_out);
        return 0;
    }
    // gate and up may differ in format: the up product reuses the gate's
    // activation digits, which do not depend on the weight format
    if (!fm_of(cg) || !fm_of(cu) || !fm_of(cd))
        return fail(-1, "m6_moe_tok: expert formats %d/%d/%d not served", cg, cu, cd);
    const int R = 8 * n_oct;
    std::vector<int> src(R, -1), pos((size_t)T * n_used, -1), fill(n_exp, 0);
    for (int i = 0; i < T * n_used; i++) {
        const int e = order[i];
        if (e < 0 || e >= n_exp) continue;
        const int row = 8 * oct0[e] + fill[e]++;
        src[row] = i / n_used;
        pos[i] = row;
    }
    if (int rc = ensure_init()) return rc;
    hipStream_t st = stream();
    const int na = (int)active.size();
    std::vector<GemmGroup> gg(na), gu(na), gd(na);
    for (int k = 0; k < na; k++) {
        const int e = active[k];
        const DracoMat* g = get_mat((const void*)(uintptr_t)ep[3 * e], cg, inter, n_in);
        const DracoMat* u = get_mat((const void*)(uintptr_t)ep[3 * e + 1], cu, inter, n_in);
        const DracoMat* d = get_mat((const void*)(uintptr_t)ep[3 * e + 2], cd, n_out, inter);
        if (!g || !u || !d) return -2;
        const int o = (cnt[e] + 7) / 8;
        gg[k] = {g->dev, oct0[e], o};
        gu[k] = {u->dev, oct0[e], o};
        gd[k] = {d->dev, oct0[e], o};
    }
    // device buffers (scratch slots 8..): inputs, gathered rows, digits, intermediates, tables
    const size_t fX = (size_t)T * n_in, fXg = (size_t)R * n_in, fI = (size_t)R * inter, fY = (size_t)R * n_out,
                 fO = (size_t)T * n_out;
    float* dX = (float*)scratch(8, sizeof(float) * fX);
    float* dXg = (float*)scratch(9, sizeof(float) * fXg);
    float* dG = (float*)scratch(10, sizeof(float) * fI);
    float* dU = (float*)scratch(11, sizeof(float) * fI);
    float* dY = (float*)scratch(12, sizeof(float) * fY);
    float* dO = (float*)scratch(13, sizeof(float) * fO);
    const size_t dbytes = draco_gemm_digit_bytes(R, n_in > inter ? n_in : inter);
    uint8_t* dD = (uint8_t*)scratch(14, dbytes);
    const size_t tb = sizeof(int) * ((size_t)R + (size_t)T * n_used) + sizeof(float) * (size_t)T * n_used +
                      sizeof(GemmGroup) * 3 * (size_t)na + 64;
    char* dT = (char*)scratch(15, tb);
    if (!dX || !dXg || !dG || !dU || !dY || !dO || !dD || !dT) return -2;
    int* dsrc = (int*)dT;
    int* dpos = dsrc + R;
    float* dwt = (float*)(dpos + (size_t)T * n_used);
    GemmGroup* dgr = (GemmGroup*)(((uintptr_t)(dwt + (size_t)T * n_used) + 15) & ~(uintptr_t)15);
    std::vector<GemmGroup> allg;
    allg.insert(allg.end(), gg.begin(), gg.end());
    allg.insert(allg.end(), gu.begin(), gu.end());
    allg.insert(allg.end(), gd.begin(), gd.end());
    DRACO_HIP(hipMemcpyAsync(dX, X, sizeof(float) * fX, hipMemcpyHostToDevice, st));
    DRACO_HIP(hipMemcpyAsync(dsrc, src.data(), sizeof(int) * R, hipMemcpyHostToDevice, st));
    DRACO_HIP(hipMemcpyAsync(dpos, pos.data(), sizeof(int) * pos.size(), hipMemcpyHostToDevice, st));
    DRACO_HIP(hipMemcpyAsync(dwt, wtop, sizeof(float) * (size_t)T * n_used, hipMemcpyHostToDevice, st));
    DRACO_HIP(hipMemcpyAsync(dgr, allg.data(), sizeof(GemmGroup) * allg.size(), hipMemcpyHostToDevice, st));
    if (draco_moe_gather_launch(dX, n_in, dsrc, R, dXg, st)) return fail(-1, "moe_tok gather rejected");
    auto grouped = [&](const float* Xin, int k_in, int code, const GemmGroup* groups, int rows, float* Y) -> int {
        DracoLayout L;
        if (draco_layout(code, rows, k_in, &L)) return fail(-1, "moe_tok layout");
        GemmArgs a = {};
        if (draco_gemm_digits_launch(Xin, R, k_in, dD, a, st)) return fail(-1, "moe_tok digits rejected");
        a.L = L;
        a.Y = Y;
        a.ldy = rows;
        a.groups = groups;
        a.n_groups = na;
        a.max_oct = max_oct;
        if (draco_gemm_grouped_launch(a, st)) return fail(-1, "moe_tok gemm rejected");
        return 0;
    };
    if (int rc = grouped(dXg, n_in, cg, dgr, inter, dG)) return rc;
    {
        // the gate and up GEMMs share the digits of Xg: reuse them for up
        DracoLayout L;
        draco_layout(cu, inter, n_in, &L);
        GemmArgs a = {};
        const size_t oct = (size_t)R / 8;
        a.xdig = reinterpret_cast<const int8_t*>(dD);
        a.xsc = reinterpret_cast<const float*>(dD + oct * ((size_t)n_in / 32) * 1024);
        a.xs32 = a.xsc + oct * ((size_t)n_in / 256) * 8;
        a.xs16 = a.xs32 + oct * ((size_t)n_in / 32) * 8;
        a.T = R;
        a.n_in = n_in;
        a.L = L;
        a.Y = dU;
        a.ldy = inter;
        a.groups = dgr + na;
        a.n_groups = na;
        a.max_oct = max_oct;
        if (draco_gemm_grouped_launch(a, st)) return fail(-1, "moe_tok up gemm rejected");
    }
    dk_swiglu(dG, dU, R * inter, st);
    if (int rc = grouped(dG, inter, cd, dgr + 2 * na, n_out, dY)) return rc;
    if (draco_moe_scatter_launch(dY, n_out, dpos, dwt, n_used, T, dO, st)) return fail(-1, "moe_tok scatter rejected");
    DRACO_HIP(hipGetLastError());
    DRACO_HIP(hipMemcpyAsync(out, dO, sizeof(float) * fO, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipStreamSynchronize(st));
    return 0;
}

std::map<const void*, MoeLayer*>& moe_layers() {
    static auto* m = new std::map<const void*, MoeLayer*>();
    return *m;
}

// m6_moe_batch4 (src/m6_layer.c:656-690): n given experts, no router --
// out = sum_j wtop[j] * down_j(silu(gate_j x0) * up_j x0) in j order, the
// caller's weights as they are (no renormalisation).  The routed launches
// with the slots fixed by the host: gate/up + SwiGLU over the n slots, then
// the down + weighted combine.
int moe_batch(const float* x0, const uint64_t* ptrs, const int* codes, const float* wtop, int n, int inter,
              int n_in, int n_out, float* out) {
    if (n < 1 || n > MOE_USED_MAX) return fail(-1, "m6_moe_batch4: %d experts (1..%d served)", n, MOE_USED_MAX);
    if (inter % 256 || n_in % 256 || n_out % 16)
        return fail(-1, "m6_moe_batch4: shape inter %d n_in %d n_out %d not served", inter, n_in, n_out);
    const int fg = fm_of(codes[0]), fd = fm_of(codes[2]);
    for (int j = 0; j < n; j++)
        if (codes[3 * j] != codes[0] || codes[3 * j + 1] != codes[0] || codes[3 * j + 2] != codes[2] || !fg || !fd)
            return fail(-1, "m6_moe_batch4: expert formats not served (one of Q4_K / Q6_K per role)");
    if (int rc = ensure_init()) return rc;
    hipStream_t st = stream();
    // device table [gate n][up n][down n] bases, then the n weights, x, act, out
    const size_t tb = sizeof(void*) * 3 * (size_t)n;
    char* d = (char*)scratch(16, tb + sizeof(float) * ((size_t)n + n_in + (size_t)n * inter + n_out) + 256);
    char* h = (char*)pinned(7, tb + sizeof(float) * ((size_t)n + n_in));
    if (!d || !h) return -2;
    const uint8_t** tab = (const uint8_t**)h;
    for (int j = 0; j < n; j++) {
        const DracoMat* g = get_mat((const void*)(uintptr_t)ptrs[3 * j], codes[3 * j], inter, n_in);
        const DracoMat* u = get_mat((const void*)(uintptr_t)ptrs[3 * j + 1], codes[3 * j + 1], inter, n_in);
        const DracoMat* dn = get_mat((const void*)(uintptr_t)ptrs[3 * j + 2], codes[3 * j + 2], n_out, inter);
        if (!g || !u || !dn) return -2;
        tab[j] = g->dev;
        tab[n + j] = u->dev;
        tab[2 * n + j] = dn->dev;
    }
    float* hw = (float*)(h + tb);
    memcpy(hw, wtop, sizeof(float) * n);
    memcpy(hw + n, x0, sizeof(float) * n_in);
    const uint8_t** dtab = (const uint8_t**)d;
    float* dw = (float*)(d + tb);
    float* dx = dw + n;
    float* dact = dx + n_in;
    float* dout = dact + (size_t)n * inter;
    DRACO_HIP(hipMemcpyAsync(d, h, tb + sizeof(float) * ((size_t)n + n_in), hipMemcpyHostToDevice, st));
    MoeArgs a = {};
    a.x = dx;
    a.n_in = n_in;
    a.n_out_e = inter;
    a.n_slots = n;
    a.base0 = dtab;
    a.base1 = dtab + n;
    a.act = dact;
    if (draco_moe_grp_launch(a, fg, true, false, false, st)) return fail(-1, "moe batch gate/up launch rejected");
    a.inter = inter;
    a.n_out = n_out;
    a.out = dout;
    a.resid = nullptr;
    a.seld = dtab + 2 * n;
    a.selw = dw;
    if (draco_moe_down_launch(a, fd, st)) return fail(-1, "moe batch down launch rejected");
    DRACO_HIP(hipGetLastError());
    float* ho = (float*)pinned(8, sizeof(float) * (size_t)n_out);
    if (!ho) return -2;
    DRACO_HIP(hipMemcpyAsync(ho, dout, sizeof(float) * n_out, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipStreamSynchronize(st));
    memcpy(out, ho, sizeof(float) * n_out);
    return 0;
}

}  // namespace

// ---- the MoE FFN of one layer inside the device decode loop --------------
struct MoeLayer {
    DracoMoeP snap;
    ExpertSet* set = nullptr;
    uint64_t epoch = 0;
    MoeWork w = {};
    float* xn = nullptr;
    char* buf = nullptr;  // own allocation behind w (router logits, activations, routing)
};

MoeLayer* draco_moe_layer(const DracoMoeP* p) {
    if (!p) {
        fail(-1, "moe layer: null parameters");
        return nullptr;
    }
    MoeLayer*& slot = moe_layers()[p];
    if (slot && slot->epoch == epoch() && memcmp(&slot->snap, p, sizeof(*p)) == 0) return slot;
    if (check_moe(p->n_exp, p->n_used, p->inter, p->n_in, p->n_out)) return nullptr;
    if (ensure_init()) return nullptr;
    if (!slot) slot = new MoeLayer();
    MoeLayer* m = slot;
    m->set = expert_set(p->ptrs, p->codes, p->gate_inp, p->n_exp, p->inter, p->n_in, p->n_out, stream());
    if (!m->set) return nullptr;
    // own buffers: captured graphs keep these addresses, so nothing shared
    // with the host-pointer entry points (whose scratch can be regrown)
    const size_t bytes = sizeof(float) * ((size_t)p->n_in + 64) + sizeof(void*) * MOE_USED_MAX +
                         sizeof(float) * ((size_t)p->n_exp + (size_t)p->n_used * p->inter + 2 * MOE_USED_MAX) + 256;
    if (m->buf) {
        hipStreamSynchronize(stream());
        hipFree(m->buf);
        m->buf = nullptr;
    }
    if (hipMalloc(&m->buf, bytes) != hipSuccess) {
        fail(-2, "moe layer: work allocation failed");
        return nullptr;
    }
    m->xn = (float*)m->buf;
    char* q = m->buf + sizeof(float) * ((size_t)p->n_in + 64);
    m->w.seld = (const uint8_t**)q;
    m->w.logits = (float*)(q + sizeof(void*) * MOE_USED_MAX);
    m->w.selw = m->w.logits + p->n_exp;
    m->w.sel = (int*)(m->w.selw + MOE_USED_MAX);
    m->w.act = (float*)(m->w.sel + MOE_USED_MAX);
    m->snap = *p;
    m->epoch = m->set->epoch;
    return m;
}

bool draco_moe_layer_pend_ok(const MoeLayer* m, const float* norm_w) { return m->snap.n_in <= 4096 && norm_w; }

bool draco_moe_layer_split_ok(const MoeLayer* m) { return m->snap.n_used % 2 == 0 && m->snap.n_used <= 16; }

int draco_moe_layer_enqueue(MoeLayer* m, const float* x, const float* norm_w, float eps, float* out,
                            const float* resid, hipStream_t st, const float* pend, float* xs, bool pend_fx,
                            float* split_out) {
    const DracoMoeP& p = m->snap;
    if (!draco_moe_layer_pend_ok(m, norm_w)) {  // wider than the router's norm prologue, or no norm weight
        if (pend) return fail(-1, "moe layer: a pending residual needs the router's RMSNorm prologue");
        dk_rmsnorm(x, norm_w, m->xn, p.n_in, eps, st);
        return enqueue_moe(m->set, m->xn, out, resid, m->w, p.n_exp, p.n_used, p.inter, p.n_in, p.n_out, st);
    }
    if (pend && !xs) return fail(-1, "moe layer: a pending residual needs its sum buffer");
    if (split_out && !draco_moe_layer_split_ok(m)) return fail(-1, "moe layer: %d experts cannot split", p.n_used);
    return enqueue_moe(m->set, x, out, resid, m->w, p.n_exp, p.n_used, p.inter, p.n_in, p.n_out, st, norm_w, eps,
                       m->xn, pend, xs, pend_fx, split_out);
}

int draco_moe_layer_enqueue_xn(MoeLayer* m, const float* xn, float* out, const float* resid, hipStream_t st) {
    const DracoMoeP& p = m->snap;
    return enqueue_moe(m->set, xn, out, resid, m->w, p.n_exp, p.n_used, p.inter, p.n_in, p.n_out, st);
}

extern "C" {

// The MoE FFN as an m6 ffn op (no reference counterpart as an op: the
// reference's qwen35 driver calls m6_granite_moe per layer from Python,
// src/qwen35_engine.py:293-307): out[n_out] = m6_granite_moe(xn, ...) with
// the arguments packed in DracoMoeP.  Called directly it runs like
// m6_granite_moe; inside M6LayerDesc it lets m6_forward_token and the device
// decode loop run MoE layers (src/m6_engine.c:61-83 with this op as ffn).
void draco_moe_ffn_op(const float* xn, void* pv, float* out) {
    const DracoMoeP* p = (const DracoMoeP*)pv;
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = granite_moe(xn, p->ptrs, p->codes, p->gate_inp, p->n_exp, p->n_used, p->inter, p->n_in, p->n_out,
                             out)) {
        fprintf(stderr, "draco_moe_ffn_op: rc %d: %s\n", rc, last_error());
        if (out && p->n_out > 0) poison(out, (size_t)p->n_out);
    }
}

// src/m6_layer.c:656-690 (bound by the reference's llama driver at import,
// src/smol_engine.py:81).  scratch is accepted and not used.
void m6_moe_batch4(const float* x0, const uint64_t* ptrs, const int* codes, const float* wtop, int n_exp, int inter,
                   int n_in, int n_out, float* scratch, float* out) {
    (void)scratch;
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = moe_batch(x0, ptrs, codes, wtop, n_exp, inter, n_in, n_out, out)) {
        fprintf(stderr, "m6_moe_batch4: rc %d: %s\n", rc, last_error());
        if (out && n_out > 0) poison(out, (size_t)n_out);  // unserved input: NaN, not stale values
    }
}

typedef int (*draco_dequant_fn)(int, const uint8_t*, int, float*);
typedef int (*draco_gemm_auto_fn)(int, const float*, const uint8_t*, int, int, int, float*);

void m6_moe_tok(draco_dequant_fn DQ, draco_gemm_auto_fn GA, float* gwbuf, const float* X, const int* order,
                const float* wtop, const uint64_t* ep, const int* ec, int T, int n_used, int inter, int n_in,
                int n_out, int n_exp, float* out, float* work, int* iwork) {
    (void)DQ;  // the device path uses its own kernels, not the caller's CPU callbacks
    (void)GA;
    (void)gwbuf;
    (void)work;
    (void)iwork;
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = moe_tok(X, order, wtop, ep, ec, T, n_used, inter, n_in, n_out, n_exp, out)) {
        // void ABI (as the reference): an input this library does not serve
        // (IQ3_S experts, mixed formats, n_used > 16, ...) leaves NaN in out,
        // so the caller's next step cannot silently read stale values
        fprintf(stderr, "m6_moe_tok: rc %d: %s\n", rc, last_error());
        if (out && T > 0 && n_out > 0) poison(out, (size_t)T * n_out);
    }
}


void m6_granite_moe(const float* x0, const uint64_t* ptrs, const int* codes, const float* gate_inp, int n_exp,
                    int n_used, int inter, int n_in, int n_out, float* scratch_unused, float* out) {
    (void)scratch_unused;  // the device path needs no host scratch
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = granite_moe(x0, ptrs, codes, gate_inp, n_exp, n_used, inter, n_in, n_out, out)) {
        fprintf(stderr, "m6_granite_moe: rc %d: %s\n", rc, last_error());
        if (out && n_out > 0) poison(out, (size_t)n_out);  // unserved input: NaN, not stale values
    }
}

int m5_gemvn_q4k(const float* x, long x_stride, const uint8_t* W, const int* idx, long per, int n_out_e,
                 int n_in, int n_exp, float* y) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    return gemvn(DRACO_Q4_K, x, x_stride, W, idx, per, n_out_e, n_in, n_exp, y);
}

int m5_gemvn_q6k(const float* x, long x_stride, const uint8_t* W, const int* idx, long per, int n_out_e,
                 int n_in, int n_exp, float* y) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    return gemvn(DRACO_Q6_K, x, x_stride, W, idx, per, n_out_e, n_in, n_exp, y);
}

// Same inputs as m6_granite_moe; returns 0 and out[0] = us per MoE FFN
// (router + routed gate/up + down/combine) from a graph replay of `iters`
// FFNs on the device (x fixed), out[1] = the routed experts' weight bytes per
// FFN + router bytes.
int draco_bench_granite_moe(const float* x0, const uint64_t* ptrs, const int* codes, const float* gate_inp,
                            int n_exp, int n_used, int inter, int n_in, int n_out, int iters, float* out) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = check_moe(n_exp, n_used, inter, n_in, n_out)) return rc;
    if (int rc = ensure_init()) return rc;
    hipStream_t st = stream();
    ExpertSet* s = expert_set(ptrs, codes, gate_inp, n_exp, inter, n_in, n_out, st);
    if (!s) return -2;
    MoeWork w;
    if (moe_work(w, n_in, n_exp, n_used, inter, n_out)) return -2;
    DRACO_HIP(hipMemcpyAsync(w.x, x0, sizeof(float) * (size_t)n_in, hipMemcpyHostToDevice, st));
    if (int rc = enqueue_moe(s, w.x, w.out, nullptr, w, n_exp, n_used, inter, n_in, n_out, st)) return rc;
    DRACO_HIP(hipStreamSynchronize(st));
    hipGraph_t graph;
    hipGraphExec_t exec;
    DRACO_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
    for (int i = 0; i < iters; i++) enqueue_moe(s, w.x, w.out, nullptr, w, n_exp, n_used, inter, n_in, n_out, st);
    DRACO_HIP(hipStreamEndCapture(st, &graph));
    DRACO_HIP(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    DRACO_HIP(hipGraphLaunch(exec, st));
    hipEvent_t e0, e1;
    DRACO_HIP(hipEventCreate(&e0));
    DRACO_HIP(hipEventCreate(&e1));
    DRACO_HIP(hipEventRecord(e0, st));
    DRACO_HIP(hipGraphLaunch(exec, st));
    DRACO_HIP(hipEventRecord(e1, st));
    DRACO_HIP(hipStreamSynchronize(st));
    float ms = 0;
    DRACO_HIP(hipEventElapsedTime(&ms, e0, e1));
    out[0] = ms * 1000.f / iters;
    const double gu = (double)draco_row_bytes(codes[0], n_in) * inter * 2;
    const double dn = (double)draco_row_bytes(codes[2], inter) * n_out;
    out[1] = (float)(n_used * (gu + dn) + 4.0 * n_exp * n_in);
    hipGraphExecDestroy(exec);
    hipGraphDestroy(graph);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    return 0;
}

}  // extern "C"
