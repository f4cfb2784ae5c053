// decode.h -- launchers of the decode-token kernels (decode.hip).
#pragma once
#include <hip/hip_runtime.h>

#include "gemv.h"

constexpr int ARGMAX_BLOCKS = 256;

// The group-shared attention kernel serves GQA groups of rep = NH / NKV q
// heads with rep a power of two in [2, 8] at HD 128 and in [2, 16] at HD 256;
// the per-head kernel serves HD in {64, 128, 256} with rep up to 16; every
// other shape (any head dim up to 512, any rep) runs the generic kernel.  (At
// HD 64 the per-head kernel is faster on MI355X: its rows are 256 bytes, so
// the re-read K / V rows stay in L2 and the per-row lane-exchange cost of the
// grouped kernel dominates.)
static inline bool attn_grouped(int NH, int NKV, int HD) {
    if (NKV < 1 || NH % NKV) return false;
    const int rep = NH / NKV;
    if (rep < 2 || (rep & (rep - 1))) return false;
    return (HD == 128 && rep <= 8) || (HD == 256 && rep <= 16);
}
static inline bool attn_per_head(int NH, int NKV, int HD) {
    return NKV >= 1 && NH % NKV == 0 && NH / NKV <= 16 && (HD == 64 || HD == 128 || HD == 256);
}

// Number of T-splits of the decode attention for a cache of max_t rows.
// Grouped kernel: about 32 rows per split at full length and at most ~512
// blocks (NKV * nsplit), at most 256 splits.  Per-head kernel: about 32 rows
// per split, at most 64 splits.  The split count is fixed by max_t so that a
// captured decode step serves every cache length.
static inline int attn_nsplit(int max_t, int NH, int NKV, int HD) {
    int n = (max_t + 31) / 32;
    if (attn_grouped(NH, NKV, HD)) {
        const int cap = (512 + NKV - 1) / NKV;
        n = n < cap ? n : cap;
        return n < 1 ? 1 : (n > 256 ? 256 : n);
    }
    return n < 1 ? 1 : (n > 64 ? 64 : n);
}

void dk_rmsnorm(const float* x, const float* w, float* out, int h, float eps, hipStream_t st);
void dk_rope_append(float* q, const float* k, const float* v, float* kc, float* vc, const float* tab,
                    const int* state, int layer, int NH, int NKV, int HD, int rot, hipStream_t st);
// split-T partials + merge; `count` is unused (kept for the caller's buffer plumbing)
// Any NH divisible by NKV and any even HD up to 512.  gate (nullable):
// out[h][d] *= sigmoid(gate[h * gstride + d]).
int dk_attention(const float* q, const float* kc, const float* vc, float* part, unsigned* count, float* out,
                 const int* state, int layer, int NH, int NKV, int HD, int max_t, float scale, hipStream_t st,
                 const float* gate = nullptr, int gstride = 0);
// The split partials only (the grouped or per-head kernel dk_attention would
// run, without the merge); -1 for the shapes only the generic kernel serves.
// part as dk_attention.
int dk_attention_parts(const float* q, const float* kc, const float* vc, float* part, const int* state, int layer,
                       int NH, int NKV, int HD, int max_t, float scale, hipStream_t st);
// Their merge fused with the o projection wo (n_in = NH * 64; Q4_K / Q6_K:
// one 256-wide input chunk per 4 heads; Q8_0: one chunk per kv group of
// NH / NKV <= 4 heads): acc[row] += round(2^32 * wo . att) over the chunks
// (int64 fixed point; acc must start at zero), acc[n_out] set when a
// contribution is not finite; zacc[0 .. zn) is cleared.  -1 for another
// shape.
// Short caches: the whole attention of every kv group fused with the Q8_0 o
// projection (head dim 64, NH / NKV <= 4), for caches of at most tcap <= 128
// rows (tcap also bounds the rows read: the call's longest cache); acc as
// dk_attn_o.  -1 for another shape.
constexpr int DK_ATT_SHORT_T = 128;
int dk_attn_o8_short(const float* q, const float* kc, const float* vc, const int* state, int layer, int NH, int NKV,
                     int HD, float scale, int tcap, const DracoMat& wo, unsigned long long* acc,
                     unsigned long long* zacc, int zn, hipStream_t st);
int dk_attn_o(const float* part, int NH, int NKV, int HD, int max_t, const DracoMat& wo, unsigned long long* acc,
              unsigned long long* zacc, int zn, hipStream_t st);
// qwen35 full attention q/k head RMSNorm + rope (NH q heads, 2 k heads of 256).
void dk_fa_prep(const float* QG, float* Qr, const float* kin, float* kout, const float* qn, const float* kn,
                const float* cs, int NH, hipStream_t st);
// The same for T tokens at positions (state ? state[0] : pos0) + t, K / V rows
// into cache rows (state ? state[1] : row0) + t (kc / vc rows of 2 x 256);
// QG rows qg_stride apart, kin / vin rows of 512, cs_tab [position][64].
void dk_fa_prep_rows(const float* QG, int qg_stride, float* Qr, const float* kin, const float* vin, float* kc,
                     float* vc, const float* qn, const float* kn, const float* cs_tab, const int* state, int pos0,
                     int row0, int NH, int T, hipStream_t st);
void dk_swiglu(float* g, const float* u, int n, hipStream_t st);
// out[i] = y[i] * sigmoid(g[0]) (n floats; g is one device float)
void dk_sigmoid_scale(const float* y, const float* g, float* out, int n, hipStream_t st);
// out[i] = y[i] * sigmoid(x . g) for a one-row F32 / F16 matrix g of n values
// (n % 4 == 0), gdot[0] = x . g; -1 for any other g
int dk_gate_scale(const float* x, const DracoMat& g, const float* y, float* out, float* gdot, int n, hipStream_t st);
// out[n_in] = dequantized row ids[cursor ? *cursor : 0] of m
void dk_embed(const DracoMat& m, const int* ids, const int* cursor, float* out, hipStream_t st);
// out[slotp ? *slotp + 1 : slot] = first index of max(x[0..n))
void dk_argmax(const float* x, int n, float* pv, int* pi, int* out, const int* slotp, int slot, hipStream_t st);
void dk_advance(int* state, int n_layer, int* tok_cursor, hipStream_t st);
void dk_pick_token(const int* ids, const int* cursor, int* cur, hipStream_t st);
