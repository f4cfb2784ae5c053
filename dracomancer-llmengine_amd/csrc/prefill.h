// prefill.h -- launchers of the chunked-prefill kernels (prefill.hip).
// All pointers are device pointers; rows are token-major ([T][width]).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "formats.h"

// key splits of the chunk attention and the partial buffer it needs (floats)
int pf_attn_nsplit(int row0, int T);
size_t pf_part_floats(int NH, int T, int HD, int nspl);

// X[t] = embedding row ids[t] (private layout of an embedding matrix)
int pf_embed(const uint8_t* base, const DracoLayout& L, const int* ids, int T, float* X, hipStream_t st);
// Xn[t] = (X[t] * inv_rms) * w, h <= 4096
int pf_rms(const float* X, const float* w, float* Xn, int T, int h, float eps, hipStream_t st);
// X[t] += Y[t], then Xn[t] = (X[t] * inv_rms) * w (h <= 4096)
int pf_add_rms(float* X, const float* Y, const float* w, float* Xn, int T, int h, float eps, hipStream_t st);
// rope of Q[t] / K[t] at position pos0 + t; K, V rows into cache row row0 + t
int pf_rope_append(float* Q, const float* K, const float* V, float* kc, float* vc, const float* tab, int pos0,
                   int row0, int T, int NH, int NKV, int HD, int rot, hipStream_t st);
// O[t] = causal attention of query row row0 + t over cache rows [0, row0 + t]
// (the shapes pf_attention_ok accepts); part holds pf_part_floats(...) floats
static inline bool pf_attention_ok(int NH, int NKV, int HD) {
    return NKV >= 1 && NH % NKV == 0 && NH / NKV <= 8 && (HD == 64 || HD == 128);
}
int pf_attention(const float* Q, const float* kc, const float* vc, float* part, float* O, int row0, int T, int NH,
                 int NKV, int HD, float scale, hipStream_t st);
// The same at head dim 256 (NH / NKV <= 16) with the qwen35 output gate:
// O[t][h*256 + d] = attention * sigmoid(gate[t * g_row + h * g_head + d])
int pf_attention256(const float* Q, const float* kc, const float* vc, float* part, float* O, int row0, int T, int NH,
                    int NKV, float scale, const float* gate, int g_row, int g_head, hipStream_t st);
// GDN gates of T tokens: B[t][e] = sigmoid(Xn[t] . bw[e]), G[t][e] =
// exp(softplus(Xn[t] . aw[e] + dt[e]) * sa[e]); bw / aw [n_vh][H]
int pf_gdn_gates(const float* Xn, int T, int H, const float* bw, const float* aw, const float* dt, const float* sa,
                 float* B, float* G, int n_vh, hipStream_t st);
// X += Y over n floats
int pf_add(float* X, const float* Y, size_t n, hipStream_t st);
