// abi_gemm.cpp -- prefill GEMM entry points.
//
// m5_gemm_auto: src/m5/m5_gemm_fused.c:231-241 (0 = done, -1 = code not served,
// the caller falls back); m5_gemm: src/m5/m5_gemm.c:249-272 (Y[T x n_out] =
// X[T x n_in] . W^T).  Host pointers.  Q4_K / Q6_K run on the f16-MFMA GEMM
// (gemmh.hip); Q8_0 and Q5_K run as one device GEMV per token.  The int8-MFMA kernels
// of gemm.hip serve the grouped expert GEMMs of m6_moe_tok only.
// m5_dequant_row: src/m5/m5_gemm.c:55-235, the GEMM library's row decoder.
#include <stdio.h>
#include <string.h>

#include <vector>

#include "decode.h"
#include "gemm.h"
#include "runtime.h"

extern "C" int draco_repack(int code, const uint8_t* src, int n_out, int n_in, uint8_t* dst);

using namespace draco;

int draco_enqueue_gemm(const DracoMat& m, const float* X, int T, float* Y, uint8_t* digits, bool have_digits,
                       hipStream_t st) {
    if (m.L.code != DRACO_Q4_K && m.L.code != DRACO_Q6_K) {  // Q8_0 and the plain formats: one GEMV per token
        for (int t = 0; t < T; t++)
            if (draco_gemv_launch(m, X + (size_t)t * m.L.n_in, Y + (size_t)t * m.L.n_out, nullptr, 0, m.L.n_out, st))
                return fail(-1, "gemm: gemv launch rejected");
        return 0;
    }
    if (!have_digits && draco_gemmh_x_launch(X, T, m.L.n_in, digits, st))
        return fail(-1, "gemm: activation launch rejected");
    GemmHArgs a = {};
    a.W = m.dev;
    a.L = m.L;
    a.n_in = m.L.n_in;
    a.T = T;
    a.xh = digits;
    a.Y = Y;
    a.ldy = m.L.n_out;
    const size_t pf = draco_gemmh_part_floats(m.L, T, a.ldy);
    if (pf) {
        // grow-only; callers that capture graphs enqueue once before capturing
        a.part = (float*)scratch(12, sizeof(float) * pf);
        if (!a.part) return -2;
    }
    if (draco_gemmh_launch(a, st)) return fail(-1, "gemm: launch rejected");
    return 0;
}

namespace {

bool served(int code) {
    return code == DRACO_Q4_K || code == DRACO_Q6_K || code == DRACO_Q8_0 || code == DRACO_Q5_K;
}

int enqueue_gemm(const DracoMat& m, const float* X, int T, float* Y, uint8_t* digits, hipStream_t st) {
    return draco_enqueue_gemm(m, X, T, Y, digits, false, st);
}

int gemm_host(int code, const float* X, const uint8_t* W, int T, int n_out, int n_in, float* Y) {
    if (!served(code)) return -1;
    if (T < 0 || n_out <= 0 || n_in <= 0 || n_in % draco_block_values(code))
        return fail(-1, "m5_gemm: bad shape T=%d %dx%d", T, n_out, n_in);
    if (T == 0) return 0;
    if (int rc = ensure_init()) return rc;
    const DracoMat* m = get_mat(W, code, n_out, n_in);
    if (!m) return -2;
    hipStream_t st = stream();
    float* dx = (float*)scratch(0, sizeof(float) * (size_t)T * n_in);
    float* dy = (float*)scratch(1, sizeof(float) * (size_t)T * n_out);
    uint8_t* dd = code == DRACO_Q8_0 ? nullptr : (uint8_t*)scratch(7, draco_gemm_digit_bytes(T, n_in));
    if (!dx || !dy || (code != DRACO_Q8_0 && !dd)) return -2;
    DRACO_HIP(hipMemcpyAsync(dx, X, sizeof(float) * (size_t)T * n_in, hipMemcpyHostToDevice, st));
    if (int rc = enqueue_gemm(*m, dx, T, dy, dd, st)) return rc;
    DRACO_HIP(hipGetLastError());
    DRACO_HIP(hipMemcpyAsync(Y, dy, sizeof(float) * (size_t)T * n_out, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipStreamSynchronize(st));
    return 0;
}

// the void fused-GEMM entries' body (below)
void gemm_void(const char* name, int code, const float* X, const uint8_t* W, int c, int n_out, int n_in, float* Y) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    int rc = served(code) ? gemm_host(code, X, W, c, n_out, n_in, Y)
                          : fail(-1, "%s: format code %d is not carried by this library", name, code);
    if (rc) {
        fprintf(stderr, "%s: rc %d: %s\n", name, rc, last_error());
        if (Y && c > 0 && n_out > 0) poison(Y, (size_t)c * n_out);
    }
}
}  // namespace

extern "C" {

int m5_gemm_auto(int code, const float* X, const uint8_t* W, int c, int n_out, int n_in, float* Y) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    return gemm_host(code, X, W, c, n_out, n_in, Y);
}

int m5_gemm(int code, const float* X, const uint8_t* W, int T, int n_out, int n_in, float* Y, float* wbuf) {
    (void)wbuf;  // the device path needs no host row buffer
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    return gemm_host(code, X, W, T, n_out, n_in, Y);
}

// The per-format fused GEMM entries (the FUSED3 instances and m5_gemm_iq3s,
// src/m5/m5_gemm_fused.c:78,211-228), Y[c x n_out] = X[c x n_in] . W^T.  The
// reference's prefill driver looks all six up when it starts and calls them
// by format instead of m5_gemm_auto (src/qwen35_prefill.py:76-80,100-104).
// They return nothing, as the reference's: a format this library does not
// carry (IQ4_XS, IQ3_S) or a failed call leaves NaN in Y and the error on
// stderr, never stale values.

void m5_gemm_q80(const float* X, const uint8_t* W, int c, int n_out, int n_in, float* Y) {
    gemm_void("m5_gemm_q80", DRACO_Q8_0, X, W, c, n_out, n_in, Y);
}
void m5_gemm_q6k(const float* X, const uint8_t* W, int c, int n_out, int n_in, float* Y) {
    gemm_void("m5_gemm_q6k", DRACO_Q6_K, X, W, c, n_out, n_in, Y);
}
void m5_gemm_q5k(const float* X, const uint8_t* W, int c, int n_out, int n_in, float* Y) {
    gemm_void("m5_gemm_q5k", DRACO_Q5_K, X, W, c, n_out, n_in, Y);
}
void m5_gemm_q4k(const float* X, const uint8_t* W, int c, int n_out, int n_in, float* Y) {
    gemm_void("m5_gemm_q4k", DRACO_Q4_K, X, W, c, n_out, n_in, Y);
}
void m5_gemm_iq4xs(const float* X, const uint8_t* W, int c, int n_out, int n_in, float* Y) {
    gemm_void("m5_gemm_iq4xs", 6, X, W, c, n_out, n_in, Y);
}
void m5_gemm_iq3s(const float* X, const uint8_t* W, int c, int n_out, int n_in, float* Y) {
    gemm_void("m5_gemm_iq3s", 2, X, W, c, n_out, n_in, Y);
}

// src/m5/m5_gemm.c:55-235: one GGUF row -> out[n_in] fp32 (0 done, -1 code
// not served).  Served: Q8_0, Q4_K, Q5_K, Q6_K, F16 (the reference also
// serves the IQ formats, which no path here carries).  The row is decoded
// on the device by the embedding decoder: from the resident copy when the
// row lies inside a registered matrix, else from the row's own bytes put in
// the private layout.
int m5_dequant_row(int code, const uint8_t* row, int n_in, float* out) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (code != DRACO_Q8_0 && code != DRACO_Q4_K && code != DRACO_Q5_K && code != DRACO_Q6_K && code != DRACO_F16)
        return -1;
    if (!row || !out || n_in <= 0 || n_in % draco_block_values(code)) {
        fail(-1, "m5_dequant_row: n_in %d is not a whole number of blocks", n_in);
        return -1;
    }
    if (ensure_init()) return -1;
    hipStream_t st = stream();
    int r = 0;
    DracoMat m;
    if (const DracoMat* rm = find_row(row, code, n_in, &r)) {
        m = *rm;
    } else {
        if (draco_layout(code, 1, n_in, &m.L)) return fail(-1, "m5_dequant_row: no layout for n_in %d", n_in);
        uint8_t* stage = (uint8_t*)pinned(0, m.L.bytes);
        m.dev = (uint8_t*)scratch(30, m.L.bytes);
        if (!stage || !m.dev) return -1;
        memset(stage, 0, m.L.bytes);
        draco_repack(code, row, 1, n_in, stage);
        if (hipMemcpyAsync(m.dev, stage, m.L.bytes, hipMemcpyHostToDevice, st) != hipSuccess)
            return fail(-1, "m5_dequant_row: upload failed");
    }
    int* ids = (int*)scratch(31, sizeof(float) * ((size_t)n_in + 64));
    float* hp = (float*)pinned(6, sizeof(float) * ((size_t)n_in + 64));
    if (!ids || !hp) return -1;
    float* dout = (float*)(ids + 64);
    *(int*)hp = r;
    if (hipMemcpyAsync(ids, hp, sizeof(int), hipMemcpyHostToDevice, st) != hipSuccess)
        return fail(-1, "m5_dequant_row: upload failed");
    dk_embed(m, ids, nullptr, dout, st);
    if (hipMemcpyAsync(hp, dout, sizeof(float) * n_in, hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return fail(-1, "m5_dequant_row: decode failed");
    memcpy(out, hp, sizeof(float) * n_in);
    return 0;
}

// Graph-replayed timing of the prefill GEMM on `n_copies` weight copies:
// out[0] us per GEMM including the activation digitization, out[1] us per
// GEMM kernel alone (digits computed once).
int draco_bench_gemm(int code, const uint8_t* W, int n_out, int n_in, int T, int n_copies, int iters, float* out) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (code != DRACO_Q4_K && code != DRACO_Q6_K) return fail(-1, "bench gemm: code %d not on the MFMA path", code);
    if (int rc = ensure_init()) return rc;
    DracoLayout L;
    if (draco_layout(code, n_out, n_in, &L) || T < 1) return fail(-1, "bench gemm: bad shape");
    if (n_copies < 1) n_copies = 1;
    std::vector<uint8_t> host(L.bytes, 0);
    draco_repack(code, W, n_out, n_in, host.data());
    std::vector<DracoMat> mats(n_copies);
    for (auto& m : mats) {
        m.L = L;
        DRACO_HIP(hipMalloc(&m.dev, L.bytes));
        DRACO_HIP(hipMemcpy(m.dev, host.data(), L.bytes, hipMemcpyHostToDevice));
    }
    std::vector<float> xh((size_t)T * n_in);
    for (size_t i = 0; i < xh.size(); i++) xh[i] = (float)((int)((i * 2654435761u) % 2001) - 1000) * 1e-3f;
    float *dx, *dy;
    uint8_t* dd;
    DRACO_HIP(hipMalloc(&dx, sizeof(float) * xh.size()));
    DRACO_HIP(hipMalloc(&dy, sizeof(float) * (size_t)T * n_out));
    DRACO_HIP(hipMalloc(&dd, draco_gemm_digit_bytes(T, n_in)));
    DRACO_HIP(hipMemcpy(dx, xh.data(), sizeof(float) * xh.size(), hipMemcpyHostToDevice));
    hipStream_t st = stream();
    // one eager product first: it sizes the K-split scratch outside the capture
    if (enqueue_gemm(mats[0], dx, T, dy, dd, st)) return -1;
    DRACO_HIP(hipStreamSynchronize(st));
    float* part = (float*)scratch(12, sizeof(float) * (draco_gemmh_part_floats(L, T, n_out) + 1));
    if (!part) return -2;
    hipEvent_t e0, e1;
    DRACO_HIP(hipEventCreate(&e0));
    DRACO_HIP(hipEventCreate(&e1));
    for (int mode = 0; mode < 2; mode++) {
        hipGraph_t graph;
        hipGraphExec_t exec;
        DRACO_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
        for (int i = 0; i < iters; i++) {
            if (mode == 0) {
                enqueue_gemm(mats[i % n_copies], dx, T, dy, dd, st);
            } else {
                GemmHArgs b = {};
                b.W = mats[i % n_copies].dev;
                b.L = L;
                b.n_in = n_in;
                b.T = T;
                b.xh = dd;
                b.Y = dy;
                b.ldy = n_out;
                b.part = part;
                draco_gemmh_launch(b, st);
            }
        }
        DRACO_HIP(hipStreamEndCapture(st, &graph));
        DRACO_HIP(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
        DRACO_HIP(hipGraphLaunch(exec, st));
        DRACO_HIP(hipEventRecord(e0, st));
        DRACO_HIP(hipGraphLaunch(exec, st));
        DRACO_HIP(hipEventRecord(e1, st));
        DRACO_HIP(hipStreamSynchronize(st));
        float ms = 0;
        DRACO_HIP(hipEventElapsedTime(&ms, e0, e1));
        out[mode] = ms * 1000.f / iters;
        hipGraphExecDestroy(exec);
        hipGraphDestroy(graph);
    }
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    for (auto& m : mats) hipFree(m.dev);
    hipFree(dx);
    hipFree(dy);
    hipFree(dd);
    return 0;
}

}  // extern "C"
