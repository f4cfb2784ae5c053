// abi_q8k.cpp -- Q8_K activations and the Q4_K / Q6_K x Q8_K GEMV.
//
// No reference counterpart: the reference has no Q8_K path (its nearest
// analogue is the Q8_0 x Q8_0 int8 dot of tests/i8dot_bench.c:63-183).  The
// block format and rounding follow llama.cpp b10819 quantize_row_q8_K_ref as
// restated by the oracle (oracle/draco_oracle.c or_quantize_q8k,
// or_q8k_block_isums, or_gemv_q8k).  Pointers are caller-owned HOST pointers
// (weights are registered and kept resident like m5_gemv's); results are
// valid when the call returns.  0 = ok, -1 = unsupported code or shape,
// -2 = device error (draco_last_error()).
#include <string.h>

#include <vector>

#include "q8k.h"
#include "runtime.h"

extern "C" int draco_repack(int code, const uint8_t* src, int n_out, int n_in, uint8_t* dst);

using namespace draco;

namespace {

int check_shape(int code, int n_out, int n_in, int nvec) {
    if (code != DRACO_Q4_K && code != DRACO_Q6_K) return fail(-1, "q8k gemv: unsupported format code %d", code);
    if (n_out <= 0 || n_in <= 0 || n_in % 256) return fail(-1, "q8k gemv: bad shape %dx%d", n_out, n_in);
    if (nvec != 1 && nvec != 4 && nvec != 8) return fail(-1, "q8k gemv: nvec %d not in {1, 4, 8}", nvec);
    return 0;
}

size_t q8k_bytes(int n, int nvec) { return (size_t)nvec * (n / 256) * Q8K_BLOCK_BYTES; }

}  // namespace

extern "C" {

// out = Q8_K blocks of nvec vectors of n floats (vector-major).
int draco_q8k_quantize(const float* x, int n, int nvec, uint8_t* out) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (n <= 0 || n % 256 || nvec < 1) return fail(-1, "q8k quantize: bad shape n=%d nvec=%d", n, nvec);
    if (int rc = ensure_init()) return rc;
    float* dx = (float*)scratch(0, sizeof(float) * (size_t)n * nvec);
    uint8_t* dq = (uint8_t*)scratch(2, q8k_bytes(n, nvec));
    if (!dx || !dq) return -2;
    hipStream_t st = stream();
    DRACO_HIP(hipMemcpyAsync(dx, x, sizeof(float) * (size_t)n * nvec, hipMemcpyHostToDevice, st));
    if (draco_q8k_quantize_launch(dx, n, nvec, dq, st)) return fail(-1, "q8k quantize launch rejected");
    DRACO_HIP(hipGetLastError());
    DRACO_HIP(hipMemcpyAsync(out, dq, q8k_bytes(n, nvec), hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipStreamSynchronize(st));
    return 0;
}

// y[v * n_out + r] = W[r,:] . dequant(xq[v]) for v < nvec (xq: Q8_K blocks).
int draco_gemv_q8k(int code, const uint8_t* xq, int nvec, const uint8_t* W, int n_out, int n_in, float* y) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = check_shape(code, n_out, n_in, nvec)) return rc;
    if (int rc = ensure_init()) return rc;
    const DracoMat* m = get_mat(W, code, n_out, n_in);
    if (!m) return -2;
    uint8_t* dq = (uint8_t*)scratch(2, q8k_bytes(n_in, nvec));
    float* dy = (float*)scratch(1, sizeof(float) * (size_t)n_out * nvec);
    if (!dq || !dy) return -2;
    hipStream_t st = stream();
    DRACO_HIP(hipMemcpyAsync(dq, xq, q8k_bytes(n_in, nvec), hipMemcpyHostToDevice, st));
    Q8Launch a = {};
    a.base = m->dev;
    a.L = m->L;
    a.n_in = n_in;
    a.xq = dq;
    a.y = dy;
    a.y_stride = n_out;
    if (draco_gemv_q8k_launch(a, nvec, false, st)) return fail(-1, "q8k gemv launch rejected");
    DRACO_HIP(hipGetLastError());
    DRACO_HIP(hipMemcpyAsync(y, dy, sizeof(float) * (size_t)n_out * nvec, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipStreamSynchronize(st));
    return 0;
}

// fp32 activations quantized on the device, then the Q8_K GEMV.
int draco_gemv_q8k_f32(int code, const float* x, int nvec, const uint8_t* W, int n_out, int n_in, float* y) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = check_shape(code, n_out, n_in, nvec)) return rc;
    if (int rc = ensure_init()) return rc;
    const DracoMat* m = get_mat(W, code, n_out, n_in);
    if (!m) return -2;
    float* dx = (float*)scratch(0, sizeof(float) * (size_t)n_in * nvec);
    uint8_t* dq = (uint8_t*)scratch(2, q8k_bytes(n_in, nvec) + Q8K_IMAGE_PAD);
    float* dy = (float*)scratch(1, sizeof(float) * (size_t)n_out * nvec);
    if (!dx || !dq || !dy) return -2;
    hipStream_t st = stream();
    DRACO_HIP(hipMemcpyAsync(dx, x, sizeof(float) * (size_t)n_in * nvec, hipMemcpyHostToDevice, st));
    Q8Launch a = {};
    a.base = m->dev;
    a.L = m->L;
    a.n_in = n_in;
    if (nvec == 1 && draco_gemv_q8k_fused_ok(code, n_in)) {
        a.xf = dx;  // one vector: the GEMV launch quantizes it itself
    } else {
        // the quantizer writes the GEMV's image of the blocks (same values)
        if (draco_q8k_quantize_launch(dx, n_in, nvec, dq, st, true)) return fail(-1, "q8k quantize launch rejected");
        a.xq = dq;
        a.img = true;
    }
    a.y = dy;
    a.y_stride = n_out;
    if (draco_gemv_q8k_launch(a, nvec, false, st)) return fail(-1, "q8k gemv launch rejected");
    DRACO_HIP(hipGetLastError());
    DRACO_HIP(hipMemcpyAsync(y, dy, sizeof(float) * (size_t)n_out * nvec, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipStreamSynchronize(st));
    return 0;
}

// Integer super-block sums of the Q8_K GEMV, as computed by the GPU kernel:
// isc[r * nb + b], imn[r * nb + b] (nb = n_in / 256), one activation vector.
int draco_q8k_isums(int code, const uint8_t* xq, const uint8_t* W, int n_out, int n_in, int32_t* isc,
                    int32_t* imn) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = check_shape(code, n_out, n_in, 1)) return rc;
    if (int rc = ensure_init()) return rc;
    const DracoMat* m = get_mat(W, code, n_out, n_in);
    if (!m) return -2;
    const size_t ni = (size_t)n_out * (n_in / 256);
    uint8_t* dq = (uint8_t*)scratch(2, q8k_bytes(n_in, 1));
    float* dy = (float*)scratch(1, sizeof(float) * (size_t)n_out);
    int32_t* di = (int32_t*)scratch(3, sizeof(int32_t) * ni * 2);
    if (!dq || !dy || !di) return -2;
    hipStream_t st = stream();
    DRACO_HIP(hipMemcpyAsync(dq, xq, q8k_bytes(n_in, 1), hipMemcpyHostToDevice, st));
    Q8Launch a = {};
    a.base = m->dev;
    a.L = m->L;
    a.n_in = n_in;
    a.xq = dq;
    a.y = dy;
    a.y_stride = n_out;
    a.isc = di;
    a.imn = di + ni;
    if (draco_gemv_q8k_launch(a, 1, true, st)) return fail(-1, "q8k isums launch rejected");
    DRACO_HIP(hipGetLastError());
    DRACO_HIP(hipMemcpyAsync(isc, di, sizeof(int32_t) * ni, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipMemcpyAsync(imn, di + ni, sizeof(int32_t) * ni, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipStreamSynchronize(st));
    return 0;
}

// Timing of the Q8_K GEMV on `n_copies` rotating weight copies, activations
// (nvec vectors, fixed pseudo-random fp32) quantized on the device once per
// launch pair.  Each figure is one HIP event pair around a graph replay of
// `iters` launches:
//   out[0] us per GEMV launch (activations quantized once, outside the replay)
//   out[1] us per (quantize + GEMV) pair
int draco_bench_gemv_q8k(int code, const uint8_t* W, int n_out, int n_in, int nvec, int n_copies, int iters,
                         float* out) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = check_shape(code, n_out, n_in, nvec)) return rc;
    if (int rc = ensure_init()) return rc;
    DracoLayout L;
    if (draco_layout(code, n_out, n_in, &L)) return fail(-1, "bench: bad shape");
    if (n_copies < 1) n_copies = 1;
    std::vector<uint8_t> host(L.bytes, 0);
    draco_repack(code, W, n_out, n_in, host.data());
    std::vector<uint8_t*> dev(n_copies, nullptr);
    for (auto& p : dev) {
        DRACO_HIP(hipMalloc(&p, L.bytes));
        DRACO_HIP(hipMemcpy(p, host.data(), L.bytes, hipMemcpyHostToDevice));
    }
    std::vector<float> xh((size_t)n_in * nvec);
    for (size_t i = 0; i < xh.size(); i++) xh[i] = (float)((int)((i * 2654435761u) % 2001) - 1000) * 1e-3f;
    float *dx, *dy;
    uint8_t* dq;
    DRACO_HIP(hipMalloc(&dx, sizeof(float) * xh.size()));
    DRACO_HIP(hipMalloc(&dy, sizeof(float) * (size_t)n_out * nvec));
    DRACO_HIP(hipMalloc(&dq, q8k_bytes(n_in, nvec) + Q8K_IMAGE_PAD));
    DRACO_HIP(hipMemcpy(dx, xh.data(), sizeof(float) * xh.size(), hipMemcpyHostToDevice));
    hipStream_t st = stream();
    auto gemv = [&](int i) {  // as draco_gemv_q8k_f32: the quantizer's GEMV image
        Q8Launch a = {};
        a.base = dev[i % n_copies];
        a.L = L;
        a.n_in = n_in;
        a.xq = dq;
        a.img = true;
        a.y = dy;
        a.y_stride = n_out;
        return draco_gemv_q8k_launch(a, nvec, false, st);
    };
    if (draco_q8k_quantize_launch(dx, n_in, nvec, dq, st, true)) return fail(-1, "bench: quantize rejected");
    for (int i = 0; i < n_copies; i++)
        if (gemv(i)) return fail(-1, "bench: gemv rejected");
    DRACO_HIP(hipStreamSynchronize(st));
    hipEvent_t e0, e1;
    DRACO_HIP(hipEventCreate(&e0));
    DRACO_HIP(hipEventCreate(&e1));
    auto gemv_fx = [&](int i) {  // as draco_gemv_q8k_f32 at nvec 1: the GEMV quantizes x itself
        Q8Launch a = {};
        a.base = dev[i % n_copies];
        a.L = L;
        a.n_in = n_in;
        a.xf = dx;
        a.y = dy;
        a.y_stride = n_out;
        return draco_gemv_q8k_launch(a, 1, false, st);
    };
    out[2] = 0.f;
    const bool fx = nvec == 1 && draco_gemv_q8k_fused_ok(code, n_in);
    for (int mode = 0; mode < (fx ? 3 : 2); mode++) {
        hipGraph_t graph;
        hipGraphExec_t exec;
        DRACO_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
        for (int i = 0; i < iters; i++) {
            if (mode == 1) draco_q8k_quantize_launch(dx, n_in, nvec, dq, st, true);
            if (mode == 2) gemv_fx(i);
            else gemv(i);
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
    for (auto p : dev) hipFree(p);
    hipFree(dx);
    hipFree(dy);
    hipFree(dq);
    return 0;
}

}  // extern "C"
