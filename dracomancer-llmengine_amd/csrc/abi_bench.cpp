// abi_bench.cpp -- device-resident timing entry points (no reference
// counterpart; the reference times its kernels from Python,
// tests/gemv_callcost.py:103-161).
//
// draco_bench_gemv uploads `n_copies` copies of one weight matrix at distinct
// device addresses and rotates through them, so a working set larger than the
// 256 MB Infinity Cache (MALL) forces every launch to stream from HBM.
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "runtime.h"

extern "C" int draco_repack(int code, const uint8_t* src, int n_out, int n_in, uint8_t* dst);

using namespace draco;

extern "C" {

// out[0] mean us per launch from per-launch event pairs
// out[1] us per launch from one event pair around the whole loop
// out[2] min us, out[3] median us (per-launch pairs)
// out[4] us per launch of the same `iters` launches captured in a HIP graph
//        and replayed (one event pair around each replay; the median of
//        five replays after a warm one): back-to-back kernels with no host
//        gaps, the figure comparable to a profiler's per-kernel duration.
//        `out` holds at least 5 floats.
int draco_bench_gemv(int code, const uint8_t* W, int n_out, int n_in, int n_copies, int iters,
                     float* out) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = ensure_init()) return rc;
    if (!draco_gemv_supported(code)) return fail(-1, "bench: unsupported code %d", code);
    DracoMat base;
    if (draco_layout(code, n_out, n_in, &base.L)) return fail(-1, "bench: bad shape");
    if (n_copies < 1) n_copies = 1;
    std::vector<uint8_t> host(base.L.bytes, 0);
    draco_repack(code, W, n_out, n_in, host.data());
    std::vector<DracoMat> mats(n_copies, base);
    for (auto& m : mats) {
        DRACO_HIP(hipMalloc(&m.dev, base.L.bytes));
        DRACO_HIP(hipMemcpy(m.dev, host.data(), base.L.bytes, hipMemcpyHostToDevice));
    }
    std::vector<float> xh(n_in);
    for (int i = 0; i < n_in; i++) xh[i] = (float)((i * 37) % 101 - 50) * 0.02f;
    float *dx, *dy;
    DRACO_HIP(hipMalloc(&dx, sizeof(float) * n_in));
    DRACO_HIP(hipMalloc(&dy, sizeof(float) * n_out));
    DRACO_HIP(hipMemcpy(dx, xh.data(), sizeof(float) * n_in, hipMemcpyHostToDevice));
    hipStream_t st = stream();
    for (int i = 0; i < 2 * n_copies; i++) draco_gemv_launch(mats[i % n_copies], dx, dy, nullptr, 0, n_out, st);
    DRACO_HIP(hipStreamSynchronize(st));
    std::vector<hipEvent_t> ev(2 * iters + 2);
    for (auto& e : ev) DRACO_HIP(hipEventCreate(&e));
    DRACO_HIP(hipEventRecord(ev[2 * iters], st));
    for (int i = 0; i < iters; i++) {
        DRACO_HIP(hipEventRecord(ev[2 * i], st));
        draco_gemv_launch(mats[i % n_copies], dx, dy, nullptr, 0, n_out, st);
        DRACO_HIP(hipEventRecord(ev[2 * i + 1], st));
    }
    DRACO_HIP(hipEventRecord(ev[2 * iters + 1], st));
    DRACO_HIP(hipStreamSynchronize(st));
    std::vector<float> t(iters);
    double sum = 0;
    for (int i = 0; i < iters; i++) {
        float ms = 0;
        DRACO_HIP(hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]));
        t[i] = ms * 1000.f;
        sum += t[i];
    }
    float tot = 0;
    DRACO_HIP(hipEventElapsedTime(&tot, ev[2 * iters], ev[2 * iters + 1]));
    // graph replay of the same rotation
    hipGraph_t graph;
    hipGraphExec_t exec;
    DRACO_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
    for (int i = 0; i < iters; i++) draco_gemv_launch(mats[i % n_copies], dx, dy, nullptr, 0, n_out, st);
    DRACO_HIP(hipStreamEndCapture(st, &graph));
    DRACO_HIP(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    DRACO_HIP(hipGraphLaunch(exec, st));  // warm
    float reps[5];
    for (int r = 0; r < 5; r++) {
        DRACO_HIP(hipEventRecord(ev[0], st));
        DRACO_HIP(hipGraphLaunch(exec, st));
        DRACO_HIP(hipEventRecord(ev[1], st));
        DRACO_HIP(hipStreamSynchronize(st));
        DRACO_HIP(hipEventElapsedTime(&reps[r], ev[0], ev[1]));
    }
    std::sort(reps, reps + 5);
    const float gms = reps[2];
    hipGraphExecDestroy(exec);
    hipGraphDestroy(graph);
    // calibration for hardware byte counters: one device-to-device copy of a
    // whole weight copy (L.bytes read, L.bytes written) after the timed work
    if (n_copies > 1) {
        DRACO_HIP(hipMemcpyAsync(mats[1].dev, mats[0].dev, base.L.bytes, hipMemcpyDeviceToDevice, st));
        DRACO_HIP(hipStreamSynchronize(st));
    }
    std::vector<float> s = t;
    std::sort(s.begin(), s.end());
    out[0] = (float)(sum / iters);
    out[1] = tot * 1000.f / iters;
    out[2] = s[0];
    out[3] = s[iters / 2];
    out[4] = gms * 1000.f / iters;
    for (auto& e : ev) hipEventDestroy(e);
    for (auto& m : mats) hipFree(m.dev);
    hipFree(dx);
    hipFree(dy);
    return 0;
}

// Launch overhead probe: `iters` back-to-back empty kernels, in a plain
// stream and replayed from a captured graph.  out[0] us/launch stream,
// out[1] us/launch graph.
__global__ void k_empty(int* p) {
    if (p && threadIdx.x == 0 && blockIdx.x == 0x7fffffff) p[0] = 1;
}

int draco_bench_launch(int iters, float* out) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = ensure_init()) return rc;
    hipStream_t st = stream();
    hipEvent_t a, b;
    DRACO_HIP(hipEventCreate(&a));
    DRACO_HIP(hipEventCreate(&b));
    for (int i = 0; i < 10; i++) hipLaunchKernelGGL(k_empty, dim3(256), dim3(256), 0, st, nullptr);
    DRACO_HIP(hipEventRecord(a, st));
    for (int i = 0; i < iters; i++) hipLaunchKernelGGL(k_empty, dim3(256), dim3(256), 0, st, nullptr);
    DRACO_HIP(hipEventRecord(b, st));
    DRACO_HIP(hipEventSynchronize(b));
    float ms = 0;
    DRACO_HIP(hipEventElapsedTime(&ms, a, b));
    out[0] = ms * 1000.f / iters;
    hipGraph_t graph;
    hipGraphExec_t exec;
    DRACO_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
    for (int i = 0; i < iters; i++) hipLaunchKernelGGL(k_empty, dim3(256), dim3(256), 0, st, nullptr);
    DRACO_HIP(hipStreamEndCapture(st, &graph));
    DRACO_HIP(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    DRACO_HIP(hipGraphLaunch(exec, st));
    DRACO_HIP(hipStreamSynchronize(st));
    DRACO_HIP(hipEventRecord(a, st));
    DRACO_HIP(hipGraphLaunch(exec, st));
    DRACO_HIP(hipEventRecord(b, st));
    DRACO_HIP(hipEventSynchronize(b));
    DRACO_HIP(hipEventElapsedTime(&ms, a, b));
    out[1] = ms * 1000.f / iters;
    hipGraphExecDestroy(exec);
    hipGraphDestroy(graph);
    hipEventDestroy(a);
    hipEventDestroy(b);
    return 0;
}

}  // extern "C"
