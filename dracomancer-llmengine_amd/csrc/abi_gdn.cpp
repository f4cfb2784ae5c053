// abi_gdn.cpp -- Gated-DeltaNet scan entry points.
//
// m6_gdn_scan: src/m6_gdn_scan.c:18-93 (host pointers; S and tail are updated
// in place, as in the reference).  The host ABI uploads the inputs and the
// state, runs the scan on the device and downloads ON, S and tail.
#include <stdio.h>
#include <string.h>

#include "gdn.h"
#include "runtime.h"

using namespace draco;

namespace {

int gdn_host(const float* QKV, const float* Z, const float* B, const float* G, const float* conv,
             const float* ssm_norm, float* tail, float* S, int T, int n_qkv, int n_vh, float* ON) {
    if (n_vh < 1 || T < 0 || n_qkv <= n_vh * 128 || (n_qkv - n_vh * 128) % 256)
        return fail(-1, "m6_gdn_scan: n_qkv %d / n_vh %d not a 128-wide q/k/v split", n_qkv, n_vh);
    if (T == 0) return 0;
    if (int rc = ensure_init()) return rc;
    hipStream_t st = stream();
    const size_t nq = (size_t)T * n_qkv, nz = (size_t)T * n_vh * 128, nbg = (size_t)T * n_vh,
                 ns = (size_t)n_vh * 128 * 128, nt = (size_t)n_qkv * 3, nc = (size_t)n_qkv * 4;
    const size_t npss = (size_t)T * n_vh * GDN_PSS_STRIDE;
    float* d = (float*)scratch(6, sizeof(float) * (nq + 2 * nz + 2 * nbg + ns + nt + nc + 128 + npss));
    if (!d) return -2;
    GdnArgs a = {};
    float* p = d;
    float* dq = p; p += nq;
    float* dz = p; p += nz;
    float* db = p; p += nbg;
    float* dg = p; p += nbg;
    float* dc = p; p += nc;
    float* dn = p; p += 128;
    float* dt = p; p += nt;
    float* ds = p; p += ns;
    float* dpss = p; p += npss;
    float* don = p;
    // a state the per-layer GDN op holds on the device is scanned in place
    // there (the caller's arrays hold only its sample); any other is uploaded
    float *rs = nullptr, *rt = nullptr;
    const bool resident = draco_gdn_state_current(S, tail, ns, nt, &rs, &rt);
    if (resident) {
        ds = rs;
        dt = rt;
    }
    DRACO_HIP(hipMemcpyAsync(dq, QKV, sizeof(float) * nq, hipMemcpyHostToDevice, st));
    DRACO_HIP(hipMemcpyAsync(dz, Z, sizeof(float) * nz, hipMemcpyHostToDevice, st));
    DRACO_HIP(hipMemcpyAsync(db, B, sizeof(float) * nbg, hipMemcpyHostToDevice, st));
    DRACO_HIP(hipMemcpyAsync(dg, G, sizeof(float) * nbg, hipMemcpyHostToDevice, st));
    DRACO_HIP(hipMemcpyAsync(dc, conv, sizeof(float) * nc, hipMemcpyHostToDevice, st));
    DRACO_HIP(hipMemcpyAsync(dn, ssm_norm, sizeof(float) * 128, hipMemcpyHostToDevice, st));
    if (!resident) {
        DRACO_HIP(hipMemcpyAsync(dt, tail, sizeof(float) * nt, hipMemcpyHostToDevice, st));
        DRACO_HIP(hipMemcpyAsync(ds, S, sizeof(float) * ns, hipMemcpyHostToDevice, st));
    }
    a.QKV = dq;
    a.Z = dz;
    a.B = db;
    a.G = dg;
    a.conv = dc;
    a.ssm_norm = dn;
    a.tail = dt;
    a.S = ds;
    a.ON = don;
    a.T = T;
    a.n_qkv = n_qkv;
    a.n_vh = n_vh;
    a.nhq = (n_qkv - n_vh * 128) / 256;
    a.nspl = T == 1 ? 1 : draco_gdn_split(false);  // one token: nothing to take the split's rms
    a.PSS = dpss;
    if (draco_gdn_scan_launch(a, st)) return fail(-1, "gdn scan launch rejected");
    DRACO_HIP(hipGetLastError());
    DRACO_HIP(hipMemcpyAsync(ON, don, sizeof(float) * nz, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipMemcpyAsync(S, ds, sizeof(float) * ns, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipMemcpyAsync(tail, dt, sizeof(float) * nt, hipMemcpyDeviceToHost, st));
    DRACO_HIP(hipStreamSynchronize(st));
    // the caller's arrays now hold the whole state, as the mirrors do
    if (resident) draco_gdn_state_written(S, ds);
    return 0;
}

}  // namespace

extern "C" {

void m6_gdn_scan(const float* QKV, const float* Z, const float* B, const float* G, const float* conv,
                 const float* ssm_norm, float* tail, float* S, int T, int n_qkv, int n_vh, float* ON,
                 float* work) {
    (void)work;  // the device path needs no host scratch
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (int rc = gdn_host(QKV, Z, B, G, conv, ssm_norm, tail, S, T, n_qkv, n_vh, ON))
        fprintf(stderr, "m6_gdn_scan: rc %d: %s\n", rc, last_error());
}

// Device-resident timing of the scan with the same inputs as m6_gdn_scan
// (state and tail are copied, the caller's arrays are not modified):
// out[0] us per token scanning T tokens in chunks of `chunk` tokens (one
// launch per chunk), out[1] us per single-token launch (n_dec decode steps
// after the prefill), both from graph replays.
int draco_bench_gdn_scan(const float* QKV, const float* Z, const float* B, const float* G, const float* conv,
                         const float* ssm_norm, const float* tail, const float* S, int T, int n_qkv, int n_vh,
                         int chunk, int n_dec, float* out) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (n_vh < 1 || T < 1 || chunk < 1 || n_dec < 0 || n_dec > T || n_qkv <= n_vh * 128 ||
        (n_qkv - n_vh * 128) % 256)
        return fail(-1, "bench gdn: bad shape");
    if (int rc = ensure_init()) return rc;
    hipStream_t st = stream();
    const size_t nq = (size_t)T * n_qkv, nz = (size_t)T * n_vh * 128, nbg = (size_t)T * n_vh,
                 ns = (size_t)n_vh * 128 * 128, nt = (size_t)n_qkv * 3, nc = (size_t)n_qkv * 4;
    float *dq, *dz, *db, *dg, *dc, *dn, *dt, *ds, *don, *dpss;
    DRACO_HIP(hipMalloc(&dpss, sizeof(float) * (size_t)(chunk > 1 ? chunk : 1) * n_vh * GDN_PSS_STRIDE));
    DRACO_HIP(hipMalloc(&dq, sizeof(float) * nq));
    DRACO_HIP(hipMalloc(&dz, sizeof(float) * nz));
    DRACO_HIP(hipMalloc(&db, sizeof(float) * nbg));
    DRACO_HIP(hipMalloc(&dg, sizeof(float) * nbg));
    DRACO_HIP(hipMalloc(&dc, sizeof(float) * nc));
    DRACO_HIP(hipMalloc(&dn, sizeof(float) * 128));
    DRACO_HIP(hipMalloc(&dt, sizeof(float) * nt));
    DRACO_HIP(hipMalloc(&ds, sizeof(float) * ns));
    DRACO_HIP(hipMalloc(&don, sizeof(float) * nz));
    DRACO_HIP(hipMemcpy(dq, QKV, sizeof(float) * nq, hipMemcpyHostToDevice));
    DRACO_HIP(hipMemcpy(dz, Z, sizeof(float) * nz, hipMemcpyHostToDevice));
    DRACO_HIP(hipMemcpy(db, B, sizeof(float) * nbg, hipMemcpyHostToDevice));
    DRACO_HIP(hipMemcpy(dg, G, sizeof(float) * nbg, hipMemcpyHostToDevice));
    DRACO_HIP(hipMemcpy(dc, conv, sizeof(float) * nc, hipMemcpyHostToDevice));
    DRACO_HIP(hipMemcpy(dn, ssm_norm, sizeof(float) * 128, hipMemcpyHostToDevice));
    DRACO_HIP(hipMemcpy(dt, tail, sizeof(float) * nt, hipMemcpyHostToDevice));
    DRACO_HIP(hipMemcpy(ds, S, sizeof(float) * ns, hipMemcpyHostToDevice));
    auto args = [&](int t0, int n) {
        GdnArgs a = {};
        a.QKV = dq + (size_t)t0 * n_qkv;
        a.Z = dz + (size_t)t0 * n_vh * 128;
        a.B = db + (size_t)t0 * n_vh;
        a.G = dg + (size_t)t0 * n_vh;
        a.conv = dc;
        a.ssm_norm = dn;
        a.tail = dt;
        a.S = ds;
        a.ON = don + (size_t)t0 * n_vh * 128;
        a.T = n;
        a.n_qkv = n_qkv;
        a.n_vh = n_vh;
        a.nhq = (n_qkv - n_vh * 128) / 256;
        a.nspl = n == 1 ? 1 : draco_gdn_split(false);
        a.PSS = dpss;
        return a;
    };
    hipEvent_t e0, e1;
    DRACO_HIP(hipEventCreate(&e0));
    DRACO_HIP(hipEventCreate(&e1));
    for (int mode = 0; mode < 2; mode++) {
        if (mode == 1 && n_dec == 0) {
            out[1] = 0.f;
            break;
        }
        hipGraph_t graph;
        hipGraphExec_t exec;
        DRACO_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
        if (mode == 0) {
            for (int t0 = 0; t0 < T; t0 += chunk) draco_gdn_scan_launch(args(t0, T - t0 < chunk ? T - t0 : chunk), st);
        } else {
            for (int t = 0; t < n_dec; t++) draco_gdn_scan_launch(args(t, 1), st);
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
        out[mode] = ms * 1000.f / (mode == 0 ? T : n_dec);
        hipGraphExecDestroy(exec);
        hipGraphDestroy(graph);
    }
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    for (float* p : {dq, dz, db, dg, dc, dn, dt, ds, don, dpss}) hipFree(p);
    return 0;
}

}  // extern "C"
