// abi_m5.cpp -- the per-format kernel-library ABI (drop-in for m5_kern*.so).
//
// Reference interface: src/m5_kern_scalar.c:146-165 (typedefs
// src/m6_layer.c:29-30).  All pointers are caller-owned HOST pointers; y is
// valid when the call returns.  Return 0 = ok, -1 = unsupported code or
// shape, -2 = device error (message via draco_last_error()).
#include <string.h>

#include "runtime.h"

using namespace draco;

namespace {

int gemv_host(int code, const float* x, const uint8_t* W, int n_out, int n_in, float* y, int o0,
              int o1) {
    if (!draco_gemv_supported(code)) return fail(-1, "m5_gemv: unsupported format code %d", code);
    const int bv = draco_block_values(code);
    if (n_in <= 0 || n_out <= 0 || n_in % bv) return fail(-1, "m5_gemv: bad shape %dx%d", n_out, n_in);
    if (o0 < 0 || o1 > n_out || o0 > o1) return fail(-1, "m5_gemv_range: bad range [%d,%d)", o0, o1);
    if (o0 == o1) return 0;
    if (int rc = ensure_init()) return rc;
    const DracoMat* m = get_mat(W, code, n_out, n_in);
    if (!m) return -2;
    float* dx = (float*)scratch(0, sizeof(float) * (size_t)n_in);
    float* dy = (float*)scratch(1, sizeof(float) * (size_t)n_out);
    if (!dx || !dy) return -2;
    hipStream_t st = stream();
    DRACO_HIP(hipMemcpyAsync(dx, x, sizeof(float) * (size_t)n_in, hipMemcpyHostToDevice, st));
    if (draco_gemv_launch(*m, dx, dy, nullptr, o0, o1, st)) return fail(-1, "gemv launch rejected");
    DRACO_HIP(hipGetLastError());
    DRACO_HIP(hipMemcpyAsync(y + o0, dy + o0, sizeof(float) * (size_t)(o1 - o0), hipMemcpyDeviceToHost,
                             st));
    DRACO_HIP(hipStreamSynchronize(st));
    return 0;
}

}  // namespace

extern "C" {

int m5_scalar_supported(int code) { return draco_gemv_supported(code) ? 1 : 0; }

int m5_gemv(int code, const float* x, const uint8_t* W, int n_out, int n_in, float* y) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    return gemv_host(code, x, W, n_out, n_in, y, 0, n_out);
}

int m5_gemv_range(int code, const float* x, const uint8_t* W, int n_out, int n_in, float* y, int o0,
                  int o1) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    return gemv_host(code, x, W, n_out, n_in, y, o0, o1);
}

const char* draco_last_error(void) { return last_error(); }

int draco_forget(const void* host) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    return forget(host);
}

void draco_reset(void) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    forget_all();
}

size_t draco_resident_bytes(void) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    return resident_bytes();
}

const char* draco_version(void) { return "draco_hip/1 gfx950"; }

}  // extern "C"
