/*
 * draco_hip.h -- C ABI of libdraco_hip.so, the MI355X (gfx950) implementation
 * of the Dracomancer per-token decode path.
 *
 * Every entry point named m5_* / m6_* has the exact signature and meaning of
 * the reference function it replaces (cited file:line under the reference
 * tree).  All pointer arguments of those are caller-owned HOST pointers, as
 * in the reference; results are in host memory when the call returns.
 * Weights are uploaded (and repacked into a private device layout) on first
 * sight and then stay resident, keyed by their host address; their bytes must
 * not change while registered (draco_forget() drops an entry).
 *
 * Return codes: 0 ok, -1 unsupported code/shape (fail loudly, as the
 * reference's -1), -2 device error.  draco_last_error() describes the last
 * failure.  The library serialises callers with one mutex (the reference is
 * non-reentrant too: src/m6_layer.c:29-46).
 */
#ifndef DRACO_HIP_H
#define DRACO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- per-format kernel-library ABI (drop-in for m5_kern*.so) ----------- */

/* src/m5_kern_scalar.c:146-148.  1 if `code` is served (0 Q8_0, 4 Q6_K,
 * 5 Q4_K, 7 F16, 9 F32). */
int m5_scalar_supported(int code);

/* src/m5_kern_scalar.c:150-156.  y[n_out] = W[n_out x n_in] . x */
int m5_gemv(int code, const float* x, const uint8_t* W, int n_out, int n_in, float* y);

/* src/m5_kern_scalar.c:158-165.  Rows [o0,o1) only, written at their absolute
 * index in y; other entries of y are not touched. */
int m5_gemv_range(int code, const float* x, const uint8_t* W, int n_out, int n_in, float* y,
                  int o0, int o1);

/* ---- library utilities (no reference counterpart) ----------------------- */

const char* draco_last_error(void);
const char* draco_version(void);
/* Drop the device copy / mirror registered for a host buffer; returns count. */
int draco_forget(const void* host);
/* Drop every device copy and mirror. */
void draco_reset(void);
size_t draco_resident_bytes(void);

/* Device timing probes (weights rotated over n_copies device copies so the
 * working set can exceed the 256 MB MALL).  out[0] mean us per launch from
 * per-launch event pairs, out[1] us per launch over the whole loop, out[2]
 * min, out[3] median. */
int draco_bench_gemv(int code, const uint8_t* W, int n_out, int n_in, int n_copies, int iters,
                     float* out);
/* out[0] us per empty-kernel launch in a stream, out[1] in a replayed graph. */
int draco_bench_launch(int iters, float* out);

/* Host-side byte work (pure CPU, callable without a GPU). */
int draco_quantize(int code, const float* x, int n_rows, int n_in, uint8_t* out);
size_t draco_layout_query(int code, int n_out, int n_in, size_t* off4);
int draco_repack(int code, const uint8_t* src, int n_out, int n_in, uint8_t* dst);
int draco_unpack(int code, const uint8_t* src, int n_out, int n_in, uint8_t* dst);
void draco_rope_table(int max_t, int rot, float base, float* tab);
float draco_f16_to_f32(uint16_t h);
uint16_t draco_f32_to_f16(float f);

#ifdef __cplusplus
}
#endif
#endif /* DRACO_HIP_H */
