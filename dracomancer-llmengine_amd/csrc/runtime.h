// runtime.h -- process-wide device state behind the C ABI.
//
// One HIP stream per process, one device (DRACO_DEVICE, default 0), a
// residency registry that maps caller-owned host weight buffers to their
// device copies, device mirrors of caller-owned state arrays (KV caches), and
// grow-only scratch.  The library is non-reentrant like the reference (whose
// globals make it so, src/m6_layer.c:29-46); every public entry point takes
// the one mutex, so concurrent callers are serialised rather than racing.
#pragma once
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "gemv.h"

namespace draco {

std::recursive_mutex& api_mutex();

// Initialise device + stream on first use.  0 = ok.
int ensure_init();
hipStream_t stream();
// Device address of the no-alloc entry point's static staging array on
// `device` (noalloc.hip); called by ensure_init with that device current.
int noalloc_setup(int device);

// Record an error message (readable through draco_last_error()).
int fail(int rc, const char* fmt, ...);
const char* last_error();

#define DRACO_HIP(expr)                                                                    \
    do {                                                                                   \
        hipError_t e_ = (expr);                                                            \
        if (e_ != hipSuccess)                                                              \
            return ::draco::fail(-2, "%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), \
                                 __FILE__, __LINE__);                                      \
    } while (0)

// Eviction epoch: bumped whenever a registered weight or mirror is dropped or
// replaced.  Anything that caches DracoMat pointers or mirror addresses must
// rebuild when the epoch it was built at is no longer current.
uint64_t epoch();

// Weight residency.  Returns nullptr (and records an error) on failure.
// The host buffer must hold n_out rows of GGUF format `code`; its contents are
// assumed immutable while registered (draco_forget drops an entry).
const DracoMat* get_mat(const void* host, int code, int n_out, int n_in);
int forget(const void* host);
// The registered matrix (format code, n_in) whose host rows hold `row` at a
// row start; *r = the row's index.  nullptr when none does.
const DracoMat* find_row(const void* row, int code, int n_in, int* r);
// Device copy of a caller-owned fp32 array of n floats (norm weights, conv
// taps, ...), registered like a weight.  tcols > 0: the host array is
// [n / tcols][tcols] and the device copy is its transpose [tcols][n / tcols].
const float* get_vec(const float* host, size_t n, int tcols = 0);
void forget_all();
size_t resident_bytes();

// Device mirror of a caller-owned host array (KV caches and other state).
// `fresh` is set when the mirror was (re)allocated and holds no data yet.
void* get_mirror(const void* host, size_t bytes, bool* fresh);
// The same, but a mirror too small for `bytes` is replaced by a larger one
// that keeps its first `keep` bytes (`fresh` is then false).
void* grow_mirror(const void* host, size_t bytes, size_t keep, bool* fresh);
int mirror_invalidate(const void* host);
int mirror_pull(const void* host, size_t bytes);   // device -> host
int mirror_push(const void* host, size_t bytes);   // host -> device

// Fill a caller's host output with quiet NaN: the void entry points (as the
// reference's, which return nothing) leave it so when they fail, so a caller
// that cannot see the error does not read stale values as a result.
void poison(float* host, size_t n);

// Grow-only device scratch in numbered slots.
void* scratch(int slot, size_t bytes);
// Grow-only pinned host staging in numbered slots.
void* pinned(int slot, size_t bytes);

}  // namespace draco
