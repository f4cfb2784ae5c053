// noalloc.hip -- the allocation-free variant of draco_gemv_q8k_f32.
//
// No reference counterpart.  For callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc): the Q8_K blocks of x, which draco_gemv_q8k_f32 stages in a
// library-allocated buffer, are staged here in a file-scope device array of
// fixed size instead.  Each GPU holds its own copy of the array for the life
// of the process; its device address is taken once per device at library
// set-up (draco_noalloc_setup, called from ensure_init with the device
// current) and only that address is ever handed to kernels.
//
// Every call on a GPU shares that GPU's array: calls that overlap on one GPU
// (two streams, or two host threads with their own streams) race on it.
// Nothing in the array needs clearing between calls: the quantize launch of a
// call writes every byte (scale, 256 quants, 16 block sums per block) that the
// GEMV launch of the same call reads.
#include <hip/hip_runtime.h>

#include "q8k.h"
#include "runtime.h"

// 1 MiB: nvec * (n_in / 256) * 292 + 16 bytes at most.  The shapes served
// are bounded more tightly by the GEMV, whose LDS holds the same image (at
// most about 150 KiB of it: n_in up to 16896 at nvec 8, 67584 at nvec 1).
constexpr size_t NOALLOC_Q8K_BYTES = 1u << 20;
constexpr int NOALLOC_MAX_DEVICES = 64;

// The staging array.  File scope, outside any namespace: the compiler gives a
// static device variable whose address host code takes (HIP_SYMBOL below) a
// global symbol in the code object, which hipGetSymbolAddress looks up.  (Its
// name must not collide with draco::scratch, the grow-only allocator, which
// an unqualified name inside namespace draco would find first.)
static __device__ __align__(256) uint8_t noalloc_q8k_stage[NOALLOC_Q8K_BYTES];

namespace {

void* g_scratch_ptr[NOALLOC_MAX_DEVICES] = {};

}  // namespace

namespace draco {

// Called by ensure_init() once per device, with that device current.
int noalloc_setup(int device) {
    if (device < 0 || device >= NOALLOC_MAX_DEVICES) return fail(-2, "noalloc: device %d out of range", device);
    if (g_scratch_ptr[device]) return 0;
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(::noalloc_q8k_stage));
    if (e != hipSuccess || !p)
        return fail(-2, "noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
    g_scratch_ptr[device] = p;
    return 0;
}

}  // namespace draco

using namespace draco;

extern "C" {

// Bytes of the static staging array (the largest nvec * (n_in / 256) * 292 +
// 16).  A request within it can still exceed the GEMV's LDS image (160 KiB
// for the image and the block's reduction space); such calls return -1
// before anything is enqueued.
size_t draco_noalloc_capacity(void) { return NOALLOC_Q8K_BYTES; }

// draco_gemv_q8k_f32 with device pointers and no allocation: x [nvec][n_in]
// fp32, W the weights in this library's device layout (draco_repack output,
// draco_layout_query bytes), y [nvec][n_out] fp32.  Enqueued on `stream`
// (NULL: the library's stream), not waited for.  0 ok, -1 unsupported code or
// shape or staging larger than draco_noalloc_capacity(), -2 device error.
int draco_gemv_q8k_f32_noalloc(int code, const float* x, int nvec, const uint8_t* W, int n_out, int n_in, float* y,
                               void* stream) {
    std::lock_guard<std::recursive_mutex> g(api_mutex());
    if (code != DRACO_Q4_K && code != DRACO_Q6_K) return fail(-1, "noalloc q8k gemv: unsupported format code %d", code);
    if (n_out <= 0 || n_in <= 0 || n_in % 256) return fail(-1, "noalloc q8k gemv: bad shape %dx%d", n_out, n_in);
    if (nvec != 1 && nvec != 4 && nvec != 8) return fail(-1, "noalloc q8k gemv: nvec %d not in {1, 4, 8}", nvec);
    if (!x || !W || !y) return fail(-1, "noalloc q8k gemv: null pointer");
    const size_t need = (size_t)nvec * (size_t)(n_in / 256) * Q8K_BLOCK_BYTES + Q8K_IMAGE_PAD;
    if (need > NOALLOC_Q8K_BYTES)
        return fail(-1, "noalloc q8k gemv: %zu bytes of Q8_K staging exceed the %zu-byte static array", need,
                    NOALLOC_Q8K_BYTES);
    // the GEMV's own limits first: nothing is enqueued for a call it would refuse
    if (!draco_gemv_q8k_shape_ok(code, n_in, nvec, true, false))
        return fail(-1, "noalloc q8k gemv: rows of %d values at nvec %d exceed the GEMV's LDS image", n_in, nvec);
    if (int rc = ensure_init()) return rc;
    int dev = 0;
    DRACO_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES || !g_scratch_ptr[dev]) {
        if (int rc = noalloc_setup(dev)) return rc;
    }
    uint8_t* stage = (uint8_t*)g_scratch_ptr[dev];
    DracoLayout L;
    if (draco_layout(code, n_out, n_in, &L)) return fail(-1, "noalloc q8k gemv: no layout for %dx%d", n_out, n_in);
    hipStream_t st = stream ? (hipStream_t)stream : draco::stream();
    if (draco_q8k_quantize_launch(x, n_in, nvec, stage, st, true)) return fail(-1, "noalloc q8k quantize rejected");
    Q8Launch a = {};
    a.base = W;
    a.L = L;
    a.n_in = n_in;
    a.xq = stage;
    a.img = true;
    a.y = y;
    a.y_stride = n_out;
    if (draco_gemv_q8k_launch(a, nvec, false, st)) return fail(-1, "noalloc q8k gemv launch rejected");
    DRACO_HIP(hipGetLastError());
    return 0;
}

}  // extern "C"
