// tile_frag.h -- one wave's operands of a (tile, super-block) item of the
// Q4_K / Q6_K tile layout (formats.h), shared by the fp32-activation GEMV
// (gemv.hip) and the Q8_K-activation GEMV (q8k.hip).
//
// Lane l = j + 16*g (row j of the 16-row tile, lane group g = 0..3).
#pragma once
#include <hip/hip_runtime.h>

#include "dev_common.h"
#include "formats.h"

typedef int v4i __attribute__((ext_vector_type(4)));

struct Frag {
    uint4 a, b, c;   // Q4_K: qs r=0, qs r=1, header.  Q6_K: ql A, ql B, qh
    uint32_t sc, d;  // Q6_K: 4 scales, d
};

__device__ __forceinline__ void load_q4(const uint8_t* item, int lane, Frag& f) {
    f.a = ldu4(item + 16 * lane);
    f.b = ldu4(item + 1024 + 16 * lane);
    f.c = ldu4(item + 2048 + 16 * (lane & 15));
    f.sc = 0u;
    f.d = 0u;
}

__device__ __forceinline__ void load_q6(const uint8_t* item, int lane, Frag& f) {
    f.a = ldu4(item + 16 * lane);
    f.b = ldu4(item + 1024 + 16 * lane);
    f.c = ldu4(item + 2048 + 16 * lane);
    f.sc = *reinterpret_cast<const uint32_t*>(item + 3072 + 4 * lane);
    f.d = *reinterpret_cast<const uint16_t*>(item + 3328 + 2 * (lane & 15));
}

__device__ __forceinline__ float fold(const v4i C) {
    const int i0 = (C[0] << 7) + C[1], i1 = (C[2] << 7) + C[3];
    return fmaf((float)i1, 6.103515625e-05f, (float)i0);
}

// A operand of one int8 MFMA: 16 bytes at p, or zeros for lanes that hold
// no activation row (p == nullptr is never passed: callers point those lanes
// at a zeroed LDS region instead, so the load is unconditional).
__device__ __forceinline__ v4i lds_v4i(const int8_t* p) { return *reinterpret_cast<const v4i*>(p); }
