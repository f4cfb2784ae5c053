// q8k.h -- internal interface of the Q8_K quantizer and the Q4_K/Q6_K x Q8_K
// GEMV kernels (q8k.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "formats.h"

struct Q8Launch {
    const uint8_t* base;  // weights, tile layout (formats.h)
    DracoLayout L;
    int n_in;
    const uint8_t* xq;    // nvec * (n_in/256) Q8_K blocks, vector-major (device);
                          // with img: the GEMV image of those blocks (below)
    bool img;
    const float* xf;      // optional (nvec 1, not img / isums): fp32 x, quantized to
                          // Q8_K inside the GEMV launch (xq unused)
    float* y;             // y[v * y_stride + row]
    int y_stride;
    int row0, row1;       // rows computed (row1 == 0: n_out)
    int32_t* isc;         // optional (ISUMS launches): [n_out][nb] integer sums
    int32_t* imn;
    // filled by draco_gemv_q8k_launch
    int tile0, n_tiles;
};

// Quantize nvec vectors of n floats (n % 256 == 0) into Q8_K blocks.  With
// image, out receives the same values as the GEMV's LDS image instead of
// blocks: q8 [nvec][n] int8, the group sums [n/256][nvec][16] as f16 (exact:
// |sum| <= 2032), d [n/256][nvec] float, contiguous (the same byte count as
// the blocks; buffers for it need Q8K_IMAGE_PAD bytes more, which the GEMV's
// 16-byte copy may read).
constexpr int Q8K_IMAGE_PAD = 16;
int draco_q8k_quantize_launch(const float* x, int n, int nvec, uint8_t* out, hipStream_t st, bool image = false);
// nvec in {1, 4, 8}; isums requires nvec == 1.
int draco_gemv_q8k_launch(Q8Launch& a, int nvec, bool isums, hipStream_t st);
// Whether draco_gemv_q8k_launch serves rows n_in wide for nvec vectors (the
// Q8_K image of x and the block's reduction space fit the CU's 160 KiB of
// LDS), checked before anything is enqueued.
int draco_gemv_q8k_shape_ok(int code, int n_in, int nvec, bool img, bool isums);
// Whether one vector of rows n_in wide can be quantized inside the GEMV
// launch (Q8Launch.xf): the block's half-waves cover the row's super-blocks
// in one pass (n_in <= 4096 at 8 waves, 8192 at 16).  Longer rows measured
// slower fused than as a quantizer launch plus the GEMV (4096x14336:
// 14.5 us against 10.6 us).
int draco_gemv_q8k_fused_ok(int code, int n_in);
