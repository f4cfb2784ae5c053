// gemv.h -- internal interface between the C-ABI layer and the GEMV kernels.
#pragma once
#include <hip/hip_runtime.h>

#include "formats.h"

// A weight matrix resident on the device in the private layout of formats.h.
struct DracoMat {
    DracoLayout L;
    uint8_t* dev;  // device base address
};

// y[r] = (yadd ? yadd[r] : 0) + W[r,:] . x  for r in [row0, row1); all device pointers.
int draco_gemv_launch(const DracoMat& m, const float* x, float* y, const float* yadd, int row0,
                      int row1, hipStream_t st);
int draco_gemv_supported(int code);
