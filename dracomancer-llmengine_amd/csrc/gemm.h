// gemm.h -- internal interface of the prefill GEMM kernels (gemm.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "formats.h"

struct GemmArgs {
    const uint8_t* W;   // weights, Q4_K / Q6_K tile layout
    DracoLayout L;
    int n_in, T;
    // digitized activations (draco_gemm_digits_launch)
    const int8_t* xdig;
    const float* xsc;
    const float* xs32;
    const float* xs16;
    float* Y;           // Y[t * ldy + row]
    int ldy;
};

// device bytes of the digit buffer for T tokens of length n_in
size_t draco_gemm_digit_bytes(int T, int n_in);
// digitize X[T][n_in] (device) into buf; fills a.xdig/xsc/xs32/xs16, a.T, a.n_in
int draco_gemm_digits_launch(const float* X, int T, int n_in, uint8_t* buf, GemmArgs& a, hipStream_t st);
int draco_gemm_launch(GemmArgs& a, hipStream_t st);
