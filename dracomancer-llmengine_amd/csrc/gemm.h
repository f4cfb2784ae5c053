// gemm.h -- internal interface of the prefill GEMM kernels (gemm.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "formats.h"

// One group of a grouped GEMM (e.g. one expert): its weights and its tokens,
// octets [oct0, oct0 + n_oct) of the digit buffer.
struct GemmGroup {
    const uint8_t* W;
    int oct0, n_oct;
};

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
    // grouped launch (nullptr: one group = W, all tokens)
    const GemmGroup* groups;  // device array [n_groups]
    int n_groups;
    int max_oct;              // largest n_oct of any group
};

// device bytes of the digit buffer for T tokens of length n_in
size_t draco_gemm_digit_bytes(int T, int n_in);
// digitize X[T][n_in] (device) into buf; fills a.xdig/xsc/xs32/xs16, a.T, a.n_in
int draco_gemm_digits_launch(const float* X, int T, int n_in, uint8_t* buf, GemmArgs& a, hipStream_t st);
int draco_gemm_launch(GemmArgs& a, hipStream_t st);

// ---- f16-MFMA GEMM (gemmh.hip): the plain (non-grouped) prefill path ----
struct GemmHArgs {
    const uint8_t* W;    // weights, Q4_K / Q6_K tile layout
    DracoLayout L;
    int n_in, T;
    const uint8_t* xh;   // activations from draco_gemmh_x_launch
    float* Y;            // Y[t * ldy + row]
    int ldy;
    float* part;         // K-split partials, draco_gemmh_part_floats(L, T, ldy) floats (nullable when 0)
};
size_t draco_gemmh_x_bytes(int T, int n_in);
int draco_gemmh_x_launch(const float* X, int T, int n_in, uint8_t* buf, hipStream_t st);
size_t draco_gemmh_part_floats(const DracoLayout& L, int T, int ldy);
int draco_gemmh_launch(GemmHArgs& a, hipStream_t st);

struct DracoMat;
// Y[t][row] = X[t] . W[row] for T token rows (X, Y device, token-major).
// Q4_K / Q6_K: X's activation operands (f16 hi/lo) into `digits`
// (draco_gemm_digit_bytes(T, n_in) bytes), skipped when have_digits says they
// are already there for this X, then the f16-MFMA GEMM; other formats (Q8_0,
// F32, F16): one GEMV per token.
int draco_enqueue_gemm(const DracoMat& m, const float* X, int T, float* Y, uint8_t* digits, bool have_digits,
                       hipStream_t st);
// Y[t] for the tokens of every group against that group's W (same shape for all groups)
int draco_gemm_grouped_launch(GemmArgs& a, hipStream_t st);
