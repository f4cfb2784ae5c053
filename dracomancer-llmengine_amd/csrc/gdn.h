// gdn.h -- internal interface of the Gated-DeltaNet scan kernel (gdn.hip).
#pragma once
#include <hip/hip_runtime.h>

struct GdnArgs {
    const float* QKV;       // [T][n_qkv]   (q heads, k heads, v heads; 128 each)
    const float* Z;         // [T][n_vh*128]
    const float* B;         // [T][n_vh]    beta
    const float* G;         // [T][n_vh]    decay (= exp(alpha))
    const float* conv;      // [n_qkv][4]
    const float* ssm_norm;  // [128]
    float* tail;            // [n_qkv][3]   conv history, updated
    float* S;               // [n_vh][128 k][128 v], updated
    float* ON;              // [T][n_vh*128]
    int T, n_qkv, n_vh, nhq;
};

int draco_gdn_scan_launch(const GdnArgs& a, hipStream_t st);
