// gdn.h -- internal interface of the Gated-DeltaNet scan kernel (gdn.hip).
#pragma once
#include <hip/hip_runtime.h>

// floats per (token, V head) in GdnArgs::PSS (one per wave of the head's
// blocks); a split decode step fills 16
constexpr int GDN_PSS_STRIDE = 64;

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
    // decode step only (draco_gdn_step_launch): B and G are computed in the
    // kernel from the layer input, src/m6_layer.c:237-256
    const float* h1;         // [H] layer input (before the attention RMSNorm)
    const float* attn_norm;  // [H]
    const float* bw;         // [n_vh][H] beta projection (the reference's [H][n_vh], transposed)
    const float* aw;         // [n_vh][H] alpha projection
    const float* ssm_a;      // [n_vh]
    const float* ssm_dt;     // [n_vh]
    int H;                   // <= 4096, multiple of 4
    // nullable: the gates' two dots already formed ([n_vh] xn.beta_wt rows,
    // then [n_vh] xn.alpha_wt rows, by the in-projection launch); the kernel
    // then reads them instead of dotting h1 with bw / aw itself
    const float* glog;
    // column split: nspl blocks per V head (1, 2, 4 or 8; 0 = 1).  Above 1
    // the gated rms runs in a second launch (or in the consumer) and needs
    // PSS [T][n_vh][GDN_PSS_STRIDE] floats (the waves' partial sums).
    int nspl;
    float* PSS;
    // split only: leave ON = (o / sqrt(128)) * ssm_norm * silu(z) and PSS
    // for the consumer, which scales each head by its rms itself (the
    // ssm_out GEMV's GNORM prologue) instead of a k_gdn_gnorm launch
    bool defer_gnorm;
};

// blocks per V head for the decode step / for scans of several tokens
// (draco_set_gdn_split changes them)
int draco_gdn_split(bool decode);

int draco_gdn_scan_launch(const GdnArgs& a, hipStream_t st);
// One decode token (T must be 1): the scan step with beta = sigmoid(xn.bw),
// decay = exp(softplus(xn.aw + dt) * a), xn = rms(h1) * attn_norm (eps 1e-6).
int draco_gdn_step_launch(const GdnArgs& a, hipStream_t st);

// State residency shared by m6_gdn_attn (abi_qwen.cpp) and m6_gdn_scan
// (abi_gdn.cpp).  The per-layer GDN op keeps the caller's ssm / tail on the
// device and writes back only a sample of the state; a scan on the same
// arrays must start from the device state.  draco_gdn_state_current returns
// true with the mirrors when the caller's ssm still carries the op's last
// written-back sample (the device holds the current state); otherwise false,
// and the op's record is dropped so that its next call uploads the caller's
// arrays.  draco_gdn_state_written records, after a scan on those mirrors
// wrote the whole state back to the caller, the sample the caller now holds.
bool draco_gdn_state_current(const float* ssm, const float* tail, size_t ns, size_t nt, float** dS, float** dT);
void draco_gdn_state_written(const float* ssm, const float* dS);
