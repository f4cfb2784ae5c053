// moe.h -- internal interface of the MoE kernels (moe.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "formats.h"

constexpr int MOE_EXP_MAX = 512;   // experts in the router (the reference's lg[512])
constexpr int MOE_USED_MAX = 64;   // selected experts / grouped slots per launch

struct MoeArgs {
    // activations
    const float* x;          // shared x, or slot j at x + j * x_stride
    long x_stride;           // floats (0: shared)
    const float* norm_w;     // RMSNorm of x in the prologue (do_norm)
    int do_norm;
    float eps;
    int n_in;                // rows' length of the grouped matrices
    int n_out_e;             // rows per grouped matrix
    int n_slots;             // selected experts (routed) or grouped slots
    // routing (k_moe_grp ROUTE)
    const float* logits;
    int n_exp;
    const uint8_t* const* base0;  // [n_exp] (routed) or [n_slots]: gate / grouped matrix bases (tile layout)
    const uint8_t* const* base1;  // [n_exp] up bases
    const uint8_t* const* base2;  // [n_exp] down bases
    int* sel;                // published routing: expert ids [n_used]
    float* selw;             // weights [n_used]
    const uint8_t** seld;    // down bases of the selected experts [n_used]
    // outputs
    float* act;              // routed: [n_used][n_out_e] SwiGLU activations
    float* y;                // grouped: [n_slots][n_out_e]
    // down + combine (k_moe_down)
    int inter;
    int n_out;
    float* out;
    const float* resid;      // optional: out = resid + sum
    int split;               // 1: two halves of the slots, sums to out[0..n_out) and out[n_out..2 n_out), no resid
};

// norm_w set (n_in <= 4096): x is normalised first, xn = (x * rms^-1) * norm_w
// (eps), and stored to xn_out for the expert launches.  pend (norm_w set):
// the input is x + pend[0..n_in) + pend[n_in..2 n_in), or with pend_fx
// x + 2^-32 pend_i (int64 fixed point, a flag at [n_in] making it NaN),
// stored to xs_out.
int draco_moe_logits_launch(const float* x, const float* gate_inp, int n_exp, int n_in, float* logits,
                            hipStream_t st, const float* norm_w = nullptr, float eps = 0.f,
                            float* xn_out = nullptr, const float* pend = nullptr, float* xs_out = nullptr,
                            bool pend_fx = false);
// fm: 1 = Q4_K, 2 = Q6_K.  route (+dual): gate/up of the routed experts;
// otherwise the grouped GEMV (xper: per-slot x).
int draco_moe_grp_launch(MoeArgs& a, int fm, bool dual, bool xper, bool route, hipStream_t st);
int draco_moe_down_launch(MoeArgs& a, int fm, hipStream_t st);
// slots per grouped launch when every slot has its own x of length n_in
int draco_moe_xper_slots(int n_in);

// The MoE FFN as an m6 ffn op's parameters (include/draco_hip.h DracoMoeP):
// m6_granite_moe's arguments (src/m6_layer.c:771) in one struct.
struct DracoMoeP {
    const uint64_t* ptrs;   // [3 * n_exp] host pointers: gate, up, down per expert
    const int* codes;       // [3 * n_exp]
    const float* gate_inp;  // [n_exp][n_in] fp32 router
    int n_exp, n_used, inter, n_in, n_out;
    float* scratch;         // the reference op's host scratch (unused here)
};

// One decoder layer's MoE FFN for the device decode loop (abi_m6.cpp): the
// expert set resolved once, per-layer work buffers of its own (a captured
// graph keeps pointing at them).  nullptr + fail() on error.
struct MoeLayer;
MoeLayer* draco_moe_layer(const DracoMoeP* p);
// out = resid + MoE(RMSNorm(x) * norm_w), device pointers; out may alias x
// and resid (x is read by the norm launch before anything is written).
// With pend ([2][n_in], the o projection's split-K partials) the input is
// x + pend[0..n_in) + pend[n_in..2 n_in) (with pend_fx: the fused attention
// merge + o projection's int64 fixed-point sums, x + 2^-32 pend_i), formed by
// the router launch and stored to xs, which is then the residual (resid is
// not read); pend needs the router's RMSNorm prologue
// (draco_moe_layer_pend_ok).
// With split_out ([2][n_out]; an even number of selected experts, at most
// 16) the down launch writes the weighted sums of the two halves of the
// slots there instead of out = resid + sum: the caller's consumer forms
// resid + half 0 + half 1 (draco_moe_layer_split_ok).
int draco_moe_layer_enqueue(MoeLayer* m, const float* x, const float* norm_w, float eps, float* out,
                            const float* resid, hipStream_t st, const float* pend = nullptr, float* xs = nullptr,
                            bool pend_fx = false, float* split_out = nullptr);
bool draco_moe_layer_split_ok(const MoeLayer* m);
bool draco_moe_layer_pend_ok(const MoeLayer* m, const float* norm_w);
// out = resid + MoE(xn) for an input that is already normalised (the qwen35
// FFN input x2n, src/qwen35_engine.py:325)
int draco_moe_layer_enqueue_xn(MoeLayer* m, const float* xn, float* out, const float* resid, hipStream_t st);

// token-batched MoE helpers
int draco_moe_gather_launch(const float* X, int n_in, const int* src, int rows, float* Xg, hipStream_t st);
int draco_moe_scatter_launch(const float* Yd, int n_out, const int* pos, const float* wt, int n_used, int T, float* out,
                             hipStream_t st);
