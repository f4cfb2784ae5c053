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

// ---- fused segment GEMV --------------------------------------------------
// One launch computes several matrices (segments) that share the input x.
// Q4_K and Q6_K segments may be mixed in one launch; Q8_0 segments must all be
// Q8_0.
// Optional prologue: x <- x * (1/sqrt(mean(x^2)+eps)) * norm_w (RMSNorm,
// src/m6_engine.c:31-37), computed by every block.  Per-segment epilogue:
enum {
    EPI_STORE = 0,      // y[r] = dot
    EPI_RESID = 1,      // y[r] = yadd[r] + dot   (y may alias yadd)
    EPI_ROPE_Q = 2,     // pairs (2i, 2i+1) rotated by the rope table -> y
    EPI_ROPE_K = 3,     // rotated pairs -> kcache row T
    EPI_V_APPEND = 4,   // -> vcache row T
    EPI_SWIGLU = 5,     // dual segment: y[r] = silu(dot_gate) * dot_up  (seg i = gate, seg i+1 = up)
    EPI_ARGMAX = 6,     // y[r] = dot, per-block argmax partials, then a finalize launch
                        // writes tokens[*cursor + 1] and advances the token state
};

struct SegDesc {
    const uint8_t* base;
    DracoLayout L;
    float* y;
    const float* yadd;
    int epi;
    int row0, row1;   // rows computed: [row0, row1); row1 == 0 means n_out
    // filled by draco_seg_launch
    int first_block;  // Q8_0 path: first grid block of this segment
    int n_blocks;
    int first_tile;   // Q4_K/Q6_K path: first global tile index of this segment
    int n_tiles;
    int tile0;        // first 16-row tile of the row range
};

constexpr int SEG_MAX = 4;

struct SegLaunch {
    SegDesc seg[SEG_MAX];
    int nseg;
    int total_tiles;      // filled by draco_seg_launch (Q4_K/Q6_K path)
    int n_in;
    const float* x;
    const float* norm_w;  // nullable
    // 0 none; 1 RMSNorm of x (norm_w, eps); 2 (Q4_K / Q6_K, one EPI_RESID
    // segment) the GDN gated rms of 128-wide groups: x = the scan's gated
    // output, scaled per group by rsqrt(sum of the group's 16 partial sums of
    // squares in kc [group][64] / 128 + eps); 3 (Q4_K / Q6_K) RMSNorm of
    // the pending residual x + p0 + p1, the two split-K
    // partials p at am_val ([2][n_in]), the sum stored to xn_out by block 0
    int do_norm;
    // 2: split-K (Q4_K / Q6_K, one EPI_STORE segment over the whole matrix,
    // do_norm 0 or 2, row widths draco_dq_ksplit_waves accepts):
    // y[r] = the first half's dot, y[n_out + r] = the second half's
    int ksplit;
    float eps;
    float* xn_out;        // nullable: block 0 writes the normalised x here (do_norm 3: the raw x + p0 + p1)
    // rope / KV epilogue context
    const float* rope_tab;  // [pos][rot/2][cos, sin]
    const int* state;       // [pos, tlen per layer ...]
    int layer;
    int head_dim, rot, kv_dim;
    float* kc;
    float* vc;
    // argmax epilogue context
    float* am_val;      // [n_blocks] partials
    int* am_idx;
    int* tokens;
    const int* cursor;  // token written to tokens[*cursor + 1], then *cursor += 1
    int* advance_state; // nullable: pos and every layer's tlen += 1
    int advance_layers;
    const uint8_t* emb; // with emb_out set: the new token's row of emb (layout emb_L) -> emb_out
    DracoLayout emb_L;
    float* emb_out;
    // Row dots riding on a normalising launch (do_norm 1 or 3, two or more
    // Q4_K / Q6_K store or residual segments, no SwiGLU pair, not split-K,
    // rows of 8 to 16 super-blocks): the last
    // 2 gdot_n blocks of the grid each dot one fp32 row -- rows [0, gdot_n)
    // of gdot_w0, then [0, gdot_n) of gdot_w1, n_in wide, contiguous -- with
    // the normalised x (x * norm_w * 1/rms) into gdot_out[0 .. 2 gdot_n).
    // draco_seg_launch sets gdot_done when the launch computed them (a
    // launch that cannot -- too few blocks, n_in above 8 floats per thread,
    // another epilogue -- leaves it 0 and the caller computes them itself).
    const float* gdot_w0;
    const float* gdot_w1;
    float* gdot_out;
    int gdot_n;
    int gdot_done;
};

// Builds grid ranges for every segment and launches the fused kernel.
int draco_seg_launch(SegLaunch& a, hipStream_t st);

// Launch shape of a Q4_K / Q6_K segment launch (k_dq), chosen on the host
// from the row width, the tile count and the variant.  Every shape returned
// keeps the kernel's coverage invariants: the prologue digitises (and
// normalises) every input value an item multiplies, the items of a tile (or
// of a split-K half) cover every super-block of its rows exactly once, the
// row-dot loads cover n_in, and the LDS image fits a CU.
struct DqShape {
    int nw;      // waves per block
    int grid;    // blocks
    int ipt1;    // one item per wave and tile (rows of at most nw super-blocks)
    int ks;      // split-K launch (halves of each row)
    int gd;      // row dots ride on the launch
    int xp_max;  // float4s of x per thread the prologue holds
};
// variant: dual = SwiGLU pair; ksplit = 2 for split-K; do_norm as SegLaunch;
// gd_n = rows per weight of the row dots the caller asks for (0: none;
// segment kinds already checked); cus = compute units of the device.
// Returns 0 with the shape, or -1 when no k_dq instance serves the request.
int draco_dq_shape(int n_in, int tiles, bool dual, int ksplit, int do_norm, int gd_n, int cus, DqShape& s);
// Waves of the split-K instance for rows n_in wide (do_norm 0 or 2), 0 if
// none covers them; callers that plan a split-K launch ask this first.
int draco_dq_ksplit_waves(int n_in, int do_norm);
