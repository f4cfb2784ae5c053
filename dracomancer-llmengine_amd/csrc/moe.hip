// moe.hip -- top-k MoE expert FFN for decode and the grouped expert GEMV (gfx950).
//
// Reference: m6_granite_moe / topk_idx / moe_experts, src/m6_layer.c:699-821:
//   logits[e] = x . gate_inp[e]; probs = softmax(logits); idx = stable top-k
//   (largest first, lowest index on ties); wtop = probs[idx] / max(sum, 2^-14);
//   act_j = silu(W_gate[e_j] x) * (W_up[e_j] x); out = sum_j wtop_j * (W_down[e_j] act_j).
// and the grouped expert GEMV m5_gemvn_q4k/q6k, src/m5/m5_batch8_k.c:80-183:
//   y[j] = W[idx[j]] . x_j, x_j = x + j*x_stride.
//
// Launches for one MoE FFN:
//   k_moe_logits   one block per expert row of the fp32 router (tree sum);
//                  optionally the layer's RMSNorm first (xn stored by block 0)
//   k_moe_grp      ROUTE: every block recomputes softmax / top-k / weights from
//                  the logits (softmax by one wave, top-k as a parallel rank of
//                  every expert, the bases read ahead) and runs the selected experts'
//                  gate and up tiles together (16 rows x 256 values per item,
//                  int8 MFMA on the digits of x as in gemv.hip) with a SwiGLU
//                  epilogue into act[j]; block 0 publishes the routing.
//   k_moe_down     one output tile per block, wave j = selected expert j over
//                  its act_j digits; the epilogue forms sum_j wtop_j * y_j in j
//                  order, so the combine needs no extra pass.
// k_moe_grp without ROUTE is the grouped GEMV (shared x, or per-expert x for up
// to MOE_XPER_MAX experts per launch).
//
// Numerics: the router sums in a wave tree and the softmax sum in a wave tree
// (the reference sums sequentially), so logits and weights agree to fp32
// rounding; top-k can differ from the reference only when two probabilities
// are within that rounding of each other.
#include <hip/hip_runtime.h>

#include <mutex>

#include "moe.h"
#include "tile_frag.h"

namespace {

constexpr int XP_MAXV = 4;

// One block per router row: every thread's loads are issued together (up to
// 4 float4 pairs per step), then a wave-tree sum and the 4 wave sums in order.
// NORM (n_in <= 4096, one step): x is the layer input and every block first
// forms xn = (x * rms^-1) * norm_w itself (the same sums in every block, so
// every block gets the same xn); block 0 also stores xn for the expert
// launches, which then need no RMSNorm launch of their own.
// PRES (with NORM): x is a pending residual, x + pend[0..n_in) +
// pend[n_in..2 n_in) (PRES 1: the split-K partials of the o projection) or
// x + 2^-32 pend_i (PRES 2: the fused attention merge + o projection's int64
// fixed-point sums, a flag at [n_in] making the input NaN), formed in every
// block; block 0 also stores the sum to xs_out (the residual of the expert
// down launch).
// The pointers the first loads need lead the arguments (the first 14
// dwords arrive in SGPRs), and the flag is read by a vector load, so no
// argument or flag load is waited for before the x and row requests.
template <bool NORM, int PRES = 0>
__global__ __launch_bounds__(256) void k_moe_logits(const float* __restrict__ x, const float* __restrict__ pend,
                                                    const float* __restrict__ norm_w, const float* __restrict__ gi,
                                                    int n_in, int n_exp, float* __restrict__ logits, float eps,
                                                    float* __restrict__ xn_out, float* __restrict__ xs_out) {
    __shared__ float part[4], sq[4];
    constexpr int U = 4;
    const int e = blockIdx.x, tid = threadIdx.x;
    const float* w = gi + (size_t)e * n_in;
    float acc = 0.f;
    for (int i0 = tid * 4; i0 < n_in; i0 += U * 1024) {
        float4 a[U], b[U], nw[U], p0[U], p1[U];
        longlong2 q0[PRES == 2 ? U : 1], q1[PRES == 2 ? U : 1];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = i0 + u * 1024;
            a[u] = i < n_in ? ld4(x + i) : make_float4(0.f, 0.f, 0.f, 0.f);
            b[u] = i < n_in ? ld4(w + i) : make_float4(0.f, 0.f, 0.f, 0.f);
            if (NORM) nw[u] = i < n_in ? ld4(norm_w + i) : make_float4(0.f, 0.f, 0.f, 0.f);
            if (PRES == 1) {
                p0[u] = i < n_in ? ld4(pend + i) : make_float4(0.f, 0.f, 0.f, 0.f);
                p1[u] = i < n_in ? ld4(pend + n_in + i) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
            if constexpr (PRES == 2) {
                const int ic = i < n_in ? i : 0;
                const longlong2* A = reinterpret_cast<const longlong2*>(pend) + ic / 2;
                q0[u] = A[0];
                q1[u] = A[1];
            }
        }
        // the flag after the batch's loads (a vector load: it is waited for
        // where it is used, behind them)
        const long long pflag = PRES == 2 ? load_flag(reinterpret_cast<const long long*>(pend) + n_in) : 0;
        if (PRES) {
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = i0 + u * 1024;
                if constexpr (PRES == 1) {
                    a[u].x = (a[u].x + p0[u].x) + p1[u].x;
                    a[u].y = (a[u].y + p0[u].y) + p1[u].y;
                    a[u].z = (a[u].z + p0[u].z) + p1[u].z;
                    a[u].w = (a[u].w + p0[u].w) + p1[u].w;
                } else if (i < n_in) {
                    constexpr float S = 2.3283064365386963e-10f;  // 2^-32
                    if (pflag) {
                        a[u].x = a[u].y = a[u].z = a[u].w = __builtin_nanf("");
                    } else {
                        a[u].x += (float)q0[u].x * S; a[u].y += (float)q0[u].y * S;
                        a[u].z += (float)q1[u].x * S; a[u].w += (float)q1[u].y * S;
                    }
                }
                if (e == 0 && i < n_in) *reinterpret_cast<float4*>(xs_out + i) = a[u];
            }
        }
        if (NORM) {
            float ss = 0.f;
#pragma unroll
            for (int u = 0; u < U; u++) {
                ss = fmaf(a[u].x, a[u].x, ss);
                ss = fmaf(a[u].y, a[u].y, ss);
                ss = fmaf(a[u].z, a[u].z, ss);
                ss = fmaf(a[u].w, a[u].w, ss);
            }
            ss = wave_sum(ss);
            if ((tid & 63) == 0) sq[tid >> 6] = ss;
            lds_barrier();
            const float inv = 1.f / sqrtf(((sq[0] + sq[1]) + (sq[2] + sq[3])) / (float)n_in + eps);
#pragma unroll
            for (int u = 0; u < U; u++) {
                a[u].x = a[u].x * inv * nw[u].x;
                a[u].y = a[u].y * inv * nw[u].y;
                a[u].z = a[u].z * inv * nw[u].z;
                a[u].w = a[u].w * inv * nw[u].w;
                const int i = i0 + u * 1024;
                if (e == 0 && i < n_in) *reinterpret_cast<float4*>(xn_out + i) = a[u];
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            acc = fmaf(a[u].x, b[u].x, acc);
            acc = fmaf(a[u].y, b[u].y, acc);
            acc = fmaf(a[u].z, b[u].z, acc);
            acc = fmaf(a[u].w, b[u].w, acc);
        }
    }
    acc = wave_sum(acc);
    if ((tid & 63) == 0) part[tid >> 6] = acc;
    lds_barrier();
    if (tid == 0) logits[e] = (part[0] + part[1]) + (part[2] + part[3]);
}

// Routing (src/m6_layer.c:774-821) in two parallel steps instead of n_used
// sequential argmax rounds.  softmax_wave: one wave turns the logits into
// probabilities sp[0, n_exp) (max and sum by wave trees; sp[n_exp, 512) =
// -1, below every probability).  rank_part: the rank of expert e is the
// number of experts ahead of it in the reference's stable order (higher
// probability, or the same probability and a lower index); the ranks are a
// permutation of [0, n_exp), so the experts of rank < n_used are exactly the
// sequential top-k, rank = slot.  Four adjacent lanes count one expert's
// rank over a quarter of the experts each and add their counts with DPP.
__device__ __forceinline__ void softmax_wave(const float* __restrict__ logits, int n_exp, float* sp) {
    constexpr int PER = MOE_EXP_MAX / 64;
    const int lane = threadIdx.x & 63;
    float p[PER];
    float mx = -1e30f;
#pragma unroll
    for (int q = 0; q < PER; q++) {
        const int e = lane + 64 * q;
        p[q] = e < n_exp ? logits[e] : -1e30f;
        mx = fmaxf(mx, p[q]);
    }
    mx = wave_max(mx);
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < PER; q++) {
        const int e = lane + 64 * q;
        if (e < n_exp) {
            p[q] = expf(p[q] - mx);
            s += p[q];
        }
    }
    const float inv = 1.f / wave_sum(s);
#pragma unroll
    for (int q = 0; q < PER; q++) sp[lane + 64 * q] = lane + 64 * q < n_exp ? p[q] * inv : -1.f;
}

// experts ahead of e among sp[f0, f0 + span) (span a multiple of 4; entries
// past n_exp are -1 and never ahead)
__device__ __forceinline__ int rank_part(const float* sp, int e, int f0, int span) {
    const float pe = sp[e];
    const float4* s4 = reinterpret_cast<const float4*>(sp);
    int r = 0;
#pragma unroll 4
    for (int f = f0; f < f0 + span; f += 4) {
        const float4 v = s4[f >> 2];
        r += (v.x > pe || (v.x == pe && f < e)) + (v.y > pe || (v.y == pe && f + 1 < e)) +
             (v.z > pe || (v.z == pe && f + 2 < e)) + (v.w > pe || (v.w == pe && f + 3 < e));
    }
    return r;
}

// Grouped expert GEMV over 16-row tiles: tile T -> slot s = T / tpe, local
// tile T % tpe of expert e_s.  ROUTE: e_s from the routing prologue, gate/up
// (DUAL) with SwiGLU into a.act; otherwise e_s = a.idx[s] and y[s][row].
// XPER: slot s reads x + s * x_stride (digits of every slot in LDS).
template <int NW, int FM, bool DUAL, bool XPER, bool ROUTE>
// The prologue's arguments come first as scalars the dispatcher preloads
// into SGPRs (a struct argument is never preloaded): x, the norm weight
// (null: none), the logits, the three expert base tables, the width and the
// expert count.
__global__ __launch_bounds__(64 * NW) void k_moe_grp(const float* __restrict__ px, const float* __restrict__ pnw,
                                                     const float* __restrict__ plog,
                                                     const uint8_t* const* __restrict__ pb0,
                                                     const uint8_t* const* __restrict__ pb1,
                                                     const uint8_t* const* __restrict__ pb2, int pn_in, int pn_exp,
                                                     const MoeArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int NT = 64 * NW;
    constexpr size_t IB = FM == 1 ? DRACO_Q4T_ITEM : DRACO_Q6T_ITEM;
    const int n_in = pn_in, nb = n_in >> 8, ng = n_in >> 4, n4 = n_in >> 2;
    const int nx = XPER ? a.n_slots : 1;  // digit sets
    int8_t* xd = reinterpret_cast<int8_t*>(smem);                            // [nx][ng][4][16]
    int8_t* zero = xd + (size_t)nx * ng * 64;                                // 1 KB of zeros
    float2* xsm = reinterpret_cast<float2*>(zero + 1024);                    // [nx][ng]
    float* red = reinterpret_cast<float*>(xsm + (size_t)nx * ng);            // [2][NW][16] (+ norm)
    int* sidx = reinterpret_cast<int*>(red + 2 * NW * 16 + 64);              // [MOE_USED_MAX]
    float* swt = reinterpret_cast<float*>(sidx + MOE_USED_MAX);
    const uint8_t** sb0 = reinterpret_cast<const uint8_t**>(swt + MOE_USED_MAX);  // [MOE_USED_MAX] bases
    const uint8_t** sb1 = sb0 + MOE_USED_MAX;
    const uint8_t** sb2 = sb1 + MOE_USED_MAX;  // block 0: the selected experts' down bases (published)
    float* sp = reinterpret_cast<float*>(sb2 + MOE_USED_MAX);                      // [MOE_EXP_MAX] probabilities

    const int tid = threadIdx.x, lane = tid & 63, j = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int bx = blockIdx.x;

    // x loads first (independent of the routing)
    float4 xv[XP_MAXV], wv[XP_MAXV];
    const int nvals4 = nx * n4;
#pragma unroll
    for (int q = 0; q < XP_MAXV; q++) {
        const int i4 = tid + q * NT;
        if (i4 < nvals4) {
            const int s = XPER ? i4 / n4 : 0, o = i4 - s * n4;
            xv[q] = ld4(px + (size_t)s * a.x_stride + 4 * o);
            if (pnw) wv[q] = ld4(pnw + 4 * o);
        }
    }
    // routing / expert bases
    if (ROUTE) {
        // expert e = tid / 4 + k * EPP is ranked by lanes 4e'..4e'+3 (part
        // tid % 4); part 0 reads its bases while wave 0 reads the logits.
        // Slots default to expert 0 (every slot is overwritten below unless
        // the probabilities hold a NaN, which then cannot index out of range)
        constexpr int EPP = NT / 4, NPASS = (MOE_EXP_MAX + EPP - 1) / EPP;
        const int part = tid & 3;
        // Block 0 also reads the down bases it publishes, with the others (a
        // read after the ranking would add a memory round trip to block 0)
        const uint8_t* rb0[NPASS];
        const uint8_t* rb1[NPASS];
        const uint8_t* rb2[NPASS];
#pragma unroll
        for (int k = 0; k < NPASS; k++) {
            const int e = (tid >> 2) + k * EPP;
            const bool mine = part == 0 && e < pn_exp;
            rb0[k] = mine ? pb0[e] : nullptr;
            rb1[k] = (DUAL && mine) ? pb1[e] : nullptr;
            rb2[k] = (bx == 0 && mine) ? pb2[e] : nullptr;
        }
        const int n_slots = a.n_slots;  // read after the loads above are issued
        if (tid < n_slots) {
            sidx[tid] = 0;
            swt[tid] = 0.f;
            sb0[tid] = pb0[0];
            if (DUAL) sb1[tid] = pb1[0];
            if (bx == 0) sb2[tid] = pb2[0];
        }
        if (w == 0) softmax_wave(plog, pn_exp, sp);
        lds_barrier();
        const int span = ((pn_exp + 15) >> 4) << 2;  // a quarter, rounded up to whole float4s
#pragma unroll
        for (int k = 0; k < NPASS; k++) {
            if (k * EPP >= pn_exp) break;  // uniform
            const int e = (tid >> 2) + k * EPP;
            int r = e < pn_exp ? rank_part(sp, e, part * span, span) : 0;
            r = group_reduce<4>(r, OpAdd{});
            if (part == 0 && e < pn_exp && r < n_slots) {
                sidx[r] = e;
                swt[r] = sp[e];
                sb0[r] = rb0[k];
                if (DUAL) sb1[r] = rb1[k];
                if (bx == 0) sb2[r] = rb2[k];
            }
        }
    } else if (tid < a.n_slots) {
        sb0[tid] = pb0[tid];
        if (DUAL) sb1[tid] = pb1[tid];
    }
    for (int i = tid; i < 256; i += NT) reinterpret_cast<uint32_t*>(zero)[i] = 0u;
    lds_barrier();
    // the tile walk (its arguments read after the prologue's loads are issued)
    const int G = gridDim.x;
    const int n_slots = a.n_slots, tpe = a.n_out_e >> 4;
    const int total = n_slots * tpe;
    const int ipt = (nb + NW - 1) / NW;
    const int my_tiles = bx < total ? (total - bx + G - 1) / G : 0;
    const int n_items = my_tiles * ipt;

    // the slots' bases, one per lane (n_slots <= MOE_USED_MAX = 64)
    static_assert(MOE_USED_MAX <= 64, "one slot per lane");
    const int ls = lane < n_slots ? lane : 0;
    const uint8_t* lb0 = sb0[ls];
    const uint8_t* lb1 = DUAL ? sb1[ls] : lb0;
    auto load = [&](int T, int b, Frag& f, Frag& f2) {
        const int s = T / tpe, lt = T - s * tpe;
        const size_t off = ((size_t)lt * nb + b) * IB;
        const uint8_t* p0 = lane_ptr(lb0, s) + off;
        if (FM == 1) load_q4b(p0, lane, f);
        else load_q6b(p0, lane, f);
        if (DUAL) {
            const uint8_t* p1 = lane_ptr(lb1, s) + off;
            if (FM == 1) load_q4b(p1, lane, f2);
            else load_q6b(p1, lane, f2);
        }
    };
    Frag P0, P1, Q0, Q1;
    int ct = bx, cb = w, cp = 0;
    load(ct < total ? ct : total - 1, cb < nb ? cb : nb - 1, P0, Q0);

    // digits (RMSNorm first when asked; one norm for the shared x)
    float inv = 1.f;
    if (a.do_norm) {
        float ss = 0.f;
#pragma unroll
        for (int q = 0; q < XP_MAXV; q++)
            if (tid + q * NT < n4) {
                const float4 v = xv[q];
                ss = fmaf(v.x, v.x, ss);
                ss = fmaf(v.y, v.y, ss);
                ss = fmaf(v.z, v.z, ss);
                ss = fmaf(v.w, v.w, ss);
            }
        ss = wave_sum(ss);
        if (lane == 0) red[2 * NW * 16 + w] = ss;
        lds_barrier();
        float tot = 0.f;
#pragma unroll
        for (int i = 0; i < NW; i++) tot += red[2 * NW * 16 + i];
        inv = 1.f / sqrtf(tot / (float)n_in + a.eps);
    }
#pragma unroll
    for (int q = 0; q < XP_MAXV; q++) {
        const int i4 = tid + q * NT;
        if (i4 >= nvals4) break;
        float4 v = xv[q];
        if (a.do_norm) {
            if (pnw) {
                const float4 nw = wv[q];
                v.x = v.x * inv * nw.x; v.y = v.y * inv * nw.y; v.z = v.z * inv * nw.z; v.w = v.w * inv * nw.w;
            } else {
                v.x *= inv; v.y *= inv; v.z *= inv; v.w *= inv;
            }
        }
        const int s = XPER ? i4 / n4 : 0, o = i4 - s * n4;
        digits4(v, o, xd + (size_t)s * ng * 64, xsm + (size_t)s * ng);
    }
    lds_barrier();

    const bool adig = (j >> 2) == g;
    const int gl4 = 4 * (g >> 1) + (g & 1), gl6 = 8 * (g >> 1) + (g & 1);
    float aD = 0.f, aM = 0.f, aD2 = 0.f, aM2 = 0.f;
    auto step = [&](int i, Frag& cur, Frag& nxt, Frag& cur2, Frag& nxt2) {
        int nt = ct, nbk = cb + NW, np = cp + 1;
        if (np == ipt) {
            np = 0;
            nbk = w;
            nt = ct + G;
        }
        const bool real = i + 1 < n_items && nbk < nb;
        load(real ? nt : ct, real ? nbk : (w < nb ? w : nb - 1), nxt, nxt2);
        if (cb < nb) {
            const int s = XPER ? ct / tpe : 0;
            const int8_t* xs = xd + (size_t)s * ng * 64;
            const float2* ms = xsm + (size_t)s * ng;
            float cD, cM, cD2 = 0.f, cM2 = 0.f;
            if (FM == 1) {
                const int8_t* xa = adig ? xs + (size_t)cb * 1024 + (gl4 * 4 + (j & 3)) * 16 : zero;
                const float2 r = dot_q4(cur, xa, ms, cb * 16 + gl4, g);
                cD = r.x;
                cM = r.y;
                if (DUAL) {
                    const float2 r2 = dot_q4(cur2, xa, ms, cb * 16 + gl4, g);
                    cD2 = r2.x;
                    cM2 = r2.y;
                }
            } else {
                const int8_t* xa = adig ? xs + (size_t)cb * 1024 + (gl6 * 4 + (j & 3)) * 16 : zero;
                cD = dot_q6(cur, xa, ms, cb * 16 + gl6);
                cM = 0.f;
                if (DUAL) cD2 = dot_q6(cur2, xa, ms, cb * 16 + gl6);
            }
            aD += cD;
            aM += cM;
            if (DUAL) {
                aD2 += cD2;
                aM2 += cM2;
            }
        }
        if (cp == ipt - 1) {
            float acc = aD - aM, acc2 = aD2 - aM2;
            acc = rows_sum(acc);
            if (DUAL) acc2 = rows_sum(acc2);
            if (lane < 16) {
                red[w * 16 + j] = acc;
                if (DUAL) red[(NW + w) * 16 + j] = acc2;
            }
            lds_barrier();
            if (tid < 16) {
                float v = 0.f, v2 = 0.f;
#pragma unroll
                for (int q = 0; q < NW; q++) {
                    v += red[q * 16 + tid];
                    if (DUAL) v2 += red[(NW + q) * 16 + tid];
                }
                const int s = ct / tpe, row = (ct - s * tpe) * 16 + tid;
                float* y = (DUAL ? a.act : a.y) + (size_t)s * a.n_out_e;
                if (DUAL) y[row] = (v / (1.f + expf(-v))) * v2;
                else y[row] = v;
            }
            lds_barrier();
            aD = aM = aD2 = aM2 = 0.f;
        }
        ct = nt;
        cb = nbk;
        cp = np;
    };
    for (int i = 0; i < n_items; i += 2) {
        step(i, P0, P1, Q0, Q1);
        if (i + 1 >= n_items) break;
        step(i + 1, P1, P0, Q1, Q0);
    }
    // publish the routing (weights renormalised in slot order) for the down
    // launch, last: stores before the first weight requests would make them
    // wait for the stores (the LDS routing tables are not rewritten above)
    if (ROUTE && bx == 0 && tid < n_slots) {
        float ws = 0.f;
        for (int t = 0; t < n_slots; t++) ws += swt[t];
        if (ws < 6.103515625e-5f) ws = 6.103515625e-5f;
        a.sel[tid] = sidx[tid];
        a.selw[tid] = swt[tid] / ws;
        a.seld[tid] = sb2[tid];
    }
}

// Down projection of the routed experts plus the weighted combine.  Block =
// one 16-row output tile at a time; wave j (< n_used) = expert slot j, which
// walks the nb super-blocks of its down rows over act_j's digits, three
// super-blocks in flight; the first three are requested before act_j is
// read and digitized.  SPLIT: twice the blocks, block b = tile b % tiles of
// half h = b / tiles, whose waves take slots h n/2 .. h n/2 + n/2 - 1 and
// whose weighted sum (slot order) goes to out[h n_out + row], no residual:
// the consumer forms resid + half 0 + half 1.
template <int NW, int FM, bool SPLIT = false>
// Leading scalars as k_moe_grp's (preloaded): the selected experts' down
// bases, the activations, the routing weights, the output and residual, the
// inner width, the output rows and the slot count.
__global__ __launch_bounds__(64 * NW) void k_moe_down(const uint8_t* const* __restrict__ pseld,
                                                      const float* __restrict__ pact, const float* __restrict__ pselw,
                                                      float* __restrict__ pout, const float* __restrict__ presid,
                                                      int pinter, int pn_out, int pn_slots, const MoeArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int NT = 64 * NW;
    constexpr size_t IB = FM == 1 ? DRACO_Q4T_ITEM : DRACO_Q6T_ITEM;
    const int inter = pinter, nb = inter >> 8, ng = inter >> 4, n4 = inter >> 2;
    const int tiles = pn_out >> 4;
    const int half = SPLIT ? (int)blockIdx.x / tiles : 0;
    const int n_used = SPLIT ? pn_slots / 2 : pn_slots;  // this block's slots
    const int so = half * n_used;                            // its first slot
    int8_t* xd = reinterpret_cast<int8_t*>(smem);                      // [n_used][ng][64]
    int8_t* zero = xd + (size_t)n_used * ng * 64;
    float2* xsm = reinterpret_cast<float2*>(zero + 1024);              // [n_used][ng]
    float* red = reinterpret_cast<float*>(xsm + (size_t)n_used * ng);  // [NW][16]
    float* swt = red + NW * 16;                                        // [MOE_USED_MAX]

    const int tid = threadIdx.x, lane = tid & 63, j = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool active = w < n_used;
    // this wave's expert base (routing published by k_moe_grp)
    const uint8_t* base = pseld[so + (active ? w : 0)];
    // item b of tile t (b clamped: a repeated item is already in flight)
    auto ld = [&](int t, int b, Frag& f) {
        const uint8_t* p = base + ((size_t)t * nb + (b < nb ? b : nb - 1)) * IB;
        if (FM == 1) load_q4b(p, lane, f);
        else load_q6b(p, lane, f);
    };
    // act loads (all slots; every float4 of a batch requested together,
    // clamped index) and the combine weight before the expert weights: the
    // act arrives first, so the digits are formed while the weights stream
    const int nvals4 = n_used * n4;
    constexpr int AB = 4;
    float4 av[AB];
    auto act_batch = [&](int b0) {
#pragma unroll
        for (int k = 0; k < AB; k++) {
            const int i4 = b0 + tid + k * NT, ic = i4 < nvals4 ? i4 : nvals4 - 1;
            const int s = ic / n4, o = ic - s * n4;
            av[k] = ld4(pact + (size_t)(so + s) * inter + 4 * o);
        }
    };
    act_batch(0);
    const float swv = pselw[so + (tid < n_used ? tid : n_used - 1)];
    // requested unconditionally (a wave past the used slots or a block past
    // the tiles re-reads real items), so the act waits above count exactly
    Frag P0, P1, P2;
    int t = SPLIT ? (int)blockIdx.x - half * tiles : (int)blockIdx.x;
    {
        const int tl = t < tiles ? t : tiles - 1;
        ld(tl, 0, P0);
        ld(tl, 1, P1);
        ld(tl, 2, P2);
    }
    for (int i = tid; i < 256; i += NT) reinterpret_cast<uint32_t*>(zero)[i] = 0u;
    for (int b0 = 0; b0 < nvals4; b0 += AB * NT) {
        if (b0 > 0) act_batch(b0);
#pragma unroll
        for (int k = 0; k < AB; k++) {
            const int i4 = b0 + tid + k * NT;
            if (i4 < nvals4) {
                const int s = i4 / n4, o = i4 - s * n4;
                digits4(av[k], o, xd + (size_t)s * ng * 64, xsm + (size_t)s * ng);
            }
        }
    }
    if (tid < n_used) swt[tid] = swv;
    lds_barrier();
    const bool adig = (j >> 2) == g;
    const int gl4 = 4 * (g >> 1) + (g & 1), gl6 = 8 * (g >> 1) + (g & 1);
    const int8_t* xs = xd + (size_t)(active ? w : 0) * ng * 64;
    const float2* ms = xsm + (size_t)(active ? w : 0) * ng;
    for (; t < tiles; t += gridDim.x) {
        float aD = 0.f, aM = 0.f;
        if (active) {
            auto dot = [&](const Frag& f, int b) {
                if (FM == 1) {
                    const int8_t* xa = adig ? xs + (size_t)b * 1024 + (gl4 * 4 + (j & 3)) * 16 : zero;
                    const float2 r = dot_q4(f, xa, ms, b * 16 + gl4, g);
                    aD += r.x;
                    aM += r.y;
                } else {
                    const int8_t* xa = adig ? xs + (size_t)b * 1024 + (gl6 * 4 + (j & 3)) * 16 : zero;
                    aD += dot_q6(f, xa, ms, b * 16 + gl6);
                }
            };
            const int tn = SPLIT ? tiles : t + (int)gridDim.x;  // the next tile's first items follow this tile's last
            for (int b = 0; b < nb; b += 3) {
                dot(P0, b);
                if (b + 3 < nb) ld(t, b + 3, P0);
                else if (tn < tiles) ld(tn, 0, P0);
                if (b + 1 < nb) {
                    dot(P1, b + 1);
                    if (b + 4 < nb) ld(t, b + 4, P1);
                    else if (tn < tiles) ld(tn, 1, P1);
                }
                if (b + 2 < nb) {
                    dot(P2, b + 2);
                    if (b + 5 < nb) ld(t, b + 5, P2);
                    else if (tn < tiles) ld(tn, 2, P2);
                }
            }
        }
        float acc = aD - aM;
        acc = rows_sum(acc);
        if (lane < 16) red[w * 16 + j] = acc;
        lds_barrier();
        if (tid < 16) {
            float o = 0.f;
            for (int s = 0; s < n_used; s++) o += swt[s] * red[s * 16 + tid];  // j order, like the reference
            const int row = t * 16 + tid;
            if (SPLIT) pout[(size_t)half * pn_out + row] = o;
            else pout[row] = presid ? presid[row] + o : o;
        }
        lds_barrier();
        if (SPLIT) break;  // one tile per block
    }
}

// Token-batched MoE (prefill): gather the token rows of every expert segment
// (src[row] = token or -1 for padding), and the deterministic scatter
// out[t] = sum_k w[t,k] * Yd[pos[t,k]] in k order (src/m6_moe_tok.c:148-159).
__global__ __launch_bounds__(256) void k_moe_gather(const float* __restrict__ X, int n_in, const int* __restrict__ src,
                                                    float* __restrict__ Xg) {
    const int row = blockIdx.x, t = src[row];
    for (int i = threadIdx.x * 4; i < n_in; i += 1024) {
        const float4 v = t >= 0 ? ld4(X + (size_t)t * n_in + i) : make_float4(0.f, 0.f, 0.f, 0.f);
        *reinterpret_cast<float4*>(Xg + (size_t)row * n_in + i) = v;
    }
}

__global__ __launch_bounds__(256) void k_moe_scatter(const float* __restrict__ Yd, int n_out, const int* __restrict__ pos,
                                                     const float* __restrict__ wt, int n_used, float* __restrict__ out) {
    const int t = blockIdx.x;
    for (int r = threadIdx.x; r < n_out; r += 256) {
        float o = 0.f;
        for (int k = 0; k < n_used; k++) {
            const int p = pos[t * n_used + k];
            if (p < 0) continue;
            o += wt[t * n_used + k] * Yd[(size_t)p * n_out + r];
        }
        out[(size_t)t * n_out + r] = o;
    }
}

int cu_count() {
    static int n = 0;
    static std::once_flag once;
    std::call_once(once, [] {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
    });
    return n;
}

template <class K>
void allow_big_lds(K kern) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024);
}

template <int NW, int FM, bool DUAL, bool XPER, bool ROUTE>
void launch_grp(const MoeArgs& a, int grid, size_t lds, hipStream_t st) {
    static std::once_flag once;
    std::call_once(once, [] { allow_big_lds(&k_moe_grp<NW, FM, DUAL, XPER, ROUTE>); });
    hipLaunchKernelGGL((k_moe_grp<NW, FM, DUAL, XPER, ROUTE>), dim3(grid), dim3(64 * NW), lds, st, a.x,
                       a.do_norm ? a.norm_w : nullptr, a.logits, a.base0, a.base1, a.base2, a.n_in, a.n_exp, a);
}

template <int NW, int FM, bool SPLIT = false>
void launch_down(const MoeArgs& a, int grid, size_t lds, hipStream_t st) {
    static std::once_flag once;
    std::call_once(once, [] { allow_big_lds(&k_moe_down<NW, FM, SPLIT>); });
    hipLaunchKernelGGL((k_moe_down<NW, FM, SPLIT>), dim3(grid), dim3(64 * NW), lds, st, a.seld, a.act, a.selw, a.out,
                       a.resid, a.inter, a.n_out, a.n_slots, a);
}

int grp_nw(int n_in) {
    const int nb = n_in / 256;
    int nw = nb >= 8 ? 8 : 4;
    while (n_in > XP_MAXV * 4 * 64 * nw && nw < 16) nw *= 2;
    return nw;
}

template <int NW>
int dispatch_grp(const MoeArgs& a, int fm, bool dual, bool xper, bool route, int grid, size_t lds, hipStream_t st) {
    if (route) {
        if (!dual) return -1;
        if (fm == 1) launch_grp<NW, 1, true, false, true>(a, grid, lds, st);
        else launch_grp<NW, 2, true, false, true>(a, grid, lds, st);
        return 0;
    }
    if (dual) {  // gate/up + SwiGLU of slots fixed by the host (m6_moe_batch4)
        if (xper) return -1;
        if (fm == 1) launch_grp<NW, 1, true, false, false>(a, grid, lds, st);
        else launch_grp<NW, 2, true, false, false>(a, grid, lds, st);
        return 0;
    }
    if (fm == 1) {
        if (xper) launch_grp<NW, 1, false, true, false>(a, grid, lds, st);
        else launch_grp<NW, 1, false, false, false>(a, grid, lds, st);
    } else {
        if (xper) launch_grp<NW, 2, false, true, false>(a, grid, lds, st);
        else launch_grp<NW, 2, false, false, false>(a, grid, lds, st);
    }
    return 0;
}

}  // namespace

int draco_moe_logits_launch(const float* x, const float* gate_inp, int n_exp, int n_in, float* logits,
                            hipStream_t st, const float* norm_w, float eps, float* xn_out, const float* pend,
                            float* xs_out, bool pend_fx) {
    if (n_exp < 1 || n_exp > MOE_EXP_MAX || n_in % 4) return -1;
    if (pend && (!norm_w || !xs_out)) return -1;
    if (norm_w) {
        if (n_in > 4096 || !xn_out) return -1;
        if (pend && pend_fx)
            hipLaunchKernelGGL((k_moe_logits<true, 2>), dim3(n_exp), dim3(256), 0, st, x, pend, norm_w, gate_inp,
                               n_in, n_exp, logits, eps, xn_out, xs_out);
        else if (pend)
            hipLaunchKernelGGL((k_moe_logits<true, 1>), dim3(n_exp), dim3(256), 0, st, x, pend, norm_w, gate_inp,
                               n_in, n_exp, logits, eps, xn_out, xs_out);
        else
            hipLaunchKernelGGL((k_moe_logits<true>), dim3(n_exp), dim3(256), 0, st, x, nullptr, norm_w, gate_inp,
                               n_in, n_exp, logits, eps, xn_out, nullptr);
        return 0;
    }
    hipLaunchKernelGGL((k_moe_logits<false>), dim3(n_exp), dim3(256), 0, st, x, nullptr, nullptr, gate_inp, n_in,
                       n_exp, logits, 0.f, nullptr, nullptr);
    return 0;
}

// ROUTE + DUAL (gate/up of the routed experts) or the plain grouped GEMV.
int draco_moe_grp_launch(MoeArgs& a, int fm, bool dual, bool xper, bool route, hipStream_t st) {
    const int n_in = a.n_in;
    if (n_in % 256 || a.n_out_e % 16 || a.n_slots < 1 || a.n_slots > MOE_USED_MAX) return -1;
    if (route && (a.n_exp < a.n_slots || a.n_exp > MOE_EXP_MAX)) return -1;
    const int nw = grp_nw(n_in);
    const int nx = xper ? a.n_slots : 1;
    if ((size_t)nx * (n_in / 4) > (size_t)XP_MAXV * 64 * nw) return -1;  // prologue capacity
    const size_t lds = (size_t)nx * (n_in / 16) * 72 + 1024 + (2 * 16 * 16 + 64) * 4 + MOE_USED_MAX * 32 +
                       MOE_EXP_MAX * 4;
    if (lds > 160 * 1024) return -1;
    const int total = a.n_slots * (a.n_out_e / 16);
    // ROUTE: every block repeats the routing (softmax + rank of the experts),
    // so at most one block per CU (configs[3] FFN, 384 tiles: 16.3 -> 15.7 us)
    const int cap = route ? cu_count() : cu_count() * (nw == 4 ? 4 : (nw == 8 ? 2 : 1));
    const int grid = total < cap ? total : cap;
    if (nw == 4) return dispatch_grp<4>(a, fm, dual, xper, route, grid, lds, st);
    if (nw == 8) return dispatch_grp<8>(a, fm, dual, xper, route, grid, lds, st);
    return dispatch_grp<16>(a, fm, dual, xper, route, grid, lds, st);
}

int draco_moe_xper_slots(int n_in) {
    if (n_in <= 0 || n_in % 256) return 0;
    return (XP_MAXV * 64 * grp_nw(n_in) * 4) / n_in;
}

namespace {

// One k_moe_down launch over at most 16 slots (a wave per slot).
int moe_down_chunk(const MoeArgs& a, int fm, hipStream_t st) {
    const int nw = a.n_slots <= 4 ? 4 : (a.n_slots <= 8 ? 8 : 16);
    if (a.n_slots * (a.inter / 4) > 4096 * 4) return -1;
    const size_t lds = (size_t)a.n_slots * (a.inter / 16) * 72 + 1024 + (size_t)nw * 16 * 4 + MOE_USED_MAX * 4;
    if (lds > 160 * 1024) return -1;
    const int tiles = a.n_out / 16;
    if (nw == 4) {
        if (fm == 1) launch_down<4, 1>(a, tiles, lds, st);
        else launch_down<4, 2>(a, tiles, lds, st);
    } else if (nw == 8) {
        if (fm == 1) launch_down<8, 1>(a, tiles, lds, st);
        else launch_down<8, 2>(a, tiles, lds, st);
    } else {
        if (fm == 1) launch_down<16, 1>(a, tiles, lds, st);
        else launch_down<16, 2>(a, tiles, lds, st);
    }
    return 0;
}

}  // namespace

// More than 16 selected experts (the reference serves up to 64,
// src/m6_layer.c:797): launches of 16 slots each, in slot order, the first
// adding the residual and each later one adding its sum to the output
// (out = ((resid + S_0..15) + S_16..31) + ...).
int draco_moe_down_launch(MoeArgs& a, int fm, hipStream_t st) {
    if (a.inter % 256 || a.n_out % 16 || a.n_slots < 1 || a.n_slots > MOE_USED_MAX) return -1;
    if (a.split) {
        // two halves of the slots, one launch of twice the tiles; each half's
        // weighted sum to out[h n_out ..] (no residual)
        const int nh = a.n_slots / 2;
        if (a.n_slots % 2 || nh > 8 || nh * (a.inter / 4) > 4096 * 4) return -1;
        const int nw = nh <= 4 ? 4 : 8;
        const size_t lds = (size_t)nh * (a.inter / 16) * 72 + 1024 + (size_t)nw * 16 * 4 + MOE_USED_MAX * 4;
        if (lds > 160 * 1024) return -1;
        const int grid = 2 * (a.n_out / 16);
        if (nw == 4) {
            if (fm == 1) launch_down<4, 1, true>(a, grid, lds, st);
            else launch_down<4, 2, true>(a, grid, lds, st);
        } else if (fm == 1) {
            launch_down<8, 1, true>(a, grid, lds, st);
        } else {
            launch_down<8, 2, true>(a, grid, lds, st);
        }
        return 0;
    }
    for (int c0 = 0; c0 < a.n_slots; c0 += 16) {
        MoeArgs c = a;
        c.n_slots = a.n_slots - c0 < 16 ? a.n_slots - c0 : 16;
        c.sel = a.sel + c0;
        c.selw = a.selw + c0;
        c.seld = a.seld + c0;
        c.act = a.act + (size_t)c0 * a.inter;
        if (c0 > 0) c.resid = a.out;
        if (int rc = moe_down_chunk(c, fm, st)) return rc;
    }
    return 0;
}

int draco_moe_gather_launch(const float* X, int n_in, const int* src, int rows, float* Xg, hipStream_t st) {
    if (n_in % 4 || rows < 1) return -1;
    hipLaunchKernelGGL(k_moe_gather, dim3(rows), dim3(256), 0, st, X, n_in, src, Xg);
    return 0;
}

int draco_moe_scatter_launch(const float* Yd, int n_out, const int* pos, const float* wt, int n_used, int T, float* out,
                             hipStream_t st) {
    if (T < 1) return -1;
    hipLaunchKernelGGL(k_moe_scatter, dim3(T), dim3(256), 0, st, Yd, n_out, pos, wt, n_used, out);
    return 0;
}
