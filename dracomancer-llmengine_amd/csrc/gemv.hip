// gemv.hip -- fp32-activation GEMV over block-quantized weights (gfx950).
//
//   y[r] = sum_k W[r][k] * x[k]
//
// Reference semantics: dot_row / m5_gemv_range, src/m5_kern_scalar.c:48-165
// (decoded weight w = d*sc*q - dmin*m for Q4_K, d*sc*(q-32) for Q6_K, d*q
// for Q8_0).  The summation order differs from the reference's sequential
// loop (a wave tree), so results agree to fp32 rounding, not bitwise.
//
// Mapping: one wave64 owns R consecutive rows.  A row is cut into "units"
// (16 quant bytes for Q4_K, 48 for Q6_K, one 32-value block for Q8_0); lane
// l takes units l, l+64, ...  Each unit's x slice is loaded once and reused
// for the wave's R rows (and for the paired row of a second matrix in the
// SwiGLU dual mode).  The block scale is applied once per 16/32 values to an
// inner dot of integer-valued weights:
//   Q4_K: d*sc_j*(sum q*x) - dmin*m_j*(sum x)
//   Q6_K: d*sc_g*((sum (q+32)*x) - 32*(sum x))
//   Q8_0: d*(sum q*x)
// which is the reference's per-weight expression regrouped.
//
// The fused segment kernel (k_seg) adds an RMSNorm prologue and epilogues
// (rope + KV append, residual add, SwiGLU, argmax) so a llama layer needs
// five launches instead of thirteen.
#include <hip/hip_runtime.h>

#include "dev_common.h"
#include "formats.h"
#include "gemv.h"

namespace {

constexpr int SEG_R = 2;                  // rows per wave in k_seg
constexpr int SEG_ROWS = 4 * SEG_R;       // rows per block (4 waves)

// ------------------------------------------------------------- traits --
struct FQ4K {
    static constexpr int UPB = 8;   // units per 256-value block
    static constexpr int NX = 32;   // x values per unit
    static constexpr int NS = 2;    // partial x sums per unit
    __device__ static void xslice(const float* x, int u, float* xv, float* sx) {
        const int b = u >> 3, j2 = (u & 7) >> 1, k0 = (u & 1) * 16;
        const float* p = x + b * 256 + j2 * 64 + k0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 a = ld4(p + 4 * i), c = ld4(p + 32 + 4 * i);
            xv[4 * i] = a.x; xv[4 * i + 1] = a.y; xv[4 * i + 2] = a.z; xv[4 * i + 3] = a.w;
            xv[16 + 4 * i] = c.x; xv[17 + 4 * i] = c.y; xv[18 + 4 * i] = c.z; xv[19 + 4 * i] = c.w;
        }
        sx[0] = sx[1] = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            sx[0] += xv[i];
            sx[1] += xv[16 + i];
        }
    }
    __device__ static float dot(const uint8_t* base, const DracoLayout& L, int row, int u, const float* xv,
                                const float* sx) {
        const size_t blk = (size_t)row * L.nb + (u >> 3);
        const uint4 q = ldu4(base + L.off[0] + blk * 128 + (size_t)(u & 7) * 16);
        const uint4 h = ldu4(base + L.off[1] + blk * 16);
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
        float sl = 0.f, sh = 0.f;
#pragma unroll
        for (int dw = 0; dw < 4; dw++) {
            const uint32_t lo = qw[dw] & 0x0F0F0F0Fu, hi = (qw[dw] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                sl = fmaf(ubyte_f(lo, k), xv[4 * dw + k], sl);
                sh = fmaf(ubyte_f(hi, k), xv[16 + 4 * dw + k], sh);
            }
        }
        // six-bit scales/mins of sub-blocks 2*j2 and 2*j2+1 (src/m5_kern_scalar.c:39-46)
        const int j2 = (u & 7) >> 1;
        const float d = h2f((uint16_t)(h.x & 0xFFFF)), dmin = h2f((uint16_t)(h.x >> 16));
        const int s0 = 16 * (j2 & 1), s1 = s0 + 8;  // bit offsets of bytes (2*j2)&3, (2*j2+1)&3
        int sc0, m0, sc1, m1;
        if (j2 < 2) {
            sc0 = (h.y >> s0) & 63;
            m0 = (h.z >> s0) & 63;
            sc1 = (h.y >> s1) & 63;
            m1 = (h.z >> s1) & 63;
        } else {
            sc0 = ((h.w >> s0) & 15) | (((h.y >> (s0 + 6)) & 3) << 4);
            m0 = ((h.w >> (s0 + 4)) & 15) | (((h.z >> (s0 + 6)) & 3) << 4);
            sc1 = ((h.w >> s1) & 15) | (((h.y >> (s1 + 6)) & 3) << 4);
            m1 = ((h.w >> (s1 + 4)) & 15) | (((h.z >> (s1 + 6)) & 3) << 4);
        }
        return (d * (float)sc0 * sl - dmin * (float)m0 * sx[0]) + (d * (float)sc1 * sh - dmin * (float)m1 * sx[1]);
    }
};

// unit (b, g, c) = ql[64g+16c..+16] (A), ql[64g+32+16c..+16] (B), qh[32g+16c..+16]:
//   A.lo -> values 128g+16c+i      scale group 8g+c
//   B.lo -> values 128g+32+16c+i   scale group 8g+c+2
//   A.hi -> values 128g+64+16c+i   scale group 8g+c+4
//   B.hi -> values 128g+96+16c+i   scale group 8g+c+6
// (the GGUF bit map of src/m5_kern_scalar.c:115-142 regrouped by qh byte)
struct FQ6K {
    static constexpr int UPB = 4, NX = 64, NS = 4;
    __device__ static void xslice(const float* x, int u, float* xv, float* sx) {
        const int b = u >> 2, g = (u >> 1) & 1, c = u & 1;
        const float* p = x + b * 256 + 128 * g + 16 * c;
#pragma unroll
        for (int run = 0; run < 4; run++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 a = ld4(p + 32 * run + 4 * i);
                xv[16 * run + 4 * i] = a.x; xv[16 * run + 4 * i + 1] = a.y;
                xv[16 * run + 4 * i + 2] = a.z; xv[16 * run + 4 * i + 3] = a.w;
            }
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < 16; i++) s += xv[16 * run + i];
            sx[run] = s;
        }
    }
    __device__ static float dot(const uint8_t* base, const DracoLayout& L, int row, int u, const float* xv,
                                const float* sx) {
        const int g = (u >> 1) & 1, c = u & 1;
        const size_t blk = (size_t)row * L.nb + (u >> 2);
        const uint4 qa = ldu4(base + L.off[0] + blk * 128 + 64 * g + 16 * c);
        const uint4 qb = ldu4(base + L.off[0] + blk * 128 + 64 * g + 32 + 16 * c);
        const uint4 hv = ldu4(base + L.off[1] + blk * 64 + 32 * g + 16 * c);
        const uint4 sv = ldu4(base + L.off[2] + blk * 16);
        const float d = h2f(*reinterpret_cast<const uint16_t*>(base + L.off[3] + blk * 2));
        const uint32_t A[4] = {qa.x, qa.y, qa.z, qa.w};
        const uint32_t B[4] = {qb.x, qb.y, qb.z, qb.w};
        const uint32_t H[4] = {hv.x, hv.y, hv.z, hv.w};
        float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dw = 0; dw < 4; dw++) {
            const uint32_t v0 = (A[dw] & 0x0F0F0F0Fu) | ((H[dw] << 4) & 0x30303030u);
            const uint32_t v1 = (B[dw] & 0x0F0F0F0Fu) | ((H[dw] << 2) & 0x30303030u);
            const uint32_t v2 = ((A[dw] >> 4) & 0x0F0F0F0Fu) | (H[dw] & 0x30303030u);
            const uint32_t v3 = ((B[dw] >> 4) & 0x0F0F0F0Fu) | ((H[dw] >> 2) & 0x30303030u);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                s[0] = fmaf(ubyte_f(v0, k), xv[4 * dw + k], s[0]);
                s[1] = fmaf(ubyte_f(v1, k), xv[16 + 4 * dw + k], s[1]);
                s[2] = fmaf(ubyte_f(v2, k), xv[32 + 4 * dw + k], s[2]);
                s[3] = fmaf(ubyte_f(v3, k), xv[48 + 4 * dw + k], s[3]);
            }
        }
        const uint32_t S[4] = {sv.x, sv.y, sv.z, sv.w};
        float part = 0.f;
#pragma unroll
        for (int run = 0; run < 4; run++) {
            const int gi = 8 * g + c + 2 * run;
            const float dsc = d * (float)(int)(int8_t)(S[gi >> 2] >> (8 * (gi & 3)));
            part += dsc * (s[run] - 32.f * sx[run]);
        }
        return part;
    }
};

struct FQ80 {
    static constexpr int UPB = 1, NX = 32, NS = 1;
    __device__ static void xslice(const float* x, int u, float* xv, float* sx) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 a = ld4(x + u * 32 + 4 * i);
            xv[4 * i] = a.x; xv[4 * i + 1] = a.y; xv[4 * i + 2] = a.z; xv[4 * i + 3] = a.w;
        }
        sx[0] = 0.f;
    }
    __device__ static float dot(const uint8_t* base, const DracoLayout& L, int row, int u, const float* xv,
                                const float* sx) {
        (void)sx;
        const size_t blk = (size_t)row * L.nb + u;
        const uint4 q0 = ldu4(base + L.off[0] + blk * 32), q1 = ldu4(base + L.off[0] + blk * 32 + 16);
        const float d = h2f(*reinterpret_cast<const uint16_t*>(base + L.off[1] + blk * 2));
        const uint32_t Q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        float s = 0.f;
#pragma unroll
        for (int dw = 0; dw < 8; dw++)
#pragma unroll
            for (int k = 0; k < 4; k++) s = fmaf(sbyte_f(Q[dw], k), xv[4 * dw + k], s);
        return d * s;
    }
};

// R row dots of one wave (plus the same rows of a second matrix when DUAL)
template <class F, int R, bool DUAL>
__device__ __forceinline__ void rows_dot(const SegDesc& s, const SegDesc& s2, const float* xs, int r0,
                                         float* acc) {
    const int lane = threadIdx.x & 63;
    const int U = s.L.nb * F::UPB;
    const int n_out = s.L.n_out;
    for (int u = lane; u < U; u += 64) {
        float xv[F::NX], sx[F::NS];
        F::xslice(xs, u, xv, sx);
#pragma unroll
        for (int i = 0; i < R; i++)
            if (r0 + i < n_out) {
                acc[i] += F::dot(s.base, s.L, r0 + i, u, xv, sx);
                if (DUAL) acc[R + i] += F::dot(s2.base, s2.L, r0 + i, u, xv, sx);
            }
    }
}


__device__ __forceinline__ void am_merge(float& v, int& i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

// ------------------------------------------------------ fused segments --
// One instantiation per weight format (all segments of a launch share it)
// and per dual mode, so the register budget is that of one format.
template <class F, bool DUAL>
__global__ __launch_bounds__(256) void k_seg(const SegLaunch a) {
    extern __shared__ float xsh[];
    __shared__ float red[4];
    __shared__ float amv[4 * SEG_R];
    __shared__ int ami[4 * SEG_R];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    int si = 0;
    for (int i = 1; i < a.nseg; i++)
        if ((int)blockIdx.x >= a.seg[i].first_block) si = i;
    const SegDesc& s = a.seg[si];
    const SegDesc& s2 = a.seg[DUAL ? si + 1 : si];

    // prologue: RMSNorm of x into LDS (every block; same order -> same result)
    const float* xs = a.x;
    if (a.do_norm) {
        float ss = 0.f;
        for (int i = tid; i < a.n_in; i += 256) {
            const float v = a.x[i];
            xsh[i] = v;
            ss = fmaf(v, v, ss);
        }
        ss = wave_sum(ss);
        if (lane == 0) red[wv] = ss;
        __syncthreads();
        const float tot = (red[0] + red[1]) + (red[2] + red[3]);
        const float inv = 1.f / sqrtf(tot / (float)a.n_in + a.eps);
        for (int i = tid; i < a.n_in; i += 256) {
            const float v = a.norm_w ? xsh[i] * inv * a.norm_w[i] : xsh[i] * inv;
            xsh[i] = v;
            if (a.xn_out && blockIdx.x == 0) a.xn_out[i] = v;
        }
        __syncthreads();
        xs = xsh;
    }

    const int r0 = ((int)blockIdx.x - s.first_block) * SEG_ROWS + wv * SEG_R;
    float acc[2 * SEG_R];
#pragma unroll
    for (int i = 0; i < 2 * SEG_R; i++) acc[i] = 0.f;
    rows_dot<F, SEG_R, DUAL>(s, s2, xs, r0, acc);
#pragma unroll
    for (int i = 0; i < (DUAL ? 2 : 1) * SEG_R; i++) acc[i] = wave_sum(acc[i]);

    const int n_out = s.L.n_out;
    switch (s.epi) {
    case EPI_STORE:
    case EPI_ARGMAX:
        if (lane == 0)
            for (int i = 0; i < SEG_R; i++)
                if (r0 + i < n_out) s.y[r0 + i] = acc[i];
        break;
    case EPI_RESID:
        if (lane == 0)
            for (int i = 0; i < SEG_R; i++)
                if (r0 + i < n_out) s.y[r0 + i] = s.yadd[r0 + i] + acc[i];
        break;
    case EPI_SWIGLU:
        if (lane == 0)
            for (int i = 0; i < SEG_R; i++)
                if (r0 + i < n_out) {
                    const float g = acc[i];
                    s.y[r0 + i] = (g / (1.f + expf(-g))) * acc[SEG_R + i];
                }
        break;
    case EPI_ROPE_Q:
    case EPI_ROPE_K:
        if (lane == 0) {
            // rows r0, r0+1 are one consecutive pair of a head (src/m6_engine.c:134-143)
            const int d = r0 % a.head_dim;
            float o0 = acc[0], o1 = acc[1];
            if (d < a.rot) {
                const int pos = a.state[0];
                const float* ang = a.rope_tab + ((size_t)pos * (a.rot / 2) + d / 2) * 2;
                const float c = ang[0], sn = ang[1];
                const float x0 = acc[0], x1 = acc[1];
                o0 = x0 * c - x1 * sn;
                o1 = x0 * sn + x1 * c;
            }
            if (s.epi == EPI_ROPE_Q) {
                if (r0 < n_out) s.y[r0] = o0;
                if (r0 + 1 < n_out) s.y[r0 + 1] = o1;
            } else {
                float* dst = a.kc + (size_t)a.state[1 + a.layer] * a.kv_dim;
                if (r0 < n_out) dst[r0] = o0;
                if (r0 + 1 < n_out) dst[r0 + 1] = o1;
            }
        }
        break;
    case EPI_V_APPEND:
        if (lane == 0) {
            float* dst = a.vc + (size_t)a.state[1 + a.layer] * a.kv_dim;
            for (int i = 0; i < SEG_R; i++)
                if (r0 + i < n_out) dst[r0 + i] = acc[i];
        }
        break;
    default:
        break;
    }

    if (s.epi != EPI_ARGMAX) return;
    // per-block argmax partial; k_argmax_finalize (next launch) reduces them
    if (lane == 0)
        for (int i = 0; i < SEG_R; i++) {
            amv[wv * SEG_R + i] = (r0 + i < n_out) ? acc[i] : -INFINITY;
            ami[wv * SEG_R + i] = (r0 + i < n_out) ? r0 + i : 0x7fffffff;
        }
    __syncthreads();
    if (tid == 0) {
        float v = amv[0];
        int idx = ami[0];
        for (int i = 1; i < 4 * SEG_R; i++) am_merge(v, idx, amv[i], ami[i]);
        const int bi = (int)blockIdx.x - s.first_block;
        a.am_val[bi] = v;
        a.am_idx[bi] = idx;
    }
}

// Reduce the head's per-block argmax partials (np.argmax semantics: first
// index of the maximum), write tokens[*cursor + 1] and advance the token
// state.  One block; runs after k_seg in stream order.
__global__ __launch_bounds__(256) void k_argmax_finalize(const float* __restrict__ pv, const int* __restrict__ pi,
                                                         int nb, int* __restrict__ tokens, int* cursor,
                                                         int* state, int n_layer) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    float v = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = tid; i < nb; i += 256) am_merge(v, idx, pv[i], pi[i]);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) am_merge(v, idx, __shfl_xor(v, m, 64), __shfl_xor(idx, m, 64));
    if (lane == 0) {
        sv[wv] = v;
        si[wv] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; w++) am_merge(v, idx, sv[w], si[w]);
        const int cur = cursor ? cursor[0] : -1;
        tokens[cur + 1] = idx;
        if (state) {
            state[0] += 1;
            for (int l = 0; l < n_layer; l++) state[1 + l] += 1;
        }
        if (cursor) cursor[0] += 1;
    }
}

// ------------------------------------------------------------ F32 / F16 --
template <int R, bool HALF>
__global__ __launch_bounds__(256) void k_gemv_plain(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                    float* __restrict__ y, const float* __restrict__ yadd,
                                                    int row0, int row1, int n_in) {
    const int lane = threadIdx.x & 63;
    const int r0 = row0 + (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * R;
    if (r0 >= row1) return;
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; i++) acc[i] = 0.f;
    for (int k = lane; k < n_in; k += 64) {
        const float xv = x[k];
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int r = r0 + i;
            if (r < row1) {
                float wv;
                if (HALF) wv = h2f(reinterpret_cast<const uint16_t*>(w)[(size_t)r * n_in + k]);
                else wv = reinterpret_cast<const float*>(w)[(size_t)r * n_in + k];
                acc[i] = fmaf(wv, xv, acc[i]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < R; i++) {
        const float s = wave_sum(acc[i]);
        const int r = r0 + i;
        if (lane == 0 && r < row1) y[r] = (yadd ? yadd[r] : 0.f) + s;
    }
}

}  // namespace

int draco_seg_launch(SegLaunch& a, hipStream_t st) {
    if (a.nseg < 1 || a.nseg > SEG_MAX) return -1;
    int blocks = 0;
    for (int i = 0; i < a.nseg; i++) {
        SegDesc& s = a.seg[i];
        if (s.L.code != DRACO_Q4_K && s.L.code != DRACO_Q6_K && s.L.code != DRACO_Q8_0) return -1;
        if (s.L.n_in != a.n_in) return -1;
        s.first_block = blocks;
        s.n_blocks = (s.L.n_out + SEG_ROWS - 1) / SEG_ROWS;
        if (s.epi == EPI_SWIGLU) {
            if (i + 1 >= a.nseg) return -1;
            const SegDesc& u = a.seg[i + 1];
            if (u.L.code != s.L.code || u.L.n_out != s.L.n_out) return -1;
            blocks += s.n_blocks;
            a.seg[i + 1].first_block = 1 << 30;  // never selected: computed with its gate
            a.seg[i + 1].n_blocks = 0;
            i++;
            continue;
        }
        if ((s.epi == EPI_ROPE_Q || s.epi == EPI_ROPE_K) && ((s.L.n_out & 1) || (a.head_dim & 1))) return -1;
        blocks += s.n_blocks;
    }
    const int code = a.seg[0].L.code;
    bool dual = false;
    for (int i = 0; i < a.nseg; i++) {
        if (a.seg[i].L.code != code) return -1;  // one format per launch
        dual = dual || a.seg[i].epi == EPI_SWIGLU;
    }
    if (dual && a.nseg != 2) return -1;
    const size_t shm = a.do_norm ? sizeof(float) * (size_t)a.n_in : 0;
    const dim3 g(blocks), b(256);
    if (code == DRACO_Q4_K) {
        if (dual) hipLaunchKernelGGL((k_seg<FQ4K, true>), g, b, shm, st, a);
        else hipLaunchKernelGGL((k_seg<FQ4K, false>), g, b, shm, st, a);
    } else if (code == DRACO_Q6_K) {
        if (dual) hipLaunchKernelGGL((k_seg<FQ6K, true>), g, b, shm, st, a);
        else hipLaunchKernelGGL((k_seg<FQ6K, false>), g, b, shm, st, a);
    } else {
        if (dual) hipLaunchKernelGGL((k_seg<FQ80, true>), g, b, shm, st, a);
        else hipLaunchKernelGGL((k_seg<FQ80, false>), g, b, shm, st, a);
    }
    if (a.seg[0].epi == EPI_ARGMAX)
        hipLaunchKernelGGL(k_argmax_finalize, dim3(1), dim3(256), 0, st, a.am_val, a.am_idx, a.seg[0].n_blocks,
                           a.tokens, const_cast<int*>(a.cursor), a.advance_state, a.advance_layers);
    return 0;
}

int draco_gemv_launch(const DracoMat& m, const float* x, float* y, const float* yadd, int row0, int row1,
                      hipStream_t st) {
    if (row0 < 0 || row1 > m.L.n_out || row0 > row1) return -1;
    if (row0 == row1) return 0;
    const int code = m.L.code;
    if (code == DRACO_Q4_K || code == DRACO_Q6_K || code == DRACO_Q8_0) {
        // a row range is a segment over rows [row0, row1): shift the row origin by
        // offsetting y and describing only those rows
        SegLaunch a = {};
        a.nseg = 1;
        a.n_in = m.L.n_in;
        a.x = x;
        SegDesc& s = a.seg[0];
        s.L = m.L;
        s.L.n_out = row1 - row0;
        // rows start at row0: advance every region base by row0 rows
        const size_t nb = (size_t)m.L.nb;
        s.base = m.dev;
        if (row0) {
            // regions are row-major [n_out][nb][...]: per-region offsets move by row0 rows
            size_t per[4] = {0, 0, 0, 0};
            if (code == DRACO_Q4_K) { per[0] = 128; per[1] = 16; }
            else if (code == DRACO_Q6_K) { per[0] = 128; per[1] = 64; per[2] = 16; per[3] = 2; }
            else { per[0] = 32; per[1] = 2; }
            for (int i = 0; i < 4; i++) s.L.off[i] += per[i] * nb * (size_t)row0;
        }
        s.y = y + row0;
        s.yadd = yadd ? yadd + row0 : nullptr;
        s.epi = yadd ? EPI_RESID : EPI_STORE;
        return draco_seg_launch(a, st);
    }
    const int R = 1;
    const int waves = row1 - row0;
    const dim3 grid((waves + 3) / 4), block(256);
    if (code == DRACO_F32)
        hipLaunchKernelGGL((k_gemv_plain<R, false>), grid, block, 0, st, m.dev, x, y, yadd, row0, row1, m.L.n_in);
    else if (code == DRACO_F16)
        hipLaunchKernelGGL((k_gemv_plain<R, true>), grid, block, 0, st, m.dev, x, y, yadd, row0, row1, m.L.n_in);
    else
        return -1;
    return 0;
}

int draco_gemv_supported(int code) {
    return code == DRACO_Q4_K || code == DRACO_Q6_K || code == DRACO_Q8_0 || code == DRACO_F32 ||
           code == DRACO_F16;
}
