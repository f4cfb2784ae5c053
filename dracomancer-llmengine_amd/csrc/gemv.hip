// gemv.hip -- fp32-activation GEMV over block-quantized weights (gfx950).
//
//   y[r] = (yadd ? yadd[r] : 0) + sum_k W[r][k] * x[k],   r in [row0, row1)
//
// Reference semantics: dot_row / m5_gemv_range, src/m5_kern_scalar.c:48-165
// (rows at absolute index; decoded weight value w = d*sc*q - dmin*m for Q4_K,
// d*sc*(q-32) for Q6_K, d*q for Q8_0).  The summation order differs from the
// reference's sequential loop (a wave tree), so results agree to fp32
// rounding, not bitwise.
//
// Mapping (one wave64 per R consecutive rows): a row is cut into "units" of
// 16-byte quant vectors; lane l takes units l, l+64, ...  Each unit's x slice
// is loaded once per lane and reused for the R rows the wave owns, then every
// row is reduced across the wave.  Per unit the kernel applies the block scale
// once to an inner integer-valued dot:
//   Q4_K: sum_j d*sc_j*(sum q*x) - dmin*m_j*(sum x)
//   Q6_K: sum_g d*sc_g*((sum (q+32)*x) - 32*(sum x))
// which is the reference's per-weight expression regrouped.
#include <hip/hip_runtime.h>

#include "dev_common.h"
#include "formats.h"
#include "gemv.h"

namespace {

// ---------------------------------------------------------------- Q4_K --
// unit = 16 qs bytes of block b: low nibbles -> sub-block 2*j2, high -> 2*j2+1,
// elements k0..k0+15, where (j2, k0) = ((u&7)>>1, (u&1)*16).
__device__ __forceinline__ void q4k_scales(uint4 h, int j2, float& dsc0, float& dm0, float& dsc1,
                                           float& dm1) {
    const float d = h2f((uint16_t)(h.x & 0xFFFF)), dmin = h2f((uint16_t)(h.x >> 16));
    const int j0 = (2 * j2) & 3, j1 = (2 * j2 + 1) & 3;
    const uint32_t s0 = h.y, s4 = h.z, s8 = h.w;
    int sc0, m0, sc1, m1;
    if (j2 < 2) {
        sc0 = (s0 >> (8 * j0)) & 63;
        m0 = (s4 >> (8 * j0)) & 63;
        sc1 = (s0 >> (8 * j1)) & 63;
        m1 = (s4 >> (8 * j1)) & 63;
    } else {
        sc0 = ((s8 >> (8 * j0)) & 15) | (((s0 >> (8 * j0 + 6)) & 3) << 4);
        m0 = ((s8 >> (8 * j0 + 4)) & 15) | (((s4 >> (8 * j0 + 6)) & 3) << 4);
        sc1 = ((s8 >> (8 * j1)) & 15) | (((s0 >> (8 * j1 + 6)) & 3) << 4);
        m1 = ((s8 >> (8 * j1 + 4)) & 15) | (((s4 >> (8 * j1 + 6)) & 3) << 4);
    }
    dsc0 = d * (float)sc0;
    dm0 = dmin * (float)m0;
    dsc1 = d * (float)sc1;
    dm1 = dmin * (float)m1;
}

template <int R>
__global__ __launch_bounds__(256) void k_gemv_q4k(const uint8_t* __restrict__ qs,
                                                  const uint8_t* __restrict__ hd,
                                                  const float* __restrict__ x, float* __restrict__ y,
                                                  const float* __restrict__ yadd, int row0, int row1,
                                                  int nb) {
    const int lane = threadIdx.x & 63;
    const int r0 = row0 + (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * R;
    if (r0 >= row1) return;
    const int U = nb * 8;
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; i++) acc[i] = 0.f;
    for (int u = lane; u < U; u += 64) {
        const int b = u >> 3, j2 = (u & 7) >> 1, k0 = (u & 1) * 16;
        const float* xp = x + b * 256 + j2 * 64 + k0;
        float xl[16], xh[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 a = ld4(xp + 4 * i), c = ld4(xp + 32 + 4 * i);
            xl[4 * i] = a.x; xl[4 * i + 1] = a.y; xl[4 * i + 2] = a.z; xl[4 * i + 3] = a.w;
            xh[4 * i] = c.x; xh[4 * i + 1] = c.y; xh[4 * i + 2] = c.z; xh[4 * i + 3] = c.w;
        }
        float sxl = 0.f, sxh = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) { sxl += xl[i]; sxh += xh[i]; }
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int r = r0 + i;
            if (r < row1) {
                const size_t blk = (size_t)r * nb + b;
                const uint4 q = ldu4(qs + blk * 128 + (size_t)(u & 7) * 16);
                const uint4 h = ldu4(hd + blk * 16);
                const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
                float sl = 0.f, sh = 0.f;
#pragma unroll
                for (int dw = 0; dw < 4; dw++) {
                    const uint32_t lo = qw[dw] & 0x0F0F0F0Fu, hi = (qw[dw] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        sl = fmaf(ubyte_f(lo, k), xl[4 * dw + k], sl);
                        sh = fmaf(ubyte_f(hi, k), xh[4 * dw + k], sh);
                    }
                }
                float dsc0, dm0, dsc1, dm1;
                q4k_scales(h, j2, dsc0, dm0, dsc1, dm1);
                acc[i] += (dsc0 * sl - dm0 * sxl) + (dsc1 * sh - dm1 * sxh);
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

// ---------------------------------------------------------------- Q6_K --
// unit (b, g, c) = ql[64g+16c..+16] (A), ql[64g+32+16c..+16] (B), qh[32g+16c..+16]:
//   A.lo -> values 128g+16c+i      scale group 8g+c
//   B.lo -> values 128g+32+16c+i   scale group 8g+c+2
//   A.hi -> values 128g+64+16c+i   scale group 8g+c+4
//   B.hi -> values 128g+96+16c+i   scale group 8g+c+6
// (the GGUF bit map of src/m5_kern_scalar.c:115-142 regrouped by qh byte)
template <int R>
__global__ __launch_bounds__(256) void k_gemv_q6k(const uint8_t* __restrict__ ql,
                                                  const uint8_t* __restrict__ qh,
                                                  const uint8_t* __restrict__ scb,
                                                  const uint8_t* __restrict__ db,
                                                  const float* __restrict__ x, float* __restrict__ y,
                                                  const float* __restrict__ yadd, int row0, int row1,
                                                  int nb) {
    const int lane = threadIdx.x & 63;
    const int r0 = row0 + (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * R;
    if (r0 >= row1) return;
    const int U = nb * 4;
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; i++) acc[i] = 0.f;
    for (int u = lane; u < U; u += 64) {
        const int b = u >> 2, g = (u >> 1) & 1, c = u & 1;
        const float* xp = x + b * 256 + 128 * g + 16 * c;
        float xv[4][16];
        float sx[4];
#pragma unroll
        for (int run = 0; run < 4; run++) {
            sx[run] = 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 a = ld4(xp + 32 * run + 4 * i);
                xv[run][4 * i] = a.x; xv[run][4 * i + 1] = a.y;
                xv[run][4 * i + 2] = a.z; xv[run][4 * i + 3] = a.w;
            }
#pragma unroll
            for (int i = 0; i < 16; i++) sx[run] += xv[run][i];
        }
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int r = r0 + i;
            if (r < row1) {
                const size_t blk = (size_t)r * nb + b;
                const uint4 qa = ldu4(ql + blk * 128 + 64 * g + 16 * c);
                const uint4 qb = ldu4(ql + blk * 128 + 64 * g + 32 + 16 * c);
                const uint4 hv = ldu4(qh + blk * 64 + 32 * g + 16 * c);
                const uint4 sv = ldu4(scb + blk * 16);
                const float d = h2f(*reinterpret_cast<const uint16_t*>(db + blk * 2));
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
                        s[0] = fmaf(ubyte_f(v0, k), xv[0][4 * dw + k], s[0]);
                        s[1] = fmaf(ubyte_f(v1, k), xv[1][4 * dw + k], s[1]);
                        s[2] = fmaf(ubyte_f(v2, k), xv[2][4 * dw + k], s[2]);
                        s[3] = fmaf(ubyte_f(v3, k), xv[3][4 * dw + k], s[3]);
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
                acc[i] += part;
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

// ---------------------------------------------------------------- Q8_0 --
template <int R>
__global__ __launch_bounds__(256) void k_gemv_q80(const uint8_t* __restrict__ qs,
                                                  const uint8_t* __restrict__ db,
                                                  const float* __restrict__ x, float* __restrict__ y,
                                                  const float* __restrict__ yadd, int row0, int row1,
                                                  int nb) {
    const int lane = threadIdx.x & 63;
    const int r0 = row0 + (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * R;
    if (r0 >= row1) return;
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; i++) acc[i] = 0.f;
    for (int b = lane; b < nb; b += 64) {
        float xv[32];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 a = ld4(x + b * 32 + 4 * i);
            xv[4 * i] = a.x; xv[4 * i + 1] = a.y; xv[4 * i + 2] = a.z; xv[4 * i + 3] = a.w;
        }
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int r = r0 + i;
            if (r < row1) {
                const size_t blk = (size_t)r * nb + b;
                const uint4 q0 = ldu4(qs + blk * 32), q1 = ldu4(qs + blk * 32 + 16);
                const float d = h2f(*reinterpret_cast<const uint16_t*>(db + blk * 2));
                const uint32_t Q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
                float s = 0.f;
#pragma unroll
                for (int dw = 0; dw < 8; dw++)
#pragma unroll
                    for (int k = 0; k < 4; k++) s = fmaf(sbyte_f(Q[dw], k), xv[4 * dw + k], s);
                acc[i] += d * s;
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

// ------------------------------------------------------------ F32 / F16 --
template <int R, bool HALF>
__global__ __launch_bounds__(256) void k_gemv_plain(const uint8_t* __restrict__ w,
                                                    const float* __restrict__ x, float* __restrict__ y,
                                                    const float* __restrict__ yadd, int row0, int row1,
                                                    int n_in) {
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

template <int R>
int launch_r(const DracoMat& m, const float* x, float* y, const float* yadd, int row0, int row1,
             hipStream_t st) {
    const int rows = row1 - row0;
    const int waves = (rows + R - 1) / R;
    const dim3 grid((waves + 3) / 4), block(256);
    const uint8_t* b = m.dev;
    switch (m.L.code) {
    case DRACO_Q4_K:
        hipLaunchKernelGGL(k_gemv_q4k<R>, grid, block, 0, st, b + m.L.off[0], b + m.L.off[1], x, y,
                           yadd, row0, row1, m.L.nb);
        break;
    case DRACO_Q6_K:
        hipLaunchKernelGGL(k_gemv_q6k<R>, grid, block, 0, st, b + m.L.off[0], b + m.L.off[1],
                           b + m.L.off[2], b + m.L.off[3], x, y, yadd, row0, row1, m.L.nb);
        break;
    case DRACO_Q8_0:
        hipLaunchKernelGGL(k_gemv_q80<R>, grid, block, 0, st, b + m.L.off[0], b + m.L.off[1], x, y,
                           yadd, row0, row1, m.L.nb);
        break;
    case DRACO_F32:
        hipLaunchKernelGGL((k_gemv_plain<R, false>), grid, block, 0, st, b, x, y, yadd, row0, row1,
                           m.L.n_in);
        break;
    case DRACO_F16:
        hipLaunchKernelGGL((k_gemv_plain<R, true>), grid, block, 0, st, b, x, y, yadd, row0, row1,
                           m.L.n_in);
        break;
    default:
        return -1;
    }
    return 0;
}

}  // namespace

int draco_gemv_launch(const DracoMat& m, const float* x, float* y, const float* yadd, int row0,
                      int row1, hipStream_t st) {
    if (row0 < 0 || row1 > m.L.n_out || row0 >= row1) return row0 == row1 ? 0 : -1;
    const int rows = row1 - row0;
    if (rows >= 8192) return launch_r<4>(m, x, y, yadd, row0, row1, st);
    if (rows >= 2048) return launch_r<2>(m, x, y, yadd, row0, row1, st);
    return launch_r<1>(m, x, y, yadd, row0, row1, st);
}

int draco_gemv_supported(int code) {
    return code == DRACO_Q4_K || code == DRACO_Q6_K || code == DRACO_Q8_0 || code == DRACO_F32 ||
           code == DRACO_F16;
}
