/*
 * draco_oracle.c -- CPU restatement of the Dracomancer per-token decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline).  The product path (libdraco_hip.so) never links,
 * loads or calls it.
 *
 * Every function restates one reference function (file:line under the
 * reference tree, src/...) with the same floating-point operation order, so a
 * strict build (-ffp-contract=off) of this file is bit-identical to a strict
 * build of the reference sources on the same inputs.  That identity is checked
 * by tests/test_oracle_golden.py against fixtures the compiled reference wrote.
 *
 * Functions whose reference cannot be compiled here (m5_gemm.c /
 * m5_gemm_fused.c need a header that is not in the tree) are pinned by
 * invariants instead; their docstrings say which.
 *
 * OR_MUTANT (compile-time, default 0) plants one known slip for the pin
 * tests to catch (tests/test_oracle_pins.py builds each mutant into a
 * temporary library and checks that its pins fail): 1 Q4_K nibble swap and
 * 2 Q4_K min term dropped in or_dequant_row, 3 Q6_K high-bit shift taken
 * from the wrong index, 4 or_gemm output transposed, 5 or_moe_tok weighting
 * every slot by slot 0's weight.  The shipped liboracle.so is built with 0.
 *
 * Q8_K (activation quantizer) and the integer block dots have no reference in
 * the tree at all.  They follow llama.cpp's published quantize_row_q8_K_ref /
 * ggml_vec_dot_q4_K_q8_K / ggml_vec_dot_q6_K_q8_K algorithm (ggml-quants.c,
 * llama.cpp b10819, the version the reference pins) and are pinned by
 * closed-form invariants (tests/test_oracle_q8k.py).
 */
#include <stdint.h>
#include <stddef.h>
#include <string.h>
#include <stdlib.h>
#include <math.h>
#include <omp.h>

#ifndef OR_MUTANT
#define OR_MUTANT 0
#endif

/* ------------------------------------------------------------------ */
/* a1  IEEE half -> float, exact incl. subnormals                      */
/*     src/m5_kern_scalar.c:9-21                                       */
/* ------------------------------------------------------------------ */
float or_f16(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t ex = (h >> 10) & 0x1Fu, mant = h & 0x3FFu, bits;
    if (ex == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            float v = (float)mant * 5.9604644775390625e-8f;   /* mant * 2^-24 */
            uint32_t vb;
            memcpy(&vb, &v, 4);
            bits = sign | vb;
        }
    } else if (ex == 31) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((ex + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline float ld_f16(const uint8_t* p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return or_f16(h);
}

/* ------------------------------------------------------------------ */
/* a2  bytes per row by format code                                    */
/*     src/m6_engine.c:40-54, src/m5_kern_scalar.c:26-36               */
/* ------------------------------------------------------------------ */
size_t or_rowbytes(int code, int n_in) {
    switch (code) {
    case 0: return (size_t)(n_in / 32) * 34;    /* Q8_0 */
    case 3: return (size_t)(n_in / 256) * 176;  /* Q5_K */
    case 4: return (size_t)(n_in / 256) * 210;  /* Q6_K */
    case 5: return (size_t)(n_in / 256) * 144;  /* Q4_K */
    case 7: return (size_t)n_in * 2;            /* F16 */
    case 9: return (size_t)n_in * 4;            /* F32 */
    default: return 0;
    }
}

/* src/m5_kern_scalar.c:146-148 */
int or_supported(int code) {
    return code == 0 || code == 3 || code == 4 || code == 5 || code == 7 || code == 9;
}

/* a3  12 packed bytes -> 8 six-bit scales + 8 six-bit mins (Q4_K/Q5_K)
 *     src/m5_kern_scalar.c:39-46 */
static void kq_scales(const uint8_t* s, float* sc, float* mn) {
    for (int i = 0; i < 4; i++) {
        sc[i] = (float)(s[i] & 0x3F);
        sc[4 + i] = (float)((s[8 + i] & 0x0F) | ((s[i] >> 2) & 0x30));
        mn[i] = (float)(s[4 + i] & 0x3F);
        mn[4 + i] = (float)((s[8 + i] >> 4) | ((s[4 + i] >> 2) & 0x30));
    }
}

/* ------------------------------------------------------------------ */
/* a4/a6/a7  scalar row dot in the reference's exact loop order        */
/*     src/m5_kern_scalar.c:48-144                                     */
/* ------------------------------------------------------------------ */
static float row_dot(int code, const uint8_t* row, const float* x, int n_in) {
    float dot = 0.f;
    if (code == 9) {                                       /* F32 */
        for (int i = 0; i < n_in; i++) {
            float w;
            memcpy(&w, row + (size_t)i * 4, 4);
            dot += w * x[i];
        }
        return dot;
    }
    if (code == 7) {                                       /* F16 */
        for (int i = 0; i < n_in; i++) dot += ld_f16(row + (size_t)i * 2) * x[i];
        return dot;
    }
    if (code == 0) {                                       /* Q8_0: d f16, 32 x i8 */
        const int nb = n_in / 32;
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = row + (size_t)b * 34;
            const float d = ld_f16(blk);
            float acc = 0.f;
            for (int i = 0; i < 32; i++) acc += (float)(int8_t)blk[2 + i] * x[b * 32 + i];
            dot += d * acc;
        }
        return dot;
    }
    if (code == 5) {                                       /* Q4_K: d dmin sc12 qs128 */
        const int nb = n_in / 256;
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = row + (size_t)b * 144;
            const float d = ld_f16(blk), dmin = ld_f16(blk + 2);
            float sc[8], mn[8];
            kq_scales(blk + 4, sc, mn);
            const uint8_t* qs = blk + 16;
            for (int j = 0; j < 8; j++) {
                const float dsc = d * sc[j], dm = dmin * mn[j];
                const uint8_t* qb = qs + (j >> 1) * 32;   /* one 32-byte run feeds sub-blocks 2i, 2i+1 */
                const int hi = j & 1;
                float acc = 0.f;
                for (int k = 0; k < 32; k++) {
                    const float qv = (float)(hi ? (qb[k] >> 4) : (qb[k] & 0xF));
                    const float w = dsc * qv - dm;
                    acc += w * x[b * 256 + j * 32 + k];
                }
                dot += acc;
            }
        }
        return dot;
    }
    if (code == 3) {                                       /* Q5_K: d dmin sc12 qh32 qs128 */
        const int nb = n_in / 256;
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = row + (size_t)b * 176;
            const float d = ld_f16(blk), dmin = ld_f16(blk + 2);
            float sc[8], mn[8];
            kq_scales(blk + 4, sc, mn);
            const uint8_t* qh = blk + 16;
            const uint8_t* qs = blk + 48;
            for (int j = 0; j < 8; j++) {
                const float dsc = d * sc[j], dm = dmin * mn[j];
                const uint8_t* qb = qs + (j >> 1) * 32;
                const int hi = j & 1;
                float acc = 0.f;
                for (int k = 0; k < 32; k++) {
                    const int nib = hi ? (qb[k] >> 4) : (qb[k] & 0xF);
                    const int top = (qh[k] >> j) & 1;
                    const float w = dsc * (float)(nib | (top << 4)) - dm;
                    acc += w * x[b * 256 + j * 32 + k];
                }
                dot += acc;
            }
        }
        return dot;
    }
    if (code == 4) {                                       /* Q6_K: ql128 qh64 sc16 d */
        const int nb = n_in / 256;
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = row + (size_t)b * 210;
            const uint8_t* ql = blk;
            const uint8_t* qh = blk + 128;
            const int8_t* sc = (const int8_t*)(blk + 192);
            const float d = ld_f16(blk + 208);
            for (int r = 0; r < 8; r++) {
                /* 32-value row r of the block: r = 4*g + 2*nibsel + odd */
                const int g = r >> 2, nibsel = (r >> 1) & 1, odd = r & 1, shift = (r & 3) * 2;
                for (int h = 0; h < 2; h++) {
                    const float dsc = d * (float)sc[r * 2 + h];
                    float acc = 0.f;
                    for (int k = 0; k < 16; k++) {
                        const int kk = h * 16 + k;
                        const int lo4 = (ql[g * 64 + odd * 32 + kk] >> (nibsel * 4)) & 0xF;
                        const int hi2 = (qh[g * 32 + kk] >> shift) & 0x3;
                        acc += (float)((lo4 | (hi2 << 4)) - 32) * x[b * 256 + r * 32 + kk];
                    }
                    dot += dsc * acc;
                }
            }
        }
        return dot;
    }
    return 0.f;
}

/* a8  m5_gemv / m5_gemv_range  src/m5_kern_scalar.c:150-165.
 * Rows are independent, so the row loop may run in parallel without
 * changing a single bit of y. */
int or_gemv_range(int code, const float* x, const uint8_t* W, int n_out, int n_in,
                  float* y, int o0, int o1) {
    (void)n_out;
    if (!or_supported(code)) return -1;
    const size_t rs = or_rowbytes(code, n_in);
    #pragma omp parallel for schedule(static) if (o1 - o0 >= 64)
    for (int r = o0; r < o1; r++) y[r] = row_dot(code, W + rs * (size_t)r, x, n_in);
    return 0;
}

int or_gemv(int code, const float* x, const uint8_t* W, int n_out, int n_in, float* y) {
    return or_gemv_range(code, x, W, n_out, n_in, y, 0, n_out);
}

/* ------------------------------------------------------------------ */
/* a12  independent row dequantizer  src/m5/m5_gemm.c:55-235           */
/*      (Q8_0 :56-68, Q4_K :142-169, Q6_K :193-211).  The value of     */
/*      each weight equals what row_dot multiplies by x.  Pinned by    */
/*      tests/test_oracle_pins.py: every row equals the one-hot        */
/*      columns of or_gemv (bitwise pinned to the compiled scalar      */
/*      kernel) and the independent numpy decoders, bit for bit.       */
/* ------------------------------------------------------------------ */
int or_dequant_row(int code, const uint8_t* row, int n_in, float* out) {
    if (code == 0) {
        for (int b = 0; b < n_in / 32; b++) {
            const uint8_t* blk = row + (size_t)b * 34;
            const float d = ld_f16(blk);
            for (int i = 0; i < 32; i++) out[b * 32 + i] = (float)(int8_t)blk[2 + i] * d;
        }
        return 0;
    }
    if (code == 5) {
        for (int b = 0; b < n_in / 256; b++) {
            const uint8_t* blk = row + (size_t)b * 144;
            const float d = ld_f16(blk), dmin = ld_f16(blk + 2);
            float sc[8], mn[8];
            kq_scales(blk + 4, sc, mn);
            const uint8_t* qs = blk + 16;
            for (int j = 0; j < 8; j++) {
                const float dsc = d * sc[j], dm = dmin * mn[j];
                const uint8_t* qb = qs + (j >> 1) * 32;
                for (int k = 0; k < 32; k++) {
#if OR_MUTANT == 1
                    const float qv = (float)((j & 1) ? (qb[k] & 0xF) : (qb[k] >> 4));
#else
                    const float qv = (float)((j & 1) ? (qb[k] >> 4) : (qb[k] & 0xF));
#endif
#if OR_MUTANT == 2
                    out[b * 256 + j * 32 + k] = dsc * qv;
                    (void)dm;
#else
                    out[b * 256 + j * 32 + k] = dsc * qv - dm;
#endif
                }
            }
        }
        return 0;
    }
    if (code == 4) {
        for (int b = 0; b < n_in / 256; b++) {
            const uint8_t* blk = row + (size_t)b * 210;
            const uint8_t* ql = blk;
            const uint8_t* qh = blk + 128;
            const int8_t* sc = (const int8_t*)(blk + 192);
            const float d = ld_f16(blk + 208);
            for (int p = 0; p < 256; p++) {
                const uint8_t lb = ql[(p >> 7) * 64 + (p & 63)];
                const int lo4 = ((p >> 6) & 1) ? (lb >> 4) : (lb & 0x0F);
#if OR_MUTANT == 3
                const int hi2 = (qh[(p >> 7) * 32 + (p & 31)] >> (((p >> 6) & 3) * 2)) & 3;
#else
                const int hi2 = (qh[(p >> 7) * 32 + (p & 31)] >> (((p >> 5) & 3) * 2)) & 3;
#endif
                const int q = (lo4 | (hi2 << 4)) - 32;
                out[b * 256 + p] = d * (float)sc[p >> 4] * (float)q;
            }
        }
        return 0;
    }
    if (code == 3) {  /* Q5_K, src/m5/m5_gemm.c:212-231: (q*d)*sc - dmin*m */
        for (int b = 0; b < n_in / 256; b++) {
            const uint8_t* blk = row + (size_t)b * 176;
            const float d = ld_f16(blk), dmin = ld_f16(blk + 2);
            float sc[8], mn[8];
            kq_scales(blk + 4, sc, mn);
            const uint8_t* qh = blk + 16;
            const uint8_t* qs = blk + 48;
            for (int p = 0; p < 256; p++) {
                const uint8_t qsb = qs[(p >> 6) * 32 + (p & 31)];
                const int nib = ((p >> 5) & 1) ? (qsb >> 4) : (qsb & 0x0F);
                const int bit = (qh[p & 31] >> (p >> 5)) & 1;
                const int g = p >> 5;
                out[b * 256 + p] = (float)(nib + (bit ? 16 : 0)) * d * sc[g] - dmin * mn[g];
            }
        }
        return 0;
    }
    if (code == 7) {
        for (int i = 0; i < n_in; i++) out[i] = ld_f16(row + (size_t)i * 2);
        return 0;
    }
    if (code == 9) {
        memcpy(out, row, sizeof(float) * (size_t)n_in);
        return 0;
    }
    return -1;
}

/* ------------------------------------------------------------------ */
/* a14  ggml rms_norm  src/m6_engine.c:31-37                           */
/* ------------------------------------------------------------------ */
void or_rms_norm(const float* x, const float* w, int h, float eps, float* out) {
    float ms = 0.f;
    for (int i = 0; i < h; i++) ms += x[i] * x[i];
    const float inv = 1.f / sqrtf(ms / (float)h + eps);
    if (w) for (int i = 0; i < h; i++) out[i] = x[i] * inv * w[i];
    else   for (int i = 0; i < h; i++) out[i] = x[i] * inv;
}

/* ------------------------------------------------------------------ */
/* a15-a18  llama-family token step.  Struct layouts are the           */
/* reference's ctypes-visible ones (src/m6_engine.c:21-28, :270-273,   */
/* :396-406) so one descriptor array drives the oracle, the compiled   */
/* reference and the HIP engine alike.                                 */
/* ------------------------------------------------------------------ */
typedef void (*or_attn_fn)(const float* xn, void* p, int pos, float* out);
typedef void (*or_ffn_fn)(const float* xn, void* p, float* out);

typedef struct {
    const float* attn_norm;
    const float* ffn_norm;
    or_attn_fn attn;
    void* attn_p;
    or_ffn_fn ffn;
    void* ffn_p;
} OrLayerDesc;

typedef struct {
    const uint8_t *wq, *wk, *wv, *wo;
    int cq, ck, cv, co;
    int n_head, n_kv, head_dim, hidden, rot;
    float rope_base;
    float* kcache;
    float* vcache;
    int* tlen;
    int max_t;
    float* work;
} OrLlamaAttnP;

typedef struct {
    const uint8_t *g, *u, *d;
    int cg, cu, cd, n_ff, h;
} OrDenseP;

/* consecutive-pair rope on the first `rot` dims  src/m6_engine.c:134-143 */
static void rope_pairs(float* v, int rot, int pos, float base) {
    for (int i = 0; i < rot / 2; i++) {
        const float theta = (float)pos * powf(base, -2.0f * (float)i / (float)rot);
        const float c = cosf(theta), s = sinf(theta);
        const float a = v[2 * i], b = v[2 * i + 1];
        v[2 * i] = a * c - b * s;
        v[2 * i + 1] = a * s + b * c;
    }
}

/* llama_attn_core with kq_scale = 1/sqrt(head_dim)  src/m6_engine.c:425-517 */
void or_llama_attn_op(const float* xn, void* pv, int pos, float* out) {
    OrLlamaAttnP* p = (OrLlamaAttnP*)pv;
    const int NH = p->n_head, NKV = p->n_kv, HD = p->head_dim, H = p->hidden;
    const int QD = NH * HD, KD = NKV * HD, T = *p->tlen, Tn = T + 1;
    const float scale = 1.0f / sqrtf((float)HD);
    float* q = p->work;
    float* k = q + QD;
    float* v = k + KD;
    float* sc = v + KD;
    const int rep = NH / NKV;
    or_gemv(p->cq, xn, p->wq, QD, H, q);
    or_gemv(p->ck, xn, p->wk, KD, H, k);
    or_gemv(p->cv, xn, p->wv, KD, H, v);
    for (int h = 0; h < NH; h++) rope_pairs(q + h * HD, p->rot, pos, p->rope_base);
    for (int h = 0; h < NKV; h++) rope_pairs(k + h * HD, p->rot, pos, p->rope_base);
    memcpy(p->kcache + (size_t)T * KD, k, sizeof(float) * KD);
    memcpy(p->vcache + (size_t)T * KD, v, sizeof(float) * KD);
    #pragma omp parallel for schedule(static)
    for (int h = 0; h < NH; h++) {
        const int kv = h / rep;
        const float* qh = q + h * HD;
        float* sh = sc + (size_t)h * p->max_t;
        float mx = -1e30f;
        for (int t = 0; t < Tn; t++) {
            const float* kt = p->kcache + (size_t)t * KD + kv * HD;
            float s = 0.f;
            for (int i = 0; i < HD; i++) s += qh[i] * kt[i];
            s *= scale;
            sh[t] = s;
            if (s > mx) mx = s;
        }
        float sum = 0.f;
        for (int t = 0; t < Tn; t++) {
            sh[t] = expf(sh[t] - mx);
            sum += sh[t];
        }
        const float inv = 1.f / sum;
        float oh[512];
        for (int i = 0; i < HD; i++) oh[i] = 0.f;
        for (int t = 0; t < Tn; t++) {
            const float pw = sh[t] * inv;
            const float* vt = p->vcache + (size_t)t * KD + kv * HD;
            for (int i = 0; i < HD; i++) oh[i] += pw * vt[i];
        }
        /* the reference writes the head output over q (the head's own slot) */
        memcpy(q + h * HD, oh, sizeof(float) * HD);
    }
    or_gemv(p->co, q, p->wo, H, QD, out);
    *p->tlen = Tn;
}

/* SwiGLU dense FFN  src/m6_engine.c:275-303 */
void or_dense_op(const float* xn, void* pv, float* out) {
    OrDenseP* p = (OrDenseP*)pv;
    const int FF = p->n_ff, H = p->h;
    float* g = (float*)malloc(sizeof(float) * (size_t)FF);
    float* u = (float*)malloc(sizeof(float) * (size_t)FF);
    or_gemv(p->cg, xn, p->g, FF, H, g);
    or_gemv(p->cu, xn, p->u, FF, H, u);
    for (int i = 0; i < FF; i++) {
        const float gv = g[i];
        g[i] = (gv / (1.f + expf(-gv))) * u[i];
    }
    or_gemv(p->cd, g, p->d, H, FF, out);
    free(g);
    free(u);
}

/* m6_forward_token  src/m6_engine.c:61-83 (the duplicate ffn-norm at :71 is
 * dead work and omitted; the norm that feeds the FFN is the one at :76). */
int or_forward_token(float* x, int h, float eps, int pos, const OrLayerDesc* layers,
                     int n_layer, float* scratch) {
    const int span = h + 64;
    float* xn = scratch;
    float* sub = scratch + 2 * span;
    for (int il = 0; il < n_layer; il++) {
        const OrLayerDesc* L = layers + il;
        or_rms_norm(x, L->attn_norm, h, eps, xn);
        L->attn(xn, L->attn_p, pos, sub);
        for (int i = 0; i < h; i++) x[i] += sub[i];
        or_rms_norm(x, L->ffn_norm, h, eps, xn);
        L->ffn(xn, L->ffn_p, sub);
        for (int i = 0; i < h; i++) x[i] += sub[i];
    }
    return 0;
}

/* m6_head_op  src/m6_engine.c:373-391 */
int or_head_op(const float* x, const float* final_norm, int h, float eps,
               const uint8_t* head_w, int code, int vocab, float* logits, float* scratch) {
    or_rms_norm(x, final_norm, h, eps, scratch);
    return or_gemv(code, scratch, head_w, vocab, h, logits);
}

/* a19  greedy pick: np.argmax over a float64 copy (src/smol_engine.py:212,
 * src/draco_engine_server.py:754) -- first index wins ties, and numpy ranks
 * NaN above every number, so the first NaN's index is the result when any
 * value is NaN. */
int or_argmax(const float* v, int n) {
    for (int i = 0; i < n; i++) if (v[i] != v[i]) return i;
    int best = 0;
    for (int i = 1; i < n; i++) if (v[i] > v[best]) best = i;
    return best;
}

/* ------------------------------------------------------------------ */
/* a20  softmax router + stable top-k + renorm + expert FFN            */
/*      src/m6_layer.c:771-802 (router), :808-821 (top-k),             */
/*      :699-764 (experts; the weighted sum runs j = 0..n_used-1)      */
/* ------------------------------------------------------------------ */
void or_topk(const float* v, int n, int k, int* out) {
    char used[4096];
    for (int i = 0; i < n; i++) used[i] = 0;
    for (int t = 0; t < k; t++) {
        int best = -1;
        float bv = -1e30f;
        for (int i = 0; i < n; i++) {
            if (used[i]) continue;
            if (v[i] > bv) { bv = v[i]; best = i; }
        }
        out[t] = best;
        used[best] = 1;
    }
}

/* Route one token.  probs[n_exp] (softmax), idx[n_used], wtop[n_used]. */
void or_moe_route(const float* x0, const float* gate_inp, int n_exp, int n_used, int n_in,
                  float* probs, int* idx, float* wtop) {
    for (int e = 0; e < n_exp; e++) {
        const float* w = gate_inp + (size_t)e * n_in;
        float acc = 0.f;
        for (int i = 0; i < n_in; i++) acc += x0[i] * w[i];
        probs[e] = acc;
    }
    float mx = -1e30f;
    for (int e = 0; e < n_exp; e++) if (probs[e] > mx) mx = probs[e];
    float s = 0.f;
    for (int e = 0; e < n_exp; e++) { probs[e] = expf(probs[e] - mx); s += probs[e]; }
    const float inv = 1.f / s;
    for (int e = 0; e < n_exp; e++) probs[e] *= inv;
    or_topk(probs, n_exp, n_used, idx);
    float ws = 0.f;
    for (int j = 0; j < n_used; j++) { wtop[j] = probs[idx[j]]; ws += wtop[j]; }
    if (ws < 6.103515625e-5f) ws = 6.103515625e-5f;
    for (int j = 0; j < n_used; j++) wtop[j] /= ws;
}

void or_granite_moe(const float* x0, const uint64_t* ptrs, const int* codes,
                    const float* gate_inp, int n_exp, int n_used,
                    int inter, int n_in, int n_out, float* scratch, float* out) {
    float probs[4096], wtop[64];
    int idx[64];
    or_moe_route(x0, gate_inp, n_exp, n_used, n_in, probs, idx, wtop);
    float* gu = scratch;
    float* uu = gu + (size_t)n_used * inter;
    float* act = uu + (size_t)n_used * inter;
    float* yd = act + (size_t)n_used * inter;
    for (int j = 0; j < n_used; j++) {
        const int e = idx[j];
        or_gemv(codes[3 * e + 0], x0, (const uint8_t*)(uintptr_t)ptrs[3 * e + 0], inter, n_in,
                gu + (size_t)j * inter);
        or_gemv(codes[3 * e + 1], x0, (const uint8_t*)(uintptr_t)ptrs[3 * e + 1], inter, n_in,
                uu + (size_t)j * inter);
    }
    for (int i = 0; i < n_used * inter; i++) {
        const float gv = gu[i];
        act[i] = (gv / (1.f + expf(-gv))) * uu[i];
    }
    for (int j = 0; j < n_used; j++) {
        const int e = idx[j];
        or_gemv(codes[3 * e + 2], act + (size_t)j * inter,
                (const uint8_t*)(uintptr_t)ptrs[3 * e + 2], n_out, inter, yd + (size_t)j * n_out);
    }
    for (int i = 0; i < n_out; i++) {
        float a = 0.f;
        for (int j = 0; j < n_used; j++) a += wtop[j] * yd[(size_t)j * n_out + i];
        out[i] = a;
    }
}

/* The MoE FFN as an m6 ffn op (OrLayerDesc.ffn): m6_granite_moe's arguments
 * packed in one struct (the product's DracoMoeP, field for field), as the
 * reference's qwen35 driver passes them per layer (src/qwen35_engine.py:
 * 293-307, the MoE half of _ffn).  scratch >= 3*n_used*inter + n_used*n_out. */
typedef struct {
    const uint64_t* ptrs;
    const int* codes;
    const float* gate_inp;
    int n_exp, n_used, inter, n_in, n_out;
    float* scratch;
} OrMoeP;

void or_moe_ffn_op(const float* xn, void* pv, float* out) {
    const OrMoeP* p = (const OrMoeP*)pv;
    or_granite_moe(xn, p->ptrs, p->codes, p->gate_inp, p->n_exp, p->n_used, p->inter, p->n_in, p->n_out,
                   p->scratch, out);
}

/* gemv_any's inline F32 branch, src/m6_layer.c:148-174: four 16-lane fma
 * accumulators over 64-value steps (a 16-value tail into the first), the
 * lane sums (a0+a1)+(a2+a3), GCC's _mm512_reduce_add_ps tree, then the
 * scalar tail.  Every other code goes to the scalar kernels (or_gemv). */
static float hsum16(const float* a);
static void or_gemv_any(int code, const float* x, const uint8_t* buf, int n_out, int n_in, float* y) {
    if (code != 9) {
        or_gemv(code, x, buf, n_out, n_in, y);
        return;
    }
    const float* w = (const float*)buf;
    for (int r = 0; r < n_out; r++) {
        const float* wr = w + (size_t)r * n_in;
        float a[4][16] = {{0}};
        int i = 0;
        for (; i + 63 < n_in; i += 64)
            for (int q = 0; q < 4; q++)
                for (int l = 0; l < 16; l++) a[q][l] = fmaf(wr[i + 16 * q + l], x[i + 16 * q + l], a[q][l]);
        for (; i + 15 < n_in; i += 16)
            for (int l = 0; l < 16; l++) a[0][l] = fmaf(wr[i + l], x[i + l], a[0][l]);
        float t[16];
        for (int l = 0; l < 16; l++) t[l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
        float s = hsum16(t);
        for (; i < n_in; i++) s = fmaf(wr[i], x[i], s);
        y[r] = s;
    }
}

/* a21  qwen35moe shared expert  src/m6_engine.c:1111-1127: SwiGLU FFN
 * scaled by sigmoid of the one-row gate product.  shp/shc = {gate, up, down,
 * gate_inp}; sh holds [gate | up] and then the activation in its first half. */
void or_granite_shexp(const float* x, const uint64_t* shp, const int* shc, float* sg, float* sh,
                      float* shg, float* out, int shi, int h) {
    or_gemv_any(shc[3], x, (const uint8_t*)(uintptr_t)shp[3], 1, h, sg);
    or_gemv_any(shc[0], x, (const uint8_t*)(uintptr_t)shp[0], shi, h, sh);
    or_gemv_any(shc[1], x, (const uint8_t*)(uintptr_t)shp[1], shi, h, sh + shi);
    for (int i = 0; i < shi; i++) {
        const float gv = sh[i];
        sh[i] = (gv / (1.f + expf(-gv))) * sh[shi + i];
    }
    or_gemv_any(shc[2], sh, (const uint8_t*)(uintptr_t)shp[2], h, shi, shg);
    const float gate = 1.f / (1.f + expf(-sg[0]));
    for (int i = 0; i < h; i++) out[i] = shg[i] * gate;
}

/* ------------------------------------------------------------------ */
/* a24  GDN token-serial scan  src/m6_gdn_scan.c:18-93                 */
/* ------------------------------------------------------------------ */
#define GDN_SV 128
#define GDN_EPS 1e-6f

/* one token of the delta rule for V head h; S_h is [128 k][128 v] */
static void gdn_head_step(float* S_h, const float* kj, const float* qj, const float* vh,
                          float g, float b, float* o) {
    float sk[GDN_SV], dl[GDN_SV];
    for (int kk = 0; kk < GDN_SV; kk++)
        for (int vv = 0; vv < GDN_SV; vv++) S_h[kk * GDN_SV + vv] *= g;
    for (int vv = 0; vv < GDN_SV; vv++) sk[vv] = 0.f;
    for (int kk = 0; kk < GDN_SV; kk++) {
        const float kv = kj[kk];
        for (int vv = 0; vv < GDN_SV; vv++) sk[vv] += S_h[kk * GDN_SV + vv] * kv;
    }
    for (int vv = 0; vv < GDN_SV; vv++) dl[vv] = (vh[vv] - sk[vv]) * b;
    for (int kk = 0; kk < GDN_SV; kk++) {
        const float kv = kj[kk];
        for (int vv = 0; vv < GDN_SV; vv++) S_h[kk * GDN_SV + vv] += kv * dl[vv];
    }
    for (int vv = 0; vv < GDN_SV; vv++) sk[vv] = 0.f;
    for (int kk = 0; kk < GDN_SV; kk++) {
        const float qv = qj[kk];
        for (int vv = 0; vv < GDN_SV; vv++) sk[vv] += S_h[kk * GDN_SV + vv] * qv;
    }
    for (int vv = 0; vv < GDN_SV; vv++) o[vv] = sk[vv];
}

/* depthwise 4-tap conv + silu with the 3-sample tail shift
 * (src/m6_gdn_scan.c:30-38, src/m6_layer.c:262-270) */
static void gdn_conv(const float* qkv, const float* conv, float* tail, float* cout, int n_qkv) {
    for (int i = 0; i < n_qkv; i++) {
        const float* wk = conv + i * 4;
        const float acc = wk[0] * tail[i * 3] + wk[1] * tail[i * 3 + 1] + wk[2] * tail[i * 3 + 2]
                        + wk[3] * qkv[i];
        cout[i] = acc / (1.f + expf(-acc));
        tail[i * 3] = tail[i * 3 + 1];
        tail[i * 3 + 1] = tail[i * 3 + 2];
        tail[i * 3 + 2] = qkv[i];
    }
}

void or_gdn_scan(const float* QKV, const float* Z, const float* B, const float* G,
                 const float* conv, const float* ssm_norm, float* tail,
                 float* S, int T, int n_qkv, int n_vh, float* ON, float* work) {
    const int NHQ = (n_qkv - n_vh * GDN_SV) / (2 * GDN_SV);
    const float scale = 1.f / sqrtf((float)GDN_SV);
    float* cout = work;
    for (int t = 0; t < T; t++) {
        gdn_conv(QKV + (size_t)t * n_qkv, conv, tail, cout, n_qkv);
        for (int j = 0; j < 2 * NHQ; j++) {                 /* sum-form l2 norm */
            float* hv = cout + j * GDN_SV;
            float n2 = 0.f;
            for (int u = 0; u < GDN_SV; u++) n2 += hv[u] * hv[u];
            const float inv = 1.f / (sqrtf(n2) > GDN_EPS ? sqrtf(n2) : GDN_EPS);
            for (int u = 0; u < GDN_SV; u++) hv[u] *= inv;
        }
        const float* z = Z + (size_t)t * n_vh * GDN_SV;
        #pragma omp parallel for schedule(static)
        for (int h = 0; h < n_vh; h++) {
            const int j = h % NHQ;
            float oh[GDN_SV];
            gdn_head_step(S + (size_t)h * GDN_SV * GDN_SV, cout + NHQ * GDN_SV + j * GDN_SV,
                          cout + j * GDN_SV, cout + 2 * NHQ * GDN_SV + h * GDN_SV,
                          G[t * n_vh + h], B[t * n_vh + h], oh);
            float ms2 = 0.f;
            for (int vv = 0; vv < GDN_SV; vv++) { oh[vv] = oh[vv] * scale; ms2 += oh[vv] * oh[vv]; }
            const float inv2 = 1.f / sqrtf(ms2 / GDN_SV + GDN_EPS);
            float* on = ON + (size_t)t * n_vh * GDN_SV + (size_t)h * GDN_SV;
            for (int vv = 0; vv < GDN_SV; vv++) {
                const float zv = z[h * GDN_SV + vv];
                on[vv] = oh[vv] * inv2 * ssm_norm[vv] * (zv / (1.f + expf(-zv)));
            }
        }
    }
}

/* ------------------------------------------------------------------ */
/* a23  GDN decode op (qwen35 linear-attention layer, one token)       */
/*      src/m6_layer.c:189-364.  Hidden width 2048 and 16 q/k heads    */
/*      are fixed, as in the reference (src/m6_layer.c:11-13).         */
/*      Struct layout = the reference's GdnW (src/m6_layer.c:189-202,  */
/*      ctypes twin src/qwen35_engine.py:137-146).                     */
/* ------------------------------------------------------------------ */
#define QW_H 2048
#define QW_NKH 16

typedef struct {
    const float* attn_norm;
    const uint8_t* qkv_buf; int qkv_code;
    const uint8_t* gate_buf; int gate_code;
    const float* beta_wt;   /* [2048][n_vh] */
    const float* alpha_wt;
    const float* ssm_a;
    const float* ssm_dt;
    const float* conv;      /* [n_qkv][4] */
    const float* ssm_norm;  /* [128] */
    const uint8_t* ssm_out_buf; int ssm_out_code;
    const float* post_norm;
    int n_qkv; int n_vh; int d_in;
} OrGdnW;

/* x2_out = h1 + ssm_out(gated rms(delta rule(l2norm(conv(qkv(rms(h1))))))),
 * x2n = rms(x2_out) * post_norm; ssm [n_vh][128][128] and tail [n_qkv][3]
 * updated in place.  The reference sums the post-norm square in per-thread
 * partials (src/m6_layer.c:343-361); this restatement sums sequentially, so
 * x2n agrees to fp32 rounding, every other output bit for bit. */
int or_gdn_attn(const float* h1, const OrGdnW* w, float* ssm, float* tail,
                float* x2n, float* x2_out) {
    const int NQKV = w->n_qkv, NVH = w->n_vh, DIN = w->d_in;
    if (NVH < 1 || NVH > 64 || NQKV != 2 * QW_NKH * GDN_SV + NVH * GDN_SV || DIN != NVH * GDN_SV) return -1;
    float* xn = (float*)malloc(sizeof(float) * (QW_H + 2 * (size_t)NQKV + 2 * (size_t)NVH * GDN_SV + QW_H));
    float* qkv = xn + QW_H;
    float* cout = qkv + NQKV;
    float* z = cout + NQKV;
    float* on = z + NVH * GDN_SV;
    float* attn = on + NVH * GDN_SV;
    float ms = 0.f;
    for (int i = 0; i < QW_H; i++) ms += h1[i] * h1[i];
    float inv = 1.f / sqrtf(ms / (float)QW_H + GDN_EPS);
    for (int i = 0; i < QW_H; i++) xn[i] = h1[i] * inv * w->attn_norm[i];
    or_gemv(w->qkv_code, xn, w->qkv_buf, NQKV, QW_H, qkv);
    or_gemv(w->gate_code, xn, w->gate_buf, NVH * GDN_SV, QW_H, z);
    /* beta = sigmoid(x.Wb), alpha = softplus(x.Wa + dt) * a  (:240-256) */
    float beta[64], gdec[64], bacc[64], aacc[64];
    for (int i = 0; i < NVH; i++) bacc[i] = aacc[i] = 0.f;
    for (int t = 0; t < QW_H; t++) {
        const float xt = xn[t];
        for (int i = 0; i < NVH; i++) {
            bacc[i] += w->beta_wt[(size_t)t * NVH + i] * xt;
            aacc[i] += w->alpha_wt[(size_t)t * NVH + i] * xt;
        }
    }
    for (int i = 0; i < NVH; i++) {
        beta[i] = 1.f / (1.f + expf(-bacc[i]));
        const float av = aacc[i] + w->ssm_dt[i];
        const float sp = av > 0 ? av + log1pf(expf(-av)) : log1pf(expf(av));
        gdec[i] = expf(sp * w->ssm_a[i]);
    }
    gdn_conv(qkv, w->conv, tail, cout, NQKV);                      /* :262-270 */
    for (int j = 0; j < 2 * QW_NKH; j++) {                          /* :274-280 */
        float* hv = cout + j * GDN_SV;
        float n2 = 0.f;
        for (int u = 0; u < GDN_SV; u++) n2 += hv[u] * hv[u];
        const float r = 1.f / fmaxf(sqrtf(n2), GDN_EPS);
        for (int u = 0; u < GDN_SV; u++) hv[u] *= r;
    }
    const float scale = 1.f / sqrtf((float)GDN_SV);
    for (int h = 0; h < NVH; h++) {                                 /* :283-331 */
        const int j = h % QW_NKH;
        float oh[GDN_SV];
        gdn_head_step(ssm + (size_t)h * GDN_SV * GDN_SV, cout + QW_NKH * GDN_SV + j * GDN_SV,
                      cout + j * GDN_SV, cout + 2 * QW_NKH * GDN_SV + h * GDN_SV, gdec[h], beta[h], oh);
        float ms2 = 0.f;
        for (int vv = 0; vv < GDN_SV; vv++) { oh[vv] = oh[vv] * scale; ms2 += oh[vv] * oh[vv]; }
        const float inv2 = 1.f / sqrtf(ms2 / GDN_SV + GDN_EPS);
        for (int vv = 0; vv < GDN_SV; vv++) {
            const float zv = z[h * GDN_SV + vv];
            on[h * GDN_SV + vv] = oh[vv] * inv2 * w->ssm_norm[vv] * (zv / (1.f + expf(-zv)));
        }
    }
    or_gemv(w->ssm_out_code, on, w->ssm_out_buf, QW_H, DIN, attn);  /* :332-340 */
    ms = 0.f;
    for (int i = 0; i < QW_H; i++) { x2_out[i] = h1[i] + attn[i]; ms += x2_out[i] * x2_out[i]; }
    inv = 1.f / sqrtf(ms / (float)QW_H + GDN_EPS);
    for (int i = 0; i < QW_H; i++) x2n[i] = x2_out[i] * inv * w->post_norm[i];
    free(xn);
    return 0;
}

/* ------------------------------------------------------------------ */
/* a25  qwen35 full attention (one token)  src/m6_layer.c:375-518.     */
/*      Head dim 256, 2 KV heads, rope on pairs (t, t+32), t < 32.     */
/*      Struct layout = the reference's FullW (src/m6_layer.c:375-387, */
/*      ctypes twin src/qwen35_engine.py:149-157).                     */
/* ------------------------------------------------------------------ */
typedef struct {
    const float* attn_norm;
    const uint8_t* q_buf; int q_code;   /* nh*512 rows: per head q[256] | gate[256] */
    const uint8_t* k_buf; int k_code;   /* 512 rows */
    const uint8_t* v_buf; int v_code;   /* 512 rows */
    const float* q_norm;                /* [256] */
    const float* k_norm;
    const uint8_t* o_buf; int o_code;   /* 2048 rows, nh*256 wide */
    const float* post_norm;
    const float* rope_inv;              /* [32] */
    int nh;
} OrFullW;

/* Kr/Vc: Told cached rows of [2][256]; the new row is computed here and
 * returned in kr_new (normed + roped) / v_new.  Every output is bitwise the
 * reference's on the same inputs (sequential sums throughout there too). */
int or_full_attn(const float* h1, const OrFullW* w, const float* Kr, const float* Vc, int Told,
                 int pos0, float* x2n, float* x2_out, float* kr_new, float* v_new) {
    const int HD = 256, NKV = 2, HALF = 32, NH = w->nh;
    if (NH < NKV || NH % NKV || NH > 64 || Told < 0) return -1;
    const int NQG = NH * 2 * HD, T = Told + 1;
    float* xn = (float*)malloc(sizeof(float) * ((size_t)QW_H * 2 + NQG + 2 * (size_t)NH * HD + T));
    float* QG = xn + QW_H;
    float* Qr = QG + NQG;
    float* ao = Qr + NH * HD;
    float* attn = ao + NH * HD;
    float* sc = attn + QW_H;
    float ms = 0.f;
    for (int i = 0; i < QW_H; i++) ms += h1[i] * h1[i];
    float inv = 1.f / sqrtf(ms / (float)QW_H + GDN_EPS);
    for (int i = 0; i < QW_H; i++) xn[i] = h1[i] * inv * w->attn_norm[i];
    or_gemv(w->q_code, xn, w->q_buf, NQG, QW_H, QG);
    or_gemv(w->k_code, xn, w->k_buf, NKV * HD, QW_H, kr_new);
    or_gemv(w->v_code, xn, w->v_buf, NKV * HD, QW_H, v_new);
    for (int kv = 0; kv < NKV; kv++) {                    /* :427-441 k: x *= (r * w) */
        float* kh = kr_new + kv * HD;
        float n2 = 0.f;
        for (int t = 0; t < HD; t++) n2 += kh[t] * kh[t];
        n2 = 1.f / sqrtf(n2 / HD + GDN_EPS);
        for (int t = 0; t < HD; t++) kh[t] *= n2 * w->k_norm[t];
        for (int t = 0; t < HALF; t++) {
            const float ang = (float)pos0 * w->rope_inv[t];
            const float c = cosf(ang), s = sinf(ang);
            const float a = kh[t], b = kh[t + HALF];
            kh[t] = a * c - b * s;
            kh[t + HALF] = a * s + b * c;
        }
    }
    for (int h = 0; h < NH; h++) {                        /* :443-457 q: (x * r) * w */
        const float* qh = QG + h * 2 * HD;
        float* qo = Qr + h * HD;
        float n2 = 0.f;
        for (int t = 0; t < HD; t++) n2 += qh[t] * qh[t];
        n2 = 1.f / sqrtf(n2 / HD + GDN_EPS);
        for (int t = 0; t < HD; t++) qo[t] = qh[t] * n2 * w->q_norm[t];
        for (int t = 0; t < HALF; t++) {
            const float ang = (float)pos0 * w->rope_inv[t];
            const float c = cosf(ang), s = sinf(ang);
            const float a = qo[t], b = qo[t + HALF];
            qo[t] = a * c - b * s;
            qo[t + HALF] = a * s + b * c;
        }
    }
    const float scale = 1.f / sqrtf((float)HD);
    for (int h = 0; h < NH; h++) {                        /* :459-499 */
        const int kv = h / (NH / NKV);
        const float* qh = Qr + h * HD;
        for (int t = 0; t < T; t++) {
            const float* krow = t < Told ? Kr + (size_t)t * NKV * HD + kv * HD : kr_new + kv * HD;
            float acc = 0.f;
            for (int d = 0; d < HD; d++) acc += qh[d] * krow[d];
            sc[t] = acc * scale;
        }
        float mx = sc[0];
        for (int t = 1; t < T; t++) if (sc[t] > mx) mx = sc[t];
        float sum = 0.f;
        for (int t = 0; t < T; t++) { sc[t] = expf(sc[t] - mx); sum += sc[t]; }
        const float rsum = 1.f / sum;
        float* oh = ao + h * HD;
        for (int d = 0; d < HD; d++) oh[d] = 0.f;
        for (int t = 0; t < T; t++) {
            const float p = sc[t] * rsum;
            const float* vrow = t < Told ? Vc + (size_t)t * NKV * HD + kv * HD : v_new + kv * HD;
            for (int d = 0; d < HD; d++) oh[d] += p * vrow[d];
        }
    }
    for (int h = 0; h < NH; h++) {                        /* :500-505 sigmoid gate */
        float* oh = ao + h * HD;
        const float* gh = QG + h * 2 * HD + HD;
        for (int d = 0; d < HD; d++) oh[d] *= 1.f / (1.f + expf(-gh[d]));
    }
    or_gemv(w->o_code, ao, w->o_buf, QW_H, NH * HD, attn);
    ms = 0.f;
    for (int i = 0; i < QW_H; i++) { x2_out[i] = h1[i] + attn[i]; ms += x2_out[i] * x2_out[i]; }
    inv = 1.f / sqrtf(ms / (float)QW_H + GDN_EPS);
    for (int i = 0; i < QW_H; i++) x2n[i] = x2_out[i] * inv * w->post_norm[i];
    free(xn);
    return 0;
}

/* ------------------------------------------------------------------ */
/* a22  token-batched MoE  src/m6_moe_tok.c:44-161, restated with the  */
/* per-token expert FFN of the decode path.  Pinned by                 */
/* tests/test_oracle_pins.py: (1) token-batched == token-serial, bit   */
/* for bit (the reference's own gate, src/prefill_chunk_gate.py:25-46):*/
/* every (token, slot) runs the same scalar GEMVs as or_granite_moe's  */
/* expert phase and the scatter adds slots in k order; (2) within      */
/* 1e-5 of the compiled src/m6_moe_tok.c (tests/golden/moetok.npz),    */
/* whose dots are 16-lane FMA trees.                                   */
/* ------------------------------------------------------------------ */
void or_moe_tok(const float* X, const int* order, const float* wtop,
                const uint64_t* ep, const int* ec, int T, int n_used, int inter,
                int n_in, int n_out, int n_exp, float* out) {
    memset(out, 0, sizeof(float) * (size_t)T * n_out);
    #pragma omp parallel
    {
        float* gu = (float*)malloc(sizeof(float) * (size_t)inter * 3);
        float* uu = gu + inter;
        float* act = uu + inter;
        float* yd = (float*)malloc(sizeof(float) * (size_t)n_out);
        #pragma omp for schedule(static)
        for (int t = 0; t < T; t++) {
            float* o = out + (size_t)t * n_out;
            for (int k = 0; k < n_used; k++) {
                const int e = order[t * n_used + k];
                if (e < 0 || e >= n_exp) continue;
                const float* xt = X + (size_t)t * n_in;
                or_gemv_range(ec[3 * e], xt, (const uint8_t*)(uintptr_t)ep[3 * e], inter, n_in, gu, 0, inter);
                or_gemv_range(ec[3 * e + 1], xt, (const uint8_t*)(uintptr_t)ep[3 * e + 1], inter, n_in, uu, 0, inter);
                for (int i = 0; i < inter; i++) {
                    const float gv = gu[i];
                    act[i] = (gv / (1.f + expf(-gv))) * uu[i];
                }
                or_gemv_range(ec[3 * e + 2], act, (const uint8_t*)(uintptr_t)ep[3 * e + 2], n_out, inter, yd, 0, n_out);
#if OR_MUTANT == 5
                const float w = wtop[t * n_used];
#else
                const float w = wtop[t * n_used + k];
#endif
                for (int r = 0; r < n_out; r++) o[r] += w * yd[r];
            }
        }
        free(gu);
        free(yd);
    }
}

/* ------------------------------------------------------------------ */
/* a26  prefill GEMM  Y[T x n_out] = X[T x n_in] . W^T                 */
/* m5_gemm semantics (src/m5/m5_gemm.c:249-272): dequantize each row   */
/* once (a12), then one dot per token.  The reference's dot is a       */
/* 16-lane AVX-512 tree; this restatement sums sequentially, so it is  */
/* pinned by invariants (tests/test_oracle_pins.py: == stacked GEMVs  */
/* within 1e-6, one-hot token rows give the dequantized columns bit    */
/* for bit), not bitwise -- m5_gemm.c cannot be built here (its header */
/* iq3s_grid.h is absent from the tree).                               */
/* ------------------------------------------------------------------ */
int or_gemm(int code, const float* X, const uint8_t* W, int T, int n_out, int n_in, float* Y) {
    if (!or_supported(code)) return -1;
    const size_t rs = or_rowbytes(code, n_in);
    #pragma omp parallel
    {
        float* wb = (float*)malloc(sizeof(float) * (size_t)n_in);
        #pragma omp for schedule(dynamic, 4)
        for (int r = 0; r < n_out; r++) {
            or_dequant_row(code, W + (size_t)r * rs, n_in, wb);
            for (int t = 0; t < T; t++) {
                const float* xt = X + (size_t)t * n_in;
                float s = 0.f;
                for (int i = 0; i < n_in; i++) s += wb[i] * xt[i];
#if OR_MUTANT == 4
                Y[(size_t)r * T + t] = s;
#else
                Y[(size_t)t * n_out + r] = s;
#endif
            }
        }
        free(wb);
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* a5  AVX-512 grouped Q4_K / Q6_K GEMV in m5_batch8_k.c lane order    */
/*     src/m5/m5_batch8_k.c:28-183 (the o0/o1 redundancy fixed: every  */
/*     row is computed once).  A 16-lane accumulator is emulated with  */
/*     fmaf, and the final horizontal sum follows GCC's                */
/*     _mm512_reduce_add_ps tree (halves 8+8, 4+4, 2+2, 1+1).          */
/* ------------------------------------------------------------------ */
static float hsum16(const float* a) {
    float t8[8], t4[4], t2[2];
    for (int i = 0; i < 8; i++) t8[i] = a[i] + a[i + 8];
    for (int i = 0; i < 4; i++) t4[i] = t8[i] + t8[i + 4];
    for (int i = 0; i < 2; i++) t2[i] = t4[i] + t4[i + 2];
    return t2[0] + t2[1];
}

static float sum32_lanes(const float* xp) {
    float s[16];
    for (int l = 0; l < 16; l++) s[l] = xp[l] + xp[l + 16];
    return hsum16(s);
}

int or_gemvn_q4k(const float* x, long x_stride, const uint8_t* W, const int* idx, long per,
                 int n_out_e, int n_in, int n_exp, float* y) {
    const int nb = n_in / 256;
    if (nb <= 0 || n_in % 256 != 0 || nb > 256) return -1;
    #pragma omp parallel for schedule(static)
    for (int e = 0; e < n_exp; e++) {
        const uint8_t* Wb = W + (int64_t)idx[e] * per;
        const float* xe = x + (int64_t)e * x_stride;
        float sx[256 * 8];
        for (int b = 0; b < nb; b++)
            for (int g = 0; g < 8; g++) sx[b * 8 + g] = sum32_lanes(xe + b * 256 + g * 32);
        for (int o = 0; o < n_out_e; o++) {
            const uint8_t* rowp = Wb + (size_t)o * nb * 144;
            float acc[16] = {0};
            for (int b = 0; b < nb; b++) {
                const uint8_t* blk = rowp + (size_t)b * 144;
                const float d = ld_f16(blk), dmin = ld_f16(blk + 2);
                float sc[8], mn[8];
                kq_scales(blk + 4, sc, mn);
                float scf[8], minf[8];
                for (int i = 0; i < 8; i++) { scf[i] = d * sc[i]; minf[i] = dmin * mn[i]; }
                const uint8_t* qs = blk + 16;
                const float* xp = xe + b * 256;
                for (int g = 0; g < 8; g++) {
                    const uint8_t* qb = qs + (g >> 1) * 32;
                    const int hi = g & 1;
                    float dotv[16];
                    for (int l = 0; l < 16; l++) {
                        const float f0 = (float)(hi ? (qb[l] >> 4) : (qb[l] & 0xF));
                        const float f1 = (float)(hi ? (qb[16 + l] >> 4) : (qb[16 + l] & 0xF));
                        dotv[l] = fmaf(f1, xp[g * 32 + 16 + l], f0 * xp[g * 32 + l]);
                    }
                    for (int l = 0; l < 16; l++) acc[l] = fmaf(scf[g], dotv[l], acc[l]);
                    acc[0] = fmaf(-minf[g], sx[b * 8 + g], acc[0]);
                    for (int l = 1; l < 16; l++) acc[l] = fmaf(-minf[g], 0.f, acc[l]);
                }
            }
            y[(int64_t)e * n_out_e + o] = hsum16(acc);
        }
    }
    return 0;
}

int or_gemvn_q6k(const float* x, long x_stride, const uint8_t* W, const int* idx, long per,
                 int n_out_e, int n_in, int n_exp, float* y) {
    const int nb = n_in / 256;
    if (nb <= 0 || n_in % 256 != 0) return -1;
    #pragma omp parallel for schedule(static)
    for (int e = 0; e < n_exp; e++) {
        const uint8_t* Wb = W + (int64_t)idx[e] * per;
        const float* xe = x + (int64_t)e * x_stride;
        for (int o = 0; o < n_out_e; o++) {
            const uint8_t* rowp = Wb + (size_t)o * nb * 210;
            float acc[16] = {0};
            for (int b = 0; b < nb; b++) {
                const uint8_t* blk = rowp + (size_t)b * 210;
                const uint8_t* ql = blk;
                const uint8_t* qh = blk + 128;
                const int8_t* sc = (const int8_t*)(blk + 192);
                const float d = ld_f16(blk + 208);
                const float* xs = xe + b * 256;
                float scf[16];
                for (int i = 0; i < 16; i++) scf[i] = d * (float)sc[i];
                for (int sb = 0; sb < 2; sb++)
                    for (int g2 = 0; g2 < 4; g2++) {
                        const uint8_t* l16 = ql + sb * 64 + g2 * 16;
                        const uint8_t* h16 = qh + sb * 32 + (g2 & 1) * 16;
                        const int base = sb * 8 + g2;
                        const int sh0 = ((base >> 1) & 3) * 2;
                        const int sh1 = (((base + 4) >> 1) & 3) * 2;
                        for (int l = 0; l < 16; l++) {
                            const int q = ((l16[l] & 0xF) | (((h16[l] >> sh0) & 3) << 4)) - 32;
                            acc[l] = fmaf((float)q * scf[base], xs[base * 16 + l], acc[l]);
                        }
                        for (int l = 0; l < 16; l++) {
                            const int q = (((l16[l] >> 4) & 0xF) | (((h16[l] >> sh1) & 3) << 4)) - 32;
                            acc[l] = fmaf((float)q * scf[base + 4], xs[(base + 4) * 16 + l], acc[l]);
                        }
                    }
            }
            y[(int64_t)e * n_out_e + o] = hsum16(acc);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* a10/a11  Q8_K activations and integer block dots (no reference in  */
/* the tree; llama.cpp b10819 ggml-quants.c published algorithm).      */
/* Block: { float d; int8 qs[256]; int16 bsums[16]; } = 292 bytes.     */
/* ------------------------------------------------------------------ */
#define Q8K_BYTES 292

static inline int nearest_even(float v) { return (int)rintf(v); }

void or_quantize_q8k(const float* x, int n, uint8_t* out) {
    for (int b = 0; b < n / 256; b++) {
        const float* xb = x + (size_t)b * 256;
        uint8_t* blk = out + (size_t)b * Q8K_BYTES;
        float amax = 0.f, mx = 0.f;
        for (int j = 0; j < 256; j++) {
            const float ax = fabsf(xb[j]);
            if (ax > amax) { amax = ax; mx = xb[j]; }
        }
        int8_t qs[256];
        int16_t bs[16];
        float d = 0.f;
        if (amax == 0.f) {
            memset(qs, 0, sizeof qs);
        } else {
            const float iscale = -127.f / mx;
            for (int j = 0; j < 256; j++) {
                const int v = nearest_even(iscale * xb[j]);
                qs[j] = (int8_t)(v < 127 ? v : 127);
            }
            d = 1.f / iscale;
        }
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int i = 0; i < 16; i++) s += qs[g * 16 + i];
            bs[g] = (int16_t)s;
        }
        memcpy(blk, &d, 4);
        memcpy(blk + 4, qs, 256);
        memcpy(blk + 260, bs, 32);
    }
}

/* Integer parts of one super-block dot.
 *   Q4_K: isc = sum_j sc_j * sum_{k in sub-block j} q4 * q8 ; imn = sum_j m_j * (bsum_2j + bsum_2j+1)
 *   Q6_K: isc = sum_g sc_g * sum_{k in group g} q6 * q8      ; imn = 0
 * Exact int32 (|isc| < 2^31 for every valid block). */
void or_q8k_block_isums(int code, const uint8_t* wblk, const uint8_t* xblk, int32_t* isc, int32_t* imn) {
    const int8_t* q8 = (const int8_t*)(xblk + 4);
    int16_t bs[16];
    memcpy(bs, xblk + 260, 32);
    if (code == 5) {
        const uint8_t* s = wblk + 4;
        const uint8_t* qs = wblk + 16;
        int sc[8], mn[8];
        for (int i = 0; i < 4; i++) {
            sc[i] = s[i] & 0x3F;
            sc[4 + i] = (s[8 + i] & 0x0F) | ((s[i] >> 2) & 0x30);
            mn[i] = s[4 + i] & 0x3F;
            mn[4 + i] = (s[8 + i] >> 4) | ((s[4 + i] >> 2) & 0x30);
        }
        int32_t a = 0, m = 0;
        for (int j = 0; j < 8; j++) {
            const uint8_t* qb = qs + (j >> 1) * 32;
            int32_t t = 0;
            for (int k = 0; k < 32; k++) {
                const int q = (j & 1) ? (qb[k] >> 4) : (qb[k] & 0xF);
                t += q * q8[j * 32 + k];
            }
            a += sc[j] * t;
            m += mn[j] * (bs[2 * j] + bs[2 * j + 1]);
        }
        *isc = a;
        *imn = m;
        return;
    }
    if (code == 4) {
        const uint8_t* ql = wblk;
        const uint8_t* qh = wblk + 128;
        const int8_t* sc = (const int8_t*)(wblk + 192);
        int32_t a = 0;
        for (int g = 0; g < 16; g++) {
            int32_t t = 0;
            for (int i = 0; i < 16; i++) {
                const int p = g * 16 + i;
                const uint8_t lb = ql[(p >> 7) * 64 + (p & 63)];
                const int lo4 = ((p >> 6) & 1) ? (lb >> 4) : (lb & 0x0F);
                const int hi2 = (qh[(p >> 7) * 32 + (p & 31)] >> (((p >> 5) & 3) * 2)) & 3;
                t += ((lo4 | (hi2 << 4)) - 32) * q8[p];
            }
            a += sc[g] * t;
        }
        *isc = a;
        *imn = 0;
        return;
    }
    *isc = 0;
    *imn = 0;
}

/* y[r] = sum_b ( (d8 * d) * isc_b - (d8 * dmin) * imn_b ), blocks in order. */
int or_gemv_q8k(int code, const uint8_t* xq, const uint8_t* W, int n_out, int n_in, float* y) {
    if (code != 4 && code != 5) return -1;
    const int nb = n_in / 256;
    const size_t rs = or_rowbytes(code, n_in);
    #pragma omp parallel for schedule(static) if (n_out >= 64)
    for (int r = 0; r < n_out; r++) {
        const uint8_t* row = W + (size_t)r * rs;
        float sum = 0.f;
        for (int b = 0; b < nb; b++) {
            const uint8_t* xb = xq + (size_t)b * Q8K_BYTES;
            float d8;
            memcpy(&d8, xb, 4);
            int32_t isc, imn;
            if (code == 5) {
                const uint8_t* wb = row + (size_t)b * 144;
                or_q8k_block_isums(5, wb, xb, &isc, &imn);
                const float d = d8 * ld_f16(wb), dmin = d8 * ld_f16(wb + 2);
                sum += d * (float)isc - dmin * (float)imn;
            } else {
                const uint8_t* wb = row + (size_t)b * 210;
                or_q8k_block_isums(4, wb, xb, &isc, &imn);
                const float d = d8 * ld_f16(wb + 208);
                sum += d * (float)isc;
            }
        }
        y[r] = sum;
    }
    return 0;
}

/* batch of nx activation rows: Y[t][r] */
int or_gemm_q8k(int code, const uint8_t* XQ, const uint8_t* W, int nx, int n_out, int n_in, float* Y) {
    const size_t xs = (size_t)(n_in / 256) * Q8K_BYTES;
    for (int t = 0; t < nx; t++) {
        const int rc = or_gemv_q8k(code, XQ + xs * t, W, n_out, n_in, Y + (size_t)t * n_out);
        if (rc) return rc;
    }
    return 0;
}

void or_set_threads(int n) { omp_set_num_threads(n); }
int or_get_threads(void) { return omp_get_max_threads(); }
