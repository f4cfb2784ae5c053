/*
 * draco_hip.h -- C ABI of libdraco_hip.so, the MI355X (gfx950) implementation
 * of the Dracomancer per-token decode path.
 *
 * Every entry point named m5_* / m6_* has the exact signature and meaning of
 * the reference function it replaces (cited file:line under the reference
 * tree).  All pointer arguments of those are caller-owned HOST pointers, as
 * in the reference; results are in host memory when the call returns.
 * Weights are uploaded (and repacked into a private device layout) on first
 * sight and then stay resident, keyed by their host address; their bytes must
 * not change while registered (draco_forget() drops an entry).
 *
 * Return codes: 0 ok, -1 unsupported code/shape (fail loudly, as the
 * reference's -1), -2 device error.  draco_last_error() describes the last
 * failure.  The library serialises callers with one mutex (the reference is
 * non-reentrant too: src/m6_layer.c:29-46).
 */
#ifndef DRACO_HIP_H
#define DRACO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- per-format kernel-library ABI (drop-in for m5_kern*.so) ----------- */

/* src/m5_kern_scalar.c:146-148.  1 if `code` is served (0 Q8_0, 3 Q5_K,
 * 4 Q6_K, 5 Q4_K, 7 F16, 9 F32: the reference scalar kernel's set). */
int m5_scalar_supported(int code);

/* src/m5_kern_scalar.c:150-156.  y[n_out] = W[n_out x n_in] . x */
int m5_gemv(int code, const float* x, const uint8_t* W, int n_out, int n_in, float* y);

/* src/m5_kern_scalar.c:158-165.  Rows [o0,o1) only, written at their absolute
 * index in y; other entries of y are not touched. */
int m5_gemv_range(int code, const float* x, const uint8_t* W, int n_out, int n_in, float* y,
                  int o0, int o1);

/* ---- layer-engine ABI (drop-in for m6_engine.so, llama path) ------------ */

/* Descriptor and parameter structs, field for field src/m6_engine.c:21-28,
 * :270-273 and :396-406 (ctypes mirrors: src/smol_engine.py:97-115). */
typedef void (*m6_attn_op)(const float* xn, void* p, int pos, float* out);
typedef void (*m6_ffn_op)(const float* xn, void* p, float* out);
typedef struct {
    const float* attn_norm;
    const float* ffn_norm;
    m6_attn_op attn;
    void* attn_p;
    m6_ffn_op ffn;
    void* ffn_p;
} M6LayerDesc;
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
} M6LlamaAttnP;
typedef struct {
    const uint8_t *g, *u, *d;
    int cg, cu, cd, n_ff, h;
} M6DenseP;

/* src/m6_engine.c:31-37 */
void m6_rms_norm(const float* x, const float* w, int h, float eps, float* out);
/* src/m6_engine.c:40-54 */
size_t m6_rowbytes(int code, int n_in);
/* src/m6_engine.c:85 */
const char* m6_engine_version(void);
/* src/m6_layer.c:123-140; kernel-slot paths accepted and ignored (returns 0). */
int m6_init_dl(const char* p012, const char* p3, const char* p4, const char* p56, const char* ps);
/* src/m6_layer.c:94-100; accepted (returns 0); Q5_0 (code 8) GEMVs return -1. */
int m6_init_extra_dl(const char* p50);
/* src/m6_layer.c:108-120 (the opt-in IQ3_S kernel slot, bound by
 * src/qwen35_engine.py:103-108 when DRACO_IQ3_FAST=1).  IQ3_S is not carried:
 * returns 1 ("could not load"), which the driver reports and goes on. */
int m6_init_iq3_dl(const char* p12);
/* src/m6_engine.c:61-83.  x[h] updated in place; every layer's *tlen += 1.
 * Layers whose ops are this library's m6_llama_attn_op / m6_dense_op run on
 * the device (KV caches mirrored on the device, see draco_state_pull/push);
 * any other op pointer returns -1. */
int m6_forward_token(float* x, int h, float eps, int pos, const M6LayerDesc* layers, int n_layer,
                     float* scratch);
/* src/m6_engine.c:373-391.  scratch[h] receives the normalised x. */
int m6_head_op(const float* x, const float* final_norm, int h, float eps, const uint8_t* head_w,
               int code, int vocab, float* logits, float* scratch);
/* src/m6_engine.c:514-517 (llama_attn_core, kq_scale 1/sqrt(head_dim)). */
void m6_llama_attn_op(const float* xn, void* p, int pos, float* out);
/* src/m6_engine.c:275-303 */
void m6_dense_op(const float* xn, void* p, float* out);
/* src/m6_engine.c:1111-1127 (qwen35moe shared expert).  shp/shc = {gate,
 * up, down, gate_inp}: out[h] = down(SwiGLU(gate.x, up.x)) *
 * sigmoid(gate_inp.x).  Also leaves shg[h] (ungated), sg[0] (gate logit) and
 * sh[0, shi) (activation); sh[shi, 2 shi) is scratch. */
void m6_granite_shexp(const float* x, const uint64_t* shp, const int* shc, float* sg, float* sh, float* shg,
                      float* out, int shi, int h);
/* Timing (no reference counterpart): m6_granite_shexp's device work
 * graph-replayed `iters` times, weights rotated over n_copies device copies;
 * out[0] = us per call, out[1] = weight bytes per call. */
int draco_bench_shexp(const float* x, const uint64_t* shp, const int* shc, int shi, int h, int n_copies,
                      int iters, float* out);

/* ---- state sync hooks (no reference counterpart: the reference's KV state
 * is the host arrays themselves, src/draco_engine_server.py:907-922) ------ */

/* device KV mirrors -> caller's kcache/vcache (rows [0, tlen)) */
int draco_state_pull(const void* layers, int n_layer);
/* caller's kcache/vcache (rows [0, tlen)) -> device KV mirrors */
int draco_state_push(const void* layers, int n_layer);

/* ---- device-resident greedy loop (no reference counterpart: the
 * reference's loop is Python, src/smol_engine.py:203-213) ----------------
 * Feeds prompt[0..n_prompt) from the current tlen, then generates n_gen
 * tokens by argmax (first index on ties), all on the device.
 * prompt[0..n_prompt-1) goes through the chunked prefill below (token-serial
 * decode steps when the chunk size is 0); the last prompt token goes through
 * the first decode step.  With use_graph the token-serial prefill step and
 * the decode step are captured as HIP graphs and replayed.
 * out_hidden[h] = x after the last forward (nullable); stats[0] = decode ms,
 * stats[1] = prefill ms of the n_prompt - 1 tokens (nullable). */
int draco_llama_generate(const void* layers, int n_layer, int h, float eps,
                         const float* final_norm, const uint8_t* head_w, int head_code, int vocab,
                         const uint8_t* emb_w, int emb_code, const int* prompt, int n_prompt,
                         int n_gen, int use_graph, int* out_tokens, float* out_hidden,
                         float* stats);

/* ---- chunked prefill of the llama family: the reference's forward_chunk
 * contract (src/qwen35_prefill.py:209-210, src/draco_engine_server.py:836-842:
 * afterwards the engine state is that of forward(ids[i], pos + i) run token
 * by token), which the reference implements for qwen35 only ----------------
 * ids[0..n) at positions pos .. pos + n - 1, in chunks of the chunk size:
 * per layer one RMSNorm, the q/k/v, o, gate/up and down products as f16-MFMA
 * GEMMs over the chunk's tokens (exact f16 operands, fp32 accumulation), rope + KV append at rows tlen .. tlen + n - 1
 * (device mirrors) and causal attention; every tlen advances by n.
 * out_x[h] (host, nullable) = hidden state of the last token after the last
 * layer (the x m6_forward_token leaves).  0 = ok. */
int draco_llama_prefill(const void* layers, int n_layer, int h, float eps, const uint8_t* emb_w, int emb_code,
                        int vocab, const int* ids, int n, int pos, float* out_x);
/* tokens per prefill chunk (default 256; 0 = draco_llama_generate feeds its
 * prompt token by token).  Returns the previous value; n < 0 only queries. */
int draco_set_prefill_chunk(int n);
/* No reference counterpart: the llama decode layers' attention split merge
 * fused with the o projection (1, the default, where the shape allows: head
 * dim 64, 32 q heads, K-quant o and gate/up) or run as two launches (0).
 * Returns the previous setting; on < 0 only queries. */
int draco_set_attn_o_fusion(int on);
/* No reference counterpart: MoE decode layers followed by a K-quant layer
 * leave their expert down launch's two half sums pending for the next
 * layer's q/k/v launch to add (1, the default) or add them with the residual
 * themselves (0).  Returns the previous setting; on < 0 only queries. */
int draco_set_moe_split(int on);
/* No reference counterpart: with the attention merge fused (above), Q8_0
 * llama layers whose caches stay within 128 rows during a call run the whole
 * attention inside the o projection's launch (1, the default) instead of a
 * split attention launch before it (0).  Returns the previous setting; on < 0
 * only queries. */
int draco_set_attn_short(int on);
/* No reference counterpart: waves per block of the group-shared decode
 * attention kernel (head dims 128 / 256): 4, 8 (the default) or 16; other
 * values only query.  Returns the previous setting. */
int draco_set_gqa_waves(int n);
/* No reference counterpart: blocks per CU of the persistent Q8_0 GEMV that
 * serves single-matrix launches of at least 16384 rows (the vocabulary
 * head; 2, the default), or 0 for the 8-rows-per-block kernel.  Values
 * outside 0..8 only query.  Returns the previous setting. */
int draco_set_seg_rows(int n);
/* No reference counterpart: the GDN decode step at 8 blocks per V head with
 * the gates' dots from the in-projection runs the barrier-free kernel in
 * blocks of 1 or 2 (the default) waves, or (0) the split scan kernel's decode
 * form.  Other values only query.  Returns the previous setting. */
int draco_set_gdn_dec(int waves);

/* ---- library utilities (no reference counterpart) ----------------------- */

const char* draco_last_error(void);
const char* draco_version(void);
/* Drop the device copy / mirror registered for a host buffer; returns count. */
int draco_forget(const void* host);
/* Drop every device copy and mirror. */
void draco_reset(void);
size_t draco_resident_bytes(void);

/* ---- MoE ----------------------------------------------------------------
 * m6_granite_moe: src/m6_layer.c:771-802 -- router (fp32 gate_inp
 * [n_exp][n_in]) -> softmax -> stable top-n_used -> renormalised weights ->
 * per expert silu(gate.x)*(up.x) -> down -> weighted sum into out[n_out].
 * ptrs/codes: 3 per expert (gate, up, down), host pointers.  Served: Q4_K /
 * Q6_K experts, n_exp <= 512, n_used <= 64, inter and n_in multiples of 256,
 * n_out a multiple of 16.  `scratch` is not used (the reference's host scratch
 * is not needed by the device path).  Errors are printed (void, as the
 * reference). */
void m6_granite_moe(const float* x0, const uint64_t* ptrs, const int* codes, const float* gate_inp, int n_exp,
                    int n_used, int inter, int n_in, int n_out, float* scratch, float* out);
/* m6_moe_tok: src/m6_moe_tok.c:44-161 -- token-batched MoE FFN for prefill:
 * out[T][n_out] = sum over k (ascending) of wtop[t*n_used+k] * expert
 * order[t*n_used+k] applied to X[t] (gate/up -> silu*up -> down).  ep/ec: 3
 * host pointers / codes per expert.  Served: Q4_K / Q6_K experts (one format
 * per role across experts), inter and n_in multiples of 256, n_out a
 * multiple of 16.  DQ, GA, gwbuf, work and iwork are accepted and not used
 * (the device path runs its own grouped GEMMs).  Unserved input (e.g. IQ3_S
 * experts) is reported on stderr and leaves NaN in out (void, as the
 * reference; m6_granite_moe does the same). */
void m6_moe_tok(int (*DQ)(int, const uint8_t*, int, float*),
                int (*GA)(int, const float*, const uint8_t*, int, int, int, float*), float* gwbuf, const float* X,
                const int* order, const float* wtop, const uint64_t* ep, const int* ec, int T, int n_used, int inter,
                int n_in, int n_out, int n_exp, float* out, float* work, int* iwork);
/* m5_gemvn_q4k / m5_gemvn_q6k: src/m5/m5_batch8_k.c:80-183.  y[e * n_out_e + r]
 * = (W + idx[e] * per)[r] . (x + e * x_stride) for e < n_exp.  Returns -1 for
 * n_in % 256 != 0 (as the reference) or n_out_e % 16 != 0. */
int m5_gemvn_q4k(const float* x, long x_stride, const uint8_t* W, const int* idx, long per, int n_out_e,
                 int n_in, int n_exp, float* y);
/* m6_moe_batch4: src/m6_layer.c:656-690 (bound at import by the reference's
 * llama driver, src/smol_engine.py:81) -- n_exp given experts, no router:
 * out[n_out] = sum over j (ascending) of wtop[j] * down_j(silu(gate_j x0) *
 * (up_j x0)), the weights as given.  ptrs/codes: 3 per expert (host).
 * Served: Q4_K / Q6_K (one format per role), n_exp <= 64, inter and n_in
 * multiples of 256, n_out a multiple of 16; anything else prints the error
 * and leaves NaN in out (void, as the reference).  scratch is not used. */
void m6_moe_batch4(const float* x0, const uint64_t* ptrs, const int* codes, const float* wtop, int n_exp, int inter,
                   int n_in, int n_out, float* scratch, float* out);
int m5_gemvn_q6k(const float* x, long x_stride, const uint8_t* W, const int* idx, long per, int n_out_e,
                 int n_in, int n_exp, float* y);
/* The MoE FFN as an m6 ffn op (no reference counterpart as an op: the
 * reference's qwen35 driver calls m6_granite_moe per layer from Python,
 * src/qwen35_engine.py:293-307): the arguments of m6_granite_moe in one
 * struct.  In an M6LayerDesc it lets m6_forward_token and
 * draco_llama_generate run MoE layers on the device (the configs[3] stack);
 * called directly it is m6_granite_moe(xn, ...) into out[n_out].  scratch
 * is the reference op's host scratch (3*n_used*inter + n_used*n_out floats;
 * not used by the device path). */
typedef struct {
    const uint64_t* ptrs;   /* [3 * n_exp] gate, up, down per expert */
    const int* codes;       /* [3 * n_exp] */
    const float* gate_inp;  /* [n_exp][n_in] fp32 router */
    int n_exp, n_used, inter, n_in, n_out;
    float* scratch;
} DracoMoeP;
void draco_moe_ffn_op(const float* xn, void* p, float* out);
/* No reference counterpart: out[0] us per MoE FFN (router + routed gate/up +
 * down/combine) from a graph replay of `iters` FFNs, out[1] bytes per FFN. */
int draco_bench_granite_moe(const float* x0, const uint64_t* ptrs, const int* codes, const float* gate_inp,
                            int n_exp, int n_used, int inter, int n_in, int n_out, int iters, float* out);

/* ---- Prefill GEMM: Y[T x n_out] = X[T x n_in] . W^T ----------------------
 * m5_gemm_auto: src/m5/m5_gemm_fused.c:231-241 (0 done, -1 code not served:
 * the caller falls back).  m5_gemm: src/m5/m5_gemm.c:249-272.  Host pointers.
 * Served: Q4_K and Q6_K on f16 MFMA (exact operands), Q8_0 and Q5_K as
 * per-token device GEMVs.
 * `wbuf` is not used. */
int m5_gemm_auto(int code, const float* X, const uint8_t* W, int c, int n_out, int n_in, float* Y);
int m5_gemm(int code, const float* X, const uint8_t* W, int T, int n_out, int n_in, float* Y, float* wbuf);
/* The per-format fused GEMMs of src/m5/m5_gemm_fused.c:78,211-228 (the
 * FUSED3 instances and m5_gemm_iq3s), which the reference's prefill driver
 * looks up by name (src/qwen35_prefill.py:76-80) and calls per format
 * (:100-104): Y[c x n_out] = X[c x n_in] . W^T, as m5_gemm_auto for their
 * code.  void, as the reference's: IQ4_XS and IQ3_S (not carried here) and
 * failures print the error and leave NaN in Y. */
void m5_gemm_q80(const float* X, const uint8_t* W, int c, int n_out, int n_in, float* Y);
void m5_gemm_q6k(const float* X, const uint8_t* W, int c, int n_out, int n_in, float* Y);
void m5_gemm_q5k(const float* X, const uint8_t* W, int c, int n_out, int n_in, float* Y);
void m5_gemm_q4k(const float* X, const uint8_t* W, int c, int n_out, int n_in, float* Y);
void m5_gemm_iq4xs(const float* X, const uint8_t* W, int c, int n_out, int n_in, float* Y);
void m5_gemm_iq3s(const float* X, const uint8_t* W, int c, int n_out, int n_in, float* Y);
/* m5_dequant_row: src/m5/m5_gemm.c:55-235 -- one GGUF row (host) ->
 * out[n_in] fp32, decoded on the device (from the resident copy when the row
 * lies inside a registered matrix).  0 done, -1 code not served: served are
 * Q8_0, Q4_K, Q5_K, Q6_K and F16 (the reference also decodes the IQ
 * formats). */
int m5_dequant_row(int code, const uint8_t* row, int n_in, float* out);
/* No reference counterpart: out[0] us per GEMM including the activation
 * digitization, out[1] us for the GEMM kernel alone (graph replays over
 * n_copies weight copies). */
int draco_bench_gemm(int code, const uint8_t* W, int n_out, int n_in, int T, int n_copies, int iters, float* out);

/* ---- Gated-DeltaNet scan ---------------------------------------------------
 * m6_gdn_scan: src/m6_gdn_scan.c:18-93.  QKV[T*n_qkv] (q heads, k heads, v
 * heads, 128 wide), Z[T*n_vh*128], B (beta) and G (= exp(alpha)) [T*n_vh],
 * conv[n_qkv*4], ssm_norm[128]; tail[n_qkv*3] and S[n_vh*128*128] are updated
 * in place; ON[T*n_vh*128].  Host pointers; `work` is not used. */
void m6_gdn_scan(const float* QKV, const float* Z, const float* B, const float* G, const float* conv,
                 const float* ssm_norm, float* tail, float* S, int T, int n_qkv, int n_vh, float* ON,
                 float* work);
/* No reference counterpart: device-resident timing with the same inputs (the
 * caller's S and tail are not modified).  out[0] us per token scanning T tokens
 * in launches of `chunk` tokens, out[1] us per single-token launch (n_dec
 * steps). */
int draco_bench_gdn_scan(const float* QKV, const float* Z, const float* B, const float* G, const float* conv,
                         const float* ssm_norm, const float* tail, const float* S, int T, int n_qkv, int n_vh,
                         int chunk, int n_dec, float* out);

/* ---- qwen35 hybrid layers (decode, one token) ----------------------------
 * Descriptors field for field src/m6_layer.c:189-202 (GdnW) and :375-387
 * (FullW); ctypes twins src/qwen35_engine.py:137-157.  Hidden width 2048,
 * 16 GDN q/k heads, head dims 128 (GDN) / 256 (full attention) and 2 KV heads
 * are fixed, as in the reference.  Host pointers; the caller's state arrays
 * (ssm, tail) are updated in place and Kr / Vc are read, as there.  Served
 * projection formats: Q4_K, Q6_K, Q8_0 (fused launches) and F16 / F32.
 * `buf` and `scores` are the reference's host scratch and are not used.
 * Errors are printed (void, as the reference). */
typedef struct {
    const float* attn_norm;
    const uint8_t* qkv_buf; int qkv_code;
    const uint8_t* gate_buf; int gate_code;
    const float* beta_wt;   /* [2048][n_vh] */
    const float* alpha_wt;  /* [2048][n_vh] */
    const float* ssm_a;
    const float* ssm_dt;
    const float* conv;      /* [n_qkv][4] */
    const float* ssm_norm;  /* [128] */
    const uint8_t* ssm_out_buf; int ssm_out_code;
    const float* post_norm;
    int n_qkv; int n_vh; int d_in;
} GdnW;

typedef struct {
    const float* attn_norm;
    const uint8_t* q_buf; int q_code;   /* nh*512 rows: per head q[256] | gate[256] */
    const uint8_t* k_buf; int k_code;   /* 512 rows */
    const uint8_t* v_buf; int v_code;   /* 512 rows */
    const float* q_norm;                /* [256] */
    const float* k_norm;                /* [256] */
    const uint8_t* o_buf; int o_code;   /* 2048 rows, nh*256 wide */
    const float* post_norm;
    const float* rope_inv;              /* [32] */
    int nh;                             /* even, <= 32 */
} FullW;

/* m6_gdn_attn: src/m6_layer.c:205-364.  h1[2048] -> x2n, x2_out; the state
 * ssm [n_vh][128][128] and tail [n_qkv][3] advances in device mirrors keyed by
 * the arrays' addresses (loaded from them when first seen).  Each call writes
 * the first 128 state floats back into ssm; when the caller's ssm no longer
 * holds them bit for bit at the next call (a reset that zeroed the arrays, a
 * restored snapshot), both arrays are loaded again.  draco_array_pull copies
 * the state back in full. */
void m6_gdn_attn(const float* h1, const GdnW* w, float* ssm, float* tail, float* buf, float* x2n,
                 float* x2_out);
/* m6_full_attn: src/m6_layer.c:389-518.  Kr / Vc: Told cached rows of
 * [2][256]; kr_new / v_new receive the new row (k normed + roped), which the
 * caller appends at row Told as the reference's driver does.  The rows live
 * in device mirrors keyed by Kr / Vc: rows the device has not held are
 * uploaded, and up to 17 held rows are compared with the caller's (first
 * float of each) per call, a mismatch reloading rows [0, Told). */
void m6_full_attn(const float* h1, const FullW* w, const float* Kr, const float* Vc, int Told, int pos0,
                  float* buf, float* scores, float* x2n, float* x2_out, float* kr_new, float* v_new);
/* No reference counterpart: device-resident timing of one op (kind 0 GDN with
 * w a GdnW*, state from ssm_or_kr / tail_or_vc; kind 1 full attention with w a
 * FullW*, told cached rows from ssm_or_kr / tail_or_vc).  Host arrays are not
 * modified.  out[0] us per op (graph replay of `iters` ops), out[1] weight
 * bytes per op, out[2] algorithmic HBM bytes per op. */
int draco_bench_qwen_op(int kind, const void* w, const float* h1, const float* ssm_or_kr, const float* tail_or_vc,
                        int told, int iters, float* out);
/* No reference counterpart (the reference's state arrays are host memory):
 * a state array's device mirror -> its first `bytes` (pull), and the caller's
 * array -> the mirror (push, e.g. after restoring a snapshot into it). */
int draco_array_pull(void* host, size_t bytes);
int draco_array_push(const void* host, size_t bytes);

/* ---- the qwen35 hybrid stack on the device --------------------------------
 * No reference counterpart as one call: the reference's driver composes the
 * per-layer ops in Python (src/qwen35_engine.py:310-327 per token,
 * src/qwen35_prefill.py:209-239 per chunk).  One DracoQwenLayer per layer:
 * the layer op (kind 0 m6_gdn_attn with a GdnW, kind 1 m6_full_attn with a
 * FullW), its state arrays (GDN: ssm [n_vh][128][128] and tail [n_qkv][3];
 * full attention: Kr and Vc [max_t][2][256]) and the FFN of x2n added to
 * x2_out (ffn_kind 0 none, 1 dense with an M6DenseP, 2 MoE with a
 * DracoMoeP).  Token t of a sequence sits at position pos0 + t and writes
 * cache row pos0 + t (Told = pos, as the reference passes them).  The state
 * lives on the device (mirrors keyed by the state arrays' addresses, loaded
 * from them when first seen); draco_qwen_state_pull / push move it to and
 * from the caller's arrays (snapshot, or after zeroing them for a reset). */
typedef struct {
    int kind;            /* 0 GDN, 1 full attention */
    const void* w;       /* const GdnW* / const FullW* */
    float* state0;       /* GDN ssm / full-attention Kr */
    float* state1;       /* GDN tail / full-attention Vc */
    int max_t;           /* full attention: rows of Kr / Vc */
    int ffn_kind;        /* 0 none, 1 dense, 2 MoE */
    const void* ffn;     /* const M6DenseP* / const DracoMoeP* */
} DracoQwenLayer;

/* One token: x[2048] (host, in / out) through every layer at position pos. */
int draco_qwen_forward(float* x, int h, int pos, const void* layers, int n_layer);
/* forward_chunk: ids[0..n) at positions pos0 .. pos0 + n - 1 in chunks
 * (draco_set_qwen_chunk, default 64): projections as f16-MFMA GEMMs over the
 * chunk, the GDN scan token-serial, causal gated attention over the cache;
 * out_x[2048] (host, nullable) = the last token's hidden row.  Layers with a
 * MoE FFN are not served here (-1; draco_qwen_generate feeds them token by
 * token). */
int draco_qwen_prefill(const void* layers, int n_layer, int h, const uint8_t* emb_w, int emb_code, int vocab,
                       const int* ids, int n, int pos0, float* out_x);
int draco_set_qwen_chunk(int n);
/* No reference counterpart: blocks per V head of the GDN scan (1, 2, 4 or 8;
 * negative keeps a setting) for the decode step of the layer ops and stacks
 * and for multi-token scans (defaults 8 and 8).  Split above 1, each head's
 * 128 state columns spread over that many workgroups and the gated rms runs
 * after them: in the ssm_out GEMV's prologue for decode steps with a Q4_K /
 * Q6_K ssm_out (other formats keep one workgroup per head), as a second
 * launch for scans.  A single-token m6_gdn_scan runs unsplit.
 * Returns the previous values as decode * 16 + scan. */
int draco_set_gdn_split(int decode_split, int scan_split);
/* Greedy generation from position pos0 (prompt through the chunked prefill
 * except its last token, then n_gen argmax tokens; graph-replayed steps with
 * use_graph); the head is RMSNorm(final_norm, eps) + head_w, as m6_head_op.
 * stats[0] = decode ms, stats[1] = prompt ms (nullable). */
int draco_qwen_generate(const void* layers, int n_layer, int h, float eps, const float* final_norm,
                        const uint8_t* head_w, int head_code, int vocab, const uint8_t* emb_w, int emb_code, int pos0,
                        const int* prompt, int n_prompt, int n_gen, int use_graph, int* out_tokens, float* out_hidden,
                        float* stats);
/* device state -> caller's arrays (GDN in full; Kr / Vc rows [0, rows)) */
int draco_qwen_state_pull(const void* layers, int n_layer, int rows);
/* caller's arrays -> device state */
int draco_qwen_state_push(const void* layers, int n_layer, int rows);

/* ---- Q8_K activations and the Q4_K / Q6_K x Q8_K GEMV --------------------
 * No reference counterpart: the reference has no Q8_K path (nearest analogue:
 * the Q8_0 x Q8_0 int8 dot of tests/i8dot_bench.c:63-183).  Block format
 * {float d; int8 qs[256]; int16 bsums[16]} (292 bytes) and rounding of
 * llama.cpp b10819 quantize_row_q8_K_ref.  Host pointers; weights are
 * registered and kept resident like m5_gemv's.  0 ok, -1 unsupported, -2
 * device error. */
/* out: nvec * (n/256) blocks, vector-major. */
int draco_q8k_quantize(const float* x, int n, int nvec, uint8_t* out);
/* y[v * n_out + r] for v < nvec, nvec in {1, 4, 8}; xq as above. */
int draco_gemv_q8k(int code, const uint8_t* xq, int nvec, const uint8_t* W, int n_out, int n_in, float* y);
/* x fp32 (nvec vectors of n_in), quantized to Q8_K on the device (one vector
 * of rows up to 4096 wide: inside the GEMV launch, with the quantizer's
 * operations; otherwise a quantizer launch first). */
int draco_gemv_q8k_f32(int code, const float* x, int nvec, const uint8_t* W, int n_out, int n_in, float* y);
/* Integer super-block sums of one vector: isc[r * nb + b], imn[r * nb + b]. */
int draco_q8k_isums(int code, const uint8_t* xq, const uint8_t* W, int n_out, int n_in, int32_t* isc,
                    int32_t* imn);
/* No reference counterpart.  For callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): draco_gemv_q8k_f32 with DEVICE pointers and no allocation.
 * x [nvec][n_in] fp32, W the weights already in this library's device layout
 * (draco_repack of the GGUF rows; draco_layout_query bytes), y [nvec][n_out]
 * fp32.  The Q8_K values of x are staged in a static device array of
 * draco_noalloc_capacity() bytes (1 MiB: nvec * n_in / 256 * 292 + 16 bytes
 * at most; larger requests return -1, as do rows whose Q8_K image does not
 * fit the GEMV's 160 KiB of LDS -- n_in above 16896 at nvec 8 -- both before
 * anything is enqueued).  Enqueued on `stream` (a hipStream_t;
 * NULL = the library's stream) and not waited for.  Every call on one GPU
 * shares that GPU's staging array: calls that overlap on one GPU race. */
int draco_gemv_q8k_f32_noalloc(int code, const float* x, int nvec, const uint8_t* W, int n_out, int n_in, float* y,
                               void* stream);
size_t draco_noalloc_capacity(void);
/* out[0] us per Q8_K GEMV launch, out[1] us per (quantize + GEMV) pair,
 * out[2] (nvec 1, rows up to 4096 wide; else 0) us per GEMV launch that
 * quantizes fp32 x itself (what draco_gemv_q8k_f32 runs for one vector of
 * such rows), all from a graph replay of `iters`
 * launches over n_copies weight copies.  out holds 3 floats. */
int draco_bench_gemv_q8k(int code, const uint8_t* W, int n_out, int n_in, int nvec, int n_copies, int iters,
                         float* out);

/* Device timing probes (weights rotated over n_copies device copies so the
 * working set can exceed the 256 MB MALL).  out[0] mean us per launch from
 * per-launch event pairs, out[1] us per launch over the whole loop, out[2]
 * min, out[3] median, out[4] us per launch from a graph replay of the same
 * launches (out holds at least 5 floats). */
int draco_bench_gemv(int code, const uint8_t* W, int n_out, int n_in, int n_copies, int iters,
                     float* out);
/* out[0] us per empty-kernel launch in a stream, out[1] in a replayed graph. */
int draco_bench_launch(int iters, float* out);

/* Launch planning of the Q4_K / Q6_K segment GEMV (no reference counterpart;
 * pure host logic, callable without a GPU, for tests): the shape the library
 * would launch for rows n_in wide in `tiles` 16-row tiles -- dual = SwiGLU
 * pair, ksplit 2 = split-K, do_norm = prologue kind (0 none, 1 RMSNorm, 2 GDN
 * gated rms, 3 RMSNorm of a pending residual), gd_n = row dots requested, cus
 * = compute units.  out[6] = {waves per block, grid, one item per wave,
 * split-K, row dots, float4s of x per thread in the prologue}.  Returns 0, or
 * -1 when no instance covers the request. */
int draco_dq_plan(int n_in, int tiles, int dual, int ksplit, int do_norm, int gd_n, int cus, int* out);

/* Host-side byte work (pure CPU, callable without a GPU). */
int draco_quantize(int code, const float* x, int n_rows, int n_in, uint8_t* out);
size_t draco_layout_query(int code, int n_out, int n_in, size_t* off4);
int draco_repack(int code, const uint8_t* src, int n_out, int n_in, uint8_t* dst);
int draco_unpack(int code, const uint8_t* src, int n_out, int n_in, uint8_t* dst);
void draco_rope_table(int max_t, int rot, float base, float* tab);
float draco_f16_to_f32(uint16_t h);
uint16_t draco_f32_to_f16(float f);

#ifdef __cplusplus
}
#endif
#endif /* DRACO_HIP_H */
