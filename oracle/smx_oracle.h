/*
 * smx_oracle.h -- CPU restatement of SmallMind's quantized transformer forward path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP path in
 * smallmind_amd/.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and only as the checker or the timed CPU baseline -- never as a product fallback.
 *
 * Every function restates a reference routine (C#, /root/reference, cited file:line).  Built
 * with gcc -O2 -ffp-contract=off so that no a*b+c is fused unless written as fmaf().
 *
 * Parity status per function (what pins it) is recorded in the header comment of
 * smx_oracle.c.
 */
#ifndef SMX_ORACLE_H
#define SMX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type ids (GgufTensorType.cs:6-52). */
enum {
    SMXO_F32 = 0, SMXO_F16 = 1, SMXO_Q4_0 = 2, SMXO_Q8_0 = 8,
    SMXO_Q4_K = 12, SMXO_Q5_K = 13, SMXO_Q6_K = 14,
    /* SMQ Q8Tensor / Q4Tensor blocks re-laid per 32 elements: fp32 scale + codes */
    SMXO_SMQ_Q8 = 1010, SMXO_SMQ_Q4 = 1011
};

/* ---- block formats ------------------------------------------------------------------ */
int     smxo_block_elems(int type);          /* elements per block, 0 if unknown         */
int     smxo_block_bytes(int type);          /* bytes per block, 0 if unknown            */
float   smxo_half_to_float(uint16_t h);      /* GgufModelLoader.cs:919-956               */
uint16_t smxo_float_to_half(float f);        /* IEEE binary16, round-to-nearest-even     */

/* Dequantize n elements of GGUF-layout blocks (GgufModelLoader.cs:419-917). 0 = ok. */
int smxo_dequant(int type, const uint8_t *src, int64_t n, float *dst);

/* Quantize n elements into GGUF-layout blocks.  Q8_0 / Q4_0 follow Q8Tensor.Quantize /
 * Q4Tensor.Quantize (Q8Tensor.cs:72-128, Q4Tensor.cs:75-134) at block 32 with an fp16
 * scale; the K-quant encoders are this build's own (the reference has none) and emit bytes
 * in exactly the layout the reference decoder reads.  0 = ok. */
int smxo_quantize(int type, const float *src, int64_t n, uint8_t *dst);

/* The reference's own SMQ-style quantizers (block b, fp32 scales). */
void smxo_quantize_ref_q8(const float *src, int n, int block, int8_t *q, float *scales);
void smxo_quantize_ref_q4(const float *src, int n, int block, uint8_t *data, float *scales);
int  smxo_decode_nibble(int nibble);        /* Q4Tensor.cs:140-143 */
/* Q8Tensor.Dequantize (scheme 10) / Q4Tensor.Dequantize (scheme 11) of a flattened SMQ tensor:
 * n elements, one fp32 scale per `block` consecutive elements.  0 = ok. */
int  smxo_dequant_smq(int scheme, const uint8_t *data, const float *scales, int64_t n, int block,
                      float *dst);

/* y[n] = sum_k dequant(W)[n][k] * x[k], accumulated in double. W is [N][K] GGUF rows. */
int smxo_gemv_f64(int type, const uint8_t *W, int N, int K, const float *x, double *y);

/* ---- elementwise / norm ops --------------------------------------------------------- */
void  smxo_rmsnorm(const float *x, const float *g, float *y, int rows, int n, float eps);
void  smxo_layernorm(const float *x, const float *g, const float *b, float *y, int rows, int n,
                     float eps);
void  smxo_rope_tables(int max_pos, int head_dim, float theta, float *cos_t, float *sin_t);
void  smxo_rope_apply(float *data, int pos0, int n_heads, int seq, int head_dim,
                      const float *cos_t, const float *sin_t);
float smxo_fastexp(float x);
void  smxo_scale_mask_softmax(float *scores, float scale, int seq, int k_seq, int cache_off);
void  smxo_gelu(const float *x, float *y, int n);
void  smxo_silu_mul(const float *g, const float *u, float *y, int n);

/* ---- model -------------------------------------------------------------------------- */
typedef struct smxo_model smxo_model;
typedef struct smxo_session smxo_session;

enum { SMXO_ARCH_LLAMA = 0, SMXO_ARCH_GPT2 = 1 };

smxo_model *smxo_model_create(int arch, int vocab, int ctx, int d, int n_layer, int n_head,
                              int n_kv_head, int ff, float rope_theta, float norm_eps);
/* Tensor by GGUF name; weights are dequantized to fp32 at load as GgufModelLoader does. */
int  smxo_model_set_tensor(smxo_model *m, const char *name, int type, const uint8_t *bytes,
                           int64_t n_elems);
int  smxo_model_finalize(smxo_model *m);
void smxo_model_destroy(smxo_model *m);

/* TransformerModel.Forward(idx[1,T], 0) without a KV cache; writes logits of every row
 * when all_rows != 0 ([T][V]) else of the last row only ([V]). */
int smxo_forward_nocache(smxo_model *m, const int32_t *tokens, int T, float *logits,
                         int all_rows);

/* KV-cached single-token step at position pos (cache written correctly). */
smxo_session *smxo_session_create(smxo_model *m, int max_ctx);
int  smxo_session_step(smxo_session *s, int32_t token, int pos, float *logits);
/* T tokens at positions pos0..pos0+T-1 in one pass (batched linears); bit-identical to T
 * smxo_session_step calls in order.  logits_last (may be NULL): the last token's logits. */
int  smxo_session_prefill(smxo_session *s, const int32_t *tokens, int T, int pos0, float *logits_last);
/* One token for each of n distinct sessions of one model (token i at pos[i] of ss[i]) in one
 * pass; logits [n][V] (may be NULL).  Bit-identical to n smxo_session_step calls. */
int  smxo_multi_step(smxo_session *const *ss, const int32_t *tokens, const int *pos, int n, float *logits);
/* Tokens of any sessions of one model in one pass: token i at pos[i] of ss[i] attends to
 * positions 0..pos[i] of its session, each of which this call or an earlier one writes (several
 * prompts prefilled together).  logits: rows lg_from..n-1 ([n - lg_from][V]) or NULL. */
int  smxo_step_tokens(smxo_session *const *ss, const int32_t *tokens, const int *pos, int n, float *logits,
                      int lg_from);
void smxo_session_destroy(smxo_session *s);

/* Threads used by the linears and attention (0 = all; results do not depend on it). */
void smxo_set_threads(int n);
int  smxo_get_threads(void);

/* Greedy decode with the cached step: prefill n_prompt tokens, then generate n_new tokens
 * (argmax, lowest index on ties).  Writes out_tokens[n_new]; returns elapsed ns of the
 * steps that produced a token in *decode_ns and of the rest in *prefill_ns. */
int smxo_generate_greedy(smxo_model *m, const int32_t *prompt, int n_prompt, int n_new,
                         int32_t *out_tokens, int64_t *prefill_ns, int64_t *decode_ns);

int smxo_argmax(const float *v, int n);
/* Next-token sampling (InferenceSession.cs:565-606); returns the id drawn at u. */
int smxo_sample(const float *logits, int n, const int32_t *ctx, int n_ctx, float temperature, int top_k,
                double top_p, double min_p, float rep, float presence, float frequency, int window, double u,
                float *probs_out);

/* Deterministic N(0, std) fill (splitmix64 + Box-Muller), the oracle twin of smx_fill_normal. */
void smxo_fill_normal(uint64_t seed, int64_t n, float std, float *out);

#ifdef __cplusplus
}
#endif
#endif
