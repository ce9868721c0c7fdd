/*
 * smx.h -- C-ABI of libsmx.so, the MI355X (gfx950) backend for SmallMind's quantized
 * transformer forward path.
 *
 * Plain C types only.  Every entry point returns an int status (0 = SMX_OK, < 0 = error);
 * smx_last_error() returns a thread-local message for the last failing call on the calling
 * thread.  Pointers named *_dev are HIP device pointers; `stream` is a hipStream_t (NULL =
 * the library context's stream for model/session calls, the null stream for operator calls).
 *
 * Reference interfaces each group replaces (paths relative to the SmallMind repository):
 *   operator level  IWeightTensor            src/SmallMind.Quantization/Abstractions/IWeightTensor.cs:7-42
 *   dequantization  GgufModelLoader.Convert* src/SmallMind.Runtime/GgufModelLoader.cs:419-956
 *   quantization    Q8Tensor/Q4Tensor.Quantize src/SmallMind.Quantization/Tensors/Q8Tensor.cs:72-128,
 *                                            Q4Tensor.cs:75-134
 *   model level     TransformerModel.Forward src/SmallMind.Transformers/Core/TransformerModel.cs:272-344
 *                   + Enable/Reset/DisableKVCache (:476-506)
 *   session level   InferenceSession.GenerateNextTokenAsync src/SmallMind.Runtime/InferenceSession.cs:478-607
 */
#ifndef SMX_H
#define SMX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SMX_API __attribute__((visibility("default")))

enum smx_status {
    SMX_OK = 0,
    SMX_EINVAL = -1,        /* bad argument / shape mismatch (ArgumentException in the reference) */
    SMX_ENOMEM = -2,        /* device allocation failed */
    SMX_EDEVICE = -3,       /* HIP runtime error */
    SMX_EBUSY = -4,         /* session already in use on another thread (InferenceSession.cs:127-144) */
    SMX_EUNSUPPORTED = -5,  /* tensor type or shape the backend does not implement */
    SMX_ESTATE = -6,        /* call out of order (e.g. model not finalized) */
    SMX_ERANGE = -7,        /* position / token out of range (TransformerModel.cs:282-285) */
    SMX_ECANCELED = -8,     /* generation stopped by smx_session_cancel (the OperationCanceledException of
                               InferenceSession's CancellationToken checks, InferenceSession.cs:211, :481) */
    SMX_ETIMEDOUT = -9      /* generation stopped at the session's time limit (InferenceTimeoutException,
                               InferenceSession.cs:164-172, :287-291) */
};

/* GGUF tensor type ids (src/SmallMind.Quantization/IO/Gguf/GgufTensorType.cs:6-52). */
enum smx_type {
    SMX_TYPE_F32 = 0,
    SMX_TYPE_F16 = 1,
    SMX_TYPE_Q4_0 = 2,
    SMX_TYPE_Q8_0 = 8,
    SMX_TYPE_Q4_K = 12,
    SMX_TYPE_Q5_K = 13,
    SMX_TYPE_Q6_K = 14,
    /* SmallMind's own SMQ blocks (Q8Tensor / Q4Tensor, src/SmallMind.Quantization/Tensors/Q8Tensor.cs,
     * Q4Tensor.cs): 1000 + the SMQ QuantScheme id (QuantScheme.cs: Q8_0 = 10, Q4_0 = 11).  As
     * upload bytes they are laid out in 32-element blocks, each the fp32 scale of the SMQ block
     * holding those elements followed by the codes (32 int8 / 16 bytes of two's-complement nibbles,
     * element 2i in the low nibble) -- see smx_smq_pack. */
    SMX_TYPE_SMQ_Q8 = 1010,
    SMX_TYPE_SMQ_Q4 = 1011
};

/* ---- library ----------------------------------------------------------------------------- */
SMX_API const char *smx_version(void);
SMX_API const char *smx_last_error(void);
/* Elements / bytes per GGUF block; 0 for unknown types. */
SMX_API int smx_type_block_elems(int type);
SMX_API int smx_type_block_bytes(int type);
/* GGUF bytes of one row of k elements (k must be a multiple of the block size), else -1. */
SMX_API int64_t smx_type_row_bytes(int type, int64_t k);

/* ---- dequantization / quantization (device pointers) ----------------------------------- */
/* Replaces GgufModelLoader.ReadAndDequantizeTensor -> Convert{Q8_0,Q4_0,Q4_K,Q5_K,Q6_K,F16,F32}
 * (GgufModelLoader.cs:419-917): n elements of GGUF-layout blocks -> fp32, bit-identical. */
SMX_API int smx_dequant(int type, const void *blocks_dev, int64_t n, float *out_dev, void *stream);
/* Replaces Q8Tensor.Quantize / Q4Tensor.Quantize (Q8Tensor.cs:72-128, Q4Tensor.cs:75-134),
 * emitting GGUF block layout (block 32, fp16 scale) for Q8_0/Q4_0, plus this build's K-quant
 * encoders for Q4_K/Q5_K/Q6_K.  n must be a multiple of the block size. */
SMX_API int smx_quantize(int type, const float *x_dev, int64_t n, void *blocks_dev, void *stream);
/* Seeded N(0, std) fill used to synthesise weights (counter-based, splitmix64 + Box-Muller).
 * Replaces the seeded weight initialisation of Tensor.InitializeXavier/Random (Tensor.cs:262-285). */
SMX_API int smx_fill_normal(uint64_t seed, int64_t n, float std, float *out_dev, void *stream);

/* ---- operator level: IWeightTensor ----------------------------------------------------- */
typedef struct smx_weight smx_weight;
/* Creates a device weight [rows][cols] (GGUF dims ne0 = cols) from GGUF-layout blocks.
 * The bytes are copied and repacked into the backend layout; the repack is lossless.
 * blocks_on_device != 0: blocks is a device pointer, else a host pointer.
 * Replaces the IWeightTensor implementations (Q8WeightTensor.cs, Q4KWeightTensor.cs, ...). */
SMX_API int smx_weight_create(int type, int64_t rows, int64_t cols, const void *blocks,
                              int blocks_on_device, smx_weight **out);
SMX_API int smx_weight_info(const smx_weight *w, int *type, int64_t *rows, int64_t *cols);
/* IWeightTensor.MatMul (IWeightTensor.cs:33) on device pointers, queued on `stream`:
 * out[m][n] = act[m][k] . W^T with k == cols and n == rows (the GGUF-loader semantics
 * y = x W^T).  Output fully overwritten.  SMX_EINVAL on dimension mismatch, as the reference
 * throws ArgumentException (Q8WeightTensor.cs:43-48).  From m >= 4 rows the matrix-core GEMM's
 * activation parts use device memory kept per weight (grown to the largest m seen; uses on
 * different streams are ordered), or a stream-ordered allocation under graph capture. */
SMX_API int smx_weight_matmul(const smx_weight *w, const float *act_dev, float *out_dev, int m,
                              int k, int n, void *stream);
/* IWeightTensor.MatMul with the reference's operands in host memory (IWeightTensor.cs:33,
 * ReadOnlySpan<float> activations, Span<float> output): act is m*k floats, out m*n floats, both
 * owned by the caller and borrowed for the call, which is synchronous.  Checks and results as
 * smx_weight_matmul.  The device staging is kept per weight and grows to the largest m seen, so
 * repeated calls allocate nothing; concurrent calls on one weight are serialised. */
SMX_API int smx_weight_matmul_host(const smx_weight *w, const float *act, float *out, int m, int k, int n);
/* IWeightTensor.ToFloat32 (IWeightTensor.cs:41) into caller-owned host memory of rows*cols floats
 * ([rows][cols], bit-identical to the reference dequantization); synchronous. */
SMX_API int smx_weight_to_float32_host(const smx_weight *w, float *out);
/* smx_weight_matmul without any device allocation: no counterpart in the reference.  For callers
 * that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same results as smx_weight_matmul.  From m >= 4 rows the activation parts go to a
 * fixed 16 MiB scratch array per GPU: calls needing more (ceil(m/16) * k/32 * 3072 bytes) return
 * SMX_EINVAL.  Every call on one GPU shares that array, so calls that overlap on one GPU (other
 * streams, other threads) race: the caller serialises them. */
SMX_API int smx_weight_matmul_noalloc(const smx_weight *w, const float *act_dev, float *out_dev, int m,
                                      int k, int n, void *stream);
/* IWeightTensor.ToFloat32 (IWeightTensor.cs:41): [rows][cols] fp32, bit-identical to the
 * reference dequantization of the original blocks. */
SMX_API int smx_weight_to_float32(const smx_weight *w, float *out_dev, void *stream);
SMX_API int smx_weight_destroy(smx_weight *w);

/* ---- elementwise / attention operators (device pointers) -------------------------------- */
/* RMSNormOps.RMSNorm (src/SmallMind.Core/Core/RMSNormOps.cs:28-219). */
SMX_API int smx_rmsnorm(const float *x_dev, const float *gamma_dev, float *y_dev, int rows, int n,
                        float eps, void *stream);
/* LayerNormOps.LayerNorm (src/SmallMind.Core/Core/LayerNormOps.cs:27-280). */
SMX_API int smx_layernorm(const float *x_dev, const float *gamma_dev, const float *beta_dev,
                          float *y_dev, int rows, int n, float eps, void *stream);
/* RotaryEmbedding.PrecomputeTables (src/SmallMind.Transformers/Core/RotaryEmbedding.cs:45-60),
 * host buffers [max_pos][head_dim/2]. */
SMX_API int smx_rope_tables(int max_pos, int head_dim, float theta, float *cos_host,
                            float *sin_host);
/* RotaryEmbedding.ApplyRotationInPlace (RotaryEmbedding.cs:85-121) on data [heads][seq][hd]
 * at positions pos0..pos0+seq-1; tables are device copies of smx_rope_tables output. */
SMX_API int smx_rope(float *data_dev, int n_heads, int seq, int head_dim, int pos0,
                     const float *cos_dev, const float *sin_dev, void *stream);
/* OptimizedOps.FusedScaleMaskSoftmax (src/SmallMind.Core/Optimized/OptimizedOps.cs:39-93),
 * in place on [seq][k_seq] with FastExp (src/SmallMind.Core/Utilities/MathUtils.cs:20-32). */
SMX_API int smx_scale_mask_softmax(float *scores_dev, float scale, int seq, int k_seq,
                                   int cache_offset, void *stream);
/* One decode position of MultiHeadAttention (MultiHeadAttention.cs:676-844): q [n_head][hd],
 * k_cache [n_kv_head][hd][ctx_stride] (dimension-major), v_cache [n_kv_head][ctx_stride][hd],
 * each holding n_pos positions, out [n_head][hd].  The scores use device memory kept per device
 * (grown to the largest request seen; uses on different streams are ordered). */
SMX_API int smx_attention_decode(const float *q_dev, const float *k_cache_dev,
                                 const float *v_cache_dev, float *out_dev, int n_head,
                                 int n_kv_head, int head_dim, int ctx_stride, int n_pos,
                                 void *stream);
/* Causal attention of n_tok consecutive query tokens at positions p_first .. p_first+n_tok-1
 * over the KV cache: MultiHeadAttention.Forward with T > 1 (MultiHeadAttention.cs:206-297;
 * scores :676-745, OptimizedOps.FusedScaleMaskSoftmax OptimizedOps.cs:39-93, W.V :810-845).
 * q [n_tok][n_head][hd], k_cache [n_kv_head][hd][ctx_stride], v_cache
 * [n_kv_head][ctx_stride][hd] holding positions 0 .. p_first+n_tok-1, out [n_tok][n_head][hd].
 * head_dim 64; n_head / n_kv_head must divide 32. */
SMX_API int smx_attention_prefill(const float *q_dev, const float *k_cache_dev,
                                  const float *v_cache_dev, float *out_dev, int n_head,
                                  int n_kv_head, int head_dim, int ctx_stride, int p_first,
                                  int n_tok, void *stream);
/* ActivationOps.FusedSiLUMul (src/SmallMind.Core/Simd/ActivationOps.cs:565-580). */
SMX_API int smx_silu_mul(const float *gate_dev, const float *up_dev, float *y_dev, int64_t n,
                         void *stream);
/* ActivationOps.GELU (ActivationOps.cs:217-296). */
SMX_API int smx_gelu(const float *x_dev, float *y_dev, int64_t n, void *stream);
/* Greedy next-token selection (replaces the T->0 limit of InferenceSession.cs:565-606):
 * index of the maximum, lowest index on ties. */
SMX_API int smx_argmax(const float *x_dev, int n, int32_t *out_dev, void *stream);
/* Measurement helper; it has no counterpart in the reference.  Reads `bytes` of device
 * memory (a multiple of 16, < 4 GiB) with 16-byte loads spread over the whole GPU and writes
 * nothing: the streaming-read ceiling a GEMV's bandwidth is compared with (bench.py). */
SMX_API int smx_stream_read(const void *src_dev, uint64_t bytes, void *stream);
/* Next-token sampling options (ProductionInferenceOptions.cs:19-87); each stage is skipped at
 * its neutral value. */
typedef struct smx_sampling {
    float temperature;          /* Temperature: logits * (1 / T); 1 = off */
    int32_t top_k;              /* TopK: keep logits >= the k-th largest; 0 = off */
    double top_p;               /* TopP (a double, as ProductionInferenceOptions.cs:31 and the
                                   float-sum >= double comparison of InferenceSession.cs:896 have it);
                                   >= 1 = off */
    float min_p;                /* MinP: drop p < max p * min_p; 0 = off */
    float repetition_penalty;   /* RepetitionPenalty: l > 0 ? l / r : l * r; 1 = off */
    float presence_penalty;     /* PresencePenalty: l - presence */
    float frequency_penalty;    /* FrequencyPenalty: l - count * frequency */
    int32_t repetition_window;  /* RepetitionWindow: recent tokens penalised; 0 = min(n, 256) */
} smx_sampling;
/* The reference's sampling pipeline on the device (InferenceSession.cs:565-606: penalties ->
 * temperature -> top-k -> softmax -> top-p -> min-p -> inverse-CDF draw, with the stages of
 * :628-936 and SampleFromProbs :708-724).  logits (n floats) and context (n_context token ids,
 * oldest first) are device memory; u in [0, 1) is the uniform draw the reference takes from
 * Random.NextDouble.  probs (n floats, device) receives the final distribution and token
 * (device) the sampled id.  Ties at the top-k / top-p cutoffs are all kept. */
SMX_API int smx_sample(const float *logits_dev, int n, const int32_t *context_dev, int n_context,
                       const smx_sampling *params, double u, float *probs_dev, int32_t *token_dev,
                       void *stream);

/* ---- model / session level --------------------------------------------------------------- */
typedef struct smx_context smx_context;
typedef struct smx_model smx_model;
typedef struct smx_session smx_session;

enum smx_arch { SMX_ARCH_LLAMA = 0, SMX_ARCH_GPT2 = 1 };

/* ModelConfig (src/SmallMind.Transformers/ModelConfig.cs:142-258).  llama: RoPE, RMSNorm,
 * SwiGLU, optional biases; gpt2: learned positions, LayerNorm, GELU MLP of 4*d, biases. */
typedef struct smx_model_config {
    int32_t arch;
    int32_t vocab;
    int32_t ctx;          /* ContextLength (block size) */
    int32_t d_model;
    int32_t n_layer;
    int32_t n_head;
    int32_t n_kv_head;
    int32_t d_ff;         /* FeedForwardLength (ignored for gpt2: 4*d_model) */
    float rope_theta;
    float norm_eps;
    int32_t reserved[6];  /* must be zero */
} smx_model_config;

typedef struct smx_gen_stats {
    double prefill_ms;    /* GPU time of the steps that only filled the KV cache */
    double decode_ms;     /* GPU time of the steps that produced a token */
    int32_t n_prefill_steps;
    int32_t n_decode_steps;
} smx_gen_stats;

SMX_API int smx_context_create(int device, smx_context **out);
SMX_API int smx_context_destroy(smx_context *ctx);

SMX_API int smx_model_create(smx_context *ctx, const smx_model_config *cfg, smx_model **out);
/* Uploads one GGUF tensor by its GGUF name (token_embd.weight, blk.N.attn_q.weight, ...).
 * dims are GGUF order (dims[0] = ne0 = fastest).  Q/K/V are merged into one fused matrix as
 * GgufModelLoader.MergeQKVWeights does (GgufModelLoader.cs:1027-1110); gate/up rows are
 * interleaved for the fused SwiGLU kernel.  bytes_on_device selects a device or host source. */
SMX_API int smx_model_upload_tensor(smx_model *m, const char *name, int type,
                                    const int64_t *dims, int ndims, const void *bytes,
                                    size_t nbytes, int bytes_on_device);
/* Validates the tensor set and ties output.weight to token_embd.weight when absent
 * (GgufModelLoader.HandleWeightTying, GgufModelLoader.cs:1126-1147). */
SMX_API int smx_model_finalize(smx_model *m);
/* Loads a GGUF v2/v3 file (GgufReader.ReadModelInfo, GgufReader.cs:39-102, through
 * GgufModelLoader, GgufModelLoader.cs:63-77): the configuration from its metadata as
 * ModelConfig.FromGgufMetadata derives it (ModelConfig.cs:142-214: llama, mistral*, phi*,
 * gpt2), then every tensor uploaded from a read-only memory map of the file and the model
 * finalized.  Tensor data is read at the data section + each tensor entry's offset (GGUF
 * specification).  SMX_EINVAL for a malformed or unreadable file, SMX_EUNSUPPORTED for other
 * architectures, versions or tensor types. */
SMX_API int smx_model_load_gguf(smx_context *ctx, const char *path, smx_model **out);
/* Parses a GGUF file's header, metadata and tensor table and returns the derived
 * configuration and the tensor count; no device work. */
SMX_API int smx_gguf_read_config(const char *path, smx_model_config *cfg, int64_t *n_tensors);
/* Loads a SmallMind .smq file (SmqModelLoader.LoadFromSmq, src/SmallMind.Runtime/SmqModelLoader.cs:
 * 29-100, reading through SmqReader, src/SmallMind.Quantization/IO/Smq/SmqReader.cs:33-293) into
 * SmallMind's GPT-2 style TransformerModel.  cfg (arch must be SMX_ARCH_GPT2) plays the role of the
 * reference's ModelConfig argument; NULL takes the configuration from the file's metadata
 * (vocab_size, block_size, embed_dim, num_layers, num_heads; d_ff = 4 * embed_dim).  Tensors are
 * matched by TransformerModel.GetNamedParameters names (TransformerModel.cs:545-728); a file
 * none of whose tensor names is a parameter name (the param_NNNN / tensor_NNN files of the
 * quantize command, QuantizeCommand.cs:63-97) is matched by parameter order.  Q8_0 / Q4_0 weight
 * matrices stay quantized on the device (SMX_TYPE_SMQ_Q8 / _Q4, the file's fp32 scales
 * unchanged); norm weights and biases are dequantized as SmqModelLoader.DequantizeTensor does
 * (SmqModelLoader.cs:320-360).  SMX_EINVAL for a malformed file, SMX_EUNSUPPORTED for F16
 * entries, other data types, or matrices whose columns or block size are not multiples of 32. */
SMX_API int smx_model_load_smq(smx_context *ctx, const char *path, const smx_model_config *cfg,
                               smx_model **out);
/* Parses an .smq file's header, metadata and tensor directory and returns the configuration its
 * metadata describes and the tensor count; no device work. */
SMX_API int smx_smq_read_config(const char *path, smx_model_config *cfg, int64_t *n_tensors);
/* Re-lays one rank-2 Q8Tensor / Q4Tensor (codes `data` as stored in the .smq file: rows * cols
 * int8, or (rows * cols + 1) / 2 nibble bytes; `scales`: one fp32 per block_size consecutive
 * elements of the flattened tensor; Q8Tensor.cs:17-60, Q4Tensor.cs:17-62) into the upload layout
 * of SMX_TYPE_SMQ_Q8 / _Q4: per 32 elements, the scale of their block then their codes.  No
 * value changes.  cols and block_size must be multiples of 32; out_bytes must equal
 * rows * cols / 32 * (36 for Q8, 20 for Q4).  Host memory only. */
SMX_API int smx_smq_pack(int type, const void *data, const float *scales, int64_t rows, int64_t cols,
                         int block_size, void *out, size_t out_bytes);
SMX_API int smx_model_weight_bytes(const smx_model *m, int64_t *bytes);
SMX_API int smx_model_destroy(smx_model *m);

/* Continuous batching.  The reference's BatchedInferenceEngine groups queued requests
 * (BatchedInferenceEngine.cs:186-200) and then runs each request of a group on its own
 * (ProcessBatchPrefillOnlyAsync, :241-259); here the members share every weight read.  A batcher
 * holds up to max_members sessions of one model, all created with max_ctx.  smx_batcher_add
 * prefills the session's prompt and makes it a member; the session stays marked in use
 * (SMX_EBUSY for its own calls and for smx_session_destroy) until smx_batcher_remove or
 * smx_batcher_destroy, which leave it as smx_session_generate would.  smx_batcher_step runs
 * n_steps steps for all members at once (one token each, at each member's own position)
 * and writes out_tokens[member][n_steps] in member order: members keep the order they were added
 * in, a removal closes the gap.  Members may join and leave between steps.  The model cannot be
 * destroyed while a batcher exists.  Before each step smx_batcher_step checks every member's cancel
 * request and time limit: on one it stops after the steps already run, returns SMX_ECANCELED /
 * SMX_ETIMEDOUT with those steps' tokens in out_tokens (the rest -1), and every member stays a
 * member (a timed-out member stays timed out until removed). */
typedef struct smx_batcher smx_batcher;
SMX_API int smx_batcher_create(smx_model *m, int max_members, int max_ctx, smx_batcher **out);
SMX_API int smx_batcher_add(smx_batcher *b, smx_session *s, const int32_t *prompt, int n_prompt);
/* As smx_batcher_add, but each of this member's tokens is drawn by the sampling pipeline of
 * smx_session_generate_sampled (same options, same draw stream for this seed) instead of argmax. */
SMX_API int smx_batcher_add_sampled(smx_batcher *b, smx_session *s, const int32_t *prompt, int n_prompt,
                                    const smx_sampling *params, uint64_t seed);
SMX_API int smx_batcher_remove(smx_batcher *b, smx_session *s);
/* Returns the number of members (>= 0), or a negative status. */
SMX_API int smx_batcher_count(const smx_batcher *b);
SMX_API int smx_batcher_step(smx_batcher *b, int n_steps, int32_t *out_tokens);
SMX_API int smx_batcher_destroy(smx_batcher *b);

SMX_API int smx_session_create(smx_model *m, int max_ctx, smx_session **out);
/* TransformerModel.Forward(idx[1,T], positionOffset) with the KV cache enabled: runs
 * n_tokens tokens at positions pos_offset.. and writes the last row's logits (vocab floats,
 * host memory) when logits_out != NULL.  SMX_ERANGE when pos_offset + n_tokens > max_ctx. */
SMX_API int smx_session_forward(smx_session *s, const int32_t *tokens, int n_tokens,
                                int pos_offset, float *logits_out);
/* Greedy generation entirely on the device: prefill the prompt, then n_new tokens by argmax.
 * out_tokens (host, n_new).  logits_out (host, n_new*vocab) may be NULL.
 * A prompt longer than the session context is cropped to its last max_ctx tokens, as
 * InferenceSession crops the context before prefill (InferenceSession.cs:494-508); the n_new
 * tokens must then fit: cropped length + n_new - 1 <= max_ctx, else SMX_ERANGE (the block-size
 * check of TransformerModel.cs:280-283 that a later decode step would fail).
 * The host checks, before the prefill and between graph launches (every 8 tokens at most), for
 * a cancel request (smx_session_cancel) and the session's time limit (smx_session_set_max_time).
 * On either it stops, and returns SMX_ECANCELED or SMX_ETIMEDOUT: out_tokens then holds the k
 * tokens produced so far (the first k tokens of the uninterrupted run) followed by -1, and
 * stats->n_decode_steps = k.  The session is left as after a generation of k tokens (untouched
 * when the stop comes before the prefill). */
SMX_API int smx_session_generate(smx_session *s, const int32_t *prompt, int n_prompt, int n_new,
                                 int32_t *out_tokens, float *logits_out, smx_gen_stats *stats);
/* Requests that the generation running on the session stop (the CancellationToken that
 * InferenceSession.GenerateAsync checks before every token, InferenceSession.cs:211, :481).
 * Callable from any thread, also while another thread is inside a call on s; it takes no lock
 * and touches no device state.  The request stays set until a generation call on s observes it
 * (smx_session_generate, smx_session_generate_sampled, smx_batch_generate, smx_batcher_step of a
 * batcher s belongs to): that call returns SMX_ECANCELED and clears it, so a request made
 * while no call runs cancels the next one at its first check, as an already-cancelled token does.
 * smx_session_reset clears it too.  s must stay alive for the duration of the call. */
SMX_API int smx_session_cancel(smx_session *s);
/* The MaxTimeMs limit (ProductionInferenceOptions.cs:124, applied at InferenceSession.cs:164-172):
 * a generation call on s that is still running max_time_ms after it started stops at its next
 * check with SMX_ETIMEDOUT.  For a batcher member the clock starts when it joins.  0 = no limit
 * (the default); negative values give SMX_EINVAL, as ProductionInferenceOptions.Validate
 * (ProductionInferenceOptions.cs:188-190).  Callable from any thread. */
SMX_API int smx_session_set_max_time(smx_session *s, int32_t max_time_ms);
/* Generation with the reference's sampling pipeline (InferenceSession.GenerateNextTokenAsync,
 * InferenceSession.cs:478-606) on the device: as smx_session_generate, but every new token is
 * drawn by the stages of smx_sample over the context so far (prompt and generated tokens), with
 * draw i = the top 53 bits of splitmix64(seed + i) as a double in [0, 1) (the reference draws
 * from System.Random, which is not reproduced).  Prompt cropping, cancellation and the time limit
 * as in smx_session_generate (checks between tokens). */
SMX_API int smx_session_generate_sampled(smx_session *s, const int32_t *prompt, int n_prompt, int n_new,
                                         const smx_sampling *params, uint64_t seed, int32_t *out_tokens,
                                         float *logits_out, smx_gen_stats *stats);
/* Greedy generation for n_sessions sessions of one model in lockstep: each session's prompt
 * is prefilled, then every decode step advances all sessions by one token, reading each weight
 * once per step for all of them (the reference serves sessions one at a time:
 * BatchedInferenceEngine, InferenceSession.cs:478-546 per session).  prompts holds the prompts
 * back to back, prompt_lens[i] tokens for session i; out_tokens is [n_sessions][n_new] (host).
 * The sessions must be distinct, share one model and have the same max_ctx; each ends as
 * smx_session_generate would leave it.  stats (may be NULL) sums the prefill steps.  A cancel
 * request or time limit of any listed session stops all of them between steps (SMX_ECANCELED /
 * SMX_ETIMEDOUT, the first k tokens of every session in out_tokens, the rest -1). */
SMX_API int smx_batch_generate(smx_session *const *sessions, int n_sessions, const int32_t *prompts,
                               const int32_t *prompt_lens, int n_new, int32_t *out_tokens,
                               smx_gen_stats *stats);
/* ResetKVCache (TransformerModel.cs:476-506): next forward starts at position 0. */
SMX_API int smx_session_reset(smx_session *s);
SMX_API int smx_session_destroy(smx_session *s);

#ifdef __cplusplus
}
#endif
#endif
