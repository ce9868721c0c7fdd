// smx_internal.h -- definitions shared by the kernels and the host runtime of libsmx.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <stdlib.h>

#include <string>

#include "../../include/smx.h"

namespace smx {

// ---- backend ("smx") weight layouts -------------------------------------------------------
//
// All layouts are row-major over the [rows][cols] weight; every row is an integral number of
// blocks.  Each row's main-stream bytes are a multiple of 16, so every 16-byte load is aligned.
//
//  Q4_0  main: [row][blk][16]   nibbles as in GGUF (element 2i low, 2i+1 high)
//        d   : [row][blk] fp16
//  Q8_0  main: [row][blk][32]   int8 as in GGUF
//        d   : [row][blk] fp16
//  Q4_K  main: [row][sb][144]   the GGUF super-block unchanged (16 B header + 128 B qs)
//  Q5_K  main: [row][sb][176]   header 16 B | qh' 32 B | ql 128 B.  qh' is a bit permutation of
//                               GGUF qh: dword j (elements 32j..32j+31), byte k, bit (2g+p)
//                               holds the high bit of element 32j + 8g + 2k + p.
//  Q6_K  main: [row][sb][208]   ql 128 B | qh' 64 B | int8 scales 16 B;  d: [row][sb] fp16.
//                               qh' chunk c = dwords (D0, D1) at 128 + 8c; D_p byte k bits
//                               (2g, 2g+1) hold the two high bits of element 32c + 8g + 2k + p.
//  F16   main: [row][chunk][64]  fp16 values (GGUF F16 rows unchanged)
//  F32   main: [row][chunk][128] fp32 values (GGUF F32 rows unchanged)
//  SQ8   main: [row][blk][32]   int8 codes of SmallMind's Q8Tensor (SMQ files);
//        d   : [row][blk] fp32 scale (the scale of the SMQ block holding the 32 elements)
//  SQ4   main: [row][blk][16]   nibbles of Q4Tensor (element 2i low, 2i+1 high, two's complement);
//        d   : [row][blk] fp32 scale
//
// The permutations put the high bits of the four elements that share one byte position of a
// 4-byte group of ql at the same bit offset of four consecutive bytes, so one shift and one
// and-or rebuild four 5-/6-bit codes.
//
// Upload ("source") layouts: the GGUF blocks for the GGUF formats and F16 / F32 rows; for SQ8 /
// SQ4 blocks of 32 elements, each the fp32 scale followed by the codes (36 / 20 bytes), which
// an SMQ tensor of any block size that is a multiple of 32 is re-laid into without rounding.

enum Fmt {
    FMT_Q4_0 = 0, FMT_Q8_0 = 1, FMT_Q4_K = 2, FMT_Q5_K = 3, FMT_Q6_K = 4,
    FMT_F16 = 5, FMT_F32 = 6, FMT_SQ8 = 7, FMT_SQ4 = 8, FMT_COUNT = 9
};

__host__ __device__ constexpr bool fmt_kquant(int f) { return f == FMT_Q4_K || f == FMT_Q5_K || f == FMT_Q6_K; }
__host__ __device__ constexpr bool fmt_dense(int f) { return f == FMT_F16 || f == FMT_F32; }
__host__ __device__ constexpr int fmt_block_elems(int f) { return fmt_kquant(f) ? 256 : 32; }
__host__ __device__ constexpr int fmt_main_bytes(int f)
{
    return f == FMT_Q4_0 ? 16 : f == FMT_Q8_0 ? 32 : f == FMT_Q4_K ? 144 : f == FMT_Q5_K ? 176 : f == FMT_Q6_K ? 208
         : f == FMT_F16 ? 64 : f == FMT_F32 ? 128 : f == FMT_SQ8 ? 32 : 16;
}
__host__ __device__ constexpr bool fmt_has_d(int f)
{
    return f == FMT_Q4_0 || f == FMT_Q8_0 || f == FMT_Q6_K || f == FMT_SQ8 || f == FMT_SQ4;
}
// bytes per block of the d stream
__host__ __device__ constexpr int fmt_d_bytes(int f) { return f == FMT_SQ8 || f == FMT_SQ4 ? 4 : fmt_has_d(f) ? 2 : 0; }
// bytes per block of the upload layout
__host__ __device__ constexpr int fmt_gguf_bytes(int f)
{
    return f == FMT_Q4_0 ? 18 : f == FMT_Q8_0 ? 34 : f == FMT_Q4_K ? 144 : f == FMT_Q5_K ? 176 : f == FMT_Q6_K ? 210
         : f == FMT_F16 ? 64 : f == FMT_F32 ? 128 : f == FMT_SQ8 ? 36 : 20;
}

int fmt_from_type(int type);   // -1 if not a weight-matrix type

struct WView {
    int fmt;              // Fmt
    // 1: the matrix is kept resident in the MALL and read with plain loads; 0: its loads
    // carry the non-temporal hint (streamed past the caches)
    int cache = 0;
    const uint8_t *q;     // main stream
    const uint16_t *d;    // fp16 scale stream or nullptr
    int64_t rows, cols;
    int nb;               // blocks per row
};

// ---- GEMV prologue / epilogue selectors ---------------------------------------------------
enum Pro { PRO_NONE = 0, PRO_RMS = 1, PRO_LN = 2 };
enum Epi {
    EPI_STORE = 0,   // out[r] = acc + bias
    EPI_RESID = 1,   // out[r] = resid[r] + (acc + bias)
    EPI_SILU = 2,    // rows interleaved gate/up: out[i] = silu(g) * u
    EPI_GELU = 3,    // out[r] = gelu(acc + bias)
    EPI_QKV = 4,     // rows [Q | K | V]: RoPE on Q/K, Q -> out, K/V -> caches at *pos
    EPI_ARGMAX = 5   // out[r] = acc + bias; each workgroup's best row -> wg_val/wg_idx, then a
                     // one-workgroup kernel takes the argmax over them (lowest index on ties)
                     // -> *amax_out and, with `tokens`, tokens[*tok_pos + 1], ++*tok_pos
};

// Device ranges read ahead into the memory-side cache (MALL) by extra workgroups of the
// one-launch decode attention: the weights of the GEMV that follows it in the decode step.
struct Prefetch {
    static constexpr int kMax = 8;
    const uint8_t *p[kMax];
    uint32_t bytes[kMax];
    int n;
};
constexpr unsigned kPrefetchWgs = 128;   // workgroups appended to a launch that prefetches

struct GemvArgs {
    WView w;
    const float *x;        // [m][cols]
    int64_t x_stride;
    float *out;            // [m][out_stride]
    int64_t out_stride;
    const float *bias;     // [rows] or nullptr (interleaved like the rows for EPI_SILU)
    const float *resid;    // EPI_RESID
    const float *gamma;    // PRO_RMS / PRO_LN
    const float *beta;     // PRO_LN
    float eps;
    int pro, epi;
    // EPI_QKV
    int d_model, kv_dim, head_dim, ctx_stride, use_rope;
    float *k_cache;             // [n_kv_head][head_dim][ctx_stride] of this layer
    float *v_cache;             // [n_kv_head][ctx_stride][head_dim] of this layer
    const float *rope_cos, *rope_sin;   // [ctx][head_dim/2]
    const int32_t *pos;         // device position (nullptr: use pos_val)
    int pos_val;
    // activation source: x (x_embed == 0) or the exact dequantised embedding row emb_row of
    // `emb` plus, when embp.q != nullptr, row embp_row of `embp` (learned positions)
    int x_embed;
    WView emb, embp;
    int64_t emb_row, embp_row;
    // EPI_ARGMAX (m == 1): per-workgroup partials [grid] and the outputs
    float *wg_val;
    int32_t *wg_idx;
    int32_t *amax_out, *tokens, *tok_pos;
    // EPI_ARGMAX with x_next set: the selected token's embedding row (+ the learned position
    // row of the next position when next_embp.q is set) is written to x_next, ready for the
    // next decode step
    float *x_next;
    WView next_emb, next_embp;
    // x_parts = 2 (m == 1, no norm): the activation vector is x + x[x_part_stride], two partial
    // sums added in that order (the two-chunk decode attention output).  Kept last: the
    // kernels read the leading fields first.
    int x_parts;
    int64_t x_part_stride;
};

hipError_t launch_gemv(const GemvArgs &a, int m, hipStream_t s);

// Launch shape of the fused GEMV for a [rows][cols] matrix: R rows per wave, S waves per row
// group splitting K, C chunks of 32 elements per lane, 4/S row groups per 4-wave workgroup
// (workgroup b owns rows [b*n, (b+1)*n), n = R*4/S).  One round of 64*S*C chunks covers the
// whole row for the staged launches.
enum GemvShape {
    GS_R4S1, GS_R2S1, GS_R2S2, GS_R4S2, GS_R2S4,   // C = 1
    GS_R4S1H2,                                     // K <= 1024, tall: rows on each half of a wave
    GS_R4S4,                                       // K <= 8192
    GS_R4S2C3, GS_R4S2C4,                          // K <= 12288 / 16384 (plain GEMVs)
    GS_WIDE                                        // R=2, S=4, C=2 (plain GEMVs, few rows)
};
// Every workgroup stages the whole activation vector (K floats), so the longer the rows, the
// more rows one staged copy should serve; short matrices keep more, smaller workgroups in
// flight.  Measured on MI355X (graph-timed, weights from HBM): 2048 x 5632 Q8_0 5.20 us with two
// rows per workgroup (R2S4), 4.75 us with eight (2 rows x 3 chunks per wave, one wave per row
// group); 2048 x 8192 Q5_K 6.05 us (R2S4), 5.53 (R4S4), 6.50 (R2S1C4); 4096 x 11008 Q4_0 12.1 us
// (R2S4C2), 9.2 us (R4S2C3).  In the decode step the 2048 x 5632 down projection runs faster as
// R4S4 (4 rows per workgroup, 512 workgroups) than with 8 rows per workgroup (256 workgroups,
// one wave per SIMD): configs[2] decode 1880 -> 1908 tok/s.
inline GemvShape gemv_shape(int64_t rows, int64_t cols)
{
    const int64_t nch = cols / 32;
    // (half-wave rows: configs[0]'s 50257 x 768 head 18.3 -> 12.9 us, decode 4250 -> 4380 tok/s;
    // on its 768-3072-row matrices the full-wave shape stayed faster)
    if (nch <= 32 && rows >= 8192) return GS_R4S1H2;
    if (nch <= 64) return rows >= 8192 ? GS_R4S1 : GS_R2S1;
    if (nch <= 128) return rows >= 4096 ? GS_R4S2 : GS_R2S2;
    if (rows < 1024) return nch <= 256 ? GS_R2S4 : GS_WIDE;
    if (nch <= 256) return GS_R4S4;
    if (nch <= 384) return GS_R4S2C3;
    return nch <= 512 ? GS_R4S2C4 : GS_WIDE;
}

// ---- quantized GEMM on the matrix cores for M activation rows (tokens) ------------------------
// y[M][rows] = norm(x)[M][cols] W^T with the GEMV's prologues and epilogues applied per token.
// For EPI_QKV every token carries its own position and KV cache (several sessions may share
// one launch): K/V rows go to kc_tok[t] / vc_tok[t] + layer_off at position tok_pos[t].
struct QgemmArgs {
    WView w;
    const uint8_t *xp;          // activation parts (k_qprep output)
    int M;
    float *y;                   // [M][y_stride]
    int64_t y_stride;
    const float *bias;          // [rows] or nullptr (interleaved like the rows for EPI_SILU)
    int epi;                    // EPI_STORE / EPI_RESID / EPI_GELU / EPI_SILU / EPI_QKV
    // EPI_SILU / EPI_GELU: when set, the outputs go to yp as the activation parts of the next
    // GEMM (qgemm_xp_bytes(M, width) bytes) instead of y
    uint8_t *yp;
    // EPI_QKV
    int d_model, kv_dim, head_dim, use_rope, ctx_stride;
    int64_t layer_off;
    float *const *kc_tok;
    float *const *vc_tok;
    const int32_t *tok_pos;
    const float *rope_cos, *rope_sin;
    // RMSNorm folded across two GEMMs (up to 16 tokens, rows of whole 256-element super-blocks):
    // RMSNorm(x) W^T = r (.) ((gamma (.) x) W^T), r = 1 / sqrt(sum x^2 / K + eps) per token.
    // Producer (EPI_RESID): with np set, the new residual x also goes to np as the activation
    // parts of gamma (.) x (ngamma = the next norm's gamma) and the per-token sums of x^2 over
    // each 16-row tile to nss[tile][M].  Consumer: with rss set, xp holds those parts and each
    // token's products are scaled by r before the epilogue, with sum x^2 = the rss_n tile sums
    // rss[p][tok] added in order.
    uint8_t *np;
    const float *ngamma;
    float *nss;
    const float *rss;
    int rss_n;
    float r_eps;
};
// Scratch bytes of the activation parts for M tokens of K elements.
size_t qgemm_xp_bytes(int M, int K);
// Prepares the parts of the (normalised, PRO_RMS / PRO_LN) activations into xp, then runs the
// GEMM.  a.xp must point at qgemm_xp_bytes(a.M, cols) bytes of scratch.  With x == nullptr
// (and PRO_NONE) a.xp already holds the parts, written by the producing kernel.
hipError_t launch_qgemm(const QgemmArgs &a, const float *x, int64_t x_stride, int pro,
                        const float *gamma, const float *beta, float eps, hipStream_t s);

// ---- other kernels -------------------------------------------------------------------------
hipError_t launch_dequant_gguf(int type, const void *blocks, int64_t n, float *out, hipStream_t s);
hipError_t launch_quantize_gguf(int type, const float *x, int64_t n, void *blocks, hipStream_t s);
hipError_t launch_fill_normal(uint64_t seed, int64_t n, float std, float *out, hipStream_t s);
// GGUF rows [rows][cols] -> smx layout rows dst_row = row_off + r * row_step.
hipError_t launch_repack(int fmt, const uint8_t *gguf, int64_t rows, int64_t cols, uint8_t *dst_q,
                         uint16_t *dst_d, int64_t dst_rows, int64_t row_off, int64_t row_step,
                         hipStream_t s);
hipError_t launch_dequant_smx(const WView &w, int64_t row0, int64_t nrows, float *out, hipStream_t s);

hipError_t launch_rmsnorm(const float *x, const float *g, float *y, int rows, int n, float eps, hipStream_t s);
hipError_t launch_layernorm(const float *x, const float *g, const float *b, float *y, int rows, int n,
                            float eps, hipStream_t s);
hipError_t launch_rope(float *data, int n_heads, int seq, int hd, int pos0, const float *c,
                       const float *sn, hipStream_t s);
hipError_t launch_softmax(float *scores, float scale, int seq, int k_seq, int cache_off, hipStream_t s);
// Decode attention as two launches spread over the chip: scores per (KV head, position block)
// into `scores` (attention_scores_floats(n_head, max_pos) floats: rows of max_pos rounded up
// to a multiple of 4), then softmax + P.V per (head, 16-dimension slice).  Positions up to
// max_pos (<= ctx_stride) are covered; pos_dev (if set) gives n_pos - 1.
// With max_chunks >= 2, contexts of 2305..4608 positions run as two workgroups per (head,
// slice) that write two partial outputs, out[0] and out[n_head * hd], to be summed by the
// caller; attention_pv_chunks says how many partial outputs a call writes.
size_t attention_scores_floats(int n_head, int max_pos);
int attention_pv_chunks(int max_pos, int max_chunks);
hipError_t launch_attention_split(const float *q, const float *kc, const float *vc, float *out,
                                  float *scores, int n_head, int n_kv_head, int hd, int ctx_stride,
                                  const int32_t *pos_dev, int n_pos_fixed, int max_pos, hipStream_t s,
                                  int max_chunks = 1, const Prefetch *pf = nullptr);
hipError_t launch_sample(const float *logits, int n, const int32_t *ctx, int n_ctx, const smx_sampling &sp,
                         double u, float *probs, int32_t *out, hipStream_t s);
// Device state of a sampled generation: the options, the seed of the draw stream and the
// number of draws taken.  Draw i is uniform_draw(seed, i).
struct SampleState {
    smx_sampling params;
    uint64_t seed;
    uint64_t counter;
};
// splitmix64(seed + i) scaled to a double in [0, 1) (the top 53 bits)
__host__ __device__ inline double uniform_draw(uint64_t seed, uint64_t i)
{
    uint64_t z = seed + i + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z = z ^ (z >> 31);
    return (double)(z >> 11) * (1.0 / 9007199254740992.0);
}
hipError_t launch_sample_rows(const float *logits, int n, int64_t stride, int M, int32_t *const *tok_arr,
                              const int32_t *pos, int32_t *ids, SampleState *st, const int32_t *on, float *probs,
                              hipStream_t s);
hipError_t launch_sample_step(const float *logits, int n, int32_t *tokens, int32_t *pos, SampleState *st,
                              float *probs, hipStream_t s);
hipError_t launch_silu_mul(const float *g, const float *u, float *y, int64_t n, hipStream_t s);
hipError_t launch_gelu(const float *x, float *y, int64_t n, hipStream_t s);
// Reads bytes (a multiple of 16, < 4 GiB) of device memory and discards them (smx_stream_read).
hipError_t launch_stream_read(const void *src, uint64_t bytes, hipStream_t s);
hipError_t launch_argmax(const float *x, int n, int32_t *out, int32_t *tokens, int32_t *pos,
                         hipStream_t s);
// Argmax over n (value, index) pairs, lowest index on ties; same outputs as launch_argmax.
hipError_t launch_argmax_pairs(const float *val, const int32_t *idx, int n, int32_t *out,
                               int32_t *tokens, int32_t *pos, hipStream_t s);
// The same, then the selected token's embedding row (+ learned position row pos + 1 when posw
// is set) written to x_next: the embedding lookup of the next decode step.
hipError_t launch_argmax_embed(const float *val, const int32_t *idx, int n, int32_t *out,
                               int32_t *tokens, int32_t *pos, const WView &tok, const WView *posw,
                               float *x_next, hipStream_t s);
hipError_t launch_embed(const WView &tok, const WView *posw, const int32_t *tokens,
                        const int32_t *pos, float *x, hipStream_t s);
hipError_t launch_advance(int32_t *pos, hipStream_t s);
// Token batches (prefill chunks, several sessions in lockstep): embedding rows, decode
// attention per (token, head) with per-token position and KV cache, argmax per logits row.
hipError_t launch_embed_tokens(const WView &tok, const WView *posw, const int32_t *ids,
                               const int32_t *pos, float *x, int64_t x_stride, int M, hipStream_t s);
// Causal attention of M consecutive tokens of one session at positions p_first .. (prefill
// chunks) on the matrix cores: q [M][q_stride] (head h at h*hd), kc / vc the layer's cache
// ([n_kv_head][hd][ctx_stride] / [n_kv_head][ctx_stride][hd]), out [M][out_stride].
bool attention_prefill_supported(int n_head, int n_kv_head, int hd);
// With out_parts set, the outputs are written as the activation parts of the next GEMM
// (xp_store, token tok_off + t, element h*hd + d) instead of out.
hipError_t launch_attention_prefill(const float *q, int q_stride, const float *kc, const float *vc, float *out,
                                    int out_stride, int n_head, int n_kv_head, int hd, int ctx_stride,
                                    int p_first, int M, hipStream_t s, uint8_t *out_parts = nullptr,
                                    int tok_off = 0);
// Several sessions' runs of a token batch in one launch: workgroup b takes the rows
// blk[2b] .. blk[2b] + blk[2b+1] - 1 of the batch (at most attention_prefill_block_rows rows, all
// of one run), with that session's cache (kc_tok / vc_tok of its first row, plus layer_off) and
// the first row's position; q, out and the parts are addressed by batch row.
struct PrefillBlocks {
    const int32_t *blk;
    float *const *kc_tok, *const *vc_tok;
    const int32_t *pos;
    int64_t layer_off;
};
int attention_prefill_block_rows(int n_head, int n_kv_head);
hipError_t launch_attention_prefill_blocks(const float *q, int q_stride, float *out, int out_stride, int n_head,
                                           int n_kv_head, int hd, int ctx_stride, int n_blocks,
                                           const PrefillBlocks &pb, hipStream_t s, uint8_t *out_parts = nullptr);
hipError_t launch_attention_tokens(const float *q, int64_t q_stride, float *const *kc_tok,
                                   float *const *vc_tok, int64_t layer_off, float *out,
                                   int64_t out_stride, int n_head, int n_kv_head, int hd,
                                   int ctx_stride, const int32_t *tok_pos, int M, hipStream_t s,
                                   uint8_t *out_parts = nullptr);
hipError_t launch_argmax_rows(const float *x, int n, int64_t stride, int M, int32_t *tok_next,
                              int32_t *tok_pos, int32_t *const *tok_arr, hipStream_t s);

// ---- errors and block geometry (host_common.cpp) ------------------------------------------
void set_error(const std::string &msg);
const char *last_error();
int type_block_elems(int type);   // elements per block (1 for F32 / F16), 0 if unknown
int type_block_bytes(int type);   // bytes per block, 0 if unknown

}  // namespace smx
