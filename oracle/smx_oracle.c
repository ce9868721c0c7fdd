/*
 * smx_oracle.c -- CPU restatement of SmallMind's quantized transformer forward path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the timed CPU baseline.  Never
 * linked into, or called from, the product library.
 *
 * Reference: justinamiller/SmallMind (C#/.NET 10), read as text.  The reference cannot be
 * compiled or run in this environment (no .NET toolchain), so this file restates it.
 *
 * What pins each function (tests/test_oracle.py):
 *   smxo_half_to_float      all 65,536 patterns vs numpy.float16 (IEEE closed form)
 *   smxo_float_to_half      all finite half values round-trip; RNE ties vs numpy.float16
 *   smxo_decode_nibble      the reference's own table (QuantKernelsTests.cs:149-158)
 *   smxo_dequant (5 types)  blocks assembled field by field from chosen integers by an
 *                           independent numpy bit packer, checked against sc*q-m computed
 *                           from those integers; block sizes/bytes (KQuantTensorTests.cs:19-29,
 *                           :145-155); random bytes vs committed golden vectors
 *   smxo_quantize           round-trip error bounds, half-even ties, known small cases
 *   smxo_quantize_ref_q8/q4 hand-computed cases from the Quantize formulas
 *   smxo_dequant_smq        hand cases (nibble order, two's complement, short last block);
 *                           the reference's benchmark-model.smq: every Q8 block's max |code|
 *                           is 127 (or all zero with scale 1), LayerNorm gammas decode to 1.0
 *                           and biases to 0.0 (tests/test_smq.py)
 *   SMQ upload blocks       smx_smq_pack's layout decoded equals smxo_dequant_smq of the
 *   (types 1010 / 1011)     original flattened tensor
 *   smxo_gemv_f64           numpy float64 matmul on the dequantized matrix
 *   smxo_rmsnorm/layernorm  the reference's closed-form tests (RMSNormOpsTests.cs:145-163,
 *                           LayerNormOpsTests.cs:206-229) and numpy float64
 *   smxo_rope_*             position-0 identity (RotaryEmbeddingTests.cs:33-57), pair norm
 *                           preservation, angle closed form
 *   smxo_fastexp            the Pade [2/2] closed form at chosen points incl. the clamp
 *   smxo_scale_mask_softmax row sums, causal zeros, numpy restatement with FastExp
 *   smxo_gelu/silu_mul      closed forms; fused == separate (ActivationOpsTests.cs:24-57)
 *   smxo_forward_nocache    T=1 reduces to V-row pass-through; causal invariance; numpy
 *                           float64 forward built from torch/numpy library ops
 *   smxo_session_step       equals smxo_forward_nocache row by row (cache == no-cache)
 *   smxo_sample             neutral options = plain softmax draw; top_k = 1 and tiny top_p
 *                           give the argmax; penalties, temperature, top-k, top-p, min-p each
 *                           against a numpy restatement of the stage on chosen logits; the
 *                           draw against the inverse CDF
 */
#include "smx_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#ifdef _OPENMP
#include <omp.h>
#endif
#include <immintrin.h>

/* ------------------------------------------------------------------------------------ */
/* fp16                                                                                 */
/* ------------------------------------------------------------------------------------ */

static float bits_to_float(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t float_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* Restates GgufModelLoader.HalfToFloat (GgufModelLoader.cs:919-956): subnormals are
 * renormalised, Inf/NaN keep their payload, everything else is a rebias. */
float smxo_half_to_float(uint16_t half)
{
    uint32_t sign = (uint32_t)(half >> 15) & 1u;
    uint32_t exponent = (uint32_t)(half >> 10) & 0x1Fu;
    uint32_t mantissa = (uint32_t)half & 0x3FFu;
    uint32_t result;
    if (exponent == 0) {
        if (mantissa == 0) {
            result = sign << 31;
        } else {
            exponent = 1;
            while ((mantissa & 0x400u) == 0) { mantissa <<= 1; exponent--; }
            mantissa &= 0x3FFu;
            result = (sign << 31) | ((exponent + (127 - 15)) << 23) | (mantissa << 13);
        }
    } else if (exponent == 0x1F) {
        result = (sign << 31) | 0x7F800000u | (mantissa << 13);
    } else {
        result = (sign << 31) | ((exponent + (127 - 15)) << 23) | (mantissa << 13);
    }
    return bits_to_float(result);
}

/* IEEE binary32 -> binary16, round to nearest even.  Used by the encoders to store block
 * scales (the GPU encoder carries the same integer routine). */
uint16_t smxo_float_to_half(float f)
{
    uint32_t x = float_to_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (ax >= 0x47800000u) return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return (uint16_t)sign;
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;
        uint32_t hm = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7FFFFFu) >> 13);
    uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ------------------------------------------------------------------------------------ */
/* block formats                                                                        */
/* ------------------------------------------------------------------------------------ */

int smxo_block_elems(int type)
{
    switch (type) {
    case SMXO_F32: case SMXO_F16: return 1;
    case SMXO_Q4_0: case SMXO_Q8_0: case SMXO_SMQ_Q8: case SMXO_SMQ_Q4: return 32;
    case SMXO_Q4_K: case SMXO_Q5_K: case SMXO_Q6_K: return 256;
    default: return 0;
    }
}

int smxo_block_bytes(int type)
{
    switch (type) {
    case SMXO_F32: return 4;
    case SMXO_F16: return 2;
    case SMXO_Q4_0: return 18;   /* fp16 d + 16 B nibbles */
    case SMXO_Q8_0: return 34;   /* fp16 d + 32 int8 */
    case SMXO_Q4_K: return 144;  /* d, dmin, 12 B scales, 128 B qs (Q4KTensor / KQuantTensorTests.cs:27) */
    case SMXO_Q5_K: return 176;  /* d, dmin, 12 B scales, 32 B qh, 128 B ql (GgufModelLoader.cs:836) */
    case SMXO_Q6_K: return 210;  /* 128 B ql, 64 B qh, 16 B int8 scales, fp16 d (KQuantTensorTests.cs:153) */
    case SMXO_SMQ_Q8: return 36; /* fp32 scale of the SMQ block + 32 int8 (upload layout) */
    case SMXO_SMQ_Q4: return 20; /* fp32 scale of the SMQ block + 16 B nibbles */
    default: return 0;
    }
}

/* Q4Tensor.DecodeNibble (Q4Tensor.cs:140-143): 4-bit two's complement. */
int smxo_decode_nibble(int nibble) { return nibble < 8 ? nibble : nibble - 16; }

/* Unpacks the 8 six-bit scales (bytes 0-5) and 8 six-bit mins (bytes 6-11) of a Q4_K/Q5_K
 * scale field, sequentially as GgufModelLoader.cs:688-705 does. */
static void unpack_k_scales(const uint8_t *s, uint8_t sc[8], uint8_t mn[8])
{
    sc[0] = (uint8_t)(s[0] & 0x3F);
    sc[1] = (uint8_t)((s[0] >> 6) | ((s[1] & 0x0F) << 2));
    sc[2] = (uint8_t)((s[1] >> 4) | ((s[2] & 0x03) << 4));
    sc[3] = (uint8_t)((s[2] >> 2) & 0x3F);
    sc[4] = (uint8_t)(s[3] & 0x3F);
    sc[5] = (uint8_t)((s[3] >> 6) | ((s[4] & 0x0F) << 2));
    sc[6] = (uint8_t)((s[4] >> 4) | ((s[5] & 0x03) << 4));
    sc[7] = (uint8_t)((s[5] >> 2) & 0x3F);
    mn[0] = (uint8_t)(s[6] & 0x3F);
    mn[1] = (uint8_t)((s[6] >> 6) | ((s[7] & 0x0F) << 2));
    mn[2] = (uint8_t)((s[7] >> 4) | ((s[8] & 0x03) << 4));
    mn[3] = (uint8_t)((s[8] >> 2) & 0x3F);
    mn[4] = (uint8_t)(s[9] & 0x3F);
    mn[5] = (uint8_t)((s[9] >> 6) | ((s[10] & 0x0F) << 2));
    mn[6] = (uint8_t)((s[10] >> 4) | ((s[11] & 0x03) << 4));
    mn[7] = (uint8_t)((s[11] >> 2) & 0x3F);
}

static void pack_k_scales(const int sc[8], const int mn[8], uint8_t *s)
{
    uint64_t a = 0, b = 0;
    for (int j = 0; j < 8; j++) {
        a |= (uint64_t)(sc[j] & 63) << (6 * j);
        b |= (uint64_t)(mn[j] & 63) << (6 * j);
    }
    for (int i = 0; i < 6; i++) { s[i] = (uint8_t)(a >> (8 * i)); s[6 + i] = (uint8_t)(b >> (8 * i)); }
}

/* ConvertQ8_0Tensor (GgufModelLoader.cs:464-492): y = (sbyte)q * d. */
static void dq_q8_0(const uint8_t *b, float *y, int n)
{
    float scale = smxo_half_to_float(rd16(b));
    for (int i = 0; i < n; i++) y[i] = (float)(int8_t)b[2 + i] * scale;
}

/* ConvertQ4_0Tensor (GgufModelLoader.cs:494-534): element 2i = low nibble of byte i,
 * element 2i+1 = high nibble, decoded as two's complement. */
static void dq_q4_0(const uint8_t *b, float *y, int n)
{
    float scale = smxo_half_to_float(rd16(b));
    for (int i = 0; i < n; i += 2) {
        uint8_t packed = b[2 + i / 2];
        y[i] = (float)smxo_decode_nibble(packed & 0xF) * scale;
        if (i + 1 < n) y[i + 1] = (float)smxo_decode_nibble((packed >> 4) & 0xF) * scale;
    }
}

/* ConvertQ4_KTensor (GgufModelLoader.cs:657-741): y = sc*q - m with sc = d*scale[j],
 * m = dmin*min[j]; multiply then subtract, two roundings. */
static void dq_q4_k(const uint8_t *b, float *y, int n)
{
    float d = smxo_half_to_float(rd16(b));
    float dmin = smxo_half_to_float(rd16(b + 2));
    uint8_t sc6[8], mn6[8];
    unpack_k_scales(b + 4, sc6, mn6);
    const uint8_t *qs = b + 16;
    for (int j = 0; j < 8; j++) {
        float sc = d * (float)sc6[j];
        float m = dmin * (float)mn6[j];
        int start = j * 32;
        int end = start + 32 < n ? start + 32 : n;
        for (int i = start; i < end; i++) y[i] = 0.0f;   /* the reference array starts zeroed */
        for (int i = 0; i < (end - start) / 2; i++) {
            uint8_t packed = qs[j * 16 + i];
            int q0 = packed & 0xF, q1 = (packed >> 4) & 0xF;
            float t0 = sc * (float)q0;
            y[start + 2 * i] = t0 - m;
            if (start + 2 * i + 1 < end) {
                float t1 = sc * (float)q1;
                y[start + 2 * i + 1] = t1 - m;
            }
        }
    }
}

/* ConvertQ5_KTensor (GgufModelLoader.cs:748-840): q = (hb<<4 | low4) - 16,
 * y = sc*q - m.  (The compatibility decoder in StubDecoders.cs:399-403 omits the -16; the
 * load path above is the one the runtime uses.) */
static void dq_q5_k(const uint8_t *b, float *y, int n)
{
    float d = smxo_half_to_float(rd16(b));
    float dmin = smxo_half_to_float(rd16(b + 2));
    uint8_t sc6[8], mn6[8];
    unpack_k_scales(b + 4, sc6, mn6);
    const uint8_t *qh = b + 16, *ql = b + 48;
    for (int j = 0; j < 8; j++) {
        float sc = d * (float)sc6[j];
        float m = dmin * (float)mn6[j];
        int start = j * 32;
        int end = start + 32 < n ? start + 32 : n;
        for (int i = 0; i < end - start; i++) {
            int v = j * 32 + i;
            int hb = ((qh[v / 8] >> (v % 8)) & 1) << 4;
            int low4 = (v % 2 == 0) ? (ql[v / 2] & 0xF) : ((ql[v / 2] >> 4) & 0xF);
            int q = (hb | low4) - 16;
            float t = sc * (float)q;
            y[start + i] = t - m;
        }
    }
}

/* ConvertQ6_KTensor (GgufModelLoader.cs:849-917): q = low4 | high2<<4,
 * y = (d*(sbyte)scale[j]) * (q-32). */
static void dq_q6_k(const uint8_t *b, float *y, int n)
{
    const uint8_t *ql = b, *qh = b + 128, *scales = b + 192;
    float d = smxo_half_to_float(rd16(b + 208));
    for (int j = 0; j < 16; j++) {
        float sc = d * (float)(int8_t)scales[j];
        int start = j * 16;
        int end = start + 16 < n ? start + 16 : n;
        for (int i = 0; i < end - start; i++) {
            int v = j * 16 + i;
            int low4 = (v % 2 == 0) ? (ql[v / 2] & 0xF) : ((ql[v / 2] >> 4) & 0xF);
            int high2 = (qh[v / 4] >> ((v % 4) * 2)) & 0x3;
            int q = low4 | (high2 << 4);
            y[start + i] = sc * (float)(q - 32);
        }
    }
}

/* Q8Tensor.Dequantize / Q4Tensor.Dequantize (Q8Tensor.cs:131-157, Q4Tensor.cs:150-176): element
 * i of the flattened tensor is code(i) * scales[i / block], one fp32 multiply; Q4 element i is
 * the low (i even) or high (i odd) nibble of byte i / 2, two's complement. */
int smxo_dequant_smq(int scheme, const uint8_t *data, const float *scales, int64_t n, int block, float *dst)
{
    if ((scheme != 10 && scheme != 11) || block <= 0 || n < 0) return -1;
    for (int64_t i = 0; i < n; i++) {
        int q;
        if (scheme == 10) q = (int8_t)data[i];
        else q = smxo_decode_nibble((i % 2 == 0) ? (data[i / 2] & 0xF) : ((data[i / 2] >> 4) & 0xF));
        dst[i] = (float)q * scales[i / block];
    }
    return 0;
}

/* The 32-element upload layout of SMQ blocks: fp32 scale, then the codes as in the file. */
static void dq_smq32(int type, const uint8_t *b, float *y, int n)
{
    float scale;
    memcpy(&scale, b, 4);
    smxo_dequant_smq(type == SMXO_SMQ_Q8 ? 10 : 11, b + 4, &scale, n, 32, y);
}

int smxo_dequant(int type, const uint8_t *src, int64_t n, float *dst)
{
    int be = smxo_block_elems(type), bb = smxo_block_bytes(type);
    if (!be || n < 0) return -1;
    if (type == SMXO_F32) { memcpy(dst, src, (size_t)n * 4); return 0; }
    if (type == SMXO_F16) {
        for (int64_t i = 0; i < n; i++) dst[i] = smxo_half_to_float(rd16(src + 2 * i));
        return 0;
    }
    int64_t nb = (n + be - 1) / be;
    for (int64_t blk = 0; blk < nb; blk++) {
        int cnt = (int)((n - blk * be) < be ? (n - blk * be) : be);
        const uint8_t *b = src + blk * bb;
        float *y = dst + blk * be;
        switch (type) {
        case SMXO_Q8_0: dq_q8_0(b, y, cnt); break;
        case SMXO_Q4_0: dq_q4_0(b, y, cnt); break;
        case SMXO_Q4_K: dq_q4_k(b, y, cnt); break;
        case SMXO_Q5_K: dq_q5_k(b, y, cnt); break;
        case SMXO_Q6_K: dq_q6_k(b, y, cnt); break;
        case SMXO_SMQ_Q8: case SMXO_SMQ_Q4: dq_smq32(type, b, y, cnt); break;
        default: return -1;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------------------ */
/* quantizers                                                                           */
/* ------------------------------------------------------------------------------------ */

static float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* Q8Tensor.Quantize (Q8Tensor.cs:72-128): scale = maxAbs/127 (1 if zero), q = round-half-
 * even(clamp(x*(1/scale), -127, 127)). */
void smxo_quantize_ref_q8(const float *src, int n, int block, int8_t *q, float *scales)
{
    int nb = (n + block - 1) / block;
    for (int b = 0; b < nb; b++) {
        int s = b * block, e = s + block < n ? s + block : n;
        float maxAbs = 0.0f;
        for (int i = s; i < e; i++) { float a = fabsf(src[i]); if (a > maxAbs) maxAbs = a; }
        float scale = maxAbs > 0.0f ? maxAbs / 127.0f : 1.0f;
        scales[b] = scale;
        float inv = 1.0f / scale;
        for (int i = s; i < e; i++) {
            float t = src[i] * inv;
            q[i] = (int8_t)(int)rintf(clampf(t, -127.0f, 127.0f));
        }
    }
}

/* Q4Tensor.Quantize (Q4Tensor.cs:75-134): scale = maxAbs/7, q = round(clamp(x/scale,-8,7)),
 * even index -> low nibble, odd -> high nibble, over the flattened tensor. */
void smxo_quantize_ref_q4(const float *src, int n, int block, uint8_t *data, float *scales)
{
    int nb = (n + block - 1) / block;
    for (int b = 0; b < nb; b++) {
        int s = b * block, e = s + block < n ? s + block : n;
        float maxAbs = 0.0f;
        for (int i = s; i < e; i++) { float a = fabsf(src[i]); if (a > maxAbs) maxAbs = a; }
        float scale = maxAbs > 0.0f ? maxAbs / 7.0f : 1.0f;
        scales[b] = scale;
        float inv = 1.0f / scale;
        for (int i = s; i < e; i++) {
            float t = src[i] * inv;
            int c = (int)rintf(clampf(t, -8.0f, 7.0f));
            if (i % 2 == 0) data[i / 2] = (uint8_t)(c & 0xF);
            else data[i / 2] = (uint8_t)((data[i / 2] & 0x0F) | ((c & 0xF) << 4));
        }
    }
}

static float block_maxabs(const float *x, int n)
{
    float m = 0.0f;
    for (int i = 0; i < n; i++) { float a = fabsf(x[i]); if (a > m) m = a; }
    return m;
}

/* Q8_0 block: the reference quantizer at block 32 with the scale stored as fp16. */
static void q_q8_0(const float *x, uint8_t *b)
{
    float maxAbs = block_maxabs(x, 32);
    float scale = maxAbs > 0.0f ? maxAbs / 127.0f : 1.0f;
    float inv = 1.0f / scale;
    uint16_t h = smxo_float_to_half(scale);
    b[0] = (uint8_t)h; b[1] = (uint8_t)(h >> 8);
    for (int i = 0; i < 32; i++) {
        float t = x[i] * inv;
        b[2 + i] = (uint8_t)(int8_t)(int)rintf(clampf(t, -127.0f, 127.0f));
    }
}

/* Q4_0 block with reference semantics: two's-complement nibbles, sequential pairs. */
static void q_q4_0(const float *x, uint8_t *b)
{
    float maxAbs = block_maxabs(x, 32);
    float scale = maxAbs > 0.0f ? maxAbs / 7.0f : 1.0f;
    float inv = 1.0f / scale;
    uint16_t h = smxo_float_to_half(scale);
    b[0] = (uint8_t)h; b[1] = (uint8_t)(h >> 8);
    for (int i = 0; i < 16; i++) {
        float t0 = x[2 * i] * inv, t1 = x[2 * i + 1] * inv;
        int c0 = (int)rintf(clampf(t0, -8.0f, 7.0f));
        int c1 = (int)rintf(clampf(t1, -8.0f, 7.0f));
        b[2 + i] = (uint8_t)((c0 & 0xF) | ((c1 & 0xF) << 4));
    }
}

/* Q4_K encoder (this build's own; the reference decodes Q4_K but cannot encode it).
 * Per 32-element sub-block: range [min(0,min x), max x] over 15 steps; scales and mins
 * quantized to 6 bits against fp16 super-block d = max scale/63, dmin = max min/63. */
static void q_q4_k(const float *x, uint8_t *b)
{
    float scl[8], mnv[8], maxs = 0.0f, maxm = 0.0f;
    for (int j = 0; j < 8; j++) {
        const float *s = x + 32 * j;
        float lo = 0.0f, hi = s[0];
        for (int i = 0; i < 32; i++) { if (s[i] < lo) lo = s[i]; if (s[i] > hi) hi = s[i]; }
        scl[j] = (hi - lo) / 15.0f;
        mnv[j] = -lo;
        if (scl[j] > maxs) maxs = scl[j];
        if (mnv[j] > maxm) maxm = mnv[j];
    }
    uint16_t d16 = smxo_float_to_half(maxs / 63.0f);
    uint16_t m16 = smxo_float_to_half(maxm / 63.0f);
    float df = smxo_half_to_float(d16), mf = smxo_half_to_float(m16);
    int ls[8], lm[8];
    for (int j = 0; j < 8; j++) {
        ls[j] = df > 0.0f ? (int)clampf(rintf(scl[j] / df), 0.0f, 63.0f) : 0;
        lm[j] = mf > 0.0f ? (int)clampf(rintf(mnv[j] / mf), 0.0f, 63.0f) : 0;
    }
    b[0] = (uint8_t)d16; b[1] = (uint8_t)(d16 >> 8);
    b[2] = (uint8_t)m16; b[3] = (uint8_t)(m16 >> 8);
    pack_k_scales(ls, lm, b + 4);
    for (int j = 0; j < 8; j++) {
        float sc = df * (float)ls[j];
        float m = mf * (float)lm[j];
        for (int i = 0; i < 16; i++) {
            int q[2];
            for (int t = 0; t < 2; t++) {
                float v = x[32 * j + 2 * i + t] + m;
                q[t] = sc > 0.0f ? (int)clampf(rintf(v / sc), 0.0f, 15.0f) : 0;
            }
            b[16 + 16 * j + i] = (uint8_t)(q[0] | (q[1] << 4));
        }
    }
}

/* Q5_K encoder (own): symmetric per sub-block, scale = maxAbs/15, mins zero, so the
 * reference decode y = sc*(q-16) - 0 recovers x. */
static void q_q5_k(const float *x, uint8_t *b)
{
    float scl[8], maxs = 0.0f;
    for (int j = 0; j < 8; j++) {
        scl[j] = block_maxabs(x + 32 * j, 32) / 15.0f;
        if (scl[j] > maxs) maxs = scl[j];
    }
    uint16_t d16 = smxo_float_to_half(maxs / 63.0f);
    float df = smxo_half_to_float(d16);
    int ls[8], lm[8];
    for (int j = 0; j < 8; j++) {
        ls[j] = df > 0.0f ? (int)clampf(rintf(scl[j] / df), 0.0f, 63.0f) : 0;
        lm[j] = 0;
    }
    memset(b, 0, 176);
    b[0] = (uint8_t)d16; b[1] = (uint8_t)(d16 >> 8);
    pack_k_scales(ls, lm, b + 4);
    uint8_t *qh = b + 16, *ql = b + 48;
    for (int j = 0; j < 8; j++) {
        float sc = df * (float)ls[j];
        for (int i = 0; i < 32; i++) {
            int v = 32 * j + i;
            int q = sc > 0.0f ? (int)clampf(rintf(x[v] / sc), -16.0f, 15.0f) + 16 : 16;
            if (q & 16) qh[v / 8] |= (uint8_t)(1u << (v % 8));
            if (v % 2 == 0) ql[v / 2] |= (uint8_t)(q & 0xF);
            else ql[v / 2] |= (uint8_t)((q & 0xF) << 4);
        }
    }
}

/* Q6_K encoder (own): per 16-element sub-block scale = maxAbs/31 quantized to int8 against
 * fp16 d = max scale/127; q-32 = round(x/(d*scale)) in [-32, 31]. */
static void q_q6_k(const float *x, uint8_t *b)
{
    float scl[16], maxs = 0.0f;
    for (int j = 0; j < 16; j++) {
        scl[j] = block_maxabs(x + 16 * j, 16) / 31.0f;
        if (scl[j] > maxs) maxs = scl[j];
    }
    uint16_t d16 = smxo_float_to_half(maxs / 127.0f);
    float df = smxo_half_to_float(d16);
    memset(b, 0, 210);
    uint8_t *ql = b, *qh = b + 128;
    for (int j = 0; j < 16; j++) {
        int ls = df > 0.0f ? (int)clampf(rintf(scl[j] / df), -128.0f, 127.0f) : 0;
        b[192 + j] = (uint8_t)(int8_t)ls;
        float sc = df * (float)ls;
        for (int i = 0; i < 16; i++) {
            int v = 16 * j + i;
            int q = sc > 0.0f ? (int)clampf(rintf(x[v] / sc), -32.0f, 31.0f) + 32 : 32;
            if (v % 2 == 0) ql[v / 2] |= (uint8_t)(q & 0xF);
            else ql[v / 2] |= (uint8_t)((q & 0xF) << 4);
            qh[v / 4] |= (uint8_t)(((q >> 4) & 3) << ((v % 4) * 2));
        }
    }
    b[208] = (uint8_t)d16; b[209] = (uint8_t)(d16 >> 8);
}

int smxo_quantize(int type, const float *src, int64_t n, uint8_t *dst)
{
    int be = smxo_block_elems(type), bb = smxo_block_bytes(type);
    if (!be || n < 0 || n % be) return -1;
    if (type == SMXO_F32) { memcpy(dst, src, (size_t)n * 4); return 0; }
    if (type == SMXO_F16) {
        for (int64_t i = 0; i < n; i++) {
            uint16_t h = smxo_float_to_half(src[i]);
            dst[2 * i] = (uint8_t)h; dst[2 * i + 1] = (uint8_t)(h >> 8);
        }
        return 0;
    }
    for (int64_t blk = 0; blk < n / be; blk++) {
        const float *x = src + blk * be;
        uint8_t *b = dst + blk * bb;
        switch (type) {
        case SMXO_Q8_0: q_q8_0(x, b); break;
        case SMXO_Q4_0: q_q4_0(x, b); break;
        case SMXO_Q4_K: q_q4_k(x, b); break;
        case SMXO_Q5_K: q_q5_k(x, b); break;
        case SMXO_Q6_K: q_q6_k(x, b); break;
        case SMXO_SMQ_Q8: case SMXO_SMQ_Q4: {   /* the reference quantizer at block 32 */
            float scale;
            if (type == SMXO_SMQ_Q8) smxo_quantize_ref_q8(x, 32, 32, (int8_t *)(b + 4), &scale);
            else smxo_quantize_ref_q4(x, 32, 32, b + 4, &scale);
            memcpy(b, &scale, 4);
            break;
        }
        default: return -1;
        }
    }
    return 0;
}

int smxo_gemv_f64(int type, const uint8_t *W, int N, int K, const float *x, double *y)
{
    int be = smxo_block_elems(type), bb = smxo_block_bytes(type);
    if (!be || K % be) return -1;
    size_t row_bytes = (size_t)(K / be) * bb;
    float *row = (float *)malloc(sizeof(float) * (size_t)K);
    if (!row) return -2;
    for (int n = 0; n < N; n++) {
        smxo_dequant(type, W + (size_t)n * row_bytes, K, row);
        double acc = 0.0;
        for (int k = 0; k < K; k++) acc += (double)row[k] * (double)x[k];
        y[n] = acc;
    }
    free(row);
    return 0;
}

/* ------------------------------------------------------------------------------------ */
/* norms, RoPE, softmax, activations                                                    */
/* ------------------------------------------------------------------------------------ */

/* Sum reduction in the reference's Vector<float> order for n >= 128 (8 lanes, then a
 * horizontal sum, then the scalar tail), sequential otherwise (RMSNormOps.cs:56-112). */
static float vec_sum_sq(const float *x, int n)
{
    if (n >= 128) {
        float lane[8] = {0};
        int f = 0;
        for (; f <= n - 8; f += 8)
            for (int l = 0; l < 8; l++) { float p = x[f + l] * x[f + l]; lane[l] = lane[l] + p; }
        float s = 0.0f;
        for (int l = 0; l < 8; l++) s += lane[l];
        for (; f < n; f++) { float p = x[f] * x[f]; s += p; }
        return s;
    }
    float s = 0.0f;
    for (int i = 0; i < n; i++) { float p = x[i] * x[i]; s += p; }
    return s;
}

/* RMSNormOps.RMSNorm (RMSNormOps.cs:28-219): invRms = 1/sqrt(sumSq/n + eps),
 * y = gamma * (x * invRms). */
void smxo_rmsnorm(const float *x, const float *g, float *y, int rows, int n, float eps)
{
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * n;
        float *yr = y + (size_t)r * n;
        float sumSq = vec_sum_sq(xr, n);
        float invRms = 1.0f / sqrtf(sumSq / (float)n + eps);
        for (int i = 0; i < n; i++) { float t = xr[i] * invRms; yr[i] = g[i] * t; }
    }
}

/* LayerNormOps.LayerNorm (LayerNormOps.cs:27-280): two-pass mean/variance,
 * invStd = 1/sqrt(var + eps), y = fma(gamma, (x-mean)*invStd, beta). */
void smxo_layernorm(const float *x, const float *g, const float *b, float *y, int rows, int n,
                    float eps)
{
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * n;
        float *yr = y + (size_t)r * n;
        float mean, sq = 0.0f;
        if (n >= 128) {
            float lane[8] = {0};
            int f = 0;
            for (; f <= n - 8; f += 8) for (int l = 0; l < 8; l++) lane[l] += xr[f + l];
            float s = 0.0f;
            for (int l = 0; l < 8; l++) s += lane[l];
            for (; f < n; f++) s += xr[f];
            mean = s / (float)n;
            float lq[8] = {0};
            f = 0;
            for (; f <= n - 8; f += 8)
                for (int l = 0; l < 8; l++) { float dd = xr[f + l] - mean; float p = dd * dd; lq[l] += p; }
            for (int l = 0; l < 8; l++) sq += lq[l];
            for (; f < n; f++) { float dd = xr[f] - mean; float p = dd * dd; sq += p; }
        } else {
            float s = 0.0f;
            for (int i = 0; i < n; i++) s += xr[i];
            mean = s / (float)n;
            for (int i = 0; i < n; i++) { float dd = xr[i] - mean; float p = dd * dd; sq += p; }
        }
        float var = sq / (float)n;
        float invStd = 1.0f / sqrtf(var + eps);
        for (int i = 0; i < n; i++) {
            float t = (xr[i] - mean) * invStd;
            yr[i] = fmaf(g[i], t, b[i]);
        }
    }
}

/* RotaryEmbedding.PrecomputeTables (RotaryEmbedding.cs:45-60):
 * freq = 1/pow(theta, 2i/hd), angle = pos*freq, layout [pos][hd/2]. */
void smxo_rope_tables(int max_pos, int head_dim, float theta, float *cos_t, float *sin_t)
{
    int half = head_dim / 2;
    for (int pos = 0; pos < max_pos; pos++)
        for (int i = 0; i < half; i++) {
            float expo = (2.0f * (float)i) / (float)head_dim;
            float freq = 1.0f / powf(theta, expo);
            float angle = (float)pos * freq;
            sin_t[pos * half + i] = sinf(angle);
            cos_t[pos * half + i] = cosf(angle);
        }
}

/* RotaryEmbedding.ApplyRotationInPlace (RotaryEmbedding.cs:85-121): adjacent pairs
 * (2i, 2i+1); data layout [head][seq][hd]. */
void smxo_rope_apply(float *data, int pos0, int n_heads, int seq, int head_dim,
                     const float *cos_t, const float *sin_t)
{
    int half = head_dim / 2;
    for (int h = 0; h < n_heads; h++)
        for (int s = 0; s < seq; s++) {
            int pos = pos0 + s;
            float *v = data + ((size_t)h * seq + s) * head_dim;
            for (int i = 0; i < half; i++) {
                float x0 = v[2 * i], x1 = v[2 * i + 1];
                float c = cos_t[pos * half + i], sn = sin_t[pos * half + i];
                float a = x0 * c, bb = x1 * sn, cc = x0 * sn, dd = x1 * c;
                v[2 * i] = a - bb;
                v[2 * i + 1] = cc + dd;
            }
        }
}

/* MathUtils.FastExp (MathUtils.cs:20-32): clamp to [-87.3, 88.7], then the Pade [2/2]
 * ratio (1 + x/2 + x^2/12) / (1 - x/2 + x^2/12) with 1/12 written as 0.08333333f. */
float smxo_fastexp(float x)
{
    x = fmaxf(-87.3f, fminf(x, 88.7f));
    float x2 = x * x;
    float h = x * 0.5f, q = x2 * 0.08333333f;
    float num = 1.0f + h; num = num + q;
    float den = 1.0f - h; den = den + q;
    return num / den;
}

/* OptimizedOps.FusedScaleMaskSoftmax (OptimizedOps.cs:39-93), in place on a [seq][k_seq]
 * row block: max of s*scale over the valid columns, e = FastExp(s*scale - max), normalise
 * by multiplying with 1/sum, zero the masked tail. */
void smxo_scale_mask_softmax(float *scores, float scale, int seq, int k_seq, int cache_off)
{
    for (int i = 0; i < seq; i++) {
        float *row = scores + (size_t)i * k_seq;
        int valid = cache_off + i + 1;
        float maxVal = -INFINITY;
        for (int j = 0; j < valid; j++) { float s = row[j] * scale; if (s > maxVal) maxVal = s; }
        float sum = 0.0f;
        for (int j = 0; j < valid; j++) {
            float s = row[j] * scale;
            float e = smxo_fastexp(s - maxVal);
            row[j] = e;
            sum += e;
        }
        float invSum = 1.0f / sum;
        for (int j = 0; j < valid; j++) row[j] *= invSum;
        for (int j = valid; j < k_seq; j++) row[j] = 0.0f;
    }
}

/* ActivationOps.GELU, vector form (ActivationOps.cs:262-276). */
void smxo_gelu(const float *in, float *out, int n)
{
    for (int i = 0; i < n; i++) {
        float x = in[i];
        float x2 = x * x;
        float x3 = x2 * x;
        float t3 = 0.044715f * x3;
        float inner = 0.7978845608f * (x + t3);
        inner = fmaxf(-10.0f, fminf(10.0f, inner));
        float inner2 = inner * inner;
        float num = inner * (27.0f + inner2);
        float den = 27.0f + 9.0f * inner2;
        float th = num / den;
        float hx = 0.5f * x;
        out[i] = hx * (1.0f + th);
    }
}

/* ActivationOps.FusedSiLUMul (ActivationOps.cs:565-580) with FastSigmoid (:304-309):
 * sigmoid of the clamped input, multiplied by the unclamped input. */
void smxo_silu_mul(const float *g, const float *u, float *y, int n)
{
    for (int i = 0; i < n; i++) {
        float x = g[i];
        float c = fmaxf(-20.0f, fminf(x, 20.0f));
        float sig = 1.0f / (1.0f + expf(-c));
        float silu = x * sig;
        y[i] = silu * u[i];
    }
}

int smxo_argmax(const float *v, int n)
{
    int best = 0;
    for (int i = 1; i < n; i++) if (v[i] > v[best]) best = i;
    return best;
}

/* ---- next-token sampling (InferenceSession.cs:565-606) ------------------------------------ */
static int cmp_float_asc(const void *a, const void *b)
{
    const float x = *(const float *)a, y = *(const float *)b;
    return (x > y) - (x < y);
}

typedef struct { float p; int i; } smxo_pi;
static int cmp_prob_desc(const void *a, const void *b)
{
    const smxo_pi *x = (const smxo_pi *)a, *y = (const smxo_pi *)b;
    if (x->p != y->p) return x->p < y->p ? 1 : -1;
    return x->i - y->i;   /* ties by index (the reference's sort leaves their order open) */
}

/* NormalizeProbabilities (InferenceSession.cs:969-1010): p * (1 / sum) when sum > 0. */
static void smxo_normalize(float *p, int n)
{
    float sum = 0.0f;
    for (int i = 0; i < n; i++) sum += p[i];
    if (sum > 0.0f) {
        const float inv = 1.0f / sum;
        for (int i = 0; i < n; i++) p[i] = p[i] * inv;
    }
}

/* The whole pipeline: penalties (:765-843), temperature (:741-763), top-k (:628-664), softmax
 * (:666-706), top-p (:845-912), min-p (:914-936), SampleFromProbs (:708-724) with the draw u.
 * probs_out receives the final distribution; returns the sampled id. */
int smxo_sample(const float *logits, int n, const int32_t *ctx, int n_ctx, float temperature, int top_k,
                double top_p, double min_p, float rep, float presence, float frequency, int window, double u,
                float *probs_out)
{
    float *l = (float *)malloc((size_t)n * sizeof(float));
    memcpy(l, logits, (size_t)n * sizeof(float));
    if (rep != 1.0f || presence != 0.0f || frequency != 0.0f) {
        const int win = window > 0 ? window : (n_ctx < 256 ? n_ctx : 256);
        const int start = n_ctx - win > 0 ? n_ctx - win : 0;
        const int aw = n_ctx - start;
        int *ids = (int *)malloc((size_t)(aw > 0 ? aw : 1) * sizeof(int));
        int *cnt = (int *)malloc((size_t)(aw > 0 ? aw : 1) * sizeof(int));
        int seen = 0;
        for (int i = start; i < n_ctx; i++) {
            int f = -1;
            for (int j = 0; j < seen; j++)
                if (ids[j] == ctx[i]) { f = j; break; }
            if (f >= 0) cnt[f]++;
            else { ids[seen] = ctx[i]; cnt[seen] = 1; seen++; }
        }
        for (int j = 0; j < seen; j++) {
            const int t = ids[j];
            if (t < 0 || t >= n) continue;
            if (rep != 1.0f) l[t] = l[t] > 0 ? l[t] / rep : l[t] * rep;
            if (presence != 0.0f) l[t] -= presence;
            if (frequency != 0.0f) l[t] -= (float)cnt[j] * frequency;
        }
        free(ids);
        free(cnt);
    }
    if (temperature != 1.0f) {
        const float inv = 1.0f / temperature;
        for (int i = 0; i < n; i++) l[i] *= inv;
    }
    if (top_k > 0 && top_k < n) {
        float *srt = (float *)malloc((size_t)n * sizeof(float));
        memcpy(srt, l, (size_t)n * sizeof(float));
        qsort(srt, (size_t)n, sizeof(float), cmp_float_asc);
        const float kth = srt[n - 1 - (top_k - 1)];   /* descending order, index k - 1 */
        for (int i = 0; i < n; i++) l[i] = l[i] >= kth ? l[i] : -INFINITY;
        free(srt);
    }
    float *p = probs_out;
    float mx = -INFINITY;
    for (int i = 0; i < n; i++)
        if (l[i] != -INFINITY) mx = fmaxf(mx, l[i]);
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        p[i] = l[i] != -INFINITY ? expf(l[i] - mx) : 0.0f;
        sum += p[i];
    }
    if (sum > 0.0f)
        for (int i = 0; i < n; i++) p[i] /= sum;
    if (top_p < 1.0) {
        smxo_pi *o = (smxo_pi *)malloc((size_t)n * sizeof(smxo_pi));
        for (int i = 0; i < n; i++) { o[i].p = p[i]; o[i].i = i; }
        qsort(o, (size_t)n, sizeof(smxo_pi), cmp_prob_desc);
        float cum = 0.0f;
        int cut = n;
        for (int i = 0; i < n; i++) {
            cum += o[i].p;
            if (cum >= top_p) { cut = i + 1; break; }
        }
        for (int i = cut; i < n; i++) p[o[i].i] = 0.0f;
        free(o);
        smxo_normalize(p, n);
    }
    if (min_p > 0.0) {
        float pm = -INFINITY;
        for (int i = 0; i < n; i++) pm = fmaxf(pm, p[i]);
        const float thr = pm * (float)min_p;
        for (int i = 0; i < n; i++)
            if (p[i] < thr) p[i] = 0.0f;
        smxo_normalize(p, n);
    }
    free(l);
    double cum = 0.0;
    for (int i = 0; i < n; i++) {
        cum += p[i];
        if (cum >= u) return i;
    }
    return n - 1;
}

static uint64_t splitmix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void smxo_fill_normal(uint64_t seed, int64_t n, float std, float *out)
{
    for (int64_t i = 0; i < n; i++) {
        uint64_t r = splitmix64(seed * 0xD1B54A32D192ED03ull + (uint64_t)(i >> 1));
        float u1 = (float)((r >> 40) + 1) * 5.9604644775390625e-08f;
        float u2 = (float)(r & 0xFFFFFFu) * 5.9604644775390625e-08f;
        float rad = sqrtf(-2.0f * logf(u1));
        float th = 6.283185307179586f * u2;
        float z = (i & 1) ? rad * sinf(th) : rad * cosf(th);
        out[i] = std * z;
    }
}

/* ------------------------------------------------------------------------------------ */
/* model                                                                                */
/* ------------------------------------------------------------------------------------ */

static float *interleave8(float *W, int N, int K);

typedef struct {
    float *attn_g, *attn_b;
    float *wq, *wk, *wv, *bq, *bk, *bv;   /* as uploaded */
    float *wqkv, *bqkv;                   /* merged [Q;K;V] rows (GgufModelLoader.cs:1027-1110) */
    float *wo, *bo, *ffn_g, *ffn_b;
    float *wg, *bg, *wu, *bu, *wd, *bd;
} olayer;

struct smxo_model {
    int arch, vocab, ctx, d, L, H, Hkv, hd, ff, kvdim, nqkv, hidden;
    float theta, eps;
    float *tok, *pos, *out_g, *out_b, *head;
    olayer *layers;
    float *cos_t, *sin_t;
    int finalized;
};

struct smxo_session {
    smxo_model *m;
    int max_ctx;
    float *kc, *vc;     /* [L][Hkv][max_ctx][hd] */
};

smxo_model *smxo_model_create(int arch, int vocab, int ctx, int d, int n_layer, int n_head,
                              int n_kv_head, int ff, float rope_theta, float norm_eps)
{
    if (vocab <= 0 || ctx <= 0 || d <= 0 || n_layer <= 0 || n_head <= 0 || n_kv_head <= 0) return NULL;
    if (d % n_head || n_head % n_kv_head || (d / n_head) % 2) return NULL;
    smxo_model *m = (smxo_model *)calloc(1, sizeof(smxo_model));
    m->arch = arch; m->vocab = vocab; m->ctx = ctx; m->d = d; m->L = n_layer;
    m->H = n_head; m->Hkv = n_kv_head; m->hd = d / n_head; m->ff = ff;
    m->kvdim = n_kv_head * m->hd; m->nqkv = d + 2 * m->kvdim;
    m->hidden = arch == SMXO_ARCH_GPT2 ? 4 * d : ff;   /* MLP is fixed at 4*d (MLP.cs:25-26) */
    m->theta = rope_theta; m->eps = norm_eps;
    m->layers = (olayer *)calloc((size_t)n_layer, sizeof(olayer));
    return m;
}

static float **tensor_slot(smxo_model *m, const char *name, int64_t *expect)
{
    int d = m->d, kv = m->kvdim, hid = m->hidden;
    if (!strcmp(name, "token_embd.weight")) { *expect = (int64_t)m->vocab * d; return &m->tok; }
    if (!strcmp(name, "position_embd.weight")) { *expect = (int64_t)m->ctx * d; return &m->pos; }
    if (!strcmp(name, "output_norm.weight")) { *expect = d; return &m->out_g; }
    if (!strcmp(name, "output_norm.bias")) { *expect = d; return &m->out_b; }
    if (!strcmp(name, "output.weight")) { *expect = (int64_t)m->vocab * d; return &m->head; }
    int li; char rest[64];
    if (sscanf(name, "blk.%d.%63s", &li, rest) != 2 || li < 0 || li >= m->L) return NULL;
    olayer *l = &m->layers[li];
    struct { const char *n; float **p; int64_t e; } tab[] = {
        {"attn_norm.weight", &l->attn_g, d}, {"attn_norm.bias", &l->attn_b, d},
        {"attn_q.weight", &l->wq, (int64_t)d * d}, {"attn_k.weight", &l->wk, (int64_t)kv * d},
        {"attn_v.weight", &l->wv, (int64_t)kv * d}, {"attn_q.bias", &l->bq, d},
        {"attn_k.bias", &l->bk, kv}, {"attn_v.bias", &l->bv, kv},
        {"attn_qkv.weight", &l->wqkv, (int64_t)m->nqkv * d}, {"attn_qkv.bias", &l->bqkv, m->nqkv},
        {"attn_output.weight", &l->wo, (int64_t)d * d}, {"attn_output.bias", &l->bo, d},
        {"ffn_norm.weight", &l->ffn_g, d}, {"ffn_norm.bias", &l->ffn_b, d},
        {"ffn_gate.weight", &l->wg, (int64_t)hid * d}, {"ffn_gate.bias", &l->bg, hid},
        {"ffn_up.weight", &l->wu, (int64_t)hid * d}, {"ffn_up.bias", &l->bu, hid},
        {"ffn_down.weight", &l->wd, (int64_t)d * hid}, {"ffn_down.bias", &l->bd, d},
    };
    for (size_t i = 0; i < sizeof(tab) / sizeof(tab[0]); i++)
        if (!strcmp(rest, tab[i].n)) { *expect = tab[i].e; return tab[i].p; }
    return NULL;
}

int smxo_model_set_tensor(smxo_model *m, const char *name, int type, const uint8_t *bytes,
                          int64_t n_elems)
{
    int64_t expect = 0;
    if (m->finalized) return -5;
    float **slot = tensor_slot(m, name, &expect);
    if (!slot) return -1;
    if (expect != n_elems) return -2;
    float *buf = (float *)malloc(sizeof(float) * (size_t)n_elems);
    if (!buf) return -3;
    /* whole blocks per chunk, dequantized in parallel (each element depends on its block only) */
    const int be = smxo_block_elems(type), bb = smxo_block_bytes(type);
    if (!be || n_elems % be) { free(buf); return -4; }
    const int64_t chunk = (int64_t)be * 4096, nchunk = (n_elems + chunk - 1) / chunk;
    int bad = 0;
#pragma omp parallel for schedule(static) num_threads(smxo_get_threads()) reduction(|:bad)
    for (int64_t c = 0; c < nchunk; c++) {
        const int64_t e0 = c * chunk, n = n_elems - e0 < chunk ? n_elems - e0 : chunk;
        bad |= smxo_dequant(type, bytes + e0 / be * bb, n, buf + e0) != 0;
    }
    if (bad) { free(buf); return -4; }
    free(*slot);
    *slot = buf;
    return 0;
}

static float *concat3(const float *a, size_t na, const float *b, size_t nb, const float *c, size_t nc)
{
    float *r = (float *)malloc(sizeof(float) * (na + nb + nc));
    memcpy(r, a, na * 4); memcpy(r + na, b, nb * 4); memcpy(r + na + nb, c, nc * 4);
    return r;
}

int smxo_model_finalize(smxo_model *m)
{
    int d = m->d, kv = m->kvdim;
    if (m->finalized) return 0;
    if (!m->tok || !m->out_g) return -1;
    if (m->arch == SMXO_ARCH_GPT2 && (!m->pos || !m->out_b)) return -1;
    if (!m->head) {   /* HandleWeightTying (GgufModelLoader.cs:1126-1147) */
        m->head = (float *)malloc(sizeof(float) * (size_t)m->vocab * d);
        memcpy(m->head, m->tok, sizeof(float) * (size_t)m->vocab * d);
    }
    for (int i = 0; i < m->L; i++) {
        olayer *l = &m->layers[i];
        if (!l->wqkv) {
            if (!l->wq || !l->wk || !l->wv) return -2;
            l->wqkv = concat3(l->wq, (size_t)d * d, l->wk, (size_t)kv * d, l->wv, (size_t)kv * d);
        }
        if (!l->bqkv && (l->bq || l->bk || l->bv)) {
            float *z = (float *)calloc((size_t)m->nqkv, 4);
            if (l->bq) memcpy(z, l->bq, (size_t)d * 4);
            if (l->bk) memcpy(z + d, l->bk, (size_t)kv * 4);
            if (l->bv) memcpy(z + d + kv, l->bv, (size_t)kv * 4);
            l->bqkv = z;
        }
        if (!l->attn_g || !l->ffn_g || !l->wo || !l->wu || !l->wd) return -3;
        if (m->arch == SMXO_ARCH_LLAMA && !l->wg) return -3;
        if (m->arch == SMXO_ARCH_GPT2 && (!l->attn_b || !l->ffn_b)) return -3;
    }
    /* the linears' weights in the 8-row interleaved layout linear() reads */
    for (int i = 0; i < m->L; i++) {
        olayer *l = &m->layers[i];
        if (l->wq && l->wqkv != l->wq) { free(l->wq); free(l->wk); free(l->wv); l->wq = l->wk = l->wv = NULL; }
        l->wqkv = interleave8(l->wqkv, m->nqkv, d);
        l->wo = interleave8(l->wo, d, d);
        l->wg = interleave8(l->wg, m->hidden, d);
        l->wu = interleave8(l->wu, m->hidden, d);
        l->wd = interleave8(l->wd, d, m->hidden);
    }
    m->head = interleave8(m->head, m->vocab, d);
    if (m->arch == SMXO_ARCH_LLAMA) {
        m->cos_t = (float *)malloc(sizeof(float) * (size_t)m->ctx * (m->hd / 2));
        m->sin_t = (float *)malloc(sizeof(float) * (size_t)m->ctx * (m->hd / 2));
        smxo_rope_tables(m->ctx, m->hd, m->theta, m->cos_t, m->sin_t);
    }
    m->finalized = 1;
    return 0;
}

void smxo_model_destroy(smxo_model *m)
{
    if (!m) return;
    for (int i = 0; i < m->L; i++) {
        olayer *l = &m->layers[i];
        float *ps[] = {l->attn_g, l->attn_b, l->wq, l->wk, l->wv, l->bq, l->bk, l->bv, l->wqkv,
                       l->bqkv, l->wo, l->bo, l->ffn_g, l->ffn_b, l->wg, l->bg, l->wu, l->bu,
                       l->wd, l->bd};
        for (size_t k = 0; k < sizeof(ps) / sizeof(ps[0]); k++) free(ps[k]);
    }
    free(m->layers); free(m->tok); free(m->pos); free(m->out_g); free(m->out_b);
    free(m->head); free(m->cos_t); free(m->sin_t); free(m);
}

/* Linear.ForwardFP32 (NeuralNet.cs:233-298): y = x * W^T, then + bias.  Every output is one
 * chain of fused multiply-adds over k = 0..K-1 in order, starting from 0, then the bias add:
 * the same arithmetic whatever the tiling, thread count or vector width, so the threaded and
 * vectorised form below gives bit-identical outputs to a single-threaded scalar loop
 * (tests/test_oracle.py checks this).  Weights are kept as 8-row blocks interleaved by k,
 * Wi[block][k][8] (rows past N zero), so one vector load serves 8 rows' chains; row blocks run
 * over the threads, and with several tokens, 8 tokens share each weight load. */
static int g_threads = 0;   /* 0: OpenMP default */

void smxo_set_threads(int n) { g_threads = n > 0 ? n : 0; }

int smxo_get_threads(void)
{
#ifdef _OPENMP
    return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
    return 1;
#endif
}

/* [N][K] row-major -> [ceil(N/8)][K][8]; frees W. */
static float *interleave8(float *W, int N, int K)
{
    if (!W) return NULL;
    const int nb = (N + 7) / 8;
    float *Wi = (float *)aligned_alloc(32, sizeof(float) * (size_t)nb * K * 8);
#pragma omp parallel for schedule(static) num_threads(smxo_get_threads())
    for (int b = 0; b < nb; b++)
        for (int k = 0; k < K; k++)
            for (int r = 0; r < 8; r++) {
                const int n = b * 8 + r;
                Wi[((size_t)b * K + k) * 8 + r] = n < N ? W[(size_t)n * K + k] : 0.0f;
            }
    free(W);
    return Wi;
}

static void linear(const float *x, int T, int K, const float *Wi, const float *bias, int N, float *y)
{
    const int nb = (N + 7) / 8;
    const int nth = smxo_get_threads();
    if (T == 1) {
        /* four row blocks per pass: four independent chains per lane */
        const int ng = (nb + 3) / 4;
#pragma omp parallel for schedule(static) num_threads(nth)
        for (int g = 0; g < ng; g++) {
            const int b0 = g * 4, nbg = nb - b0 < 4 ? nb - b0 : 4;
            __m256 acc[4];
            const float *w[4];
            for (int j = 0; j < 4; j++) {
                acc[j] = _mm256_setzero_ps();
                w[j] = Wi + (size_t)(b0 + (j < nbg ? j : 0)) * K * 8;
            }
            for (int k = 0; k < K; k++) {
                const __m256 xv = _mm256_broadcast_ss(x + k);
                for (int j = 0; j < 4; j++) acc[j] = _mm256_fmadd_ps(xv, _mm256_load_ps(w[j] + (size_t)k * 8), acc[j]);
            }
            for (int j = 0; j < nbg; j++) {
                float out[8];
                _mm256_storeu_ps(out, acc[j]);
                for (int r = 0; r < 8 && (b0 + j) * 8 + r < N; r++) y[(b0 + j) * 8 + r] = out[r];
            }
        }
    } else {
        /* tokens transposed into tiles of 8: xt[tile][k][8], zero-padded */
        const int nt = (T + 7) / 8;
        float *xt = (float *)aligned_alloc(32, sizeof(float) * (size_t)nt * K * 8);
        for (int tt = 0; tt < nt; tt++)
            for (int k = 0; k < K; k++)
                for (int l = 0; l < 8; l++) {
                    int t = tt * 8 + l;
                    xt[((size_t)tt * K + k) * 8 + l] = t < T ? x[(size_t)t * K + k] : 0.0f;
                }
#pragma omp parallel for schedule(dynamic, 1) num_threads(nth)
        for (int b = 0; b < nb; b++) {
            const int n0 = b * 8, rows = N - n0 < 8 ? N - n0 : 8;
            const float *w = Wi + (size_t)b * K * 8;
            for (int tt = 0; tt < nt; tt++) {
                const float *xp = xt + (size_t)tt * K * 8;
                __m256 acc[8];
                for (int r = 0; r < 8; r++) acc[r] = _mm256_setzero_ps();
                for (int k = 0; k < K; k++) {
                    const __m256 xv = _mm256_load_ps(xp + (size_t)k * 8);
                    for (int r = 0; r < 8; r++)
                        acc[r] = _mm256_fmadd_ps(_mm256_broadcast_ss(w + (size_t)k * 8 + r), xv, acc[r]);
                }
                float out[8][8];
                for (int r = 0; r < 8; r++) _mm256_storeu_ps(out[r], acc[r]);
                for (int l = 0; l < 8 && tt * 8 + l < T; l++)
                    for (int r = 0; r < rows; r++) y[(size_t)(tt * 8 + l) * N + n0 + r] = out[r][l];
            }
        }
        free(xt);
    }
    if (bias)
        for (int t = 0; t < T; t++) {
            float *yt = y + (size_t)t * N;
            for (int i = 0; i < N; i++) yt[i] = yt[i] + bias[i];
        }
}

static void norm_rows(const smxo_model *m, const float *x, const float *g, const float *b,
                      float *y, int rows)
{
    if (m->arch == SMXO_ARCH_LLAMA) smxo_rmsnorm(x, g, y, rows, m->d, m->eps);
    else smxo_layernorm(x, g, b, y, rows, m->d, m->eps);
}

/* Embedding (NeuralNet.cs:376-391) plus, for GPT-2, the learned position row
 * (TransformerModel.cs:299-326, :355-434). */
static void embed(const smxo_model *m, int32_t tok, int pos, float *x)
{
    const float *e = m->tok + (size_t)tok * m->d;
    if (m->arch == SMXO_ARCH_GPT2) {
        const float *p = m->pos + (size_t)pos * m->d;
        for (int i = 0; i < m->d; i++) x[i] = e[i] + p[i];
    } else {
        memcpy(x, e, sizeof(float) * (size_t)m->d);
    }
}

/* MLP / GatedMLP on rows of h (GatedMLP.cs:51-93, MLP.cs:36-58); out = [T][d]. */
static void mlp(const smxo_model *m, const olayer *l, const float *h, int T, float *t1, float *t2,
                float *out)
{
    int d = m->d, hid = m->hidden;
    if (m->arch == SMXO_ARCH_LLAMA) {
        linear(h, T, d, l->wg, l->bg, hid, t1);
        linear(h, T, d, l->wu, l->bu, hid, t2);
        smxo_silu_mul(t1, t2, t1, T * hid);
    } else {
        linear(h, T, d, l->wu, l->bu, hid, t2);
        smxo_gelu(t2, t1, T * hid);
    }
    linear(t1, T, hid, l->wd, l->bd, d, out);
}

int smxo_forward_nocache(smxo_model *m, const int32_t *tokens, int T, float *logits, int all_rows)
{
    if (!m->finalized || T <= 0 || T > m->ctx) return -1;
    for (int t = 0; t < T; t++) if (tokens[t] < 0 || tokens[t] >= m->vocab) return -2;
    int d = m->d, H = m->H, Hkv = m->Hkv, hd = m->hd, kv = m->kvdim, N = m->nqkv;
    int hid = m->hidden;
    float scale = 1.0f / sqrtf((float)hd);          /* MultiHeadAttention.cs:686 */
    int group = H / Hkv;
    float *x = (float *)malloc(sizeof(float) * (size_t)T * d);
    float *h = (float *)malloc(sizeof(float) * (size_t)T * d);
    float *qkv = (float *)malloc(sizeof(float) * (size_t)T * N);
    float *q = (float *)malloc(sizeof(float) * (size_t)H * T * hd);
    float *k = (float *)malloc(sizeof(float) * (size_t)Hkv * T * hd);
    float *v = (float *)malloc(sizeof(float) * (size_t)Hkv * T * hd);
    float *y = (float *)malloc(sizeof(float) * (size_t)T * d);
    float *o = (float *)malloc(sizeof(float) * (size_t)T * d);
    float *t1 = (float *)malloc(sizeof(float) * (size_t)T * hid);
    float *t2 = (float *)malloc(sizeof(float) * (size_t)T * hid);
    for (int t = 0; t < T; t++) embed(m, tokens[t], t, x + (size_t)t * d);
    for (int li = 0; li < m->L; li++) {
        const olayer *l = &m->layers[li];
        norm_rows(m, x, l->attn_g, l->attn_b, h, T);
        linear(h, T, d, l->wqkv, l->bqkv, N, qkv);
        /* ExtractAndReshapeQ/KVInPlace (MultiHeadAttention.cs:395-462) */
        for (int t = 0; t < T; t++) {
            const float *r = qkv + (size_t)t * N;
            for (int hh = 0; hh < H; hh++)
                memcpy(q + ((size_t)hh * T + t) * hd, r + hh * hd, sizeof(float) * hd);
            for (int hh = 0; hh < Hkv; hh++) {
                memcpy(k + ((size_t)hh * T + t) * hd, r + d + hh * hd, sizeof(float) * hd);
                memcpy(v + ((size_t)hh * T + t) * hd, r + d + kv + hh * hd, sizeof(float) * hd);
            }
        }
        if (m->arch == SMXO_ARCH_LLAMA) {     /* no cache: position offset 0 */
            smxo_rope_apply(q, 0, H, T, hd, m->cos_t, m->sin_t);
            smxo_rope_apply(k, 0, Hkv, T, hd, m->cos_t, m->sin_t);
        }
#pragma omp parallel for schedule(dynamic, 1) num_threads(smxo_get_threads())
        for (int hh = 0; hh < H; hh++) {
            float *att = (float *)malloc(sizeof(float) * (size_t)T * T);
            int kvh = hh / group;
            const float *qh = q + (size_t)hh * T * hd;
            const float *kh = k + (size_t)kvh * T * hd;
            const float *vh = v + (size_t)kvh * T * hd;
            for (int i = 0; i < T; i++)
                for (int j = 0; j < T; j++) {
                    float s = 0.0f;
                    for (int e = 0; e < hd; e++) s = fmaf(qh[i * hd + e], kh[j * hd + e], s);
                    att[i * T + j] = s;
                }
            smxo_scale_mask_softmax(att, scale, T, T, 0);
            for (int i = 0; i < T; i++) {
                float acc[512];
                for (int e = 0; e < hd; e++) acc[e] = 0.0f;
                for (int j = 0; j < T; j++) {
                    float p = att[i * T + j];
                    for (int e = 0; e < hd; e++) acc[e] = fmaf(p, vh[j * hd + e], acc[e]);
                }
                /* ReshapeAttentionOutputInPlace (MultiHeadAttention.cs:643-667) */
                memcpy(y + (size_t)i * d + hh * hd, acc, sizeof(float) * hd);
            }
            free(att);
        }
        linear(y, T, d, l->wo, l->bo, d, o);
        for (size_t i = 0; i < (size_t)T * d; i++) x[i] = x[i] + o[i];   /* TransformerBlock.cs:170 */
        norm_rows(m, x, l->ffn_g, l->ffn_b, h, T);
        mlp(m, l, h, T, t1, t2, o);
        for (size_t i = 0; i < (size_t)T * d; i++) x[i] = x[i] + o[i];   /* TransformerBlock.cs:184 */
    }
    int r0 = all_rows ? 0 : T - 1;
    norm_rows(m, x + (size_t)r0 * d, m->out_g, m->out_b, h, T - r0);
    linear(h, T - r0, d, m->head, NULL, m->vocab, logits);
    free(x); free(h); free(qkv); free(q); free(k); free(v); free(y); free(o);
    free(t1); free(t2);
    return 0;
}

smxo_session *smxo_session_create(smxo_model *m, int max_ctx)
{
    if (!m->finalized || max_ctx <= 0 || max_ctx > m->ctx) return NULL;
    smxo_session *s = (smxo_session *)calloc(1, sizeof(smxo_session));
    size_t cache = (size_t)m->L * m->Hkv * max_ctx * m->hd;
    s->m = m; s->max_ctx = max_ctx;
    s->kc = (float *)calloc(cache, 4); s->vc = (float *)calloc(cache, 4);
    if (!s->kc || !s->vc) { smxo_session_destroy(s); return NULL; }
    return s;
}

void smxo_session_destroy(smxo_session *s)
{
    if (!s) return;
    free(s->kc); free(s->vc); free(s);
}

/* Tokens tok[i] of sessions ss[i] at positions pos[i], i < T, through the model with each
 * session's KV cache (written and read with the same stride: the intent stated in
 * GoldenValues.cs:71-83).  A session may appear several times at consecutive positions (a
 * prefill run) or once per token (several sessions stepping together).  Per layer every token's
 * K/V is written before any attention reads the cache, and token i attends to positions
 * 0..pos[i] of its own session, so the outputs are bit-identical to T single-token steps in
 * order.  logits: rows lg_from..T-1 ([T - lg_from][V]), or NULL. */
static int step_batch(smxo_model *m, smxo_session *const *ss, const int32_t *tok, const int *pos, int T,
                      float *logits, int lg_from)
{
    int d = m->d, H = m->H, Hkv = m->Hkv, hd = m->hd, kv = m->kvdim, N = m->nqkv, hid = m->hidden;
    float scale = 1.0f / sqrtf((float)hd);
    int group = H / Hkv, maxL = 1;
    for (int i = 0; i < T; i++) {
        if (pos[i] < 0 || pos[i] >= ss[i]->max_ctx || tok[i] < 0 || tok[i] >= m->vocab) return -1;
        if (pos[i] + 1 > maxL) maxL = pos[i] + 1;
    }
    const int nth = smxo_get_threads();
    float *x = (float *)malloc(sizeof(float) * (size_t)T * d);
    float *h = (float *)malloc(sizeof(float) * (size_t)T * d);
    float *qkv = (float *)malloc(sizeof(float) * (size_t)T * N);
    float *y = (float *)malloc(sizeof(float) * (size_t)T * d);
    float *t1 = (float *)malloc(sizeof(float) * (size_t)T * hid);
    float *t2 = (float *)malloc(sizeof(float) * (size_t)T * hid);
    float *t3 = (float *)malloc(sizeof(float) * (size_t)T * d);
    float *sc = (float *)malloc(sizeof(float) * (size_t)nth * maxL);
    for (int i = 0; i < T; i++) embed(m, tok[i], pos[i], x + (size_t)i * d);
    for (int li = 0; li < m->L; li++) {
        const olayer *l = &m->layers[li];
        norm_rows(m, x, l->attn_g, l->attn_b, h, T);
        linear(h, T, d, l->wqkv, l->bqkv, N, qkv);
        for (int i = 0; i < T; i++) {
            float *q = qkv + (size_t)i * N, *k = q + d, *v = q + d + kv;
            if (m->arch == SMXO_ARCH_LLAMA) {
                smxo_rope_apply(q, pos[i], H, 1, hd, m->cos_t, m->sin_t);
                smxo_rope_apply(k, pos[i], Hkv, 1, hd, m->cos_t, m->sin_t);
            }
            const smxo_session *s = ss[i];
            for (int hh = 0; hh < Hkv; hh++) {
                size_t base = (((size_t)li * Hkv + hh) * s->max_ctx + pos[i]) * hd;
                memcpy(s->kc + base, k + hh * hd, 4 * (size_t)hd);
                memcpy(s->vc + base, v + hh * hd, 4 * (size_t)hd);
            }
        }
        /* MultiHeadAttention.cs:676-844 per (token, head) */
#pragma omp parallel for schedule(dynamic, 1) num_threads(nth)
        for (int ih = 0; ih < T * H; ih++) {
            int i = ih / H, hh = ih % H;
#ifdef _OPENMP
            float *scores = sc + (size_t)omp_get_thread_num() * maxL;
#else
            float *scores = sc;
#endif
            const smxo_session *s = ss[i];
            int kvh = hh / group, L = pos[i] + 1;
            const float *kh = s->kc + ((size_t)li * Hkv + kvh) * s->max_ctx * hd;
            const float *vh = s->vc + ((size_t)li * Hkv + kvh) * s->max_ctx * hd;
            const float *qh = qkv + (size_t)i * N + hh * hd;
            for (int j = 0; j < L; j++) {
                float acc = 0.0f;
                for (int e = 0; e < hd; e++) acc = fmaf(qh[e], kh[(size_t)j * hd + e], acc);
                scores[j] = acc;
            }
            smxo_scale_mask_softmax(scores, scale, 1, L, pos[i]);
            float acc[512];
            for (int e = 0; e < hd; e++) acc[e] = 0.0f;
            for (int j = 0; j < L; j++)
                for (int e = 0; e < hd; e++) acc[e] = fmaf(scores[j], vh[(size_t)j * hd + e], acc[e]);
            memcpy(y + (size_t)i * d + hh * hd, acc, 4 * (size_t)hd);
        }
        linear(y, T, d, l->wo, l->bo, d, t3);
        for (size_t i = 0; i < (size_t)T * d; i++) x[i] = x[i] + t3[i];   /* TransformerBlock.cs:170 */
        norm_rows(m, x, l->ffn_g, l->ffn_b, h, T);
        mlp(m, l, h, T, t1, t2, t3);
        for (size_t i = 0; i < (size_t)T * d; i++) x[i] = x[i] + t3[i];   /* TransformerBlock.cs:184 */
    }
    if (logits && lg_from < T) {
        norm_rows(m, x + (size_t)lg_from * d, m->out_g, m->out_b, h, T - lg_from);
        linear(h, T - lg_from, d, m->head, NULL, m->vocab, logits);
    }
    free(x); free(h); free(qkv); free(y); free(t1); free(t2); free(t3); free(sc);
    return 0;
}

int smxo_session_step(smxo_session *s, int32_t token, int pos, float *logits)
{
    return step_batch(s->m, &s, &token, &pos, 1, logits, 0);
}

int smxo_session_prefill(smxo_session *s, const int32_t *tokens, int T, int pos0, float *logits_last)
{
    if (T <= 0 || pos0 < 0 || pos0 + T > s->max_ctx) return -1;
    smxo_session **ss = (smxo_session **)malloc(sizeof(*ss) * (size_t)T);
    int *pos = (int *)malloc(sizeof(int) * (size_t)T);
    for (int i = 0; i < T; i++) { ss[i] = s; pos[i] = pos0 + i; }
    int rc = step_batch(s->m, ss, tokens, pos, T, logits_last, T - 1);
    free(ss); free(pos);
    return rc;
}

int smxo_step_tokens(smxo_session *const *ss, const int32_t *tokens, const int *pos, int n, float *logits,
                     int lg_from)
{
    if (n <= 0 || lg_from < 0) return -1;
    for (int i = 0; i < n; i++) if (ss[i]->m != ss[0]->m) return -1;
    return step_batch(ss[0]->m, ss, tokens, pos, n, logits, lg_from);
}

int smxo_multi_step(smxo_session *const *ss, const int32_t *tokens, const int *pos, int n, float *logits)
{
    if (n <= 0) return -1;
    for (int i = 0; i < n; i++) {
        if (ss[i]->m != ss[0]->m) return -1;
        for (int j = 0; j < i; j++) if (ss[j] == ss[i]) return -1;
    }
    return step_batch(ss[0]->m, ss, tokens, pos, n, logits, 0);
}

static int64_t now_ns(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (int64_t)ts.tv_sec * 1000000000ll + ts.tv_nsec;
}

int smxo_generate_greedy(smxo_model *m, const int32_t *prompt, int n_prompt, int n_new,
                         int32_t *out_tokens, int64_t *prefill_ns, int64_t *decode_ns)
{
    /* InferenceSession.GenerateNextTokenAsync crops the context to its last blockSize tokens
     * before the prefill (InferenceSession.cs:494-508) */
    if (n_prompt > m->ctx) {
        prompt += n_prompt - m->ctx;
        n_prompt = m->ctx;
    }
    if (n_prompt <= 0 || n_new <= 0 || n_prompt + n_new - 1 > m->ctx) return -1;
    smxo_session *s = smxo_session_create(m, n_prompt + n_new - 1);
    if (!s) return -2;
    float *logits = (float *)malloc(sizeof(float) * (size_t)m->vocab);
    int64_t t0 = now_ns();
    if (n_prompt > 1) smxo_session_prefill(s, prompt, n_prompt - 1, 0, NULL);
    int64_t t1 = now_ns();
    int32_t tok = prompt[n_prompt - 1];
    for (int i = 0; i < n_new; i++) {
        smxo_session_step(s, tok, n_prompt - 1 + i, logits);
        tok = smxo_argmax(logits, m->vocab);
        out_tokens[i] = tok;
    }
    int64_t t2 = now_ns();
    if (prefill_ns) *prefill_ns = t1 - t0;
    if (decode_ns) *decode_ns = t2 - t1;
    free(logits);
    smxo_session_destroy(s);
    return 0;
}
