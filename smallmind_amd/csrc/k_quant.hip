// k_quant.hip -- block-format kernels: GGUF dequantization, encoders, weight repacking.
//
// GGUF-layout dequantization restates GgufModelLoader.Convert*Tensor (GgufModelLoader.cs:
// 419-917) element for element; Q8_0/Q4_0 encoders restate Q8Tensor.Quantize /
// Q4Tensor.Quantize (Q8Tensor.cs:72-128, Q4Tensor.cs:75-134) at block 32 with an fp16 scale;
// the K-quant encoders are this build's own and write the layout the reference decodes.
#include "smx_formats.h"

namespace smx {

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float rd_half_exact(const uint8_t *p) { return h2f_exact(ld_u16(p)); }

// ---- GGUF dequantization: one thread per 32 elements ---------------------------------------
__device__ void unpack_k_scales(const uint8_t *s, uint32_t *sc, uint32_t *mn)
{
    sc[0] = s[0] & 0x3Fu;
    sc[1] = (s[0] >> 6) | ((s[1] & 0x0Fu) << 2);
    sc[2] = (s[1] >> 4) | ((s[2] & 0x03u) << 4);
    sc[3] = (s[2] >> 2) & 0x3Fu;
    sc[4] = s[3] & 0x3Fu;
    sc[5] = (s[3] >> 6) | ((s[4] & 0x0Fu) << 2);
    sc[6] = (s[4] >> 4) | ((s[5] & 0x03u) << 4);
    sc[7] = (s[5] >> 2) & 0x3Fu;
    mn[0] = s[6] & 0x3Fu;
    mn[1] = (s[6] >> 6) | ((s[7] & 0x0Fu) << 2);
    mn[2] = (s[7] >> 4) | ((s[8] & 0x03u) << 4);
    mn[3] = (s[8] >> 2) & 0x3Fu;
    mn[4] = s[9] & 0x3Fu;
    mn[5] = (s[9] >> 6) | ((s[10] & 0x0Fu) << 2);
    mn[6] = (s[10] >> 4) | ((s[11] & 0x03u) << 4);
    mn[7] = (s[11] >> 2) & 0x3Fu;
}

__global__ void k_dequant_gguf(int type, const uint8_t *__restrict__ src, int64_t n,
                               float *__restrict__ out)
{
    const int64_t chunk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t e0 = chunk * 32;
    if (e0 >= n) return;
    const int cnt = (int)(n - e0 < 32 ? n - e0 : 32);
    float *y = out + e0;
    if (type == SMX_TYPE_F32) {
        const float *f = (const float *)src + e0;
        for (int i = 0; i < cnt; i++) y[i] = f[i];
    } else if (type == SMX_TYPE_F16) {
        for (int i = 0; i < cnt; i++) y[i] = rd_half_exact(src + 2 * (e0 + i));
    } else if (type == SMX_TYPE_SMQ_Q8 || type == SMX_TYPE_SMQ_Q4) {
        // Q8Tensor.Dequantize / Q4Tensor.Dequantize (Q8Tensor.cs:131-157, Q4Tensor.cs:150-178):
        // code * scale, one fp32 multiply; 32-element blocks of [fp32 scale | codes]
        const bool q8 = type == SMX_TYPE_SMQ_Q8;
        const uint8_t *b = src + chunk * (q8 ? 36 : 20);
        const float d = __uint_as_float((uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) |
                                        ((uint32_t)b[3] << 24));
        for (int i = 0; i < cnt; i++) {
            int q;
            if (q8) {
                q = (int8_t)b[4 + i];
            } else {
                const uint32_t n = (b[4 + i / 2] >> (4 * (i & 1))) & 15u;
                q = n < 8 ? (int)n : (int)n - 16;   // Q4Tensor.DecodeNibble (Q4Tensor.cs:140-143)
            }
            y[i] = (float)q * d;
        }
    } else if (type == SMX_TYPE_Q8_0) {   // GgufModelLoader.cs:464-492
        const uint8_t *b = src + chunk * 34;
        const float d = rd_half_exact(b);
        for (int i = 0; i < cnt; i++) y[i] = (float)(int8_t)b[2 + i] * d;
    } else if (type == SMX_TYPE_Q4_0) {   // GgufModelLoader.cs:494-534
        const uint8_t *b = src + chunk * 18;
        const float d = rd_half_exact(b);
        for (int i = 0; i < cnt; i += 2) {
            uint32_t packed = b[2 + i / 2];
            int lo = (int)(packed & 15u), hi = (int)((packed >> 4) & 15u);
            y[i] = (float)(lo < 8 ? lo : lo - 16) * d;
            if (i + 1 < cnt) y[i + 1] = (float)(hi < 8 ? hi : hi - 16) * d;
        }
    } else {
        const int64_t sbi = e0 / 256;
        const int j = (int)((e0 % 256) / 32);
        if (type == SMX_TYPE_Q6_K) {   // GgufModelLoader.cs:849-917, 16-element sub-blocks
            const uint8_t *b = src + sbi * 210;
            const float d = rd_half_exact(b + 208);
            for (int i = 0; i < cnt; i++) {
                int v = j * 32 + i;
                float sc = d * (float)(int8_t)b[192 + v / 16];
                uint32_t low4 = (v % 2 == 0) ? (b[v / 2] & 15u) : ((b[v / 2] >> 4) & 15u);
                uint32_t high2 = (b[128 + v / 4] >> ((v % 4) * 2)) & 3u;
                int q = (int)(low4 | (high2 << 4));
                y[i] = sc * (float)(q - 32);
            }
        } else {
            const int bytes = type == SMX_TYPE_Q4_K ? 144 : 176;
            const uint8_t *b = src + sbi * bytes;
            const float d = rd_half_exact(b), dmin = rd_half_exact(b + 2);
            uint32_t sc6[8], mn6[8];
            unpack_k_scales(b + 4, sc6, mn6);
            const float sc = d * (float)sc6[j];
            const float m = dmin * (float)mn6[j];
            if (type == SMX_TYPE_Q4_K) {   // GgufModelLoader.cs:657-741
                // The reference loop runs i < count/2, so an odd tail element stays zero.
                for (int i = 0; i < cnt; i++) y[i] = 0.0f;
                for (int i = 0; i < cnt / 2; i++) {
                    uint32_t packed = b[16 + j * 16 + i];
                    float t0 = sc * (float)(packed & 15u);
                    y[2 * i] = t0 - m;
                    if (2 * i + 1 < cnt) {
                        float t1 = sc * (float)((packed >> 4) & 15u);
                        y[2 * i + 1] = t1 - m;
                    }
                }
            } else {   // Q5_K, GgufModelLoader.cs:748-840
                for (int i = 0; i < cnt; i++) {
                    int v = j * 32 + i;
                    uint32_t hb = ((b[16 + v / 8] >> (v % 8)) & 1u) << 4;
                    uint32_t low4 = (v % 2 == 0) ? (b[48 + v / 2] & 15u) : ((b[48 + v / 2] >> 4) & 15u);
                    int q = (int)(hb | low4) - 16;
                    float t = sc * (float)q;
                    y[i] = t - m;
                }
            }
        }
    }
}

// ---- encoders: one thread per block --------------------------------------------------------
__device__ __forceinline__ float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

__device__ float block_maxabs(const float *x, int n)
{
    float m = 0.0f;
    for (int i = 0; i < n; i++) { float a = fabsf(x[i]); if (a > m) m = a; }
    return m;
}

__device__ void st16(uint8_t *p, uint32_t h) { p[0] = (uint8_t)h; p[1] = (uint8_t)(h >> 8); }

__device__ void pack_k_scales(const int *sc, const int *mn, uint8_t *s)
{
    uint64_t a = 0, b = 0;
    for (int j = 0; j < 8; j++) {
        a |= (uint64_t)(sc[j] & 63) << (6 * j);
        b |= (uint64_t)(mn[j] & 63) << (6 * j);
    }
    for (int i = 0; i < 6; i++) { s[i] = (uint8_t)(a >> (8 * i)); s[6 + i] = (uint8_t)(b >> (8 * i)); }
}

__device__ void enc_q8_0(const float *x, uint8_t *b)
{
    float maxAbs = block_maxabs(x, 32);
    float scale = maxAbs > 0.0f ? maxAbs / 127.0f : 1.0f;
    float inv = 1.0f / scale;
    st16(b, f2h_rne(scale));
    for (int i = 0; i < 32; i++) {
        float t = x[i] * inv;
        b[2 + i] = (uint8_t)(int8_t)(int)rintf(clampf(t, -127.0f, 127.0f));
    }
}

__device__ void enc_q4_0(const float *x, uint8_t *b)
{
    float maxAbs = block_maxabs(x, 32);
    float scale = maxAbs > 0.0f ? maxAbs / 7.0f : 1.0f;
    float inv = 1.0f / scale;
    st16(b, f2h_rne(scale));
    for (int i = 0; i < 16; i++) {
        float t0 = x[2 * i] * inv, t1 = x[2 * i + 1] * inv;
        int c0 = (int)rintf(clampf(t0, -8.0f, 7.0f));
        int c1 = (int)rintf(clampf(t1, -8.0f, 7.0f));
        b[2 + i] = (uint8_t)((c0 & 0xF) | ((c1 & 0xF) << 4));
    }
}

// Q8Tensor.Quantize / Q4Tensor.Quantize (Q8Tensor.cs:72-128, Q4Tensor.cs:75-134) as written, fp32
// scale kept, at 32-element blocks: the SMQ upload layout (fp32 scale, then the codes).
__device__ void enc_smq_q8(const float *x, uint8_t *b)
{
    float maxAbs = block_maxabs(x, 32);
    float scale = maxAbs > 0.0f ? maxAbs / 127.0f : 1.0f;
    float inv = 1.0f / scale;
    const uint32_t u = __float_as_uint(scale);
    for (int i = 0; i < 4; i++) b[i] = (uint8_t)(u >> (8 * i));
    for (int i = 0; i < 32; i++) {
        float t = x[i] * inv;
        b[4 + i] = (uint8_t)(int8_t)(int)rintf(clampf(t, -127.0f, 127.0f));
    }
}

__device__ void enc_smq_q4(const float *x, uint8_t *b)
{
    float maxAbs = block_maxabs(x, 32);
    float scale = maxAbs > 0.0f ? maxAbs / 7.0f : 1.0f;
    float inv = 1.0f / scale;
    const uint32_t u = __float_as_uint(scale);
    for (int i = 0; i < 4; i++) b[i] = (uint8_t)(u >> (8 * i));
    for (int i = 0; i < 16; i++) {
        float t0 = x[2 * i] * inv, t1 = x[2 * i + 1] * inv;
        int c0 = (int)rintf(clampf(t0, -8.0f, 7.0f));
        int c1 = (int)rintf(clampf(t1, -8.0f, 7.0f));
        b[4 + i] = (uint8_t)((c0 & 0xF) | ((c1 & 0xF) << 4));
    }
}

__device__ void enc_q4_k(const float *x, uint8_t *b)
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
    uint32_t d16 = f2h_rne(maxs / 63.0f), m16 = f2h_rne(maxm / 63.0f);
    float df = h2f_exact(d16), mf = h2f_exact(m16);
    int ls[8], lm[8];
    for (int j = 0; j < 8; j++) {
        ls[j] = df > 0.0f ? (int)clampf(rintf(scl[j] / df), 0.0f, 63.0f) : 0;
        lm[j] = mf > 0.0f ? (int)clampf(rintf(mnv[j] / mf), 0.0f, 63.0f) : 0;
    }
    st16(b, d16);
    st16(b + 2, m16);
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

__device__ void enc_q5_k(const float *x, uint8_t *b)
{
    float scl[8], maxs = 0.0f;
    for (int j = 0; j < 8; j++) {
        scl[j] = block_maxabs(x + 32 * j, 32) / 15.0f;
        if (scl[j] > maxs) maxs = scl[j];
    }
    uint32_t d16 = f2h_rne(maxs / 63.0f);
    float df = h2f_exact(d16);
    int ls[8], lm[8];
    for (int j = 0; j < 8; j++) {
        ls[j] = df > 0.0f ? (int)clampf(rintf(scl[j] / df), 0.0f, 63.0f) : 0;
        lm[j] = 0;
    }
    for (int i = 0; i < 176; i++) b[i] = 0;
    st16(b, d16);
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

__device__ void enc_q6_k(const float *x, uint8_t *b)
{
    float scl[16], maxs = 0.0f;
    for (int j = 0; j < 16; j++) {
        scl[j] = block_maxabs(x + 16 * j, 16) / 31.0f;
        if (scl[j] > maxs) maxs = scl[j];
    }
    uint32_t d16 = f2h_rne(maxs / 127.0f);
    float df = h2f_exact(d16);
    for (int i = 0; i < 210; i++) b[i] = 0;
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
    st16(b + 208, d16);
}

__global__ void k_quantize(int type, const float *__restrict__ x, int64_t nblocks,
                           uint8_t *__restrict__ out)
{
    const int64_t blk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= nblocks) return;
    switch (type) {
    case SMX_TYPE_Q8_0: enc_q8_0(x + blk * 32, out + blk * 34); break;
    case SMX_TYPE_Q4_0: enc_q4_0(x + blk * 32, out + blk * 18); break;
    case SMX_TYPE_Q4_K: enc_q4_k(x + blk * 256, out + blk * 144); break;
    case SMX_TYPE_Q5_K: enc_q5_k(x + blk * 256, out + blk * 176); break;
    case SMX_TYPE_Q6_K: enc_q6_k(x + blk * 256, out + blk * 210); break;
    case SMX_TYPE_SMQ_Q8: enc_smq_q8(x + blk * 32, out + blk * 36); break;
    case SMX_TYPE_SMQ_Q4: enc_smq_q4(x + blk * 32, out + blk * 20); break;
    case SMX_TYPE_F16: {
        uint32_t h = f2h_rne(x[blk]);
        out[2 * blk] = (uint8_t)h;
        out[2 * blk + 1] = (uint8_t)(h >> 8);
        break;
    }
    default: break;
    }
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void k_fill_normal(uint64_t seed, int64_t n, float std, float *__restrict__ out)
{
    const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // pair index
    if (2 * p >= n) return;
    uint64_t r = splitmix64(seed * 0xD1B54A32D192ED03ull + (uint64_t)p);
    float u1 = (float)((r >> 40) + 1) * 5.9604644775390625e-08f;
    float u2 = (float)(r & 0xFFFFFFu) * 5.9604644775390625e-08f;
    float rad = sqrtf(-2.0f * logf(u1));
    float th = 6.283185307179586f * u2;
    out[2 * p] = std * (rad * cosf(th));
    if (2 * p + 1 < n) out[2 * p + 1] = std * (rad * sinf(th));
}

// ---- GGUF -> backend layout ------------------------------------------------------------------
__global__ void k_repack(int fmt, const uint8_t *__restrict__ src, int64_t rows, int nb,
                         uint8_t *__restrict__ dq, uint16_t *__restrict__ dd, int64_t row_off,
                         int64_t row_step)
{
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * nb) return;
    const int64_t r = idx / nb;
    const int b = (int)(idx % nb);
    const int64_t dr = row_off + r * row_step;
    const int gb = fmt_gguf_bytes(fmt), mb = fmt_main_bytes(fmt);
    const uint8_t *s = src + idx * gb;
    uint8_t *o = dq + (dr * nb + b) * mb;
    if (fmt == FMT_F16 || fmt == FMT_F32) {
        for (int i = 0; i < mb; i++) o[i] = s[i];
    } else if (fmt == FMT_SQ8 || fmt == FMT_SQ4) {
        ((uint32_t *)dd)[dr * nb + b] = (uint32_t)s[0] | ((uint32_t)s[1] << 8) | ((uint32_t)s[2] << 16) |
                                        ((uint32_t)s[3] << 24);
        for (int i = 0; i < mb; i++) o[i] = s[4 + i];
    } else if (fmt == FMT_Q4_0 || fmt == FMT_Q8_0) {
        dd[dr * nb + b] = (uint16_t)ld_u16(s);
        for (int i = 0; i < mb; i++) o[i] = s[2 + i];
    } else if (fmt == FMT_Q4_K) {
        for (int i = 0; i < 144; i++) o[i] = s[i];
    } else if (fmt == FMT_Q5_K) {
        for (int i = 0; i < 16; i++) o[i] = s[i];
        for (int i = 0; i < 128; i++) o[48 + i] = s[48 + i];
        const uint8_t *qh = s + 16;
        for (int j = 0; j < 8; j++)
            for (int k = 0; k < 4; k++) {
                uint32_t byte = 0;
                for (int g = 0; g < 4; g++)
                    for (int p = 0; p < 2; p++) {
                        int v = 32 * j + 8 * g + 2 * k + p;
                        byte |= ((qh[v >> 3] >> (v & 7)) & 1u) << (2 * g + p);
                    }
                o[16 + 4 * j + k] = (uint8_t)byte;
            }
    } else {   // Q6_K
        for (int i = 0; i < 128; i++) o[i] = s[i];
        for (int i = 0; i < 16; i++) o[192 + i] = s[192 + i];
        dd[dr * nb + b] = (uint16_t)ld_u16(s + 208);
        const uint8_t *qh = s + 128;
        for (int c = 0; c < 8; c++)
            for (int p = 0; p < 2; p++)
                for (int k = 0; k < 4; k++) {
                    uint32_t byte = 0;
                    for (int g = 0; g < 4; g++) {
                        int v = 32 * c + 8 * g + 2 * k + p;
                        byte |= ((qh[v >> 2] >> (2 * (v & 3))) & 3u) << (2 * g);
                    }
                    o[128 + 8 * c + 4 * p + k] = (uint8_t)byte;
                }
    }
}

template <int F>
__global__ void k_dequant_smx(WView w, int64_t row0, int64_t nrows, float *__restrict__ out)
{
    const int nch = (int)(w.cols / 32);
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= nrows * nch) return;
    const int64_t r = idx / nch;
    const int c = (int)(idx % nch);
    float y[32];
    decode_chunk_exact<F>(w, row0 + r, c, y);
    float *o = out + r * w.cols + (int64_t)c * 32;
#pragma unroll
    for (int i = 0; i < 32; i += 4) *(float4 *)(o + i) = make_float4(y[i], y[i + 1], y[i + 2], y[i + 3]);
}

unsigned grid_for(int64_t n) { return (unsigned)((n + kThreads - 1) / kThreads); }

}  // namespace

int fmt_from_type(int type)
{
    switch (type) {
    case SMX_TYPE_Q4_0: return FMT_Q4_0;
    case SMX_TYPE_Q8_0: return FMT_Q8_0;
    case SMX_TYPE_Q4_K: return FMT_Q4_K;
    case SMX_TYPE_Q5_K: return FMT_Q5_K;
    case SMX_TYPE_Q6_K: return FMT_Q6_K;
    case SMX_TYPE_F16: return FMT_F16;
    case SMX_TYPE_F32: return FMT_F32;
    case SMX_TYPE_SMQ_Q8: return FMT_SQ8;
    case SMX_TYPE_SMQ_Q4: return FMT_SQ4;
    default: return -1;
    }
}

hipError_t launch_dequant_gguf(int type, const void *blocks, int64_t n, float *out, hipStream_t s)
{
    const int64_t chunks = (n + 31) / 32;
    if (chunks == 0) return hipSuccess;
    hipLaunchKernelGGL(k_dequant_gguf, dim3(grid_for(chunks)), dim3(kThreads), 0, s, type,
                       (const uint8_t *)blocks, n, out);
    return hipGetLastError();
}

hipError_t launch_quantize_gguf(int type, const float *x, int64_t n, void *blocks, hipStream_t s)
{
    const int be = type == SMX_TYPE_F16 ? 1
                 : (type == SMX_TYPE_Q8_0 || type == SMX_TYPE_Q4_0 || type == SMX_TYPE_SMQ_Q8 || type == SMX_TYPE_SMQ_Q4)
                     ? 32 : 256;
    const int64_t nblocks = n / be;
    if (nblocks == 0) return hipSuccess;
    hipLaunchKernelGGL(k_quantize, dim3(grid_for(nblocks)), dim3(kThreads), 0, s, type, x, nblocks,
                       (uint8_t *)blocks);
    return hipGetLastError();
}

hipError_t launch_fill_normal(uint64_t seed, int64_t n, float std, float *out, hipStream_t s)
{
    const int64_t pairs = (n + 1) / 2;
    if (pairs == 0) return hipSuccess;
    hipLaunchKernelGGL(k_fill_normal, dim3(grid_for(pairs)), dim3(kThreads), 0, s, seed, n, std, out);
    return hipGetLastError();
}

hipError_t launch_repack(int fmt, const uint8_t *gguf, int64_t rows, int64_t cols, uint8_t *dst_q,
                         uint16_t *dst_d, int64_t dst_rows, int64_t row_off, int64_t row_step,
                         hipStream_t s)
{
    (void)dst_rows;
    const int nb = (int)(cols / fmt_block_elems(fmt));
    const int64_t total = rows * nb;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_repack, dim3(grid_for(total)), dim3(kThreads), 0, s, fmt, gguf, rows, nb,
                       dst_q, dst_d, row_off, row_step);
    return hipGetLastError();
}

hipError_t launch_dequant_smx(const WView &w, int64_t row0, int64_t nrows, float *out, hipStream_t s)
{
    const int f = w.fmt;
    const int64_t total = nrows * (w.cols / 32);
    if (total == 0) return hipSuccess;
    const dim3 g(grid_for(total)), b(kThreads);
    switch (f) {
    case FMT_Q4_0: hipLaunchKernelGGL(k_dequant_smx<FMT_Q4_0>, g, b, 0, s, w, row0, nrows, out); break;
    case FMT_Q8_0: hipLaunchKernelGGL(k_dequant_smx<FMT_Q8_0>, g, b, 0, s, w, row0, nrows, out); break;
    case FMT_Q4_K: hipLaunchKernelGGL(k_dequant_smx<FMT_Q4_K>, g, b, 0, s, w, row0, nrows, out); break;
    case FMT_Q5_K: hipLaunchKernelGGL(k_dequant_smx<FMT_Q5_K>, g, b, 0, s, w, row0, nrows, out); break;
    case FMT_Q6_K: hipLaunchKernelGGL(k_dequant_smx<FMT_Q6_K>, g, b, 0, s, w, row0, nrows, out); break;
    case FMT_F16: hipLaunchKernelGGL(k_dequant_smx<FMT_F16>, g, b, 0, s, w, row0, nrows, out); break;
    case FMT_F32: hipLaunchKernelGGL(k_dequant_smx<FMT_F32>, g, b, 0, s, w, row0, nrows, out); break;
    case FMT_SQ8: hipLaunchKernelGGL(k_dequant_smx<FMT_SQ8>, g, b, 0, s, w, row0, nrows, out); break;
    case FMT_SQ4: hipLaunchKernelGGL(k_dequant_smx<FMT_SQ4>, g, b, 0, s, w, row0, nrows, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace smx
