// k_gemv.hip -- fused dequantize-GEMV for Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K weights.
//
// y[r] = sum_k W[r][k] * x[k] for a row-major [rows][cols] weight in the backend layout
// (smx_internal.h).  Replaces Linear.ForwardFP32 / IWeightTensor.MatMul for batch-1 decode
// (NeuralNet.cs:145-298) and the fused C# kernels (MatMulF32Q8.cs, MatMulF32Q4.cs,
// FusedQ4KMatMul.cs, FusedQ6KMatMul.cs), computing y = x W^T as the GGUF loader path does.
//
// Work decomposition (one workgroup = 4 wave64s):
//   * the activation row is staged once per workgroup in LDS, optionally normalised on the way
//     (RMSNorm / LayerNorm prologue, so the norm never makes its own HBM round trip);
//   * a wave owns R consecutive weight rows; lane l walks the 32-element chunks l, l+64, ...
//     of all R rows, so the 32 activations it needs are read from LDS once per R rows;
//   * each chunk is one 16 B (or 32 B) vector load per row; codes are unpacked with and/shift
//     into bytes and converted with the byte-select converts, block scales are factored out
//     of the 32-term sum (sum (sc*q - m) x = sc * sum q x - m * sum x, using per-16-element
//     activation sums precomputed in LDS);
//   * the R partial sums are reduce-scattered across the wave (R values cost 2R-1 shuffles
//     instead of 6R), then one lane applies the epilogue.
#include "smx_device.h"
#include "smx_formats.h"

namespace smx {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

// Byte b of v as fp32 in one v_cvt_f32_ubyte<b> (the compiler would otherwise re-extract each
// nibble with a bit-field extract first).
__device__ __forceinline__ float ub(uint32_t v, int b)
{
    float r;
    switch (b) {
    case 0: asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v)); break;
    case 1: asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v)); break;
    case 2: asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v)); break;
    default: asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v)); break;
    }
    return r;
}

__device__ __forceinline__ float xget(const float4 *xv, int e)
{
    const float4 v = xv[e >> 2];
    switch (e & 3) {
    case 0: return v.x;
    case 1: return v.y;
    case 2: return v.z;
    default: return v.w;
    }
}

// sum over the 8 elements 8g..8g+7 of a chunk whose codes sit in two dwords: `lo` holds the
// even elements (8g, 8g+2, 8g+4, 8g+6) in bytes 0..3, `hi` the odd ones.
__device__ __forceinline__ float dot8(uint32_t lo, uint32_t hi, const float4 *xv, int g, float acc)
{
    const int e = 8 * g;
    acc = __builtin_fmaf(ub(lo, 0), xget(xv, e + 0), acc);
    acc = __builtin_fmaf(ub(hi, 0), xget(xv, e + 1), acc);
    acc = __builtin_fmaf(ub(lo, 1), xget(xv, e + 2), acc);
    acc = __builtin_fmaf(ub(hi, 1), xget(xv, e + 3), acc);
    acc = __builtin_fmaf(ub(lo, 2), xget(xv, e + 4), acc);
    acc = __builtin_fmaf(ub(hi, 2), xget(xv, e + 5), acc);
    acc = __builtin_fmaf(ub(lo, 3), xget(xv, e + 6), acc);
    acc = __builtin_fmaf(ub(hi, 3), xget(xv, e + 7), acc);
    return acc;
}

template <int S>
__device__ __forceinline__ uint32_t shl(uint32_t v)
{
    if constexpr (S >= 0) return v << S;
    else return v >> (-S);
}

// ---- per-format raw chunk data + dot ------------------------------------------------------
template <int F> struct Raw;

template <> struct Raw<FMT_Q4_0> {
    uint4 q; uint32_t d;
    __device__ __forceinline__ void load(const WView &w, int64_t row, int c)
    {
        const int64_t blk = row * w.nb + c;
        q = *(const uint4 *)(w.q + blk * 16);
        d = w.d[blk];
    }
    __device__ __forceinline__ float dot(const float4 *xv, float xa, float xb, int) const
    {
        const uint32_t v[4] = {q.x ^ 0x88888888u, q.y ^ 0x88888888u, q.z ^ 0x88888888u, q.w ^ 0x88888888u};
        float s0 = 0.0f, s1 = 0.0f;
        s0 = dot8(v[0] & 0x0F0F0F0Fu, (v[0] >> 4) & 0x0F0F0F0Fu, xv, 0, s0);
        s1 = dot8(v[1] & 0x0F0F0F0Fu, (v[1] >> 4) & 0x0F0F0F0Fu, xv, 1, s1);
        s0 = dot8(v[2] & 0x0F0F0F0Fu, (v[2] >> 4) & 0x0F0F0F0Fu, xv, 2, s0);
        s1 = dot8(v[3] & 0x0F0F0F0Fu, (v[3] >> 4) & 0x0F0F0F0Fu, xv, 3, s1);
        // codes are (n ^ 8) = value + 8 (Q4Tensor.DecodeNibble two's complement)
        return h2f(d) * ((s0 + s1) - 8.0f * (xa + xb));
    }
};

template <> struct Raw<FMT_Q8_0> {
    uint4 q0, q1; uint32_t d;
    __device__ __forceinline__ void load(const WView &w, int64_t row, int c)
    {
        const int64_t blk = row * w.nb + c;
        const uint4 *p = (const uint4 *)(w.q + blk * 32);
        q0 = p[0];
        q1 = p[1];
        d = w.d[blk];
    }
    __device__ __forceinline__ float dot(const float4 *xv, float, float, int) const
    {
        const uint32_t v[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        float s[2] = {0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < 8; k++)
#pragma unroll
            for (int b = 0; b < 4; b++)
                s[k & 1] = __builtin_fmaf((float)(int8_t)(v[k] >> (8 * b)), xget(xv, 4 * k + b), s[k & 1]);
        return h2f(d) * (s[0] + s[1]);
    }
};

template <> struct Raw<FMT_Q4_K> {
    uint4 h, q;
    __device__ __forceinline__ void load(const WView &w, int64_t row, int c)
    {
        const uint8_t *base = w.q + (row * w.nb + (c >> 3)) * 144;
        h = *(const uint4 *)base;
        q = *(const uint4 *)(base + 16 + 16 * (c & 7));
    }
    __device__ __forceinline__ float dot(const float4 *xv, float xa, float xb, int c) const
    {
        const int j = c & 7;
        const float sc = h2f(h.x & 0xFFFFu) * (float)kq_scale6(h.y, h.z, h.w, j, 0);
        const float m = h2f(h.x >> 16) * (float)kq_scale6(h.y, h.z, h.w, j, 1);
        const uint32_t v[4] = {q.x, q.y, q.z, q.w};
        float s0 = 0.0f, s1 = 0.0f;
        s0 = dot8(v[0] & 0x0F0F0F0Fu, (v[0] >> 4) & 0x0F0F0F0Fu, xv, 0, s0);
        s1 = dot8(v[1] & 0x0F0F0F0Fu, (v[1] >> 4) & 0x0F0F0F0Fu, xv, 1, s1);
        s0 = dot8(v[2] & 0x0F0F0F0Fu, (v[2] >> 4) & 0x0F0F0F0Fu, xv, 2, s0);
        s1 = dot8(v[3] & 0x0F0F0F0Fu, (v[3] >> 4) & 0x0F0F0F0Fu, xv, 3, s1);
        return __builtin_fmaf(sc, s0 + s1, -(m * (xa + xb)));
    }
};

template <> struct Raw<FMT_Q5_K> {
    uint4 h, q; uint32_t H;
    __device__ __forceinline__ void load(const WView &w, int64_t row, int c)
    {
        const uint8_t *base = w.q + (row * w.nb + (c >> 3)) * 176;
        const int j = c & 7;
        h = *(const uint4 *)base;
        H = *(const uint32_t *)(base + 16 + 4 * j);
        q = *(const uint4 *)(base + 48 + 16 * j);
    }
    __device__ __forceinline__ float dot(const float4 *xv, float xa, float xb, int c) const
    {
        const int j = c & 7;
        const float sc = h2f(h.x & 0xFFFFu) * (float)kq_scale6(h.y, h.z, h.w, j, 0);
        const float m = h2f(h.x >> 16) * (float)kq_scale6(h.y, h.z, h.w, j, 1);
        const uint32_t v[4] = {q.x, q.y, q.z, q.w};
        float s0 = 0.0f, s1 = 0.0f;
        // high bit of element 8g+2k+p sits at bit 8k + 2g + p of H -> move it to bit 8k + 4.
        s0 = dot8((v[0] & 0x0F0F0F0Fu) | (shl<4>(H) & 0x10101010u),
                  ((v[0] >> 4) & 0x0F0F0F0Fu) | (shl<3>(H) & 0x10101010u), xv, 0, s0);
        s1 = dot8((v[1] & 0x0F0F0F0Fu) | (shl<2>(H) & 0x10101010u),
                  ((v[1] >> 4) & 0x0F0F0F0Fu) | (shl<1>(H) & 0x10101010u), xv, 1, s1);
        s0 = dot8((v[2] & 0x0F0F0F0Fu) | (H & 0x10101010u),
                  ((v[2] >> 4) & 0x0F0F0F0Fu) | (shl<-1>(H) & 0x10101010u), xv, 2, s0);
        s1 = dot8((v[3] & 0x0F0F0F0Fu) | (shl<-2>(H) & 0x10101010u),
                  ((v[3] >> 4) & 0x0F0F0F0Fu) | (shl<-3>(H) & 0x10101010u), xv, 3, s1);
        const float xs = xa + xb;
        // y = sc*(q-16) - m  =>  sum y x = sc*(sum q x - 16 sum x) - m sum x
        return __builtin_fmaf(sc, (s0 + s1) - 16.0f * xs, -(m * xs));
    }
};

template <> struct Raw<FMT_Q6_K> {
    uint4 q; uint2 D; uint32_t scw, d;
    __device__ __forceinline__ void load(const WView &w, int64_t row, int c)
    {
        const int64_t sbi = row * w.nb + (c >> 3);
        const uint8_t *base = w.q + sbi * 208;
        const int cc = c & 7;
        q = *(const uint4 *)(base + 16 * cc);
        D = *(const uint2 *)(base + 128 + 8 * cc);
        scw = *(const uint16_t *)(base + 192 + 2 * cc);
        d = w.d[sbi];
    }
    __device__ __forceinline__ float dot(const float4 *xv, float xa, float xb, int) const
    {
        const uint32_t v[4] = {q.x, q.y, q.z, q.w};
        float sa = 0.0f, sb = 0.0f;
        // two high bits of element 8g+2k+p sit at bits 8k + 2g of D_p -> move to 8k + 4.
        sa = dot8((v[0] & 0x0F0F0F0Fu) | (shl<4>(D.x) & 0x30303030u),
                  ((v[0] >> 4) & 0x0F0F0F0Fu) | (shl<4>(D.y) & 0x30303030u), xv, 0, sa);
        sa = dot8((v[1] & 0x0F0F0F0Fu) | (shl<2>(D.x) & 0x30303030u),
                  ((v[1] >> 4) & 0x0F0F0F0Fu) | (shl<2>(D.y) & 0x30303030u), xv, 1, sa);
        sb = dot8((v[2] & 0x0F0F0F0Fu) | (D.x & 0x30303030u),
                  ((v[2] >> 4) & 0x0F0F0F0Fu) | (D.y & 0x30303030u), xv, 2, sb);
        sb = dot8((v[3] & 0x0F0F0F0Fu) | (shl<-2>(D.x) & 0x30303030u),
                  ((v[3] >> 4) & 0x0F0F0F0Fu) | (shl<-2>(D.y) & 0x30303030u), xv, 3, sb);
        const float df = h2f(d);
        const float sca = df * (float)(int8_t)(scw & 0xFFu);
        const float scb = df * (float)(int8_t)(scw >> 8);
        // y = (d*scale)*(q-32) per 16-element sub-block
        return __builtin_fmaf(sca, sa - 32.0f * xa, scb * (sb - 32.0f * xb));
    }
};

// ---- prologue: stage (normalised) activations in LDS ----------------------------------------
// LDS layout: xT[i][c] (float4, i = 0..7 parts of chunk c) so that lanes reading consecutive
// chunks hit consecutive 16 B words; xsA[c], xsB[c] = sums of elements 0..15 / 16..31.
__device__ __forceinline__ void stage_x(const GemvArgs &a, const float *__restrict__ x, int K,
                                        float *lds, float *red)
{
    const int nch = K / 32;
    float4 *xT = (float4 *)lds;
    float *xsA = lds + K, *xsB = xsA + nch;
    float scale = 1.0f, mean = 0.0f;
    if (a.pro == PRO_RMS) {
        float ss = 0.0f;
        for (int i = threadIdx.x; i < K; i += kThreads) { float v = x[i]; float p = v * v; ss += p; }
        ss = block_sum<kWaves>(ss, red);
        scale = 1.0f / sqrtf(ss / (float)K + a.eps);   // RMSNormOps.cs:114
    } else if (a.pro == PRO_LN) {
        float s = 0.0f;
        for (int i = threadIdx.x; i < K; i += kThreads) s += x[i];
        s = block_sum<kWaves>(s, red);
        mean = s / (float)K;                            // LayerNormOps.cs:92
        float sq = 0.0f;
        for (int i = threadIdx.x; i < K; i += kThreads) { float dd = x[i] - mean; float p = dd * dd; sq += p; }
        sq = block_sum<kWaves>(sq, red);
        scale = 1.0f / sqrtf(sq / (float)K + a.eps);    // LayerNormOps.cs:119
    }
    for (int i4 = threadIdx.x; i4 < K / 4; i4 += kThreads) {
        float4 v = ((const float4 *)x)[i4];
        if (a.pro == PRO_RMS) {
            const float4 g = ((const float4 *)a.gamma)[i4];
            v.x = g.x * (v.x * scale); v.y = g.y * (v.y * scale);
            v.z = g.z * (v.z * scale); v.w = g.w * (v.w * scale);
        } else if (a.pro == PRO_LN) {
            const float4 g = ((const float4 *)a.gamma)[i4];
            const float4 b = ((const float4 *)a.beta)[i4];
            v.x = __builtin_fmaf(g.x, (v.x - mean) * scale, b.x);
            v.y = __builtin_fmaf(g.y, (v.y - mean) * scale, b.y);
            v.z = __builtin_fmaf(g.z, (v.z - mean) * scale, b.z);
            v.w = __builtin_fmaf(g.w, (v.w - mean) * scale, b.w);
        }
        const int c = i4 >> 3, part = i4 & 7;
        xT[part * nch + c] = v;
    }
    __syncthreads();
    for (int c = threadIdx.x; c < nch; c += kThreads) {
        float sa = 0.0f, sb = 0.0f;
#pragma unroll
        for (int part = 0; part < 4; part++) {
            const float4 v = xT[part * nch + c];
            sa += (v.x + v.y) + (v.z + v.w);
            const float4 u = xT[(part + 4) * nch + c];
            sb += (u.x + u.y) + (u.z + u.w);
        }
        xsA[c] = sa;
        xsB[c] = sb;
    }
    __syncthreads();
}

// ---- epilogue ---------------------------------------------------------------------------------
__device__ __forceinline__ void rope_pair(float &v0, float &v1, int pair, int pos, const GemvArgs &a)
{
    const int half = a.head_dim / 2;
    const float c = a.rope_cos[(int64_t)pos * half + pair], s = a.rope_sin[(int64_t)pos * half + pair];
    const float x0 = v0, x1 = v1;
    const float t0 = x0 * c, t1 = x1 * s, t2 = x0 * s, t3 = x1 * c;
    v0 = t0 - t1;   // RotaryEmbedding.cs:115-116
    v1 = t2 + t3;
}

template <int R>
__device__ __forceinline__ void epilogue(const GemvArgs &a, const float *t, int64_t row0, int64_t N,
                                         int my)
{
    float *out = a.out + (int64_t)my * a.out_stride;
    float v[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        v[r] = t[r];
        if (a.bias && row0 + r < N) v[r] = v[r] + a.bias[row0 + r];
    }
    switch (a.epi) {
    case EPI_STORE:
#pragma unroll
        for (int r = 0; r < R; r++) if (row0 + r < N) out[row0 + r] = v[r];
        break;
    case EPI_RESID: {
        const float *res = a.resid + (int64_t)my * a.out_stride;
#pragma unroll
        for (int r = 0; r < R; r++) if (row0 + r < N) out[row0 + r] = res[row0 + r] + v[r];
        break;
    }
    case EPI_GELU:
#pragma unroll
        for (int r = 0; r < R; r++) if (row0 + r < N) out[row0 + r] = gelu_pade(v[r]);
        break;
    case EPI_SILU:
#pragma unroll
        for (int r = 0; r < R; r += 2)
            if (row0 + r + 1 < N) out[(row0 + r) / 2] = silu_mul(v[r], v[r + 1]);
        break;
    case EPI_QKV: {
        const int pos = *a.pos;
        const int d = a.d_model, kv = a.kv_dim, hd = a.head_dim;
#pragma unroll
        for (int r = 0; r < R; r += 2) {
            const int64_t row = row0 + r;
            if (row + 1 >= N) break;
            float v0 = v[r], v1 = v[r + 1];
            if (row < d) {
                if (a.use_rope) rope_pair(v0, v1, (int)(row % hd) / 2, pos, a);
                out[row] = v0;
                out[row + 1] = v1;
            } else if (row < d + kv) {
                const int64_t kr = row - d;
                if (a.use_rope) rope_pair(v0, v1, (int)(kr % hd) / 2, pos, a);
                float *dst = a.k_cache + ((kr / hd) * a.ctx_stride + pos) * hd + (kr % hd);
                dst[0] = v0;
                dst[1] = v1;
            } else {
                const int64_t vr = row - d - kv;
                float *dst = a.v_cache + ((vr / hd) * a.ctx_stride + pos) * hd + (vr % hd);
                dst[0] = v0;
                dst[1] = v1;
            }
        }
        break;
    }
    default: break;
    }
}

template <int F, int R>
__global__ __launch_bounds__(kThreads) void k_gemv(GemvArgs a)
{
    extern __shared__ float4 smem4[];
    float *lds = (float *)smem4;
    __shared__ float red[16];
    const int K = (int)a.w.cols;
    const int nch = K / 32;
    const int my = blockIdx.y;
    stage_x(a, a.x + (int64_t)my * a.x_stride, K, lds, red);

    const float4 *xT = (const float4 *)lds;
    const float *xsA = lds + K, *xsB = xsA + nch;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t N = a.w.rows;
    const int64_t row0 = ((int64_t)blockIdx.x * kWaves + wave) * R;
    if (row0 >= N) return;

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

    for (int c = lane; c < nch; c += 64) {
        Raw<F> raw[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int64_t row = row0 + r < N ? row0 + r : N - 1;
            raw[r].load(a.w, row, c);
        }
        float4 xv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) xv[i] = xT[i * nch + c];
        const float xa = xsA[c], xb = xsB[c];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] += raw[r].dot(xv, xa, xb, c);
    }

    // reduce-scatter: after the first log2(R) steps lane group r (64/R lanes) holds row r.
    float k;
    if constexpr (R == 4) {
        const bool up = lane & 32;
        float s0 = up ? acc[0] : acc[2], s1 = up ? acc[1] : acc[3];
        float k0 = up ? acc[2] : acc[0], k1 = up ? acc[3] : acc[1];
        k0 += __shfl_xor(s0, 32, 64);
        k1 += __shfl_xor(s1, 32, 64);
        const bool u16 = lane & 16;
        float s = u16 ? k0 : k1;
        k = u16 ? k1 : k0;
        k += __shfl_xor(s, 16, 64);
    } else if constexpr (R == 2) {
        const bool up = lane & 32;
        float s = up ? acc[0] : acc[1];
        k = up ? acc[1] : acc[0];
        k += __shfl_xor(s, 32, 64);
        k += __shfl_xor(k, 16, 64);
    } else {
        k = acc[0];
        k += __shfl_xor(k, 32, 64);
        k += __shfl_xor(k, 16, 64);
    }
    k += __shfl_xor(k, 8, 64);
    k += __shfl_xor(k, 4, 64);
    k += __shfl_xor(k, 2, 64);
    k += __shfl_xor(k, 1, 64);
    float t[R];
#pragma unroll
    for (int r = 0; r < R; r++) t[r] = __shfl(k, r * (64 / R), 64);
    if (lane == 0) epilogue<R>(a, t, row0, N, my);
}

template <int F, int R>
hipError_t launch_fr(const GemvArgs &a, int m, hipStream_t s)
{
    const int64_t waves = (a.w.rows + R - 1) / R;
    const dim3 grid((unsigned)((waves + kWaves - 1) / kWaves), (unsigned)m);
    const size_t lds = (size_t)a.w.cols * 4 + (size_t)(a.w.cols / 32) * 8;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void *)k_gemv<F, R>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((k_gemv<F, R>), grid, dim3(kThreads), lds, s, a);
    return hipGetLastError();
}

template <int F>
hipError_t launch_f(const GemvArgs &a, int m, hipStream_t s)
{
    // Pairs of rows must share a wave for the SwiGLU and RoPE epilogues, so R >= 2.
    if (a.w.rows >= 8192) return launch_fr<F, 4>(a, m, s);
    return launch_fr<F, 2>(a, m, s);
}

}  // namespace

hipError_t launch_gemv(const GemvArgs &a, int m, hipStream_t s)
{
    switch (a.w.fmt) {
    case FMT_Q4_0: return launch_f<FMT_Q4_0>(a, m, s);
    case FMT_Q8_0: return launch_f<FMT_Q8_0>(a, m, s);
    case FMT_Q4_K: return launch_f<FMT_Q4_K>(a, m, s);
    case FMT_Q5_K: return launch_f<FMT_Q5_K>(a, m, s);
    case FMT_Q6_K: return launch_f<FMT_Q6_K>(a, m, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace smx
