// smx_gemv.h -- the per-wave fused dequantize-GEMV used by k_gemv.hip.
//
// gemv_wave<F, R>(a, row0, my) computes rows row0..row0+R-1 of y = W x for activation row
// `my`, applies the prologue (none / RMSNorm / LayerNorm of x) and the epilogue.  It uses no
// LDS and no workgroup barrier, so any wave can run any row group.
#pragma once

#include "smx_device.h"
#include "smx_formats.h"
#include "smx_internal.h"

namespace smx {

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

// dot8 for 4-bit codes (every byte of lo / hi below 16), scaled by 2^-9: a byte 0000qqqq read
// as an OCP E4M3 value is exactly q * 2^-9 (subnormal for q < 8, exponent 1 above), so one
// v_cvt_pk_f32_fp8 turns two codes into floats.  The products and partial sums are the
// dot8 ones times 2^-9 exactly (a power-of-two scaling commutes with fp32 rounding away from
// the subnormal range), in the same order; callers fold 512 into the block scale.
__device__ __forceinline__ float dot8_nib(uint32_t lo, uint32_t hi, const float4 *xv, int g, float acc)
{
    typedef float f2 __attribute__((ext_vector_type(2)));
    const int e = 8 * g;
    const f2 l01 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false), l23 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
    const f2 h01 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false), h23 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
    acc = __builtin_fmaf(l01.x, xget(xv, e + 0), acc);
    acc = __builtin_fmaf(h01.x, xget(xv, e + 1), acc);
    acc = __builtin_fmaf(l01.y, xget(xv, e + 2), acc);
    acc = __builtin_fmaf(h01.y, xget(xv, e + 3), acc);
    acc = __builtin_fmaf(l23.x, xget(xv, e + 4), acc);
    acc = __builtin_fmaf(h23.x, xget(xv, e + 5), acc);
    acc = __builtin_fmaf(l23.y, xget(xv, e + 6), acc);
    acc = __builtin_fmaf(h23.y, xget(xv, e + 7), acc);
    return acc;
}

template <int S>
__device__ __forceinline__ uint32_t shl(uint32_t v)
{
    if constexpr (S >= 0) return v << S;
    else return v >> (-S);
}

// Weight loads.  NT = true sets the non-temporal hint (the `nt` bit of global_load): the
// bytes of a large matrix are read once per launch and not again until the same matrix comes
// round in the next decode step, hundreds of megabytes later, so they should not displace what
// the next kernels reuse (the KV cache rows, activations, matrices kept in the MALL).  Matrices
// the runtime keeps resident in the 256 MB MALL (WView::cache) are read with plain loads.
template <bool NT>
__device__ __forceinline__ uint4 ldw4(const uint8_t *p)
{
    if constexpr (NT) {
        typedef unsigned u4 __attribute__((ext_vector_type(4)));
        const u4 v = __builtin_nontemporal_load((const u4 *)p);
        return make_uint4(v.x, v.y, v.z, v.w);
    } else {
        return *(const uint4 *)p;
    }
}
template <bool NT>
__device__ __forceinline__ uint2 ldw2(const uint8_t *p)
{
    if constexpr (NT) {
        typedef unsigned u2 __attribute__((ext_vector_type(2)));
        const u2 v = __builtin_nontemporal_load((const u2 *)p);
        return make_uint2(v.x, v.y);
    } else {
        return *(const uint2 *)p;
    }
}
template <bool NT>
__device__ __forceinline__ uint32_t ldw1(const void *p)
{
    if constexpr (NT) return __builtin_nontemporal_load((const uint32_t *)p);
    else return *(const uint32_t *)p;
}
template <bool NT>
__device__ __forceinline__ uint32_t ldwh(const void *p)
{
    if constexpr (NT) return __builtin_nontemporal_load((const uint16_t *)p);
    else return *(const uint16_t *)p;
}
template <bool NT>
__device__ __forceinline__ float4 ldwf4(const uint8_t *p)
{
    const uint4 v = ldw4<NT>(p);
    return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}

// ---- per-format raw chunk data + dot ------------------------------------------------------
template <int F> struct Raw;

template <> struct Raw<FMT_Q4_0> {
    uint4 q; uint32_t d;
    __device__ __forceinline__ void load(const WView &w, int64_t row, int c)
    {
        const int64_t blk = row * w.nb + c;
        q = ldw4<true>(w.q + blk * 16);
        d = ldwh<true>(w.d + blk);
    }
    // 32-bit offsets (the whole matrix is below 4 GiB): `row_blk` = row * blocks per row.
    template <bool NT = true> __device__ __forceinline__ void load32(const WView &w, uint32_t row_blk, int c)
    {
        const uint32_t blk = row_blk + (uint32_t)c;
        q = ldw4<NT>(w.q + blk * 16u);
        d = ldwh<NT>(w.d + blk);
    }
    __device__ __forceinline__ float dot(const float4 *xv, float xa, float xb, int) const
    {
        const uint32_t v[4] = {q.x ^ 0x88888888u, q.y ^ 0x88888888u, q.z ^ 0x88888888u, q.w ^ 0x88888888u};
        float s0 = 0.0f, s1 = 0.0f;
        s0 = dot8_nib(v[0] & 0x0F0F0F0Fu, (v[0] >> 4) & 0x0F0F0F0Fu, xv, 0, s0);
        s1 = dot8_nib(v[1] & 0x0F0F0F0Fu, (v[1] >> 4) & 0x0F0F0F0Fu, xv, 1, s1);
        s0 = dot8_nib(v[2] & 0x0F0F0F0Fu, (v[2] >> 4) & 0x0F0F0F0Fu, xv, 2, s0);
        s1 = dot8_nib(v[3] & 0x0F0F0F0Fu, (v[3] >> 4) & 0x0F0F0F0Fu, xv, 3, s1);
        // codes are (n ^ 8) = value + 8 (Q4Tensor.DecodeNibble two's complement); sums are
        // scaled by 2^-9 (dot8_nib), the scale by 512
        return (h2f(d) * 512.0f) * ((s0 + s1) - 0.015625f * (xa + xb));
    }
};

template <> struct Raw<FMT_Q8_0> {
    uint4 q0, q1; uint32_t d;
    __device__ __forceinline__ void load(const WView &w, int64_t row, int c)
    {
        const int64_t blk = row * w.nb + c;
        q0 = ldw4<true>(w.q + blk * 32);
        q1 = ldw4<true>(w.q + blk * 32 + 16);
        d = ldwh<true>(w.d + blk);
    }
    template <bool NT = true> __device__ __forceinline__ void load32(const WView &w, uint32_t row_blk, int c)
    {
        const uint32_t blk = row_blk + (uint32_t)c;
        q0 = ldw4<NT>(w.q + blk * 32u);
        q1 = ldw4<NT>(w.q + blk * 32u + 16u);
        d = ldwh<NT>(w.d + blk);
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
        h = ldw4<true>(base);
        q = ldw4<true>(base + 16 + 16 * (c & 7));
    }
    template <bool NT = true> __device__ __forceinline__ void load32(const WView &w, uint32_t row_blk, int c)
    {
        const uint32_t off = (row_blk + ((uint32_t)c >> 3)) * 144u;
        h = ldw4<NT>(w.q + off);
        q = ldw4<NT>(w.q + off + 16u + 16u * ((uint32_t)c & 7u));
    }
    __device__ __forceinline__ float dot(const float4 *xv, float xa, float xb, int c) const
    {
        const int j = c & 7;
        const float sc = h2f(h.x & 0xFFFFu) * (float)kq_scale6(h.y, h.z, h.w, j, 0);
        const float m = h2f(h.x >> 16) * (float)kq_scale6(h.y, h.z, h.w, j, 1);
        const uint32_t v[4] = {q.x, q.y, q.z, q.w};
        float s0 = 0.0f, s1 = 0.0f;
        s0 = dot8_nib(v[0] & 0x0F0F0F0Fu, (v[0] >> 4) & 0x0F0F0F0Fu, xv, 0, s0);
        s1 = dot8_nib(v[1] & 0x0F0F0F0Fu, (v[1] >> 4) & 0x0F0F0F0Fu, xv, 1, s1);
        s0 = dot8_nib(v[2] & 0x0F0F0F0Fu, (v[2] >> 4) & 0x0F0F0F0Fu, xv, 2, s0);
        s1 = dot8_nib(v[3] & 0x0F0F0F0Fu, (v[3] >> 4) & 0x0F0F0F0Fu, xv, 3, s1);
        return __builtin_fmaf(sc * 512.0f, s0 + s1, -(m * (xa + xb)));   // sums scaled by 2^-9
    }
};

template <> struct Raw<FMT_Q5_K> {
    uint4 h, q; uint32_t H;
    __device__ __forceinline__ void load(const WView &w, int64_t row, int c)
    {
        const uint8_t *base = w.q + (row * w.nb + (c >> 3)) * 176;
        const int j = c & 7;
        h = ldw4<true>(base);
        H = ldw1<true>(base + 16 + 4 * j);
        q = ldw4<true>(base + 48 + 16 * j);
    }
    template <bool NT = true> __device__ __forceinline__ void load32(const WView &w, uint32_t row_blk, int c)
    {
        const uint32_t off = (row_blk + ((uint32_t)c >> 3)) * 176u, j = (uint32_t)c & 7u;
        h = ldw4<NT>(w.q + off);
        H = ldw1<NT>(w.q + off + 16u + 4u * j);
        q = ldw4<NT>(w.q + off + 48u + 16u * j);
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
        q = ldw4<true>(base + 16 * cc);
        D = ldw2<true>(base + 128 + 8 * cc);
        scw = ldwh<true>(base + 192 + 2 * cc);
        d = ldwh<true>(w.d + sbi);
    }
    template <bool NT = true> __device__ __forceinline__ void load32(const WView &w, uint32_t row_blk, int c)
    {
        const uint32_t sb = row_blk + ((uint32_t)c >> 3), off = sb * 208u, cc = (uint32_t)c & 7u;
        q = ldw4<NT>(w.q + off + 16u * cc);
        D = ldw2<NT>(w.q + off + 128u + 8u * cc);
        scw = ldwh<NT>(w.q + off + 192u + 2u * cc);
        d = ldwh<NT>(w.d + sb);
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

// F16 / F32 rows (unquantized GGUF matrices): a chunk is 32 values; fp16 converts exactly.
template <> struct Raw<FMT_F16> {
    uint4 v[4];
    __device__ __forceinline__ void load(const WView &w, int64_t row, int c)
    {
        const uint8_t *p = w.q + (row * w.nb + c) * 64;
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = ldw4<true>(p + 16 * i);
    }
    template <bool NT = true> __device__ __forceinline__ void load32(const WView &w, uint32_t row_blk, int c)
    {
        const uint8_t *p = w.q + (row_blk + (uint32_t)c) * 64u;
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = ldw4<NT>(p + 16 * i);
    }
    __device__ __forceinline__ float dot(const float4 *xv, float, float, int) const
    {
        const uint32_t u[16] = {v[0].x, v[0].y, v[0].z, v[0].w, v[1].x, v[1].y, v[1].z, v[1].w,
                                v[2].x, v[2].y, v[2].z, v[2].w, v[3].x, v[3].y, v[3].z, v[3].w};
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            s0 = __builtin_fmaf(h2f(u[k] & 0xFFFFu), xget(xv, 2 * k), s0);
            s1 = __builtin_fmaf(h2f(u[k] >> 16), xget(xv, 2 * k + 1), s1);
        }
        return s0 + s1;
    }
};

template <> struct Raw<FMT_F32> {
    float4 v[8];
    __device__ __forceinline__ void load(const WView &w, int64_t row, int c)
    {
        const uint8_t *p = w.q + (row * w.nb + c) * 128;
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = ldwf4<true>(p + 16 * i);
    }
    template <bool NT = true> __device__ __forceinline__ void load32(const WView &w, uint32_t row_blk, int c)
    {
        const uint8_t *p = w.q + (row_blk + (uint32_t)c) * 128u;
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = ldwf4<NT>(p + 16 * i);
    }
    __device__ __forceinline__ float dot(const float4 *xv, float, float, int) const
    {
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            s0 = __builtin_fmaf(v[i].x, xv[i].x, s0);
            s1 = __builtin_fmaf(v[i].y, xv[i].y, s1);
            s0 = __builtin_fmaf(v[i].z, xv[i].z, s0);
            s1 = __builtin_fmaf(v[i].w, xv[i].w, s1);
        }
        return s0 + s1;
    }
};

// SMQ blocks (Q8Tensor / Q4Tensor): the Q8_0 / Q4_0 codes with an fp32 scale per 32 elements
// (the d stream read as 32-bit words).
template <> struct Raw<FMT_SQ8> {
    Raw<FMT_Q8_0> b;
    __device__ __forceinline__ void load(const WView &w, int64_t row, int c)
    {
        const int64_t blk = row * w.nb + c;
        b.q0 = ldw4<true>(w.q + blk * 32);
        b.q1 = ldw4<true>(w.q + blk * 32 + 16);
        b.d = ldw1<true>((const uint32_t *)w.d + blk);
    }
    template <bool NT = true> __device__ __forceinline__ void load32(const WView &w, uint32_t row_blk, int c)
    {
        const uint32_t blk = row_blk + (uint32_t)c;
        b.q0 = ldw4<NT>(w.q + blk * 32u);
        b.q1 = ldw4<NT>(w.q + blk * 32u + 16u);
        b.d = ldw1<NT>((const uint32_t *)w.d + blk);
    }
    __device__ __forceinline__ float dot(const float4 *xv, float, float, int) const
    {
        const uint32_t v[8] = {b.q0.x, b.q0.y, b.q0.z, b.q0.w, b.q1.x, b.q1.y, b.q1.z, b.q1.w};
        float s[2] = {0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < 8; k++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                s[k & 1] = __builtin_fmaf((float)(int8_t)(v[k] >> (8 * j)), xget(xv, 4 * k + j), s[k & 1]);
        return __uint_as_float(b.d) * (s[0] + s[1]);
    }
};

template <> struct Raw<FMT_SQ4> {
    uint4 q; uint32_t d;
    __device__ __forceinline__ void load(const WView &w, int64_t row, int c)
    {
        const int64_t blk = row * w.nb + c;
        q = ldw4<true>(w.q + blk * 16);
        d = ldw1<true>((const uint32_t *)w.d + blk);
    }
    template <bool NT = true> __device__ __forceinline__ void load32(const WView &w, uint32_t row_blk, int c)
    {
        const uint32_t blk = row_blk + (uint32_t)c;
        q = ldw4<NT>(w.q + blk * 16u);
        d = ldw1<NT>((const uint32_t *)w.d + blk);
    }
    __device__ __forceinline__ float dot(const float4 *xv, float xa, float xb, int) const
    {
        // as Q4_0: codes n ^ 8 = value + 8, sums scaled by 2^-9 (dot8_nib), the scale by 512
        const uint32_t v[4] = {q.x ^ 0x88888888u, q.y ^ 0x88888888u, q.z ^ 0x88888888u, q.w ^ 0x88888888u};
        float s0 = 0.0f, s1 = 0.0f;
        s0 = dot8_nib(v[0] & 0x0F0F0F0Fu, (v[0] >> 4) & 0x0F0F0F0Fu, xv, 0, s0);
        s1 = dot8_nib(v[1] & 0x0F0F0F0Fu, (v[1] >> 4) & 0x0F0F0F0Fu, xv, 1, s1);
        s0 = dot8_nib(v[2] & 0x0F0F0F0Fu, (v[2] >> 4) & 0x0F0F0F0Fu, xv, 2, s0);
        s1 = dot8_nib(v[3] & 0x0F0F0F0Fu, (v[3] >> 4) & 0x0F0F0F0Fu, xv, 3, s1);
        return (__uint_as_float(d) * 512.0f) * ((s0 + s1) - 0.015625f * (xa + xb));
    }
};

// ---- prologue: per-wave norm statistics --------------------------------------------------
struct NormStat {
    float scale, mean;
};

// RMSNorm: scale = 1/sqrt(sum x^2 / K + eps) (RMSNormOps.cs:114); LayerNorm: mean = sum x / K,
// scale = 1/sqrt(sum (x-mean)^2 / K + eps) (LayerNormOps.cs:92-119).  Computed by the whole
// wave with a fixed order, so every wave obtains the same bits.
__device__ __forceinline__ NormStat wave_norm_stat(const GemvArgs &a, const float *__restrict__ x, int K)
{
    NormStat st{1.0f, 0.0f};
    const int lane = lane_id();
    if (a.pro == PRO_RMS) {
        float ss = 0.0f;
        for (int base = 0; base < K / 4; base += 64 * 8) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {   // eight independent loads in flight per lane
                const int i4 = base + u * 64 + lane;
                v[u] = i4 < K / 4 ? ((const float4 *)x)[i4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                float p;
                p = v[u].x * v[u].x; ss += p;
                p = v[u].y * v[u].y; ss += p;
                p = v[u].z * v[u].z; ss += p;
                p = v[u].w * v[u].w; ss += p;
            }
        }
        ss = wave_sum(ss);
        st.scale = 1.0f / sqrtf(ss / (float)K + a.eps);
    } else if (a.pro == PRO_LN) {
        float s = 0.0f;
        for (int i4 = lane; i4 < K / 4; i4 += 64) {
            const float4 v = ((const float4 *)x)[i4];
            s += v.x; s += v.y; s += v.z; s += v.w;
        }
        s = wave_sum(s);
        const float mean = s / (float)K;
        float sq = 0.0f;
        for (int i4 = lane; i4 < K / 4; i4 += 64) {
            const float4 v = ((const float4 *)x)[i4];
            float dd, p;
            dd = v.x - mean; p = dd * dd; sq += p;
            dd = v.y - mean; p = dd * dd; sq += p;
            dd = v.z - mean; p = dd * dd; sq += p;
            dd = v.w - mean; p = dd * dd; sq += p;
        }
        sq = wave_sum(sq);
        st.mean = mean;
        st.scale = 1.0f / sqrtf(sq / (float)K + a.eps);
    }
    return st;
}

// Loads activation chunk c (32 floats), normalised as the reference norms produce them.
__device__ __forceinline__ void load_x_chunk(const GemvArgs &a, const float *__restrict__ x, int c,
                                             const NormStat &st, float4 *xv)
{
    const float4 *xp = (const float4 *)(x + 32 * c);
#pragma unroll
    for (int i = 0; i < 8; i++) xv[i] = xp[i];
    if (a.pro == PRO_RMS) {
        const float4 *gp = (const float4 *)(a.gamma + 32 * c);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 g = gp[i];
            float4 &v = xv[i];
            v.x = g.x * (v.x * st.scale); v.y = g.y * (v.y * st.scale);     // RMSNormOps.cs:137-139
            v.z = g.z * (v.z * st.scale); v.w = g.w * (v.w * st.scale);
        }
    } else if (a.pro == PRO_LN) {
        const float4 *gp = (const float4 *)(a.gamma + 32 * c);
        const float4 *bp = (const float4 *)(a.beta + 32 * c);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 g = gp[i], b = bp[i];
            float4 &v = xv[i];
            v.x = __builtin_fmaf(g.x, (v.x - st.mean) * st.scale, b.x);   // LayerNormOps.cs:185
            v.y = __builtin_fmaf(g.y, (v.y - st.mean) * st.scale, b.y);
            v.z = __builtin_fmaf(g.z, (v.z - st.mean) * st.scale, b.z);
            v.w = __builtin_fmaf(g.w, (v.w - st.mean) * st.scale, b.w);
        }
    }
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
__device__ __forceinline__ void gemv_epilogue(const GemvArgs &a, const float *t, int64_t row0,
                                              int64_t N, int my)
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
        // Q -> out; K -> k_cache [kv_head][head_dim][ctx_stride] (dimension-major, so decode
        // attention reads consecutive positions); V -> v_cache [kv_head][ctx_stride][head_dim].
        const int pos = a.pos ? *a.pos : a.pos_val;
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
                float *dst = a.k_cache + kr * a.ctx_stride + pos;
                dst[0] = v0;
                dst[a.ctx_stride] = v1;
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

// Reduce-scatter of R per-lane partial sums: after log2(R) exchange steps lane group r
// (64/R lanes) holds row r; lane 0 then gathers the R totals.
template <int R>
__device__ __forceinline__ void wave_reduce_rows(const float *acc, float *t)
{
    const int lane = lane_id();
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
#pragma unroll
    for (int r = 0; r < R; r++) t[r] = __shfl(k, r * (64 / R), 64);
}

// Normalises the lane's 32 activations held in registers (one chunk per lane covers the whole
// vector), computing the statistic with one wave reduction.
__device__ __forceinline__ void norm_in_regs(const GemvArgs &a, float4 *xv, int c, bool active, int K)
{
    NormStat st{1.0f, 0.0f};
    if (a.pro == PRO_RMS) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float p;
            p = xv[i].x * xv[i].x; ss += p;
            p = xv[i].y * xv[i].y; ss += p;
            p = xv[i].z * xv[i].z; ss += p;
            p = xv[i].w * xv[i].w; ss += p;
        }
        ss = wave_sum(ss);
        st.scale = 1.0f / sqrtf(ss / (float)K + a.eps);
    } else {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) { s += xv[i].x; s += xv[i].y; s += xv[i].z; s += xv[i].w; }
        s = wave_sum(s);
        st.mean = s / (float)K;
        float sq = 0.0f;
        if (active) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float dd, p;
                dd = xv[i].x - st.mean; p = dd * dd; sq += p;
                dd = xv[i].y - st.mean; p = dd * dd; sq += p;
                dd = xv[i].z - st.mean; p = dd * dd; sq += p;
                dd = xv[i].w - st.mean; p = dd * dd; sq += p;
            }
        }
        sq = wave_sum(sq);
        st.scale = 1.0f / sqrtf(sq / (float)K + a.eps);
    }
    if (!active) return;
    if (a.pro == PRO_RMS) {
        const float4 *gp = (const float4 *)(a.gamma + 32 * c);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 g = gp[i];
            float4 &v = xv[i];
            v.x = g.x * (v.x * st.scale); v.y = g.y * (v.y * st.scale);     // RMSNormOps.cs:137-139
            v.z = g.z * (v.z * st.scale); v.w = g.w * (v.w * st.scale);
        }
    } else {
        const float4 *gp = (const float4 *)(a.gamma + 32 * c);
        const float4 *bp = (const float4 *)(a.beta + 32 * c);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 g = gp[i], b = bp[i];
            float4 &v = xv[i];
            v.x = __builtin_fmaf(g.x, (v.x - st.mean) * st.scale, b.x);   // LayerNormOps.cs:185
            v.y = __builtin_fmaf(g.y, (v.y - st.mean) * st.scale, b.y);
            v.z = __builtin_fmaf(g.z, (v.z - st.mean) * st.scale, b.z);
            v.w = __builtin_fmaf(g.w, (v.w - st.mean) * st.scale, b.w);
        }
    }
}

// Exact decode of chunk c of row `row` of any backend-layout weight (embedding gathers).
__device__ __forceinline__ void decode_chunk_any(const WView &w, int64_t row, int c, float *y)
{
    switch (w.fmt) {
    case FMT_Q4_0: decode_chunk_exact<FMT_Q4_0>(w, row, c, y); break;
    case FMT_Q8_0: decode_chunk_exact<FMT_Q8_0>(w, row, c, y); break;
    case FMT_Q4_K: decode_chunk_exact<FMT_Q4_K>(w, row, c, y); break;
    case FMT_Q5_K: decode_chunk_exact<FMT_Q5_K>(w, row, c, y); break;
    case FMT_Q6_K: decode_chunk_exact<FMT_Q6_K>(w, row, c, y); break;
    case FMT_F16: decode_chunk_exact<FMT_F16>(w, row, c, y); break;
    case FMT_F32: decode_chunk_exact<FMT_F32>(w, row, c, y); break;
    case FMT_SQ8: decode_chunk_exact<FMT_SQ8>(w, row, c, y); break;
    default: decode_chunk_exact<FMT_SQ4>(w, row, c, y); break;
    }
}

// Raw activation chunk c: from x, or the embedding row (+ learned position row) dequantised
// exactly as Embedding.Forward / AddPositionEmbeddings produce it (NeuralNet.cs:576-592,
// TransformerModel.cs:355-434).
__device__ __forceinline__ void fetch_x_chunk(const GemvArgs &a, const float *__restrict__ x, int c,
                                              float4 *xv)
{
    if (a.x_embed) {
        float v[32];
        decode_chunk_any(a.emb, a.emb_row, c, v);
        if (a.embp.q) {
            float p[32];
            decode_chunk_any(a.embp, a.embp_row, c, p);
#pragma unroll
            for (int i = 0; i < 32; i++) v[i] = v[i] + p[i];
        }
#pragma unroll
        for (int i = 0; i < 8; i++) xv[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    } else {
        const float4 *xp = (const float4 *)(x + 32 * c);
#pragma unroll
        for (int i = 0; i < 8; i++) xv[i] = xp[i];
    }
}

// Issues the weight loads of the first chunk of rows row0..row0+R-1 (lane l -> chunk l).
template <int F, int R>
__device__ __forceinline__ void gemv_prefetch(const WView &w, int64_t row0, Raw<F> *cur)
{
    const int lane = lane_id();
    if (lane < (int)(w.cols / 32)) {
#pragma unroll
        for (int r = 0; r < R; r++) cur[r].load(w, row0 + r < w.rows ? row0 + r : w.rows - 1, lane);
    }
}

// Row totals t[R] (valid in every lane) of rows row0..row0+R-1 for activation row `my`.
// `cur` holds the first chunk's weights when `loaded`, else they are loaded here first.
template <int F, int R>
__device__ __forceinline__ void gemv_compute(const GemvArgs &a, int64_t row0, int my, Raw<F> *cur,
                                             bool loaded, float *t)
{
    const int64_t N = a.w.rows;
    const int lane = lane_id();
    const int K = (int)a.w.cols;
    const int nch = K / 32;
    const float *x = a.x + (int64_t)my * a.x_stride;

    // 1. weight loads of the first chunk go out before the activation prologue.
    if (!loaded) gemv_prefetch<F, R>(a.w, row0, cur);

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    if (nch <= 64) {
        // One chunk per lane covers the whole activation vector: load it once, take the norm
        // statistic from registers, normalise in place.
        const bool active = lane < nch;
        float4 xv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) xv[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (active) fetch_x_chunk(a, x, lane, xv);
        if (a.pro != PRO_NONE) norm_in_regs(a, xv, lane, active, K);
        if (active) {
            float xa = 0.0f, xb = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                xa += (xv[i].x + xv[i].y) + (xv[i].z + xv[i].w);
                xb += (xv[i + 4].x + xv[i + 4].y) + (xv[i + 4].z + xv[i + 4].w);
            }
#pragma unroll
            for (int r = 0; r < R; r++) acc[r] = cur[r].dot(xv, xa, xb, lane);
        }
    } else {
        // 2. general K: norm statistic over the whole vector, then the chunk loop
        const NormStat st = wave_norm_stat(a, x, K);
        for (int c = lane; c < nch; c += 64) {
            if (c != lane) {
#pragma unroll
                for (int r = 0; r < R; r++) cur[r].load(a.w, row0 + r < N ? row0 + r : N - 1, c);
            }
            float4 xv[8];
            load_x_chunk(a, x, c, st, xv);
            float xa = 0.0f, xb = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                xa += (xv[i].x + xv[i].y) + (xv[i].z + xv[i].w);
                xb += (xv[i + 4].x + xv[i + 4].y) + (xv[i + 4].z + xv[i + 4].w);
            }
#pragma unroll
            for (int r = 0; r < R; r++) acc[r] += cur[r].dot(xv, xa, xb, c);
        }
    }
    wave_reduce_rows<R>(acc, t);
}

template <int F, int R>
__device__ __forceinline__ void gemv_wave(const GemvArgs &a, int64_t row0, int my)
{
    if (row0 >= a.w.rows) return;
    Raw<F> cur[R];
    float t[R];
    gemv_compute<F, R>(a, row0, my, cur, false, t);
    if ((threadIdx.x & 63) == 0) gemv_epilogue<R>(a, t, row0, a.w.rows, my);
}

}  // namespace smx
