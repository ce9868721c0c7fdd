// smx_formats.h -- exact (reference-rounding) decoders for the backend weight layouts.
//
// decode_chunk_exact<F>() produces the 32 fp32 values of chunk c (elements 32c..32c+31) of a
// row, rounding exactly as GgufModelLoader.Convert*Tensor does (GgufModelLoader.cs:464-917):
// one fp32 multiply for Q8_0/Q4_0/Q6_K element values, multiply-then-subtract for Q4_K/Q5_K.
#pragma once

#include "smx_device.h"
#include "smx_internal.h"

namespace smx {

// Six-bit scale (sel = 0) or min (sel = 1) j of a Q4_K/Q5_K header, read from the 12-byte field
// as one little-endian bit stream per half (GgufModelLoader.cs:688-705).
__device__ __forceinline__ uint32_t kq_scale6(uint32_t h1, uint32_t h2, uint32_t h3, int j, int sel)
{
    // h1 = bytes 4..7, h2 = bytes 8..11, h3 = bytes 12..15 of the super-block: the scales sit
    // at bits 6j, the mins at bits 48 + 6j of the 96-bit stream h3:h2:h1.  One funnel shift
    // (v_alignbit_b32) of the two words holding the field extracts it without 64-bit values.
    const uint32_t b = 6u * (uint32_t)j + (sel ? 48u : 0u);
    const uint32_t wd = b >> 5;
    const uint32_t lo = wd == 0 ? h1 : wd == 1 ? h2 : h3;
    const uint32_t hi = wd == 0 ? h2 : wd == 1 ? h3 : 0u;
    return __builtin_amdgcn_alignbit(hi, lo, b & 31u) & 63u;
}

template <int F>
__device__ __forceinline__ void decode_chunk_exact(const WView &w, int64_t row, int c, float *y)
{
    if constexpr (F == FMT_F16 || F == FMT_F32) {   // ConvertF16Tensor / F32 (GgufModelLoader.cs:438-462)
        const uint8_t *q = w.q + (row * w.nb + c) * fmt_main_bytes(F);
#pragma unroll
        for (int i = 0; i < 32; i++)
            y[i] = F == FMT_F16 ? h2f_exact(((const uint16_t *)q)[i]) : ((const float *)q)[i];
    } else if constexpr (F == FMT_SQ8 || F == FMT_SQ4) {
        // Q8Tensor.Dequantize / Q4Tensor.Dequantize (Q8Tensor.cs:130-160, Q4Tensor.cs:150-178):
        // code * scale, one fp32 multiply
        const int64_t blk = row * w.nb + c;
        const float d = __uint_as_float(((const uint32_t *)w.d)[blk]);
        const uint8_t *q = w.q + blk * fmt_main_bytes(F);
        if constexpr (F == FMT_SQ4) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t b = q[i];
                int lo = (int)(b & 15u), hi = (int)(b >> 4);
                lo = lo < 8 ? lo : lo - 16;   // Q4Tensor.DecodeNibble (Q4Tensor.cs:140-143)
                hi = hi < 8 ? hi : hi - 16;
                y[2 * i] = (float)lo * d;
                y[2 * i + 1] = (float)hi * d;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 32; i++) y[i] = (float)(int8_t)q[i] * d;
        }
    } else if constexpr (F == FMT_Q4_0 || F == FMT_Q8_0) {
        const int64_t blk = row * w.nb + c;
        const float d = h2f_exact(w.d[blk]);
        const uint8_t *q = w.q + blk * fmt_main_bytes(F);
        if constexpr (F == FMT_Q4_0) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                uint32_t b = q[i];
                int lo = (int)(b & 15u), hi = (int)(b >> 4);
                lo = lo < 8 ? lo : lo - 16;   // Q4Tensor.DecodeNibble (Q4Tensor.cs:140-143)
                hi = hi < 8 ? hi : hi - 16;
                y[2 * i] = (float)lo * d;
                y[2 * i + 1] = (float)hi * d;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 32; i++) y[i] = (float)(int8_t)q[i] * d;
        }
    } else if constexpr (F == FMT_Q4_K || F == FMT_Q5_K) {
        const int sb = c >> 3, j = c & 7;
        const uint8_t *base = w.q + (row * w.nb + sb) * fmt_main_bytes(F);
        const uint32_t *hw = (const uint32_t *)base;
        const float d = h2f_exact(hw[0] & 0xFFFFu), dmin = h2f_exact(hw[0] >> 16);
        const float sc = d * (float)kq_scale6(hw[1], hw[2], hw[3], j, 0);
        const float m = dmin * (float)kq_scale6(hw[1], hw[2], hw[3], j, 1);
        if constexpr (F == FMT_Q4_K) {
            const uint8_t *qs = base + 16 + 16 * j;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                uint32_t b = qs[i];
                float t0 = sc * (float)(b & 15u);
                float t1 = sc * (float)(b >> 4);
                y[2 * i] = t0 - m;
                y[2 * i + 1] = t1 - m;
            }
        } else {
            const uint32_t H = *(const uint32_t *)(base + 16 + 4 * j);
            const uint8_t *ql = base + 48 + 16 * j;
#pragma unroll
            for (int e = 0; e < 32; e++) {
                const int g = e >> 3, k = (e & 7) >> 1, p = e & 1;
                uint32_t hb = (H >> (8 * k + 2 * g + p)) & 1u;
                uint32_t low = (ql[e >> 1] >> (4 * (e & 1))) & 15u;
                int q = (int)((hb << 4) | low) - 16;
                float t = sc * (float)q;
                y[e] = t - m;
            }
        }
    } else {   // Q6_K
        const int sb = c >> 3, cc = c & 7;
        const uint8_t *base = w.q + (row * w.nb + sb) * 208;
        const float d = h2f_exact(w.d[row * w.nb + sb]);
        const uint32_t D0 = *(const uint32_t *)(base + 128 + 8 * cc);
        const uint32_t D1 = *(const uint32_t *)(base + 128 + 8 * cc + 4);
        const float sca = d * (float)(int8_t)base[192 + 2 * cc];
        const float scb = d * (float)(int8_t)base[192 + 2 * cc + 1];
        const uint8_t *ql = base + 16 * cc;
#pragma unroll
        for (int e = 0; e < 32; e++) {
            const int g = e >> 3, k = (e & 7) >> 1, p = e & 1;
            uint32_t hi2 = ((p ? D1 : D0) >> (8 * k + 2 * g)) & 3u;
            uint32_t low = (ql[e >> 1] >> (4 * (e & 1))) & 15u;
            int q = (int)(low | (hi2 << 4));
            y[e] = (e < 16 ? sca : scb) * (float)(q - 32);
        }
    }
}

}  // namespace smx
