// smx_device.h -- device helpers shared by the HIP kernels of libsmx.so.
//
// Everything here is compiled with -ffp-contract=off: a*b+c is never fused unless written
// as __builtin_fmaf, so the scalar formulas below round exactly like the C# reference.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace smx {

// fp16 bits -> fp32, bit-identical to GgufModelLoader.HalfToFloat (GgufModelLoader.cs:919-956)
// for every pattern: subnormals are exact (m * 2^-24 is a normal fp32), Inf/NaN keep payload.
__device__ __forceinline__ float h2f_exact(uint32_t h)
{
    uint32_t sign = (h >> 15) & 1u, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    uint32_t r = e == 0x1F ? ((sign << 31) | 0x7F800000u | (m << 13))
                           : ((sign << 31) | ((e + 112u) << 23) | (m << 13));
    return __uint_as_float(r);
}

// fp16 bits -> fp32 with the hardware conversion (exact for all finite values; used in the
// GEMV hot loops where NaN payloads do not matter).
__device__ __forceinline__ float h2f(uint32_t h)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// fp32 -> fp16 bits, round to nearest even; the same integer routine as the oracle's
// smxo_float_to_half, so CPU and GPU encoders store identical scales.
__device__ __forceinline__ uint32_t f2h_rne(float f)
{
    uint32_t x = __float_as_uint(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u);
    if (ax >= 0x47800000u) return sign | 0x7C00u;
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return sign;
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;
        uint32_t hm = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (hm & 1u))) hm++;
        return sign | hm;
    }
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7FFFFFu) >> 13);
    uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return sign | h;
}

// MathUtils.FastExp (src/SmallMind.Core/Utilities/MathUtils.cs:20-32).
__device__ __forceinline__ float fastexp(float x)
{
    x = fmaxf(-87.3f, fminf(x, 88.7f));
    float x2 = x * x;
    float h = x * 0.5f, q = x2 * 0.08333333f;
    float num = 1.0f + h;
    num = num + q;
    float den = 1.0f - h;
    den = den + q;
    return num / den;
}

// ActivationOps.GELU vector form (src/SmallMind.Core/Simd/ActivationOps.cs:262-276).
__device__ __forceinline__ float gelu_pade(float x)
{
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
    return hx * (1.0f + th);
}

// ActivationOps.FusedSiLUMul element (ActivationOps.cs:565-580, FastSigmoid :304-309).
__device__ __forceinline__ float silu_mul(float x, float u)
{
    float c = fmaxf(-20.0f, fminf(x, 20.0f));
    float sig = 1.0f / (1.0f + expf(-c));
    float silu = x * sig;
    return silu * u;
}

// Thread index passed through an opaque instruction, so the compiler treats values derived from
// it as lane-varying and recomputes lane-dependent addresses where they are used instead of
// hoisting them and keeping them live (which spills registers in the larger kernels).  Costs
// one v_mov per call site.
__device__ __forceinline__ int opaque_tid()
{
    int t;
    asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"((int)threadIdx.x));
    return t;
}
__device__ __forceinline__ int lane_id() { return opaque_tid() & 63; }
// Wave index within the workgroup as a scalar (wave-uniform) value, so task indices and row
// addresses derived from it live in SGPRs.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// Load of a wave-uniform value through the scalar data cache (s_load, counted by lgkmcnt), so
// it neither waits for nor delays the vector-memory loads in flight.  The address must be the
// same in every lane, and the data must not be written by the running kernel before the load.
template <typename T>
__device__ __forceinline__ T ld_uniform(const T *p)
{
    return *(const __attribute__((address_space(4))) T *)p;
}

// ---- wave64 / block reductions ------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Sum over each row of 16 lanes with DPP (quad swaps, half-row and row mirrors): no LDS
// traffic.  Every lane of a row ends with the same bits (each step adds a commuted pair).
// All 64 lanes must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_sum(float v)
{
    v += dpp_mov<0xB1>(v);    // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v);   // row_half_mirror
    v += dpp_mov<0x140>(v);   // row_mirror
    return v;
}
// Wave-uniform total of v over all 64 lanes (all lanes active): row sums, then the four row
// totals read into scalars and added in a fixed order.
__device__ __forceinline__ float wave_sum_uniform(float v)
{
    v = row16_sum(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

// bf16 bits of f, rounded to nearest even.
__device__ __forceinline__ uint32_t bf16_rne(float f)
{
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Activation parts of the matrix-core GEMM (k_qgemm): f = hi + mid + lo, three bf16 values each
// rounded to nearest even, stored for element k = 32 s + 8 g + 4 h + q of token m at
// Xp[m / 16][s][part][g][m % 16] dword q, half h (2 bytes each; nsb = sub-blocks per token).
__device__ __forceinline__ void xp_store(uint8_t *xp, int nsb, int m, int k, float f)
{
    const uint32_t hi = bf16_rne(f);
    const float r1 = f - __uint_as_float(hi << 16);
    const uint32_t mid = bf16_rne(r1);
    const float r2 = r1 - __uint_as_float(mid << 16);
    const int s = k >> 5, e = k & 31, g = e >> 3, j = e & 7;
    uint8_t *b = xp + ((size_t)(m >> 4) * nsb + s) * 3 * 1024 + (g * 16 + (m & 15)) * 16 + (j & 3) * 4 + (j >> 2) * 2;
    *(uint16_t *)b = (uint16_t)hi;
    *(uint16_t *)(b + 1024) = (uint16_t)mid;
    *(uint16_t *)(b + 2048) = (uint16_t)bf16_rne(r2);
}

// v_permlane32_swap_b32 (gfx950): lanes 32..63 of `a` trade places with lanes 0..31 of `b`;
// .x is the new `a`, .y the new `b`.
__device__ __forceinline__ float2 swap32(float a, float b)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// v_permlane16_swap_b32 (gfx950): the odd 16-lane rows of `a` trade places with the even rows
// of `b`; .x is the new `a`, .y the new `b`.
__device__ __forceinline__ float2 swap16(float a, float b)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Totals of R per-lane partials (R = 2 or 4) over the wave, transposed: row r's total ends up
// in every lane of block r (lanes [r*64/R, (r+1)*64/R)).  The lane swaps fold the halves so
// that each add combines two rows' partials at once, then each 16-lane row is summed with
// DPP: 2 + R/2 swaps and adds plus 4 DPP adds, against 11 instructions per row for separate
// wave sums.  All lanes must be active.
template <int R>
__device__ __forceinline__ float wave_totals_t(const float *acc)
{
    static_assert(R == 2 || R == 4, "two or four rows per wave");
    float c;
    if constexpr (R == 4) {
        const float2 p0 = swap32(acc[0], acc[2]);   // lanes 0..31: row 0, 32..63: row 2
        const float2 p1 = swap32(acc[1], acc[3]);   // lanes 0..31: row 1, 32..63: row 3
        const float2 q = swap16(p0.x + p0.y, p1.x + p1.y);
        c = q.x + q.y;                              // 16-lane rows: rows 0, 1, 2, 3
    } else {
        const float2 p = swap32(acc[0], acc[1]);    // lanes 0..31: row 0, 32..63: row 1
        const float b = p.x + p.y;
        const float2 q = swap16(b, b);
        c = q.x + q.y;
    }
    return row16_sum(c);
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Block-wide sum for blockDim.x == 64 * nw (nw <= 16); red must hold 16 floats.  Every
// thread receives the same value; the order of additions is fixed, so every block that sums
// the same data gets the same bits.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float *red)
{
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < NW; i++) t += red[i];
    return t;
}

template <int NW>
__device__ __forceinline__ float block_max(float v, float *red)
{
    v = wave_max(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = red[0];
#pragma unroll
    for (int i = 1; i < NW; i++) t = fmaxf(t, red[i]);
    return t;
}

__device__ __forceinline__ uint32_t ld_u32_unaligned(const uint8_t *p)
{
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p)
{
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8);
}

}  // namespace smx
