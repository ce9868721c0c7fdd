// k_qgemm.hip -- quantized GEMM Y[M][N] = X[M][K] . W[N][K]^T on the bf16 matrix cores, for
// several activation rows at once (m >= 16: batched decode of many sessions, prefill chunks,
// IWeightTensor.MatMul with m > 1; NeuralNet.cs:145-298, MatMulF32Q8.cs:23-80).
//
// Exactness.  The MFMA inputs are bf16, the reference computes in fp32.  Both sides are made
// exact:
//   * weights enter as their integer codes, which bf16 represents exactly: 128 + q is built
//     with one and-or per pair of codes (bf16 0x4300 | q; Q8_0 codes go through a conversion),
//     and the block scales are applied to the fp32 result of each 32-element sub-block;
//   * activations enter as three bf16 parts, x = hi + mid + lo (8 + 8 + 8 significant bits),
//     so every product code x part is exact and the MFMA accumulates in fp32.
// A fourth product with an all-ones weight operand gives sum(x) per sub-block, which removes
// the +128 code offset and supplies the min term of Q4_K/Q5_K:
//   y += sc * (C - off * sum x) - m * sum x        (C = sum (128 + q) x over the sub-block).
//
// MFMA v_mfma_f32_16x16x32_bf16: A = activation parts (16 tokens x 32 k), B = weight codes
// (32 k x 16 weight rows), D[token][row].  Lane l supplies token / weight row l % 16 and the
// 8 k-values of group l / 16; D lane l holds tokens 4*(l/16)+0..3 of weight row l % 16.  The
// order of the 8 k-values inside a group is free as long as A and B agree; both use
// element order {0,4,1,5,2,6,3,7}, the order in which ((v >> 4p) & 0x000F000F) lays out two
// nibble codes per 32-bit pair.
//
// Work decomposition: a workgroup is 4 waves that split the sub-blocks of K between them
// (wave w takes sub-blocks w, w+4, ...) for RT row tiles of 16 weight rows and TT token tiles
// of 16 tokens; the four partial tiles are summed in LDS in a fixed order.
//
// Activation parts come from k_qprep: Xp[tt][s][p][g][t][8 bf16] (1 KB per (token tile,
// sub-block, part), lane l reads 16 bytes at l*16).
#include <algorithm>
#include <type_traits>

#include "smx_device.h"
#include "smx_formats.h"
#include "smx_internal.h"

namespace smx {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v)
{
    bf16x8 r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

__device__ __forceinline__ f32x4 mfma(uint4 a, uint4 b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// bf16 of an fp32 holding an integer of at most 8 significant bits (exact: the low 16 bits are 0)
__device__ __forceinline__ uint32_t pack_hi16(float lo, float hi)
{
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// (a & m) | (b & ~m) and the bf16 pair 128 + (e & m) per 16-bit half, one v_bitop3_b32 each
// (truth-table index = 4 * bit of the first operand + 2 * second + third)
__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t a, uint32_t b)
{
    return __builtin_amdgcn_bitop3_b32(a, m, b, 0xE2);   // m ? a : b
}
__device__ __forceinline__ uint32_t code_pair(uint32_t e, uint32_t m)
{
    return __builtin_amdgcn_bitop3_b32(e, m, 0x43004300u, 0xEA);   // (e & m) | 0x43004300
}

// ---- per-format weight operand --------------------------------------------------------------
// load(): the raw words of (row, sub-block s, k-group g) -- codes and scale fields -- issued
// one sub-block ahead of use; codes(): 4 bf16 pairs (element p, element p + 4) of the group's
// 8 codes; scale(): the per-(row, sub-block) scale terms.
struct RawQ {
    uint4 h;          // K-quant super-block header
    uint32_t v, v2;   // code bytes of the group
    uint32_t H, H2;   // high bits (Q5_K: qh'; Q6_K: D0, D1)
    uint32_t d;       // fp16 scale (Q4_0, Q8_0, Q6_K) / Q6_K int8 scale pair in the high half
};
struct Scl {
    float sc, sc2, m;   // Q6_K uses sc (first 16 elements) and sc2 (second 16)
};

template <int F> struct QW;

// Q4_0: block = sub-block of 32; codes n ^ 8 (value = code - 8): offset 128 + 8.
template <> struct QW<FMT_Q4_0> {
    static constexpr float kOff = 136.0f;
    static constexpr bool kHalves = false;
    __device__ __forceinline__ static RawQ load(const WView &w, uint32_t row, int s, int g)
    {
        RawQ r{};
        const uint32_t blk = row * (uint32_t)w.nb + (uint32_t)s;
        r.v = *(const uint32_t *)(w.q + blk * 16u + 4u * g);
        r.d = w.d[blk];
        return r;
    }
    __device__ __forceinline__ static uint4 codes(const RawQ &r, int)
    {
        const uint32_t v = r.v ^ 0x88888888u;
        return make_uint4((v & 0x000F000Fu) | 0x43004300u, ((v >> 4) & 0x000F000Fu) | 0x43004300u,
                          ((v >> 8) & 0x000F000Fu) | 0x43004300u, ((v >> 12) & 0x000F000Fu) | 0x43004300u);
    }
    __device__ __forceinline__ static Scl scale(const RawQ &r, int) { return {h2f(r.d), 0.0f, 0.0f}; }
};

// Q8_0: int8 codes; bf16(b ^ 0x80) = value + 128 (exact integers up to 255).
template <> struct QW<FMT_Q8_0> {
    static constexpr float kOff = 128.0f;
    static constexpr bool kHalves = false;
    __device__ __forceinline__ static RawQ load(const WView &w, uint32_t row, int s, int g)
    {
        RawQ r{};
        const uint32_t blk = row * (uint32_t)w.nb + (uint32_t)s;
        const uint2 v = *(const uint2 *)(w.q + blk * 32u + 8u * g);
        r.v = v.x;
        r.v2 = v.y;
        r.d = w.d[blk];
        return r;
    }
    __device__ __forceinline__ static uint4 codes(const RawQ &r, int)
    {
        const uint32_t a = r.v ^ 0x80808080u, b = r.v2 ^ 0x80808080u;
        // pair p = (element p, element p + 4) = (byte p of a, byte p of b)
        float a0, a1, a2, a3, b0, b1, b2, b3;
        asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(a0) : "v"(a));
        asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(a1) : "v"(a));
        asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(a2) : "v"(a));
        asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(a3) : "v"(a));
        asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(b0) : "v"(b));
        asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(b1) : "v"(b));
        asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(b2) : "v"(b));
        asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(b3) : "v"(b));
        return make_uint4(pack_hi16(a0, b0), pack_hi16(a1, b1), pack_hi16(a2, b2), pack_hi16(a3, b3));
    }
    __device__ __forceinline__ static Scl scale(const RawQ &r, int) { return {h2f(r.d), 0.0f, 0.0f}; }
};

// SMQ blocks (Q8Tensor / Q4Tensor): the Q8_0 / Q4_0 codes with an fp32 scale per 32 elements.
template <> struct QW<FMT_SQ8> {
    static constexpr float kOff = 128.0f;
    static constexpr bool kHalves = false;
    __device__ __forceinline__ static RawQ load(const WView &w, uint32_t row, int s, int g)
    {
        RawQ r{};
        const uint32_t blk = row * (uint32_t)w.nb + (uint32_t)s;
        const uint2 v = *(const uint2 *)(w.q + blk * 32u + 8u * g);
        r.v = v.x;
        r.v2 = v.y;
        r.d = ((const uint32_t *)w.d)[blk];
        return r;
    }
    __device__ __forceinline__ static uint4 codes(const RawQ &r, int g) { return QW<FMT_Q8_0>::codes(r, g); }
    __device__ __forceinline__ static Scl scale(const RawQ &r, int) { return {__uint_as_float(r.d), 0.0f, 0.0f}; }
};

template <> struct QW<FMT_SQ4> {
    static constexpr float kOff = 136.0f;
    static constexpr bool kHalves = false;
    __device__ __forceinline__ static RawQ load(const WView &w, uint32_t row, int s, int g)
    {
        RawQ r{};
        const uint32_t blk = row * (uint32_t)w.nb + (uint32_t)s;
        r.v = *(const uint32_t *)(w.q + blk * 16u + 4u * g);
        r.d = ((const uint32_t *)w.d)[blk];
        return r;
    }
    __device__ __forceinline__ static uint4 codes(const RawQ &r, int g) { return QW<FMT_Q4_0>::codes(r, g); }
    __device__ __forceinline__ static Scl scale(const RawQ &r, int) { return {__uint_as_float(r.d), 0.0f, 0.0f}; }
};

// Q4_K: sub-block s = qs bytes 16 + 16*(s % 8) of super-block s / 8.
template <> struct QW<FMT_Q4_K> {
    static constexpr float kOff = 128.0f;
    static constexpr bool kHalves = false;
    __device__ __forceinline__ static RawQ load(const WView &w, uint32_t row, int s, int g)
    {
        RawQ r{};
        const uint32_t base = (row * (uint32_t)w.nb + ((uint32_t)s >> 3)) * 144u;
        r.h = *(const uint4 *)(w.q + base);
        r.v = *(const uint32_t *)(w.q + base + 16u + 16u * ((uint32_t)s & 7u) + 4u * g);
        return r;
    }
    __device__ __forceinline__ static uint4 codes(const RawQ &r, int)
    {
        const uint32_t v = r.v;
        return make_uint4((v & 0x000F000Fu) | 0x43004300u, ((v >> 4) & 0x000F000Fu) | 0x43004300u,
                          ((v >> 8) & 0x000F000Fu) | 0x43004300u, ((v >> 12) & 0x000F000Fu) | 0x43004300u);
    }
    __device__ __forceinline__ static Scl scale(const RawQ &r, int s)
    {
        const int j = s & 7;
        return {h2f(r.h.x & 0xFFFFu) * (float)kq_scale6(r.h.y, r.h.z, r.h.w, j, 0), 0.0f,
                h2f(r.h.x >> 16) * (float)kq_scale6(r.h.y, r.h.z, r.h.w, j, 1)};
    }
};

// Q5_K: codes = ql nibble | high bit (bit-permuted qh'), value = q - 16: offset 128 + 16.
template <> struct QW<FMT_Q5_K> {
    static constexpr float kOff = 144.0f;
    static constexpr bool kHalves = false;
    __device__ __forceinline__ static RawQ load(const WView &w, uint32_t row, int s, int g)
    {
        RawQ r{};
        const uint32_t base = (row * (uint32_t)w.nb + ((uint32_t)s >> 3)) * 176u;
        const uint32_t j = (uint32_t)s & 7u;
        r.h = *(const uint4 *)(w.q + base);
        r.v = *(const uint32_t *)(w.q + base + 48u + 16u * j + 4u * g);
        r.H = *(const uint32_t *)(w.q + base + 16u + 4u * j);
        return r;
    }
    __device__ __forceinline__ static uint4 codes(const RawQ &r, int g)
    {
        // The high bit of element 8g + 2k + p sits at bit 8k + 2g + p of H, so hg = H >> 2g
        // holds it at bit 8k + p.  e0 / e1 = the 5-bit codes of the even / odd elements
        // 2k / 2k + 1 in bits 0-4 of byte k (bits 5-7 are don't-care); pair q = (element q,
        // element q + 4) is then bytes 0 and 2 of e_{q%2} >> 8(q/2).
        const uint32_t v = r.v, hg = r.H >> (2 * g);
        const uint32_t e0 = bfi(0x0F0F0F0Fu, v, hg << 4), e1 = bfi(0x0F0F0F0Fu, v >> 4, hg << 3);
        return make_uint4(code_pair(e0, 0x001F001Fu), code_pair(e1, 0x001F001Fu), code_pair(e0 >> 8, 0x001F001Fu),
                          code_pair(e1 >> 8, 0x001F001Fu));
    }
    __device__ __forceinline__ static Scl scale(const RawQ &r, int s)
    {
        const int j = s & 7;
        return {h2f(r.h.x & 0xFFFFu) * (float)kq_scale6(r.h.y, r.h.z, r.h.w, j, 0), 0.0f,
                h2f(r.h.x >> 16) * (float)kq_scale6(r.h.y, r.h.z, r.h.w, j, 1)};
    }
};

// Q6_K: 6-bit codes, value = q - 32: offset 128 + 32; two 16-element scales per sub-block.
template <> struct QW<FMT_Q6_K> {
    static constexpr float kOff = 160.0f;
    static constexpr bool kHalves = true;
    __device__ __forceinline__ static RawQ load(const WView &w, uint32_t row, int s, int g)
    {
        RawQ r{};
        const uint32_t sb = row * (uint32_t)w.nb + ((uint32_t)s >> 3);
        const uint32_t base = sb * 208u, cc = (uint32_t)s & 7u;
        r.v = *(const uint32_t *)(w.q + base + 16u * cc + 4u * g);
        const uint2 D = *(const uint2 *)(w.q + base + 128u + 8u * cc);
        r.H = D.x;
        r.H2 = D.y;
        r.d = (uint32_t)w.d[sb] | ((uint32_t)*(const uint16_t *)(w.q + base + 192u + 2u * cc) << 16);
        return r;
    }
    __device__ __forceinline__ static uint4 codes(const RawQ &r, int g)
    {
        // The two high bits of element 8g + 2k + p sit at bits 8k + 2g of D_p, so
        // dp = D_p >> 2g holds them at bits 8k, 8k + 1: e_p = the 6-bit codes of the elements
        // 2k + p in bits 0-5 of byte k, and pair q = bytes 0 and 2 of e_{q%2} >> 8(q/2).
        const uint32_t v = r.v;
        const uint32_t e0 = bfi(0x0F0F0F0Fu, v, (r.H >> (2 * g)) << 4);
        const uint32_t e1 = bfi(0x0F0F0F0Fu, v >> 4, (r.H2 >> (2 * g)) << 4);
        return make_uint4(code_pair(e0, 0x003F003Fu), code_pair(e1, 0x003F003Fu), code_pair(e0 >> 8, 0x003F003Fu),
                          code_pair(e1 >> 8, 0x003F003Fu));
    }
    __device__ __forceinline__ static Scl scale(const RawQ &r, int)
    {
        const float d = h2f(r.d & 0xFFFFu);
        return {d * (float)(int8_t)((r.d >> 16) & 0xFFu), d * (float)(int8_t)(r.d >> 24), 0.0f};
    }
};

constexpr uint4 kZero4 = {0u, 0u, 0u, 0u};

// acc + sc * (C - off * sum x) - m * sum x as two fused steps: acc + sc*C - (sc*off + m) * sum x
// (cs = sc * off + m precomputed per row and sub-block).
// Activation part p of (token tile tt, sub-block s) for this lane: a wave-uniform base plus the
// lane's 32-bit byte offset, so each load is one scalar-base instruction with no per-lane
// 64-bit address arithmetic.
__device__ __forceinline__ uint4 ld_part(const uint8_t *xp, int tt, int nsb, int s, int p, uint32_t lane16)
{
    const uint8_t *base = xp + (((size_t)tt * nsb + s) * 3 + p) * 1024;
    return *(const uint4 *)(base + lane16);
}

__device__ __forceinline__ float accumulate1(float acc, float sc, float cs, float c, float sx)
{
    return __builtin_fmaf(sc, c, __builtin_fmaf(-cs, sx, acc));
}
// Two 16-element halves with their own scales (Q6_K): acc + sc*(Ca - off*sa) + sc2*(Cb - off*sb).
__device__ __forceinline__ float accumulate2(float acc, float sc, float sc2, float ca, float cb, float sa, float sb,
                                             float off)
{
    acc = __builtin_fmaf(-(sc * off), sa, acc);
    acc = __builtin_fmaf(-(sc2 * off), sb, acc);
    acc = __builtin_fmaf(sc, ca, acc);
    return __builtin_fmaf(sc2, cb, acc);
}
constexpr uint32_t kOnes = 0x3F803F80u;   // bf16 1.0 pair

// Inputs of the EPI_QKV epilogue for one (token, row) value, loaded by the caller ahead of the
// epilogue: the token's position, the RoPE factors of the row's pair (when it is rotated) and
// the token's K or V cache base (for K / V rows).
struct QkvPre {
    uint32_t pos;   // never negative: widening it is a zero extension, which waits for no load
    float c, sn;
    float *cache;
};

// Epilogue of one output value per (token, weight row); all lanes of the wave must call it
// (adjacent weight rows are exchanged with DPP for the paired SwiGLU / RoPE epilogues).
// Returns the new residual value for EPI_RESID with a.np set (0 for rows / tokens outside the
// output), else 0.  With pre, EPI_RESID takes the residual and the next norm's gamma from
// pres / pg, and EPI_QKV its position, RoPE factors and cache base from qp (all loaded by the
// caller before the epilogue) instead of loading them here, so the epilogue's stores do not
// wait for loads: vector-memory waits count stores as well, so a load between two stores
// would also wait for the first store.
__device__ __forceinline__ float qgemm_epilogue(const QgemmArgs &a, float v, uint32_t row, int tok, bool live,
                                                bool pre = false, float pres = 0.0f, float pg = 0.0f,
                                                QkvPre qp = QkvPre{0, 0.0f, 0.0f, nullptr})
{
    const uint32_t N = (uint32_t)a.w.rows;
    if (a.bias && row < N) v = v + a.bias[row];
    // value of the neighbouring weight row (lane li ^ 1 holds row ^ 1)
    const float nb = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
    if (!live || row >= N || tok >= a.M) return 0.0f;
    float *yr = a.y + (int64_t)tok * a.y_stride;
    switch (a.epi) {
    case EPI_STORE: yr[row] = v; break;
    case EPI_RESID: {
        const float xn = (pre ? pres : yr[row]) + v;
        yr[row] = xn;
        if (a.np) {   // the next GEMM's parts of gamma (.) x (RMSNormOps.cs:137-139 up to the factor r)
            xp_store(a.np, (int)(N >> 5), tok, (int)row, (pre ? pg : a.ngamma[row]) * xn);
            return xn;
        }
        break;
    }
    case EPI_GELU:
        if (a.yp) xp_store(a.yp, (int)(N >> 5), tok, (int)row, gelu_pade(v));
        else yr[row] = gelu_pade(v);
        break;
    case EPI_SILU:
        // rows interleave gate / up: out[i] = silu(gate_i) * up_i
        if (!(row & 1)) {
            const float y = silu_mul(v, nb);
            if (a.yp) xp_store(a.yp, (int)(N >> 6), tok, (int)(row >> 1), y);
            else yr[row >> 1] = y;
        }
        break;
    case EPI_QKV: {
        if (row & 1) break;
        const int d = a.d_model, kv = a.kv_dim, hd = a.head_dim, r = (int)row;
        const uint32_t pos = pre ? qp.pos : (uint32_t)a.tok_pos[tok];
        float v0 = v, v1 = nb;
        if (a.use_rope && r < d + kv) {
            const int pair = ((r < d ? r : r - d) % hd) / 2, half = hd / 2;
            const float c = pre ? qp.c : a.rope_cos[(int64_t)pos * half + pair];
            const float sn = pre ? qp.sn : a.rope_sin[(int64_t)pos * half + pair];
            const float t0 = v0 * c, t1 = v1 * sn, t2 = v0 * sn, t3 = v1 * c;   // RotaryEmbedding.cs:115-116
            v0 = t0 - t1;
            v1 = t2 + t3;
        }
        if (r < d) {
            yr[r] = v0;
            yr[r + 1] = v1;
        } else if (r < d + kv) {
            float *dst = (pre ? qp.cache : a.kc_tok[tok]) + a.layer_off + (int64_t)(r - d) * a.ctx_stride + pos;
            dst[0] = v0;
            dst[a.ctx_stride] = v1;
        } else {
            const int vr = r - d - kv;
            float *dst = (pre ? qp.cache : a.vc_tok[tok]) + a.layer_off + ((int64_t)(vr / hd) * a.ctx_stride + pos) * hd + (vr % hd);
            dst[0] = v0;
            dst[1] = v1;
        }
        break;
    }
    default: break;
    }
    return 0.0f;
}

template <int F, int RT, int TT, int NW, int SB>
__global__ __launch_bounds__(64 * NW) void k_qgemm(QgemmArgs a)
{
    using Q = QW<F>;
    const WView &w = a.w;
    const uint8_t *__restrict__ xp = a.xp;
    const int M = a.M;
    __shared__ f32x4 s_part[NW - 1][RT * TT][64];
    const int wv = wave_id();
    const int lane = lane_id();
    const int g = lane >> 4, li = lane & 15;
    const uint32_t lane16 = (uint32_t)lane * 16u;
    const uint32_t N = (uint32_t)w.rows;
    const int nsb = (int)(w.cols >> 5);
    const uint32_t row_base = blockIdx.x * (16 * RT);
    const int tt0 = blockIdx.y * TT;
    const int ntt = (M + 15) >> 4;

    f32x4 acc[RT][TT];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int t = 0; t < TT; t++) acc[r][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // weight rows of this lane (B operand column l % 16), clamped to the matrix
    uint32_t wrow[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const uint32_t rr = row_base + 16 * r + li;
        wrow[r] = rr < N ? rr : N - 1;
    }
    const uint4 ones_a = Q::kHalves ? (g < 2 ? make_uint4(kOnes, kOnes, kOnes, kOnes) : kZero4)
                                    : make_uint4(kOnes, kOnes, kOnes, kOnes);
    const uint4 ones_b = g >= 2 ? make_uint4(kOnes, kOnes, kOnes, kOnes) : kZero4;

    // Wave wv takes sub-blocks wv, wv + NW, ...; SB of them at a time, all of whose loads (raw
    // weight words and activation parts) are issued before any is consumed.
    for (int s0 = wv; s0 < nsb; s0 += NW * SB) {
        RawQ raw[SB][RT];
        uint4 xa[SB][TT][3];
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const int s = s0 + u * NW < nsb ? s0 + u * NW : nsb - 1;
#pragma unroll
            for (int t = 0; t < TT; t++) {
                const int tt = tt0 + t < ntt ? tt0 + t : ntt - 1;
#pragma unroll
                for (int p = 0; p < 3; p++)
                    xa[u][t][p] = ld_part(xp, tt, nsb, s, p, lane16);
            }
#pragma unroll
            for (int r = 0; r < RT; r++) raw[u][r] = Q::load(w, wrow[r], s, g);
        }
        // keep the whole batch of loads ahead of the first use
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const int s = s0 + u * NW;
            const float ok = s < nsb ? 1.0f : 0.0f;   // past the end: clamped duplicate, adds 0
            uint4 wc[RT];
            Scl sc[RT];
#pragma unroll
            for (int r = 0; r < RT; r++) {
                wc[r] = Q::codes(raw[u][r], g);
                sc[r] = Q::scale(raw[u][r], s);
            }
            // sum(x) per token (and per half for Q6_K): the same for every weight row
#pragma unroll
            for (int t = 0; t < TT; t++) {
                f32x4 sa = {0.0f, 0.0f, 0.0f, 0.0f}, sb = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int p = 0; p < 3; p++) {
                    sa = mfma(xa[u][t][p], ones_a, sa);
                    if constexpr (Q::kHalves) sb = mfma(xa[u][t][p], ones_b, sb);
                }
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    if constexpr (Q::kHalves) {
                        const uint4 ca = g < 2 ? wc[r] : kZero4, cb = g >= 2 ? wc[r] : kZero4;
                        f32x4 da = {0.0f, 0.0f, 0.0f, 0.0f}, db = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                        for (int p = 0; p < 3; p++) {
                            da = mfma(xa[u][t][p], ca, da);
                            db = mfma(xa[u][t][p], cb, db);
                        }
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            acc[r][t][i] = accumulate2(acc[r][t][i], ok * sc[r].sc, ok * sc[r].sc2, da[i], db[i], sa[i], sb[i],
                                                       Q::kOff);
                    } else {
                        f32x4 dc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                        for (int p = 0; p < 3; p++) dc = mfma(xa[u][t][p], wc[r], dc);
                        const float c = ok * sc[r].sc, cs = ok * (sc[r].sc * Q::kOff + sc[r].m);
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[r][t][i] = accumulate1(acc[r][t][i], c, cs, dc[i], sa[i]);
                    }
                }
            }
        }
    }

    // sum the NW waves' partial tiles in a fixed order; wave 0 stores
    if (wv > 0) {
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int t = 0; t < TT; t++) s_part[wv - 1][r * TT + t][lane] = acc[r][t];
    }
    __syncthreads();
    if (wv != 0) return;
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int t = 0; t < TT; t++) {
            f32x4 v = acc[r][t];
#pragma unroll
            for (int k = 0; k < NW - 1; k++) {
                const f32x4 o = s_part[k][r * TT + t][lane];
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] += o[i];
            }
            const uint32_t row = row_base + 16 * r + li;
#pragma unroll
            for (int i = 0; i < 4; i++) qgemm_epilogue(a, v[i], row, (tt0 + t) * 16 + 4 * g + i, true);
        }
}

// ---- unquantized weights (F16 / F32) --------------------------------------------------------
// The FP32 Linear on F16 / F32 matrices (NeuralNet.cs:233-298, F32WeightTensor.cs:9-60).  The
// weights have no block scale to factor out, so they enter as bf16 parts of their own, exactly:
// an fp16 value (11 significant bits) is hi + lo, an fp32 value hi + mid + lo (8 + 8 + 8), each
// part a round-to-nearest-even bf16 of the remainder.  Every product of a weight part and an
// activation part is exact in fp32; the MFMA sums them (6 products per element for F16, 9 for
// F32).  Same operand layout, work split and epilogue as k_qgemm; no sum(x) term.
template <int F> struct DW {
    static constexpr int kParts = F == FMT_F16 ? 2 : 3;
    // the 8 weights of (row, sub-block s, k-group g) as fp32, element order 0..7
    __device__ __forceinline__ static void load(const WView &w, uint32_t row, int s, int g, float *v)
    {
        const uint8_t *p = w.q + ((size_t)row * (uint32_t)w.nb + (uint32_t)s) * fmt_main_bytes(F);
        if constexpr (F == FMT_F16) {
            const uint4 h = *(const uint4 *)(p + 16 * g);
            const uint32_t u[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[2 * i] = h2f(u[i] & 0xFFFFu);
                v[2 * i + 1] = h2f(u[i] >> 16);
            }
        } else {
            const float4 a = *(const float4 *)(p + 32 * g), b = *(const float4 *)(p + 32 * g + 16);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        }
    }
    // bf16 parts in the operand order (pair q = element q, element q + 4)
    __device__ __forceinline__ static void parts(const float *v, uint4 *o)
    {
        uint32_t pt[3][8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t h = bf16_rne(v[k]);
            const float r1 = v[k] - __uint_as_float(h << 16);
            const uint32_t m = bf16_rne(r1);
            pt[0][k] = h;
            pt[1][k] = m;
            if constexpr (kParts == 3) pt[2][k] = bf16_rne(r1 - __uint_as_float(m << 16));
        }
#pragma unroll
        for (int p = 0; p < kParts; p++)
            o[p] = make_uint4(pt[p][0] | (pt[p][4] << 16), pt[p][1] | (pt[p][5] << 16), pt[p][2] | (pt[p][6] << 16),
                              pt[p][3] | (pt[p][7] << 16));
    }
};

template <int F, int RT, int TT, int NW, int SB>
__global__ __launch_bounds__(64 * NW) void k_dgemm(QgemmArgs a)
{
    using D = DW<F>;
    constexpr int NP = D::kParts;
    const WView &w = a.w;
    const uint8_t *__restrict__ xp = a.xp;
    const int M = a.M;
    __shared__ f32x4 s_part[NW - 1][RT * TT][64];
    const int wv = wave_id();
    const int lane = lane_id();
    const int g = lane >> 4, li = lane & 15;
    const uint32_t lane16 = (uint32_t)lane * 16u;
    const uint32_t N = (uint32_t)w.rows;
    const int nsb = (int)(w.cols >> 5);
    const uint32_t row_base = blockIdx.x * (16 * RT);
    const int tt0 = blockIdx.y * TT;
    const int ntt = (M + 15) >> 4;

    f32x4 acc[RT][TT];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int t = 0; t < TT; t++) acc[r][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    uint32_t wrow[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const uint32_t rr = row_base + 16 * r + li;
        wrow[r] = rr < N ? rr : N - 1;
    }

    for (int s0 = wv; s0 < nsb; s0 += NW * SB) {
        float wf[SB][RT][8];
        uint4 xa[SB][TT][3];
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const int s = s0 + u * NW < nsb ? s0 + u * NW : nsb - 1;
#pragma unroll
            for (int t = 0; t < TT; t++) {
                const int tt = tt0 + t < ntt ? tt0 + t : ntt - 1;
#pragma unroll
                for (int p = 0; p < 3; p++) xa[u][t][p] = ld_part(xp, tt, nsb, s, p, lane16);
            }
#pragma unroll
            for (int r = 0; r < RT; r++) D::load(w, wrow[r], s, g, wf[u][r]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < SB; u++) {
            if (s0 + u * NW >= nsb) break;   // wave-uniform: past the end of K
#pragma unroll
            for (int r = 0; r < RT; r++) {
                uint4 wp[NP];
                D::parts(wf[u][r], wp);
#pragma unroll
                for (int t = 0; t < TT; t++)
#pragma unroll
                    for (int q = 0; q < NP; q++)
#pragma unroll
                        for (int p = 0; p < 3; p++) acc[r][t] = mfma(xa[u][t][p], wp[q], acc[r][t]);
            }
        }
    }

    if (wv > 0) {
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int t = 0; t < TT; t++) s_part[wv - 1][r * TT + t][lane] = acc[r][t];
    }
    __syncthreads();
    if (wv != 0) return;
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int t = 0; t < TT; t++) {
            f32x4 v = acc[r][t];
#pragma unroll
            for (int k = 0; k < NW - 1; k++) {
                const f32x4 o = s_part[k][r * TT + t][lane];
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] += o[i];
            }
            const uint32_t row = row_base + 16 * r + li;
#pragma unroll
            for (int i = 0; i < 4; i++) qgemm_epilogue(a, v[i], row, (tt0 + t) * 16 + 4 * g + i, true);
        }
}

// ---- LDS-staged variant --------------------------------------------------------------------
// The lane-per-(row, k-group) operand layout makes direct weight loads touch 16 rows (16 cache
// lines) per instruction for 4 useful bytes each.  Here every wave copies its weight tile --
// 16*RT rows x one 256-element super-block -- into its own LDS region with coalesced 16-byte
// loads (the next super-block's copy in flight while the current one is multiplied), and reads
// the operand dwords from LDS.  RT row tiles per wave share each activation-part load.
// Waves of a workgroup take contiguous super-block ranges of K.
// kBytes: main-stream bytes per row and super-block; kDW: dwords of the d stream per row and
// super-block (8 fp16 scales, one fp16 scale, or 8 fp32 scales).
template <int F> struct Stage;
template <> struct Stage<FMT_Q4_0> { static constexpr int kBytes = 128, kDW = 4; };
template <> struct Stage<FMT_Q8_0> { static constexpr int kBytes = 256, kDW = 4; };
template <> struct Stage<FMT_Q4_K> { static constexpr int kBytes = 144, kDW = 0; };
template <> struct Stage<FMT_Q5_K> { static constexpr int kBytes = 176, kDW = 0; };
template <> struct Stage<FMT_Q6_K> { static constexpr int kBytes = 208, kDW = 1; };
template <> struct Stage<FMT_SQ4> { static constexpr int kBytes = 128, kDW = 8; };
template <> struct Stage<FMT_SQ8> { static constexpr int kBytes = 256, kDW = 8; };

__device__ __forceinline__ uint32_t lds_u32(const uint8_t *p) { return *(const uint32_t *)p; }

// Raw operand words of (tile row, sub-block j of the staged super-block, k-group g) from LDS:
// `row` points at the row's staged main bytes, `dr` at its staged fp16 scales (packed in
// dwords).  Staged data is written and read as 32-bit words only, so the compiler cannot
// treat a narrower read as independent of the staging stores and move it above them.
template <int F>
__device__ __forceinline__ RawQ stage_raw(const uint8_t *row, const uint32_t *dr, int j, int g)
{
    RawQ r{};
    if constexpr (F == FMT_Q4_0) {
        r.v = lds_u32(row + 16 * j + 4 * g);
        r.d = (dr[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
    } else if constexpr (F == FMT_SQ4) {
        r.v = lds_u32(row + 16 * j + 4 * g);
        r.d = dr[j];
    } else if constexpr (F == FMT_SQ8) {
        r.v = lds_u32(row + 32 * j + 8 * g);
        r.v2 = lds_u32(row + 32 * j + 8 * g + 4);
        r.d = dr[j];
    } else if constexpr (F == FMT_Q8_0) {
        r.v = lds_u32(row + 32 * j + 8 * g);
        r.v2 = lds_u32(row + 32 * j + 8 * g + 4);
        r.d = (dr[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
    } else if constexpr (F == FMT_Q4_K) {
        r.h = make_uint4(lds_u32(row), lds_u32(row + 4), lds_u32(row + 8), lds_u32(row + 12));
        r.v = lds_u32(row + 16 + 16 * j + 4 * g);
    } else if constexpr (F == FMT_Q5_K) {
        r.h = make_uint4(lds_u32(row), lds_u32(row + 4), lds_u32(row + 8), lds_u32(row + 12));
        r.v = lds_u32(row + 48 + 16 * j + 4 * g);
        r.H = lds_u32(row + 16 + 4 * j);
    } else {
        r.v = lds_u32(row + 16 * j + 4 * g);
        r.H = lds_u32(row + 128 + 8 * j);
        r.H2 = lds_u32(row + 128 + 8 * j + 4);
        const uint32_t scw = (lds_u32(row + 192 + 4 * (j >> 1)) >> (16 * (j & 1))) & 0xFFFFu;
        r.d = (dr[0] & 0xFFFFu) | (scw << 16);
    }
    return r;
}

// Tile order of a launch with several token-tile groups.  The 2-D grid (row tile x, token group
// y) runs the row tiles fastest, and workgroups land on the 8 XCDs round robin, so each XCD works
// on 1/8 of W for ~1.5 token groups at a time: W's slice plus those groups' activation parts
// exceed the XCD's 4 MB L2, and W is fetched again for every token group.  With G > 0 the grid
// is 1-D and workgroup i runs tile t = (i % 8) * chunk + i / 8 of a panel-major order (panels of
// G token groups whose parts stay in the L2, row tiles in a panel with the G groups fastest), so
// each XCD works through one contiguous chunk of that order: the parts of its panel stay
// resident and each W tile is read once per panel by G workgroups in a row.
struct TileSched {
    uint32_t R, T;       // row tiles, token-tile groups
    uint32_t G, chunk;   // groups per panel (0: the 2-D grid), tiles per XCD
};

// TS > 1 (one token tile only): the tile's 16 tokens are split over TS workgroups of 16 / TS
// tokens each (grid y).  Each workgroup still multiplies whole 16 x 16 MFMA tiles, but it loads
// the activation parts of its own tokens only (the other token lanes repeat them) and stores
// only their outputs: the parts of the whole K, which every workgroup of a row tile reads, are
// most of what a one-token-tile workgroup moves into its CU, and the split also spreads a
// matrix of few row tiles over more CUs.  No partial sums cross workgroups.
template <int F, int RT, int TT, int NW, int TS = 1>
__global__ __launch_bounds__(64 * NW) void k_qgemm_st(QgemmArgs a, TileSched ts)
{
    static_assert(TS == 1 || (TT == 1 && (TS == 2 || TS == 4)), "token split of one token tile into 8 or 4");
    using Q = QW<F>;
    using G = Stage<F>;
    constexpr int R16 = 16 * RT;
    constexpr int RS = G::kBytes + 4;                       // row stride: dword pad, odd in dwords
    constexpr int NPC = (R16 * G::kBytes / 16 + 63) / 64;   // 16-byte pieces per lane
    // dword accesses below: the byte array must be dword (here 16-byte) aligned
    __shared__ __align__(16) uint8_t s_w[NW][R16 * RS];
    __shared__ __align__(16) uint32_t s_d[NW][R16][G::kDW > 0 ? G::kDW : 1];
    __shared__ f32x4 s_part[NW - 1][RT * TT][64];
    const WView &w = a.w;
    const uint8_t *__restrict__ xp = a.xp;
    const int M = a.M;
    const int wv = wave_id();
    const int lane = lane_id();
    const int g = lane >> 4, li = lane & 15;
    const uint32_t lane16 = (uint32_t)lane * 16u;
    const uint32_t N = (uint32_t)w.rows;
    const int nsb = (int)(w.cols >> 5), nsup = nsb >> 3;
    uint32_t bx = blockIdx.x, by = blockIdx.y;
    // one token tile (the lockstep step): never scheduled, and the latency-bound launch reads
    // no schedule argument (reading and testing it cost 2 % of the configs[4] step)
    if constexpr (TT > 1) {
        if (ts.G) {   // wave-uniform: the whole workgroup takes the same branch
            const uint32_t i = blockIdx.x, t = (i & 7u) * ts.chunk + (i >> 3);
            if (t >= ts.R * ts.T) return;
            const uint32_t pt = ts.R * ts.G, panel = t / pt, rem = t - panel * pt;
            const uint32_t gp = min(ts.G, ts.T - panel * ts.G);
            bx = rem / gp;
            by = panel * ts.G + (rem - bx * gp);
        }
    }
    const uint32_t row_base = bx * R16;
    // token split: this workgroup's tokens are tlo .. tlo + TW - 1 of the single token tile
    constexpr int TW = 16 / TS;
    const int tlo = TS > 1 ? (int)by * TW : 0;
    const int tt0 = TS > 1 ? 0 : (int)by * TT;
    const int ntt = (M + 15) >> 4;
    // lanes whose results are this workgroup's tokens (tokens 4g .. 4g + 3; TW is a multiple of
    // 4).  A lane supplies token li's parts to the MFMA; lanes of the other tokens read those of
    // token tlo + li % TW instead, so the loads touch only this workgroup's tokens' lines and
    // need no mask or select (the duplicated tokens' results are not stored).
    const bool tlive = TS == 1 || (uint32_t)(4 * g - tlo) < (uint32_t)TW;
    const uint32_t xl16 = TS == 1 ? lane16 : (uint32_t)(16 * g + tlo + (li & (TW - 1))) * 16u;
    const uint32_t row_bytes = (uint32_t)nsup * G::kBytes;
    // contiguous super-block range of this wave
    const int per = (nsup + NW - 1) / NW;
    const int sup0 = wv * per, sup1 = sup0 + per < nsup ? sup0 + per : nsup;

    f32x4 acc[RT][TT];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int t = 0; t < TT; t++) acc[r][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const uint4 ones_a = Q::kHalves ? (g < 2 ? make_uint4(kOnes, kOnes, kOnes, kOnes) : kZero4)
                                    : make_uint4(kOnes, kOnes, kOnes, kOnes);
    const uint4 ones_b = g >= 2 ? make_uint4(kOnes, kOnes, kOnes, kOnes) : kZero4;

    // Folded RMSNorm (one token tile): the tile sums of x^2 of wave wv's tokens wv + NW*j are
    // requested here and reduced after the main loop.
    constexpr int RJ = TT == 1 ? (16 + NW - 1) / NW : 1, RP = 4;   // tokens per wave, sums per lane
    __shared__ float s_r[16];
    float rl[RJ][RP];
    const bool fold = TT == 1 && a.rss != nullptr;
    if (fold) {
#pragma unroll
        for (int j = 0; j < RJ; j++) {
            const int tk = min(tt0 * 16 + wv + NW * j, M - 1);
#pragma unroll
            for (int q = 0; q < RP; q++) {
                const int p = lane + 64 * q;
                rl[j][q] = p < a.rss_n ? a.rss[(int64_t)p * M + tk] : 0.0f;
            }
        }
    }

    // EPI_RESID with one 16 x 16 tile per wave: wave 0's residual values (and the next norm's
    // gamma) are requested at entry, so the epilogue waits for no load.  EPI_QKV likewise: the
    // positions of wave 0's tokens at entry, their RoPE factors and cache bases (which depend
    // on the positions) right after the main loop, ahead of the cross-wave reduction.
    constexpr bool PRE = TT == 1 && RT == 1;
    const bool pre = PRE && (a.epi == EPI_RESID || a.epi == EPI_QKV);
    const bool preq = PRE && a.epi == EPI_QKV;
    float pres[4] = {0.0f, 0.0f, 0.0f, 0.0f}, pg = 0.0f;
    QkvPre qp[4] = {};
    if (pre && wv == 0 && tlive) {
        const uint32_t rc = min(row_base + (uint32_t)li, N - 1);
        if (preq) {
#pragma unroll
            for (int i = 0; i < 4; i++) qp[i].pos = a.tok_pos[min(tt0 * 16 + 4 * g + i, M - 1)];
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) pres[i] = a.y[(int64_t)min(tt0 * 16 + 4 * g + i, M - 1) * a.y_stride + rc];
            if (a.np) pg = a.ngamma[rc];
        }
    }

    // staging loads of one super-block: piece p -> (row p / (kBytes/16), 16-byte column)
    uint4 wp[NPC];
    uint4 dp = kZero4, dp2 = kZero4;
    auto issue = [&](int sup) {
#pragma unroll
        for (int k = 0; k < NPC; k++) {
            const int p = lane + 64 * k;
            const int row = p / (G::kBytes / 16), col = p % (G::kBytes / 16);
            uint32_t gr = row_base + (uint32_t)row;
            gr = gr < N ? gr : N - 1;
            wp[k] = p < R16 * G::kBytes / 16
                        ? *(const uint4 *)(w.q + gr * row_bytes + (uint32_t)sup * G::kBytes + 16u * col)
                        : kZero4;
        }
        if constexpr (G::kDW == 4) {
            if (lane < R16) {
                uint32_t gr = row_base + (uint32_t)lane;
                gr = gr < N ? gr : N - 1;
                dp = *(const uint4 *)(w.d + (gr * (uint32_t)nsb + (uint32_t)sup * 8));
            }
        } else if constexpr (G::kDW == 8) {
            if (lane < R16) {
                uint32_t gr = row_base + (uint32_t)lane;
                gr = gr < N ? gr : N - 1;
                const uint4 *dq = (const uint4 *)((const uint32_t *)w.d + (gr * (uint32_t)nsb + (uint32_t)sup * 8));
                dp = dq[0];
                dp2 = dq[1];
            }
        } else if constexpr (G::kDW == 1) {
            if (lane < R16) {
                uint32_t gr = row_base + (uint32_t)lane;
                gr = gr < N ? gr : N - 1;
                dp.x = w.d[gr * (uint32_t)nsup + (uint32_t)sup];
            }
        }
    };
    auto stage = [&]() {
        // the previous super-block's reads of the tile stay above these stores
        asm volatile("" ::: "memory");
        uint8_t *dst = s_w[wv];
#pragma unroll
        for (int k = 0; k < NPC; k++) {
            const int p = lane + 64 * k;
            if (p < R16 * G::kBytes / 16) {
                const int row = p / (G::kBytes / 16), col = p % (G::kBytes / 16);
                uint32_t *o = (uint32_t *)(dst + row * RS + 16 * col);
                o[0] = wp[k].x;
                o[1] = wp[k].y;
                o[2] = wp[k].z;
                o[3] = wp[k].w;
            }
        }
        if constexpr (G::kDW == 4 || G::kDW == 8) {
            if (lane < R16) {
                uint32_t *o = s_d[wv][lane];
                o[0] = dp.x; o[1] = dp.y; o[2] = dp.z; o[3] = dp.w;
                if constexpr (G::kDW == 8) { o[4] = dp2.x; o[5] = dp2.y; o[6] = dp2.z; o[7] = dp2.w; }
            }
        } else if constexpr (G::kDW == 1) {
            if (lane < R16) s_d[wv][lane][0] = dp.x;
        }
        // keep every read of the staged tile below these stores
        asm volatile("" ::: "memory");
    };

    if (sup0 < sup1) issue(sup0);
    for (int sup = sup0; sup < sup1; sup++) {
        stage();                               // this wave's LDS region only: in-order LDS ops
        if (sup + 1 < sup1) issue(sup + 1);    // next super-block in flight
        // XU sub-blocks of activation parts in flight at once (fewer with more token tiles, and
        // two for the 16-wave SMQ Q8 tile, whose two staged scale words per sub-block would
        // otherwise push it past the 128 registers of a 1024-thread workgroup)
        constexpr int XU = TT == 1 ? (F == FMT_SQ8 && NW == 16 ? 2 : 4) : 1;
#pragma unroll
        for (int h = 0; h < 8 / XU; h++) {
            uint4 xa[XU][TT][3];
#pragma unroll
            for (int u = 0; u < XU; u++) {
                const int s = sup * 8 + XU * h + u;
#pragma unroll
                for (int t = 0; t < TT; t++) {
                    const int tt = tt0 + t < ntt ? tt0 + t : ntt - 1;
#pragma unroll
                    for (int p = 0; p < 3; p++)
                        xa[u][t][p] = ld_part(xp, tt, nsb, s, p, xl16);
                }
            }
#pragma unroll
            for (int u = 0; u < XU; u++) {
                const int j = XU * h + u;
                uint4 wc[RT];
                Scl sc[RT];
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    const int row = 16 * r + li;
                    const RawQ raw = stage_raw<F>(s_w[wv] + row * RS, s_d[wv][row], j, g);
                    wc[r] = Q::codes(raw, g);
                    sc[r] = Q::scale(raw, j);
                }
#pragma unroll
                for (int t = 0; t < TT; t++) {
                    f32x4 sa = {0.0f, 0.0f, 0.0f, 0.0f}, sb = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int p = 0; p < 3; p++) {
                        sa = mfma(xa[u][t][p], ones_a, sa);
                        if constexpr (Q::kHalves) sb = mfma(xa[u][t][p], ones_b, sb);
                    }
#pragma unroll
                    for (int r = 0; r < RT; r++) {
                        if constexpr (Q::kHalves) {
                            const uint4 ca = g < 2 ? wc[r] : kZero4, cb = g >= 2 ? wc[r] : kZero4;
                            f32x4 da = {0.0f, 0.0f, 0.0f, 0.0f}, db = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                            for (int p = 0; p < 3; p++) {
                                da = mfma(xa[u][t][p], ca, da);
                                db = mfma(xa[u][t][p], cb, db);
                            }
#pragma unroll
                            for (int i = 0; i < 4; i++)
                                acc[r][t][i] = accumulate2(acc[r][t][i], sc[r].sc, sc[r].sc2, da[i], db[i], sa[i], sb[i],
                                                           Q::kOff);
                        } else {
                            f32x4 dc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                            for (int p = 0; p < 3; p++) dc = mfma(xa[u][t][p], wc[r], dc);
                            const float c = sc[r].sc, cs = sc[r].sc * Q::kOff + sc[r].m;
#pragma unroll
                            for (int i = 0; i < 4; i++) acc[r][t][i] = accumulate1(acc[r][t][i], c, cs, dc[i], sa[i]);
                        }
                    }
                }
            }
        }
    }

    if (preq && wv == 0 && tlive) {
        const int d = a.d_model, kv = a.kv_dim, hd = a.head_dim, half = hd / 2;
        const int r = (int)min(row_base + (uint32_t)li, N - 1);
        const int pair = ((r < d ? r : r - d) % hd) / 2;
        const bool rot = a.use_rope && r < d + kv && !(r & 1);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tk = min(tt0 * 16 + 4 * g + i, M - 1);
            qp[i].c = rot ? a.rope_cos[(int64_t)qp[i].pos * half + pair] : 0.0f;
            qp[i].sn = rot ? a.rope_sin[(int64_t)qp[i].pos * half + pair] : 0.0f;
            qp[i].cache = r < d ? nullptr : (r < d + kv ? a.kc_tok[tk] : a.vc_tok[tk]);
        }
    }
    if (fold) {   // r = 1 / sqrt(sum x^2 / K + eps) (RMSNormOps.cs:114)
#pragma unroll
        for (int j = 0; j < RJ; j++) {
            float t = rl[j][0];
#pragma unroll
            for (int q = 1; q < RP; q++) t += rl[j][q];
            t = wave_sum_uniform(t);
            if (lane == 0 && wv + NW * j < 16) s_r[wv + NW * j] = 1.0f / sqrtf(t / (float)w.cols + a.r_eps);
        }
    }
    // sum the NW waves' partial tiles in a fixed order; wave 0 applies the epilogue
    if (wv > 0) {
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int t = 0; t < TT; t++) s_part[wv - 1][r * TT + t][lane] = acc[r][t];
    }
    __syncthreads();
    if (wv != 0) return;
    float rs[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if (fold) {
#pragma unroll
        for (int i = 0; i < 4; i++) rs[i] = s_r[4 * g + i];
    }
    const bool emit = TT == 1 && a.np != nullptr;   // producer of a folded norm
#pragma unroll
    for (int r = 0; r < RT; r++) {
        float sq[TT][4];
#pragma unroll
        for (int t = 0; t < TT; t++) {
            f32x4 v = acc[r][t];
#pragma unroll
            for (int k = 0; k < NW - 1; k++) {
                const f32x4 o = s_part[k][r * TT + t][lane];
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] += o[i];
            }
            const uint32_t row = row_base + 16 * r + li;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float xn = qgemm_epilogue(a, v[i] * rs[i], row, (tt0 + t) * 16 + 4 * g + i, tlive, pre, pres[i],
                                                pg, qp[i]);
                sq[t][i] = xn * xn;
            }
        }
        if (emit) {   // x^2 summed over the tile's 16 rows (the 16 lanes of a row of lanes)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float t = row16_sum(sq[0][i]);
                const int tok = tt0 * 16 + 4 * g + i;
                if (li == 0 && tok < M && tlive) a.nss[(int64_t)(row_base / 16 + r) * M + tok] = t;
            }
        }
    }
}

// ---- row-split variant for one token tile ---------------------------------------------------
// Up to 16 tokens, the K-split workgroups above each read the activation parts of the whole K
// for their own 16-32 rows (6 bytes per token and k against 0.69 bytes per Q5_K weight), and
// a wave can only hold a few sub-blocks of them in registers, so its part loads queue behind
// its weight loads.  Here a workgroup of NW = NR * NKH waves owns NR row tiles (16 rows each)
// and the whole K: wave (r, h) multiplies row tile r by the sub-blocks h * 8 / NKH ... of every
// super-block.  Super-block by super-block, a slot of an NS-slot LDS ring receives the
// super-block's activation parts (24 KB, read by every wave) and its NR * 16 rows of weights,
// both loaded straight into LDS (global_load_lds_dwordx4, no registers) NS - 1 super-blocks
// ahead of use; one barrier per super-block publishes a slot.  Each wave issues the same
// number of loads per super-block (every one with at least one active lane), so the wait for
// a slot is a fixed vector-memory count.  The loads into LDS are issued by inline assembly:
// through the builtin, the compiler cannot tell the slots apart in this kernel and waits for
// every load into LDS in flight before each LDS read, which leaves no load in flight across a
// super-block's multiplications.  The explicit wait before each barrier is what orders a
// slot's reads after its loads.
template <int F, int NR> struct RsSlot {
    uint4 xp[24][64];                  // [sub-block][part] x (64 lanes x 16 bytes)
    uint4 w[NR * Stage<F>::kBytes];    // NR * 16 rows x kBytes, row-major, in 16-byte pieces
};

template <int N> using ic = std::integral_constant<int, N>;

// 16 bytes per lane from global address g into LDS at l + 16 * lane (l wave-uniform; M0 holds
// it, with the one wait state between the M0 write and the load)
__device__ __forceinline__ void lds_dma16(const void *g, void *l)
{
    const uint32_t la = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)l;
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(la) : "memory");
}

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4 left
// alone, lgkmcnt 11:8): the wave's vector-memory loads older than its last n have landed and
// its own LDS reads have completed
template <int N> __device__ __forceinline__ void wait_vm_lds()
{
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

template <int F, int NR, int NKH, int NS>
__global__ __launch_bounds__(64 * NR * NKH) void k_qgemm_rs(QgemmArgs a)
{
    using Q = QW<F>;
    constexpr int kB = Stage<F>::kBytes;
    constexpr int NW = NR * NKH, JP = 8 / NKH;
    constexpr int WP = NR * kB;            // 16-byte weight pieces per super-block
    constexpr int PPW = WP / NW;           // ... per wave
    constexpr int WI = (PPW + 63) / 64;    // weight loads per wave and super-block
    constexpr int NPW = 24 / NW;           // part loads per wave and super-block
    constexpr int L = WI + NPW;            // vector-memory instructions per wave and super-block
    static_assert(Stage<F>::kDW == 0, "weights without a separate scale stream");
    static_assert(WP % NW == 0 && 24 % NW == 0 && 8 % NKH == 0 && NS >= 2 && NS <= 4, "work split");
    static_assert((NS - 2) * L < 64, "vmcnt range");
    __shared__ RsSlot<F, NR> slot[NS];
    __shared__ f32x4 s_part[NKH > 1 ? NKH - 1 : 1][NR][64];
    __shared__ float s_r[16];
    const WView &w = a.w;
    const int M = a.M;
    const int wv = wave_id();
    const int r = wv % NR, h = wv / NR;
    const int lane = lane_id();
    const int g = lane >> 4, li = lane & 15;
    const uint32_t N = (uint32_t)w.rows;
    const int nsup = (int)(w.cols >> 8);
    const uint32_t row_base = blockIdx.x * (16u * NR);
    const uint32_t row_bytes = (uint32_t)nsup * kB;
    const uint32_t my_row = row_base + 16u * r + (uint32_t)li;

    // loads of super-block sup into a slot: this wave's parts (instructions wv * NPW ...) and
    // its share of the weight pieces (wv * PPW ...)
    auto issue = [&](int sup, auto &S) {
        const uint8_t *xs = a.xp + (size_t)sup * (24u * 1024u) + (uint32_t)lane * 16u;
#pragma unroll
        for (int k = 0; k < NPW; k++) {
            const int c = wv * NPW + k;
            lds_dma16(xs + c * 1024, &S.xp[c][0]);
        }
#pragma unroll
        for (int k = 0; k < WI; k++) {
            const int q = wv * PPW + 64 * k + lane;
            if (64 * k + lane < PPW) {
                const int rw = q / (kB / 16), col = q % (kB / 16);
                const uint32_t gr = min(row_base + (uint32_t)rw, N - 1);
                lds_dma16(w.q + gr * row_bytes + (uint32_t)sup * kB + 16u * col, &S.w[wv * PPW + 64 * k]);
            }
        }
    };
    // the first super-blocks' loads go out before anything else
#pragma unroll
    for (int i = 0; i < NS - 1; i++)
        if (i < nsup) issue(i, slot[i]);

    // Folded RMSNorm: the tile sums of x^2 of wave wv's tokens wv + NW*j, requested here and
    // reduced after the main loop.
    constexpr int RJ = (16 + NW - 1) / NW, RP = 4;
    float rl[RJ][RP];
    const bool fold = a.rss != nullptr;
    if (fold) {
#pragma unroll
        for (int j = 0; j < RJ; j++) {
            const int tk = min(wv + NW * j, M - 1);
#pragma unroll
            for (int q = 0; q < RP; q++) {
                const int p = lane + 64 * q;
                rl[j][q] = p < a.rss_n ? a.rss[(int64_t)p * M + tk] : 0.0f;
            }
        }
    }
    // The epilogue waves' residual values and next-norm gamma (EPI_RESID), or their tokens'
    // positions (EPI_QKV), requested at entry so that the epilogue's stores wait for no load.
    const bool pre = a.epi == EPI_RESID || a.epi == EPI_QKV;
    const bool preq = a.epi == EPI_QKV;
    float pres[4] = {0.0f, 0.0f, 0.0f, 0.0f}, pg = 0.0f;
    QkvPre qp[4] = {};
    if (pre && h == 0) {
        const uint32_t rc = min(my_row, N - 1);
        if (preq) {
#pragma unroll
            for (int i = 0; i < 4; i++) qp[i].pos = a.tok_pos[min(4 * g + i, M - 1)];
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) pres[i] = a.y[(int64_t)min(4 * g + i, M - 1) * a.y_stride + rc];
            if (a.np) pg = a.ngamma[rc];
        }
    }

    // Publishes the slot of super-block i: this wave's loads of it have landed (the loads of
    // the n_after later super-blocks already issued may still be in flight), then every wave's.
    // The wave's LDS reads of the previous super-block's slot have completed too, so the loads
    // that go into that slot after the barrier cannot overtake them.
    auto sync = [&](int n_after) {
        asm volatile("" ::: "memory");
        if (NS > 3 && n_after >= 2) wait_vm_lds<(NS > 3 ? 2 * L : 0)>();
        else if (NS > 2 && n_after >= 1) wait_vm_lds<(NS > 2 ? L : 0)>();
        else wait_vm_lds<0>();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const uint4 ones = make_uint4(kOnes, kOnes, kOnes, kOnes);
    auto compute = [&](const auto &S) {
        const uint8_t *wrow = (const uint8_t *)S.w + (16 * r + li) * kB;
        auto body = [&](auto hc) {
            constexpr int H = decltype(hc)::value;
#pragma unroll
            for (int jj = 0; jj < JP; jj++) {
                const int j = H * JP + jj;
                uint4 xa[3];
#pragma unroll
                for (int p = 0; p < 3; p++) xa[p] = S.xp[3 * j + p][lane];
                const RawQ raw = stage_raw<F>(wrow, nullptr, j, g);
                const uint4 wc = Q::codes(raw, g);
                const Scl sc = Q::scale(raw, j);
                f32x4 sa = {0.0f, 0.0f, 0.0f, 0.0f}, dc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int p = 0; p < 3; p++) sa = mfma(xa[p], ones, sa);
#pragma unroll
                for (int p = 0; p < 3; p++) dc = mfma(xa[p], wc, dc);
                const float c = sc.sc, cs = sc.sc * Q::kOff + sc.m;
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i] = accumulate1(acc[i], c, cs, dc[i], sa[i]);
            }
        };
        if constexpr (NKH == 1) body(ic<0>{});
        else if constexpr (NKH == 2) { if (h == 0) body(ic<0>{}); else body(ic<1>{}); }
        else if constexpr (NKH == 4) {
            if (h == 0) body(ic<0>{}); else if (h == 1) body(ic<1>{}); else if (h == 2) body(ic<2>{}); else body(ic<3>{});
        } else {
            switch (h) {
            case 0: body(ic<0>{}); break;
            case 1: body(ic<1>{}); break;
            case 2: body(ic<2>{}); break;
            case 3: body(ic<3>{}); break;
            case 4: body(ic<4>{}); break;
            case 5: body(ic<5>{}); break;
            case 6: body(ic<6>{}); break;
            default: body(ic<7>{}); break;
            }
        }
    };
    // super-block i lives in slot i % NS; its loads were issued NS - 1 super-blocks earlier,
    // into the slot that super-block i - 1 used, which every wave finished reading before the
    // barrier of step i
    for (int i = 0; i < nsup; i++) {
        sync(min(NS - 2, nsup - 1 - i));
        if (i + NS - 1 < nsup) issue(i + NS - 1, slot[(i + NS - 1) % NS]);
        compute(slot[i % NS]);
    }

    if (preq && h == 0) {
        const int d = a.d_model, kv = a.kv_dim, hd = a.head_dim, half = hd / 2;
        const int rr = (int)min(my_row, N - 1);
        const int pair = ((rr < d ? rr : rr - d) % hd) / 2;
        const bool rot = a.use_rope && rr < d + kv && !(rr & 1);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tk = min(4 * g + i, M - 1);
            qp[i].c = rot ? a.rope_cos[(int64_t)qp[i].pos * half + pair] : 0.0f;
            qp[i].sn = rot ? a.rope_sin[(int64_t)qp[i].pos * half + pair] : 0.0f;
            qp[i].cache = rr < d ? nullptr : (rr < d + kv ? a.kc_tok[tk] : a.vc_tok[tk]);
        }
    }
    if (fold) {   // r = 1 / sqrt(sum x^2 / K + eps) (RMSNormOps.cs:114)
#pragma unroll
        for (int j = 0; j < RJ; j++) {
            float t = rl[j][0];
#pragma unroll
            for (int q = 1; q < RP; q++) t += rl[j][q];
            t = wave_sum_uniform(t);
            if (lane == 0 && wv + NW * j < 16) s_r[wv + NW * j] = 1.0f / sqrtf(t / (float)w.cols + a.r_eps);
        }
    }
    // sum the NKH partial tiles of each row tile in a fixed order; wave (r, 0) applies the
    // epilogue
    if (NKH > 1 && h > 0) s_part[h - 1][r][lane] = acc;
    __syncthreads();   // s_part, and the folded-norm factors in s_r
    if (h != 0) return;
    float rs[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if (fold) {
#pragma unroll
        for (int i = 0; i < 4; i++) rs[i] = s_r[4 * g + i];
    }
    f32x4 v = acc;
#pragma unroll
    for (int k = 0; k < NKH - 1; k++) {
        const f32x4 o = s_part[k][r][lane];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] += o[i];
    }
    float sq[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float xn = qgemm_epilogue(a, v[i] * rs[i], my_row, 4 * g + i, true, pre, pres[i], pg, qp[i]);
        sq[i] = xn * xn;
    }
    if (a.np != nullptr) {   // producer of a folded norm: x^2 summed over the tile's 16 rows
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float t = row16_sum(sq[i]);
            const int tok = 4 * g + i;
            if (li == 0 && tok < M) a.nss[(int64_t)(row_base / 16 + r) * M + tok] = t;
        }
    }
}

// Activation parts: token m, sub-block s, part p -> Xp[m/16][s][p][g][m%16][perm] (bf16).
// x = hi + mid + lo with hi = bf16(x), mid = bf16(x - hi), lo = bf16(x - hi - mid), each
// rounded to nearest even (bf16_rne, xp_store); tokens beyond M (tile padding) are zero.

// Parts and stores of one item (8 elements of sub-block s, group g) of token row t of tile tt.
__device__ __forceinline__ void qprep_store(const float *v, uint8_t *__restrict__ xp, int nsb, int tt, int t, int i)
{
    const int s = i >> 2, g = i & 3;
    uint32_t part[3][8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const float f = v[k];
        const uint32_t h = bf16_rne(f);
        const float r1 = f - __uint_as_float(h << 16);
        const uint32_t mm = bf16_rne(r1);
        const float r2 = r1 - __uint_as_float(mm << 16);
        part[0][k] = h;
        part[1][k] = mm;
        part[2][k] = bf16_rne(r2);
    }
#pragma unroll
    for (int p = 0; p < 3; p++) {
        // pair q = (element q, element q + 4)
        uint4 o;
        o.x = part[p][0] | (part[p][4] << 16);
        o.y = part[p][1] | (part[p][5] << 16);
        o.z = part[p][2] | (part[p][6] << 16);
        o.w = part[p][3] | (part[p][7] << 16);
        *(uint4 *)(xp + (((size_t)tt * nsb + s) * 3 + p) * 1024 + (g * 16 + t) * 16) = o;
    }
}

__device__ __forceinline__ void unpack8(const float4 &a, const float4 &b, float *v)
{
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// One workgroup per token (rows M..Mp-1 of the last tile are zero): the norm statistic of the
// row (RMSNorm: RMSNormOps.cs:114; LayerNorm: LayerNormOps.cs:92-119), the normalised value in
// the reference's operation order (gamma * (x * invRms); fma(gamma, (x - mean) * invStd, beta)),
// then its three bf16 parts at Xp[m/16][s][p][g][m%16][perm].  Thread j holds items j + 256 u
// (u < IPT, K <= 2048 * IPT): the row, gamma and beta are loaded in one batch before the
// statistic, so the kernel makes one round trip to memory.
template <int IPT>
__global__ __launch_bounds__(256) void k_qprep(const float *__restrict__ x, int64_t x_stride, int M, int K,
                                               int pro, const float *__restrict__ gamma,
                                               const float *__restrict__ beta, float eps,
                                               uint8_t *__restrict__ xp)
{
    __shared__ float red[16];
    const int m = blockIdx.x;
    const int nsb = K >> 5, items = K >> 3;   // item = 8 elements (sub-block s, group g)
    const int tt = m >> 4, t = m & 15;
    const float *xr = x + (int64_t)m * x_stride;
    const int tid = threadIdx.x;
    if (m >= M) {   // padding row of the last tile
        float z[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        for (int i = tid; i < items; i += 256) qprep_store(z, xp, nsb, tt, t, i);
        return;
    }
    float4 xa[IPT][2], ga[IPT][2], ba[IPT][2];
#pragma unroll
    for (int u = 0; u < IPT; u++) {
        const int i = tid + 256 * u;
        if (i < items) {
            xa[u][0] = ((const float4 *)xr)[2 * i];
            xa[u][1] = ((const float4 *)xr)[2 * i + 1];
            if (pro != PRO_NONE) {
                ga[u][0] = ((const float4 *)gamma)[2 * i];
                ga[u][1] = ((const float4 *)gamma)[2 * i + 1];
            }
            if (pro == PRO_LN) {
                ba[u][0] = ((const float4 *)beta)[2 * i];
                ba[u][1] = ((const float4 *)beta)[2 * i + 1];
            }
        }
    }
    float sc = 1.0f, mean = 0.0f;
    if (pro == PRO_RMS) {
        float ss = 0.0f;
#pragma unroll
        for (int u = 0; u < IPT; u++)
            if (tid + 256 * u < items) {
                float v[8];
                unpack8(xa[u][0], xa[u][1], v);
#pragma unroll
                for (int k = 0; k < 8; k++) { const float q = v[k] * v[k]; ss += q; }
            }
        ss = block_sum<4>(ss, red);
        sc = 1.0f / sqrtf(ss / (float)K + eps);
    } else if (pro == PRO_LN) {
        float tsum = 0.0f;
#pragma unroll
        for (int u = 0; u < IPT; u++)
            if (tid + 256 * u < items) {
                float v[8];
                unpack8(xa[u][0], xa[u][1], v);
#pragma unroll
                for (int k = 0; k < 8; k++) tsum += v[k];
            }
        mean = block_sum<4>(tsum, red) / (float)K;
        float sq = 0.0f;
#pragma unroll
        for (int u = 0; u < IPT; u++)
            if (tid + 256 * u < items) {
                float v[8];
                unpack8(xa[u][0], xa[u][1], v);
#pragma unroll
                for (int k = 0; k < 8; k++) { const float dd = v[k] - mean; const float q = dd * dd; sq += q; }
            }
        sq = block_sum<4>(sq, red);
        sc = 1.0f / sqrtf(sq / (float)K + eps);
    }
#pragma unroll
    for (int u = 0; u < IPT; u++) {
        const int i = tid + 256 * u;
        if (i >= items) continue;
        float v[8];
        unpack8(xa[u][0], xa[u][1], v);
        if (pro == PRO_RMS) {
            float gg[8];
            unpack8(ga[u][0], ga[u][1], gg);
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = gg[k] * (v[k] * sc);
        } else if (pro == PRO_LN) {
            float gg[8], be[8];
            unpack8(ga[u][0], ga[u][1], gg);
            unpack8(ba[u][0], ba[u][1], be);
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = __builtin_fmaf(gg[k], (v[k] - mean) * sc, be[k]);
        }
        qprep_store(v, xp, nsb, tt, t, i);
    }
}

// Rows longer than 2048 * 4: the same with the row read twice in loops.
__global__ __launch_bounds__(256) void k_qprep_long(const float *__restrict__ x, int64_t x_stride, int M, int K,
                                                    int pro, const float *__restrict__ gamma,
                                                    const float *__restrict__ beta, float eps,
                                                    uint8_t *__restrict__ xp)
{
    __shared__ float red[16];
    const int m = blockIdx.x;
    const int nsb = K >> 5, items = K >> 3;
    const float *xr = x + (int64_t)m * x_stride;
    const bool live = m < M;
    float sc = 1.0f, mean = 0.0f;
    if (live && pro == PRO_RMS) {
        float ss = 0.0f;
        for (int i = threadIdx.x; i < items; i += 256) {
            float v[8];
            unpack8(((const float4 *)xr)[2 * i], ((const float4 *)xr)[2 * i + 1], v);
#pragma unroll
            for (int k = 0; k < 8; k++) { const float q = v[k] * v[k]; ss += q; }
        }
        ss = block_sum<4>(ss, red);
        sc = 1.0f / sqrtf(ss / (float)K + eps);
    } else if (live && pro == PRO_LN) {
        float tsum = 0.0f;
        for (int i = threadIdx.x; i < items; i += 256) {
            float v[8];
            unpack8(((const float4 *)xr)[2 * i], ((const float4 *)xr)[2 * i + 1], v);
#pragma unroll
            for (int k = 0; k < 8; k++) tsum += v[k];
        }
        mean = block_sum<4>(tsum, red) / (float)K;
        float sq = 0.0f;
        for (int i = threadIdx.x; i < items; i += 256) {
            float v[8];
            unpack8(((const float4 *)xr)[2 * i], ((const float4 *)xr)[2 * i + 1], v);
#pragma unroll
            for (int k = 0; k < 8; k++) { const float dd = v[k] - mean; const float q = dd * dd; sq += q; }
        }
        sq = block_sum<4>(sq, red);
        sc = 1.0f / sqrtf(sq / (float)K + eps);
    }
    const int tt = m >> 4, t = m & 15;
    for (int i = threadIdx.x; i < items; i += 256) {
        float v[8];
        if (live) {
            unpack8(((const float4 *)xr)[2 * i], ((const float4 *)xr)[2 * i + 1], v);
            if (pro == PRO_RMS) {
                float gg[8];
                unpack8(((const float4 *)gamma)[2 * i], ((const float4 *)gamma)[2 * i + 1], gg);
#pragma unroll
                for (int k = 0; k < 8; k++) v[k] = gg[k] * (v[k] * sc);
            } else if (pro == PRO_LN) {
                float gg[8], be[8];
                unpack8(((const float4 *)gamma)[2 * i], ((const float4 *)gamma)[2 * i + 1], gg);
                unpack8(((const float4 *)beta)[2 * i], ((const float4 *)beta)[2 * i + 1], be);
#pragma unroll
                for (int k = 0; k < 8; k++) v[k] = __builtin_fmaf(gg[k], (v[k] - mean) * sc, be[k]);
            }
        } else {
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = 0.0f;
        }
        qprep_store(v, xp, nsb, tt, t, i);
    }
}

template <int F, int RT, int TT, int NW, int SB>
hipError_t launch_frt(const QgemmArgs &a, hipStream_t s)
{
    const dim3 grid((unsigned)((a.w.rows + 16 * RT - 1) / (16 * RT)), (unsigned)(((a.M + 15) / 16 + TT - 1) / TT));
    hipLaunchKernelGGL((k_qgemm<F, RT, TT, NW, SB>), grid, dim3(64 * NW), 0, s, a);
    return hipGetLastError();
}

template <int F, int RT, int TT, int NW, int TS = 1>
hipError_t launch_st(const QgemmArgs &a, hipStream_t s)
{
    const uint32_t R = (uint32_t)((a.w.rows + 16 * RT - 1) / (16 * RT));
    // with a token split, one workgroup per 16 / TS tokens of the (single) token tile
    const uint32_t T = TS > 1 ? (uint32_t)((a.M + 16 / TS - 1) / (16 / TS))
                              : (uint32_t)(((a.M + 15) / 16 + TT - 1) / TT);
    if (TS > 1 && a.M > 16) return hipErrorInvalidValue;
    TileSched ts{R, T, 0, 0};
    dim3 grid(R, T);
    // From 1024 tokens: panels of G token groups whose activation parts (TT tiles x K/32
    // sub-blocks x 3 KB each) fill ~1.5 MB of an XCD's 4 MB L2.  Measured (configs[3] Q8_0 at
    // 2048 tokens): L2 fills 2-2.3x lower (gate/up 16x -> 8.6x the algorithmic bytes), kernel
    // times 0-2 % lower; at 511 tokens the 2-D order is 2-5 % faster, so shorter chunks keep it.
    if (TT > 1 && T > 1 && a.M >= 1024) {
        const uint64_t group_bytes = (uint64_t)TT * (uint64_t)(a.w.cols / 32) * 3072u;
        ts.G = (uint32_t)std::min<uint64_t>(T, std::max<uint64_t>(1, (3u << 19) / group_bytes));
        ts.chunk = (R * T + 7) / 8;
        grid = dim3(8 * ts.chunk, 1);
    }
    hipLaunchKernelGGL((k_qgemm_st<F, RT, TT, NW, TS>), grid, dim3(64 * NW), 0, s, a, ts);
    return hipGetLastError();
}

template <int F, int NR, int NKH, int NS>
hipError_t launch_rs(const QgemmArgs &a, hipStream_t s)
{
    const dim3 grid((unsigned)((a.w.rows + 16 * NR - 1) / (16 * NR)));
    hipLaunchKernelGGL((k_qgemm_rs<F, NR, NKH, NS>), grid, dim3(64 * NR * NKH), 0, s, a);
    return hipGetLastError();
}

template <int F>
hipError_t launch_f(const QgemmArgs &a, hipStream_t s)
{
    // Rows of whole 256-element super-blocks: LDS-staged weight tiles.  Up to 16 tokens: one
    // token tile per workgroup (16 waves splitting K from 8192 up).  More: per wave RT x 16
    // rows by TT x 16 tokens, NW waves splitting K; chosen by measurement (matrix-core GEMM
    // with its k_qprep, weights resident) at 256-token chunks and at the 512 / 2048-token
    // chunks of the configs[2] / configs[3] prompts:
    //  - K-quants (Q4_K / Q5_K): tall matrices 64 rows x 32 tokens, 4 waves; few rows or long
    //    K (O, down) the same above 320 tokens (Q4_K O 47.8 -> 39.7 us, down 92.0 -> 82.0 at
    //    512), 32 x 64 with 8 waves up to 320; other shapes (QKV) 32 x 32, 4 waves (Q4_K QKV 52.5
    //    -> 45.9 us at 512, Q5_K 52.1 -> 50.4 at 256);
    //  - Q8_0 / Q4_0 / SMQ: 32 x 64, 4 waves; few rows or long K with 8 waves below 1024
    //    tokens (Q8_0 O 165 -> 131 us, down 346 -> 317 at 2048 tokens with 4);
    //  - Q6_K: 32 x 64 with 8 waves on few rows or long K, else 16 x 64.
    if (a.w.cols % 256 == 0) {
        const bool tall = a.w.rows >= 8192;
        if (a.M > 16) {
            const bool narrow = a.w.cols > 4096 || a.w.rows <= 2048;
            if constexpr (F == FMT_Q4_K || F == FMT_Q5_K) {
                if (tall || (narrow && a.M > 320)) return launch_st<F, 4, 2, 4>(a, s);
                if (narrow) return launch_st<F, 2, 4, 8>(a, s);
                return launch_st<F, 2, 2, 4>(a, s);
            }
            if constexpr (F == FMT_Q6_K) return narrow ? launch_st<F, 2, 4, 8>(a, s) : launch_st<F, 1, 4, 8>(a, s);
            // (SMQ Q8's two staged scale words per sub-block do not fit 8 waves' registers)
            if constexpr (F != FMT_SQ8)
                if (narrow && a.M < 1024) return launch_st<F, 2, 4, 8>(a, s);
            return launch_st<F, 2, 4, 4>(a, s);
        }
        // tall K-quant matrices up to one workgroup of 64 rows per CU: the row-split kernel
        // (configs[4] gate/up 16.9 -> 13.6 us); up to 192 rows per CU, 12 row tiles of 16 rows
        // per workgroup, each wave all of K, a two-slot ring (117 KB of LDS: one workgroup per
        // CU in a single round; the 64-row form took three rounds on the 49152-row head, which
        // the K-split kernel's several workgroups per CU beat): configs[4] step 1.536 -> 1.528 ms
        if constexpr (F == FMT_Q4_K || F == FMT_Q5_K) {
            if (tall && a.w.rows <= 256 * 64) return launch_rs<F, 4, 2, 3>(a, s);
            if (tall && a.w.rows <= 256 * 192) return launch_rs<F, 12, 1, 2>(a, s);
        }
        // 16 waves of >= 2 super-blocks (Q6_K and Q4_0 would spill at 128 registers)
        if constexpr (F != FMT_Q6_K && F != FMT_Q4_0)
            if (a.w.cols >= 8192) return a.M > 8 ? launch_st<F, 1, 1, 16, 2>(a, s) : launch_st<F, 1, 1, 16>(a, s);
        return tall ? launch_st<F, 2, 1, 4>(a, s) : launch_st<F, 1, 1, 8>(a, s);
    }
    // Rows of 32-element blocks only (K-quant rows are whole super-blocks).  Up to 16 tokens:
    // one token tile, 16 waves per workgroup splitting K, 4 sub-blocks per wave in flight.  More
    // tokens: 4 token tiles per workgroup (the weight codes are reused across 64 tokens), 4
    // waves, 2 sub-blocks in flight.
    if constexpr (F == FMT_Q4_K || F == FMT_Q5_K || F == FMT_Q6_K) {
        return hipErrorInvalidValue;
    } else {
        if (a.M > 16) return launch_frt<F, 1, 4, 4, 2>(a, s);
        if (a.w.rows >= 16 * 2 * 512) return launch_frt<F, 2, 1, 16, 4>(a, s);
        return launch_frt<F, 1, 1, 16, 4>(a, s);
    }
}

template <int F, int RT, int TT, int NW, int SB>
hipError_t launch_drt(const QgemmArgs &a, hipStream_t s)
{
    const dim3 grid((unsigned)((a.w.rows + 16 * RT - 1) / (16 * RT)), (unsigned)(((a.M + 15) / 16 + TT - 1) / TT));
    hipLaunchKernelGGL((k_dgemm<F, RT, TT, NW, SB>), grid, dim3(64 * NW), 0, s, a);
    return hipGetLastError();
}

// F16 / F32 weights: the decomposition of the unstaged quantized kernel (4 token tiles per
// workgroup above 16 tokens, else one tile and 16 waves splitting K).
template <int F>
hipError_t launch_d(const QgemmArgs &a, hipStream_t s)
{
    constexpr int SB = F == FMT_F32 ? 2 : 4;   // F32 with 4 in flight would spill at 128 registers
    if (a.M > 16) return launch_drt<F, 1, 4, 4, 2>(a, s);
    if (a.w.rows >= 16 * 2 * 512) return launch_drt<F, 2, 1, 16, SB>(a, s);
    return launch_drt<F, 1, 1, 16, SB>(a, s);
}

}  // namespace

size_t qgemm_xp_bytes(int M, int K) { return (size_t)(((int64_t)M + 15) / 16) * (size_t)(K / 32) * 3 * 1024; }

hipError_t launch_qgemm(const QgemmArgs &a, const float *x, int64_t x_stride, int pro,
                        const float *gamma, const float *beta, float eps, hipStream_t s)
{
    if (a.M <= 0 || a.w.cols % 32 != 0 || (pro != PRO_NONE && !gamma) || (pro == PRO_LN && !beta))
        return hipErrorInvalidValue;
    if ((a.epi == EPI_SILU || a.epi == EPI_QKV) && (a.w.rows & 1)) return hipErrorInvalidValue;
    if ((uint64_t)a.w.rows * (uint64_t)a.w.nb * (uint64_t)fmt_main_bytes(a.w.fmt) >= (1ull << 32))
        return hipErrorInvalidValue;
    const int K = (int)a.w.cols;
    if ((!x && pro != PRO_NONE) || (a.yp && (a.epi == EPI_SILU ? a.w.rows % 64 : a.w.rows % 32)) ||
        (a.yp && a.epi != EPI_SILU && a.epi != EPI_GELU))
        return hipErrorInvalidValue;
    // folded RMSNorm: one token tile on the staged path (block formats only)
    if ((a.rss || a.np) && (a.M > 16 || K % 256 != 0 || fmt_dense(a.w.fmt))) return hipErrorInvalidValue;
    if (a.rss && (x || pro != PRO_NONE || a.rss_n < 1 || a.rss_n > 256)) return hipErrorInvalidValue;
    if (a.np && (a.epi != EPI_RESID || a.w.rows % 32 != 0 || !a.ngamma || !a.nss)) return hipErrorInvalidValue;
    const unsigned mp = (unsigned)((a.M + 15) / 16 * 16);
    int ipt = (K / 8 + 255) / 256;
#define SMX_QPREP(KN) hipLaunchKernelGGL(KN, dim3(mp), dim3(256), 0, s, x, x_stride, a.M, K, pro, gamma, beta, eps, (uint8_t *)a.xp)
    if (!x) ipt = -1;   // the parts are already in a.xp (written by the producing kernel)
    switch (ipt) {
    case -1: break;
    case 1: SMX_QPREP(k_qprep<1>); break;
    case 2: SMX_QPREP(k_qprep<2>); break;
    case 3: SMX_QPREP(k_qprep<3>); break;
    case 4: SMX_QPREP(k_qprep<4>); break;
    default: SMX_QPREP(k_qprep_long); break;
    }
#undef SMX_QPREP
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    switch (a.w.fmt) {
    case FMT_Q4_0: return launch_f<FMT_Q4_0>(a, s);
    case FMT_Q8_0: return launch_f<FMT_Q8_0>(a, s);
    case FMT_SQ4: return launch_f<FMT_SQ4>(a, s);
    case FMT_SQ8: return launch_f<FMT_SQ8>(a, s);
    case FMT_Q4_K: return launch_f<FMT_Q4_K>(a, s);
    case FMT_Q5_K: return launch_f<FMT_Q5_K>(a, s);
    case FMT_Q6_K: return launch_f<FMT_Q6_K>(a, s);
    case FMT_F16: return launch_d<FMT_F16>(a, s);
    case FMT_F32: return launch_d<FMT_F32>(a, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace smx
