// k_attn_prefill.hip -- causal attention of a run of consecutive tokens of one session over its
// KV cache, on the fp32 matrix cores (prefill chunks).
//
// Reference: MultiHeadAttention.Forward with T > 1 tokens over the KV cache
// (MultiHeadAttention.cs:206-297): scores Q.K^T per head (ComputeAttentionScoresInPlace,
// :676-745, MatMulOps.MatMulTransposeB), OptimizedOps.FusedScaleMaskSoftmax
// (OptimizedOps.cs:39-93) -- for query i at position p_first + i: s_j = (q.k_j) * scale for
// j <= p_first + i, max, e_j = FastExp(s_j - max) (MathUtils.cs:20-32), sum, w_j = e_j / sum --
// then out = W.V (ApplyAttentionInPlace, :810-845).
//
// The softmax needs the exact row maximum before any exponential (the Pade FastExp is not
// multiplicative, so flash-style online rescaling would not reproduce the reference), so the
// kernel makes two passes over the keys: pass 1 computes the scores and the row maxima, pass 2
// recomputes the same scores (same instruction sequence, same bits), exponentiates, sums and
// accumulates E.V.  The output is (sum_j e_j v_j) / sum, the reference's sum_j (e_j / sum) v_j
// up to rounding.
//
// Work decomposition.  A workgroup owns 32 query rows of one KV head: 32 / G tokens x the G
// query heads that share the KV head (GQA), so every K/V element it loads serves 32 rows.  Its
// 8 waves split the keys in 16-key tiles (wave w: tiles w, w + 8, ...).  A wave loads one tile
// at a time: without a register copy of the next tile the kernel takes 115 VGPRs and two
// workgroups fit a CU, whose other waves hide the loads (prefill +0.6-1.3 % against one
// workgroup per CU with the next tile's loads in flight).  Partial maxima, sums and
// outputs of the 8 waves are combined through LDS in a fixed order.
//
// Matrix cores: v_mfma_f32_16x16x4_f32 (fp32 products, fp32 accumulation).
//   S^T = K . Q^T per (16-key tile, 16-row block): A = K (lane: key l % 16, dimension
//   4j + l / 16 for step j), B = Q^T (lane: query l % 16, same dimension); D lane l holds keys
//   4(l/16) + i of query l % 16.
//   O = E . V per (16-row block, 16-dimension block): A = E (lane: query l % 16, key
//   4(l/16) + j for step j -- exactly the scores lane l already holds), B = V (lane: dimension
//   l % 16, key 4(l/16) + j); D lane l holds queries 4(l/16) + i of dimension l % 16.
// K is dimension-major [HD][ctx_stride] and V position-major [ctx_stride][HD]: for one step,
// lanes l % 16 read 16 consecutive floats of one row, four rows per load instruction.
#include "smx_device.h"
#include "smx_internal.h"

namespace smx {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mma(float a, float b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr int kHD = 64;          // head dimension of this kernel
constexpr int kRows = 32;        // query rows per workgroup (two 16-row blocks)
constexpr int kWaves = 8;
constexpr int kPitch = kHD + 4;  // LDS row pitch of the partial outputs (conflict-free writes)

// Maximum / sum over the four 16-lane rows (lanes l, l^16, l^32, l^48), the same bits in all.
__device__ __forceinline__ float rows_max(float v)
{
    float2 p = swap32(v, v);
    v = fmaxf(p.x, p.y);
    p = swap16(v, v);
    return fmaxf(p.x, p.y);
}
__device__ __forceinline__ float rows_sum(float v)
{
    float2 p = swap32(v, v);
    v = p.x + p.y;
    p = swap16(v, v);
    return p.x + p.y;
}

// With pb.blk set (several sessions' runs of a batch in one launch), workgroup b's rows, cache
// and first position come from the block table instead of the arguments: q, out and tok_off
// move to the block's first batch row, and the block is a run of M <= TT tokens at t0 = 0.
__global__ __launch_bounds__(kWaves * 64) void k_attn_prefill(
    const float *__restrict__ q, int q_stride, const float *__restrict__ kc, const float *__restrict__ vc,
    float *__restrict__ out, int out_stride, int n_head, int n_kv_head, int ctx_stride, int p_first, int M,
    uint8_t *__restrict__ out_parts, int tok_off, PrefillBlocks pb)
{
    extern __shared__ float s_out[];          // [kWaves][kRows][kPitch]
    __shared__ float s_max[kWaves][kRows], s_sum[kWaves][kRows], s_inv[kRows];
    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const int li = lane & 15, g = lane >> 4;
    const int G = n_head / n_kv_head, TT = kRows / G;
    const int kvh = blockIdx.y;
    int t0 = blockIdx.x * TT;
    if (pb.blk) {   // uniform over the workgroup
        const int r0 = pb.blk[2 * blockIdx.x];
        M = pb.blk[2 * blockIdx.x + 1];
        t0 = 0;
        kc = pb.kc_tok[r0] + pb.layer_off;
        vc = pb.vc_tok[r0] + pb.layer_off;
        p_first = pb.pos[r0];
        q += (int64_t)r0 * q_stride;
        out += (int64_t)r0 * out_stride;
        tok_off += r0;
    }
    const float scale = 1.0f / sqrtf((float)kHD);   // MultiHeadAttention.cs:682

    // this lane's query in row block rb: row 16 rb + li
    int npos[2];
    float qv[2][16];
#pragma unroll
    for (int rb = 0; rb < 2; rb++) {
        const int r = 16 * rb + li;
        const int t = min(t0 + r / G, M - 1), h = kvh * G + r % G;
        npos[rb] = p_first + t + 1;
        const float *qr = q + (int64_t)t * q_stride + (int64_t)h * kHD;
#pragma unroll
        for (int j = 0; j < 16; j++) qv[rb][j] = qr[4 * j + g];
    }
    const int n_max = p_first + min(t0 + TT, M);   // keys 0 .. n_max-1 are written cache entries
    const int n_tiles = (n_max + 15) >> 4;
    // K and V of one KV head span less than 4 GiB: uniform base + 32-bit offsets
    const float *K = kc + (int64_t)kvh * kHD * ctx_stride;
    const float *V = vc + (int64_t)kvh * ctx_stride * kHD;
    const uint32_t cs = (uint32_t)ctx_stride;

    auto load_k = [&](int ti, float *dst) {
        const uint32_t key = (uint32_t)min(16 * ti + li, ctx_stride - 1);
#pragma unroll
        for (int j = 0; j < 16; j++) dst[j] = K[(uint32_t)(4 * j + g) * cs + key];
    };
    auto load_v = [&](int ti, float (*dst)[4]) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t key = (uint32_t)min(16 * ti + 4 * g + j, ctx_stride - 1);
#pragma unroll
            for (int mb = 0; mb < 4; mb++) dst[j][mb] = V[key * kHD + 16 * mb + li];
        }
    };
    // scores of one tile: s[rb][i] = key 16 ti + 4 g + i, query li of row block rb (scaled)
    auto scores = [&](const float *kv, float (*s)[4]) {
        f32x4 a0 = {0.0f, 0.0f, 0.0f, 0.0f}, a1 = a0;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            a0 = mma(kv[j], qv[0][j], a0);
            a1 = mma(kv[j], qv[1][j], a1);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            s[0][i] = a0[i] * scale;
            s[1][i] = a1[i] * scale;
        }
    };

    // ---- pass 1: row maxima -----------------------------------------------------------------
    float mx[2] = {-INFINITY, -INFINITY};
    {
        float kv[16];
        int ti = w;
        for (; ti < n_tiles; ti += kWaves) {
            load_k(ti, kv);
            float s[2][4];
            scores(kv, s);
#pragma unroll
            for (int rb = 0; rb < 2; rb++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (16 * ti + 4 * g + i < npos[rb]) mx[rb] = fmaxf(mx[rb], s[rb][i]);
        }
    }
#pragma unroll
    for (int rb = 0; rb < 2; rb++) {
        mx[rb] = rows_max(mx[rb]);
        if (g == 0) s_max[w][16 * rb + li] = mx[rb];
    }
    __syncthreads();
#pragma unroll
    for (int rb = 0; rb < 2; rb++) {
        float m = s_max[0][16 * rb + li];
#pragma unroll
        for (int v = 1; v < kWaves; v++) m = fmaxf(m, s_max[v][16 * rb + li]);
        mx[rb] = m;
    }

    // ---- pass 2: exponentials, sums and E.V --------------------------------------------------
    float sum[2] = {0.0f, 0.0f};
    f32x4 o[2][4];
#pragma unroll
    for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int mb = 0; mb < 4; mb++) o[rb][mb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    {
        float kv[16], vv[4][4];
        int ti = w;
        for (; ti < n_tiles; ti += kWaves) {
            load_k(ti, kv);
            load_v(ti, vv);
            float s[2][4];
            scores(kv, s);
#pragma unroll
            for (int rb = 0; rb < 2; rb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const bool ok = 16 * ti + 4 * g + i < npos[rb];
                    const float e = ok ? fastexp(s[rb][i] - mx[rb]) : 0.0f;
                    s[rb][i] = e;
                    sum[rb] += e;
                }
            // V rows past the written cache entries may hold anything: zero them (0 * NaN)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const bool ok = 16 * ti + 4 * g + j < n_max;
#pragma unroll
                for (int mb = 0; mb < 4; mb++) {
                    const float vz = ok ? vv[j][mb] : 0.0f;
                    o[0][mb] = mma(s[0][j], vz, o[0][mb]);
                    o[1][mb] = mma(s[1][j], vz, o[1][mb]);
                }
            }

        }
    }
    // partial sums and outputs of this wave to LDS
#pragma unroll
    for (int rb = 0; rb < 2; rb++) {
        const float sm = rows_sum(sum[rb]);
        if (g == 0) s_sum[w][16 * rb + li] = sm;
#pragma unroll
        for (int mb = 0; mb < 4; mb++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                s_out[(w * kRows + 16 * rb + 4 * g + i) * kPitch + 16 * mb + li] = o[rb][mb][i];
    }
    __syncthreads();
    if (tid < kRows) {
        float sm = s_sum[0][tid];
#pragma unroll
        for (int v = 1; v < kWaves; v++) sm += s_sum[v][tid];
        s_inv[tid] = 1.0f / sm;
    }
    __syncthreads();
    // combine: thread -> (row r, 4 dimensions)
    const int r = tid >> 4, d4 = (tid & 15) * 4;
    float4 acc = *(const float4 *)&s_out[r * kPitch + d4];
#pragma unroll
    for (int v = 1; v < kWaves; v++) {
        const float4 p = *(const float4 *)&s_out[(v * kRows + r) * kPitch + d4];
        acc.x += p.x; acc.y += p.y; acc.z += p.z; acc.w += p.w;
    }
    const int t = t0 + r / G;
    if (t < M) {
        const float inv = s_inv[r];
        acc.x *= inv; acc.y *= inv; acc.z *= inv; acc.w *= inv;
        const int h = kvh * G + r % G;
        if (out_parts) {
            const int nsb = n_head * kHD / 32, k = h * kHD + d4;
            xp_store(out_parts, nsb, tok_off + t, k, acc.x);
            xp_store(out_parts, nsb, tok_off + t, k + 1, acc.y);
            xp_store(out_parts, nsb, tok_off + t, k + 2, acc.z);
            xp_store(out_parts, nsb, tok_off + t, k + 3, acc.w);
        } else {
            *(float4 *)(out + (int64_t)t * out_stride + (int64_t)h * kHD + d4) = acc;
        }
    }
}

}  // namespace

bool attention_prefill_supported(int n_head, int n_kv_head, int hd)
{
    if (hd != kHD || n_kv_head <= 0 || n_head % n_kv_head) return false;
    const int G = n_head / n_kv_head;
    return G <= kRows && kRows % G == 0;
}

hipError_t launch_attention_prefill(const float *q, int q_stride, const float *kc, const float *vc, float *out,
                                    int out_stride, int n_head, int n_kv_head, int hd, int ctx_stride,
                                    int p_first, int M, hipStream_t s, uint8_t *out_parts, int tok_off)
{
    if (!attention_prefill_supported(n_head, n_kv_head, hd) || M <= 0 || p_first < 0 || ((n_head * hd) & 31) ||
        p_first + M > ctx_stride || (q_stride & 3) || (out_stride & 3) || tok_off < 0)
        return hipErrorInvalidValue;
    const size_t lds = (size_t)kWaves * kRows * kPitch * 4;
    const hipError_t e = hipFuncSetAttribute((const void *)k_attn_prefill,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    const int TT = kRows / (n_head / n_kv_head);
    const dim3 grid((unsigned)((M + TT - 1) / TT), (unsigned)n_kv_head);
    hipLaunchKernelGGL(k_attn_prefill, grid, dim3(kWaves * 64), lds, s, q, q_stride, kc, vc, out, out_stride,
                       n_head, n_kv_head, ctx_stride, p_first, M, out_parts, tok_off, PrefillBlocks{});
    return hipGetLastError();
}

int attention_prefill_block_rows(int n_head, int n_kv_head) { return kRows / (n_head / n_kv_head); }

hipError_t launch_attention_prefill_blocks(const float *q, int q_stride, float *out, int out_stride, int n_head,
                                           int n_kv_head, int hd, int ctx_stride, int n_blocks,
                                           const PrefillBlocks &pb, hipStream_t s, uint8_t *out_parts)
{
    if (!attention_prefill_supported(n_head, n_kv_head, hd) || n_blocks <= 0 || !pb.blk || !pb.kc_tok ||
        !pb.vc_tok || !pb.pos || ((n_head * hd) & 31) || (q_stride & 3) || (out_stride & 3))
        return hipErrorInvalidValue;
    const size_t lds = (size_t)kWaves * kRows * kPitch * 4;
    const hipError_t e = hipFuncSetAttribute((const void *)k_attn_prefill,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    const dim3 grid((unsigned)n_blocks, (unsigned)n_kv_head);
    hipLaunchKernelGGL(k_attn_prefill, grid, dim3(kWaves * 64), lds, s, q, q_stride, nullptr, nullptr, out,
                       out_stride, n_head, n_kv_head, ctx_stride, 0, 0, out_parts, 0, pb);
    return hipGetLastError();
}

}  // namespace smx
