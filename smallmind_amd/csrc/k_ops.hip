// k_ops.hip -- norms, RoPE, softmax, decode attention, activations, embedding, argmax.
#include "smx_device.h"
#include "smx_formats.h"
#include "smx_attn.h"
#include "smx_prefetch.h"

namespace smx {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

// RMSNormOps.RMSNorm (RMSNormOps.cs:28-219): one workgroup per row.
__global__ __launch_bounds__(kThreads) void k_rmsnorm(const float *__restrict__ x,
                                                      const float *__restrict__ g,
                                                      float *__restrict__ y, int n, float eps)
{
    __shared__ float red[16];
    const float *xr = x + (int64_t)blockIdx.x * n;
    float *yr = y + (int64_t)blockIdx.x * n;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += kThreads) { float v = xr[i]; float p = v * v; ss += p; }
    ss = block_sum<kWaves>(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += kThreads) { float t = xr[i] * inv; yr[i] = g[i] * t; }
}

// LayerNormOps.LayerNorm (LayerNormOps.cs:27-280): two-pass mean / variance, affine by FMA.
__global__ __launch_bounds__(kThreads) void k_layernorm(const float *__restrict__ x,
                                                        const float *__restrict__ g,
                                                        const float *__restrict__ b,
                                                        float *__restrict__ y, int n, float eps)
{
    __shared__ float red[16];
    const float *xr = x + (int64_t)blockIdx.x * n;
    float *yr = y + (int64_t)blockIdx.x * n;
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += kThreads) s += xr[i];
    s = block_sum<kWaves>(s, red);
    const float mean = s / (float)n;
    float sq = 0.0f;
    for (int i = threadIdx.x; i < n; i += kThreads) { float dd = xr[i] - mean; float p = dd * dd; sq += p; }
    sq = block_sum<kWaves>(sq, red);
    const float inv = 1.0f / sqrtf(sq / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += kThreads) {
        float t = (xr[i] - mean) * inv;
        yr[i] = __builtin_fmaf(g[i], t, b[i]);
    }
}

// RotaryEmbedding.ApplyRotationInPlace (RotaryEmbedding.cs:85-121), data [heads][seq][hd].
__global__ void k_rope(float *__restrict__ data, int n_heads, int seq, int hd, int pos0,
                       const float *__restrict__ c, const float *__restrict__ sn)
{
    const int half = hd / 2;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)n_heads * seq * half) return;
    const int i = (int)(idx % half);
    const int64_t hs = idx / half;
    const int s = (int)(hs % seq);
    const int pos = pos0 + s;
    float *v = data + hs * hd;
    const float x0 = v[2 * i], x1 = v[2 * i + 1];
    const float cc = c[(int64_t)pos * half + i], ss = sn[(int64_t)pos * half + i];
    const float t0 = x0 * cc, t1 = x1 * ss, t2 = x0 * ss, t3 = x1 * cc;
    v[2 * i] = t0 - t1;
    v[2 * i + 1] = t2 + t3;
}

// OptimizedOps.FusedScaleMaskSoftmax (OptimizedOps.cs:39-93): one workgroup per row.
__global__ __launch_bounds__(kThreads) void k_softmax(float *__restrict__ scores, float scale,
                                                      int k_seq, int cache_off)
{
    __shared__ float red[16];
    float *row = scores + (int64_t)blockIdx.x * k_seq;
    const int valid = cache_off + (int)blockIdx.x + 1;
    float mx = -INFINITY;
    for (int j = threadIdx.x; j < valid; j += kThreads) mx = fmaxf(mx, row[j] * scale);
    mx = block_max<kWaves>(mx, red);
    float sum = 0.0f;
    for (int j = threadIdx.x; j < valid; j += kThreads) {
        float s = row[j] * scale;
        float e = fastexp(s - mx);
        row[j] = e;
        sum += e;
    }
    sum = block_sum<kWaves>(sum, red);
    const float inv = 1.0f / sum;
    for (int j = threadIdx.x; j < k_seq; j += kThreads) row[j] = j < valid ? row[j] * inv : 0.0f;
}

// Attention of one (token, head) by a whole workgroup (attention_head), as used by the token
// batches below: 256 threads; for head_dim 64 the score pass (one position per thread) covers
// 256 positions and the P.V pass (32 positions per thread) 512 per round of loads.  Measured
// on configs[4] (16 sessions x 32 heads, ~320 positions): 1.561 -> 1.545 ms per lockstep step
// against 512 threads x 16 positions (171 VGPRs, two waves per SIMD, no spills); 256 x 16 and
// 128 x 16 fell in between.
template <int HD> struct AttnCfg {
    static constexpr int NT = 256;
    static constexpr int U = HD <= 64 ? 32 : 8;
};

// Decode attention split over the whole chip in two launches (one workgroup per head would
// stream the head's K and V through one CU).  The kernel boundary between them
// supplies the exact maximum over all positions that the Pade FastExp needs before any
// exponential (MathUtils.cs:20-32; MultiHeadAttention.cs:676-844).
//
// 1. k_attn_scores: workgroup = (KV head, block of 32 positions).  The block of K
//    ([HD][32], dimension-major) is staged in LDS once and serves every query head of the
//    group: thread (position tl, head slot hs) computes q_h . k_t for heads h = hs, hs+8, ...
//    with the same FMA order as attention_head (dimension 0 first), then multiplies by
//    1/sqrt(HD).  Scores go to sc_out[head][ctx_stride].
// 2. k_attn_pv: workgroup = (query head, slice of 16 dimensions).  Each workgroup reads the
//    head's scores, takes the exact max, FastExp(s - max), the sum (fixed reduction order,
//    so every slice of a head obtains the same bits), scales by 1/sum, and accumulates
//    P.V for its slice (V is position-major, so a position's slice is 64 contiguous bytes).
constexpr int kScorePB = 32;    // positions per score workgroup
constexpr int kPvSlice = 16;    // dimensions per P.V workgroup
constexpr int kPvChunk = 2304;  // positions per workgroup of the two-chunk P.V (128 lanes x 18)


template <int HD>
__global__ __launch_bounds__(256) void k_attn_scores(const float *__restrict__ q, const float *__restrict__ kc,
                                                     float *__restrict__ sc_out, int n_head, int n_kv_head,
                                                     int ctx_stride, int sc_stride, const int32_t *__restrict__ pos_dev,
                                                     int n_pos_fixed, int nblk)
{
    __shared__ float ks[HD][kScorePB];
    extern __shared__ float4 qs4[];   // [G][HD / 4]
    const int G = n_head / n_kv_head, GQ4 = G * HD / 4;
    const int g = blockIdx.x / nblk, blk = blockIdx.x % nblk;
    const int t0 = blk * kScorePB;
    const int tid = threadIdx.x, tl = tid & (kScorePB - 1), hs = tid >> 5;
    const float *K = kc + (int64_t)g * HD * ctx_stride;
    const int t = t0 + tl;
    // The loads do not wait for the position: every column index is clamped into the cache
    // row (valid memory), and columns at or past n_pos are never stored.
    const int tc = min(t, ctx_stride - 1);
    float kr[HD / 8];
#pragma unroll
    for (int i = 0; i < HD / 8; i++) kr[i] = K[(int64_t)(hs + 8 * i) * ctx_stride + tc];
    const float4 *qg = (const float4 *)(q + (int64_t)g * G * HD);
    float4 qr[2];   // the first 2048 floats of the group's queries
#pragma unroll
    for (int i = 0; i < 2; i++) qr[i] = qg[min(tid + 256 * i, GQ4 - 1)];
    const int n_pos = pos_dev ? ld_uniform(pos_dev) + 1 : n_pos_fixed;
#pragma unroll
    for (int i = 0; i < HD / 8; i++) ks[hs + 8 * i][tl] = kr[i];
#pragma unroll
    for (int i = 0; i < 2; i++)
        if (tid + 256 * i < GQ4) qs4[tid + 256 * i] = qr[i];
    for (int i = tid + 512; i < GQ4; i += 256) qs4[i] = qg[i];   // groups beyond 2048 floats
    if (t0 >= n_pos) return;   // uniform over the workgroup
    __syncthreads();
    const float *qs = (const float *)qs4;
    const float scale = 1.0f / sqrtf((float)HD);   // MultiHeadAttention.cs:686
    for (int hg = hs; hg < G; hg += 8) {
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < HD; e++) s = __builtin_fmaf(qs[hg * HD + e], ks[e][tl], s);
        if (t < n_pos) sc_out[(int64_t)(g * G + hg) * sc_stride + t] = s * scale;
    }
}

// NCH = 2: the positions are split over two workgroups per (head, slice), each taking its
// half (NB positions) and writing a partial output at out + chunk * n_head * HD; the O
// projection sums the two (GemvArgs::x_parts).  Both compute the softmax statistics over all
// positions in the same order, so they use the same max, sum and weights.
template <int HD, int U, int NT, int NCH>
__global__ __launch_bounds__(NT) void k_attn_pv(const float *__restrict__ scores, const float *__restrict__ vc,
                                                float *__restrict__ out, int n_head, int n_kv_head,
                                                int ctx_stride, int sc_stride, const int32_t *__restrict__ pos_dev,
                                                int n_pos_fixed)
{
    constexpr int NW = NT / 64;         // waves
    constexpr int NS = HD / kPvSlice;   // slices per head
    constexpr int C4 = kPvSlice / 4;    // float4 columns per slice
    constexpr int PL = NT / C4;         // position lanes
    // U: consecutive positions per lane in the first batch (sized by the launcher to the
    // session's context, so the first batch loads no rows past it)
    constexpr int NB = PL * U;          // positions of the first batch
    extern __shared__ float p[];        // [n_pos], only for n_pos > NB
    __shared__ float red[16];
    __shared__ float4 part[NW][C4];
    // Workgroups are dealt to the 8 XCDs round-robin; consecutive (head, slice) indices are
    // grouped per XCD so that the query heads of one KV head share that XCD's L2.
    const int T = n_head * NS * NCH, b = blockIdx.x;
    const int Lc = (T % 8 == 0) ? (b % 8) * (T / 8) + b / 8 : b;
    const int L = Lc / NCH, chunk = Lc % NCH;
    const int h = L / NS, slice = L % NS;
    const int kvh = h / (n_head / n_kv_head);
    const int tid = threadIdx.x;
    const int c4 = tid % C4, pl = tid / C4;
    const float *srow = scores + (int64_t)h * sc_stride;
    const char *Vb = (const char *)(vc + (int64_t)kvh * ctx_stride * HD + slice * kPvSlice);
    auto vload = [&](int j) {
        return *(const float4 *)(Vb + 4u * ((uint32_t)j * HD + 4u * (uint32_t)c4));
    };
    // Lane pl owns positions j0 .. j0 + U - 1 of the first batch.  Its scores and V rows are
    // all loaded up front, before the position is known, with indices clamped into the cache
    // row (valid memory; entries at or past n_pos are dropped by selection, never multiplied),
    // so the scores arrive first and V streams in while the softmax is computed.
    const int j0 = chunk * NB + pl * U;
    // NCH = 1: the lane's own positions' scores; NCH = 2: positions tid + NT*u of both chunks
    // for the statistics (NPT per thread)
    constexpr int NPT = NCH == 1 ? U : 2 * NB / NT;
    float sv[NPT];
    if constexpr (NCH == 1) {
#pragma unroll
        for (int u = 0; u < U; u += 4) {
            const int j = min(j0 + u, sc_stride - 4);   // sc_stride is a multiple of 4
            const float4 t = *(const float4 *)(srow + j);
            sv[u] = t.x; sv[u + 1] = t.y; sv[u + 2] = t.z; sv[u + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int u = 0; u < NPT; u++) sv[u] = srow[min(tid + NT * u, sc_stride - 1)];
    }
    __builtin_amdgcn_sched_barrier(0);
    float4 vv[U];
#pragma unroll
    for (int u = 0; u < U; u++) vv[u] = vload(min(j0 + u, ctx_stride - 1));
    __builtin_amdgcn_sched_barrier(0);
    const int n_pos = pos_dev ? ld_uniform(pos_dev) + 1 : n_pos_fixed;
    float pu[U];
    if constexpr (NCH == 2) {
        // statistics over all positions (the same order in every workgroup of the head), the
        // weights of every position into LDS, then this lane's
        float mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < NPT; u++)
            if (tid + NT * u < n_pos) mx = fmaxf(mx, sv[u]);
        mx = block_max<NW>(mx, red);
        float sum = 0.0f;
#pragma unroll
        for (int u = 0; u < NPT; u++) {
            const float e = tid + NT * u < n_pos ? fastexp(sv[u] - mx) : 0.0f;
            sv[u] = e;
            sum += e;
        }
        sum = block_sum<NW>(sum, red);
        const float inv = 1.0f / sum;
#pragma unroll
        for (int u = 0; u < NPT; u++)
            if (tid + NT * u < n_pos) p[tid + NT * u] = sv[u] * inv;
        __syncthreads();
#pragma unroll
        for (int u = 0; u < U; u++) pu[u] = p[min(j0 + u, n_pos - 1)];   // j0 + u >= n_pos: dropped below
    } else if (n_pos <= NB) {
        // Whole softmax in registers.  The C4 = 4 lanes of a position lane form a DPP quad
        // holding the same positions: lane c4 takes the exact max over its quarter, computes
        // FastExp for positions j0 + 4*c4 .. +3 and the quad shares the results; the sum runs
        // over every lane once per position, in the same order in every workgroup of the head.
        static_assert(C4 == 4 && U % 4 == 0, "one quarter of the positions per lane of a quad");
        constexpr int UQ = U / 4;
        float mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < U; u++)
            if (j0 + u < n_pos) mx = fmaxf(mx, sv[u]);
        mx = block_max<NW>(mx, red);
        float e[UQ], sum = 0.0f;
#pragma unroll
        for (int k = 0; k < UQ; k++) {
            const int u = UQ * c4 + k;
            float sk = sv[k];
#pragma unroll
            for (int i = 1; i < 4; i++) sk = c4 == i ? sv[UQ * i + k] : sk;
            e[k] = j0 + u < n_pos ? fastexp(sk - mx) : 0.0f;
            sum += e[k];
        }
        sum = block_sum<NW>(sum, red);
        const float inv = 1.0f / sum;
#pragma unroll
        for (int k = 0; k < UQ; k++) {
            e[k] = e[k] * inv;
            pu[k] = dpp_mov<0x00>(e[k]);             // quad_perm [0,0,0,0]
            pu[UQ + k] = dpp_mov<0x55>(e[k]);        // quad_perm [1,1,1,1]
            pu[2 * UQ + k] = dpp_mov<0xAA>(e[k]);    // quad_perm [2,2,2,2]
            pu[3 * UQ + k] = dpp_mov<0xFF>(e[k]);    // quad_perm [3,3,3,3]
        }
    } else {
        // long contexts: the scores of all positions pass through LDS, loaded in batches of
        // eight per thread (all loads of a batch in flight before any is used)
        float mx = -INFINITY;
        for (int jb = tid; jb < n_pos; jb += NT * 8) {
            float sb[8];
#pragma unroll
            for (int u = 0; u < 8; u++) sb[u] = srow[min(jb + NT * u, sc_stride - 1)];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int j = jb + NT * u;
                if (j < n_pos) {
                    p[j] = sb[u];
                    mx = fmaxf(mx, sb[u]);
                }
            }
        }
        mx = block_max<NW>(mx, red);
        float sum = 0.0f;
        for (int j = tid; j < n_pos; j += NT) {
            const float e = fastexp(p[j] - mx);
            p[j] = e;
            sum += e;
        }
        sum = block_sum<NW>(sum, red);
        const float inv = 1.0f / sum;
        for (int j = tid; j < n_pos; j += NT) p[j] = p[j] * inv;
        __syncthreads();
#pragma unroll
        for (int u = 0; u < U; u++) pu[u] = p[j0 + u];   // j0 + u < NB < n_pos
    }

    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int u = 0; u < U; u++) {
        if (j0 + u < n_pos) {
            const float pp = pu[u];
            acc.x = __builtin_fmaf(pp, vv[u].x, acc.x);
            acc.y = __builtin_fmaf(pp, vv[u].y, acc.y);
            acc.z = __builtin_fmaf(pp, vv[u].z, acc.z);
            acc.w = __builtin_fmaf(pp, vv[u].w, acc.w);
        }
    }
    // positions beyond the first batch (n_pos > NB): batches of U2 rows per lane, each batch's
    // loads (clamped into the row, dropped by selection) issued before the previous batch's
    // multiply-adds
    constexpr int U2 = 16;
    if (NCH == 1 && n_pos > NB) {
        float4 v2[U2];
        auto load2 = [&](int jb) {
#pragma unroll
            for (int u = 0; u < U2; u++) v2[u] = vload(min(jb + u * PL, ctx_stride - 1));
        };
        int jb = NB + pl;
        load2(jb);
        for (; jb < n_pos; jb += PL * U2) {
            float4 cur[U2];
#pragma unroll
            for (int u = 0; u < U2; u++) cur[u] = v2[u];
            if (jb + PL * U2 < n_pos) load2(jb + PL * U2);
#pragma unroll
            for (int u = 0; u < U2; u++) {
                const int j = jb + u * PL;
                if (j < n_pos) {
                    const float pp = p[j];
                    acc.x = __builtin_fmaf(pp, cur[u].x, acc.x);
                    acc.y = __builtin_fmaf(pp, cur[u].y, acc.y);
                    acc.z = __builtin_fmaf(pp, cur[u].z, acc.z);
                    acc.w = __builtin_fmaf(pp, cur[u].w, acc.w);
                }
            }
        }
    }
    // lanes with the same column: butterfly over lane bits C4, 2*C4, ..., 32; then the waves
#pragma unroll
    for (int m = C4; m < 64; m <<= 1) {
        acc.x += __shfl_xor(acc.x, m);
        acc.y += __shfl_xor(acc.y, m);
        acc.z += __shfl_xor(acc.z, m);
        acc.w += __shfl_xor(acc.w, m);
    }
    const int w = tid >> 6;
    if ((tid & 63) < C4) part[w][c4] = acc;
    __syncthreads();
    if (tid < C4) {
        float4 o = part[0][tid];
#pragma unroll
        for (int i = 1; i < NW; i++) {
            const float4 v = part[i][tid];
            o.x += v.x; o.y += v.y; o.z += v.z; o.w += v.w;
        }
        ((float4 *)(out + (int64_t)chunk * n_head * HD + (int64_t)h * HD + slice * kPvSlice))[tid] = o;
    }
}

// Decode attention of contexts up to NT * P <= 1024 positions in one launch (HD <= 64, cache
// rows 16-byte aligned: ctx_stride % 4 == 0): the workgroup = (query head, slice of 16
// dimensions) of k_attn_pv computes its head's scores itself instead of reading them from a
// previous launch.  Score phase: thread (dimension quarter dq, position group pg) loads, for
// each of P passes of NT positions, the keys of positions 4pg..4pg+3 over its HD/4
// dimensions as float4 rows of the dimension-major cache (a wave's load of one dimension is
// 1 KB contiguous) and forms four partial dot products with q read through the scalar
// cache; the quarters are added in LDS in a fixed order and scaled by 1/sqrt(HD).  Every key
// and V row of the workgroup is requested at entry, except with three passes, whose last
// pass's keys reuse the registers of the first.  Few large-register threads beat many small ones here:
// at the same context a workgroup of 1024 threads takes ~2.5 us longer than one of 256.
// Every workgroup of a head reads the head's K (n_pos * HD * 4 bytes; L2 serves all but the
// first).
template <int HD, int NT, int P>
__global__ __launch_bounds__(NT) void k_attn_dec(const float *__restrict__ q, const float *__restrict__ kc,
                                                 const float *__restrict__ vc, float *__restrict__ out,
                                                 int n_head, int n_kv_head, int ctx_stride,
                                                 const int32_t *__restrict__ pos_dev, int n_pos_fixed, Prefetch pf)
{
    if ((int)blockIdx.x >= n_head * (HD / kPvSlice)) {   // workgroups past the attention grid
        prefetch_slice(pf, (int)blockIdx.x - n_head * (HD / kPvSlice),
                       (int)gridDim.x - n_head * (HD / kPvSlice), NT);
        return;
    }
    constexpr int NW = NT / 64;
    constexpr int NS = HD / kPvSlice;   // slices per head
    constexpr int C4 = kPvSlice / 4;    // float4 columns per slice
    constexpr int U = 4 * P;            // consecutive positions per P.V lane (NT / C4 lanes)
    constexpr int NPG = NT / 4;         // position groups per pass
    constexpr int DQ = HD / 4;          // dimensions per quarter
    constexpr int NP = NT * P;          // positions covered
    static_assert(HD <= 64 && NP <= 1024 && NT % 256 == 0, "short-context decode attention");
    __shared__ __align__(16) float ps[4][NP];
    __shared__ __align__(16) float p[NP];
    __shared__ float red[16];
    __shared__ float4 part[NW][C4];
    const int T = n_head * NS, b = blockIdx.x;
    const int L = (T % 8 == 0) ? (b % 8) * (T / 8) + b / 8 : b;   // heads of a KV head share an XCD
    const int h = L / NS, slice = L % NS;
    const int kvh = h / (n_head / n_kv_head);
    const int tid = opaque_tid();
    const int c4 = tid % C4, j0 = (tid / C4) * U;
    const int dq = __builtin_amdgcn_readfirstlane(tid / NPG), pg = tid % NPG;
    const char *Kb = (const char *)(kc + (int64_t)kvh * HD * ctx_stride + (int64_t)dq * DQ * ctx_stride);
    const char *Vb = (const char *)(vc + (int64_t)kvh * ctx_stride * HD + slice * kPvSlice);
    // every load is issued before the position is known, with indices clamped into the cache
    // row (valid memory); entries at or past n_pos are dropped by selection, never multiplied
    const int lastg = ctx_stride / 4 - 1;
    auto kload = [&](float4 *kv, int pass, int lim) {
        const uint32_t pc = 4u * (uint32_t)min(pg + NPG * pass, lim);
#pragma unroll
        for (int e = 0; e < DQ; e++) kv[e] = *(const float4 *)(Kb + 4u * ((uint32_t)e * (uint32_t)ctx_stride + pc));
    };
    const float *qd = q + (int64_t)h * HD + dq * DQ;
    auto kdot = [&](const float4 *kv, int pass) {
        float4 sp = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int e = 0; e < DQ; e++) {
            const float qe = ld_uniform(qd + e);
            sp.x = __builtin_fmaf(qe, kv[e].x, sp.x);
            sp.y = __builtin_fmaf(qe, kv[e].y, sp.y);
            sp.z = __builtin_fmaf(qe, kv[e].z, sp.z);
            sp.w = __builtin_fmaf(qe, kv[e].w, sp.w);
        }
        *(float4 *)&ps[dq][4 * (pg + NPG * pass)] = sp;
    };
    constexpr int PA = P <= 2 ? P : P - 1;   // passes loaded at entry (registers: 16 * DQ * PA)
    float4 kv[PA][DQ];
#pragma unroll
    for (int i = 0; i < PA; i++) kload(kv[i], i, lastg);
    float4 vv[U];
#pragma unroll
    for (int u = 0; u < U; u++)
        vv[u] = *(const float4 *)(Vb + 4u * ((uint32_t)min(j0 + u, ctx_stride - 1) * HD + 4u * (uint32_t)c4));
    __builtin_amdgcn_sched_barrier(0);
    const int n_pos = pos_dev ? ld_uniform(pos_dev) + 1 : n_pos_fixed;
    kdot(kv[0], 0);
    if constexpr (PA < P) {
        // the last pass is issued once the position is known: groups past it re-read the last
        // written group instead of streaming cache entries not yet written
        __builtin_amdgcn_sched_barrier(0);
        kload(kv[0], P - 1, min(lastg, (n_pos - 1) >> 2));
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 1; i < PA; i++) kdot(kv[i], i);
    if constexpr (PA < P) kdot(kv[0], P - 1);
    __syncthreads();
    float sc[P], mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < P; i++) {
        const int j = tid + NT * i;
        float s = ps[0][j];
#pragma unroll
        for (int k = 1; k < 4; k++) s += ps[k][j];
        sc[i] = s * (1.0f / sqrtf((float)HD));   // MultiHeadAttention.cs:686
        if (j < n_pos) mx = fmaxf(mx, sc[i]);
    }
    mx = block_max<NW>(mx, red);
    float ev[P], sum = 0.0f;
#pragma unroll
    for (int i = 0; i < P; i++) {
        ev[i] = tid + NT * i < n_pos ? fastexp(sc[i] - mx) : 0.0f;
        sum += ev[i];
    }
    sum = block_sum<NW>(sum, red);
    const float inv = 1.0f / sum;
#pragma unroll
    for (int i = 0; i < P; i++) p[tid + NT * i] = ev[i] * inv;
    __syncthreads();
    float pu[U];
#pragma unroll
    for (int u = 0; u < U; u += 4) {
        const float4 pq = *(const float4 *)&p[j0 + u];
        pu[u] = pq.x; pu[u + 1] = pq.y; pu[u + 2] = pq.z; pu[u + 3] = pq.w;
    }
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int u = 0; u < U; u++) {
        if (j0 + u < n_pos) {
            acc.x = __builtin_fmaf(pu[u], vv[u].x, acc.x);
            acc.y = __builtin_fmaf(pu[u], vv[u].y, acc.y);
            acc.z = __builtin_fmaf(pu[u], vv[u].z, acc.z);
            acc.w = __builtin_fmaf(pu[u], vv[u].w, acc.w);
        }
    }
#pragma unroll
    for (int m = C4; m < 64; m <<= 1) {
        acc.x += __shfl_xor(acc.x, m);
        acc.y += __shfl_xor(acc.y, m);
        acc.z += __shfl_xor(acc.z, m);
        acc.w += __shfl_xor(acc.w, m);
    }
    const int w = tid >> 6;
    if ((tid & 63) < C4) part[w][c4] = acc;
    __syncthreads();
    if (tid < C4) {
        float4 o = part[0][tid];
#pragma unroll
        for (int i = 1; i < NW; i++) {
            const float4 v = part[i][tid];
            o.x += v.x; o.y += v.y; o.z += v.z; o.w += v.w;
        }
        ((float4 *)(out + (int64_t)h * HD + slice * kPvSlice))[tid] = o;
    }
}

__global__ void k_silu_mul(const float *__restrict__ g, const float *__restrict__ u,
                           float *__restrict__ y, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = silu_mul(g[i], u[i]);
}

__global__ void k_gelu(const float *__restrict__ x, float *__restrict__ y, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = gelu_pade(x[i]);
}

// Thread-local argmax scan of x[tid], x[tid + T], ... in batches of U loads issued before any
// compare (one memory round trip per batch instead of one per element).  Indices ascend within
// a thread, so `>` keeps the lowest index of equal values.
template <int U>
__device__ __forceinline__ void argmax_scan(const float *__restrict__ x, int n, int tid, int T, float &best, int &idx)
{
    for (int base = tid; base < n; base += U * T) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = base + u * T;
            v[u] = i < n ? x[i] : -INFINITY;
        }
#pragma unroll
        for (int u = 0; u < U; u++)
            if (v[u] > best) { best = v[u]; idx = base + u * T; }
    }
}

// The same over (value, index) pairs: (v, i) wins over (best, idx) when larger, or equal with a
// lower index.
template <int U>
__device__ __forceinline__ void argmax_scan_pairs(const float *__restrict__ val, const int32_t *__restrict__ ix,
                                                  int n, int tid, int T, float &best, int &idx)
{
    for (int base = tid; base < n; base += U * T) {
        float v[U];
        int k[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = base + u * T;
            v[u] = i < n ? val[i] : -INFINITY;
            k[u] = i < n ? ix[i] : 0x7FFFFFFF;
        }
#pragma unroll
        for (int u = 0; u < U; u++)
            if (v[u] > best || (v[u] == best && k[u] < idx)) { best = v[u]; idx = k[u]; }
    }
}

// Argmax with the lowest index on ties.  With `tokens`/`pos` set it also appends the token to
// the device token array and advances the device position (end of a decode step).
__global__ __launch_bounds__(1024) void k_argmax(const float *__restrict__ x, int n,
                                                 int32_t *__restrict__ out,
                                                 int32_t *__restrict__ tokens,
                                                 int32_t *__restrict__ pos)
{
    __shared__ float bv[16];
    __shared__ int bi[16];
    float best = -INFINITY;
    int idx = 0x7FFFFFFF;
    argmax_scan<16>(x, n, threadIdx.x, blockDim.x, best, idx);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(idx, o, 64);
        if (ov > best || (ov == best && oi < idx)) { best = ov; idx = oi; }
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { bv[w] = best; bi[w] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int nw = blockDim.x >> 6;
        best = bv[0];
        idx = bi[0];
        for (int i = 1; i < nw; i++)
            if (bv[i] > best || (bv[i] == best && bi[i] < idx)) { best = bv[i]; idx = bi[i]; }
        if (idx == 0x7FFFFFFF) idx = 0;
        if (out) *out = idx;
        if (tokens && pos) {
            const int p = *pos;
            tokens[p + 1] = idx;
            *pos = p + 1;
        }
    }
}

// Argmax over (value, index) pairs (per-workgroup partials of the head GEMV), lowest index on
// ties; same outputs as k_argmax.
__global__ __launch_bounds__(256) void k_argmax_pairs(const float *__restrict__ val,
                                                      const int32_t *__restrict__ idx, int n,
                                                      int32_t *__restrict__ out,
                                                      int32_t *__restrict__ tokens,
                                                      int32_t *__restrict__ pos)
{
    __shared__ float bv[4];
    __shared__ int bi[4];
    float best = -INFINITY;
    int bidx = 0x7FFFFFFF;
    argmax_scan_pairs<16>(val, idx, n, threadIdx.x, 256, best, bidx);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bidx, o, 64);
        if (ov > best || (ov == best && oi < bidx)) { best = ov; bidx = oi; }
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { bv[w] = best; bi[w] = bidx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        best = bv[0];
        bidx = bi[0];
        for (int k = 1; k < 4; k++)
            if (bv[k] > best || (bv[k] == best && bi[k] < bidx)) { best = bv[k]; bidx = bi[k]; }
        if (bidx == 0x7FFFFFFF) bidx = 0;
        if (out) *out = bidx;
        if (tokens && pos) {
            const int p = *pos;
            tokens[p + 1] = bidx;
            *pos = p + 1;
        }
    }
}

__global__ void k_advance(int32_t *pos)
{
    if (threadIdx.x == 0) *pos = *pos + 1;
}

// Chunk c of a row of any weight layout, dequantised exactly (decode_chunk_exact).
// One pass over an embedding row: y = row (ADD = false) or y = y + row (ADD = true), each thread
// decoding whole 32-element chunks in registers and writing them as float4.
template <int F, bool ADD>
__device__ __forceinline__ void embed_pass(const WView &w, int64_t row, float *y)
{
    const int nch = (int)(w.cols / 32);
    for (int c = threadIdx.x; c < nch; c += blockDim.x) {
        float v[32];
        decode_chunk_exact<F>(w, row, c, v);
        float4 *y4 = (float4 *)(y + (int64_t)c * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float4 o = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
            if constexpr (ADD) {
                const float4 a = y4[i];
                o = make_float4(a.x + o.x, a.y + o.y, a.z + o.z, a.w + o.w);
            }
            y4[i] = o;
        }
    }
}

template <bool ADD>
__device__ void embed_pass_any(const WView &w, int64_t row, float *y)
{
    switch (w.fmt) {
    case FMT_Q4_0: embed_pass<FMT_Q4_0, ADD>(w, row, y); break;
    case FMT_Q8_0: embed_pass<FMT_Q8_0, ADD>(w, row, y); break;
    case FMT_Q4_K: embed_pass<FMT_Q4_K, ADD>(w, row, y); break;
    case FMT_Q5_K: embed_pass<FMT_Q5_K, ADD>(w, row, y); break;
    case FMT_Q6_K: embed_pass<FMT_Q6_K, ADD>(w, row, y); break;
    case FMT_F16: embed_pass<FMT_F16, ADD>(w, row, y); break;
    case FMT_F32: embed_pass<FMT_F32, ADD>(w, row, y); break;
    case FMT_SQ8: embed_pass<FMT_SQ8, ADD>(w, row, y); break;
    default: embed_pass<FMT_SQ4, ADD>(w, row, y); break;
    }
}

// Embedding gather (NeuralNet.cs:376-391, row copies :576-592) with the row dequantised
// exactly, plus the learned position row for GPT-2 (TransformerModel.cs:299-326): the token row
// is stored, then the position row added to it (tok + pos, the reference's operand order); each
// thread handles the same chunks in both passes.
__device__ __forceinline__ void embed_row(const WView &w, int64_t row, float *y, const WView &pw, bool has_pos,
                                          int64_t prow)
{
    embed_pass_any<false>(w, row, y);
    if (has_pos) embed_pass_any<true>(pw, prow, y);
}

__global__ __launch_bounds__(kThreads) void k_embed(WView w, WView pw, int has_pos,
                                                    const int32_t *__restrict__ tokens,
                                                    const int32_t *__restrict__ pos,
                                                    float *__restrict__ x)
{
    const int p = *pos;
    int64_t tok = tokens[p];
    if (tok < 0 || tok >= w.rows) tok = 0;   // the host validates tokens; never read out of bounds
    embed_row(w, tok, x, pw, has_pos != 0, p);
}

// End of a decode step with the next step's embedding folded in: argmax over the head's
// per-workgroup (value, index) pairs (lowest index on ties), token appended at tokens[pos + 1],
// position advanced, and x_next = emb[token] (+ pos_emb[pos + 1]).  The position is read up
// front, before the reduction, so it costs no round trip of its own.
__global__ __launch_bounds__(kThreads) void k_argmax_embed(const float *__restrict__ val,
                                                           const int32_t *__restrict__ idx, int n,
                                                           int32_t *__restrict__ out,
                                                           int32_t *__restrict__ tokens,
                                                           int32_t *__restrict__ pos, WView w, WView pw,
                                                           int has_pos, float *__restrict__ x_next)
{
    __shared__ float bv[kWaves];
    __shared__ int bi[kWaves];
    __shared__ int s_p;
    // only thread 0 touches the position in memory (read here, advanced at the end); the
    // other threads take it from LDS after the barrier
    int p = 0;
    if (threadIdx.x == 0) p = *pos;
    float best = -INFINITY;
    int bidx = 0x7FFFFFFF;
    argmax_scan_pairs<16>(val, idx, n, threadIdx.x, kThreads, best, bidx);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bidx, o, 64);
        if (ov > best || (ov == best && oi < bidx)) { best = ov; bidx = oi; }
    }
    const int wv = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { bv[wv] = best; bi[wv] = bidx; }
    if (threadIdx.x == 0) s_p = p;
    __syncthreads();
    p = s_p;
    best = bv[0];
    bidx = bi[0];
#pragma unroll
    for (int k = 1; k < kWaves; k++)
        if (bv[k] > best || (bv[k] == best && bi[k] < bidx)) { best = bv[k]; bidx = bi[k]; }
    if (bidx == 0x7FFFFFFF) bidx = 0;
    int64_t tok = bidx;
    if (tok < 0 || tok >= w.rows) tok = 0;
    // the learned position row of the next position (clamped: after the last step of a full
    // context it is never used)
    const int64_t prow = has_pos ? (p + 1 < pw.rows ? p + 1 : pw.rows - 1) : 0;
    embed_row(w, tok, x_next, pw, has_pos != 0, prow);
    // token and position stores last: a wait for the embedding row's loads also waits for
    // every earlier store of the wave (the vector-memory counter counts both)
    if (threadIdx.x == 0) {
        if (out) *out = bidx;
        tokens[p + 1] = bidx;
        *pos = p + 1;
    }
}

// Embedding rows of a token batch: x[t] = emb[tok[t]] (+ pos_emb[pos[t]]), one workgroup per
// token.
__global__ __launch_bounds__(kThreads) void k_embed_tokens(WView w, WView pw, int has_pos,
                                                           const int32_t *__restrict__ tok,
                                                           const int32_t *__restrict__ pos,
                                                           float *__restrict__ x, int64_t x_stride)
{
    const int t = blockIdx.x;
    int64_t id = tok[t];
    if (id < 0 || id >= w.rows) id = 0;   // the host validates tokens; never read out of bounds
    const int p = pos[t];
    float *xr = x + (int64_t)t * x_stride;
    embed_row(w, id, xr, pw, has_pos != 0, p);
}

// Decode attention for a token batch: token t (its own position and KV cache) x head h.
template <int HD>
__global__ __launch_bounds__(AttnCfg<HD>::NT) void k_attention_tokens(
    const float *__restrict__ q, int64_t q_stride, float *const *__restrict__ kc_tok,
    float *const *__restrict__ vc_tok, int64_t layer_off, float *__restrict__ out, int64_t out_stride,
    int n_head, int n_kv_head, int ctx_stride, const int32_t *__restrict__ tok_pos, uint8_t *__restrict__ out_parts)
{
    constexpr int NT = AttnCfg<HD>::NT;
    extern __shared__ float4 smem4[];
    __shared__ AttnSmem<HD, NT> sm;
    const int b = blockIdx.x, t = blockIdx.y;
    const int h = (n_head % 8 == 0) ? (b % 8) * (n_head / 8) + b / 8 : b;
    const int kvh = h / (n_head / n_kv_head);
    const int n_pos = tok_pos[t] + 1;
    const int64_t off = layer_off + (int64_t)kvh * ctx_stride * HD;
    attention_head<HD, NT, AttnCfg<HD>::U>(q + (int64_t)t * q_stride + (int64_t)h * HD, kc_tok[t] + off,
                                           vc_tok[t] + off, out + (int64_t)t * out_stride + (int64_t)h * HD,
                                           n_pos, ctx_stride, (float *)smem4, sm, out_parts, n_head * HD / 32, t,
                                           h * HD);
}

// Argmax of each row of logits [M][n] (lowest index on ties); with `tok_arr`, appends the
// token to row t's session token array at tok_pos[t] + 1 and advances tok_pos[t]; tok_next
// receives the token for the next step.
__global__ __launch_bounds__(1024) void k_argmax_rows(const float *__restrict__ x, int n, int64_t stride,
                                                      int32_t *__restrict__ tok_next,
                                                      int32_t *__restrict__ tok_pos,
                                                      int32_t *const *__restrict__ tok_arr)
{
    __shared__ float bv[16];
    __shared__ int bi[16];
    const float *xr = x + (int64_t)blockIdx.x * stride;
    float best = -INFINITY;
    int idx = 0x7FFFFFFF;
    argmax_scan<16>(xr, n, threadIdx.x, blockDim.x, best, idx);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(idx, o, 64);
        if (ov > best || (ov == best && oi < idx)) { best = ov; idx = oi; }
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { bv[w] = best; bi[w] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        best = bv[0];
        idx = bi[0];
        for (int i = 1; i < (int)(blockDim.x >> 6); i++)
            if (bv[i] > best || (bv[i] == best && bi[i] < idx)) { best = bv[i]; idx = bi[i]; }
        if (idx == 0x7FFFFFFF) idx = 0;
        const int t = blockIdx.x;
        tok_next[t] = idx;
        if (tok_arr) {
            const int p = tok_pos[t];
            tok_arr[t][p + 1] = idx;
            tok_pos[t] = p + 1;
        }
    }
}

unsigned grid_for(int64_t n, int t = kThreads) { return (unsigned)((n + t - 1) / t); }

}  // namespace

hipError_t launch_rmsnorm(const float *x, const float *g, float *y, int rows, int n, float eps, hipStream_t s)
{
    hipLaunchKernelGGL(k_rmsnorm, dim3(rows), dim3(kThreads), 0, s, x, g, y, n, eps);
    return hipGetLastError();
}

hipError_t launch_layernorm(const float *x, const float *g, const float *b, float *y, int rows, int n,
                            float eps, hipStream_t s)
{
    hipLaunchKernelGGL(k_layernorm, dim3(rows), dim3(kThreads), 0, s, x, g, b, y, n, eps);
    return hipGetLastError();
}

hipError_t launch_rope(float *data, int n_heads, int seq, int hd, int pos0, const float *c,
                       const float *sn, hipStream_t s)
{
    const int64_t total = (int64_t)n_heads * seq * (hd / 2);
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_rope, dim3(grid_for(total)), dim3(kThreads), 0, s, data, n_heads, seq, hd,
                       pos0, c, sn);
    return hipGetLastError();
}

hipError_t launch_softmax(float *scores, float scale, int seq, int k_seq, int cache_off, hipStream_t s)
{
    hipLaunchKernelGGL(k_softmax, dim3(seq), dim3(kThreads), 0, s, scores, scale, k_seq, cache_off);
    return hipGetLastError();
}

template <int HD, int U, int NT, int NCH = 1>
hipError_t launch_pv(dim3 g2, size_t p_lds, const float *scores, const float *vc, float *out, int n_head,
                     int n_kv_head, int ctx_stride, int sc_stride, const int32_t *pos_dev, int n_pos_fixed,
                     hipStream_t s)
{
    const void *fp = (const void *)k_attn_pv<HD, U, NT, NCH>;
    if (p_lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(fp, hipFuncAttributeMaxDynamicSharedMemorySize, (int)p_lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((k_attn_pv<HD, U, NT, NCH>), dim3(g2.x * NCH), dim3(NT), p_lds, s, scores, vc, out, n_head,
                       n_kv_head, ctx_stride, sc_stride, pos_dev, n_pos_fixed);
    return hipGetLastError();
}

template <int HD>
hipError_t launch_attn_hd(dim3 g1, dim3 g2, size_t q_lds, size_t p_lds, int U, int NT, const float *q, const float *kc,
                          const float *vc, float *out, float *scores, int n_head, int n_kv_head, int ctx_stride,
                          int sc_stride, const int32_t *pos_dev, int n_pos_fixed, int nblk, hipStream_t s)
{
    hipLaunchKernelGGL(k_attn_scores<HD>, g1, dim3(256), q_lds, s, q, kc, scores, n_head, n_kv_head, ctx_stride,
                       sc_stride, pos_dev, n_pos_fixed, nblk);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
#define SMX_PV(U_, NT_) launch_pv<HD, U_, NT_>(g2, p_lds, scores, vc, out, n_head, n_kv_head, ctx_stride, sc_stride, pos_dev, n_pos_fixed, s)
    if (NT == 256) {
        switch (U) {
        case 4: return SMX_PV(4, 256);
        case 8: return SMX_PV(8, 256);
        case 12: return SMX_PV(12, 256);
        default: return SMX_PV(16, 256);
        }
    }
    if (NT == 512) {
        switch (U) {
        case 16: return SMX_PV(16, 512);
        case 24: return SMX_PV(24, 512);
        default: return SMX_PV(36, 512);
        }
    }
#undef SMX_PV
    // two workgroups per (head, slice), 512 threads, 18 positions per lane each (configs[3]
    // decode at ~4.1K positions 1338 -> 1382 tok/s against 256 threads x 36; 1024 x 9: 1350)
    return launch_pv<HD, 18, 512, 2>(g2, p_lds, scores, vc, out, n_head, n_kv_head, ctx_stride, sc_stride, pos_dev,
                                     n_pos_fixed, s);
}

template <int HD, int NT, int P>
hipError_t launch_dec(dim3 g, const float *q, const float *kc, const float *vc, float *out, int n_head,
                      int n_kv_head, int ctx_stride, const int32_t *pos_dev, int n_pos_fixed, hipStream_t s,
                      const Prefetch *pf)
{
    Prefetch p{};
    unsigned extra = 0;
    if (pf && pf->n > 0) {
        p = *pf;
        extra = kPrefetchWgs;
    }
    hipLaunchKernelGGL((k_attn_dec<HD, NT, P>), dim3(g.x + extra), dim3(NT), 0, s, q, kc, vc, out, n_head, n_kv_head,
                       ctx_stride, pos_dev, n_pos_fixed, p);
    return hipGetLastError();
}

// One launch for contexts up to 1024 positions: 256 threads with 1-3 passes of 256
// positions, 512 threads with two passes above 768 positions
template <int HD>
hipError_t launch_dec_hd(dim3 g, int max_pos, const float *q, const float *kc, const float *vc, float *out,
                         int n_head, int n_kv_head, int ctx_stride, const int32_t *pos_dev, int n_pos_fixed,
                         hipStream_t s, const Prefetch *pf)
{
    if (max_pos <= 256) return launch_dec<HD, 256, 1>(g, q, kc, vc, out, n_head, n_kv_head, ctx_stride, pos_dev, n_pos_fixed, s, pf);
    if (max_pos <= 512) return launch_dec<HD, 256, 2>(g, q, kc, vc, out, n_head, n_kv_head, ctx_stride, pos_dev, n_pos_fixed, s, pf);
    if (max_pos <= 768) return launch_dec<HD, 256, 3>(g, q, kc, vc, out, n_head, n_kv_head, ctx_stride, pos_dev, n_pos_fixed, s, pf);
    return launch_dec<HD, 512, 2>(g, q, kc, vc, out, n_head, n_kv_head, ctx_stride, pos_dev, n_pos_fixed, s, pf);
}

hipError_t launch_attn_dec(dim3 g, int max_pos, int hd, const float *q, const float *kc, const float *vc,
                           float *out, int n_head, int n_kv_head, int ctx_stride, const int32_t *pos_dev,
                           int n_pos_fixed, hipStream_t s, const Prefetch *pf)
{
    switch (hd) {
    case 16: return launch_dec_hd<16>(g, max_pos, q, kc, vc, out, n_head, n_kv_head, ctx_stride, pos_dev, n_pos_fixed, s, pf);
    case 32: return launch_dec_hd<32>(g, max_pos, q, kc, vc, out, n_head, n_kv_head, ctx_stride, pos_dev, n_pos_fixed, s, pf);
    case 64: return launch_dec_hd<64>(g, max_pos, q, kc, vc, out, n_head, n_kv_head, ctx_stride, pos_dev, n_pos_fixed, s, pf);
    default: return hipErrorInvalidValue;
    }
}

size_t attention_scores_floats(int n_head, int max_pos) { return (size_t)n_head * ((max_pos + 3) & ~3); }

int attention_pv_chunks(int max_pos, int max_chunks)
{
    return max_chunks >= 2 && max_pos > kPvChunk && max_pos <= 2 * kPvChunk ? 2 : 1;
}

hipError_t launch_attention_split(const float *q, const float *kc, const float *vc, float *out,
                                  float *scores, int n_head, int n_kv_head, int hd, int ctx_stride,
                                  const int32_t *pos_dev, int n_pos_fixed, int max_pos, hipStream_t s,
                                  int max_chunks, const Prefetch *pf)
{
    if (hd % kPvSlice || hd > 128 || n_head % n_kv_head || max_pos > ctx_stride || max_pos < 1)
        return hipErrorInvalidValue;
    const int sc_stride = (max_pos + 3) & ~3;
    const int G = n_head / n_kv_head;
    const int nblk = (max_pos + kScorePB - 1) / kScorePB;
    const size_t q_lds = (size_t)G * hd * 4, p_lds = (size_t)max_pos * 4;
    if (q_lds > 64 * 1024 || p_lds > 160 * 1024) return hipErrorInvalidValue;
    const dim3 g1((unsigned)(n_kv_head * nblk)), g2((unsigned)(n_head * (hd / kPvSlice)));
    if (hd <= 64 && max_pos <= 1024 && ctx_stride % 4 == 0) return launch_attn_dec(g2, max_pos, hd, q, kc, vc, out, n_head, n_kv_head,
                                                             ctx_stride, pos_dev, n_pos_fixed, s, pf);
    // positions per lane sized to the session context so that every V row of the context is
    // loaded in the first batch, all of its loads in flight: 256 threads (64 position lanes)
    // up to 1024 positions, 512 threads (128 position lanes) up to 4608
    // (two workgroups per (head, slice), when the caller sums two partial outputs: NT 0)
    const int NT = attention_pv_chunks(max_pos, max_chunks) == 2 ? 0 : max_pos <= 1024 ? 256 : 512;
    const int U = max_pos <= 256 ? 4 : max_pos <= 512 ? 8 : max_pos <= 768 ? 12 : max_pos <= 1024 ? 16
                : max_pos <= 2048 ? 16 : max_pos <= 3072 ? 24 : 36;
    switch (hd) {
    case 16: return launch_attn_hd<16>(g1, g2, q_lds, p_lds, U, NT, q, kc, vc, out, scores, n_head, n_kv_head, ctx_stride, sc_stride, pos_dev, n_pos_fixed, nblk, s);
    case 32: return launch_attn_hd<32>(g1, g2, q_lds, p_lds, U, NT, q, kc, vc, out, scores, n_head, n_kv_head, ctx_stride, sc_stride, pos_dev, n_pos_fixed, nblk, s);
    case 64: return launch_attn_hd<64>(g1, g2, q_lds, p_lds, U, NT, q, kc, vc, out, scores, n_head, n_kv_head, ctx_stride, sc_stride, pos_dev, n_pos_fixed, nblk, s);
    case 128: return launch_attn_hd<128>(g1, g2, q_lds, p_lds, U, NT, q, kc, vc, out, scores, n_head, n_kv_head, ctx_stride, sc_stride, pos_dev, n_pos_fixed, nblk, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_silu_mul(const float *g, const float *u, float *y, int64_t n, hipStream_t s)
{
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_silu_mul, dim3(grid_for(n)), dim3(kThreads), 0, s, g, u, y, n);
    return hipGetLastError();
}

hipError_t launch_gelu(const float *x, float *y, int64_t n, hipStream_t s)
{
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_gelu, dim3(grid_for(n)), dim3(kThreads), 0, s, x, y, n);
    return hipGetLastError();
}

// Streaming read of one device range (16-byte loads, 8 per thread in flight; the values only
// feed an empty asm statement): the HBM read ceiling the GEMV is measured against.
__global__ __launch_bounds__(256) void k_stream_read(Prefetch pf) { prefetch_slice(pf, (int)blockIdx.x, (int)gridDim.x, 256); }

hipError_t launch_stream_read(const void *src, uint64_t bytes, hipStream_t s)
{
    if (!src || bytes == 0 || bytes % 16 || bytes >= (1ull << 32)) return hipErrorInvalidValue;
    Prefetch pf{};
    pf.p[0] = (const uint8_t *)src;
    pf.bytes[0] = (uint32_t)bytes;
    pf.n = 1;
    // about one workgroup per 16 KB, rounded down to a whole number of workgroups per CU (256
    // to 4096): with a partial last round the CUs holding one workgroup more set the time (13 MB
    // through 795 workgroups 4.69 us, 768 or 512 workgroups 4.40-4.42 us, 640 4.61, 384 5.15)
    uint64_t wgs = bytes / 16384 / 256 * 256;
    wgs = wgs < 256 ? 256 : wgs > 4096 ? 4096 : wgs;
    hipLaunchKernelGGL(k_stream_read, dim3((unsigned)wgs), dim3(256), 0, s, pf);
    return hipGetLastError();
}

hipError_t launch_argmax(const float *x, int n, int32_t *out, int32_t *tokens, int32_t *pos,
                         hipStream_t s)
{
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, s, x, n, out, tokens, pos);
    return hipGetLastError();
}

hipError_t launch_argmax_pairs(const float *val, const int32_t *idx, int n, int32_t *out,
                               int32_t *tokens, int32_t *pos, hipStream_t s)
{
    hipLaunchKernelGGL(k_argmax_pairs, dim3(1), dim3(256), 0, s, val, idx, n, out, tokens, pos);
    return hipGetLastError();
}

hipError_t launch_argmax_embed(const float *val, const int32_t *idx, int n, int32_t *out,
                               int32_t *tokens, int32_t *pos, const WView &tok, const WView *posw,
                               float *x_next, hipStream_t s)
{
    WView pw = posw ? *posw : tok;
    hipLaunchKernelGGL(k_argmax_embed, dim3(1), dim3(kThreads), 0, s, val, idx, n, out, tokens, pos, tok, pw,
                       posw ? 1 : 0, x_next);
    return hipGetLastError();
}

hipError_t launch_embed(const WView &tok, const WView *posw, const int32_t *tokens,
                        const int32_t *pos, float *x, hipStream_t s)
{
    WView pw = posw ? *posw : tok;
    hipLaunchKernelGGL(k_embed, dim3(1), dim3(kThreads), 0, s, tok, pw, posw ? 1 : 0, tokens, pos, x);
    return hipGetLastError();
}

hipError_t launch_embed_tokens(const WView &tok, const WView *posw, const int32_t *ids,
                               const int32_t *pos, float *x, int64_t x_stride, int M, hipStream_t s)
{
    WView pw = posw ? *posw : tok;
    hipLaunchKernelGGL(k_embed_tokens, dim3(M), dim3(kThreads), 0, s, tok, pw, posw ? 1 : 0, ids, pos, x, x_stride);
    return hipGetLastError();
}

hipError_t launch_attention_tokens(const float *q, int64_t q_stride, float *const *kc_tok,
                                   float *const *vc_tok, int64_t layer_off, float *out,
                                   int64_t out_stride, int n_head, int n_kv_head, int hd,
                                   int ctx_stride, const int32_t *tok_pos, int M, hipStream_t s,
                                   uint8_t *out_parts)
{
    if (out_parts && (n_head * hd) % 32) return hipErrorInvalidValue;
    const size_t lds = (size_t)ctx_stride * 4;
    const void *fn = nullptr;
    switch (hd) {
    case 16: fn = (const void *)k_attention_tokens<16>; break;
    case 32: fn = (const void *)k_attention_tokens<32>; break;
    case 64: fn = (const void *)k_attention_tokens<64>; break;
    case 128: fn = (const void *)k_attention_tokens<128>; break;
    default: return hipErrorInvalidValue;
    }
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    const dim3 grid((unsigned)n_head, (unsigned)M);
#define SMX_ATT_T(HD) hipLaunchKernelGGL(k_attention_tokens<HD>, grid, dim3(AttnCfg<HD>::NT), lds, s, q, q_stride, kc_tok, vc_tok, layer_off, out, out_stride, n_head, n_kv_head, ctx_stride, tok_pos, out_parts)
    switch (hd) {
    case 16: SMX_ATT_T(16); break;
    case 32: SMX_ATT_T(32); break;
    case 64: SMX_ATT_T(64); break;
    default: SMX_ATT_T(128); break;
    }
#undef SMX_ATT_T
    return hipGetLastError();
}

hipError_t launch_argmax_rows(const float *x, int n, int64_t stride, int M, int32_t *tok_next,
                              int32_t *tok_pos, int32_t *const *tok_arr, hipStream_t s)
{
    hipLaunchKernelGGL(k_argmax_rows, dim3(M), dim3(1024), 0, s, x, n, stride, tok_next, tok_pos, tok_arr);
    return hipGetLastError();
}

hipError_t launch_advance(int32_t *pos, hipStream_t s)
{
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(64), 0, s, pos);
    return hipGetLastError();
}

}  // namespace smx
