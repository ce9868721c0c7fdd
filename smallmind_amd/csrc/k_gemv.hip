// k_gemv.hip -- fused dequantize-GEMV for Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K weights, SmallMind's
// SMQ Q8 / Q4 blocks (fp32 scales) and unquantized F16 / F32 matrices.
//
// y[r] = sum_k W[r][k] * x[k] for a row-major [rows][cols] weight in the backend layout
// (smx_internal.h).  Replaces Linear.ForwardFP32 / IWeightTensor.MatMul for batch-1 decode
// (NeuralNet.cs:145-298) and the fused C# kernels (MatMulF32Q8.cs, MatMulF32Q4.cs,
// FusedQ4KMatMul.cs, FusedQ6KMatMul.cs), computing y = x W^T as the GGUF loader path does.
//
// Work decomposition.  A workgroup is 4 wave64s.  A "row group" of R consecutive rows is owned
// by S waves (S = 1, 2 or 4) that split the 32-element chunks of K between them; lane l of wave
// ws takes chunks (ws + S*j)*64 + l for j < C, so one pass ("round") covers 64*S*C chunks and
// every lane holds at most C chunks of x and C*R chunks of weights in registers.  Rows of at
// most 32 chunks (K <= 1024) on tall matrices put a row group on each half of a wave (HW = 2),
// and with a fused norm at K <= 1024 every wave stages its own copy of the activations
// (STG = 4), so the prologue needs no workgroup barrier.
//
// Latency is the budget at decode sizes (a 3 MB matrix is 0.4 us of HBM time), so each wave
// issues all of its loads before it consumes any of them, in the order in which it needs them:
//   1. the activation vector (+ gamma / beta of a fused RMSNorm / LayerNorm), loaded by the
//      whole workgroup with coalesced 16-byte loads (L2-resident);
//   2. the weight chunks of all R rows (HBM);
//   3. the epilogue operands (bias, residual, RoPE table entries, KV position) as scalar loads.
// Vector-memory loads complete in issue order, so (1) is consumed while (2) is in flight: the
// norm statistic is reduced across the workgroup (DPP within waves, LDS across them), the
// normalised vector is staged in LDS with a bank-conflict-free swizzle, and each lane reads
// its 32-element chunks from there -- one copy of the activations per workgroup instead of
// one strided copy per wave.
// Codes are unpacked with and/shift into bytes and converted with v_cvt_f32_ubyte*; block
// scales are factored out of each 32-term sum (sum (sc*q - m) x = sc * sum q x - m * sum x).
// The R per-lane partials are summed across the wave transposed (lane swaps fold two rows per
// add, then DPP within 16-lane rows), combined across the S waves in LDS in a fixed order, and
// the R rows' epilogues run on R lanes at once.
//
// Compiled once per block format (SMX_GEMV_FMT) so the instantiations build in parallel.
#include "smx_device.h"
#include "smx_formats.h"
#include "smx_gemv.h"

#ifndef SMX_GEMV_FMT
#error "compile with -DSMX_GEMV_FMT=<Fmt>"
#endif

namespace smx {

namespace {

// Epilogue classes: EC_SIMPLE covers EPI_STORE / EPI_RESID / EPI_GELU (selected at run time).
enum { EC_SIMPLE = 0, EC_SILU = 1, EC_QKV = 2, EC_ARGMAX = 3 };

// Epilogue operands of one row group, loaded before the dot products (wave-uniform values).
template <int R, int EC>
struct EpiIn {
    float bias[R];
    float res[R];
    float cs[R / 2], sn[R / 2];
    int pos;
};

template <int R, int EC>
__device__ __forceinline__ void epi_load(const GemvArgs &a, uint32_t row0, uint32_t N, int my,
                                         EpiIn<R, EC> &e)
{
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t row = row0 + r < N ? row0 + r : N - 1;
        e.bias[r] = a.bias ? ld_uniform(a.bias + row) : 0.0f;
        e.res[r] = 0.0f;
        if constexpr (EC == EC_SIMPLE)
            if (a.epi == EPI_RESID) e.res[r] = ld_uniform(a.resid + (int64_t)my * a.out_stride + row);
    }
    e.pos = 0;
    if constexpr (EC == EC_QKV) e.pos = a.pos ? ld_uniform(a.pos) : a.pos_val;
}

// R wave-uniform values moved to the first lane of each lane block: lane r*64/R receives v[r],
// the other lanes 0.  v_writelane moves a scalar into one lane with no compares or selects
// (a lane-indexed select chain over v can be folded into an indexed access, which puts the
// array in scratch memory).
template <int R>
__device__ __forceinline__ float spread(const float *v)
{
    float o = 0.0f;
#pragma unroll
    for (int r = 0; r < R; r++) asm("v_writelane_b32 %0, %1, %2" : "+v"(o) : "s"(v[r]), "i"(r * (64 / R)));
    return o;
}

// RoPE table entries of the group's row pairs, loaded once the activation vector is staged.
// They depend on the position, a scalar load, and go through the vector path on purpose:
// scalar loads share a counter with LDS operations and return out of order, so one still
// outstanding would hold up every later LDS wait of the dot products.  Issued after the
// weights, they are not waited for until the epilogue.
template <int R, int EC>
__device__ __forceinline__ void epi_load_rope(const GemvArgs &a, uint32_t row0, EpiIn<R, EC> &e)
{
    const int half = a.head_dim / 2, d = a.d_model, kv = a.kv_dim;
    const int z = opaque_tid() >> 30;   // 0, but lane-varying to the compiler: vector loads
#pragma unroll
    for (int p = 0; p < R / 2; p++) {
        const int row = (int)row0 + 2 * p;
        int pair = -1;
        if (a.use_rope && row < d) pair = (row % a.head_dim) / 2;
        else if (a.use_rope && row < d + kv) pair = ((row - d) % a.head_dim) / 2;
        e.cs[p] = pair >= 0 ? a.rope_cos[(int64_t)e.pos * half + pair + z] : 1.0f;
        e.sn[p] = pair >= 0 ? a.rope_sin[(int64_t)e.pos * half + pair + z] : 0.0f;
    }
}

// Lane-indexed pick of one of P values that are the same in every lane (i >= P gives the last).
template <int P>
__device__ __forceinline__ float pick(const float *v, int i)
{
    float o = v[P - 1];
#pragma unroll
    for (int r = P - 2; r >= 0; r--) o = i == r ? v[r] : o;
    return o;
}

// Epilogue of one row group.  Called by the whole wave with c = the transposed row totals
// (wave_totals_t: row r in lane block r of 64/R lanes), so the R rows leave from R lanes in
// one store instruction.  SwiGLU and QKV work on row pairs: a lane swap brings rows 2p and
// 2p+1 together in lane 32p, and the pairs are computed in parallel (each SwiGLU output is a
// long exp/divide chain).
template <int R, int EC>
__device__ __forceinline__ void epi_store(const GemvArgs &a, float c, const EpiIn<R, EC> &e,
                                          uint32_t row0, uint32_t N, int my, int lane)
{
    constexpr int LB = 64 / R;
    const int rl = lane / LB;   // row of this lane's block
    float *out = a.out + (int64_t)my * a.out_stride;
    if constexpr (EC == EC_SIMPLE || EC == EC_ARGMAX) {
        if (lane % LB != 0 || row0 + (uint32_t)rl >= N) return;
        float y = c;
        if constexpr (EC == EC_SIMPLE) {
            if (a.epi == EPI_RESID) y = spread<R>(e.res) + c;
            else if (a.epi == EPI_GELU) y = gelu_pade(c);
        }
        out[row0 + rl] = y;
        return;
    }
    const float2 pr = R == 4 ? swap16(c, c) : swap32(c, c);   // lane 32p: rows 2p, 2p+1
    const int p = lane >> 5;
    if ((lane & 31) != 0 || p >= R / 2) return;
    const uint32_t row = row0 + 2u * (uint32_t)p;
    if (row + 1u >= N) return;
    if constexpr (EC == EC_SILU) {
        // rows interleave gate / up: out[i] = silu(gate_i) * up_i
        out[row / 2] = silu_mul(pr.x, pr.y);
    } else {
        // rows [Q | K | V]: RoPE on Q and K pairs (RotaryEmbedding.cs:115-116); Q -> out,
        // K -> k_cache [kv_head][head_dim][ctx_stride] (dimension-major), V -> v_cache
        // [kv_head][ctx_stride][head_dim].
        const int d = a.d_model, kv = a.kv_dim, hd = a.head_dim, pos = e.pos;
        const int r = (int)row;
        float v0 = pr.x, v1 = pr.y;
        if (a.use_rope && r < d + kv) {
            const float cs = pick<R / 2>(e.cs, p), sn = pick<R / 2>(e.sn, p);
            const float t0 = v0 * cs, t1 = v1 * sn, t2 = v0 * sn, t3 = v1 * cs;
            v0 = t0 - t1;
            v1 = t2 + t3;
        }
        if (r < d) {
            out[r] = v0;
            out[r + 1] = v1;
        } else if (r < d + kv) {
            float *dst = a.k_cache + (int64_t)(r - d) * a.ctx_stride + pos;
            dst[0] = v0;
            dst[a.ctx_stride] = v1;
        } else {
            const int vr = r - d - kv;
            float *dst = a.v_cache + ((int64_t)(vr / hd) * a.ctx_stride + pos) * hd + (vr % hd);
            dst[0] = v0;
            dst[1] = v1;
        }
    }
}

// (v, i) beats (bv, bi): larger value, or equal value and lower index (NaN never wins).
__device__ __forceinline__ bool am_better(float v, int i, float bv, int bi)
{
    return v > bv || (v == bv && i < bi);
}

// Workgroup-wide sum (4 waves), the same bits in every thread.
__device__ __forceinline__ float wg_sum(float v, float *slot, int w)
{
    v = wave_sum_uniform(v);
    if (lane_id() == 0) slot[w] = v;
    __syncthreads();
    return (slot[0] + slot[1]) + (slot[2] + slot[3]);
}

// Position of float4 i4 of the activation vector in the staged LDS copy: float4 i of chunk c
// sits at 8c + (i ^ (c & 7)), so the eight 16-byte reads of a lane's 128-byte chunk fall on
// distinct banks across consecutive lanes.
__device__ __forceinline__ int xs_pos(int c, int i) { return 8 * c + (i ^ (c & 7)); }

// STG = 3 is STG = 1 with the activation vector given as two partial sums x + x[x_part_stride]
// (no norm), added in that order while staging.
// STG = 1 (K <= 8192) / 2 (K <= 16384, no norm): the workgroup loads the activation vector
// with coalesced loads (thread t: float4 t, t+256, ...), applies the fused norm and stages it
// in LDS; lanes then read their chunks from LDS.  STG = 0 (no norm, K > 16384): lanes read
// their chunks from global memory.
// NT: the weights are read with the non-temporal hint (streamed); false for matrices the
// runtime keeps resident in the MALL (WView::cache).  A template argument, not a branch on
// the flag: with both load sequences in one kernel the plain one ran ~10 % slower.
// HW = 2 (rows of at most 32 chunks, K <= 1024): each half of a wave takes its own R rows, lanes
// 32h + l taking chunk l of rows row0 + R*h ..., so a wave covers 2R rows with every lane busy
// instead of leaving the lanes past the row's chunks idle; the rows are reduced one half at a
// time (the other half's partials zeroed).
template <int F, int R, int S, int C, int PRO, int EC, int STG, bool NT, int HW = 1>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a)
{
    static_assert(STG || PRO == PRO_NONE, "a fused norm needs the staged activation path");
    static_assert(HW == 1 || (HW == 2 && S == 1 && C == 1 && STG), "half-wave rows: one chunk per lane");
    constexpr int G = 4 / S;    // row groups per workgroup
    // STG = 4 (K <= 1024, S = 1): every wave loads the whole activation vector, takes the norm
    // statistic with wave reductions and stages its own copy in LDS, so the prologue has no
    // workgroup barrier (the waves need nothing from each other)
    constexpr bool WAVE = STG == 4;
    static_assert(!WAVE || S == 1, "wave-private staging: each wave owns whole rows");
    constexpr int TSTEP = WAVE ? 64 : 256;   // threads sharing the staging loads
    constexpr int KPT = WAVE ? 4 : STG == 2 ? 16 : 8;   // staged float4 per thread: K <= 4*TSTEP*KPT
    static_assert(STG != 2 || PRO == PRO_NONE, "the wide staging is for plain GEMVs");
    __shared__ float s_red[4][R];
    __shared__ float s_st[2][4];
    extern __shared__ float4 xs[];
    const int w = wave_id();
    const int grp = w / S, ws = w % S;
    const int lane = lane_id();
    const uint32_t N = (uint32_t)a.w.rows;
    const int K = (int)a.w.cols, nch = K >> 5, K4 = K >> 2;
    float4 *const xsb = WAVE ? xs + w * K4 : xs;   // this wave's staged copy (STG 4)
    const uint32_t row0 = (blockIdx.x * G + grp) * R * HW;
    const int my = blockIdx.y;
    const float *x = a.x + (int64_t)my * a.x_stride;
    const int half = HW == 2 ? lane >> 5 : 0, cl = HW == 2 ? lane & 31 : lane;
    const uint32_t rh = row0 + (uint32_t)(R * half);   // first row of this lane's half
    uint32_t rb[R];   // row * blocks-per-row (rows past the end re-read the last row)
#pragma unroll
    for (int r = 0; r < R; r++) rb[r] = (rh + r < N ? rh + r : N - 1) * (uint32_t)a.w.nb;

    // 1. activations (+ norm parameters): coalesced, issued first
    const int tid = STG ? (WAVE ? (opaque_tid() & 63) : opaque_tid()) : 0;
    float4 xr[STG ? KPT : 1], gr[PRO != PRO_NONE ? KPT : 1], br[PRO == PRO_LN ? KPT : 1];
    constexpr bool TWO = STG == 3;   // x = x + x[x_part_stride] (two partial sums)
    static_assert(!TWO || PRO == PRO_NONE, "partial sums are added before any norm");
    float4 x2[TWO ? KPT : 1];
    if constexpr (STG) {
#pragma unroll
        for (int k = 0; k < KPT; k++) {
            const int i4 = tid + TSTEP * k;
            if (i4 < K4) {
                xr[k] = ((const float4 *)x)[i4];
                if constexpr (PRO != PRO_NONE) gr[k] = ((const float4 *)a.gamma)[i4];
                if constexpr (PRO == PRO_LN) br[k] = ((const float4 *)a.beta)[i4];
            }
        }
        if constexpr (TWO) {
#pragma unroll
            for (int k = 0; k < KPT; k++) {
                const int i4 = tid + TSTEP * k;
                if (i4 < K4) x2[k] = ((const float4 *)(x + a.x_part_stride))[i4];
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // 2. weights of the first round
    int cj[C];
    bool on[C];
    Raw<F> wr[C][R];
#pragma unroll
    for (int j = 0; j < C; j++) {
        const int c = (ws + S * j) * (64 / HW) + cl;
        on[j] = c < nch;
        cj[j] = on[j] ? c : nch - 1;
    }
#pragma unroll
    for (int j = 0; j < C; j++)
#pragma unroll
        for (int r = 0; r < R; r++) wr[j][r].template load32<NT>(a.w, rb[r], cj[j]);
    __builtin_amdgcn_sched_barrier(0);
    // 3. epilogue operands (of each half's rows)
    EpiIn<R, EC> e[HW];
#pragma unroll
    for (int h = 0; h < HW; h++) epi_load<R, EC>(a, row0 + (uint32_t)(R * h), N, my, e[h]);
    __builtin_amdgcn_sched_barrier(0);
    // 4. norm statistic over the workgroup, normalise, stage in LDS
    if constexpr (STG) {
        float sc = 1.0f, mean = 0.0f;
        if constexpr (PRO == PRO_RMS) {
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < KPT; k++)
                if (tid + TSTEP * k < K4) {
                    float q;
                    q = xr[k].x * xr[k].x; ss += q;
                    q = xr[k].y * xr[k].y; ss += q;
                    q = xr[k].z * xr[k].z; ss += q;
                    q = xr[k].w * xr[k].w; ss += q;
                }
            ss = WAVE ? wave_sum_uniform(ss) : wg_sum(ss, s_st[0], w);
            sc = 1.0f / sqrtf(ss / (float)K + a.eps);   // RMSNormOps.cs:114
        } else if constexpr (PRO == PRO_LN) {
            float t = 0.0f;
#pragma unroll
            for (int k = 0; k < KPT; k++)
                if (tid + TSTEP * k < K4) { t += xr[k].x; t += xr[k].y; t += xr[k].z; t += xr[k].w; }
            mean = (WAVE ? wave_sum_uniform(t) : wg_sum(t, s_st[0], w)) / (float)K;   // LayerNormOps.cs:92-101
            float sq = 0.0f;
#pragma unroll
            for (int k = 0; k < KPT; k++)
                if (tid + TSTEP * k < K4) {
                    float dd, q;
                    dd = xr[k].x - mean; q = dd * dd; sq += q;
                    dd = xr[k].y - mean; q = dd * dd; sq += q;
                    dd = xr[k].z - mean; q = dd * dd; sq += q;
                    dd = xr[k].w - mean; q = dd * dd; sq += q;
                }
            sq = WAVE ? wave_sum_uniform(sq) : wg_sum(sq, s_st[1], w);
            sc = 1.0f / sqrtf(sq / (float)K + a.eps);     // LayerNormOps.cs:103-119
        }
#pragma unroll
        for (int k = 0; k < KPT; k++) {
            const int i4 = tid + TSTEP * k;
            if (i4 < K4) {
                float4 v = xr[k];
                if constexpr (TWO) { v.x += x2[k].x; v.y += x2[k].y; v.z += x2[k].z; v.w += x2[k].w; }
                if constexpr (PRO == PRO_RMS) {   // RMSNormOps.cs:137-139: gamma * (x * invRms)
                    const float4 g = gr[k];
                    v.x = g.x * (v.x * sc); v.y = g.y * (v.y * sc);
                    v.z = g.z * (v.z * sc); v.w = g.w * (v.w * sc);
                } else if constexpr (PRO == PRO_LN) {   // LayerNormOps.cs:185
                    const float4 g = gr[k], b = br[k];
                    v.x = __builtin_fmaf(g.x, (v.x - mean) * sc, b.x);
                    v.y = __builtin_fmaf(g.y, (v.y - mean) * sc, b.y);
                    v.z = __builtin_fmaf(g.z, (v.z - mean) * sc, b.z);
                    v.w = __builtin_fmaf(g.w, (v.w - mean) * sc, b.w);
                }
                xsb[xs_pos(i4 >> 3, i4 & 7)] = v;
            }
        }
        // wave-private staging: a wave's LDS operations complete in issue order, so its reads
        // below see its writes; otherwise every wave reads what all of them staged
        if constexpr (WAVE) __builtin_amdgcn_wave_barrier();
        else __syncthreads();
    }

    if constexpr (EC == EC_QKV) {
#pragma unroll
        for (int h = 0; h < HW; h++) epi_load_rope<R, EC>(a, row0 + (uint32_t)(R * h), e[h]);
    }

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    // 5. activation chunks (LDS or global) and dot products.  A staged launch covers K in one
    // round; only the unstaged fallback (K > 16384) loops, which keeps the loop's register
    // cost out of the common instances.
    auto round = [&]() {
#pragma unroll
        for (int j = 0; j < C; j++) {
            float4 xv[8];
            if constexpr (STG) {
#pragma unroll
                for (int i = 0; i < 8; i++) xv[i] = xsb[xs_pos(cj[j], i)];
            } else {
                const float4 *xp = (const float4 *)(x + 32 * cj[j]);
#pragma unroll
                for (int i = 0; i < 8; i++) xv[i] = xp[i];
            }
            float xa = 0.0f, xb = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                xa += (xv[i].x + xv[i].y) + (xv[i].z + xv[i].w);
                xb += (xv[i + 4].x + xv[i + 4].y) + (xv[i + 4].z + xv[i + 4].w);
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float p = wr[j][r].dot(xv, xa, xb, cj[j]);
                acc[r] += on[j] ? p : 0.0f;
            }
        }
    };
    round();
    if constexpr (!STG) {
        for (int base = 64 * S * C; base < nch; base += 64 * S * C) {
#pragma unroll
            for (int j = 0; j < C; j++) {
                const int c = base + (ws + S * j) * 64 + lane;
                on[j] = c < nch;
                cj[j] = on[j] ? c : nch - 1;
#pragma unroll
                for (int r = 0; r < R; r++) wr[j][r].template load32<NT>(a.w, rb[r], cj[j]);
            }
            round();
        }
    }

    // 6. reduction across the wave (row r's total in lane block r), then across the S waves
    // of the row group in a fixed order; with half-wave rows, one half at a time
    constexpr int LB = 64 / R;
    float t[HW][R];   // the row totals (argmax epilogue)
#pragma unroll
    for (int h = 0; h < HW; h++) {
        float ah[R];
#pragma unroll
        for (int r = 0; r < R; r++) ah[r] = HW == 1 || half == h ? acc[r] : 0.0f;
        float c = wave_totals_t<R>(ah);
        if constexpr (S > 1) {
            if (lane % LB == 0) s_red[w][lane / LB] = c;
            __syncthreads();
            float v = s_red[grp * S][lane / LB];
#pragma unroll
            for (int s = 1; s < S; s++) v += s_red[grp * S + s][lane / LB];
            c = v;
        }
        if (a.bias) c += spread<R>(e[h].bias);   // in the first lane of each block
        const uint32_t r0 = row0 + (uint32_t)(R * h);
        if (ws == 0 && r0 < N) epi_store<R, EC>(a, c, e[h], r0, N, my, lane);
        if constexpr (EC == EC_ARGMAX) {
#pragma unroll
            for (int r = 0; r < R; r++) t[h][r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(c), r * LB));
        }
    }
    if constexpr (EC == EC_ARGMAX) {
        __shared__ float s_bv[4];
        __shared__ int s_bi[4];
        if (ws == 0 && lane == 0) {
            float bv = -INFINITY;
            int bi = 0x7FFFFFFF;
#pragma unroll
            for (int h = 0; h < HW; h++)
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t row = row0 + (uint32_t)(R * h + r);
                    if (row < N && am_better(t[h][r], (int)row, bv, bi)) { bv = t[h][r]; bi = (int)row; }
                }
            s_bv[grp] = bv;
            s_bi[grp] = bi;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float bv = s_bv[0];
            int bi = s_bi[0];
#pragma unroll
            for (int g = 1; g < G; g++)
                if (am_better(s_bv[g], s_bi[g], bv, bi)) { bv = s_bv[g]; bi = s_bi[g]; }
            a.wg_val[blockIdx.x] = bv;
            a.wg_idx[blockIdx.x] = bi;
        }
    }
}

template <int R, int S, int C, int PRO, int EC, int STG, int HW = 1>
hipError_t launch_v(const GemvArgs &a, int m, hipStream_t s)
{
    constexpr int F = SMX_GEMV_FMT;
    // a staged launch runs one round of 64*S*C/HW chunks: it must cover the row
    if (STG && a.w.cols > (int64_t)64 / HW * S * C * 32) return hipErrorInvalidValue;
    const int64_t groups = (a.w.rows + R * HW - 1) / (R * HW);
    const dim3 grid((unsigned)((groups + (4 / S) - 1) / (4 / S)), (unsigned)m);
    if (STG == 4 && a.w.cols > 1024) return hipErrorInvalidValue;
    const size_t lds = STG ? (size_t)a.w.cols * 4 * (STG == 4 ? 4 : 1) : 0;
    if (a.w.cache) hipLaunchKernelGGL((k_gemv<F, R, S, C, PRO, EC, STG, false, HW>), grid, dim3(256), lds, s, a);
    else hipLaunchKernelGGL((k_gemv<F, R, S, C, PRO, EC, STG, true, HW>), grid, dim3(256), lds, s, a);
    if constexpr (EC == EC_ARGMAX) {
        // the per-workgroup partials are reduced by a one-workgroup kernel; the kernel boundary
        // makes them visible without a device-scope fence in each of the many workgroups
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        if (a.x_next)
            return launch_argmax_embed(a.wg_val, a.wg_idx, (int)grid.x, a.amax_out, a.tokens, a.tok_pos,
                                       a.next_emb, a.next_embp.q ? &a.next_embp : nullptr, a.x_next, s);
        return launch_argmax_pairs(a.wg_val, a.wg_idx, (int)grid.x, a.amax_out, a.tokens, a.tok_pos, s);
    }
    return hipGetLastError();
}

// Shape selection (gemv_shape): S waves split K so that one round covers it (up to 4 waves x 64
// lanes x C chunks); R = 2 or 4 rows per wave.  The activation
// vector is staged in LDS (up to 8192 floats with a fused norm, 16384 without).
template <int PRO, int EC>
hipError_t launch_pe(const GemvArgs &a, int m, hipStream_t s)
{
    const int64_t K = a.w.cols;
    if constexpr (PRO == PRO_NONE && EC == EC_SIMPLE) {
        // two partial activation vectors (STG 3: staged like STG 1, K <= 8192)
        if (a.x_parts == 2) {
            if (K > 8192) return hipErrorInvalidValue;
            switch (gemv_shape(a.w.rows, K)) {
            case GS_R4S1H2:
            case GS_R4S1: return launch_v<4, 1, 1, PRO, EC, 3>(a, m, s);
            case GS_R2S1: return launch_v<2, 1, 1, PRO, EC, 3>(a, m, s);
            case GS_R2S2: return launch_v<2, 2, 1, PRO, EC, 3>(a, m, s);
            case GS_R4S2: return launch_v<4, 2, 1, PRO, EC, 3>(a, m, s);
            case GS_R4S4: return launch_v<4, 4, 1, PRO, EC, 3>(a, m, s);
            default: return launch_v<2, 4, 1, PRO, EC, 3>(a, m, s);
            }
        }
    }
    switch (gemv_shape(a.w.rows, K)) {
    case GS_WIDE:
    case GS_R4S2C3:
    case GS_R4S2C4:
        if constexpr (PRO == PRO_NONE && EC == EC_SIMPLE) {   // K > 8192: no fused norm
            if (K > 16384) return launch_v<2, 4, 2, PRO, EC, 0>(a, m, s);
            // F32 chunks are 128 bytes: 4 rows x 3-4 chunks in flight would not fit the
            // registers (the C = 4 instance spills 436 bytes per lane and returned wrong sums)
            if constexpr (SMX_GEMV_FMT == FMT_F32) {
                return launch_v<2, 4, 2, PRO, EC, 2>(a, m, s);
            } else {
                switch (gemv_shape(a.w.rows, K)) {
                case GS_R4S2C3: return launch_v<4, 2, 3, PRO, EC, 2>(a, m, s);
                case GS_R4S2C4: return launch_v<4, 2, 4, PRO, EC, 2>(a, m, s);
                default: return launch_v<2, 4, 2, PRO, EC, 2>(a, m, s);
                }
            }
        }
        return hipErrorInvalidValue;
    // K <= 1024 with a fused norm: wave-private staging (no workgroup barrier in the prologue)
    case GS_R4S1H2:
        if constexpr (PRO != PRO_NONE) return launch_v<4, 1, 1, PRO, EC, 4, 2>(a, m, s);
        else return launch_v<4, 1, 1, PRO, EC, 1, 2>(a, m, s);
    case GS_R4S1:
        if constexpr (PRO != PRO_NONE)
            if (K <= 1024) return launch_v<4, 1, 1, PRO, EC, 4>(a, m, s);
        return launch_v<4, 1, 1, PRO, EC, 1>(a, m, s);
    case GS_R2S1:
        if constexpr (PRO != PRO_NONE)
            if (K <= 1024) return launch_v<2, 1, 1, PRO, EC, 4>(a, m, s);
        return launch_v<2, 1, 1, PRO, EC, 1>(a, m, s);
    case GS_R2S2: return launch_v<2, 2, 1, PRO, EC, 1>(a, m, s);
    case GS_R4S2: return launch_v<4, 2, 1, PRO, EC, 1>(a, m, s);
    case GS_R4S4: return launch_v<4, 4, 1, PRO, EC, 1>(a, m, s);
    default: return launch_v<2, 4, 1, PRO, EC, 1>(a, m, s);   // GS_R2S4: nch <= 256
    }
}

}  // namespace

#define SMX_CAT2(a, b) a##b
#define SMX_CAT(a, b) SMX_CAT2(a, b)

hipError_t SMX_CAT(launch_gemv_fmt, SMX_GEMV_FMT)(const GemvArgs &a, int m, hipStream_t s)
{
    switch (a.epi) {
    case EPI_STORE:
    case EPI_RESID:
    case EPI_GELU:
        if (a.pro == PRO_NONE) return launch_pe<PRO_NONE, EC_SIMPLE>(a, m, s);
        if (a.pro == PRO_RMS) return launch_pe<PRO_RMS, EC_SIMPLE>(a, m, s);
        return launch_pe<PRO_LN, EC_SIMPLE>(a, m, s);
    case EPI_SILU:
        if (a.pro == PRO_RMS) return launch_pe<PRO_RMS, EC_SILU>(a, m, s);
        return hipErrorInvalidValue;
    case EPI_QKV:
        if (a.pro == PRO_RMS) return launch_pe<PRO_RMS, EC_QKV>(a, m, s);
        if (a.pro == PRO_LN) return launch_pe<PRO_LN, EC_QKV>(a, m, s);
        return hipErrorInvalidValue;
    case EPI_ARGMAX:
        if (m != 1 || !a.wg_val || !a.wg_idx) return hipErrorInvalidValue;
        if (a.pro == PRO_RMS) return launch_pe<PRO_RMS, EC_ARGMAX>(a, m, s);
        if (a.pro == PRO_LN) return launch_pe<PRO_LN, EC_ARGMAX>(a, m, s);
        return hipErrorInvalidValue;
    default:
        return hipErrorInvalidValue;
    }
}

}  // namespace smx
