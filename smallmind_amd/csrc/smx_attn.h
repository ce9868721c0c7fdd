// smx_attn.h -- decode attention of one query head, executed by one whole workgroup.
//
// One decode position of MultiHeadAttention (MultiHeadAttention.cs:676-844): raw scores q.k,
// scale, max, FastExp(s*scale - max) (MathUtils.cs:20-32), normalise by 1/sum
// (OptimizedOps.cs:39-93), then P.V (:810-844).  The softmax is two-pass (global max first)
// because the Pade FastExp is not multiplicative, so an online rescaling would not reproduce
// the reference.
//
// Cache layouts: K is dimension-major [kv_head][HD][ctx_stride] so that lanes reading
// consecutive positions issue coalesced loads; V is position-major [kv_head][ctx_stride][HD]
// so that lanes reading consecutive dimensions of one position are coalesced.  Every load
// batch is a fully unrolled set of independent loads, so a thread keeps many requests in
// flight instead of one round trip per loop iteration.
#pragma once

#include "smx_device.h"

namespace smx {

template <int HD, int NT>
struct AttnSmem {
    static constexpr int D4 = HD / 4;
    static constexpr int NPL = NT / D4;
    float4 qs[D4];
    float4 part[NPL][D4];
    float red[16];
};

// sc: LDS scratch of at least n_pos floats.  All NT threads of the workgroup must call this.
// U: positions per thread per P.V load batch (one batch = one round trip to memory).
// With parts set, the output is written as activation parts of the next GEMM instead of out:
// xp_store(parts, parts_nsb, parts_tok, parts_k0 + d, out[d]).
template <int HD, int NT, int U = 8>
__device__ __forceinline__ void attention_head(const float *__restrict__ qh, const float *__restrict__ K,
                                               const float *__restrict__ V, float *__restrict__ out,
                                               int n_pos, int ctx_stride, float *sc,
                                               AttnSmem<HD, NT> &sm, uint8_t *parts = nullptr,
                                               int parts_nsb = 0, int parts_tok = 0, int parts_k0 = 0)
{
    constexpr int D4 = HD / 4;
    constexpr int NPL = NT / D4;
    constexpr int NW = NT / 64;
    const float scale = 1.0f / sqrtf((float)HD);   // MultiHeadAttention.cs:686
    const int tid = opaque_tid();
    if (tid < D4) sm.qs[tid] = ((const float4 *)qh)[tid];
    __syncthreads();

    // K and V of one KV head span less than 4 GiB, so every load is a uniform base plus a
    // 32-bit byte offset (no 64-bit address per load held in registers).
    // The pointers are cast to the global address space: global loads are counted by the
    // vector-memory counter alone (flat loads also by the LDS counter), so the waits for the
    // LDS reads of q do not also wait for every K load in flight.
    typedef const __attribute__((address_space(1))) char gchar;
    typedef const __attribute__((address_space(1))) float gfloat;
    typedef float gf4 __attribute__((ext_vector_type(4)));
    gchar *Kb = (gchar *)K, *Vb = (gchar *)V;
    float mx = -INFINITY;
    for (int j = tid; j < n_pos; j += NT) {
        float kv[HD];
#pragma unroll
        for (int e = 0; e < HD; e++) kv[e] = *(gfloat *)(Kb + 4u * ((uint32_t)e * (uint32_t)ctx_stride + (uint32_t)j));
        // q is read from LDS (broadcast) at each use: held in registers across the position
        // loop it would take HD VGPRs and, at 1024 threads, force the K loads to serialize.
        int z = 0;
        asm volatile("" : "+s"(z));
        float s = 0.0f;
#pragma unroll
        for (int e4 = 0; e4 < D4; e4++) {
            const float4 qv = sm.qs[e4 + z];
            s = __builtin_fmaf(qv.x, kv[4 * e4 + 0], s);
            s = __builtin_fmaf(qv.y, kv[4 * e4 + 1], s);
            s = __builtin_fmaf(qv.z, kv[4 * e4 + 2], s);
            s = __builtin_fmaf(qv.w, kv[4 * e4 + 3], s);
        }
        const float t = s * scale;
        sc[j] = t;
        mx = fmaxf(mx, t);
    }
    mx = block_max<NW>(mx, sm.red);
    float sum = 0.0f;
    for (int j = tid; j < n_pos; j += NT) {
        const float e = fastexp(sc[j] - mx);
        sc[j] = e;
        sum += e;
    }
    sum = block_sum<NW>(sum, sm.red);
    const float inv = 1.0f / sum;
    for (int j = tid; j < n_pos; j += NT) sc[j] = sc[j] * inv;
    __syncthreads();

    // P.V: thread = (position lane pl, float4 column c4); U rows in flight per thread
    const int c4 = tid % D4, pl = tid / D4;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int j0 = pl; j0 < n_pos; j0 += NPL * U) {
        float4 vv[U];
        float pp[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int j = j0 + u * NPL;
            const bool ok = j < n_pos;
            const gf4 t = ok ? *(const __attribute__((address_space(1))) gf4 *)(Vb + 16u * ((uint32_t)j * (HD / 4) + (uint32_t)c4))
                             : gf4{0.0f, 0.0f, 0.0f, 0.0f};
            vv[u] = make_float4(t.x, t.y, t.z, t.w);
            pp[u] = ok ? sc[j] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            acc.x = __builtin_fmaf(pp[u], vv[u].x, acc.x);
            acc.y = __builtin_fmaf(pp[u], vv[u].y, acc.y);
            acc.z = __builtin_fmaf(pp[u], vv[u].z, acc.z);
            acc.w = __builtin_fmaf(pp[u], vv[u].w, acc.w);
        }
    }
    sm.part[pl][c4] = acc;
    __syncthreads();
    if (tid < D4) {
        float4 o = sm.part[0][tid];
        for (int p = 1; p < NPL; p++) {
            const float4 v = sm.part[p][tid];
            o.x += v.x; o.y += v.y; o.z += v.z; o.w += v.w;
        }
        if (parts) {
            const int k = parts_k0 + 4 * tid;
            xp_store(parts, parts_nsb, parts_tok, k, o.x);
            xp_store(parts, parts_nsb, parts_tok, k + 1, o.y);
            xp_store(parts, parts_nsb, parts_tok, k + 2, o.z);
            xp_store(parts, parts_nsb, parts_tok, k + 3, o.w);
        } else {
            ((float4 *)out)[tid] = o;
        }
    }
    __syncthreads();   // sm and sc may be reused by the caller right away
}

}  // namespace smx
