// k_decode.hip -- persistent decode: every step of a prefill or a greedy generation in one
// cooperative launch.
//
// One step is TransformerModel.Forward for one token with the KV cache on
// (TransformerModel.cs:272-344, TransformerBlock.cs:153-187) followed, for token-producing
// steps, by greedy selection.  The phases of a step run on all workgroups and are separated
// by a device-wide barrier:
//
//   per layer:  norm + QKV GEMV (+RoPE, K/V append; layer 0 reads the embedding row directly)
//            |  attention (one workgroup per query head)
//            |  O GEMV + residual
//            |  norm + gate/up GEMV + SwiGLU (or fc1 + GELU)
//            |  down GEMV + residual
//   head:       final norm + head GEMV, per-workgroup argmax partials | argmax
//
// The barrier is a monotonically increasing arrival counter.  Every wait is bounded: a
// workgroup that spins past kSpinLimit raises the abort flag, every other waiter sees it and
// leaves, and the host reports the failure, so no wave can be left waiting.
#include "smx_attn.h"
#include "smx_gemv.h"

namespace smx {

namespace {

constexpr int kNT = kDecodeThreads;
constexpr int kNW = kNT / 64;
constexpr unsigned kSpinLimit = 1u << 22;

// Returns false when the launch is being aborted.
__device__ __forceinline__ bool grid_sync(const DecodeArgs &A, unsigned nwg, unsigned &epoch, int *s_ok)
{
    unsigned *bar = A.bar;
    int *abort_flag = A.abort_flag;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long *tr = nullptr;
        if (A.trace && (int)epoch < A.trace_cap) {
            tr = A.trace + ((unsigned long long)epoch * nwg + blockIdx.x) * 2;
            tr[0] = __builtin_amdgcn_s_memrealtime();
        }
        epoch += 1;
        const unsigned target = epoch * nwg;
        // release: this workgroup's writes of the phase become visible device-wide first
        __hip_atomic_fetch_add(bar, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        int ok = 1;
        unsigned spins = 0;
        while (true) {
            const unsigned v = __hip_atomic_load(bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if ((int)(v - target) >= 0) break;
            if (__hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                ok = 0;
                break;
            }
            if (++spins > kSpinLimit) {
                __hip_atomic_store(abort_flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        // acquire: the other workgroups' writes are visible to this workgroup from here on
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        if (tr) tr[1] = __builtin_amdgcn_s_memrealtime();
        *s_ok = ok;
    }
    __syncthreads();
    return *s_ok != 0;
}

__device__ __forceinline__ void better(float &bv, int &bi, float v, int i)
{
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// Head GEMV tasks of this wave; tracks the wave's (max, lowest index) over its rows.
template <int FH>
__device__ __forceinline__ void head_tasks(const GemvArgs &g, int64_t gw, int64_t W, int vocab,
                                           float *lout, float &best, int &bidx)
{
    const int lane = threadIdx.x & 63;
    const int64_t ntask = (vocab + 3) / 4;
    for (int64_t t = gw; t < ntask; t += W) {
        Raw<FH> cur[4];
        float tt[4];
        gemv_compute<FH, 4>(g, 4 * t, 0, cur, false, tt);
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = (int)(4 * t + r);
                if (row < vocab) {
                    lout[row] = tt[r];
                    if (tt[r] > best) {   // rows of a wave ascend, so > keeps the lowest index
                        best = tt[r];
                        bidx = row;
                    }
                }
            }
        }
    }
}

template <int F, int HD>
__global__ __launch_bounds__(kNT) void k_decode(DecodeArgs A)
{
    extern __shared__ float4 smem4[];
    float *sc = (float *)smem4;                     // attention scores [max_ctx]
    __shared__ AttnSmem<HD, kNT> asm_;
    __shared__ int s_ok, s_tok;
    __shared__ float s_bv[kNW];
    __shared__ int s_bi[kNW];

    const unsigned nwg = gridDim.x;
    const int wg = blockIdx.x, wv = wave_id(), lane = threadIdx.x & 63;
    const int64_t W = (int64_t)nwg * kNW;
    const int64_t gw = (int64_t)wv * nwg + wg;      // consecutive tasks land on different CUs
    unsigned epoch = 0;
    const int nch_d = A.d / 32;
    const bool fuse_embed = nch_d <= 64;
    const int pro = A.llama ? PRO_RMS : PRO_LN;
    int tok = A.tokens[A.pos0];

    for (int s = 0; s < A.n_steps; s++) {
        const int pos = A.pos0 + s;
        if (tok < 0 || tok >= A.vocab) tok = 0;     // the host validates tokens
        if (!fuse_embed) {
            GemvArgs e{};
            e.x_embed = 1;
            e.emb = A.tok;
            e.emb_row = tok;
            e.embp = A.posw;
            e.embp_row = pos;
            for (int64_t c = gw * 64 + lane; c < nch_d; c += W * 64) {
                float4 xv[8];
                fetch_x_chunk(e, A.x, (int)c, xv);
#pragma unroll
                for (int i = 0; i < 8; i++) ((float4 *)(A.x + 32 * c))[i] = xv[i];
            }
            if (!grid_sync(A, nwg, epoch, &s_ok)) return;
        }
        for (int l = 0; l < A.n_layer; l++) {
            const LayerDesc &L = A.layers[l];
            {   // norm + QKV (+RoPE, K/V append)
                GemvArgs g{};
                g.w = L.qkv;
                g.x = A.x;
                g.out = A.q;
                g.bias = L.bqkv;
                g.gamma = L.attn_g;
                g.beta = L.attn_b;
                g.eps = A.eps;
                g.pro = pro;
                g.epi = EPI_QKV;
                g.d_model = A.d;
                g.kv_dim = A.kv_dim;
                g.head_dim = HD;
                g.ctx_stride = A.max_ctx;
                g.use_rope = A.llama;
                g.k_cache = L.kc;
                g.v_cache = L.vc;
                g.rope_cos = A.rope_cos;
                g.rope_sin = A.rope_sin;
                g.pos = nullptr;
                g.pos_val = pos;
                if (l == 0 && fuse_embed) {
                    g.x_embed = 1;
                    g.emb = A.tok;
                    g.emb_row = tok;
                    g.embp = A.posw;
                    g.embp_row = pos;
                }
                const int64_t ntask = (A.nqkv + 1) / 2;
                for (int64_t t = gw; t < ntask; t += W) gemv_wave<F, 2>(g, 2 * t, 0);
                if (l == 0 && fuse_embed && gw == 0 && lane < nch_d) {
                    // the residual stream starts from the embedding row
                    float4 xv[8];
                    fetch_x_chunk(g, A.x, lane, xv);
#pragma unroll
                    for (int i = 0; i < 8; i++) ((float4 *)(A.x + 32 * lane))[i] = xv[i];
                }
            }
            if (!grid_sync(A, nwg, epoch, &s_ok)) return;
            // attention, one query head per workgroup
            for (int h = wg; h < A.n_head; h += (int)nwg) {
                const int kvh = h / (A.n_head / A.n_kv_head);
                const int64_t off = (int64_t)kvh * A.max_ctx * HD;
                attention_head<HD, kNT>(A.q + (int64_t)h * HD, L.kc + off, L.vc + off,
                                        A.att + (int64_t)h * HD, pos + 1, A.max_ctx, sc, asm_);
            }
            if (!grid_sync(A, nwg, epoch, &s_ok)) return;
            {   // O projection + residual
                GemvArgs g{};
                g.w = L.o;
                g.x = A.att;
                g.out = A.x;
                g.resid = A.x;
                g.bias = L.bo;
                g.pro = PRO_NONE;
                g.epi = EPI_RESID;
                const int64_t ntask = (L.o.rows + 1) / 2;
                for (int64_t t = gw; t < ntask; t += W) gemv_wave<F, 2>(g, 2 * t, 0);
            }
            if (!grid_sync(A, nwg, epoch, &s_ok)) return;
            {   // norm + gate/up (SwiGLU) or fc1 (GELU)
                GemvArgs g{};
                g.w = L.gu;
                g.x = A.x;
                g.out = A.h;
                g.bias = L.bgu;
                g.gamma = L.ffn_g;
                g.beta = L.ffn_b;
                g.eps = A.eps;
                g.pro = pro;
                g.epi = A.llama ? EPI_SILU : EPI_GELU;
                const int64_t ntask = (L.gu.rows + 3) / 4;
                for (int64_t t = gw; t < ntask; t += W) gemv_wave<F, 4>(g, 4 * t, 0);
            }
            if (!grid_sync(A, nwg, epoch, &s_ok)) return;
            {   // down projection + residual
                GemvArgs g{};
                g.w = L.down;
                g.x = A.h;
                g.out = A.x;
                g.resid = A.x;
                g.bias = L.bdown;
                g.pro = PRO_NONE;
                g.epi = EPI_RESID;
                const int64_t ntask = (L.down.rows + 1) / 2;
                for (int64_t t = gw; t < ntask; t += W) gemv_wave<F, 2>(g, 2 * t, 0);
            }
            if (!grid_sync(A, nwg, epoch, &s_ok)) return;
        }
        if (s >= A.head_from) {
            // final norm + head GEMV with per-wave argmax
            GemvArgs g{};
            g.w = A.head;
            g.x = A.x;
            g.gamma = A.out_g;
            g.beta = A.out_b;
            g.eps = A.eps;
            g.pro = pro;
            float *lout = A.logits_all ? A.logits_all + (int64_t)(s - A.head_from) * A.vocab : A.logits;
            float best = -INFINITY;
            int bidx = 0x7FFFFFFF;
            switch (A.head.fmt) {
            case FMT_Q4_0: head_tasks<FMT_Q4_0>(g, gw, W, A.vocab, lout, best, bidx); break;
            case FMT_Q8_0: head_tasks<FMT_Q8_0>(g, gw, W, A.vocab, lout, best, bidx); break;
            case FMT_Q4_K: head_tasks<FMT_Q4_K>(g, gw, W, A.vocab, lout, best, bidx); break;
            case FMT_Q5_K: head_tasks<FMT_Q5_K>(g, gw, W, A.vocab, lout, best, bidx); break;
            default: head_tasks<FMT_Q6_K>(g, gw, W, A.vocab, lout, best, bidx); break;
            }
            if (lane == 0) {
                s_bv[wv] = best;
                s_bi[wv] = bidx;
            }
            __syncthreads();
            if (threadIdx.x == 0) {
                float b = s_bv[0];
                int i = s_bi[0];
                for (int k = 1; k < kNW; k++) better(b, i, s_bv[k], s_bi[k]);
                A.wg_val[wg] = b;
                A.wg_idx[wg] = i;
            }
            if (!grid_sync(A, nwg, epoch, &s_ok)) return;
            // every workgroup reduces the partials itself, so the next step needs no barrier
            float b = -INFINITY;
            int i = 0x7FFFFFFF;
            for (int k = threadIdx.x; k < (int)nwg; k += kNT) better(b, i, A.wg_val[k], A.wg_idx[k]);
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(b, o, 64);
                const int oi = __shfl_xor(i, o, 64);
                better(b, i, ov, oi);
            }
            if (lane == 0) {
                s_bv[wv] = b;
                s_bi[wv] = i;
            }
            __syncthreads();
            if (threadIdx.x == 0) {
                float bb = s_bv[0];
                int ii = s_bi[0];
                for (int k = 1; k < kNW; k++) better(bb, ii, s_bv[k], s_bi[k]);
                s_tok = ii == 0x7FFFFFFF ? 0 : ii;
                if (wg == 0) A.tokens[pos + 1] = s_tok;
            }
            __syncthreads();
            tok = s_tok;
        } else {
            tok = A.tokens[pos + 1];                   // next prompt token (written by the host)
        }
    }
    if (wg == 0 && threadIdx.x == 0) *A.pos = A.pos0 + A.n_steps;
}

}  // namespace

// This file is compiled once per block format (-DSMX_DECODE_FMT=<Fmt>) so the instantiations
// build in parallel; each object exports the accessor of its own format.
#ifndef SMX_DECODE_FMT
#error "compile k_decode.hip with -DSMX_DECODE_FMT=<Fmt>"
#endif
#define SMX_CAT2(a, b) a##b
#define SMX_CAT(a, b) SMX_CAT2(a, b)
const void *SMX_CAT(decode_kernel_fmt, SMX_DECODE_FMT)(int hd)
{
    switch (hd) {
    case 16: return (const void *)k_decode<SMX_DECODE_FMT, 16>;
    case 32: return (const void *)k_decode<SMX_DECODE_FMT, 32>;
    case 64: return (const void *)k_decode<SMX_DECODE_FMT, 64>;
    case 128: return (const void *)k_decode<SMX_DECODE_FMT, 128>;
    default: return nullptr;
    }
}

}  // namespace smx
