// k_sample.hip -- next-token sampling on the device, in the reference's pipeline order
// (InferenceSession.SampleNextToken, InferenceSession.cs:565-606):
//   1. repetition / presence / frequency penalties over the recent context (:765-843)
//   2. temperature: logits * (1 / T) (:741-763)
//   3. top-k: keep logits >= the k-th largest (:628-664)
//   4. softmax: exp(l - max) / sum over the finite logits (:666-706)
//   5. top-p: keep the largest probabilities whose running sum first reaches p, renormalise
//      by 1 / sum (:845-912, NormalizeProbabilities :969-1010)
//   6. min-p: zero probabilities below max * min_p, renormalise (:914-936)
//   7. sample: the first index whose running (double) sum of probabilities reaches u (:708-724)
// One workgroup of 1024 threads; the vocabulary stays in global memory (probs, n floats).
// Selections are exact: the k-th largest logit and the top-p threshold are found by binary
// search over the float bit patterns.  Where the reference sorts, ties at the cutoff are all
// kept here (the reference's unstable Array.Sort keeps an arbitrary subset of them), and sums
// run in tree order rather than in sorted or index order.
#include "smx_device.h"
#include "smx_internal.h"

namespace smx {

namespace {

constexpr int kT = 1024;
constexpr int kW = kT / 64;

// Order-preserving unsigned image of a float (larger float -> larger key).
__device__ __forceinline__ uint32_t fkey(float f)
{
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float kfloat(uint32_t k)
{
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

template <typename T>
__device__ T block_sum_t(T v, T *red)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    T t = 0;
#pragma unroll
    for (int i = 0; i < kW; i++) t += red[i];
    return t;
}

__device__ uint32_t block_count(uint32_t v, uint32_t *red) { return block_sum_t<uint32_t>(v, red); }

// NormalizeProbabilities (InferenceSession.cs:969-1010): p * (1 / sum) when sum > 0.
// s is this thread's partial sum of probs.
__device__ void renorm(float *probs, int n, float s, float *red)
{
    const float sum = block_sum_t<float>(s, red);
    if (sum > 0.0f) {
        const float inv = 1.0f / sum;
        for (int i = threadIdx.x; i < n; i += kT) probs[i] = probs[i] * inv;
    }
    __syncthreads();
}

// The pipeline; every thread of the workgroup calls it, and thread 0 receives the token.
__device__ int sample_pipeline(const float *__restrict__ logits, int n, const int32_t *__restrict__ ctx, int n_ctx,
                               const smx_sampling &sp, double u, float *__restrict__ probs)
{
    __shared__ float redf[kW];
    __shared__ uint32_t redu[kW];
    __shared__ double s_cum[kT];
    const int tid = threadIdx.x;

    for (int i = tid; i < n; i += kT) probs[i] = logits[i];
    __syncthreads();

    // 1. penalties: each distinct token of the window once (the first thread holding it)
    if (sp.repetition_penalty != 1.0f || sp.presence_penalty != 0.0f || sp.frequency_penalty != 0.0f) {
        const int win = sp.repetition_window > 0 ? sp.repetition_window : min(n_ctx, 256);
        const int start = max(0, n_ctx - win);
        for (int j = start + tid; j < n_ctx; j += kT) {
            const int t = ctx[j];
            bool first = true;
            for (int q = start; q < j && first; q++) first = ctx[q] != t;
            if (!first || t < 0 || t >= n) continue;
            int count = 0;
            for (int q = start; q < n_ctx; q++) count += ctx[q] == t;
            float l = probs[t];
            if (sp.repetition_penalty != 1.0f)
                l = l > 0.0f ? l / sp.repetition_penalty : l * sp.repetition_penalty;
            if (sp.presence_penalty != 0.0f) l = l - sp.presence_penalty;
            if (sp.frequency_penalty != 0.0f) l = l - (float)count * sp.frequency_penalty;
            probs[t] = l;
        }
        __threadfence_block();
        __syncthreads();
    }
    // 2. temperature
    if (sp.temperature != 1.0f) {
        const float inv = 1.0f / sp.temperature;
        for (int i = tid; i < n; i += kT) probs[i] = probs[i] * inv;
        __syncthreads();
    }
    // 3. top-k: the k-th largest key, bit by bit from the top (largest key with >= k at or above)
    if (sp.top_k > 0 && sp.top_k < n) {
        uint32_t key = 0;
        for (int b = 31; b >= 0; b--) {
            const uint32_t cand = key | (1u << b);
            uint32_t c = 0;
            for (int i = tid; i < n; i += kT) c += fkey(probs[i]) >= cand;
            if (block_count(c, redu) >= (uint32_t)sp.top_k) key = cand;
        }
        const float kth = kfloat(key);
        for (int i = tid; i < n; i += kT) probs[i] = probs[i] >= kth ? probs[i] : -INFINITY;
        __syncthreads();
    }
    // 4. softmax over the finite logits
    float mx = -INFINITY;
    for (int i = tid; i < n; i += kT)
        if (probs[i] != -INFINITY) mx = fmaxf(mx, probs[i]);
    mx = block_max<kW>(mx, redf);
    float s = 0.0f;
    for (int i = tid; i < n; i += kT) {
        const float l = probs[i];
        const float e = l != -INFINITY ? expf(l - mx) : 0.0f;
        probs[i] = e;
        s += e;
    }
    float sum = block_sum_t<float>(s, redf);
    if (sum > 0.0f)
        for (int i = tid; i < n; i += kT) probs[i] = probs[i] / sum;
    __syncthreads();
    // 5. top-p: threshold t = the largest probability with sum(p >= t) >= top_p
    if (sp.top_p < 1.0) {
        uint32_t key = 0;   // probabilities are >= 0: their bit patterns order like the values
        for (int b = 30; b >= 0; b--) {
            const uint32_t cand = key | (1u << b);
            const float t = __uint_as_float(cand);
            float c = 0.0f;
            for (int i = tid; i < n; i += kT) c += probs[i] >= t ? probs[i] : 0.0f;
            const float f = block_sum_t<float>(c, redf);
            if ((double)f >= sp.top_p && f > 0.0f) key = cand;   // float sum against the double TopP
        }
        const float t = __uint_as_float(key);
        s = 0.0f;
        for (int i = tid; i < n; i += kT) {
            const float p = probs[i] >= t ? probs[i] : 0.0f;
            probs[i] = p;
            s += p;
        }
        renorm(probs, n, s, redf);
    }
    // 6. min-p
    if (sp.min_p > 0.0f) {
        float pm = 0.0f;
        for (int i = tid; i < n; i += kT) pm = fmaxf(pm, probs[i]);
        pm = block_max<kW>(pm, redf);
        const float thr = pm * sp.min_p;
        s = 0.0f;
        for (int i = tid; i < n; i += kT) {
            const float p = probs[i] < thr ? 0.0f : probs[i];
            probs[i] = p;
            s += p;
        }
        renorm(probs, n, s, redf);
    }
    // 7. inverse-CDF draw: thread t owns the contiguous range [t*chunk, (t+1)*chunk)
    const int chunk = (n + kT - 1) / kT;
    const int lo = tid * chunk, hi = min(n, lo + chunk);
    double cs = 0.0;
    for (int i = lo; i < hi; i++) cs += (double)probs[i];
    s_cum[tid] = cs;
    __syncthreads();
    if (tid == 0) {
        double run = 0.0;
        int owner = -1;
        for (int t = 0; t < kT && owner < 0; t++) {
            if (run + s_cum[t] >= u) owner = t;
            else run += s_cum[t];
        }
        int tok = n - 1;   // SampleFromProbs' fallback
        if (owner >= 0) {
            const int a = owner * chunk, e = min(n, a + chunk);
            for (int i = a; i < e; i++) {
                run += (double)probs[i];
                if (run >= u) { tok = i; break; }
            }
        }
        return tok;
    }
    return 0;
}

__global__ __launch_bounds__(kT) void k_sample(const float *__restrict__ logits, int n,
                                               const int32_t *__restrict__ ctx, int n_ctx, smx_sampling sp,
                                               double u, float *__restrict__ probs, int32_t *__restrict__ out)
{
    const int tok = sample_pipeline(logits, n, ctx, n_ctx, sp, u, probs);
    if (threadIdx.x == 0) *out = tok;
}

// End of a sampled decode step: the context is tokens[0..pos] (prompt and generated so far),
// u = the st->counter-th draw of the stream seeded by st->seed; the token is appended at
// tokens[pos + 1], the position advanced and the draw counter incremented.
__global__ __launch_bounds__(kT) void k_sample_step(const float *__restrict__ logits, int n,
                                                    int32_t *__restrict__ tokens, int32_t *__restrict__ pos,
                                                    SampleState *__restrict__ st, float *__restrict__ probs)
{
    const int p = *pos;
    const smx_sampling sp = st->params;
    const double u = uniform_draw(st->seed, st->counter);
    const int tok = sample_pipeline(logits, n, tokens, p + 1, sp, u, probs);
    if (threadIdx.x == 0) {
        tokens[p + 1] = tok;
        *pos = p + 1;
        st->counter = st->counter + 1;
    }
}

// Members of a lockstep step (one logits row each), after k_argmax_rows has appended each
// member's greedy token at tokens[pos] and advanced pos: a member with sampling on replaces
// that token (and the next step's input id) with the pipeline's draw over tokens[0..pos-1].
__global__ __launch_bounds__(kT) void k_sample_rows(const float *__restrict__ logits, int n, int64_t stride,
                                                    int32_t *const *__restrict__ tok_arr,
                                                    const int32_t *__restrict__ pos, int32_t *__restrict__ ids,
                                                    SampleState *__restrict__ st, const int32_t *__restrict__ on,
                                                    float *__restrict__ probs)
{
    const int r = blockIdx.x;
    if (!on[r]) return;   // the same for the whole workgroup
    const int p = pos[r];
    const smx_sampling sp = st[r].params;
    const double u = uniform_draw(st[r].seed, st[r].counter);
    const int tok = sample_pipeline(logits + (size_t)r * stride, n, tok_arr[r], p, sp, u, probs + (size_t)r * n);
    if (threadIdx.x == 0) {
        tok_arr[r][p] = tok;
        ids[r] = tok;
        st[r].counter = st[r].counter + 1;
    }
}

}  // namespace

hipError_t launch_sample_rows(const float *logits, int n, int64_t stride, int M, int32_t *const *tok_arr,
                              const int32_t *pos, int32_t *ids, SampleState *st, const int32_t *on, float *probs,
                              hipStream_t s)
{
    hipLaunchKernelGGL(k_sample_rows, dim3(M), dim3(kT), 0, s, logits, n, stride, tok_arr, pos, ids, st, on, probs);
    return hipGetLastError();
}

hipError_t launch_sample(const float *logits, int n, const int32_t *ctx, int n_ctx, const smx_sampling &sp,
                         double u, float *probs, int32_t *out, hipStream_t s)
{
    hipLaunchKernelGGL(k_sample, dim3(1), dim3(kT), 0, s, logits, n, ctx, n_ctx, sp, u, probs, out);
    return hipGetLastError();
}

hipError_t launch_sample_step(const float *logits, int n, int32_t *tokens, int32_t *pos, SampleState *st,
                              float *probs, hipStream_t s)
{
    hipLaunchKernelGGL(k_sample_step, dim3(1), dim3(kT), 0, s, logits, n, tokens, pos, st, probs);
    return hipGetLastError();
}

}  // namespace smx
