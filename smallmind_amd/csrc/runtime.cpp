// runtime.cpp -- host runtime and C-ABI of libsmx.so.
//
// Model-level boundary: TransformerModel.Forward + KV cache (TransformerModel.cs:272-344,
// :476-506) and the per-token driver InferenceSession.GenerateNextTokenAsync
// (InferenceSession.cs:478-607).  A decode step is one pass of fused kernels:
//
//   embed -> per layer [ norm+QKV GEMV (+RoPE, K/V append) -> attention -> O GEMV (+residual)
//                        -> norm+gate/up GEMV (+SwiGLU | GELU) -> down GEMV (+residual) ]
//         -> final norm + head GEMV -> argmax (token appended, position advanced on device)
//
// The token array and the position live in device memory, so a step is captured once as a
// hipGraph per session and replayed without host round trips.
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <map>
#include <mutex>
#include <memory>
#include <string>
#include <vector>

#include "smx_internal.h"

using namespace smx;

#define SMX_FAIL(code, ...)                                          \
    do {                                                             \
        char _b[512];                                                \
        snprintf(_b, sizeof(_b), __VA_ARGS__);                       \
        set_error(_b);                                               \
        return (code);                                               \
    } while (0)

#define SMX_HIP(expr)                                                                       \
    do {                                                                                    \
        hipError_t _e = (expr);                                                             \
        if (_e != hipSuccess) SMX_FAIL(_e == hipErrorOutOfMemory ? SMX_ENOMEM : SMX_EDEVICE, \
                                       "%s: %s", #expr, hipGetErrorString(_e));             \
    } while (0)

namespace {

// A weight matrix in the backend layout.
struct Mat {
    int fmt = -1;
    int64_t rows = 0, cols = 0;
    uint8_t *q = nullptr;
    uint16_t *d = nullptr;
    uint64_t rows_loaded = 0;   // bitmask of uploaded row groups (QKV: 1,2,4; gate/up: 1,2)
    int cache = 0;              // kept resident in the MALL (plain loads), see plan_mall_residency

    WView view() const
    {
        WView v;
        v.fmt = fmt;
        v.q = q;
        v.d = d;
        v.rows = rows;
        v.cols = cols;
        v.nb = fmt < 0 ? 0 : (int)(cols / fmt_block_elems(fmt));
        v.cache = cache;
        return v;
    }
    int64_t bytes() const
    {
        if (fmt < 0) return 0;
        const int64_t nb = cols / fmt_block_elems(fmt);
        return rows * nb * (fmt_main_bytes(fmt) + fmt_d_bytes(fmt));
    }
    void release()
    {
        if (q) (void)hipFree(q);
        if (d) (void)hipFree(d);
        q = nullptr;
        d = nullptr;
        fmt = -1;
    }
};

// Allocates m as [rows][cols] of fmt; no-op when already allocated with the same geometry.
int mat_alloc(Mat &m, int fmt, int64_t rows, int64_t cols)
{
    if (m.fmt >= 0) {
        if (m.fmt != fmt || m.rows != rows || m.cols != cols)
            SMX_FAIL(SMX_EUNSUPPORTED, "fused matrix parts must share one quantization type "
                                       "(have type fmt %d, got fmt %d)", m.fmt, fmt);
        return SMX_OK;
    }
    const int64_t nb = cols / fmt_block_elems(fmt);
    // the kernels address a matrix with 32-bit byte offsets, so larger ones are refused here,
    // before any size arithmetic could wrap into a short allocation (callers bound cols)
    if (rows > (INT64_C(1) << 32) || (uint64_t)rows * (uint64_t)nb * (uint64_t)fmt_main_bytes(fmt) >= (1ull << 32))
        SMX_FAIL(SMX_EUNSUPPORTED, "matrix [%lld x %lld] exceeds the 4 GiB the kernels address", (long long)rows,
                 (long long)cols);
    SMX_HIP(hipMalloc((void **)&m.q, (size_t)(rows * nb * fmt_main_bytes(fmt))));
    if (fmt_has_d(fmt)) SMX_HIP(hipMalloc((void **)&m.d, (size_t)(rows * nb * fmt_d_bytes(fmt))));
    m.fmt = fmt;
    m.rows = rows;
    m.cols = cols;
    return SMX_OK;
}

// Copies GGUF rows (host or device) into rows row_off + r*row_step of m.
int mat_upload(Mat &m, const void *bytes, int64_t rows, int64_t cols, int on_device,
               int64_t row_off, int64_t row_step, hipStream_t s)
{
    const size_t nbytes = (size_t)(rows * (cols / fmt_block_elems(m.fmt)) * fmt_gguf_bytes(m.fmt));
    const uint8_t *src = (const uint8_t *)bytes;
    uint8_t *staging = nullptr;
    if (!on_device) {
        SMX_HIP(hipMalloc((void **)&staging, nbytes));
        hipError_t e = hipMemcpyAsync(staging, bytes, nbytes, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) { (void)hipFree(staging); SMX_HIP(e); }
        src = staging;
    }
    hipError_t e = launch_repack(m.fmt, src, rows, cols, m.q, m.d, m.rows, row_off, row_step, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (staging) (void)hipFree(staging);
    SMX_HIP(e);
    return SMX_OK;
}

// Device memory reused across calls instead of allocated per call: grown on demand (to the
// largest request seen), with its uses on different streams ordered by an event -- each use
// waits for the previous one.  The caller holds the mutex that guards it.
struct Scratch {
    void *p = nullptr;
    size_t cap = 0;
    hipEvent_t last = nullptr;
    bool used = false;
};

// Returns S.p with at least `need` bytes, ready for a use queued on stream s.
int scratch_acquire(Scratch &S, size_t need, hipStream_t s, void **out)
{
    if (!S.last) SMX_HIP(hipEventCreateWithFlags(&S.last, hipEventDisableTiming));
    if (need > S.cap) {
        if (S.used) SMX_HIP(hipEventSynchronize(S.last));   // every earlier use has finished
        if (S.p) (void)hipFree(S.p);
        S.p = nullptr;
        S.cap = 0;
        SMX_HIP(hipMalloc(&S.p, need));
        S.cap = need;
    } else if (S.used) {
        SMX_HIP(hipStreamWaitEvent(s, S.last, 0));
    }
    *out = S.p;
    return SMX_OK;
}

// Marks the end of a use queued on stream s.
int scratch_release(Scratch &S, hipStream_t s)
{
    SMX_HIP(hipEventRecord(S.last, s));
    S.used = true;
    return SMX_OK;
}

void scratch_free(Scratch &S)
{
    if (S.used && S.last) (void)hipEventSynchronize(S.last);
    if (S.p) (void)hipFree(S.p);
    if (S.last) (void)hipEventDestroy(S.last);
    S = Scratch{};
}

// Whether work queued on s is being captured into a graph (stream-ordered allocations are then
// recorded as graph nodes, made once when the graph is instantiated).
bool capturing(hipStream_t s)
{
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(s, &st) == hipSuccess && st == hipStreamCaptureStatusActive;
}

}  // namespace

// The context stream carries model uploads only (serialised by mu); every session and batcher
// runs on a stream of its own, so a graph capture on one never records another thread's work.
struct smx_context {
    int device = 0;
    hipStream_t stream = nullptr;
    std::mutex mu;
};

struct smx_weight {
    int type = 0;
    int device = 0;
    Mat mat;
    // reused device memory, guarded by mu: the GEMM's activation parts, and the staging of the
    // host-memory entry points (activations in, products or dequantized rows out) with the
    // stream they run on
    std::mutex mu;
    Scratch xp, act, out;
    hipStream_t host_stream = nullptr;
};

struct Layer {
    Mat qkv, o, gu, down;
    std::vector<float> attn_g, attn_b, ffn_g, ffn_b, bqkv, bo, bgu, bdown;
    bool has_bqkv = false, has_bgu = false;
    float *d_attn_g = nullptr, *d_attn_b = nullptr, *d_ffn_g = nullptr, *d_ffn_b = nullptr;
    float *d_bqkv = nullptr, *d_bo = nullptr, *d_bgu = nullptr, *d_bdown = nullptr;
};

struct smx_model {
    smx_context *ctx = nullptr;
    smx_model_config cfg{};
    int hd = 0, kvdim = 0, nqkv = 0, hidden = 0;
    bool llama = true;
    Mat tok, pos, head;
    bool head_tied = false;
    std::vector<float> out_g, out_b;
    float *d_out_g = nullptr, *d_out_b = nullptr;
    std::vector<Layer> layers;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    bool dense_layers = false;   // some layer matrix is F16 / F32 (no folded norms)
    int64_t mall_kept = 0;       // bytes of the matrices kept resident in the MALL
    bool finalized = false;
    std::atomic<int> sessions{0};
};

// Device state for running a batch of tokens through the model at once: a prefill chunk of
// one session, or one token of each of several sessions stepping in lockstep.  Token t has
// its own id, position, KV cache (kc/vc: the session's layer-0 cache base) and token array.
struct TokBatch {
    int cap = 0, logits_rows = 0;
    float *x = nullptr, *q = nullptr, *att = nullptr, *h = nullptr, *logits = nullptr;
    uint8_t *xp = nullptr;    // activation parts prepared by k_qprep (QKV, gate/up, head)
    uint8_t *xp2 = nullptr;   // activation parts written by the producing kernel (O, down)
    float *ss = nullptr;      // folded RMSNorm: per-16-row-tile sums of x^2 [d_model / 16][cap]
    int32_t *ids = nullptr, *pos = nullptr;
    float **kc = nullptr, **vc = nullptr;
    int32_t **tok_arr = nullptr;
    int32_t *blk = nullptr;   // prefill attention blocks of several sessions' runs: (row, rows) pairs
};

struct smx_session {
    smx_model *m = nullptr;
    hipStream_t stream = nullptr;   // this session's work, its graph captures and replays
    int max_ctx = 0;
    // KV cache row length: max_ctx rounded up to 4 positions, so K rows are 16-byte aligned
    // (the one-launch decode attention reads them as float4)
    int ctx_stride = 0;
    // the decode step reads the model's MALL-resident matrices with plain loads and the rest
    // with the non-temporal hint (false: every matrix with plain loads)
    bool mall_plan = true;
    float *kc = nullptr, *vc = nullptr;
    float *x = nullptr, *q = nullptr, *att = nullptr, *h = nullptr, *logits = nullptr;
    float *scores = nullptr;   // decode attention scores [n_head][max_ctx]
    int32_t *tokens = nullptr, *pos = nullptr, *amax = nullptr;
    // argmax fused into the head GEMV: per-workgroup partials
    float *head_val = nullptr;
    int32_t *head_idx = nullptr;
    // g_decode looks up the embedding of tokens[pos]; g_decode_next follows a decode step, whose
    // argmax already wrote the embedding row of the token it appended
    hipGraphExec_t g_prefill = nullptr, g_decode = nullptr, g_decode_next = nullptr;
    // kDecodeBlock chained decode steps in one graph: one launch per block of tokens when no
    // per-step logits are copied out
    hipGraphExec_t g_decode_block = nullptr;
    // sampled generation: the step graph (embedding, layers, head logits, sampling), its device
    // state and the probability scratch, made on first use
    hipGraphExec_t g_sample = nullptr;
    SampleState *samp = nullptr;
    float *probs = nullptr;
    TokBatch pb;            // prefill chunks on the matrix cores (allocated on first use)
    hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
    std::atomic<int> busy{0};
    // generation control: smx_session_cancel sets `cancel` from any thread (the generation that
    // observes it stops and clears it); smx_session_set_max_time sets the time limit (0 = none)
    std::atomic<int> cancel{0};
    std::atomic<int32_t> max_time_ms{0};
};

namespace {

void free_dev(void *p)
{
    if (p) (void)hipFree(p);
}

int upload_floats(float **dst, const std::vector<float> &v, hipStream_t s)
{
    if (v.empty()) return SMX_OK;
    SMX_HIP(hipMalloc((void **)dst, v.size() * 4));
    SMX_HIP(hipMemcpyAsync(*dst, v.data(), v.size() * 4, hipMemcpyHostToDevice, s));
    return SMX_OK;
}

// Parses "blk.N.rest" -> N and rest; returns -1 for non-layer names.
int parse_layer(const char *name, std::string &rest)
{
    int li = -1, consumed = 0;
    if (sscanf(name, "blk.%d.%n", &li, &consumed) == 1 && consumed > 0) {
        rest = name + consumed;
        return li;
    }
    rest = name;
    return -1;
}

// Builds the step's kernel sequence on stream s (captured into a graph by the caller).
// with_embed = false: x already holds the step's embedding row, written by the previous decode
// step's argmax (a step with a head folds the next step's embedding lookup into its argmax).
// The weight streams of a matrix as prefetch ranges (its main bytes, then its scale stream).
void add_prefetch(Prefetch &pf, const Mat &M)
{
    if (M.fmt < 0) return;
    const uint64_t nb = (uint64_t)(M.cols / fmt_block_elems(M.fmt));
    const uint64_t qb = (uint64_t)M.rows * nb * fmt_main_bytes(M.fmt), db = (uint64_t)M.rows * nb * fmt_d_bytes(M.fmt);
    if (M.q && qb && qb < (1ull << 32) && pf.n < Prefetch::kMax) {
        pf.p[pf.n] = M.q;
        pf.bytes[pf.n++] = (uint32_t)qb;
    }
    if (M.d && db && db < (1ull << 32) && pf.n < Prefetch::kMax) {
        pf.p[pf.n] = (const uint8_t *)M.d;
        pf.bytes[pf.n++] = (uint32_t)db;
    }
}

// A matrix as the decode step reads it (plain or non-temporal loads, smx_session::mall_plan).
static WView step_view(const smx_session *S, const Mat &w)
{
    WView v = w.view();
    if (!S->mall_plan) v.cache = 1;
    return v;
}

int enqueue_step(smx_session *S, bool with_head, bool with_embed, hipStream_t s, bool sample = false)
{
    smx_model *m = S->m;
    const smx_model_config &c = m->cfg;
    const int Hkv = c.n_kv_head, hd = m->hd;
    const size_t layer_cache = (size_t)Hkv * S->ctx_stride * hd;
    WView posw = m->pos.view();
    if (with_embed)
        SMX_HIP(launch_embed(m->tok.view(), m->llama ? nullptr : &posw, S->tokens, S->pos, S->x, s));
    for (int l = 0; l < c.n_layer; l++) {
        Layer &L = m->layers[l];
        GemvArgs a{};
        a.w = step_view(S, L.qkv);
        a.x = S->x;
        a.out = S->q;
        a.bias = L.d_bqkv;
        a.gamma = L.d_attn_g;
        a.beta = L.d_attn_b;
        a.eps = c.norm_eps;
        a.pro = m->llama ? PRO_RMS : PRO_LN;
        a.epi = EPI_QKV;
        a.d_model = c.d_model;
        a.kv_dim = m->kvdim;
        a.head_dim = hd;
        a.ctx_stride = S->ctx_stride;
        a.use_rope = m->llama ? 1 : 0;
        a.k_cache = S->kc + l * layer_cache;
        a.v_cache = S->vc + l * layer_cache;
        a.rope_cos = m->rope_cos;
        a.rope_sin = m->rope_sin;
        a.pos = S->pos;
        SMX_HIP(launch_gemv(a, 1, s));

        // long contexts: two partial attention outputs, summed by the O projection's staging
        const int att_parts = attention_pv_chunks(S->max_ctx, 2);
        // Idle CUs of the attention launch read the O projection's weights into the MALL, where
        // the next kernel finds them (measured: +0.9% decode tok/s on configs[2]; prefetching
        // gate/up and down as well lengthens the attention launch by more than it saves).
        Prefetch pf{};
        add_prefetch(pf, L.o);
        SMX_HIP(launch_attention_split(S->q, a.k_cache, a.v_cache, S->att, S->scores, c.n_head, Hkv, hd,
                                       S->ctx_stride, S->pos, 0, S->max_ctx, s, 2, &pf));

        GemvArgs o{};
        o.w = step_view(S, L.o);
        o.x = S->att;
        o.x_parts = att_parts;
        o.x_part_stride = (int64_t)c.n_head * hd;
        o.out = S->x;
        o.resid = S->x;
        o.bias = L.d_bo;
        o.pro = PRO_NONE;
        o.epi = EPI_RESID;
        SMX_HIP(launch_gemv(o, 1, s));

        GemvArgs g{};
        g.w = step_view(S, L.gu);
        g.x = S->x;
        g.out = S->h;
        g.bias = L.d_bgu;
        g.gamma = L.d_ffn_g;
        g.beta = L.d_ffn_b;
        g.eps = c.norm_eps;
        g.pro = m->llama ? PRO_RMS : PRO_LN;
        g.epi = m->llama ? EPI_SILU : EPI_GELU;
        SMX_HIP(launch_gemv(g, 1, s));

        GemvArgs dn{};
        dn.w = step_view(S, L.down);
        dn.x = S->h;
        dn.out = S->x;
        dn.resid = S->x;
        dn.bias = L.d_bdown;
        dn.pro = PRO_NONE;
        dn.epi = EPI_RESID;
        SMX_HIP(launch_gemv(dn, 1, s));
    }
    if (with_head && sample) {   // logits, then the sampling pipeline appends the token
        GemvArgs hgt{};
        hgt.w = step_view(S, m->head);
        hgt.x = S->x;
        hgt.out = S->logits;
        hgt.gamma = m->d_out_g;
        hgt.beta = m->d_out_b;
        hgt.eps = c.norm_eps;
        hgt.pro = m->llama ? PRO_RMS : PRO_LN;
        hgt.epi = EPI_STORE;
        SMX_HIP(launch_gemv(hgt, 1, s));
        SMX_HIP(launch_sample_step(S->logits, c.vocab, S->tokens, S->pos, S->samp, S->probs, s));
    } else if (with_head) {
        GemvArgs hgt{};
        hgt.w = step_view(S, m->head);
        hgt.x = S->x;
        hgt.out = S->logits;
        hgt.gamma = m->d_out_g;
        hgt.beta = m->d_out_b;
        hgt.eps = c.norm_eps;
        hgt.pro = m->llama ? PRO_RMS : PRO_LN;
        hgt.epi = EPI_ARGMAX;
        hgt.wg_val = S->head_val;
        hgt.wg_idx = S->head_idx;
        hgt.amax_out = S->amax;
        hgt.tokens = S->tokens;
        hgt.tok_pos = S->pos;
        hgt.x_next = S->x;   // x is dead once the head has read it
        hgt.next_emb = m->tok.view();
        if (!m->llama) hgt.next_embp = posw;
        SMX_HIP(launch_gemv(hgt, 1, s));
    } else {
        SMX_HIP(launch_advance(S->pos, s));
    }
    return SMX_OK;
}

constexpr int kDecodeBlock = 8;

// Between graph launches a generation stops early on the caller's request: smx_session_cancel
// (the reference checks its CancellationToken before every token, InferenceSession.cs:211,
// :481) or the session's time limit (MaxTimeMs, InferenceSession.cs:164-172, :287-291).
struct StopCheck {
    std::vector<std::atomic<int> *> flags;
    std::chrono::steady_clock::time_point deadline{};
    bool timed = false;
    // one deadline for the call: the smallest positive limit among the sessions
    void add(smx_session *S, std::chrono::steady_clock::time_point t0)
    {
        flags.push_back(&S->cancel);
        const int32_t ms = S->max_time_ms.load();
        if (ms > 0) {
            const auto d = t0 + std::chrono::milliseconds(ms);
            if (!timed || d < deadline) deadline = d;
            timed = true;
        }
    }
    // SMX_OK to go on, else the status the call returns; a cancel request is consumed
    int poll()
    {
        for (std::atomic<int> *f : flags)
            if (f->exchange(0) != 0) return SMX_ECANCELED;
        if (timed && std::chrono::steady_clock::now() >= deadline) return SMX_ETIMEDOUT;
        return SMX_OK;
    }
};

// Keeps the host at most `depth` launches ahead of the device: after each launch an event is
// recorded, and the host waits for the one `depth` launches back.  The device always has queued
// work, and a stop request takes effect within `depth` launches.
class Pacer {
    static constexpr int kRing = 16;
    hipEvent_t ev_[kRing] = {};
    hipStream_t s_;
    int depth_;
    long n_ = 0;

public:
    Pacer(hipStream_t s, int depth) : s_(s), depth_(std::min(std::max(depth, 1), kRing - 1)) {}
    ~Pacer()
    {
        for (hipEvent_t e : ev_) if (e) (void)hipEventDestroy(e);
    }
    hipError_t launched()
    {
        hipEvent_t &e = ev_[n_ % kRing];
        hipError_t r = e ? hipSuccess : hipEventCreateWithFlags(&e, hipEventDisableTiming);
        if (r == hipSuccess) r = hipEventRecord(e, s_);
        n_++;
        if (r == hipSuccess && n_ > depth_) r = hipEventSynchronize(ev_[(n_ - 1 - depth_) % kRing]);
        return r;
    }
};

// Captures `steps` consecutive steps (steps > 1: chained decode steps) into one graph.
int capture_step(smx_session *S, bool with_head, bool with_embed, hipGraphExec_t *out, int steps = 1,
                 bool sample = false)
{
    hipStream_t s = S->stream;
    hipGraph_t graph = nullptr;
    SMX_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    int rc = SMX_OK;
    for (int i = 0; i < steps && rc == SMX_OK; i++) rc = enqueue_step(S, with_head, with_embed, s, sample);
    hipError_t e = hipStreamEndCapture(s, &graph);
    if (rc != SMX_OK) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc;
    }
    SMX_HIP(e);
    e = hipGraphInstantiate(out, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    SMX_HIP(e);
    return SMX_OK;
}

void batch_free(TokBatch &B)
{
    free_dev(B.x); free_dev(B.q); free_dev(B.att); free_dev(B.h); free_dev(B.logits);
    free_dev(B.xp); free_dev(B.xp2); free_dev(B.ss); free_dev(B.ids); free_dev(B.pos); free_dev(B.kc); free_dev(B.vc);
    free_dev(B.tok_arr); free_dev(B.blk);
    B = TokBatch{};
}

int batch_alloc(const smx_model *m, TokBatch &B, int cap, int logits_rows)
{
    const smx_model_config &c = m->cfg;
    const int64_t maxk = m->hidden > c.d_model ? m->hidden : c.d_model;
    hipError_t e = hipSuccess;
    auto A = [&](void **p, size_t n) { if (e == hipSuccess) e = hipMalloc(p, n); };
    A((void **)&B.x, (size_t)cap * c.d_model * 4);
    A((void **)&B.q, (size_t)cap * m->nqkv * 4);
    A((void **)&B.att, (size_t)cap * c.d_model * 4);
    A((void **)&B.h, (size_t)cap * maxk * 4);
    A((void **)&B.logits, (size_t)logits_rows * c.vocab * 4);
    A((void **)&B.xp, qgemm_xp_bytes(cap, (int)maxk));
    A((void **)&B.xp2, qgemm_xp_bytes(cap, (int)maxk));
    A((void **)&B.ss, (size_t)((c.d_model + 15) / 16) * cap * 4);
    A((void **)&B.ids, (size_t)cap * 4);
    A((void **)&B.pos, (size_t)cap * 4);
    A((void **)&B.kc, (size_t)cap * sizeof(float *));
    A((void **)&B.vc, (size_t)cap * sizeof(float *));
    A((void **)&B.tok_arr, (size_t)cap * sizeof(int32_t *));
    A((void **)&B.blk, (size_t)cap * 2 * 4);   // every block holds at least one row
    if (e != hipSuccess) {
        batch_free(B);
        SMX_HIP(e);
    }
    B.cap = cap;
    B.logits_rows = logits_rows;
    return SMX_OK;
}

// Rows row0 .. row0+count-1 of a token batch are consecutive tokens p_first .. of one session
// (a prefill chunk, or one session's part of a batch of several sessions' prompts): their
// attention runs as one causal block over that session's cache instead of per (token, head).
struct PrefillRun {
    const float *kc, *vc;
    int p_first;
    int row0 = 0, count = -1;   // count < 0: all M rows
};

// Runs tokens 0..M-1 of B (ids, pos, kc, vc filled on the device) through every layer on the
// matrix-core GEMM path, writing K/V into each token's cache; the final norm + head run on rows
// head_from..M-1 into B.logits.  Same graph as enqueue_step, per token.
// With n_blk > 0, B.blk holds the runs split into attention blocks (attention_prefill_blocks),
// and the prefill attention of all runs is one launch per layer.
int run_tokens(const smx_model *m, TokBatch &B, int M, int ctx_stride, int head_from, hipStream_t s,
               const PrefillRun *run, int n_run = 1, int n_blk = 0)
{
    const smx_model_config &c = m->cfg;
    const int d = c.d_model, hd = m->hd, Hkv = c.n_kv_head;
    const int pro = m->llama ? PRO_RMS : PRO_LN;
    // host-side bounds of the batch buffers: M rows fit the buffers, the head rows fit the logits
    // buffer, and every prefill run lies inside the M rows
    if (M <= 0 || M > B.cap) SMX_FAIL(SMX_EINVAL, "run_tokens: %d rows for a batch of %d", M, B.cap);
    if (n_blk < 0 || n_blk > M || (n_blk > 0 && !run))
        SMX_FAIL(SMX_EINVAL, "run_tokens: %d attention blocks for %d rows", n_blk, M);
    if (head_from < M && (head_from < 0 || M - head_from > B.logits_rows))
        SMX_FAIL(SMX_EINVAL, "run_tokens: head rows %d..%d for %d logits rows", head_from, M - 1, B.logits_rows);
    for (int i = 0; run && i < n_run; i++) {
        const int cnt = run[i].count < 0 ? M : run[i].count;
        if (run[i].row0 < 0 || cnt <= 0 || run[i].row0 + cnt > M || run[i].p_first < 0 ||
            (int64_t)run[i].p_first + cnt > ctx_stride)
            SMX_FAIL(SMX_EINVAL, "run_tokens: prefill run %d (rows %d + %d at position %d) outside the batch of %d "
                     "rows or the cache row of %d", i, run[i].row0, cnt, run[i].p_first, M, ctx_stride);
    }
    // Up to 16 tokens, RMSNorm is folded into the GEMMs around it: the O and down projections
    // write the next norm's input as parts of gamma (.) x plus per-tile sums of x^2, and the
    // QKV (after layer 0) and gate/up GEMMs scale by 1 / rms -- no k_qprep launch per norm.
    // (the GEMMs reduce up to 256 tile sums per token: d_model up to 4096)
    const bool fold = m->llama && M <= 16 && d % 256 == 0 && d <= 4096 && m->hidden % 256 == 0 && !m->dense_layers;
    WView posw = m->pos.view();
    SMX_HIP(launch_embed_tokens(m->tok.view(), m->llama ? nullptr : &posw, B.ids, B.pos, B.x, d, M, s));
    for (int l = 0; l < c.n_layer; l++) {
        const Layer &L = m->layers[l];
        const bool fold_in = fold && l > 0;   // QKV parts written by the previous down projection
        const int64_t layer_off = (int64_t)l * Hkv * ctx_stride * hd;
        QgemmArgs a{};
        a.w = L.qkv.view();
        a.xp = B.xp;
        a.M = M;
        a.y = B.q;
        a.y_stride = m->nqkv;
        a.bias = L.d_bqkv;
        a.epi = EPI_QKV;
        a.d_model = d;
        a.kv_dim = m->kvdim;
        a.head_dim = hd;
        a.use_rope = m->llama ? 1 : 0;
        a.ctx_stride = ctx_stride;
        a.layer_off = layer_off;
        a.kc_tok = B.kc;
        a.vc_tok = B.vc;
        a.tok_pos = B.pos;
        a.rope_cos = m->rope_cos;
        a.rope_sin = m->rope_sin;
        if (fold_in) {
            a.rss = B.ss;
            a.rss_n = d / 16;
            a.r_eps = c.norm_eps;
            SMX_HIP(launch_qgemm(a, nullptr, d, PRO_NONE, nullptr, nullptr, 0.0f, s));
        } else {
            SMX_HIP(launch_qgemm(a, B.x, d, pro, L.d_attn_g, L.d_attn_b, c.norm_eps, s));
        }
        // attention writes the O projection's activation parts directly (no k_qprep launch)
        if (run && n_blk > 0 && attention_prefill_supported(c.n_head, Hkv, hd)) {
            const PrefillBlocks pb{B.blk, B.kc, B.vc, B.pos, layer_off};
            SMX_HIP(launch_attention_prefill_blocks(B.q, m->nqkv, B.att, d, c.n_head, Hkv, hd, ctx_stride, n_blk, pb,
                                                    s, B.xp2));
        } else if (run && attention_prefill_supported(c.n_head, Hkv, hd)) {
            for (int i = 0; i < n_run; i++) {
                const PrefillRun &r = run[i];
                const int cnt = r.count < 0 ? M : r.count;
                SMX_HIP(launch_attention_prefill(B.q + (int64_t)r.row0 * m->nqkv, m->nqkv, r.kc + layer_off,
                                                 r.vc + layer_off, B.att + (int64_t)r.row0 * d, d, c.n_head, Hkv, hd,
                                                 ctx_stride, r.p_first, cnt, s, B.xp2, r.row0));
            }
        } else
            SMX_HIP(launch_attention_tokens(B.q, m->nqkv, B.kc, B.vc, layer_off, B.att, d, c.n_head, Hkv, hd,
                                            ctx_stride, B.pos, M, s, B.xp2));
        QgemmArgs o{};
        o.w = L.o.view();
        o.xp = B.xp2;
        o.M = M;
        o.y = B.x;
        o.y_stride = d;
        o.bias = L.d_bo;
        o.epi = EPI_RESID;
        if (fold) {
            o.np = B.xp;
            o.ngamma = L.d_ffn_g;
            o.nss = B.ss;
        }
        SMX_HIP(launch_qgemm(o, nullptr, d, PRO_NONE, nullptr, nullptr, 0.0f, s));
        QgemmArgs g{};
        g.w = L.gu.view();
        g.xp = B.xp;
        g.M = M;
        g.y = B.h;
        g.y_stride = m->hidden;
        g.bias = L.d_bgu;
        g.epi = m->llama ? EPI_SILU : EPI_GELU;
        g.yp = B.xp2;   // the down projection's activation parts
        if (fold) {
            g.rss = B.ss;
            g.rss_n = d / 16;
            g.r_eps = c.norm_eps;
            SMX_HIP(launch_qgemm(g, nullptr, d, PRO_NONE, nullptr, nullptr, 0.0f, s));
        } else {
            SMX_HIP(launch_qgemm(g, B.x, d, pro, L.d_ffn_g, L.d_ffn_b, c.norm_eps, s));
        }
        QgemmArgs dn{};
        dn.w = L.down.view();
        dn.xp = B.xp2;
        dn.M = M;
        dn.y = B.x;
        dn.y_stride = d;
        dn.bias = L.d_bdown;
        dn.epi = EPI_RESID;
        if (fold && l + 1 < c.n_layer) {
            dn.np = B.xp;
            dn.ngamma = m->layers[l + 1].d_attn_g;
            dn.nss = B.ss;
        }
        SMX_HIP(launch_qgemm(dn, nullptr, m->hidden, PRO_NONE, nullptr, nullptr, 0.0f, s));
    }
    if (head_from < M && fmt_dense(m->head.fmt)) {
        // an unquantized head: the fused GEMV (norm prologue per row), one pass per row
        GemvArgs hg{};
        hg.w = m->head.view();
        hg.x = B.x + (int64_t)head_from * d;
        hg.x_stride = d;
        hg.out = B.logits;
        hg.out_stride = c.vocab;
        hg.gamma = m->d_out_g;
        hg.beta = m->d_out_b;
        hg.eps = c.norm_eps;
        hg.pro = pro;
        hg.epi = EPI_STORE;
        SMX_HIP(launch_gemv(hg, M - head_from, s));
    } else if (head_from < M) {
        QgemmArgs hq{};
        hq.w = m->head.view();
        hq.xp = B.xp;
        hq.M = M - head_from;
        hq.y = B.logits;
        hq.y_stride = c.vocab;
        hq.epi = EPI_STORE;
        SMX_HIP(launch_qgemm(hq, B.x + (int64_t)head_from * d, d, pro, m->d_out_g, m->d_out_b, c.norm_eps, s));
    }
    return SMX_OK;
}

// Tokens of one session per prefill chunk on the matrix-core path: long chunks give the GEMMs
// more token tiles per weight read and fewer launches (configs[2] 512-token prompt 50.6K ->
// 58.9K tok/s as one chunk instead of two; configs[3] 4096 tokens 38.0K / 43.6K / 46.0K /
// 46.3K tok/s at 256 / 1024 / 2048 / 4096-token chunks).  The chunk buffers hold at least 256
// tokens: a session of 83 positions with 96-token buffers ended its process with a host
// segmentation fault once.  Reading the paths that depend on the buffer size found no
// out-of-bounds access (the GEMM clamps its part loads to the last token tile, the prefill
// attention clamps keys to the cache row, the host arrays hold cap entries with M <= cap, and
// run_tokens now checks those bounds); with no cause shown, no smaller size has run since.
constexpr int kPrefillChunk = 2048, kPrefillChunkMin = 256;

// Runs tokens[0..n) of session S at positions p0.. through the model in chunks (K/V written
// to the session cache).  With want_head, the last token's logits land in S->logits and its
// argmax is appended to the session token array at p0 + n with the device position advanced
// to p0 + n, exactly as a decode step leaves them; without, the device position is untouched.
// Prompts shorter than kPrefillMin tokens go through the per-token decode graph instead.
constexpr int kPrefillMin = 8;
int prefill_tokens(smx_session *S, const int32_t *tokens_host, int n, int p0, bool want_head, hipStream_t s)
{
    smx_model *m = S->m;
    // chunk length: kPrefillChunk, or the session's whole context when that is shorter (the
    // chunk buffers are sized for it), and at least kPrefillChunkMin tokens
    const int chunk = std::max(kPrefillChunkMin, std::min(kPrefillChunk, (S->max_ctx + 15) & ~15));
    if (!S->pb.cap) {
        int rc = batch_alloc(m, S->pb, chunk, 1);
        if (rc != SMX_OK) return rc;
        std::vector<float *> kc((size_t)chunk, S->kc), vc((size_t)chunk, S->vc);
        std::vector<int32_t *> ta((size_t)chunk, S->tokens);
        SMX_HIP(hipMemcpyAsync(S->pb.kc, kc.data(), kc.size() * sizeof(float *), hipMemcpyHostToDevice, s));
        SMX_HIP(hipMemcpyAsync(S->pb.vc, vc.data(), vc.size() * sizeof(float *), hipMemcpyHostToDevice, s));
        SMX_HIP(hipMemcpyAsync(S->pb.tok_arr, ta.data(), ta.size() * sizeof(int32_t *), hipMemcpyHostToDevice, s));
        SMX_HIP(hipStreamSynchronize(s));
    }
    TokBatch &B = S->pb;
    if (chunk > B.cap) SMX_FAIL(SMX_EINVAL, "prefill_tokens: chunk %d exceeds the buffers of %d rows", chunk, B.cap);
    std::vector<int32_t> pos((size_t)chunk);
    for (int i0 = 0; i0 < n; i0 += chunk) {
        const int M = n - i0 < chunk ? n - i0 : chunk;
        for (int i = 0; i < M; i++) pos[(size_t)i] = p0 + i0 + i;
        SMX_HIP(hipMemcpyAsync(B.ids, tokens_host + i0, (size_t)M * 4, hipMemcpyHostToDevice, s));
        SMX_HIP(hipMemcpyAsync(B.pos, pos.data(), (size_t)M * 4, hipMemcpyHostToDevice, s));
        const bool last = i0 + M == n;
        const PrefillRun run{S->kc, S->vc, p0 + i0};
        int rc = run_tokens(m, B, M, S->ctx_stride, (want_head && last) ? M - 1 : M, s, &run);
        if (rc != SMX_OK) return rc;
        // the host arrays are reused by the next chunk: let this chunk's copies finish
        SMX_HIP(hipStreamSynchronize(s));
    }
    if (want_head) {
        // token array / position exactly as after a decode step at position p0 + n - 1
        const int32_t plast = p0 + n - 1;
        SMX_HIP(hipMemcpyAsync(S->pos, &plast, 4, hipMemcpyHostToDevice, s));
        SMX_HIP(launch_argmax_rows(B.logits, m->cfg.vocab, m->cfg.vocab, 1, S->amax, S->pos, B.tok_arr, s));
        SMX_HIP(hipMemcpyAsync(S->logits, B.logits, (size_t)m->cfg.vocab * 4, hipMemcpyDeviceToDevice, s));
        SMX_HIP(hipStreamSynchronize(s));
    }
    return SMX_OK;
}

// Chunk buffer size for a prefill of n tokens: up to kPrefillChunk, at least kPrefillChunkMin.
int prefill_cap(int64_t n)
{
    const int64_t r = (n + 15) & ~(int64_t)15;
    return (int)std::max<int64_t>(kPrefillChunkMin, std::min<int64_t>(kPrefillChunk, r));
}

// The prompts of several sessions of one model (all but each prompt's last token) through the
// matrix-core path together: their tokens are packed into chunks of up to P.cap rows, each
// row carrying its own session's cache and position, so the GEMMs see long chunks instead of
// one short prompt at a time; each session's rows of a chunk attend over its own cache.
int prefill_sessions(smx_model *m, TokBatch &P, smx_session *const *sessions, int n, const int32_t *prompts,
                     const int64_t *off, const int *lens, hipStream_t s)
{
    const int cap = P.cap, ctx_stride = sessions[0]->ctx_stride;
    std::vector<int32_t> ids((size_t)cap), pos((size_t)cap);
    std::vector<float *> kc((size_t)cap), vc((size_t)cap);
    std::vector<int32_t *> ta((size_t)cap);
    std::vector<PrefillRun> runs;
    // the runs of a chunk split into prefill-attention blocks (batch row, rows): one attention
    // launch per layer for all sessions of the chunk instead of one per run
    const smx_model_config &c = m->cfg;
    const bool blocks = attention_prefill_supported(c.n_head, c.n_kv_head, m->hd);
    const int TB = blocks ? attention_prefill_block_rows(c.n_head, c.n_kv_head) : 1;
    std::vector<int32_t> blk((size_t)cap * 2);
    int M = 0;
    auto flush = [&]() -> int {
        if (M == 0) return SMX_OK;
        int nb = 0;
        if (blocks && runs.size() > 1) {
            for (const PrefillRun &r : runs)
                for (int t = 0; t < r.count; t += TB) {
                    blk[(size_t)(2 * nb)] = r.row0 + t;
                    blk[(size_t)(2 * nb + 1)] = std::min(TB, r.count - t);
                    nb++;
                }
            SMX_HIP(hipMemcpyAsync(P.blk, blk.data(), (size_t)nb * 8, hipMemcpyHostToDevice, s));
        }
        SMX_HIP(hipMemcpyAsync(P.ids, ids.data(), (size_t)M * 4, hipMemcpyHostToDevice, s));
        SMX_HIP(hipMemcpyAsync(P.pos, pos.data(), (size_t)M * 4, hipMemcpyHostToDevice, s));
        SMX_HIP(hipMemcpyAsync(P.kc, kc.data(), (size_t)M * sizeof(float *), hipMemcpyHostToDevice, s));
        SMX_HIP(hipMemcpyAsync(P.vc, vc.data(), (size_t)M * sizeof(float *), hipMemcpyHostToDevice, s));
        SMX_HIP(hipMemcpyAsync(P.tok_arr, ta.data(), (size_t)M * sizeof(int32_t *), hipMemcpyHostToDevice, s));
        const int rc = run_tokens(m, P, M, ctx_stride, M, s, runs.data(), (int)runs.size(), nb);
        if (rc != SMX_OK) return rc;
        // the host arrays are reused by the next chunk: let this chunk's copies finish
        SMX_HIP(hipStreamSynchronize(s));
        M = 0;
        runs.clear();
        return SMX_OK;
    };
    for (int i = 0; i < n; i++) {
        smx_session *S = sessions[i];
        const int32_t *tp = prompts + off[i];
        int left = lens[i] - 1, p = 0;
        while (left > 0) {
            const int take = std::min(left, cap - M);
            PrefillRun r{S->kc, S->vc, p};
            r.row0 = M;
            r.count = take;
            runs.push_back(r);
            for (int j = 0; j < take; j++) {
                ids[(size_t)(M + j)] = tp[p + j];
                pos[(size_t)(M + j)] = p + j;
                kc[(size_t)(M + j)] = S->kc;
                vc[(size_t)(M + j)] = S->vc;
                ta[(size_t)(M + j)] = S->tokens;
            }
            M += take;
            p += take;
            left -= take;
            if (M == cap) {
                const int rc = flush();
                if (rc != SMX_OK) return rc;
            }
        }
    }
    return flush();
}

struct BusyGuard {
    std::atomic<int> &flag;
    bool ok;
    explicit BusyGuard(std::atomic<int> &f) : flag(f)
    {
        int expected = 0;
        ok = flag.compare_exchange_strong(expected, 1);
    }
    ~BusyGuard()
    {
        if (ok) flag.store(0);
    }
};

}  // namespace

// =============================================================================================
// C-ABI
// =============================================================================================
extern "C" {

SMX_API const char *smx_version(void) { return "smx 0.1.0 (gfx950)"; }
SMX_API int smx_dequant(int type, const void *blocks_dev, int64_t n, float *out_dev, void *stream)
{
    if (!type_block_elems(type)) SMX_FAIL(SMX_EUNSUPPORTED, "smx_dequant: unsupported type %d", type);
    if (n < 0 || (n > 0 && (!blocks_dev || !out_dev))) SMX_FAIL(SMX_EINVAL, "smx_dequant: bad arguments");
    SMX_HIP(launch_dequant_gguf(type, blocks_dev, n, out_dev, (hipStream_t)stream));
    return SMX_OK;
}

SMX_API int smx_quantize(int type, const float *x_dev, int64_t n, void *blocks_dev, void *stream)
{
    const int be = type_block_elems(type);
    if (!be || type == SMX_TYPE_F32) SMX_FAIL(SMX_EUNSUPPORTED, "smx_quantize: unsupported type %d", type);
    if (n < 0 || n % be) SMX_FAIL(SMX_EINVAL, "smx_quantize: n=%lld is not a multiple of %d", (long long)n, be);
    if (n > 0 && (!x_dev || !blocks_dev)) SMX_FAIL(SMX_EINVAL, "smx_quantize: null pointer");
    SMX_HIP(launch_quantize_gguf(type, x_dev, n, blocks_dev, (hipStream_t)stream));
    return SMX_OK;
}

SMX_API int smx_fill_normal(uint64_t seed, int64_t n, float std, float *out_dev, void *stream)
{
    if (n < 0 || (n > 0 && !out_dev)) SMX_FAIL(SMX_EINVAL, "smx_fill_normal: bad arguments");
    SMX_HIP(launch_fill_normal(seed, n, std, out_dev, (hipStream_t)stream));
    return SMX_OK;
}

// ---- IWeightTensor --------------------------------------------------------------------------
SMX_API int smx_weight_create(int type, int64_t rows, int64_t cols, const void *blocks,
                              int blocks_on_device, smx_weight **out)
{
    if (!out || !blocks) SMX_FAIL(SMX_EINVAL, "smx_weight_create: null argument");
    *out = nullptr;
    const int fmt = fmt_from_type(type);
    if (fmt < 0) SMX_FAIL(SMX_EUNSUPPORTED, "smx_weight_create: type %d is not a weight-matrix type", type);
    if (rows <= 0 || cols <= 0 || cols % fmt_block_elems(fmt))
        SMX_FAIL(SMX_EINVAL, "smx_weight_create: cols=%lld must be a positive multiple of %d",
                 (long long)cols, fmt_block_elems(fmt));
    if (cols > 16384) SMX_FAIL(SMX_EUNSUPPORTED, "smx_weight_create: cols=%lld exceeds 16384", (long long)cols);
    int dev = 0;
    SMX_HIP(hipGetDevice(&dev));
    smx_weight *w = new smx_weight();
    w->type = type;
    w->device = dev;
    int rc = mat_alloc(w->mat, fmt, rows, cols);
    // standalone weights stream with the non-temporal hint, except Q6_K: its three loads per
    // 208-byte super-block ran 25 % slower with it (32000 x 2048: 15.4 against 12.0 us)
    w->mat.cache = fmt == FMT_Q6_K ? 1 : 0;
    if (rc == SMX_OK) rc = mat_upload(w->mat, blocks, rows, cols, blocks_on_device, 0, 1, nullptr);
    if (rc != SMX_OK) {
        w->mat.release();
        delete w;
        return rc;
    }
    *out = w;
    return SMX_OK;
}

SMX_API int smx_weight_info(const smx_weight *w, int *type, int64_t *rows, int64_t *cols)
{
    if (!w) SMX_FAIL(SMX_EINVAL, "smx_weight_info: null weight");
    if (type) *type = w->type;
    if (rows) *rows = w->mat.rows;
    if (cols) *cols = w->mat.cols;
    return SMX_OK;
}

// Activation rows from which IWeightTensor.MatMul uses the matrix-core GEMM instead of one
// GEMV pass per row.
constexpr int kQgemmMinRows = 4;

}  // extern "C"

namespace {
int weight_check(const smx_weight *w, int m, int k, int n, const char *fn)
{
    if (k != w->mat.cols || n != w->mat.rows)
        SMX_FAIL(SMX_EINVAL, "%s: k=%d must equal cols=%lld and n=%d rows=%lld", fn, k, (long long)w->mat.cols, n,
                 (long long)w->mat.rows);
    if (m <= 0 || m > 65535) SMX_FAIL(SMX_EINVAL, "%s: m=%d out of range", fn, m);
    return SMX_OK;
}

// out[m][n] = act[m][k] W^T on device pointers, queued on st.  The caller holds w->mu.
int weight_matmul_dev(smx_weight *w, const float *act_dev, float *out_dev, int m, int k, int n, hipStream_t st)
{
    if (m < kQgemmMinRows) {
        GemvArgs a{};
        a.w = w->mat.view();
        a.x = act_dev;
        a.x_stride = k;
        a.out = out_dev;
        a.out_stride = n;
        a.pro = PRO_NONE;
        a.epi = EPI_STORE;
        SMX_HIP(launch_gemv(a, m, st));
        return SMX_OK;
    }
    // several activation rows: one pass over the weights on the matrix cores
    QgemmArgs q{};
    q.w = w->mat.view();
    q.M = m;
    q.y = out_dev;
    q.y_stride = n;
    q.epi = EPI_STORE;
    const size_t need = qgemm_xp_bytes(m, k);
    if (capturing(st)) {
        // under graph capture the parts are a stream-ordered allocation recorded in the graph
        uint8_t *xp = nullptr;
        SMX_HIP(hipMallocAsync((void **)&xp, need, st));
        q.xp = xp;
        const hipError_t e = launch_qgemm(q, act_dev, k, PRO_NONE, nullptr, nullptr, 0.0f, st);
        const hipError_t f = hipFreeAsync(xp, st);
        SMX_HIP(e);
        SMX_HIP(f);
        return SMX_OK;
    }
    void *xp = nullptr;
    int rc = scratch_acquire(w->xp, need, st, &xp);
    if (rc != SMX_OK) return rc;
    q.xp = (const uint8_t *)xp;
    const hipError_t e = launch_qgemm(q, act_dev, k, PRO_NONE, nullptr, nullptr, 0.0f, st);
    rc = scratch_release(w->xp, st);
    SMX_HIP(e);
    return rc;
}

// Host staging of the host-memory entry points: the weight's own stream and reused device
// buffers.  The caller holds w->mu.
int host_stage(smx_weight *w, size_t in_bytes, size_t out_bytes, void **in_dev, void **out_dev)
{
    SMX_HIP(hipSetDevice(w->device));
    if (!w->host_stream) SMX_HIP(hipStreamCreateWithFlags(&w->host_stream, hipStreamNonBlocking));
    int rc = SMX_OK;
    if (in_bytes && (rc = scratch_acquire(w->act, in_bytes, w->host_stream, in_dev)) != SMX_OK) return rc;
    return scratch_acquire(w->out, out_bytes, w->host_stream, out_dev);
}
}  // namespace

extern "C" {

SMX_API int smx_weight_matmul(const smx_weight *w, const float *act_dev, float *out_dev, int m,
                              int k, int n, void *stream)
{
    if (!w || !act_dev || !out_dev) SMX_FAIL(SMX_EINVAL, "smx_weight_matmul: null argument");
    int rc = weight_check(w, m, k, n, "smx_weight_matmul");
    if (rc != SMX_OK) return rc;
    smx_weight *W = const_cast<smx_weight *>(w);   // the weight is read-only; its scratch is not
    std::lock_guard<std::mutex> lock(W->mu);
    return weight_matmul_dev(W, act_dev, out_dev, m, k, n, (hipStream_t)stream);
}

SMX_API int smx_weight_matmul_host(const smx_weight *w, const float *act, float *out, int m, int k, int n)
{
    if (!w || !act || !out) SMX_FAIL(SMX_EINVAL, "smx_weight_matmul_host: null argument");
    int rc = weight_check(w, m, k, n, "smx_weight_matmul_host");
    if (rc != SMX_OK) return rc;
    smx_weight *W = const_cast<smx_weight *>(w);
    std::lock_guard<std::mutex> lock(W->mu);
    const size_t in_bytes = (size_t)m * k * 4, out_bytes = (size_t)m * n * 4;
    void *a = nullptr, *o = nullptr;
    if ((rc = host_stage(W, in_bytes, out_bytes, &a, &o)) != SMX_OK) return rc;
    hipStream_t st = W->host_stream;
    SMX_HIP(hipMemcpyAsync(a, act, in_bytes, hipMemcpyHostToDevice, st));
    rc = weight_matmul_dev(W, (const float *)a, (float *)o, m, k, n, st);
    if (rc == SMX_OK) {
        const hipError_t e = hipMemcpyAsync(out, o, out_bytes, hipMemcpyDeviceToHost, st);
        if (e != hipSuccess) {
            set_error(hipGetErrorString(e));
            rc = SMX_EDEVICE;
        }
    }
    const int r1 = scratch_release(W->act, st), r2 = scratch_release(W->out, st);
    SMX_HIP(hipStreamSynchronize(st));
    return rc != SMX_OK ? rc : r1 != SMX_OK ? r1 : r2;
}

SMX_API int smx_weight_to_float32_host(const smx_weight *w, float *out)
{
    if (!w || !out) SMX_FAIL(SMX_EINVAL, "smx_weight_to_float32_host: null argument");
    smx_weight *W = const_cast<smx_weight *>(w);
    std::lock_guard<std::mutex> lock(W->mu);
    const size_t out_bytes = (size_t)w->mat.rows * w->mat.cols * 4;
    void *o = nullptr;
    int rc = host_stage(W, 0, out_bytes, nullptr, &o);
    if (rc != SMX_OK) return rc;
    hipStream_t st = W->host_stream;
    hipError_t e = launch_dequant_smx(w->mat.view(), 0, w->mat.rows, (float *)o, st);
    if (e == hipSuccess) e = hipMemcpyAsync(out, o, out_bytes, hipMemcpyDeviceToHost, st);
    rc = scratch_release(W->out, st);
    const hipError_t f = hipStreamSynchronize(st);
    SMX_HIP(e);
    SMX_HIP(f);
    return rc;
}

}  // extern "C"

// Scratch of smx_weight_matmul_noalloc: the matrix-core GEMM's activation parts live in this
// file-scope device array instead of an allocation.  Each GPU holds its own copy for the life
// of the process.  Host code never passes the array's name to a kernel or a copy (in host code
// it names a host-side stand-in): it uses the per-device address from hipGetSymbolAddress.
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t *g_scratch_ptr[kMaxDevices] = {};
// smx_attention_decode's scores, per device, reused across calls (kept until the process ends)
std::mutex g_attn_mu;
Scratch g_attn_scratch[kMaxDevices];

// The device address of `scratch` on the current device, looked up once per device.
int noalloc_scratch(uint8_t **out)
{
    int dev = -1;
    SMX_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) SMX_FAIL(SMX_EUNSUPPORTED, "smx_weight_matmul_noalloc: device %d", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        SMX_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (!ptr) SMX_FAIL(SMX_EDEVICE, "smx_weight_matmul_noalloc: no device address for the scratch array");
        g_scratch_ptr[dev] = (uint8_t *)ptr;
    }
    *out = g_scratch_ptr[dev];
    return SMX_OK;
}
}  // namespace

extern "C" {

SMX_API int smx_weight_matmul_noalloc(const smx_weight *w, const float *act_dev, float *out_dev, int m, int k,
                                      int n, void *stream)
{
    if (!w || !act_dev || !out_dev) SMX_FAIL(SMX_EINVAL, "smx_weight_matmul_noalloc: null argument");
    int rc = weight_check(w, m, k, n, "smx_weight_matmul_noalloc");
    if (rc != SMX_OK) return rc;
    hipStream_t st = (hipStream_t)stream;
    if (m < kQgemmMinRows) {   // the GEMV path uses no scratch
        GemvArgs a{};
        a.w = w->mat.view();
        a.x = act_dev;
        a.x_stride = k;
        a.out = out_dev;
        a.out_stride = n;
        a.pro = PRO_NONE;
        a.epi = EPI_STORE;
        SMX_HIP(launch_gemv(a, m, st));
        return SMX_OK;
    }
    const size_t need = qgemm_xp_bytes(m, k);
    if (need > kNoAllocScratchBytes)
        SMX_FAIL(SMX_EINVAL, "smx_weight_matmul_noalloc: m=%d, k=%d needs %zu bytes of scratch; the limit is %zu "
                             "(ceil(m/16) * k/32 * 3072 bytes)", m, k, need, kNoAllocScratchBytes);
    uint8_t *xp = nullptr;
    if ((rc = noalloc_scratch(&xp)) != SMX_OK) return rc;
    // k_qprep writes every byte of the parts it uses (padding rows as zeros): nothing to clear
    QgemmArgs q{};
    q.w = w->mat.view();
    q.xp = xp;
    q.M = m;
    q.y = out_dev;
    q.y_stride = n;
    q.epi = EPI_STORE;
    SMX_HIP(launch_qgemm(q, act_dev, k, PRO_NONE, nullptr, nullptr, 0.0f, st));
    return SMX_OK;
}

SMX_API int smx_weight_to_float32(const smx_weight *w, float *out_dev, void *stream)
{
    if (!w || !out_dev) SMX_FAIL(SMX_EINVAL, "smx_weight_to_float32: null argument");
    SMX_HIP(launch_dequant_smx(w->mat.view(), 0, w->mat.rows, out_dev, (hipStream_t)stream));
    return SMX_OK;
}

SMX_API int smx_weight_destroy(smx_weight *w)
{
    if (!w) return SMX_OK;
    (void)hipSetDevice(w->device);
    scratch_free(w->xp);
    scratch_free(w->act);
    scratch_free(w->out);
    if (w->host_stream) (void)hipStreamDestroy(w->host_stream);
    w->mat.release();
    delete w;
    return SMX_OK;
}

// ---- elementwise / attention operators -------------------------------------------------------
SMX_API int smx_rmsnorm(const float *x, const float *g, float *y, int rows, int n, float eps, void *stream)
{
    if (!x || !g || !y || rows <= 0 || n <= 0) SMX_FAIL(SMX_EINVAL, "smx_rmsnorm: bad arguments");
    SMX_HIP(launch_rmsnorm(x, g, y, rows, n, eps, (hipStream_t)stream));
    return SMX_OK;
}

SMX_API int smx_layernorm(const float *x, const float *g, const float *b, float *y, int rows, int n,
                          float eps, void *stream)
{
    if (!x || !g || !b || !y || rows <= 0 || n <= 0) SMX_FAIL(SMX_EINVAL, "smx_layernorm: bad arguments");
    SMX_HIP(launch_layernorm(x, g, b, y, rows, n, eps, (hipStream_t)stream));
    return SMX_OK;
}

SMX_API int smx_rope_tables(int max_pos, int head_dim, float theta, float *cos_host, float *sin_host)
{
    if (max_pos <= 0 || head_dim <= 0 || head_dim % 2 || !cos_host || !sin_host)
        SMX_FAIL(SMX_EINVAL, "smx_rope_tables: head_dim must be even and positive");
    const int half = head_dim / 2;
    for (int pos = 0; pos < max_pos; pos++)
        for (int i = 0; i < half; i++) {
            const float expo = (2.0f * (float)i) / (float)head_dim;
            const float freq = 1.0f / powf(theta, expo);   // RotaryEmbedding.cs:52
            const float angle = (float)pos * freq;
            sin_host[pos * half + i] = sinf(angle);
            cos_host[pos * half + i] = cosf(angle);
        }
    return SMX_OK;
}

SMX_API int smx_rope(float *data, int n_heads, int seq, int head_dim, int pos0, const float *c,
                     const float *sn, void *stream)
{
    if (!data || !c || !sn || n_heads <= 0 || seq <= 0 || head_dim <= 0 || head_dim % 2 || pos0 < 0)
        SMX_FAIL(SMX_EINVAL, "smx_rope: bad arguments");
    SMX_HIP(launch_rope(data, n_heads, seq, head_dim, pos0, c, sn, (hipStream_t)stream));
    return SMX_OK;
}

SMX_API int smx_scale_mask_softmax(float *scores, float scale, int seq, int k_seq, int cache_offset,
                                   void *stream)
{
    if (!scores || seq <= 0 || k_seq <= 0 || cache_offset < 0 || cache_offset + seq > k_seq)
        SMX_FAIL(SMX_EINVAL, "smx_scale_mask_softmax: need 0 <= cache_offset and cache_offset+seq <= k_seq");
    SMX_HIP(launch_softmax(scores, scale, seq, k_seq, cache_offset, (hipStream_t)stream));
    return SMX_OK;
}

SMX_API int smx_attention_decode(const float *q, const float *kc, const float *vc, float *out,
                                 int n_head, int n_kv_head, int head_dim, int ctx_stride, int n_pos,
                                 void *stream)
{
    if (!q || !kc || !vc || !out) SMX_FAIL(SMX_EINVAL, "smx_attention_decode: null pointer");
    if (n_head <= 0 || n_kv_head <= 0 || n_head % n_kv_head)
        SMX_FAIL(SMX_EINVAL, "smx_attention_decode: n_head must be a multiple of n_kv_head");
    if (head_dim != 16 && head_dim != 32 && head_dim != 64 && head_dim != 128)
        SMX_FAIL(SMX_EUNSUPPORTED, "smx_attention_decode: head_dim must be 16, 32, 64 or 128");
    if (n_pos <= 0 || n_pos > ctx_stride || ctx_stride > 40000)
        SMX_FAIL(SMX_EINVAL, "smx_attention_decode: need 1 <= n_pos <= ctx_stride <= 40000");
    hipStream_t st = (hipStream_t)stream;
    const size_t need = attention_scores_floats(n_head, n_pos) * 4;
    if (capturing(st)) {   // a stream-ordered allocation recorded in the caller's graph
        float *scores = nullptr;
        SMX_HIP(hipMallocAsync((void **)&scores, need, st));
        const hipError_t e = launch_attention_split(q, kc, vc, out, scores, n_head, n_kv_head, head_dim,
                                                    ctx_stride, nullptr, n_pos, n_pos, st);
        const hipError_t f = hipFreeAsync(scores, st);
        SMX_HIP(e);
        SMX_HIP(f);
        return SMX_OK;
    }
    // the scores scratch of this device, reused call after call
    int dev = -1;
    SMX_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) SMX_FAIL(SMX_EUNSUPPORTED, "smx_attention_decode: device %d", dev);
    std::lock_guard<std::mutex> lock(g_attn_mu);
    void *scores = nullptr;
    int rc = scratch_acquire(g_attn_scratch[dev], need, st, &scores);
    if (rc != SMX_OK) return rc;
    const hipError_t e = launch_attention_split(q, kc, vc, out, (float *)scores, n_head, n_kv_head, head_dim,
                                                ctx_stride, nullptr, n_pos, n_pos, st);
    rc = scratch_release(g_attn_scratch[dev], st);
    SMX_HIP(e);
    return rc;
}

SMX_API int smx_attention_prefill(const float *q, const float *kc, const float *vc, float *out,
                                  int n_head, int n_kv_head, int head_dim, int ctx_stride, int p_first,
                                  int n_tok, void *stream)
{
    if (!q || !kc || !vc || !out) SMX_FAIL(SMX_EINVAL, "smx_attention_prefill: null pointer");
    if (n_head <= 0 || n_kv_head <= 0 || n_head % n_kv_head)
        SMX_FAIL(SMX_EINVAL, "smx_attention_prefill: n_head must be a multiple of n_kv_head");
    if (!attention_prefill_supported(n_head, n_kv_head, head_dim))
        SMX_FAIL(SMX_EUNSUPPORTED, "smx_attention_prefill: needs head_dim 64 and n_head / n_kv_head dividing 32");
    if (n_tok <= 0 || p_first < 0 || (int64_t)p_first + n_tok > ctx_stride || ctx_stride > 1000000)
        SMX_FAIL(SMX_EINVAL, "smx_attention_prefill: need 0 <= p_first, p_first + n_tok <= ctx_stride <= 1000000");
    const int row = n_head * head_dim;
    SMX_HIP(launch_attention_prefill(q, row, kc, vc, out, row, n_head, n_kv_head, head_dim, ctx_stride, p_first,
                                     n_tok, (hipStream_t)stream));
    return SMX_OK;
}

SMX_API int smx_silu_mul(const float *g, const float *u, float *y, int64_t n, void *stream)
{
    if (!g || !u || !y || n < 0) SMX_FAIL(SMX_EINVAL, "smx_silu_mul: bad arguments");
    SMX_HIP(launch_silu_mul(g, u, y, n, (hipStream_t)stream));
    return SMX_OK;
}

SMX_API int smx_gelu(const float *x, float *y, int64_t n, void *stream)
{
    if (!x || !y || n < 0) SMX_FAIL(SMX_EINVAL, "smx_gelu: bad arguments");
    SMX_HIP(launch_gelu(x, y, n, (hipStream_t)stream));
    return SMX_OK;
}

SMX_API int smx_argmax(const float *x, int n, int32_t *out, void *stream)
{
    if (!x || !out || n <= 0) SMX_FAIL(SMX_EINVAL, "smx_argmax: bad arguments");
    SMX_HIP(launch_argmax(x, n, out, nullptr, nullptr, (hipStream_t)stream));
    return SMX_OK;
}

SMX_API int smx_stream_read(const void *src, uint64_t bytes, void *stream)
{
    if (!src || bytes == 0 || bytes % 16 || bytes >= (1ull << 32))
        SMX_FAIL(SMX_EINVAL, "smx_stream_read: need a device pointer and 0 < bytes < 4 GiB, a multiple of 16");
    SMX_HIP(launch_stream_read(src, bytes, (hipStream_t)stream));
    return SMX_OK;
}

SMX_API int smx_sample(const float *logits, int n, const int32_t *context, int n_context, const smx_sampling *p,
                       double u, float *probs, int32_t *token, void *stream)
{
    if (!logits || !probs || !token || !p || n <= 0 || n_context < 0 || (n_context > 0 && !context))
        SMX_FAIL(SMX_EINVAL, "smx_sample: bad arguments");
    if (!(p->temperature > 0.0f) || p->top_k < 0 || p->repetition_window < 0 || !(u >= 0.0 && u < 1.0))
        SMX_FAIL(SMX_EINVAL, "smx_sample: need temperature > 0, top_k >= 0, repetition_window >= 0, 0 <= u < 1");
    SMX_HIP(launch_sample(logits, n, context, n_context, *p, u, probs, token, (hipStream_t)stream));
    return SMX_OK;
}

// ---- context / model ----------------------------------------------------------------------------
SMX_API int smx_context_create(int device, smx_context **out)
{
    if (!out) SMX_FAIL(SMX_EINVAL, "smx_context_create: null out");
    *out = nullptr;
    int count = 0;
    SMX_HIP(hipGetDeviceCount(&count));
    if (device < 0 || device >= count) SMX_FAIL(SMX_EINVAL, "smx_context_create: device %d of %d", device, count);
    SMX_HIP(hipSetDevice(device));
    smx_context *c = new smx_context();
    c->device = device;
    hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete c;
        SMX_HIP(e);
    }
    *out = c;
    return SMX_OK;
}

SMX_API int smx_context_destroy(smx_context *c)
{
    if (!c) return SMX_OK;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
    return SMX_OK;
}

SMX_API int smx_model_create(smx_context *ctx, const smx_model_config *cfg, smx_model **out)
{
    if (!ctx || !cfg || !out) SMX_FAIL(SMX_EINVAL, "smx_model_create: null argument");
    *out = nullptr;
    const smx_model_config &c = *cfg;
    if (c.arch != SMX_ARCH_LLAMA && c.arch != SMX_ARCH_GPT2)
        SMX_FAIL(SMX_EUNSUPPORTED, "smx_model_create: arch %d", c.arch);
    if (c.vocab <= 0 || c.ctx <= 0 || c.d_model <= 0 || c.n_layer <= 0 || c.n_head <= 0 || c.n_kv_head <= 0)
        SMX_FAIL(SMX_EINVAL, "smx_model_create: non-positive dimension");
    if (c.d_model % c.n_head) SMX_FAIL(SMX_EINVAL, "smx_model_create: d_model %% n_head != 0");
    if (c.n_head % c.n_kv_head) SMX_FAIL(SMX_EINVAL, "smx_model_create: n_head %% n_kv_head != 0");
    const int hd = c.d_model / c.n_head;
    if (hd != 16 && hd != 32 && hd != 64 && hd != 128)
        SMX_FAIL(SMX_EUNSUPPORTED, "smx_model_create: head_dim %d (supported: 16, 32, 64, 128)", hd);
    if (c.arch == SMX_ARCH_LLAMA && c.d_ff <= 0) SMX_FAIL(SMX_EINVAL, "smx_model_create: d_ff");
    // the weight uploads take rows of at most 16384 elements (d_model and the MLP width); the
    // other limits keep every derived size (QKV width, MLP width, cache and logits bytes) far
    // inside its type whatever a file's metadata says
    const int64_t mlp = c.arch == SMX_ARCH_LLAMA ? c.d_ff : 4 * (int64_t)c.d_model;
    if (c.d_model > 16384 || mlp > 16384 || c.vocab > (1 << 24) || c.ctx > (1 << 24) || c.n_layer > 4096)
        SMX_FAIL(SMX_EUNSUPPORTED, "smx_model_create: d_model %d, MLP width %lld, vocab %d, ctx %d, %d layers exceed "
                 "d_model, MLP width <= 16384, vocab, ctx <= 2^24, layers <= 4096", c.d_model, (long long)mlp, c.vocab,
                 c.ctx, c.n_layer);
    for (int i = 0; i < 6; i++) if (c.reserved[i]) SMX_FAIL(SMX_EINVAL, "smx_model_create: reserved fields must be 0");
    smx_model *m = new smx_model();
    m->ctx = ctx;
    m->cfg = c;
    m->hd = hd;
    m->kvdim = c.n_kv_head * hd;
    m->nqkv = c.d_model + 2 * m->kvdim;
    m->llama = c.arch == SMX_ARCH_LLAMA;
    m->hidden = m->llama ? c.d_ff : 4 * c.d_model;   // MLP.cs:25-26
    m->layers.resize(c.n_layer);
    *out = m;
    return SMX_OK;
}

static int model_upload_vec(smx_model *m, std::vector<float> &dst, int64_t n, int64_t off,
                            int64_t step, int64_t total, int type, const int64_t *dims, int ndims,
                            const void *bytes, size_t nbytes, int on_device)
{
    if (type != SMX_TYPE_F32) SMX_FAIL(SMX_EUNSUPPORTED, "1-D tensors must be F32 (got type %d)", type);
    if (ndims != 1 || dims[0] != n) SMX_FAIL(SMX_EINVAL, "1-D tensor has %lld elements, expected %lld",
                                             (long long)(ndims >= 1 ? dims[0] : -1), (long long)n);
    if (nbytes != (size_t)n * 4) SMX_FAIL(SMX_EINVAL, "1-D tensor byte size %zu != %lld", nbytes, (long long)n * 4);
    std::vector<float> tmp((size_t)n);
    if (on_device) {
        SMX_HIP(hipMemcpy(tmp.data(), bytes, nbytes, hipMemcpyDeviceToHost));
    } else {
        memcpy(tmp.data(), bytes, nbytes);
    }
    if (dst.empty()) dst.assign((size_t)total, 0.0f);
    for (int64_t i = 0; i < n; i++) dst[(size_t)(off + i * step)] = tmp[(size_t)i];
    (void)m;
    return SMX_OK;
}

SMX_API int smx_model_upload_tensor(smx_model *m, const char *name, int type, const int64_t *dims,
                                    int ndims, const void *bytes, size_t nbytes, int bytes_on_device)
{
    if (!m || !name || !dims || !bytes) SMX_FAIL(SMX_EINVAL, "smx_model_upload_tensor: null argument");
    if (m->finalized) SMX_FAIL(SMX_ESTATE, "smx_model_upload_tensor: model already finalized");
    std::lock_guard<std::mutex> lock(m->ctx->mu);
    SMX_HIP(hipSetDevice(m->ctx->device));
    const smx_model_config &c = m->cfg;
    const int64_t d = c.d_model, kv = m->kvdim, hid = m->hidden;
    std::string rest;
    const int li = parse_layer(name, rest);
    if (li >= c.n_layer) SMX_FAIL(SMX_EINVAL, "%s: layer index out of range", name);

    // 1-D tensors (norm weights and biases).
    if (ndims == 1) {
        if (li < 0) {
            if (rest == "output_norm.weight") return model_upload_vec(m, m->out_g, d, 0, 1, d, type, dims, ndims, bytes, nbytes, bytes_on_device);
            if (rest == "output_norm.bias") return model_upload_vec(m, m->out_b, d, 0, 1, d, type, dims, ndims, bytes, nbytes, bytes_on_device);
            SMX_FAIL(SMX_EINVAL, "%s: unknown 1-D tensor", name);
        }
        Layer &L = m->layers[li];
        const int64_t nq = m->nqkv;
        if (rest == "attn_norm.weight") return model_upload_vec(m, L.attn_g, d, 0, 1, d, type, dims, ndims, bytes, nbytes, bytes_on_device);
        if (rest == "attn_norm.bias") return model_upload_vec(m, L.attn_b, d, 0, 1, d, type, dims, ndims, bytes, nbytes, bytes_on_device);
        if (rest == "ffn_norm.weight") return model_upload_vec(m, L.ffn_g, d, 0, 1, d, type, dims, ndims, bytes, nbytes, bytes_on_device);
        if (rest == "ffn_norm.bias") return model_upload_vec(m, L.ffn_b, d, 0, 1, d, type, dims, ndims, bytes, nbytes, bytes_on_device);
        if (rest == "attn_q.bias") { L.has_bqkv = true; return model_upload_vec(m, L.bqkv, d, 0, 1, nq, type, dims, ndims, bytes, nbytes, bytes_on_device); }
        if (rest == "attn_k.bias") { L.has_bqkv = true; return model_upload_vec(m, L.bqkv, kv, d, 1, nq, type, dims, ndims, bytes, nbytes, bytes_on_device); }
        if (rest == "attn_v.bias") { L.has_bqkv = true; return model_upload_vec(m, L.bqkv, kv, d + kv, 1, nq, type, dims, ndims, bytes, nbytes, bytes_on_device); }
        if (rest == "attn_qkv.bias") { L.has_bqkv = true; return model_upload_vec(m, L.bqkv, nq, 0, 1, nq, type, dims, ndims, bytes, nbytes, bytes_on_device); }
        if (rest == "attn_output.bias") return model_upload_vec(m, L.bo, d, 0, 1, d, type, dims, ndims, bytes, nbytes, bytes_on_device);
        if (rest == "ffn_down.bias") return model_upload_vec(m, L.bdown, d, 0, 1, d, type, dims, ndims, bytes, nbytes, bytes_on_device);
        if (m->llama) {
            if (rest == "ffn_gate.bias") { L.has_bgu = true; return model_upload_vec(m, L.bgu, hid, 0, 2, 2 * hid, type, dims, ndims, bytes, nbytes, bytes_on_device); }
            if (rest == "ffn_up.bias") { L.has_bgu = true; return model_upload_vec(m, L.bgu, hid, 1, 2, 2 * hid, type, dims, ndims, bytes, nbytes, bytes_on_device); }
        } else if (rest == "ffn_up.bias") {
            L.has_bgu = true;
            return model_upload_vec(m, L.bgu, hid, 0, 1, hid, type, dims, ndims, bytes, nbytes, bytes_on_device);
        }
        SMX_FAIL(SMX_EINVAL, "%s: unknown 1-D tensor", name);
    }

    // 2-D weights: dims = {cols (ne0), rows}.
    if (ndims != 2) SMX_FAIL(SMX_EINVAL, "%s: expected 1 or 2 dims, got %d", name, ndims);
    const int64_t cols = dims[0], rows = dims[1];
    const int fmt = fmt_from_type(type);
    if (fmt < 0) SMX_FAIL(SMX_EUNSUPPORTED, "%s: weight type %d is not a supported block format", name, type);
    if (cols <= 0 || rows <= 0 || cols % fmt_block_elems(fmt))
        SMX_FAIL(SMX_EINVAL, "%s: ne0=%lld is not a multiple of the block size %d", name, (long long)cols, fmt_block_elems(fmt));
    const int64_t blocks = cols / fmt_block_elems(fmt), bb = fmt_gguf_bytes(fmt);
    if (rows > INT64_MAX / blocks / bb)
        SMX_FAIL(SMX_EINVAL, "%s: shape [%lld x %lld] is too large", name, (long long)rows, (long long)cols);
    const size_t expect = (size_t)(rows * blocks * bb);
    if (nbytes != expect) SMX_FAIL(SMX_EINVAL, "%s: %zu bytes, expected %zu", name, nbytes, expect);
    hipStream_t s = m->ctx->stream;

    struct Target { Mat *mat; int64_t rows_total, cols, rows, off, step; uint64_t bit; };
    Target t{nullptr, 0, 0, 0, 0, 1, 1};
    if (li < 0) {
        if (rest == "token_embd.weight") t = {&m->tok, c.vocab, d, c.vocab, 0, 1, 1};
        else if (rest == "position_embd.weight") t = {&m->pos, c.ctx, d, c.ctx, 0, 1, 1};
        else if (rest == "output.weight") t = {&m->head, c.vocab, d, c.vocab, 0, 1, 1};
        else SMX_FAIL(SMX_EINVAL, "%s: unknown tensor", name);
    } else {
        Layer &L = m->layers[li];
        if (rest == "attn_q.weight") t = {&L.qkv, m->nqkv, d, d, 0, 1, 1};
        else if (rest == "attn_k.weight") t = {&L.qkv, m->nqkv, d, kv, d, 1, 2};
        else if (rest == "attn_v.weight") t = {&L.qkv, m->nqkv, d, kv, d + kv, 1, 4};
        else if (rest == "attn_qkv.weight") t = {&L.qkv, m->nqkv, d, m->nqkv, 0, 1, 7};
        else if (rest == "attn_output.weight") t = {&L.o, d, d, d, 0, 1, 1};
        else if (rest == "ffn_down.weight") t = {&L.down, d, hid, d, 0, 1, 1};
        else if (m->llama && rest == "ffn_gate.weight") t = {&L.gu, 2 * hid, d, hid, 0, 2, 1};
        else if (m->llama && rest == "ffn_up.weight") t = {&L.gu, 2 * hid, d, hid, 1, 2, 2};
        else if (!m->llama && rest == "ffn_up.weight") t = {&L.gu, hid, d, hid, 0, 1, 3};
        else SMX_FAIL(SMX_EINVAL, "%s: unknown tensor", name);
    }
    if (cols != t.cols || rows != t.rows)
        SMX_FAIL(SMX_EINVAL, "%s: shape [%lld x %lld], expected [%lld x %lld]", name, (long long)rows,
                 (long long)cols, (long long)t.rows, (long long)t.cols);
    // F16 / F32 matrices load like the block formats (GgufModelLoader.cs:438-462 loads any 2-D
    // tensor so): the GEMV and the matrix-core GEMM take them unquantized
    if (cols > 16384) SMX_FAIL(SMX_EUNSUPPORTED, "%s: ne0=%lld exceeds 16384", name, (long long)cols);
    int rc = mat_alloc(*t.mat, fmt, t.rows_total, t.cols);
    if (rc != SMX_OK) return rc;
    rc = mat_upload(*t.mat, bytes, rows, cols, bytes_on_device, t.off, t.step, s);
    if (rc != SMX_OK) return rc;
    t.mat->rows_loaded |= t.bit;
    return SMX_OK;
}

// Which weight matrices stay resident in the 256 MB memory-side cache (MALL).  A decode step
// reads every matrix once, hundreds of megabytes per token, so a matrix read with plain loads
// is evicted before its next use unless the rest streams past the cache: the GEMV reads the
// kept matrices with plain loads and all others with the non-temporal hint.  Kept are the
// layer matrices of at most 4 MiB, smallest first, up to 128 MiB in total (their launches are
// latency-bound: a 2-3 MB matrix is 0.3 us of HBM time in a ~3.5 us launch, and served from
// the MALL it finishes sooner), and the head up to 64 MiB (its three loads per 208-byte Q6_K
// super-block run ~25 % slower with the non-temporal hint).  The large matrices (gate/up,
// down) gain least from residency and would crowd out the rest, so they stream.
// Measured on the configs[2] decode step, one box: all plain loads 1580 tok/s, all
// non-temporal 1649, this plan 1684.
constexpr int64_t kMallMaxMat = 4ll << 20, kMallLayerBudget = 128ll << 20, kMallHeadMax = 64ll << 20;
// A session keeps the plan only when the kept matrices and its whole KV cache fit in the MALL
// with room to spare; otherwise nothing stays resident from one token to the next and every
// matrix is read with plain loads (configs[3]: 4K-token context, 190 MB of KV cache: plain
// loads 1261 tok/s against 1230 with the plan).
constexpr int64_t kMallUsable = 224ll << 20;

static void plan_mall_residency(smx_model *m)
{
    std::vector<Mat *> cand;
    for (Layer &L : m->layers)
        for (Mat *w : {&L.qkv, &L.o, &L.gu, &L.down})
            if (w->bytes() <= kMallMaxMat) cand.push_back(w);
    std::stable_sort(cand.begin(), cand.end(), [](const Mat *a, const Mat *b) { return a->bytes() < b->bytes(); });
    int64_t left = kMallLayerBudget;
    m->mall_kept = 0;
    for (Mat *w : cand) {
        if (w->bytes() > left) break;
        w->cache = 1;
        left -= w->bytes();
        m->mall_kept += w->bytes();
    }
    if (m->head.bytes() <= kMallHeadMax) {
        m->head.cache = 1;
        m->mall_kept += m->head.bytes();
    }
}

SMX_API int smx_model_finalize(smx_model *m)
{
    if (!m) SMX_FAIL(SMX_EINVAL, "smx_model_finalize: null model");
    std::lock_guard<std::mutex> lock(m->ctx->mu);
    if (m->finalized) return SMX_OK;
    SMX_HIP(hipSetDevice(m->ctx->device));
    const smx_model_config &c = m->cfg;
    hipStream_t s = m->ctx->stream;
    if (m->tok.fmt < 0) SMX_FAIL(SMX_ESTATE, "finalize: token_embd.weight missing");
    if (m->out_g.empty()) SMX_FAIL(SMX_ESTATE, "finalize: output_norm.weight missing");
    if (!m->llama && (m->pos.fmt < 0 || m->out_b.empty()))
        SMX_FAIL(SMX_ESTATE, "finalize: gpt2 needs position_embd.weight and output_norm.bias");
    if (m->head.fmt < 0) {   // GgufModelLoader.HandleWeightTying (GgufModelLoader.cs:1126-1147)
        m->head = m->tok;
        m->head_tied = true;
    }
    for (int l = 0; l < c.n_layer; l++) {
        Layer &L = m->layers[l];
        if (L.qkv.rows_loaded != 7) SMX_FAIL(SMX_ESTATE, "finalize: layer %d Q/K/V incomplete", l);
        if (L.o.fmt < 0 || L.down.fmt < 0) SMX_FAIL(SMX_ESTATE, "finalize: layer %d attn_output/ffn_down missing", l);
        if (L.gu.rows_loaded != 3) SMX_FAIL(SMX_ESTATE, "finalize: layer %d ffn gate/up incomplete", l);
        if (L.attn_g.empty() || L.ffn_g.empty()) SMX_FAIL(SMX_ESTATE, "finalize: layer %d norm weights missing", l);
        if (!m->llama && (L.attn_b.empty() || L.ffn_b.empty()))
            SMX_FAIL(SMX_ESTATE, "finalize: layer %d LayerNorm biases missing", l);
        m->dense_layers = m->dense_layers || fmt_dense(L.qkv.fmt) || fmt_dense(L.o.fmt) || fmt_dense(L.gu.fmt) ||
                          fmt_dense(L.down.fmt);
        int rc;
        if ((rc = upload_floats(&L.d_attn_g, L.attn_g, s)) || (rc = upload_floats(&L.d_attn_b, L.attn_b, s)) ||
            (rc = upload_floats(&L.d_ffn_g, L.ffn_g, s)) || (rc = upload_floats(&L.d_ffn_b, L.ffn_b, s)) ||
            (rc = upload_floats(&L.d_bqkv, L.bqkv, s)) || (rc = upload_floats(&L.d_bo, L.bo, s)) ||
            (rc = upload_floats(&L.d_bgu, L.bgu, s)) || (rc = upload_floats(&L.d_bdown, L.bdown, s)))
            return rc;
    }
    int rc;
    if ((rc = upload_floats(&m->d_out_g, m->out_g, s)) || (rc = upload_floats(&m->d_out_b, m->out_b, s)))
        return rc;
    if (m->llama) {
        const size_t half = (size_t)m->hd / 2;
        std::vector<float> cs((size_t)c.ctx * half), sn((size_t)c.ctx * half);
        smx_rope_tables(c.ctx, m->hd, c.rope_theta, cs.data(), sn.data());
        if ((rc = upload_floats(&m->rope_cos, cs, s)) || (rc = upload_floats(&m->rope_sin, sn, s))) return rc;
    }
    SMX_HIP(hipStreamSynchronize(s));
    plan_mall_residency(m);
    m->finalized = true;
    return SMX_OK;
}

SMX_API int smx_model_weight_bytes(const smx_model *m, int64_t *bytes)
{
    if (!m || !bytes) SMX_FAIL(SMX_EINVAL, "smx_model_weight_bytes: null argument");
    int64_t b = m->tok.bytes() + m->pos.bytes() + (m->head_tied ? 0 : m->head.bytes());
    for (const Layer &L : m->layers) b += L.qkv.bytes() + L.o.bytes() + L.gu.bytes() + L.down.bytes();
    *bytes = b;
    return SMX_OK;
}

SMX_API int smx_model_destroy(smx_model *m)
{
    if (!m) return SMX_OK;
    if (m->sessions.load() != 0) SMX_FAIL(SMX_ESTATE, "smx_model_destroy: sessions or batchers still open");
    (void)hipSetDevice(m->ctx->device);
    if (!m->head_tied) m->head.release();
    m->tok.release();
    m->pos.release();
    for (Layer &L : m->layers) {
        L.qkv.release(); L.o.release(); L.gu.release(); L.down.release();
        free_dev(L.d_attn_g); free_dev(L.d_attn_b); free_dev(L.d_ffn_g); free_dev(L.d_ffn_b);
        free_dev(L.d_bqkv); free_dev(L.d_bo); free_dev(L.d_bgu); free_dev(L.d_bdown);
    }
    free_dev(m->d_out_g); free_dev(m->d_out_b); free_dev(m->rope_cos); free_dev(m->rope_sin);
    delete m;
    return SMX_OK;
}

// ---- session ------------------------------------------------------------------------------------
SMX_API int smx_session_destroy(smx_session *S);

SMX_API int smx_session_create(smx_model *m, int max_ctx, smx_session **out)
{
    if (!m || !out) SMX_FAIL(SMX_EINVAL, "smx_session_create: null argument");
    *out = nullptr;
    if (!m->finalized) SMX_FAIL(SMX_ESTATE, "smx_session_create: model not finalized");
    if (max_ctx <= 0 || max_ctx > m->cfg.ctx)
        SMX_FAIL(SMX_EINVAL, "smx_session_create: max_ctx %d not in [1, %d]", max_ctx, m->cfg.ctx);
    SMX_HIP(hipSetDevice(m->ctx->device));
    smx_session *S = new smx_session();
    S->m = m;
    S->max_ctx = max_ctx;
    S->ctx_stride = (max_ctx + 3) & ~3;
    m->sessions.fetch_add(1);
    const smx_model_config &c = m->cfg;
    const size_t cache = (size_t)c.n_layer * c.n_kv_head * S->ctx_stride * m->hd * 4;
    S->mall_plan = m->mall_kept + 2 * (int64_t)cache <= kMallUsable;
    const size_t maxv = (size_t)(m->hidden > c.d_model ? m->hidden : c.d_model);
    hipError_t e = hipSuccess;
    auto A = [&](void **p, size_t n) { if (e == hipSuccess) e = hipMalloc(p, n); };
    A((void **)&S->kc, cache);
    A((void **)&S->vc, cache);
    A((void **)&S->x, (size_t)c.d_model * 4);
    A((void **)&S->q, (size_t)m->nqkv * 4);
    A((void **)&S->att, (size_t)2 * c.d_model * 4);   // two partial outputs at long contexts
    A((void **)&S->scores, attention_scores_floats(c.n_head, max_ctx) * 4);
    A((void **)&S->h, maxv * 4);
    A((void **)&S->logits, (size_t)c.vocab * 4);
    A((void **)&S->tokens, (size_t)(max_ctx + 1) * 4);
    A((void **)&S->pos, 4);
    A((void **)&S->amax, 4);
    // the head GEMV has at most one workgroup per two vocabulary rows
    A((void **)&S->head_val, (size_t)(c.vocab / 2 + 1) * 4);
    A((void **)&S->head_idx, (size_t)(c.vocab / 2 + 1) * 4);
    for (int i = 0; i < 3 && e == hipSuccess; i++) e = hipEventCreate(&S->ev[i]);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&S->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipMemsetAsync(S->tokens, 0, (size_t)(max_ctx + 1) * 4, S->stream);
    if (e == hipSuccess) e = hipMemsetAsync(S->pos, 0, 4, S->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(S->stream);
    if (e != hipSuccess) {
        smx_session_destroy(S);
        SMX_HIP(e);
    }
    int rc = capture_step(S, false, true, &S->g_prefill);
    if (rc == SMX_OK) rc = capture_step(S, true, true, &S->g_decode);
    if (rc == SMX_OK) rc = capture_step(S, true, false, &S->g_decode_next);
    if (rc == SMX_OK) rc = capture_step(S, true, false, &S->g_decode_block, kDecodeBlock);
    if (rc != SMX_OK) {
        std::string msg = smx::last_error();
        smx_session_destroy(S);
        SMX_FAIL(rc, "%s", msg.c_str());
    }
    *out = S;
    return SMX_OK;
}

static int check_tokens(const smx_session *S, const int32_t *t, int n)
{
    for (int i = 0; i < n; i++)
        if (t[i] < 0 || t[i] >= S->m->cfg.vocab)
            SMX_FAIL(SMX_ERANGE, "token %d at index %d outside [0, %d)", t[i], i, S->m->cfg.vocab);
    return SMX_OK;
}

SMX_API int smx_session_forward(smx_session *S, const int32_t *tokens, int n_tokens, int pos_offset,
                                float *logits_out)
{
    if (!S || !tokens || n_tokens <= 0 || pos_offset < 0) SMX_FAIL(SMX_EINVAL, "smx_session_forward: bad arguments");
    BusyGuard guard(S->busy);
    if (!guard.ok) SMX_FAIL(SMX_EBUSY, "smx_session_forward: session in use on another thread");
    if ((int64_t)pos_offset + n_tokens > S->max_ctx)
        SMX_FAIL(SMX_ERANGE, "sequence length %d + offset %d exceeds block size %d", n_tokens, pos_offset, S->max_ctx);
    int rc = check_tokens(S, tokens, n_tokens);
    if (rc != SMX_OK) return rc;
    SMX_HIP(hipSetDevice(S->m->ctx->device));
    hipStream_t s = S->stream;
    const int32_t p0 = pos_offset;
    SMX_HIP(hipMemcpyAsync(S->tokens + pos_offset, tokens, (size_t)n_tokens * 4, hipMemcpyHostToDevice, s));
    SMX_HIP(hipMemcpyAsync(S->pos, &p0, 4, hipMemcpyHostToDevice, s));
    if (n_tokens >= kPrefillMin) {
        if ((rc = prefill_tokens(S, tokens, n_tokens, pos_offset, true, s)) != SMX_OK) return rc;
    } else {
        for (int i = 0; i + 1 < n_tokens; i++) SMX_HIP(hipGraphLaunch(S->g_prefill, s));
        SMX_HIP(hipGraphLaunch(S->g_decode, s));
    }
    if (logits_out)
        SMX_HIP(hipMemcpyAsync(logits_out, S->logits, (size_t)S->m->cfg.vocab * 4, hipMemcpyDeviceToHost, s));
    SMX_HIP(hipStreamSynchronize(s));
    return SMX_OK;
}

// The prompt a generation prefills: its last max_ctx tokens (InferenceSession.cs:494-508).
static void crop_prompt(const smx_session *S, const int32_t *&prompt, int &n_prompt)
{
    if (n_prompt > S->max_ctx) {
        prompt += n_prompt - S->max_ctx;
        n_prompt = S->max_ctx;
    }
}

// After a generation of n_new requested tokens stopped (rc != SMX_OK) or finished: copies the
// `done` tokens produced to out_tokens, fills the rest with -1 and fills stats.
static int finish_generation(smx_session *S, int n_prompt, int n_new, int done, int32_t *out_tokens,
                             smx_gen_stats *stats, int rc)
{
    hipStream_t s = S->stream;
    if (done > 0)
        SMX_HIP(hipMemcpyAsync(out_tokens, S->tokens + n_prompt, (size_t)done * 4, hipMemcpyDeviceToHost, s));
    SMX_HIP(hipStreamSynchronize(s));
    for (int i = done; i < n_new; i++) out_tokens[i] = -1;
    if (stats) {
        float a = 0.0f, b = 0.0f;
        SMX_HIP(hipEventElapsedTime(&a, S->ev[0], S->ev[1]));
        SMX_HIP(hipEventElapsedTime(&b, S->ev[1], S->ev[2]));
        stats->prefill_ms = a;
        stats->decode_ms = b;
        stats->n_prefill_steps = n_prompt - 1;
        stats->n_decode_steps = done;
    }
    if (rc == SMX_ECANCELED) SMX_FAIL(rc, "generation cancelled after %d of %d tokens", done, n_new);
    if (rc == SMX_ETIMEDOUT)
        SMX_FAIL(rc, "generation stopped at the session's %d ms time limit after %d of %d tokens",
                 (int)S->max_time_ms.load(), done, n_new);
    return rc;
}

// Prefills all prompt tokens but the last (their logits are not needed) and leaves the device
// position at the last one.
static int prefill_prompt(smx_session *S, const int32_t *prompt, int n_prompt, hipStream_t s)
{
    int rc = SMX_OK;
    if (n_prompt - 1 >= kPrefillMin) {
        if ((rc = prefill_tokens(S, prompt, n_prompt - 1, 0, false, s)) != SMX_OK) return rc;
        const int32_t plast = n_prompt - 1;
        SMX_HIP(hipMemcpyAsync(S->pos, &plast, 4, hipMemcpyHostToDevice, s));
    } else {
        for (int i = 0; i + 1 < n_prompt; i++) SMX_HIP(hipGraphLaunch(S->g_prefill, s));
    }
    return SMX_OK;
}

SMX_API int smx_session_generate(smx_session *S, const int32_t *prompt, int n_prompt, int n_new,
                                 int32_t *out_tokens, float *logits_out, smx_gen_stats *stats)
{
    if (!S || !prompt || !out_tokens || n_prompt <= 0 || n_new <= 0)
        SMX_FAIL(SMX_EINVAL, "smx_session_generate: bad arguments");
    BusyGuard guard(S->busy);
    if (!guard.ok) SMX_FAIL(SMX_EBUSY, "smx_session_generate: session in use on another thread");
    crop_prompt(S, prompt, n_prompt);
    if ((int64_t)n_prompt + n_new - 1 > S->max_ctx)
        SMX_FAIL(SMX_ERANGE, "prompt %d + new tokens %d exceed the session context %d", n_prompt, n_new, S->max_ctx);
    int rc = check_tokens(S, prompt, n_prompt);
    if (rc != SMX_OK) return rc;
    StopCheck stop;
    stop.add(S, std::chrono::steady_clock::now());
    SMX_HIP(hipSetDevice(S->m->ctx->device));
    hipStream_t s = S->stream;
    const int V = S->m->cfg.vocab;
    const int32_t zero = 0;
    SMX_HIP(hipEventRecord(S->ev[0], s));
    int done = 0, halt = stop.poll();
    if (halt == SMX_OK) {
        SMX_HIP(hipMemcpyAsync(S->tokens, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice, s));
        SMX_HIP(hipMemcpyAsync(S->pos, &zero, 4, hipMemcpyHostToDevice, s));
        if ((rc = prefill_prompt(S, prompt, n_prompt, s)) != SMX_OK) return rc;
    }
    SMX_HIP(hipEventRecord(S->ev[1], s));
    Pacer pace(s, logits_out ? 1 : 2);
    while (halt == SMX_OK && done < n_new) {
        if ((halt = stop.poll()) != SMX_OK) break;
        if (done > 0 && !logits_out && n_new - done >= kDecodeBlock) {
            SMX_HIP(hipGraphLaunch(S->g_decode_block, s));
            done += kDecodeBlock;
        } else {
            SMX_HIP(hipGraphLaunch(done == 0 ? S->g_decode : S->g_decode_next, s));
            if (logits_out)
                SMX_HIP(hipMemcpyAsync(logits_out + (size_t)done * V, S->logits, (size_t)V * 4, hipMemcpyDeviceToHost, s));
            done++;
        }
        SMX_HIP(pace.launched());
    }
    SMX_HIP(hipEventRecord(S->ev[2], s));
    return finish_generation(S, n_prompt, n_new, done, out_tokens, stats, halt);
}

SMX_API int smx_session_cancel(smx_session *S)
{
    if (!S) SMX_FAIL(SMX_EINVAL, "smx_session_cancel: null session");
    S->cancel.store(1);
    return SMX_OK;
}

SMX_API int smx_session_set_max_time(smx_session *S, int32_t max_time_ms)
{
    if (!S || max_time_ms < 0) SMX_FAIL(SMX_EINVAL, "smx_session_set_max_time: bad arguments");
    S->max_time_ms.store(max_time_ms);
    return SMX_OK;
}

SMX_API int smx_session_generate_sampled(smx_session *S, const int32_t *prompt, int n_prompt, int n_new,
                                         const smx_sampling *params, uint64_t seed, int32_t *out_tokens,
                                         float *logits_out, smx_gen_stats *stats)
{
    if (!S || !prompt || !out_tokens || !params || n_prompt <= 0 || n_new <= 0)
        SMX_FAIL(SMX_EINVAL, "smx_session_generate_sampled: bad arguments");
    if (!(params->temperature > 0.0f) || params->top_k < 0 || params->repetition_window < 0)
        SMX_FAIL(SMX_EINVAL, "smx_session_generate_sampled: need temperature > 0, top_k >= 0, repetition_window >= 0");
    BusyGuard guard(S->busy);
    if (!guard.ok) SMX_FAIL(SMX_EBUSY, "smx_session_generate_sampled: session in use on another thread");
    crop_prompt(S, prompt, n_prompt);
    if ((int64_t)n_prompt + n_new - 1 > S->max_ctx)
        SMX_FAIL(SMX_ERANGE, "prompt %d + new tokens %d exceed the session context %d", n_prompt, n_new, S->max_ctx);
    int rc = check_tokens(S, prompt, n_prompt);
    if (rc != SMX_OK) return rc;
    StopCheck stop;
    stop.add(S, std::chrono::steady_clock::now());
    SMX_HIP(hipSetDevice(S->m->ctx->device));
    hipStream_t s = S->stream;
    const int V = S->m->cfg.vocab;
    if (!S->samp || !S->probs) {   // both or neither: the sampling graph reads both
        free_dev(S->samp);
        free_dev(S->probs);
        S->samp = nullptr;
        S->probs = nullptr;
        SampleState *samp = nullptr;
        float *probs = nullptr;
        hipError_t e = hipMalloc((void **)&samp, sizeof(SampleState));
        if (e == hipSuccess) e = hipMalloc((void **)&probs, (size_t)V * 4);
        if (e != hipSuccess) {
            free_dev(samp);
            SMX_HIP(e);
        }
        S->samp = samp;
        S->probs = probs;
    }
    if (!S->g_sample && (rc = capture_step(S, true, true, &S->g_sample, 1, true)) != SMX_OK) return rc;
    const SampleState st{*params, seed, 0};
    const int32_t zero = 0;
    SMX_HIP(hipEventRecord(S->ev[0], s));
    int done = 0, halt = stop.poll();
    if (halt == SMX_OK) {
        SMX_HIP(hipMemcpyAsync(S->samp, &st, sizeof(st), hipMemcpyHostToDevice, s));
        SMX_HIP(hipMemcpyAsync(S->tokens, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice, s));
        SMX_HIP(hipMemcpyAsync(S->pos, &zero, 4, hipMemcpyHostToDevice, s));
        if ((rc = prefill_prompt(S, prompt, n_prompt, s)) != SMX_OK) return rc;
    }
    SMX_HIP(hipEventRecord(S->ev[1], s));
    Pacer pace(s, 8);
    while (halt == SMX_OK && done < n_new) {
        if ((halt = stop.poll()) != SMX_OK) break;
        SMX_HIP(hipGraphLaunch(S->g_sample, s));
        if (logits_out)
            SMX_HIP(hipMemcpyAsync(logits_out + (size_t)done * V, S->logits, (size_t)V * 4, hipMemcpyDeviceToHost, s));
        done++;
        SMX_HIP(pace.launched());
    }
    SMX_HIP(hipEventRecord(S->ev[2], s));
    return finish_generation(S, n_prompt, n_new, done, out_tokens, stats, halt);
}

// Upper bound on sessions per lockstep batch (one token tile of the GEMM per 16 sessions).
constexpr int kMaxBatchSessions = 256;

SMX_API int smx_batch_generate(smx_session *const *sessions, int n_sessions, const int32_t *prompts,
                               const int32_t *prompt_lens, int n_new, int32_t *out_tokens,
                               smx_gen_stats *stats)
{
    if (!sessions || !prompts || !prompt_lens || !out_tokens || n_sessions <= 0 || n_new <= 0)
        SMX_FAIL(SMX_EINVAL, "smx_batch_generate: bad arguments");
    if (n_sessions > kMaxBatchSessions)
        SMX_FAIL(SMX_EINVAL, "smx_batch_generate: %d sessions exceed the limit %d", n_sessions, kMaxBatchSessions);
    smx_model *m = sessions[0] ? sessions[0]->m : nullptr;
    if (!m) SMX_FAIL(SMX_EINVAL, "smx_batch_generate: null session");
    const int max_ctx = sessions[0]->max_ctx;
    std::vector<int64_t> off((size_t)n_sessions + 1, 0);
    for (int i = 0; i < n_sessions; i++) {
        smx_session *S = sessions[i];
        if (!S) SMX_FAIL(SMX_EINVAL, "smx_batch_generate: null session %d", i);
        if (S->m != m) SMX_FAIL(SMX_EINVAL, "smx_batch_generate: session %d belongs to another model", i);
        if (S->max_ctx != max_ctx) SMX_FAIL(SMX_EINVAL, "smx_batch_generate: sessions differ in max_ctx");
        for (int j = 0; j < i; j++)
            if (sessions[j] == S) SMX_FAIL(SMX_EINVAL, "smx_batch_generate: session %d listed twice", i);
        const int n = prompt_lens[i];
        if (n <= 0) SMX_FAIL(SMX_EINVAL, "smx_batch_generate: empty prompt for session %d", i);
        if ((int64_t)n + n_new - 1 > max_ctx)
            SMX_FAIL(SMX_ERANGE, "prompt %d + new tokens %d exceed the session context %d", n, n_new, max_ctx);
        off[(size_t)i + 1] = off[(size_t)i] + n;
    }
    std::vector<std::unique_ptr<BusyGuard>> guards;
    StopCheck stop;
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < n_sessions; i++) {
        guards.emplace_back(new BusyGuard(sessions[i]->busy));
        if (!guards.back()->ok) SMX_FAIL(SMX_EBUSY, "smx_batch_generate: session %d in use on another thread", i);
        int rc = check_tokens(sessions[i], prompts + off[(size_t)i], prompt_lens[i]);
        if (rc != SMX_OK) return rc;
        stop.add(sessions[i], t0);
    }
    int halt = stop.poll();
    if (halt != SMX_OK) {
        for (int64_t i = 0; i < (int64_t)n_sessions * n_new; i++) out_tokens[i] = -1;
        if (stats) *stats = smx_gen_stats{0.0, 0.0, 0, 0};
        SMX_FAIL(halt, "smx_batch_generate: stopped before the prefill (%s)",
                 halt == SMX_ECANCELED ? "cancel request" : "time limit");
    }
    SMX_HIP(hipSetDevice(m->ctx->device));
    // every listed session is held by this call: the first one's stream carries the batch
    hipStream_t s = sessions[0]->stream;
    const int V = m->cfg.vocab, n = n_sessions;
    hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
    TokBatch D;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int rc = SMX_OK;
    auto cleanup = [&]() {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        batch_free(D);
        for (hipEvent_t e : ev) if (e) (void)hipEventDestroy(e);
    };
#define SMX_BHIP(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { cleanup(); SMX_HIP(e_); } } while (0)
    for (auto &e : ev) SMX_BHIP(hipEventCreate(&e));
    // prefill every session's prompt except its last token, all sessions together
    int64_t n_prefill = 0;
    for (int i = 0; i < n; i++) n_prefill += prompt_lens[i] - 1;
    TokBatch P;   // allocated outside the timed region
    if (n_prefill > 0 && (rc = batch_alloc(m, P, prefill_cap(n_prefill), 1)) != SMX_OK) {
        cleanup();
        return rc;
    }
    SMX_BHIP(hipEventRecord(ev[0], s));
    for (int i = 0; i < n; i++)
        SMX_BHIP(hipMemcpyAsync(sessions[i]->tokens, prompts + off[(size_t)i], (size_t)prompt_lens[i] * 4,
                                hipMemcpyHostToDevice, s));
    if (n_prefill > 0) {
        rc = prefill_sessions(m, P, sessions, n, prompts, off.data(), prompt_lens, s);
        batch_free(P);
        if (rc != SMX_OK) {
            cleanup();
            return rc;
        }
    }
    SMX_BHIP(hipEventRecord(ev[1], s));
    // one token per session per step
    if ((rc = batch_alloc(m, D, n, n)) != SMX_OK) {
        cleanup();
        return rc;
    }
    {
        std::vector<int32_t> ids((size_t)n), pos((size_t)n);
        std::vector<float *> kc((size_t)n), vc((size_t)n);
        std::vector<int32_t *> ta((size_t)n);
        for (int i = 0; i < n; i++) {
            ids[(size_t)i] = prompts[off[(size_t)i] + prompt_lens[i] - 1];
            pos[(size_t)i] = prompt_lens[i] - 1;
            kc[(size_t)i] = sessions[i]->kc;
            vc[(size_t)i] = sessions[i]->vc;
            ta[(size_t)i] = sessions[i]->tokens;
        }
        SMX_BHIP(hipMemcpyAsync(D.ids, ids.data(), (size_t)n * 4, hipMemcpyHostToDevice, s));
        SMX_BHIP(hipMemcpyAsync(D.pos, pos.data(), (size_t)n * 4, hipMemcpyHostToDevice, s));
        SMX_BHIP(hipMemcpyAsync(D.kc, kc.data(), (size_t)n * sizeof(float *), hipMemcpyHostToDevice, s));
        SMX_BHIP(hipMemcpyAsync(D.vc, vc.data(), (size_t)n * sizeof(float *), hipMemcpyHostToDevice, s));
        SMX_BHIP(hipMemcpyAsync(D.tok_arr, ta.data(), (size_t)n * sizeof(int32_t *), hipMemcpyHostToDevice, s));
        SMX_BHIP(hipStreamSynchronize(s));
    }
    // capture one lockstep step: all layers for the n tokens, head, argmax (appends each
    // session's token at pos + 1 and advances pos on the device)
    SMX_BHIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    rc = run_tokens(m, D, n, sessions[0]->ctx_stride, 0, s, nullptr);
    if (rc == SMX_OK) {
        const hipError_t e = launch_argmax_rows(D.logits, V, V, n, D.ids, D.pos, D.tok_arr, s);
        if (e != hipSuccess) { set_error(hipGetErrorString(e)); rc = SMX_EDEVICE; }
    }
    const hipError_t ce = hipStreamEndCapture(s, &graph);
    if (rc != SMX_OK) {
        cleanup();
        return rc;
    }
    SMX_BHIP(ce);
    SMX_BHIP(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    int done = 0;
    {
        Pacer pace(s, 2);
        while (done < n_new && (halt = stop.poll()) == SMX_OK) {
            SMX_BHIP(hipGraphLaunch(exec, s));
            done++;
            SMX_BHIP(pace.launched());
        }
    }
    SMX_BHIP(hipEventRecord(ev[2], s));
    for (int i = 0; i < n; i++) {
        if (done > 0)
            SMX_BHIP(hipMemcpyAsync(out_tokens + (size_t)i * n_new, sessions[i]->tokens + prompt_lens[i],
                                    (size_t)done * 4, hipMemcpyDeviceToHost, s));
        SMX_BHIP(hipMemcpyAsync(sessions[i]->pos, D.pos + i, 4, hipMemcpyDeviceToDevice, s));
    }
    SMX_BHIP(hipStreamSynchronize(s));
    for (int i = 0; i < n; i++)
        for (int k = done; k < n_new; k++) out_tokens[(size_t)i * n_new + k] = -1;
    if (stats) {
        float a = 0.0f, b = 0.0f;
        SMX_BHIP(hipEventElapsedTime(&a, ev[0], ev[1]));
        SMX_BHIP(hipEventElapsedTime(&b, ev[1], ev[2]));
        stats->prefill_ms = a;
        stats->decode_ms = b;
        stats->n_prefill_steps = (int32_t)n_prefill;
        stats->n_decode_steps = done;
    }
#undef SMX_BHIP
    cleanup();
    if (halt != SMX_OK)
        SMX_FAIL(halt, "smx_batch_generate: stopped after %d of %d steps (%s)", done, n_new,
                 halt == SMX_ECANCELED ? "cancel request" : "time limit");
    return SMX_OK;
}

// Continuous batching: sessions join (after their own prefill) and leave between steps; every
// step runs all current members through the layers as one token batch (one token each, each at
// its own position) and appends each member's greedy token.  One captured graph per member
// count, made on first use.
struct smx_batcher {
    smx_model *m = nullptr;
    hipStream_t stream = nullptr;   // member prefills, step captures and replays
    int cap = 0, max_ctx = 0;
    TokBatch D;
    std::vector<smx_session *> slot;
    std::vector<int32_t> id, pos;   // per member: token to process next and its position
    std::vector<SampleState> samp;  // per member: sampling options, seed and draws taken
    std::vector<int32_t> on;        // per member: 1 = sampled, 0 = greedy
    std::vector<std::chrono::steady_clock::time_point> joined;   // per member: when it joined
    SampleState *d_samp = nullptr;  // device copies, max_members entries
    int32_t *d_on = nullptr;
    float *d_probs = nullptr;       // sampling scratch, max_members x vocab
    std::map<int, hipGraphExec_t> graphs;   // key: 2 * members + (any member sampled)
    bool dirty = true;              // member arrays on the device are stale
    std::atomic<int> busy{0};
};

SMX_API int smx_batcher_create(smx_model *m, int max_members, int max_ctx, smx_batcher **out)
{
    if (!m || !out || max_members <= 0 || max_ctx <= 0) SMX_FAIL(SMX_EINVAL, "smx_batcher_create: bad arguments");
    if (max_members > kMaxBatchSessions)
        SMX_FAIL(SMX_EINVAL, "smx_batcher_create: %d members exceed the limit %d", max_members, kMaxBatchSessions);
    *out = nullptr;
    SMX_HIP(hipSetDevice(m->ctx->device));
    auto *B = new smx_batcher();
    B->m = m;
    B->cap = max_members;
    B->max_ctx = max_ctx;
    int rc = batch_alloc(m, B->D, max_members, max_members);
    hipError_t e = hipSuccess;
    if (rc == SMX_OK) e = hipStreamCreateWithFlags(&B->stream, hipStreamNonBlocking);
    if (rc == SMX_OK && e == hipSuccess) e = hipMalloc((void **)&B->d_samp, (size_t)max_members * sizeof(SampleState));
    if (rc == SMX_OK && e == hipSuccess) e = hipMalloc((void **)&B->d_on, (size_t)max_members * 4);
    if (rc == SMX_OK && e == hipSuccess) e = hipMalloc((void **)&B->d_probs, (size_t)max_members * m->cfg.vocab * 4);
    if (rc != SMX_OK || e != hipSuccess) {
        batch_free(B->D);
        free_dev(B->d_samp); free_dev(B->d_on); free_dev(B->d_probs);
        if (B->stream) (void)hipStreamDestroy(B->stream);
        delete B;
        if (rc != SMX_OK) return rc;
        SMX_FAIL(SMX_ENOMEM, "smx_batcher_create: %s", hipGetErrorString(e));
    }
    m->sessions.fetch_add(1);   // the model outlives its batchers as it outlives its sessions
    *out = B;
    return SMX_OK;
}

static int batcher_add(smx_batcher *B, smx_session *S, const int32_t *prompt, int n_prompt,
                       const smx_sampling *params, uint64_t seed)
{
    if (!B || !S || !prompt || n_prompt <= 0) SMX_FAIL(SMX_EINVAL, "smx_batcher_add: bad arguments");
    if (params && (!(params->temperature > 0.0f) || params->top_k < 0 || params->repetition_window < 0))
        SMX_FAIL(SMX_EINVAL, "smx_batcher_add_sampled: need temperature > 0, top_k >= 0, repetition_window >= 0");
    BusyGuard guard(B->busy);
    if (!guard.ok) SMX_FAIL(SMX_EBUSY, "smx_batcher_add: batcher in use on another thread");
    if (S->m != B->m) SMX_FAIL(SMX_EINVAL, "smx_batcher_add: session belongs to another model");
    if (S->max_ctx != B->max_ctx) SMX_FAIL(SMX_EINVAL, "smx_batcher_add: session max_ctx %d, batcher %d", S->max_ctx, B->max_ctx);
    if ((int)B->slot.size() >= B->cap) SMX_FAIL(SMX_ERANGE, "smx_batcher_add: all %d member slots in use", B->cap);
    if (n_prompt > S->max_ctx) SMX_FAIL(SMX_ERANGE, "smx_batcher_add: prompt %d exceeds the context %d", n_prompt, S->max_ctx);
    int rc = check_tokens(S, prompt, n_prompt);
    if (rc != SMX_OK) return rc;
    // the session stays marked in use while it is a member
    int expected = 0;
    if (!S->busy.compare_exchange_strong(expected, 1))
        SMX_FAIL(SMX_EBUSY, "smx_batcher_add: session in use (on another thread or in a batcher)");
    auto release = [&]() { S->busy.store(0); };
    hipStream_t s = B->stream;
    hipError_t e = hipSetDevice(B->m->ctx->device);
    if (e == hipSuccess) e = hipMemcpyAsync(S->tokens, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) {
        release();
        SMX_HIP(e);
    }
    if (n_prompt > 1 && (rc = prefill_tokens(S, prompt, n_prompt - 1, 0, false, s)) != SMX_OK) {
        release();
        return rc;
    }
    B->slot.push_back(S);
    B->id.push_back(prompt[n_prompt - 1]);
    B->pos.push_back(n_prompt - 1);
    B->samp.push_back(params ? SampleState{*params, seed, 0} : SampleState{});
    B->on.push_back(params ? 1 : 0);
    B->joined.push_back(std::chrono::steady_clock::now());
    B->dirty = true;
    return SMX_OK;
}

SMX_API int smx_batcher_add(smx_batcher *B, smx_session *S, const int32_t *prompt, int n_prompt)
{
    return batcher_add(B, S, prompt, n_prompt, nullptr, 0);
}

SMX_API int smx_batcher_add_sampled(smx_batcher *B, smx_session *S, const int32_t *prompt, int n_prompt,
                                    const smx_sampling *params, uint64_t seed)
{
    if (!params) SMX_FAIL(SMX_EINVAL, "smx_batcher_add_sampled: null params");
    return batcher_add(B, S, prompt, n_prompt, params, seed);
}

// Leaves the session where smx_session_generate would: its position is that of its last token.
SMX_API int smx_batcher_remove(smx_batcher *B, smx_session *S)
{
    if (!B || !S) SMX_FAIL(SMX_EINVAL, "smx_batcher_remove: bad arguments");
    BusyGuard guard(B->busy);
    if (!guard.ok) SMX_FAIL(SMX_EBUSY, "smx_batcher_remove: batcher in use on another thread");
    size_t i = 0;
    while (i < B->slot.size() && B->slot[i] != S) i++;
    if (i == B->slot.size()) SMX_FAIL(SMX_EINVAL, "smx_batcher_remove: session is not a member");
    SMX_HIP(hipSetDevice(B->m->ctx->device));
    hipStream_t s = B->stream;
    const int32_t p = B->pos[i];
    SMX_HIP(hipMemcpyAsync(S->pos, &p, 4, hipMemcpyHostToDevice, s));
    SMX_HIP(hipStreamSynchronize(s));
    B->slot.erase(B->slot.begin() + (std::ptrdiff_t)i);
    B->id.erase(B->id.begin() + (std::ptrdiff_t)i);
    B->pos.erase(B->pos.begin() + (std::ptrdiff_t)i);
    B->samp.erase(B->samp.begin() + (std::ptrdiff_t)i);
    B->on.erase(B->on.begin() + (std::ptrdiff_t)i);
    B->joined.erase(B->joined.begin() + (std::ptrdiff_t)i);
    B->dirty = true;
    S->busy.store(0);
    return SMX_OK;
}

SMX_API int smx_batcher_count(const smx_batcher *B)
{
    if (!B) SMX_FAIL(SMX_EINVAL, "smx_batcher_count: null batcher");
    return (int)B->slot.size();
}

SMX_API int smx_batcher_step(smx_batcher *B, int n_steps, int32_t *out_tokens)
{
    if (!B || !out_tokens || n_steps <= 0) SMX_FAIL(SMX_EINVAL, "smx_batcher_step: bad arguments");
    BusyGuard guard(B->busy);
    if (!guard.ok) SMX_FAIL(SMX_EBUSY, "smx_batcher_step: batcher in use on another thread");
    const int n = (int)B->slot.size();
    if (n == 0) SMX_FAIL(SMX_EINVAL, "smx_batcher_step: no members");
    for (int i = 0; i < n; i++)
        if ((int64_t)B->pos[(size_t)i] + n_steps > B->max_ctx)
            SMX_FAIL(SMX_ERANGE, "smx_batcher_step: member %d at position %d + %d steps exceeds the context %d", i,
                     B->pos[(size_t)i], n_steps, B->max_ctx);
    smx_model *m = B->m;
    SMX_HIP(hipSetDevice(m->ctx->device));
    hipStream_t s = B->stream;
    TokBatch &D = B->D;
    if (B->dirty) {
        std::vector<float *> kc((size_t)n), vc((size_t)n);
        std::vector<int32_t *> ta((size_t)n);
        for (int i = 0; i < n; i++) {
            kc[(size_t)i] = B->slot[(size_t)i]->kc;
            vc[(size_t)i] = B->slot[(size_t)i]->vc;
            ta[(size_t)i] = B->slot[(size_t)i]->tokens;
        }
        SMX_HIP(hipMemcpyAsync(D.ids, B->id.data(), (size_t)n * 4, hipMemcpyHostToDevice, s));
        SMX_HIP(hipMemcpyAsync(D.pos, B->pos.data(), (size_t)n * 4, hipMemcpyHostToDevice, s));
        SMX_HIP(hipMemcpyAsync(D.kc, kc.data(), (size_t)n * sizeof(float *), hipMemcpyHostToDevice, s));
        SMX_HIP(hipMemcpyAsync(D.vc, vc.data(), (size_t)n * sizeof(float *), hipMemcpyHostToDevice, s));
        SMX_HIP(hipMemcpyAsync(D.tok_arr, ta.data(), (size_t)n * sizeof(int32_t *), hipMemcpyHostToDevice, s));
        SMX_HIP(hipMemcpyAsync(B->d_samp, B->samp.data(), (size_t)n * sizeof(SampleState), hipMemcpyHostToDevice, s));
        SMX_HIP(hipMemcpyAsync(B->d_on, B->on.data(), (size_t)n * 4, hipMemcpyHostToDevice, s));
        SMX_HIP(hipStreamSynchronize(s));
        B->dirty = false;
    }
    bool any = false;
    for (int v : B->on) any = any || v;
    hipGraphExec_t &exec = B->graphs[2 * n + (any ? 1 : 0)];
    if (!exec) {
        hipGraph_t graph = nullptr;
        SMX_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
        int rc = run_tokens(m, D, n, B->slot[0]->ctx_stride, 0, s, nullptr);
        if (rc == SMX_OK) {
            const int V = m->cfg.vocab;
            hipError_t e = launch_argmax_rows(D.logits, V, V, n, D.ids, D.pos, D.tok_arr, s);
            if (e == hipSuccess && any)
                e = launch_sample_rows(D.logits, V, V, n, D.tok_arr, D.pos, D.ids, B->d_samp, B->d_on, B->d_probs, s);
            if (e != hipSuccess) { set_error(hipGetErrorString(e)); rc = SMX_EDEVICE; }
        }
        const hipError_t ce = hipStreamEndCapture(s, &graph);
        if (rc == SMX_OK && ce == hipSuccess) {
            const hipError_t ie = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
            if (ie != hipSuccess) { exec = nullptr; set_error(hipGetErrorString(ie)); rc = SMX_EDEVICE; }
        } else if (rc == SMX_OK) {
            set_error(hipGetErrorString(ce));
            rc = SMX_EDEVICE;
        }
        if (graph) (void)hipGraphDestroy(graph);
        if (rc != SMX_OK) {
            B->graphs.erase(2 * n + (any ? 1 : 0));
            return rc;
        }
    }
    StopCheck stop;
    for (int i = 0; i < n; i++) stop.add(B->slot[(size_t)i], B->joined[(size_t)i]);
    int done = 0, halt = SMX_OK;
    {
        Pacer pace(s, 2);
        while (done < n_steps && (halt = stop.poll()) == SMX_OK) {
            SMX_HIP(hipGraphLaunch(exec, s));
            done++;
            SMX_HIP(pace.launched());
        }
    }
    if (done == 1 && n_steps == 1)   // the step's tokens are also each member's next input id: one copy
        SMX_HIP(hipMemcpyAsync(out_tokens, D.ids, (size_t)n * 4, hipMemcpyDeviceToHost, s));
    else if (done > 0)
        for (int i = 0; i < n; i++)
            SMX_HIP(hipMemcpyAsync(out_tokens + (size_t)i * n_steps, B->slot[(size_t)i]->tokens + B->pos[(size_t)i] + 1,
                                   (size_t)done * 4, hipMemcpyDeviceToHost, s));
    SMX_HIP(hipStreamSynchronize(s));
    for (int i = 0; i < n; i++) {
        if (done > 0) {
            B->pos[(size_t)i] += done;
            B->id[(size_t)i] = out_tokens[(size_t)i * n_steps + done - 1];
            if (B->on[(size_t)i]) B->samp[(size_t)i].counter += (uint64_t)done;
        }
        for (int k = done; k < n_steps; k++) out_tokens[(size_t)i * n_steps + k] = -1;
    }
    if (halt != SMX_OK)
        SMX_FAIL(halt, "smx_batcher_step: stopped after %d of %d steps (%s)", done, n_steps,
                 halt == SMX_ECANCELED ? "cancel request" : "time limit");
    return SMX_OK;
}

SMX_API int smx_batcher_destroy(smx_batcher *B)
{
    if (!B) return SMX_OK;
    (void)hipSetDevice(B->m->ctx->device);
    (void)hipStreamSynchronize(B->stream);
    for (auto &g : B->graphs) if (g.second) (void)hipGraphExecDestroy(g.second);
    for (size_t i = 0; i < B->slot.size(); i++) {
        const int32_t p = B->pos[i];
        (void)hipMemcpy(B->slot[i]->pos, &p, 4, hipMemcpyHostToDevice);
        B->slot[i]->busy.store(0);
    }
    batch_free(B->D);
    free_dev(B->d_samp); free_dev(B->d_on); free_dev(B->d_probs);
    if (B->stream) (void)hipStreamDestroy(B->stream);
    B->m->sessions.fetch_sub(1);
    delete B;
    return SMX_OK;
}

SMX_API int smx_session_reset(smx_session *S)
{
    if (!S) SMX_FAIL(SMX_EINVAL, "smx_session_reset: null session");
    BusyGuard guard(S->busy);
    if (!guard.ok) SMX_FAIL(SMX_EBUSY, "smx_session_reset: session in use on another thread");
    S->cancel.store(0);
    SMX_HIP(hipSetDevice(S->m->ctx->device));
    const int32_t zero = 0;
    SMX_HIP(hipMemcpyAsync(S->pos, &zero, 4, hipMemcpyHostToDevice, S->stream));
    SMX_HIP(hipStreamSynchronize(S->stream));
    return SMX_OK;
}

SMX_API int smx_session_destroy(smx_session *S)
{
    if (!S) return SMX_OK;
    if (S->busy.load() != 0)
        SMX_FAIL(SMX_EBUSY, "smx_session_destroy: session in use (on another thread or in a batcher)");
    (void)hipSetDevice(S->m->ctx->device);
    if (S->g_prefill) (void)hipGraphExecDestroy(S->g_prefill);
    if (S->g_decode) (void)hipGraphExecDestroy(S->g_decode);
    if (S->g_decode_next) (void)hipGraphExecDestroy(S->g_decode_next);
    if (S->g_decode_block) (void)hipGraphExecDestroy(S->g_decode_block);
    if (S->g_sample) (void)hipGraphExecDestroy(S->g_sample);
    for (hipEvent_t e : S->ev) if (e) (void)hipEventDestroy(e);
    if (S->stream) {
        (void)hipStreamSynchronize(S->stream);
        (void)hipStreamDestroy(S->stream);
    }
    free_dev(S->kc); free_dev(S->vc); free_dev(S->x); free_dev(S->q); free_dev(S->att); free_dev(S->scores);
    free_dev(S->h); free_dev(S->logits); free_dev(S->tokens); free_dev(S->pos); free_dev(S->amax);
    free_dev(S->head_val); free_dev(S->head_idx);
    batch_free(S->pb);
    free_dev(S->samp); free_dev(S->probs);
    S->m->sessions.fetch_sub(1);
    delete S;
    return SMX_OK;
}

}  // extern "C"
