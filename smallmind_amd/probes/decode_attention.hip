// decode_attention.hip -- measurement probe: the two decode-attention designs of k_ops.hip timed
// against each other at the configs[2] head layout (32 query heads, 4 KV heads, head_dim 64).
//
//   one-launch  k_attn_dec: workgroup = (query head, 16-dimension slice); each computes its
//               head's scores over all positions itself (reads the KV head's whole K), takes the
//               exact max, FastExp, the sum and its slice of P.V.
//   two-launch  k_attn_scores (workgroup = (KV head, 32-position block), K block read once for
//               all 8 query heads) then k_attn_pv (workgroup = (query head, slice)); the kernel
//               boundary supplies the exact maximum over all positions.
//
// 200 calls of each are captured in a HIP graph and replayed; K/V rotate over 24 layer copies
// (48 MB, more than the L2s hold) as in a decode step.  Prints microseconds per call and the
// largest difference between the two outputs.
//
// Build and run (repository root):
//   hipcc -O3 -std=c++17 --offload-arch=gfx950 -ffp-contract=off \
//     -Xclang -target-feature -Xclang -packed-fp32-ops \
//     smallmind_amd/probes/decode_attention.hip -o /tmp/decode_attention
//   /tmp/decode_attention
#include "../csrc/k_ops.hip"
#include <cstdio>
#include <vector>
#include <cstdlib>
using namespace smx;
#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e_), __LINE__); exit(1);} } while (0)
int main() {
    const int H = 32, HKV = 4, HD = 64, CTX = 1024;
    std::vector<float> hq(H * HD), hk((size_t)HKV * HD * CTX), hv((size_t)HKV * CTX * HD);
    srand(1);
    for (auto &x : hq) x = (rand() / (float)RAND_MAX - 0.5f);
    for (auto &x : hk) x = (rand() / (float)RAND_MAX - 0.5f);
    for (auto &x : hv) x = (rand() / (float)RAND_MAX - 0.5f);
    float *q, *kc0, *vc0, *oa, *ob, *sc;
    const int NL = 24;   // layer copies: K/V not resident in L2, as in a decode step
    CK(hipMalloc(&q, hq.size() * 4)); CK(hipMalloc(&kc0, hk.size() * 4 * NL)); CK(hipMalloc(&vc0, hv.size() * 4 * NL));
    CK(hipMalloc(&oa, H * HD * 4)); CK(hipMalloc(&ob, H * HD * 4)); CK(hipMalloc(&sc, H * CTX * 4));
    CK(hipMemcpy(q, hq.data(), hq.size() * 4, hipMemcpyHostToDevice));
    for (int l = 0; l < NL; l++) {
        CK(hipMemcpy(kc0 + l * hk.size(), hk.data(), hk.size() * 4, hipMemcpyHostToDevice));
        CK(hipMemcpy(vc0 + l * hv.size(), hv.data(), hv.size() * 4, hipMemcpyHostToDevice));
    }
    hipStream_t s; CK(hipStreamCreate(&s));
    hipEvent_t e0, e1; CK(hipEventCreate(&e0)); CK(hipEventCreate(&e1));
    const int N = 200;
    for (int n_pos : {160, 384, 512, 768, 1024}) {
        const int sc_stride = (n_pos + 3) & ~3;
        const int nblk = (n_pos + kScorePB - 1) / kScorePB;
        const dim3 g1((unsigned)(HKV * nblk)), g2((unsigned)(H * (HD / kPvSlice)));
        const size_t q_lds = (size_t)(H / HKV) * HD * 4, p_lds = (size_t)n_pos * 4;
        const int U = n_pos <= 256 ? 4 : n_pos <= 512 ? 8 : n_pos <= 768 ? 12 : 16;
        for (int v = 0; v < 2; v++) {
            int li = 0;
            auto launch = [&]() {
                const float *kc = kc0 + (li % NL) * hk.size(), *vc = vc0 + (li % NL) * hv.size();
                li++;
                if (v == 0) return launch_attn_dec(g2, n_pos, HD, q, kc, vc, oa, H, HKV, CTX, nullptr, n_pos, s, nullptr);
                return launch_attn_hd<64>(g1, g2, q_lds, p_lds, U, 256, q, kc, vc, ob, sc, H, HKV, CTX, sc_stride,
                                          nullptr, n_pos, nblk, s);
            };
            CK(launch()); CK(hipStreamSynchronize(s));
            hipGraph_t g; hipGraphExec_t ge;
            CK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
            for (int i = 0; i < N; i++) CK(launch());
            CK(hipStreamEndCapture(s, &g));
            CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
            CK(hipGraphLaunch(ge, s)); CK(hipStreamSynchronize(s));
            float best = 1e9;
            for (int r = 0; r < 5; r++) {
                CK(hipEventRecord(e0, s)); CK(hipGraphLaunch(ge, s)); CK(hipEventRecord(e1, s));
                CK(hipEventSynchronize(e1));
                float ms; CK(hipEventElapsedTime(&ms, e0, e1)); if (ms < best) best = ms;
            }
            printf("n_pos %4d variant %s: %.3f us per call\n", n_pos, v == 0 ? "one-launch" : "two-launch", best * 1000.0f / N);
            CK(hipGraphExecDestroy(ge)); CK(hipGraphDestroy(g));
        }
        std::vector<float> a(H * HD), b(H * HD);
        CK(hipMemcpy(a.data(), oa, a.size() * 4, hipMemcpyDeviceToHost));
        CK(hipMemcpy(b.data(), ob, b.size() * 4, hipMemcpyDeviceToHost));
        double md = 0; for (size_t i = 0; i < a.size(); i++) md = fmax(md, fabs(a[i] - b[i]));
        printf("  max |A-B| %.3g\n", md);
    }
    return 0;
}
