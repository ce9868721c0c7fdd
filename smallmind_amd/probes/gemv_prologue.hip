// gemv_prologue.hip -- measurement probe: what the fused RMSNorm prologue and SwiGLU epilogue
// cost the Q4_K gate/up GEMV of the configs[2] decode step (11264 x 2048), next to the plain
// GEMV that bench.py's roofline line times.  200 launches over rotating weight copies (>= 600
// MB, streamed from HBM) are captured in a graph and replayed (best of 5); each variant runs
// with x warm (the same vector every launch) and with x freshly written by a small kernel
// before each GEMV, as the O projection writes it in the decode step ("touch": its own cost
// is printed and included in those lines).
//
// Build and run (repository root, after __graft_entry__.build(), which leaves k_ops.o):
//   hipcc -O3 -std=c++17 --offload-arch=gfx950 -ffp-contract=off -Xclang -target-feature -Xclang -packed-fp32-ops \
//     -DSMX_GEMV_FMT=2 -c smallmind_amd/probes/gemv_prologue.hip -o /tmp/gemv_prologue.o
//   hipcc --offload-arch=gfx950 /tmp/gemv_prologue.o smallmind_amd/_build/k_ops.o -o /tmp/gemv_prologue
//   /tmp/gemv_prologue
#include "../csrc/k_gemv.hip"
#include <cstdio>
#include <vector>
#include <algorithm>
#include <cstdlib>
using namespace smx;
#define CK(...) do { hipError_t e_ = (__VA_ARGS__); if (e_ != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e_), __LINE__); exit(1);} } while (0)

__global__ void kfill(uint8_t *p, size_t n, uint32_t seed)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i < n / 4; i += (size_t)gridDim.x * blockDim.x) {
        uint32_t x = (uint32_t)i * 2654435761u ^ seed;
        x ^= x >> 13; x *= 0x5bd1e995u; x ^= x >> 15;
        ((uint32_t *)p)[i] = x & 0x3BFF3BFFu;
    }
}
// writes x (as the O projection's residual epilogue would): 2048 floats, 8 workgroups
__global__ void ktouch(float *x, int n, float v)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = v + 0.001f * (float)(i & 63);
}

int main()
{
    const int N = 11264, K = 2048;
    const size_t wbytes = (size_t)N * (K / 256) * 144;
    const int copies = (int)((600u << 20) / wbytes + 1);
    uint8_t *wq; CK(hipMalloc(&wq, wbytes * copies));
    hipLaunchKernelGGL(kfill, dim3(4096), dim3(256), 0, 0, wq, wbytes * copies, 3u);
    float *x, *g, *out, *res;
    CK(hipMalloc(&x, K * 4)); CK(hipMalloc(&g, K * 4)); CK(hipMalloc(&out, N * 4)); CK(hipMalloc(&res, N * 4));
    std::vector<float> h(K, 0.5f);
    CK(hipMemcpy(x, h.data(), K * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(g, h.data(), K * 4, hipMemcpyHostToDevice));
    hipStream_t s; CK(hipStreamCreate(&s));
    hipEvent_t e0, e1; CK(hipEventCreate(&e0)); CK(hipEventCreate(&e1));
    const int L = 200;
    auto timeit = [&](const char *name, auto launch) {
        hipGraph_t gr; hipGraphExec_t ge;
        CK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
        for (int i = 0; i < L; i++) launch(i);
        CK(hipStreamEndCapture(s, &gr));
        CK(hipGraphInstantiate(&ge, gr, nullptr, nullptr, 0));
        CK(hipGraphLaunch(ge, s)); CK(hipStreamSynchronize(s));
        float best = 1e9;
        for (int r = 0; r < 5; r++) {
            CK(hipEventRecord(e0, s)); CK(hipGraphLaunch(ge, s)); CK(hipEventRecord(e1, s));
            CK(hipEventSynchronize(e1));
            float ms; CK(hipEventElapsedTime(&ms, e0, e1)); best = std::min(best, ms);
        }
        printf("%-52s %7.3f us per step\n", name, best * 1000.0f / L);
        fflush(stdout);
        CK(hipGraphExecDestroy(ge)); CK(hipGraphDestroy(gr));
    };
    GemvArgs a{};
    a.w.fmt = FMT_Q4_K; a.w.rows = N; a.w.cols = K; a.w.nb = K / 256; a.w.cache = 0;
    a.x = x; a.x_stride = K; a.out = out; a.out_stride = N; a.gamma = g; a.eps = 1e-5f;
    auto plain = [&](int i) { GemvArgs b = a; b.w.q = wq + (size_t)(i % copies) * wbytes; b.pro = PRO_NONE; b.epi = EPI_STORE;
                              CK(launch_v<4, 1, 1, PRO_NONE, EC_SIMPLE, 1>(b, 1, s)); };
    auto rms = [&](int i) { GemvArgs b = a; b.w.q = wq + (size_t)(i % copies) * wbytes; b.pro = PRO_RMS; b.epi = EPI_STORE;
                            CK(launch_v<4, 1, 1, PRO_RMS, EC_SIMPLE, 1>(b, 1, s)); };
    auto silu = [&](int i) { GemvArgs b = a; b.w.q = wq + (size_t)(i % copies) * wbytes; b.pro = PRO_RMS; b.epi = EPI_SILU;
                             CK(launch_v<4, 1, 1, PRO_RMS, EC_SILU, 1>(b, 1, s)); };
    auto touch = [&](int i) { hipLaunchKernelGGL(ktouch, dim3(8), dim3(256), 0, s, x, K, 0.5f + 1e-3f * (i & 7)); };
    for (int rep = 0; rep < 2; rep++) {
        timeit("plain (roofline kernel), x warm", plain);
        timeit("RMSNorm prologue, x warm", rms);
        timeit("RMSNorm + SwiGLU (in-step form), x warm", silu);
        timeit("touch kernel alone", touch);
        timeit("touch + plain", [&](int i) { touch(i); plain(i); });
        timeit("touch + RMSNorm", [&](int i) { touch(i); rms(i); });
        timeit("touch + RMSNorm + SwiGLU", [&](int i) { touch(i); silu(i); });
    }
    return 0;
}
