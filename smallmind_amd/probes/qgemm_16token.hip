// qgemm_16token.hip -- measurement probe: the staged matrix-core GEMM (k_qgemm_st) at one token
// tile (16 tokens: the configs[4] lockstep step, Q5_K, K = 2048 / 8192), weights rotating over
// >= 600 MB so that every launch streams them from HBM.
//
//   1. Per-wave timeline: a copy of k_qgemm_st's one-token-tile path (same loads, staging and
//      products, plain store epilogue) that records s_memrealtime (100 MHz) at entry, when the
//      first super-block's weights have arrived (staged), after the first half super-block's
//      products (its activation parts have arrived), after each super-block, at the end of the
//      main loop and at the end.  Medians and 90th percentiles over waves and launches.
//   2. Launch times of the product kernel's tiles <RT, NW> (eager launches, HIP events), with
//      the largest difference between tiles' outputs.
//
// Build and run (repository root):
//   hipcc -O3 -std=c++17 --offload-arch=gfx950 -ffp-contract=off -Xclang -target-feature -Xclang -packed-fp32-ops \
//     -c smallmind_amd/probes/qgemm_16token.hip -o /tmp/qgemm_16token.o && hipcc --offload-arch=gfx950 /tmp/qgemm_16token.o -o /tmp/qgemm_16token
//   /tmp/qgemm_16token
#include "../csrc/k_qgemm.hip"
#include <cstdio>
#include <vector>
#include <algorithm>
#include <cstdlib>
using namespace smx;
#define CK(...) do { hipError_t e_ = (__VA_ARGS__); if (e_ != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e_), __LINE__); exit(1);} } while (0)

namespace smx { namespace {
constexpr int NSLOT = 8;
template <int F, int RT, int TT, int NW>
__global__ __launch_bounds__(64 * NW) void k_ts(QgemmArgs a, uint64_t *ts)
{
    uint64_t t[NSLOT];
#pragma unroll
    for (int i = 0; i < NSLOT; i++) t[i] = 0;
    t[0] = __builtin_amdgcn_s_memrealtime();
    using Q = QW<F>;
    using G = Stage<F>;
    constexpr int R16 = 16 * RT;
    constexpr int RS = G::kBytes + 4;
    constexpr int NPC = (R16 * G::kBytes / 16 + 63) / 64;
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
    const uint32_t row_base = blockIdx.x * R16;
    const int tt0 = blockIdx.y * TT;
    const int ntt = (M + 15) >> 4;
    const uint32_t row_bytes = (uint32_t)nsup * G::kBytes;
    const int per = (nsup + NW - 1) / NW;
    const int sup0 = wv * per, sup1 = sup0 + per < nsup ? sup0 + per : nsup;
    f32x4 acc[RT][TT];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int tq = 0; tq < TT; tq++) acc[r][tq] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const uint4 ones_a = make_uint4(kOnes, kOnes, kOnes, kOnes);
    uint4 wp[NPC];
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
    };
    auto stage = [&]() {
        asm volatile("" ::: "memory");
        uint8_t *dst = s_w[wv];
#pragma unroll
        for (int k = 0; k < NPC; k++) {
            const int p = lane + 64 * k;
            if (p < R16 * G::kBytes / 16) {
                const int row = p / (G::kBytes / 16), col = p % (G::kBytes / 16);
                uint32_t *o = (uint32_t *)(dst + row * RS + 16 * col);
                o[0] = wp[k].x; o[1] = wp[k].y; o[2] = wp[k].z; o[3] = wp[k].w;
            }
        }
        asm volatile("" ::: "memory");
    };
    if (sup0 < sup1) issue(sup0);
    int it = 0;
    for (int sup = sup0; sup < sup1; sup++, it++) {
        stage();
        if (it < 2) t[1 + 3 * it] = __builtin_amdgcn_s_memrealtime();
        if (sup + 1 < sup1) issue(sup + 1);
        constexpr int XU = 4;
#pragma unroll
        for (int h = 0; h < 8 / XU; h++) {
            uint4 xa[XU][TT][3];
#pragma unroll
            for (int u = 0; u < XU; u++) {
                const int s = sup * 8 + XU * h + u;
#pragma unroll
                for (int tq = 0; tq < TT; tq++) {
                    const int tt = tt0 + tq < ntt ? tt0 + tq : ntt - 1;
#pragma unroll
                    for (int p = 0; p < 3; p++) xa[u][tq][p] = ld_part(xp, tt, nsb, s, p, lane16);
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
                for (int tq = 0; tq < TT; tq++) {
                    f32x4 sa = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int p = 0; p < 3; p++) sa = mfma(xa[u][tq][p], ones_a, sa);
#pragma unroll
                    for (int r = 0; r < RT; r++) {
                        f32x4 dc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                        for (int p = 0; p < 3; p++) dc = mfma(xa[u][tq][p], wc[r], dc);
                        const float c = sc[r].sc, cs = sc[r].sc * Q::kOff + sc[r].m;
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[r][tq][i] = accumulate1(acc[r][tq][i], c, cs, dc[i], sa[i]);
                    }
                }
            }
            if (it < 2 && h == 0) {
                // force completion of this h's arithmetic before the stamp
                float z = acc[0][0][0];
                asm volatile("" : "+v"(z));
                acc[0][0][0] = z;
                t[2 + 3 * it] = __builtin_amdgcn_s_memrealtime();
            }
        }
        if (it < 2) t[3 + 3 * it] = __builtin_amdgcn_s_memrealtime();
    }
    t[6] = __builtin_amdgcn_s_memrealtime();
    if (wv > 0) {
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int tq = 0; tq < TT; tq++) s_part[wv - 1][r * TT + tq][lane] = acc[r][tq];
    }
    __syncthreads();
    if (wv == 0) {
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int tq = 0; tq < TT; tq++) {
                f32x4 v = acc[r][tq];
#pragma unroll
                for (int k = 0; k < NW - 1; k++) {
                    const f32x4 o = s_part[k][r * TT + tq][lane];
#pragma unroll
                    for (int i = 0; i < 4; i++) v[i] += o[i];
                }
                const uint32_t row = row_base + 16 * r + li;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int tok = (tt0 + tq) * 16 + 4 * g + i;
                    if (row < N && tok < M) a.y[(int64_t)tok * a.y_stride + row] = v[i];
                }
            }
    }
    t[7] = __builtin_amdgcn_s_memrealtime();
    if (lane == 0) {
        const size_t wid = ((size_t)blockIdx.y * gridDim.x + blockIdx.x) * NW + wv;
#pragma unroll
        for (int i = 0; i < NSLOT; i++) ts[wid * NSLOT + i] = t[i];
    }
}
}}

__global__ void kfill(uint8_t *p, size_t n, uint32_t seed)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i < n / 4; i += (size_t)gridDim.x * blockDim.x) {
        uint32_t x = (uint32_t)i * 2654435761u ^ seed;
        x ^= x >> 13; x *= 0x5bd1e995u; x ^= x >> 15;
        // keep fp16 fields finite: clear the top exponent bit of every 16-bit half
        ((uint32_t *)p)[i] = x & 0xBFFFBFFFu;
    }
}

template <int F, int RT, int TT, int NW>
void run(const char *name, int N, int K, int reps)
{
    const int M = 16;
    const size_t wbytes = (size_t)N * (K / 256) * Stage<F>::kBytes;
    const int copies = (int)std::max<size_t>(2, (600u << 20) / wbytes + 1);
    uint8_t *wq; CK(hipMalloc(&wq, wbytes * copies));
    hipLaunchKernelGGL(kfill, dim3(4096), dim3(256), 0, 0, wq, wbytes * copies, 7u);
    const size_t xpb = qgemm_xp_bytes(M, K);
    uint8_t *xp; CK(hipMalloc(&xp, xpb));
    hipLaunchKernelGGL(kfill, dim3(256), dim3(256), 0, 0, xp, xpb, 9u);
    float *y; CK(hipMalloc(&y, (size_t)M * N * 4));
    const dim3 grid((unsigned)((N + 16 * RT - 1) / (16 * RT)), 1);
    const size_t nwaves = (size_t)grid.x * NW;
    uint64_t *ts; CK(hipMalloc(&ts, nwaves * NSLOT * 8 * reps));
    QgemmArgs a{};
    a.w.fmt = F; a.w.rows = N; a.w.cols = K; a.w.nb = K / 256; a.w.d = nullptr;
    a.xp = xp; a.M = M; a.y = y; a.y_stride = N; a.epi = EPI_STORE;
    CK(hipDeviceSynchronize());
    for (int r = 0; r < reps; r++) {
        a.w.q = wq + (size_t)(r % copies) * wbytes;
        hipLaunchKernelGGL((k_ts<F, RT, TT, NW>), grid, dim3(64 * NW), 0, 0, a, ts + nwaves * NSLOT * r);
    }
    CK(hipGetLastError());
    CK(hipDeviceSynchronize());
    std::vector<uint64_t> h(nwaves * NSLOT * reps);
    CK(hipMemcpy(h.data(), ts, h.size() * 8, hipMemcpyDeviceToHost));
    // per rep: span; per wave: slot deltas relative to entry (10 ns ticks) -> medians over waves and reps (last half)
    std::vector<double> span;
    std::vector<std::vector<double>> d(NSLOT);
    std::vector<double> entry_spread;
    for (int r = reps / 2; r < reps; r++) {
        const uint64_t *b = h.data() + nwaves * NSLOT * r;
        uint64_t mn = ~0ull, mx = 0, emx = 0;
        for (size_t wi = 0; wi < nwaves; wi++) {
            mn = std::min(mn, b[wi * NSLOT]);
            mx = std::max(mx, b[wi * NSLOT + 7]);
            emx = std::max(emx, b[wi * NSLOT]);
        }
        span.push_back((mx - mn) * 10.0);
        entry_spread.push_back((emx - mn) * 10.0);
        for (size_t wi = 0; wi < nwaves; wi++)
            for (int s = 1; s < NSLOT; s++)
                if (b[wi * NSLOT + s]) d[s].push_back(((double)b[wi * NSLOT + s] - (double)b[wi * NSLOT]) * 10.0);
    }
    auto med = [](std::vector<double> v) { if (v.empty()) return -1.0; std::sort(v.begin(), v.end()); return v[v.size() / 2]; };
    auto p90 = [](std::vector<double> v) { if (v.empty()) return -1.0; std::sort(v.begin(), v.end()); return v[v.size() * 9 / 10]; };
    printf("%-28s N=%5d K=%5d grid=%u x %d waves: span med %.0f ns, entry spread med %.0f ns\n", name, N, K, grid.x, NW,
           med(span), med(entry_spread));
    const char *lab[NSLOT] = {"entry", "stage0(W0 in)", "h0 done (P in)", "sup0 done", "stage1(W1 in)", "h0' done", "loop end", "end"};
    for (int s = 1; s < NSLOT; s++)
        if (!d[s].empty()) printf("   %-16s med %6.0f ns  p90 %6.0f ns\n", lab[s], med(d[s]), p90(d[s]));
    fflush(stdout);
    CK(hipFree(wq)); CK(hipFree(xp)); CK(hipFree(y)); CK(hipFree(ts));
}

struct Shape { const char *name; int N, K; };

template <int F, int RT, int TT, int NW>
double time_tile(const Shape &sh, uint8_t *wq, size_t wbytes, int copies, uint8_t *xp, float *y, int reps, std::vector<float> *out)
{
    QgemmArgs a{};
    a.w.fmt = F; a.w.rows = sh.N; a.w.cols = sh.K; a.w.nb = sh.K / 256; a.w.d = nullptr;
    a.xp = xp; a.M = 16; a.y = y; a.y_stride = sh.N; a.epi = EPI_STORE;
    hipEvent_t e0, e1; CK(hipEventCreate(&e0)); CK(hipEventCreate(&e1));
    for (int r = 0; r < copies; r++) { a.w.q = wq + (size_t)r * wbytes; CK(launch_st<F, RT, TT, NW>(a, 0)); }
    CK(hipDeviceSynchronize());
    CK(hipEventRecord(e0, 0));
    for (int r = 0; r < reps; r++) { a.w.q = wq + (size_t)(r % copies) * wbytes; CK(launch_st<F, RT, TT, NW>(a, 0)); }
    CK(hipEventRecord(e1, 0));
    CK(hipEventSynchronize(e1));
    float ms; CK(hipEventElapsedTime(&ms, e0, e1));
    if (out) {
        a.w.q = wq;
        CK(launch_st<F, RT, TT, NW>(a, 0));
        CK(hipDeviceSynchronize());
        out->resize((size_t)16 * sh.N);
        CK(hipMemcpy(out->data(), y, out->size() * 4, hipMemcpyDeviceToHost));
    }
    CK(hipEventDestroy(e0)); CK(hipEventDestroy(e1));
    return ms * 1000.0 / reps;
}

template <int RT, int NW>
void one(const Shape &sh, uint8_t *wq, size_t wbytes, int copies, uint8_t *xp, float *y, std::vector<float> &ref, bool first)
{
    std::vector<float> o;
    const double us = time_tile<FMT_Q5_K, RT, 1, NW>(sh, wq, wbytes, copies, xp, y, 400, &o);
    double md = 0, mr = 0;
    if (first) ref = o;
    for (size_t i = 0; i < o.size(); i++) { md = std::max(md, (double)fabsf(o[i] - ref[i])); mr = std::max(mr, (double)fabsf(ref[i])); }
    const double gbs = (double)wbytes / (us * 1e-6) / 1e9;
    printf("  %-20s <RT=%d,NW=%2d>  %7.2f us/launch  %6.0f GB/s  max|d|/max|ref| %.2e\n", sh.name, RT, NW, us, gbs, md / (mr > 0 ? mr : 1));
    fflush(stdout);
}

void tile_sweep()
{
    const Shape shapes[] = {{"QKV 6144x2048", 6144, 2048}, {"O 2048x2048", 2048, 2048},
                            {"gate/up 16384x2048", 16384, 2048}, {"down 2048x8192", 2048, 8192}};
    for (const Shape &sh : shapes) {
        const size_t wbytes = (size_t)sh.N * (sh.K / 256) * Stage<FMT_Q5_K>::kBytes;
        const int copies = (int)std::max<size_t>(2, (600u << 20) / wbytes + 1);
        uint8_t *wq; CK(hipMalloc(&wq, wbytes * copies));
        hipLaunchKernelGGL(kfill, dim3(4096), dim3(256), 0, 0, wq, wbytes, 7u);
        for (int c = 1; c < copies; c++) CK(hipMemcpy(wq + (size_t)c * wbytes, wq, wbytes, hipMemcpyDeviceToDevice));
        const size_t xpb = qgemm_xp_bytes(16, sh.K);
        uint8_t *xp; CK(hipMalloc(&xp, xpb));
        hipLaunchKernelGGL(kfill, dim3(256), dim3(256), 0, 0, xp, xpb, 9u);
        float *y; CK(hipMalloc(&y, (size_t)16 * sh.N * 4));
        std::vector<float> ref;
        one<1, 16>(sh, wq, wbytes, copies, xp, y, ref, true);
        one<1, 8>(sh, wq, wbytes, copies, xp, y, ref, false);
        one<1, 4>(sh, wq, wbytes, copies, xp, y, ref, false);
        one<2, 4>(sh, wq, wbytes, copies, xp, y, ref, false);
        one<2, 8>(sh, wq, wbytes, copies, xp, y, ref, false);
        CK(hipFree(wq)); CK(hipFree(xp)); CK(hipFree(y));
    }
}

int main()
{
    printf("== per-wave timeline (instrumented copy of the one-token-tile path)\n");
    run<FMT_Q5_K, 1, 1, 8>("Q5_K QKV <1,1,8>", 6144, 2048, 40);
    run<FMT_Q5_K, 1, 1, 8>("Q5_K O <1,1,8>", 2048, 2048, 40);
    run<FMT_Q5_K, 2, 1, 4>("Q5_K gate/up <2,1,4>", 16384, 2048, 40);
    run<FMT_Q5_K, 1, 1, 16>("Q5_K down <1,1,16>", 2048, 8192, 40);
    printf("== launch times of the product kernel's tiles\n");
    tile_sweep();
    return 0;
}
