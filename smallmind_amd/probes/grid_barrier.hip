// grid_barrier.hip -- measurement probe: what a device-wide barrier inside one cooperative kernel
// costs on this GPU, next to what a kernel boundary costs inside a HIP graph.
//
// A persistent decode kernel replaces each kernel boundary of the decode step with a grid
// barrier; it can only win if a barrier is cheaper than a boundary.  Four barrier forms are
// timed over 2000 barriers at grids of 256, 128 and 64 workgroups (one per CU at most, launched
// cooperatively so all are resident), each with a visibility check: after every barrier each
// workgroup reads a value another workgroup wrote before it.  Every spin is bounded (an abort
// flag ends the kernel if a barrier does not complete).  Then empty kernels of several grid
// sizes are replayed back to back in a graph: the per-launch time is the boundary cost.
//
// Build and run (repository root):
//   hipcc -O3 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops \\
//     smallmind_amd/probes/grid_barrier.hip -o /tmp/grid_barrier
//   /tmp/grid_barrier
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>

#define CK(x)                                                                              \
    do {                                                                                   \
        hipError_t e_ = (x);                                                               \
        if (e_ != hipSuccess) {                                                            \
            printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);          \
            exit(1);                                                                       \
        }                                                                                  \
    } while (0)

constexpr unsigned kSpin = 1u << 20;

__device__ inline void st_agent(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline float ld_agent(const float *p) { return __hip_atomic_load((float *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// V: 0 = one counter, release add + acquire fence (reference); 1 = one counter, relaxed, data written
// through with agent-scope stores, read with agent-scope loads; 2 = flag per workgroup (no atomic
// contention), polled by one wave, data as in 1; 3 = flag array, release/acquire fences, plain data
template <int V>
__global__ __launch_bounds__(256) void kbar(unsigned *bar, unsigned *flags, int *abort_flag, int n, float *data,
                                            int *errors)
{
    __shared__ int ok;
    const unsigned nwg = gridDim.x, b = blockIdx.x;
    int err = 0;
    for (int i = 1; i <= n; i++) {
        // write 64 floats (a GEMV phase's output slice)
        float *mine = data + ((size_t)(i & 1) * nwg + b) * 64;
        if (threadIdx.x < 64) {
            if constexpr (V == 0 || V == 3) mine[threadIdx.x] = (float)(i * 1000 + b);
            else st_agent(mine + threadIdx.x, (float)(i * 1000 + b));
        }
        if constexpr (V == 1 || V == 2) __builtin_amdgcn_s_waitcnt(0);   // stores complete before arrival
        __syncthreads();
        if (threadIdx.x < 64) {
            unsigned spins = 0;
            int good = 1;
            if constexpr (V == 0 || V == 1) {
                if (threadIdx.x == 0) {
                    if constexpr (V == 0) __hip_atomic_fetch_add(bar, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
                    else __hip_atomic_fetch_add(bar, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    const unsigned target = (unsigned)i * nwg;
                    while ((int)(__hip_atomic_load(bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - target) < 0) {
                        if (++spins > kSpin) { good = 0; break; }
                    }
                    if constexpr (V == 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
                    ok = good;
                }
            } else {
                if (threadIdx.x == 0) {
                    if constexpr (V == 3) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
                    __hip_atomic_store(flags + b, (unsigned)i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                // wave 0 polls every flag: lane l checks flags l, l+64, ...
                while (true) {
                    int done = 1;
                    for (unsigned w = threadIdx.x; w < nwg; w += 64)
                        done &= (int)(__hip_atomic_load(flags + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - (unsigned)i) >= 0;
                    if (__all(done)) break;
                    if (++spins > kSpin) { good = 0; break; }
                }
                if constexpr (V == 3) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
                if (threadIdx.x == 0) ok = good;
            }
        }
        __syncthreads();
        if (!ok) {
            if (threadIdx.x == 0) atomicExch(abort_flag, 1);
            return;
        }
        // read the slice of workgroup (b + 37 * i) % nwg
        const unsigned o = (b + 37u * (unsigned)i) % nwg;
        const float *theirs = data + ((size_t)(i & 1) * nwg + o) * 64;
        if (threadIdx.x < 64) {
            float v = (V == 0 || V == 3) ? theirs[threadIdx.x] : ld_agent(theirs + threadIdx.x);
            if (v != (float)(i * 1000 + o)) err++;
        }
    }
    if (err) atomicAdd(errors, err);
}

__global__ void kempty(float *p) { if (threadIdx.x == 0 && blockIdx.x == 0 && p[0] == 12345.0f) p[1] = 1.0f; }

template <int V>
void run(int grid, int n, unsigned *bar, unsigned *flags, int *ab, float *data, int *errs, hipStream_t s, const char *name)
{
    CK(hipMemset(bar, 0, 4));
    CK(hipMemset(flags, 0, 4096 * 4));
    CK(hipMemset(ab, 0, 4));
    CK(hipMemset(errs, 0, 4));
    CK(hipDeviceSynchronize());
    void *args[] = {&bar, &flags, &ab, &n, &data, &errs};
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    CK(hipEventRecord(e0, s));
    CK(hipLaunchCooperativeKernel((const void *)kbar<V>, dim3(grid), dim3(256), args, 0, s));
    CK(hipEventRecord(e1, s));
    CK(hipStreamSynchronize(s));
    float ms = 0;
    CK(hipEventElapsedTime(&ms, e0, e1));
    int f = 0, e = 0;
    CK(hipMemcpy(&f, ab, 4, hipMemcpyDeviceToHost));
    CK(hipMemcpy(&e, errs, 4, hipMemcpyDeviceToHost));
    printf("grid %4d %-44s %7.3f us/barrier  abort=%d visibility_errors=%d\n", grid, name, ms * 1000.0f / n, f, e);
    fflush(stdout);
    CK(hipEventDestroy(e0));
    CK(hipEventDestroy(e1));
}

int main()
{
    int cus = 0;
    CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    printf("CUs %d\n", cus);
    unsigned *bar, *flags;
    int *ab, *errs;
    float *data;
    CK(hipMalloc(&bar, 256));
    CK(hipMalloc(&flags, 4096 * 4));
    CK(hipMalloc(&ab, 256));
    CK(hipMalloc(&errs, 256));
    CK(hipMalloc(&data, 2 * 4096 * 64 * 4));
    hipStream_t s;
    CK(hipStreamCreate(&s));
    const int n = 2000;
    for (int grid : {cus, cus / 2, 64}) {
        run<1>(grid, 10, bar, flags, ab, data, errs, s, "warmup");
        run<0>(grid, n, bar, flags, ab, data, errs, s, "V0 counter, release/acquire");
        run<1>(grid, n, bar, flags, ab, data, errs, s, "V1 counter, relaxed, write-through data");
        run<2>(grid, n, bar, flags, ab, data, errs, s, "V2 flag array, write-through data");
        run<3>(grid, n, bar, flags, ab, data, errs, s, "V3 flag array, release/acquire fences");
    }
    // empty kernels back to back in a graph, at several grid sizes (workgroup dispatch cost)
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    for (int grid : {1, 64, cus, 1024, 4096}) {
        hipGraph_t g;
        hipGraphExec_t ge;
        CK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
        for (int i = 0; i < 200; i++) hipLaunchKernelGGL(kempty, dim3(grid), dim3(256), 0, s, data);
        CK(hipGetLastError());
        CK(hipStreamEndCapture(s, &g));
        CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        CK(hipGraphLaunch(ge, s));
        CK(hipStreamSynchronize(s));
        CK(hipEventRecord(e0, s));
        for (int r = 0; r < 10; r++) CK(hipGraphLaunch(ge, s));
        CK(hipEventRecord(e1, s));
        CK(hipStreamSynchronize(s));
        float ms = 0;
        CK(hipEventElapsedTime(&ms, e0, e1));
        printf("empty kernel in a graph (grid %4d x 256 threads): %.3f us per launch\n", grid, ms * 1000.0f / 2000);
        CK(hipGraphExecDestroy(ge));
        CK(hipGraphDestroy(g));
    }
    return 0;
}
