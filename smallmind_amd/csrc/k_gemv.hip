// k_gemv.hip -- fused dequantize-GEMV for Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K weights.
//
// y[r] = sum_k W[r][k] * x[k] for a row-major [rows][cols] weight in the backend layout
// (smx_internal.h).  Replaces Linear.ForwardFP32 / IWeightTensor.MatMul for batch-1 decode
// (NeuralNet.cs:145-298) and the fused C# kernels (MatMulF32Q8.cs, MatMulF32Q4.cs,
// FusedQ4KMatMul.cs, FusedQ6KMatMul.cs), computing y = x W^T as the GGUF loader path does.
//
// Work decomposition: a wave64 owns R consecutive weight rows and is independent of every
// other wave (no LDS, no workgroup barrier).  Lane l walks the 32-element chunks l, l+64, ...
//   1. the weight loads of the wave's first chunk are issued before anything else, so HBM
//      latency overlaps the activation prologue;
//   2. the activation chunk is read from global memory (L1/L2 resident: every wave reads the
//      same vector); a RMSNorm / LayerNorm prologue is computed by the wave itself with
//      shuffles (deterministic, identical in every wave), so the norm never takes its own
//      kernel or HBM round trip;
//   3. codes are unpacked with and/shift into bytes and converted with v_cvt_f32_ubyte*, and
//      block scales are factored out of the 32-term sums (sum (sc*q - m) x =
//      sc * sum q x - m * sum x);
//   4. the R partial sums are reduce-scattered across the wave and one lane applies the
//      epilogue (bias, residual, SwiGLU, GELU, or RoPE + KV-cache append).
#include "smx_device.h"
#include "smx_formats.h"
#include "smx_gemv.h"

namespace smx {

namespace {

template <int F, int R>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a)
{
    const int64_t wave = ((int64_t)blockIdx.x * (blockDim.x >> 6)) + wave_id();
    gemv_wave<F, R>(a, wave * R, blockIdx.y);
}

template <int F, int R>
hipError_t launch_fr(const GemvArgs &a, int m, hipStream_t s)
{
    const int64_t waves = (a.w.rows + R - 1) / R;
    const dim3 grid((unsigned)((waves + 3) / 4), (unsigned)m);
    hipLaunchKernelGGL((k_gemv<F, R>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int F>
hipError_t launch_f(const GemvArgs &a, int m, hipStream_t s)
{
    // Pairs of rows must share a wave for the SwiGLU and RoPE epilogues, so R >= 2.
    if (a.w.rows >= 8192) return launch_fr<F, 4>(a, m, s);
    return launch_fr<F, 2>(a, m, s);
}

}  // namespace

hipError_t launch_gemv(const GemvArgs &a, int m, hipStream_t s)
{
    switch (a.w.fmt) {
    case FMT_Q4_0: return launch_f<FMT_Q4_0>(a, m, s);
    case FMT_Q8_0: return launch_f<FMT_Q8_0>(a, m, s);
    case FMT_Q4_K: return launch_f<FMT_Q4_K>(a, m, s);
    case FMT_Q5_K: return launch_f<FMT_Q5_K>(a, m, s);
    case FMT_Q6_K: return launch_f<FMT_Q6_K>(a, m, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace smx
