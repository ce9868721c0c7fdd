// gemv_dispatch.cpp -- routes a fused GEMV to the instantiation compiled for its block format
// (k_gemv.hip is built once per format) after checking the shape limits the kernels assume.
#include "smx_internal.h"

namespace smx {

hipError_t launch_gemv_fmt0(const GemvArgs &a, int m, hipStream_t s);
hipError_t launch_gemv_fmt1(const GemvArgs &a, int m, hipStream_t s);
hipError_t launch_gemv_fmt2(const GemvArgs &a, int m, hipStream_t s);
hipError_t launch_gemv_fmt3(const GemvArgs &a, int m, hipStream_t s);
hipError_t launch_gemv_fmt4(const GemvArgs &a, int m, hipStream_t s);
hipError_t launch_gemv_fmt5(const GemvArgs &a, int m, hipStream_t s);
hipError_t launch_gemv_fmt6(const GemvArgs &a, int m, hipStream_t s);
hipError_t launch_gemv_fmt7(const GemvArgs &a, int m, hipStream_t s);
hipError_t launch_gemv_fmt8(const GemvArgs &a, int m, hipStream_t s);

hipError_t launch_gemv(const GemvArgs &a, int m, hipStream_t s)
{
    // Weight offsets are 32-bit inside the kernels; columns come in whole 32-element chunks.
    if (a.w.rows <= 0 || a.w.cols <= 0 || a.w.cols % 32 != 0 || m <= 0 || m > 65535)
        return hipErrorInvalidValue;
    if ((uint64_t)a.w.rows * (uint64_t)a.w.nb * (uint64_t)fmt_main_bytes(a.w.fmt) >= (1ull << 32))
        return hipErrorInvalidValue;
    // two partial activation vectors: staged paths only (K <= 16384), no fused norm, one row
    if (a.x_parts > 2 || (a.x_parts == 2 && (m != 1 || a.pro != PRO_NONE || a.x_embed || a.w.cols > 8192 || a.epi == EPI_SILU || a.epi == EPI_QKV ||
                               a.epi == EPI_ARGMAX)))
        return hipErrorInvalidValue;
    switch (a.w.fmt) {
    case FMT_Q4_0: return launch_gemv_fmt0(a, m, s);
    case FMT_Q8_0: return launch_gemv_fmt1(a, m, s);
    case FMT_Q4_K: return launch_gemv_fmt2(a, m, s);
    case FMT_Q5_K: return launch_gemv_fmt3(a, m, s);
    case FMT_Q6_K: return launch_gemv_fmt4(a, m, s);
    case FMT_F16: return launch_gemv_fmt5(a, m, s);
    case FMT_F32: return launch_gemv_fmt6(a, m, s);
    case FMT_SQ8: return launch_gemv_fmt7(a, m, s);
    case FMT_SQ4: return launch_gemv_fmt8(a, m, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace smx
