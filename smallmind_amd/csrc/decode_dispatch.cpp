// decode_dispatch.cpp -- picks the persistent decode kernel for a block format / head size,
// sizes its grid (one co-resident workgroup per CU) and launches it cooperatively, which
// guarantees that every workgroup of the grid is resident at once, as the device-wide barrier
// inside the kernel requires.
#include "smx_internal.h"

namespace smx {

const void *decode_kernel_fmt0(int hd);
const void *decode_kernel_fmt1(int hd);
const void *decode_kernel_fmt2(int hd);
const void *decode_kernel_fmt3(int hd);
const void *decode_kernel_fmt4(int hd);

namespace {

const void *pick(int fmt, int hd)
{
    switch (fmt) {
    case FMT_Q4_0: return decode_kernel_fmt0(hd);
    case FMT_Q8_0: return decode_kernel_fmt1(hd);
    case FMT_Q4_K: return decode_kernel_fmt2(hd);
    case FMT_Q5_K: return decode_kernel_fmt3(hd);
    case FMT_Q6_K: return decode_kernel_fmt4(hd);
    default: return nullptr;
    }
}

}  // namespace

int decode_grid(int fmt, int hd, size_t lds, int device)
{
    static_assert(FMT_Q4_0 == 0 && FMT_Q8_0 == 1 && FMT_Q4_K == 2 && FMT_Q5_K == 3 && FMT_Q6_K == 4,
                  "decode_kernel_fmtN accessors are numbered by Fmt");
    const void *fn = pick(fmt, hd);
    if (!fn) return 0;
    int coop = 0, cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, device) != hipSuccess || !coop)
        return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
    if (lds > 64 * 1024 &&
        hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kDecodeThreads, lds) != hipSuccess ||
        per_cu < 1)
        return 0;
    return cus;
}

hipError_t launch_decode(const DecodeArgs &a, int fmt, int grid, size_t lds, hipStream_t s)
{
    const void *fn = pick(fmt, a.hd);
    if (!fn) return hipErrorInvalidValue;
    DecodeArgs copy = a;
    void *args[] = {&copy};
    return hipLaunchCooperativeKernel(fn, dim3(grid), dim3(kDecodeThreads), args, (unsigned)lds, s);
}

}  // namespace smx
