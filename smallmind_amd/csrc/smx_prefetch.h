// smx_prefetch.h -- extra workgroups of a launch that read weight ranges into the MALL.
//
// The decode step's GEMVs are latency-bound at their sizes and run measurably shorter with their
// weights in the 256 MB memory-side cache than from HBM; the decode attention, which leaves half
// the CUs idle, carries Prefetch ranges for the GEMV after it.
#pragma once

#include "smx_internal.h"

namespace smx {

// Workgroup w of nw reads its share of every range (16-byte loads, 8 per thread in flight) so
// that the lines sit in the MALL when the later kernel reads them.  The loaded values only feed
// an empty asm statement, which keeps the loads.
__device__ __forceinline__ void prefetch_slice(const Prefetch &pf, int w, int nw, int nt)
{
    const uint32_t tid = threadIdx.x;
    uint32_t acc = 0;
    for (int r = 0; r < pf.n; r++) {
        const uint32_t n16 = pf.bytes[r] >> 4;
        const uint32_t b0 = (uint32_t)((uint64_t)n16 * (uint32_t)w / (uint32_t)nw);
        const uint32_t b1 = (uint32_t)((uint64_t)n16 * (uint32_t)(w + 1) / (uint32_t)nw);
        const uint4 *src = (const uint4 *)pf.p[r];
        for (uint32_t i = b0 + tid; i < b1; i += 8u * (uint32_t)nt) {
            uint4 v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint32_t j = i + (uint32_t)k * (uint32_t)nt;
                v[k] = j < b1 ? src[j] : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int k = 0; k < 8; k++) acc ^= v[k].x ^ v[k].w;
        }
    }
    asm volatile("" ::"v"(acc));
}

}  // namespace smx
