"""Measurement probe: the fused dequant-GEMV (IWeightTensor.MatMul with m = 1) at the decode
shapes whose roofline fractions are tracked -- the configs[2] Q4_K layer matrices and the
configs[1] Q4_0 shapes -- each launched over rotating weight copies (>= 600 MB, beyond the
256 MB MALL) so that every launch streams its weights from HBM.  Launches are eager (no
graph) so that rocprofv3 counter passes see every dispatch; the HIP-event figure therefore
includes the launch gaps and reads above the kernel duration rocprofv3 reports.

    python smallmind_amd/probes/gemv_shapes.py [--launches 200]
"""
from __future__ import annotations

import argparse
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))

SHAPES = [("configs[2] QKV", 12, 2560, 2048), ("configs[2] O", 12, 2048, 2048),
          ("configs[2] gate/up", 12, 11264, 2048), ("configs[2] down", 12, 2048, 5632),
          ("configs[1]", 2, 4096, 4096), ("configs[1]", 2, 11008, 4096), ("configs[1]", 2, 4096, 11008)]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--launches", type=int, default=200)
    args = ap.parse_args()
    import torch

    from smallmind_amd.quantization import GpuWeightTensor, fill_normal, quantize, row_bytes
    for label, qt, N, K in SHAPES:
        wbytes = N * row_bytes(qt, K)
        copies = max(2, (600 << 20) // wbytes + 1)
        blocks = quantize(qt, fill_normal(N * 3 + K, N * K, 0.02))
        ws = [GpuWeightTensor(qt, N, K, blocks) for _ in range(copies)]
        del blocks
        x = torch.randn(K, device="cuda")
        y = torch.empty(N, device="cuda")
        for w in ws:
            w.mat_mul(x, y, 1, K, N)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(args.launches):
            ws[i % copies].mat_mul(x, y, 1, K, N)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / args.launches
        print(f"{label:20s} type {qt:2d} {N:6d} x {K:5d}  {wbytes:9d} B  {us:7.2f} us per eager launch  "
              f"{wbytes / (us * 1e-6) / 1e9:7.1f} GB/s", flush=True)
        for w in ws:
            w.close()
        del ws


if __name__ == "__main__":
    main()
