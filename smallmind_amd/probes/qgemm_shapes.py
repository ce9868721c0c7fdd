"""Measurement probe: the matrix-core GEMM (IWeightTensor.MatMul with m >= 4 -> k_qprep +
k_qgemm_st) at the layer shapes of the prefill chunks (256 tokens, and the 511 / 2048-token
chunks of the configs[2] / configs[3] prompts) and of the 16-session lockstep decode, for the block formats of configs[2] (Q4_K), configs[3] (Q8_0) and configs[4]
(Q5_K).  Launches are eager (no graph) so that rocprofv3 counter passes see every dispatch.

Prints one line per shape: microseconds per call (HIP events over `--reps` calls, weights
resident), useful TFLOP/s (2 M N K per call) and its fraction of the 2.5 PFLOP/s bf16 dense
peak.

    python smallmind_amd/probes/qgemm_shapes.py [--reps 20]
"""
from __future__ import annotations

import argparse
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))

# (label, GGUF type, rows N, cols K): the four layer matrices of each model
LLAMA_1B = [("qkv", 2560, 2048), ("o", 2048, 2048), ("gate_up", 11264, 2048), ("down", 2048, 5632)]
SMOLLM_17B = [("qkv", 6144, 2048), ("o", 2048, 2048), ("gate_up", 16384, 2048), ("down", 2048, 8192)]
# M: 256-token chunks, the prefill chunks of the configs' prompts (configs[2]: 511 tokens in one
# chunk; configs[3]: 2048-token chunks) and the 16-session lockstep step
CASES = ([("configs[2] Q4_K", 12, LLAMA_1B, (256, 511)), ("configs[3] Q8_0", 8, LLAMA_1B, (256, 2048)),
          ("configs[4] Q5_K", 13, SMOLLM_17B, (256, 16))])


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=20)
    args = ap.parse_args()
    import torch

    from smallmind_amd.quantization import GpuWeightTensor, fill_normal, quantize
    for label, qt, shapes, ms in CASES:
        for name, N, K in shapes:
            w = GpuWeightTensor(qt, N, K, quantize(qt, fill_normal(N + K, N * K, 0.02)))
            for M in ms:
                x = torch.randn(M, K, device="cuda")
                y = torch.empty(M, N, device="cuda")
                for _ in range(3):
                    w.mat_mul(x, y, M, K, N)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(args.reps):
                    w.mat_mul(x, y, M, K, N)
                e1.record()
                torch.cuda.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / args.reps
                tf = 2.0 * M * N * K / (us * 1e-6) / 1e12
                print(f"{label:16s} {name:8s} M={M:5d} N={N:6d} K={K:5d}  {us:8.2f} us  {tf:7.2f} TFLOP/s  "
                      f"{tf / 2500.0:.4f} of bf16 peak", flush=True)
            w.close()


if __name__ == "__main__":
    main()
