"""Benchmark: batch-1 greedy decode of the LLaMA-style 1.1B Q4_K model on one MI355X.

One step = one request of the configs[2] workload: a 512-token seeded prompt (prefilled
through the KV cache) and 256 greedy tokens, all on the device.  `value` is decode tokens/s
(GPU-event time of the token-producing steps).  The dominant kernel -- the fused gate/up
Q4_K GEMV (k_gemv<Q4_K,R=4>, 11264 x 2048) -- is then timed on its own with HIP events over
rotating weight copies larger than the 256 MB MALL, giving the roofline figure.  The CPU
baseline is the oracle's reference-faithful path (fp32 weights dequantized at load, one
thread) timed on a bounded sample of the same model.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "decode tok/s batch1 + quant GEMV HBM GB/s (% of peak), LLaMA-1B Q4_K"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gemv_roofline(n_iter: int = 200):
    """Times the gate/up-shaped fused Q4_K GEMV (11264 x 2048, x in LDS, RMSNorm-free store
    epilogue -- the same kernel instance) on the current stream over >512 MB of weights."""
    import torch

    from smallmind_amd.quantization import GpuWeightTensor, fill_normal, quantize
    N, K = 2 * 5632, 2048
    wbytes = N * (K // 256) * 144
    copies = max(2, (600 << 20) // wbytes + 1)
    blocks = quantize(12, fill_normal(3, N * K, 0.02))
    ws = [GpuWeightTensor(12, N, K, blocks) for _ in range(copies)]
    del blocks
    x = torch.randn(K, device="cuda")
    y = torch.empty(N, device="cuda")
    for w in ws:
        w.mat_mul(x, y, 1, K, N)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(n_iter):
        ws[i % copies].mat_mul(x, y, 1, K, N)
    e1.record()
    torch.cuda.synchronize()
    avg_s = e0.elapsed_time(e1) * 1e-3 / n_iter
    alg = wbytes + K * 4 + N * 4          # weights + activations in + outputs
    for w in ws:
        w.close()
    return {"kernel": "k_gemv<Q4_K,R=4> (fused dequant-GEMV, 11264x2048)", "avg_us": avg_s * 1e6,
            "bytes": alg, "gbs": alg / avg_s / 1e9, "copies": copies}


def cpu_baseline(kept, wl, budget_s: float = 15.0):
    import numpy as np

    import oracle as O
    cfg = wl.config
    t0 = time.time()
    om = O.OracleModel(O.ARCH_LLAMA, cfg.vocab_size, cfg.context_length, cfg.embedding_length,
                       cfg.block_count, cfg.head_count, cfg.head_count_kv, cfg.feed_forward_length,
                       cfg.rope_freq_base, cfg.norm_eps)
    for name, (qt, dims, data) in kept.items():
        om.set_tensor(name, qt, data.cpu().numpy(), int(np.prod(dims)))
    om.finalize()
    load_s = time.time() - t0
    prompt = np.arange(4, dtype=np.int32) * 97 % cfg.vocab_size
    _, _, dec1 = om.generate_greedy(prompt, 1)
    n = max(2, min(64, int(budget_s / max(dec1, 1e-3))))
    toks, pre, dec = om.generate_greedy(prompt, n)
    return {"value": n / dec, "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"same seeded configs[2] weights, fp32 dequantized at load ({load_s:.1f} s), "
                      f"4-token prompt then {n} greedy decode steps, single thread, "
                      f"{platform.processor() or platform.machine()} x{os.cpu_count()} host"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--workload", default="llama-1.1b-q4_k")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-roofline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each box has one "
              "MI355X; see DESIGN.md for how the path would shard).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from smallmind_amd.model import GpuTransformerModel
    from smallmind_amd.synthetic import WORKLOADS, load_synthetic_on_device, prompt_tokens
    wl = WORKLOADS[args.workload]
    cfg = wl.config
    log(f"building {args.workload} on device")
    model = GpuTransformerModel(cfg)
    kept = load_synthetic_on_device(model, wl, seed=42, keep_blocks=not args.no_cpu_baseline)
    wbytes = model.weight_bytes()
    max_ctx = wl.prompt_len + wl.new_tokens
    sess = model.create_session(max_ctx)
    prompt = prompt_tokens(7, wl.prompt_len, cfg.vocab_size)
    for i in range(args.warmup):
        sess.generate_greedy(prompt, wl.new_tokens)
        log(f"warmup {i + 1}/{args.warmup} done")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dec_ms = pre_ms = 0.0
    tokens = None
    for i in range(args.steps):
        tokens, st = sess.generate_greedy(prompt, wl.new_tokens)
        dec_ms += st["decode_ms"]
        pre_ms += st["prefill_ms"]
        log(f"step {i + 1}/{args.steps}: decode {st['decode_ms']:.1f} ms, prefill {st['prefill_ms']:.1f} ms")
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    dec_tok_s = args.steps * wl.new_tokens / (dec_ms * 1e-3)
    pre_tok_s = args.steps * (wl.prompt_len - 1) / (pre_ms * 1e-3)
    hd = cfg.head_dim
    mean_pos = wl.prompt_len + wl.new_tokens / 2
    kv_bytes = 2 * cfg.block_count * cfg.head_count_kv * hd * 4 * mean_pos
    token_bytes = wbytes + kv_bytes
    out = {
        "metric": METRIC, "value": round(dec_tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall * 1e3 / args.steps, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded N(0,0.02) weights encoded on device; seeded uniform prompt)",
        "config": {"workload": f"{args.workload}: configs[2] LLaMA-style 1.1B (22L, d2048, 32/4 heads, "
                               f"ff5632, V32000), Q4_K layers + Q6_K embedding/head, batch 1, "
                               f"{wl.prompt_len}-token prompt + {wl.new_tokens} greedy tokens",
                   "batch": 1, "prompt_len": wl.prompt_len, "new_tokens": wl.new_tokens},
        "prefill_tok_s": round(pre_tok_s, 2),
        "decode_ms_per_token": round(dec_ms / (args.steps * wl.new_tokens), 4),
        "decode_effective_gbs": round(token_bytes / (dec_ms * 1e-3 / (args.steps * wl.new_tokens)) / 1e9, 1),
        "bytes_per_token": int(token_bytes),
        "first_tokens": [int(t) for t in tokens[:8]],
    }
    if not args.no_roofline:
        log("timing the dominant GEMV kernel")
        g = gemv_roofline()
        out["roofline"] = {"bound": "hbm", "achieved": round(g["gbs"], 1), "peak": HBM_PEAK_GBS,
                           "unit": "GB/s", "frac": round(g["gbs"] / HBM_PEAK_GBS, 4), "traffic": None,
                           "kernel": g["kernel"], "avg_us": round(g["avg_us"], 3),
                           "bytes_per_launch": g["bytes"]}
    sess.close()
    if not args.no_cpu_baseline:
        log("timing the CPU baseline (oracle, one thread)")
        out["cpu_baseline"] = cpu_baseline(kept, wl)
    del kept
    model.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
