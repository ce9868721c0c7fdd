"""Benchmark: batch-1 greedy decode of the LLaMA-style 1.1B Q4_K model on one MI355X.

One step = one request of the configs[2] workload: a 512-token seeded prompt (prefilled
through the KV cache) and 256 greedy tokens, all on the device.  `value` is decode tokens/s
(GPU-event time of the token-producing steps).  The dominant kernel -- the fused Q4_K GEMV at
the gate/up shape (11264 x 2048) -- is then timed on its own with HIP events around replays of
a captured graph of launches over rotating weight copies larger than the 256 MB MALL, giving
the roofline figure; the configs[1] Q4_0 GEMV shapes are timed the same way.  The CPU
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


def gemv_timing(qt: int, N: int, K: int, seed: int, min_bytes: int = 600 << 20, reps: int = 10):
    """Average launch duration of the fused GEMV y = W x (smx_weight_matmul) for one [N, K]
    weight of block type `qt`, on the current torch stream, with HIP events around replays of a
    captured graph of back-to-back launches that cycle over enough distinct weight copies
    (>= 600 MB) to defeat the 256 MB MALL: every launch streams its weights from HBM."""
    import torch

    from smallmind_amd.quantization import GpuWeightTensor, fill_normal, quantize, row_bytes
    wbytes = N * row_bytes(qt, K)
    copies = max(2, min_bytes // wbytes + 1)
    blocks = quantize(qt, fill_normal(seed, N * K, 0.02))
    ws = [GpuWeightTensor(qt, N, K, blocks) for _ in range(copies)]
    del blocks
    x = torch.randn(K, device="cuda")
    y = torch.empty(N, device="cuda")
    n_launch = max(copies, 64)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        for w in ws:
            w.mat_mul(x, y, 1, K, N)
        with torch.cuda.graph(g, stream=s):
            for i in range(n_launch):
                ws[i % copies].mat_mul(x, y, 1, K, N)
        g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            g.replay()
        e1.record(s)
    torch.cuda.synchronize()
    avg_s = e0.elapsed_time(e1) * 1e-3 / (reps * n_launch)
    alg = wbytes + K * 4 + N * 4          # weights + activations in + outputs
    del g
    for w in ws:
        w.close()
    return {"avg_us": avg_s * 1e6, "bytes": alg, "gbs": alg / avg_s / 1e9, "copies": copies,
            "launches": reps * n_launch}


def gemv_roofline():
    """The dominant decode kernel: the fused Q4_K GEMV at the gate/up shape (11264 x 2048)."""
    g = gemv_timing(12, 2 * 5632, 2048, seed=3)
    g["kernel"] = "k_gemv<Q4_K,R=4,S=1> (fused dequant-GEMV, gate/up shape 11264x2048)"
    return g


def c2_gemv_lines():
    """configs[1] (C2): Q4_0 GEMV at the three reference shapes."""
    from smallmind_amd.synthetic import GEMV_SHAPES
    out = []
    for i, (N, K) in enumerate(GEMV_SHAPES):
        g = gemv_timing(2, N, K, seed=10 + i)
        out.append({"shape": [N, K], "avg_us": round(g["avg_us"], 3), "bytes": g["bytes"],
                    "gbs": round(g["gbs"], 1), "frac": round(g["gbs"] / HBM_PEAK_GBS, 4)})
    return out


def other_configs():
    """configs[0], [3] and [4] measured on the same build: GPT-2-small Q8_0 decode; LLaMA-1.1B
    Q8_0 with a 4096-token prefill (matrix-core GEMM chunks) then decode at ~4.1K context; and
    SmolLM-1.7B Q5_K with 16 sessions (256-token prompts, 128 tokens each) in lockstep."""
    import torch

    from smallmind_amd.model import GpuInferenceSession, GpuTransformerModel
    from smallmind_amd.synthetic import WORKLOADS, load_synthetic_on_device, prompt_tokens
    out = {}
    for key in ("gpt2-small-q8_0", "llama-1.1b-q8_0-4k"):
        wl = WORKLOADS[key]
        log(f"other configs: {key}")
        model = GpuTransformerModel(wl.config)
        load_synthetic_on_device(model, wl, seed=42, keep_blocks=False)
        sess = model.create_session(wl.prompt_len + wl.new_tokens)
        prompt = prompt_tokens(7, wl.prompt_len, wl.config.vocab_size)
        sess.generate_greedy(prompt, 8)                      # warmup
        toks, st = sess.generate_greedy(prompt, wl.new_tokens)
        out[key] = {"prompt_len": wl.prompt_len, "new_tokens": wl.new_tokens,
                    "prefill_tok_s": round((wl.prompt_len - 1) / (st["prefill_ms"] * 1e-3), 1),
                    "decode_tok_s": round(wl.new_tokens / (st["decode_ms"] * 1e-3), 1),
                    "weight_bytes": int(model.weight_bytes())}
        sess.close()
        model.close()
        torch.cuda.synchronize()
    wl = WORKLOADS["smollm-1.7b-q5_k"]
    log("other configs: smollm-1.7b-q5_k (16 sessions in lockstep)")
    model = GpuTransformerModel(wl.config)
    load_synthetic_on_device(model, wl, seed=42, keep_blocks=False)
    sess = [model.create_session(wl.prompt_len + wl.new_tokens) for _ in range(wl.sessions)]
    prompts = [prompt_tokens(100 + i, wl.prompt_len, wl.config.vocab_size) for i in range(wl.sessions)]
    GpuInferenceSession.generate_greedy_batch(sess, prompts, 8)        # warmup
    toks, st = GpuInferenceSession.generate_greedy_batch(sess, prompts, wl.new_tokens)
    out["smollm-1.7b-q5_k"] = {
        "sessions": wl.sessions, "prompt_len": wl.prompt_len, "new_tokens": wl.new_tokens,
        "prefill_tok_s": round(st["prefill_steps"] / (st["prefill_ms"] * 1e-3), 1),
        "decode_tok_s_aggregate": round(wl.sessions * wl.new_tokens / (st["decode_ms"] * 1e-3), 1),
        "decode_ms_per_step": round(st["decode_ms"] / wl.new_tokens, 4),
        "weight_bytes": int(model.weight_bytes())}
    # the same 16 requests through the continuous batcher, one step per call as a serving loop
    # runs it (each call returns its tokens to the host before the next step is queued)
    import time

    from smallmind_amd.model import ContinuousBatcher
    log("other configs: smollm-1.7b-q5_k through the continuous batcher")
    b = ContinuousBatcher(model, wl.sessions, wl.prompt_len + wl.new_tokens)
    for x, p in zip(sess, prompts):
        b.add(x, p)
    for _ in range(4):
        b.step(1)                                                     # warmup (graph capture)
    n_steps = wl.new_tokens - 8
    t0 = time.perf_counter()
    for _ in range(n_steps):
        b.step(1)
    dt = time.perf_counter() - t0
    b.close()
    out["smollm-1.7b-q5_k"]["continuous_batcher_ms_per_step"] = round(dt * 1e3 / n_steps, 4)
    out["smollm-1.7b-q5_k"]["continuous_batcher_tok_s_aggregate"] = round(wl.sessions * n_steps / dt, 1)
    for x in sess:
        x.close()
    model.close()
    return out


PMC_SUMMARY = os.path.join(ROOT, "profiles", "gemv_q4k_11264x2048_pmc.md")


def traffic_from_profiles():
    """HBM bytes per launch of the roofline kernel from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by what the counter reads for a plain
    copy kernel of known size), or None when no summary is present."""
    if not os.path.exists(PMC_SUMMARY):
        return None
    with open(PMC_SUMMARY) as f:
        for line in f:
            if line.startswith("hbm_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    return None


def copy_calibration(n_bytes: int = 1 << 30, reps: int = 5):
    """A plain device copy of known size (reads n_bytes, writes n_bytes per launch), run under
    rocprofv3 --pmc to scale FETCH_SIZE / WRITE_SIZE to bytes."""
    import torch
    a = torch.empty(n_bytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n_bytes, "copy_bytes_written": n_bytes, "launches": reps}),
          flush=True)


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
    ap.add_argument("--roofline-only", action="store_true",
                    help="time only the dominant GEMV kernel (for rocprofv3 --pmc passes)")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the configs[0]/[3]/[4] measurements")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run a 1 GiB device copy (counter calibration for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each box has one "
              "MI355X; see DESIGN.md for how the path would shard).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    if args.copy_calibration:
        copy_calibration()
        return
    if args.roofline_only:
        g = gemv_roofline()
        print(json.dumps({"roofline_kernel": g["kernel"], "avg_us": round(g["avg_us"], 3),
                          "bytes_per_launch": g["bytes"], "gbs": round(g["gbs"], 1),
                          "launches": g["launches"]}), flush=True)
        return

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
                           "unit": "GB/s", "frac": round(g["gbs"] / HBM_PEAK_GBS, 4),
                           "traffic": traffic_from_profiles(),
                           "kernel": g["kernel"], "avg_us": round(g["avg_us"], 3),
                           "bytes_per_launch": g["bytes"]}
        log("timing the configs[1] Q4_0 GEMV shapes")
        out["c2_q4_0_gemv"] = c2_gemv_lines()
    sess.close()
    model.close()
    if not args.no_other_configs:
        out["other_configs"] = other_configs()
    if not args.no_cpu_baseline:
        log("timing the CPU baseline (oracle, one thread)")
        out["cpu_baseline"] = cpu_baseline(kept, wl)
    del kept
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
