"""Benchmark: batch-1 greedy decode of the LLaMA-style 1.1B Q4_K model on one MI355X.

One step = one request of the configs[2] workload: a 512-token seeded prompt (prefilled
through the KV cache) and 256 greedy tokens, all on the device.  `value` is decode tokens/s
(GPU-event time of the token-producing steps).  The metric's kernel -- the fused Q4_K GEMV at
the gate/up shape (11264 x 2048), the largest weight stream of the decode step -- is then timed
on its own with HIP events around replays of a captured graph of launches over rotating weight
copies larger than the 256 MB MALL, giving the roofline figure, next to a plain streaming read of
the same bytes per launch and of 1 GiB per launch timed the same way (measured ceilings); the
configs[1] Q4_0 GEMV shapes are timed the same way.  The CPU baseline is the oracle on the same model at the same
positions: reference-faithful (fp32 weights dequantized at load, one thread) and on all cores.
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


MFMA_BF16_PEAK_TFLOPS = 2500.0


def layer_gemm_flops(cfg) -> float:
    """FLOPs of one token through the layer matrices (QKV, O, gate/up or up, down): 2 N K each."""
    d, kv, hid = cfg.embedding_length, cfg.kv_dim, cfg.hidden_dim
    gu = 2 * hid if cfg.architecture == "llama" else hid
    return 2.0 * cfg.block_count * ((d + 2 * kv) * d + d * d + gu * d + d * hid)


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


def stream_read_timing(n_bytes: int, min_bytes: int = 600 << 20, reps: int = 10):
    """The HBM streaming-read ceiling (smx_stream_read: 16-byte loads over the whole GPU, nothing
    written), timed like gemv_timing: HIP events around replays of a captured graph of launches
    that each read n_bytes of a different buffer, cycling over >= 600 MB."""
    import torch

    from smallmind_amd._lib import call
    n_bytes = (n_bytes + 15) // 16 * 16
    copies = max(2, min_bytes // n_bytes + 1)
    bufs = [torch.empty(n_bytes, dtype=torch.uint8, device="cuda").fill_(1) for _ in range(copies)]
    n_launch = max(copies, 64)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        for b in bufs:
            call("smx_stream_read", b.data_ptr(), n_bytes, s.cuda_stream)
        with torch.cuda.graph(g, stream=s):
            for i in range(n_launch):
                call("smx_stream_read", bufs[i % copies].data_ptr(), n_bytes, s.cuda_stream)
        g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            g.replay()
        e1.record(s)
    torch.cuda.synchronize()
    avg_s = e0.elapsed_time(e1) * 1e-3 / (reps * n_launch)
    del g, bufs
    return {"bytes": n_bytes, "avg_us": round(avg_s * 1e6, 3), "gbs": round(n_bytes / avg_s / 1e9, 1)}


def gemv_roofline():
    """The metric's kernel: the fused Q4_K GEMV at the gate/up shape (11264 x 2048)."""
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


# Decode GEMV shapes whose roofline fractions are tracked (label, GGUF type, rows N, cols K):
# the configs[2] Q4_K layer matrices and the configs[1] Q4_0 shapes.
GEMV_TRACKED = [("configs[2] QKV", 12, 2560, 2048), ("configs[2] O", 12, 2048, 2048),
                ("configs[2] gate/up", 12, 11264, 2048), ("configs[2] down", 12, 2048, 5632),
                ("configs[1]", 2, 4096, 4096), ("configs[1]", 2, 11008, 4096), ("configs[1]", 2, 4096, 11008)]


def gemv_shapes(launches: int):
    """--gemv-shapes: the fused dequant-GEMV (IWeightTensor.MatMul, m = 1) at GEMV_TRACKED, each
    launched over rotating weight copies (>= 600 MB, beyond the 256 MB MALL) so every launch
    streams its weights from HBM.  Launches are eager (no graph) so rocprofv3 counter passes see
    every dispatch; the HIP-event figure includes the launch gaps."""
    import torch

    from smallmind_amd.quantization import GpuWeightTensor, fill_normal, quantize, row_bytes
    for label, qt, N, K in GEMV_TRACKED:
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
        for i in range(launches):
            ws[i % copies].mat_mul(x, y, 1, K, N)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / launches
        print(f"{label:20s} type {qt:2d} {N:6d} x {K:5d}  {wbytes:9d} B  {us:7.2f} us per eager launch  "
              f"{wbytes / (us * 1e-6) / 1e9:7.1f} GB/s", flush=True)
        for w in ws:
            w.close()
        del ws


# Matrix-core GEMM shapes (label, GGUF type, layer matrices (name, N, K), token counts M): the
# 256-token chunk, the configs' prompt chunks (configs[2]: 511 tokens; configs[3]: 2048) and the
# 16-session lockstep step of configs[4].
_LLAMA_1B = [("qkv", 2560, 2048), ("o", 2048, 2048), ("gate_up", 11264, 2048), ("down", 2048, 5632)]
_SMOLLM_17B = [("qkv", 6144, 2048), ("o", 2048, 2048), ("gate_up", 16384, 2048), ("down", 2048, 8192)]
QGEMM_TRACKED = [("configs[2] Q4_K", 12, _LLAMA_1B, (256, 511)), ("configs[3] Q8_0", 8, _LLAMA_1B, (256, 2048)),
                 ("configs[4] Q5_K", 13, _SMOLLM_17B, (256, 16))]


def qgemm_shapes(reps: int):
    """--qgemm-shapes: the matrix-core GEMM (IWeightTensor.MatMul with m >= 4: k_qprep +
    k_qgemm_st) at QGEMM_TRACKED, eager launches with the weights resident; one line per shape
    with microseconds per call, useful TFLOP/s (2 M N K) and its fraction of the 2.5 PFLOP/s
    bf16 dense peak."""
    import torch

    from smallmind_amd.quantization import GpuWeightTensor, fill_normal, quantize
    for label, qt, shapes, ms in QGEMM_TRACKED:
        for name, N, K in shapes:
            w = GpuWeightTensor(qt, N, K, quantize(qt, fill_normal(N + K, N * K, 0.02)))
            for M in ms:
                x = torch.randn(M, K, device="cuda")
                y = torch.empty(M, N, device="cuda")
                for _ in range(3):
                    w.mat_mul(x, y, M, K, N)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(reps):
                    w.mat_mul(x, y, M, K, N)
                e1.record()
                torch.cuda.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / reps
                tf = 2.0 * M * N * K / (us * 1e-6) / 1e12
                print(f"{label:16s} {name:8s} M={M:5d} N={N:6d} K={K:5d}  {us:8.2f} us  {tf:7.2f} TFLOP/s  "
                      f"{tf / MFMA_BF16_PEAK_TFLOPS:.4f} of bf16 peak", flush=True)
            w.close()


def decode_step_bytes(wl, mean_pos: float) -> int:
    """Algorithmic HBM bytes of one decode step (one token for each of wl.sessions sessions): every
    layer matrix and the head once per step, one embedding row (and one learned-position row)
    per token -- the tables themselves are not streamed unless the head is tied to them -- all
    norm weights and biases, and each session's K/V of mean_pos positions (fp32)."""
    from smallmind_amd.quantization import row_bytes
    from smallmind_amd.synthetic import tensor_specs
    cfg = wl.config
    total = 0
    for s in tensor_specs(cfg, wl.layer_type, wl.embd_type, wl.head_type):
        if len(s.dims) == 1:
            total += 4 * s.n
        elif s.name in ("token_embd.weight", "position_embd.weight"):
            total += wl.sessions * row_bytes(s.qtype, s.dims[0])
            if s.name == "token_embd.weight" and wl.head_type is None:   # tied: the head reads it all
                total += s.dims[1] * row_bytes(s.qtype, s.dims[0])
        else:
            total += s.dims[1] * row_bytes(s.qtype, s.dims[0])
    kv_per_pos = 2 * cfg.block_count * cfg.head_count_kv * cfg.head_dim * 4
    return int(total + wl.sessions * kv_per_pos * mean_pos)


def mean_attended(wl) -> float:
    """Decode token i (0-based) sits at position prompt_len - 1 + i and attends to prompt_len + i
    positions; the mean over the new tokens."""
    return wl.prompt_len + (wl.new_tokens - 1) / 2


def other_configs():
    """configs[0], [3] and [4] measured on the same build: GPT-2-small Q8_0 decode; LLaMA-1.1B
    Q8_0 with a 4096-token prefill (matrix-core GEMM chunks) then decode at ~4.1K context; and
    SmolLM-1.7B Q5_K with 16 sessions (256-token prompts, 128 tokens each) in lockstep."""
    import numpy as np
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
        tok_s = wl.new_tokens / (st["decode_ms"] * 1e-3)
        step_bytes = decode_step_bytes(wl, mean_attended(wl))
        pre_tok_s = (wl.prompt_len - 1) / (st["prefill_ms"] * 1e-3)
        out[key] = {"prompt_len": wl.prompt_len, "new_tokens": wl.new_tokens,
                    "prefill_tok_s": round(pre_tok_s, 1),
                    "prefill_mfma_frac": round(layer_gemm_flops(wl.config) * pre_tok_s / 1e12
                                               / MFMA_BF16_PEAK_TFLOPS, 4),
                    "decode_tok_s": round(tok_s, 1),
                    "weight_bytes": int(model.weight_bytes()),
                    "bytes_per_token": step_bytes,
                    "decode_effective_gbs": round(step_bytes * tok_s / 1e9, 1),
                    "hbm_frac": round(step_bytes * tok_s / 1e9 / HBM_PEAK_GBS, 4),
                    "first_tokens": [int(t) for t in toks[:8]]}
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
    step_bytes = decode_step_bytes(wl, mean_attended(wl))
    step_s = st["decode_ms"] * 1e-3 / wl.new_tokens
    out["smollm-1.7b-q5_k"] = {
        "sessions": wl.sessions, "prompt_len": wl.prompt_len, "new_tokens": wl.new_tokens,
        "prefill_tok_s": round(st["prefill_steps"] / (st["prefill_ms"] * 1e-3), 1),
        "prefill_mfma_frac": round(layer_gemm_flops(wl.config) * st["prefill_steps"] / (st["prefill_ms"] * 1e-3)
                                   / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
        "decode_tok_s_aggregate": round(wl.sessions * wl.new_tokens / (st["decode_ms"] * 1e-3), 1),
        "decode_ms_per_step": round(st["decode_ms"] / wl.new_tokens, 4),
        "weight_bytes": int(model.weight_bytes()),
        "bytes_per_step": step_bytes,
        "decode_effective_gbs": round(step_bytes / step_s / 1e9, 1),
        "hbm_frac": round(step_bytes / step_s / 1e9 / HBM_PEAK_GBS, 4)}
    # the same 16 requests through the continuous batcher, one step per call as a serving loop
    # runs it (each call returns its tokens to the host before the next step is queued)
    import time

    from smallmind_amd.model import ContinuousBatcher
    log("other configs: smollm-1.7b-q5_k through the continuous batcher")
    b = ContinuousBatcher(model, wl.sessions, wl.prompt_len + wl.new_tokens)
    for x, p in zip(sess, prompts):
        b.add(x, p)
    got = [b.step(1) for _ in range(4)]                               # warmup (graph capture)
    n_steps = wl.new_tokens - 8
    t0 = time.perf_counter()
    for _ in range(n_steps):
        got.append(b.step(1))
    dt = time.perf_counter() - t0
    b.close()
    # the batcher's tokens are the lockstep run's (same prompts, same model)
    got = np.concatenate(got, axis=1)
    out["smollm-1.7b-q5_k"]["continuous_batcher_tokens_match_lockstep"] = bool(
        np.array_equal(got, toks[:, :got.shape[1]]))
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


def cpu_baseline(kept, wl, budget_s: float = 12.0):
    """The oracle on the host's cores, on the headline workload's positions: the 511 prompt
    tokens are prefilled (all cores, untimed), then decode steps from position 511 on are timed
    -- first the reference-faithful way (fp32 weights dequantized at load, the single-threaded
    M = 1 GEMV of MatMulOps.cs:1176), then on every core (the same fp32 arithmetic over all
    threads; not the reference's threading).
    Each mode runs about budget_s seconds."""
    import numpy as np

    import oracle as O
    from smallmind_amd.synthetic import prompt_tokens
    cfg = wl.config
    t0 = time.time()
    om = O.OracleModel(O.ARCH_LLAMA, cfg.vocab_size, cfg.context_length, cfg.embedding_length,
                       cfg.block_count, cfg.head_count, cfg.head_count_kv, cfg.feed_forward_length,
                       cfg.rope_freq_base, cfg.norm_eps)
    for name, (qt, dims, data) in kept.items():
        om.set_tensor(name, qt, data.cpu().numpy(), int(np.prod(dims)))
    om.finalize()
    load_s = time.time() - t0
    prompt = prompt_tokens(7, wl.prompt_len, cfg.vocab_size)
    n_all = O.get_threads()
    out = {}
    for mode, threads in (("reference", 1), ("all_cores", n_all)):
        O.set_threads(n_all)
        s = om.session(wl.prompt_len + 256)
        s.prefill(prompt[:-1], 0)
        O.set_threads(threads)
        tok, pos, n, t_dec = int(prompt[-1]), wl.prompt_len - 1, 0, 0.0
        while t_dec < budget_s and n < 256:
            t1 = time.perf_counter()
            tok = int(np.argmax(s.step(tok, pos)))
            t_dec += time.perf_counter() - t1
            pos += 1
            n += 1
        out[mode] = (n / t_dec, n, threads)
        del s
    O.set_threads(0)
    v, n, _ = out["reference"]
    va, na, ta = out["all_cores"]
    cpu = f"{platform.processor() or platform.machine()} x{os.cpu_count()} host"
    return {"value": round(v, 3), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"oracle on the same seeded configs[2] weights (fp32, dequantized at load in {load_s:.1f} s), "
                      f"the {wl.prompt_len - 1}-token prompt prefilled untimed, then {n} greedy decode steps "
                      f"at positions {wl.prompt_len - 1}..{wl.prompt_len - 2 + n} timed on one thread "
                      f"(the reference's single-threaded M=1 GEMV); {cpu}",
            "all_cores": {"value": round(va, 3), "unit": "tok/s", "cores": ta,
                          "sample": f"{na} decode steps from position {wl.prompt_len - 1}, linears and attention "
                                    f"over {ta} threads (same fp32 arithmetic; not the reference's threading)"}}


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
    ap.add_argument("--gemv-shapes", action="store_true",
                    help="time the fused GEMV at the tracked decode shapes (eager launches, for rocprofv3)")
    ap.add_argument("--qgemm-shapes", action="store_true",
                    help="time the matrix-core GEMM at the tracked prefill / lockstep shapes (eager launches)")
    ap.add_argument("--launches", type=int, default=200, help="launches per shape for --gemv-shapes")
    ap.add_argument("--reps", type=int, default=20, help="calls per shape for --qgemm-shapes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each box has one "
              "MI355X). A single session would shard as tensor parallelism (QKV and gate/up rows "
              "split, O and down split over K with two 8 KB all-reduces per layer); independent "
              "sessions as data parallelism.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    if args.copy_calibration:
        copy_calibration()
        return
    if args.gemv_shapes:
        gemv_shapes(args.launches)
        return
    if args.qgemm_shapes:
        qgemm_shapes(args.reps)
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
    token_bytes = decode_step_bytes(wl, mean_attended(wl))
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
        # matrix-core use of the prefill: useful GEMM FLOPs of the layer matrices (2 N K per
        # token) per second over the whole prefill time, against the 2.5 PFLOP/s bf16 dense peak
        "prefill_gemm_tflops": round(layer_gemm_flops(cfg) * pre_tok_s / 1e12, 2),
        "prefill_mfma_frac": round(layer_gemm_flops(cfg) * pre_tok_s / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
        "decode_ms_per_token": round(dec_ms / (args.steps * wl.new_tokens), 4),
        "decode_effective_gbs": round(token_bytes / (dec_ms * 1e-3 / (args.steps * wl.new_tokens)) / 1e9, 1),
        "bytes_per_token": int(token_bytes),
        "bytes_per_token_note": f"layers + head + one embedding row + norms + K/V at the mean attended "
                                f"position {mean_attended(wl):.1f}",
        "hbm_frac": round(token_bytes / (dec_ms * 1e-3 / (args.steps * wl.new_tokens)) / 1e9 / HBM_PEAK_GBS, 4),
        "first_tokens": [int(t) for t in tokens[:8]],
    }
    if not args.no_roofline:
        log("timing the dominant GEMV kernel")
        g = gemv_roofline()
        # the metric's kernel: the quantized GEMV (the decode step's largest byte stream)
        out["roofline"] = {"bound": "hbm", "achieved": round(g["gbs"], 1), "peak": HBM_PEAK_GBS,
                           "unit": "GB/s", "frac": round(g["gbs"] / HBM_PEAK_GBS, 4),
                           "traffic": traffic_from_profiles(),
                           "kernel": g["kernel"], "avg_us": round(g["avg_us"], 3),
                           "bytes_per_launch": g["bytes"]}
        # measured ceilings: a plain streaming read of the same bytes per launch (same launch
        # floor, same ramp) and of 1 GiB per launch (the sustained read rate)
        log("timing the streaming-read ceiling")
        same = stream_read_timing(g["bytes"])
        big = stream_read_timing(1 << 30, min_bytes=2 << 30, reps=3)
        out["roofline"]["read_ceiling"] = {
            "same_bytes": same, "one_gib": big,
            "frac_of_same_bytes_read": round(g["gbs"] / same["gbs"], 4),
            "frac_of_sustained_read": round(g["gbs"] / big["gbs"], 4)}
        log("timing the configs[1] Q4_0 GEMV shapes")
        out["c2_q4_0_gemv"] = c2_gemv_lines()
    sess.close()
    model.close()
    if not args.no_other_configs:
        out["other_configs"] = other_configs()
    if not args.no_cpu_baseline:
        log("timing the CPU baseline (oracle: one thread, then all cores)")
        out["cpu_baseline"] = cpu_baseline(kept, wl)
    del kept
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
