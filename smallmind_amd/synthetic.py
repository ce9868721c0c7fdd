"""Synthetic workloads of the benchmark configurations (seeded weights, seeded prompts).

The reference initialises weights from a seeded generator (Tensor.cs:262-285) and quantizes
them with its own quantizer (Q8Tensor.Quantize / Q4Tensor.Quantize, the `quantize` CLI command
QuantizeCommand.cs:87-97).  Here each tensor is drawn N(0, 0.02) on the device with a per-tensor
seed and encoded on the device into GGUF blocks, then uploaded like a GGUF tensor.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from ._lib import F32, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0
from .model import ModelConfig


@dataclass
class TensorSpec:
    name: str
    qtype: int
    dims: tuple          # GGUF order: ne0 (fastest) first
    kind: str            # "weight" | "norm" | "bias"

    @property
    def n(self) -> int:
        return int(np.prod(self.dims))


@dataclass
class Workload:
    config: ModelConfig
    layer_type: int
    embd_type: int
    head_type: int | None      # None: output tied to token_embd
    prompt_len: int
    new_tokens: int
    sessions: int = 1


WORKLOADS = {
    # GPT-2-small, Q8_0 everywhere, tied head, 32-token prompt + 128 tokens
    "gpt2-small-q8_0": Workload(ModelConfig("gpt2", 50257, 1024, 768, 12, 12, 12, 3072),
                                Q8_0, Q8_0, None, 32, 128),
    # LLaMA-style 1.1B, Q4_K layers, Q6_K embedding and head, 512 + 256
    "llama-1.1b-q4_k": Workload(ModelConfig("llama", 32000, 2048, 2048, 22, 32, 4, 5632),
                                Q4_K, Q6_K, Q6_K, 512, 256),
    # same model, Q8_0 layers, Q6_K head, 4096 + 128
    "llama-1.1b-q8_0-4k": Workload(ModelConfig("llama", 32000, 4224, 2048, 22, 32, 4, 5632),
                                   Q8_0, Q6_K, Q6_K, 4096, 128),
    # SmolLM-style 1.7B, Q5_K, tied embeddings, 16 sessions x (256 + 128)
    "smollm-1.7b-q5_k": Workload(ModelConfig("llama", 49152, 2048, 2048, 24, 32, 32, 8192),
                                 Q5_K, Q5_K, None, 256, 128, sessions=16),
}

# isolated Q4_0 GEMV shapes (rows N, cols K)
GEMV_SHAPES = [(4096, 4096), (11008, 4096), (4096, 11008)]


def tensor_specs(cfg: ModelConfig, layer_type: int, embd_type: int, head_type: int | None):
    d, V, kv, hid = cfg.embedding_length, cfg.vocab_size, cfg.kv_dim, cfg.hidden_dim
    specs = [TensorSpec("token_embd.weight", embd_type, (d, V), "weight")]
    gpt2 = cfg.architecture == "gpt2"
    if gpt2:
        specs.append(TensorSpec("position_embd.weight", embd_type, (d, cfg.context_length), "weight"))
    for i in range(cfg.block_count):
        p = f"blk.{i}."
        specs.append(TensorSpec(p + "attn_norm.weight", F32, (d,), "norm"))
        if gpt2:
            specs.append(TensorSpec(p + "attn_norm.bias", F32, (d,), "bias0"))
            specs.append(TensorSpec(p + "attn_qkv.weight", layer_type, (d, d + 2 * kv), "weight"))
            specs.append(TensorSpec(p + "attn_qkv.bias", F32, (d + 2 * kv,), "bias"))
        else:
            specs.append(TensorSpec(p + "attn_q.weight", layer_type, (d, d), "weight"))
            specs.append(TensorSpec(p + "attn_k.weight", layer_type, (d, kv), "weight"))
            specs.append(TensorSpec(p + "attn_v.weight", layer_type, (d, kv), "weight"))
        specs.append(TensorSpec(p + "attn_output.weight", layer_type, (d, d), "weight"))
        if gpt2:
            specs.append(TensorSpec(p + "attn_output.bias", F32, (d,), "bias"))
        specs.append(TensorSpec(p + "ffn_norm.weight", F32, (d,), "norm"))
        if gpt2:
            specs.append(TensorSpec(p + "ffn_norm.bias", F32, (d,), "bias0"))
            specs.append(TensorSpec(p + "ffn_up.weight", layer_type, (d, hid), "weight"))
            specs.append(TensorSpec(p + "ffn_up.bias", F32, (hid,), "bias"))
        else:
            specs.append(TensorSpec(p + "ffn_gate.weight", layer_type, (d, hid), "weight"))
            specs.append(TensorSpec(p + "ffn_up.weight", layer_type, (d, hid), "weight"))
        specs.append(TensorSpec(p + "ffn_down.weight", layer_type, (hid, d), "weight"))
        if gpt2:
            specs.append(TensorSpec(p + "ffn_down.bias", F32, (d,), "bias"))
    specs.append(TensorSpec("output_norm.weight", F32, (d,), "norm"))
    if gpt2:
        specs.append(TensorSpec("output_norm.bias", F32, (d,), "bias0"))
    if head_type is not None:
        specs.append(TensorSpec("output.weight", head_type, (d, V), "weight"))
    return specs


def tensor_seed(seed: int, index: int) -> int:
    return (seed * 1000003 + index * 7919 + 1) & 0xFFFFFFFFFFFFFFFF


def load_synthetic_on_device(model, wl: Workload, seed: int, keep_blocks: bool = False):
    """Draws every tensor on the device, encodes it and uploads it to `model`.
    Returns {name: (qtype, dims, device uint8 blocks or fp32 vector)} when keep_blocks."""
    import torch

    from .quantization import fill_normal, quantize
    kept = {}
    specs = tensor_specs(wl.config, wl.layer_type, wl.embd_type, wl.head_type)
    for i, s in enumerate(specs):
        if s.kind == "norm":
            data = torch.ones(s.n, dtype=torch.float32, device="cuda")
        elif s.kind == "bias0":
            data = torch.zeros(s.n, dtype=torch.float32, device="cuda")
        elif s.kind == "bias":
            data = fill_normal(tensor_seed(seed, i), s.n, 0.02)
        else:
            x = fill_normal(tensor_seed(seed, i), s.n, 0.02)
            data = quantize(s.qtype, x)
            del x
        model.load_tensor(s.name, s.qtype, s.dims, data)
        if keep_blocks:
            kept[s.name] = (s.qtype, s.dims, data)
    model.finalize()
    return kept


def prompt_tokens(seed: int, n: int, vocab: int) -> np.ndarray:
    """Seeded uniform token ids."""
    return np.random.default_rng(seed).integers(0, vocab, size=n, dtype=np.int64).astype(np.int32)


__all__ = ["WORKLOADS", "GEMV_SHAPES", "Workload", "TensorSpec", "tensor_specs",
           "load_synthetic_on_device", "prompt_tokens", "tensor_seed", "Q4_0"]
