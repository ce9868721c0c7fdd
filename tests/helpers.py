"""Shared builders for the parity tests: one set of seeded GGUF bytes feeds both the CPU oracle
and the GPU backend."""
from __future__ import annotations

import numpy as np

import oracle as O
from oracle import smq as OS
from smallmind_amd import smq as S

TYPES = {"Q4_0": O.Q4_0, "Q8_0": O.Q8_0, "Q4_K": O.Q4_K, "Q5_K": O.Q5_K, "Q6_K": O.Q6_K}
# every weight-matrix format of the backend: the GGUF blocks, SmallMind's SMQ blocks and the
# unquantized F16 / F32 matrices
ALL_TYPES = dict(TYPES, SMQ_Q8=O.SMQ_Q8, SMQ_Q4=O.SMQ_Q4, F16=O.F16, F32=O.F32)


def random_blocks(qtype: int, nblocks: int, seed: int) -> np.ndarray:
    """Random bytes for every field, with the fp16 scale fields forced finite (the reference's
    HalfToFloat keeps NaN payloads, which no fp32 product reproduces bit-for-bit)."""
    rng = np.random.default_rng(seed)
    if qtype == O.F32:   # finite values over a wide range of magnitudes
        v = rng.normal(0, 1, nblocks) * np.exp2(rng.integers(-30, 30, nblocks))
        return v.astype(np.float32).view(np.uint8)
    bb = O.BLOCK_BYTES[qtype]
    b = rng.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)
    if qtype == O.F16:   # every finite half pattern
        h = b.reshape(-1).view(np.uint16)
        h[(h & 0x7C00) == 0x7C00] &= 0xBBFF
        return b.reshape(-1)
    if qtype in (O.SMQ_Q8, O.SMQ_Q4):   # random codes, finite fp32 scales of moderate size
        sc = (rng.normal(0, 1, nblocks) * np.exp2(rng.integers(-12, 4, nblocks))).astype(np.float32)
        b[:, :4] = sc.view(np.uint8).reshape(nblocks, 4)
        return b.reshape(-1)

    def finite_half(col):
        h = b[:, col].astype(np.uint16) | (b[:, col + 1].astype(np.uint16) << 8)
        bad = (h & 0x7C00) == 0x7C00
        h = np.where(bad, h & 0xBBFF, h)   # clear one exponent bit
        b[:, col] = (h & 0xFF).astype(np.uint8)
        b[:, col + 1] = (h >> 8).astype(np.uint8)

    if qtype in (O.Q4_0, O.Q8_0, O.Q4_K, O.Q5_K):
        finite_half(0)
    if qtype in (O.Q4_K, O.Q5_K):
        finite_half(2)
    if qtype == O.Q6_K:
        finite_half(208)
    return b.reshape(-1)


def quantized(qtype: int, shape, seed: int, std: float = 0.02):
    x = np.random.default_rng(seed).normal(0.0, std, size=int(np.prod(shape))).astype(np.float32)
    return O.quantize(qtype, x)


def model_specs(cfg, layer_type, embd_type, head_type):
    from smallmind_amd.synthetic import tensor_specs
    return tensor_specs(cfg, layer_type, embd_type, head_type)


def build_pair(cfg, layer_type, embd_type, head_type, seed=1234, random_norms=True, with_gpu=True):
    """Returns (oracle_model, gpu_model or None, {name: (qtype, dims, host bytes)})."""
    rng = np.random.default_rng(seed)
    arch = O.ARCH_GPT2 if cfg.architecture == "gpt2" else O.ARCH_LLAMA
    om = O.OracleModel(arch, cfg.vocab_size, cfg.context_length, cfg.embedding_length,
                       cfg.block_count, cfg.head_count, cfg.head_count_kv, cfg.feed_forward_length,
                       cfg.rope_freq_base, cfg.norm_eps)
    gm = None
    if with_gpu:
        from smallmind_amd.model import GpuTransformerModel
        gm = GpuTransformerModel(cfg)
    tensors = {}
    for s in model_specs(cfg, layer_type, embd_type, head_type):
        if s.kind == "norm":
            data = (rng.normal(1.0, 0.1, s.n) if random_norms else np.ones(s.n)).astype(np.float32)
        elif s.kind == "bias0":
            data = (rng.normal(0.0, 0.05, s.n) if random_norms else np.zeros(s.n)).astype(np.float32)
        elif s.kind == "bias":
            data = rng.normal(0.0, 0.02, s.n).astype(np.float32)
        else:
            data = O.quantize(s.qtype, rng.normal(0.0, 0.02, s.n).astype(np.float32))
        om.set_tensor(s.name, s.qtype, data, s.n)
        if gm is not None:
            gm.load_tensor(s.name, s.qtype, s.dims, data)
        tensors[s.name] = (s.qtype, s.dims, data)
    om.finalize()
    if gm is not None:
        gm.finalize()
    return om, gm, tensors


def rel_err(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def oracle_from_kept(cfg, kept):
    """The oracle model of a GPU model built by load_synthetic_on_device(keep_blocks=True): the
    same device-encoded bytes, copied to the host."""
    arch = O.ARCH_GPT2 if cfg.architecture == "gpt2" else O.ARCH_LLAMA
    om = O.OracleModel(arch, cfg.vocab_size, cfg.context_length, cfg.embedding_length,
                       cfg.block_count, cfg.head_count, cfg.head_count_kv, cfg.feed_forward_length,
                       cfg.rope_freq_base, cfg.norm_eps)
    for name, (qt, dims, data) in kept.items():
        om.set_tensor(name, qt, data.cpu().numpy(), int(np.prod(dims)))
    om.finalize()
    return om


def check_greedy_against_oracle(osess, prompt, toks, logits, tol, prefilled=False):
    """Walks the oracle session through the GPU run: every step's logits within tol
    (max|d| / max|ref|) and every greedy token identical.  Returns the worst error."""
    if not prefilled and len(prompt) > 1:
        osess.prefill(prompt[:-1], 0)
    tok, worst = int(prompt[-1]), 0.0
    for i in range(len(toks)):
        ref = osess.step(tok, len(prompt) - 1 + i)
        err = rel_err(logits[i], ref)
        worst = max(worst, err)
        assert err <= tol, (i, err)
        ref_tok = int(np.argmax(ref))
        assert int(toks[i]) == ref_tok, (i, int(toks[i]), ref_tok)
        tok = ref_tok
    return worst


def gpt2_smq_tensors(cfg, scheme, block, seed, named):
    """A GPT-2 TransformerModel's parameters quantized as the SMQ tools do (every parameter,
    1-D ones as [1][n]), in parameter order."""
    rng = np.random.default_rng(seed)
    d, V, T, hid = cfg.embedding_length, cfg.vocab_size, cfg.context_length, 4 * cfg.embedding_length
    shapes = [(V, d), (T, d)]
    for _ in range(cfg.block_count):
        shapes += [(1, d), (1, d), (3 * d, d), (1, 3 * d), (d, d), (1, d), (1, d), (1, d), (hid, d), (1, hid),
                   (d, hid), (1, d)]
    shapes += [(1, d), (1, d), (V, d)]
    names = OS.gpt2_parameter_names(cfg.block_count)
    out = []
    for i, (shp, name) in enumerate(zip(shapes, names)):
        n = shp[0] * shp[1]
        if name.endswith("norm.weight"):
            x = rng.normal(1.0, 0.1, n)
        elif name.endswith(".bias"):
            x = rng.normal(0.0, 0.05, n)
        else:
            x = rng.normal(0.0, 0.02, n)
        q, sc = (O.quantize_ref_q8 if scheme == S.Q8_0 else O.quantize_ref_q4)(x.astype(np.float32), block)
        out.append(S.SmqTensor(name if named else f"param_{i:04d}", scheme, shp, q, sc, block))
    return out


def c_consumer() -> str:
    """The C99 consumer of the C-ABI (tests/capi/smx_consumer.c), which the build links next to
    libsmx.so; built here (gcc) if it is absent."""
    import importlib.util
    import os
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    path = os.path.join(root, "tests", "capi", "smx_consumer")
    if not os.path.exists(path):
        spec = importlib.util.spec_from_file_location("smx_build", os.path.join(root, "smallmind_amd", "build.py"))
        b = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(b)
        b.build_consumer()
    return path
