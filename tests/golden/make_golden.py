"""Writes the committed golden vectors under tests/golden/ from the CPU oracle.

The reference holds no golden vectors for this path (its K-quant value tests are skipped and
its golden logits are placeholders), so these fixtures freeze the oracle's outputs once the
oracle has been pinned by tests/test_oracle.py; both the oracle (regression) and the GPU path
(parity) are checked against them.

    python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402
from tests.helpers import TYPES, random_blocks  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main():
    for name, qt in TYPES.items():
        b = random_blocks(qt, 64, 1000 + qt)
        n = 64 * O.BLOCK_ELEMS[qt]
        y = O.dequant(qt, b, n)
        np.savez_compressed(os.path.join(HERE, f"dequant_{name}.npz"), blocks=b, out=y,
                            sha256=np.array(sha(y)))
    rng = np.random.default_rng(2024)
    N, K = 256, 512
    W = O.quantize(O.Q4_0, rng.normal(0, 0.02, N * K).astype(np.float32))
    x = rng.normal(0, 1, K).astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "gemv_Q4_0_256x512.npz"), W=W, x=x,
                        y=O.gemv_f64(O.Q4_0, W, N, K, x))

    # tiny llama-style model: 2 layers, d=64, 4 heads / 2 KV heads, ff=128, V=128, Q4_K
    # layers + Q6_K head would need K >= 256, so the tiny model uses Q8_0 / Q4_0 blocks.
    cfg = dict(vocab=128, ctx=32, d=64, L=2, H=4, Hkv=2, ff=128)
    om = O.OracleModel(O.ARCH_LLAMA, cfg["vocab"], cfg["ctx"], cfg["d"], cfg["L"], cfg["H"],
                       cfg["Hkv"], cfg["ff"])
    tensors = {}
    d, kv, ff, V = cfg["d"], cfg["d"] // cfg["H"] * cfg["Hkv"], cfg["ff"], cfg["vocab"]
    spec = [("token_embd.weight", O.Q8_0, (d, V)), ("output.weight", O.Q4_0, (d, V)),
            ("output_norm.weight", O.F32, (d,))]
    for i in range(cfg["L"]):
        p = f"blk.{i}."
        spec += [(p + "attn_norm.weight", O.F32, (d,)), (p + "attn_q.weight", O.Q8_0, (d, d)),
                 (p + "attn_k.weight", O.Q8_0, (d, kv)), (p + "attn_v.weight", O.Q8_0, (d, kv)),
                 (p + "attn_output.weight", O.Q4_0, (d, d)), (p + "ffn_norm.weight", O.F32, (d,)),
                 (p + "ffn_gate.weight", O.Q8_0, (d, ff)), (p + "ffn_up.weight", O.Q8_0, (d, ff)),
                 (p + "ffn_down.weight", O.Q4_0, (ff, d))]
    rng = np.random.default_rng(77)
    arrays = {}
    for name, qt, dims in spec:
        n = int(np.prod(dims))
        if qt == O.F32:
            data = rng.normal(1.0, 0.1, n).astype(np.float32)
        else:
            data = O.quantize(qt, rng.normal(0, 0.05, n).astype(np.float32))
        om.set_tensor(name, qt, data, n)
        tensors[name] = (qt, dims)
        arrays["t:" + name] = data.view(np.uint8)
        arrays["q:" + name] = np.array([qt, *dims], np.int64)
    om.finalize()
    prompt = rng.integers(0, V, 6).astype(np.int32)
    sess = om.session(16)
    for p_, t in enumerate(prompt[:-1]):
        sess.step(int(t), p_, want_logits=False)
    tok, logits, toks = int(prompt[-1]), [], []
    for i in range(8):
        lg = sess.step(tok, len(prompt) - 1 + i)
        logits.append(lg)
        tok = O.lib().smxo_argmax(lg.ctypes.data_as(__import__("ctypes").c_void_p), V)
        toks.append(tok)
    np.savez_compressed(os.path.join(HERE, "tiny_llama_8steps.npz"), prompt=prompt,
                        logits=np.stack(logits), tokens=np.array(toks, np.int32),
                        config=np.array([cfg[k] for k in ("vocab", "ctx", "d", "L", "H", "Hkv", "ff")]),
                        **arrays)
    print("golden vectors written to", HERE)


if __name__ == "__main__":
    main()
