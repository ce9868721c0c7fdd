"""Committed golden vectors (tests/golden/, written by make_golden.py): the oracle must keep
reproducing them (CPU) and the GPU path must match them (gpu)."""
import hashlib
import os

import numpy as np
import pytest

import oracle as O
from tests.helpers import TYPES, rel_err

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


@pytest.mark.parametrize("name", list(TYPES))
def test_oracle_reproduces_dequant_golden(name):
    z = _load(f"dequant_{name}.npz")
    y = O.dequant(TYPES[name], z["blocks"], z["out"].size)
    assert np.array_equal(y.view(np.uint32), z["out"].view(np.uint32))
    assert hashlib.sha256(y.tobytes()).hexdigest() == str(z["sha256"])


def test_oracle_reproduces_gemv_golden():
    z = _load("gemv_Q4_0_256x512.npz")
    assert np.array_equal(O.gemv_f64(O.Q4_0, z["W"], 256, 512, z["x"]), z["y"])


def _tiny_tensors(z):
    out = {}
    for k in z.files:
        if k.startswith("q:"):
            name = k[2:]
            meta = z[k]
            out[name] = (int(meta[0]), tuple(int(v) for v in meta[1:]), z["t:" + name])
    return out


def test_oracle_reproduces_tiny_model_golden():
    z = _load("tiny_llama_8steps.npz")
    V, ctx, d, L, H, Hkv, ff = (int(v) for v in z["config"])
    om = O.OracleModel(O.ARCH_LLAMA, V, ctx, d, L, H, Hkv, ff)
    for name, (qt, dims, data) in _tiny_tensors(z).items():
        om.set_tensor(name, qt, data, int(np.prod(dims)))
    om.finalize()
    prompt = z["prompt"]
    full = om.forward_nocache(np.concatenate([prompt, z["tokens"][:-1]]), all_rows=True)
    for i in range(8):
        assert rel_err(full[len(prompt) - 1 + i], z["logits"][i]) < 1e-6


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(TYPES))
def test_gpu_dequant_golden(gpu, name):
    import torch

    from smallmind_amd.quantization import dequantize
    z = _load(f"dequant_{name}.npz")
    got = dequantize(TYPES[name], torch.from_numpy(z["blocks"]).cuda(), z["out"].size).cpu().numpy()
    assert hashlib.sha256(got.tobytes()).hexdigest() == str(z["sha256"])


@pytest.mark.gpu
def test_gpu_gemv_golden(gpu):
    import torch

    from smallmind_amd.quantization import GpuWeightTensor
    z = _load("gemv_Q4_0_256x512.npz")
    w = GpuWeightTensor(O.Q4_0, 256, 512, z["W"])
    y = torch.empty((1, 256), device="cuda")
    w.mat_mul(torch.from_numpy(z["x"]).cuda(), y, 1, 512, 256)
    assert rel_err(y.cpu().numpy()[0], z["y"]) < 2e-5
    w.close()


@pytest.mark.gpu
def test_gpu_tiny_model_golden(gpu):
    from smallmind_amd.model import GpuTransformerModel, ModelConfig
    z = _load("tiny_llama_8steps.npz")
    V, ctx, d, L, H, Hkv, ff = (int(v) for v in z["config"])
    gm = GpuTransformerModel(ModelConfig("llama", V, ctx, d, L, H, Hkv, ff))
    for name, (qt, dims, data) in _tiny_tensors(z).items():
        gm.load_tensor(name, qt, dims, data)
    gm.finalize()
    s = gm.create_session(16)
    toks, _, logits = s.generate_greedy(z["prompt"], 8, return_logits=True)
    assert list(toks) == list(z["tokens"])
    for i in range(8):
        assert rel_err(logits[i], z["logits"][i]) < 1e-3
    s.close()
    gm.close()
