"""GGUF files: the writer (smallmind_amd.gguf) and the backend's reader (smx_gguf_read_config,
the parsing half of smx_model_load_gguf), checked on the CPU.  The derived configuration
follows ModelConfig.FromGgufMetadata (ModelConfig.cs:142-214); the header / metadata / tensor
table layout follows GgufReader.ReadModelInfo (GgufReader.cs:39-102)."""
import struct

import numpy as np
import pytest

import oracle as O
from smallmind_amd import gguf as G
from smallmind_amd.model import ModelConfig
from tests.helpers import build_pair

CFG = ModelConfig("llama", 300, 96, 256, 2, 8, 2, 512, 500000.0, 1e-6)


def _tensors(cfg, lt=O.Q4_K, et=O.Q6_K, ht=O.Q6_K, seed=3):
    _, _, t = build_pair(cfg, lt, et, ht, seed=seed, with_gpu=False)
    return [(name, q, dims, data) for name, (q, dims, data) in t.items()]


def _read(path):
    from smallmind_amd.model import read_gguf_config
    return read_gguf_config(str(path))


def test_config_round_trip(tmp_path):
    p = tmp_path / "m.gguf"
    G.write_gguf(str(p), G.model_metadata(CFG), _tensors(CFG))
    got = _read(p)
    assert got == ModelConfig("llama", 300, 96, 256, 2, 8, 2, 512, 500000.0, np.float32(1e-6))


def test_gpt2_config_and_layer_norm_epsilon(tmp_path):
    cfg = ModelConfig("gpt2", 200, 64, 128, 1, 4, 4, 512, 10000.0, 1e-5)
    p = tmp_path / "g.gguf"
    G.write_gguf(str(p), G.model_metadata(cfg), _tensors(cfg, O.Q8_0, O.Q8_0, None))
    got = _read(p)
    assert (got.architecture, got.vocab_size, got.embedding_length, got.head_count_kv) == ("gpt2", 200, 128, 4)
    assert got.norm_eps == np.float32(1e-5)


def test_defaults_and_vocab_inference(tmp_path):
    """Without head_count_kv, feed_forward_length, rope.freq_base or an epsilon the defaults
    apply (head_count, 4 d, 10000, 1e-5); the vocabulary comes from tokenizer.ggml.tokens, or
    else from token_embd.weight; mistral* reads the llama keys."""
    base = [("general.architecture", G.STRING, "mistral-7b"), ("llama.context_length", G.U32, 96),
            ("llama.embedding_length", G.U32, 256), ("llama.block_count", G.U32, 2),
            ("llama.attention.head_count", G.U32, 8)]
    toks = [("tokenizer.ggml.tokens", G.ARRAY, (G.STRING, [f"t{i}" for i in range(77)]))]
    emb = [("token_embd.weight", O.Q8_0, (256, 123), np.zeros(123 * 8 * 34, np.uint8))]
    p = tmp_path / "a.gguf"
    G.write_gguf(str(p), base + toks, emb)
    got = _read(p)
    assert (got.architecture, got.vocab_size, got.head_count_kv, got.feed_forward_length) == ("llama", 77, 8, 1024)
    assert got.rope_freq_base == 10000.0 and got.norm_eps == np.float32(1e-5)
    G.write_gguf(str(p), base, emb)
    assert _read(p).vocab_size == 123


def test_alignment_padding_between_tensors(tmp_path):
    """A 301-row Q8_0 embedding (301 x 272 bytes) is not a multiple of the alignment, so the
    next tensor starts after padding; the tensor table is read to the end and the file size is
    the aligned data section plus every tensor padded to the alignment."""
    import ctypes

    from smallmind_amd import _lib
    cfg = ModelConfig("llama", 301, 96, 256, 2, 8, 2, 512)
    p = tmp_path / "pad.gguf"
    t = _tensors(cfg, O.Q8_0, O.Q8_0, O.Q8_0)
    sizes = [np.asarray(d).view(np.uint8).size for _, _, _, d in t]
    assert any(n % 64 for n in sizes)
    G.write_gguf(str(p), G.model_metadata(cfg), t, alignment=64)
    c = _lib.ModelConfigC()
    n = ctypes.c_int64()
    _lib.call("smx_gguf_read_config", str(p).encode(), ctypes.byref(c), ctypes.byref(n))
    assert n.value == len(t) and c.vocab == 301
    data = sum((k + 63) // 64 * 64 for k in sizes)
    assert (p.stat().st_size - data) % 64 == 0


@pytest.mark.parametrize("case", ["magic", "version", "arch", "truncated", "missing", "alignment", "missing_file"])
def test_malformed_files_are_rejected(tmp_path, case):
    from smallmind_amd._lib import SmxError
    p = tmp_path / f"{case}.gguf"
    meta = G.model_metadata(CFG)
    tens = _tensors(CFG)[:3]
    expect = -1
    if case == "magic":
        G.write_gguf(str(p), meta, tens)
        p.write_bytes(b"GGUX" + p.read_bytes()[4:])
    elif case == "version":
        G.write_gguf(str(p), meta, tens, version=1)
        expect = -5
    elif case == "arch":
        G.write_gguf(str(p), [("general.architecture", G.STRING, "bert")] + meta[1:], tens)
        expect = -5
    elif case == "truncated":
        G.write_gguf(str(p), meta, tens)
        raw = p.read_bytes()
        hdr = 4 + 4 + 8 + 8
        p.write_bytes(raw[:hdr + 40])   # inside the metadata
    elif case == "missing":
        G.write_gguf(str(p), [m for m in meta if not m[0].endswith("context_length")], tens)
    elif case == "alignment":
        raw_meta = [m for m in meta] + [("general.alignment", G.U32, 48)]
        # write_gguf sets its own alignment entry; patch the value in place
        G.write_gguf(str(p), raw_meta, tens, alignment=32)
        raw = bytearray(p.read_bytes())
        key = G._str("general.alignment") + struct.pack("<I", G.U32)
        i = raw.index(key) + len(key)
        raw[i:i + 4] = struct.pack("<I", 48)
        p.write_bytes(bytes(raw))
    else:
        p = tmp_path / "absent.gguf"
    with pytest.raises(SmxError) as e:
        _read(p)
    assert e.value.code == expect
