"""GGUF v3 writer for fixtures and model export.

Writes the layout GgufReader reads (GgufReader.cs:39-102): "GGUF", version 3, tensor and
metadata counts, metadata entries (GGUF string key, u32 value type, value), tensor entries
(name, n_dims, dims fastest first, GGML type, offset), and the data section at the next
multiple of general.alignment.  Each tensor starts at an offset aligned to that alignment (the
GGUF specification); with tensor sizes that are multiples of the alignment the offsets also
equal GgufReader's running sum of sizes (GgufReader.cs:94-100).  Reading is done by the
backend (smx_model_load_gguf / smx_gguf_read_config).
"""
from __future__ import annotations

import struct
from typing import Iterable

import numpy as np

# GGUF metadata value types (GgufValueType.cs)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
           U64: "<Q", I64: "<q", F64: "<d"}


def _str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, value) -> bytes:
    if vtype == STRING:
        return _str(value)
    if vtype == ARRAY:
        etype, items = value
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(_value(etype, x) for x in items)
    return struct.pack(_SCALAR[vtype], value)


def model_metadata(config, name: str = "smallmind-amd") -> list[tuple[str, int, object]]:
    """The metadata ModelConfig.FromGgufMetadata reads back (ModelConfig.cs:142-214) for a
    smallmind_amd.model.ModelConfig."""
    a = config.architecture
    eps_key = "attention.layer_norm_rms_epsilon" if a == "llama" else "attention.layer_norm_epsilon"
    return [("general.architecture", STRING, a), ("general.name", STRING, name),
            (f"{a}.vocab_size", U32, config.vocab_size), (f"{a}.context_length", U32, config.context_length),
            (f"{a}.embedding_length", U32, config.embedding_length), (f"{a}.block_count", U32, config.block_count),
            (f"{a}.feed_forward_length", U32, config.feed_forward_length),
            (f"{a}.attention.head_count", U32, config.head_count),
            (f"{a}.attention.head_count_kv", U32, config.head_count_kv),
            (f"{a}.rope.freq_base", F32, float(config.rope_freq_base)), (f"{a}.{eps_key}", F32, float(config.norm_eps))]


def write_gguf(path: str, metadata: Iterable[tuple[str, int, object]],
               tensors: Iterable[tuple[str, int, tuple, bytes | np.ndarray]], alignment: int = 32,
               version: int = 3) -> None:
    """metadata: (key, GGUF value type, value) -- arrays as (element type, list); tensors:
    (name, GGML type id, dims fastest first, raw block bytes or fp32 array)."""
    meta = [m for m in metadata if m[0] != "general.alignment"]
    meta.append(("general.alignment", U32, int(alignment)))
    tens = []
    for name, ttype, dims, data in tensors:
        raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1).tobytes() if isinstance(data, np.ndarray) else bytes(data)
        tens.append((name, int(ttype), tuple(int(d) for d in dims), raw))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tens), len(meta))
    head += b"".join(_str(k) + struct.pack("<I", t) + _value(t, v) for k, t, v in meta)
    offsets, off = [], 0
    for _, _, _, raw in tens:
        offsets.append(off)
        off = (off + len(raw) + alignment - 1) // alignment * alignment
    for (name, ttype, dims, _), o in zip(tens, offsets):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ttype, o)
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        for (_, _, _, raw), o in zip(tens, offsets):
            f.write(raw)
            f.write(b"\0" * ((-len(raw)) % alignment))
