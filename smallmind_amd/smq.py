"""SmallMind .smq writer for model export and fixtures.

Writes the layout SmqWriter.WriteModel writes (src/SmallMind.Quantization/IO/Smq/SmqWriter.cs;
format in SmqFormat.cs:15-121): "SMQv0001", u32 version 1, u32 header size 32, u32 tensor
count, u32 metadata JSON length, u64 reserved; the UTF-8 JSON metadata; one 156-byte entry per
tensor (name padded to 64 bytes, u32 data type, i32 rank, i32 dims[8], u32 block size, u64 data
offset / length, u64 aux offset / length, 16 reserved bytes); then each tensor's data followed by
its scales (aux), in directory order, starting right after the directory.  Reading is done by
the backend (smx_model_load_smq / smx_smq_read_config).
"""
from __future__ import annotations

import json
import struct
from dataclasses import dataclass
from typing import Iterable

import numpy as np

F32, F16, Q8_0, Q4_0 = 1, 2, 10, 11   # QuantScheme ids (src/SmallMind.Quantization/Tensors/QuantScheme.cs)
_ENTRY = struct.Struct("<64sIi8iIQQQQ16x")


@dataclass
class SmqTensor:
    """One directory entry.  Q8_0: `data` holds rows*cols int8 codes; Q4_0: (rows*cols+1)//2
    bytes of two's-complement nibbles, element 2i in the low nibble (Q4Tensor.cs:17-62); both
    with one fp32 scale per `block_size` consecutive elements.  F32: `data` the float32 values,
    `scales` None."""
    name: str
    scheme: int
    dims: tuple
    data: np.ndarray
    scales: np.ndarray | None = None
    block_size: int = 0

    def payload(self) -> tuple[bytes, bytes]:
        n = int(np.prod(self.dims))
        if self.scheme == F32:
            d = np.ascontiguousarray(self.data, np.float32).reshape(-1)
            if d.size != n:
                raise ValueError(f"{self.name}: {d.size} values for dims {self.dims}")
            return d.tobytes(), b""
        if self.scheme not in (Q8_0, Q4_0):
            raise ValueError(f"{self.name}: scheme {self.scheme} is not written")
        if len(self.dims) != 2 or self.block_size <= 0:
            raise ValueError(f"{self.name}: quantized tensors are rank 2 with a positive block size")
        d = np.ascontiguousarray(self.data).view(np.uint8).reshape(-1)
        want = n if self.scheme == Q8_0 else (n + 1) // 2
        sc = np.ascontiguousarray(self.scales, np.float32).reshape(-1)
        if d.size != want or sc.size != -(-n // self.block_size):
            raise ValueError(f"{self.name}: {d.size} data bytes / {sc.size} scales for dims {self.dims}")
        return d.tobytes(), sc.tobytes()


def write_smq(path: str, tensors: Iterable[SmqTensor], metadata: dict | None = None) -> int:
    """Writes the tensors in the given order; returns the file size."""
    tensors = list(tensors)
    meta = json.dumps(metadata, separators=(",", ":")).encode("utf-8") if metadata else b""
    payloads = [t.payload() for t in tensors]
    off = 32 + len(meta) + _ENTRY.size * len(tensors)
    entries = []
    for t, (d, a) in zip(tensors, payloads):
        name = t.name.encode("utf-8")
        if len(name) > 63 or len(t.dims) > 8:
            raise ValueError(f"{t.name}: name longer than 63 bytes or rank above 8")
        dims = list(t.dims) + [0] * (8 - len(t.dims))
        doff = off
        aoff = off + len(d) if a else 0
        off += len(d) + len(a)
        entries.append(_ENTRY.pack(name, t.scheme, len(t.dims), *dims, t.block_size, doff, len(d), aoff, len(a)))
    with open(path, "wb") as f:
        f.write(b"SMQv0001" + struct.pack("<IIIIQ", 1, 32, len(tensors), len(meta), 0))
        f.write(meta)
        for e in entries:
            f.write(e)
        for d, a in payloads:
            f.write(d)
            f.write(a)
        return f.tell()


def gpt2_metadata(config, name: str = "smallmind-amd") -> dict:
    """The metadata keys the SMQ tools write for a GPT-2 TransformerModel (string values, as
    CreateBenchmarkModel does) from a smallmind_amd.model.ModelConfig."""
    return {"model_name": name, "format_version": "1", "vocab_size": str(config.vocab_size),
            "block_size": str(config.context_length), "embed_dim": str(config.embedding_length),
            "num_layers": str(config.block_count), "num_heads": str(config.head_count)}
