"""SmallMind .smq files on the CPU: the checker's own reader and model loader.

TEST INFRASTRUCTURE ONLY.  Imported by tests/ as the checker for the backend's SMQ loader
(smx_model_load_smq); the product package never imports it.

Restates SmqReader (src/SmallMind.Quantization/IO/Smq/SmqReader.cs:33-293; layout in
SmqFormat.cs:15-121) and SmqModelLoader.LoadWeights (src/SmallMind.Runtime/SmqModelLoader.cs:
119-205): header, JSON metadata, 156-byte tensor entries, Q8/Q4 payloads dequantized with
Q8Tensor.Dequantize / Q4Tensor.Dequantize (oracle.dequant_smq), F32 payloads as stored.
"""
from __future__ import annotations

import json
import struct

import numpy as np

from . import ARCH_GPT2, F32, OracleModel, dequant_smq

MAGIC = b"SMQv0001"
ENTRY = struct.Struct("<64sIi8iIQQQQ16x")   # SmqFormat.TensorEntry: 156 bytes
SCHEME_F32, SCHEME_F16, SCHEME_Q8, SCHEME_Q4 = 1, 2, 10, 11   # QuantScheme.cs


class SmqError(ValueError):
    pass


def read_smq(data: bytes):
    """Returns (metadata dict, [entry dict]) with each entry's dims, scheme, block size and
    its values dequantized to float32 (flattened, row-major over dims)."""
    if len(data) < 32 or data[:8] != MAGIC:
        raise SmqError("Invalid magic header")
    version, hsize, count, mlen, _ = struct.unpack_from("<IIIIQ", data, 8)
    if version != 1:
        raise SmqError(f"Unsupported format version {version}")
    if hsize != 32 or 32 + mlen > len(data):
        raise SmqError("truncated header")
    meta = json.loads(data[32:32 + mlen].decode("utf-8")) if mlen else {}
    off = 32 + mlen
    if off + count * ENTRY.size > len(data):
        raise SmqError("truncated tensor directory")
    out = []
    for i in range(count):
        f = ENTRY.unpack_from(data, off + i * ENTRY.size)
        name = f[0].split(b"\0", 1)[0].decode("utf-8")
        scheme, rank = f[1], f[2]
        dims = tuple(f[3:3 + rank])
        block, doff, dlen, aoff, alen = f[11], f[12], f[13], f[14], f[15]
        if doff + dlen > len(data) or aoff + alen > len(data):
            raise SmqError(f"{name}: data beyond the end of the file")
        n = int(np.prod(dims)) if dims else 0
        raw = np.frombuffer(data, np.uint8, dlen, doff)
        if scheme == SCHEME_F32:
            if dlen != 4 * n:
                raise SmqError(f"{name}: F32 length")
            vals = raw.view(np.float32).copy()
        elif scheme in (SCHEME_Q8, SCHEME_Q4):
            nblk = -(-n // block)
            if dlen != (n if scheme == SCHEME_Q8 else (n + 1) // 2) or alen != 4 * nblk:
                raise SmqError(f"{name}: payload length")
            scales = np.frombuffer(data, np.float32, nblk, aoff) if aoff % 4 == 0 else \
                np.frombuffer(bytes(data[aoff:aoff + alen]), np.float32)
            vals = dequant_smq(scheme, raw, scales, n, block)
        else:
            raise SmqError(f"{name}: data type {scheme}")
        out.append({"name": name, "scheme": scheme, "dims": dims, "block": block, "values": vals})
    return meta, out


def gpt2_parameter_names(n_layer: int) -> list[str]:
    """GetNamedParameters names (TransformerModel.cs:545-728) of the GPT-2 TransformerModel in
    the order its Parameters list registers them (TransformerModel.cs:132-144,
    TransformerBlock.cs:64-72, MultiHeadAttention.cs:114-115, MLP.cs:32-33)."""
    names = ["token_embd.weight", "pos_embd.weight"]
    for l in range(n_layer):
        p = f"blk.{l}."
        names += [p + "attn_norm.weight", p + "attn_norm.bias", p + "attn_qkv.weight", p + "attn_qkv.bias",
                  p + "attn_output.weight", p + "attn_output.bias", p + "ffn_norm.weight", p + "ffn_norm.bias",
                  p + "ffn_up.weight", p + "ffn_up.bias", p + "ffn_down.weight", p + "ffn_down.bias"]
    return names + ["output_norm.weight", "output_norm.bias", "output.weight"]


def config_from_metadata(meta: dict) -> dict:
    g = lambda k: int(meta[k])
    d = g("embed_dim")
    return dict(vocab=g("vocab_size"), ctx=g("block_size"), d=d, n_layer=g("num_layers"), n_head=g("num_heads"),
                ff=4 * d)


def oracle_from_smq(data: bytes, cfg: dict | None = None) -> tuple[OracleModel, dict]:
    """The GPT-2 TransformerModel an .smq file describes, as an OracleModel on the dequantized
    values.  Tensors whose names are parameter names are matched by name; a file with none is
    matched by parameter order."""
    meta, ents = read_smq(data)
    cfg = cfg or config_from_metadata(meta)
    order = gpt2_parameter_names(cfg["n_layer"])
    named = [e for e in ents if e["name"] in order]
    if named:
        pairs = [(e["name"], e) for e in named]
    else:
        if len(ents) != len(order):
            raise SmqError(f"{len(ents)} unnamed tensors for {len(order)} parameters")
        pairs = list(zip(order, ents))
    m = OracleModel(ARCH_GPT2, cfg["vocab"], cfg["ctx"], cfg["d"], cfg["n_layer"], cfg["n_head"], cfg["n_head"],
                    cfg["ff"], 10000.0, 1e-5)
    for name, e in pairs:
        oname = "position_embd.weight" if name == "pos_embd.weight" else name
        m.set_tensor(oname, F32, e["values"], e["values"].size)
    m.finalize()
    return m, cfg
