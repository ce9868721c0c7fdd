"""SmallMind .smq files on the CPU: the checker's reader (oracle.smq) pinned on the reference's
own model file and on closed forms, the writer (smallmind_amd.smq) and the backend's parser
(smx_smq_read_config, the parsing half of smx_model_load_smq), and the re-layout of Q8Tensor /
Q4Tensor blocks for upload (smx_smq_pack).  The round-trip and malformed-file cases follow the
reference's SmqRoundTripTests.cs (round trips :12-155, validator cases :262-360)."""
import hashlib
import json
import os
import struct

import numpy as np
import pytest

import oracle as O
from oracle import smq as OS
from smallmind_amd import smq as S
from smallmind_amd.model import ModelConfig

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "benchmark_model.smq")
GOLDEN_SHA = "82033e7e615c4b245b8de99ad3f34e04def1b3df23275f8c42862be9d2c047cc"


def _golden() -> bytes:
    with open(GOLDEN, "rb") as f:
        b = f.read()
    assert hashlib.sha256(b).hexdigest() == GOLDEN_SHA
    return b


# ---- the checker's reader, pinned on the reference's model file -------------------------------

def test_reference_model_directory_and_payload_layout():
    """benchmark-model.smq: 29 Q8_0 tensors at block 32 whose payloads tile the file after the
    directory with no gap (SmqWriter assigns offsets by a running sum), data then scales."""
    b = _golden()
    meta, ents = OS.read_smq(b)
    assert meta["vocab_size"] == "50" and meta["embed_dim"] == "64" and meta["num_layers"] == "2"
    assert len(ents) == 29 and all(e["scheme"] == OS.SCHEME_Q8 and e["block"] == 32 for e in ents)
    assert [e["name"] for e in ents] == [f"tensor_{i:03d}" for i in range(29)]
    mlen = struct.unpack_from("<I", b, 20)[0]
    off = 32 + mlen + 29 * 156
    for i in range(29):
        f = OS.ENTRY.unpack_from(b, 32 + mlen + 156 * i)
        doff, dlen, aoff, alen = f[12], f[13], f[14], f[15]
        assert doff == off and aoff == doff + dlen
        off = aoff + alen
    assert off == len(b)
    # shapes in GPT-2 parameter order (rows = out features): embeddings, per layer ln1, qkv,
    # proj, ln2, fc1, fc2 (1-D parameters stored as [1][n]), final norm, lm head
    dims = [e["dims"] for e in ents]
    assert dims[0] == (50, 64) and dims[1] == (32, 64) and dims[28] == (50, 64)
    assert dims[4] == (192, 64) and dims[10] == (256, 64) and dims[12] == (64, 256) and dims[13] == (1, 64)


def test_reference_model_values_follow_q8_quantize_closed_forms():
    """Q8Tensor.Quantize (Q8Tensor.cs:72-128) fixes two things a misread file breaks: every
    block's largest |code| is 127 (scale = maxAbs / 127), or the block is all zero with scale
    1.  The untrained model's LayerNorm gammas are ones and its biases zeros, so they dequantize
    to 127 * (1/127 in fp32) = 1.0 exactly and to 0.0."""
    b = _golden()
    meta, ents = OS.read_smq(b)
    mlen = struct.unpack_from("<I", b, 20)[0]
    for i, e in enumerate(ents):
        f = OS.ENTRY.unpack_from(b, 32 + mlen + 156 * i)
        n = int(np.prod(e["dims"]))
        codes = np.frombuffer(b, np.int8, n, f[12]).astype(np.int32).reshape(-1, 32)
        scales = np.frombuffer(b[f[14]:f[14] + f[15]], np.float32)
        mx = np.abs(codes).max(axis=1)
        assert np.all((mx == 127) | ((mx == 0) & (scales == 1.0))), e["name"]
        # the dequantized values are code * scale, element by element
        assert np.array_equal(e["values"], (codes.astype(np.float32) * scales[:, None]).reshape(-1))
    names = OS.gpt2_parameter_names(2)
    for name, e in zip(names, ents):
        if name.endswith("norm.weight"):
            assert np.all(e["values"] == 1.0), name
        if name.endswith(".bias"):
            assert np.all(e["values"] == 0.0), name


def test_dequant_smq_hand_cases():
    """Q4Tensor.Dequantize: element 2i is the low nibble of byte i, two's complement
    (DecodeNibble, Q4Tensor.cs:140-143); Q8: signed bytes; one scale per block of the flattened
    tensor, the last block short."""
    q4 = np.array([0x8F, 0x71, 0x08], np.uint8)   # nibbles (lo, hi): (15, 8), (1, 7), (8, 0)
    got = O.dequant_smq(11, q4, np.array([0.5, 2.0], np.float32), 5, 4)
    assert got.tolist() == [-0.5, -4.0, 0.5, 3.5, -16.0]
    q8 = np.array([127, 129, 0, 255, 1], np.uint8)   # 127, -127, 0, -1, 1
    got = O.dequant_smq(10, q8, np.array([0.25, -3.0], np.float32), 5, 3)
    assert got.tolist() == [31.75, -31.75, 0.0, 3.0, -3.0]


def test_oracle_model_from_reference_file_runs():
    om, cfg = OS.oracle_from_smq(_golden())
    assert cfg == dict(vocab=50, ctx=32, d=64, n_layer=2, n_head=4, ff=256)
    toks = om.generate_greedy(np.array([1, 2, 3], np.int32), 8)[0]
    assert len(toks) == 8 and all(0 <= t < 50 for t in toks)


# ---- writer / backend parser round trips ------------------------------------------------------

@pytest.mark.parametrize("scheme,block", [(S.Q8_0, 8), (S.Q4_0, 8), (S.Q8_0, 64), (S.Q4_0, 32)])
def test_round_trip_preserves_codes_and_scales(tmp_path, scheme, block):
    """SmqRoundTrip_Q8Tensor/Q4Tensor_PreservesData: rows, cols, block size, every code byte
    and every scale survive write + read."""
    rng = np.random.default_rng(block + scheme)
    rows, cols = 16, 64
    x = rng.uniform(-1, 1, rows * cols).astype(np.float32)
    q, sc = (O.quantize_ref_q8 if scheme == S.Q8_0 else O.quantize_ref_q4)(x, block)
    p = tmp_path / "t.smq"
    S.write_smq(str(p), [S.SmqTensor("layer1.wq", scheme, (rows, cols), q, sc, block)], {"model_name": "t"})
    meta, ents = OS.read_smq(p.read_bytes())
    assert meta == {"model_name": "t"} and len(ents) == 1
    e = ents[0]
    assert (e["name"], e["dims"], e["block"], e["scheme"]) == ("layer1.wq", (rows, cols), block, scheme)
    assert np.array_equal(e["values"], O.dequant_smq(scheme, q, sc, rows * cols, block))


def test_mixed_model_metadata_and_backend_config(tmp_path):
    """SmqRoundTrip_MixedQ8Q4Model / _Metadata_RoundTrips, and smx_smq_read_config's view of
    the same file: the GPT-2 configuration from the metadata, the tensor count."""
    from smallmind_amd.model import read_smq_config
    cfg = ModelConfig("gpt2", 300, 48, 128, 3, 4, 4, 512)
    rng = np.random.default_rng(1)
    q8, s8 = O.quantize_ref_q8(rng.normal(0, 1, 32).astype(np.float32), 4)
    q4, s4 = O.quantize_ref_q4(rng.normal(0, 1, 128).astype(np.float32), 8)
    f32 = rng.normal(0, 1, 12).astype(np.float32)
    p = tmp_path / "m.smq"
    S.write_smq(str(p), [S.SmqTensor("layer1.wq", S.Q8_0, (4, 8), q8, s8, 4),
                         S.SmqTensor("layer1.wk", S.Q4_0, (8, 16), q4, s4, 8),
                         S.SmqTensor("norm", S.F32, (12,), f32)], S.gpt2_metadata(cfg, "mixed"))
    meta, ents = OS.read_smq(p.read_bytes())
    assert [e["name"] for e in ents] == ["layer1.wq", "layer1.wk", "norm"]
    assert meta["model_name"] == "mixed" and meta["vocab_size"] == "300"
    assert np.array_equal(ents[2]["values"], f32)
    c = read_smq_config(str(p))
    assert (c.architecture, c.vocab_size, c.context_length, c.embedding_length, c.block_count, c.head_count,
            c.head_count_kv, c.feed_forward_length) == ("gpt2", 300, 48, 128, 3, 4, 4, 512)
    # the reference file: configuration from its string-valued metadata
    c = read_smq_config(GOLDEN)
    assert (c.vocab_size, c.context_length, c.embedding_length, c.block_count, c.head_count) == (50, 32, 64, 2, 4)


@pytest.mark.parametrize("case", ["magic", "version", "truncated_dir", "truncated_data", "payload_length",
                                  "f16", "missing_meta", "missing_file"])
def test_malformed_files_are_rejected(tmp_path, case):
    """SmqValidator_InvalidMagicHeader / _WrongVersion / _TruncatedFile and the payload length
    checks of SmqReader (SmqReader.cs:153-293): SMX_EINVAL, or SMX_EUNSUPPORTED for a version
    or data type the reader does not take."""
    from smallmind_amd._lib import SmxError
    from smallmind_amd.model import read_smq_config
    cfg = ModelConfig("gpt2", 300, 48, 128, 3, 4, 4, 512)
    q, sc = O.quantize_ref_q8(np.linspace(-1, 1, 64).astype(np.float32), 32)
    t = S.SmqTensor("w", S.Q8_0, (2, 32), q, sc, 32)
    p = tmp_path / f"{case}.smq"
    meta = S.gpt2_metadata(cfg)
    S.write_smq(str(p), [t], meta)
    raw = bytearray(p.read_bytes())
    mlen = struct.unpack_from("<I", raw, 20)[0]
    expect = -1
    if case == "magic":
        raw[:8] = b"SMQv0002"
    elif case == "version":
        raw[8:12] = struct.pack("<I", 2)
        expect = -5
    elif case == "truncated_dir":
        raw = raw[:32 + mlen + 100]
    elif case == "truncated_data":
        raw = raw[:-10]
    elif case == "payload_length":
        e = 32 + mlen
        raw[e + 116:e + 124] = struct.pack("<Q", 63)   # data length != rows * cols
    elif case == "f16":
        raw[32 + mlen + 64:32 + mlen + 68] = struct.pack("<I", S.F16)
        expect = -5
    elif case == "missing_meta":
        S.write_smq(str(p), [t], {"model_name": "x"})
        raw = bytearray(p.read_bytes())
    if case == "missing_file":
        p = tmp_path / "absent.smq"
    else:
        p.write_bytes(bytes(raw))
    with pytest.raises(SmxError) as e:
        read_smq_config(str(p))
    assert e.value.code == expect


# ---- upload layout --------------------------------------------------------------------------

@pytest.mark.parametrize("qtype,block", [(1010, 32), (1010, 64), (1011, 32), (1011, 128)])
def test_smq_pack_layout_and_values(qtype, block):
    """smx_smq_pack: per 32 elements, the fp32 scale of their SMQ block then their codes; the
    packed blocks decode (oracle, upload layout) to Q8Tensor / Q4Tensor.Dequantize of the
    original tensor."""
    from smallmind_amd.quantization import smq_pack
    rows, cols = 6, 128
    x = np.random.default_rng(qtype + block).normal(0, 1, rows * cols).astype(np.float32)
    q, sc = (O.quantize_ref_q8 if qtype == 1010 else O.quantize_ref_q4)(x, block)
    got = smq_pack(qtype, q, sc, rows, cols, block)
    bb = 36 if qtype == 1010 else 20
    qb = np.ascontiguousarray(q).view(np.uint8)
    for k in range(rows * cols // 32):
        blk = got[k * bb:(k + 1) * bb]
        assert blk[:4].view(np.float32)[0] == sc[32 * k // block]
        code_bytes = qb[32 * k:32 * k + 32] if qtype == 1010 else qb[16 * k:16 * k + 16]
        assert np.array_equal(blk[4:], code_bytes)
    scheme = 10 if qtype == 1010 else 11
    assert np.array_equal(O.dequant(qtype, got, rows * cols), O.dequant_smq(scheme, q, sc, rows * cols, block))


def test_smq_pack_rejects_blocks_that_straddle_chunks():
    from smallmind_amd._lib import SmxError
    from smallmind_amd.quantization import smq_pack
    q, sc = O.quantize_ref_q8(np.ones(96, np.float32), 48)
    with pytest.raises(SmxError):
        smq_pack(1010, q, sc, 2, 48, 48)   # cols not a multiple of 32
    q, sc = O.quantize_ref_q8(np.ones(128, np.float32), 16)
    with pytest.raises(SmxError):
        smq_pack(1010, q, sc, 2, 64, 16)   # block of 16: two scales per 32-element chunk


def test_writer_output_is_what_smqwriter_lays_out(tmp_path):
    """Header fields, JSON metadata and the 156-byte entry of one tensor, byte by byte."""
    q, sc = O.quantize_ref_q8(np.arange(64, dtype=np.float32), 32)
    p = tmp_path / "one.smq"
    n = S.write_smq(str(p), [S.SmqTensor("a.weight", S.Q8_0, (2, 32), q, sc, 32)], {"k": "v"})
    b = p.read_bytes()
    assert n == len(b)
    meta = json.dumps({"k": "v"}, separators=(",", ":")).encode()
    assert b[:8] == b"SMQv0001" and struct.unpack_from("<IIIIQ", b, 8) == (1, 32, 1, len(meta), 0)
    assert b[32:32 + len(meta)] == meta
    e = 32 + len(meta)
    assert b[e:e + 8] == b"a.weight" and b[e + 8:e + 64] == bytes(56)
    assert struct.unpack_from("<Ii8iI", b, e + 64) == (10, 2, 2, 32, 0, 0, 0, 0, 0, 0, 32)
    data = e + 156
    assert struct.unpack_from("<QQQQ", b, e + 108) == (data, 64, data + 64, 8)
    assert b[e + 140:e + 156] == bytes(16)
    assert b[data:data + 64] == np.ascontiguousarray(q).tobytes() and b[data + 64:] == sc.tobytes()


def test_smq_pack_refuses_sizes_past_64_bits():
    """rows x cols whose byte counts would not fit 64 bits are refused before any arithmetic on
    them (the product itself would overflow); the small buffers are never touched."""
    import ctypes

    from smallmind_amd import _lib
    from smallmind_amd._lib import SmxError
    data = np.zeros(64, np.int8)
    scales = np.ones(4, np.float32)
    out = np.zeros(64, np.uint8)
    for rows, cols in [(2**40, 2**40), (2**62, 32), (2**31, 2**31)]:
        with pytest.raises(SmxError, match="too large"):
            _lib.call("smx_smq_pack", 1010, data.ctypes.data_as(ctypes.c_void_p),
                      scales.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), ctypes.c_int64(rows),
                      ctypes.c_int64(cols), 32, out.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(out.size))
