"""Pins the CPU oracle (oracle/smx_oracle.c) before it is trusted as the GPU checker.

Every check is independent of the oracle's own code: closed forms, the reference's own test
values, numpy library routines, an independent bit packer, and invariants chosen so that a
dropped term, a wrong index or a transposed operand fails one of them.
"""
import numpy as np
import pytest

import oracle as O
from tests.helpers import rel_err

# ---------------------------------------------------------------------------------------------
# fp16 (GgufModelLoader.HalfToFloat, GgufModelLoader.cs:919-956)
# ---------------------------------------------------------------------------------------------


def _h2f_all():
    # through the F16 tensor path (an array write), so signalling NaNs are not quieted by a
    # float return value on the way back to Python
    return O.dequant(O.F16, np.arange(65536, dtype=np.uint16).view(np.uint8), 65536)


def test_half_to_float_all_patterns_vs_ieee():
    got = _h2f_all().view(np.uint32)
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32).view(np.uint32)
    exp = (h >> 10) & 0x1F
    finite = exp != 0x1F
    assert np.array_equal(got[finite], ref[finite])
    # Inf/NaN keep sign and payload: sign<<31 | 0x7F800000 | mantissa<<13 (reference formula)
    hh = h[~finite].astype(np.uint32)
    closed = ((hh >> 15) << 31) | 0x7F800000 | ((hh & 0x3FF) << 13)
    assert np.array_equal(got[~finite], closed)


def test_float_to_half_roundtrip_and_rne_vs_numpy():
    h = np.arange(65536, dtype=np.uint16)
    finite = ((h >> 10) & 0x1F) != 0x1F
    f = h.view(np.float16).astype(np.float32)
    back = np.array([O.float_to_half(float(v)) for v in f[finite]], np.uint16)
    # +0/-0 and every finite value round-trip exactly
    assert np.array_equal(back, h[finite])
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.normal(0, 1, 3000).astype(np.float32),
        rng.normal(0, 1e-5, 2000).astype(np.float32),            # half subnormal range
        (rng.uniform(-70000, 70000, 1000)).astype(np.float32),    # overflow boundary
        # exact ties between adjacent half values (normal and subnormal)
        ((f[finite][:-1].astype(np.float64) + f[finite][1:].astype(np.float64)) / 2)[::37].astype(np.float32),
    ])
    x = x[np.isfinite(x)]
    ours = np.array([O.float_to_half(float(v)) for v in x], np.uint16)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


# ---------------------------------------------------------------------------------------------
# block formats
# ---------------------------------------------------------------------------------------------


def test_decode_nibble_reference_table():
    # QuantKernelsTests.cs:149-158
    lib = O.lib()
    assert [lib.smxo_decode_nibble(n) for n in (0, 1, 7, 8, 9, 15)] == [0, 1, 7, -8, -7, -1]


def test_block_geometry_matches_reference_tests():
    # KQuantTensorTests.cs:19-29 (Q4_K 256/144), :145-155 (Q6_K 256/210)
    assert (O.BLOCK_ELEMS[O.Q4_K], O.BLOCK_BYTES[O.Q4_K]) == (256, 144)
    assert (O.BLOCK_ELEMS[O.Q6_K], O.BLOCK_BYTES[O.Q6_K]) == (256, 210)
    lib = O.lib()
    for t in (O.Q4_0, O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K):
        assert lib.smxo_block_elems(t) == O.BLOCK_ELEMS[t]
        assert lib.smxo_block_bytes(t) == O.BLOCK_BYTES[t]


# An independent packer: builds blocks field by field from integers, following the byte
# layout the reference decoder reads, and the expected values from the same integers.

def _f16(v):
    return np.float16(v).view(np.uint16)


def _put16(b, off, h):
    b[off] = int(h) & 0xFF
    b[off + 1] = int(h) >> 8


def _pack_bits(values, width):
    acc = 0
    for i, v in enumerate(values):
        acc |= int(v) << (width * i)
    nbytes = len(values) * width // 8
    return [(acc >> (8 * i)) & 0xFF for i in range(nbytes)]


F = np.float32


def _known_q8_0(rng):
    d = rng.choice([0.5, 0.0078125, 3.0, 1e-6, -0.25])
    q = rng.integers(-128, 128, 32)
    b = np.zeros(34, np.uint8)
    _put16(b, 0, _f16(d))
    b[2:] = (q & 0xFF).astype(np.uint8)
    df = F(np.float16(d))
    return b, np.array([F(int(v)) * df for v in q], F)


def _known_q4_0(rng):
    d = rng.choice([0.5, 0.0078125, 3.0, 1e-6, -0.25])
    q = rng.integers(-8, 8, 32)
    b = np.zeros(18, np.uint8)
    _put16(b, 0, _f16(d))
    for i in range(16):   # element 2i low nibble, 2i+1 high nibble (two's complement)
        b[2 + i] = (int(q[2 * i]) & 0xF) | ((int(q[2 * i + 1]) & 0xF) << 4)
    df = F(np.float16(d))
    return b, np.array([F(int(v)) * df for v in q], F)


def _known_kq(rng, five_bit):
    d, dmin = rng.choice([0.5, 0.0078125, 3.0, 1e-5]), rng.choice([0.25, 0.001, 2.0])
    sc6 = rng.integers(0, 64, 8)
    mn6 = rng.integers(0, 64, 8)
    q = rng.integers(0, 32 if five_bit else 16, 256)
    b = np.zeros(176 if five_bit else 144, np.uint8)
    _put16(b, 0, _f16(d))
    _put16(b, 2, _f16(dmin))
    b[4:10] = _pack_bits(sc6, 6)    # 8 six-bit scales, one little-endian bit stream
    b[10:16] = _pack_bits(mn6, 6)   # 8 six-bit mins
    low = q & 0xF
    qs_off = 48 if five_bit else 16
    for i in range(128):
        b[qs_off + i] = int(low[2 * i]) | (int(low[2 * i + 1]) << 4)
    if five_bit:
        b[16:48] = _pack_bits((q >> 4) & 1, 1)   # element v -> bit v of qh
    df, dmf = F(np.float16(d)), F(np.float16(dmin))
    y = np.empty(256, F)
    for v in range(256):
        j = v // 32
        sc, m = df * F(int(sc6[j])), dmf * F(int(mn6[j]))
        qq = int(q[v]) - (16 if five_bit else 0)
        y[v] = F(sc * F(qq)) - m
    return b, y


def _known_q6_k(rng):
    d = rng.choice([0.5, 0.0078125, 3.0, 1e-5, -0.125])
    sc = rng.integers(-128, 128, 16)
    q = rng.integers(0, 64, 256)
    b = np.zeros(210, np.uint8)
    for i in range(128):
        b[i] = int(q[2 * i] & 0xF) | (int(q[2 * i + 1] & 0xF) << 4)
    b[128:192] = _pack_bits((q >> 4) & 3, 2)     # element v -> bits 2v..2v+1 of qh
    b[192:208] = (sc & 0xFF).astype(np.uint8)
    _put16(b, 208, _f16(d))
    df = F(np.float16(d))
    y = np.array([F(df * F(int(sc[v // 16]))) * F(int(q[v]) - 32) for v in range(256)], F)
    return b, y


KNOWN = {O.Q8_0: _known_q8_0, O.Q4_0: _known_q4_0, O.Q4_K: lambda r: _known_kq(r, False),
         O.Q5_K: lambda r: _known_kq(r, True), O.Q6_K: _known_q6_k}


@pytest.mark.parametrize("qtype", list(KNOWN))
def test_dequant_known_answers_from_independent_packer(qtype):
    rng = np.random.default_rng(qtype)
    for _ in range(40):
        b, y = KNOWN[qtype](rng)
        got = O.dequant(qtype, b, y.size)
        assert np.array_equal(got.view(np.uint32), y.view(np.uint32))


def test_q5_k_subtracts_16_like_the_load_path():
    # GgufModelLoader.cs:830 centres 5-bit codes by 16 (the compat decoder in StubDecoders.cs
    # does not); a block with d=1, dmin=0, scale 1 and code 0 decodes to -16.
    b = np.zeros(176, np.uint8)
    _put16(b, 0, _f16(1.0))
    b[4:10] = _pack_bits([1] * 8, 6)
    assert np.all(O.dequant(O.Q5_K, b, 256) == -16.0)


def test_q4_k_partial_block_leaves_odd_tail_zero():
    # GgufModelLoader.cs:723 loops i < count/2, so a sub-block with an odd element count
    # never writes its last element.
    rng = np.random.default_rng(3)
    b, y = _known_kq(rng, False)
    got = O.dequant(O.Q4_K, b, 37)
    assert np.array_equal(got[:36].view(np.uint32), y[:36].view(np.uint32))
    assert got[36] == 0.0


# ---------------------------------------------------------------------------------------------
# quantizers (Q8Tensor.Quantize / Q4Tensor.Quantize and the build's encoders)
# ---------------------------------------------------------------------------------------------


def test_reference_q8_quantizer_hand_cases():
    x = np.array([127.0, 63.5, -127.0, 0.5, 1.5, 2.5, -2.5, 0.0], np.float32)
    q, s = O.quantize_ref_q8(x, block=8)
    assert s[0] == 1.0
    assert q.tolist() == [127, 64, -127, 0, 2, 2, -2, 0]      # MathF.Round is half-to-even
    q, s = O.quantize_ref_q8(np.zeros(4, np.float32), block=4)
    assert s[0] == 1.0 and q.tolist() == [0, 0, 0, 0]


def test_reference_q4_quantizer_hand_cases():
    x = np.array([7.0, -7.0, 3.5, 2.5, -8.0, 0.4, 100.0, -0.5], np.float32)
    data, s = O.quantize_ref_q4(x[:6], block=6)
    assert s[0] == np.float32(8.0) / np.float32(7.0)
    codes = [O.lib().smxo_decode_nibble((int(data[i // 2]) >> (4 * (i % 2))) & 0xF) for i in range(6)]
    inv = np.float32(1.0) / s[0]
    assert codes == [int(np.rint(np.clip(np.float32(v) * inv, -8, 7))) for v in x[:6]]
    data, s = O.quantize_ref_q4(np.array([7.0, -7.0, 3.5, 2.5], np.float32), block=4)
    assert s[0] == 1.0
    codes = [O.lib().smxo_decode_nibble((int(data[i // 2]) >> (4 * (i % 2))) & 0xF) for i in range(4)]
    assert codes == [7, -7, 4, 2]


@pytest.mark.parametrize("qtype,tol", [(O.Q8_0, 0.006), (O.Q4_0, 0.08), (O.Q4_K, 0.07),
                                       (O.Q5_K, 0.035), (O.Q6_K, 0.018)])
def test_encoder_roundtrip_error_bound(qtype, tol):
    rng = np.random.default_rng(qtype)
    x = rng.normal(0, 0.02, 256 * 64).astype(np.float32)
    y = O.dequant(qtype, O.quantize(qtype, x), x.size)
    be = 16 if qtype == O.Q6_K else 32   # elements sharing one scale
    err = np.abs(y - x).reshape(-1, be).max(1) / np.abs(x).reshape(-1, be).max(1)
    assert err.max() < tol * 2 and np.median(err) < tol


def test_q8_0_encoder_exact_on_grid():
    s = np.float32(2.0 ** -7)
    q = np.random.default_rng(1).integers(-127, 128, 64)
    q[0], q[32] = 127, -127
    x = (q * s).astype(np.float32)
    assert np.array_equal(O.dequant(O.Q8_0, O.quantize(O.Q8_0, x), 64), x)


def test_q4_0_encoder_uses_reference_nibble_semantics():
    x = np.array([7, -7, 1, -1, 0, 3, -3, 2] * 4, np.float32)
    b = O.quantize(O.Q4_0, x)
    assert np.array_equal(O.dequant(O.Q4_0, b, 32), x)
    # element 1 (-7) is the high nibble of byte 0, two's complement 0b1001
    assert b[2] == (7 | (9 << 4))


# ---------------------------------------------------------------------------------------------
# GEMV
# ---------------------------------------------------------------------------------------------


@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K])
def test_gemv_f64_equals_numpy_on_dequantized(qtype):
    rng = np.random.default_rng(7)
    N, K = 48, 512
    W = O.quantize(qtype, rng.normal(0, 0.02, N * K).astype(np.float32))
    x = rng.normal(0, 1, K).astype(np.float32)
    Wf = O.dequant(qtype, W, N * K).reshape(N, K).astype(np.float64)
    assert np.allclose(O.gemv_f64(qtype, W, N, K, x), Wf @ x.astype(np.float64), rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------------------------
# norms, RoPE, softmax, activations
# ---------------------------------------------------------------------------------------------


def test_rmsnorm_reference_closed_form():
    # RMSNormOpsTests.cs:145-163
    x = np.array([0.5, 1.5, 2.5, 3.5], np.float32)
    g = np.array([1.2, 0.8, 1.5, 0.5], np.float32)
    y = O.rmsnorm(x, g)
    inv = 1.0 / np.sqrt((0.25 + 2.25 + 6.25 + 12.25) / 4 + 1e-5)
    assert np.allclose(y, g * x * inv, atol=1e-4)


def test_layernorm_reference_closed_form():
    # LayerNormOpsTests.cs:206-229: mean 5, variance 5
    x = np.array([2, 4, 6, 8], np.float32)
    y = O.layernorm(x, np.ones(4, np.float32), np.zeros(4, np.float32))
    assert np.allclose(y, (x - 5) / np.sqrt(5 + 1e-5), atol=1e-4)


@pytest.mark.parametrize("n", [64, 768, 2048, 2050])
def test_norms_vs_float64(n):
    rng = np.random.default_rng(n)
    x = rng.normal(0, 3, (3, n)).astype(np.float32)
    g = rng.normal(1, 0.2, n).astype(np.float32)
    b = rng.normal(0, 0.2, n).astype(np.float32)
    xd = x.astype(np.float64)
    rms = xd / np.sqrt((xd ** 2).mean(-1, keepdims=True) + 1e-5) * g
    assert rel_err(O.rmsnorm(x, g), rms) < 2e-6
    mu = xd.mean(-1, keepdims=True)
    ln = (xd - mu) / np.sqrt(((xd - mu) ** 2).mean(-1, keepdims=True) + 1e-5) * g + b
    assert rel_err(O.layernorm(x, g, b), ln) < 2e-6


def test_rope_position0_identity_and_angles():
    c, s = O.rope_tables(512, 4, 10000.0)
    # RotaryEmbeddingTests.cs:33-57: position 0 is the identity
    q = np.array([[[1, 0, 1, 0]]], np.float32)
    k = np.array([[[0, 1, 0, 1]]], np.float32)
    assert np.array_equal(O.rope_apply(q, 0, c, s), q)
    assert np.array_equal(O.rope_apply(k, 0, c, s), k)
    c, s = O.rope_tables(64, 64, 10000.0)
    pos = np.arange(64)[:, None].astype(np.float64)
    freq = 1.0 / 10000.0 ** (2 * np.arange(32) / 64.0)
    assert np.allclose(c, np.cos(pos * freq), atol=2e-5)
    assert np.allclose(s, np.sin(pos * freq), atol=2e-5)


def test_rope_rotates_adjacent_pairs_as_complex_multiply():
    rng = np.random.default_rng(5)
    c, s = O.rope_tables(32, 8, 10000.0)
    x = rng.normal(0, 1, (3, 5, 8)).astype(np.float32)
    y = O.rope_apply(x, 7, c, s)
    z = (x[..., 0::2] + 1j * x[..., 1::2]) * (c[7:12] + 1j * s[7:12])[None]
    assert np.allclose(y[..., 0::2], z.real, atol=1e-6)
    assert np.allclose(y[..., 1::2], z.imag, atol=1e-6)
    assert np.allclose(np.hypot(y[..., 0::2], y[..., 1::2]), np.hypot(x[..., 0::2], x[..., 1::2]), atol=1e-6)


def test_fastexp_pade_closed_form():
    assert O.fastexp(0.0) == 1.0
    assert abs(O.fastexp(-1.0) - 7.0 / 19.0) < 1e-7          # (1-1/2+1/12)/(1+1/2+1/12)
    assert abs(O.fastexp(2.0) - (1 + 1 + 4 / 12) / (1 - 1 + 4 / 12)) < 1e-6
    assert O.fastexp(-1000.0) == O.fastexp(-87.3)            # clamp
    assert O.fastexp(1000.0) == O.fastexp(88.7)


def test_softmax_rows_mask_and_uniform():
    rng = np.random.default_rng(2)
    s = rng.normal(0, 2, (5, 9)).astype(np.float32)
    p = O.scale_mask_softmax(s, 0.125, cache_off=4)
    for i in range(5):
        valid = 4 + i + 1
        assert abs(p[i, :valid].sum() - 1) < 1e-6
        assert np.all(p[i, valid:] == 0)
        e = np.array([O.fastexp(float(np.float32(v) * np.float32(0.125)) - float((s[i, :valid] * np.float32(0.125)).max()))
                      for v in s[i, :valid]])
        assert np.allclose(p[i, :valid], e / e.sum(), rtol=1e-6)
    u = O.scale_mask_softmax(np.ones((1, 6), np.float32), 1.0, cache_off=5)
    assert np.allclose(u, 1 / 6)


def test_gelu_pade_closed_form():
    for x in [-3.0, -0.7, 0.0, 0.3, 1.0, 4.0, 12.0]:
        inner = 0.7978845608 * (x + 0.044715 * x ** 3)
        inner = max(-10.0, min(10.0, inner))
        t = inner * (27 + inner ** 2) / (27 + 9 * inner ** 2)
        assert abs(O.gelu(np.array([x], np.float32))[0] - 0.5 * x * (1 + t)) < 1e-5 * max(1, abs(x))


@pytest.mark.parametrize("n", [7, 15, 16, 31, 64, 127, 256])
def test_silu_mul_fused_equals_separate(n):
    # ActivationOpsTests.cs:24-57
    rng = np.random.default_rng(n)
    g = rng.normal(0, 4, n).astype(np.float32)
    u = rng.normal(0, 1, n).astype(np.float32)
    gd = g.astype(np.float64)
    sep = gd / (1 + np.exp(-np.clip(gd, -20, 20))) * u
    assert np.allclose(O.silu_mul(g, u), sep, atol=1e-4)


# ---------------------------------------------------------------------------------------------
# forward
# ---------------------------------------------------------------------------------------------


def _np_forward(cfg, tensors, tokens):
    """float64 numpy forward of the reference graph from library-level operations."""
    d, H, Hkv = cfg.embedding_length, cfg.head_count, cfg.head_count_kv
    hd, kv = d // H, (d // H) * Hkv
    W = {}
    for name, (qt, dims, data) in tensors.items():
        n = int(np.prod(dims))
        v = O.dequant(qt, data, n).astype(np.float64)
        W[name] = v.reshape(dims[::-1]) if len(dims) == 2 else v
    gpt2 = cfg.architecture == "gpt2"
    T = len(tokens)
    x = W["token_embd.weight"][tokens]
    if gpt2:
        x = x + W["position_embd.weight"][:T]

    def norm(v, g, b):
        if gpt2:
            mu = v.mean(-1, keepdims=True)
            return (v - mu) / np.sqrt(((v - mu) ** 2).mean(-1, keepdims=True) + cfg.norm_eps) * g + b
        return v / np.sqrt((v ** 2).mean(-1, keepdims=True) + cfg.norm_eps) * g

    c, s = O.rope_tables(cfg.context_length, hd, cfg.rope_freq_base)
    rot = (c[:T] + 1j * s[:T]).astype(np.complex128)
    fe = np.vectorize(lambda z: O.fastexp(float(z)))
    for i in range(cfg.block_count):
        p = f"blk.{i}."
        h = norm(x, W[p + "attn_norm.weight"], W.get(p + "attn_norm.bias"))
        if gpt2:
            qkv = h @ W[p + "attn_qkv.weight"].T + W[p + "attn_qkv.bias"]
            q, k, v = qkv[:, :d], qkv[:, d:d + kv], qkv[:, d + kv:]
        else:
            q, k, v = h @ W[p + "attn_q.weight"].T, h @ W[p + "attn_k.weight"].T, h @ W[p + "attn_v.weight"].T
        q = q.reshape(T, H, hd).transpose(1, 0, 2)
        k = k.reshape(T, Hkv, hd).transpose(1, 0, 2)
        v = v.reshape(T, Hkv, hd).transpose(1, 0, 2)
        if not gpt2:
            def rope(a):
                z = (a[..., 0::2] + 1j * a[..., 1::2]) * rot[None]
                out = np.empty_like(a)
                out[..., 0::2], out[..., 1::2] = z.real, z.imag
                return out
            q, k = rope(q), rope(k)
        k = np.repeat(k, H // Hkv, axis=0)
        v = np.repeat(v, H // Hkv, axis=0)
        sc = (q @ k.transpose(0, 2, 1)) / np.sqrt(hd)
        mask = np.tril(np.ones((T, T), bool))
        sc = np.where(mask, sc, -np.inf)
        e = np.where(mask, fe(sc - sc.max(-1, keepdims=True)), 0.0)
        att = (e / e.sum(-1, keepdims=True)) @ v
        y = att.transpose(1, 0, 2).reshape(T, d)
        o = y @ W[p + "attn_output.weight"].T + (W[p + "attn_output.bias"] if gpt2 else 0)
        x = x + o
        h = norm(x, W[p + "ffn_norm.weight"], W.get(p + "ffn_norm.bias"))
        if gpt2:
            f = h @ W[p + "ffn_up.weight"].T + W[p + "ffn_up.bias"]
            inner = np.clip(0.7978845608 * (f + 0.044715 * f ** 3), -10, 10)
            f = 0.5 * f * (1 + inner * (27 + inner ** 2) / (27 + 9 * inner ** 2))
            m = f @ W[p + "ffn_down.weight"].T + W[p + "ffn_down.bias"]
        else:
            g = h @ W[p + "ffn_gate.weight"].T
            u = h @ W[p + "ffn_up.weight"].T
            m = (g / (1 + np.exp(-np.clip(g, -20, 20))) * u) @ W[p + "ffn_down.weight"].T
        x = x + m
    h = norm(x, W["output_norm.weight"], W.get("output_norm.bias"))
    head = W.get("output.weight", W["token_embd.weight"])
    return h @ head.T


TINY = {
    "llama": dict(architecture="llama", vocab_size=300, context_length=40, embedding_length=256,
                  block_count=2, head_count=4, head_count_kv=2, feed_forward_length=512),
    "gpt2": dict(architecture="gpt2", vocab_size=300, context_length=40, embedding_length=128,
                 block_count=2, head_count=2, head_count_kv=2, feed_forward_length=512),
}


def _tiny(arch):
    from smallmind_amd.model import ModelConfig
    from tests.helpers import build_pair
    cfg = ModelConfig(**TINY[arch])
    lt = O.Q4_K if arch == "llama" else O.Q8_0
    om, _, tensors = build_pair(cfg, lt, O.Q6_K if arch == "llama" else O.Q8_0,
                                O.Q6_K if arch == "llama" else None, seed=11, with_gpu=False)
    return cfg, om, tensors


@pytest.mark.parametrize("arch", ["llama", "gpt2"])
def test_forward_nocache_vs_numpy_float64(arch):
    cfg, om, tensors = _tiny(arch)
    toks = np.random.default_rng(4).integers(0, cfg.vocab_size, 12).astype(np.int32)
    got = om.forward_nocache(toks, all_rows=True)
    ref = _np_forward(cfg, tensors, toks)
    assert rel_err(got, ref) < 1e-5


@pytest.mark.parametrize("arch", ["llama", "gpt2"])
def test_forward_is_causal_and_cache_equals_nocache(arch):
    cfg, om, _ = _tiny(arch)
    rng = np.random.default_rng(9)
    toks = rng.integers(0, cfg.vocab_size, 16).astype(np.int32)
    full = om.forward_nocache(toks, all_rows=True)
    toks2 = toks.copy()
    toks2[10:] = rng.integers(0, cfg.vocab_size, 6)
    full2 = om.forward_nocache(toks2, all_rows=True)
    assert np.array_equal(full[:10], full2[:10])
    assert not np.array_equal(full[10:], full2[10:])
    sess = om.session(32)
    for p, t in enumerate(toks):
        assert np.array_equal(sess.step(int(t), p), full[p])


def test_single_token_attention_passes_v_through():
    # With one position the softmax weight is FastExp(0)/FastExp(0) = 1 exactly, so the
    # attention output of head h is the V row of its KV head.
    s = np.zeros((1, 1), np.float32)
    assert O.scale_mask_softmax(s, 0.125)[0, 0] == 1.0


@pytest.mark.parametrize("arch", ["llama", "gpt2"])
def test_threaded_batched_paths_are_bit_identical(arch):
    """The oracle's linears run row blocks over threads and 8 tokens per vector; every output
    keeps its own fma chain over k in order, so one thread, all threads, a batched prefill and a
    multi-session step must agree bit for bit with single-token steps.  Ragged shapes: vocab
    300 (a partial 8-row block and a partial group of four blocks), 13 tokens (a partial tile)."""
    cfg, om, _ = _tiny(arch)
    rng = np.random.default_rng(17)
    toks = rng.integers(0, cfg.vocab_size, 13).astype(np.int32)
    n0 = O.get_threads()
    try:
        O.set_threads(1)
        full1 = om.forward_nocache(toks, all_rows=True)
        s1 = om.session(32)
        steps1 = [s1.step(int(t), p) for p, t in enumerate(toks)]
        O.set_threads(3)
        assert np.array_equal(om.forward_nocache(toks, all_rows=True), full1)
    finally:
        O.set_threads(0)
    assert O.get_threads() == n0
    assert np.array_equal(om.forward_nocache(toks, all_rows=True), full1)
    s2 = om.session(32)
    last = s2.prefill(toks[:9], 0, want_logits=True)
    assert np.array_equal(last, steps1[8])
    for p in range(9, 13):                       # steps continue on the prefilled cache
        assert np.array_equal(s2.step(int(toks[p]), p), steps1[p])
    # three sessions at different positions in one pass vs one step each
    prompts = [rng.integers(0, cfg.vocab_size, n).astype(np.int32) for n in (5, 1, 11)]
    sa = [om.session(32) for _ in prompts]
    sb = [om.session(32) for _ in prompts]
    for a, b, p in zip(sa, sb, prompts):
        if len(p) > 1:
            a.prefill(p[:-1], 0)
            b.prefill(p[:-1], 0)
    tk = [int(p[-1]) for p in prompts]
    for step in range(3):
        pos = [len(p) - 1 + step for p in prompts]
        multi = om.multi_step(sa, tk, pos)
        single = [b.step(t, q) for b, t, q in zip(sb, tk, pos)]
        assert np.array_equal(multi, np.stack(single))
        tk = [int(np.argmax(r)) for r in single]


def test_prefill_many_equals_prefill_each():
    """Several prompts prefilled in one pass leave every session's cache as its own prefill
    does: the next step's logits are bit-identical."""
    cfg, om, _ = _tiny("llama")
    rng = np.random.default_rng(23)
    prompts = [rng.integers(0, cfg.vocab_size, n).astype(np.int32) for n in (7, 2, 12)]
    sa = [om.session(32) for _ in prompts]
    sb = [om.session(32) for _ in prompts]
    om.prefill_many(sa, [p[:-1] for p in prompts])
    for b, p in zip(sb, prompts):
        for q, t in enumerate(p[:-1]):
            b.step(int(t), q, want_logits=False)
    for a, b, p in zip(sa, sb, prompts):
        assert np.array_equal(a.step(int(p[-1]), len(p) - 1), b.step(int(p[-1]), len(p) - 1))


def test_generate_crops_the_prompt_to_the_block_size():
    """InferenceSession.cs:494-508: a context longer than blockSize is cropped to its last
    blockSize tokens before the prefill.  The oracle's generate (the C restatement) against a
    step-by-step run of the explicitly cropped prompt; one more token than the block holds is
    refused, as TransformerModel.Forward refuses a position past the block (:280-283)."""
    from smallmind_amd.model import ModelConfig
    from tests.helpers import build_pair
    cfg = ModelConfig("llama", 200, 24, 64, 2, 4, 2, 128)
    om, _, _ = build_pair(cfg, O.Q4_K, O.Q6_K, O.Q6_K, seed=5, with_gpu=False)
    prompt = np.random.default_rng(2).integers(0, cfg.vocab_size, 40).astype(np.int32)
    toks, _, _ = om.generate_greedy(prompt, 1)
    s = om.session(24)
    for p, t in enumerate(prompt[-24:-1]):
        s.step(int(t), p, want_logits=False)
    ref = s.step(int(prompt[-1]), 23)
    assert int(toks[0]) == int(np.argmax(ref))
    with pytest.raises(ValueError):
        om.generate_greedy(prompt, 2)
    short, _, _ = om.generate_greedy(prompt[-20:], 5)
    assert short.shape == (5,)
