"""ctypes front-end of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker or the timed CPU baseline.  The product package
(smallmind_amd) never imports this module.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 8, 12, 13, 14
SMQ_Q8, SMQ_Q4 = 1010, 1011   # SMQ Q8Tensor / Q4Tensor blocks re-laid per 32 (fp32 scale + codes)
ARCH_LLAMA, ARCH_GPT2 = 0, 1

BLOCK_ELEMS = {F32: 1, F16: 1, Q4_0: 32, Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, SMQ_Q8: 32, SMQ_Q4: 32}
BLOCK_BYTES = {F32: 4, F16: 2, Q4_0: 18, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210, SMQ_Q8: 36, SMQ_Q4: 20}


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "liboracle.so"], cwd=_HERE, check=True)
    return _LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        c_f32p = ctypes.POINTER(ctypes.c_float)
        vp = ctypes.c_void_p
        L.smxo_half_to_float.restype = ctypes.c_float
        L.smxo_half_to_float.argtypes = [ctypes.c_uint16]
        L.smxo_float_to_half.restype = ctypes.c_uint16
        L.smxo_float_to_half.argtypes = [ctypes.c_float]
        L.smxo_dequant.argtypes = [ctypes.c_int, vp, ctypes.c_int64, vp]
        L.smxo_quantize.argtypes = [ctypes.c_int, vp, ctypes.c_int64, vp]
        L.smxo_quantize_ref_q8.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp, vp]
        L.smxo_quantize_ref_q4.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp, vp]
        L.smxo_dequant_smq.argtypes = [ctypes.c_int, vp, vp, ctypes.c_int64, ctypes.c_int, vp]
        L.smxo_gemv_f64.argtypes = [ctypes.c_int, vp, ctypes.c_int, ctypes.c_int, vp, vp]
        L.smxo_rmsnorm.argtypes = [vp, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_float]
        L.smxo_layernorm.argtypes = [vp, vp, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_float]
        L.smxo_rope_tables.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_float, vp, vp]
        L.smxo_rope_apply.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp]
        L.smxo_fastexp.restype = ctypes.c_float
        L.smxo_fastexp.argtypes = [ctypes.c_float]
        L.smxo_scale_mask_softmax.argtypes = [vp, ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.smxo_gelu.argtypes = [vp, vp, ctypes.c_int]
        L.smxo_silu_mul.argtypes = [vp, vp, vp, ctypes.c_int]
        L.smxo_argmax.argtypes = [vp, ctypes.c_int]
        L.smxo_sample.argtypes = [vp, ctypes.c_int, vp, ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_double,
                                  ctypes.c_double, ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_int,
                                  ctypes.c_double, vp]
        L.smxo_fill_normal.argtypes = [ctypes.c_uint64, ctypes.c_int64, ctypes.c_float, vp]
        L.smxo_model_create.restype = vp
        L.smxo_model_create.argtypes = [ctypes.c_int] * 8 + [ctypes.c_float, ctypes.c_float]
        L.smxo_model_set_tensor.argtypes = [vp, ctypes.c_char_p, ctypes.c_int, vp, ctypes.c_int64]
        L.smxo_model_finalize.argtypes = [vp]
        L.smxo_model_destroy.argtypes = [vp]
        L.smxo_forward_nocache.argtypes = [vp, vp, ctypes.c_int, vp, ctypes.c_int]
        L.smxo_session_create.restype = vp
        L.smxo_session_create.argtypes = [vp, ctypes.c_int]
        L.smxo_session_step.argtypes = [vp, ctypes.c_int32, ctypes.c_int, vp]
        L.smxo_session_prefill.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, vp]
        L.smxo_multi_step.argtypes = [vp, vp, vp, ctypes.c_int, vp]
        L.smxo_step_tokens.argtypes = [vp, vp, vp, ctypes.c_int, vp, ctypes.c_int]
        L.smxo_set_threads.argtypes = [ctypes.c_int]
        L.smxo_get_threads.restype = ctypes.c_int
        L.smxo_session_destroy.argtypes = [vp]
        L.smxo_generate_greedy.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, vp, vp, vp]
        _ = c_f32p
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def half_to_float(h: int) -> float:
    return lib().smxo_half_to_float(h)


def float_to_half(f: float) -> int:
    return lib().smxo_float_to_half(f)


def row_bytes(qtype: int, k: int) -> int:
    return k // BLOCK_ELEMS[qtype] * BLOCK_BYTES[qtype]


def dequant(qtype: int, blocks: np.ndarray, n: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks).reshape(-1).view(np.uint8)
    out = np.empty(n, np.float32)
    rc = lib().smxo_dequant(qtype, _p(blocks), n, _p(out))
    if rc:
        raise ValueError(f"smxo_dequant failed ({rc})")
    return out


def quantize(qtype: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    n = x.size
    if n % BLOCK_ELEMS[qtype]:
        raise ValueError("length must be a multiple of the block size")
    out = np.zeros(n // BLOCK_ELEMS[qtype] * BLOCK_BYTES[qtype], np.uint8)
    rc = lib().smxo_quantize(qtype, _p(x), n, _p(out))
    if rc:
        raise ValueError(f"smxo_quantize failed ({rc})")
    return out


def quantize_ref_q8(x: np.ndarray, block: int = 64):
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.zeros(x.size, np.int8)
    s = np.zeros((x.size + block - 1) // block, np.float32)
    lib().smxo_quantize_ref_q8(_p(x), x.size, block, _p(q), _p(s))
    return q, s


def quantize_ref_q4(x: np.ndarray, block: int = 64):
    x = np.ascontiguousarray(x, dtype=np.float32)
    d = np.zeros((x.size + 1) // 2, np.uint8)
    s = np.zeros((x.size + block - 1) // block, np.float32)
    lib().smxo_quantize_ref_q4(_p(x), x.size, block, _p(d), _p(s))
    return d, s


def dequant_smq(scheme: int, data: np.ndarray, scales: np.ndarray, n: int, block: int) -> np.ndarray:
    """Q8Tensor.Dequantize (scheme 10) / Q4Tensor.Dequantize (scheme 11) of n flattened elements."""
    d = np.ascontiguousarray(data).view(np.uint8)
    sc = np.ascontiguousarray(scales, dtype=np.float32)
    out = np.empty(n, np.float32)
    if lib().smxo_dequant_smq(scheme, _p(d), _p(sc), n, block, _p(out)):
        raise ValueError("dequant_smq failed")
    return out


def gemv_f64(qtype: int, W: np.ndarray, N: int, K: int, x: np.ndarray) -> np.ndarray:
    W = np.ascontiguousarray(W, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(N, np.float64)
    rc = lib().smxo_gemv_f64(qtype, _p(W), N, K, _p(x), _p(y))
    if rc:
        raise ValueError(f"smxo_gemv_f64 failed ({rc})")
    return y


def rmsnorm(x: np.ndarray, g: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = np.ascontiguousarray(g, dtype=np.float32)
    y = np.empty_like(x)
    n = x.shape[-1]
    lib().smxo_rmsnorm(_p(x), _p(g), _p(y), x.size // n, n, eps)
    return y


def layernorm(x, g, b, eps: float = 1e-5) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = np.ascontiguousarray(g, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    y = np.empty_like(x)
    n = x.shape[-1]
    lib().smxo_layernorm(_p(x), _p(g), _p(b), _p(y), x.size // n, n, eps)
    return y


def rope_tables(max_pos: int, head_dim: int, theta: float):
    c = np.empty((max_pos, head_dim // 2), np.float32)
    s = np.empty((max_pos, head_dim // 2), np.float32)
    lib().smxo_rope_tables(max_pos, head_dim, theta, _p(c), _p(s))
    return c, s


def rope_apply(data: np.ndarray, pos0: int, cos_t, sin_t) -> np.ndarray:
    """data: [heads][seq][hd] float32, rotated in a copy."""
    d = np.ascontiguousarray(data, dtype=np.float32).copy()
    h, s, hd = d.shape
    lib().smxo_rope_apply(_p(d), pos0, h, s, hd, _p(np.ascontiguousarray(cos_t)),
                          _p(np.ascontiguousarray(sin_t)))
    return d


def fastexp(x: float) -> float:
    return lib().smxo_fastexp(x)


def scale_mask_softmax(scores: np.ndarray, scale: float, cache_off: int = 0) -> np.ndarray:
    s = np.ascontiguousarray(scores, dtype=np.float32).copy()
    seq, kseq = s.shape
    lib().smxo_scale_mask_softmax(_p(s), scale, seq, kseq, cache_off)
    return s


def gelu(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().smxo_gelu(_p(x), _p(y), x.size)
    return y


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    y = np.empty_like(g)
    lib().smxo_silu_mul(_p(g), _p(u), _p(y), g.size)
    return y


def sample(logits: np.ndarray, u: float, context=(), temperature: float = 1.0, top_k: int = 0,
           top_p: float = 1.0, min_p: float = 0.0, repetition_penalty: float = 1.0,
           presence_penalty: float = 0.0, frequency_penalty: float = 0.0, window: int = 0):
    """(token, final probabilities) of the reference's sampling pipeline at the draw u."""
    lg = np.ascontiguousarray(logits, np.float32)
    ctx = np.ascontiguousarray(np.asarray(context, np.int32))
    probs = np.empty_like(lg)
    tok = lib().smxo_sample(_p(lg), lg.size, _p(ctx) if ctx.size else None, ctx.size, temperature, top_k, top_p,
                            min_p, repetition_penalty, presence_penalty, frequency_penalty, window, u, _p(probs))
    return int(tok), probs


def set_threads(n: int) -> None:
    """Threads for the oracle's linears and attention (0 = all cores).  Results are
    bit-identical for every thread count."""
    lib().smxo_set_threads(int(n))


def get_threads() -> int:
    return int(lib().smxo_get_threads())


def fill_normal(seed: int, n: int, std: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().smxo_fill_normal(seed, n, std, _p(out))
    return out


class OracleModel:
    """The reference forward (TransformerModel.Forward) on fp32 weights dequantized at load."""

    def __init__(self, arch, vocab, ctx, d, n_layer, n_head, n_kv_head, ff, rope_theta=10000.0,
                 norm_eps=1e-5):
        self.vocab = vocab
        self._h = lib().smxo_model_create(arch, vocab, ctx, d, n_layer, n_head, n_kv_head, ff,
                                          rope_theta, norm_eps)
        if not self._h:
            raise ValueError("invalid oracle model shape")

    def set_tensor(self, name: str, qtype: int, data: np.ndarray, n_elems: int):
        data = np.ascontiguousarray(data).view(np.uint8)
        rc = lib().smxo_model_set_tensor(self._h, name.encode(), qtype, _p(data), n_elems)
        if rc:
            raise ValueError(f"set_tensor({name}) failed ({rc})")

    def finalize(self):
        rc = lib().smxo_model_finalize(self._h)
        if rc:
            raise ValueError(f"finalize failed ({rc})")

    def forward_nocache(self, tokens, all_rows=False) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty((t.size if all_rows else 1) * self.vocab, np.float32)
        rc = lib().smxo_forward_nocache(self._h, _p(t), t.size, _p(out), int(all_rows))
        if rc:
            raise ValueError(f"forward_nocache failed ({rc})")
        return out.reshape(-1, self.vocab) if all_rows else out

    def session(self, max_ctx: int) -> "OracleSession":
        return OracleSession(self, max_ctx)

    def multi_step(self, sessions, tokens, positions) -> np.ndarray:
        """One token per session (distinct sessions of this model) in one batched pass;
        logits [n][V], bit-identical to n OracleSession.step calls."""
        n = len(sessions)
        hs = (ctypes.c_void_p * n)(*[s._h for s in sessions])
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        p = np.ascontiguousarray(positions, dtype=np.int32)
        out = np.empty((n, self.vocab), np.float32)
        rc = lib().smxo_multi_step(hs, _p(t), _p(p), n, _p(out))
        if rc:
            raise ValueError(f"multi_step failed ({rc})")
        return out

    def prefill_many(self, sessions, prompts):
        """Each session's prompt at positions 0.. in one batched pass (all prompts' tokens share
        every weight load); bit-identical to prefilling each session token by token."""
        ss, toks, pos = [], [], []
        for s, p in zip(sessions, prompts):
            p = np.asarray(p, np.int32).reshape(-1)
            ss += [s._h] * p.size
            toks.append(p)
            pos.append(np.arange(p.size, dtype=np.int32))
        n = len(ss)
        if n == 0:
            return
        hs = (ctypes.c_void_p * n)(*ss)
        t = np.ascontiguousarray(np.concatenate(toks), dtype=np.int32)
        q = np.ascontiguousarray(np.concatenate(pos), dtype=np.int32)
        rc = lib().smxo_step_tokens(hs, _p(t), _p(q), n, None, n)
        if rc:
            raise ValueError(f"step_tokens failed ({rc})")

    def generate_greedy(self, prompt, n_new):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(n_new, np.int32)
        pre = ctypes.c_int64(0)
        dec = ctypes.c_int64(0)
        rc = lib().smxo_generate_greedy(self._h, _p(p), p.size, n_new, _p(out),
                                        ctypes.byref(pre), ctypes.byref(dec))
        if rc:
            raise ValueError(f"generate_greedy failed ({rc})")
        return out, pre.value * 1e-9, dec.value * 1e-9

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.smxo_model_destroy(h)
            self._h = None


class OracleSession:
    def __init__(self, model: OracleModel, max_ctx: int):
        self.model = model
        self._h = lib().smxo_session_create(model._h, max_ctx)
        if not self._h:
            raise ValueError("session create failed")

    def step(self, token: int, pos: int, want_logits=True):
        out = np.empty(self.model.vocab, np.float32) if want_logits else None
        rc = lib().smxo_session_step(self._h, token, pos, _p(out) if want_logits else None)
        if rc:
            raise ValueError(f"session_step failed ({rc})")
        return out

    def prefill(self, tokens, pos0: int = 0, want_logits: bool = False):
        """tokens at positions pos0.. in one batched pass (bit-identical to step() per token);
        returns the last token's logits when want_logits."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty(self.model.vocab, np.float32) if want_logits else None
        rc = lib().smxo_session_prefill(self._h, _p(t), t.size, pos0, _p(out) if want_logits else None)
        if rc:
            raise ValueError(f"session_prefill failed ({rc})")
        return out

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.smxo_session_destroy(h)
            self._h = None
