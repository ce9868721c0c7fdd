"""Operator level of the backend: the IWeightTensor mirror and the per-op entry points.

Mirrors SmallMind.Quantization's operator boundary (IWeightTensor.cs:7-42): a weight knows its
Rows / Cols / Scheme, multiplies activations (`MatMul`, y = x W^T with k == Cols, n == Rows) and
dequantizes to fp32 (`ToFloat32`).  Dimension mismatches raise ValueError as the reference
raises ArgumentException (Q8WeightTensor.cs:43-48).

Device memory is held in torch tensors purely as allocation/stream plumbing; every computation
is a call into libsmx.so.
"""
from __future__ import annotations

import ctypes
from enum import IntEnum

import numpy as np

from . import _lib
from ._lib import SmxError, call


class GgufTensorType(IntEnum):
    """GGUF tensor type ids (GgufTensorType.cs:6-52) the backend implements, and SmallMind's own
    SMQ Q8Tensor / Q4Tensor blocks (1000 + QuantScheme id, QuantScheme.cs) in their upload
    layout (per 32 elements: the fp32 scale of their SMQ block, then the codes; smq_pack)."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q8_0 = 8
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    SMQ_Q8 = 1010
    SMQ_Q4 = 1011


BLOCK_ELEMS = {0: 1, 1: 1, 2: 32, 8: 32, 12: 256, 13: 256, 14: 256, 1010: 32, 1011: 32}
BLOCK_BYTES = {0: 4, 1: 2, 2: 18, 8: 34, 12: 144, 13: 176, 14: 210, 1010: 36, 1011: 20}


def smq_pack(qtype: int, data, scales, rows: int, cols: int, block_size: int) -> np.ndarray:
    """A Q8Tensor / Q4Tensor (codes as stored in an .smq file, fp32 scales per block_size
    elements of the flattened tensor) re-laid as SMX_TYPE_SMQ_Q8 / _Q4 upload bytes; no value
    changes (smx_smq_pack, host memory)."""
    d = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
    sc = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
    out = np.empty(rows * cols // 32 * BLOCK_BYTES[int(qtype)], np.uint8)
    call("smx_smq_pack", int(qtype), d.ctypes.data_as(ctypes.c_void_p), sc.ctypes.data_as(ctypes.c_void_p),
         rows, cols, block_size, out.ctypes.data_as(ctypes.c_void_p), out.size)
    return out


def _torch():
    import torch
    return torch


def _ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    torch = _torch()
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _require_cuda(*ts):
    for t in ts:
        if not t.is_cuda:
            raise ValueError("operands must be device (cuda) tensors")
        if not t.is_contiguous():
            raise ValueError("operands must be contiguous")


def row_bytes(qtype: int, k: int) -> int:
    be = BLOCK_ELEMS[int(qtype)]
    if k % be:
        raise ValueError(f"row length {k} is not a multiple of the block size {be}")
    return k // be * BLOCK_BYTES[int(qtype)]


def dequantize(qtype: int, blocks, n: int):
    """GGUF blocks (device uint8 tensor) -> fp32 device tensor, bit-identical to
    GgufModelLoader.Convert*Tensor (GgufModelLoader.cs:419-917)."""
    torch = _torch()
    _require_cuda(blocks)
    out = torch.empty(n, dtype=torch.float32, device=blocks.device)
    call("smx_dequant", int(qtype), _ptr(blocks), n, _ptr(out), _stream())
    return out


def quantize(qtype: int, x):
    """fp32 device tensor -> GGUF blocks (device uint8 tensor) with the backend encoders."""
    torch = _torch()
    _require_cuda(x)
    n = x.numel()
    be = BLOCK_ELEMS[int(qtype)]
    if n % be:
        raise ValueError(f"{n} elements is not a multiple of the block size {be}")
    out = torch.empty(n // be * BLOCK_BYTES[int(qtype)], dtype=torch.uint8, device=x.device)
    call("smx_quantize", int(qtype), _ptr(x), n, _ptr(out), _stream())
    return out


def fill_normal(seed: int, n: int, std: float, device="cuda"):
    torch = _torch()
    out = torch.empty(n, dtype=torch.float32, device=device)
    call("smx_fill_normal", ctypes.c_uint64(seed), n, std, _ptr(out), _stream())
    return out


class GpuWeightTensor:
    """IWeightTensor backed by a repacked device weight (IWeightTensor.cs:7-42)."""

    def __init__(self, qtype: int, rows: int, cols: int, blocks):
        self._h = ctypes.c_void_p()
        if isinstance(blocks, np.ndarray) or isinstance(blocks, (bytes, bytearray)):
            buf = np.ascontiguousarray(np.frombuffer(blocks, np.uint8) if not isinstance(blocks, np.ndarray)
                                       else blocks.view(np.uint8).reshape(-1))
            if buf.size != rows * row_bytes(qtype, cols):
                raise ValueError("block buffer size does not match rows x cols")
            call("smx_weight_create", int(qtype), rows, cols, buf.ctypes.data_as(ctypes.c_void_p), 0,
                 ctypes.byref(self._h))
        else:
            _require_cuda(blocks)
            if blocks.numel() * blocks.element_size() != rows * row_bytes(qtype, cols):
                raise ValueError("block buffer size does not match rows x cols")
            _torch().cuda.synchronize()
            call("smx_weight_create", int(qtype), rows, cols, _ptr(blocks), 1, ctypes.byref(self._h))
        self.rows, self.cols, self.scheme = rows, cols, GgufTensorType(int(qtype))

    @property
    def Rows(self) -> int:
        return self.rows

    @property
    def Cols(self) -> int:
        return self.cols

    def mat_mul(self, activations, output, m: int, k: int, n: int):
        """IWeightTensor.MatMul: output[m][n] = activations[m][k] . W^T (k == Cols, n == Rows)."""
        _require_cuda(activations, output)
        if k != self.cols or n != self.rows:
            raise ValueError(f"k={k} must equal Cols={self.cols} and n={n} Rows={self.rows}")
        if activations.numel() < m * k or output.numel() < m * n:
            raise ValueError("activation/output buffers are too small")
        call("smx_weight_matmul", self._h, _ptr(activations), _ptr(output), m, k, n, _stream())
        return output

    def mat_mul_host(self, activations: np.ndarray, m: int, k: int, n: int, output: np.ndarray | None = None):
        """IWeightTensor.MatMul with host operands, as the reference takes them
        (ReadOnlySpan<float> activations, Span<float> output): numpy float32 arrays of at least
        m*k and m*n elements; synchronous (smx_weight_matmul_host)."""
        a = np.ascontiguousarray(activations, dtype=np.float32).reshape(-1)
        if output is None:
            output = np.empty((m, n), np.float32)
        if a.size < m * k or output.size < m * n or not output.flags.c_contiguous or output.dtype != np.float32:
            raise ValueError("activation/output buffers are too small or not contiguous float32")
        call("smx_weight_matmul_host", self._h, a.ctypes.data_as(ctypes.c_void_p),
             output.ctypes.data_as(ctypes.c_void_p), m, k, n)
        return output

    def to_float32_host(self) -> np.ndarray:
        """IWeightTensor.ToFloat32 into host memory: [Rows][Cols] float32 (smx_weight_to_float32_host)."""
        out = np.empty((self.rows, self.cols), np.float32)
        call("smx_weight_to_float32_host", self._h, out.ctypes.data_as(ctypes.c_void_p))
        return out

    def to_float32(self):
        """IWeightTensor.ToFloat32: [Rows][Cols] fp32 on the device."""
        torch = _torch()
        out = torch.empty((self.rows, self.cols), dtype=torch.float32, device="cuda")
        call("smx_weight_to_float32", self._h, _ptr(out), _stream())
        return out

    def close(self):
        if getattr(self, "_h", None) and self._h.value and _lib._lib is not None:
            _lib._lib.smx_weight_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        self.close()


# ---- elementwise / attention operators (device tensors) -----------------------------------------
def rmsnorm(x, gamma, eps: float = 1e-5):
    torch = _torch()
    _require_cuda(x, gamma)
    n = x.shape[-1]
    y = torch.empty_like(x)
    call("smx_rmsnorm", _ptr(x), _ptr(gamma), _ptr(y), x.numel() // n, n, eps, _stream())
    return y


def layernorm(x, gamma, beta, eps: float = 1e-5):
    torch = _torch()
    _require_cuda(x, gamma, beta)
    n = x.shape[-1]
    y = torch.empty_like(x)
    call("smx_layernorm", _ptr(x), _ptr(gamma), _ptr(beta), _ptr(y), x.numel() // n, n, eps, _stream())
    return y


def rope_tables(max_pos: int, head_dim: int, theta: float = 10000.0):
    c = np.empty((max_pos, head_dim // 2), np.float32)
    s = np.empty((max_pos, head_dim // 2), np.float32)
    call("smx_rope_tables", max_pos, head_dim, theta, c.ctypes.data_as(ctypes.c_void_p),
         s.ctypes.data_as(ctypes.c_void_p))
    return c, s


def rope_(data, pos0: int, cos_t, sin_t):
    """In place on data [heads][seq][hd]."""
    _require_cuda(data, cos_t, sin_t)
    h, s, hd = data.shape
    call("smx_rope", _ptr(data), h, s, hd, pos0, _ptr(cos_t), _ptr(sin_t), _stream())
    return data


def scale_mask_softmax_(scores, scale: float, cache_offset: int = 0):
    _require_cuda(scores)
    seq, kseq = scores.shape
    call("smx_scale_mask_softmax", _ptr(scores), scale, seq, kseq, cache_offset, _stream())
    return scores


def attention_decode(q, k_cache, v_cache, n_head: int, n_kv_head: int, head_dim: int,
                     ctx_stride: int, n_pos: int):
    torch = _torch()
    _require_cuda(q, k_cache, v_cache)
    out = torch.empty(n_head * head_dim, dtype=torch.float32, device=q.device)
    call("smx_attention_decode", _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), n_head,
         n_kv_head, head_dim, ctx_stride, n_pos, _stream())
    return out


def attention_prefill(q, k_cache, v_cache, n_head: int, n_kv_head: int, head_dim: int,
                      ctx_stride: int, p_first: int, n_tok: int):
    torch = _torch()
    _require_cuda(q, k_cache, v_cache)
    out = torch.empty(n_tok * n_head * head_dim, dtype=torch.float32, device=q.device)
    call("smx_attention_prefill", _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), n_head,
         n_kv_head, head_dim, ctx_stride, p_first, n_tok, _stream())
    return out


def silu_mul(gate, up):
    torch = _torch()
    _require_cuda(gate, up)
    y = torch.empty_like(gate)
    call("smx_silu_mul", _ptr(gate), _ptr(up), _ptr(y), gate.numel(), _stream())
    return y


def gelu(x):
    torch = _torch()
    _require_cuda(x)
    y = torch.empty_like(x)
    call("smx_gelu", _ptr(x), _ptr(y), x.numel(), _stream())
    return y


def argmax(x) -> int:
    torch = _torch()
    _require_cuda(x)
    out = torch.empty(1, dtype=torch.int32, device=x.device)
    call("smx_argmax", _ptr(x), x.numel(), _ptr(out), _stream())
    return int(out.item())


def sample(logits, u: float, context=None, temperature: float = 1.0, top_k: int = 0, top_p: float = 1.0,
           min_p: float = 0.0, repetition_penalty: float = 1.0, presence_penalty: float = 0.0,
           frequency_penalty: float = 0.0, repetition_window: int = 0):
    """Next-token sampling in InferenceSession's order (InferenceSession.cs:565-606) on the
    device: (token, final probabilities).  logits and context (int32 token ids, oldest first)
    are cuda tensors; u in [0, 1) is the uniform draw (Random.NextDouble in the reference)."""
    torch = _torch()
    _require_cuda(logits)
    p = _lib.SamplingC(temperature, top_k, top_p, min_p, repetition_penalty, presence_penalty,
                       frequency_penalty, repetition_window)
    probs = torch.empty_like(logits)
    out = torch.empty(1, dtype=torch.int32, device=logits.device)
    n_ctx = 0 if context is None else context.numel()
    call("smx_sample", _ptr(logits), logits.numel(), _ptr(context) if n_ctx else None, n_ctx, ctypes.byref(p),
         float(u), _ptr(probs), _ptr(out), _stream())
    return int(out.item()), probs


__all__ = ["GgufTensorType", "GpuWeightTensor", "SmxError", "dequantize", "quantize", "fill_normal",
           "rmsnorm", "layernorm", "rope_tables", "rope_", "scale_mask_softmax_", "attention_decode",
           "silu_mul", "gelu", "argmax", "sample", "row_bytes", "BLOCK_ELEMS", "BLOCK_BYTES"]
