"""ctypes binding of libsmx.so (the C-ABI declared in include/smx.h).

The product path always runs through this library; there is no CPU fallback.  Importing
fails loudly when the library has not been built.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsmx.so")

# GGUF tensor type ids (GgufTensorType.cs:6-52)
F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 8, 12, 13, 14
ARCH_LLAMA, ARCH_GPT2 = 0, 1

STATUS = {0: "SMX_OK", -1: "SMX_EINVAL", -2: "SMX_ENOMEM", -3: "SMX_EDEVICE", -4: "SMX_EBUSY",
          -5: "SMX_EUNSUPPORTED", -6: "SMX_ESTATE", -7: "SMX_ERANGE", -8: "SMX_ECANCELED",
          -9: "SMX_ETIMEDOUT"}
ECANCELED, ETIMEDOUT = -8, -9

# Every function include/smx.h declares.
EXPORTS = [
    "smx_version", "smx_last_error", "smx_type_block_elems", "smx_type_block_bytes",
    "smx_type_row_bytes", "smx_dequant", "smx_quantize", "smx_fill_normal",
    "smx_weight_create", "smx_weight_info", "smx_weight_matmul", "smx_weight_matmul_noalloc",
    "smx_weight_matmul_host", "smx_weight_to_float32", "smx_weight_to_float32_host",
    "smx_weight_destroy", "smx_rmsnorm", "smx_layernorm", "smx_rope_tables", "smx_rope",
    "smx_scale_mask_softmax", "smx_attention_decode", "smx_attention_prefill", "smx_silu_mul", "smx_gelu", "smx_argmax", "smx_stream_read",
    "smx_context_create", "smx_context_destroy", "smx_model_create", "smx_model_upload_tensor",
    "smx_model_finalize", "smx_model_weight_bytes", "smx_model_destroy", "smx_session_create",
    "smx_session_forward", "smx_session_generate", "smx_session_cancel", "smx_session_set_max_time",
    "smx_batch_generate", "smx_session_reset",
    "smx_session_destroy", "smx_model_load_gguf", "smx_gguf_read_config", "smx_model_load_smq",
    "smx_smq_read_config", "smx_smq_pack", "smx_sample",
    "smx_session_generate_sampled", "smx_batcher_create", "smx_batcher_add", "smx_batcher_add_sampled", "smx_batcher_remove",
    "smx_batcher_count", "smx_batcher_step", "smx_batcher_destroy",
]


class SmxError(RuntimeError):
    def __init__(self, func: str, code: int, msg: str):
        super().__init__(f"{func} -> {STATUS.get(code, code)}: {msg}")
        self.code = code


class GenerationCancelled(SmxError):
    """SMX_ECANCELED: the generation stopped on a cancel request (the OperationCanceledException
    of InferenceSession's CancellationToken, InferenceSession.cs:211, :481).  `tokens` holds what
    was produced before the stop (the first tokens of the uninterrupted run)."""
    tokens = None


class GenerationTimeout(SmxError):
    """SMX_ETIMEDOUT: the generation stopped at the session's time limit (InferenceTimeoutException,
    InferenceSession.cs:164-172, :287-291).  `tokens` holds what was produced before the stop."""
    tokens = None


class ModelConfigC(ctypes.Structure):
    _fields_ = [("arch", ctypes.c_int32), ("vocab", ctypes.c_int32), ("ctx", ctypes.c_int32),
                ("d_model", ctypes.c_int32), ("n_layer", ctypes.c_int32),
                ("n_head", ctypes.c_int32), ("n_kv_head", ctypes.c_int32),
                ("d_ff", ctypes.c_int32), ("rope_theta", ctypes.c_float),
                ("norm_eps", ctypes.c_float), ("reserved", ctypes.c_int32 * 6)]


class SamplingC(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_int32), ("top_p", ctypes.c_double),
                ("min_p", ctypes.c_float), ("repetition_penalty", ctypes.c_float),
                ("presence_penalty", ctypes.c_float), ("frequency_penalty", ctypes.c_float),
                ("repetition_window", ctypes.c_int32)]


class GenStatsC(ctypes.Structure):
    _fields_ = [("prefill_ms", ctypes.c_double), ("decode_ms", ctypes.c_double),
                ("n_prefill_steps", ctypes.c_int32), ("n_decode_steps", ctypes.c_int32)]


_lib = None


def load() -> ctypes.CDLL:
    """Loads libsmx.so; raises ImportError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: the HIP backend has not been built "
            "(run `python -c 'import __graft_entry__ as g; g.build()'`). There is no CPU fallback.")
    # torch ships its own libamdhip64 / libhsa-runtime64 with the same SONAMEs as ROCm's.  Two
    # HIP runtimes in one process do not share the device, so when torch is present it is
    # loaded first and libsmx.so binds to the runtime already in the process.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = ctypes.CDLL(LIB_PATH)
    vp, i32, i64, f32, u64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_uint64
    pp = ctypes.POINTER(ctypes.c_void_p)
    sig = {
        "smx_version": (ctypes.c_char_p, []),
        "smx_last_error": (ctypes.c_char_p, []),
        "smx_type_block_elems": (i32, [i32]),
        "smx_type_block_bytes": (i32, [i32]),
        "smx_type_row_bytes": (i64, [i32, i64]),
        "smx_dequant": (i32, [i32, vp, i64, vp, vp]),
        "smx_quantize": (i32, [i32, vp, i64, vp, vp]),
        "smx_fill_normal": (i32, [u64, i64, f32, vp, vp]),
        "smx_weight_create": (i32, [i32, i64, i64, vp, i32, pp]),
        "smx_weight_info": (i32, [vp, ctypes.POINTER(i32), ctypes.POINTER(i64), ctypes.POINTER(i64)]),
        "smx_weight_matmul": (i32, [vp, vp, vp, i32, i32, i32, vp]),
        "smx_weight_matmul_noalloc": (i32, [vp, vp, vp, i32, i32, i32, vp]),
        "smx_weight_matmul_host": (i32, [vp, vp, vp, i32, i32, i32]),
        "smx_weight_to_float32_host": (i32, [vp, vp]),
        "smx_weight_to_float32": (i32, [vp, vp, vp]),
        "smx_weight_destroy": (i32, [vp]),
        "smx_rmsnorm": (i32, [vp, vp, vp, i32, i32, f32, vp]),
        "smx_layernorm": (i32, [vp, vp, vp, vp, i32, i32, f32, vp]),
        "smx_rope_tables": (i32, [i32, i32, f32, vp, vp]),
        "smx_rope": (i32, [vp, i32, i32, i32, i32, vp, vp, vp]),
        "smx_scale_mask_softmax": (i32, [vp, f32, i32, i32, i32, vp]),
        "smx_attention_decode": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, i32, vp]),
        "smx_attention_prefill": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, vp]),
        "smx_silu_mul": (i32, [vp, vp, vp, i64, vp]),
        "smx_gelu": (i32, [vp, vp, i64, vp]),
        "smx_argmax": (i32, [vp, i32, vp, vp]),
        "smx_stream_read": (i32, [vp, u64, vp]),
        "smx_sample": (i32, [vp, i32, vp, i32, ctypes.POINTER(SamplingC), ctypes.c_double, vp, vp, vp]),
        "smx_context_create": (i32, [i32, pp]),
        "smx_context_destroy": (i32, [vp]),
        "smx_model_create": (i32, [vp, ctypes.POINTER(ModelConfigC), pp]),
        "smx_model_upload_tensor": (i32, [vp, ctypes.c_char_p, i32, ctypes.POINTER(i64), i32, vp,
                                          ctypes.c_size_t, i32]),
        "smx_model_finalize": (i32, [vp]),
        "smx_model_load_gguf": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(vp)]),
        "smx_gguf_read_config": (i32, [ctypes.c_char_p, ctypes.POINTER(ModelConfigC), ctypes.POINTER(ctypes.c_int64)]),
        "smx_model_load_smq": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(ModelConfigC), ctypes.POINTER(vp)]),
        "smx_smq_read_config": (i32, [ctypes.c_char_p, ctypes.POINTER(ModelConfigC), ctypes.POINTER(ctypes.c_int64)]),
        "smx_smq_pack": (i32, [i32, vp, vp, i64, i64, i32, vp, ctypes.c_size_t]),
        "smx_model_weight_bytes": (i32, [vp, ctypes.POINTER(i64)]),
        "smx_model_destroy": (i32, [vp]),
        "smx_session_create": (i32, [vp, i32, pp]),
        "smx_session_forward": (i32, [vp, vp, i32, i32, vp]),
        "smx_session_generate": (i32, [vp, vp, i32, i32, vp, vp, ctypes.POINTER(GenStatsC)]),
        "smx_session_cancel": (i32, [vp]),
        "smx_session_set_max_time": (i32, [vp, ctypes.c_int32]),
        "smx_batch_generate": (i32, [vp, i32, vp, vp, i32, vp, ctypes.POINTER(GenStatsC)]),
        "smx_session_generate_sampled": (i32, [vp, vp, i32, i32, ctypes.POINTER(SamplingC), ctypes.c_uint64, vp, vp,
                                               ctypes.POINTER(GenStatsC)]),
        "smx_batcher_create": (i32, [vp, i32, i32, pp]),
        "smx_batcher_add": (i32, [vp, vp, vp, i32]),
        "smx_batcher_add_sampled": (i32, [vp, vp, vp, i32, ctypes.POINTER(SamplingC), ctypes.c_uint64]),
        "smx_batcher_remove": (i32, [vp, vp]),
        "smx_batcher_count": (i32, [vp]),
        "smx_batcher_step": (i32, [vp, i32, vp]),
        "smx_batcher_destroy": (i32, [vp]),
        "smx_session_reset": (i32, [vp]),
        "smx_session_destroy": (i32, [vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def call(name: str, *args) -> int:
    """Calls a status-returning C-ABI function and raises SmxError on failure (GenerationCancelled
    / GenerationTimeout for a stopped generation)."""
    L = load()
    rc = getattr(L, name)(*args)
    if rc != 0:
        cls = {ECANCELED: GenerationCancelled, ETIMEDOUT: GenerationTimeout}.get(rc, SmxError)
        raise cls(name, rc, (L.smx_last_error() or b"").decode(errors="replace"))
    return rc
