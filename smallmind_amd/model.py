"""Model / session level of the backend.

GpuTransformerModel replaces TransformerModel (TransformerModel.cs:81-344) for inference:
weights are uploaded by GGUF tensor name (as GgufModelLoader maps them, GgufModelLoader.cs:
117-187, with the Q/K/V merge of :1027-1110 and the weight tying of :1126-1147) and stay
quantized on the device.  GpuInferenceSession mirrors the KV-cached Forward(idx,
positionOffset) calls InferenceSession makes (InferenceSession.cs:478-546) and adds greedy
generation that runs entirely on the device.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from ._lib import ARCH_GPT2, ARCH_LLAMA, GenerationCancelled, GenerationTimeout, GenStatsC, ModelConfigC, call, load


def uniform_draw(seed: int, i: int) -> float:
    """Draw i of smx_session_generate_sampled's stream: splitmix64(seed + i), top 53 bits."""
    m = (1 << 64) - 1
    z = (seed + i + 0x9E3779B97F4A7C15) & m
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    z ^= z >> 31
    return (z >> 11) / 9007199254740992.0


@dataclass
class ModelConfig:
    """Fields of SmallMind's ModelConfig (ModelConfig.cs:142-258) the forward path reads."""
    architecture: str            # "llama" (RoPE, RMSNorm, SwiGLU) or "gpt2" (learned pos, LayerNorm, GELU)
    vocab_size: int
    context_length: int
    embedding_length: int
    block_count: int
    head_count: int
    head_count_kv: int
    feed_forward_length: int
    rope_freq_base: float = 10000.0
    norm_eps: float = 1e-5

    @property
    def head_dim(self) -> int:
        return self.embedding_length // self.head_count

    @property
    def kv_dim(self) -> int:
        return self.head_count_kv * self.head_dim

    @property
    def hidden_dim(self) -> int:
        return 4 * self.embedding_length if self.architecture == "gpt2" else self.feed_forward_length

    def to_c(self) -> ModelConfigC:
        c = ModelConfigC()
        c.arch = ARCH_GPT2 if self.architecture == "gpt2" else ARCH_LLAMA
        c.vocab = self.vocab_size
        c.ctx = self.context_length
        c.d_model = self.embedding_length
        c.n_layer = self.block_count
        c.n_head = self.head_count
        c.n_kv_head = self.head_count_kv
        c.d_ff = self.feed_forward_length
        c.rope_theta = self.rope_freq_base
        c.norm_eps = self.norm_eps
        return c


def _config_from_c(c: ModelConfigC) -> ModelConfig:
    return ModelConfig("gpt2" if c.arch == ARCH_GPT2 else "llama", c.vocab, c.ctx, c.d_model, c.n_layer,
                       c.n_head, c.n_kv_head, c.d_ff, float(c.rope_theta), float(c.norm_eps))


def read_gguf_config(path: str) -> ModelConfig:
    """The ModelConfig a GGUF file's metadata describes (smx_gguf_read_config; no device work)."""
    c = ModelConfigC()
    n = ctypes.c_int64()
    call("smx_gguf_read_config", str(path).encode(), ctypes.byref(c), ctypes.byref(n))
    return _config_from_c(c)


def read_smq_config(path: str) -> ModelConfig:
    """The GPT-2 ModelConfig an .smq file's metadata describes (vocab_size, block_size,
    embed_dim, num_layers, num_heads; smx_smq_read_config; no device work)."""
    c = ModelConfigC()
    n = ctypes.c_int64()
    call("smx_smq_read_config", str(path).encode(), ctypes.byref(c), ctypes.byref(n))
    return _config_from_c(c)


class GpuContext:
    def __init__(self, device: int = 0):
        load()
        self._h = ctypes.c_void_p()
        call("smx_context_create", device, ctypes.byref(self._h))
        self.device = device

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            call("smx_context_destroy", self._h)
            self._h = ctypes.c_void_p()


class GpuTransformerModel:
    """TransformerModel for the GPU backend (weights stay quantized on the device)."""

    def __init__(self, config: ModelConfig, context: GpuContext | None = None, device: int = 0):
        self.config = config
        self.context = context or GpuContext(device)
        self._own_ctx = context is None
        self._cfg = config.to_c()
        self._h = ctypes.c_void_p()
        call("smx_model_create", self.context._h, ctypes.byref(self._cfg), ctypes.byref(self._h))
        self._sessions = []

    @classmethod
    def from_gguf(cls, path: str, context: GpuContext | None = None, device: int = 0) -> "GpuTransformerModel":
        """Loads a GGUF file (GgufModelLoader, GgufModelLoader.cs:63-77): configuration from the
        metadata (ModelConfig.FromGgufMetadata, ModelConfig.cs:142-214), every tensor uploaded
        from a memory map of the file, the model finalized (smx_model_load_gguf)."""
        return cls._loaded(read_gguf_config(path), context, device,
                           lambda ctx, out: call("smx_model_load_gguf", ctx, str(path).encode(), out))

    @classmethod
    def from_smq(cls, path: str, config: ModelConfig | None = None, context: GpuContext | None = None,
                 device: int = 0) -> "GpuTransformerModel":
        """Loads a SmallMind .smq file into the GPT-2 TransformerModel (SmqModelLoader.LoadFromSmq,
        SmqModelLoader.cs:29-100): `config` plays the reference's ModelConfig argument, None
        takes it from the file's metadata; Q8_0 / Q4_0 weight matrices stay quantized on the
        device with the file's scales (smx_model_load_smq)."""
        config = config or read_smq_config(path)
        cfg = config.to_c()
        return cls._loaded(config, context, device,
                           lambda ctx, out: call("smx_model_load_smq", ctx, str(path).encode(), ctypes.byref(cfg),
                                                 out))

    @classmethod
    def _loaded(cls, config: ModelConfig, context, device: int, load) -> "GpuTransformerModel":
        self = cls.__new__(cls)
        self.config = config
        self.context = context or GpuContext(device)
        self._own_ctx = context is None
        self._cfg = config.to_c()
        self._h = ctypes.c_void_p()
        self._sessions = []
        try:
            load(self.context._h, ctypes.byref(self._h))
        except Exception:
            if self._own_ctx:
                self.context.close()
            raise
        return self

    def load_tensor(self, name: str, qtype: int, dims, data):
        """Uploads one GGUF tensor.  dims are GGUF order (ne0 first).  data is a host buffer
        (numpy / bytes) or a device torch tensor."""
        d = (ctypes.c_int64 * len(dims))(*[int(x) for x in dims])
        if isinstance(data, (bytes, bytearray, np.ndarray)):
            buf = np.ascontiguousarray(np.frombuffer(data, np.uint8) if not isinstance(data, np.ndarray)
                                       else data).view(np.uint8).reshape(-1)
            call("smx_model_upload_tensor", self._h, name.encode(), int(qtype), d, len(dims),
                 buf.ctypes.data_as(ctypes.c_void_p), buf.size, 0)
        else:
            import torch
            if not data.is_cuda or not data.is_contiguous():
                raise ValueError("device tensors must be contiguous cuda tensors")
            torch.cuda.synchronize()
            call("smx_model_upload_tensor", self._h, name.encode(), int(qtype), d, len(dims),
                 ctypes.c_void_p(data.data_ptr()), data.numel() * data.element_size(), 1)

    def finalize(self):
        call("smx_model_finalize", self._h)

    def weight_bytes(self) -> int:
        b = ctypes.c_int64()
        call("smx_model_weight_bytes", self._h, ctypes.byref(b))
        return b.value

    def create_session(self, max_ctx: int | None = None) -> "GpuInferenceSession":
        s = GpuInferenceSession(self, max_ctx or self.config.context_length)
        self._sessions.append(s)
        return s

    def close(self):
        for b in list(getattr(self, "_batchers", [])):
            b.close()
        self._batchers = []
        for s in list(self._sessions):
            s.close()
        self._sessions = []
        if getattr(self, "_h", None) and self._h.value:
            call("smx_model_destroy", self._h)
            self._h = ctypes.c_void_p()
        if self._own_ctx:
            self.context.close()


class GpuInferenceSession:
    """KV-cached decoding session (one HIP stream, one captured decode-step graph).

    Not thread-safe, like InferenceSession (InferenceSession.cs:127-144): concurrent use
    raises SmxError with SMX_EBUSY."""

    def __init__(self, model: GpuTransformerModel, max_ctx: int):
        self.model = model
        self.max_ctx = max_ctx
        self._h = ctypes.c_void_p()
        call("smx_session_create", model._h, max_ctx, ctypes.byref(self._h))

    def forward(self, tokens, position_offset: int, want_logits: bool = True):
        """TransformerModel.Forward(idx[1,T], positionOffset) with the KV cache enabled;
        returns the last row's logits."""
        t = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
        out = np.empty(self.model.config.vocab_size, np.float32) if want_logits else None
        call("smx_session_forward", self._h, t.ctypes.data_as(ctypes.c_void_p), t.size,
             position_offset, out.ctypes.data_as(ctypes.c_void_p) if want_logits else None)
        return out

    def generate_greedy(self, prompt, max_new_tokens: int, return_logits: bool = False):
        """Prefill + greedy decode on the device.  Returns (tokens, stats[, logits]).  A prompt
        longer than the session context is cropped to its last max_ctx tokens.  A cancel request
        or the time limit stops it between graph launches: GenerationCancelled /
        GenerationTimeout, whose `tokens` are the ones produced before the stop."""
        p = np.ascontiguousarray(prompt, dtype=np.int32).reshape(-1)
        toks = np.empty(max_new_tokens, np.int32)
        logits = (np.empty((max_new_tokens, self.model.config.vocab_size), np.float32)
                  if return_logits else None)
        st = GenStatsC()
        try:
            call("smx_session_generate", self._h, p.ctypes.data_as(ctypes.c_void_p), p.size,
                 max_new_tokens, toks.ctypes.data_as(ctypes.c_void_p),
                 logits.ctypes.data_as(ctypes.c_void_p) if return_logits else None, ctypes.byref(st))
        except (GenerationCancelled, GenerationTimeout) as e:
            e.tokens = toks[:st.n_decode_steps].copy()
            raise
        stats = {"prefill_ms": st.prefill_ms, "decode_ms": st.decode_ms,
                 "prefill_steps": st.n_prefill_steps, "decode_steps": st.n_decode_steps}
        return (toks, stats, logits) if return_logits else (toks, stats)

    def generate_sampled(self, prompt, max_new_tokens: int, seed: int = 0, temperature: float = 0.8,
                         top_k: int = 40, top_p: float = 0.95, min_p: float = 0.0, repetition_penalty: float = 1.0,
                         presence_penalty: float = 0.0, frequency_penalty: float = 0.0, repetition_window: int = 0,
                         return_logits: bool = False):
        """Prefill + decode with the reference's sampling pipeline on the device (defaults of
        ProductionInferenceOptions.cs:19-87); draw i is uniform_draw(seed, i).  Returns
        (tokens, stats[, logits]); cropping and stops as in generate_greedy."""
        from ._lib import SamplingC
        p = np.ascontiguousarray(prompt, dtype=np.int32).reshape(-1)
        toks = np.empty(max_new_tokens, np.int32)
        logits = (np.empty((max_new_tokens, self.model.config.vocab_size), np.float32)
                  if return_logits else None)
        sp = SamplingC(temperature, top_k, top_p, min_p, repetition_penalty, presence_penalty, frequency_penalty,
                       repetition_window)
        st = GenStatsC()
        try:
            call("smx_session_generate_sampled", self._h, p.ctypes.data_as(ctypes.c_void_p), p.size, max_new_tokens,
                 ctypes.byref(sp), ctypes.c_uint64(seed), toks.ctypes.data_as(ctypes.c_void_p),
                 logits.ctypes.data_as(ctypes.c_void_p) if return_logits else None, ctypes.byref(st))
        except (GenerationCancelled, GenerationTimeout) as e:
            e.tokens = toks[:st.n_decode_steps].copy()
            raise
        stats = {"prefill_ms": st.prefill_ms, "decode_ms": st.decode_ms,
                 "prefill_steps": st.n_prefill_steps, "decode_steps": st.n_decode_steps}
        return (toks, stats, logits) if return_logits else (toks, stats)

    def cancel(self):
        """Asks the running (or next) generation on this session to stop; callable from any
        thread (smx_session_cancel)."""
        call("smx_session_cancel", self._h)

    def set_max_time_ms(self, max_time_ms: int):
        """MaxTimeMs of ProductionInferenceOptions (0 = no limit): later generations stop with
        GenerationTimeout once they have run this long."""
        call("smx_session_set_max_time", self._h, int(max_time_ms))

    def reset_kv_cache(self):
        call("smx_session_reset", self._h)

    @staticmethod
    def generate_greedy_batch(sessions, prompts, max_new_tokens: int):
        """Greedy generation for several sessions of one model in lockstep (smx_batch_generate):
        every decode step advances all sessions by one token with one pass over the weights.
        Returns (tokens [n_sessions][max_new_tokens], stats)."""
        n = len(sessions)
        ps = [np.ascontiguousarray(p, dtype=np.int32).reshape(-1) for p in prompts]
        if len(ps) != n:
            raise ValueError("one prompt per session")
        flat = np.concatenate(ps).astype(np.int32)
        lens = np.array([p.size for p in ps], np.int32)
        handles = (ctypes.c_void_p * n)(*[s._h.value for s in sessions])
        toks = np.empty((n, max_new_tokens), np.int32)
        st = GenStatsC()
        try:
            call("smx_batch_generate", ctypes.cast(handles, ctypes.c_void_p), n,
                 flat.ctypes.data_as(ctypes.c_void_p), lens.ctypes.data_as(ctypes.c_void_p),
                 max_new_tokens, toks.ctypes.data_as(ctypes.c_void_p), ctypes.byref(st))
        except (GenerationCancelled, GenerationTimeout) as e:
            e.tokens = toks[:, :st.n_decode_steps].copy()
            raise
        stats = {"prefill_ms": st.prefill_ms, "decode_ms": st.decode_ms,
                 "prefill_steps": st.n_prefill_steps, "decode_steps": st.n_decode_steps}
        return toks, stats

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            call("smx_session_destroy", self._h)
            self._h = ctypes.c_void_p()
        owned = getattr(self.model, "_sessions", None)
        if owned is not None and self in owned:
            owned.remove(self)


class ContinuousBatcher:
    """Continuous batching over sessions of one model (smx_batcher_*): members join after their
    own prefill and leave between steps; each step advances every member by one greedy token
    with one pass over the weights.  The reference's BatchedInferenceEngine groups requests
    (BatchedInferenceEngine.cs:186-200) but runs each one on its own (:241-259)."""

    def __init__(self, model: "GpuTransformerModel", max_members: int, max_ctx: int):
        self.model = model
        self.max_ctx = max_ctx
        self._h = ctypes.c_void_p()
        call("smx_batcher_create", model._h, max_members, max_ctx, ctypes.byref(self._h))
        self.members: list = []
        if not hasattr(model, "_batchers"):
            model._batchers = []
        model._batchers.append(self)

    def add(self, session: "GpuInferenceSession", prompt, sampling: dict | None = None, seed: int = 0):
        """Prefills the prompt and makes the session a member; with sampling (keyword options of
        generate_sampled) its tokens are drawn as generate_sampled draws them for this seed."""
        p = np.ascontiguousarray(prompt, dtype=np.int32).reshape(-1)
        if sampling is None:
            call("smx_batcher_add", self._h, session._h, p.ctypes.data_as(ctypes.c_void_p), p.size)
        else:
            from ._lib import SamplingC
            o = dict(temperature=0.8, top_k=40, top_p=0.95, min_p=0.0, repetition_penalty=1.0,
                     presence_penalty=0.0, frequency_penalty=0.0, repetition_window=0)
            o.update(sampling)
            sp = SamplingC(o["temperature"], o["top_k"], o["top_p"], o["min_p"], o["repetition_penalty"],
                           o["presence_penalty"], o["frequency_penalty"], o["repetition_window"])
            call("smx_batcher_add_sampled", self._h, session._h, p.ctypes.data_as(ctypes.c_void_p), p.size,
                 ctypes.byref(sp), ctypes.c_uint64(seed))
        self.members.append(session)

    def remove(self, session: "GpuInferenceSession"):
        call("smx_batcher_remove", self._h, session._h)
        self.members.remove(session)

    def __len__(self):
        n = load().smx_batcher_count(self._h)
        if n < 0:
            call("smx_batcher_count", self._h)   # raises with the library's message
        return n

    def step(self, n_steps: int = 1) -> np.ndarray:
        """Tokens [n_members][n_steps], members in the order they were added.  A member's cancel
        request or time limit stops the call between steps: GenerationCancelled /
        GenerationTimeout with `tokens` = the steps that ran."""
        out = np.empty((len(self.members), n_steps), np.int32)
        try:
            call("smx_batcher_step", self._h, n_steps, out.ctypes.data_as(ctypes.c_void_p))
        except (GenerationCancelled, GenerationTimeout) as e:
            done = int((out[0] >= 0).sum()) if out.size else 0
            e.tokens = out[:, :done].copy()
            raise
        return out

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            call("smx_batcher_destroy", self._h)
            self._h = ctypes.c_void_p()
            self.members = []
        owned = getattr(self.model, "_batchers", None)
        if owned is not None and self in owned:
            owned.remove(self)


def serve_continuous(model: "GpuTransformerModel", prompts, max_new_tokens, max_members: int, max_ctx: int,
                     eos_token: int | None = None):
    """Greedy generation for a queue of requests with continuous batching: at most max_members
    requests decode together; a request leaves as soon as it has its tokens (or emits
    eos_token) and the next queued request takes its place before the next step.  Returns one
    token array per request, in request order."""
    lim = [max_new_tokens] * len(prompts) if np.isscalar(max_new_tokens) else list(max_new_tokens)
    out = [[] for _ in prompts]
    b = ContinuousBatcher(model, max_members, max_ctx)
    free = []
    active = {}    # session -> request index
    queue = list(range(len(prompts)))
    try:
        free = [model.create_session(max_ctx) for _ in range(min(max_members, len(prompts)))]
        while queue or active:
            while queue and free:
                r = queue.pop(0)
                s = free.pop()
                b.add(s, prompts[r])
                active[s] = r
            toks = b.step(1)
            for s, t in zip(list(b.members), toks[:, 0]):
                r = active[s]
                out[r].append(int(t))
                if len(out[r]) >= lim[r] or (eos_token is not None and int(t) == eos_token):
                    b.remove(s)
                    del active[s]
                    free.append(s)
    finally:
        # the batcher releases its members first; then every session of this call is closed
        # (each holds a KV cache of max_ctx positions)
        b.close()
        for s in list(free) + list(active):
            s.close()
    return [np.array(o, np.int32) for o in out]
