"""CPU checks of the C-ABI library: it loads, exports every function include/smx.h declares,
and its host-only entry points behave (no device calls here)."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "smx.h")).read()
    return sorted(set(re.findall(r"SMX_API[^;(]*?\b(smx_\w+)\s*\(", text, re.S)))


def test_library_exports_every_declared_symbol():
    from smallmind_amd import _lib
    L = _lib.load()
    declared = _declared()
    assert len(declared) >= 30
    for name in declared:
        assert hasattr(L, name), name
    assert sorted(_lib.EXPORTS) == declared


def test_type_geometry():
    from smallmind_amd import _lib
    L = _lib.load()
    for t in (O.F32, O.F16, O.Q4_0, O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K):
        assert L.smx_type_block_elems(t) == O.BLOCK_ELEMS[t]
        assert L.smx_type_block_bytes(t) == O.BLOCK_BYTES[t]
    assert L.smx_type_row_bytes(O.Q4_K, 2048) == 8 * 144
    assert L.smx_type_row_bytes(O.Q4_0, 4096) == 128 * 18
    assert L.smx_type_row_bytes(O.Q4_K, 100) == -1
    assert L.smx_type_block_elems(3) == 0    # Q4_1: not implemented by the backend


def test_rope_tables_host_entry_matches_oracle():
    from smallmind_amd.quantization import rope_tables
    c, s = rope_tables(128, 64, 10000.0)
    oc, os_ = O.rope_tables(128, 64, 10000.0)
    assert np.array_equal(c, oc) and np.array_equal(s, os_)


def test_invalid_arguments_report_errors_without_a_device():
    from smallmind_amd import _lib
    L = _lib.load()
    assert L.smx_rope_tables(4, 3, 10000.0, None, None) == -1
    assert b"even" in L.smx_last_error()
    w = ctypes.c_void_p()
    assert L.smx_weight_create(3, 4, 32, ctypes.c_void_p(1), 0, ctypes.byref(w)) == -5
    assert L.smx_quantize(O.Q4_K, None, 100, None, None) == -1


def test_model_config_struct_layout():
    from smallmind_amd._lib import ModelConfigC
    assert ctypes.sizeof(ModelConfigC) == 4 * 16


def test_cancel_and_time_limit_entry_points_check_arguments_without_a_device():
    from smallmind_amd import _lib
    L = _lib.load()
    assert L.smx_session_cancel(None) == -1
    assert L.smx_session_set_max_time(None, 5) == -1


class _StoppingLib:
    """Stand-in for libsmx.so whose generate calls stop after two tokens with status `rc`,
    filling out_tokens and stats as the library does (tokens produced, then -1)."""

    def __init__(self, rc):
        self.rc = rc

    def smx_last_error(self):
        return b"stopped"

    def _fill(self, toks_ptr, n_total, stats_ptr, done=2):
        arr = (ctypes.c_int32 * n_total).from_address(toks_ptr.value)
        for i in range(n_total):
            arr[i] = 40 + i if i < done else -1
        ctypes.cast(stats_ptr, ctypes.POINTER(self.stats_type)).contents.n_decode_steps = done

    def smx_session_generate(self, h, p, n, n_new, toks, logits, stats):
        self._fill(toks, n_new, stats)
        return self.rc


@pytest.mark.parametrize("rc,cls,reference", [(-8, "GenerationCancelled", "OperationCanceledException"),
                                              (-9, "GenerationTimeout", "InferenceTimeoutException")])
def test_stopped_generation_maps_to_the_reference_exception(monkeypatch, rc, cls, reference):
    """Status mapping of a stopped generation on the host side: the Python mirror raises
    GenerationCancelled / GenerationTimeout carrying the tokens produced before the stop, and the
    C# binding throws the reference's exception for the same status."""
    from smallmind_amd import _lib, model
    fake = _StoppingLib(rc)
    fake.stats_type = _lib.GenStatsC
    monkeypatch.setattr(_lib, "_lib", fake)
    sess = model.GpuInferenceSession.__new__(model.GpuInferenceSession)
    sess._h = ctypes.c_void_p(1)
    sess.model = type("M", (), {"config": type("C", (), {"vocab_size": 8})()})()
    with pytest.raises(getattr(_lib, cls)) as ei:
        sess.generate_greedy(np.arange(3, dtype=np.int32), 5)
    assert ei.value.code == rc
    assert list(ei.value.tokens) == [40, 41]
    sess._h = ctypes.c_void_p()
    cs = open(os.path.join(ROOT, "smallmind_amd", "bindings", "csharp", "Smx.cs")).read()
    name = {-8: "ECANCELED", -9: "ETIMEDOUT"}[rc]
    assert re.search(rf"\b{name}\s*=>\s*new {reference}\(", cs), (name, reference)


def test_build_refuses_gemv_instances_with_scratch_memory():
    """The build reads the compiler's resource remarks for the GEMV source and fails on any
    instance with scratch memory (an instance that spilled its weight registers once returned
    wrong sums)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("smx_build", os.path.join(ROOT, "smallmind_amd", "build.py"))
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    remarks = "\n".join([
        "k_gemv.hip:206:1: remark: Function Name: _ZN3smx6k_gemvILi4E [-Rpass-analysis=kernel-resource-usage]",
        "k_gemv.hip:206:1: remark:     VGPRs: 254 [-Rpass-analysis=kernel-resource-usage]",
        "k_gemv.hip:206:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
        "k_gemv.hip:206:1: remark: Function Name: _ZN3smx6k_gemvILi2E [-Rpass-analysis=kernel-resource-usage]",
        "k_gemv.hip:206:1: remark:     ScratchSize [bytes/lane]: 436 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert b._spilling_kernels(remarks) == ["_ZN3smx6k_gemvILi2E"]
    # the GEMV and the matrix-core kernels (GEMM tiles, prefill attention) are all checked
    assert {"k_gemv.hip", "k_qgemm.hip", "k_attn_prefill.hip"} <= set(b.SPILL_CHECKED)


def test_c_consumer_reads_a_model_file_through_the_header(tmp_path):
    """include/smx.h compiles as C99 with -pedantic -Werror (the build fails otherwise), and a
    C program linked against libsmx.so reads the version, the block geometry and a GGUF file's
    configuration with no device work, as the Python binding does."""
    import subprocess

    from smallmind_amd import gguf as G
    from smallmind_amd.model import ModelConfig, read_gguf_config
    from tests.helpers import build_pair, c_consumer
    cfg = ModelConfig("llama", 300, 96, 256, 2, 8, 2, 512, 500000.0, 1e-6)
    _, _, t = build_pair(cfg, O.Q4_K, O.Q6_K, O.Q6_K, seed=3, with_gpu=False)
    p = tmp_path / "m.gguf"
    G.write_gguf(str(p), G.model_metadata(cfg), [(n, q, d, x) for n, (q, d, x) in t.items()])
    r = subprocess.run([c_consumer(), "info", str(p)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    lines = dict(line.split(" ", 1) for line in r.stdout.strip().splitlines())
    assert lines["version"].startswith("smx ")
    assert lines["q4_k"].split() == ["256", "144", str(4096 // 256 * 144)]
    f = lines["config"].split()
    got = read_gguf_config(str(p))
    assert [int(x) for x in f[:8]] == [0, got.vocab_size, got.context_length, got.embedding_length, got.block_count,
                                       got.head_count, got.head_count_kv, got.feed_forward_length]
    assert np.float32(float(f[8])) == np.float32(got.rope_freq_base)
    assert np.float32(float(f[9])) == np.float32(got.norm_eps) and int(f[10]) == len(t)
