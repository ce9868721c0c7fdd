"""GPU parity of the .smq model path (smx_model_load_smq): models loaded from SmallMind's own
files generate the checker's greedy tokens with logits within 1e-3 (max|dl| / max|l_ref|), the
checker building its model from the same file with its own reader (oracle.smq).  Covers the
reference's benchmark model (Q8_0 at block 32, positional tensor names, d = 64), and written
GPT-2 models with named tensors, Q4_0 at block 32 and Q8_0 at block 64, on both the per-token
decode path and the chunked matrix-core prefill."""
import os

import numpy as np
import pytest

import oracle as O
from oracle import smq as OS
from smallmind_amd import smq as S
from smallmind_amd.model import ModelConfig
from tests.helpers import check_greedy_against_oracle, gpt2_smq_tensors, rel_err

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "benchmark_model.smq")


def _check(gm, om, prompt, n_new, ctx):
    s = gm.create_session(ctx)
    toks, stats, logits = s.generate_greedy(np.asarray(prompt, np.int32), n_new, return_logits=True)
    worst = check_greedy_against_oracle(om.session(ctx), np.asarray(prompt, np.int32), toks, logits, LOGIT_TOL)
    s.close()
    return worst


def test_reference_benchmark_model(gpu):
    """tools/CreateBenchmarkModel/benchmark-model.smq as the reference ships it: the
    configuration from its metadata, tensors tensor_000..028 matched by parameter order, Q8_0
    embeddings, position table and head kept quantized on the device."""
    from smallmind_amd.model import GpuTransformerModel
    with open(GOLDEN, "rb") as f:
        om, cfg = OS.oracle_from_smq(f.read())
    gm = GpuTransformerModel.from_smq(GOLDEN)
    c = gm.config
    assert (c.architecture, c.vocab_size, c.context_length, c.embedding_length, c.block_count,
            c.head_count) == ("gpt2", 50, 32, 64, 2, 4)
    # a short prompt (per-token prefill) and one long enough for the chunked GEMM prefill
    _check(gm, om, [1, 2, 3, 4, 5], 27, 32)
    _check(gm, om, [7, 3, 9, 11, 20, 33, 2, 5, 8, 13, 21, 34], 20, 32)
    gm.close()


@pytest.mark.parametrize("scheme,block,named", [(S.Q4_0, 32, True), (S.Q8_0, 64, False)])
def test_written_gpt2_models(gpu, tmp_path, scheme, block, named):
    from smallmind_amd.model import GpuTransformerModel
    cfg = ModelConfig("gpt2", 1000, 128, 256, 2, 4, 4, 1024)
    p = tmp_path / "m.smq"
    S.write_smq(str(p), gpt2_smq_tensors(cfg, scheme, block, 11 + block, named), S.gpt2_metadata(cfg))
    om, _ = OS.oracle_from_smq(p.read_bytes())
    gm = GpuTransformerModel.from_smq(str(p))
    rng = np.random.default_rng(block)
    _check(gm, om, rng.integers(0, 1000, 5), 64, 128)      # per-token prefill, 64 greedy steps
    _check(gm, om, rng.integers(0, 1000, 40), 48, 128)     # chunked GEMM prefill
    gm.close()


def test_explicit_config_and_missing_tensor_are_reported(gpu, tmp_path):
    """The caller's ModelConfig replaces the metadata (LoadFromSmq's config argument); a file
    lacking a parameter the model needs fails at finalize with the parameter named."""
    from smallmind_amd._lib import SmxError
    from smallmind_amd.model import GpuTransformerModel
    cfg = ModelConfig("gpt2", 1000, 128, 256, 2, 4, 4, 1024)
    tens = gpt2_smq_tensors(cfg, S.Q8_0, 32, 3, True)
    p = tmp_path / "nometa.smq"
    S.write_smq(str(p), tens, {"model_name": "no-config"})
    gm = GpuTransformerModel.from_smq(str(p), config=cfg)
    om, _ = OS.oracle_from_smq(p.read_bytes(), dict(vocab=1000, ctx=128, d=256, n_layer=2, n_head=4, ff=1024))
    _check(gm, om, [5, 6, 7], 8, 64)
    gm.close()
    q = tmp_path / "partial.smq"
    S.write_smq(str(q), [t for t in tens if t.name != "blk.1.ffn_down.weight"], S.gpt2_metadata(cfg))
    with pytest.raises(SmxError) as e:
        GpuTransformerModel.from_smq(str(q))
    assert "layer 1" in str(e.value)


def test_matrix_of_wrong_rank_is_refused_and_released(gpu, tmp_path):
    """An F32 weight matrix stored with rank 3 passes the directory checks (SmqReader takes any
    rank for F32) but is no matrix: the load fails with SMX_EUNSUPPORTED after earlier tensors were
    uploaded, and releases the partly built model (device memory back to where it was)."""
    import torch

    from smallmind_amd._lib import SmxError
    from smallmind_amd.model import GpuTransformerModel
    cfg = ModelConfig("gpt2", 1000, 128, 256, 2, 4, 4, 1024)
    tens = gpt2_smq_tensors(cfg, S.Q8_0, 32, 5, True)
    last = [t.name for t in tens if len(t.dims) == 2 and t.dims[0] > 1][-1]
    bad = [S.SmqTensor(t.name, S.F32, (t.dims[0], t.dims[1], 1),
                       np.random.default_rng(1).normal(0, 0.02, t.dims[0] * t.dims[1]).astype(np.float32))
           if t.name == last else t for t in tens]
    p = tmp_path / "rank3.smq"
    S.write_smq(str(p), bad, S.gpt2_metadata(cfg))
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(4):
        with pytest.raises(SmxError) as e:
            GpuTransformerModel.from_smq(str(p))
        assert e.value.code == -5 and "rank 3" in str(e.value)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] >= free0 - (1 << 20)
