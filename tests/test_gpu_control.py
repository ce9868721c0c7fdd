"""Generation control on the device path: cancellation from another thread, the time limit and
prompt cropping, against the reference's InferenceSession semantics.

- The reference checks its CancellationToken before every token (InferenceSession.cs:211, :481)
  and turns MaxTimeMs into InferenceTimeoutException (InferenceSession.cs:164-172, :287-291).
  Here the host checks between graph launches; a stopped call returns the tokens produced so far,
  which must be the first tokens of the uninterrupted run.
- The reference crops the context to its last blockSize tokens before the prefill
  (InferenceSession.cs:494-508); here the session's max_ctx is the block size, and the cropped run
  must equal the oracle on the explicitly cropped prompt."""
import threading
import time

import numpy as np
import pytest

import oracle as O
from smallmind_amd._lib import GenerationCancelled, GenerationTimeout, SmxError
from smallmind_amd.model import ContinuousBatcher, GpuInferenceSession, ModelConfig
from tests.helpers import build_pair

pytestmark = pytest.mark.gpu

# a small llama (configs[2] formats) with a context long enough for a generation of ~100 ms
CFG = ModelConfig("llama", 1000, 2048, 256, 3, 8, 2, 768)
N_LONG = 1900


@pytest.fixture(scope="module")
def pair(gpu):
    om, gm, _ = build_pair(CFG, O.Q4_K, O.Q6_K, O.Q6_K, seed=77)
    yield om, gm
    gm.close()


@pytest.fixture(scope="module")
def reference_run(pair):
    """The uninterrupted greedy run every stopped run must be a prefix of."""
    _, gm = pair
    prompt = np.random.default_rng(3).integers(0, CFG.vocab_size, 16).astype(np.int32)
    s = gm.create_session(2048)
    toks, _ = s.generate_greedy(prompt, N_LONG)
    s.close()
    return prompt, toks


def test_cancel_from_a_second_thread_returns_a_prefix(pair, reference_run):
    _, gm = pair
    prompt, full = reference_run
    s = gm.create_session(2048)
    started = threading.Event()
    result = {}

    def run():
        started.set()
        try:
            result["tokens"] = s.generate_greedy(prompt, N_LONG)[0]
        except GenerationCancelled as e:
            result["cancelled"] = e

    t = threading.Thread(target=run)
    t.start()
    assert started.wait(30)
    time.sleep(0.02)
    while t.is_alive():      # ctypes releases the GIL inside the generate call
        s.cancel()
        time.sleep(0.002)
    t.join()
    assert "cancelled" in result, "the generation finished before any cancel request arrived"
    e = result["cancelled"]
    assert e.code == -8
    k = len(e.tokens)
    print(f"cancelled after {k} of {N_LONG} tokens", flush=True)
    assert 0 < k < N_LONG
    assert np.array_equal(e.tokens, full[:k])
    # the request was consumed: the next generation on the session runs to the end
    toks, _ = s.generate_greedy(prompt, N_LONG)
    assert np.array_equal(toks, full)
    s.close()


def test_cancel_before_the_call_stops_it_at_its_first_check(pair, reference_run):
    _, gm = pair
    prompt, full = reference_run
    s = gm.create_session(2048)
    s.cancel()
    with pytest.raises(GenerationCancelled) as ei:
        s.generate_greedy(prompt, 64)
    assert len(ei.value.tokens) == 0
    toks, _ = s.generate_greedy(prompt, 64)
    assert np.array_equal(toks, full[:64])
    # smx_session_reset clears a pending request
    s.cancel()
    s.reset_kv_cache()
    toks, _ = s.generate_greedy(prompt, 64)
    assert np.array_equal(toks, full[:64])
    s.close()


def test_time_limit_stops_the_generation(pair, reference_run):
    _, gm = pair
    prompt, full = reference_run
    s = gm.create_session(2048)
    s.set_max_time_ms(5)
    with pytest.raises(GenerationTimeout) as ei:
        s.generate_greedy(prompt, N_LONG)
    k = len(ei.value.tokens)
    print(f"time limit: {k} of {N_LONG} tokens", flush=True)
    assert ei.value.code == -9 and k < N_LONG
    assert np.array_equal(ei.value.tokens, full[:k])
    s.set_max_time_ms(0)
    toks, _ = s.generate_greedy(prompt, N_LONG)
    assert np.array_equal(toks, full)
    with pytest.raises(SmxError) as ei:
        s.set_max_time_ms(-1)
    assert ei.value.code == -1
    s.close()


def test_sampled_generation_stops_with_a_prefix(pair, reference_run):
    _, gm = pair
    prompt, _ = reference_run
    s = gm.create_session(2048)
    ref, _ = s.generate_sampled(prompt, 600, seed=11)
    s.set_max_time_ms(3)
    with pytest.raises(GenerationTimeout) as ei:
        s.generate_sampled(prompt, 600, seed=11)
    k = len(ei.value.tokens)
    assert k < 600 and np.array_equal(ei.value.tokens, ref[:k])
    s.set_max_time_ms(0)
    s.cancel()
    with pytest.raises(GenerationCancelled) as ei:
        s.generate_sampled(prompt, 600, seed=11)
    assert len(ei.value.tokens) == 0
    s.close()


def test_over_long_prompt_is_cropped_to_the_session_context(pair):
    om, gm = pair
    rng = np.random.default_rng(9)
    prompt = rng.integers(0, CFG.vocab_size, 100).astype(np.int32)
    s = gm.create_session(64)
    toks, stats, logits = s.generate_greedy(prompt, 1, return_logits=True)
    assert stats["prefill_steps"] == 63
    # the oracle on the explicitly cropped prompt
    osess = om.session(64)
    osess.prefill(prompt[-64:-1], 0)
    ref = osess.step(int(prompt[-1]), 63)
    assert float(np.abs(logits[0] - ref).max() / np.abs(ref).max()) <= 1e-3
    assert int(toks[0]) == int(np.argmax(ref))
    # a second token would need position 64: the block-size check (TransformerModel.cs:280-283)
    with pytest.raises(SmxError) as ei:
        s.generate_greedy(prompt, 2)
    assert ei.value.code == -7
    # the same token as a generation on the cropped prompt itself
    c, _ = s.generate_greedy(prompt[-64:], 1)
    assert int(c[0]) == int(toks[0])
    s.close()


def test_batcher_step_stops_on_a_member_request(pair):
    _, gm = pair
    rng = np.random.default_rng(21)
    prompts = [rng.integers(0, CFG.vocab_size, n).astype(np.int32) for n in (9, 14)]
    ref_sessions = [gm.create_session(256) for _ in prompts]
    ref, _ = GpuInferenceSession.generate_greedy_batch(ref_sessions, prompts, 24)
    for x in ref_sessions:
        x.close()
    b = ContinuousBatcher(gm, 2, 256)
    ss = [gm.create_session(256) for _ in prompts]
    for x, p in zip(ss, prompts):
        b.add(x, p)
    got = [b.step(8)]
    ss[1].cancel()
    with pytest.raises(GenerationCancelled) as ei:
        b.step(8)
    assert ei.value.tokens.shape == (2, 0)
    got.append(b.step(8))           # both members continue where they were
    got.append(b.step(8))
    assert np.array_equal(np.concatenate(got, axis=1), ref)
    # a member's time limit counts from its join
    ss[0].set_max_time_ms(1)
    b.remove(ss[0])
    b.add(ss[0], prompts[0])
    time.sleep(0.01)
    with pytest.raises(GenerationTimeout):
        b.step(1)
    b.remove(ss[0])
    ss[0].set_max_time_ms(0)
    assert b.step(2).shape == (1, 2)
    b.close()
    for x in ss:
        x.close()


def test_batch_generate_stops_every_session(pair):
    _, gm = pair
    rng = np.random.default_rng(22)
    prompts = [rng.integers(0, CFG.vocab_size, n).astype(np.int32) for n in (5, 11, 8)]
    ss = [gm.create_session(2048) for _ in prompts]
    ref, _ = GpuInferenceSession.generate_greedy_batch(ss, prompts, 600)
    ss[2].set_max_time_ms(3)
    with pytest.raises(GenerationTimeout) as ei:
        GpuInferenceSession.generate_greedy_batch(ss, prompts, 600)
    k = ei.value.tokens.shape[1]
    assert k < 600 and np.array_equal(ei.value.tokens, ref[:, :k])
    ss[2].set_max_time_ms(0)
    ss[0].cancel()
    with pytest.raises(GenerationCancelled) as ei:
        GpuInferenceSession.generate_greedy_batch(ss, prompts, 600)
    assert ei.value.tokens.shape == (3, 0)
    got, _ = GpuInferenceSession.generate_greedy_batch(ss, prompts, 600)
    assert np.array_equal(got, ref)
    for x in ss:
        x.close()
