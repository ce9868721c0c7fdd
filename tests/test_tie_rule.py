"""The cross-path greedy token rule of the full-size tests (CPU): identical sequences, or a first
difference only at a near-tie of the reference logits resolved to the runner-up."""
import numpy as np
import pytest

from tests.test_gpu_fullsize import TIE_TOL, _same_tokens_or_near_tie


def _logits(n_steps, vocab, tie_at=None, margin=0.0):
    rng = np.random.default_rng(0)
    lg = rng.normal(0, 1, (n_steps, vocab)).astype(np.float32)
    lg[:, 3] = 10.0        # reference token 3 at every step, clear winner
    lg[:, 7] = 9.0
    if tie_at is not None:
        lg[tie_at, 7] = 10.0 - margin * 10.0   # runner-up 7 within margin of max|logit| = 10
    return lg


def test_equal_sequences_pass():
    ref = np.full(8, 3)
    assert _same_tokens_or_near_tie(ref.copy(), ref, _logits(8, 20)) is None


def test_difference_at_a_near_tie_to_the_runner_up_is_accepted():
    ref = np.full(8, 3)
    other = ref.copy()
    other[5:] = 7
    assert _same_tokens_or_near_tie(other, ref, _logits(8, 20, tie_at=5, margin=TIE_TOL / 2)) == 5


def test_difference_without_a_near_tie_fails():
    ref = np.full(8, 3)
    other = ref.copy()
    other[5] = 7
    with pytest.raises(AssertionError):
        _same_tokens_or_near_tie(other, ref, _logits(8, 20, tie_at=5, margin=TIE_TOL * 2))


def test_difference_to_a_token_other_than_the_runner_up_fails():
    ref = np.full(8, 3)
    other = ref.copy()
    other[5] = 11
    with pytest.raises(AssertionError):
        _same_tokens_or_near_tie(other, ref, _logits(8, 20, tie_at=5, margin=TIE_TOL / 2))
