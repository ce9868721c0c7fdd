"""The oracle's sampling pipeline (InferenceSession.cs:565-606) pinned against closed forms and
numpy restatements of each stage, on the CPU.  The GPU kernel is checked against it in
test_gpu_ops.py."""
import numpy as np
import pytest

import oracle as O


def _softmax64(l):
    l = np.asarray(l, np.float64)
    m = l[np.isfinite(l)].max()
    e = np.where(np.isfinite(l), np.exp(l - m), 0.0)
    return e / e.sum()


def _draw(p, u):
    c = np.cumsum(np.asarray(p, np.float64))
    i = int(np.searchsorted(c, u, side="left"))
    return min(i, len(p) - 1)


@pytest.fixture(scope="module")
def logits():
    return np.random.default_rng(11).normal(0, 2, 500).astype(np.float32)


def test_neutral_options_are_a_softmax_draw(oracle_mod, logits):
    ref = _softmax64(logits)
    for u in (0.0, 0.1, 0.5, 0.93, 0.999999):
        tok, p = O.sample(logits, u)
        assert np.abs(p - ref).max() < 1e-6
        assert tok == _draw(ref, u)


def test_top_k_one_and_tiny_top_p_give_the_argmax(oracle_mod, logits):
    am = int(np.argmax(logits))
    for kw in ({"top_k": 1}, {"top_p": 1e-9}, {"min_p": 0.999999}):
        tok, p = O.sample(logits, 0.73, **kw)
        assert tok == am and p[am] == 1.0 and p.sum() == 1.0, kw


def test_temperature_scales_logits(oracle_mod, logits):
    for t in (0.25, 0.8, 1.7):
        _, p = O.sample(logits, 0.5, temperature=t)
        inv = np.float32(1.0) / np.float32(t)
        assert np.abs(p - _softmax64(logits * inv)).max() < 1e-6


def test_top_k_keeps_the_k_largest(oracle_mod, logits):
    for k in (2, 40, 499):
        _, p = O.sample(logits, 0.5, top_k=k)
        keep = np.zeros(logits.size, bool)
        keep[np.argsort(-logits, kind="stable")[:k]] = True
        assert np.array_equal(p > 0, keep)
        assert np.abs(p - _softmax64(np.where(keep, logits, -np.inf))).max() < 1e-6


def test_top_p_keeps_the_smallest_prefix_reaching_p(oracle_mod, logits):
    base = _softmax64(logits)
    for tp in (0.3, 0.9, 0.95):
        _, p = O.sample(logits, 0.5, top_p=tp)
        order = np.argsort(-base, kind="stable")
        c = np.cumsum(base[order])
        cut = int(np.searchsorted(c, tp, side="left")) + 1
        keep = np.zeros(logits.size, bool)
        keep[order[:cut]] = True
        assert np.array_equal(p > 0, keep), tp
        assert np.abs(p - np.where(keep, base, 0) / base[keep].sum()).max() < 1e-6


def test_min_p_drops_below_a_fraction_of_the_max(oracle_mod, logits):
    base = _softmax64(logits)
    _, p = O.sample(logits, 0.5, min_p=0.1)
    keep = base >= base.max() * 0.1
    assert np.array_equal(p > 0, keep)
    assert np.abs(p - np.where(keep, base, 0) / base[keep].sum()).max() < 1e-6


def test_penalties_hand_computed(oracle_mod):
    """InferenceSession.ApplyRepetitionPenalties (:765-843): per distinct token of the window,
    l / r for l > 0 else l * r, minus presence, minus count * frequency."""
    l = np.array([1.0, 3.0, 2.0, -0.5, 0.25], np.float32)
    ctx = [4, 1, 1, 2, 3]
    _, p = O.sample(l, 0.5, context=ctx, repetition_penalty=1.5, presence_penalty=0.2, frequency_penalty=0.1)
    f = np.float32
    exp = np.array([1.0, f(3.0) / f(1.5) - f(0.2) - f(2) * f(0.1), f(2.0) / f(1.5) - f(0.2) - f(0.1),
                    f(-0.5) * f(1.5) - f(0.2) - f(0.1), f(0.25) / f(1.5) - f(0.2) - f(0.1)], np.float32)
    assert np.abs(p - _softmax64(exp)).max() < 1e-6
    # a window of 2 sees only tokens 2 and 3
    _, p2 = O.sample(l, 0.5, context=ctx, repetition_penalty=1.5, window=2)
    exp2 = l.copy()
    exp2[2] = f(2.0) / f(1.5)
    exp2[3] = f(-0.5) * f(1.5)
    assert np.abs(p2 - _softmax64(exp2)).max() < 1e-6


def test_draw_past_the_total_falls_back_to_the_last_id(oracle_mod):
    l = np.array([0.0, -np.inf, -np.inf], np.float32)
    tok, p = O.sample(l, 0.999999)
    assert tok == 0 and p[0] == 1.0
