"""CPU: the host nucleus sampler (opworks_amd.llama.sample_top_p) against
known answers of the reference's semantics (examples/llama/generate.py:83-109)
and the textbook softmax, by exact frequency counts on a seeded generator."""
import numpy as np
import pytest

from opworks_amd.llama import sample_top_p


def empirical(logits, temperature, top_p, n=40000, seed=5):
    rng = np.random.default_rng(seed)
    counts = np.bincount([sample_top_p(logits, rng, temperature, top_p) for _ in range(n)], minlength=len(logits))
    return counts / n


def test_full_distribution_is_temperature_softmax():
    logits = np.array([2.0, 1.0, 0.5, -1.0], np.float32)
    for t in (1.0, 0.5):
        p = np.exp(logits / t - (logits / t).max())
        p /= p.sum()
        assert np.allclose(empirical(logits, t, 1.0), p, atol=0.01)


def test_nucleus_keeps_the_crossing_token():
    # probabilities 0.5, 0.3, 0.15, 0.05 (logits = log p)
    p = np.array([0.5, 0.3, 0.15, 0.05])
    logits = np.log(p).astype(np.float32)
    # top_p 0.7: 0.5 <= 0.7 kept, 0.8 crosses -> kept too; renormalised over {0.5, 0.3}
    assert np.allclose(empirical(logits, 1.0, 0.7), [0.625, 0.375, 0, 0], atol=0.01)
    # top_p 0.9: 0.5, 0.8 kept, 0.95 crosses -> three tokens
    assert np.allclose(empirical(logits, 1.0, 0.9), np.array([0.5, 0.3, 0.15, 0]) / 0.95, atol=0.01)


def test_nucleus_exact_boundary_and_tiny_p():
    p = np.array([0.5, 0.3, 0.15, 0.05])
    logits = np.log(p).astype(np.float32)
    # cumulative 0.5 == top_p: searchsorted lands on it, so only the top token survives
    assert np.array_equal(empirical(logits, 1.0, 0.5, n=2000), [1, 0, 0, 0])
    # a top_p below the top probability still keeps the top token
    assert np.array_equal(empirical(logits, 1.0, 0.01, n=2000), [1, 0, 0, 0])


def test_seeded_sampling_is_reproducible():
    logits = np.random.default_rng(1).normal(size=1000).astype(np.float32)
    a = [sample_top_p(logits, np.random.default_rng(7), 0.8, 0.9) for _ in range(3)]
    b = [sample_top_p(logits, np.random.default_rng(7), 0.8, 0.9) for _ in range(3)]
    assert a == b
