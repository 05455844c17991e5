"""The sampler (src/model.rs:300-366) in the library, on the CPU, against the oracle's restatement.

The oracle is pinned by the reference's own unit tests (greedy picks the first maximum, top-k never
leaves the top k, a seed repeats its draws and top_p = 0.5 keeps only the likeliest token, a high
temperature reaches every token) and by the draw frequencies: over many draws each token's share
must match the softmax at the temperature over the top k after the nucleus cut, computed here in
float64 (a wrong sign, a dropped temperature or a misplaced cut fails it). The library's sampler
must then draw the oracle's exact tokens for the same seeds, logits and settings."""
import os
import sys

import numpy as np
import pytest

import layerstream_amd as LS

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "oracle"))
import oracle_py as O  # noqa: E402

BOTH = [("library", LS.Sampler), ("oracle", O.Sampler)]


@pytest.mark.parametrize("name,S", BOTH)
def test_reference_unit_cases(name, S):
    # greedy_picks_the_first_maximum
    assert S(0.0, 1, 1.0, 0).sample([0.1, 3.0, 3.0, -1.0]) == 1
    # top_k_never_leaves_the_top_k
    logits = np.arange(100, dtype=np.float32)
    s = S(1.0, 5, 1.0, 42)
    assert all(s.sample(logits) >= 95 for _ in range(500))
    # sampling_is_deterministic_for_a_seed_and_respects_top_p
    lg = np.array([10.0, 9.0, 0.0, 0.0, 0.0], np.float32)

    def draw(seed):
        s = S(0.8, 5, 0.5, seed)
        return [s.sample(lg) for _ in range(50)]

    assert draw(7) == draw(7)
    assert all(t == 0 for t in draw(7))
    # higher_temperature_spreads_the_choices
    s = S(2.0, 4, 1.0, 1)
    seen = {s.sample(np.array([2.0, 1.5, 1.0, 0.5], np.float32)) for _ in range(2000)}
    assert seen == {0, 1, 2, 3}


def expected_shares(logits, temperature, top_k, top_p):
    order = np.argsort(-logits.astype(np.float64), kind="stable")[: max(1, min(top_k, len(logits)))]
    z = (logits[order].astype(np.float64) - logits[order[0]]) / temperature
    p = np.exp(z)
    p /= p.sum()
    keep = len(p)
    cum = np.cumsum(p)
    hit = np.nonzero(cum >= top_p)[0]
    if len(hit):
        keep = hit[0] + 1
    q = p[:keep] / p[:keep].sum()
    out = np.zeros(len(logits))
    out[order[:keep]] = q
    return out


@pytest.mark.parametrize("temperature,top_k,top_p", [(1.0, 50, 1.0), (0.7, 8, 0.9), (1.5, 1000, 0.6), (0.3, 3, 1.0)])
def test_oracle_draws_follow_the_softmax_after_top_k_and_top_p(temperature, top_k, top_p):
    rng = np.random.default_rng(5)
    logits = (rng.standard_normal(64) * 2).astype(np.float32)
    want = expected_shares(logits, temperature, top_k, top_p)
    s = O.Sampler(temperature, top_k, top_p, 123)
    n = 40000
    counts = np.bincount([s.sample(logits) for _ in range(n)], minlength=len(logits)) / n
    assert np.all(counts[want == 0] == 0)
    assert np.max(np.abs(counts - want)) < 0.012, np.max(np.abs(counts - want))


def test_the_uniform_stream_is_uniform_and_seeded():
    s = O.Sampler(1.0, 1, 1.0, 99)
    u = np.array([s.uniform() for _ in range(20000)])
    assert u.min() >= 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 0.01 and abs(u.var() - 1 / 12) < 0.005
    a = O.Sampler(1.0, 1, 1.0, 5)
    b = O.Sampler(1.0, 1, 1.0, 6)
    assert [a.uniform() for _ in range(8)] != [b.uniform() for _ in range(8)]


def test_the_library_draws_the_oracles_tokens():
    rng = np.random.default_rng(17)
    for case in range(40):
        n = int(rng.choice([5, 64, 1000, 151936]))
        logits = (rng.standard_normal(n) * rng.uniform(0.5, 4)).astype(np.float32)
        temperature = float(rng.choice([0.0, 0.2, 0.7, 1.0, 1.8]))
        top_k = int(rng.choice([1, 2, 8, 40, 100000]))
        top_p = float(rng.choice([0.1, 0.5, 0.9, 1.0]))
        seed = int(rng.integers(0, 2**63))
        a, b = LS.Sampler(temperature, top_k, top_p, seed), O.Sampler(temperature, top_k, top_p, seed)
        got = [a.sample(logits) for _ in range(30)]
        want = [b.sample(logits) for _ in range(30)]
        assert got == want, (case, n, temperature, top_k, top_p)


def test_greedy_follows_the_argmax_rule_with_nans():
    s = LS.Sampler.greedy()
    assert s.sample([np.nan, 1.0, 2.0]) == 0  # nothing beats a NaN in front
    assert s.sample([1.0, np.nan, 2.0]) == 2
    assert s.sample([-np.inf, -np.inf]) == 0
    with pytest.raises(LS.LayerstreamError):
        s.sample([])
