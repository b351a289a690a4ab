"""The harness's host greedy sampling (cheetah_amd/workloads.greedy_token)
against the definition it implements: the last index of the maximum
(engine.rs:2247-2253), on random logits with planted ties and NaN."""
import numpy as np

from cheetah_amd import workloads


def last_max(a):
    return int(len(a) - 1 - np.argmax(a[::-1]))


def test_greedy_token_is_the_last_maximum():
    rng = np.random.default_rng(3)
    for trial in range(200):
        a = rng.standard_normal(int(rng.integers(1, 3000))).astype(np.float32)
        if trial % 3 == 0 and a.size > 1:
            # Plant the maximum at several indices.
            idx = rng.choice(a.size, size=min(a.size, int(rng.integers(2, 5))), replace=False)
            a[idx] = a.max() + 1.0
        if trial % 7 == 0:
            a[int(rng.integers(0, a.size))] = np.nan
        assert workloads.greedy_token(a) == last_max(a), trial
    assert workloads.greedy_token(np.array([5.0], np.float32)) == 0
    assert workloads.greedy_token(np.array([1.0, 2.0, 2.0, 0.5], np.float32)) == 2
