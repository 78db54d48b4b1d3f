"""The exact top-k: the C radix select against the numpy sort and brute force."""

import numpy as np
import pytest

from oracle import topk as T


def _brute(s, k):
    keyed = sorted(range(len(s)), key=lambda i: (float(s[i]), not np.signbit(s[i]), -i),
                   reverse=True)
    return sorted(keyed[:k])


@pytest.mark.parametrize("n,k", [(1, 1), (5, 3), (37, 8), (64, 64), (65, 64), (300, 17)])
def test_topk_tiny_brute_force_with_ties(n, k):
    rng = np.random.default_rng(n * 131 + k)
    for _ in range(50):
        s = rng.choice(np.array([0.0, -0.0, 1.5, -2.0, 1.5, np.inf, -np.inf], np.float32), n)
        want = _brute(s, min(k, n))
        assert T.topk_sort(s, k).tolist() == want
        assert T.topk_c(s, k).tolist() == want


def test_topk_c_equals_sort_at_scale():
    rng = np.random.default_rng(7)
    for n, k in [(32768, 2048), (4097, 2048), (2048, 2048), (100, 2048)]:
        s = rng.normal(0, 1, n).astype(np.float32)
        s[rng.integers(0, n, n // 10)] = 0.5  # a block of exact ties
        assert np.array_equal(T.topk_c(s, k), T.topk_sort(s, k))


def test_topk_rows_pads_short_rows():
    rng = np.random.default_rng(3)
    s = rng.normal(0, 1, (3, 5000)).astype(np.float32)
    lens = np.array([5000, 10, 0], np.int32)
    out = T.topk_rows(s, lens, 2048)
    assert np.array_equal(out[0], T.topk_sort(s[0], 2048))
    assert out[1, :10].tolist() == list(range(10)) and np.all(out[1, 10:] == -1)
    assert np.all(out[2] == -1)
