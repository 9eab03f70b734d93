"""The benchmark's data generator (tokenvector.inference_amd.synthetic)
against the oracle's scalar restatement of the reference's `_gi_noise`
(tv/training/gpt2_ref.tkv:1977-1991) and outlier placement: bit for bit."""
import numpy as np
import pytest

import oracle as O
from tokenvector.inference_amd import synthetic as S


@pytest.mark.parametrize("n,seed,sigma", [(0, 1, 1.0), (1, 0, 1.0), (2, 2**31 + 5, 0.02),
                                          (7, 5, 0.02), (4097, 12345, 0.01), (1_000_003, 7, 1.0)])
def test_gi_noise_matches_oracle(n, seed, sigma):
    a = O.gi_noise(n, seed, sigma)
    b = S.gi_noise(n, seed, sigma)
    assert b.dtype == np.float32 and b.shape == (n,)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_lcg31_states_are_the_recurrence():
    s, want = 123456789, []
    for _ in range(1000):
        s = (1103515245 * s + 12345) % 2**31
        want.append(s)
    assert S.lcg31_states(123456789, 1000).tolist() == want


@pytest.mark.parametrize("n,frac,seed", [(200_000, 0.001, 3), (50, 0.9, 9), (10, 1.0, 1), (10, 0.0, 1)])
def test_add_outliers_matches_oracle(n, frac, seed):
    x = O.gi_noise(n, 3, 1.0)
    a = O.add_outliers(x, frac, seed, 4, 20.0)
    b = S.add_outliers(x, frac, seed, 4, 20.0)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
