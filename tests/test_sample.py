"""Sampling (S16): the library's ifr_sample / ifr_rng against the oracle's
restatement of the reference's sample() (main.cpp:8674-8764), and the
oracle against what fixes it independently (CPU only; no device needed).

Pins of the oracle's sampler:
  * the generator is the C++ standard's mt19937: its 10000th output from the
    default seed 5489 is 4123659995 (the value the standard itself states);
  * the draw is std::uniform_real_distribution<float>(0, 1), here equal to
    float(x) * 2^-32 of the raw outputs (numpy float32 rounding);
  * temperature -> 0, top_k = 1 and a tiny top_p all reduce to the argmax;
  * frequencies over many draws match the float64 softmax of logits / T, and
    the top-k / top-p supports are the sets a float64 sort gives.
The library's sampler must then equal the oracle's draw for draw.
"""
import numpy as np
import pytest

import intfer_amd as ia
from oracle import pyoracle as po
from oracle.pyoracle import ptr


@pytest.fixture(scope="module")
def O():
    return po.oracle()


def _or_draws(O, logits, n, seed, T=1.0, k=0, p=0.0):
    g = O.or_rng_create(seed)
    try:
        lg = np.ascontiguousarray(logits, np.float32)
        return np.array([O.or_sample(ptr(lg), lg.size, k, p, T, g) for _ in range(n)])
    finally:
        O.or_rng_free(g)


def test_mt19937_matches_the_standard(O):
    g = O.or_rng_create(5489)
    try:
        for _ in range(9999):
            O.or_rng_next(g)
        assert O.or_rng_next(g) == 4123659995
    finally:
        O.or_rng_free(g)


def test_uniform_draw_is_float_of_the_raw_output(O):
    g1, g2 = O.or_rng_create(123), O.or_rng_create(123)
    try:
        raw = np.array([O.or_rng_next(g1) for _ in range(100000)], np.uint64)
        u = np.array([O.or_rng_uniform(g2) for _ in range(100000)], np.float32)
    finally:
        O.or_rng_free(g1)
        O.or_rng_free(g2)
    want = raw.astype(np.float32) * np.float32(2.0 ** -32)
    want = np.where(want >= 1, np.nextafter(np.float32(1), np.float32(0)), want).astype(np.float32)
    assert np.array_equal(u.view(np.uint32), want.view(np.uint32))


def test_library_generator_equals_oracle(O):
    for seed in (0, 1, 7, 2**32 - 1):
        r = ia.Rng(seed)
        g = O.or_rng_create(seed)
        try:
            a = np.array([r.uniform() for _ in range(20000)], np.float32)
            b = np.array([O.or_rng_uniform(g) for _ in range(20000)], np.float32)
        finally:
            O.or_rng_free(g)
            r.close()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), seed


def test_greedy_limits_are_the_argmax(O):
    rng = np.random.default_rng(3)
    for _ in range(20):
        lg = rng.standard_normal(5000).astype(np.float32)
        am = int(np.argmax(lg))
        assert set(_or_draws(O, lg, 20, 5, T=0.0).tolist()) == {am}
        assert set(_or_draws(O, lg, 20, 6, T=1.5, k=1).tolist()) == {am}
        assert set(_or_draws(O, lg, 20, 7, T=1.0, p=1e-7).tolist()) == {am}


def test_frequencies_follow_the_softmax(O):
    lg = np.array([1.0, 0.2, -0.5, 2.0, 0.9, -1.5], np.float32)
    n = 60000
    for T, k, p in ((0.7, 0, 0.0), (1.3, 3, 0.0), (1.0, 0, 0.6)):
        d = _or_draws(O, lg, n, 11, T=T, k=k, p=p)
        pr = np.exp((lg.astype(np.float64) - lg.max()) / T)
        pr /= pr.sum()
        order = np.argsort(-pr, kind="stable")
        keep = np.ones(lg.size, bool)
        if k:
            keep[order[k:]] = False
        if p:
            cut = int(np.searchsorted(np.cumsum(pr[order]), p)) + 1
            keep[order[cut:]] = False
        pr = np.where(keep, pr, 0.0)
        pr /= pr.sum()
        f = np.bincount(d, minlength=lg.size) / n
        assert set(np.nonzero(f)[0].tolist()) <= set(np.nonzero(keep)[0].tolist()), (T, k, p)
        sd = np.sqrt(pr * (1 - pr) / n)
        assert np.all(np.abs(f - pr) <= 5 * sd + 1e-9), (T, k, p, f, pr)


@pytest.mark.parametrize("V,T,k,p", [(8, 1.0, 0, 0.0), (1000, 0.8, 40, 0.0), (1000, 0.6, 0, 0.9),
                                     (4096, 1.2, 50, 0.95), (151936, 0.7, 0, 0.0), (151936, 0.9, 40, 0.9),
                                     (300, 0.0, 0, 0.0), (300, -1.0, 5, 0.5)])
def test_library_sampler_equals_oracle(O, V, T, k, p):
    rng = np.random.default_rng(V + k)
    lg = (rng.standard_normal((6, V)) * 2).astype(np.float32)
    lg[1, :5] = lg[1].max()  # tied maxima
    seed = 1234 + V
    r = ia.Rng(seed)
    g = O.or_rng_create(seed)
    try:
        for row in lg:
            for _ in range(3 if V > 10000 else 12):
                a = ia.sample(row, r, temperature=T, top_k=k, top_p=p)
                b = O.or_sample(ptr(np.ascontiguousarray(row)), V, k, p, T, g)
                assert a == b
    finally:
        O.or_rng_free(g)
        r.close()
