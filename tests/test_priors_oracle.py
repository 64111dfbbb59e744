"""Pins the oracle's restatement of the reference MCTS prior computation
(oracle.fast_exp / oracle.mcts_priors; reference src/mcts/core.h:38-44,
src/mcts/search.cpp:127-199, src/mcts/evaluator.cpp:181-224) against closed
forms, Schraudolph's published error bound and a float64 softmax."""

import numpy as np

import oracle


def test_fast_exp_exact_points():
    # x = 0 gives the pattern 127 << 23 = 1.0; x = k ln 2 gives 2^k (the
    # product lands on an integer multiple of 2^23 after float32 rounding).
    assert oracle.fast_exp(0.0) == np.float32(1.0)
    for k in (1, 2, 3, -1, -2):
        x = np.float32(k) * np.float32(np.log(2.0))
        assert oracle.fast_exp(x) == np.float32(2.0 ** k), k


def test_fast_exp_error_bound_and_clamp():
    # Schraudolph's construction is exact at x = k ln 2 and overestimates in
    # between by at most max_f (1 + f) / 2^f = 1.0861 (f = 1/ln 2 - 1).
    x = np.linspace(-80, 80, 200001, dtype=np.float32)
    ratio = oracle.fast_exp(x).astype(np.float64) / np.exp(x.astype(np.float64))
    assert ratio.min() > 0.9999 and ratio.max() < 1.0862
    # Clamp to [-88, 88] with std::min/std::max semantics: NaN -> 88.
    big, small = oracle.fast_exp(88.0), oracle.fast_exp(-88.0)
    assert oracle.fast_exp(1000.0) == big and oracle.fast_exp(np.inf) == big
    assert oracle.fast_exp(-1000.0) == small and oracle.fast_exp(np.nan) == big
    assert 0 < small < np.float32(1e-38)  # a binary32 subnormal, still positive


def test_priors_against_float64_softmax():
    rng = np.random.default_rng(3)
    logits = rng.standard_normal(1858).astype(np.float32) * 3
    for n in (1, 2, 20, 218, 256):
        idx = rng.choice(1858, size=n, replace=False)
        for temp in (1.0, 0.5, 2.2):
            p = oracle.mcts_priors(logits, idx, temp)
            l = logits[idx].astype(np.float64)
            e = oracle.fast_exp(((logits[idx] - logits[idx].max()) *
                                 (np.float32(1) / np.float32(temp))).astype(np.float32))
            want = e.astype(np.float64) / e.astype(np.float64).sum()
            assert abs(p.astype(np.float64).sum() - 1.0) < 1e-5
            np.testing.assert_allclose(p, want, rtol=2e-6, atol=1e-12)
            # FastExp tracks exp within its bound, so the priors follow the
            # temperature softmax of the logits within about 9 %.
            soft = np.exp((l - l.max()) / temp)
            soft /= soft.sum()
            assert np.all(np.abs(p - soft) <= 0.2 * soft + 1e-7)


def test_priors_out_of_range_indices_read_zero():
    logits = np.full(1858, -5.0, np.float32)
    logits[7] = 1.0
    p = oracle.mcts_priors(logits, [7, -1, 1858, 30000], 1.0)
    # Indices outside the policy read logit 0 (evaluator.cpp:198-202).
    assert p[1] == p[2] == p[3]
    assert p[0] > p[1]
    assert oracle.mcts_priors(logits, [], 1.0).size == 0
