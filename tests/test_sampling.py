"""generate's sampling step (TransformerLM::generate, src/models/transformer_lm.cpp:113-213) on the
CPU through aic_sample_tokens: over many draws from fixed logits, the token frequencies match
the distribution the reference's rules define -- softmax(logits / temperature), the top_k
largest kept and renormalised, then the smallest prefix of the descending order whose
cumulative sum reaches top_p kept and renormalised -- computed here independently in float64;
no token outside that support is ever drawn; greedy settings return the argmax; draws are a
function of the seed."""
import ctypes as C

import numpy as np
import pytest

from autonomousaicore_amd import _lib

N_DRAWS = 200_000


def draws(logits, temperature, top_k, top_p, seed, n=N_DRAWS):
    logits = np.ascontiguousarray(logits, np.float32)
    out = np.empty(n, np.int64)
    _lib.call("aic_sample_tokens", logits.ctypes.data, logits.size, C.c_float(temperature), top_k,
              C.c_float(top_p), C.c_uint64(seed), n, out.ctypes.data)
    return out


def expected(logits, temperature, top_k, top_p):
    z = logits.astype(np.float64) / temperature
    p = np.exp(z - z.max())
    p /= p.sum()
    V = p.size
    if 0 < top_k < V:
        keep = np.argsort(-p, kind="stable")[:top_k]
        q = np.zeros(V)
        q[keep] = p[keep]
        p = q / q.sum()
    if 0.0 < top_p < 1.0:
        order = np.argsort(-p, kind="stable")
        order = order[p[order] > 0]
        cut = int(np.searchsorted(np.cumsum(p[order]), top_p)) + 1  # first index reaching top_p
        q = np.zeros(V)
        q[order[:cut]] = p[order[:cut]]
        p = q / q.sum()
    return p


@pytest.mark.parametrize("temperature,top_k,top_p", [(1.0, 0, 1.0), (0.7, 10, 1.0), (1.3, 0, 0.8), (0.7, 12, 0.6),
                                                     (2.0, 3, 0.99)])
def test_frequencies_match_filtered_softmax(temperature, top_k, top_p):
    rng = np.random.default_rng(int(temperature * 10) + top_k)
    logits = (1.5 * rng.standard_normal(50)).astype(np.float32)
    p = expected(logits, temperature, top_k, top_p)
    got = np.bincount(draws(logits, temperature, top_k, top_p, seed=42), minlength=50) / N_DRAWS
    assert np.all(got[p == 0] == 0), "a token outside the filtered support was drawn"
    sigma = np.sqrt(p * (1 - p) / N_DRAWS)
    assert np.all(np.abs(got - p) <= 5 * sigma + 1e-12), np.abs(got - p).max()
    # Pearson chi-square over the support, well inside its upper tail
    sup = p > 0
    chi2 = float(np.sum((got[sup] - p[sup]) ** 2 / p[sup]) * N_DRAWS)
    dof = int(sup.sum()) - 1
    assert chi2 < dof + 6 * np.sqrt(2 * max(dof, 1))


def test_greedy_settings_take_the_argmax():
    logits = np.array([0.1, 2.5, -1.0, 2.4999, 0.0], np.float32)
    assert set(draws(logits, 0.001, 0, 1.0, 7, 100)) == {1}
    assert set(draws(logits, 1.0, 1, 1.0, 7, 100)) == {1}
    # a tiny top_p keeps only the most likely token
    assert set(draws(logits, 1.0, 0, 1e-6, 7, 100)) == {1}


def test_draws_are_a_function_of_the_seed():
    logits = np.linspace(-1, 1, 64).astype(np.float32)
    a, b = draws(logits, 1.0, 0, 1.0, 5, 1000), draws(logits, 1.0, 0, 1.0, 5, 1000)
    np.testing.assert_array_equal(a, b)
    assert not np.array_equal(a, draws(logits, 1.0, 0, 1.0, 6, 1000))
