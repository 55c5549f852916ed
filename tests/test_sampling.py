"""The C ABI's sampler (oxb_sample_logits, host code) against properties that
rs/sampling.rs:4-80 fixes, with the uniform draw u passed in so that no RNG
has to agree with the reference's `rand`:

- repetition penalty: positive logits divided, others multiplied, once per
  occurrence in the window (a duplicate is penalised twice, :14-24);
- temperature: logits * (1/T) when T != 1 (:27-33); T = 0 gives inf/NaN
  logits and the draw falls through to the last index, as in the reference;
- top-k: everything below the k-th largest value becomes -inf, values equal
  to it are kept (:36-59);
- draw: the first index whose running sum of exp(l - max) reaches u * sum
  (:61-79), so over a fine grid of u the share of each token is its softmax
  probability.
"""
import ctypes as C

import numpy as np
import pytest

from helpers import pkg


def sample(logits, temperature=1.0, top_k=0, penalty=1.0, recent=(), u=0.5):
    lg = np.ascontiguousarray(logits, np.float32).copy()
    rec = np.ascontiguousarray(recent, np.int32)
    L = pkg.lib()
    return L.oxb_sample_logits(lg.ctypes.data, lg.size, float(temperature), int(top_k),
                               float(penalty), rec.ctypes.data if rec.size else None, rec.size,
                               float(u))


def shares(logits, n=20000, **kw):
    """Fraction of a uniform grid of u that draws each token."""
    V = len(logits)
    counts = np.zeros(V)
    for u in (np.arange(n) + 0.5) / n:
        counts[sample(logits, u=u, **kw)] += 1
    return counts / n


def softmax64(x):
    x = np.asarray(x, np.float64)
    e = np.exp(x - x.max())
    return e / e.sum()


LOGITS = np.array([0.3, 2.0, -1.0, 1.5, 0.9, -0.2, 2.4, 0.0], np.float32)


def test_top1_is_the_argmax_for_any_draw():
    for u in (1e-7, 0.3, 0.999):
        assert sample(LOGITS, top_k=1, u=u) == int(np.argmax(LOGITS))
    # a draw of exactly 0 stops at index 0 whatever its probability (the
    # running sum 0 already reaches r = 0), as the reference's `cumsum >= r`
    # does; rand's f32 draw is 0 with probability 2^-24
    assert sample(LOGITS, top_k=1, u=0.0) == 0


def test_repetition_penalty_divides_positive_multiplies_negative_per_occurrence():
    lg = np.array([1.0, 2.4, 2.0, -0.5], np.float32)
    # 2.4 / 1.1 = 2.18 > 2.0: still token 1;  2.4 / 1.1^2 = 1.98 < 2.0: token 2
    assert sample(lg, top_k=1, penalty=1.1, recent=[1]) == 1
    assert sample(lg, top_k=1, penalty=1.1, recent=[1, 1]) == 2
    # a negative logit is multiplied (made smaller), never divided toward 0
    lg2 = np.array([-1.0, -1.05, -3.0], np.float32)
    assert sample(lg2, top_k=1, penalty=1.2, recent=[0]) == 1      # -1.2 < -1.05
    assert sample(lg2, top_k=1, penalty=1.2, recent=[1, 2]) == 0   # -1.26 and -3.6
    # penalty 1 and ids outside the vocabulary change nothing
    assert sample(lg, top_k=1, penalty=1.0, recent=[1, 1, 1]) == 1
    assert sample(lg, top_k=1, penalty=1.5, recent=[99, -5 & 0x7fffffff]) == 1


@pytest.mark.parametrize("T", [1.0, 0.7, 1.6])
def test_draw_shares_are_the_tempered_softmax(T):
    got = shares(LOGITS, temperature=T)
    want = softmax64(LOGITS.astype(np.float64) / T)
    assert np.abs(got - want).max() < 2e-3


@pytest.mark.parametrize("k", [1, 2, 3, 5])
def test_top_k_keeps_exactly_the_k_largest(k):
    got = shares(LOGITS, top_k=k, temperature=0.9)
    top = np.argsort(-LOGITS)[:k]
    assert set(np.nonzero(got)[0]) == set(top.tolist())
    want = np.zeros(len(LOGITS))
    want[top] = softmax64(LOGITS[top].astype(np.float64) / 0.9)
    assert np.abs(got - want).max() < 2e-3


def test_top_k_keeps_values_equal_to_the_threshold_and_k_ge_v_keeps_all():
    lg = np.array([3.0, 2.0, 2.0, 1.0], np.float32)
    assert set(np.nonzero(shares(lg, top_k=2, n=4000))[0]) == {0, 1, 2}
    for k in (0, 4, 10):
        assert set(np.nonzero(shares(lg, top_k=k, n=4000))[0]) == {0, 1, 2, 3}


def test_temperature_zero_falls_through_to_the_last_index():
    """1/0 = inf makes every logit +-inf or NaN; the running sum is NaN and
    never reaches the draw (rs/sampling.rs:27-33 has no greedy special case)."""
    assert sample(LOGITS, temperature=0.0, top_k=50, u=0.4) == len(LOGITS) - 1


def test_sampler_rejects_empty_logits():
    L = pkg.lib()
    assert L.oxb_sample_logits(None, 0, 1.0, 0, 1.0, None, 0, 0.5) == -1
