"""The oracle's token sampler (oracle_sample, restating model.cpp:1659-1728 and libstdc++'s
std::discrete_distribution) pinned on the reference's own sample() and on what the mathematics
fixes; the device sampler is checked against it in test_gpu_sample.py.

* reference: oracle/_ref/libref_sampler.so is the reference's model.cpp compiled from its source
  (oracle/Makefile.ref); its init_sampler/sample run a seeded std::mt19937 through several calls,
  and the oracle, fed the same generator's variates (Draws), must pick the same ids. Skipped when
  the reference sources were not there to build it.
* ties: std::partial_sort leaves the order of equal logits open; the oracle orders them by id. On
  logits full of ties the reference's pick and the oracle's must still be the same weight slot
  (equal logits) on every call, so the generators stay in step.
* closed forms: the draw as a step function of u whose steps are the float64 softmax
  probabilities after the top-k and top-p cuts; top-k 1 and top-p 0 give the argmax without a
  draw; the penalty's sign rule; argmax's NaN rule; the C++ standard's known answer for
  std::mt19937 (the 10000th output of the default seed is 4123659995, [rand.predef]).
"""
import numpy as np
import pytest

from gl import Draws, oracle_sample, oracle_sample_seq, ref_sample_seq, ref_sampler

REF = ref_sampler()
needs_ref = pytest.mark.skipif(REF is None, reason="oracle/_ref/libref_sampler.so not built (no /root/reference)")


def tie_free(rng, n, scale=3.0):
    v = np.unique((rng.standard_normal(n + n // 4 + 16) * scale).astype(np.float32))
    assert v.size >= n
    return rng.permutation(v[rng.choice(v.size, n, replace=False)])


def test_draws_are_std_mt19937():
    d = Draws(5489)
    raw = d.bg.random_raw(10000)
    assert int(raw[0]) == 3499211612
    assert int(raw[9999]) == 4123659995


def test_draws_are_generate_canonical():
    d = Draws(42)
    ref = Draws(42).bg.random_raw(4)
    u0 = d.peek()
    assert u0 == d.peek()                       # pending until consumed
    assert u0 == (float(ref[0]) + float(ref[1]) * 2.0 ** 32) / 2.0 ** 64
    d.consume()
    assert d.peek() == (float(ref[2]) + float(ref[3]) * 2.0 ** 32) / 2.0 ** 64
    assert 0.0 <= u0 < 1.0


PARAMS = [
    dict(temp=0.8),
    dict(temp=1.0, top_k=0, top_p=1.0),
    dict(temp=1.5, top_k=0),
    dict(temp=0.7, top_p=0.5, repeat_penalty=1.3),
    dict(temp=2.0, top_k=5000, top_p=0.99, repeat_penalty=0.7, repeat_last_n=-1),
    dict(temp=0.0, repeat_penalty=1.2),
    dict(temp=1.0, top_k=1),
    dict(temp=0.9, top_k=3, top_p=1.0, repeat_penalty=1.1, repeat_last_n=0),
]


@needs_ref
@pytest.mark.parametrize("n", [50, 32000, 151936])
def test_oracle_matches_reference_sample(n):
    rng = np.random.default_rng(n)
    x = tie_free(rng, n)
    recent = np.concatenate([rng.integers(0, n, 150), rng.integers(0, 20, 50), [-3, n + 5]]).astype(np.int32)
    calls = 32 if n < 100000 else 12
    for i, params in enumerate(PARAMS):
        seed = 1000 + i
        ref = ref_sample_seq(REF, x, recent, seed, calls, **params)
        got = oracle_sample_seq(x, recent, seed, calls, **params)
        assert got == ref, (n, params)


@needs_ref
@pytest.mark.parametrize("n", [64, 5000, 128256])
def test_oracle_ties_take_the_reference_slot(n):
    rng = np.random.default_rng(7 + n)
    x = (np.round(rng.standard_normal(n) * 8) / 4).astype(np.float32)    # many exact ties
    for params in (dict(temp=1.0), dict(temp=1.0, top_k=0, top_p=1.0), dict(temp=0.5, top_k=7),
                   dict(temp=3.0, top_k=2000, top_p=0.9)):
        ref = ref_sample_seq(REF, x, [], 77, 48, **params)
        got = oracle_sample_seq(x, [], 77, 48, **params)
        assert all(x[a] == x[b] for a, b in zip(ref, got)), (n, params)


def softmax_cut(x, temp, top_k, top_p):
    """float64 probabilities of each id after the cuts (ids ordered by value, then id)"""
    order = sorted(range(len(x)), key=lambda i: (-float(x[i]), i))
    k = top_k if 0 < top_k < len(x) else len(x)
    order = order[:k]
    p = np.exp((x[order].astype(np.float64) - float(x[order[0]])) / temp)
    p /= p.sum()
    if top_p < 1.0:
        c = np.cumsum(p)
        m = int(np.searchsorted(c, top_p) + 1)
        order, p = order[:m], p[:m] / p[:m].sum()
    out = np.zeros(len(x))
    out[order] = p
    return out


@pytest.mark.parametrize("temp,top_k,top_p", [(1.0, 0, 1.0), (0.5, 0, 1.0), (2.0, 4, 1.0), (1.0, 0, 0.8), (0.7, 5, 0.9)])
def test_draw_is_the_inverse_cdf_of_the_cut_softmax(temp, top_k, top_p):
    x = np.array([0.3, 2.0, -1.0, 1.1, 0.95, -0.2, 1.7, 0.0], dtype=np.float32)
    want = softmax_cut(x, temp, top_k, top_p)
    m = 20000
    us = (np.arange(m) + 0.5) / m
    hits = np.zeros(len(x))
    for u in us:
        tok, used = oracle_sample(x, (), float(u), temp=temp, top_k=top_k, top_p=top_p)
        assert used == (np.count_nonzero(want) >= 2)
        hits[tok] += 1
    np.testing.assert_allclose(hits / m, want, atol=1.5 / m)
    # the ids in order of u: descending value
    first = oracle_sample(x, (), 1e-9, temp=temp, top_k=top_k, top_p=top_p)[0]
    assert first == int(np.argmax(x))


def test_cuts_to_one_token_are_the_argmax_without_a_draw():
    rng = np.random.default_rng(3)
    x = tie_free(rng, 1000)
    for params in (dict(temp=1.0, top_k=1), dict(temp=1.0, top_p=0.0), dict(temp=0.0)):
        tok, used = oracle_sample(x, (), 0.999, **params)
        assert tok == int(np.argmax(x)) and not used


def test_penalty_sign_rule_and_repeats():
    # positive logits divided, negative multiplied, once per occurrence in the window
    x = np.array([2.0, 1.9, -1.0, -1.05, 0.5], dtype=np.float32)
    assert oracle_sample(x, [0], temp=0.0, repeat_penalty=1.02)[0] == 0          # 1.9608 > 1.9
    assert oracle_sample(x, [0, 0], temp=0.0, repeat_penalty=1.04)[0] == 1       # 2 / 1.04^2 < 1.9
    y = np.array([-1.0, -1.05, -3.0], dtype=np.float32)
    assert oracle_sample(y, [0], temp=0.0, repeat_penalty=1.1)[0] == 1           # -1.1 < -1.05
    # the window: the last repeat_last_n entries (negative: all of them); ids outside the row skipped
    assert oracle_sample(x, [0, 4, 4], temp=0.0, repeat_penalty=1.5, repeat_last_n=2)[0] == 0
    assert oracle_sample(x, [0, 4, 4], temp=0.0, repeat_penalty=1.5, repeat_last_n=-1)[0] == 1
    assert oracle_sample(x, [7, -1], temp=0.0, repeat_penalty=9.0)[0] == 0


def test_argmax_nan_rule():
    nan = np.float32(np.nan)
    assert oracle_sample(np.array([nan, 5, 9], np.float32), temp=0.0)[0] == 0
    assert oracle_sample(np.array([1, nan, 0.5, 3, 3], np.float32), temp=0.0)[0] == 3
