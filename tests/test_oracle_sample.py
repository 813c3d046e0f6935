"""The sampling restatement (oracle/sample.py) pinned against numpy itself.

engine.py:348-357 samples with numpy calls: np.sum, np.argsort, np.cumsum,
np.searchsorted and np.random.choice.  These tests check each step of the
restatement against those calls and against the closed forms the cutoff and
the draw must satisfy, so a wrong summation order, a wrong comparison side or
a dropped renormalisation fails here.
"""
import numpy as np
import pytest

from oracle import sample as S


@pytest.mark.parametrize("n", [1, 2, 7, 8, 9, 15, 16, 127, 128, 129, 135, 1000, 4480, 8191, 8192, 8193, 20000,
                               151936])
def test_np_sum_order_is_numpys(n):
    """np.sum of float32 vectors: buffers of 8192 added from 0, each summed
    pairwise.  Values spread over many binades so the order shows."""
    rng = np.random.default_rng(n)
    for _ in range(3):
        a = np.exp(rng.standard_normal(n) * 4).astype(np.float32)
        assert S.np_sum_order(a) == np.sum(a)


def test_np_sum_order_differs_from_other_orders():
    """The order matters at this size: a plain running sum and one pairwise
    tree over the whole vector both give other values."""
    rng = np.random.default_rng(7)
    a = np.exp(rng.standard_normal(151936) * 4).astype(np.float32)
    assert S.np_sum_order(a) == np.sum(a)
    assert S.pairwise_sum(a) != np.sum(a)
    seq = np.float32(0.0)
    for x in a[:20000]:
        seq = np.float32(seq + x)
    assert seq != np.sum(a[:20000])


def test_cumsum_is_sequential_float32():
    rng = np.random.default_rng(1)
    a = rng.random(10000).astype(np.float32)
    cs = np.cumsum(a)
    r = np.float32(0.0)
    for i, x in enumerate(a):
        r = np.float32(r + x)
        if i % 997 == 0:
            assert cs[i] == r


def test_searchsorted_compares_in_float64():
    """A python float top_p against float32 sums is compared in float64:
    0.9f < 0.9, so a running sum equal to 0.9f does not reach top_p 0.9."""
    cs = np.array([0.5, np.float32(0.9), 1.0], dtype=np.float32)
    assert np.searchsorted(cs, 0.9) == 2
    assert np.searchsorted(cs, float(np.float32(0.9))) == 1
    assert np.searchsorted(cs, np.nan) == 3  # NaN top_p: past the end, every token a candidate


@pytest.mark.parametrize("seed", range(6))
def test_draw_matches_random_state_choice(seed):
    """The explicit draw (cdf = cumsum(float64 p) / last, first > u) gives
    RandomState.choice's token for the same RandomState, whose choice takes
    exactly one random_sample() per draw."""
    rng = np.random.default_rng(100 + seed)
    V = 5000
    logits = (rng.standard_normal(V) * 2.5).astype(np.float32)
    for T, top_p in ((0.7, 0.9), (1.0, 0.95), (1.3, 0.5), (0.5, 1.0)):
        _, info = S.sample(logits, T, top_p, 0.5, exp="numpy")
        for k in range(8):
            rs = np.random.RandomState(1000 * seed + k)
            ref = int(rs.choice(info["cand"], p=info["cp"]))
            u = np.random.RandomState(1000 * seed + k).random_sample()
            tok, _ = S.sample(logits, T, top_p, u, exp="numpy")
            assert tok == ref


def test_order_without_ties_is_reversed_argsort():
    """With distinct probabilities the stable descending order is the
    reference's np.argsort(probs)[::-1]."""
    rng = np.random.default_rng(3)
    logits = rng.permutation(np.linspace(-8.0, 8.0, 5000)).astype(np.float32)  # 0.4% apart after exp
    _, info = S.sample(logits, 0.8, 0.9, 0.25, exp="numpy")
    p = info["probs"]
    assert np.unique(p[p > 0]).size == np.count_nonzero(p)
    nz = np.count_nonzero(p)
    assert np.array_equal(info["order"][:nz], np.argsort(p)[::-1][:nz])


def test_cutoff_is_minimal_prefix():
    """cutoff = the first running sum >= top_p, counted inclusively: the
    sum before it is below top_p and the sum at it reaches top_p."""
    rng = np.random.default_rng(4)
    logits = (rng.standard_normal(20000) * 2).astype(np.float32)
    for top_p in (0.1, 0.5, 0.9, 0.99):
        _, info = S.sample(logits, 1.0, top_p, 0.5)
        k = info["cutoff"] - 1
        cs = info["cs"].astype(np.float64)
        assert cs[k] >= top_p
        assert k == 0 or cs[k - 1] < top_p


def test_brute_force_frequencies_tiny_vocab():
    """Over a fine grid of u the token frequencies equal the renormalised
    candidate probabilities, and tokens outside the prefix never appear."""
    logits = np.array([2.0, 0.5, 1.0, -1.0, 1.0, 0.0], np.float32)
    T, top_p = 0.9, 0.8
    _, info = S.sample(logits, T, top_p, 0.0)
    N = 20000
    counts = np.zeros(logits.size)
    for i in range(N):
        tok, _ = S.sample(logits, T, top_p, (i + 0.5) / N)
        counts[tok] += 1
    cand = info["cand"]
    assert set(np.nonzero(counts)[0]) == set(cand.tolist())
    p = np.exp(logits.astype(np.float64) / T)
    p /= p.sum()
    order = sorted(range(logits.size), key=lambda i: (-p[i], i))
    acc, want = 0.0, []
    for i in order:
        want.append(i)
        acc += p[i]
        if acc >= top_p:
            break
    assert sorted(want) == sorted(cand.tolist())
    q = p[cand] / p[cand].sum()
    assert np.allclose(counts[cand] / N, q, atol=2.0 / N)
    # ties (logits 1.0 at ids 2 and 4) in ascending id order
    assert list(cand).index(2) < list(cand).index(4)


def test_special_cases():
    rng = np.random.default_rng(5)
    logits = (rng.standard_normal(1000) * 2).astype(np.float32)
    top = int(np.argmax(logits))
    for u in (0.0, 0.5, 0.999999):
        assert S.sample(logits, 1.0, 0.0, u)[0] == top        # cutoff 1
        assert S.sample(logits, 1.0, -3.0, u)[0] == top
        assert S.sample(logits, 0.0, 0.9, u)[0] == top        # greedy
        assert S.sample(logits, 1e-30, 0.9, u)[0] == top      # every other p underflows
    _, info = S.sample(logits, 1.0, 2.0, 0.5)                 # never reached: every token
    assert info["cutoff"] == logits.size + 1 and info["cand"].size == logits.size
    _, info = S.sample(logits, 1.0, float("nan"), 0.5)
    assert info["cand"].size == logits.size
    flat = np.zeros(64, np.float32)                           # equal logits: uniform, ids in order
    for i in range(64):
        assert S.sample(flat, 1.0, 1.0, (i + 0.5) / 64)[0] == i


def test_rounded_exp_within_two_ulp_of_numpy():
    """numpy's float32 exp against the correctly rounded value on the
    arguments a softmax meets."""
    rng = np.random.default_rng(6)
    z = (-rng.random(200000) * 90).astype(np.float32)
    a = np.exp(z).view(np.int32).astype(np.int64)
    b = np.exp(z.astype(np.float64)).astype(np.float32).view(np.int32).astype(np.int64)
    assert np.abs(a - b).max() <= 2
