"""Next-token sampling restated in numpy (tinygiant/engine.py:348-359).

TEST INFRASTRUCTURE ONLY: the checker that tests/ compare libtinygiant's
tg_sampler_run / tg_head_sample with.  Nothing in the product imports it.

The reference, per decode step with temperature > 0 (engine.py:348-357):
softmax of logits / T, the descending order of the probabilities, their
float32 running sum, the prefix up to and including the first sum >= top_p
(np.searchsorted + 1), those probabilities renormalised, and
np.random.choice over them.  Here the draw is explicit: RandomState.choice
widens p to float64, forms cdf = cumsum(p) / cdf[-1], takes ONE uniform
u = random_sample() and returns the first index with cdf > u
(searchsorted side='right'); sample() takes that u as an argument.

Two conventions the reference leaves open are fixed:
  * ties: np.argsort's default kind does not order equal values; the order
    here is descending probability, ties by ascending token id;
  * exp: exp="numpy" is the reference's float32 np.exp (within 2 ulp of the
    correctly rounded value, and CPU-dependent), exp="rounded" the fp32
    rounding of a float64 exp, which the GPU computes.
"""
from __future__ import annotations

import numpy as np

NP_BUFSIZE = 8192   # np.sum reduces a long vector in buffers of this many values
NP_PW_BLOCK = 128   # numpy's pairwise summation: unrolled base case size


def pairwise_sum(a: np.ndarray) -> np.float32:
    """numpy's pairwise summation of a float32 vector (one buffer): below 8
    values in order from 0; up to 128 values by 8 interleaved accumulators
    combined ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)), the last n % 8 values added
    in order; above, halves of n // 2 rounded down to a multiple of 8."""
    a = np.asarray(a, dtype=np.float32)
    n = a.size
    f = np.float32
    if n < 8:
        r = f(0.0)
        for x in a:
            r = f(r + x)
        return r
    if n <= NP_PW_BLOCK:
        main = n - n % 8
        r = [a[j] for j in range(8)]
        for i in range(8, main, 8):
            for j in range(8):
                r[j] = f(r[j] + a[i + j])
        res = f(f(f(r[0] + r[1]) + f(r[2] + r[3])) + f(f(r[4] + r[5]) + f(r[6] + r[7])))
        for i in range(main, n):
            res = f(res + a[i])
        return res
    n2 = n // 2
    n2 -= n2 % 8
    return f(pairwise_sum(a[:n2]) + pairwise_sum(a[n2:]))


def np_sum_order(a: np.ndarray) -> np.float32:
    """np.sum of a float32 vector restated: NP_BUFSIZE-value buffers, each
    by pairwise_sum, added one after another starting from 0.  The GPU
    sampler sums in this order; tests pin it against np.sum itself."""
    a = np.asarray(a, dtype=np.float32)
    s = np.float32(0.0)
    for c0 in range(0, a.size, NP_BUFSIZE):
        s = np.float32(s + pairwise_sum(a[c0:c0 + NP_BUFSIZE]))
    return s


def softmax_t(logits: np.ndarray, temperature: float, exp: str = "rounded") -> np.ndarray:
    """probs of engine.py:349-350: exp((l - max) / T) / sum, in float32 (the
    Python float T meets a float32 array, so the division is float32)."""
    l = np.asarray(logits, dtype=np.float32)
    z = (l - np.max(l)) / np.float32(temperature)
    if exp == "numpy":
        p = np.exp(z)
    elif exp == "rounded":
        p = np.exp(z.astype(np.float64)).astype(np.float32)
    else:
        raise ValueError(exp)
    return p / np.sum(p)


def sample(logits: np.ndarray, temperature: float, top_p: float, u: float, exp: str = "rounded"):
    """Token of engine.py:348-359 for the draw's uniform u.  Returns
    (token, info) with the intermediate arrays (None for greedy)."""
    l = np.asarray(logits, dtype=np.float32)
    if not temperature > 0:                         # engine.py:358-359
        return int(np.argmax(l)), None
    probs = softmax_t(l, temperature, exp)          # :349-350
    order = np.argsort(-probs, kind="stable")       # :351, ties by ascending id
    cs = np.cumsum(probs[order])                    # :352 (float32, in order)
    cutoff = int(np.searchsorted(cs, top_p)) + 1    # :353 (compared in float64)
    cand = order[:cutoff]                           # :354
    cp = probs[cand]
    cp = cp / np.sum(cp)                            # :355-356
    cdf = np.cumsum(cp.astype(np.float64))          # :357, RandomState.choice
    cdf /= cdf[-1]
    pos = int(np.searchsorted(cdf, u, side="right"))
    return int(cand[pos]), {"probs": probs, "order": order, "cs": cs, "cutoff": cutoff, "cand": cand, "cp": cp,
                            "cdf": cdf, "pos": pos}


def margins(info: dict, top_p: float, u: float) -> tuple:
    """Relative distance of top_p from the running sums next to the cutoff,
    and of u from the cdf values next to the drawn position: how far the
    probabilities may move before the token changes."""
    cs = info["cs"].astype(np.float64)
    k = min(info["cutoff"] - 1, cs.size - 1)
    near = cs[max(k - 1, 0):k + 1]
    m_cut = float(np.min(np.abs(near - top_p)) / max(abs(top_p), 1e-30)) if np.isfinite(top_p) else np.inf
    cdf = info["cdf"]
    pos = info["pos"]
    near = cdf[max(pos - 1, 0):pos + 1]
    m_draw = float(np.min(np.abs(near - u)))
    return m_cut, m_draw
