"""Pins the oracle's elementary functions, router, top-k, SwiGLU, grouping
and the expert / layer composition (oracle/tg_oracle.c) without the GPU.

The references here are float64 evaluations, brute-force sorts and
constructed special cases; none restates the oracle's own float32 steps.
"""
import math

import numpy as np
import pytest

U = 2.0 ** -24  # unit roundoff of float32


def ulp32(v: np.ndarray) -> np.ndarray:
    v = np.abs(np.asarray(v, np.float32))
    return np.spacing(v).astype(np.float64)


# ---------------------------------------------------------------- exp, ln, cos

def test_expf_ulp(O):
    lib = O.lib()
    xs = np.concatenate([np.linspace(-87.0, 88.0, 40001, dtype=np.float32),
                         np.array([0.0, -0.0, 1e-8, -1e-8, 0.5, -0.5, 1.0, -1.0], np.float32),
                         (np.random.default_rng(0).standard_normal(5000) * 4).astype(np.float32)])
    got = np.array([lib.tgo_expf(float(x)) for x in xs], np.float32)
    ref = np.exp(xs.astype(np.float64))
    err = np.abs(got.astype(np.float64) - ref) / ulp32(ref.astype(np.float32))
    assert err.max() <= 2.0, f"max error {err.max():.2f} ulp"


def test_expf_clamps(O):
    assert O.expf(-1000.0) == np.float32(math.exp(-87.0)) or abs(O.expf(-1000.0) / math.exp(-87) - 1) < 1e-6
    assert np.isfinite(O.expf(1000.0))
    assert O.expf(0.0) == 1.0


def test_ln_unit(O):
    lib = O.lib()
    u = np.concatenate([np.linspace(2.0 ** -24, 1.0, 20001), 2.0 ** -np.arange(0, 25)]).astype(np.float32)
    got = np.array([lib.tgo_ln_unit(float(v)) for v in u])
    assert np.max(np.abs(got - np.log(u.astype(np.float64)))) < 4e-6


def test_cos2pi(O):
    lib = O.lib()
    u = np.linspace(0.0, 1.0, 40001, endpoint=False).astype(np.float32)
    got = np.array([lib.tgo_cos2pi(float(v)) for v in u])
    assert np.max(np.abs(got - np.cos(2 * np.pi * u.astype(np.float64)))) < 2e-6


def test_normal_generator_moments(O):
    z = O.synth_normal(5, O.stream_id(0, 0, 4), 1.0, 400000).astype(np.float64)
    assert abs(z.mean()) < 0.01
    assert abs(z.std() - 1.0) < 0.01
    assert abs(np.mean(z ** 3)) < 0.02                  # skewness
    assert abs(np.mean(z ** 4) - 3.0) < 0.05            # kurtosis
    # tails of N(0,1): P(|z| > 2) = 0.0455, P(|z| > 3) = 0.0027
    assert abs(np.mean(np.abs(z) > 2) - 0.0455) < 0.002
    assert abs(np.mean(np.abs(z) > 3) - 0.0027) < 0.0005


def test_generator_is_counter_based(O):
    """Element i of a stream does not depend on how much is drawn."""
    a = O.synth_normal(9, 77, 0.02, 1000)
    b = O.synth_normal(9, 77, 0.02, 10)
    assert np.array_equal(a[:10], b)
    assert not np.array_equal(O.synth_normal(9, 78, 0.02, 10), b)
    q = O.synth_q40(9, 77, 0.02, 4, 64)
    assert np.array_equal(q, O.quantize_q4_0(O.synth_normal(9, 77, 0.02, 4 * 64)))


# ---------------------------------------------------------------- norm, router

def test_sumsq_and_rms_scale(O):
    rng = np.random.default_rng(1)
    for n in (32, 256, 2048, 4096):
        x = rng.standard_normal(n).astype(np.float32)
        exact = float(np.sum(x.astype(np.float64) ** 2))
        assert abs(O.sumsq(x) - exact) <= (32 + n // 32) * U * exact
        s = O.rms_scale(x, 1e-6)
        assert abs(s - 1.0 / math.sqrt(exact / n + 1e-6)) <= 2e-6 * s


def test_router_dot_grouped(O):
    rng = np.random.default_rng(2)
    for n in (256, 2048, 4096):
        w = (rng.standard_normal(n) * 0.02).astype(np.float32)
        x = rng.standard_normal(n).astype(np.float32)
        exact = float(w.astype(np.float64) @ x.astype(np.float64))
        mag = float(np.abs(w.astype(np.float64)) @ np.abs(x.astype(np.float64)))
        assert abs(O.router_dot(w, x) - exact) <= (32 + n // 32) * U * mag


def test_router_logits_scale(O):
    rng = np.random.default_rng(3)
    Wr = (rng.standard_normal((16, 256)) * 0.02).astype(np.float32)
    x = rng.standard_normal(256).astype(np.float32)
    s = O.rms_scale(x)
    lg = O.router_logits(Wr, x, s)
    exact = (Wr.astype(np.float64) @ x.astype(np.float64)) * s
    mag = (np.abs(Wr.astype(np.float64)) @ np.abs(x.astype(np.float64))) * s
    assert np.all(np.abs(lg - exact) <= 50 * U * mag)


# ---------------------------------------------------------------- top-k

def brute_topk(logits, k):
    order = sorted(range(len(logits)), key=lambda e: (-(logits[e] if logits[e] == logits[e] else -np.inf), e))
    return order[:k]


@pytest.mark.parametrize("E,k", [(16, 4), (128, 8), (64, 1), (8, 8)])
def test_topk_bruteforce(O, E, k):
    rng = np.random.default_rng(E * 10 + k)
    for _ in range(50):
        lg = rng.standard_normal(E).astype(np.float32)
        idx, w = O.topk_softmax(lg, k)
        assert idx.tolist() == brute_topk(lg.tolist(), k)


def test_topk_ties_lower_index_first(O):
    lg = np.zeros(32, np.float32)
    lg[[3, 9, 10, 30]] = 2.0
    lg[[1, 2]] = 1.0
    idx, w = O.topk_softmax(lg, 6)
    assert idx.tolist() == [3, 9, 10, 30, 1, 2]
    assert w[0] == w[1] == w[2] == w[3] and w[4] == w[5]


def test_topk_nan_ranks_last(O):
    """A NaN logit ranks as -inf: below every number, and tied with -inf,
    where the lower index goes first."""
    lg = np.array([np.nan, 0.5, -1.0, np.nan, 2.0, -np.inf], np.float32)
    idx, _ = O.topk_softmax(lg, 5)
    assert idx.tolist() == [4, 1, 2, 0, 3]


def test_topk_weights_are_renormalised_softmax(O):
    """engine.py:233-236: exp(l - lmax) / sum over the k; equals the full
    softmax restricted to the top k and renormalised."""
    rng = np.random.default_rng(4)
    for _ in range(100):
        lg = (rng.standard_normal(128) * 0.3).astype(np.float32)
        idx, w = O.topk_softmax(lg, 8)
        assert np.all(w > 0)
        assert np.all(np.diff(w.astype(np.float64)) <= 0)  # descending logits, descending weights
        assert abs(float(np.sum(w.astype(np.float64))) - 1.0) <= 8 * U
        full = np.exp(lg.astype(np.float64) - lg.max())
        full /= full.sum()
        ref = full[idx] / full[idx].sum()
        assert np.all(np.abs(w - ref) <= 8 * U * ref)


def test_topk_reference_weights_shape(O):
    """The combine weights of tools/nws_q8dot_bench.c:369 are a valid top-8
    weight vector: softmax of their logs reproduces them."""
    ref = np.array([.15, .14, .13, .13, .12, .11, .11, .11], np.float64)
    lg = np.full(16, -10.0, np.float32)
    lg[:8] = np.log(ref).astype(np.float32)
    idx, w = O.topk_softmax(lg, 8)
    assert idx.tolist() == [0, 1, 2, 3, 4, 5, 6, 7]
    assert np.all(np.abs(w - ref / ref.sum()) < 1e-6)


# ---------------------------------------------------------------- SwiGLU

def test_silu_mul(O):
    rng = np.random.default_rng(5)
    g = np.concatenate([rng.standard_normal(5000) * 3, [0.0, -80.0, 80.0, -100.0]]).astype(np.float32)
    u = rng.standard_normal(g.size).astype(np.float32)
    got = np.array([O.silu_mul(a, b) for a, b in zip(g, u)])
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    ref = g64 / (1 + np.exp(-g64)) * u64
    # below g = -88 the exponential's argument is clamped: the result is
    # then at most |g u| e^-88 instead of |g u| e^g, both negligible
    clamp = np.where(g64 < -88, np.abs(g64 * u64) * math.exp(-87), 0.0)
    assert np.all(np.abs(got - ref) <= 8 * U * np.abs(ref) + clamp + 1e-37)


# ---------------------------------------------------------------- grouping

def test_group_by_expert(O):
    rng = np.random.default_rng(6)
    T, k, E = 64, 8, 128
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    counts, offsets, perm, uniq = O.group_by_expert(idx, E)
    flat = idx.ravel()
    assert np.array_equal(counts, np.bincount(flat, minlength=E))
    assert offsets[0] == 0 and np.array_equal(np.diff(offsets), counts)
    assert np.array_equal(perm, np.argsort(flat, kind="stable"))
    assert uniq == len(np.unique(flat))


# ---------------------------------------------------------------- expert / layer

def deq_tensor(O, buf, rows, cols):
    return O.dequantize_q4_0(buf, rows * cols).astype(np.float64).reshape(rows, cols)


def test_expert_stages_against_float64(O):
    """gate/up rows, SiLU*up, Q8_0(h) and down rows of one expert, each stage
    against float64 on the same quantized inputs (role of
    libtinygiant.c:555-595)."""
    H, I = 512, 128
    ex = np.concatenate([O.synth_q40(3, O.stream_id(0, 0, t), 0.02, r, c)
                         for t, (r, c) in enumerate([(I, H), (I, H), (H, I)])])
    x = O.synth_normal(3, O.stream_id(0, 0, 4), 1.0, H)
    xq = O.quantize_q8_0(x)
    r = O.expert(ex, H, I, xq)
    gb = I * H // 32 * 18
    Wg = deq_tensor(O, ex[:gb], I, H)
    Wu = deq_tensor(O, ex[gb:2 * gb], I, H)
    Wd = deq_tensor(O, ex[2 * gb:], H, I)
    xd = O.dequantize_q8_0(xq, H).astype(np.float64)
    tol = lambda W, v: (H // 32 + 1) * U * (np.abs(W) @ np.abs(v))
    assert np.all(np.abs(r["gate"] - Wg @ xd) <= tol(Wg, xd))
    assert np.all(np.abs(r["up"] - Wu @ xd) <= tol(Wu, xd))
    g64, u64 = r["gate"].astype(np.float64), r["up"].astype(np.float64)
    href = g64 / (1 + np.exp(-g64)) * u64
    assert np.all(np.abs(r["h"] - href) <= 8 * U * np.abs(href) + 1e-37)
    assert np.array_equal(r["hq"], O.quantize_q8_0(r["h"]))
    hd = O.dequantize_q8_0(r["hq"], I).astype(np.float64)
    assert np.all(np.abs(r["down"] - Wd @ hd) <= (I // 32 + 1) * U * (np.abs(Wd) @ np.abs(hd)))


@pytest.mark.parametrize("H,I,E,k,T", [(256, 64, 16, 4, 3), (512, 128, 32, 8, 2)])
def test_moe_layer_against_float64(O, H, I, E, k, T):
    """engine.py:229-258 with Q4_0 experts: routing equals the brute-force
    top-k of float64 logits (where no near-tie), and the layer output equals
    the float64 composition within the Q8 quantization error (the
    reference's test 1b measures the same effect, csrc/test_libtinygiant.c:140-165)."""
    layer, router = O.synth_layer(11, 0, H, I, E)
    x = O.synth_normal(11, O.stream_id(0, 3, 4), 1.0, T * H).reshape(T, H)
    out, idx, w, xq = O.moe_layer(layer, router, H, I, E, k, x)
    eb = O.expert_bytes(H, I)
    gb = I * H // 32 * 18
    for t in range(T):
        x64 = x[t].astype(np.float64)
        xn = x64 / math.sqrt(np.mean(x64 ** 2) + 1e-6)
        lg = router.astype(np.float64) @ xn
        order = np.argsort(-lg, kind="stable")
        gap = lg[order[k - 1]] - lg[order[k]]
        if gap > 1e-4:
            assert sorted(idx[t].tolist()) == sorted(order[:k].tolist())
        assert np.array_equal(xq[t], O.quantize_q8_0(xn.astype(np.float32)))
        ref = np.zeros(H)
        for j in range(k):
            e = idx[t, j]
            ex = layer[e * eb:(e + 1) * eb]
            g = deq_tensor(O, ex[:gb], I, H) @ xn
            u = deq_tensor(O, ex[gb:2 * gb], I, H) @ xn
            h = g / (1 + np.exp(-g)) * u
            ref += float(w[t, j]) * (deq_tensor(O, ex[2 * gb:], H, I) @ h)
        rel = np.max(np.abs(out[t] - ref)) / np.max(np.abs(ref))
        assert rel < 3e-2, rel


def test_moe_stack_is_residual_composition(O):
    H, I, E, k = 256, 64, 16, 4
    L0, R0 = O.synth_layer(12, 0, H, I, E)
    L1, R1 = O.synth_layer(12, 1, H, I, E)
    x = O.synth_normal(12, O.stream_id(0, 0, 4), 1.0, 2 * H).reshape(2, H)
    got, trace = O.moe_stack([L0, L1], [R0, R1], H, I, E, k, x)
    o0, i0, _, _ = O.moe_layer(L0, R0, H, I, E, k, x)
    x1 = x + o0
    o1, i1, _, _ = O.moe_layer(L1, R1, H, I, E, k, x1)
    assert np.array_equal(got, x1 + o1)
    assert np.array_equal(trace[0], i0) and np.array_equal(trace[1], i1)
