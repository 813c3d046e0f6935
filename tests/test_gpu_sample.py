"""GPU parity of next-token sampling (tg_sampler_run, tg_head_sample) with
the numpy restatement of tinygiant/engine.py:348-359 (oracle/sample.py).

Bar, per call:
  * the probabilities bit-identical to the restatement with the correctly
    rounded exp, which the GPU computes (every later step, summation orders
    included, is numpy's), and the token identical;
  * the token identical to the restatement with numpy's own float32 exp (the
    reference's arithmetic), unless top_p or u lies closer to a running sum
    than that exp's 2-ulp rounding can move it (then the decision is not
    determined by the reference's arithmetic either; counted and reported).
Vocabulary 151,936 (Qwen3) with logit sets whose cutoffs run from a handful
of tokens (candidates sorted in LDS) to every token (the global-memory sort),
ties, -inf logits, edge values of top_p and u, the greedy path and errors.
"""
import ctypes

import numpy as np
import pytest

from oracle import sample as S
from tests.conftest import gpu_note

torch = pytest.importorskip("torch")  # before the library: torch brings its own HIP runtime

pytestmark = pytest.mark.gpu

V_QWEN = 151936
TG_E_INVALID = -1
US = (0.0, 0.123456789, 0.5, 0.87, 0.999999)


def ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


def logit_set(name, V, seed):
    rng = np.random.default_rng(seed)
    if name == "llm":
        return (rng.standard_normal(V) * 2.5).astype(np.float32)
    if name == "peaked":
        l = rng.standard_normal(V).astype(np.float32)
        l[rng.choice(V, min(12, V), replace=False)] = (14.0 + rng.random(min(12, V))).astype(np.float32)
        return l
    if name == "flat":
        return (rng.standard_normal(V) * 0.5).astype(np.float32)
    if name == "ties":
        return np.round(rng.standard_normal(V) * 3).astype(np.float32)
    if name == "neginf":
        l = (rng.standard_normal(V) * 2).astype(np.float32)
        l[rng.random(V) < 0.5] = -np.inf
        return l
    raise ValueError(name)


@pytest.fixture(scope="module")
def sampler_factory(tglib):
    made = []

    def make(V):
        s = tglib.tg_sampler_create(V)
        assert s, tglib.tg_last_error()
        made.append(s)
        return s
    yield make
    for s in made:
        tglib.tg_sampler_destroy(s)


def run(L, s, logits, T, top_p, u, probs=None):
    tok = ctypes.c_int32(-7)
    rc = L.tg_sampler_run(s, ptr(logits), 0, T, top_p, u, ctypes.byref(tok), None if probs is None else ptr(probs))
    return rc, tok.value


def check_case(L, s, logits, T, top_p, us=US):
    V = logits.size
    near = 0
    for u in us:
        probs = np.full(V, np.nan, np.float32)
        rc, tok = run(L, s, logits, np.float32(T), top_p, u, probs)
        assert rc == 0, L.tg_last_error().decode()
        ref_tok, info = S.sample(logits, T, top_p, u, exp="rounded")
        assert np.array_equal(probs.view(np.uint32), info["probs"].view(np.uint32)), "probabilities"
        assert tok == ref_tok, f"u={u}: token {tok} vs {ref_tok} (cutoff {info['cutoff']})"
        np_tok, np_info = S.sample(logits, T, top_p, u, exp="numpy")
        if np_tok != tok:
            m = S.margins(np_info, top_p, u)
            assert min(m) < 1e-5, f"u={u}: token {tok} vs numpy's {np_tok} with decision margins {m}"
            near += 1
    return near


@pytest.mark.parametrize("name", ["llm", "peaked", "flat", "ties", "neginf"])
@pytest.mark.parametrize("T,top_p", [(0.6, 0.9), (1.0, 0.95), (1.0, 0.5), (1.5, 0.9), (1.0, 1.0)])
def test_sample_vocab_151936(tglib, sampler_factory, name, T, top_p):
    gpu_note(f"tg_sampler_run V={V_QWEN} {name} T={T} top_p={top_p}")
    s = sampler_factory(V_QWEN)
    logits = logit_set(name, V_QWEN, 11)
    near = check_case(tglib, s, logits, T, top_p)
    print(f"  cutoff {S.sample(logits, T, top_p, 0.5)[1]['cutoff']}, near-boundary draws {near}")


@pytest.mark.parametrize("top_p", [0.0, -1.0, 1e-9, 0.999, 2.0, float("nan"), float("inf")])
def test_sample_top_p_edges(tglib, sampler_factory, top_p):
    gpu_note(f"tg_sampler_run V={V_QWEN} top_p={top_p}")
    s = sampler_factory(V_QWEN)
    check_case(tglib, s, logit_set("llm", V_QWEN, 12), 0.9, top_p, us=(0.0, 0.61, 0.999999))


@pytest.mark.parametrize("V", [1, 2, 7, 100, 129, 8192, 8193, 20000, 524288])
def test_sample_vocab_sizes(tglib, sampler_factory, V):
    gpu_note(f"tg_sampler_run V={V}")
    s = sampler_factory(V)
    for name, T, top_p in (("llm", 1.0, 0.9), ("flat", 1.2, 0.97), ("peaked", 0.7, 0.6)):
        check_case(tglib, s, logit_set(name, V, V), T, top_p, us=(0.05, 0.5, 0.95))


def test_sample_uniform_and_extreme_temperatures(tglib, sampler_factory):
    gpu_note("tg_sampler_run equal logits, T extremes")
    V = 4096
    s = sampler_factory(V)
    flat = np.zeros(V, np.float32)
    for i in (0, 1, 1000, 4095):  # equal probabilities: ids in order, u picks id floor(u V)
        rc, tok = run(tglib, s, flat, np.float32(1.0), 1.0, (i + 0.5) / V)
        assert rc == 0 and tok == i
    l = logit_set("llm", V, 3)
    check_case(tglib, s, l, 1e-30, 0.9)        # every other p underflows
    check_case(tglib, s, l, 1e30, 0.9)         # every p is 1
    check_case(tglib, s, l, float(np.float32(3e38)), 0.5)


def test_sample_greedy_and_errors(tglib, sampler_factory):
    gpu_note("tg_sampler_run greedy and error returns")
    V = 50000
    s = sampler_factory(V)
    l = logit_set("ties", V, 5)
    for T in (0.0, -1.0, float("nan")):  # engine.py:358-359: np.argmax, first of the ties
        rc, tok = run(tglib, s, l, np.float32(T), 0.9, 2.0)
        assert rc == 0 and tok == int(np.argmax(l))
    for bad in (np.nan, np.inf):
        b = l.copy()
        b[777] = bad
        rc, tok = run(tglib, s, b, np.float32(1.0), 0.9, 0.5)
        assert rc == TG_E_INVALID and b"NaN" in tglib.tg_last_error()
    rc, _ = run(tglib, s, np.full(V, -np.inf, np.float32), np.float32(1.0), 0.9, 0.5)
    assert rc == TG_E_INVALID
    for u in (1.0, -0.25, float("nan")):
        rc, _ = run(tglib, s, l, np.float32(1.0), 0.9, u)
        assert rc == TG_E_INVALID
    rc, tok = run(tglib, s, l, np.float32(1.0), 0.9, 0.5)  # a good call after the errors
    assert rc == 0 and tok == S.sample(l, 1.0, 0.9, 0.5)[0]
    assert not tglib.tg_sampler_create(0)
    assert not tglib.tg_sampler_create(524289)


def test_sample_device_logits(tglib, sampler_factory):
    """Logits already in HBM (a torch tensor) sample without a copy."""
    gpu_note("tg_sampler_run device logits")
    V = V_QWEN
    s = sampler_factory(V)
    l = logit_set("llm", V, 21)
    dl = torch.from_numpy(l).to("cuda:0")
    torch.cuda.synchronize()
    for u in (0.2, 0.7):
        tok = ctypes.c_int32(-1)
        rc = tglib.tg_sampler_run(s, ctypes.c_void_p(dl.data_ptr()), 1, np.float32(0.8), 0.92, u,
                                  ctypes.byref(tok), None)
        assert rc == 0, tglib.tg_last_error()
        assert tok.value == S.sample(l, 0.8, 0.92, u)[0]


def test_head_sample(O, tglib):
    """tg_head_sample: the head's logits (bit-identical to the oracle's norm +
    fp32 matvec) sampled on the device."""
    vocab, embed = 32000, 1024
    gpu_note(f"tg_head_sample vocab={vocab} embed={embed}")
    rng = np.random.default_rng(9)
    W = rng.standard_normal((vocab, embed), dtype=np.float32) * np.float32(0.05)
    nw = rng.normal(1.0, 0.1, embed).astype(np.float32)
    h = tglib.tg_head_create(ptr(W), ptr(nw), vocab, embed)
    assert h, tglib.tg_last_error()
    try:
        for i, (T, top_p, u) in enumerate(((0.7, 0.9, 0.3), (1.0, 0.95, 0.8), (0.0, 0.9, 0.5), (1.2, 1.0, 0.01))):
            x = rng.normal(0, 1, embed).astype(np.float32)
            ref_logits, _ = O.output_head(W, nw, x, 1e-6)
            out = np.zeros(vocab, np.float32)
            tok = ctypes.c_int32(-1)
            rc = tglib.tg_head_sample(h, ptr(x), 1e-6, np.float32(T), top_p, u, ptr(out), ctypes.byref(tok))
            assert rc == 0, tglib.tg_last_error()
            assert np.array_equal(out.view(np.uint32), ref_logits.view(np.uint32))
            assert tok.value == S.sample(ref_logits, T, top_p, u)[0]
    finally:
        tglib.tg_head_destroy(h)
