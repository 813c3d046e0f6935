"""Pins where the FFN norm weight enters the oracle's MoE block
(engine.py:229-236: normed = rms_norm(x, ffn_norms[i]); logits =
routers[i] @ normed; the experts run on normed).

References: float64 evaluations of the reference's formula, and a
power-of-two weight, under which every float32 step scales exactly, so the
result is known without restating the oracle's steps.
"""
import math

import numpy as np

U = 2.0 ** -24


def deq_tensor(O, buf, rows, cols):
    return O.dequantize_q4_0(buf, rows * cols).astype(np.float64).reshape(rows, cols)


def test_router_dot_g_unit_and_none(O):
    rng = np.random.default_rng(1)
    w = rng.standard_normal(512).astype(np.float32)
    x = rng.standard_normal(512).astype(np.float32)
    assert O.router_dot_g(w, None, x) == O.router_dot(w, x)
    assert O.router_dot_g(w, np.ones(512, np.float32), x) == O.router_dot(w, x)


def test_router_dot_g_against_float64(O):
    """(w * g) . x against float64 within the chain's error bound."""
    rng = np.random.default_rng(2)
    for _ in range(20):
        w = (rng.standard_normal(2048) * 0.02).astype(np.float32)
        g = (1.0 + 0.1 * rng.standard_normal(2048)).astype(np.float32)
        x = rng.standard_normal(2048).astype(np.float32)
        got = O.router_dot_g(w, g, x)
        wg = w.astype(np.float64) * g.astype(np.float64)
        ref = float(wg @ x.astype(np.float64))
        bound = (32 + 64 + 2) * U * float(np.abs(wg) @ np.abs(x.astype(np.float64)))
        assert abs(got - ref) <= bound


def test_norm_weight_power_of_two(O):
    """g = 2 everywhere: Q8_0(normed) keeps its quants and doubles its
    scales, the logits double, so the selected experts stay the same.  A
    weight applied to the sum of squares, dropped from the expert input or
    applied twice fails one of these."""
    H, I, E, k, T = 256, 64, 16, 4, 3
    layer, router = O.synth_layer(21, 0, H, I, E)
    x = O.synth_normal(21, O.stream_id(0, 1, 4), 1.0, T * H).reshape(T, H)
    _, idx1, _, xq1 = O.moe_layer(layer, router, H, I, E, k, x)
    _, idx2, _, xq2 = O.moe_layer(layer, router, H, I, E, k, x, norm=np.full(H, 2.0, np.float32))
    assert np.array_equal(idx1, idx2)
    b1 = xq1.reshape(T, H // 32, 34)
    b2 = xq2.reshape(T, H // 32, 34)
    assert np.array_equal(b1[:, :, 2:], b2[:, :, 2:])  # the int8 quants
    d1 = b1[:, :, :2].copy().view(np.float16).astype(np.float32)
    d2 = b2[:, :, :2].copy().view(np.float16).astype(np.float32)
    assert np.array_equal(d2, 2 * d1)
    for t in range(T):
        s = O.rms_scale(x[t])
        for e in range(E):
            l1 = O.router_dot_g(router[e], None, x[t]) * np.float32(s)
            l2 = O.router_dot_g(router[e], np.full(H, 2.0, np.float32), x[t]) * np.float32(s)
            assert l2 == 2 * l1


def test_norm_weight_layer_against_float64(O):
    """N(1, 0.1) norm weight: routing equals the float64 top-k of
    routers @ (x / rms(x) * g) where no near-tie, the expert input is
    Q8_0 of (x * s) * g element by element (tg_rms_norm's order,
    libtinygiant.c:338), and the output equals the float64 composition
    within the Q8 quantisation error."""
    H, I, E, k, T = 512, 128, 32, 8, 3
    rng = np.random.default_rng(22)
    g = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    layer, router = O.synth_layer(22, 0, H, I, E)
    x = O.synth_normal(22, O.stream_id(0, 2, 4), 1.0, T * H).reshape(T, H)
    out, idx, w, xq = O.moe_layer(layer, router, H, I, E, k, x, norm=g)
    eb = O.expert_bytes(H, I)
    gb = I * H // 32 * 18
    for t in range(T):
        x64 = x[t].astype(np.float64)
        xn = x64 / math.sqrt(np.mean(x64 ** 2) + 1e-6) * g.astype(np.float64)
        lg = router.astype(np.float64) @ xn
        order = np.argsort(-lg, kind="stable")
        if lg[order[k - 1]] - lg[order[k]] > 1e-4:
            assert sorted(idx[t].tolist()) == sorted(order[:k].tolist())
        s32 = np.float32(O.rms_scale(x[t]))
        xn32 = (x[t] * s32) * g  # float32 elementwise, as tg_rms_norm
        assert np.array_equal(xq[t], O.quantize_q8_0(xn32))
        ref = np.zeros(H)
        for j in range(k):
            ex = layer[idx[t, j] * eb:(idx[t, j] + 1) * eb]
            gg = deq_tensor(O, ex[:gb], I, H) @ xn
            uu = deq_tensor(O, ex[gb:2 * gb], I, H) @ xn
            h = gg / (1 + np.exp(-gg)) * uu
            ref += float(w[t, j]) * (deq_tensor(O, ex[2 * gb:], H, I) @ h)
        assert np.max(np.abs(out[t] - ref)) / np.max(np.abs(ref)) < 3e-2


def test_norm_weight_stack_composition(O):
    H, I, E, k = 256, 64, 16, 4
    rng = np.random.default_rng(23)
    L0, R0 = O.synth_layer(23, 0, H, I, E)
    L1, R1 = O.synth_layer(23, 1, H, I, E)
    g0 = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    g1 = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    x = O.synth_normal(23, O.stream_id(0, 0, 4), 1.0, 2 * H).reshape(2, H)
    got, _ = O.moe_stack([L0, L1], [R0, R1], H, I, E, k, x, norms=[g0, g1])
    o0, _, _, _ = O.moe_layer(L0, R0, H, I, E, k, x, norm=g0)
    x1 = x + o0
    o1, _, _, _ = O.moe_layer(L1, R1, H, I, E, k, x1, norm=g1)
    assert np.array_equal(got, x1 + o1)
