"""Pins the oracle's restatement of the reference's attention decode step, its
RoPE and the transformer layer (csrc/libtinygiant.c:344-551, 662-702) with
checks that do not reuse the oracle's code:

- RoPE against a float64 rotation, and the identity at cos 1 / sin 0 exactly;
- attention (f32 weights) against a float64 numpy restatement of the same
  steps (projections, per-head RMS norm, RoPE, GQA softmax attention over the
  cache with the new row, output projection), normwise within 2e-5;
- attention with Q4_K / f16 weights against float64 on the dequantized
  weights and the Q8-quantized activations (the two points where the
  reference quantizes), normwise within 2e-5;
- the one-position case (kv_len 0), which reduces to the output projection of
  the value rows (softmax of one score is exactly 1), bit for bit, and the
  cache rows: the new row at kv_len, every other row untouched;
- the transformer layer against the composition of its pieces, bit for bit.
"""
import numpy as np
import pytest


def rope_tables(kv_max, half, base=10000.0):
    inv = base ** (-np.arange(half, dtype=np.float64) / half)
    ang = np.arange(kv_max, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rms64(v, w, eps=1e-6):
    v = np.asarray(v, np.float64)
    return v / np.sqrt(np.mean(v * v) + eps) * np.asarray(w, np.float64)


def rope64(x, n_heads, hd, c, s):
    x = np.asarray(x, np.float64).reshape(n_heads, hd).copy()
    half = hd // 2
    c = np.asarray(c, np.float64)
    s = np.asarray(s, np.float64)
    x1, x2 = x[:, :half].copy(), x[:, half:].copy()
    x[:, :half] = x1 * c - x2 * s
    x[:, half:] = x1 * s + x2 * c
    return x.reshape(-1)


def attn64(q, kn, v, kv_k, kv_v, kv_len, n_heads, n_kv_heads, hd):
    """GQA attention in float64 over the cache rows 0..kv_len-1 and the new row."""
    ratio = n_heads // n_kv_heads
    out = np.zeros(n_heads * hd)
    for h in range(n_heads):
        kh = h // ratio
        K = np.vstack([kv_k[kh, :kv_len].astype(np.float64), kn[kh * hd:(kh + 1) * hd][None, :]])
        V = np.vstack([kv_v[kh, :kv_len].astype(np.float64), v[kh * hd:(kh + 1) * hd][None, :]])
        sc = K @ q[h * hd:(h + 1) * hd] / np.sqrt(hd)
        p = np.exp(sc - sc.max())
        p /= p.sum()
        out[h * hd:(h + 1) * hd] = p @ V
    return out


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


GEOM = dict(embed=256, n_heads=4, n_kv_heads=2, hd=64, kv_max=16)


def make_f32(rng, g):
    e, H, KV, hd = g["embed"], g["n_heads"], g["n_kv_heads"], g["hd"]
    w = dict(
        wq=rng.normal(0, 0.05, (H * hd, e)).astype(np.float32),
        wk=rng.normal(0, 0.05, (KV * hd, e)).astype(np.float32),
        wv=rng.normal(0, 0.05, (KV * hd, e)).astype(np.float32),
        wo=rng.normal(0, 0.05, (e, H * hd)).astype(np.float32),
        qn=rng.normal(1.0, 0.1, hd).astype(np.float32),
        kn=rng.normal(1.0, 0.1, hd).astype(np.float32),
    )
    return w


def test_rope_rotation(O):
    rng = np.random.default_rng(3)
    n_heads, hd, kv_max = 3, 64, 12
    c, s = rope_tables(kv_max, hd // 2)
    x = rng.normal(0, 1, n_heads * hd).astype(np.float32)
    for pos in (0, 5, 11):
        got = O.rope(x, n_heads, hd, c, s, pos)
        assert rel(got, rope64(x, n_heads, hd, c[pos], s[pos])) < 4e-7, pos
    # cos 1 / sin 0 (position 0 of the tables): the identity, bit for bit
    got = O.rope(x, n_heads, hd, c, s, 0)
    assert np.array_equal(got.view(np.uint32), x.view(np.uint32))


@pytest.mark.parametrize("kv_len", [0, 1, 7, 15])
def test_attention_f32_vs_float64(O, kv_len):
    g = GEOM
    rng = np.random.default_rng(10 + kv_len)
    w = make_f32(rng, g)
    c, s = rope_tables(g["kv_max"], g["hd"] // 2)
    kv_k = rng.normal(0, 1, (g["n_kv_heads"], g["kv_max"], g["hd"])).astype(np.float32)
    kv_v = rng.normal(0, 1, (g["n_kv_heads"], g["kv_max"], g["hd"])).astype(np.float32)
    k0, v0 = kv_k.copy(), kv_v.copy()
    x = rng.normal(0, 1, g["embed"]).astype(np.float32)
    pos = kv_len
    out = O.attention_decode(False, w["wq"], w["wk"], w["wv"], w["wo"], w["qn"], w["kn"], kv_k, kv_v, kv_len,
                             g["kv_max"], c, s, x, g["embed"], g["n_heads"], g["n_kv_heads"], g["hd"], pos)
    hd, H, KV = g["hd"], g["n_heads"], g["n_kv_heads"]
    q = w["wq"].astype(np.float64) @ x
    k = w["wk"].astype(np.float64) @ x
    v = w["wv"].astype(np.float64) @ x
    qn = np.concatenate([rms64(q[h * hd:(h + 1) * hd], w["qn"]) for h in range(H)])
    kn = np.concatenate([rms64(k[h * hd:(h + 1) * hd], w["kn"]) for h in range(KV)])
    qn = rope64(qn, H, hd, c[pos], s[pos])
    kn = rope64(kn, KV, hd, c[pos], s[pos])
    ao = attn64(qn, kn, v, k0, v0, kv_len, H, KV, hd)
    ref = w["wo"].astype(np.float64) @ ao
    assert rel(out, ref) < 2e-5
    # the cache: the new row at kv_len, every other row unchanged
    for h in range(KV):
        assert rel(kv_k[h, kv_len], kn[h * hd:(h + 1) * hd]) < 2e-6
        assert rel(kv_v[h, kv_len], v[h * hd:(h + 1) * hd]) < 2e-6
    mask = np.ones(g["kv_max"], bool)
    mask[kv_len] = False
    assert np.array_equal(kv_k[:, mask], k0[:, mask]) and np.array_equal(kv_v[:, mask], v0[:, mask])


def test_attention_one_position_is_value_projection(O):
    """kv_len 0: one score, softmax weight exactly 1, so each head's output is
    its kv head's value row and the result is the output projection of those
    rows (the reference's own f32 matvec), bit for bit."""
    g = GEOM
    rng = np.random.default_rng(21)
    w = make_f32(rng, g)
    c, s = rope_tables(g["kv_max"], g["hd"] // 2)
    kv_k = np.zeros((g["n_kv_heads"], g["kv_max"], g["hd"]), np.float32)
    kv_v = np.zeros_like(kv_k)
    x = rng.normal(0, 1, g["embed"]).astype(np.float32)
    out = O.attention_decode(False, w["wq"], w["wk"], w["wv"], w["wo"], w["qn"], w["kn"], kv_k, kv_v, 0,
                             g["kv_max"], c, s, x, g["embed"], g["n_heads"], g["n_kv_heads"], g["hd"], 0)
    v = O.matvec_f32(w["wv"], x)
    hd, ratio = g["hd"], g["n_heads"] // g["n_kv_heads"]
    ao = np.concatenate([v[(h // ratio) * hd:(h // ratio + 1) * hd] for h in range(g["n_heads"])])
    ref = O.matvec_f32(w["wo"], ao)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(kv_v[:, 0].reshape(-1).view(np.uint32), v.view(np.uint32))


def q4k_rows(O, rng, nrows, ncols):
    from tests.test_oracle_legacy import pack_scales
    bpr = ncols // 256
    n = nrows * bpr
    blk = np.zeros((n, 144), np.uint8)
    blk[:, 0:2] = rng.uniform(0.0005, 0.002, n).astype(np.float16).view(np.uint8).reshape(n, 2)
    blk[:, 2:4] = rng.uniform(0.0, 0.002, n).astype(np.float16).view(np.uint8).reshape(n, 2)
    for i in range(n):
        blk[i, 4:16] = pack_scales(rng.integers(0, 64, 8), rng.integers(0, 64, 8))
    blk[:, 16:] = rng.integers(0, 256, (n, 128), dtype=np.uint8)
    flat = blk.reshape(-1)
    deq = np.concatenate([O.dequant_q4k_block(blk[i]) for i in range(n)]).reshape(nrows, ncols)
    return flat, deq.astype(np.float64)


def q8k_deq(O, x):
    """x after the reference's 256-value Q8 quantization, as float64."""
    blocks = O.quantize_q8k(x)
    out = []
    for b in blocks:
        out.append(np.float64(b["scale"]) * b["qs"].astype(np.float64))
    return np.concatenate(out)


def test_attention_q4_vs_float64(O):
    g = dict(GEOM, embed=512, hd=128, n_heads=2, n_kv_heads=1)
    rng = np.random.default_rng(33)
    e, H, KV, hd, kv_len = g["embed"], g["n_heads"], g["n_kv_heads"], g["hd"], 6
    wq, dq = q4k_rows(O, rng, H * hd, e)
    wk, dk = q4k_rows(O, rng, KV * hd, e)
    wo, do = q4k_rows(O, rng, e, H * hd)
    wv = rng.normal(0, 0.05, (KV * hd, e)).astype(np.float16)
    qn_w = rng.normal(1.0, 0.1, hd).astype(np.float32)
    kn_w = rng.normal(1.0, 0.1, hd).astype(np.float32)
    c, s = rope_tables(g["kv_max"], hd // 2)
    kv_k = rng.normal(0, 1, (KV, g["kv_max"], hd)).astype(np.float32)
    kv_v = rng.normal(0, 1, (KV, g["kv_max"], hd)).astype(np.float32)
    k0, v0 = kv_k.copy(), kv_v.copy()
    x = rng.normal(0, 1, e).astype(np.float32)
    out = O.attention_decode(True, wq, wk, wv.view(np.uint16), wo, qn_w, kn_w, kv_k, kv_v, kv_len, g["kv_max"], c,
                             s, x, e, H, KV, hd, kv_len)
    xq = q8k_deq(O, x)
    q = dq @ xq
    k = dk @ xq
    v = wv.astype(np.float64) @ x
    qn = rope64(np.concatenate([rms64(q[h * hd:(h + 1) * hd], qn_w) for h in range(H)]), H, hd, c[kv_len], s[kv_len])
    kn = rope64(np.concatenate([rms64(k[h * hd:(h + 1) * hd], kn_w) for h in range(KV)]), KV, hd, c[kv_len],
                s[kv_len])
    ao = attn64(qn, kn, v, k0, v0, kv_len, H, KV, hd)
    # the output projection quantizes the attention output (fp32) to Q8 first
    ref = do @ q8k_deq(O, ao.astype(np.float32))
    assert rel(out, ref) < 2e-5  # the Q8 points are reproduced, so the fp32 error alone remains
    assert rel(kv_k[0, kv_len], kn) < 2e-6


def test_transformer_layer_composition(O):
    """The layer equals its pieces in the reference's order, bit for bit:
    norm, attention, residual add, norm, experts from zero, residual add."""
    from tests.test_gpu_legacy import expert_operands
    g = dict(GEOM, embed=512)
    rng = np.random.default_rng(44)
    e, H, KV, hd, kv_len, inter = g["embed"], g["n_heads"], g["n_kv_heads"], g["hd"], 3, 256
    w = make_f32(rng, g)
    an = rng.normal(1.0, 0.1, e).astype(np.float32)
    fn = rng.normal(1.0, 0.1, e).astype(np.float32)
    c, s = rope_tables(g["kv_max"], hd // 2)
    kv_k = rng.normal(0, 1, (KV, g["kv_max"], hd)).astype(np.float32)
    kv_v = rng.normal(0, 1, (KV, g["kv_max"], hd)).astype(np.float32)
    kk, vv = kv_k.copy(), kv_v.copy()
    fmts = [0, 1, 0]
    ex = [expert_operands(rng, e, inter, f) for f in fmts]
    ew = np.array([0.5, 0.3, 0.2], np.float32)
    x = rng.normal(0, 1, e).astype(np.float32)
    x_layer = x.copy()
    O.transformer_layer(w["wq"], w["wk"], w["wv"], w["wo"], an, w["qn"], w["kn"], fn, kv_k, kv_v, kv_len,
                        g["kv_max"], c, s, [a[0] for a in ex], [a[1] for a in ex], [a[2] for a in ex], fmts, ew,
                        x_layer, e, inter, H, KV, hd, kv_len)
    xr = x.copy()
    nrm = O.rms_norm(xr, an, 1e-6)
    att = O.attention_decode(False, w["wq"], w["wk"], w["wv"], w["wo"], w["qn"], w["kn"], kk, vv, kv_len,
                             g["kv_max"], c, s, nrm, e, H, KV, hd, kv_len)
    xr = (xr + att).astype(np.float32)
    nrm = O.rms_norm(xr, fn, 1e-6)
    mo = np.zeros(e, np.float32)
    for (gt, up, dn), f, wi in zip(ex, fmts, ew):
        mo = O.expert_forward_mixed(gt, up, dn, f, nrm, mo, wi, e, inter)
    xr = (xr + mo).astype(np.float32)
    assert np.array_equal(x_layer.view(np.uint32), xr.view(np.uint32))
    assert np.array_equal(kv_k.view(np.uint32), kk.view(np.uint32))
    assert np.array_equal(kv_v.view(np.uint32), vv.view(np.uint32))


def test_output_head_oracle(O):
    """The output head composes the pinned norm and matvec; its product
    agrees with numpy's W @ x (the reference's own op, in BLAS order) to fp32
    rounding, and its token is numpy's argmax of the same logits, ties to the
    first index."""
    rng = np.random.default_rng(11)
    vocab, embed = 3001, 512
    W = rng.normal(0, 0.02, (vocab, embed)).astype(np.float32)
    nw = rng.normal(1, 0.1, embed).astype(np.float32)
    x = rng.normal(0, 1, embed).astype(np.float32)
    logits, tok = O.output_head(W, nw, x, 1e-6)
    xn = O.rms_norm(x, nw, 1e-6)
    ref = W.astype(np.float64) @ xn.astype(np.float64)
    bound = 4 * embed * np.finfo(np.float32).eps * (np.abs(W).astype(np.float64) @ np.abs(xn).astype(np.float64))
    assert np.all(np.abs(logits - ref) <= bound)
    assert np.all(np.abs(logits - W @ xn) <= bound)
    assert tok == int(np.argmax(logits))
    # a tie: two rows equal to the best one, the first index wins
    W2 = W.copy()
    W2[7] = W2[tok]
    W2[2900] = W2[tok]
    _, tok2 = O.output_head(W2, nw, x, 1e-6)
    assert tok2 == min(7, tok)
