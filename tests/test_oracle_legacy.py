"""Pins the oracle's restatements of the reference's legacy formats (Q4_K,
Q6_K, f16, the 256-element Q8 activations and the expert forward of
csrc/libtinygiant.c) against checks that do not reuse the oracle's code:

- the 6-bit scale/min packing of Q4_K through a packer written from the block
  layout (round trip), and known answers built from the reference test's
  constants d = 0x3400 (0.25) and dmin = 0x2C00 (0.0625)
  (csrc/test_libtinygiant.c:66-67);
- Q6_K dequantization against a numpy restatement in ggml's element order;
- the Q8 activation quantizer against its definition (amax / 127, RNE);
- the dot products against a float64 scalar Q8 reference and a float64
  dequantize-then-dot, with the reference test's own thresholds (test 1a:
  1e-4 relative, test 2: 1e-4 absolute, test 3: 1% relative on 768 x 2048,
  csrc/test_libtinygiant.c:104-240);
- f16 / f32 matrix-vector products, the RMS norm and the expert forward
  against float64 compositions.
"""
import numpy as np
import pytest


def f16(bits):
    return np.array([bits], dtype=np.uint16).view(np.float16).astype(np.float32)[0]


# ------------------------------------------------------------------ Q4_K

def pack_scales(sc, m):
    """12-byte Q4_K scale field from 8 six-bit scales and 8 six-bit mins:
    bytes 0..3 hold sc[0..3] (low 6 bits) and the top 2 bits of sc[4..7];
    bytes 4..7 hold m[0..3] and the top 2 bits of m[4..7]; bytes 8..11 hold
    the low 4 bits of sc[4..7] (low nibble) and of m[4..7] (high nibble)."""
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4)
    return s


def q4k_block(d_bits, dmin_bits, sc, m, nib):
    """nib: 256 values 0..15 in element order (element g*64 + j is the low
    nibble of byte g*32 + j, element g*64 + 32 + j its high nibble)."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([d_bits], np.uint16).view(np.uint8)
    b[2:4] = np.array([dmin_bits], np.uint16).view(np.uint8)
    b[4:16] = pack_scales(sc, m)
    nib = np.asarray(nib, np.uint8).reshape(4, 2, 32)
    b[16:] = (nib[:, 0, :] | (nib[:, 1, :] << 4)).ravel()
    return b


def q4k_dequant_np(d, dmin, sc, m, nib):
    """float64 values d * sc_g * q - dmin * m_g, sub-block g = element // 32."""
    nib = np.asarray(nib, np.float64)
    g = np.arange(256) // 32
    return d * np.asarray(sc, np.float64)[g] * nib - dmin * np.asarray(m, np.float64)[g]


def test_q4k_scale_min_roundtrip(O):
    rng = np.random.default_rng(1)
    for _ in range(200):
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        s = pack_scales(sc, m)
        for j in range(8):
            assert O.scale_min_k4(j, s) == (sc[j], m[j]), j


def test_q4k_dequant_known_answers(O):
    """d = 0.25, dmin = 0.0625 (the reference test's block constants): every
    value d*sc*q - dmin*m is exact in float32, so the match is bit for bit."""
    rng = np.random.default_rng(2)
    for _ in range(50):
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        nib = rng.integers(0, 16, 256)
        blk = q4k_block(0x3400, 0x2C00, sc, m, nib)
        want = q4k_dequant_np(0.25, 0.0625, sc, m, nib).astype(np.float32)
        got = O.dequant_q4k_block(blk)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def random_q4k_rows(rng, rows, bpr):
    out = np.zeros((rows, bpr * 144), np.uint8)
    for r in range(rows):
        for b in range(bpr):
            out[r, b * 144:(b + 1) * 144] = q4k_block(
                int(rng.choice([0x3400, 0x2C00, 0x2000, 0x3000])), int(rng.choice([0x2C00, 0x2400, 0x2000])),
                rng.integers(0, 64, 8), rng.integers(0, 64, 8), rng.integers(0, 16, 256))
    return out


def q8k_np(x):
    """The Q8 activation blocks of 256: scale = amax/127 (0 -> all zero),
    q = rne(x * 127/amax), returned as (q int, scale float32)."""
    x = np.asarray(x, np.float32).reshape(-1, 256)
    amax = np.max(np.abs(x), axis=1)
    inv = np.where(amax > 0, np.float32(127.0) / np.where(amax > 0, amax, 1), 0).astype(np.float32)
    q = np.rint(x * inv[:, None]).astype(np.int32)
    return q, (amax / np.float32(127.0)).astype(np.float32)


def test_q8k_quantizer_definition(O):
    rng = np.random.default_rng(3)
    for scale in (1e-3, 0.05, 3.0):
        x = (rng.standard_normal(2048) * scale).astype(np.float32)
        x[:256] = 0.0  # an all-zero block
        xq = O.quantize_q8k(x)
        q, s = q8k_np(x)
        assert np.array_equal(xq["qs"].astype(np.int32), q)
        assert np.array_equal(xq["scale"].view(np.uint32), s.view(np.uint32))
        assert np.array_equal(xq["sum"], q.sum(axis=1))


def test_dot_q4k_q8_vs_scalar_q8_reference(O):
    """Reference test 1a: the Q8 dot against a scalar Q8 reference on the same
    Q8 input (here float64 over the integer dot products), rel < 1e-4."""
    rng = np.random.default_rng(4)
    worst = 0.0
    for trial in range(100):
        row = random_q4k_rows(rng, 1, 1)[0]
        x = ((rng.random(256) - 0.5) * 0.1).astype(np.float32)
        xq = O.quantize_q8k(x)
        got = O.dot_q4k_q8(row, xq)
        q, s = q8k_np(x)
        d, dmin = f16(int(row[0]) | (int(row[1]) << 8)), f16(int(row[2]) | (int(row[3]) << 8))
        sc = [O.scale_min_k4(j, row[4:16])[0] for j in range(8)]
        m = [O.scale_min_k4(j, row[4:16])[1] for j in range(8)]
        nib = np.stack([row[16:].reshape(4, 32) & 0xF, row[16:].reshape(4, 32) >> 4], 1).reshape(256)
        g = np.arange(256) // 32
        want = float(s[0]) * sum(float(d) * sc[k] * float(np.dot(nib[g == k], q[0][g == k]))
                                 - float(dmin) * m[k] * float(q[0][g == k].sum()) for k in range(8))
        denom = abs(want) if abs(want) > 1e-3 else 1.0
        worst = max(worst, abs(got - want) / denom)
    assert worst < 1e-4, worst


def test_scalar_q4k_dot_vs_dequant(O):
    """Reference test 2: the dequantize-style scalar dot against dequantize
    then a float64 dot, absolute error < 1e-4."""
    rng = np.random.default_rng(5)
    worst = 0.0
    for trial in range(100):
        W = random_q4k_rows(rng, 1, 1)
        x = ((rng.random(256) - 0.5) * 0.1).astype(np.float32)
        got = O.matmul_q4k_scalar(W, x, 1, 256)[0]
        want = float(np.dot(O.dequant_q4k_block(W[0]).astype(np.float64), x.astype(np.float64)))
        worst = max(worst, abs(got - want))
    assert worst < 1e-4, worst


def test_matmul_q4k_768x2048(O):
    """Reference test 3: 768 x 2048, the matrix product against a float64
    scalar Q8 reference on the same Q8 input, relative error < 1%; and the
    Q8 path against dequantize-then-dot within the Q8 error (normwise)."""
    rng = np.random.default_rng(6)
    rows, cols = 768, 2048
    bpr = cols // 256
    W = random_q4k_rows(rng, rows, bpr)
    x = ((rng.random(cols) - 0.5) * 0.02).astype(np.float32)
    got = O.matmul_q4k(W, x, rows, cols)
    q, s = q8k_np(x)
    blocks = W.reshape(rows, bpr, 144)
    d = blocks[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    dmin = blocks[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    qs = blocks[:, :, 16:].reshape(rows, bpr, 4, 32)
    nib = np.stack([qs & 0xF, qs >> 4], 3).reshape(rows, bpr, 8, 32).astype(np.int64)
    sc = np.zeros((rows, bpr, 8)); m = np.zeros((rows, bpr, 8))
    for r in range(rows):
        for b in range(bpr):
            for j in range(8):
                sc[r, b, j], m[r, b, j] = O.scale_min_k4(j, blocks[r, b, 4:16])
    qx = q.reshape(bpr, 8, 32).astype(np.int64)
    idot = np.einsum("rbgj,bgj->rbg", nib, qx)
    isum = qx.sum(axis=2)
    want = np.einsum("b,rbg->r", s.astype(np.float64),
                     d[:, :, None] * sc * idot - dmin[:, :, None] * m * isum[None, :, :])
    denom = np.where(np.abs(want) > 1e-3, np.abs(want), 1.0)
    assert float(np.max(np.abs(got - want) / denom)) < 0.01
    ref = O.matmul_q4k_scalar(W, x, rows, cols)
    assert float(np.max(np.abs(got - ref))) / float(np.max(np.abs(ref))) < 0.02


# ------------------------------------------------------------------ Q6_K

def q6k_dequant_np(block):
    """ggml's Q6_K element order: in each half of 128, element l (+32, +64,
    +96) takes the low (high) nibble of ql[l] / ql[l + 32] and two bits of
    qh[l]; scale sc[l // 16 + 2i]; value d * sc * (q - 32)."""
    ql, qh = block[:128].astype(np.int32), block[128:192].astype(np.int32)
    sc = block[192:208].view(np.int8).astype(np.float32)
    d = f16(int(block[208]) | (int(block[209]) << 8))
    y = np.zeros(256, np.float32)
    for half in range(2):
        for l in range(32):
            a, b2, h = ql[half * 64 + l], ql[half * 64 + l + 32], qh[half * 32 + l]
            q = [(a & 0xF) | (((h >> 0) & 3) << 4), (b2 & 0xF) | (((h >> 2) & 3) << 4),
                 (a >> 4) | (((h >> 4) & 3) << 4), (b2 >> 4) | (((h >> 6) & 3) << 4)]
            for i in range(4):
                y[half * 128 + l + 32 * i] = d * sc[half * 8 + l // 16 + 2 * i] * np.float32(q[i] - 32)
    return y


def random_q6k_rows(rng, rows, bpr):
    out = rng.integers(0, 256, (rows, bpr * 210)).astype(np.uint8)
    for r in range(rows):
        for b in range(bpr):
            blk = out[r, b * 210:(b + 1) * 210]
            blk[192:208] = rng.integers(-64, 64, 16).astype(np.int8).view(np.uint8)
            blk[208:210] = np.array([int(rng.choice([0x2000, 0x2400, 0x1C00]))], np.uint16).view(np.uint8)
    return out


def test_q6k_dequant_vs_ggml_order(O):
    rng = np.random.default_rng(7)
    for _ in range(50):
        blk = random_q6k_rows(rng, 1, 1)[0]
        got = O.dequant_q6k_block(blk)
        want = q6k_dequant_np(blk)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q6k_dequant_known_answer(O):
    """d = 0.25, every scale 2, ql / qh chosen so element e holds q = e % 64:
    value 0.5 * (e % 64 - 32), exact."""
    blk = np.zeros(210, np.uint8)
    q = np.arange(256) % 64
    for half in range(2):
        for l in range(32):
            e = [half * 128 + l + 32 * i for i in range(4)]
            blk[half * 64 + l] = (q[e[0]] & 0xF) | ((q[e[2]] & 0xF) << 4)
            blk[half * 64 + l + 32] = (q[e[1]] & 0xF) | ((q[e[3]] & 0xF) << 4)
            blk[128 + half * 32 + l] = (q[e[0]] >> 4) | ((q[e[1]] >> 4) << 2) | ((q[e[2]] >> 4) << 4) | ((q[e[3]] >> 4) << 6)
    blk[192:208] = 2
    blk[208:210] = np.array([0x3400], np.uint16).view(np.uint8)
    want = (0.5 * (q - 32)).astype(np.float32)
    assert np.array_equal(O.dequant_q6k_block(blk), want)


def test_dot_q6k_q8_vs_scalar_q8_reference(O):
    rng = np.random.default_rng(8)
    worst = 0.0
    for trial in range(50):
        blk = random_q6k_rows(rng, 1, 2)[0]
        x = ((rng.random(512) - 0.5) * 0.1).astype(np.float32)
        xq = O.quantize_q8k(x)
        got = O.dot_q6k_q8(blk, xq)
        q, s = q8k_np(x)
        want = 0.0
        for b in range(2):
            deq = q6k_dequant_np(blk[b * 210:(b + 1) * 210]).astype(np.float64)  # d * sc * (q - 32)
            want += float(s[b]) * float(np.dot(deq, q[b]))
        denom = abs(want) if abs(want) > 1e-3 else 1.0
        worst = max(worst, abs(got - want) / denom)
    assert worst < 1e-4, worst


def test_matmul_q6k_vs_dequant(O):
    rng = np.random.default_rng(9)
    rows, cols = 256, 768
    W = random_q6k_rows(rng, rows, cols // 256)
    x = ((rng.random(cols) - 0.5) * 0.05).astype(np.float32)
    got = O.matmul_q6k(W, x, rows, cols)
    deq = np.stack([np.concatenate([q6k_dequant_np(W[r, b * 210:(b + 1) * 210]) for b in range(cols // 256)])
                    for r in range(rows)]).astype(np.float64)
    ref = deq @ x.astype(np.float64)
    assert float(np.max(np.abs(got - ref))) / float(np.max(np.abs(ref))) < 0.01


# ------------------------------------------------------- f16 / f32 / norm

def test_matvec_f16_f32(O):
    rng = np.random.default_rng(10)
    A = (rng.standard_normal((96, 512)) * 0.05).astype(np.float32)
    x = rng.standard_normal(512).astype(np.float32)
    ref16 = A.astype(np.float16).astype(np.float64) @ x.astype(np.float64)
    got16 = O.matvec_f16(A.astype(np.float16), x)
    assert float(np.max(np.abs(got16 - ref16))) / float(np.max(np.abs(ref16))) < 1e-5
    ref32 = A.astype(np.float64) @ x.astype(np.float64)
    got32 = O.matvec_f32(A, x)
    assert float(np.max(np.abs(got32 - ref32))) / float(np.max(np.abs(ref32))) < 1e-5


def test_rms_norm(O):
    rng = np.random.default_rng(11)
    x = rng.standard_normal(2048).astype(np.float32) * 3
    w = rng.standard_normal(2048).astype(np.float32)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 * x64) + 1e-6) * w.astype(np.float64)
    got = O.rms_norm(x, w, 1e-6)
    assert float(np.max(np.abs(got - ref))) / float(np.max(np.abs(ref))) < 1e-5


# ------------------------------------------------------------ expert forward

@pytest.mark.parametrize("down_format", [0, 1, 2])
def test_expert_forward_mixed_vs_float64(O, down_format):
    """gate / up Q4_K, down Q4_K (0), f16 (1) or Q6_K (2): out += w * down(SiLU(gate x) * up x),
    against the float64 composition of the dequantized weights, within the
    error of the two Q8 activation quantizations (a few percent)."""
    rng = np.random.default_rng(20 + down_format)
    embed, inter, weight = 512, 256, 0.375
    gate = random_q4k_rows(rng, inter, embed // 256)
    up = random_q4k_rows(rng, inter, embed // 256)
    deq = lambda W, n: np.stack([np.concatenate([O.dequant_q4k_block(W[r, b * 144:(b + 1) * 144])
                                                 for b in range(n // 256)]) for r in range(W.shape[0])])
    Wg, Wu = deq(gate, embed).astype(np.float64), deq(up, embed).astype(np.float64)
    if down_format == 0:
        down = random_q4k_rows(rng, embed, inter // 256)
        Wd = deq(down, inter).astype(np.float64)
    elif down_format == 1:
        Wd16 = (rng.standard_normal((embed, inter)) * 0.05).astype(np.float16)
        down = Wd16
        Wd = Wd16.astype(np.float64)
    else:
        down = random_q6k_rows(rng, embed, inter // 256)
        Wd = np.stack([np.concatenate([q6k_dequant_np(down[r, b * 210:(b + 1) * 210]) for b in range(inter // 256)])
                       for r in range(embed)]).astype(np.float64)
    x = ((rng.random(embed) - 0.5) * 0.1).astype(np.float32)
    out0 = rng.standard_normal(embed).astype(np.float32)
    out = O.expert_forward_mixed(gate, up, np.ascontiguousarray(down), down_format, x, out0.copy(), weight,
                                 embed, inter)
    g = Wg @ x.astype(np.float64)
    u = Wu @ x.astype(np.float64)
    h = g / (1.0 + np.exp(-g)) * u
    want = out0.astype(np.float64) + weight * (Wd @ h)
    delta_got = out.astype(np.float64) - out0
    delta_want = want - out0
    err = float(np.max(np.abs(delta_got - delta_want))) / float(np.max(np.abs(delta_want)))
    assert err < 0.05, err
