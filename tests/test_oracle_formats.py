"""Pins the oracle's number formats (oracle/tg_oracle.c) without the GPU.

Each check is chosen so that a plausible slip in the oracle fails it: a
wrong nibble order, a dropped -8 offset, a wrong rounding mode, a swapped
scale.  The checks are closed forms (dequantized float64 products equal the
integer block sums times the scales), exhaustive comparisons with numpy's
IEEE conversions, special cases (zero blocks, clamps, exact half-way
values), and the f16 constants the reference's own tests use
(csrc/test_libtinygiant.c:66-67, tools/nws_fused_bench.c:80).
"""
import numpy as np
import pytest


# ---------------------------------------------------------------- halves

def test_f16_to_f32_exhaustive(O):
    """All 65,536 codes against numpy's float16 -> float32 (libtinygiant.c:24-33)."""
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.f16_to_f32_n(codes)
    ref = codes.view(np.float16).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("code,value", [(0x3400, 0.25), (0x2C00, 0.0625), (0x2000, 0.0078125),
                                        (0x3C00, 1.0), (0xC000, -2.0), (0x0001, 2.0 ** -24),
                                        (0x7BFF, 65504.0)])
def test_f16_reference_constants(O, code, value):
    """Scale constants of csrc/test_libtinygiant.c:66-67 and tools/nws_fused_bench.c:80."""
    assert O.f16_to_f32(code) == value


def test_f32_to_f16_matches_numpy(O):
    """Round to nearest even, subnormal halves, overflow to inf (numpy's cast)."""
    lib = O.lib()
    rng = np.random.default_rng(0)
    vals = [0.0, -0.0, 1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25,
            2.0 ** -25 * 1.0000001, 2.0 ** -26, 6.1e-5, 6.097e-5, 1e-8, np.inf, -np.inf]
    # exact half-way points between adjacent halves (ties go to even)
    h = np.arange(0x0400, 0x7BFF, 997, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    vals += list(((lo + hi) / 2).astype(np.float32))
    vals += list(rng.standard_normal(20000).astype(np.float32) * np.float32(0.02))
    vals += list((rng.standard_normal(5000) * 1e-5).astype(np.float32))
    vals += list((rng.standard_normal(5000) * 3e4).astype(np.float32))
    x = np.array(vals, dtype=np.float32)
    got = np.array([lib.tgo_f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------- Q4_0

def unpack_q4_0(q: np.ndarray):
    """(d float32 [nb], q 0..15 int [nb, 32]) of relayout Q4_0 bytes."""
    blk = q.reshape(-1, 18)
    d = blk[:, :2].copy().view(np.float16).astype(np.float32).ravel()
    qs = blk[:, 2:].astype(np.int64)
    return d, np.concatenate([qs & 15, qs >> 4], axis=1)


def unpack_q8_0(q: np.ndarray):
    blk = q.reshape(-1, 34)
    d = blk[:, :2].copy().view(np.float16).astype(np.float32).ravel()
    return d, blk[:, 2:].view(np.int8).astype(np.int64)


def test_q4_0_zero_block(O):
    out = O.quantize_q4_0(np.zeros(32, np.float32))
    # d = 0 / -8 = -0.0: half code 0x8000
    assert out[0] == 0 and out[1] == 0x80
    assert np.all(out[2:] == 0x88)  # q = 8 in both nibbles, value 0


def test_q4_0_clamp_and_sign(O):
    """d = m / -8 for the signed max m: m itself maps to q = 0, -m to the
    clamped q = 15 (16 before the clamp)."""
    x = np.zeros(32, np.float32)
    x[5] = -4.0
    x[20] = 4.0  # same magnitude, later: the first one (negative) is m
    q = O.quantize_q4_0(x)
    d, qs = unpack_q4_0(q)
    assert d[0] == np.float32(0.5)
    assert qs[0, 5] == 0 and qs[0, 20] == 15
    assert np.all(qs[0, [i for i in range(32) if i not in (5, 20)]] == 8)
    x2 = -x
    d2, qs2 = unpack_q4_0(O.quantize_q4_0(x2))
    assert d2[0] == np.float32(-0.5) and qs2[0, 5] == 0 and qs2[0, 20] == 15


def test_q4_0_element_order(O):
    """Element j < 16 in the low nibble of byte j, j + 16 in the high nibble."""
    x = np.zeros(32, np.float32)
    x[0] = -8.0   # m: d = 1, q = 0
    x[3] = 3.0    # q = 11 in the low nibble of byte 3
    x[19] = -5.0  # q = 3 in the high nibble of byte 3
    q = O.quantize_q4_0(x)
    assert q[2 + 3] == (11 | (3 << 4))
    assert q[2 + 0] == (0 | (8 << 4))


def test_q4_0_matches_numpy_rule_and_error_bound(O):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(32 * 4096) * 0.02).astype(np.float32)
    q = O.quantize_q4_0(x)
    d, qs = unpack_q4_0(q)
    xb = x.reshape(-1, 32)
    # numpy statement of the rule, vectorised
    am = np.argmax(np.abs(xb), axis=1)
    m = xb[np.arange(xb.shape[0]), am]
    dd = (m / np.float32(-8.0)).astype(np.float32)
    idd = np.where(dd != 0, np.float32(1.0) / dd, np.float32(0.0)).astype(np.float32)
    qr = np.minimum(15, np.trunc((xb * idd[:, None]).astype(np.float32) + np.float32(8.5))).astype(np.int64)
    assert np.array_equal(d, dd.astype(np.float16).astype(np.float32))
    assert np.array_equal(qs, qr)
    # dequantization error: at most half a step (a full step at the clamp),
    # plus the half-precision rounding of d times |q - 8| <= 8
    deq = O.dequantize_q4_0(q, x.size).reshape(-1, 32)
    assert np.array_equal(deq, (d[:, None] * (qs - 8)).astype(np.float32))
    err = np.abs(deq.astype(np.float64) - xb)
    bound = np.abs(d)[:, None] * 1.0 + 8 * np.abs(d.astype(np.float64) - dd)[:, None] + 1e-12
    assert np.all(err <= bound)


# ---------------------------------------------------------------- Q8_0

def test_q8_0_zero_block(O):
    out = O.quantize_q8_0(np.zeros(64, np.float32))
    assert np.all(out == 0)


def test_q8_0_amax_maps_to_127(O):
    rng = np.random.default_rng(2)
    x = rng.standard_normal(32 * 100).astype(np.float32)
    d, qs = unpack_q8_0(O.quantize_q8_0(x))
    xb = x.reshape(-1, 32)
    am = np.argmax(np.abs(xb), axis=1)
    assert np.array_equal(qs[np.arange(100), am], np.where(xb[np.arange(100), am] > 0, 127, -127))
    assert np.all(np.abs(qs) <= 127)


def test_q8_0_round_half_even(O):
    """amax = 127 makes the multiplier exactly 1: x = k + 1/2 must round to
    the even neighbour (vcvtnq_s32_f32, libtinygiant.c:81)."""
    halves = np.array([0.5, 1.5, 2.5, 3.5, -0.5, -1.5, -2.5, -3.5, 10.5, 11.5, -10.5, 126.5], np.float32)
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:1 + halves.size] = halves
    d, qs = unpack_q8_0(O.quantize_q8_0(x))
    assert d[0] == np.float32(1.0)
    assert qs[0, 0] == 127
    assert qs[0, 1:1 + halves.size].tolist() == [0, 2, 2, 4, 0, -2, -2, -4, 10, 12, -10, 126]


def test_q8_0_error_bound(O):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(32 * 2000).astype(np.float32)
    q = O.quantize_q8_0(x)
    d, qs = unpack_q8_0(q)
    deq = O.dequantize_q8_0(q, x.size).reshape(-1, 32)
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    dexact = amax.astype(np.float64) / 127
    # half a step of the exact scale, plus the half rounding of d times |q|
    bound = dexact[:, None] * 0.5 * (1 + 1e-6) + np.abs(d - dexact)[:, None] * 127 + 1e-12
    assert np.all(np.abs(deq.astype(np.float64) - xb) <= bound)


# ---------------------------------------------------------------- block dot

def test_block_dot_bruteforce(O):
    rng = np.random.default_rng(4)
    W = O.quantize_q4_0((rng.standard_normal(32 * 300) * 0.02).astype(np.float32))
    X = O.quantize_q8_0(rng.standard_normal(32 * 300).astype(np.float32))
    _, qw = unpack_q4_0(W)
    _, qx = unpack_q8_0(X)
    lib = O.lib()
    for b in range(300):
        got = lib.tgo_block_dot_q40_q80(W[b * 18:].ctypes.data, X[b * 34:].ctypes.data)
        assert got == int(np.sum((qw[b] - 8) * qx[b]))
        # sum (q - 8) x = sum q x - 8 sum x
        assert got == int(np.sum(qw[b] * qx[b]) - 8 * np.sum(qx[b]))


def test_block_dot_extremes(O):
    """|S| reaches 32 * 8 * 128 = 32768 only at q_w = 0, q_x = -128."""
    w = np.zeros(18, np.uint8)       # d = 0, all nibbles 0 -> (q - 8) = -8
    x = np.zeros(34, np.uint8)
    x[2:] = np.uint8(0x80)           # -128
    assert O.lib().tgo_block_dot_q40_q80(w.ctypes.data, x.ctypes.data) == 32768
    w[2:] = 0xFF                     # q = 15 -> 7
    x[2:] = np.uint8(127)
    assert O.lib().tgo_block_dot_q40_q80(w.ctypes.data, x.ctypes.data) == 7 * 127 * 32


def test_block_sums_layout(O):
    rng = np.random.default_rng(5)
    rows, cols = 7, 96
    W = O.quantize_q4_0((rng.standard_normal(rows * cols) * 0.02).astype(np.float32))
    X = O.quantize_q8_0(rng.standard_normal(cols).astype(np.float32))
    S = O.block_sums(W, rows, cols, X)
    _, qw = unpack_q4_0(W)
    _, qx = unpack_q8_0(X)
    ref = np.einsum("rbi,bi->rb", (qw - 8).reshape(rows, cols // 32, 32), qx)
    assert np.array_equal(S, ref)


# ---------------------------------------------------------------- row dot

@pytest.mark.parametrize("rows,cols", [(3, 32), (64, 2048), (128, 768)])
def test_row_dot_against_float64_dequantized_product(O, rows, cols):
    """Sum_i dequant(w)_i dequant(x)_i equals sum_b dw_b dx_b S_b exactly in
    real arithmetic, so the float64 dequantized product is the exact value
    the oracle rounds; its fp32 chain of nb fmas stays within (nb + 1) u of
    sum |terms| (u = 2^-24)."""
    rng = np.random.default_rng(rows + cols)
    W = O.quantize_q4_0((rng.standard_normal(rows * cols) * 0.02).astype(np.float32))
    X = O.quantize_q8_0(rng.standard_normal(cols).astype(np.float32))
    got = O.matvec_q40(W, rows, cols, X).astype(np.float64)
    wd = O.dequantize_q4_0(W, rows * cols).astype(np.float64).reshape(rows, cols)
    xd = O.dequantize_q8_0(X, cols).astype(np.float64)
    exact = wd @ xd
    mag = np.abs(wd) @ np.abs(xd)
    nb = cols // 32
    assert np.all(np.abs(got - exact) <= (nb + 1) * 2.0 ** -24 * mag + 1e-30)
    # and the row dot is the per-block chain, not a transposed product
    assert not np.allclose(got, wd.T[:rows, :] @ xd if rows == cols else -exact)


def test_row_dot_chain_order(O):
    """The blocks are accumulated sequentially b = 0..nb-1 with one fma each:
    with terms 1, 2^-25, 2^-25 (in that order) the chain keeps 1.0 (each
    addition of 2^-25 ties to even), while summing the small terms first
    would give 1 + 2^-24."""
    # block b: S_b * dw_b * dx_b = target_b, built from w and x bytes
    def blk_w(d):
        w = np.zeros(18, np.uint8)
        w[:2] = np.array([d], np.float16).view(np.uint8)
        w[2:] = 0x88
        w[2] = 0x89  # element 0: q = 9 -> +1
        return w
    def blk_x(d):
        x = np.zeros(34, np.uint8)
        x[:2] = np.array([d], np.float16).view(np.uint8)
        x[2] = 1
        return x
    W = np.concatenate([blk_w(1.0), blk_w(2.0 ** -13), blk_w(2.0 ** -13)])
    X = np.concatenate([blk_x(1.0), blk_x(2.0 ** -12), blk_x(2.0 ** -12)])
    assert O.row_dot(W, X, 3) == np.float32(1.0)
    W2 = np.concatenate([blk_w(2.0 ** -13), blk_w(2.0 ** -13), blk_w(1.0)])
    X2 = np.concatenate([blk_x(2.0 ** -12), blk_x(2.0 ** -12), blk_x(1.0)])
    assert O.row_dot(W2, X2, 3) == np.float32(1.0 + 2.0 ** -24)


# ---------------------------------------------------------------- planar form

@pytest.mark.parametrize("rows,nb", [(1, 1), (5, 3), (64, 24)])
def test_planar_roundtrip(O, rows, nb):
    rng = np.random.default_rng(rows * nb)
    aos = rng.integers(0, 256, rows * nb * 18, dtype=np.uint8)
    pl = O.to_planar(aos, rows, nb)
    blk = aos.reshape(-1, 18)
    n = rows * nb
    assert np.array_equal(pl[:16 * n].reshape(n, 16), blk[:, 2:])
    assert np.array_equal(pl[16 * n:].reshape(n, 2), blk[:, :2])
    assert np.array_equal(O.from_planar(pl, rows, nb), aos)
