"""GPU parity of the reference's legacy entry points (Q4_K / Q6_K / f16 /
f32 products, RMS norm, expert forward) against the CPU oracle.

The entry points are called exactly as the reference's ctypes surface calls
them (tinygiant/_lib.py:39-74): host numpy buffers, synchronous.  Every
kernel performs the reference's arithmetic in its own order with
contraction off, so each fp32 result must equal the oracle's bit for bit;
the reference's own threshold for the stack (max relative error 1e-5) is
asserted as well, so a failure reports both.  Inputs are seeded: Q4_K blocks
from a packer written from the block layout (finite fp16 d / dmin, 6-bit
scales and mins, random nibbles), Q6_K blocks as random bytes with a finite
fp16 d, f16 matrices from N(0, 0.02).
"""
import ctypes

import numpy as np
import pytest

from tests.conftest import gpu_note
from tests.test_oracle_legacy import pack_scales

pytestmark = pytest.mark.gpu

REL_TOL = 1e-5


def ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


def f16_bits(v):
    return np.asarray(v, np.float32).astype(np.float16).view(np.uint16)


def q4k_matrix(rng, nrows, bpr):
    """nrows x bpr Q4_K blocks, row-major (144 bytes each)."""
    n = nrows * bpr
    blk = np.zeros((n, 144), np.uint8)
    d = f16_bits(rng.uniform(0.0005, 0.004, n))
    dmin = f16_bits(rng.uniform(0.0, 0.004, n))
    blk[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    blk[:, 2:4] = dmin.view(np.uint8).reshape(n, 2)
    for i in range(n):
        blk[i, 4:16] = pack_scales(rng.integers(0, 64, 8), rng.integers(0, 64, 8))
    blk[:, 16:] = rng.integers(0, 256, (n, 128), dtype=np.uint8)
    return blk.reshape(-1)


def q6k_matrix(rng, nrows, bpr):
    n = nrows * bpr
    blk = rng.integers(0, 256, (n, 210), dtype=np.uint8)
    blk[:, 208:210] = f16_bits(rng.uniform(0.0002, 0.002, n)).view(np.uint8).reshape(n, 2)
    return blk.reshape(-1)


def f16_matrix(rng, nrows, ncols):
    return f16_bits(rng.normal(0.0, 0.02, nrows * ncols))


def assert_exact(got, ref, what):
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    den = max(float(np.max(np.abs(ref))), 1e-30)
    rel = float(np.max(np.abs(got.astype(np.float64) - ref))) / den
    assert rel <= REL_TOL, f"{what}: normwise relative error {rel:.3e}"
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"{what}: not bit-identical (rel {rel:.2e})"


@pytest.fixture(scope="module")
def L(tglib):
    return tglib


@pytest.mark.parametrize("nrows,ncols", [(1, 256), (64, 512), (768, 2048), (2048, 768), (37, 300), (5, 100)])
def test_matmul_q4k(O, L, nrows, ncols):
    gpu_note(f"tg_matmul_q4k {nrows}x{ncols}")
    rng = np.random.default_rng(nrows * 7 + ncols)
    bpr = ncols // 256
    W = q4k_matrix(rng, nrows, bpr)
    x = rng.normal(0.0, 1.0, ncols).astype(np.float32)
    out = np.full(nrows, -1.0, np.float32)
    L.tg_matmul_q4k(ptr(W), ptr(x), ptr(out), nrows, ncols)
    assert_exact(out, O.matmul_q4k(W, x, nrows, ncols), f"q4k {nrows}x{ncols}")


@pytest.mark.parametrize("nrows,ncols", [(1, 256), (2048, 768), (33, 1024)])
def test_matmul_q4k_scalar(O, L, nrows, ncols):
    gpu_note(f"tg_matmul_q4k_scalar {nrows}x{ncols}")
    rng = np.random.default_rng(nrows + 3 * ncols)
    bpr = ncols // 256
    W = q4k_matrix(rng, nrows, bpr)
    x = rng.normal(0.0, 1.0, ncols).astype(np.float32)
    out = np.zeros(nrows, np.float32)
    L.tg_matmul_q4k_scalar(ptr(W), ptr(x), ptr(out), nrows, ncols)
    assert_exact(out, O.matmul_q4k_scalar(W, x, nrows, ncols), f"q4k scalar {nrows}x{ncols}")


@pytest.mark.parametrize("nrows,ncols", [(1, 256), (2048, 768), (70, 1280)])
def test_matmul_q6k(O, L, nrows, ncols):
    gpu_note(f"tg_matmul_q6k {nrows}x{ncols}")
    rng = np.random.default_rng(5 * nrows + ncols)
    bpr = ncols // 256
    W = q6k_matrix(rng, nrows, bpr)
    x = rng.normal(0.0, 1.0, ncols).astype(np.float32)
    out = np.zeros(nrows, np.float32)
    L.tg_matmul_q6k(ptr(W), ptr(x), ptr(out), nrows, ncols)
    assert_exact(out, O.matmul_q6k(W, x, nrows, ncols), f"q6k {nrows}x{ncols}")


@pytest.mark.parametrize("half", [True, False])
# (33, 8200) and (9, 16391) stage x through LDS in more than one chunk of
# 8192 columns, the last one ragged
@pytest.mark.parametrize("nrows,ncols", [(2048, 768), (3, 7), (129, 777), (16, 8), (33, 8200), (9, 16391)])
def test_matvec_f16_f32(O, L, half, nrows, ncols):
    gpu_note(f"tg_{'f16' if half else 'f32'}_matvec {nrows}x{ncols}")
    rng = np.random.default_rng(nrows + ncols + half)
    x = rng.normal(0.0, 1.0, ncols).astype(np.float32)
    out = np.zeros(nrows, np.float32)
    if half:
        A = f16_matrix(rng, nrows, ncols)
        L.tg_f16_matvec(ptr(A), ptr(x), ptr(out), nrows, ncols)
        ref = O.matvec_f16(A.view(np.float16).reshape(nrows, ncols), x)
    else:
        A = rng.normal(0.0, 0.02, nrows * ncols).astype(np.float32)
        L.tg_f32_matvec(ptr(A), ptr(x), ptr(out), nrows, ncols)
        ref = O.matvec_f32(A.reshape(nrows, ncols), x)
    assert_exact(out, ref, f"matvec half={half} {nrows}x{ncols}")


# 6150 and 8195 stage the row in more than one chunk of 4096 (6150: the
# second chunk ragged), 4099 and 8195 leave a tail of 3
@pytest.mark.parametrize("dim", [2048, 1001, 3, 4099, 6150, 8195])
def test_rms_norm(O, L, dim):
    gpu_note(f"tg_rms_norm {dim}")
    rng = np.random.default_rng(dim)
    x = rng.normal(0.0, 1.0, dim).astype(np.float32)
    w = rng.normal(1.0, 0.1, dim).astype(np.float32)
    out = np.zeros(dim, np.float32)
    L.tg_rms_norm(ptr(x), ptr(w), ptr(out), dim, ctypes.c_float(1e-6))
    assert_exact(out, O.rms_norm(x, w, 1e-6), f"rms_norm {dim}")


def expert_operands(rng, embed, inter, fmt):
    gate = q4k_matrix(rng, inter, embed // 256)
    up = q4k_matrix(rng, inter, embed // 256)
    if fmt == 1:
        down = f16_matrix(rng, embed, inter)
    elif fmt == 2:
        down = q6k_matrix(rng, embed, inter // 256)
    else:
        down = q4k_matrix(rng, embed, inter // 256)
    return gate, up, down


@pytest.mark.parametrize("fmt", [0, 1, 2])
@pytest.mark.parametrize("embed,inter", [(2048, 768), (512, 256)])
def test_expert_forward_mixed(O, L, fmt, embed, inter):
    gpu_note(f"tg_expert_forward_mixed fmt={fmt} {embed}x{inter}")
    rng = np.random.default_rng(fmt * 1000 + embed + inter)
    gate, up, down = expert_operands(rng, embed, inter, fmt)
    x = rng.normal(0.0, 1.0, embed).astype(np.float32)
    out0 = rng.normal(0.0, 0.1, embed).astype(np.float32)  # the output accumulates
    out = out0.copy()
    L.tg_expert_forward_mixed(ptr(gate), ptr(up), ptr(down), fmt, ptr(x), ptr(out), ctypes.c_float(0.13),
                              embed, inter)
    ref = O.expert_forward_mixed(gate, up, down, fmt, x, out0.copy(), 0.13, embed, inter)
    assert_exact(out, ref, f"expert fmt={fmt}")


def test_expert_forward_contiguous(O, L):
    """tg_expert_forward: gate | up | down (Q4_K) in one buffer."""
    gpu_note("tg_expert_forward 2048x768")
    rng = np.random.default_rng(77)
    embed, inter = 2048, 768
    gate, up, down = expert_operands(rng, embed, inter, 0)
    blob = np.concatenate([gate, up, down])
    x = rng.normal(0.0, 1.0, embed).astype(np.float32)
    out0 = rng.normal(0.0, 0.1, embed).astype(np.float32)
    out = out0.copy()
    L.tg_expert_forward(ptr(blob), ptr(x), ptr(out), ctypes.c_float(0.25), embed, inter)
    ref = O.expert_forward_mixed(gate, up, down, 0, x, out0.copy(), 0.25, embed, inter)
    assert_exact(out, ref, "expert contiguous")


@pytest.mark.parametrize("n", [8, 1, 3, 17])
def test_moe_forward(O, L, n):
    """tg_moe_forward: output zeroed, then the weighted experts in order; for
    8 experts the reference's own combine weights {.15, .14, .13, ...}
    (tools/nws_q8dot_bench.c:369).  Up to 16 experts run in three launches
    over all of them, 17 expert by expert."""
    gpu_note(f"tg_moe_forward {n} experts 2048x768")
    rng = np.random.default_rng(91 + n)
    embed, inter = 2048, 768
    experts = [np.concatenate(expert_operands(rng, embed, inter, 0)) for _ in range(n)]
    if n == 8:
        w = np.array([0.15, 0.14, 0.13, 0.13, 0.12, 0.11, 0.11, 0.11], np.float32)
    else:
        w = rng.uniform(0.02, 0.3, n).astype(np.float32)
    x = rng.normal(0.0, 1.0, embed).astype(np.float32)
    out = np.full(embed, 7.0, np.float32)  # overwritten, not accumulated
    ptrs = (ctypes.c_void_p * n)(*[e.ctypes.data for e in experts])
    L.tg_moe_forward(ptrs, ptr(w), n, ptr(x), ptr(out), embed, inter)
    ref = O.moe_forward_q4k(experts, w, x, embed, inter)
    assert_exact(out, ref, "moe_forward")


# ---------------------------------------------------------------- attention

def attn_case(rng, q4, embed, n_heads, n_kv, hd, kv_max):
    from tests.test_oracle_attention import rope_tables
    q_dim, kv_dim = n_heads * hd, n_kv * hd
    if q4:
        wq = q4k_matrix(rng, q_dim, embed // 256)
        wk = q4k_matrix(rng, kv_dim, embed // 256)
        wv = f16_matrix(rng, kv_dim, embed)
        wo = q4k_matrix(rng, embed, q_dim // 256)
    else:
        wq = rng.normal(0, 0.03, q_dim * embed).astype(np.float32)
        wk = rng.normal(0, 0.03, kv_dim * embed).astype(np.float32)
        wv = rng.normal(0, 0.03, kv_dim * embed).astype(np.float32)
        wo = rng.normal(0, 0.03, embed * q_dim).astype(np.float32)
    qn = rng.normal(1.0, 0.1, hd).astype(np.float32)
    kn = rng.normal(1.0, 0.1, hd).astype(np.float32)
    c, s = rope_tables(kv_max, hd // 2)
    kv_k = rng.normal(0, 1, (n_kv, kv_max, hd)).astype(np.float32)
    kv_v = rng.normal(0, 1, (n_kv, kv_max, hd)).astype(np.float32)
    x = rng.normal(0, 1, embed).astype(np.float32)
    return wq, wk, wv, wo, qn, kn, c, s, kv_k, kv_v, x


@pytest.mark.parametrize("q4", [False, True])
@pytest.mark.parametrize("embed,n_heads,n_kv,hd,kv_max,kv_len",
                         [(512, 4, 2, 64, 16, 0), (512, 4, 2, 64, 16, 9), (2048, 32, 4, 128, 300, 257),
                          (256, 2, 1, 130, 8, 7),
                          # 12 query heads per kv head (two head groups), 1031 positions (three chunks)
                          (768, 12, 1, 64, 1100, 1030),
                          # one query head per kv head
                          (512, 4, 4, 128, 40, 33),
                          # hd not a multiple of 4 over two chunks, 3 heads per kv head
                          (256, 6, 2, 130, 600, 520),
                          # the largest head
                          (1024, 2, 1, 512, 20, 17),
                          # 2091 positions: the softmax runs over two chunks
                          (256, 2, 1, 128, 2100, 2090)])
def test_attention_decode(O, L, q4, embed, n_heads, n_kv, hd, kv_max, kv_len):
    if q4 and (n_heads * hd) % 256:
        pytest.skip("Q4_K output projection needs q_dim % 256 == 0")
    gpu_note(f"tg_attention_decode{'_q4' if q4 else ''} E={embed} H={n_heads}/{n_kv} hd={hd} kv_len={kv_len}")
    rng = np.random.default_rng(embed + 7 * kv_len + q4)
    wq, wk, wv, wo, qn, kn, c, s, kv_k, kv_v, x = attn_case(rng, q4, embed, n_heads, n_kv, hd, kv_max)
    gk, gv = kv_k.copy(), kv_v.copy()
    out = np.zeros(embed, np.float32)
    fn = L.tg_attention_decode_q4 if q4 else L.tg_attention_decode
    fn(ptr(wq), ptr(wk), ptr(wv), ptr(wo), ptr(qn), ptr(kn), ptr(gk), ptr(gv), kv_len, kv_max, ptr(c), ptr(s),
       ptr(x), ptr(out), embed, n_heads, n_kv, hd, kv_len)
    rk, rv = kv_k.copy(), kv_v.copy()
    ref = O.attention_decode(q4, wq, wk, wv, wo, qn, kn, rk, rv, kv_len, kv_max, c, s, x, embed, n_heads, n_kv, hd,
                             kv_len)
    assert_exact(out, ref, "attention output")
    assert np.array_equal(gk.view(np.uint32), rk.view(np.uint32)), "key cache"
    assert np.array_equal(gv.view(np.uint32), rv.view(np.uint32)), "value cache"


def test_transformer_layer(O, L):
    """tg_transformer_layer: attention + experts (Q4_K and f16 down) on one
    token, x and the caches updated in place, against the oracle."""
    gpu_note("tg_transformer_layer E=2048 H=32/4 hd=128 kv_len=40, 4 experts")
    rng = np.random.default_rng(123)
    embed, n_heads, n_kv, hd, kv_max, kv_len, inter = 2048, 32, 4, 128, 64, 40, 768
    wq, wk, wv, wo, qn, kn, c, s, kv_k, kv_v, x = attn_case(rng, False, embed, n_heads, n_kv, hd, kv_max)
    an = rng.normal(1.0, 0.1, embed).astype(np.float32)
    fn_ = rng.normal(1.0, 0.1, embed).astype(np.float32)
    fmts = [0, 1, 0, 1]
    ex = [expert_operands(rng, embed, inter, f) for f in fmts]
    ew = np.array([0.4, 0.3, 0.2, 0.1], np.float32)
    gx, gk, gv = x.copy(), kv_k.copy(), kv_v.copy()
    n = len(ex)
    arr = lambda lst: (ctypes.c_void_p * n)(*[a.ctypes.data for a in lst])
    dif = np.array(fmts, np.int32)
    L.tg_transformer_layer(ptr(wq), ptr(wk), ptr(wv), ptr(wo), ptr(an), ptr(qn), ptr(kn), ptr(fn_), ptr(gk), ptr(gv),
                           kv_len, kv_max, ptr(c), ptr(s), arr([e[0] for e in ex]), arr([e[1] for e in ex]),
                           arr([e[2] for e in ex]), ptr(dif), ptr(ew), n, ptr(gx), embed, inter, n_heads, n_kv, hd,
                           kv_len)
    rx, rk, rv = x.copy(), kv_k.copy(), kv_v.copy()
    O.transformer_layer(wq, wk, wv, wo, an, qn, kn, fn_, rk, rv, kv_len, kv_max, c, s, [e[0] for e in ex],
                        [e[1] for e in ex], [e[2] for e in ex], fmts, ew, rx, embed, inter, n_heads, n_kv, hd, kv_len)
    assert_exact(gx, rx, "transformer layer x")
    assert np.array_equal(gk.view(np.uint32), rk.view(np.uint32)), "key cache"
    assert np.array_equal(gv.view(np.uint32), rv.view(np.uint32)), "value cache"


@pytest.mark.parametrize("vocab,embed,case", [(1000, 256, "plain"), (5003, 2048, "tie"), (4097, 1001, "nan"),
                                              (151936, 2048, "plain"), (700, 8300, "plain")])
def test_output_head(O, L, vocab, embed, case):
    """tg_head_forward: logits bit-identical to the oracle's norm + fp32
    matvec, token = numpy's argmax (ties to the first index, NaN largest)."""
    gpu_note(f"tg_head_forward vocab={vocab} embed={embed} {case}")
    rng = np.random.default_rng(vocab + embed)
    W = rng.standard_normal((vocab, embed), dtype=np.float32) * np.float32(0.02)
    nw = rng.normal(1.0, 0.1, embed).astype(np.float32)
    x = rng.normal(0, 1, embed).astype(np.float32)
    if case == "tie":
        best = int(np.argmax(O.output_head(W, nw, x)[0]))
        W[vocab - 1] = W[best]
        W[3] = W[best]
    elif case == "nan":
        W[vocab // 2, 5] = np.nan
        W[vocab - 2, 0] = np.nan
    ref, ref_tok = O.output_head(W, nw, x, 1e-6)
    h = L.tg_head_create(ptr(W), ptr(nw), vocab, embed)
    assert h, L.tg_last_error()
    try:
        out = np.zeros(vocab, np.float32)
        tok = ctypes.c_int32(-1)
        assert L.tg_head_forward(h, ptr(x), 1e-6, ptr(out), ctypes.byref(tok)) == 0, L.tg_last_error()
        if case == "nan":  # NaN rows: same positions; every other logit bit-identical
            nan = np.isnan(ref)
            assert np.array_equal(np.isnan(out), nan)
            assert np.array_equal(out[~nan].view(np.uint32), ref[~nan].view(np.uint32))
        else:
            assert_exact(out, ref, "logits")
        assert tok.value == ref_tok
        tok2 = ctypes.c_int32(-1)  # the token alone, logits not copied back
        assert L.tg_head_forward(h, ptr(x), 1e-6, None, ctypes.byref(tok2)) == 0, L.tg_last_error()
        assert tok2.value == ref_tok
    finally:
        L.tg_head_destroy(h)
    if case == "tie":
        assert ref_tok == 3
    if case == "nan":
        assert ref_tok == vocab // 2
