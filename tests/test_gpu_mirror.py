"""HBM residency of tg_mlock ranges for the reference's legacy entry points.

The reference pins hot experts by calling tg_mlock on the mmap views of
their gate / up / down tensors (tinygiant/cache.py:31-67) and pins the
attention weights the same way (engine.py:134-139).  tg_mlock keeps that
contract and may also copy a range to HBM once; the legacy calls then read
those operands from HBM.  By default only ranges in read-only mappings are
copied (the reference's expert views); writable memory only in
TG_MIRROR_ALL.  Checked here: outputs stay bit-identical to the oracle, the
operands are read from the copies (hit counters, no copy per call), a range
rewritten after the lock (its first bytes, or in bulk inside) is read from
host memory again, writable memory is not copied by default, and copies of
read-only mmap views of a layer file serve tg_moe_forward.
"""
import ctypes
import mmap

import numpy as np
import pytest

from tests.conftest import gpu_note
from tests.test_gpu_legacy import assert_exact, attn_case, expert_operands, ptr

pytestmark = pytest.mark.gpu


def stats(L):
    b, r, h, m = ctypes.c_size_t(), ctypes.c_int(), ctypes.c_uint64(), ctypes.c_uint64()
    L.tg_mirror_stats(ctypes.byref(b), ctypes.byref(r), ctypes.byref(h), ctypes.byref(m))
    return b.value, r.value, h.value, m.value


def lock(L, a):
    L.tg_mlock(ctypes.c_void_p(a.ctypes.data), ctypes.c_size_t(a.nbytes))  # mlock may be refused by RLIMIT_MEMLOCK


MIRROR_OFF, MIRROR_READONLY, MIRROR_ALL = 0, 1, 2


@pytest.fixture
def L(tglib):
    """The library with no copies held, in TG_MIRROR_ALL (the operands below
    are writable numpy arrays); the default mode again afterwards."""
    tglib.tg_mirror_drop(None, 0)
    assert tglib.tg_mirror_mode(MIRROR_ALL) == MIRROR_ALL
    yield tglib
    tglib.tg_mirror_mode(MIRROR_READONLY)
    tglib.tg_mirror_drop(None, 0)
    assert stats(tglib)[:2] == (0, 0)


@pytest.mark.parametrize("fmt", [0, 1, 2])
def test_expert_forward_mixed_from_mirror(O, L, fmt):
    gpu_note(f"tg_mlock + tg_expert_forward_mixed fmt={fmt} 2048x768")
    embed, inter = 2048, 768
    rng = np.random.default_rng(500 + fmt)
    gate, up, down = expert_operands(rng, embed, inter, fmt)
    for a in (gate, up, down):
        lock(L, a)
    b0, r0, h0, m0 = stats(L)
    assert r0 == 3 and b0 == gate.nbytes + up.nbytes + down.nbytes
    for i in range(3):
        x = rng.normal(0.0, 1.0, embed).astype(np.float32)
        out0 = rng.normal(0.0, 0.1, embed).astype(np.float32)
        out = out0.copy()
        L.tg_expert_forward_mixed(ptr(gate), ptr(up), ptr(down), fmt, ptr(x), ptr(out), ctypes.c_float(0.2),
                                  embed, inter)
        assert_exact(out, O.expert_forward_mixed(gate, up, down, fmt, x, out0.copy(), 0.2, embed, inter), "expert")
    _, _, h1, m1 = stats(L)
    assert (h1 - h0, m1 - m0) == (9, 0)  # every weight read from HBM, none copied


def test_rewritten_range_is_copied_again(O, L):
    gpu_note("tg_mlock, range rewritten, tg_expert_forward_mixed")
    embed, inter = 512, 256
    rng = np.random.default_rng(7)
    gate, up, down = expert_operands(rng, embed, inter, 0)
    for a in (gate, up, down):
        lock(L, a)
    gate[0:16] = rng.integers(0, 256, 16, dtype=np.uint8)  # first bytes change after the lock
    _, _, h0, m0 = stats(L)
    x = rng.normal(0.0, 1.0, embed).astype(np.float32)
    out = np.zeros(embed, np.float32)
    L.tg_expert_forward_mixed(ptr(gate), ptr(up), ptr(down), 0, ptr(x), ptr(out), ctypes.c_float(0.5), embed, inter)
    assert_exact(out, O.expert_forward_mixed(gate, up, down, 0, x, np.zeros(embed, np.float32), 0.5, embed, inter),
                 "expert after rewrite")
    _, r1, h1, m1 = stats(L)
    assert (h1 - h0, m1 - m0, r1) == (2, 1, 2)  # the stale copy is dropped


def test_interior_rewrite_is_seen(O, L):
    """A locked buffer reloaded in place (its middle half rewritten): the
    spread samples differ, the copy is dropped, the call reads host memory."""
    gpu_note("tg_mlock, middle of a range rewritten, tg_expert_forward_mixed")
    embed, inter = 512, 256
    rng = np.random.default_rng(8)
    gate, up, down = expert_operands(rng, embed, inter, 0)
    for a in (gate, up, down):
        lock(L, a)
    n = up.nbytes
    up[n // 4: 3 * n // 4] = expert_operands(rng, embed, inter, 0)[1][n // 4: 3 * n // 4]
    _, _, h0, m0 = stats(L)
    x = rng.normal(0.0, 1.0, embed).astype(np.float32)
    out = np.zeros(embed, np.float32)
    L.tg_expert_forward_mixed(ptr(gate), ptr(up), ptr(down), 0, ptr(x), ptr(out), ctypes.c_float(0.5), embed, inter)
    assert_exact(out, O.expert_forward_mixed(gate, up, down, 0, x, np.zeros(embed, np.float32), 0.5, embed, inter),
                 "expert after an interior rewrite")
    _, r1, h1, m1 = stats(L)
    assert (h1 - h0, m1 - m0, r1) == (2, 1, 2)


def test_unsampled_rewrite_keeps_copy_in_mirror_all(O, L):
    """The documented limit of TG_MIRROR_ALL: one byte rewritten away from the
    hashed ends and the sampled words is not seen; the call reads the copy,
    i.e. the bytes as locked."""
    gpu_note("tg_mlock (TG_MIRROR_ALL), one unsampled byte rewritten")
    embed, inter = 512, 256
    rng = np.random.default_rng(9)
    gate, up, down = expert_operands(rng, embed, inter, 0)
    for a in (gate, up, down):
        lock(L, a)
    locked = up.copy()
    n = up.nbytes
    step = (n - 8) // 15
    pos = step // 2 + 100  # between the first and second sampled words, past the hashed head
    assert 64 <= pos and pos + 8 < step
    up[pos] ^= 0x5A
    x = rng.normal(0.0, 1.0, embed).astype(np.float32)
    out = np.zeros(embed, np.float32)
    _, _, h0, m0 = stats(L)
    L.tg_expert_forward_mixed(ptr(gate), ptr(up), ptr(down), 0, ptr(x), ptr(out), ctypes.c_float(0.5), embed, inter)
    assert_exact(out, O.expert_forward_mixed(gate, locked, down, 0, x, np.zeros(embed, np.float32), 0.5, embed,
                                             inter), "expert from the copy")
    _, _, h1, m1 = stats(L)
    assert (h1 - h0, m1 - m0) == (3, 0)


def test_writable_range_not_copied_by_default(O, L):
    """Default mode: tg_mlock of writable memory copies nothing, so every
    call reads host memory as the reference's does."""
    gpu_note("tg_mlock of writable memory in the default mode")
    assert L.tg_mirror_mode(MIRROR_READONLY) == MIRROR_READONLY
    embed, inter = 512, 256
    rng = np.random.default_rng(10)
    gate, up, down = expert_operands(rng, embed, inter, 0)
    for a in (gate, up, down):
        lock(L, a)
    assert stats(L)[:2] == (0, 0)
    up[len(up) // 2] ^= 0x11  # read from host memory: seen
    x = rng.normal(0.0, 1.0, embed).astype(np.float32)
    out = np.zeros(embed, np.float32)
    _, _, h0, m0 = stats(L)
    L.tg_expert_forward_mixed(ptr(gate), ptr(up), ptr(down), 0, ptr(x), ptr(out), ctypes.c_float(0.5), embed, inter)
    assert_exact(out, O.expert_forward_mixed(gate, up, down, 0, x, np.zeros(embed, np.float32), 0.5, embed, inter),
                 "expert from host memory")
    _, _, h1, m1 = stats(L)
    assert (h1 - h0, m1 - m0) == (0, 3)


def _moe_on_views(O, L, mm, parts, gb, eb, rng):
    embed, inter, n = 2048, 768, len(parts)
    views = [[np.frombuffer(mm, np.uint8, count=sz, offset=e * eb + off)
              for off, sz in ((0, gb), (gb, gb), (2 * gb, eb - 2 * gb))] for e in range(n)]
    for v in views:
        for a in v:
            lock(L, a)
    assert stats(L)[:2] == (n * eb, 3 * n)
    w = np.array([0.15, 0.14, 0.13, 0.13, 0.12, 0.11, 0.11, 0.11], np.float32)
    x = rng.normal(0.0, 1.0, embed).astype(np.float32)
    out = np.full(embed, 7.0, np.float32)
    _, _, h0, m0 = stats(L)
    ptrs = (ctypes.c_void_p * n)(*[v[0].ctypes.data for v in views])
    L.tg_moe_forward(ptrs, ptr(w), n, ptr(x), ptr(out), embed, inter)
    experts = [np.concatenate(p) for p in parts]
    assert_exact(out, O.moe_forward_q4k(experts, w, x, embed, inter), "moe_forward from mirrors")
    _, _, h1, m1 = stats(L)
    assert (h1 - h0, m1 - m0) == (3 * n, 0)


def test_moe_forward_on_mmap_views(O, L, tmp_path):
    """Experts in a layer file, mapped read-only and viewed per tensor as the
    reference's ExpertCache does, locked, then tg_moe_forward on them."""
    gpu_note("tg_mlock on mmap views + tg_moe_forward 8 experts 2048x768")
    embed, inter, n = 2048, 768, 8
    rng = np.random.default_rng(31)
    parts = [expert_operands(rng, embed, inter, 0) for _ in range(n)]
    f = tmp_path / "layer_000.q4.bin"
    np.concatenate([np.concatenate(p) for p in parts]).tofile(f)
    gb, eb = parts[0][0].nbytes, sum(a.nbytes for a in parts[0])
    assert L.tg_mirror_mode(MIRROR_READONLY) == MIRROR_READONLY  # the default copies read-only views
    with open(f, "rb") as fd:
        mm = mmap.mmap(fd.fileno(), 0, access=mmap.ACCESS_READ)
        _moe_on_views(O, L, mm, parts, gb, eb, rng)
        L.tg_mirror_drop(None, 0)  # before the mapping goes
        mm.close()


def test_transformer_layer_from_mirror(O, L):
    gpu_note("tg_mlock attention weights + experts, tg_transformer_layer")
    rng = np.random.default_rng(321)
    embed, n_heads, n_kv, hd, kv_max, kv_len, inter = 2048, 32, 4, 128, 64, 40, 768
    wq, wk, wv, wo, qn, kn, c, s, kv_k, kv_v, x = attn_case(rng, False, embed, n_heads, n_kv, hd, kv_max)
    an = rng.normal(1.0, 0.1, embed).astype(np.float32)
    fn_ = rng.normal(1.0, 0.1, embed).astype(np.float32)
    fmts = [0, 1]
    ex = [expert_operands(rng, embed, inter, f) for f in fmts]
    for a in (wq, wk, wv, wo, qn, kn, an, fn_, *[t for e in ex for t in e]):
        lock(L, a)
    ew = np.array([0.6, 0.4], np.float32)
    n = len(ex)
    arr = lambda lst: (ctypes.c_void_p * n)(*[a.ctypes.data for a in lst])
    dif = np.array(fmts, np.int32)
    _, _, h0, m0 = stats(L)
    gx, gk, gv = x.copy(), kv_k.copy(), kv_v.copy()
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
    _, _, h1, m1 = stats(L)
    assert (h1 - h0, m1 - m0) == (8 + 3 * n, 0)
