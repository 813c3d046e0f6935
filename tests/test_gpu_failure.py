"""The failure channel of the one-token launches, forced from the host.

The ROUTED and FUSED launches hand h between their blocks through tagged
words in device memory, and every wait for such a word is bounded.  The
reference's entry points have no error channel (csrc/libtinygiant.c:555,
599, 647 return void); the new entry points report a wait that ran out of
tries: the rows come back NaN, tg_moe_layer_q40 and tg_moe_stack_q40 return
TG_E_HIP, and so does tg_arena_status after a device-pointer call.

tg_debug_fault_inject lowers the poll bound and leaves one h line
unpublished, so every reader of that line gives up while each kernel still
runs to its end (nothing here faults or hangs the GPU).  After the hook is
cleared, the next call on the same arena is bit-exact again."""
import ctypes

import numpy as np
import pytest

from tests.conftest import gpu_note

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TG_E_HIP = -4
SPIN = 64  # tries per poll while the hook is set


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.fixture
def inject(tglib):
    """Sets the hook for the block of the test that asks for it; always
    cleared afterwards."""
    def set_(spin, drop):
        assert tglib.tg_debug_fault_inject(spin, drop) == 0
    yield set_
    tglib.tg_debug_fault_inject(0, -1)


def layer_dev(lib, a, layer, x, T=1, name="tg_moe_layer_q40_dev"):
    out = torch.empty_like(x)
    st = torch.cuda.current_stream().cuda_stream
    rc = getattr(lib, name)(a.handle, layer, x.data_ptr(), out.data_ptr(), T, None, None, ctypes.c_float(1e-6), st)
    assert rc == 0, lib.tg_last_error()
    return out


def host_layer(lib, a, layer, x):
    out = np.empty_like(x)
    idx = np.empty((x.shape[0], a.top_k), np.int32)
    w = np.empty((x.shape[0], a.top_k), np.float32)
    rc = lib.tg_moe_layer_q40(a.handle, layer, x.ctypes.data, out.ctypes.data, x.shape[0], idx.ctypes.data,
                              w.ctypes.data, ctypes.c_float(1e-6))
    return rc, out


def host_stack(lib, a, x, l0, n):
    y = x.copy()
    rc = lib.tg_moe_stack_q40(a.handle, y.ctypes.data, y.shape[0], l0, n, ctypes.c_float(1e-6))
    return rc, y


@pytest.mark.parametrize("H,I,E,k", [(2048, 768, 128, 8), (4096, 1536, 128, 8)])
def test_routed_poll_failure_is_reported_and_recovers(O, tglib, inject, H, I, E, k):
    """30B shape (whole units) and 235B shape (half units) on the routed
    one-token launch."""
    from tinygiant_amd.arena import HBMExpertArena
    a = HBMExpertArena(2, E, H, I, k)
    try:
        a.set_decode_path(4)  # ROUTED: raises where the shape does not take it
        for l in range(2):
            a.synth_layer(l, 4242)
        x = O.synth_normal(4242, O.stream_id(0, 9, 4), 1.0, H).reshape(1, H)
        xd = torch.from_numpy(x).cuda()
        gpu_note(f"fault hook H={H}: clean call")
        ref = layer_dev(tglib, a, 0, xd).cpu().numpy()
        assert tglib.tg_arena_status(a.handle) == 0
        assert np.isfinite(ref).all()
        rc, ref_h = host_layer(tglib, a, 0, x)
        assert rc == 0 and np.array_equal(bits(ref_h), bits(ref))
        rc, ref_s = host_stack(tglib, a, x, 0, 2)
        assert rc == 0 and np.isfinite(ref_s).all()

        gpu_note(f"fault hook H={H}: line 0 withheld, {SPIN} tries per poll, device-pointer call")
        inject(SPIN, 0)
        bad = layer_dev(tglib, a, 0, xd).cpu().numpy()
        assert np.isnan(bad).all(), "every block reads every unit: all rows NaN"
        assert tglib.tg_arena_status(a.handle) == TG_E_HIP
        assert "ran out of tries" in tglib.tg_last_error().decode()
        assert tglib.tg_arena_status(a.handle) == 0, "reported once"

        gpu_note(f"fault hook H={H}: host layer call")
        rc, out = host_layer(tglib, a, 1, x)
        assert rc == TG_E_HIP and np.isnan(out).all()
        gpu_note(f"fault hook H={H}: host stack call")
        rc, y = host_stack(tglib, a, x, 0, 2)
        assert rc == TG_E_HIP and np.isnan(y).all()
        assert tglib.tg_arena_status(a.handle) == 0

        gpu_note(f"fault hook H={H}: no-alloc call")
        bad = layer_dev(tglib, a, 0, xd, name="tg_moe_layer_q40_noalloc_dev").cpu().numpy()
        assert np.isnan(bad).all()
        assert tglib.tg_arena_status(a.handle) == TG_E_HIP
        assert "no-alloc" in tglib.tg_last_error().decode()

        gpu_note(f"fault hook H={H}: cleared, the same calls again")
        tglib.tg_debug_fault_inject(0, -1)
        for rep in range(2):
            got = layer_dev(tglib, a, 0, xd).cpu().numpy()
            assert np.array_equal(bits(got), bits(ref)), f"rep {rep}"
        got = layer_dev(tglib, a, 0, xd, name="tg_moe_layer_q40_noalloc_dev").cpu().numpy()
        assert np.array_equal(bits(got), bits(ref))
        rc, out = host_layer(tglib, a, 0, x)
        assert rc == 0 and np.array_equal(bits(out), bits(ref))
        rc, y = host_stack(tglib, a, x, 0, 2)
        assert rc == 0 and np.array_equal(bits(y), bits(ref_s))
        assert tglib.tg_arena_status(a.handle) == 0
    finally:
        tglib.tg_debug_fault_inject(0, -1)
        a.close()


def test_recovered_call_matches_oracle(O, tglib, inject):
    """After a reported failure the routed call equals the oracle bit for bit
    (the withheld line's old tag never matches a later generation)."""
    from tinygiant_amd.arena import HBMExpertArena
    H, I, E, k = 2048, 768, 128, 8
    lb, r = O.synth_layer(77, 0, H, I, E)
    a = HBMExpertArena(1, E, H, I, k)
    try:
        a.load_layer(0, lb)
        a.load_router(0, r)
        x = O.synth_normal(77, O.stream_id(0, 3, 4), 1.0, H).reshape(1, H)
        xd = torch.from_numpy(x).cuda()
        gpu_note("fault hook then oracle: withheld unit 5")
        inject(SPIN, 5)
        assert np.isnan(layer_dev(tglib, a, 0, xd).cpu().numpy()).all()
        assert tglib.tg_arena_status(a.handle) == TG_E_HIP
        tglib.tg_debug_fault_inject(0, -1)
        ref, _, _, _ = O.moe_layer(lb, r, H, I, E, k, x)
        got = layer_dev(tglib, a, 0, xd).cpu().numpy()
        assert np.array_equal(bits(got), bits(ref))
        assert tglib.tg_arena_status(a.handle) == 0
    finally:
        a.close()


def test_fused_gate_up_down_wait_failure(O, tglib, inject):
    """The batched path's fused gate/up + down launch: the down blocks of a
    work item wait (bounded) until the item's gate/up blocks have stored h.
    With the hook, the gate/up blocks of item 0 (all entries of the lowest
    expert any token selected, at 16 tokens) never count in: exactly the
    tokens that selected that expert come back NaN, every other row is
    bit-exact, the host call returns TG_E_HIP, and the next call on the same
    arena equals the oracle again."""
    import os
    from tinygiant_amd.arena import HBMExpertArena
    H, I, E, k, T = 2048, 768, 128, 8, 16
    lb, r = O.synth_layer(91, 0, H, I, E)
    a = HBMExpertArena(1, E, H, I, k)
    old = os.environ.get("TG_FUSE_GD")
    os.environ["TG_FUSE_GD"] = "1"
    try:
        a.load_layer(0, lb)
        a.load_router(0, r)
        x = O.synth_normal(91, O.stream_id(0, 5, 4), 1.0, T * H).reshape(T, H)
        ref, ridx, _, _ = O.moe_layer(lb, r, H, I, E, k, x)
        gpu_note("fused gate/up + down: clean call")
        rc, out = host_layer(tglib, a, 0, x)
        assert rc == 0 and np.array_equal(bits(out), bits(ref))

        gpu_note("fused gate/up + down: item 0 never counted in, 4096 tries per wait")
        inject(4096, 0)
        rc, bad = host_layer(tglib, a, 0, x)
        assert rc == TG_E_HIP
        assert "ran out of tries" in tglib.tg_last_error().decode()
        hit = (ridx == ridx.min()).any(axis=1)
        nan_rows = np.isnan(bad).any(axis=1)
        assert hit.any() and np.array_equal(nan_rows, hit), (np.nonzero(nan_rows)[0], np.nonzero(hit)[0])
        assert np.isnan(bad[hit]).all()
        assert np.array_equal(bits(bad[~hit]), bits(ref[~hit]))

        gpu_note("fused gate/up + down: hook cleared")
        tglib.tg_debug_fault_inject(0, -1)
        for rep in range(2):
            rc, out = host_layer(tglib, a, 0, x)
            assert rc == 0 and np.array_equal(bits(out), bits(ref)), f"rep {rep}"
        assert tglib.tg_arena_status(a.handle) == 0
    finally:
        tglib.tg_debug_fault_inject(0, -1)
        if old is None:
            os.environ.pop("TG_FUSE_GD", None)
        else:
            os.environ["TG_FUSE_GD"] = old
        a.close()


def test_fused_x16_wait_failure(O, tglib, inject):
    """The fused gate/up + down launch of the 16 x 16 items (about 250
    entries per expert): with the hook, item 0's gate/up blocks never count
    in, so its down blocks' waits run out: some rows come back NaN, the host
    call returns TG_E_HIP, and the next call on the same arena equals the
    oracle again."""
    import os
    from tinygiant_amd.arena import HBMExpertArena
    H, I, E, k, T = 512, 256, 32, 8, 1000
    lb, r = O.synth_layer(97, 0, H, I, E)
    a = HBMExpertArena(1, E, H, I, k)
    old = os.environ.get("TG_FUSE_GD16")
    os.environ["TG_FUSE_GD16"] = "1"
    try:
        a.load_layer(0, lb)
        a.load_router(0, r)
        x = O.synth_normal(97, O.stream_id(0, 7, 4), 1.0, T * H).reshape(T, H)
        ref, _, _, _ = O.moe_layer(lb, r, H, I, E, k, x)
        gpu_note("fused 16 x 16 gate/up + down: clean call")
        rc, out = host_layer(tglib, a, 0, x)
        assert rc == 0 and np.array_equal(bits(out), bits(ref))

        gpu_note("fused 16 x 16 gate/up + down: item 0 never counted in, 4096 tries per wait")
        inject(4096, 0)
        rc, bad = host_layer(tglib, a, 0, x)
        assert rc == TG_E_HIP
        assert "ran out of tries" in tglib.tg_last_error().decode()
        nan_rows = np.isnan(bad).any(axis=1)
        assert 0 < nan_rows.sum() < T
        assert np.array_equal(bits(bad[~nan_rows]), bits(ref[~nan_rows]))

        gpu_note("fused 16 x 16 gate/up + down: hook cleared")
        tglib.tg_debug_fault_inject(0, -1)
        for rep in range(2):
            rc, out = host_layer(tglib, a, 0, x)
            assert rc == 0 and np.array_equal(bits(out), bits(ref)), f"rep {rep}"
        assert tglib.tg_arena_status(a.handle) == 0
    finally:
        tglib.tg_debug_fault_inject(0, -1)
        if old is None:
            os.environ.pop("TG_FUSE_GD16", None)
        else:
            os.environ["TG_FUSE_GD16"] = old
        a.close()
