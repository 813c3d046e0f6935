"""GPU parity of the one-launch decode path (persistent kernel over every
layer of a stack, one token) against the oracle and against the per-layer
kernel path, on identical bytes.  Every result must be bit-identical."""
import numpy as np
import pytest

from tests.conftest import gpu_note

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def make_arena(O, n_layers, H, I, E, k, seed):
    from tinygiant_amd.arena import HBMExpertArena
    a = HBMExpertArena(n_layers, E, H, I, k)
    layers, routers = [], []
    for L in range(n_layers):
        lb, r = O.synth_layer(seed, L, H, I, E)
        a.load_layer(L, lb)
        a.load_router(L, r)
        layers.append(lb)
        routers.append(r)
    return a, layers, routers


@pytest.mark.parametrize("H,I,E,k,L", [(256, 64, 16, 4, 4), (512, 96, 32, 8, 3), (2048, 768, 128, 8, 3)])
def test_persist_stack_matches_oracle(O, tglib, H, I, E, k, L):
    gpu_note(f"persist stack H={H} I={I} E={E} k={k} L={L}")
    from tinygiant_amd.moe import MoEBlock
    a, layers, routers = make_arena(O, L, H, I, E, k, seed=41)
    try:
        a.set_decode_path(a.DECODE_PERSISTENT)
        for tok in range(3):
            x0 = O.synth_normal(41, O.stream_id(0, tok, 4), 1.0, H).reshape(1, H)
            ref, trace = O.moe_stack(layers, routers, H, I, E, k, x0)
            xd = dev(x0)
            idx, w = MoEBlock(a).step_trace(xd)
            a.status()
            assert np.array_equal(host(idx), trace[:, 0, :]), f"routing token {tok}"
            got = host(xd)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), \
                f"x after {L} layers, token {tok}: max |diff| {np.max(np.abs(got - ref)):.3e}"
    finally:
        a.close()


def test_persist_equals_per_layer_path_deep(O, tglib):
    """48 layers of the full shape: the persistent path and the per-layer
    kernels give the same bytes, routing and weights, token after token."""
    gpu_note("persist vs per-layer, 48 layers, H=2048")
    from tinygiant_amd.arena import HBMExpertArena
    from tinygiant_amd.moe import MoEBlock
    H, I, E, k, L = 2048, 768, 128, 8, 48
    a = HBMExpertArena(L, E, H, I, k)
    try:
        for l in range(L):
            a.synth_layer(l, seed=7)
        blk = MoEBlock(a)
        for tok in range(4):
            x0 = O.synth_normal(7, O.stream_id(0, 100 + tok, 4), 1.0, H).reshape(1, H)
            a.set_decode_path(a.DECODE_PERSISTENT)
            xp = dev(x0)
            ip, wp = blk.step_trace(xp)
            a.status()
            a.set_decode_path(a.DECODE_PER_LAYER)
            xl = dev(x0)
            il, wl = blk.step_trace(xl)
            assert np.array_equal(host(ip), host(il)), f"routing token {tok}"
            assert np.array_equal(host(wp).view(np.uint32), host(wl).view(np.uint32)), f"weights token {tok}"
            assert np.array_equal(host(xp).view(np.uint32), host(xl).view(np.uint32)), f"x token {tok}"
    finally:
        a.close()


def test_persist_back_to_back_launches(O, tglib):
    """Many one-token calls queued without host synchronisation (the
    counters are cleared on the stream before every launch)."""
    gpu_note("persist back-to-back x32")
    from tinygiant_amd.moe import MoEBlock
    H, I, E, k, L = 512, 96, 32, 8, 6
    a, layers, routers = make_arena(O, L, H, I, E, k, seed=5)
    try:
        a.set_decode_path(a.DECODE_PERSISTENT)
        X = O.synth_normal(5, O.stream_id(0, 0, 4), 1.0, 32 * H).reshape(32, H)
        xs = [dev(X[t:t + 1]) for t in range(32)]
        blk = MoEBlock(a)
        for t in range(32):
            blk.step(xs[t])
        a.status()
        for t in (0, 13, 31):
            ref, _ = O.moe_stack(layers, routers, H, I, E, k, X[t:t + 1])
            assert np.array_equal(host(xs[t]).view(np.uint32), ref.view(np.uint32)), f"token {t}"
    finally:
        a.close()
