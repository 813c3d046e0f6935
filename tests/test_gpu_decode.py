"""GPU parity of the one-token decode paths: ROUTED (one launch per layer
that also routes, from router partials the layer before it leaves), FUSED
(routing kernel, then one launch for gate/up and down with h handed over as
tagged words) and PER_LAYER (routing, gate/up and down as three kernels).
All must equal the oracle bit for bit, layer by layer and through a stack
(with the routing of every layer), and must agree with each other when
calls alternate on one arena (the tag generations of the exchange words
carry over between paths)."""
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


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


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


PATHS = {"routed": 4, "fused": 3, "per_layer": 2}


@pytest.mark.parametrize("path", ["routed", "fused", "per_layer"])
@pytest.mark.parametrize("H,I,E,k", [(256, 64, 16, 4), (512, 96, 32, 8), (1024, 256, 64, 8), (2048, 768, 128, 8)])
def test_one_token_layer_matches_oracle(O, tglib, path, H, I, E, k):
    gpu_note(f"one-token layer path={path} H={H} I={I} E={E} k={k}")
    from tinygiant_amd.moe import MoEBlock
    a, layers, routers = make_arena(O, 1, H, I, E, k, seed=91)
    try:
        a.set_decode_path(PATHS[path])
        blk = MoEBlock(a)
        for rep in range(3):  # repeated calls: fresh tag generations each time
            x = O.synth_normal(91, O.stream_id(0, rep, 4), 1.0, H).reshape(1, H)
            ref, ridx, rw, _ = O.moe_layer(layers[0], routers[0], H, I, E, k, x)
            out, idx, w = blk.forward(0, dev(x), return_routing=True)
            assert np.array_equal(host(idx), ridx)
            assert np.array_equal(bits(host(w)), bits(rw))
            got = host(out)
            assert np.array_equal(bits(got), bits(ref)), f"rep {rep}: max |diff| {np.max(np.abs(got - ref)):.3e}"
        a.status()
    finally:
        a.close()


@pytest.mark.parametrize("graphs", [False, True])
@pytest.mark.parametrize("path", ["routed", "fused", "per_layer"])
@pytest.mark.parametrize("H,I,E,k,L", [(256, 64, 16, 4, 5), (2048, 768, 128, 8, 4)])
def test_one_token_stack_matches_oracle(O, tglib, path, H, I, E, k, L, graphs):
    gpu_note(f"one-token stack path={path} H={H} L={L} graphs={graphs}")
    from tinygiant_amd.moe import MoEBlock
    a, layers, routers = make_arena(O, L, H, I, E, k, seed=92)
    try:
        a.set_decode_path(PATHS[path])
        a.set_graphs(graphs)
        x0 = O.synth_normal(92, O.stream_id(0, 1, 4), 1.0, H).reshape(1, H)
        ref, _ = O.moe_stack(layers, routers, H, I, E, k, x0)
        src = dev(x0)
        xd = dev(x0)
        for rep in range(3):  # with graphs on, calls after the first replay the graph it captured
            xd.copy_(src)
            MoEBlock(a).step(xd)
            got = host(xd)
            assert np.array_equal(bits(got), bits(ref)), f"rep {rep}: max |diff| {np.max(np.abs(got - ref)):.3e}"
        a.status()
    finally:
        a.close()


def test_paths_alternate_on_one_arena(O, tglib):
    """Routed, fused and per-layer calls interleaved on the same arena: each
    call's words carry a fresh generation, so no call can read another's."""
    gpu_note("one-token paths alternating")
    from tinygiant_amd.moe import MoEBlock
    H, I, E, k = 512, 96, 32, 8
    a, layers, routers = make_arena(O, 2, H, I, E, k, seed=93)
    order = ["routed", "fused", "routed", "per_layer", "fused", "routed", "routed", "per_layer", "fused"]
    try:
        blk = MoEBlock(a)
        for rep, path in enumerate(order):
            a.set_decode_path(PATHS[path])
            layer = rep % 2
            x = O.synth_normal(93, O.stream_id(layer, rep, 4), 1.0, H).reshape(1, H)
            ref, ridx, _, _ = O.moe_layer(layers[layer], routers[layer], H, I, E, k, x)
            out, idx, _ = blk.forward(layer, dev(x), return_routing=True)
            assert np.array_equal(host(idx), ridx)
            assert np.array_equal(bits(host(out)), bits(ref))
        a.status()
    finally:
        a.close()


def test_235b_shape_layer(O, tglib):
    """Qwen3-235B-A22B layer shape (H=4096, I=1536) on the default one-token
    path (the fused launch where its register budget allows, else three
    kernels)."""
    gpu_note("one-token layer H=4096 I=1536")
    from tinygiant_amd.moe import MoEBlock
    H, I, E, k = 4096, 1536, 128, 8
    a, layers, routers = make_arena(O, 1, H, I, E, k, seed=94)
    try:
        x = O.synth_normal(94, O.stream_id(0, 0, 4), 1.0, H).reshape(1, H)
        ref, ridx, rw, _ = O.moe_layer(layers[0], routers[0], H, I, E, k, x)
        out, idx, w = MoEBlock(a).forward(0, dev(x), return_routing=True)
        assert np.array_equal(host(idx), ridx)
        assert np.array_equal(bits(host(w)), bits(rw))
        assert np.array_equal(bits(host(out)), bits(ref))
        a.status()
    finally:
        a.close()


@pytest.mark.parametrize("path", ["routed", "per_layer"])
def test_stack_trace_matches_oracle(O, tglib, path):
    """The routing of every layer of a stack call (trace entry point) and the
    final x, against the oracle's stack trace."""
    gpu_note(f"one-token stack trace path={path}")
    from tinygiant_amd.moe import MoEBlock
    H, I, E, k, L = 1024, 256, 64, 8, 6
    a, layers, routers = make_arena(O, L, H, I, E, k, seed=95)
    try:
        a.set_decode_path(PATHS[path])
        x0 = O.synth_normal(95, O.stream_id(0, 2, 4), 1.0, H).reshape(1, H)
        ref, trace = O.moe_stack(layers, routers, H, I, E, k, x0)
        xd = dev(x0)
        idx, w = MoEBlock(a).step_trace(xd)
        assert np.array_equal(host(idx), trace[:, 0, :])
        assert np.array_equal(bits(host(xd)), bits(ref))
        a.status()
    finally:
        a.close()


def test_routed_stack_sub_ranges(O, tglib):
    """Routed stack calls over layer sub-ranges (the prologue forms the
    partials of the first layer of each call) give the oracle's stack."""
    gpu_note("routed stack sub-ranges")
    from tinygiant_amd.moe import MoEBlock
    H, I, E, k, L = 512, 96, 32, 8, 5
    a, layers, routers = make_arena(O, L, H, I, E, k, seed=96)
    try:
        a.set_decode_path(PATHS["routed"])
        x0 = O.synth_normal(96, O.stream_id(0, 3, 4), 1.0, H).reshape(1, H)
        ref, _ = O.moe_stack(layers, routers, H, I, E, k, x0)
        xd = dev(x0)
        blk = MoEBlock(a)
        blk.step(xd, 0, 2)
        blk.step(xd, 2, 1)
        blk.step(xd, 3, 2)
        assert np.array_equal(bits(host(xd)), bits(ref))
        a.status()
    finally:
        a.close()


@pytest.mark.parametrize("H,I", [(4096, 768), (2048, 1536)])
def test_deep_unit_variants_stack(O, tglib, H, I):
    """The routed launch's deep variants off the 235B shape, two layers
    against the oracle's stack.  H=4096, I=768: units of eight loads per
    thread but fewer units (192) than blocks (256), so whole units (down
    scales and residual rows staged in LDS, down loads after the unit).
    H=2048, I=1536: more units (384) than blocks (256, eight rows each), so
    half units of two loads per thread (nbH = 64), three per block."""
    gpu_note(f"one-token stack H={H} I={I} L=2 (deep unit variants)")
    from tinygiant_amd.moe import MoEBlock
    E, k, L = 128, 8, 2
    a, layers, routers = make_arena(O, L, H, I, E, k, seed=98)
    try:
        x0 = O.synth_normal(98, O.stream_id(0, 5, 4), 1.0, H).reshape(1, H)
        ref, trace = O.moe_stack(layers, routers, H, I, E, k, x0)
        xd = dev(x0)
        idx, w = MoEBlock(a).step_trace(xd)
        assert np.array_equal(host(idx), trace[:, 0, :])
        assert np.array_equal(bits(host(xd)), bits(ref))
        a.status()
    finally:
        a.close()


def test_235b_shape_stack(O, tglib):
    """Qwen3-235B-A22B shape through two layers on the default one-token path
    (the routed launch: 16-row chunks, two per router group, two gate/up
    units on some blocks), against the oracle's stack."""
    gpu_note("one-token stack H=4096 I=1536 L=2")
    from tinygiant_amd.moe import MoEBlock
    H, I, E, k, L = 4096, 1536, 128, 8, 2
    a, layers, routers = make_arena(O, L, H, I, E, k, seed=97)
    try:
        x0 = O.synth_normal(97, O.stream_id(0, 5, 4), 1.0, H).reshape(1, H)
        ref, trace = O.moe_stack(layers, routers, H, I, E, k, x0)
        xd = dev(x0)
        idx, w = MoEBlock(a).step_trace(xd)
        assert np.array_equal(host(idx), trace[:, 0, :])
        assert np.array_equal(bits(host(xd)), bits(ref))
        a.status()
    finally:
        a.close()
