"""GPU parity with a non-unit FFN norm weight (engine.py:229-230 runs the
MoE block on rms_norm(x) * ffn_norms[i]) on every path, and the Q4_0 cache
loader (relayout files -> HBM arena) end to end.  Every result must equal
the oracle bit for bit."""
import numpy as np
import pytest

from tests.conftest import gpu_note

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

DECODE = {"routed": 4, "fused": 3, "per_layer": 2}
BATCH = {"grouped": 1, "grouped_dot": 3, "per_token": 2}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def norm_arena(O, L, H, I, E, k, seed):
    from tinygiant_amd.arena import HBMExpertArena
    rng = np.random.default_rng(seed)
    a = HBMExpertArena(L, E, H, I, k)
    layers, routers, norms = [], [], []
    for l in range(L):
        lb, r = O.synth_layer(seed, l, H, I, E)
        g = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
        # router before and after the norm: both orders must give router * g
        if l % 2:
            a.load_norm(l, g)
            a.load_router(l, r)
        else:
            a.load_router(l, r)
            a.load_norm(l, g)
        a.load_layer(l, lb)
        layers.append(lb)
        routers.append(r)
        norms.append(g)
    return a, layers, routers, norms


@pytest.mark.parametrize("path,T", [("routed", 1), ("fused", 1), ("per_layer", 1), ("grouped", 5),
                                    ("grouped", 40), ("grouped_dot", 17), ("per_token", 3)])
@pytest.mark.parametrize("H,I,E,k", [(512, 96, 32, 8), (2048, 768, 128, 8)])
def test_norm_weight_layer(O, tglib, path, T, H, I, E, k):
    gpu_note(f"norm weight layer path={path} T={T} H={H}")
    from tinygiant_amd.moe import MoEBlock
    a, layers, routers, norms = norm_arena(O, 1, H, I, E, k, seed=71)
    try:
        if path in DECODE:
            a.set_decode_path(DECODE[path])
        else:
            a.set_batch_path(BATCH[path])
        x = O.synth_normal(71, O.stream_id(0, T, 4), 1.0, T * H).reshape(T, H)
        ref, ridx, rw, _ = O.moe_layer(layers[0], routers[0], H, I, E, k, x, norm=norms[0])
        out, idx, w = MoEBlock(a).forward(0, dev(x), return_routing=True)
        assert np.array_equal(host(idx), ridx)
        assert np.array_equal(bits(host(w)), bits(rw))
        got = host(out)
        assert np.array_equal(bits(got), bits(ref)), f"max |diff| {np.max(np.abs(got - ref)):.3e}"
        a.status()
    finally:
        a.close()


@pytest.mark.parametrize("path", ["routed", "fused", "per_layer"])
def test_norm_weight_stack(O, tglib, path):
    """The routed path forms each layer's router partials in the layer
    before it, so the next layer's weight is folded in there."""
    gpu_note(f"norm weight stack path={path}")
    from tinygiant_amd.moe import MoEBlock
    H, I, E, k, L = 1024, 256, 64, 8, 5
    a, layers, routers, norms = norm_arena(O, L, H, I, E, k, seed=72)
    try:
        a.set_decode_path(DECODE[path])
        x0 = O.synth_normal(72, O.stream_id(0, 0, 4), 1.0, H).reshape(1, H)
        ref, trace = O.moe_stack(layers, routers, H, I, E, k, x0, norms=norms)
        xd = dev(x0)
        idx, _ = MoEBlock(a).step_trace(xd)
        assert np.array_equal(host(idx), trace[:, 0, :])
        assert np.array_equal(bits(host(xd)), bits(ref))
        a.status()
    finally:
        a.close()


def test_cache_dir_loader_round_trip(O, tglib, tmp_path):
    """relayout.write_cache -> HBMExpertArena.from_cache_dir: the layer bytes
    come back unchanged, and a stack over the loaded arena equals the
    oracle's on the same files (norm weights included)."""
    gpu_note("Q4_0 cache loader round trip")
    from tinygiant_amd import relayout
    from tinygiant_amd.arena import HBMExpertArena
    from tinygiant_amd.moe import MoEBlock
    H, I, E, k, L = 512, 96, 32, 8, 3
    rng = np.random.default_rng(73)
    layers, routers, norms = [], [], []
    for l in range(L):
        lb, r = O.synth_layer(73, l, H, I, E)
        layers.append(lb)
        routers.append(r)
        norms.append((1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    relayout.write_cache(tmp_path, layers, routers, k, norms=norms)
    a = HBMExpertArena.from_cache_dir(tmp_path)
    try:
        assert (a.n_layers, a.n_experts, a.embed_dim, a.inter_dim, a.top_k) == (L, E, H, I, k)
        for l in range(L):
            assert np.array_equal(a.read_layer(l), layers[l])
        x0 = O.synth_normal(73, O.stream_id(0, 0, 4), 1.0, 2 * H).reshape(2, H)
        ref, _ = O.moe_stack(layers, routers, H, I, E, k, x0, norms=norms)
        xd = dev(x0)
        MoEBlock(a).step(xd)
        assert np.array_equal(bits(host(xd)), bits(ref))
        a.status()
    finally:
        a.close()
