"""Oracle parity of the benchmark configurations at their full shapes.

  config 2  the 48-layer Qwen3-30B-A3B-shaped stack, one token, default
            (routed) path: bit-exact against the oracle's stack, and within
            the 1e-3 stack tolerance
  config 3  64 tokens through one 30B layer with Zipf(1.1)-skewed routing
            (grouped int8-MFMA path)
  config 4  2048 tokens through one 30B layer (prefill: multi-tile work items
            of ~128 entries per expert)
  config 4  the full prefill: 2048 tokens through all 48 layers on the grouped
            path, compared with the oracle after every layer on every 8th
            token (tokens do not interact in the MoE block, so the oracle's
            stack over a subset of the tokens is the reference for them),
            bit for bit and within 1e-3 at the end
  config 5  32 tokens through one Qwen3-235B-A22B layer (H=4096, I=1536) with
            Zipf(1.1)-skewed routing (grouped path); and one token through
            all 94 layers of the 235B stack with Zipf-skewed routers on the
            default (routed) path, every layer's routing and the final x
            against the oracle's stack, bit for bit and within 1e-3

The experts are generated on the device (the generator is bit-identical to
the host's) and read back for the oracle, which checks every token's routing
(ids and weights) and output bit for bit.  Reference behaviour:
tinygiant/engine.py:229-258, csrc/libtinygiant.c:555-655.
"""
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


def rel_err(got, ref):
    """Normwise max relative error max|got - ref| / max|ref|."""
    ref64 = np.asarray(ref, dtype=np.float64)
    return float(np.max(np.abs(np.asarray(got, dtype=np.float64) - ref64)) / np.max(np.abs(ref64)))


def check_layer(O, a, layer_bytes, router, H, I, E, k, x, norm=None):
    from tinygiant_amd.moe import MoEBlock
    ref, ridx, rw, _ = O.moe_layer(layer_bytes, router, H, I, E, k, x, norm=norm)
    out, idx, w = MoEBlock(a).forward(0, dev(x), return_routing=True)
    got_idx = host(idx)
    assert np.array_equal(got_idx, ridx), f"{int(np.sum(got_idx != ridx))} ids differ"
    assert np.array_equal(bits(host(w)), bits(rw))
    got = host(out)
    assert rel_err(got, ref) <= 1e-5
    assert np.array_equal(bits(got), bits(ref)), f"max |diff| {np.max(np.abs(got - ref)):.3e}"
    a.status()
    return ridx


def zipf_case(O, H, I, E, k, T, seed):
    from tinygiant_amd.arena import HBMExpertArena
    from tinygiant_amd.synth import fit_zipf_exponent, zipf_skew
    rng = np.random.default_rng(seed)
    router, shift = zipf_skew(rng, E, H)
    a = HBMExpertArena(1, E, H, I, k)
    try:
        a.synth_layer(0, seed)
        a.load_router(0, router)
        a.set_batch_path(a.BATCH_GROUPED)
        lb = a.read_layer(0)
        x = (rng.standard_normal((T, H)).astype(np.float32) + shift).astype(np.float32)
        idx = check_layer(O, a, lb, router, H, I, E, k, x)
    finally:
        a.close()
    uniq = len(np.unique(idx))
    s = fit_zipf_exponent(idx, E)
    gpu_note(f"  {uniq} distinct experts, fitted rank-frequency exponent {s:.2f}")
    assert uniq < E  # the skew concentrates the routing


def test_config3_batched_zipf_30b(O, tglib):
    gpu_note("config 3: T=64 H=2048 I=768 E=128 k=8, Zipf routers, grouped")
    zipf_case(O, 2048, 768, 128, 8, 64, seed=301)


def test_config5_batched_zipf_235b(O, tglib):
    gpu_note("config 5: T=32 H=4096 I=1536 E=128 k=8, Zipf routers, grouped")
    zipf_case(O, 4096, 1536, 128, 8, 32, seed=501)


def test_config4_prefill_layer_30b(O, tglib):
    """2048 tokens, N(0, 0.02) routers: ~128 entries per expert, so every
    selected expert runs multi-tile MFMA items."""
    gpu_note("config 4: T=2048 H=2048 I=768 E=128 k=8, grouped MFMA")
    from tinygiant_amd.arena import HBMExpertArena
    H, I, E, k, T = 2048, 768, 128, 8, 2048
    seed = 401
    a = HBMExpertArena(1, E, H, I, k)
    try:
        a.synth_layer(0, seed)
        router = O.synth_normal(seed, O.stream_id(0, 0, 3), 0.02, E * H).reshape(E, H)
        lb = a.read_layer(0)
        x = O.synth_normal(seed, O.stream_id(0, 0, 4), 1.0, T * H).reshape(T, H)
        idx = check_layer(O, a, lb, router, H, I, E, k, x)
        counts = np.bincount(idx.ravel(), minlength=E)
        gpu_note(f"  entries per expert: max {counts.max()}, min {counts.min()}")
        assert counts.max() > 96  # items of more than three M-tiles occur
    finally:
        a.close()


@pytest.mark.parametrize("with_norm", [False, True])
def test_config2_stack_48_layers(O, tglib, with_norm):
    """One token through the 48-layer 30B stack on the default (routed)
    path, launched layer by layer, against the oracle's layer-by-layer
    stack: bit for bit, and within the 1e-3 tolerance allowed after the full
    stack.  The second case loads N(1, 0.1) FFN norm weights into every
    layer."""
    gpu_note(f"config 2: 48 layers H=2048, one token, norm={with_norm}")
    from tinygiant_amd.arena import HBMExpertArena
    from tinygiant_amd.moe import MoEBlock
    H, I, E, k, L = 2048, 768, 128, 8, 48
    seed = 201
    rng = np.random.default_rng(seed)
    a = HBMExpertArena(L, E, H, I, k)
    try:
        norms = []
        for l in range(L):
            a.synth_layer(l, seed)
            if with_norm:
                g = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
                a.load_norm(l, g)
                norms.append(g)
        x0 = O.synth_normal(seed, O.stream_id(0, 0, 4), 1.0, H).reshape(1, H)
        xd = dev(x0)
        MoEBlock(a).step(xd)
        got = host(xd)
        a.status()
        x = x0.copy()
        for l in range(L):  # the oracle one layer at a time (340 MB of host bytes each)
            router = O.synth_normal(seed, O.stream_id(l, 0, 3), 0.02, E * H).reshape(E, H)
            x, _ = O.moe_stack([a.read_layer(l)], [router], H, I, E, k, x,
                               norms=[norms[l]] if with_norm else None)
        err = rel_err(got, x)
        gpu_note(f"  stack rel err {err:.2e}")
        assert err <= 1e-3
        assert np.array_equal(bits(got), bits(x)), f"max |diff| {np.max(np.abs(got - x)):.3e}"
    finally:
        a.close()


def test_config4_prefill_stack_48_layers(O, tglib):
    """2048 tokens through the 48-layer 30B stack (grouped int8-MFMA path,
    one stack call per layer), checked after every layer against the
    oracle's stack on every 8th token, bit for bit; 1e-3 at the end."""
    gpu_note("config 4: 2048 tokens x 48 layers H=2048, grouped MFMA, oracle on every 8th token per layer")
    from tinygiant_amd.arena import HBMExpertArena
    from tinygiant_amd.moe import MoEBlock
    H, I, E, k, L, T = 2048, 768, 128, 8, 48, 2048
    seed = 402
    a = HBMExpertArena(L, E, H, I, k)
    try:
        for l in range(L):
            a.synth_layer(l, seed)
        a.set_batch_path(a.BATCH_GROUPED)
        x0 = O.synth_normal(seed, O.stream_id(0, 0, 4), 1.0, T * H).reshape(T, H)
        sample = np.arange(0, T, 8)
        xs = x0[sample].copy()
        xd = dev(x0)
        blk = MoEBlock(a)
        for l in range(L):
            blk.step(xd, l, 1)
            got = host(xd)[sample]
            a.status()
            router = O.synth_normal(seed, O.stream_id(l, 0, 3), 0.02, E * H).reshape(E, H)
            xs, _ = O.moe_stack([a.read_layer(l)], [router], H, I, E, k, xs)
            assert np.array_equal(bits(got), bits(xs)), \
                f"layer {l}: {int(np.sum(bits(got) != bits(xs)))} values differ, max |diff| {np.max(np.abs(got - xs)):.3e}"
            if l % 8 == 7:
                gpu_note(f"  layer {l} bit-exact")
        err = rel_err(got, xs)
        gpu_note(f"  48 layers bit-exact on {sample.size} tokens, rel err {err:.2e}")
        assert err <= 1e-3
    finally:
        a.close()


def zipf_stack_routers(rng, L, E, H, beta=0.6):
    """Per-layer routers N(0, 0.02) plus a per-expert bias along one shared
    direction u (the construction of synth.zipf_skew, one u for the whole
    stack), and the token shift c u."""
    from tinygiant_amd.synth import zipf_router_bias
    u = rng.standard_normal(H)
    u /= np.linalg.norm(u)
    c = 0.5 * np.sqrt(H)
    rms = np.sqrt(1.0 + c * c / H)
    bias = zipf_router_bias(E, beta * 0.02 * np.sqrt(H) / rms)
    routers = []
    for _ in range(L):
        r = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
        r += (bias[:, None] * (rms / c) * u[None, :]).astype(np.float32)
        routers.append(r)
    return routers, (c * u).astype(np.float32)


def test_config5_decode_stack_94_layers_zipf(O, tglib):
    """One token through all 94 layers of the 235B-shaped stack (127.7 GB of
    experts generated on the device) with Zipf-skewed routers, on the default
    routed path with the routing of every layer recorded.  The oracle runs
    the same stack layer by layer on the experts the GPU selected, read back
    one by one (an expert the oracle selects but the GPU did not would be
    zero bytes and change its output)."""
    gpu_note("config 5: one token x 94 layers H=4096 I=1536, Zipf routers, routed path")
    from tinygiant_amd.arena import HBMExpertArena
    from tinygiant_amd.moe import MoEBlock
    from tinygiant_amd.synth import fit_zipf_exponent
    H, I, E, k, L = 4096, 1536, 128, 8, 94
    seed = 502
    rng = np.random.default_rng(seed)
    routers, shift = zipf_stack_routers(rng, L, E, H)
    a = HBMExpertArena(L, E, H, I, k)
    try:
        for l in range(L):
            a.synth_layer(l, seed)
            a.load_router(l, routers[l])
        x0 = (O.synth_normal(seed, O.stream_id(0, 0, 4), 1.0, H).reshape(1, H) + shift).astype(np.float32)
        xd = dev(x0)
        idx, w = MoEBlock(a).step_trace(xd)
        got, gidx, gw = host(xd), host(idx).reshape(L, k), host(w).reshape(L, k)
        a.status()
        gpu_note(f"  routing over the stack: {len(np.unique(gidx))} distinct experts, "
                 f"fitted exponent {fit_zipf_exponent(gidx, E):.2f}")
        layer = np.zeros(a.layer_bytes, np.uint8)
        eb = a.expert_bytes
        x = x0.copy()
        for l in range(L):
            layer[:] = 0
            for e in gidx[l]:
                layer[e * eb:(e + 1) * eb] = a.read_expert(l, int(e))
            x, tr = O.moe_stack([layer], [routers[l]], H, I, E, k, x)
            assert np.array_equal(tr[0, 0], gidx[l]), f"layer {l}: routing {tr[0, 0]} vs {gidx[l]}"
            if l % 16 == 15:
                gpu_note(f"  oracle through layer {l}")
        err = rel_err(got, x)
        gpu_note(f"  94 layers: stack rel err {err:.2e}")
        assert err <= 1e-3
        assert np.array_equal(bits(got), bits(x)), f"max |diff| {np.max(np.abs(got - x)):.3e}"
    finally:
        a.close()


def test_config5_batched_stack_94_layers_zipf(O, tglib):
    """32 tokens through all 94 layers of the 235B-shaped stack with
    Zipf-skewed routers on the grouped path (one-tile items: the routing
    launch builds the work items, gate/up and down run in one launch).  After
    every layer all 32 rows equal the oracle's stack bit for bit (the oracle
    reads each layer back from the arena); 1e-3 at the end."""
    gpu_note("config 5: 32 tokens x 94 layers H=4096 I=1536, Zipf routers, grouped path")
    from tinygiant_amd.arena import HBMExpertArena
    from tinygiant_amd.moe import MoEBlock
    H, I, E, k, L, T = 4096, 1536, 128, 8, 94, 32
    seed = 503
    rng = np.random.default_rng(seed)
    routers, shift = zipf_stack_routers(rng, L, E, H)
    a = HBMExpertArena(L, E, H, I, k)
    try:
        for l in range(L):
            a.synth_layer(l, seed)
            a.load_router(l, routers[l])
        a.set_batch_path(a.BATCH_GROUPED)
        x0 = (O.synth_normal(seed, O.stream_id(0, 0, 4), 1.0, T * H).reshape(T, H) + shift).astype(np.float32)
        xd = dev(x0)
        blk = MoEBlock(a)
        xs = x0.copy()
        uniq = []
        for l in range(L):
            blk.step(xd, l, 1)
            got = host(xd)
            a.status()
            xs, tr = O.moe_stack([a.read_layer(l)], [routers[l]], H, I, E, k, xs)
            uniq.append(len(np.unique(tr[0])))
            assert np.array_equal(bits(got), bits(xs)), \
                f"layer {l}: {int(np.sum(bits(got) != bits(xs)))} values differ, max |diff| {np.max(np.abs(got - xs)):.3e}"
            if l % 16 == 15:
                gpu_note(f"  layer {l} bit-exact ({uniq[-1]} distinct experts)")
        err = rel_err(got, xs)
        gpu_note(f"  94 layers bit-exact, {np.mean(uniq):.1f} distinct experts per layer, rel err {err:.2e}")
        assert err <= 1e-3
    finally:
        a.close()
