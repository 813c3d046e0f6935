"""GPU parity of the grouped (batched decode / prefill) MoE path: tokens are
grouped by expert and every selected expert's weights are read once per
layer.  Results must equal the oracle (and the per-token path) bit for bit,
whatever the order of the tokens inside each group."""
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


def make_arena(O, n_layers, H, I, E, k, seed, routers=None):
    from tinygiant_amd.arena import HBMExpertArena
    a = HBMExpertArena(n_layers, E, H, I, k)
    layers, rs = [], []
    for L in range(n_layers):
        lb, r = O.synth_layer(seed, L, H, I, E)
        if routers is not None:
            r = routers[L]
        a.load_layer(L, lb)
        a.load_router(L, r)
        layers.append(lb)
        rs.append(r)
    return a, layers, rs


# router chains: 16-token tiles (T 17, 64), 32-token tiles with a partial last tile (T 100)
@pytest.mark.parametrize("H,I,E,k,T", [(256, 64, 16, 4, 5), (256, 64, 16, 4, 33), (512, 96, 32, 8, 17),
                                       (256, 352, 16, 4, 40), (2048, 768, 128, 8, 64), (512, 96, 32, 8, 100)])
def test_grouped_layer_matches_oracle(O, tglib, H, I, E, k, T):
    gpu_note(f"grouped layer H={H} I={I} E={E} k={k} T={T}")
    from tinygiant_amd.moe import MoEBlock
    a, layers, routers = make_arena(O, 1, H, I, E, k, seed=61)
    try:
        a.set_batch_path(a.BATCH_GROUPED)
        x = O.synth_normal(61, O.stream_id(0, T, 4), 1.0, T * H).reshape(T, H)
        ref, ridx, rw, _ = O.moe_layer(layers[0], routers[0], H, I, E, k, x)
        out, idx, w = MoEBlock(a).forward(0, dev(x), return_routing=True)
        assert np.array_equal(host(idx), ridx)
        assert np.array_equal(bits(host(w)), bits(rw))
        got = host(out)
        assert np.array_equal(bits(got), bits(ref)), f"max |diff| {np.max(np.abs(got - ref)):.3e}"
    finally:
        a.close()


def test_grouped_equals_per_token_path(O, tglib):
    gpu_note("grouped vs per-token, full shape, T=64")
    from tinygiant_amd.arena import HBMExpertArena
    from tinygiant_amd.moe import MoEBlock
    H, I, E, k, T = 2048, 768, 128, 8, 64
    a = HBMExpertArena(2, E, H, I, k)
    try:
        for l in range(2):
            a.synth_layer(l, seed=3)
        x = dev(O.synth_normal(3, O.stream_id(0, 0, 4), 1.0, T * H).reshape(T, H))
        blk = MoEBlock(a)
        a.set_batch_path(a.BATCH_GROUPED)
        g = host(blk.forward(1, x))
        xg = x.clone()
        blk.step(xg)
        a.set_batch_path(a.BATCH_PER_TOKEN)
        p = host(blk.forward(1, x))
        xp = x.clone()
        blk.step(xp)
        assert np.array_equal(bits(g), bits(p))
        assert np.array_equal(bits(host(xg)), bits(host(xp)))
    finally:
        a.close()


def test_grouped_large_groups(O, tglib):
    """Every token routed to the same k experts: each group holds all T
    tokens, more than one LDS chunk."""
    gpu_note("grouped, all tokens on the same experts, T=40")
    from tinygiant_amd.moe import MoEBlock
    H, I, E, k, T = 512, 96, 32, 8, 40
    rng = np.random.default_rng(8)
    v = rng.standard_normal(H).astype(np.float32)
    Wr = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    for e in range(k):
        Wr[e] += np.float32(0.5 - 0.05 * e) * v / np.float32(np.sqrt(H))
    a, layers, routers = make_arena(O, 1, H, I, E, k, seed=8, routers=[Wr])
    try:
        a.set_batch_path(a.BATCH_GROUPED)
        x = (v[None, :] + 0.1 * rng.standard_normal((T, H))).astype(np.float32)
        ref, ridx, rw, _ = O.moe_layer(layers[0], routers[0], H, I, E, k, x)
        assert len(np.unique(ridx)) == k, "construction must send every token to the same experts"
        out, idx, w = MoEBlock(a).forward(0, dev(x), return_routing=True)
        assert np.array_equal(host(idx), ridx)
        assert np.array_equal(bits(host(out)), bits(ref))
    finally:
        a.close()


@pytest.mark.parametrize("H,I,E,k,T,L", [(256, 64, 16, 4, 3, 4), (2048, 768, 128, 8, 8, 2)])
def test_grouped_stack_matches_oracle(O, tglib, H, I, E, k, T, L):
    gpu_note(f"grouped stack H={H} T={T} L={L}")
    from tinygiant_amd.moe import MoEBlock
    a, layers, routers = make_arena(O, L, H, I, E, k, seed=71)
    try:
        x0 = O.synth_normal(71, O.stream_id(0, 1, 4), 1.0, T * H).reshape(T, H)
        ref, _ = O.moe_stack(layers, routers, H, I, E, k, x0)
        xd = dev(x0)
        MoEBlock(a).step(xd)
        assert np.array_equal(bits(host(xd)), bits(ref))
    finally:
        a.close()


def test_grouped_single_token(O, tglib):
    gpu_note("grouped forced for T=1")
    from tinygiant_amd.moe import MoEBlock
    H, I, E, k = 512, 96, 32, 8
    a, layers, routers = make_arena(O, 1, H, I, E, k, seed=9)
    try:
        a.set_batch_path(a.BATCH_GROUPED)
        x = O.synth_normal(9, O.stream_id(0, 2, 4), 1.0, H).reshape(1, H)
        ref, ridx, _, _ = O.moe_layer(layers[0], routers[0], H, I, E, k, x)
        out, idx, _ = MoEBlock(a).forward(0, dev(x), return_routing=True)
        assert np.array_equal(host(idx), ridx)
        assert np.array_equal(bits(host(out)), bits(ref))
    finally:
        a.close()


@pytest.mark.parametrize("H,I,E,k,T", [(512, 96, 32, 8, 200), (256, 352, 16, 4, 300), (2048, 768, 128, 8, 600)])
def test_mfma_layer_matches_oracle_many_tiles(O, tglib, H, I, E, k, T):
    """Groups spanning several 32-entry M-tiles of the int8-MFMA path."""
    gpu_note(f"mfma grouped layer H={H} T={T}")
    from tinygiant_amd.moe import MoEBlock
    a, layers, routers = make_arena(O, 1, H, I, E, k, seed=83)
    try:
        a.set_batch_path(a.BATCH_GROUPED)
        x = O.synth_normal(83, O.stream_id(0, T, 4), 1.0, T * H).reshape(T, H)
        ref, ridx, rw, _ = O.moe_layer(layers[0], routers[0], H, I, E, k, x)
        out, idx, w = MoEBlock(a).forward(0, dev(x), return_routing=True)
        assert np.array_equal(host(idx), ridx)
        got = host(out)
        assert np.array_equal(bits(got), bits(ref)), f"max |diff| {np.max(np.abs(got - ref)):.3e}"
    finally:
        a.close()


@pytest.mark.parametrize("T", [64, 1024, 2048])
def test_mfma_equals_dot_path(O, tglib, T):
    """The int8-MFMA tiles and the packed-dot kernels give the same bytes
    (full shape, up to a 2048-token prefill batch)."""
    gpu_note(f"mfma vs dot, full shape, T={T}")
    from tinygiant_amd.arena import HBMExpertArena
    from tinygiant_amd.moe import MoEBlock
    H, I, E, k = 2048, 768, 128, 8
    a = HBMExpertArena(1, E, H, I, k)
    try:
        a.synth_layer(0, seed=19)
        x = dev(O.synth_normal(19, O.stream_id(0, 5, 4), 1.0, T * H).reshape(T, H))
        blk = MoEBlock(a)
        a.set_batch_path(a.BATCH_GROUPED)
        m = host(blk.forward(0, x))
        a.set_batch_path(a.BATCH_GROUPED_DOT)
        d = host(blk.forward(0, x))
        assert np.array_equal(bits(m), bits(d))
    finally:
        a.close()


def test_mfma16_every_item_size(O, tglib):
    """Prefill-sized batches run 16 x 16 int8 MFMA tiles on items of up to
    160 entries (10 column tiles of 16).  A Zipf(1.1)-skewed router gives
    groups from a handful of entries (one column tile) to experts split over
    several items; the layer must equal the oracle bit for bit."""
    from tinygiant_amd.moe import MoEBlock
    from tinygiant_amd.synth import zipf_skew
    H, I, E, k, T = 512, 256, 32, 8, 1000
    gpu_note(f"mfma16 item sizes H={H} I={I} E={E} T={T} zipf")
    rng = np.random.default_rng(5)
    router, shift = zipf_skew(rng, E, H)
    a, layers, routers = make_arena(O, 1, H, I, E, k, seed=29, routers=[router])
    try:
        a.set_batch_path(a.BATCH_GROUPED)
        x = (O.synth_normal(29, O.stream_id(0, T, 4), 1.0, T * H).reshape(T, H) + shift[None, :]).astype(np.float32)
        ref, ridx, rw, _ = O.moe_layer(layers[0], routers[0], H, I, E, k, x)
        counts = np.bincount(ridx.reshape(-1), minlength=E)
        # the sizes this test is about: one-tile groups, whole items, experts over several items
        assert counts[counts > 0].min() <= 16 and counts.max() > 320, counts
        assert np.any((counts > 32) & (counts < 160)), counts
        out, idx, w = MoEBlock(a).forward(0, dev(x), return_routing=True)
        assert np.array_equal(host(idx), ridx)
        got = host(out)
        assert np.array_equal(bits(got), bits(ref)), f"max |diff| {np.max(np.abs(got - ref)):.3e}"
    finally:
        a.close()


def test_fused_combine_counts_across_calls(O, tglib):
    """With TG_FUSE_COMBINE=1 the one-tile and 16 x 16 down launches also
    combine (off by default: measured slower than k_combine): each block counts
    its entries in at (token, 128-row tile) in the arena's scratch, and the
    block that brings a count to k folds that token's k rows over its tile
    and sets the count back to zero.  Calls of different sizes on one arena
    (one-tile items, two-tile items whose combine is a launch of its own,
    16 x 16 items), each made twice, must equal the oracle bit for bit every
    time: no call leaves a count behind for the next."""
    import os
    from tinygiant_amd.moe import MoEBlock
    H, I, E, k = 512, 256, 32, 8
    a, layers, routers = make_arena(O, 1, H, I, E, k, seed=37)
    old = os.environ.get("TG_FUSE_COMBINE")
    os.environ["TG_FUSE_COMBINE"] = "1"  # the library reads it per call
    try:
        a.set_batch_path(a.BATCH_GROUPED)
        blk = MoEBlock(a)
        # entries per expert 10 (one tile), 250 (16 x 16), 24 (two tiles)
        for i, T in enumerate((40, 1000, 96, 40, 1000)):
            x = O.synth_normal(37, O.stream_id(0, i, 4), 1.0, T * H).reshape(T, H)
            ref, _, _, _ = O.moe_layer(layers[0], routers[0], H, I, E, k, x)
            xd = dev(x)
            for rep in range(2):
                gpu_note(f"fused combine H={H} T={T} call {i} rep {rep}")
                got = host(blk.forward(0, xd))
                assert np.array_equal(bits(got), bits(ref)), f"T={T} rep {rep}: max |diff| {np.max(np.abs(got - ref)):.3e}"
    finally:
        if old is None:
            os.environ.pop("TG_FUSE_COMBINE", None)
        else:
            os.environ["TG_FUSE_COMBINE"] = old
        a.close()


# (H, I, E, k, token counts): one-tile items with a gate/up K of 8 chunks
# (activations staged once) and of 16 (staged per chunk), the placed-entry
# grouping below 128 tokens and the listing one from 128; 16 x 16 items
# (about 250 and 160 entries per expert: whole items, and experts split over
# two items)
@pytest.mark.parametrize("H,I,E,k,Ts", [(512, 256, 32, 8, (40, 9, 64)), (2048, 768, 128, 8, (64, 200, 3)),
                                        (4096, 1536, 128, 8, (32, 5)), (512, 256, 32, 8, (1000, 640, 1000))])
def test_fused_gate_up_down_across_calls(O, tglib, H, I, E, k, Ts):
    """Gate/up and down of the one-tile and the 16 x 16 work items run in one
    launch (down blocks wait, bounded, for their item's gate/up blocks to
    store h; the kernel that builds the work items clears the per-item counts
    for every call).  Calls of different sizes on one arena, each made with
    the default launches and with every alternative switched on (TG_FUSE_GD=0
    and TG_FUSE_GD16=0: the two launches; TG_ROUTE_GROUP=0 and TG_GROUP_PAR=0:
    the grouping kernel, building the entry lists itself from 128 tokens; all
    read per call), equal the oracle bit for bit."""
    import os
    from tinygiant_amd.moe import MoEBlock
    a, layers, routers = make_arena(O, 1, H, I, E, k, seed=41)
    switches = ("TG_FUSE_GD", "TG_FUSE_GD16", "TG_ROUTE_GROUP", "TG_GROUP_PAR")
    old = {v: os.environ.get(v) for v in switches}
    try:
        blk = MoEBlock(a)
        for i, T in enumerate(Ts):
            x = O.synth_normal(41, O.stream_id(0, i, 4), 1.0, T * H).reshape(T, H)
            ref, _, _, _ = O.moe_layer(layers[0], routers[0], H, I, E, k, x)
            xd = dev(x)
            for mode in ("1", "0", "1"):
                for v in switches:
                    os.environ[v] = mode
                gpu_note(f"fused gate/up + down H={H} T={T} defaults={mode}")
                got = host(blk.forward(0, xd))
                assert np.array_equal(bits(got), bits(ref)), \
                    f"T={T} mode {mode}: max |diff| {np.max(np.abs(got - ref)):.3e}"
        assert tglib.tg_arena_status(a.handle) == 0
    finally:
        for v, val in old.items():
            if val is None:
                os.environ.pop(v, None)
            else:
                os.environ[v] = val
        a.close()
