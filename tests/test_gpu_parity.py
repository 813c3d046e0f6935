"""GPU parity: the gfx950 kernels against the CPU oracle on identical bytes.

Integer and byte results (Q8_0 bytes, block sums, top-k indices, synthetic
weights, planar repack) must be bit-exact.  The fp32 results are also
compared bit for bit, because every kernel performs the oracle's exact
operation order; the stated tolerance (max relative error 1e-5, normwise
max|a-b| / max|b|) is asserted as well so a failure reports both.
"""
import numpy as np
import pytest

from tests.conftest import gpu_note

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

REL_TOL = 1e-5


def call(name, *args):
    from tinygiant_amd._lib import call as _call
    return _call(name, *args)


def stream():
    return torch.cuda.current_stream().cuda_stream


def dev(a: np.ndarray) -> "torch.Tensor":
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def assert_fp32_parity(got, ref, what):
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    assert got.shape == ref.shape, what
    denom = max(float(np.max(np.abs(ref))), 1e-30)
    rel = float(np.max(np.abs(got.astype(np.float64) - ref))) / denom
    assert rel <= REL_TOL, f"{what}: normwise relative error {rel:.3e} > {REL_TOL}"
    nbad = int(np.sum(got.view(np.uint32) != ref.view(np.uint32)))
    assert nbad == 0, f"{what}: {nbad} of {got.size} values differ in bits (rel err {rel:.3e})"


# ---------------------------------------------------------------- generators

@pytest.mark.parametrize("n", [1, 1000, 65536 + 7])
def test_synth_normal_bitexact(O, tglib, n):
    gpu_note(f"synth_normal n={n}")
    sid = O.stream_id(3, 0, 3)
    ref = O.synth_normal(11, sid, 0.02, n)
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    call("tg_synth_normal_dev", 11, sid, 0.02, n, out.data_ptr(), stream())
    assert np.array_equal(host(out).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(1, 32), (96, 512), (768, 2048), (2048, 768)])
def test_synth_q40_bitexact(O, tglib, rows, cols):
    gpu_note(f"synth_q40 {rows}x{cols}")
    sid = O.stream_id(2, 5, 1)
    nb = cols // 32
    ref = O.to_planar(O.synth_q40(3, sid, 0.02, rows, cols), rows, nb)
    out = torch.empty(rows * nb * 18, dtype=torch.uint8, device="cuda")
    call("tg_synth_q40_dev", 3, sid, 0.02, rows, cols, out.data_ptr(), stream())
    assert np.array_equal(host(out), ref)


# ---------------------------------------------------------------- formats

@pytest.mark.parametrize("rows,nb", [(1, 1), (37, 24), (768, 64)])
def test_planar_repack_roundtrip(O, tglib, rows, nb):
    gpu_note(f"repack {rows}x{nb}")
    rng = np.random.default_rng(rows * 1000 + nb)
    aos = rng.integers(0, 256, rows * nb * 18, dtype=np.uint8)
    src = dev(aos)
    pl = torch.empty(aos.size, dtype=torch.uint8, device="cuda")
    back = torch.empty(aos.size, dtype=torch.uint8, device="cuda")
    call("tg_q40_to_planar_dev", src.data_ptr(), pl.data_ptr(), rows, nb, stream())
    call("tg_q40_from_planar_dev", pl.data_ptr(), back.data_ptr(), rows, nb, stream())
    assert np.array_equal(host(pl), O.to_planar(aos, rows, nb))
    assert np.array_equal(host(back), aos)


def q8_cases():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(32 * 64).astype(np.float32)
    x[:32] = 0.0                                   # amax = 0
    x[32:64] = np.arange(32, dtype=np.float32) - 15.5  # half-way multiples
    x[64:96] = np.float32(1e-30)                   # tiny values
    x[96:128] = np.linspace(-127, 127, 32).astype(np.float32) / 64  # +-amax
    return x


@pytest.mark.parametrize("which", ["cases", "large"])
def test_quantize_q8_0_bitexact(O, tglib, which):
    x = q8_cases() if which == "cases" else np.random.default_rng(9).standard_normal(2048 * 40).astype(np.float32)
    gpu_note(f"quantize_q8_0 {which} n={x.size}")
    xd = dev(x)
    out = torch.empty(x.size // 32 * 34, dtype=torch.uint8, device="cuda")
    call("tg_q40_quantize_q8_0_dev", xd.data_ptr(), out.data_ptr(), x.size, stream())
    assert np.array_equal(host(out), O.quantize_q8_0(x))


@pytest.mark.parametrize("rows,cols", [(5, 32), (64, 2048), (2048, 768), (768, 4096)])
def test_block_sums_bitexact(O, tglib, rows, cols):
    gpu_note(f"block_sums {rows}x{cols}")
    nb = cols // 32
    W = O.synth_q40(7, O.stream_id(0, 1, 0), 0.02, rows, cols)
    x = O.synth_normal(7, O.stream_id(0, 0, 4), 1.0, cols)
    xq = O.quantize_q8_0(x)
    ref = O.block_sums(W, rows, cols, xq)
    wd, xqd = dev(O.to_planar(W, rows, nb)), dev(xq)
    sums = torch.empty((rows, nb), dtype=torch.int32, device="cuda")
    call("tg_q40_block_sums_dev", wd.data_ptr(), rows, cols, xqd.data_ptr(), sums.data_ptr(), stream())
    assert np.array_equal(host(sums), ref)


@pytest.mark.parametrize("rows,cols", [(1, 32), (17, 256), (768, 2048), (2048, 768), (1536, 4096)])
def test_matvec_bitexact(O, tglib, rows, cols):
    gpu_note(f"matvec {rows}x{cols}")
    nb = cols // 32
    W = O.synth_q40(8, O.stream_id(1, 2, 2), 0.02, rows, cols)
    xq = O.quantize_q8_0(O.synth_normal(8, O.stream_id(1, 0, 4), 1.0, cols))
    ref = O.matvec_q40(W, rows, cols, xq)
    wd, xqd = dev(O.to_planar(W, rows, nb)), dev(xq)
    out = torch.empty(rows, dtype=torch.float32, device="cuda")
    call("tg_q40_matvec_dev", wd.data_ptr(), rows, cols, xqd.data_ptr(), out.data_ptr(), stream())
    assert_fp32_parity(host(out), ref, f"matvec {rows}x{cols}")


# ---------------------------------------------------------------- router

@pytest.mark.parametrize("E,H,k,T", [(16, 256, 4, 5), (128, 2048, 8, 4), (128, 4096, 8, 2), (20, 256, 4, 13),
                                     (128, 2048, 8, 64), (128, 4096, 8, 32), (20, 256, 4, 150),
                                     (128, 2048, 8, 300)])
def test_router_topk_exact(O, tglib, E, H, k, T):
    gpu_note(f"router E={E} H={H} k={k} T={T}")
    Wr = O.synth_normal(4, O.stream_id(0, 0, 3), 0.02, E * H).reshape(E, H)
    x = O.synth_normal(4, O.stream_id(0, 1, 4), 1.0, T * H).reshape(T, H)
    logits = torch.empty((T, E), dtype=torch.float32, device="cuda")
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    wrd, xd = dev(Wr), dev(x)
    call("tg_router_topk_dev", wrd.data_ptr(), xd.data_ptr(), E, H, k, 1e-6, T, logits.data_ptr(),
         idx.data_ptr(), w.data_ptr(), stream())
    gl, gi, gw = host(logits), host(idx), host(w)
    for t in range(T):
        rl = O.router_logits(Wr, x[t], O.rms_scale(x[t]))
        ri, rw = O.topk_softmax(rl, k)
        assert np.array_equal(gl[t].view(np.uint32), rl.view(np.uint32)), f"logits token {t}"
        assert np.array_equal(gi[t], ri), f"top-k token {t}"
        assert np.array_equal(gw[t].view(np.uint32), rw.view(np.uint32)), f"weights token {t}"


def test_router_topk_ties(O, tglib):
    """Exactly equal logits: the lower expert index ranks first."""
    gpu_note("router ties")
    E, H, k = 64, 256, 8
    Wr = np.zeros((E, H), np.float32)
    Wr[:, 0] = 1.0
    for e in (3, 9, 10, 40, 41, 63):
        Wr[e, 0] = 2.0               # six-way tie at the top
    Wr[50, 0] = 1.5
    x = np.zeros((1, H), np.float32)
    x[0, 0] = 4.0
    idx = torch.empty((1, k), dtype=torch.int32, device="cuda")
    w = torch.empty((1, k), dtype=torch.float32, device="cuda")
    logits = torch.empty((1, E), dtype=torch.float32, device="cuda")
    wrd, xd = dev(Wr), dev(x)
    call("tg_router_topk_dev", wrd.data_ptr(), xd.data_ptr(), E, H, k, 1e-6, 1, logits.data_ptr(),
         idx.data_ptr(), w.data_ptr(), stream())
    assert host(idx)[0].tolist() == [3, 9, 10, 40, 41, 63, 50, 0]
    ri, rw = O.topk_softmax(host(logits)[0], k)
    assert ri.tolist() == [3, 9, 10, 40, 41, 63, 50, 0]
    assert np.array_equal(host(w)[0].view(np.uint32), rw.view(np.uint32))


# ---------------------------------------------------------------- MoE layer

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


@pytest.mark.parametrize("H,I,E,k,T", [(256, 64, 16, 4, 3), (512, 96, 32, 8, 2), (2048, 768, 128, 8, 2)])
def test_moe_layer_bitexact(O, tglib, H, I, E, k, T):
    gpu_note(f"moe layer H={H} I={I} E={E} k={k} T={T}")
    from tinygiant_amd.moe import MoEBlock
    a, layers, routers = make_arena(O, 1, H, I, E, k, seed=21)
    try:
        x = O.synth_normal(21, O.stream_id(0, 7, 4), 1.0, T * H).reshape(T, H)
        ref, ridx, rw, _ = O.moe_layer(layers[0], routers[0], H, I, E, k, x)
        blk = MoEBlock(a)
        out, idx, w = blk.forward(0, dev(x), return_routing=True)
        assert np.array_equal(host(idx), ridx)
        assert np.array_equal(host(w).view(np.uint32), rw.view(np.uint32))
        assert_fp32_parity(host(out), ref, f"moe_out H={H}")
        # host-pointer entry point: same bytes
        hout, hidx, hw = blk.forward_host(0, x)
        assert np.array_equal(hidx, ridx)
        assert np.array_equal(hout.view(np.uint32), ref.view(np.uint32))
    finally:
        a.close()


def test_arena_roundtrip_and_offsets(O, tglib):
    gpu_note("arena roundtrip")
    H, I, E, k = 256, 64, 16, 4
    a, layers, _ = make_arena(O, 2, H, I, E, k, seed=5)
    try:
        for L in range(2):
            assert np.array_equal(a.read_layer(L), layers[L])
        eb = O.expert_bytes(H, I)
        for e in (0, 1, E - 1):
            info = a.expert_offset(e)
            assert info["offset"] == e * eb
            assert info["sizes"] == {"gate": I * H // 32 * 18, "up": I * H // 32 * 18, "down": H * I // 32 * 18}
    finally:
        a.close()


@pytest.mark.parametrize("H,I,E", [(256, 64, 16), (2048, 768, 128)])
def test_arena_synth_matches_host_generator(O, tglib, H, I, E):
    gpu_note(f"arena synth H={H} I={I} E={E}")
    from tinygiant_amd.arena import HBMExpertArena
    a = HBMExpertArena(1, E, H, I, 8 if E >= 8 else 4)
    try:
        a.synth_layer(0, seed=77)
        lb, _ = O.synth_layer(77, 0, H, I, E)
        assert np.array_equal(a.read_layer(0), lb)
    finally:
        a.close()


@pytest.mark.parametrize("H,I,E,k,T,L", [(256, 64, 16, 4, 2, 4), (2048, 768, 128, 8, 1, 3)])
def test_moe_stack_bitexact(O, tglib, H, I, E, k, T, L):
    gpu_note(f"moe stack H={H} L={L} T={T}")
    from tinygiant_amd.moe import MoEBlock
    a, layers, routers = make_arena(O, L, H, I, E, k, seed=33)
    try:
        x0 = O.synth_normal(33, O.stream_id(0, 9, 4), 1.0, T * H).reshape(T, H)
        ref, _ = O.moe_stack(layers, routers, H, I, E, k, x0)
        xd = dev(x0)
        MoEBlock(a).step(xd)
        assert_fp32_parity(host(xd), ref, f"stack H={H} L={L}")
        xh = MoEBlock(a).step_host(x0)
        assert np.array_equal(xh.view(np.uint32), ref.view(np.uint32))
    finally:
        a.close()


def test_moe_layer_deterministic(O, tglib):
    gpu_note("determinism")
    from tinygiant_amd.moe import MoEBlock
    H, I, E, k = 2048, 768, 128, 8
    from tinygiant_amd.arena import HBMExpertArena
    a = HBMExpertArena(1, E, H, I, k)
    try:
        a.synth_layer(0, seed=1)
        x = dev(O.synth_normal(1, O.stream_id(0, 0, 4), 1.0, 8 * H).reshape(8, H))
        blk = MoEBlock(a)
        r1 = host(blk.forward(0, x))
        r2 = host(blk.forward(0, x))
        assert np.array_equal(r1.view(np.uint32), r2.view(np.uint32))
    finally:
        a.close()
