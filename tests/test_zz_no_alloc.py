"""tg_moe_layer_q40_noalloc_dev (the layer call that allocates nothing: its
scratch is a fixed device array per GPU) against tg_moe_layer_q40_dev, the
entry point it mirrors, through the C-ABI: bit for bit, on consecutive
calls whose token count shrinks (the array keeps the last call's contents),
on the one-token routed path and the grouped path, replays of a captured
call between direct calls of other shapes and token counts, plus the size
limit."""
import ctypes

import numpy as np
import pytest

from tests.conftest import gpu_note

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def bits(t):
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint32)


def layer_call(lib, name, a, layer, x, T, k):
    out = torch.empty_like(x)
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    rc = getattr(lib, name)(a.handle, layer, x.data_ptr(), out.data_ptr(), T, idx.data_ptr(), w.data_ptr(),
                            ctypes.c_float(1e-6), st)
    assert rc == 0, lib.tg_last_error()
    return out, idx, w


@pytest.mark.parametrize("H,I,E,k,Ts", [(512, 96, 32, 8, (40, 1, 3, 1)), (2048, 768, 128, 8, (64, 1))])
def test_noalloc_layer_matches_dev_entry(O, tglib, H, I, E, k, Ts):
    from tinygiant_amd.arena import HBMExpertArena
    a = HBMExpertArena(2, E, H, I, k)
    try:
        rng = np.random.default_rng(H + I)
        for l in range(2):
            lb, r = O.synth_layer(81, l, H, I, E)
            a.load_layer(l, lb)
            a.load_router(l, r)
            a.load_norm(l, (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32))
        for rep, T in enumerate(Ts):
            layer = rep % 2
            gpu_note(f"no-alloc layer H={H} T={T} layer={layer} call {rep}")
            x = torch.from_numpy(O.synth_normal(82, O.stream_id(layer, rep, 4), 1.0, T * H).reshape(T, H)).cuda()
            o1, i1, w1 = layer_call(tglib, "tg_moe_layer_q40_noalloc_dev", a, layer, x, T, k)
            o2, i2, w2 = layer_call(tglib, "tg_moe_layer_q40_dev", a, layer, x, T, k)
            assert np.array_equal(bits(i1), bits(i2))
            assert np.array_equal(bits(w1), bits(w2))
            assert np.array_equal(bits(o1), bits(o2)), f"call {rep} (T={T})"
        a.status()
    finally:
        a.close()


def test_noalloc_graph_replays_between_other_shapes(O, tglib):
    """A one-token no-alloc call captured in a HIP graph, replayed after
    direct no-alloc calls of another shape and of another token count (which
    leave other tagged words in the array): every replay equals the direct
    tg_moe_layer_q40_dev call bit for bit (the array's header decides on the
    device whether the words must be cleared)."""
    from tinygiant_amd.arena import HBMExpertArena
    k = 8
    A = HBMExpertArena(1, 128, 2048, 768, k)
    B = HBMExpertArena(1, 32, 512, 96, k)
    try:
        A.synth_layer(0, 31)
        B.synth_layer(0, 32)
        xa = torch.from_numpy(O.synth_normal(33, O.stream_id(0, 0, 4), 1.0, 2048).reshape(1, 2048)).cuda()
        ref, ridx, rw = layer_call(tglib, "tg_moe_layer_q40_dev", A, 0, xa, 1, k)
        ref_b = bits(ref)
        gpu_note("no-alloc call captured (H=2048, T=1)")
        out = torch.empty_like(xa)
        idx = torch.empty((1, k), dtype=torch.int32, device="cuda")
        w = torch.empty((1, k), dtype=torch.float32, device="cuda")
        g = torch.cuda.CUDAGraph()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, capture_error_mode="thread_local"):
            st = torch.cuda.current_stream().cuda_stream
            rc = tglib.tg_moe_layer_q40_noalloc_dev(A.handle, 0, xa.data_ptr(), out.data_ptr(), 1, idx.data_ptr(),
                                                    w.data_ptr(), ctypes.c_float(1e-6), st)
        assert rc == 0, tglib.tg_last_error()
        between = [(B, 512, 3), (A, 2048, 5), (B, 512, 1), (A, 2048, 1)]
        for rep, (arena, H, T) in enumerate(between):
            gpu_note(f"  direct no-alloc call H={H} T={T}, then replay {rep}")
            x = torch.from_numpy(O.synth_normal(34, O.stream_id(0, rep, 4), 1.0, T * H).reshape(T, H)).cuda()
            o1, _, _ = layer_call(tglib, "tg_moe_layer_q40_noalloc_dev", arena, 0, x, T, k)
            o2, _, _ = layer_call(tglib, "tg_moe_layer_q40_dev", arena, 0, x, T, k)
            assert np.array_equal(bits(o1), bits(o2)), f"direct call {rep}"
            out.fill_(0.0)
            g.replay()
            assert np.array_equal(bits(out), ref_b), f"replay {rep}"
            assert np.array_equal(bits(idx), bits(ridx)) and np.array_equal(bits(w), bits(rw))
        del g
        A.status()
    finally:
        A.close()
        B.close()


def test_noalloc_layer_rejects_oversize(O, tglib):
    from tinygiant_amd.arena import HBMExpertArena
    gpu_note("no-alloc layer size limit")
    H, I, E, k, T = 2048, 768, 128, 8, 4096
    a = HBMExpertArena(1, E, H, I, k)
    try:
        x = torch.zeros((T, H), dtype=torch.float32, device="cuda")
        out = torch.empty_like(x)
        rc = tglib.tg_moe_layer_q40_noalloc_dev(a.handle, 0, x.data_ptr(), out.data_ptr(), T, None, None,
                                                ctypes.c_float(1e-6), None)
        assert rc == -1
        msg = tglib.tg_last_error().decode()
        assert "no-alloc" in msg and "at most" in msg, msg
        gpu_note(f"  {msg}")
    finally:
        a.close()
