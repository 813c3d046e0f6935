"""GPU outputs against the committed golden fixtures (tests/golden/), with no
oracle in the loop: weights and tokens are generated on the device from the
fixture's seeds (the device generator is bit-identical to the host one), one
token goes through the MoE layer on every path that serves it, and the
expert ids, weights and outputs must equal the stored bit patterns."""
import hashlib
import os

import numpy as np
import pytest

from tests.conftest import gpu_note

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "moe_q40_golden.npz")
# decode paths (tg_arena_set_decode_path) and batch paths (tg_arena_set_batch_path)
PATHS = {"routed": (4, 0), "fused": (3, 0), "per_layer": (2, 0), "grouped_mfma": (0, 1), "grouped_dot": (0, 3)}


@pytest.fixture(scope="module")
def G():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bits(t):
    torch.cuda.synchronize()
    return np.ascontiguousarray(t.cpu().numpy().astype(np.float32)).view(np.uint32)


def device_token(seed, H):
    from tinygiant_amd._lib import call
    from tinygiant_amd.synth import stream_id
    x = torch.empty((1, H), dtype=torch.float32, device="cuda")
    call("tg_synth_normal_dev", seed, stream_id(0, 0, 4), 1.0, H, x.data_ptr(),
         torch.cuda.current_stream().cuda_stream)
    return x


def run_layer(H, I, E, k, seed, path):
    from tinygiant_amd.arena import HBMExpertArena
    from tinygiant_amd.moe import MoEBlock
    a = HBMExpertArena(1, E, H, I, k)
    try:
        a.synth_layer(0, seed)
        dec, bat = PATHS[path]
        a.set_decode_path(dec)
        a.set_batch_path(bat)
        out, idx, w = MoEBlock(a).forward(0, device_token(seed, H), return_routing=True)
        res = bits(out)[0], idx.cpu().numpy()[0], bits(w)[0]
        a.status()
        return res
    finally:
        a.close()


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_small_layer_golden_gpu(tglib, G, seed, path):
    gpu_note(f"golden small layer seed={seed} path={path}")
    out, idx, w = run_layer(256, 64, 16, 4, seed, path)
    assert np.array_equal(idx, G[f"s{seed}_idx"])
    assert np.array_equal(w, G[f"s{seed}_w"])
    assert np.array_equal(out, G[f"s{seed}_out"])


@pytest.mark.parametrize("path", ["routed", "fused", "per_layer", "grouped_mfma"])
def test_full_30b_layer_golden_gpu(tglib, G, path):
    gpu_note(f"golden 30B layer path={path}")
    out, idx, w = run_layer(2048, 768, 128, 8, 7, path)
    assert np.array_equal(idx, G["full_idx"])
    assert np.array_equal(w, G["full_w"])
    assert np.array_equal(out[::64], G["full_out_rows"])
    assert hashlib.sha256(out.tobytes()).hexdigest() == bytes(G["full_out_sha"]).decode()
