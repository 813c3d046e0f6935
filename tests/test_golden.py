"""The oracle against the committed golden fixtures (tests/golden/, written by
tests/golden/make_golden.py): for seeds 0, 1, 2 at H=256, I=64, E=16, k=4, one
Q4_0 x Q8_0 block, one row dot, one expert forward and one MoE layer for one
token, and one full Qwen3-30B-A3B-shaped layer (outputs as a SHA-256 plus every
64th row).  Every value is compared bit for bit, so any change of the
generator, a format or an operation order shows up here first."""
import hashlib
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "moe_q40_golden.npz")


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def text(a):
    return bytes(np.asarray(a, np.uint8)).decode()


def bits(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32)).view(np.uint32)


@pytest.fixture(scope="module")
def G():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_small_layer_golden(O, G, seed):
    H, I, E, k = 256, 64, 16, 4
    layer, router = O.synth_layer(seed, 0, H, I, E)
    x = O.synth_normal(seed, O.stream_id(0, 0, 4), 1.0, H).reshape(1, H)
    assert text(G[f"s{seed}_in_sha"]) == sha(layer) + sha(router) + sha(x), "generator changed"
    out, idx, w, xq = O.moe_layer(layer, router, H, I, E, k, x)
    assert np.array_equal(xq[0], G[f"s{seed}_xq"])
    assert np.array_equal(idx[0], G[f"s{seed}_idx"])
    assert np.array_equal(bits(w[0]), G[f"s{seed}_w"])
    assert np.array_equal(bits(out[0]), G[f"s{seed}_out"])
    eb = O.expert_bytes(H, I)
    e0 = int(G[f"s{seed}_expert_id"][0])
    assert e0 == int(idx[0, 0])
    ex = layer[e0 * eb:(e0 + 1) * eb]
    ef = O.expert(ex, H, I, xq[0])
    for part in ("gate", "up", "down"):
        assert np.array_equal(bits(ef[part]), G[f"s{seed}_expert_{part}"]), part
    assert np.array_equal(ef["hq"], G[f"s{seed}_expert_hq"])
    nb = H // 32
    row0 = ex[:nb * 18]
    assert np.array_equal(bits([O.row_dot(row0, xq[0], nb)]), G[f"s{seed}_row_dot"])
    assert np.array_equal(O.block_sums(row0[:18], 1, 32, xq[0][:34]).ravel(), G[f"s{seed}_block_sum"])


def test_full_30b_layer_golden(O, G):
    H, I, E, k = 2048, 768, 128, 8
    layer, router = O.synth_layer(7, 0, H, I, E)
    x = O.synth_normal(7, O.stream_id(0, 0, 4), 1.0, H).reshape(1, H)
    assert text(G["full_in_sha"]) == sha(layer) + sha(router) + sha(x), "generator changed"
    out, idx, w, xq = O.moe_layer(layer, router, H, I, E, k, x)
    assert text(G["full_xq_sha"]) == sha(xq[0])
    assert np.array_equal(idx[0], G["full_idx"])
    assert np.array_equal(bits(w[0]), G["full_w"])
    assert np.array_equal(bits(out[0][::64]), G["full_out_rows"])
    assert text(G["full_out_sha"]) == sha(bits(out[0]))
