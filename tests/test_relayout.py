"""The Q4_0 cache writer (tinygiant_amd.relayout) against the reference's
cache contract: the layer file layout and index.json keys that
tinygiant/relayout.py:142-157,276-299 writes and tinygiant/cache.py:32-57
reads (per-expert offset, gate/up/down sizes in that order, tensor
formats).  CPU only."""
import json

import numpy as np
import pytest

from tinygiant_amd import relayout


def make(O, L=2, H=256, I=64, E=8, seed=5, with_norm=True):
    rng = np.random.default_rng(seed)
    layers, routers, norms = [], [], []
    for l in range(L):
        lb, r = O.synth_layer(seed, l, H, I, E)
        layers.append(lb)
        routers.append(r)
        norms.append((1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    return layers, routers, (norms if with_norm else None)


def test_index_schema_and_offsets(O, tmp_path):
    H, I, E, k = 256, 64, 8, 4
    layers, routers, norms = make(O, H=H, I=I, E=E)
    index = relayout.write_cache(tmp_path, layers, routers, k, norms=norms)
    on_disk = json.loads((tmp_path / "index.json").read_text())
    assert on_disk == json.loads(json.dumps(index))
    assert on_disk["magic"] == "NWSMOE01" and on_disk["dtype"] == "q4_0"
    assert (on_disk["n_layers"], on_disk["n_experts"], on_disk["n_experts_used"], on_disk["embed_dim"],
            on_disk["inter_dim"]) == (2, E, k, H, I)
    gate = I * (H // 32) * 18
    down = H * (I // 32) * 18
    eb = 2 * gate + down
    assert on_disk["q4_sizes"] == {"gate": {"out_dim": I, "in_dim": H}, "up": {"out_dim": I, "in_dim": H},
                                   "down": {"out_dim": H, "in_dim": I}}
    for L in range(2):
        info = on_disk["layers"][str(L)]
        assert info["file"] == f"layer_{L:03d}.q4.bin"
        assert info["total_bytes"] == E * eb
        assert info["tensor_formats"] == {"gate": "q4_0", "up": "q4_0", "down": "q4_0"}
        data = np.fromfile(tmp_path / info["file"], dtype=np.uint8)
        assert np.array_equal(data, layers[L])
        for e in range(E):
            ent = info["expert_offsets"][str(e)]
            assert ent == {"offset": e * eb, "sizes": {"gate": gate, "up": gate, "down": down}}
            assert list(ent["sizes"]) == ["gate", "up", "down"]  # EXPERT_KEYS_ORDER, cache.py:47
        r = np.fromfile(tmp_path / info["router_file"], dtype=np.float32).reshape(E, H)
        assert np.array_equal(r, routers[L])
        g = np.fromfile(tmp_path / info["norm_file"], dtype=np.float32)
        assert np.array_equal(g, norms[L])


def test_views_like_the_reference_cache(O, tmp_path):
    """Slicing the layer file at each expert's offset with the recorded sizes
    in gate, up, down order (cache.py:41-57) gives that expert's tensors."""
    H, I, E = 256, 64, 8
    layers, routers, _ = make(O, L=1, H=H, I=I, E=E, with_norm=False)
    index = relayout.write_cache(tmp_path, layers, routers, 4)
    info = index["layers"]["0"]
    assert "norm_file" not in info
    mm = np.fromfile(tmp_path / info["file"], dtype=np.uint8)
    parts = relayout.split_layer_bytes(layers[0], E, H, I)
    for e in range(E):
        ent = info["expert_offsets"][str(e)]
        pos = ent["offset"]
        for key in ["gate", "up", "down"]:
            n = ent["sizes"][key]
            assert np.array_equal(mm[pos:pos + n], parts[e][key])
            pos += n


def test_split_rejects_wrong_size():
    with pytest.raises(ValueError):
        relayout.split_layer_bytes(np.zeros(100, np.uint8), 8, 256, 64)
    with pytest.raises(ValueError):
        relayout.q40_tensor_bytes(64, 100)


def test_from_cache_dir_rejects_other_dtypes(tmp_path):
    """The arena loader takes Q4_0 caches only (the reference's own q4_k
    caches go through the legacy entry points); it says so before it needs a
    device."""
    from tinygiant_amd.arena import HBMExpertArena
    (tmp_path / "index.json").write_text(json.dumps({"dtype": "q4_k", "layers": {}}))
    with pytest.raises(ValueError, match="q4_k"):
        HBMExpertArena.from_cache_dir(tmp_path)
