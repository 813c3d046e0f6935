"""All-experts-resident HBM arena: the MI355X replacement of ExpertCache.

The reference keeps experts in per-layer files (tinygiant/relayout.py:142-157)
and serves them through mmap views, optional mlock pinning and the OS page
cache (tinygiant/cache.py:14-160).  On one MI355X every expert of the model
fits in HBM (Qwen3-30B-A3B Q4_0: 16.3 GB of 288 GB), so the three tiers
collapse into one device allocation.  Per-expert offsets and gate/up/down
sizes are the relayout file's, and get() answers with the same keys the
reference's cache does.
"""
from __future__ import annotations

import ctypes
import json
from pathlib import Path

import numpy as np

from . import _lib
from ._lib import call, require_lib

EXPERT_KEYS_ORDER = ["gate", "up", "down"]  # tinygiant/_constants.py:13


class HBMExpertArena:
    """Device-resident experts and routers for n_layers MoE layers."""

    def __init__(self, n_layers: int, n_experts: int, embed_dim: int, inter_dim: int, top_k: int = 8):
        lib = require_lib()
        ptr = lib.tg_arena_create(n_layers, n_experts, embed_dim, inter_dim, top_k)
        if not ptr:
            raise _lib.TinyGiantError("tg_arena_create", -1, lib.tg_last_error().decode())
        self._ptr = ptr
        self.n_layers = n_layers
        self.n_experts = n_experts
        self.embed_dim = embed_dim
        self.inter_dim = inter_dim
        self.top_k = top_k
        self.expert_bytes = lib.tg_arena_expert_bytes(ptr)
        self.layer_bytes = lib.tg_arena_layer_bytes(ptr)
        self.hits = 0
        self.access_counts: dict = {}

    # ------------------------------------------------------------ lifecycle
    @property
    def handle(self) -> int:
        if not self._ptr:
            raise ValueError("arena is closed")
        return self._ptr

    def close(self) -> None:
        if getattr(self, "_ptr", None):
            require_lib().tg_arena_destroy(self._ptr)
            self._ptr = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass

    # ------------------------------------------------------------ decode path
    DECODE_AUTO, DECODE_PER_LAYER, DECODE_FUSED, DECODE_ROUTED = 0, 2, 3, 4

    def set_decode_path(self, path: int) -> None:
        """One-token calls.  ROUTED: one launch per layer that also routes
        (from router partial sums the layer before it leaves, plus one
        prologue launch per call); FUSED: per layer a routing kernel and
        one launch for gate/up and down; PER_LAYER: routing, gate/up and
        down as three kernels; AUTO: ROUTED, else FUSED, else PER_LAYER, as
        the shape allows.  ROUTED and FUSED need every block of their launch
        resident at once: run nothing else on the device beside them."""
        call("tg_arena_set_decode_path", self.handle, int(path))

    def set_graphs(self, on: bool) -> None:
        """Stack calls launched layer by layer (False, the default) or
        replayed as a HIP graph captured on the first call with the same x,
        token count, layer range and eps (True).  Same bytes either way."""
        call("tg_arena_set_graphs", self.handle, int(bool(on)))

    BATCH_AUTO, BATCH_GROUPED, BATCH_PER_TOKEN, BATCH_GROUPED_DOT = 0, 1, 2, 3

    def set_batch_path(self, path: int) -> None:
        """GROUPED: tokens grouped by expert, each selected expert read once
        per layer, on int8 MFMA tiles; GROUPED_DOT: the same grouping on
        packed int8 dot instructions; PER_TOKEN: every token reads its own
        experts; AUTO: GROUPED for two or more tokens."""
        call("tg_arena_set_batch_path", self.handle, int(path))

    def status(self) -> None:
        """Wait for the device; raise if an earlier asynchronous call failed
        on the device (a hand-off poll that ran out of tries)."""
        call("tg_arena_status", self.handle)

    # ------------------------------------------------------------ contents
    def load_layer(self, layer: int, data) -> None:
        """Upload one relayout layer file's bytes (bytes or uint8 array)."""
        buf = np.frombuffer(data, dtype=np.uint8) if isinstance(data, (bytes, bytearray, memoryview)) \
            else np.ascontiguousarray(data, dtype=np.uint8)
        call("tg_arena_load_layer", self.handle, layer, buf.ctypes.data, buf.size)

    def load_router(self, layer: int, router: np.ndarray) -> None:
        r = np.ascontiguousarray(router, dtype=np.float32)
        call("tg_arena_load_router", self.handle, layer, r.ctypes.data, r.size)

    def load_norm(self, layer: int, norm: np.ndarray) -> None:
        """Upload one layer's FFN norm weight [H] (engine.py:229-230's
        ffn_norms[i]); until then a layer runs on a unit weight."""
        g = np.ascontiguousarray(norm, dtype=np.float32)
        call("tg_arena_load_norm", self.handle, layer, g.ctypes.data, g.size)

    def read_layer(self, layer: int) -> np.ndarray:
        out = np.empty(self.layer_bytes, dtype=np.uint8)
        call("tg_arena_read_layer", self.handle, layer, out.ctypes.data, out.size)
        return out

    def read_expert(self, layer: int, expert: int) -> np.ndarray:
        """One expert's gate | up | down bytes in the relayout layout."""
        out = np.empty(self.expert_bytes, dtype=np.uint8)
        call("tg_arena_read_expert", self.handle, layer, expert, out.ctypes.data, out.size)
        return out

    def synth_layer(self, layer: int, seed: int, sigma: float = 0.02) -> None:
        """Fill a layer with the synthetic N(0, sigma) Q4_0 workload on the GPU."""
        call("tg_arena_synth_layer", self.handle, layer, int(seed), float(sigma))

    def expert_offset(self, expert: int) -> dict:
        """index.json-style entry: {"offset", "sizes": {gate, up, down}}."""
        off, g, u, d = (ctypes.c_size_t() for _ in range(4))
        call("tg_arena_expert_offset", self.handle, expert, ctypes.byref(off), ctypes.byref(g),
             ctypes.byref(u), ctypes.byref(d))
        return {"offset": off.value, "sizes": {"gate": g.value, "up": u.value, "down": d.value}}

    def get(self, layer: int, expert: int) -> dict:
        """Lookup with ExpertCache.get's bookkeeping (cache.py:154-160); the
        weights stay on the device, so the answer is their location."""
        if not (0 <= layer < self.n_layers and 0 <= expert < self.n_experts):
            raise KeyError((layer, expert))
        key = (layer, expert)
        self.access_counts[key] = self.access_counts.get(key, 0) + 1
        self.hits += 1
        info = self.expert_offset(expert)
        info["layer"] = layer
        info["_formats"] = {k: "q4_0" for k in EXPERT_KEYS_ORDER}
        return info

    # ------------------------------------------------------------ loaders
    @classmethod
    def from_cache_dir(cls, cache_dir, top_k: int | None = None) -> "HBMExpertArena":
        """Load a Q4_0 relayout cache (index.json + layer_NNN.q4.bin +
        router_NNN.f32.bin [+ norm_NNN.f32.bin]) written by
        tinygiant_amd.relayout."""
        cache_dir = Path(cache_dir)
        index = json.loads((cache_dir / "index.json").read_text())
        if index.get("dtype") != "q4_0":
            raise ValueError(f"cache dtype {index.get('dtype')!r} is not q4_0")
        layers = sorted(int(k) for k in index["layers"])
        if layers != list(range(len(layers))):
            raise ValueError("cache must hold layers 0..n-1")
        a = cls(len(layers), index["n_experts"], index["embed_dim"], index["inter_dim"],
                top_k or index["n_experts_used"])
        for L in layers:
            info = index["layers"][str(L)]
            for e in range(a.n_experts):
                ref = info["expert_offsets"][str(e)]
                if ref != a.expert_offset(e):
                    raise ValueError(f"layer {L} expert {e}: offsets {ref} differ from the arena's")
            data = np.fromfile(cache_dir / info["file"], dtype=np.uint8)
            a.load_layer(L, data)
            router = np.fromfile(cache_dir / info["router_file"], dtype=np.float32)
            a.load_router(L, router)
            if "norm_file" in info:
                a.load_norm(L, np.fromfile(cache_dir / info["norm_file"], dtype=np.float32))
        return a
