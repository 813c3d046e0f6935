"""Q4_0 expert-contiguous cache files (the layout contract of the arena).

Mirrors tinygiant/relayout.py's q4 output for ggml type 2 (Q4_0, 18 bytes
per 32 weights): per layer one file layer_NNN.q4.bin holding experts in id
order, each expert gate | up | down, and index.json recording every
expert's offset and sizes (relayout.py:142-157, 276-299).  The reference
derives in_dim from Q4_K super-blocks (relayout.py:101-102); for Q4_0 a row
of in_dim weights is in_dim / 32 blocks of 18 bytes.  The router of each
layer is stored next to it as router_NNN.f32.bin ([n_experts x embed_dim]
fp32), and, when given, its FFN norm weight as norm_NNN.f32.bin
([embed_dim] fp32); the reference reads both from the GGUF
(engine.py:103-117).
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

MAGIC = "NWSMOE01"           # relayout.py:16
GGML_Q4_0 = 2
Q40_BLOCK_BYTES = 18
QK = 32
EXPERT_KEYS = ["gate", "up", "down"]


def q40_tensor_bytes(out_dim: int, in_dim: int) -> int:
    if in_dim % QK:
        raise ValueError("in_dim must be a multiple of 32 for Q4_0")
    return out_dim * (in_dim // QK) * Q40_BLOCK_BYTES


def expert_sizes(embed_dim: int, inter_dim: int) -> dict:
    return {"gate": q40_tensor_bytes(inter_dim, embed_dim),
            "up": q40_tensor_bytes(inter_dim, embed_dim),
            "down": q40_tensor_bytes(embed_dim, inter_dim)}


def write_layer(out_dir, layer: int, experts: list, router: np.ndarray, norm=None) -> dict:
    """experts: list of dicts {gate, up, down} of uint8 arrays (relayout
    order); norm: the layer's FFN norm weight or None.  Returns the layer's
    index entry."""
    out_dir = Path(out_dir)
    fname = f"layer_{layer:03d}.q4.bin"
    offsets = {}
    cur = 0
    with open(out_dir / fname, "wb") as f:
        for e, ex in enumerate(experts):
            sizes = {}
            start = cur
            for k in EXPERT_KEYS:
                b = np.ascontiguousarray(ex[k], dtype=np.uint8).tobytes()
                f.write(b)
                sizes[k] = len(b)
                cur += len(b)
            offsets[str(e)] = {"offset": start, "sizes": sizes}
    rname = f"router_{layer:03d}.f32.bin"
    np.ascontiguousarray(router, dtype=np.float32).tofile(out_dir / rname)
    entry = {"file": fname, "router_file": rname, "total_bytes": cur, "expert_offsets": offsets,
             "tensor_formats": {k: "q4_0" for k in EXPERT_KEYS}}
    if norm is not None:
        nname = f"norm_{layer:03d}.f32.bin"
        np.ascontiguousarray(norm, dtype=np.float32).tofile(out_dir / nname)
        entry["norm_file"] = nname
    return entry


def split_layer_bytes(data: np.ndarray, n_experts: int, embed_dim: int, inter_dim: int) -> list:
    sz = expert_sizes(embed_dim, inter_dim)
    eb = sum(sz.values())
    if data.size != eb * n_experts:
        raise ValueError("layer bytes do not match the shape")
    out = []
    for e in range(n_experts):
        base = e * eb
        g = data[base:base + sz["gate"]]
        u = data[base + sz["gate"]:base + sz["gate"] + sz["up"]]
        d = data[base + sz["gate"] + sz["up"]:base + eb]
        out.append({"gate": g, "up": u, "down": d})
    return out


def write_cache(out_dir, layers: list, routers: list, n_experts_used: int, model: str = "synthetic",
                norms=None) -> dict:
    """Write a full Q4_0 cache: layers = list of per-layer byte arrays,
    routers their [n_experts x embed_dim] fp32 routers, norms (optional)
    their FFN norm weights."""
    out_dir = Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    E, H = np.asarray(routers[0]).shape
    I = None
    per_expert = len(layers[0]) // E
    # per_expert = 3 * I * H / 32 * 18  ->  I = per_expert / (3 * H / 32 * 18)
    I = per_expert // (3 * (H // QK) * Q40_BLOCK_BYTES)
    index = {"magic": MAGIC, "version": 3, "model": model, "n_layers": len(layers), "n_experts": E,
             "n_experts_used": n_experts_used, "embed_dim": H, "inter_dim": I, "dtype": "q4_0",
             "q4_sizes": {"gate": {"out_dim": I, "in_dim": H}, "up": {"out_dim": I, "in_dim": H},
                          "down": {"out_dim": H, "in_dim": I}},
             "tensor_formats": {k: "q4_0" for k in EXPERT_KEYS}, "layers": {}}
    for L, (data, router) in enumerate(zip(layers, routers)):
        experts = split_layer_bytes(np.asarray(data, dtype=np.uint8), E, H, I)
        index["layers"][str(L)] = write_layer(out_dir, L, experts, router,
                                              None if norms is None else norms[L])
    (out_dir / "index.json").write_text(json.dumps(index, indent=2))
    return index
