"""Writes the golden fixtures under tests/golden/ from the C oracle.

The fixtures fix, for seeds 0, 1, 2 at a small layer shape (H=256, I=64, E=16,
k=4) and for one full Qwen3-30B-A3B-shaped layer (H=2048, I=768, E=128, k=8):
one Q4_0 x Q8_0 block, one row dot, one expert forward and one MoE layer for
one token.  Inputs are not stored: they come from the seeded generator
(SplitMix64 + Box-Muller, bit-identical on host and GPU), and the fixture keeps
a SHA-256 of every generated input so a change of the generator is caught.
Floats are stored as their bit patterns (uint32), so comparisons are exact.

Run from the repository root:  python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402

SMALL = dict(H=256, I=64, E=16, k=4)
FULL = dict(H=2048, I=768, E=128, k=8)
SEEDS = (0, 1, 2)
FULL_SEED = 7


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def bits(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32)).view(np.uint32)


def small_case(seed: int) -> dict:
    H, I, E, k = SMALL["H"], SMALL["I"], SMALL["E"], SMALL["k"]
    layer, router = O.synth_layer(seed, 0, H, I, E)
    x = O.synth_normal(seed, O.stream_id(0, 0, 4), 1.0, H).reshape(1, H)
    out, idx, w, xq = O.moe_layer(layer, router, H, I, E, k, x)
    eb = O.expert_bytes(H, I)
    e0 = int(idx[0, 0])
    ex = layer[e0 * eb:(e0 + 1) * eb]
    ef = O.expert(ex, H, I, xq[0])
    nb = H // 32
    row0 = ex[:nb * 18]                      # gate row 0 of the first selected expert
    blk_w, blk_x = row0[:18], xq[0][:34]     # its first block and the first Q8_0 block of x
    return {
        f"s{seed}_in_sha": np.frombuffer((sha(layer) + sha(router) + sha(x)).encode(), np.uint8),
        f"s{seed}_xq": xq[0],
        f"s{seed}_block_sum": O.block_sums(blk_w, 1, 32, blk_x).astype(np.int32).ravel(),
        f"s{seed}_row_dot": bits([O.row_dot(row0, xq[0], nb)]),
        f"s{seed}_expert_id": np.array([e0], np.int32),
        f"s{seed}_expert_gate": bits(ef["gate"]),
        f"s{seed}_expert_up": bits(ef["up"]),
        f"s{seed}_expert_hq": ef["hq"],
        f"s{seed}_expert_down": bits(ef["down"]),
        f"s{seed}_idx": idx[0].astype(np.int32),
        f"s{seed}_w": bits(w[0]),
        f"s{seed}_out": bits(out[0]),
    }


def full_case() -> dict:
    H, I, E, k = FULL["H"], FULL["I"], FULL["E"], FULL["k"]
    layer, router = O.synth_layer(FULL_SEED, 0, H, I, E)
    x = O.synth_normal(FULL_SEED, O.stream_id(0, 0, 4), 1.0, H).reshape(1, H)
    out, idx, w, xq = O.moe_layer(layer, router, H, I, E, k, x)
    return {
        "full_in_sha": np.frombuffer((sha(layer) + sha(router) + sha(x)).encode(), np.uint8),
        "full_out_sha": np.frombuffer(sha(bits(out[0])).encode(), np.uint8),
        "full_out_rows": bits(out[0][::64]),
        "full_xq_sha": np.frombuffer(sha(xq[0]).encode(), np.uint8),
        "full_idx": idx[0].astype(np.int32),
        "full_w": bits(w[0]),
    }


def main() -> int:
    data = {}
    for s in SEEDS:
        data.update(small_case(s))
    data.update(full_case())
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "moe_q40_golden.npz")
    np.savez_compressed(path, **data)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(data)} arrays)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
