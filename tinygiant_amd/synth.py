"""Synthetic workload streams (counter-based, generated on the device).

Every synthetic tensor is one counter stream of the library's generator
(tg_synth_normal_dev, tg_arena_synth_layer): SplitMix64 keyed by (seed,
stream), one N(0, 1) draw per element, so a tensor's bytes depend only on
(seed, stream, index) and not on how or where they are generated.
"""
from __future__ import annotations

import numpy as np

KIND_GATE, KIND_UP, KIND_DOWN, KIND_ROUTER, KIND_TOKENS = 0, 1, 2, 3, 4


def stream_id(layer: int, index: int, kind: int) -> int:
    """Stream of one tensor: kind 0 gate, 1 up, 2 down (index = expert),
    3 router, 4 activations (index = token batch)."""
    return ((layer & 0xFFFF) << 40) | ((index & 0xFFFFFF) << 8) | (kind & 0xFF)


def zipf_router_bias(n_experts: int, tau: float = 0.54) -> np.ndarray:
    """Per-expert logit offsets -tau * ln(e + 1).  Added along a direction
    that every token shares, they make expert popularity follow a power law;
    with router noise of std ~0.9 (N(0, 0.02) weights, H = 2048) tau = 0.54
    gives a rank-frequency exponent of ~1.1 for top-8."""
    return (-tau * np.log(np.arange(1, n_experts + 1))).astype(np.float32)


def fit_zipf_exponent(idx: np.ndarray, n_experts: int) -> float:
    """Least-squares slope of log frequency against log rank of the experts
    chosen in idx (any shape)."""
    cnt = np.bincount(np.asarray(idx).ravel(), minlength=n_experts).astype(np.float64)
    f = np.sort(cnt)[::-1]
    r = np.arange(1, n_experts + 1)
    m = f > 0
    if m.sum() < 2:
        return float("nan")
    return float(-np.polyfit(np.log(r[m]), np.log(f[m]), 1)[0])


def zipf_skew(rng: np.random.Generator, n_experts: int, embed_dim: int, sigma: float = 0.02):
    """Zipf(1.1)-skewed routing for one layer fed tokens x = N(0, 1) + shift.

    Returns (router, shift): router = N(0, sigma) plus, along a unit
    direction u that every token shares, the per-expert offsets of
    zipf_router_bias scaled to the logit noise; shift = c u with
    c = sqrt(H) / 2 is the component each token carries along u.  The
    reference's router has no bias term (engine.py:231), so the skew lives
    in the weights and the activations."""
    H, E = embed_dim, n_experts
    u = rng.standard_normal(H)
    u /= np.linalg.norm(u)
    c = 0.5 * np.sqrt(H)
    rms = np.sqrt(1.0 + c * c / H)
    noise_std = sigma * np.sqrt(H) / rms
    bias = zipf_router_bias(E, 0.54 * noise_std / 0.905)
    router = (rng.standard_normal((E, H)) * sigma).astype(np.float32)
    router += (bias[:, None] * (rms / c) * u[None, :]).astype(np.float32)
    return router, (c * u).astype(np.float32)
