"""ctypes + numpy front end of the C oracle (oracle/tg_oracle.c).

TEST INFRASTRUCTURE ONLY: the checker that tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg compare the GPU path against.  Functions
take and return numpy arrays; byte buffers are uint8 arrays in the
reference's on-disk layout (Q4_0 18-byte blocks, expert = gate|up|down,
layer = experts back to back, tinygiant/relayout.py:142-157).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libtg_oracle.so"

QK = 32
Q40_BYTES = 18
Q80_BYTES = 34

_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_U64 = ctypes.c_uint64
_SZ = ctypes.c_size_t


def build() -> Path:
    """Compile the oracle with its Makefile (host compiler only)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        alt = os.environ.get("TG_ORACLE_LIB")  # a sanitizer build of the same source (tests/test_sanitizers.py)
        if alt:
            L = ctypes.CDLL(alt)
        else:
            if not LIB_PATH.exists():
                build()
            L = ctypes.CDLL(str(LIB_PATH))
        sigs = {
            "tgo_f16_to_f32": (_F, [ctypes.c_uint16]),
            "tgo_f16_to_f32_n": (None, [_P, _SZ, _P]),
            "tgo_f32_to_f16": (ctypes.c_uint16, [_F]),
            "tgo_expf": (_F, [_F]),
            "tgo_ln_unit": (_F, [_F]),
            "tgo_cos2pi": (_F, [_F]),
            "tgo_splitmix64": (_U64, [_U64]),
            "tgo_stream_key": (_U64, [_U64, _U64]),
            "tgo_normal_at": (_F, [_U64, _U64]),
            "tgo_synth_normal": (None, [_U64, _U64, _F, _SZ, _P]),
            "tgo_synth_q40": (None, [_U64, _U64, _F, _I, _I, _P]),
            "tgo_quantize_q4_0": (None, [_P, _SZ, _P]),
            "tgo_dequantize_q4_0": (None, [_P, _SZ, _P]),
            "tgo_quantize_q8_0": (None, [_P, _SZ, _P]),
            "tgo_dequantize_q8_0": (None, [_P, _SZ, _P]),
            "tgo_block_dot_q40_q80": (ctypes.c_int32, [_P, _P]),
            "tgo_block_sums": (None, [_P, _I, _I, _P, _P]),
            "tgo_row_dot_q40_q80": (_F, [_P, _P, _I]),
            "tgo_matvec_q40": (None, [_P, _I, _I, _P, _P]),
            "tgo_q40_to_planar": (None, [_P, _I, _I, _P]),
            "tgo_q40_from_planar": (None, [_P, _I, _I, _P]),
            "tgo_sumsq": (_F, [_P, _I]),
            "tgo_rms_scale": (_F, [_P, _I, _F]),
            "tgo_router_dot": (_F, [_P, _P, _I]),
            "tgo_router_logits": (None, [_P, _I, _I, _P, _F, _P]),
            "tgo_topk_softmax": (None, [_P, _I, _I, _P, _P]),
            "tgo_silu_mul": (_F, [_F, _F]),
            "tgo_expert_q40": (None, [_P, _I, _I, _P, _P, _P, _P, _P, _P]),
            "tgo_router_dot_g": (_F, [_P, _P, _P, _I]),
            "tgo_moe_layer_q40": (None, [_P, _P, _P, _I, _I, _I, _I, _F, _P, _I, _P, _P, _P, _P]),
            "tgo_moe_stack_q40": (None, [_P, _P, _P, _I, _I, _I, _I, _I, _F, _P, _I, _P]),
            "tgo_group_by_expert": (_I, [_P, _I, _I, _I, _P, _P, _P]),
            "tgo_quantize_q8k": (None, [_P, _P, _I]),
            "tgo_scale_min_k4": (None, [_I, _P, _P, _P]),
            "tgo_dot_q4k_q8": (_F, [_P, _P, _I]),
            "tgo_matmul_q4k": (None, [_P, _P, _P, _I, _I]),
            "tgo_dot_q6k_q8": (_F, [_P, _P, _I]),
            "tgo_matmul_q6k": (None, [_P, _P, _P, _I, _I]),
            "tgo_matvec_f16": (None, [_P, _P, _P, _I, _I]),
            "tgo_matvec_f32": (None, [_P, _P, _P, _I, _I]),
            "tgo_rms_norm": (None, [_P, _P, _P, _I, _F]),
            "tgo_expert_forward_mixed": (None, [_P, _P, _P, _I, _P, _P, _F, _I, _I]),
            "tgo_moe_forward_q4k": (None, [_P, _P, _I, _P, _P, _I, _I]),
            "tgo_matmul_q4k_scalar": (None, [_P, _P, _P, _I, _I]),
            "tgo_dequant_q4k_block": (None, [_P, _P]),
            "tgo_dequant_q6k_block": (None, [_P, _P]),
            "tgo_rope": (None, [_P, _I, _I, _P, _P, _I]),
            "tgo_attention_decode": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _P, _P, _P, _P,
                                             _I, _I, _I, _I, _I]),
            "tgo_attention_decode_q4": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _P, _P, _P, _P,
                                                _I, _I, _I, _I, _I]),
            "tgo_transformer_layer": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _P, _P,
                                              _P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _I]),
            "tgo_set_threads": (_I, [_I]),
            "tgo_max_threads": (_I, []),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# Q8_K block (reference q8_block, libtinygiant.c:55-59)
Q8K_DTYPE = np.dtype([("scale", "<f4"), ("sum", "<i4"), ("qs", "i1", (256,))])

# ---------------------------------------------------------------- scalars

def f16_to_f32(h: int) -> float:
    return lib().tgo_f16_to_f32(int(h))


def f16_to_f32_n(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.size, np.float32)
    lib().tgo_f16_to_f32_n(_p(h), h.size, _p(out))
    return out


def f32_to_f16(f: float) -> int:
    return lib().tgo_f32_to_f16(float(f))


def expf(x: float) -> float:
    return lib().tgo_expf(float(x))


# ------------------------------------------------------------- synthetic

def stream_id(layer: int, expert: int, kind: int) -> int:
    """Counter stream of one tensor: kind 0 gate, 1 up, 2 down, 3 router,
    4 activations (expert = token batch id)."""
    return ((layer & 0xFFFF) << 40) | ((expert & 0xFFFFFF) << 8) | (kind & 0xFF)


def synth_normal(seed: int, stream: int, sigma: float, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().tgo_synth_normal(seed, stream, sigma, n, _p(out))
    return out


def synth_q40(seed: int, stream: int, sigma: float, rows: int, cols: int) -> np.ndarray:
    out = np.empty(rows * (cols // QK) * Q40_BYTES, dtype=np.uint8)
    lib().tgo_synth_q40(seed, stream, sigma, rows, cols, _p(out))
    return out


def synth_layer(seed: int, layer: int, H: int, I: int, E: int, sigma: float = 0.02):
    """One layer: Q4_0 experts in relayout order and the fp32 router."""
    parts = []
    for e in range(E):
        parts.append(synth_q40(seed, stream_id(layer, e, 0), sigma, I, H))
        parts.append(synth_q40(seed, stream_id(layer, e, 1), sigma, I, H))
        parts.append(synth_q40(seed, stream_id(layer, e, 2), sigma, H, I))
    experts = np.concatenate(parts)
    router = synth_normal(seed, stream_id(layer, 0, 3), sigma, E * H).reshape(E, H)
    return experts, router


def expert_bytes(H: int, I: int) -> int:
    return 3 * I * (H // QK) * Q40_BYTES


# ---------------------------------------------------------------- formats

def quantize_q4_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(x.size // QK * Q40_BYTES, dtype=np.uint8)
    lib().tgo_quantize_q4_0(_p(x), x.size, _p(out))
    return out


def dequantize_q4_0(q: np.ndarray, n: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    lib().tgo_dequantize_q4_0(_p(q), n, _p(out))
    return out


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(x.size // QK * Q80_BYTES, dtype=np.uint8)
    lib().tgo_quantize_q8_0(_p(x), x.size, _p(out))
    return out


def dequantize_q8_0(q: np.ndarray, n: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    lib().tgo_dequantize_q8_0(_p(q), n, _p(out))
    return out


def block_sums(W: np.ndarray, rows: int, cols: int, xq: np.ndarray) -> np.ndarray:
    out = np.empty((rows, cols // QK), dtype=np.int32)
    lib().tgo_block_sums(_p(np.ascontiguousarray(W)), rows, cols, _p(np.ascontiguousarray(xq)), _p(out))
    return out


def row_dot(wrow: np.ndarray, xq: np.ndarray, nb: int) -> float:
    return lib().tgo_row_dot_q40_q80(_p(np.ascontiguousarray(wrow)), _p(np.ascontiguousarray(xq)), nb)


def matvec_q40(W: np.ndarray, rows: int, cols: int, xq: np.ndarray) -> np.ndarray:
    out = np.empty(rows, dtype=np.float32)
    lib().tgo_matvec_q40(_p(np.ascontiguousarray(W)), rows, cols, _p(np.ascontiguousarray(xq)), _p(out))
    return out


def to_planar(aos: np.ndarray, rows: int, nb: int) -> np.ndarray:
    out = np.empty(rows * nb * Q40_BYTES, dtype=np.uint8)
    lib().tgo_q40_to_planar(_p(np.ascontiguousarray(aos)), rows, nb, _p(out))
    return out


def from_planar(pl: np.ndarray, rows: int, nb: int) -> np.ndarray:
    out = np.empty(rows * nb * Q40_BYTES, dtype=np.uint8)
    lib().tgo_q40_from_planar(_p(np.ascontiguousarray(pl)), rows, nb, _p(out))
    return out


# ------------------------------------------------------- router / layer

def sumsq(x: np.ndarray) -> float:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return lib().tgo_sumsq(_p(x), x.size)


def rms_scale(x: np.ndarray, eps: float = 1e-6) -> float:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return lib().tgo_rms_scale(_p(x), x.size, eps)


def router_dot(w: np.ndarray, x: np.ndarray) -> float:
    """Un-normalised grouped dot w . x (the logit is this times the norm scale)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    return lib().tgo_router_dot(_p(w), _p(x), w.size)


def router_logits(Wr: np.ndarray, x: np.ndarray, s: float) -> np.ndarray:
    """logits = s * (Wr @ x) in the grouped order, x un-normalised."""
    Wr = np.ascontiguousarray(Wr, dtype=np.float32)
    E, H = Wr.shape
    out = np.empty(E, dtype=np.float32)
    lib().tgo_router_logits(_p(Wr), E, H, _p(np.ascontiguousarray(x, dtype=np.float32)), float(s), _p(out))
    return out


def topk_softmax(logits: np.ndarray, k: int):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    idx = np.empty(k, dtype=np.int32)
    w = np.empty(k, dtype=np.float32)
    lib().tgo_topk_softmax(_p(logits), logits.size, k, _p(idx), _p(w))
    return idx, w


def silu_mul(g: float, u: float) -> float:
    return lib().tgo_silu_mul(float(g), float(u))


def expert(ex: np.ndarray, H: int, I: int, xq: np.ndarray):
    g = np.empty(I, np.float32)
    u = np.empty(I, np.float32)
    h = np.empty(I, np.float32)
    hq = np.empty(I // QK * Q80_BYTES, np.uint8)
    d = np.empty(H, np.float32)
    lib().tgo_expert_q40(_p(np.ascontiguousarray(ex)), H, I, _p(np.ascontiguousarray(xq)),
                         _p(g), _p(u), _p(h), _p(hq), _p(d))
    return dict(gate=g, up=u, h=h, hq=hq, down=d)


def router_dot_g(w: np.ndarray, g, x: np.ndarray) -> float:
    """Grouped dot (w * g) . x, the norm weight folded into the router column."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    if g is None:
        return lib().tgo_router_dot_g(_p(w), None, _p(x), w.size)
    g = np.ascontiguousarray(g, dtype=np.float32)
    return lib().tgo_router_dot_g(_p(w), _p(g), _p(x), w.size)


def moe_layer(layer: np.ndarray, Wr: np.ndarray, H: int, I: int, E: int, k: int,
              x: np.ndarray, eps: float = 1e-6, norm=None):
    """One MoE block over the rows of x; norm is the FFN norm weight (None: unit)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, H)
    T = x.shape[0]
    out = np.empty((T, H), np.float32)
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    xq = np.empty((T, H // QK * Q80_BYTES), np.uint8)
    g = None if norm is None else np.ascontiguousarray(norm, dtype=np.float32).reshape(H)
    lib().tgo_moe_layer_q40(_p(np.ascontiguousarray(layer)), _p(np.ascontiguousarray(Wr, dtype=np.float32)),
                            None if g is None else _p(g), H, I, E, k, eps, _p(x), T, _p(out), _p(idx), _p(w),
                            _p(xq))
    return out, idx, w, xq


def moe_stack(layers, routers, H: int, I: int, E: int, k: int, x: np.ndarray, eps: float = 1e-6, norms=None):
    """x <- x + MoE_l(x) over the layers; returns (x, idx_trace).  norms:
    per-layer FFN norm weights (None: unit)."""
    n = len(layers)
    x = np.array(x, dtype=np.float32, copy=True).reshape(-1, H)
    T = x.shape[0]
    keep = [np.ascontiguousarray(a) for a in layers] + [np.ascontiguousarray(r, dtype=np.float32) for r in routers]
    lp = (ctypes.c_void_p * n)(*[_p(a) for a in keep[:n]])
    rp = (ctypes.c_void_p * n)(*[_p(a) for a in keep[n:]])
    npp = None
    if norms is not None:
        keep += [np.ascontiguousarray(g, dtype=np.float32).reshape(H) for g in norms]
        npp = (ctypes.c_void_p * n)(*[_p(a) for a in keep[2 * n:]])
    trace = np.empty((n, T, k), np.int32)
    lib().tgo_moe_stack_q40(ctypes.cast(lp, ctypes.c_void_p), ctypes.cast(rp, ctypes.c_void_p),
                            None if npp is None else ctypes.cast(npp, ctypes.c_void_p),
                            n, H, I, E, k, eps, _p(x), T, _p(trace))
    return x, trace


def group_by_expert(idx: np.ndarray, E: int):
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    T, k = idx.shape
    counts = np.empty(E, np.int32)
    offsets = np.empty(E + 1, np.int32)
    perm = np.empty(T * k, np.int32)
    uniq = lib().tgo_group_by_expert(_p(idx), T, k, E, _p(counts), _p(offsets), _p(perm))
    return counts, offsets, perm, uniq


def set_threads(n: int) -> int:
    return lib().tgo_set_threads(int(n))


# ---------------------------------------------------------------- legacy

def quantize_q8k(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 256, dtype=Q8K_DTYPE)
    lib().tgo_quantize_q8k(_p(x), _p(out), x.size // 256)
    return out


def scale_min_k4(j: int, scales: np.ndarray):
    sc = ctypes.c_uint8()
    m = ctypes.c_uint8()
    lib().tgo_scale_min_k4(j, _p(np.ascontiguousarray(scales, dtype=np.uint8)), ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


def dot_q4k_q8(q4: np.ndarray, xq: np.ndarray) -> float:
    return lib().tgo_dot_q4k_q8(_p(np.ascontiguousarray(q4)), _p(xq), xq.size)


def matmul_q4k(W: np.ndarray, x: np.ndarray, nrows: int, ncols: int) -> np.ndarray:
    y = np.empty(nrows, np.float32)
    lib().tgo_matmul_q4k(_p(np.ascontiguousarray(W)), _p(np.ascontiguousarray(x, dtype=np.float32)), _p(y), nrows, ncols)
    return y


def dot_q6k_q8(q6: np.ndarray, xq: np.ndarray) -> float:
    return lib().tgo_dot_q6k_q8(_p(np.ascontiguousarray(q6)), _p(xq), xq.size)


def matmul_q6k(W: np.ndarray, x: np.ndarray, nrows: int, ncols: int) -> np.ndarray:
    y = np.empty(nrows, np.float32)
    lib().tgo_matmul_q6k(_p(np.ascontiguousarray(W)), _p(np.ascontiguousarray(x, dtype=np.float32)), _p(y), nrows, ncols)
    return y


def matvec_f16(A: np.ndarray, x: np.ndarray) -> np.ndarray:
    A = np.ascontiguousarray(A, dtype=np.float16)
    y = np.empty(A.shape[0], np.float32)
    lib().tgo_matvec_f16(_p(A), _p(np.ascontiguousarray(x, dtype=np.float32)), _p(y), A.shape[0], A.shape[1])
    return y


def matvec_f32(A: np.ndarray, x: np.ndarray) -> np.ndarray:
    A = np.ascontiguousarray(A, dtype=np.float32)
    y = np.empty(A.shape[0], np.float32)
    lib().tgo_matvec_f32(_p(A), _p(np.ascontiguousarray(x, dtype=np.float32)), _p(y), A.shape[0], A.shape[1])
    return y


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().tgo_rms_norm(_p(x), _p(np.ascontiguousarray(w, dtype=np.float32)), _p(out), x.size, eps)
    return out


def output_head(W: np.ndarray, norm_w: np.ndarray, x: np.ndarray, eps: float = 1e-6):
    """(logits, greedy token) of tinygiant/engine.py:262-266,359: logits =
    W @ rms_norm(x, norm_w) with the product in tg_f32_matvec's order
    (libtinygiant.c:299-318), token = np.argmax(logits) (first index of the
    largest value, NaN largest)."""
    logits = matvec_f32(W, rms_norm(x, norm_w, eps))
    return logits, int(np.argmax(logits))


def expert_forward_mixed(gate, up, down, down_format, x, out, weight, embed, inter):
    lib().tgo_expert_forward_mixed(_p(gate), _p(up), _p(down), down_format,
                                   _p(np.ascontiguousarray(x, dtype=np.float32)), _p(out),
                                   float(weight), embed, inter)
    return out


def moe_forward_q4k(experts, w, x, embed, inter):
    """tg_moe_forward: output zeroed, then every Q4_K expert (gate | up | down
    contiguous) accumulated with its weight, in order."""
    n = len(experts)
    ptrs = (ctypes.c_void_p * n)(*[np.ascontiguousarray(e).ctypes.data for e in experts])
    out = np.empty(embed, np.float32)
    lib().tgo_moe_forward_q4k(ctypes.cast(ptrs, ctypes.c_void_p), _p(np.ascontiguousarray(w, dtype=np.float32)), n,
                              _p(np.ascontiguousarray(x, dtype=np.float32)), _p(out), embed, inter)
    return out


def matmul_q4k_scalar(W: np.ndarray, x: np.ndarray, nrows: int, ncols: int) -> np.ndarray:
    y = np.empty(nrows, np.float32)
    lib().tgo_matmul_q4k_scalar(_p(np.ascontiguousarray(W)), _p(np.ascontiguousarray(x, dtype=np.float32)), _p(y), nrows, ncols)
    return y


def dequant_q4k_block(block: np.ndarray) -> np.ndarray:
    out = np.empty(256, np.float32)
    lib().tgo_dequant_q4k_block(_p(np.ascontiguousarray(block, dtype=np.uint8)), _p(out))
    return out


def dequant_q6k_block(block: np.ndarray) -> np.ndarray:
    out = np.empty(256, np.float32)
    lib().tgo_dequant_q6k_block(_p(np.ascontiguousarray(block, dtype=np.uint8)), _p(out))
    return out


def cpu_count() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


def rope(x: np.ndarray, n_heads: int, head_dim: int, cos_t: np.ndarray, sin_t: np.ndarray, pos: int) -> np.ndarray:
    """apply_rope_inplace on a copy of x (n_heads * head_dim floats)."""
    y = np.array(x, dtype=np.float32, copy=True)
    lib().tgo_rope(_p(y), n_heads, head_dim, _p(np.ascontiguousarray(cos_t, dtype=np.float32)),
                   _p(np.ascontiguousarray(sin_t, dtype=np.float32)), pos)
    return y


def attention_decode(q4, wq, wk, wv, wo, q_norm_w, k_norm_w, kv_k, kv_v, kv_len, kv_max, cos_t, sin_t, x, embed,
                     n_heads, n_kv_heads, head_dim, pos):
    """tg_attention_decode (q4 False: f32 weights) or tg_attention_decode_q4;
    kv_k / kv_v (float32 [n_kv_heads, kv_max, head_dim]) are updated in place.
    Returns the output (embed floats)."""
    out = np.empty(embed, np.float32)
    fn = lib().tgo_attention_decode_q4 if q4 else lib().tgo_attention_decode
    fn(_p(wq), _p(wk), _p(wv), _p(wo), _p(q_norm_w), _p(k_norm_w), _p(kv_k), _p(kv_v), kv_len, kv_max, _p(cos_t),
       _p(sin_t), _p(np.ascontiguousarray(x, dtype=np.float32)), _p(out), embed, n_heads, n_kv_heads, head_dim, pos)
    return out


def transformer_layer(wq, wk, wv, wo, attn_norm_w, q_norm_w, k_norm_w, ffn_norm_w, kv_k, kv_v, kv_len, kv_max,
                      cos_t, sin_t, gates, ups, downs, down_is_f16, expert_w, x, embed, inter, n_heads, n_kv_heads,
                      head_dim, pos):
    """tg_transformer_layer; x (float32, embed) and the caches are updated in place."""
    n = len(gates)
    arr = lambda lst: ctypes.cast((ctypes.c_void_p * n)(*[a.ctypes.data for a in lst]), ctypes.c_void_p)
    dif = np.ascontiguousarray(down_is_f16, dtype=np.int32)
    lib().tgo_transformer_layer(_p(wq), _p(wk), _p(wv), _p(wo), _p(attn_norm_w), _p(q_norm_w), _p(k_norm_w),
                                _p(ffn_norm_w), _p(kv_k), _p(kv_v), kv_len, kv_max, _p(cos_t), _p(sin_t), arr(gates),
                                arr(ups), arr(downs), _p(dif), _p(np.ascontiguousarray(expert_w, dtype=np.float32)),
                                n, _p(x), embed, inter, n_heads, n_kv_heads, head_dim, pos)
    return x
