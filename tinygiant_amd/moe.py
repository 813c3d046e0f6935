"""The MoE block on the GPU: norm -> router -> top-k -> experts -> combine.

Host-side mirror of the reference's per-layer MoE step
(tinygiant/engine.py:229-258):

    normed = rms_norm(x, ffn_norms[i])         engine.py:229-230
    logits = router @ normed                   engine.py:231
    top_k_idx, softmax over the top k          engine.py:232-236
    moe_out = sum_j w_j * expert_j(normed)     engine.py:238-257
    x += moe_out                               engine.py:258

Every step runs in libtinygiant.so's gfx950 kernels on weights resident in
an HBMExpertArena (the layer's norm weight from HBMExpertArena.load_norm);
torch is used only to hold device buffers and name the current stream.
"""
from __future__ import annotations

import numpy as np

from ._lib import call
from .arena import HBMExpertArena

RMS_EPS = 1e-6  # tinygiant/_constants.py:12


def _torch():
    import torch  # torch is plumbing only: device memory and streams
    return torch


def _stream_ptr(tensor) -> int:
    torch = _torch()
    return torch.cuda.current_stream(tensor.device).cuda_stream


def _check_dev(t, dtype, name):
    torch = _torch()
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a CUDA (HIP) tensor")
    if t.dtype != dtype or not t.is_contiguous():
        raise TypeError(f"{name} must be a contiguous {dtype} tensor")


class MoEBlock:
    """One MoE layer (or a stack of them) over an HBMExpertArena."""

    def __init__(self, arena: HBMExpertArena, eps: float = RMS_EPS):
        self.arena = arena
        self.eps = float(eps)

    # ---------------------------------------------------------- device
    def forward(self, layer: int, x, return_routing: bool = False):
        """x: [T, H] float32 CUDA tensor -> moe_out [T, H] (x unchanged)."""
        torch = _torch()
        _check_dev(x, torch.float32, "x")
        a = self.arena
        T = x.numel() // a.embed_dim
        out = torch.empty_like(x)
        idx = torch.empty((T, a.top_k), dtype=torch.int32, device=x.device)
        w = torch.empty((T, a.top_k), dtype=torch.float32, device=x.device)
        call("tg_moe_layer_q40_dev", a.handle, layer, x.data_ptr(), out.data_ptr(), T, idx.data_ptr(),
             w.data_ptr(), self.eps, _stream_ptr(x))
        return (out, idx, w) if return_routing else out

    def step(self, x, layer0: int = 0, n_layers: int | None = None):
        """x <- x + MoE_l(x) for the layers [layer0, layer0 + n_layers), in place."""
        torch = _torch()
        _check_dev(x, torch.float32, "x")
        a = self.arena
        n = a.n_layers - layer0 if n_layers is None else n_layers
        T = x.numel() // a.embed_dim
        call("tg_moe_stack_q40_dev", a.handle, x.data_ptr(), T, layer0, n, self.eps, _stream_ptr(x))
        return x

    def step_trace(self, x, layer0: int = 0, n_layers: int | None = None):
        """One token: x <- x + MoE_l(x) over the layers, in place, with the
        routing of every layer: returns (idx [n, k] int32, w [n, k] float32)."""
        torch = _torch()
        _check_dev(x, torch.float32, "x")
        a = self.arena
        if x.numel() != a.embed_dim:
            raise ValueError("step_trace takes one token")
        n = a.n_layers - layer0 if n_layers is None else n_layers
        idx = torch.empty((n, a.top_k), dtype=torch.int32, device=x.device)
        w = torch.empty((n, a.top_k), dtype=torch.float32, device=x.device)
        call("tg_moe_stack_q40_trace_dev", a.handle, x.data_ptr(), layer0, n, self.eps, idx.data_ptr(),
             w.data_ptr(), _stream_ptr(x))
        return idx, w

    # ---------------------------------------------------------- host
    def forward_host(self, layer: int, x: np.ndarray):
        """Synchronous host-pointer form (the reference's calling convention)."""
        a = self.arena
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, a.embed_dim)
        T = x.shape[0]
        out = np.empty_like(x)
        idx = np.empty((T, a.top_k), np.int32)
        w = np.empty((T, a.top_k), np.float32)
        call("tg_moe_layer_q40", a.handle, layer, x.ctypes.data, out.ctypes.data, T, idx.ctypes.data,
             w.ctypes.data, self.eps)
        return out, idx, w

    def step_host(self, x: np.ndarray, layer0: int = 0, n_layers: int | None = None) -> np.ndarray:
        a = self.arena
        x = np.array(x, dtype=np.float32, copy=True).reshape(-1, a.embed_dim)
        n = a.n_layers - layer0 if n_layers is None else n_layers
        call("tg_moe_stack_q40", a.handle, x.ctypes.data, x.shape[0], layer0, n, self.eps)
        return x
