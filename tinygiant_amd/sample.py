"""Next-token sampling on the GPU: the decode step of tinygiant/engine.py:348-359.

    if temperature > 0:  softmax(logits / T), top-p prefix, np.random.choice
    else:                np.argmax(logits)

Sampler runs that step in libtinygiant.so (tg_sampler_run).  The draw's
uniform comes from the same generator the reference's np.random.choice uses
(numpy's global RandomState unless another is given), one random_sample()
per sampled token and none for greedy tokens, so a seeded run yields the
reference's tokens.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import call, require_lib


class Sampler:
    """Device buffers for one vocabulary; call it once per decode step."""

    def __init__(self, vocab: int):
        lib = require_lib()
        ptr = lib.tg_sampler_create(int(vocab))
        if not ptr:
            raise _lib.TinyGiantError("tg_sampler_create", -1, lib.tg_last_error().decode())
        self._ptr = ptr
        self.vocab = int(vocab)

    def close(self) -> None:
        if getattr(self, "_ptr", None):
            require_lib().tg_sampler_destroy(self._ptr)
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

    def __call__(self, logits, temperature: float, top_p: float, rng=None, u: float | None = None,
                 probs: np.ndarray | None = None) -> int:
        """The next token.  logits: a numpy array (host) or a float32 CUDA
        tensor (read in place) of vocab values.  u: the draw's uniform; by
        default rng.random_sample() (numpy's global RandomState when rng is
        None) when temperature > 0.  probs: optional float32 host array that
        receives the normalised probabilities."""
        if not self._ptr:
            raise ValueError("sampler is closed")
        sample = temperature > 0
        if u is None:
            u = (rng if rng is not None else np.random).random_sample() if sample else 0.0
        on_dev = 0
        if isinstance(logits, np.ndarray):
            host = np.ascontiguousarray(logits, dtype=np.float32)
            if host.size != self.vocab:
                raise ValueError(f"{host.size} logits for a vocabulary of {self.vocab}")
            addr = host.ctypes.data
        else:
            import torch  # device logits: torch is plumbing only
            if not (isinstance(logits, torch.Tensor) and logits.is_cuda and logits.dtype == torch.float32
                    and logits.is_contiguous() and logits.numel() == self.vocab):
                raise TypeError("logits must be a numpy array or a contiguous float32 CUDA tensor of vocab values")
            torch.cuda.current_stream(logits.device).synchronize()
            addr, on_dev = logits.data_ptr(), 1
        pp = None
        if probs is not None:
            if probs.dtype != np.float32 or probs.size != self.vocab or not probs.flags.c_contiguous:
                raise TypeError("probs must be a contiguous float32 array of vocab values")
            pp = probs.ctypes.data
        tok = ctypes.c_int32(-1)
        call("tg_sampler_run", self._ptr, addr, on_dev, float(np.float32(temperature)), float(top_p), float(u),
             ctypes.byref(tok), pp)
        return tok.value
