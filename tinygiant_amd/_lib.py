"""ctypes binding of libtinygiant.so (gfx950).

find_library() and load_tinygiant_lib() keep the reference's behaviour
(tinygiant/_lib.py:9-76): the same search order (package directory, then the
directory above it; .dylib before .so), None when no library is found, and
the same argtypes for the thirteen registered symbols, so the reference's
engine binds this library unchanged.  They additionally register the new
Q4_0 entry points declared in include/tinygiant.h.

require_lib() is the strict form used by this package's own host code: it
raises when the library is missing instead of returning None, so nothing in
the MoE path can silently run without the GPU kernels.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

VP = ctypes.c_void_p
CI = ctypes.c_int
CF = ctypes.c_float
SZ = ctypes.c_size_t
U64 = ctypes.c_uint64
CD = ctypes.c_double

# (name, restype, argtypes) of the reference ABI, tinygiant/_lib.py:39-74
LEGACY_SYMBOLS = [
    ("tg_expert_forward", None, [VP, VP, VP, CF, CI, CI]),
    ("tg_expert_forward_mixed", None, [VP, VP, VP, CI, VP, VP, CF, CI, CI]),
    ("tg_matmul_q4k", None, [VP, VP, VP, CI, CI]),
    ("tg_matmul_q6k", None, [VP, VP, VP, CI, CI]),
    ("tg_rms_norm", None, [VP, VP, VP, CI, CF]),
    ("tg_f32_matvec", None, [VP, VP, VP, CI, CI]),
    ("tg_f16_matvec", None, [VP, VP, VP, CI, CI]),
    ("tg_attention_decode", None,
     [VP, VP, VP, VP, VP, VP, VP, VP, CI, CI, VP, VP, VP, VP, CI, CI, CI, CI, CI]),
    ("tg_attention_decode_q4", None,
     [VP, VP, VP, VP, VP, VP, VP, VP, CI, CI, VP, VP, VP, VP, CI, CI, CI, CI, CI]),
    ("tg_prefetch", None, [VP, SZ]),
    ("tg_prefetch_batch", None, [VP, VP, CI]),
    ("tg_mlock", ctypes.c_int, [VP, SZ]),
    ("tg_transformer_layer", None,
     [VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, CI, CI, VP, VP, VP, VP, VP, VP, VP, CI, VP,
      CI, CI, CI, CI, CI, CI]),
]

# exported by csrc/libtinygiant.c but not registered by the reference's _lib.py
UNREGISTERED_SYMBOLS = [
    ("tg_moe_forward", None, [VP, VP, CI, VP, VP, CI, CI]),
    ("tg_matmul_q4k_scalar", None, [VP, VP, VP, CI, CI]),
]

# new entry points (include/tinygiant.h)
NEW_SYMBOLS = [
    ("tg_last_error", ctypes.c_char_p, []),
    ("tg_version", ctypes.c_char_p, []),
    ("tg_gpu_init", CI, [CI]),
    ("tg_device_sync", CI, []),
    ("tg_prof_enable", CI, [CI]),
    ("tg_prof_read", CI, [ctypes.c_char_p, VP, VP]),
    ("tg_arena_create", VP, [CI, CI, CI, CI, CI]),
    ("tg_arena_destroy", None, [VP]),
    ("tg_arena_expert_bytes", SZ, [VP]),
    ("tg_arena_layer_bytes", SZ, [VP]),
    ("tg_arena_expert_offset", CI, [VP, CI, VP, VP, VP, VP]),
    ("tg_arena_load_layer", CI, [VP, CI, VP, SZ]),
    ("tg_arena_load_router", CI, [VP, CI, VP, SZ]),
    ("tg_arena_load_norm", CI, [VP, CI, VP, SZ]),
    ("tg_arena_read_layer", CI, [VP, CI, VP, SZ]),
    ("tg_arena_read_expert", CI, [VP, CI, CI, VP, SZ]),
    ("tg_arena_synth_layer", CI, [VP, CI, U64, CF]),
    ("tg_moe_layer_q40_dev", CI, [VP, CI, VP, VP, CI, VP, VP, CF, VP]),
    ("tg_moe_layer_q40", CI, [VP, CI, VP, VP, CI, VP, VP, CF]),
    ("tg_moe_layer_q40_noalloc_dev", CI, [VP, CI, VP, VP, CI, VP, VP, CF, VP]),
    ("tg_moe_stack_q40_dev", CI, [VP, VP, CI, CI, CI, CF, VP]),
    ("tg_moe_stack_q40", CI, [VP, VP, CI, CI, CI, CF]),
    ("tg_moe_stack_q40_trace_dev", CI, [VP, VP, CI, CI, CF, VP, VP, VP]),
    ("tg_arena_set_decode_path", CI, [VP, CI]),
    ("tg_arena_set_batch_path", CI, [VP, CI]),
    ("tg_arena_set_graphs", CI, [VP, CI]),
    ("tg_arena_status", CI, [VP]),
    ("tg_q40_quantize_q8_0_dev", CI, [VP, VP, CI, VP]),
    ("tg_q40_to_planar_dev", CI, [VP, VP, CI, CI, VP]),
    ("tg_q40_from_planar_dev", CI, [VP, VP, CI, CI, VP]),
    ("tg_q40_block_sums_dev", CI, [VP, CI, CI, VP, VP, VP]),
    ("tg_q40_matvec_dev", CI, [VP, CI, CI, VP, VP, VP]),
    ("tg_router_topk_dev", CI, [VP, VP, CI, CI, CI, CF, CI, VP, VP, VP, VP]),
    ("tg_stream_read_dev", CI, [VP, SZ, CI, VP, VP]),
    ("tg_synth_normal_dev", CI, [U64, U64, CF, SZ, VP, VP]),
    ("tg_synth_q40_dev", CI, [U64, U64, CF, CI, CI, VP, VP]),
    ("tg_head_create", VP, [VP, VP, CI, CI]),
    ("tg_head_forward", CI, [VP, VP, CF, VP, VP]),
    ("tg_head_destroy", None, [VP]),
    ("tg_sampler_create", VP, [CI]),
    ("tg_sampler_run", CI, [VP, VP, CI, CF, CD, CD, VP, VP]),
    ("tg_sampler_destroy", None, [VP]),
    ("tg_head_sample", CI, [VP, VP, CF, CF, CD, CD, VP, VP]),
    ("tg_mirror_drop", None, [VP, SZ]),
    ("tg_mirror_stats", None, [VP, VP, VP, VP]),
    ("tg_mirror_mode", CI, [CI]),
    ("tg_debug_fault_inject", CI, [ctypes.c_uint32, CI]),
    ("tg_clock_mfma_mhz", CI, [CI, VP, VP, VP]),
]

ALL_SYMBOLS = LEGACY_SYMBOLS + UNREGISTERED_SYMBOLS + NEW_SYMBOLS


def find_library():
    """Find the libtinygiant shared library (reference search order)."""
    pkg_dir = Path(__file__).parent
    repo_dir = pkg_dir.parent
    search = [
        pkg_dir / "libtinygiant.dylib",
        pkg_dir / "libtinygiant.so",
        repo_dir / "libtinygiant.dylib",
        repo_dir / "libtinygiant.so",
    ]
    for path in search:
        if path.exists():
            return path
    return None


def _register(lib):
    for name, res, args in ALL_SYMBOLS:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def load_tinygiant_lib(lib_path=None):
    """Load the library and register its symbols; None if it is not found."""
    if lib_path is None:
        lib_path = find_library()
    if lib_path is None:
        return None
    return _register(ctypes.CDLL(str(lib_path)))


class TinyGiantError(RuntimeError):
    """A libtinygiant entry point returned an error code."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


_LIB = None


def require_lib():
    """The loaded library, or an ImportError naming the missing build."""
    global _LIB
    if _LIB is None:
        # TINYGIANT_LIB names another build of this library (the sanitizer
        # build of tests/test_sanitizers.py); find_library keeps the
        # reference's search order
        path = os.environ.get("TINYGIANT_LIB") or find_library()
        if path is None:
            raise ImportError(
                "libtinygiant.so (gfx950) is not built; run "
                "`python -c 'import __graft_entry__ as g; g.build()'` or "
                "`python tinygiant_amd/build.py`")
        _LIB = load_tinygiant_lib(path)
    return _LIB


def check(fn: str, rc: int) -> None:
    if rc != 0:
        msg = require_lib().tg_last_error()
        raise TinyGiantError(fn, rc, msg.decode() if msg else "")


def call(name: str, *args):
    """Call a status-returning entry point and raise on error."""
    rc = getattr(require_lib(), name)(*args)
    check(name, rc)
    return rc
