"""tinygiant_amd -- TinyGiant's MoE expert hot path on MI355X (gfx950).

libtinygiant.so (built from csrc/ by build.py) exports the reference's C ABI
(csrc/libtinygiant.c) plus the Q4_0 arena / MoE entry points of
include/tinygiant.h.  Python side:

  _lib      find_library / load_tinygiant_lib (tinygiant/_lib.py mirror)
  arena     HBMExpertArena (tinygiant/cache.py's role, in HBM)
  moe       MoEBlock (tinygiant/engine.py:229-258 on the GPU)
  relayout  Q4_0 expert-contiguous cache files (tinygiant/relayout.py)
"""
from ._lib import find_library, load_tinygiant_lib, require_lib  # noqa: F401

__all__ = ["find_library", "load_tinygiant_lib", "require_lib"]
