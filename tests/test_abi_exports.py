"""The C-ABI library loads and exports every symbol include/tinygiant.h
declares, with the reference's registration (tinygiant/_lib.py:39-74).
No compute calls: these run without a GPU."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "tinygiant.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    names = re.findall(r"\b(tg_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


@pytest.fixture(scope="module")
def libpath():
    from tinygiant_amd._lib import find_library
    p = find_library()
    if p is None:
        pytest.fail("libtinygiant.so is not built (run __graft_entry__.build())")
    return p


def test_header_declares_reference_abi():
    names = declared_symbols()
    for ref in ["tg_expert_forward", "tg_expert_forward_mixed", "tg_matmul_q4k", "tg_matmul_q6k",
                "tg_rms_norm", "tg_f32_matvec", "tg_f16_matvec", "tg_attention_decode",
                "tg_attention_decode_q4", "tg_prefetch", "tg_prefetch_batch", "tg_mlock",
                "tg_transformer_layer", "tg_moe_forward", "tg_matmul_q4k_scalar"]:
        assert ref in names


def test_library_exports_every_declared_symbol(libpath):
    out = subprocess.run(["nm", "-D", "--defined-only", str(libpath)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (tg_[a-z0-9_]+)\b", out))
    missing = [n for n in declared_symbols() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"


def test_load_tinygiant_lib_registers_reference_symbols(libpath):
    from tinygiant_amd._lib import ALL_SYMBOLS, LEGACY_SYMBOLS, load_tinygiant_lib
    lib = load_tinygiant_lib(libpath)
    assert lib is not None
    for name, res, args in LEGACY_SYMBOLS:
        fn = getattr(lib, name)
        assert fn.argtypes == args
    assert {n for n, _, _ in ALL_SYMBOLS} == set(declared_symbols())


def test_reference_argtypes_match_reference_registration():
    """The thirteen registrations of tinygiant/_lib.py:39-74, restated."""
    from tinygiant_amd._lib import CF, CI, LEGACY_SYMBOLS, VP
    reg = {n: a for n, _, a in LEGACY_SYMBOLS}
    assert reg["tg_expert_forward"] == [VP, VP, VP, CF, CI, CI]
    assert reg["tg_expert_forward_mixed"] == [VP, VP, VP, CI, VP, VP, CF, CI, CI]
    assert reg["tg_rms_norm"] == [VP, VP, VP, CI, CF]
    assert len(reg["tg_attention_decode"]) == 19
    assert len(reg["tg_transformer_layer"]) == 27
    assert reg["tg_mlock"] == [VP, ctypes.c_size_t]


def test_find_library_search_order(tmp_path, monkeypatch):
    from tinygiant_amd import _lib
    p = _lib.find_library()
    assert p is not None and p.name in ("libtinygiant.so", "libtinygiant.dylib")
    assert p.parent in (Path(_lib.__file__).parent, Path(_lib.__file__).parent.parent)
