"""AddressSanitizer + UndefinedBehaviorSanitizer runs of the host code, on
the CPU (no GPU sanitizer exists on this pool, and none is needed for the
host side):

  the oracle   oracle/_san/libtg_oracle.so (gcc, `make -C oracle sanitize`)
               under every oracle, golden and relayout test
  the C-ABI    tinygiant_amd/_san/libtinygiant.so (host code sanitized, the
               gfx950 code built as usual) under the error-channel and export
               tests, which reach no kernel

Each runs in a child pytest with the sanitizer runtime preloaded, so the
first sanitizer report fails it."""
import glob
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
OPTS = {"ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=0",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}


def child_pytest(files, env_extra):
    env = dict(os.environ, **OPTS, **env_extra)
    cmd = [sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "-m", "not gpu", *files]
    r = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    tail = "\n".join((r.stdout + r.stderr).splitlines()[-30:])
    assert r.returncode == 0, tail
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error:" not in r.stderr, tail


def test_oracle_under_asan_ubsan():
    libasan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    libubsan = subprocess.run(["gcc", "-print-file-name=libubsan.so"], capture_output=True, text=True).stdout.strip()
    if not os.path.isabs(libasan) or not os.path.isabs(libubsan):
        pytest.skip("gcc's sanitizer runtimes are not installed")
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "sanitize"], check=True)
    files = sorted(str(p.relative_to(ROOT)) for p in (ROOT / "tests").glob("test_oracle_*.py"))
    files += ["tests/test_golden.py", "tests/test_relayout.py"]
    child_pytest(files, {"LD_PRELOAD": f"{libasan}:{libubsan}",
                         "TG_ORACLE_LIB": str(ROOT / "oracle" / "_san" / "libtg_oracle.so")})


def test_abi_host_code_under_asan_ubsan():
    rt = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not rt:
        pytest.skip("clang's shared ASan runtime is not installed")
    from tinygiant_amd import build
    lib = build.build_sanitized()
    child_pytest(["tests/test_abi_errors.py", "tests/test_abi_exports.py"],
                 {"LD_PRELOAD": rt[-1], "TINYGIANT_LIB": str(lib)})
