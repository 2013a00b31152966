"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

The library is rebuilt with both sanitizers on its host side only (each
-fsanitize= follows -Xarch_host, so the gfx950 code objects are built as
usual), and tests/test_capi.py (argument checks, workspace sizing, empty
batches: every path that runs without a GPU) runs against that build in a child
Python with clang's ASan runtime preloaded (it carries the UBSan handlers too).
Any report aborts the child (halt_on_error), and the test fails.  No GPU.
"""
import glob
import importlib.util
import os
import subprocess
import sys
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "distributed-hipkittens_amd")
SANITIZE = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer"]


def _recipe():
    # the build recipe by file path (importing hkmoe would need the built module)
    spec = importlib.util.spec_from_file_location("_hkmoe_build_san", os.path.join(PKG, "hkmoe", "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_capi_host_code_under_asan_and_ubsan():
    rec = _recipe()
    runtimes = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not os.path.exists(rec.HIPCC) or not runtimes:
        pytest.skip("hipcc or clang's ASan runtime not found")
    with tempfile.TemporaryDirectory() as tmp:
        lib = os.path.join(tmp, "libhkmoe.so")
        flags = [f for f in rec.HIP_FLAGS if f != "-O3"] + ["-O1", "-g"] + SANITIZE
        build = subprocess.run([rec.HIPCC, *flags, f"-I{rec.INCLUDE}", str(rec.CSRC / "capi.hip"), "-o", lib],
                               capture_output=True, text=True)
        assert build.returncode == 0, build.stderr[-3000:]
        env = dict(os.environ, HKMOE_LIB=lib, LD_PRELOAD=runtimes[-1],
                   ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
                   UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
        run = subprocess.run([sys.executable, "-m", "pytest", os.path.join(ROOT, "tests", "test_capi.py"),
                              "-q", "-p", "no:cacheprovider", "-k", "not pybind"],
                             capture_output=True, text=True, env=env, cwd=ROOT, timeout=600)
        out = run.stdout + run.stderr
        assert run.returncode == 0, out[-4000:]
        assert "AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
