"""Build recipe for the gfx950 FP8 MoE path (explicit hipcc / g++ lines).

Produces, in the package root (``distributed-hipkittens_amd/``):
  libhkmoe.so                   the C ABI (include/hkmoe.h) and every HIP kernel
  tk_kernel<EXT_SUFFIX>         the pybind11 ``dispatch_*`` module over it

The reference builds one pybind11 ``tk_kernel`` per kernel directory through
its make rules (kernels/common.mk:63-82); here one library holds the whole
path and the module links against it with an ``$ORIGIN`` rpath, so the pair
can be copied anywhere together.
"""
import os
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent.parent
CSRC = PKG_ROOT / "csrc"
INCLUDE = PKG_ROOT.parent / "include"
LIB = PKG_ROOT / "libhkmoe.so"
EXT = PKG_ROOT / ("tk_kernel" + sysconfig.get_config_var("EXT_SUFFIX"))

ARCH = os.environ.get("HKMOE_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    # packed fp32 VALU ops are kept out of every kernel on this hardware pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # fp32 '/' must be IEEE-correctly rounded (quantisation is bit-exact)
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # one-thread queue atomics stay plain atomics: the wave-level rewrite reads
    # the result right away, which waits for every load in flight
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Wno-unused-command-line-argument",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(str(c) for c in cmd), flush=True)
    res = subprocess.run([str(c) for c in cmd], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"build failed ({res.returncode}): {' '.join(map(str, cmd))}\n"
                           f"{res.stdout}\n{res.stderr}")
    return res


def _pybind_includes():
    import pybind11
    return [f"-I{pybind11.get_include()}", f"-I{sysconfig.get_paths()['include']}"]


def build(verbose=False):
    """Compile libhkmoe.so (hipcc, gfx950) and the tk_kernel module (g++)."""
    tmp_lib = LIB.with_suffix(".so.tmp")
    _run([HIPCC, *HIP_FLAGS, f"-I{INCLUDE}", CSRC / "capi.hip", "-o", tmp_lib], verbose)
    os.replace(tmp_lib, LIB)
    tmp_ext = EXT.with_name(EXT.name + ".tmp")
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
          *_pybind_includes(), f"-I{INCLUDE}", CSRC / "tk_kernel.cpp",
          f"-L{PKG_ROOT}", "-lhkmoe", "-Wl,-rpath,$ORIGIN", "-o", tmp_ext], verbose)
    os.replace(tmp_ext, EXT)
    return LIB, EXT


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(f"built {LIB} and {EXT}")
