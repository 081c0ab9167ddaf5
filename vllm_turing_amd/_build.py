"""Builds the HIP kernels in csrc/ into build/libw8a8_mi355.so with hipcc for gfx950 and loads it with ctypes.

The counterpart of vllm_turing/_build.py:33-55 (nvcc -> .so -> ctypes.CDLL): the library is rebuilt when a source
is newer than it (:42), builds are serialized across processes by an fcntl lock (:40-41), the new library is written
to a temporary name and renamed into place (:53), and the loaded handle is cached per process (:13, :54).  Each .hip
file is compiled to an object in parallel, then linked.  There is no CPU fallback: if the library cannot be built or
loaded, load() raises.

Before compiling, the SiLU lookup tables are generated into build/silu_table.inc (silu_table.py), which quant.hip
includes as read-only device data.

Flags: -O3, -ffp-contract=off (every multiply-add fusion in the kernels is an explicit __builtin_fmaf, so the float
epilogues round exactly where the reference rounds), correctly rounded float32 division (hipcc's default, never
-ffast-math), and the packed-FP32 instructions switched off.
"""
import concurrent.futures
import ctypes
import fcntl
import glob
import os
import shutil
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
_CSRC = os.path.join(_HERE, "csrc")
_BUILD = os.path.join(_HERE, "build")
_INCLUDE = os.path.join(os.path.dirname(_HERE), "include")
LIB_NAME = "w8a8_mi355"
ARCH = os.environ.get("VLLM_TURING_AMD_ARCH", "gfx950")
_libs = {}

HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def so_path(name=LIB_NAME):
    return os.path.join(_BUILD, f"lib{name}.so")


def _sources():
    return sorted(glob.glob(os.path.join(_CSRC, "*.hip")))


_GENERATOR = os.path.join(_HERE, "silu_table.py")
_SILU_INC = os.path.join(_BUILD, "silu_table.inc")


def _deps():
    return _sources() + sorted(glob.glob(os.path.join(_CSRC, "*.h"))) + \
        sorted(glob.glob(os.path.join(_INCLUDE, "*.h"))) + [_GENERATOR]


def _hipcc():
    for p in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if p and os.path.exists(p):
            return p
    raise RuntimeError("hipcc not found: the W8A8 HIP library cannot be built")


def stale(name=LIB_NAME):
    so = so_path(name)
    if not os.path.exists(so):
        return True
    t = os.path.getmtime(so)
    return any(os.path.getmtime(d) > t for d in _deps())


def build(name=LIB_NAME, force=False, verbose=False):
    """Compile csrc/*.hip for gfx950 into build/lib<name>.so (under the build lock)."""
    os.makedirs(_BUILD, exist_ok=True)
    so = so_path(name)
    with open(os.path.join(_BUILD, ".lock"), "w") as lk:
        fcntl.flock(lk, fcntl.LOCK_EX)
        if not force and not stale(name):
            return so
        hipcc = _hipcc()
        from . import silu_table
        silu_table.write_include(_SILU_INC)
        objs = []

        def compile_one(src):
            obj = os.path.join(_BUILD, os.path.basename(src)[:-4] + ".o")
            cmd = [hipcc, *HIPCC_FLAGS, f"-I{_INCLUDE}", f"-I{_BUILD}", "-c", src, "-o", obj + ".tmp"]
            r = subprocess.run(cmd, capture_output=True, text=True)
            if r.returncode != 0:
                raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
            os.replace(obj + ".tmp", obj)
            if verbose:
                print(" ".join(cmd), flush=True)
            return obj

        with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(_sources()))) as ex:
            objs = list(ex.map(compile_one, _sources()))
        cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", so + ".tmp"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc link failed:\n{r.stderr}")
        os.replace(so + ".tmp", so)
    return so


def load(name=LIB_NAME):
    """The loaded library (built first if missing or older than its sources); cached per process."""
    if name in _libs:
        return _libs[name]
    if stale(name):
        build(name)
    _libs[name] = ctypes.CDLL(so_path(name))
    return _libs[name]
