"""Build libsnapjudge_hip.so (gfx950) in-tree with hipcc.

Every source under csrc/ is compiled for gfx950 only and linked into
snapjudge_amd/libsnapjudge_hip.so next to this file, so the built library
travels with the source tree.  Objects go to snapjudge_amd/_build/.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libsnapjudge_hip.so")
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32.
# -amdgpu-mfma-vgpr-form: MFMA results go to ordinary VGPRs, so the softmax
# and epilogue math on them needs no AGPR round trips.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-I" + CSRC, "-I" + os.path.join(ROOT, "include"),
]


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [hipcc(), *HIP_FLAGS, "-x", "hip", "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{r.stderr[-6000:]}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


HOOK_SRC = os.path.join(HERE, "hook", "fast_hip.cpp")
HOOK_LIB = os.path.join(HERE, "libsnapjudge_fast_hip.so")


def build_hook(ref: str | None = None, verbose: bool = False) -> str | None:
    """Build libsnapjudge_fast_hip.so, the reference's FastSnapjudge class over
    libsnapjudge_hip.so.  It compiles against the reference's own headers
    (include/snapjudge/model.hpp for DecisionModel's fields), so it is built
    only where the reference tree exists; the built library travels with the
    source tree like libsnapjudge_hip.so.  Returns None without the headers."""
    ref = ref or os.environ.get("SNAPJUDGE_REF", "/root/reference")
    inc = os.path.join(ref, "include")
    if not os.path.exists(os.path.join(inc, "snapjudge", "model.hpp")):
        return None
    cxx = shutil.which("g++") or "g++"
    tmp = HOOK_LIB + ".tmp"
    cmd = [cxx, "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra",
           "-I" + os.path.join(ROOT, "include"), "-I" + inc,
           "-I" + os.path.join(ref, "third_party"), HOOK_SRC, "-L" + HERE, "-lsnapjudge_hip",
           "-Wl,-rpath,$ORIGIN", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hook build failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, HOOK_LIB)
    if verbose:
        print(f"built {HOOK_LIB}")
    return HOOK_LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
