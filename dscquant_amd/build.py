"""Builds libdscq.so (the gfx950 HIP kernels + C ABI) in-tree.

    python -m dscquant_amd.build          # or dscquant_amd.build.build()

Every .hip file under csrc/ is compiled by hipcc for gfx950 only and linked
into dscquant_amd/lib/libdscq.so.  Flags that matter for results:
  -ffp-contract=off        no silent a*b+c -> fma fusion; fmas are explicit
  -fno-fast-math           IEEE division / rounding as written
  -target-feature -packed-fp32-ops
                           keep hipcc from emitting packed fp32 math
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
LIB_PATH = os.path.join(LIBDIR, "libdscq.so")
OBJDIR = os.path.join(HERE, "_build")
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libdscq)")


COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-mcode-object-version=5",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def _compile(src: str, objdir: str = OBJDIR, extra: tuple = ()) -> str:
    obj = os.path.join(objdir, os.path.basename(src) + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *extra, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr}")
    # Host passes warn about the device-only feature flag; keep real warnings.
    warn = "\n".join(l for l in res.stderr.splitlines()
                     if "packed-fp32-ops" not in l and l.strip())
    if warn:
        sys.stderr.write(warn + "\n")
    return obj


def build(verbose: bool = False, lib_path: str = LIB_PATH, objdir: str = OBJDIR,
          extra_flags: tuple = ()) -> str:
    """Compile every csrc/*.hip and link libdscq.so; returns its path.

    ``extra_flags`` go on every compile and on the link (the sanitized host
    build passes ``-Xarch_host -fsanitize=...`` here, with its own paths).
    """
    os.makedirs(objdir, exist_ok=True)
    os.makedirs(os.path.dirname(lib_path), exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    jobs = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, objdir, tuple(extra_flags)), srcs))
    tmp = lib_path + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *extra_flags, *objs,
           "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, lib_path)
    if verbose:
        print(f"built {lib_path}")
    return lib_path


if __name__ == "__main__":
    build(verbose=True)
