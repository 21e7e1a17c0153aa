"""CPU sanitizer run of the host code (not collected by pytest; run it directly).

    python tests/sanitize_host.py

Builds, under dscquant_amd/_build/sanitize/:
  * the C oracle (oracle/dscq_oracle.c) with clang, AddressSanitizer and
    UndefinedBehaviorSanitizer;
  * libdscq.so with the same sanitizers on its host pass only (``-Xarch_host``):
    the argument checks, size limits, workspace sizing and dispatch of
    csrc/api.hip, gemm.hip, quantize.hip, decode.hip and noalloc.hip.  Device
    code is compiled as usual and never runs here.

Then runs the CPU test suite (``-m "not gpu"``) in a child process with the
sanitizer runtime preloaded and the two sanitized libraries swapped in
(tests/conftest.py reads DSCQ_TEST_ORACLE_LIB / DSCQ_TEST_LIBDSCQ).  Any
sanitizer report aborts the run, so the exit status is the verdict.  Leak
detection is off: the interpreter and torch keep allocations alive at exit.
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OUT = os.path.join(ROOT, "dscquant_amd", "_build", "sanitize")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]


def llvm_dir() -> str:
    return os.environ.get("ROCM_PATH", "/opt/rocm") + "/llvm"


def asan_runtime() -> str:
    hits = sorted(glob.glob(os.path.join(llvm_dir(), "lib/clang/*/lib/linux/"
                                         "libclang_rt.asan-x86_64.so")))
    if not hits:
        raise RuntimeError("clang's AddressSanitizer runtime not found under " + llvm_dir())
    return hits[-1]


def build_oracle() -> str:
    path = os.path.join(OUT, "liboracle_san.so")
    subprocess.run(["make", "-s", "-B", "-C", os.path.join(ROOT, "oracle"),
                    f"CC={llvm_dir()}/bin/clang", "SANFLAGS=" + " ".join(SAN), f"OUT={path}"],
                   check=True)
    return path


def build_libdscq() -> str:
    sys.path.insert(0, ROOT)
    from dscquant_amd import build
    flags = []
    for f in SAN:
        flags += ["-Xarch_host", f]
    return build.build(lib_path=os.path.join(OUT, "libdscq_san.so"),
                       objdir=os.path.join(OUT, "obj"), extra_flags=tuple(flags))


def main() -> int:
    oracle_lib = build_oracle()
    dscq_lib = build_libdscq()
    env = dict(os.environ,
               LD_PRELOAD=asan_runtime(),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               DSCQ_TEST_ORACLE_LIB=oracle_lib,
               DSCQ_TEST_LIBDSCQ=dscq_lib)
    # The sanitized builds, not the in-tree ones, must be what the tests load.
    probe = ("import sys; sys.path.insert(0, 'tests'); import conftest\n"
             "class C:\n    def addinivalue_line(self, *a): pass\n"
             "conftest.pytest_configure(C())\n"
             "from oracle import native; from dscquant_amd import _lib\n"
             "native.lib(); _lib.lib(); maps = open('/proc/self/maps').read()\n"
             "assert 'liboracle_san.so' in maps and 'libdscq_san.so' in maps, 'not loaded'\n")
    subprocess.run([sys.executable, "-c", probe], env=env, cwd=ROOT, check=True)
    cmd = [sys.executable, "-m", "pytest", os.path.join(ROOT, "tests"), "-q", "-m", "not gpu",
           "-p", "no:cacheprovider"]
    print("sanitized run:", " ".join(cmd), flush=True)
    return subprocess.run(cmd, env=env, cwd=ROOT).returncode


if __name__ == "__main__":
    sys.exit(main())
