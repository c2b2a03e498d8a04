"""AddressSanitizer + UndefinedBehaviorSanitizer run of the host code.

Builds the pybind modules (bindings/*.cpp with host/*.cpp) and the C oracle
(oracle/gemm_oracle.c) with -fsanitize=address,undefined into _build/asan/, next
to a copy of the Python package and the ordinary libgev2.so (device code is not
instrumented), then runs the CPU test suite (-m "not gpu") against them with the
ASan runtime preloaded into Python.  Any report aborts the run
(-fno-sanitize-recover, halt_on_error).

Usage: python ai_framework-dev_amd/sanitize.py [pytest args ...]
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig

import build as B

OUT = os.path.join(B.REPO, "_build", "asan")
PKG_OUT = os.path.join(OUT, "pkg")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]


def _sh(cmd, **kw):
    r = subprocess.run(cmd, **kw)
    if r.returncode != 0:
        raise SystemExit(f"failed ({r.returncode}): {' '.join(cmd)}")


def build() -> None:
    import pybind11

    lib = os.path.join(B.OUT_DIR, "libgev2.so")
    if not os.path.exists(lib):
        B.build_hip(False, 8)
    src_pkg = os.path.join(B.PKG, "graph_executor_v2")
    dst_pkg = os.path.join(PKG_OUT, "graph_executor_v2")
    shutil.rmtree(dst_pkg, ignore_errors=True)
    shutil.copytree(src_pkg, dst_pkg, ignore=shutil.ignore_patterns("__pycache__", "_ops_*.so"))
    ops = os.path.join(dst_pkg, "ops")
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    for mod, srcs in B.BIND_SOURCES.items():
        cmd = ["g++", "-std=c++17", "-fPIC", "-shared", "-Wall", "-fvisibility=hidden", *SAN,
               f"-I{pybind11.get_include()}", f"-I{sysconfig.get_paths()['include']}", f"-I{B.INCLUDE}",
               f"-I{B.CSRC}", *[os.path.join(B.CSRC, x) for x in srcs], "-o", os.path.join(ops, mod + suffix)]
        if mod != "_ops_common":
            cmd += [f"-L{ops}", "-lgev2", "-Wl,-rpath,$ORIGIN"]
        _sh(cmd)
    _sh(["gcc", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", *SAN,
         os.path.join(B.REPO, "oracle", "gemm_oracle.c"), "-o", os.path.join(OUT, "libgemm_oracle.so"), "-lm"])


def run(pytest_args) -> int:
    def rt(name):
        return subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()

    env = dict(os.environ)
    # libstdc++ is preloaded too: Python is not a C++ program, and ASan's
    # __cxa_throw interceptor needs the real one resolved at start-up
    env.update(LD_PRELOAD=f"{rt('libasan.so')} {rt('libstdc++.so')}",
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               GEV2_PKG_ROOT=PKG_OUT,
               GEV2_ORACLE_LIB=os.path.join(OUT, "libgemm_oracle.so"))
    cmd = [sys.executable, "-m", "pytest", os.path.join(B.REPO, "tests"), "-q", "-m", "not gpu", "-p", "no:cacheprovider",
           *pytest_args]
    return subprocess.run(cmd, env=env, cwd=B.REPO).returncode


if __name__ == "__main__":
    build()
    sys.exit(run(sys.argv[1:]))
