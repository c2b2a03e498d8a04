"""Build the gfx950 HIP library and the Python binding modules in-tree.

Outputs (next to the Python package, like the reference's CMake output dir
``python/graph_executor_v2/ops``; graph_executor_v2/CMakeLists.txt:163-182):
  graph_executor_v2/ops/libgev2.so        HIP kernels + C ABI (include/gev2_gemm.h)
  graph_executor_v2/ops/_ops_common*.so   pybind11: shared shim types
  graph_executor_v2/ops/_ops_gemm*.so     pybind11: the GEMM op surface
  graph_executor_v2/ops/_ops_conv2d*.so   pybind11: conv2d on the GEMM op
  graph_executor_v2/ops/_ops_rnn*.so      pybind11: Elman RNN on the GEMM op
  graph_executor_v2/ops/_ops_sdpa*.so     pybind11: scaled dot-product attention

Usage: python ai_framework-dev_amd/build.py [--force] [-j N]
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OUT_DIR = os.path.join(PKG, "graph_executor_v2", "ops")
BUILD_DIR = os.path.join(REPO, "_build")
INCLUDE = os.path.join(REPO, "include")

HIP_SOURCES = [
    "gemm_tile_f32.hip", "gemm_tile_bf16.hip", "gemm_tile_f16.hip",
    "gemm_dl_bf16.hip", "gemm_dl_f16.hip", "gemm_dl_f32.hip",
    "gemm_skinny.hip", "gemm_small.hip", "gemm_aux.hip", "capi.hip", "noalloc.hip", "conv.hip", "rnn.hip", "attn.hip", "probe.hip",
]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++20", "-fPIC", "-Wall", "-Wno-unused-function",
    # packed-fp32 forms are disabled for all device code (the host pass warns
    # that it does not know the feature; that is harmless)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

BIND_SOURCES = {
    "_ops_common": ["bindings/ops_common_pybind.cpp"],
    "_ops_gemm": ["bindings/gemm_pybind.cpp", "host/gemm_host.cpp"],
    "_ops_conv2d": ["bindings/conv2d_pybind.cpp", "host/conv2d_host.cpp"],
    "_ops_rnn": ["bindings/rnn_pybind.cpp", "host/rnn_host.cpp"],
    "_ops_sdpa": ["bindings/sdpa_pybind.cpp", "host/sdpa_host.cpp"],
}
HOST_HEADERS = ["host/shim.hpp", "host/gemm_host.hpp", "host/conv2d_host.hpp", "host/rnn_host.hpp",
                "host/sdpa_host.hpp"]


def _includes(path: str, seen=None) -> list[str]:
    """The file and every local header it includes (#include "..."), recursively."""
    import re
    seen = set() if seen is None else seen
    if path in seen or not os.path.exists(path):
        return []
    seen.add(path)
    with open(path) as f:
        for inc in re.findall(r'^\s*#\s*include\s+"([^"]+)"', f.read(), re.M):
            _includes(os.path.normpath(os.path.join(os.path.dirname(path), inc)), seen)
    return sorted(seen)


def _newer(target: str, deps: list[str]) -> bool:
    if not os.path.exists(target):
        return True
    t = os.path.getmtime(target)
    return any(os.path.getmtime(d) > t for d in deps if os.path.exists(d))


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def build_hip(force: bool, jobs: int) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    os.makedirs(OUT_DIR, exist_ok=True)
    objs, todo = [], []
    for src in HIP_SOURCES:
        s = os.path.join(CSRC, src)
        o = os.path.join(BUILD_DIR, src.replace(".hip", ".o"))
        objs.append(o)
        if force or _newer(o, _includes(s)):
            todo.append([HIPCC, *HIP_FLAGS, "-c", s, "-o", o])
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, todo))
    lib = os.path.join(OUT_DIR, "libgev2.so")
    if force or todo or _newer(lib, objs):
        tmp = lib + ".tmp"
        _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs,
              "-Wl,-soname,libgev2.so"])
        os.replace(tmp, lib)
    return lib


def build_bindings(force: bool, jobs: int) -> list[str]:
    import pybind11

    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    py_inc = sysconfig.get_paths()["include"]
    headers = [os.path.join(CSRC, h) for h in HOST_HEADERS] + [os.path.join(INCLUDE, "gev2_gemm.h")]
    cmds, outs = [], []
    for mod, srcs in BIND_SOURCES.items():
        paths = [os.path.join(CSRC, s) for s in srcs]
        out = os.path.join(OUT_DIR, mod + suffix)
        outs.append(out)
        if not all(os.path.exists(p) for p in paths):
            continue
        if force or _newer(out, paths + headers + [os.path.join(OUT_DIR, "libgev2.so")]):
            cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
                   "-fvisibility=hidden",
                   f"-I{pybind11.get_include()}", f"-I{py_inc}", f"-I{INCLUDE}", f"-I{CSRC}",
                   *paths, "-o", out + ".tmp"]
            if mod in ("_ops_gemm", "_ops_conv2d", "_ops_rnn", "_ops_sdpa"):
                cmd += [f"-L{OUT_DIR}", "-lgev2", "-Wl,-rpath,$ORIGIN"]
            cmds.append((cmd, out))

    def go(c):
        cmd, out = c
        _run(cmd)
        os.replace(out + ".tmp", out)

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(go, cmds))
    return outs


def build_oracle() -> None:
    """The C restatement under oracle/ (test infrastructure, not the product)."""
    odir = os.path.join(REPO, "oracle")
    if os.path.exists(os.path.join(odir, "Makefile")) and shutil.which("make"):
        _run(["make", "-s", "-C", odir])


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=min(8, os.cpu_count() or 4))
    ap.add_argument("--hip-only", action="store_true")
    args = ap.parse_args(argv)
    build_hip(args.force, args.jobs)
    if not args.hip_only:
        build_bindings(args.force, args.jobs)
    return 0


if __name__ == "__main__":
    sys.exit(main())
