"""Build libmentat_hip.so (gfx950) from mentat_amd/csrc/*.hip with hipcc (and
the host-only mentat_amd/csrc/*.cpp with the host compiler), and the host
planner extension mentat_amd/_host_plan*.so from mentat_amd/csrc/host_plan.c.

Every call recompiles all sources (objects go to mentat_amd/_build/, the
library to mentat_amd/lib/libmentat_hip.so). Usage: ``python -m mentat_amd.build``.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libmentat_hip.so")
ARCH = os.environ.get("MENTAT_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # Packed fp32 VALU ops stay disabled for all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        ln for ln in proc.stdout.splitlines() if "packed-fp32-ops' is not a recognized feature" not in ln
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    _run([HIPCC, *COMMON_FLAGS, "-c", src, "-o", obj])
    return obj


# Host-only sources (planners run on the CPU each step) go through the host compiler.
CXX = shutil.which("g++") or "g++"
HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function"]


def _compile_host(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src).replace(".cpp", "_host.o"))
    _run([CXX, *HOST_FLAGS, "-I", os.path.join(os.path.dirname(HERE), "include"), "-c", src, "-o", obj])
    return obj


# The host planner extension (CPython C API, csrc/host_plan.c) is built in-tree
# next to the package's modules.
CC = shutil.which("gcc") or "gcc"


def build_host_ext(verbose: bool = True) -> str:
    import sysconfig

    src = os.path.join(CSRC, "host_plan.c")
    out = os.path.join(HERE, "_host_plan" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out + ".tmp"
    _run([CC, "-O2", "-shared", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter",
          "-I", sysconfig.get_paths()["include"], src, "-o", tmp])
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}", file=sys.stderr)
    return out


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    host = sorted(glob.glob(os.path.join(CSRC, "*.cpp")))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = max(1, min(len(srcs) + len(host), os.cpu_count() or 1, 16))
    with cf.ThreadPoolExecutor(workers) as ex:
        jobs = [ex.submit(_compile, s) for s in srcs] + [ex.submit(_compile_host, s) for s in host]
        objs = [j.result() for j in jobs]
    srcs = srcs + host
    tmp = LIB + ".tmp"
    _run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources", file=sys.stderr)
    build_host_ext(verbose)
    return LIB


if __name__ == "__main__":
    build()
