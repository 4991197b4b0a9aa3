"""Build the gfx950 HIP library (nnr_amd/lib/libnnr_hip.so) with hipcc.

Every HIP/C++ source under nnr_amd/csrc is compiled separately (in parallel)
and linked into one shared library exporting the C ABI of include/nnr_hip.h.

Numerics flags (identical for device and host code):
  -ffp-contract=off                          no implicit a*b+c -> fma
  -fhip-fp32-correctly-rounded-divide-sqrt   IEEE division
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                             no v_pk_*_f32 generation
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "nnr_amd")
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(PKG, "host")
LIBDIR = os.path.join(PKG, "lib")
OBJDIR = os.path.join(ROOT, "_build", "obj")
LIB = os.path.join(LIBDIR, "libnnr_hip.so")
HOSTLIB = os.path.join(LIBDIR, "libnnr_host.so")
ARCH = os.environ.get("NNR_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
CXX = shutil.which("g++") or "g++"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}",
]
HOST_FLAGS = [
    "-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math",
    "-Wall", "-Wextra", "-Wno-unused-parameter",
    f"-I{os.path.join(ROOT, 'include')}", f"-I{HOST}",
]


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in p.stdout.splitlines() if "packed-fp32-ops" not in l
                    and "is not a recognized feature" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _compile(src, obj, flags, compiler):
    os.makedirs(os.path.dirname(obj), exist_ok=True)
    _run([compiler, *flags, "-c", src, "-o", obj])
    return obj


def build_hip(jobs: int | None = None, verbose: bool = False) -> str:
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC)
                  if f.endswith((".hip", ".cpp")))
    jobs = jobs or min(8, os.cpu_count() or 4)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = []
        for s in srcs:
            obj = os.path.join(OBJDIR, "hip", os.path.basename(s) + ".o")
            flags = list(HIP_FLAGS)
            if s.endswith(".cpp"):
                flags = ["-x", "hip"] + flags
            futs.append(ex.submit(_compile, s, obj, flags, HIPCC))
        for f in futs:
            objs.append(f.result())
    os.makedirs(LIBDIR, exist_ok=True)
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    if verbose:
        print(f"[nnr_amd.build] {LIB}")
    return LIB


def build_host(jobs: int | None = None, verbose: bool = False) -> str | None:
    """C++ host framework (operator_t / registry / context mirror) over the C ABI."""
    if not os.path.isdir(HOST):
        return None
    srcs = sorted(os.path.join(HOST, f) for f in os.listdir(HOST) if f.endswith(".cpp"))
    if not srcs:
        return None
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(
            s, os.path.join(OBJDIR, "host", os.path.basename(s) + ".o"), HOST_FLAGS, CXX), srcs))
    tmp = HOSTLIB + ".tmp"
    _run([CXX, "-shared", "-fPIC", "-o", tmp, *objs, f"-L{LIBDIR}", "-lnnr_hip",
          "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, HOSTLIB)
    if verbose:
        print(f"[nnr_amd.build] {HOSTLIB}")
    return HOSTLIB


def build_oracle(verbose: bool = False) -> str:
    """The CPU oracle is test infrastructure (see oracle/nnr_oracle.h)."""
    odir = os.path.join(ROOT, "oracle")
    _run(["make", "-C", odir, "-B", "CC=gcc"])
    path = os.path.join(odir, "build", "liboracle.so")
    if verbose:
        print(f"[nnr_amd.build] {path}")
    return path


def build_all(verbose: bool = True) -> None:
    build_hip(verbose=verbose)
    build_host(verbose=verbose)
    build_oracle(verbose=verbose)


if __name__ == "__main__":
    what = sys.argv[1] if len(sys.argv) > 1 else "all"
    {"all": build_all, "hip": lambda: build_hip(verbose=True),
     "host": lambda: build_host(verbose=True),
     "oracle": lambda: build_oracle(verbose=True)}[what]()
