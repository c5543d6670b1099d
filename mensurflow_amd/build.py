"""Builds the native parts of mensurflow_amd in-tree (no JIT cache, so the libraries travel
with the source tree):

* ``_lib/libmfr_rocm.so`` -- the HIP kernels and the C ABI of ``include/mfr_rocm.h``
  (hipcc, gfx950 only);
* ``_lib/libmensurflow.so`` -- the C++17 host layer (tensor, dispatcher, registry, ops and the
  ROCm backend that calls the C ABI), built by g++ without any HIP header.

Run ``python -m mensurflow_amd.build`` or ``__graft_entry__.build()``.
"""
from __future__ import annotations

import concurrent.futures
import glob
import os
import shlex
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(PKG, "host")
INCLUDE = os.path.join(ROOT, "include")
LIBDIR = os.path.join(PKG, "_lib")
OBJDIR = os.path.join(PKG, "_build")

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

# -ffp-contract=off: products and sums round separately unless a kernel asks for fma()
# explicitly, so epilogues round like the reference's separate ops.
# -packed-fp32-ops off: no v_pk_*_f32 instructions anywhere in this library.
HIP_FLAGS = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-warning-option",
    f"-I{INCLUDE}", f"-I{CSRC}",
]

# MENSURFLOW_ENABLE_TRACING: the trace spans of mensurflow/trace.hpp are compiled in (one relaxed
# atomic load per span while no hook is attached); anything built against the library defines it
# too, so it sees the same `trace::hook`.
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-DMENSURFLOW_ENABLE_TRACING",
              f"-I{INCLUDE}", f"-I{os.path.join(HOST, 'include')}", f"-I{os.path.join(HOST, 'src')}"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    out = (proc.stdout + proc.stderr).strip()
    # hipcc's host pass does not know the device feature flag; that warning is expected.
    lines = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if proc.returncode != 0:
        raise RuntimeError("command failed:\n" + " ".join(shlex.quote(c) for c in cmd) + "\n" +
                           "\n".join(lines))
    if lines:
        print("\n".join(lines), file=sys.stderr)


def _compile_all(jobs: list[list[str]]) -> None:
    workers = min(len(jobs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        for fut in [pool.submit(_run, cmd) for cmd in jobs]:
            fut.result()


def build_hip() -> str:
    """Compile every csrc/*.hip for gfx950 and link libmfr_rocm.so; returns its path."""
    os.makedirs(LIBDIR, exist_ok=True)
    os.makedirs(OBJDIR, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    objects = []
    jobs = []
    for src in sources:
        obj = os.path.join(OBJDIR, os.path.basename(src) + ".o")
        objects.append(obj)
        jobs.append([HIPCC, *HIP_FLAGS, "-c", src, "-o", obj])
    _compile_all(jobs)
    out = os.path.join(LIBDIR, "libmfr_rocm.so")
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objects,
          "-Wl,-soname,libmfr_rocm.so"])
    os.replace(tmp, out)
    return out


def build_host() -> str | None:
    """Compile the C++17 host layer (no HIP headers) into libmensurflow.so."""
    sources = sorted(glob.glob(os.path.join(HOST, "src", "**", "*.cpp"), recursive=True))
    if not sources:
        return None
    os.makedirs(LIBDIR, exist_ok=True)
    os.makedirs(OBJDIR, exist_ok=True)
    objects = []
    jobs = []
    for src in sources:
        rel = os.path.relpath(src, HOST).replace(os.sep, "_")
        obj = os.path.join(OBJDIR, rel + ".o")
        objects.append(obj)
        jobs.append(["g++", *HOST_FLAGS, "-c", src, "-o", obj])
    _compile_all(jobs)
    out = os.path.join(LIBDIR, "libmensurflow.so")
    tmp = out + ".tmp"
    _run(["g++", "-shared", "-o", tmp, *objects, f"-L{LIBDIR}", "-lmfr_rocm",
          "-Wl,-rpath,$ORIGIN", "-Wl,-soname,libmensurflow.so"])
    os.replace(tmp, out)
    return out


def build_api_bench() -> str:
    """Link host/bench/api_bench.cpp against libmensurflow.so: bench.py's timing of the
    BASELINE workloads through the C++ API."""
    out = os.path.join(LIBDIR, "mfr_api_bench")
    tmp = out + ".tmp"
    _run(["g++", *HOST_FLAGS, "-o", tmp, os.path.join(HOST, "bench", "api_bench.cpp"),
          f"-L{LIBDIR}", "-lmensurflow", "-lmfr_rocm", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, out)
    return out


def build() -> None:
    build_hip()
    if build_host() is not None:
        build_api_bench()


if __name__ == "__main__":
    build()
    print("built", LIBDIR)
