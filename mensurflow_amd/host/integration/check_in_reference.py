"""Builds mensurflow itself with this repository's ROCm backend wired in, and runs mensurflow's own
test suite against it. CPU container only: it needs the reference sources, and nothing it builds
is used by the product or leaves the work directory (`--work`; by default a fresh temporary
directory outside the repository, removed at the end).

Steps:
  1. copy the reference tree (without .git) to <work>/tree;
  2. apply rocm_wiring.patch (the additive core changes: the DeviceType, registration,
     execution and default device lists, OpId::Gemm/StridedCopy/Attention and their OpArgs
     fields, Stream::copy_d2d, device-side packing in Tensor, the fused gemm and attention
     dispatches, the CMake option, and the batched GEMM test's GPU expectation);
  3. drop in src/backends/rocm/backend.cpp and mfr_rocm.h from this repository;
  4. compile the library's sources (the list in the patched CMakeLists.txt plus the ROCm backend)
     with g++ and MENSURFLOW_HAS_ROCM=1, linked against mensurflow_amd/_lib/libmfr_rocm.so;
  5. compile and run every test the CMakeLists registers (mensurflow_add_test).

The reference's build system is not run: its CMakeLists.txt is read only for the two lists, and
the compile flags are those its Release configuration uses (-O3 -DNDEBUG, OpenMP, -ffp-contract=off
for optimizer.cpp). Without a GPU the ROCm backend reports 0 devices and the registry drops it,
so the suite checks that the wiring compiles, links and leaves the CPU path as it was; with a
gfx950 device the device-generic tests run on rocm:0 too.

Usage: python mensurflow_amd/host/integration/check_in_reference.py [--reference DIR]
       [--work DIR] [--keep] [--jobs N]
"""
from __future__ import annotations

import argparse
import concurrent.futures
import os
import re
import shutil
import subprocess
import sys
import tarfile
import tempfile
import time

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.abspath(os.path.join(HERE, "..", "..", ".."))
PATCH = os.path.join(HERE, "rocm_wiring.patch")
BACKEND = os.path.join(REPO, "mensurflow_amd", "host", "src", "backends", "rocm", "backend.cpp")
ABI_HEADER = os.path.join(REPO, "include", "mfr_rocm.h")
LIBDIR = os.path.join(REPO, "mensurflow_amd", "_lib")

CXXFLAGS = ["-std=c++17", "-O3", "-DNDEBUG", "-fPIC", "-fopenmp", "-Wall", "-Wextra"]


def log(msg: str) -> None:
    print(msg, flush=True)


def copy_tree(reference: str, dest: str) -> None:
    if os.path.exists(dest):
        shutil.rmtree(dest)
    os.makedirs(dest)
    tmp = dest + ".tar"
    with tarfile.open(tmp, "w") as tar:
        for entry in os.listdir(reference):
            if entry != ".git":
                tar.add(os.path.join(reference, entry), arcname=entry)
    with tarfile.open(tmp) as tar:
        tar.extractall(dest)
    os.remove(tmp)


def cmake_lists(tree: str) -> tuple[list[str], list[tuple[str, str]]]:
    """(library sources, [(test name, test source)]) as the CMakeLists lists them."""
    text = open(os.path.join(tree, "CMakeLists.txt")).read()
    library = re.search(r"add_library\(mensurflow\s+(.*?)\)", text, re.S)
    if library is None:
        raise RuntimeError("add_library(mensurflow ...) not found in CMakeLists.txt")
    sources = [s for s in library.group(1).split() if s.endswith(".cpp")]
    tests = re.findall(r"^mensurflow_add_test\((\w+)\s+([\w/.]+)\)", text, re.M)
    return sources, tests


def run(cmd: list[str], cwd: str, what: str) -> str:
    proc = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{' '.join(cmd)}\n{proc.stdout}{proc.stderr}")
    return proc.stdout + proc.stderr


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("--work", default=None,
                    help="work directory (default: a temporary directory, removed afterwards)")
    ap.add_argument("--keep", action="store_true", help="keep the temporary work directory")
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--test-timeout", type=int, default=600)
    args = ap.parse_args()
    if not os.path.isdir(os.path.join(args.reference, "src")):
        log(f"reference sources not found at {args.reference}")
        return 2
    if not os.path.exists(os.path.join(LIBDIR, "libmfr_rocm.so")):
        log("mensurflow_amd/_lib/libmfr_rocm.so is missing: build it first (python -m mensurflow_amd.build)")
        return 2
    temporary = args.work is None
    work = tempfile.mkdtemp(prefix="mfr_refdrop_") if temporary else args.work
    try:
        return check(args, work)
    finally:
        if temporary and not args.keep:
            shutil.rmtree(work, ignore_errors=True)


def check(args: argparse.Namespace, work: str) -> int:
    start = time.time()
    tree = os.path.join(work, "tree")
    build = os.path.join(work, "build")
    log(f"[1/5] copying {args.reference} -> {tree}")
    copy_tree(args.reference, tree)
    log("[2/5] applying rocm_wiring.patch")
    with open(PATCH) as patch:
        proc = subprocess.run(["patch", "-p1", "--forward", "--batch"], cwd=tree, stdin=patch,
                              capture_output=True, text=True)
    if proc.returncode != 0:
        log(proc.stdout + proc.stderr)
        return 1
    log("[3/5] dropping in src/backends/rocm/{backend.cpp, mfr_rocm.h}")
    rocm_dir = os.path.join(tree, "src", "backends", "rocm")
    os.makedirs(rocm_dir, exist_ok=True)
    shutil.copy(BACKEND, os.path.join(rocm_dir, "backend.cpp"))
    shutil.copy(ABI_HEADER, os.path.join(rocm_dir, "mfr_rocm.h"))

    sources, tests = cmake_lists(tree)
    sources.append("src/backends/rocm/backend.cpp")
    os.makedirs(os.path.join(build, "obj"), exist_ok=True)
    os.makedirs(os.path.join(build, "bin"), exist_ok=True)
    include = ["-I" + os.path.join(tree, "include"), "-I" + os.path.join(tree, "src")]

    def compile_one(src: str) -> tuple[str, str]:
        obj = os.path.join(build, "obj", src.replace("/", "_") + ".o")
        extra = ["-ffp-contract=off"] if src.endswith("ops/optimizer.cpp") else []
        out = run(["g++", *CXXFLAGS, *extra, "-DMENSURFLOW_HAS_ROCM=1", *include, "-c",
                   os.path.join(tree, src), "-o", obj], tree, f"compile {src}")
        return obj, out

    log(f"[4/5] compiling {len(sources)} library sources (ROCm backend included)")
    with concurrent.futures.ThreadPoolExecutor(args.jobs) as pool:
        results = list(pool.map(compile_one, sources))
    warnings = [(src, out) for src, (_, out) in zip(sources, results) if out.strip()]
    for src, out in warnings:
        if "rocm" in src:
            log(f"warnings in {src}:\n{out}")
    library = os.path.join(build, "libmensurflow.so")
    run(["g++", "-shared", "-fopenmp", "-o", library, *[obj for obj, _ in results],
         f"-L{LIBDIR}", "-lmfr_rocm", f"-Wl,-rpath,{LIBDIR}"], tree, "link libmensurflow.so")
    symbols = run(["nm", "-DC", library], tree, "nm")
    if "register_rocm_backend" not in symbols:
        log("the library does not define register_rocm_backend")
        return 1

    log(f"[5/5] compiling and running {len(tests)} tests")

    def build_test(item: tuple[str, str]) -> str:
        name, src = item
        exe = os.path.join(build, "bin", name)
        run(["g++", *CXXFLAGS, *include, "-I" + os.path.join(tree, "tests"),
             os.path.join(tree, src), "-o", exe, f"-L{build}", "-lmensurflow",
             f"-Wl,-rpath,{build}", f"-Wl,-rpath,{LIBDIR}"], tree, f"compile {name}")
        return exe

    with concurrent.futures.ThreadPoolExecutor(args.jobs) as pool:
        exes = list(pool.map(build_test, tests))
    failed = []
    for (name, _), exe in zip(tests, exes):
        t0 = time.time()
        try:
            proc = subprocess.run([exe], cwd=tree, capture_output=True, text=True,
                                  timeout=args.test_timeout)
            ok = proc.returncode == 0
            detail = (proc.stdout + proc.stderr).strip().splitlines()[-1:] if not ok else []
        except subprocess.TimeoutExpired:
            ok, detail = False, ["timed out"]
        log(f"  {'ok  ' if ok else 'FAIL'} {name} ({time.time() - t0:.1f} s) {' '.join(detail)}")
        if not ok:
            failed.append(name)
    log(f"{len(tests) - len(failed)} of {len(tests)} reference tests passed with the ROCm backend "
        f"wired in ({time.time() - start:.0f} s)")
    return 1 if failed else 0


if __name__ == "__main__":
    sys.exit(main())
