"""Builds libnpa_hip.so in-tree with hipcc for gfx950.

The device code is compiled with -ffp-contract=off (no a*b+c fusion, as in the
reference's Rust arithmetic) and with packed FP32 instructions disabled.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libnpa_hip.so")
SOURCES = ["npa_hashgrid.hip", "npa_perception.hip", "npa_update.hip", "npa_adjoint.hip", "npa_decode.hip",
           "npa_sort.hip", "npa_abi.hip", "npa_bpk.cpp"]
# npa_perception.hip and npa_update.hip compile as three objects each (NPA_PART selects which
# kernels each holds)
PARTS = {"npa_perception.hip": ["-DNPA_PART=0", "-DNPA_PART=2", "-DNPA_PART=3"],
         "npa_update.hip": ["-DNPA_PART=0", "-DNPA_PART=2", "-DNPA_PART=3"]}
ARCH = os.environ.get("NPA_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the HIP library cannot be built")


FLAGS = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Xclang", "-target-feature",
         "-Xclang", "-packed-fp32-ops", "-Wall", "-Wno-unused-variable", "-Wno-unused-function",
         # the neighbour filters combine bools with & on purpose (branch-free)
         "-Wno-bitwise-instead-of-logical"]
NOISE = "'-packed-fp32-ops' is not a recognized feature"


def command(out: str = LIB) -> list:
    """One-shot compile-and-link command (the build runs the same flags per source in parallel)."""
    return [hipcc(), f"--offload-arch={ARCH}", "-shared"] + FLAGS + ["-o", out] + \
        [os.path.join(CSRC, s) for s in SOURCES]


def _check(proc, what: str) -> str:
    errs = "\n".join(l for l in proc.stderr.splitlines() if NOISE not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {what} ({proc.returncode}):\n{errs}")
    return errs


def build(verbose: bool = False) -> str:
    """Compiles every source to an object in parallel, then links libnpa_hip.so."""
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    jobs = []
    for src in SOURCES:
        for k, part in enumerate(PARTS.get(src, [None])):
            obj = os.path.join(objdir, os.path.splitext(src)[0] + f"_{k}.o")
            cmd = [hipcc(), f"--offload-arch={ARCH}", "-c"] + FLAGS + ([part] if part else []) + \
                ["-o", obj, os.path.join(CSRC, src)]
            jobs.append((src, obj, cmd))
    with ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 1)) as pool:
        procs = list(pool.map(lambda j: subprocess.run(j[2], capture_output=True, text=True), jobs))
    log = [_check(proc, src) for (src, _, _), proc in zip(jobs, procs)]
    objs = [obj for _, obj, _ in jobs]
    tmp = LIB + ".tmp"
    link = subprocess.run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs,
                          capture_output=True, text=True)
    log.append(_check(link, "link"))
    if verbose and any(l.strip() for l in log):
        print("\n".join(log), file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
