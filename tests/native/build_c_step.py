"""Builds the native test programs: tests/native/c_step, the C caller of libnpa_hip.so (gcc, linked
against the in-tree library with an rpath to it), and tests/native/mfma_product, the check that a
matrix-core product equals the vector multiply (hipcc for gfx950)."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(HERE, "c_step")
MFMA_OUT = os.path.join(HERE, "mfma_product")


def build(out: str = OUT) -> str:
    lib_dir = os.path.join(ROOT, "burn_automata_amd")
    rpath = os.path.relpath(lib_dir, os.path.dirname(os.path.abspath(out)))
    subprocess.run(["gcc", "-O2", "-std=c11", "-Wall", "-Wextra", "-o", out, os.path.join(HERE, "c_step.c"),
                    "-L" + lib_dir, "-lnpa_hip", "-Wl,-rpath,$ORIGIN/" + rpath],
                   check=True, capture_output=True, text=True)
    return out


def build_mfma_product(out: str = MFMA_OUT) -> str:
    from burn_automata_amd import build as hip_build

    subprocess.run([hip_build.hipcc(), f"--offload-arch={hip_build.ARCH}", "-O2", "-ffp-contract=off",
                    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-x", "hip",
                    "-o", out, os.path.join(HERE, "mfma_product.cpp")],
                   check=True, capture_output=True, text=True)
    return out


if __name__ == "__main__":
    print(build())
    print(build_mfma_product())
