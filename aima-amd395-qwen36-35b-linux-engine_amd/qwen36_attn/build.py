"""Compile the gfx950 HIP sources into the in-tree C-ABI library.

``python -m qwen36_attn.build`` (run from the package root) or
``build_library()`` compiles every ``csrc/*.hip`` to an object (in parallel)
and links ``qwen36_attn/libqwen36_attn.so``.  Packed-FP32 VALU forms are
disabled (``-packed-fp32-ops``) for every source.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
CSRC = os.path.join(ROOT, "csrc")
LIB_NAME = "libqwen36_attn.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
# Host-only C++ caller of the FMHA provider ABI (dlopen, like the engine).
HARNESS_SRC = os.path.join(ROOT, "harness", "provider_harness.cpp")
HARNESS_PATH = os.path.join(PKG_DIR, "provider_harness")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Per-source code-generation flags (none needed at present).
EXTRA_FLAGS: dict[str, list[str]] = {}


def hip_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
        "-fvisibility=hidden", "-Wall", "-Wno-unused-result",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    ]


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


_NOISE = "is not a recognized feature for this target"


def _run(cmd: list[str]) -> str:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(line for line in proc.stderr.splitlines() if _NOISE not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    return err


def build_library(verbose: bool = False) -> str:
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with tempfile.TemporaryDirectory(prefix="qwen36_build_") as tmpd:
        jobs = []
        for src in srcs:
            obj = os.path.join(tmpd, os.path.basename(src) + ".o")
            cmd = [HIPCC, *hip_flags(), *EXTRA_FLAGS.get(os.path.basename(src), []),
                   "-I", CSRC, "-c", src, "-o", obj]
            jobs.append((cmd, obj))
        workers = min(len(jobs), max(1, min(8, os.cpu_count() or 1)))
        with cf.ThreadPoolExecutor(workers) as ex:
            for (cmd, _), err in zip(jobs, ex.map(lambda j: _run(j[0]), jobs)):
                if verbose:
                    print(" ".join(cmd), flush=True)
                    if err.strip():
                        print(err, file=sys.stderr)
        tmp_lib = LIB_PATH + ".tmp"
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC",
              *[o for _, o in jobs], "-o", tmp_lib, "-L", os.path.join(ROCM, "lib"),
              "-lhipblaslt", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"])
    os.replace(tmp_lib, LIB_PATH)
    build_harness(verbose)
    return LIB_PATH


def build_harness(verbose: bool = False) -> str:
    """Compile the provider harness (plain host C++ against the HIP runtime;
    it loads the library with dlopen, so it does not link it)."""
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-D__HIP_PLATFORM_AMD__",
           "-I", os.path.join(ROCM, "include"), HARNESS_SRC, "-o", HARNESS_PATH + ".tmp",
           "-L", os.path.join(ROCM, "lib"), "-lamdhip64", "-ldl",
           f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    _run(cmd)
    os.replace(HARNESS_PATH + ".tmp", HARNESS_PATH)
    return HARNESS_PATH


if __name__ == "__main__":
    print(build_library(verbose=True))
