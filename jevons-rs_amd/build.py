"""Builds the gfx950 code object and the host library in-tree.

Outputs (git-ignored, shipped with the tree):
  jevons-rs_amd/lib/jevons_qmm.hsaco    kernels, loaded at run time with hipModuleLoad
  jevons-rs_amd/lib/libjevons_qmm.so    C ABI of include/jevons_qmm.h (host code, plus the
                                        fixed device array of jv_matmul_noalloc in its own
                                        gfx950 code object)

Run as a script (``python jevons-rs_amd/build.py``) or call ``build()``.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_DIR = os.path.join(HERE, "lib")
HSACO = os.path.join(LIB_DIR, "jevons_qmm.hsaco")
SO = os.path.join(LIB_DIR, "libjevons_qmm.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

KERNEL_SRC = os.path.join(HERE, "csrc", "kernels", "qmm.hip")
HOST_SRC = os.path.join(HERE, "csrc", "host", "jevons_qmm.cpp")
TUNE_SRC = os.path.join(HERE, "csrc", "host", "tune.cpp")
GGUF_SRC = os.path.join(HERE, "csrc", "host", "gguf.cpp")
NOALLOC_SRC = os.path.join(HERE, "csrc", "host", "noalloc.hip")
NOALLOC_OBJ = os.path.join(LIB_DIR, "noalloc.o")

# Packed FP32 VALU instructions are disabled for all device code.
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "--cuda-device-only", "--no-gpu-bundle-output",
]


def kernel_cmd(out: str = HSACO) -> list[str]:
    return [os.path.join(ROCM, "bin", "hipcc"), *HIPCC_FLAGS, "-c", KERNEL_SRC, "-o", out]


def noalloc_cmd(out: str = NOALLOC_OBJ) -> list[str]:
    """Host object holding a device array (host and device passes of hipcc)."""
    return [os.path.join(ROCM, "bin", "hipcc"), "--offload-arch=gfx950", "-O2", "-std=c++17", "-fPIC",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-I", os.path.join(ROOT, "include"), "-c", NOALLOC_SRC, "-o", out]


def host_cmd(out: str = SO) -> list[str]:
    return [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra",
        "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"),
        "-I", os.path.join(ROCM, "include"), HOST_SRC, TUNE_SRC, GGUF_SRC, NOALLOC_OBJ,
        "-L", os.path.join(ROCM, "lib"), "-lamdhip64", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}",
        "-o", out,
    ]


def _run_all(jobs, verbose: bool) -> None:
    """Runs (command, output) jobs in parallel; each writes output + ".tmp", renamed on success,
    so a failed build never leaves a half-written file."""
    procs = []
    for cmd, _ in jobs:
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append(subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True))
    failed = []
    for (cmd, final), p in zip(jobs, procs):
        out, _ = p.communicate()
        # hipcc's host pass warns about the device-only target feature; keep other output.
        lines = [l for l in out.splitlines() if "packed-fp32-ops" not in l]
        if p.returncode != 0:
            failed.append((cmd, "\n".join(lines)))
        else:
            if verbose and lines:
                print("\n".join(lines))
            os.replace(final + ".tmp", final)
    if failed:
        msg = "\n\n".join(" ".join(c) + "\n" + o for c, o in failed)
        raise RuntimeError("build failed:\n" + msg)


def build(verbose: bool = False) -> None:
    os.makedirs(LIB_DIR, exist_ok=True)
    _run_all([(kernel_cmd(HSACO + ".tmp"), HSACO), (noalloc_cmd(NOALLOC_OBJ + ".tmp"), NOALLOC_OBJ)], verbose)
    _run_all([(host_cmd(SO + ".tmp"), SO)], verbose)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print("built", HSACO, SO)
