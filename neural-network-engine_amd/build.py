"""Builds the gfx950 attention library in-tree.

    python neural-network-engine_amd/build.py

produces neural-network-engine_amd/lib/libnne_attn.so (HIP kernels + C ABI) and
neural-network-engine_amd/lib/libnne_host.so (the C++ host API of host/nne.hpp,
on top of the C ABI and rocBLAS).
Every build recompiles; nothing is cached outside the repository, so the
built file travels with the tree to the GPU machine.
"""
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB_DIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIB_DIR, "libnne_attn.so")
HOST_LIB = os.path.join(LIB_DIR, "libnne_host.so")

SOURCES = ["prefill.hip", "small.hip", "splitk.hip", "splitk_plan.cpp", "qkv.hip", "deep.hip", "deep_plan.cpp", "abi.cpp", "noalloc.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # packed FP32 instructions are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def hipcc():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def _run(cmd, out, verbose):
    tmp = out + ".tmp"
    cmd = cmd + ["-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + err)
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, out)
    return out


def build_library(verbose=False):
    os.makedirs(LIB_DIR, exist_ok=True)
    cmd = [hipcc()] + HIPCC_FLAGS + [
        "-I" + os.path.join(ROOT, "include"),
        "-I" + CSRC,
    ] + [os.path.join(CSRC, s) for s in SOURCES]
    return _run(cmd, LIB, verbose)


def build_host_library(verbose=False):
    """The C++ host API; links libnne_attn.so from the same directory."""
    cmd = [hipcc()] + HIPCC_FLAGS + [
        "-I" + os.path.join(ROOT, "include"),
        "-I" + os.path.join(PKG, "host"),
        os.path.join(PKG, "host", "nne_host.hip"),
        "-L" + LIB_DIR, "-lnne_attn",
        "-L" + os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib"), "-lrocblas",
        "-Wl,-rpath,$ORIGIN",
    ]
    return _run(cmd, HOST_LIB, verbose)


def build_all(verbose=False):
    return [build_library(verbose), build_host_library(verbose)]


if __name__ == "__main__":
    for path in build_all(verbose=True):
        print(path)
