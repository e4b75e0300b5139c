"""Builds the HIP sampling library in-tree: lmrs_amd/liblmrs_sampling.so (gfx950).

Run as ``python -m lmrs_amd.build`` or through ``__graft_entry__.build()``.
The library is built by hipcc directly (no PyTorch extension machinery): it
exports the plain C-ABI of include/lmrs_sampling.h.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "liblmrs_sampling.so")

SOURCES = ["sampling_api.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # the reference never fuses multiply-add except in its affine kernel,
    # which the sources spell as an explicit fma
    "-ffp-contract=off",
    # packed-FP32 instructions are kept out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


# bench.py's measured streaming ceiling: a read-only kernel with the sampler's
# access shape, in a library of its own (not part of the sampling ABI)
PROBE_LIB = os.path.join(HERE, "liblmrs_stream_probe.so")
PROBE_SOURCES = ["stream_probe.hip"]


def build(verbose: bool = False) -> str:
    _build_one(SOURCES, LIB, verbose)
    _build_one(PROBE_SOURCES, PROBE_LIB, verbose)
    return LIB


def _build_one(sources, lib, verbose):
    srcs = [os.path.join(CSRC, s) for s in sources]
    cmd = [HIPCC, *FLAGS, "-I", os.path.join(ROOT, "include"), *srcs, "-o", lib + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns about the device-only target feature: harmless
    errs = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln]
    if res.returncode != 0:
        sys.stderr.write("\n".join(errs) + "\n")
        raise RuntimeError(f"hipcc failed ({res.returncode}) building {lib}")
    if verbose and errs:
        sys.stderr.write("\n".join(errs) + "\n")
    os.replace(lib + ".tmp", lib)


if __name__ == "__main__":
    print(build(verbose=True))
