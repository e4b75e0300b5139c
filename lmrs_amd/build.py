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

# one translation unit per kernel family, compiled in parallel, then linked
SOURCES = ["fast_nch40_pairs.hip", "sampling_api.hip", "fast_nch8.hip", "fast_nch16.hip", "fast_nch32.hip",
           "fast_nch40.hip",
           "generic_kernels.hip", "f32_kernel.hip", "lm_head.hip"]

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


def _run(cmd, verbose, what):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns about the device-only target feature: harmless
    errs = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln]
    if res.returncode != 0:
        sys.stderr.write("\n".join(errs) + "\n")
        raise RuntimeError(f"hipcc failed ({res.returncode}) building {what}")
    if verbose and errs:
        sys.stderr.write("\n".join(errs) + "\n")


def _build_one(sources, lib, verbose):
    from concurrent.futures import ThreadPoolExecutor

    inc = ["-I", os.path.join(ROOT, "include")]
    cflags = [f for f in FLAGS if f != "-shared"]
    objs = [lib + f".{os.path.splitext(s)[0]}.o" for s in sources]
    jobs = [([HIPCC, *cflags, *inc, "-c", os.path.join(CSRC, s), "-o", o], o) for s, o in zip(sources, objs)]
    with ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 1)) as ex:
        for f in [ex.submit(_run, cmd, verbose, o) for cmd, o in jobs]:
            f.result()
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", lib + ".tmp"], verbose, lib)
    for o in objs:
        os.remove(o)
    os.replace(lib + ".tmp", lib)


if __name__ == "__main__":
    print(build(verbose=True))
