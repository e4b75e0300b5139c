"""The fast kernel's explicitly issued loads are never touched before their
waits (see tests/isa_hazards.py), in every instantiation."""
import os
import subprocess

import pytest

from isa_hazards import kernel_names, scan

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    import sys

    sys.path.insert(0, ROOT)
    from lmrs_amd import build

    out = tmp_path_factory.mktemp("isa") / "sampling.s"
    flags = [f for f in build.FLAGS if f not in ("-fPIC", "-shared")]
    cmd = [build.HIPCC, *flags, "--cuda-device-only", "-S", "-I", os.path.join(ROOT, "include"),
           os.path.join(build.CSRC, "sampling_api.hip"), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        pytest.skip(f"hipcc unavailable or failed: {res.stderr[-300:]}")
    return out.read_text()


def test_fast_kernels_have_no_load_hazards(asm):
    names = kernel_names(asm, "_ZN4lmrs16bf16_fast_kernel")
    assert len(names) == 4, names
    for k in names:
        assert scan(asm, k) == [], k


def test_scanner_flags_a_reused_destination():
    planted = "\n".join([
        "kern:",
        "\t;;#ASMSTART",
        "\tglobal_load_ushort v18, v[54:55], off",
        "\t;;#ASMEND",
        "\tv_mov_b32_e32 v18, 0",
        "\ts_waitcnt vmcnt(0)",
        ".Lfunc_end0:",
    ])
    assert len(scan(planted, "kern")) == 1
    waited = planted.replace("\tv_mov_b32_e32 v18, 0\n\ts_waitcnt vmcnt(0)", "\ts_waitcnt vmcnt(0)\n\tv_mov_b32_e32 v18, 0")
    assert scan(waited, "kern") == []


def test_stream_probe_has_no_load_hazards(tmp_path):
    # bench.py's streaming-ceiling kernel issues its loads the same way
    import sys
    sys.path.insert(0, ROOT)
    from lmrs_amd import build
    out = tmp_path / "probe.s"
    flags = [f for f in build.FLAGS if f not in ("-fPIC", "-shared")]
    cmd = [build.HIPCC, *flags, "--cuda-device-only", "-S", os.path.join(build.CSRC, "stream_probe.hip"),
           "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        pytest.skip(f"hipcc unavailable or failed: {res.stderr[-300:]}")
    asm = out.read_text()
    names = kernel_names(asm, "_ZN12_GLOBAL__N_112probe_kernel")
    assert len(names) == 4, names
    for k in names:
        assert scan(asm, k) == [], k
