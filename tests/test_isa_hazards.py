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

    from concurrent.futures import ThreadPoolExecutor

    tmp = tmp_path_factory.mktemp("isa")
    flags = [f for f in build.FLAGS if f not in ("-fPIC", "-shared")]
    srcs = [s for s in build.SOURCES if s.startswith("fast_nch")]

    def one(src):
        out = tmp / (src + ".s")
        cmd = [build.HIPCC, *flags, "--cuda-device-only", "-S", "-I", os.path.join(ROOT, "include"),
               os.path.join(build.CSRC, src), "-o", str(out)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        return res, out

    with ThreadPoolExecutor(max_workers=len(srcs)) as ex:
        results = list(ex.map(one, srcs))
    for res, _ in results:
        if res.returncode != 0:
            pytest.skip(f"hipcc unavailable or failed: {res.stderr[-300:]}")
    return "\n".join(out.read_text() for _, out in results)


def test_fast_kernels_have_no_load_hazards(asm):
    names = kernel_names(asm, "_ZN4lmrs16bf16_fast_kernel")
    assert len(names) == 4, names
    pairs = kernel_names(asm, "_ZN4lmrs23bf16_fast_rounds_kernel")  # two rows per workgroup
    assert len(pairs) == 1, pairs
    for k in names + pairs:
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


def test_scanner_follows_branches():
    # a load, then a branch: the fall-through reads the destination before any
    # wait (a hazard); the taken side waits first (none); a join after both
    # sees only waited queues
    body = [
        "kern:",
        "\t;;#ASMSTART",
        "\tglobal_load_dwordx4 v[10:13], v[2:3], off nt",
        "\t;;#ASMEND",
        "\ts_cbranch_scc1 .LBB0_2",
        "\tv_mov_b32_e32 v20, v11",
        "\ts_waitcnt vmcnt(0)",
        "\ts_branch .LBB0_3",
        ".LBB0_2:",
        "\ts_waitcnt vmcnt(0)",
        "\tv_mov_b32_e32 v21, v12",
        ".LBB0_3:",
        "\tv_mov_b32_e32 v22, v13",
        "\ts_endpgm",
        ".Lfunc_end0:",
    ]
    found = scan("\n".join(body), "kern")
    assert len(found) == 1 and "v20, v11" in found[0], found
    # the same read on the taken side only, with the wait on the fall-through: a hazard
    body2 = [ln.replace("v_mov_b32_e32 v21, v12", "v_mov_b32_e32 v21, v12\n\tv_mov_b32_e32 v23, v10")
             .replace("\ts_waitcnt vmcnt(0)\n\tv_mov_b32_e32 v21", "\tv_mov_b32_e32 v21") for ln in body]
    body2 = "\n".join(body2).replace(".LBB0_2:\n\ts_waitcnt vmcnt(0)\n", ".LBB0_2:\n")
    found2 = scan(body2, "kern")
    assert any("v21, v12" in f for f in found2) and any("v23, v10" in f for f in found2), found2
    # a long branch (s_getpc / s_add_u32 / s_setpc) to a block that reads unwaited
    lb = [
        "kern:",
        "\t;;#ASMSTART",
        "\tglobal_load_dword v30, v[2:3], off",
        "\t;;#ASMEND",
        "\ts_getpc_b64 s[98:99]",
        ".Lpost_getpc0:",
        "\ts_add_u32 s98, s98, (.LBB0_9-.Lpost_getpc0)&4294967295",
        "\ts_addc_u32 s99, s99, (.LBB0_9-.Lpost_getpc0)>>32",
        "\ts_setpc_b64 s[98:99]",
        "\ts_waitcnt vmcnt(0)",
        "\tv_mov_b32_e32 v31, v30",
        ".LBB0_9:",
        "\tv_mov_b32_e32 v32, v30",
        "\ts_endpgm",
        ".Lfunc_end0:",
    ]
    found3 = scan("\n".join(lb), "kern")
    assert len(found3) == 1 and "v32, v30" in found3[0], found3


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


def test_no_bit_cast_of_a_vector_element():
    # hipcc compiles __builtin_bit_cast(T, v[i]) of an element of a vector
    # reference as a cast of v[0] (seen on the int16 chunk maximum): the
    # kernels copy elements to scalars before casting them
    import re

    csrc = os.path.join(ROOT, "lmrs_amd", "csrc")
    pat = re.compile(r"__builtin_bit_cast\([^,()]+,\s*[A-Za-z_]\w*\s*\[")
    for name in sorted(os.listdir(csrc)):
        text = open(os.path.join(csrc, name)).read()
        assert not pat.search(text), name
