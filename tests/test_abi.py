"""CPU-side checks of the drop-in boundary: the HIP library loads, exports
every entry point declared in include/*.h, and rejects bad arguments on the
host before touching a GPU (no kernel is launched by these tests)."""
import ctypes
import glob
import os
import re
import subprocess

import pytest

from lmrs_amd import sampling as S

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(lmrs_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_functions()
    assert "lmrs_sample_fwd" in names and "lmrs_process_logits_fwd" in names


def test_library_exports_every_declared_symbol():
    lib = S.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_version_string():
    assert b"gfx950" in S.lib().lmrs_sampling_version()


def test_no_workspace_is_needed():
    # every working set is in LDS and registers (no device call is made)
    L = S.lib()
    for B, V, dt, H in ((256, 128256, S.DTYPE_BF16, 2048), (512, 256000, S.DTYPE_F32, 512), (1, 1, 0, 0)):
        assert L.lmrs_sample_workspace_size(B, V, dt, H) == 0


def test_args_struct_layout_matches_header(tmp_path):
    # compile the header with the C compiler and compare every field offset
    fields = [f for f, _ in S.SampleArgs._fields_]
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "lmrs_sampling.h"\nint main(void){\n'
        + 'printf("%zu\\n", sizeof(lmrs_sample_args));\n'
        + "".join(f'printf("%zu\\n", offsetof(lmrs_sample_args, {f}));\n' for f in fields)
        + "return 0;}\n"
    )
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert got[0] == ctypes.sizeof(S.SampleArgs)
    assert got[1:] == [getattr(S.SampleArgs, f).offset for f in fields]


def _args(**kw):
    a = S.SampleArgs()
    a.dtype = kw.get("dtype", S.DTYPE_BF16)
    a.batch = kw.get("batch", 1)
    a.vocab = kw.get("vocab", 8)
    a.row_stride = kw.get("row_stride", a.vocab)
    a.logits = kw.get("logits", 0x1000)
    a.token_ids = kw.get("token_ids", 0x2000)
    a.hist_offsets = kw.get("hist_offsets", None)
    a.hist_ids = kw.get("hist_ids", None)
    return a


@pytest.mark.parametrize(
    "kw,code",
    [
        (dict(dtype=S.DTYPE_F16), S.ERR_BAD_DTYPE),
        (dict(dtype=7), S.ERR_BAD_DTYPE),
        (dict(batch=-1), S.ERR_BAD_SHAPE),
        (dict(vocab=-3), S.ERR_BAD_SHAPE),
        (dict(vocab=S.MAX_VOCAB + 1), S.ERR_BAD_SHAPE),
        (dict(vocab=16, row_stride=8), S.ERR_BAD_SHAPE),
        (dict(token_ids=None), S.ERR_NULL_ARGUMENT),
        (dict(logits=None), S.ERR_NULL_ARGUMENT),
        (dict(hist_offsets=0x3000, hist_ids=None), S.ERR_NULL_ARGUMENT),
        (dict(logits=0x1001), S.ERR_ALIGNMENT),
        (dict(batch=0), S.LMRS_OK),
    ],
)
def test_host_side_rejection(kw, code):
    a = _args(**kw)
    assert S.lib().lmrs_sample_fwd(ctypes.byref(a), None) == code


def test_null_args_pointer():
    assert S.lib().lmrs_sample_fwd(None, None) == S.ERR_NULL_ARGUMENT
    assert S.lib().lmrs_process_logits_fwd(None, None, None) == S.ERR_NULL_ARGUMENT


def test_process_needs_output():
    a = _args()
    assert S.lib().lmrs_process_logits_fwd(ctypes.byref(a), None, None) == S.ERR_NULL_ARGUMENT


def test_python_mirror_validation():
    with pytest.raises(S.SamplingError):
        S.TopK(0)
    with pytest.raises(S.SamplingError):
        S.TopP(0.0)
    with pytest.raises(S.SamplingError):
        S.TopP(1.5)
    with pytest.raises(S.SamplingError):
        S.Temperature(0.0)
    with pytest.raises(S.SamplingError):
        S.RepetitionPenalty(-1.0)
    with pytest.raises(S.SamplingError):
        S.FrequencyPresencePenalty(float("nan"), 0.0)
    with pytest.raises(S.SamplingError):
        S.BeamSearch(0)
    assert S.SamplerConfig(S.TopK(8)).with_seed(123).seed == 123
    assert S.SamplerConfig().seed == 1
    assert S.SamplerConfig().with_seed(0).seed == 1  # seed.max(1), sampler.rs:49-52
    s = S.Sampler()
    s.push_processor(S.Temperature(1.0))
    assert s.processor_count() == 1


def test_python_next_unit_matches_oracle():
    import oracle as O

    for seed in (1, 9, 42, 2**64 - 1):
        assert S.next_unit(seed) == O.next_unit(seed)


@pytest.mark.parametrize(
    "args,code",
    [
        ((0x1000, 0x2000, 0x3000, 4, 64, 100, S.DTYPE_F32, None, None), S.ERR_BAD_DTYPE),
        ((0x1000, 0x2000, 0x3000, -1, 64, 100, S.DTYPE_BF16, None, None), S.ERR_BAD_SHAPE),
        ((0x1000, 0x2000, 0x3000, 4, 60, 100, S.DTYPE_BF16, None, None), S.ERR_BAD_SHAPE),  # in % 8
        ((None, 0x2000, 0x3000, 4, 64, 100, S.DTYPE_BF16, None, None), S.ERR_NULL_ARGUMENT),
        ((0x1000, None, 0x3000, 4, 64, 100, S.DTYPE_BF16, None, None), S.ERR_NULL_ARGUMENT),
        ((0x1000, 0x2008, 0x3000, 4, 64, 100, S.DTYPE_BF16, None, None), S.ERR_ALIGNMENT),
        ((0x1000, 0x2000, 0x3000, 0, 64, 100, S.DTYPE_BF16, None, None), S.LMRS_OK),  # nothing to do
    ],
)
def test_lm_head_host_side_rejection(args, code):
    assert S.lib().lmrs_lm_head_fwd(*args) == code
