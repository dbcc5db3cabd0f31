"""The C ABI library: it loads, exports exactly what include/vsampler.h declares, and rejects
bad arguments with the documented codes before touching a GPU."""

from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from vinfer_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "vsampler.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(vsamp_\w+)\s*\(", text, re.M)))


def test_library_is_built_and_loads():
    assert _lib.LIB_PATH.exists(), "run python -m vinfer_amd.csrc.build"
    lib = _lib.load()
    assert lib.vsamp_abi_version() == _lib.ABI_VERSION


def test_abi_version_is_one_number_everywhere():
    # the header's version, the binding's, and the one the integration guide's snippet asserts
    header = int(re.search(r"#define VSAMP_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    guide = (HEADER.parents[1] / "INTEGRATION.md").read_text()
    snippet = int(re.search(r"^VSAMP_ABI_VERSION = (\d+)", guide, re.M).group(1))
    assert header == _lib.ABI_VERSION == snippet


def test_every_declared_symbol_is_exported():
    names = declared()
    assert names == sorted(_lib.EXPORTS)
    lib = _lib.load()
    for n in names:
        assert hasattr(lib, n), n


def test_header_struct_matches_the_binding(tmp_path):
    # Field names in order, and every offset and the size as the C compiler lays them out.
    text = HEADER.read_text()
    body = text[text.index("typedef struct vsamp_args") : text.index("} vsamp_args;")]
    fields = re.findall(r"^\s*[\w\s\*]+?\b(\w+);", body, re.M)
    assert fields == [f for f, _ in _lib.VsampArgs._fields_]
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    src = tmp_path / "layout.c"
    lines = [f'printf("%zu\\n", offsetof(vsamp_args, {f}));' for f in fields]
    src.write_text(
        "#include <stdio.h>\n#include <stddef.h>\n#include \"vsampler.h\"\nint main(void){"
        + "".join(lines)
        + 'printf("%zu\\n", sizeof(vsamp_args));return 0;}\n'
    )
    exe = tmp_path / "layout"
    subprocess.run([gcc, f"-I{HEADER.parent}", str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [getattr(_lib.VsampArgs, f).offset for f in fields] + [ctypes.sizeof(_lib.VsampArgs)]
    assert got == want


def test_workspace_size_formula():
    lib = _lib.load()
    assert lib.vsamp_workspace_bytes(0, 1, 0) > 0 or lib.vsamp_workspace_bytes(0, 1, 0) == 0
    n = lib.vsamp_workspace_bytes(256, 151936, 256 * 4096)
    assert n >= 256 * 4 + 3 * 4 * 256 * 4096
    assert lib.vsamp_workspace_bytes(-1, 10, 0) == 0


def _args(**kw):
    a = _lib.VsampArgs()
    a.logits, a.dtype, a.batch, a.vocab, a.row_stride = 0x1000, 0, 4, 100, 100
    a.uniforms, a.out_ids = 0x2000, 0x3000
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "kw,code,msg",
    [
        ({"dtype": 7}, 2, "dtype"),
        ({"vocab": 0}, 1, "vocab"),
        ({"row_stride": 50}, 1, "row_stride"),
        ({"batch": -1}, 1, "batch"),
        ({"uniforms": None}, 1, "uniforms"),
        ({"out_ids": None}, 1, "out_ids"),
        ({"flags": 8}, 1, "flags"),
        ({"flags": 4}, 1, "VSAMP_HIST_APPEND goes with VSAMP_HIST_RANGES"),
        ({"flags": 5}, 1, "VSAMP_HIST_APPEND needs penalties"),
        ({"draft_ids": 0x4000}, 1, "draft"),
        ({"hist_ids": 0x5000, "hist_total": 10}, 1, "hist"),
        ({"logits": None}, 1, "logits"),
    ],
)
def test_bad_arguments_are_rejected_with_their_code(kw, code, msg):
    lib = _lib.load()
    rc = lib.vsamp_sample(ctypes.byref(_args(**kw)), None)
    assert rc == code
    assert msg in lib.vsamp_last_error().decode()
    with pytest.raises(_lib.VsamplerError, match=msg):
        _lib.check(rc)


def test_empty_batch_is_a_no_op():
    lib = _lib.load()
    assert lib.vsamp_sample(ctypes.byref(_args(batch=0)), None) == 0
    assert lib.vsamp_last_error() == b""


def test_query_names_the_problem_without_a_gpu():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    reason = _lib.query(0)
    assert reason and "device" in reason


def test_host_uniforms_equal_the_python_derivation():
    # vsamp_uniforms (BLAKE2b-8 + SplitMix64 in C, on the host) against the Python derivation
    # over hashlib, whose position_seed the oracle tests pin to known values; signs, the int64
    # extremes and long decimal texts included.
    import numpy as np

    from vinfer_amd.sampling import uniform

    rng = np.random.default_rng(5)
    seeds = [0, 7, 8, -1, -(1 << 63), (1 << 63) - 1, 1 << 62, 9] + rng.integers(
        -(1 << 63), (1 << 63) - 1, 3000, dtype=np.int64
    ).tolist()
    positions = [0, 1, 2, 3, 10**12, (1 << 63) - 1, -5, 99] + rng.integers(0, 1 << 40, 3000).tolist()
    # every decimal length of both numbers, signed: 10^k - 1, 10^k, 10^k + 1 crossed
    edges = sorted({v for k in range(19) for v in (10**k - 1, 10**k, 10**k + 1)} | {(1 << 63) - 1})
    edges += [-v for v in edges if v > 0] + [-(1 << 63)]
    pairs = [(a, b) for a in edges for b in edges[::3]] + [(a, b) for a in edges[1::3] for b in edges]
    seeds += [a for a, _ in pairs]
    positions += [b for _, b in pairs]
    got = _lib.position_uniforms(seeds, positions)
    want = np.array([uniform(s, p) for s, p in zip(seeds, positions)], np.float32)
    assert np.array_equal(got, want)
    big = _lib.position_uniforms([1 << 70, 3], [4, 4])  # outside int64: the Python derivation
    assert big.tolist() == [uniform(1 << 70, 4), uniform(3, 4)]
    lib = _lib.load()
    assert lib.vsamp_uniforms(None, None, -1, None) == 1
    assert lib.vsamp_uniforms(None, None, 0, None) == 0


def test_verify_arguments_are_checked_before_any_launch():
    lib = _lib.load()
    v = _lib.VsampVerifyArgs()
    v.target = _args(batch=6, out_ids=None)
    v.draft = _args(batch=3, uniforms=None, out_ids=None)
    v.batch, v.num_draft = 3, 1
    v.draft_tokens = v.u_accept = v.u_residual = v.out_tokens = v.out_count = 0x6000
    cases = [
        ({"num_draft": 0}, "num_draft"),
        ({"batch": 2}, "target.batch"),
        ({"draft_tokens": None}, "draft_tokens"),
    ]
    for kw, msg in cases:
        w = _lib.VsampVerifyArgs.from_buffer_copy(v)
        for k, val in kw.items():
            setattr(w, k, val)
        assert lib.vsamp_verify(ctypes.byref(w), None) == 1
        assert msg in lib.vsamp_last_error().decode()
    w = _lib.VsampVerifyArgs.from_buffer_copy(v)
    w.target.out_ids = 0x3000  # outputs of the inner calls belong to the call
    assert lib.vsamp_verify(ctypes.byref(w), None) == 1 and b"leave them NULL" in lib.vsamp_last_error()
    w = _lib.VsampVerifyArgs.from_buffer_copy(v)
    w.target.out_ids = None
    w.target.hist_ids, w.target.hist_offsets, w.target.hist_total = 0x7000, 0x7100, 10
    w.target.repetition_penalty = 0x7200
    assert lib.vsamp_verify(ctypes.byref(w), None) == 1 and b"penalties" in lib.vsamp_last_error()
    assert lib.vsamp_verify_workspace_bytes(3, 1) > 0 and lib.vsamp_verify_workspace_bytes(3, 0) == 0


def test_verify_struct_matches_the_binding(tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    fields = [f for f, _ in _lib.VsampVerifyArgs._fields_]
    src = tmp_path / "vlayout.c"
    lines = [f'printf("%zu\\n", offsetof(vsamp_verify_args, {f}));' for f in fields]
    src.write_text(
        "#include <stdio.h>\n#include <stddef.h>\n#include \"vsampler.h\"\nint main(void){"
        + "".join(lines)
        + 'printf("%zu\\n", sizeof(vsamp_verify_args));return 0;}\n'
    )
    exe = tmp_path / "vlayout"
    subprocess.run([gcc, f"-I{HEADER.parent}", str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [getattr(_lib.VsampVerifyArgs, f).offset for f in fields] + [ctypes.sizeof(_lib.VsampVerifyArgs)]
    assert got == want


def test_lm_head_struct_matches_the_binding(tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    fields = [f for f, _ in _lib.VsampLmHeadArgs._fields_]
    src = tmp_path / "llayout.c"
    lines = [f'printf("%zu\\n", offsetof(vsamp_lm_head_args, {f}));' for f in fields]
    src.write_text(
        "#include <stdio.h>\n#include <stddef.h>\n#include \"vsampler.h\"\nint main(void){"
        + "".join(lines)
        + 'printf("%zu\\n", sizeof(vsamp_lm_head_args));printf("%d\\n", VSAMP_LM_TILE);return 0;}\n'
    )
    exe = tmp_path / "llayout"
    subprocess.run([gcc, f"-I{HEADER.parent}", str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [getattr(_lib.VsampLmHeadArgs, f).offset for f in fields] + [ctypes.sizeof(_lib.VsampLmHeadArgs), _lib.LM_TILE]
    assert got == want


def test_lm_head_arguments_are_checked_before_any_launch():
    lib = _lib.load()
    a = _lib.VsampLmHeadArgs()
    a.batch, a.dim, a.vocab = 2, 100, 10
    a.hidden_stride, a.weight_stride, a.logits_stride = 100, 100, 10
    assert lib.vsamp_lm_head(ctypes.byref(a), None) == 1 and b"multiple of 64" in lib.vsamp_last_error()
    a.dim = a.hidden_stride = a.weight_stride = 128
    assert lib.vsamp_lm_head(ctypes.byref(a), None) == 1 and b"must be set" in lib.vsamp_last_error()
    a.batch = 0
    assert lib.vsamp_lm_head(ctypes.byref(a), None) == 0  # (an empty batch is a no-op)
