"""ctypes binding of ``libvsampler.so`` (the C ABI in include/vsampler.h).

The library is built in-tree by ``python -m vinfer_amd.csrc.build``. Loading never falls back to
anything: if the library is missing, ``load()`` raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libvsampler.so"
ABI_VERSION = 11
ROW_STATE_BYTES = 40

VSAMP_BF16 = 0
VSAMP_F32 = 1
VSAMP_HIST_RANGES = 1
VSAMP_SPLIT_ROWS = 2
VSAMP_HIST_APPEND = 4

STATUS = {0: "ok", 1: "VSAMP_E_ARG", 2: "VSAMP_E_DTYPE", 3: "VSAMP_E_HIP", 4: "VSAMP_E_WORKSPACE", 5: "VSAMP_E_DEVICE"}

# Every symbol include/vsampler.h declares.
EXPORTS = (
    "vsamp_abi_version",
    "vsamp_query",
    "vsamp_workspace_bytes",
    "vsamp_split_workspace_bytes",
    "vsamp_sample",
    "vsamp_sample_noalloc",
    "vsamp_probs",
    "vsamp_penalized_logits",
    "vsamp_uniforms",
    "vsamp_uniforms_device",
    "vsamp_spec_advance",
    "vsamp_logprobs",
    "vsamp_logprobs_tiles",
    "vsamp_sample_tiles",
    "vsamp_sample_tile_pass",
    "vsamp_tile_stats",
    "vsamp_lm_head",
    "vsamp_sample_states",
    "vsamp_verify",
    "vsamp_verify_workspace_bytes",
    "vsamp_last_error",
)


class VsampArgs(ctypes.Structure):
    """``vsamp_args`` field for field."""

    _fields_ = [
        ("logits", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("reserved0", ctypes.c_int32),
        ("row_stride", ctypes.c_int64),
        ("temperature", ctypes.c_void_p),
        ("top_k", ctypes.c_void_p),
        ("top_p", ctypes.c_void_p),
        ("min_p", ctypes.c_void_p),
        ("repetition_penalty", ctypes.c_void_p),
        ("presence_penalty", ctypes.c_void_p),
        ("frequency_penalty", ctypes.c_void_p),
        ("hist_ids", ctypes.c_void_p),
        ("hist_offsets", ctypes.c_void_p),
        ("hist_total", ctypes.c_int64),
        ("uniforms", ctypes.c_void_p),
        ("draft_ids", ctypes.c_void_p),
        ("out_ids", ctypes.c_void_p),
        ("out_draft_prob", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("flags", ctypes.c_uint32),
        ("reserved1", ctypes.c_uint32),
    ]


LM_TILE = 128  # VSAMP_LM_TILE: logits per statistics tile


class VsampLmHeadArgs(ctypes.Structure):
    """``vsamp_lm_head_args`` field for field."""

    _fields_ = [
        ("hidden", ctypes.c_void_p),
        ("hidden_stride", ctypes.c_int64),
        ("weight", ctypes.c_void_p),
        ("weight_stride", ctypes.c_int64),
        ("logits", ctypes.c_void_p),
        ("logits_stride", ctypes.c_int64),
        ("tile_max", ctypes.c_void_p),
        ("tile_sum", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("dim", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class VsampVerifyArgs(ctypes.Structure):
    """``vsamp_verify_args`` field for field."""

    _fields_ = [
        ("target", VsampArgs),
        ("draft", VsampArgs),
        ("batch", ctypes.c_int32),
        ("num_draft", ctypes.c_int32),
        ("draft_tokens", ctypes.c_void_p),
        ("u_accept", ctypes.c_void_p),
        ("u_residual", ctypes.c_void_p),
        ("out_tokens", ctypes.c_void_p),
        ("out_count", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("draft_states", ctypes.c_void_p),
    ]


class VsamplerError(RuntimeError):
    """A failed library call; ``code`` is the VSAMP_E_* status."""

    def __init__(self, code: int, message: str) -> None:
        super().__init__(f"{STATUS.get(code, code)}: {message}")
        self.code = code


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """The loaded library (once per process); raises if it is missing or mismatched."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise FileNotFoundError(
                f"{LIB_PATH} is not built; run `python -m vinfer_amd.csrc.build` (needs hipcc)"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.vsamp_abi_version.restype = ctypes.c_int
        lib.vsamp_query.argtypes = [ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t]
        lib.vsamp_query.restype = ctypes.c_int
        lib.vsamp_workspace_bytes.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int64]
        lib.vsamp_workspace_bytes.restype = ctypes.c_size_t
        lib.vsamp_split_workspace_bytes.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int64]
        lib.vsamp_split_workspace_bytes.restype = ctypes.c_size_t
        lib.vsamp_sample.argtypes = [ctypes.POINTER(VsampArgs), ctypes.c_void_p]
        lib.vsamp_sample.restype = ctypes.c_int
        lib.vsamp_sample_noalloc.argtypes = [ctypes.POINTER(VsampArgs), ctypes.c_void_p]
        lib.vsamp_sample_noalloc.restype = ctypes.c_int
        lib.vsamp_probs.argtypes = [ctypes.POINTER(VsampArgs), ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
        lib.vsamp_probs.restype = ctypes.c_int
        lib.vsamp_penalized_logits.argtypes = [
            ctypes.POINTER(VsampArgs),
            ctypes.c_void_p,
            ctypes.c_void_p,
            ctypes.c_int64,
            ctypes.c_void_p,
        ]
        lib.vsamp_penalized_logits.restype = ctypes.c_int
        lib.vsamp_sample_states.argtypes = [ctypes.POINTER(VsampArgs), ctypes.c_void_p, ctypes.c_void_p]
        lib.vsamp_sample_states.restype = ctypes.c_int
        lib.vsamp_verify.argtypes = [ctypes.POINTER(VsampVerifyArgs), ctypes.c_void_p]
        lib.vsamp_verify.restype = ctypes.c_int
        lib.vsamp_verify_workspace_bytes.argtypes = [ctypes.c_int32, ctypes.c_int32]
        lib.vsamp_verify_workspace_bytes.restype = ctypes.c_size_t
        lib.vsamp_logprobs.argtypes = [
            ctypes.POINTER(VsampArgs),
            ctypes.c_void_p,
            ctypes.c_int32,
            ctypes.c_void_p,
            ctypes.c_void_p,
            ctypes.c_void_p,
            ctypes.c_void_p,
        ]
        lib.vsamp_logprobs.restype = ctypes.c_int
        lib.vsamp_logprobs_tiles.argtypes = [ctypes.POINTER(VsampArgs), ctypes.c_void_p, ctypes.c_void_p] + [
            ctypes.c_void_p,
            ctypes.c_int32,
            ctypes.c_void_p,
            ctypes.c_void_p,
            ctypes.c_void_p,
            ctypes.c_void_p,
        ]
        lib.vsamp_logprobs_tiles.restype = ctypes.c_int
        lib.vsamp_sample_tiles.argtypes = [ctypes.POINTER(VsampArgs), ctypes.c_void_p, ctypes.c_void_p]
        lib.vsamp_sample_tiles.restype = ctypes.c_int
        lib.vsamp_sample_tile_pass.argtypes = [ctypes.POINTER(VsampArgs), ctypes.c_void_p, ctypes.c_void_p,
                                               ctypes.c_void_p]
        lib.vsamp_sample_tile_pass.restype = ctypes.c_int
        lib.vsamp_tile_stats.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                         ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        lib.vsamp_tile_stats.restype = ctypes.c_int
        lib.vsamp_lm_head.argtypes = [ctypes.POINTER(VsampLmHeadArgs), ctypes.c_void_p]
        lib.vsamp_lm_head.restype = ctypes.c_int
        lib.vsamp_uniforms.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p]
        lib.vsamp_uniforms.restype = ctypes.c_int
        lib.vsamp_uniforms_device.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p,
                                              ctypes.c_void_p]
        lib.vsamp_uniforms_device.restype = ctypes.c_int
        lib.vsamp_spec_advance.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                                           ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        lib.vsamp_spec_advance.restype = ctypes.c_int
        lib.vsamp_last_error.restype = ctypes.c_char_p
        version = lib.vsamp_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI version {version}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def check(code: int) -> None:
    """Raise ``VsamplerError`` for a non-zero status."""
    if code != 0:
        msg = load().vsamp_last_error().decode(errors="replace")
        raise VsamplerError(code, msg)


def query(device_index: int) -> str | None:
    """``None`` if the device can run the kernels, else the library's reason."""
    buf = ctypes.create_string_buffer(256)
    code = load().vsamp_query(device_index, buf, len(buf))
    return None if code == 0 else (buf.value.decode(errors="replace") or STATUS.get(code, str(code)))


_INT64 = (-(1 << 63), 1 << 63)


def position_uniforms(seeds, positions, out=None):
    """The draw's uniforms of ``(seeds[i], positions[i])`` (``vsamp_uniforms``, on the host):
    float32 numpy array, equal to ``vinfer_amd.sampling.uniform`` element for element. Seeds
    outside int64 are not representable in the C call; such rows go through ``uniform``."""
    import numpy as np

    from vinfer_amd.sampling import uniform

    n = len(seeds)
    out = np.empty(n, np.float32) if out is None else out
    if n == 0:
        return out
    try:
        s = np.asarray(seeds, dtype=np.int64)
    except OverflowError:
        for i, (sd, p) in enumerate(zip(seeds, positions)):
            out[i] = uniform(int(sd), int(p))
        return out
    p = np.ascontiguousarray(positions, dtype=np.int64)
    s = np.ascontiguousarray(s)
    if out.dtype != np.float32 or not out.flags["C_CONTIGUOUS"] or out.shape[0] < n:
        raise ValueError("out must be a contiguous float32 array of at least n entries")
    check(load().vsamp_uniforms(s.ctypes.data, p.ctypes.data, n, out.ctypes.data))
    return out
