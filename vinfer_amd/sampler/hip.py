"""The ``hip`` sampler backend: hand-written gfx950 kernels behind the C ABI of libvsampler.so.

Registered for device type ``"cuda"`` (ROCm PyTorch reports HIP devices as ``cuda``) and the
logits dtypes bf16 and fp32. ``supports`` checks, at engine build time, that this is a ROCm
build of PyTorch, that the library loads and that the device is a gfx950 GPU
(kernels/registry.py:38-43: an unsupported context is an error, never a fallback).

Every call enqueues work on the current torch stream of the logits' device and returns without
synchronising, except ``sample`` which returns a Python ``int`` as the engine's does
(sampler.py:71, :77).
"""

from __future__ import annotations

import ctypes
import struct
import threading
from collections.abc import Sequence

import numpy as np
import torch

from vinfer_amd import _lib
from vinfer_amd.registry import BackendContext
from vinfer_amd.sampler.base import SAMPLER, require_history
from vinfer_amd.sampling import PackedParams, SamplingParams, field, pack_params, penalized, uniform

_DTYPES = {torch.bfloat16: _lib.VSAMP_BF16, torch.float32: _lib.VSAMP_F32}


def _supports(ctx: BackendContext) -> str | None:
    if torch.version.hip is None:
        return "needs a ROCm build of PyTorch"
    if not torch.cuda.is_available():
        return "no HIP device is visible"
    try:
        _lib.load()
    except Exception as e:  # the reason is reported, never swallowed into a fallback
        return f"libvsampler.so does not load: {e}"
    index = ctx.device.index if ctx.device.index is not None else torch.cuda.current_device()
    return _lib.query(index)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


@SAMPLER.register("hip", devices={"cuda"}, dtypes={torch.bfloat16, torch.float32}, supports=_supports)
class HipSampler:
    def __init__(self, ctx: BackendContext) -> None:
        self.ctx = ctx
        self._lib = _lib.load()
        # Per calling thread: the workspaces by device and the per-token call's buffers. A
        # thread's calls on one device are ordered (one stream, or the per-token call's wait), so
        # its buffers are never rewritten while a kernel reads them; two threads never share one.
        self._local = threading.local()
        # sample_batch / prepare_batch take append_history (VSAMP_HIST_APPEND)
        self.appends_history = True
        # Split small bf16 batches' rows over several workgroups (VSAMP_SPLIT_ROWS): identical
        # results, slower than whole rows on MI355X at every batch measured, so off by default.
        self.split_rows = False
        # Small batches take the tile pass in one launch (vsamp_sample_tile_pass), whose rows the
        # tile maxima decide from a few tiles; identical results. False: the row passes only.
        self.tile_pass = True

    # ---- argument checks ---------------------------------------------------------------------
    def _device(self, logits: torch.Tensor) -> torch.device:
        if logits.device.type != "cuda":
            raise ValueError(f"hip sampler needs logits on a GPU, got {logits.device}")
        if logits.dtype not in _DTYPES:
            raise ValueError(f"hip sampler supports bf16 and fp32 logits, got {logits.dtype}")
        if logits.dim() != 2 or logits.stride(1) != 1:
            raise ValueError("logits must be [B, V] with unit stride along V")
        return logits.device

    @staticmethod
    def _vec(t: torch.Tensor | None, n: int, dtype: torch.dtype, dev: torch.device, name: str):
        if t is None:
            return None
        if t.dtype != dtype or t.device != dev or t.dim() != 1 or t.shape[0] != n:
            raise ValueError(f"{name} must be a {dtype} [{n}] tensor on {dev}")
        return t.contiguous()

    def _args(self, logits, params, hist_ids, hist_offsets, uniforms=None, draft_ids=None, param_rows=None,
              append_history=False):
        dev = self._device(logits)
        B, V = logits.shape
        P = B if param_rows is None else param_rows  # parameter entries (verify: one per sequence)
        if params.batch != P:
            raise ValueError(f"params describe {params.batch} rows, logits have {B}")
        cols = {}
        for name in (
            "temperature",
            "top_p",
            "min_p",
            "repetition_penalty",
            "presence_penalty",
            "frequency_penalty",
        ):
            cols[name] = self._vec(getattr(params, name), P, torch.float32, dev, name)
        cols["top_k"] = self._vec(params.top_k, P, torch.int32, dev, "top_k")
        if (hist_ids is None) != (hist_offsets is None):
            raise ValueError("hist_ids and hist_offsets go together")
        hist_total = 0
        flags = 0
        if hist_ids is not None:
            if hist_offsets.dim() == 2:  # a [start, end) pair per row
                if (
                    hist_offsets.dtype != torch.int32
                    or hist_offsets.device != dev
                    or tuple(hist_offsets.shape) != (B, 2)
                ):
                    raise ValueError(f"hist_offsets as ranges must be a torch.int32 [{B}, 2] tensor on {dev}")
                hist_offsets = hist_offsets.contiguous()
                flags = _lib.VSAMP_HIST_RANGES
            else:
                hist_offsets = self._vec(hist_offsets, B + 1, torch.int32, dev, "hist_offsets")
            if hist_ids.dtype != torch.int32 or hist_ids.device != dev or hist_ids.dim() != 1:
                raise ValueError(f"hist_ids must be an int32 1-D tensor on {dev}")
            hist_ids = hist_ids.contiguous()
            hist_total = int(hist_ids.shape[0])
        a = _lib.VsampArgs()
        a.logits = logits.data_ptr()
        a.dtype = _DTYPES[logits.dtype]
        a.batch = B
        a.vocab = V
        a.row_stride = logits.stride(0) if B > 1 else V
        for name, t in cols.items():
            setattr(a, name, _ptr(t))
        a.hist_ids = _ptr(hist_ids) if hist_total else None
        a.hist_offsets = _ptr(hist_offsets) if hist_total else None
        a.hist_total = hist_total
        a.flags = (flags if hist_total else 0) | (_lib.VSAMP_SPLIT_ROWS if self.split_rows else 0)
        if append_history:  # (the library checks that ranges and a penalty column come with it)
            a.flags |= _lib.VSAMP_HIST_APPEND
        if uniforms is not None:
            uniforms = self._vec(uniforms, P, torch.float32, dev, "uniforms")
            a.uniforms = _ptr(uniforms)
        if draft_ids is not None:
            draft_ids = self._vec(draft_ids, B, torch.int32, dev, "draft_ids")
            a.draft_ids = _ptr(draft_ids)
        # (histories' penalty lists and, with split rows, the slices' records)
        ws_bytes = self._lib.vsamp_split_workspace_bytes if self.split_rows else self._lib.vsamp_workspace_bytes
        need = int(ws_bytes(B, V, hist_total))
        if need:
            a.workspace = self._workspace(dev, need)
            a.workspace_bytes = need
        keep = (logits, cols, hist_ids, hist_offsets, uniforms, draft_ids)
        return a, keep

    @staticmethod
    def _stream(dev: torch.device) -> ctypes.c_void_p:
        # (the raw handle of the device's current stream: what torch.cuda.current_stream(dev)
        # .cuda_stream returns, without building the Stream object, ~4 us a call)
        return ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(dev.index))

    # ---- the interface ----------------------------------------------------------------------
    def prepare_batch(self, logits, params, uniforms, hist_ids=None, hist_offsets=None, draft_ids=None,
                      append_history=False):
        """A reusable launch of ``sample_batch`` on fixed buffers: every check and the argument
        block are done once; ``PreparedStep.launch()`` then only enqueues the kernel. Outputs
        land in ``PreparedStep.ids`` / ``.draft_prob``; inputs may be refilled in place."""
        a, keep = self._args(logits, params, hist_ids, hist_offsets, uniforms, draft_ids,
                             append_history=append_history)
        if a.workspace_bytes:  # a private workspace: steps prepared together may overlap
            ws = torch.empty(a.workspace_bytes + 256, dtype=torch.uint8, device=logits.device)
            a.workspace = (ws.data_ptr() + 255) & ~255
            keep = keep + (ws,)
        B, V = logits.shape
        ids = torch.empty(B, dtype=torch.int32, device=logits.device)
        dprob = torch.empty(B, dtype=torch.float32, device=logits.device) if draft_ids is not None else None
        a.out_ids = ids.data_ptr()
        a.out_draft_prob = _ptr(dprob)
        tile_pass = None
        if self._one_launch_tiles(a, logits):  # (the step's own maxima and arrival words)
            tile_pass = (torch.empty(B * _n_tiles(V), dtype=torch.float32, device=logits.device),
                         torch.zeros(B, dtype=torch.int32, device=logits.device))
        return PreparedStep(self._lib, a, keep, ids, dprob, tile_pass=tile_pass)

    def sample_batch(self, logits, params, uniforms, hist_ids=None, hist_offsets=None, draft_ids=None,
                     append_history=False):
        """``SamplerBackend.sample_batch``; with ``append_history`` (per-row ranges into a writable
        ``hist_ids``, penalties on) each row's drawn id is also written at its range's end."""
        a, keep = self._args(logits, params, hist_ids, hist_offsets, uniforms, draft_ids,
                             append_history=append_history)
        dev = logits.device
        B = logits.shape[0]
        ids = torch.empty(B, dtype=torch.int32, device=dev)
        dprob = torch.empty(B, dtype=torch.float32, device=dev) if draft_ids is not None else None
        a.out_ids = ids.data_ptr()
        a.out_draft_prob = _ptr(dprob)
        if self._one_launch_tiles(a, logits):
            tiles, arrive = self._tiles(dev, B * _n_tiles(logits.shape[1]), B)
            _lib.check(self._lib.vsamp_sample_tile_pass(ctypes.byref(a), tiles, arrive, self._stream(dev)))
        else:
            _lib.check(self._lib.vsamp_sample(ctypes.byref(a), self._stream(dev)))
        del keep
        return ids, dprob

    def _one_launch_tiles(self, a, logits: torch.Tensor) -> bool:
        """Whether a batch takes the tile pass as one launch (``vsamp_sample_tile_pass``): rows
        few enough that their workgroups fit one round on the CUs, no split rows, and
        ``tile_pass`` on. Its greedy and top-k rows without penalties are then decided from a few
        tiles; the other rows run the row passes on one workgroup each, as ``vsamp_sample`` would
        (the same outputs either way)."""
        B, V = logits.shape
        return (self.tile_pass and not (a.flags & _lib.VSAMP_SPLIT_ROWS)
                and B * ((_n_tiles(V) + 63) // 64) <= _TILE_FUSED_WORKGROUPS)

    def probs(self, logits, params, hist_ids=None, hist_offsets=None):
        a, keep = self._args(logits, params, hist_ids, hist_offsets)
        B, V = logits.shape
        out = torch.empty(B, V, dtype=torch.float32, device=logits.device)
        _lib.check(self._lib.vsamp_probs(ctypes.byref(a), out.data_ptr(), V, self._stream(logits.device)))
        del keep
        return out

    def penalized_logits(self, logits, params, hist_ids=None, hist_offsets=None):
        a, keep = self._args(logits, params, hist_ids, hist_offsets)
        B, V = logits.shape
        dev = logits.device
        need = int(self._lib.vsamp_workspace_bytes(B, V, a.hist_total))
        if a.workspace_bytes < need:
            a.workspace = self._workspace(dev, need)
            a.workspace_bytes = need
        out = torch.empty(B, V, dtype=torch.float32, device=dev)
        counts = torch.empty(B, V, dtype=torch.int32, device=dev)
        _lib.check(
            self._lib.vsamp_penalized_logits(
                ctypes.byref(a), out.data_ptr(), counts.data_ptr(), V, self._stream(dev)
            )
        )
        del keep
        return out, counts

    def logprobs(self, logits, tokens=None, n_top=0):
        dev = self._device(logits)
        B, V = logits.shape
        if not 0 <= n_top <= 32:
            raise ValueError(f"n_top must be in [0, 32], got {n_top}")
        a = _lib.VsampArgs()
        a.logits = logits.data_ptr()
        a.dtype = _DTYPES[logits.dtype]
        a.batch, a.vocab = B, V
        a.row_stride = logits.stride(0) if B > 1 else V
        tok = self._vec(tokens.to(torch.int32) if tokens is not None else None, B, torch.int32, dev, "tokens")
        out_tok = torch.empty(B, dtype=torch.float32, device=dev) if tok is not None else None
        ids = torch.empty(B, n_top, dtype=torch.int32, device=dev)
        lps = torch.empty(B, n_top, dtype=torch.float32, device=dev)
        _lib.check(
            self._lib.vsamp_logprobs(
                ctypes.byref(a), _ptr(tok), n_top, _ptr(out_tok),
                ids.data_ptr() if n_top else None, lps.data_ptr() if n_top else None, self._stream(dev)
            )
        )
        return out_tok, ids, lps

    def lm_head(self, hidden, weight):
        """The LM head fused with the log-softmax statistics (``vsamp_lm_head``): bf16
        ``logits [B, V] = hidden [B, d] @ weight [V, d]^T`` (fp32 accumulation, rounded to bf16, as
        ``F.linear`` returns it; model.py:230-233) and, per row and 128 logits, their max and sum of
        exp(x - max). Returns ``(logits, tile_max, tile_sum)``; the statistics feed
        ``logprobs_tiles``. Up to 64 rows the fused kernel runs (d a multiple of 64); above, the
        library GEMM (``F.linear``, any d) and ``tile_stats`` over its logits."""
        for name, t in (("hidden", hidden), ("weight", weight)):
            if t.dtype != torch.bfloat16 or t.device.type != "cuda" or t.dim() != 2 or t.stride(1) != 1:
                raise ValueError(f"{name} must be a bf16 2-D tensor on a GPU with unit stride along d")
        B, d = hidden.shape
        V, d2 = weight.shape
        if d2 != d or weight.device != hidden.device:
            raise ValueError(f"weight must be [V, {d}] on {hidden.device}, got {tuple(weight.shape)} on {weight.device}")
        dev = hidden.device
        if B > _LM_OWN_ROWS:
            # above 64 rows the library's GEMM (F.linear, hipBLASLt) beats the MFMA tiles (at
            # d = 4096, V = 151936: 286-353 us against 472-525 at B = 65-256 on MI355X); the
            # statistics then come from one read of its logits
            logits = torch.nn.functional.linear(hidden, weight)
            tmax, tsum = self.tile_stats(logits)
            return logits, tmax, tsum
        nT = (V + _lib.LM_TILE - 1) // _lib.LM_TILE
        logits = torch.empty(B, V, dtype=torch.bfloat16, device=dev)
        tmax = torch.empty(B, nT, dtype=torch.float32, device=dev)
        tsum = torch.empty(B, nT, dtype=torch.float32, device=dev)
        a = _lib.VsampLmHeadArgs()
        a.hidden, a.hidden_stride = hidden.data_ptr(), hidden.stride(0) if B > 1 else d
        a.weight, a.weight_stride = weight.data_ptr(), weight.stride(0) if V > 1 else d
        a.logits, a.logits_stride = logits.data_ptr(), V
        a.tile_max, a.tile_sum = tmax.data_ptr(), tsum.data_ptr()
        a.batch, a.dim, a.vocab = B, d, V
        _lib.check(self._lib.vsamp_lm_head(ctypes.byref(a), self._stream(dev)))
        return logits, tmax, tsum

    def tile_stats(self, logits):
        """The tile statistics ``lm_head`` returns, for bf16 logits ``[B, V]`` from any GEMM
        (``vsamp_tile_stats``): per row and 128 logits, the max and the sum of exp(x - max).
        Returns ``(tile_max, tile_sum)``, fp32 ``[B, ceil(V / 128)]`` each."""
        dev = self._device(logits)
        if logits.dtype != torch.bfloat16 or logits.dim() != 2 or logits.stride(1) != 1:
            raise ValueError("tile_stats takes bf16 [B, V] logits with unit stride along V")
        B, V = logits.shape
        nT = (V + _lib.LM_TILE - 1) // _lib.LM_TILE
        tmax = torch.empty(B, nT, dtype=torch.float32, device=dev)
        tsum = torch.empty(B, nT, dtype=torch.float32, device=dev)
        _lib.check(self._lib.vsamp_tile_stats(logits.data_ptr(), logits.stride(0) if B > 1 else V, B, V,
                                              tmax.data_ptr(), tsum.data_ptr(), self._stream(dev)))
        return tmax, tsum

    def logprobs_tiles(self, logits, tile_max, tile_sum, tokens=None, n_top=0):
        """``logprobs`` over the bf16 logits ``lm_head`` wrote, with its tile statistics
        (``vsamp_logprobs_tiles``)."""
        dev = self._device(logits)
        if logits.dtype != torch.bfloat16:
            raise ValueError("logprobs_tiles takes the bf16 logits of lm_head")
        B, V = logits.shape
        nT = (V + _lib.LM_TILE - 1) // _lib.LM_TILE
        for name, t in (("tile_max", tile_max), ("tile_sum", tile_sum)):
            if t.dtype != torch.float32 or t.device != dev or tuple(t.shape) != (B, nT) or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous float32 [{B}, {nT}] tensor on {dev}")
        if not 0 <= n_top <= 32:
            raise ValueError(f"n_top must be in [0, 32], got {n_top}")
        a = _lib.VsampArgs()
        a.logits = logits.data_ptr()
        a.dtype = _DTYPES[logits.dtype]
        a.batch, a.vocab = B, V
        a.row_stride = logits.stride(0) if B > 1 else V
        tok = self._vec(tokens.to(torch.int32) if tokens is not None else None, B, torch.int32, dev, "tokens")
        out_tok = torch.empty(B, dtype=torch.float32, device=dev) if tok is not None else None
        ids = torch.empty(B, n_top, dtype=torch.int32, device=dev)
        lps = torch.empty(B, n_top, dtype=torch.float32, device=dev)
        _lib.check(
            self._lib.vsamp_logprobs_tiles(
                ctypes.byref(a), tile_max.data_ptr(), tile_sum.data_ptr(), _ptr(tok), n_top, _ptr(out_tok),
                ids.data_ptr() if n_top else None, lps.data_ptr() if n_top else None, self._stream(dev)
            )
        )
        return out_tok, ids, lps

    def _check_tiles(self, logits, tile_max) -> None:
        dev = self._device(logits)
        if logits.dtype != torch.bfloat16:
            raise ValueError("sample_tiles takes the bf16 logits of lm_head")
        B, V = logits.shape
        nT = (V + _lib.LM_TILE - 1) // _lib.LM_TILE
        if (tile_max.dtype != torch.float32 or tile_max.device != dev or tuple(tile_max.shape) != (B, nT)
                or not tile_max.is_contiguous()):
            raise ValueError(f"tile_max must be a contiguous float32 [{B}, {nT}] tensor on {dev}")

    def sample_tiles(self, logits, tile_max, params, uniforms, hist_ids=None, hist_offsets=None, draft_ids=None):
        """``sample_batch`` over the bf16 logits ``lm_head`` wrote, with its tile maxima
        (``vsamp_sample_tiles``): the same ids and draft probabilities, with greedy, top-k and
        min-p rows without penalties decided from a few tiles."""
        self._check_tiles(logits, tile_max)
        dev = logits.device
        B = logits.shape[0]
        a, keep = self._args(logits, params, hist_ids, hist_offsets, uniforms, draft_ids)
        a.flags &= ~_lib.VSAMP_SPLIT_ROWS
        ids = torch.empty(B, dtype=torch.int32, device=dev)
        dprob = torch.empty(B, dtype=torch.float32, device=dev) if draft_ids is not None else None
        a.out_ids = ids.data_ptr()
        a.out_draft_prob = _ptr(dprob)
        _lib.check(self._lib.vsamp_sample_tiles(ctypes.byref(a), tile_max.data_ptr(), self._stream(dev)))
        del keep
        return ids, dprob

    def sample_tile_pass(self, logits, params, uniforms, hist_ids=None, hist_offsets=None, draft_ids=None):
        """``sample_batch`` for small batches of bf16 or fp32 logits from any source
        (``vsamp_sample_tile_pass``): the rows' tile maxima are computed by a launch spread over
        the chip first, then greedy, top-k and min-p rows without penalties are decided from a
        few tiles. The same ids and draft probabilities as ``sample_batch``."""
        dev = self._device(logits)
        B, V = logits.shape
        a, keep = self._args(logits, params, hist_ids, hist_offsets, uniforms, draft_ids)
        a.flags &= ~_lib.VSAMP_SPLIT_ROWS
        ids = torch.empty(B, dtype=torch.int32, device=dev)
        dprob = torch.empty(B, dtype=torch.float32, device=dev) if draft_ids is not None else None
        a.out_ids = ids.data_ptr()
        a.out_draft_prob = _ptr(dprob)
        tiles, arrive = self._tiles(dev, B * ((V + _lib.LM_TILE - 1) // _lib.LM_TILE), B)
        _lib.check(self._lib.vsamp_sample_tile_pass(ctypes.byref(a), tiles, arrive, self._stream(dev)))
        del keep
        return ids, dprob

    def prepare_tiles(self, logits, tile_max, params, uniforms, hist_ids=None, hist_offsets=None, draft_ids=None):
        """``prepare_batch`` for ``sample_tiles``: a reusable launch on fixed buffers (the logits
        and tile maxima may be rewritten in place between launches)."""
        self._check_tiles(logits, tile_max)
        split, self.split_rows = self.split_rows, False
        try:
            st = self.prepare_batch(logits, params, uniforms, hist_ids, hist_offsets, draft_ids)
        finally:
            self.split_rows = split
        return PreparedStep(self._lib, st._args, st._keep + (tile_max,), st.ids, st.draft_prob, tile_max)

    def sample_states(self, logits, params, uniforms):
        """``sample_batch`` without histories, plus each row's sampling state (uint8 ``[B, 40]``,
        opaque) for a later ``verify`` of these rows as drafts (``draft_states``)."""
        a, keep = self._args(logits, params, None, None, uniforms)
        dev = logits.device
        B = logits.shape[0]
        ids = torch.empty(B, dtype=torch.int32, device=dev)
        states = torch.empty(B, _lib.ROW_STATE_BYTES // 8, dtype=torch.int64, device=dev)  # (8-byte aligned)
        a.out_ids = ids.data_ptr()
        _lib.check(self._lib.vsamp_sample_states(ctypes.byref(a), states.data_ptr(), self._stream(dev)))
        del keep
        return ids, states.view(torch.uint8).view(B, _lib.ROW_STATE_BYTES)

    def uniforms_device(self, seeds: torch.Tensor, positions: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """The draw's uniforms of ``(seeds[i], positions[i])`` computed on the device
        (``vsamp_uniforms_device``; the same values as ``sampling.uniform``, bit for bit), on the
        current stream: int64 device tensors in, a float32 device tensor out. A decode loop
        replaying its steps from a captured graph puts this in the graph and stages only the
        positions."""
        for name, t in (("seeds", seeds), ("positions", positions)):
            if t.dtype != torch.int64 or t.device.type != "cuda" or t.dim() != 1 or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous 1-D int64 tensor on a GPU")
        n = seeds.shape[0]
        if positions.shape[0] != n or positions.device != seeds.device:
            raise ValueError(f"positions must have {n} entries on {seeds.device}")
        dev = seeds.device
        if out is None:
            out = torch.empty(n, dtype=torch.float32, device=dev)
        elif out.dtype != torch.float32 or out.device != dev or out.dim() != 1 or out.shape[0] < n or not out.is_contiguous():
            raise ValueError(f"out must be a contiguous float32 tensor of at least {n} entries on {dev}")
        _lib.check(self._lib.vsamp_uniforms_device(seeds.data_ptr(), positions.data_ptr(), n, out.data_ptr(),
                                                   self._stream(dev)))
        return out

    def spec_advance(self, inputs: torch.Tensor, num_draft: int, seeds: torch.Tensor, uniforms: torch.Tensor,
                     tokens: torch.Tensor | None = None, counts: torch.Tensor | None = None) -> None:
        """A speculative loop's next-iteration inputs and uniforms on the device, in place
        (``vsamp_spec_advance``): ``inputs`` int64 ``[4 + 2 K + 1, n]`` (slot, last token, the
        token before it, its position, the draft steps' and the target's positions), moved past
        the iteration whose verified ``tokens`` ``[n, K + 1]`` and ``counts`` ``[n]`` (int32) are
        given (none: they stay), and ``uniforms`` float32 ``[(3K + 1) n]`` from ``seeds`` int64
        ``[n]``, on the current stream."""
        K = int(num_draft)
        if inputs.dtype != torch.int64 or inputs.dim() != 2 or inputs.shape[0] != 4 + 2 * K + 1 or not inputs.is_contiguous():
            raise ValueError(f"inputs must be a contiguous int64 [{4 + 2 * K + 1}, n] tensor")
        n = inputs.shape[1]
        dev = inputs.device
        if seeds.dtype != torch.int64 or seeds.shape != (n,) or seeds.device != dev or not seeds.is_contiguous():
            raise ValueError(f"seeds must be a contiguous int64 [{n}] tensor on {dev}")
        if uniforms.dtype != torch.float32 or uniforms.numel() < (3 * K + 1) * n or uniforms.device != dev or not uniforms.is_contiguous():
            raise ValueError(f"uniforms must be a contiguous float32 tensor of {(3 * K + 1) * n} entries on {dev}")
        if (tokens is None) != (counts is None):
            raise ValueError("tokens and counts are given together or not at all")
        if tokens is not None:
            if tokens.dtype != torch.int32 or tokens.shape != (n, K + 1) or not tokens.is_contiguous() or tokens.device != dev:
                raise ValueError(f"tokens must be a contiguous int32 [{n}, {K + 1}] tensor on {dev}")
            if counts.dtype != torch.int32 or counts.shape != (n,) or not counts.is_contiguous() or counts.device != dev:
                raise ValueError(f"counts must be a contiguous int32 [{n}] tensor on {dev}")
        ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        _lib.check(self._lib.vsamp_spec_advance(inputs.data_ptr(), n, K, ptr(tokens), ptr(counts), seeds.data_ptr(),
                                                uniforms.data_ptr(), self._stream(dev)))

    def verify(self, target_logits, draft_logits, draft_tokens, params, u_accept, u_residual, u_bonus,
               draft_params=None, draft_states=None):
        if target_logits.dim() != 3 or draft_logits.dim() != 3:
            raise ValueError("target_logits must be [B, K + 1, V] and draft_logits [B, K, V]")
        B, K1, V = target_logits.shape
        K = K1 - 1
        if K < 1 or tuple(draft_logits.shape) != (B, K, V):
            raise ValueError(f"draft_logits must be [{B}, {K}, {V}] for target_logits {tuple(target_logits.shape)}")
        if draft_logits.dtype != target_logits.dtype:
            raise ValueError("target and draft logits must have one dtype")
        dev = target_logits.device
        tl = target_logits.reshape(B * K1, V)
        dl = draft_logits.reshape(B * K, V)
        dparams = params if draft_params is None else draft_params
        if params.batch != B or dparams.batch != B:
            raise ValueError(f"params must describe the {B} sequences")
        drafts = draft_tokens.to(torch.int32).contiguous()
        ua = u_accept.to(torch.float32).contiguous()
        ur = u_residual.to(torch.float32).contiguous()
        for name, t, shape in (("draft_tokens", drafts, (B, K)), ("u_accept", ua, (B, K)), ("u_residual", ur, (B, K))):
            if tuple(t.shape) != shape or t.device != dev:
                raise ValueError(f"{name} must be [{B}, {K}] on {dev}")
        ub = self._vec(u_bonus.to(torch.float32), B, torch.float32, dev, "u_bonus")
        ta, tkeep = self._args(tl, params, None, None, ub, param_rows=B)
        da, dkeep = self._args(dl, dparams, None, None, None, param_rows=B)
        v = _lib.VsampVerifyArgs()
        v.target, v.draft = ta, da
        v.batch, v.num_draft = B, K
        v.draft_tokens, v.u_accept, v.u_residual = drafts.data_ptr(), ua.data_ptr(), ur.data_ptr()
        tokens = torch.empty(B, K1, dtype=torch.int32, device=dev)
        counts = torch.empty(B, dtype=torch.int32, device=dev)
        v.out_tokens, v.out_count = tokens.data_ptr(), counts.data_ptr()
        if draft_states is not None:
            ds = draft_states.reshape(B * K, _lib.ROW_STATE_BYTES)
            if ds.dtype != torch.uint8 or ds.device != dev or ds.data_ptr() % 8:
                raise ValueError("draft_states must be the uint8 [B, K, 40] states sample_states returned")
            ds = ds.contiguous()
            v.draft_states = ds.data_ptr()
        need = int(self._lib.vsamp_verify_workspace_bytes(B, K))
        ws = torch.empty(need + 256, dtype=torch.uint8, device=dev)
        v.workspace = (ws.data_ptr() + 255) & ~255
        v.workspace_bytes = need
        _lib.check(self._lib.vsamp_verify(ctypes.byref(v), self._stream(dev)))
        del tkeep, dkeep
        return tokens, counts

    def sample(
        self,
        logits: torch.Tensor,
        params: SamplingParams,
        seed: int,
        position: int,
        history: Sequence[int] | torch.Tensor | None = None,
    ) -> int:
        # (each extension field read once: the per-token call's host time is most of its cost)
        rep_p = field(params, "repetition_penalty")
        pres_p = field(params, "presence_penalty")
        freq_p = field(params, "frequency_penalty")
        pen = rep_p != 1.0 or pres_p != 0.0 or freq_p != 0.0  # (penalized(params))
        if pen and history is None:
            require_history(params, history)
        if logits.dim() != 1 and not (logits.dim() == 2 and logits.shape[0] == 1):
            raise ValueError(f"sample takes one row of logits ([V] or [1, V]), got {tuple(logits.shape)}")
        row = logits.reshape(-1)
        if row.stride(0) != 1:
            raise ValueError("logits must have unit stride")
        dev = row.device
        if dev.type != "cuda" or row.dtype not in _DTYPES:
            self._device(row.reshape(1, -1))  # (raises with the reason)
        V = row.shape[0]
        t = self._token_path(dev)
        # the row's parameters and its uniform (one pinned block the kernel reads in place)
        top_k = params.top_k
        u = uniform(seed, position)
        try:
            _WORDS.pack_into(t.mem, 0, params.temperature, params.top_p, field(params, "min_p"), rep_p, pres_p, freq_p,
                             top_k, u)
        except (struct.error, OverflowError):  # (values past fp32 or int32: numpy's conversions)
            f = t.words.view(np.float32)
            f[0], f[1], f[2] = params.temperature, params.top_p, field(params, "min_p")
            f[3], f[4], f[5] = rep_p, pres_p, freq_p
            t.words[6] = top_k
            f[7] = u
        n = len(history) if pen else 0
        a = t.args
        a.logits = row.data_ptr()
        if t.shape != (V, row.dtype):
            t.shape = (V, row.dtype)
            a.dtype, a.vocab, a.row_stride = _DTYPES[row.dtype], V, V
            # (the tile pass's maxima and arrival word: this path's own, zero until first used)
            t.tile_bufs = (torch.empty(max((V + _lib.LM_TILE - 1) // _lib.LM_TILE, 2048), dtype=torch.float32, device=dev),
                           torch.zeros(64, dtype=torch.int32, device=dev))
            t.tiles = (t.tile_bufs[0].data_ptr(), t.tile_bufs[1].data_ptr())
        if t.hist:  # (the previous call passed a history)
            a.hist_ids = a.hist_offsets = a.workspace = None
            a.hist_total = a.workspace_bytes = 0
            t.hist = False
        keep = None
        if n > 0:
            if isinstance(history, torch.Tensor) and history.device.type != "cpu":
                # (read in place when it is already an int32 vector on this device)
                keep = history.reshape(-1).to(device=dev, dtype=torch.int32).contiguous()
                hist_ptr = keep.data_ptr()
            else:
                if t.hist_host.shape[0] < n:
                    t.hist_host = torch.empty(max(n, 2 * t.hist_host.shape[0]), dtype=torch.int32, pin_memory=True)
                t.hist_host.numpy()[:n] = np.asarray(history, dtype=np.int32).reshape(-1)
                hist_ptr = t.hist_host.data_ptr()
            t.words[8], t.words[9] = 0, n
            need = int(self._lib.vsamp_workspace_bytes(1, V, n))
            a.hist_ids, a.hist_offsets, a.hist_total = hist_ptr, t.base + 32, n
            a.workspace, a.workspace_bytes = self._workspace(dev, need), need
            t.hist = True
        stream = self._stream(dev)
        out = t.out_np
        out[0] = -1
        # Greedy and top-k (<= 256) rows without penalties take the tile pass: the row's tile
        # maxima over the chip, then a few tiles, instead of the whole row on one workgroup
        # (bf16: greedy 29.9 -> 24.7 us per call, top-k 20 34.2 -> 31.0 on MI355X, as first
        # built). Rows with min-p alone do not: their candidates depend on the logits (N(0, 4) rows
        # keep ~900 tokens at min-p 0.05, more than the tile path's list), and a row handed on pays
        # both launches.
        if (self.tile_pass and n == 0 and not pen
                and (not params.temperature > 0 or 0 < top_k <= 256 and top_k < V)):
            code = self._lib.vsamp_sample_tile_pass(t.ref, t.tiles[0], t.tiles[1], stream)
        else:
            code = self._lib.vsamp_sample(t.ref, stream)
        _lib.check(code)
        # the kernel writes the id last, after every read of the parameters and the history: the
        # call returns as soon as the id reaches the pinned word (sooner than a stream
        # synchronisation returns), and a synchronisation settles it past any draw's time
        spins = 0
        while out[0] < 0:
            spins += 1
            if spins == 1 << 20:
                torch.cuda.current_stream(dev).synchronize()
                if out[0] < 0:
                    raise RuntimeError("the drawn id never reached the host")
        del keep
        return int(out[0])

    def _token_path(self, dev: torch.device) -> "_TokenPath":
        paths = self._local.__dict__.setdefault("paths", {})
        t = paths.get(dev)
        if t is None:
            t = paths[dev] = _TokenPath(dev)
        return t

    def _tiles(self, dev: torch.device, n: int, rows: int) -> tuple[int, int]:
        """Device buffers of ``n`` fp32 tile maxima and ``rows`` arrival words (zero, and left
        zero by every call), this thread's for ``dev``."""
        bufs = self._local.__dict__.setdefault("tiles", {})
        t = bufs.get(dev)
        if t is None or t[0].numel() < n or t[1].numel() < rows:
            t = bufs[dev] = (torch.empty(max(n, 2048), dtype=torch.float32, device=dev),
                             torch.zeros(max(rows, 64), dtype=torch.int32, device=dev))
        return t[0].data_ptr(), t[1].data_ptr()

    def _workspace(self, dev: torch.device, need: int) -> int:
        """A 256-byte aligned device workspace of ``need`` bytes, this thread's for ``dev``."""
        spaces = self._local.__dict__.setdefault("workspaces", {})
        w = spaces.get(dev)
        if w is None or w.numel() < need + 256:
            w = spaces[dev] = torch.empty(need + 256, dtype=torch.uint8, device=dev)
        return (w.data_ptr() + 255) & ~255


def _n_tiles(V: int) -> int:
    return (V + _lib.LM_TILE - 1) // _lib.LM_TILE


# batches up to this many workgroups (rows times workgroups per row) take the tile pass in one
# launch (the library's rule)
_TILE_FUSED_WORKGROUPS = 256
_LM_OWN_ROWS = 64  # (lm_head: the library GEMM and vsamp_tile_stats above this many rows)

# the per-token call's parameter words: temperature, top_p, min_p, the three penalties (fp32),
# top_k (int32), the uniform (fp32)
_WORDS = struct.Struct("<6fif")


class _TokenPath:
    """The per-token call's buffers on one device, reused call after call, all pinned host
    memory that the kernel reads and writes in place (mapped into the device's address space:
    no copy either way, 6 us less per call than a copy in and a copy out): the row's parameter
    words (temperature, top_p, min_p, the three penalties, top_k, the uniform, the history's
    [0, n) range), the history of a call that passes it from the host, and the drawn id. The
    call returns once the kernel has written the id, which it does after its last read of the
    rest, so nothing here is rewritten while a kernel reads it. Each calling thread has its own
    (the engine calls from one generation worker thread, serial.py:40)."""

    def __init__(self, dev: torch.device) -> None:
        self.words_t = torch.zeros(16, dtype=torch.int32, pin_memory=True)
        self.words = self.words_t.numpy()
        self.mem = memoryview(self.words).cast("B")
        self.base = self.words_t.data_ptr()
        self.shape = None  # (V, dtype) the argument block was last set up for, with its tile buffers
        self.tile_bufs = None
        self.tiles = (0, 0)
        self.hist = False  # the argument block points at a history
        self.hist_host = torch.empty(0, dtype=torch.int32, pin_memory=True)
        self.out = torch.empty(1, dtype=torch.int32, pin_memory=True)
        self.out_np = self.out.numpy()
        a = _lib.VsampArgs()
        a.batch = 1
        for i, name in enumerate(("temperature", "top_p", "min_p", "repetition_penalty", "presence_penalty",
                                  "frequency_penalty", "top_k", "uniforms")):
            setattr(a, name, self.base + 4 * i)
        a.out_ids = self.out.data_ptr()
        self.args = a
        self.ref = ctypes.byref(a)


class PreparedStep:
    """One batch's sampler launch with its argument block built (see ``prepare_batch``)."""

    def __init__(self, lib, args, keep, ids, dprob, tile_max=None, tile_pass=None) -> None:
        self._lib, self._args, self._keep = lib, args, keep
        self._ref = ctypes.byref(args)
        self.ids, self.draft_prob = ids, dprob
        self._tiles = None if tile_max is None else ctypes.c_void_p(tile_max.data_ptr())
        # (a small batch: the tile pass in one launch, on the step's own maxima and arrival words)
        self._pass = tile_pass
        self._pass_ptrs = None if tile_pass is None else tuple(ctypes.c_void_p(t.data_ptr()) for t in tile_pass)

    def launch(self, stream: int | None = None) -> None:
        """Enqueue the step on ``stream`` (a hipStream_t as int; default: torch's current)."""
        if stream is None:
            stream = torch._C._cuda_getCurrentRawStream(self.ids.device.index)
        if self._tiles is not None:
            code = self._lib.vsamp_sample_tiles(self._ref, self._tiles, ctypes.c_void_p(stream))
        elif self._pass_ptrs is not None:
            code = self._lib.vsamp_sample_tile_pass(self._ref, *self._pass_ptrs, ctypes.c_void_p(stream))
        else:
            code = self._lib.vsamp_sample(self._ref, ctypes.c_void_p(stream))
        if code:
            _lib.check(code)


__all__ = ["HipSampler", "PackedParams", "PreparedStep"]
