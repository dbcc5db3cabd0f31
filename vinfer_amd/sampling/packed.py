"""Per-row parameter arrays and token histories in the layout the kernels read.

A batch of ``B`` rows carries its ``SamplingParams`` as seven length-``B`` arrays (fp32 for the
real-valued fields, int32 for ``top_k``) and its token histories in CSR form: ``ids`` int32 of
length ``sum(L_b)`` and ``offsets`` int32 of length ``B + 1``. Real-valued fields are rounded to
fp32 once, here, exactly as the engine's sampler rounds a Python float when it meets an fp32
tensor (sampler.py:52, :62); the CPU oracle reads the same fp32 values.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import torch

from vinfer_amd.sampling.params import SamplingParams, field

F32_FIELDS = (
    "temperature",
    "top_p",
    "min_p",
    "repetition_penalty",
    "presence_penalty",
    "frequency_penalty",
)


@dataclass(frozen=True)
class PackedParams:
    """Per-row sampling parameters, each a 1-D tensor of length ``B`` on one device."""

    temperature: torch.Tensor  # f32; 0 = greedy
    top_k: torch.Tensor  # i32; 0 = off
    top_p: torch.Tensor  # f32; 1 = off
    min_p: torch.Tensor  # f32; 0 = off
    repetition_penalty: torch.Tensor  # f32; 1 = off
    presence_penalty: torch.Tensor  # f32; 0 = off
    frequency_penalty: torch.Tensor  # f32; 0 = off

    @property
    def batch(self) -> int:
        return int(self.temperature.shape[0])

    @property
    def device(self) -> torch.device:
        return self.temperature.device

    def to(self, device: torch.device | str) -> PackedParams:
        return PackedParams(**{k: getattr(self, k).to(device) for k in self.__dataclass_fields__})

    def any_penalty(self) -> bool:
        return bool(
            (self.repetition_penalty != 1).any()
            or (self.presence_penalty != 0).any()
            or (self.frequency_penalty != 0).any()
        )

    def repeat_rows(self, n: int) -> PackedParams:
        """Each row ``n`` times in a row (``B * n`` rows: row ``b * n + j`` is row ``b``)."""
        return PackedParams(**{k: getattr(self, k).repeat_interleave(n) for k in self.__dataclass_fields__})

    def select(self, rows: torch.Tensor) -> PackedParams:
        """The rows ``rows`` (an index tensor), in that order."""
        return PackedParams(**{k: getattr(self, k)[rows] for k in self.__dataclass_fields__})

    def row(self, i: int) -> dict[str, float | int]:
        """Row ``i`` as plain Python numbers (fp32 values widened exactly to float)."""
        out: dict[str, float | int] = {k: float(getattr(self, k)[i]) for k in F32_FIELDS}
        out["top_k"] = int(self.top_k[i])
        return out


def pack_params(
    params: Sequence[SamplingParams], device: torch.device | str = "cpu"
) -> PackedParams:
    """Pack one params object per row: this package's ``SamplingParams`` or the engine's own
    (sampler.py:18-27), whose missing extension fields pack as their off values."""
    cols = {k: torch.tensor([field(p, k) for p in params], dtype=torch.float32) for k in F32_FIELDS}
    top_k = torch.tensor([p.top_k for p in params], dtype=torch.int32)
    return PackedParams(top_k=top_k, **cols).to(device)


def pack_history(
    histories: Sequence[Sequence[int]], device: torch.device | str = "cpu"
) -> tuple[torch.Tensor, torch.Tensor]:
    """Token histories as CSR ``(ids int32[sum L], offsets int32[B + 1])``."""
    lengths = torch.tensor([len(h) for h in histories], dtype=torch.int64)
    offsets = torch.zeros(len(histories) + 1, dtype=torch.int64)
    torch.cumsum(lengths, 0, out=offsets[1:])
    if int(offsets[-1]) >= 2**31:
        raise ValueError("total history length must be < 2**31")
    flat = [int(t) for h in histories for t in h]
    ids = torch.tensor(flat, dtype=torch.int32) if flat else torch.zeros(0, dtype=torch.int32)
    return ids.to(device), offsets.to(torch.int32).to(device)
