"""Resolve the configured sampler backend once, for a device and dtype.

Mirrors ``resolve_kernels`` (src/vinfer/kernels/__init__.py:23-34): it runs when the engine is
built, and a backend that cannot run in that context raises ``ValueError`` there, never a
fallback. In the engine the ``sampler`` field sits beside ``attention`` and ``gdn``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from vinfer_amd.config import KernelConfig
from vinfer_amd.registry import BackendContext
from vinfer_amd.sampler import SAMPLER, SamplerBackend


@dataclass(frozen=True)
class Kernels:
    sampler: SamplerBackend


def resolve_kernels(cfg: KernelConfig, device: torch.device | str, dtype: torch.dtype) -> Kernels:
    ctx = BackendContext(torch.device(device), dtype)
    return Kernels(sampler=SAMPLER.resolve(cfg.sampler_backend, ctx))


__all__ = ["BackendContext", "Kernels", "resolve_kernels"]
