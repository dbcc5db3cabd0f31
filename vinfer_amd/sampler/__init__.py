"""Sampler backends: ``reference`` (torch, any device) and ``hip`` (gfx950 kernels)."""

from vinfer_amd.sampler import hip as _hip  # noqa: F401  (registers "hip")
from vinfer_amd.sampler import reference as _reference  # noqa: F401  (registers "reference")
from vinfer_amd.sampler.base import SAMPLER, SamplerBackend
from vinfer_amd.sampler.hip import HipSampler
from vinfer_amd.sampler.reference import ReferenceSampler

__all__ = ["SAMPLER", "HipSampler", "ReferenceSampler", "SamplerBackend"]
