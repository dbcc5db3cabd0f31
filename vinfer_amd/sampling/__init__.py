"""Sampling parameters and their packing into per-row device arrays."""

from vinfer_amd.sampling.packed import PackedParams, pack_history, pack_params
from vinfer_amd.sampling.params import (
    EXTENSION_DEFAULTS,
    SamplingParams,
    field,
    penalized,
    position_seed,
    splitmix64,
    uniform,
)

__all__ = [
    "EXTENSION_DEFAULTS",
    "PackedParams",
    "SamplingParams",
    "field",
    "pack_history",
    "pack_params",
    "penalized",
    "position_seed",
    "splitmix64",
    "uniform",
]
