"""Sampling parameters and their packing into per-row device arrays."""

from vinfer_amd.sampling.packed import PackedParams, pack_history, pack_params
from vinfer_amd.sampling.params import SamplingParams, position_seed, splitmix64, uniform

__all__ = [
    "PackedParams",
    "SamplingParams",
    "pack_history",
    "pack_params",
    "position_seed",
    "splitmix64",
    "uniform",
]
