"""Kernel selection flags for the sampler op family.

Mirrors ``KernelConfig`` (src/vinfer/config.py:22-46): one ``Literal`` flag per op family,
defaulting to ``"reference"``, parsed from ``key=value,...`` strings as on the engine's command
line (server/__main__.py:22, :53). The ``sampler_backend`` flag is the one this package adds;
``"hip"`` selects the hand-written gfx950 kernels.
"""

from __future__ import annotations

from dataclasses import dataclass, fields
from typing import Literal


@dataclass(frozen=True)
class KernelConfig:
    """Which implementation of each hot op family to use. A backend that does not support the
    device or dtype is an error at startup, not a fallback."""

    # "reference" = slow, readable implementation used as ground truth; "hip" = hand-written
    # CDNA4 (gfx950) sampler kernels behind a C ABI. The engine's own attention/gdn flags sit
    # beside this one in its KernelConfig; only the sampler family lives in this package.
    sampler_backend: Literal["reference", "hip"] = "reference"

    @classmethod
    def from_string(cls, spec: str | None) -> KernelConfig:
        """``"sampler_backend=hip,..."``; empty = defaults (config.py:31-43)."""
        values: dict[str, str] = {}
        for item in filter(None, (spec or "").split(",")):
            key, sep, value = item.partition("=")
            if not sep:
                raise ValueError(f"expected key=value in kernel spec, got {item!r}")
            values[key.strip()] = value.strip()
        known = {f.name for f in fields(cls)}
        if unknown := set(values) - known:
            raise ValueError(f"unknown kernel setting(s) {sorted(unknown)}; known: {sorted(known)}")
        return cls(**values)  # type: ignore[arg-type]

    def describe(self) -> str:
        return ",".join(f"{f.name}={getattr(self, f.name)}" for f in fields(self))
