"""Named implementations of one op family, each declaring where it can run.

Mirrors the engine's kernel-backend registry (src/vinfer/kernels/registry.py:25-88): a backend
is registered under a name with the device types and dtypes it supports plus an optional
``supports`` predicate, and is constructed as ``cls(BackendContext(device, dtype))``. Choosing
a backend that cannot run in a context raises ``ValueError`` when the engine is built; there is
never a silent fallback to another backend.
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass
from typing import Generic, TypeVar

import torch

T = TypeVar("T")


@dataclass(frozen=True)
class BackendContext:
    """Where a backend runs (registry.py:25-28)."""

    device: torch.device
    dtype: torch.dtype


@dataclass(frozen=True)
class _Entry(Generic[T]):
    factory: Callable[[BackendContext], T]
    devices: frozenset[str] | None
    dtypes: frozenset[torch.dtype] | None
    supports: Callable[[BackendContext], str | None] | None

    def unsupported(self, ctx: BackendContext) -> str | None:
        # Same check order and message texts as registry.py:38-43.
        if self.devices is not None and ctx.device.type not in self.devices:
            return f"does not run on {ctx.device.type} (supports {sorted(self.devices)})"
        if self.dtypes is not None and ctx.dtype not in self.dtypes:
            return f"does not support {ctx.dtype} (supports {sorted(map(str, self.dtypes))})"
        return self.supports(ctx) if self.supports is not None else None


class BackendRegistry(Generic[T]):
    """One registry per op family (registry.py:46-88)."""

    def __init__(self, family: str) -> None:
        self.family = family
        self._entries: dict[str, _Entry[T]] = {}

    def register(
        self,
        name: str,
        *,
        devices: set[str] | None = None,
        dtypes: set[torch.dtype] | None = None,
        supports: Callable[[BackendContext], str | None] | None = None,
    ) -> Callable[[Callable[[BackendContext], T]], Callable[[BackendContext], T]]:
        """Class decorator registering ``cls`` as ``name``; a name registers once."""

        def wrap(factory: Callable[[BackendContext], T]) -> Callable[[BackendContext], T]:
            if name in self._entries:
                raise ValueError(f"{self.family} backend {name!r} registered twice")
            self._entries[name] = _Entry(
                factory,
                frozenset(devices) if devices is not None else None,
                frozenset(dtypes) if dtypes is not None else None,
                supports,
            )
            return factory

        return wrap

    def names(self) -> list[str]:
        return sorted(self._entries)

    def unsupported(self, name: str, ctx: BackendContext) -> str | None:
        """Why ``name`` cannot run in ``ctx``, or ``None`` if it can."""
        if name not in self._entries:
            return f"unknown {self.family} backend {name!r}; available: {self.names()}"
        return self._entries[name].unsupported(ctx)

    def resolve(self, name: str, ctx: BackendContext) -> T:
        if (reason := self.unsupported(name, ctx)) is not None:
            prefix = "" if name not in self._entries else f"{self.family} backend {name!r} "
            raise ValueError(prefix + reason)
        return self._entries[name].factory(ctx)
