"""Per-request sampling parameters, per-position seeds and the per-step uniform.

``SamplingParams`` keeps every field, default and validation rule of the engine's class
(src/vinfer/runtime/sampler.py:18-41) and adds six fields the engine's API layer names but does
not implement (server/protocol.py:131-135, :142): ``repetition_penalty``, ``presence_penalty``,
``frequency_penalty`` and ``min_p`` change the draw; ``logprobs`` and ``top_logprobs`` only ask
the decode loop to report log-probabilities. Each is added with its "off" value as default, so
existing callers construct the same objects and get the same behaviour.

``position_seed`` is the engine's 63-bit seed of ``(seed, position)`` (sampler.py:44-47).
``uniform`` turns it into the one uniform ``u`` in [0, 1) that the inverse-CDF draw consumes:
a SplitMix64 finaliser of the seed, top 24 bits, times 2**-24. So a request's token depends only
on its seed, position and its own logits (the property sampler.py:5-7 states), and, unlike a
``torch.Generator`` stream (sampler.py:73), it is the same on every device.
"""

from __future__ import annotations

import hashlib
import math
from dataclasses import dataclass

_MASK64 = (1 << 64) - 1


@dataclass(frozen=True)
class SamplingParams:
    max_tokens: int = 16
    temperature: float = 1.0  # 0 = greedy
    top_k: int = 0  # 0 = off
    top_p: float = 1.0  # 1 = off
    seed: int | None = None  # None: the runtime picks one per request
    stop: tuple[str, ...] = ()
    stop_token_ids: tuple[int, ...] = ()
    ignore_eos: bool = False
    # Extensions (off by default; names and off-values as in server/protocol.py:133-135, :142).
    repetition_penalty: float = 1.0  # 1 = off; > 1 discourages tokens already in the history
    presence_penalty: float = 0.0  # 0 = off; subtracted once from every token in the history
    frequency_penalty: float = 0.0  # 0 = off; subtracted once per occurrence in the history
    min_p: float = 0.0  # 0 = off; drop tokens with p < min_p * max p
    # Reported, not sampled (names and off-values as the API layer lists them, protocol.py:131-132):
    logprobs: bool = False  # the drawn token's log-probability under the raw logits
    top_logprobs: int = 0  # and the n most likely tokens' (0 .. 20; needs logprobs)

    def __post_init__(self) -> None:
        # The first four checks and messages are sampler.py:29-37.
        if self.temperature < 0:
            raise ValueError(f"temperature must be >= 0, got {self.temperature}")
        if not 0 < self.top_p <= 1:
            raise ValueError(f"top_p must be in (0, 1], got {self.top_p}")
        if self.top_k < 0:
            raise ValueError(f"top_k must be >= 0, got {self.top_k}")
        if self.max_tokens < 1:
            raise ValueError(f"max_tokens must be >= 1, got {self.max_tokens}")
        if not (self.repetition_penalty > 0 and math.isfinite(self.repetition_penalty)):
            raise ValueError(f"repetition_penalty must be > 0, got {self.repetition_penalty}")
        for name in ("presence_penalty", "frequency_penalty"):
            if not math.isfinite(getattr(self, name)):
                raise ValueError(f"{name} must be finite, got {getattr(self, name)}")
        if not 0 <= self.min_p <= 1:
            raise ValueError(f"min_p must be in [0, 1], got {self.min_p}")
        if not 0 <= self.top_logprobs <= 20:
            raise ValueError(f"top_logprobs must be in [0, 20], got {self.top_logprobs}")
        if self.top_logprobs and not self.logprobs:
            raise ValueError("top_logprobs needs logprobs")

    @property
    def greedy(self) -> bool:
        return self.temperature == 0

    @property
    def penalized(self) -> bool:
        return penalized(self)


# The extension fields and their off values. The engine's own SamplingParams (sampler.py:18-27)
# has none of them; every reader below takes them with ``field`` so that an object of the
# engine's class, or of that class with some of these fields added, is read as "off" for each
# field it lacks.
EXTENSION_DEFAULTS: dict[str, float | int | bool] = {
    "repetition_penalty": 1.0,
    "presence_penalty": 0.0,
    "frequency_penalty": 0.0,
    "min_p": 0.0,
    "logprobs": False,
    "top_logprobs": 0,
}


def field(params, name: str):
    """``params.<name>``; for an extension field the object lacks, its off value."""
    if name in EXTENSION_DEFAULTS:
        return getattr(params, name, EXTENSION_DEFAULTS[name])
    return getattr(params, name)


def penalized(params) -> bool:
    """Whether any of the three penalties is on for ``params`` (any params object)."""
    return (
        field(params, "repetition_penalty") != 1.0
        or field(params, "presence_penalty") != 0.0
        or field(params, "frequency_penalty") != 0.0
    )


def position_seed(seed: int, position: int) -> int:
    """A 63-bit seed derived from ``(seed, position)`` (sampler.py:44-47): BLAKE2b with an
    8-byte digest of ``"{seed}:{position}"``, read little-endian, top bit cleared."""
    digest = hashlib.blake2b(f"{seed}:{position}".encode(), digest_size=8).digest()
    return int.from_bytes(digest, "little") & ((1 << 63) - 1)


def splitmix64(x: int) -> int:
    """SplitMix64 output function (Steele, Lea, Flood 2014) of ``x + golden gamma``."""
    z = (x + 0x9E3779B97F4A7C15) & _MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _MASK64
    return z ^ (z >> 31)


def uniform(seed: int, position: int) -> float:
    """The draw's uniform for ``(seed, position)``: a multiple of 2**-24 in [0, 1), exactly
    representable in fp32, so host and device see the same value."""
    return (splitmix64(position_seed(seed, position)) >> 40) * 2.0**-24
