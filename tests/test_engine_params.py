"""Both sampler backends take the engine's own ``SamplingParams``.

The engine's class (src/vinfer/runtime/sampler.py:18-41) has eight fields and none of this
package's extension fields. The runtime passes it unchanged to ``sample`` (generate.py:129), and
the registry's rule is that callers do not change (kernels/registry.py:3-7). ``EngineParams``
below has exactly those eight fields, defaults and checks. ``EngineParamsPen`` adds the four
sampling extension fields with their off defaults, as INTEGRATION.md tells a maintainer to do.
Every call with either class must equal the same call with this package's ``SamplingParams``.
The integration snippet of INTEGRATION.md is executed against a fresh registry.
"""

from __future__ import annotations

import re
import sys
import types
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import pytest
import torch

from vinfer_amd import registry as registry_mod
from vinfer_amd.registry import BackendContext
from vinfer_amd.runtime import BatchDecoder
from vinfer_amd.sampler import SAMPLER, ReferenceSampler
from vinfer_amd.sampling import SamplingParams, pack_params, penalized
from vinfer_amd.workloads import SyntheticLM

GUIDE = Path(__file__).resolve().parents[1] / "INTEGRATION.md"


@dataclass(frozen=True)
class EngineParams:
    """The engine's class: sampler.py:18-41, field for field."""

    max_tokens: int = 16
    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0
    seed: int | None = None
    stop: tuple[str, ...] = ()
    stop_token_ids: tuple[int, ...] = ()
    ignore_eos: bool = False

    def __post_init__(self) -> None:
        if self.temperature < 0:
            raise ValueError(f"temperature must be >= 0, got {self.temperature}")
        if not 0 < self.top_p <= 1:
            raise ValueError(f"top_p must be in (0, 1], got {self.top_p}")
        if self.top_k < 0:
            raise ValueError(f"top_k must be >= 0, got {self.top_k}")
        if self.max_tokens < 1:
            raise ValueError(f"max_tokens must be >= 1, got {self.max_tokens}")

    @property
    def greedy(self) -> bool:
        return self.temperature == 0


@dataclass(frozen=True)
class EngineParamsPen(EngineParams):
    """The engine's class with the four sampling extension fields added, off by default."""

    repetition_penalty: float = 1.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    min_p: float = 0.0


ENGINE_FIELDS = ("max_tokens", "temperature", "top_k", "top_p", "seed", "stop", "stop_token_ids", "ignore_eos")
PEN_FIELDS = ("repetition_penalty", "presence_penalty", "frequency_penalty", "min_p")


def ours(p) -> SamplingParams:
    """The same request as this package's ``SamplingParams``."""
    names = ENGINE_FIELDS + (PEN_FIELDS if isinstance(p, EngineParamsPen) else ())
    return SamplingParams(**{k: getattr(p, k) for k in names})


PLAIN = [
    EngineParams(temperature=0.0),
    EngineParams(temperature=0.7, top_k=20, top_p=0.8),
    EngineParams(temperature=1.2, top_p=0.5),
    EngineParams(),
]
WITH_PEN = [
    EngineParamsPen(temperature=1.0, top_p=0.95, min_p=0.05, repetition_penalty=1.05, presence_penalty=0.5,
                    frequency_penalty=0.2),
    EngineParamsPen(temperature=0.0, frequency_penalty=10.0),
    EngineParamsPen(temperature=0.8, top_k=50, min_p=0.1),
    EngineParamsPen(temperature=0.9),  # the added fields at their defaults: no history needed
]


def test_the_engine_class_shape():
    assert tuple(EngineParams.__dataclass_fields__) == ENGINE_FIELDS
    assert not hasattr(EngineParams(), "penalized") and not hasattr(EngineParams(), "min_p")
    assert not penalized(EngineParams()) and not penalized(EngineParamsPen())
    assert penalized(EngineParamsPen(presence_penalty=0.5))
    packed = pack_params([EngineParams(temperature=0.5), EngineParamsPen(min_p=0.2, repetition_penalty=1.3)])
    want = pack_params([SamplingParams(temperature=0.5), SamplingParams(min_p=0.2, repetition_penalty=1.3)])
    for k in want.__dataclass_fields__:
        assert torch.equal(getattr(packed, k), getattr(want, k)), k


def _histories(V: int):
    return [[], [3, 3, 1], list(range(0, V, 7)) + [5, 5, 5]]


def test_reference_backend_takes_the_engine_params():
    s = ReferenceSampler(BackendContext(torch.device("cpu"), torch.float32))
    g = torch.Generator().manual_seed(3)
    V = 500
    x = torch.randn(V, generator=g) * 2
    for p in PLAIN:
        for pos in range(4):
            assert s.sample(x, p, 9, pos) == s.sample(x, ours(p), 9, pos)
    for p in WITH_PEN:
        for pos, h in enumerate(_histories(V)):
            assert s.sample(x, p, 9, pos, history=h) == s.sample(x, ours(p), 9, pos, history=h)
    with pytest.raises(ValueError, match="history"):
        s.sample(x, WITH_PEN[0], 9, 0)


def test_decode_loop_takes_the_engine_params():
    model = SyntheticLM(96, dim=16, scale=3.0, dtype=torch.float32)
    s = SAMPLER.resolve("reference", BackendContext(torch.device("cpu"), torch.float32))
    reqs = [([5, 17, 3], EngineParams(max_tokens=6, seed=11, temperature=0.8, top_k=20)),
            ([1, 2], EngineParamsPen(max_tokens=6, seed=12, temperature=0.0, frequency_penalty=100.0)),
            ([7], EngineParams(max_tokens=5, seed=13))]

    def run(rs):
        dec = BatchDecoder(model, s, num_slots=2, max_seq_len=32)
        rids = [dec.submit(p, sp) for p, sp in rs]
        done = dec.run()
        return [done[r] for r in rids]

    assert run(reqs) == run([(p, ours(sp)) for p, sp in reqs])


def _snippet() -> str:
    text = GUIDE.read_text()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    block = next(b for b in blocks if "src/vinfer/kernels/sampler/__init__.py (new)" in b)
    lines = block.splitlines()
    indent = min(len(ln) - len(ln.lstrip()) for ln in lines if ln.strip())
    return "\n".join(ln[indent:] for ln in lines) + "\n"


def _engine_modules(calls: list) -> dict[str, types.ModuleType]:
    """Stand-ins for the engine modules the snippet imports: the registry is this package's
    stand-in (same API and messages); the engine's ``sample`` is recorded and answered by the
    package's reference backend."""
    ref = ReferenceSampler(BackendContext(torch.device("cpu"), torch.float32))

    def sample(logits, params, seed, position):
        calls.append((seed, position))
        return ref.sample(logits.cpu(), params, seed, position)

    mods = {name: types.ModuleType(name) for name in ("vinfer", "vinfer.kernels", "vinfer.runtime",
                                                      "vinfer.runtime.sampler")}
    mods["vinfer.kernels.registry"] = registry_mod
    mods["vinfer.runtime.sampler"].sample = sample
    mods["vinfer.runtime"].sampler = mods["vinfer.runtime.sampler"]
    mods["vinfer"].kernels, mods["vinfer"].runtime = mods["vinfer.kernels"], mods["vinfer.runtime"]
    mods["vinfer.kernels"].registry = registry_mod
    return mods


def run_snippet(calls: list) -> dict:
    ns: dict = {"__name__": "vinfer.kernels.sampler"}
    mods = _engine_modules(calls)
    saved = {k: sys.modules.get(k) for k in mods}
    sys.modules.update(mods)
    try:
        exec(compile(_snippet(), str(GUIDE), "exec"), ns)
    finally:
        for k, v in saved.items():
            if v is None:
                sys.modules.pop(k, None)
            else:
                sys.modules[k] = v
    return ns


def test_integration_snippet_registers_both_backends():
    calls: list = []
    ns = run_snippet(calls)
    reg = ns["SAMPLER"]
    assert reg is not SAMPLER and reg.names() == ["hip", "reference"]
    ref = reg.resolve("reference", BackendContext(torch.device("cpu"), torch.float32))
    x = torch.tensor([2.0, 1.0, 0.5, 0.0, -1.0, -3.0])
    assert ref.sample(x, EngineParams(temperature=0.0), 1, 0) == 0 and calls == [(1, 0)]
    if not torch.cuda.is_available():
        # the startup check says why, never a fallback (kernels/registry.py:5-7)
        with pytest.raises(ValueError, match="hip"):
            reg.resolve("hip", BackendContext(torch.device("cuda"), torch.bfloat16))


# ---- on the GPU: the hip backend through the integration snippet's registry ----------------


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_gpu_hip_backend_takes_the_engine_params(dtype):
    from oracle.sampler_oracle import classify_ties
    from oracle.sampler_oracle import sample_batch as oracle_batch
    from vinfer_amd.sampling import uniform

    dev = torch.device("cuda", 0)
    ns = run_snippet([])
    hip = ns["SAMPLER"].resolve("hip", BackendContext(dev, dtype))
    assert type(hip).__name__ == "HipSampler"
    V = 151936
    g = torch.Generator().manual_seed(21)
    x = (torch.randn(V, generator=g) * 2).to(dtype)
    row = x.to(dev)
    xs = x.float().numpy()
    print(f"engine params through the snippet's registry, V={V} {dtype}", flush=True)
    for ci, p in enumerate(PLAIN + WITH_PEN):
        q = ours(p)
        for pos, h in enumerate(_histories(V)):
            hist = h if penalized(p) else None
            tok = hip.sample(row, p, 40 + ci, pos, history=hist)
            assert tok == hip.sample(row, q, 40 + ci, pos, history=hist), (ci, pos)
            hi = np.asarray(h if penalized(p) else [], dtype=np.int32)
            res = oracle_batch(xs[None], [q.temperature], [q.top_k], [q.top_p], [q.min_p],
                               [q.repetition_penalty], [q.presence_penalty], [q.frequency_penalty],
                               hi, np.array([0, len(hi)], np.int32), [uniform(40 + ci, pos)])[0]
            if not classify_ties(res):
                assert tok == res.token, (ci, pos, tok, res.token)
    with pytest.raises(ValueError, match="history"):
        hip.sample(row, WITH_PEN[0], 1, 0)
    # the batched entry with the engine's objects packed
    B = 8
    ps = (PLAIN + WITH_PEN)[:B]
    xb = (torch.randn(B, V, generator=g) * 2).to(dtype).to(dev)
    u = torch.rand(B, generator=g).to(dev)
    a, _ = hip.sample_batch(xb, pack_params(ps, dev), u)
    b, _ = hip.sample_batch(xb, pack_params([ours(p) for p in ps], dev), u)
    assert torch.equal(a, b)
