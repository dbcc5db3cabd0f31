"""Repeated launches on the same inputs give the same outputs, bit for bit.

Every kernel here decides a row inside one workgroup (or inside one row's workgroups) through LDS
and barriers; a missing barrier shows first as a launch whose result depends on how its waves
happen to interleave, which one run against the oracle can miss. Each path below runs REPEAT
times on fixed inputs -- rows with penalties, drafts and mixed parameters, rows of massive ties
whose top-p cutoff splits a group of equal values (two member searches in one workgroup), row
states, split rows, fp32 rows through the generic path, the speculative verify with its
residual's hand-off between workgroups -- and every launch must equal the first.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from vinfer_amd import workloads
from vinfer_amd.registry import BackendContext
from vinfer_amd.sampler import SAMPLER
from vinfer_amd.sampling import SamplingParams, pack_params

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
REPEAT = 16


def hip(dtype=torch.bfloat16):
    return SAMPLER.resolve("hip", BackendContext(DEV, dtype))


def bits(t: torch.Tensor) -> torch.Tensor:
    """The tensor's bytes as integers (NaN-safe, -0.0 apart from +0.0)."""
    return t.contiguous().view(torch.uint8).cpu()


def same_every_time(fn, label: str) -> None:
    print(f"repeat {label}", flush=True)
    first = [bits(t) for t in fn() if t is not None]
    for i in range(1, REPEAT):
        out = [bits(t) for t in fn() if t is not None]
        for k, (a, b) in enumerate(zip(first, out)):
            assert torch.equal(a, b), (label, "launch", i, "output", k)


def tied_rows(B: int, V: int, seed: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Rows whose top-k and top-p cutoffs fall inside groups of equal values, and draft ids inside
    the kept part of those groups."""
    g = torch.Generator().manual_seed(seed)
    rows, drafts = [], []
    for b in range(B):
        kind = b % 3
        if kind == 0:
            x = torch.full((V,), 0.25)
        elif kind == 1:
            x = torch.randn(V, generator=g)
            x[: 300 + b] = 5.0
        else:
            x = torch.randn(V, generator=g) * 0.01
            x[b % 97 : b % 97 + 600] = 0.0390625
        rows.append(x)
        drafts.append(b % 150)
    return torch.stack(rows).to(torch.bfloat16).to(DEV), torch.tensor(drafts, dtype=torch.int32, device=DEV)


def uniforms(B: int, seed: int) -> torch.Tensor:
    return torch.from_numpy(np.random.default_rng(seed).random(B, dtype=np.float32)).to(DEV)


@pytest.mark.parametrize("name,batch,vocab", [("mixed_bf16", 64, None), ("peaked_flat", 256, None),
                                              ("large_fp32", 128, None), ("verify_bf16", 64, None)])
def test_gpu_workload_launches_repeat_exactly(name, batch, vocab):
    w = workloads.make(name, batch=batch, vocab=vocab).to(DEV)
    s = hip(w.logits.dtype)
    same_every_time(lambda: s.sample_batch(w.logits, w.params, w.uniforms, w.hist_ids, w.hist_offsets, w.draft_ids),
                    f"{name} B={batch}")


def test_gpu_split_rows_repeat_exactly():
    w = workloads.make("mixed_bf16", batch=16).to(DEV)
    s = hip()
    s.split_rows = True
    same_every_time(lambda: s.sample_batch(w.logits, w.params, w.uniforms, w.hist_ids, w.hist_offsets, w.draft_ids),
                    "mixed_bf16 split rows B=16")


@pytest.mark.parametrize("V", [4099, 8192])
def test_gpu_tied_rows_repeat_exactly_on_every_path(V):
    B = 48
    logits, draft = tied_rows(B, V, seed=V)
    s = hip()
    for T, kw in [(0.5, dict(top_k=20, top_p=0.5)), (1.0, dict(top_p=0.3))]:
        pp = pack_params([SamplingParams(temperature=T, **kw) for _ in range(B)], DEV)
        u = uniforms(B, seed=V + len(kw))
        label = f"tied V={V} T={T} {kw}"

        def row_passes():
            s.tile_pass = False
            try:
                return s.sample_batch(logits, pp, u, None, None, draft)
            finally:
                s.tile_pass = True

        same_every_time(row_passes, label + " row passes")
        same_every_time(lambda: s.sample_tile_pass(logits, pp, u, None, None, draft), label + " tile pass")
        same_every_time(lambda: s.sample_states(logits, pp, u), label + " row states")


def test_gpu_verify_repeats_exactly():
    # the verify's residual hands each rejected row's stripe sums between its workgroups: half the
    # drafts are the draft rows' argmax (mostly accepted), half random ids (mostly rejected)
    B, K, V = 96, 2, 151936
    g = torch.Generator().manual_seed(5)
    xt = torch.randn(B, K + 1, V, generator=g) * 2.5
    xq = xt[:, :K] + torch.randn(B, K, V, generator=g) * 0.5
    drafts = torch.randint(0, V, (B, K), generator=g, dtype=torch.int32)
    drafts[::2] = xq[::2].argmax(-1).to(torch.int32)
    pp = pack_params([SamplingParams(temperature=0.8, top_p=0.95) for _ in range(B)], DEV)
    rng = np.random.default_rng(6)
    ua, ur = (torch.from_numpy(rng.random((B, K), np.float32)).to(DEV) for _ in range(2))
    ub = uniforms(B, seed=7)
    xt, xq, drafts = xt.to(torch.bfloat16).to(DEV), xq.to(torch.bfloat16).to(DEV), drafts.to(DEV)
    s = hip()
    same_every_time(lambda: s.verify(xt, xq, drafts, pp, ua, ur, ub), f"verify B={B} K={K} V={V}")
