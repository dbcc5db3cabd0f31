"""Every registered sampler backend against the oracle, on this machine's devices, in fp32 and
bf16 (the pattern of the engine's tests/unit/kernels/test_backend_contract.py:1-30).

A new backend registered in ``SAMPLER`` is picked up here automatically. A backend that cannot
run in a (device, dtype) context is skipped there with its own reason (``unsupported``), so the
skip list says where each one runs. Each test runs one batch of mixed rows (greedy, top-k, top-p,
min-p, penalties with histories, draft ids) through ``sample_batch``, ``probs`` and
``penalized_logits`` and the per-token ``sample``."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.sampler_oracle import classify_ties, penalize
from tests.parity import compare_ids, oracle
from vinfer_amd.registry import BackendContext
from vinfer_amd.sampler import SAMPLER
from vinfer_amd.sampling import SamplingParams, pack_history, pack_params
from vinfer_amd.workloads import Workload

DEVICES = [torch.device("cpu"), pytest.param(torch.device("cuda", 0), marks=pytest.mark.gpu)]
DTYPES = [torch.float32, torch.bfloat16]


def _backend(name, device, dtype):
    ctx = BackendContext(device, dtype)
    if (reason := SAMPLER.unsupported(name, ctx)) is not None:
        pytest.skip(reason)
    return SAMPLER.resolve(name, ctx)


def _batch(dtype, B=12, V=700, seed=3) -> Workload:
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, V, generator=g) * 2.5).to(dtype)
    kinds = [dict(temperature=0.0), dict(temperature=0.8, top_k=20), dict(temperature=1.0, top_p=0.9),
             dict(temperature=1.2, min_p=0.05, top_p=0.95),
             dict(temperature=0.7, repetition_penalty=1.3, presence_penalty=0.5, frequency_penalty=0.2),
             dict(temperature=1.0, top_k=50, top_p=0.8, frequency_penalty=1.0)]
    params = pack_params([SamplingParams(**kinds[b % len(kinds)]) for b in range(B)])
    hist = [rng.integers(0, V, int(rng.integers(0, 40))).tolist() for _ in range(B)]
    hi, ho = pack_history(hist)
    u = torch.from_numpy(rng.random(B, dtype=np.float32))
    draft = torch.from_numpy(rng.integers(0, V, B).astype(np.int32))
    return Workload("contract", x, params, u, hi, ho, draft)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("device", DEVICES, ids=str)
@pytest.mark.parametrize("name", SAMPLER.names())
def test_sampler_backend_matches_the_oracle(name, device, dtype):
    backend = _backend(name, device, dtype)
    w = _batch(dtype)
    d = w.to(device)
    ids, dp = backend.sample_batch(d.logits, d.params, d.uniforms, d.hist_ids, d.hist_offsets, d.draft_ids)
    assert ids.dtype == torch.int32 and ids.device.type == device.type
    ties, bad = compare_ids(ids.cpu(), oracle(w), dp.cpu())
    assert not bad and ties <= 1, (bad, ties)
    # the final distribution, non-tie rows within 1e-5 relative
    pr = backend.probs(d.logits, d.params, d.hist_ids, d.hist_offsets).cpu().double().numpy()
    for b, r in enumerate(oracle(w, want_probs=True)):
        if not classify_ties(r):
            np.testing.assert_allclose(pr[b], r.probs, rtol=1e-5, atol=1e-30)
    # penalised logits and exact counts
    xs, counts = backend.penalized_logits(d.logits, d.params, d.hist_ids, d.hist_offsets)
    p = w.params
    for b in range(w.batch):
        h = w.hist_ids[int(w.hist_offsets[b]) : int(w.hist_offsets[b + 1])].numpy()
        want_x, want_c = penalize(w.logits[b].float().numpy(), h, float(p.repetition_penalty[b]),
                                  float(p.presence_penalty[b]), float(p.frequency_penalty[b]))
        assert (counts[b].cpu().numpy() == want_c).all()
        assert (xs[b].cpu().numpy().view(np.uint32) == want_x.view(np.uint32)).all()


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("device", DEVICES, ids=str)
@pytest.mark.parametrize("name", SAMPLER.names())
def test_per_token_sample_is_the_one_row_batch(name, device, dtype):
    # the engine's call (generate.py:129) draws the same token as a one-row batch with the
    # uniform of (seed, position)
    from vinfer_amd.sampling import uniform

    backend = _backend(name, device, dtype)
    w = _batch(dtype, B=6, seed=9)
    d = w.to(device)
    for b in range(w.batch):
        row = {k: getattr(w.params, k)[b].item() for k in w.params.__dataclass_fields__}
        sp = SamplingParams(**{k: (int(v) if k == "top_k" else v) for k, v in row.items()})
        hist = w.hist_ids[int(w.hist_offsets[b]) : int(w.hist_offsets[b + 1])].tolist()
        tok = backend.sample(d.logits[b], sp, 11, 40 + b, history=hist)
        u = torch.tensor([uniform(11, 40 + b)], dtype=torch.float32, device=device)
        hi = torch.tensor(hist, dtype=torch.int32, device=device) if hist else None
        ho = torch.tensor([0, len(hist)], dtype=torch.int32, device=device) if hist else None
        ids, _ = backend.sample_batch(d.logits[b : b + 1], w.params.select(torch.tensor([b])).to(device), u, hi, ho)
        assert tok == int(ids[0])
