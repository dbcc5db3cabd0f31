"""A seeded random sweep through ``sample_batch``: shapes from 97 to 262144 tokens, bf16 and fp32,
padded row strides, plain, peaked and tied rows, every parameter (greedy to T = 1.5, top-k past
the sorted lists' 256, top-p, min-p, all three penalties) and histories up to 4096 ids, each
launch run twice. Every non-tie row's id and draft probability against the oracle, and the two
launches bit for bit equal."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.parity import compare_ids, oracle
from vinfer_amd.registry import BackendContext
from vinfer_amd.sampler import SAMPLER
from vinfer_amd.sampling import SamplingParams, pack_history, pack_params
from vinfer_amd.workloads import Workload

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
CASES_PER_TEST = 10


def sweep_case(seed: int) -> tuple[Workload, torch.Tensor]:
    """The seed's workload (CPU) and its logits on the device, in a buffer with padded rows."""
    rng = np.random.default_rng(10_000 + seed)
    g = torch.Generator().manual_seed(10_000 + seed)
    V = int(rng.choice([97, 1000, 4099, 32768, 65536, 151936, 200003, 262144]))
    B = int(rng.integers(1, 40 if V > 100000 else 120))
    dtype = torch.bfloat16 if rng.random() < 0.6 else torch.float32
    kind = int(rng.integers(0, 4))
    x = torch.randn(B, V, generator=g) * float(rng.choice([0.01, 0.1, 1.0, 3.0]))
    if kind == 1:  # one token far above the rest
        x[torch.arange(B), torch.from_numpy(rng.integers(0, V, B))] += 15.0
    elif kind == 2:  # a run of equal values
        for b in range(B):
            s0 = int(rng.integers(0, max(1, V - 600)))
            x[b, s0 : s0 + int(rng.integers(1, 600))] = float(rng.choice([0.25, 5.0, 0.0]))
    x = x.to(dtype)
    pad = int(rng.choice([0, 0, 3, 8]))
    buf = torch.zeros(B, V + pad, dtype=dtype)
    buf[:, :V] = x
    params = [
        SamplingParams(
            temperature=float(rng.choice([0.0, 0.3, 0.7, 1.0, 1.5])),
            top_k=int(rng.choice([0, 0, 1, 20, 50, 256, 300, 1000, V - 1])),
            top_p=float(rng.choice([1.0, 1.0, 0.5, 0.8, 0.95, 1e-6])),
            min_p=float(rng.choice([0.0, 0.0, 0.05, 0.3])),
            repetition_penalty=float(rng.choice([1.0, 1.0, 1.05, 1.3])),
            presence_penalty=float(rng.choice([0.0, 0.0, 0.5])),
            frequency_penalty=float(rng.choice([0.0, 0.0, 0.2])),
        )
        for _ in range(B)
    ]
    hl = int(rng.choice([0, 64, 2048, 4096]))
    hi, ho = pack_history([rng.integers(0, V, int(rng.integers(0, hl + 1))).tolist() for _ in range(B)])
    u = torch.from_numpy(rng.random(B, dtype=np.float32))
    draft = torch.from_numpy(rng.integers(0, V, B).astype(np.int32))
    w = Workload(f"sweep{seed}", x, pack_params(params), u, hi, ho, draft)
    return w, buf.to(DEV)[:, :V]


@pytest.mark.parametrize("first", range(0, 6 * CASES_PER_TEST, CASES_PER_TEST))
def test_gpu_random_sweep_matches_the_oracle(first):
    for seed in range(first, first + CASES_PER_TEST):
        w, logits = sweep_case(seed)
        print(f"sweep seed {seed} B={w.batch} V={w.vocab} {w.logits.dtype} stride={logits.stride(0)}", flush=True)
        s = SAMPLER.resolve("hip", BackendContext(DEV, w.logits.dtype))
        d = w.to(DEV)
        args = (logits, d.params, d.uniforms, d.hist_ids, d.hist_offsets, d.draft_ids)
        ids, dp = s.sample_batch(*args)
        ids2, dp2 = s.sample_batch(*args)
        torch.cuda.synchronize()
        assert torch.equal(ids, ids2) and torch.equal(dp.view(torch.int32), dp2.view(torch.int32)), seed
        ties, bad = compare_ids(ids.cpu(), oracle(w), dp.cpu())
        assert not bad, (seed, bad[:5])
        assert ties <= max(2, 0.25 * w.batch), (seed, ties)
