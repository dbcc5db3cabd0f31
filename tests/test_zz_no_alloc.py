"""``vsamp_sample_noalloc`` (the library's own workspace, no allocation) against ``vsamp_sample``
(a caller workspace), through the C ABI: identical ids and draft probabilities on two calls in
a row, the second smaller, on rows that take the workspace path (fp32 rows; bf16 rows whose
history is too long for the fast path); sizes past its workspace and a caller workspace are
rejected before any launch."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from vinfer_amd import _lib
from vinfer_amd.registry import BackendContext
from vinfer_amd.sampler import SAMPLER
from vinfer_amd.sampling import pack_history, pack_params, SamplingParams
from vinfer_amd.workloads import zipf_ids

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def batch(seed, B, V, dtype, hist_len):
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, V, generator=g) * 2.0).to(dtype).to(DEV)
    params = pack_params(
        [SamplingParams(temperature=float(rng.choice([0.0, 0.7, 1.0])), top_k=int(rng.choice([0, 50])),
                        top_p=float(rng.choice([1.0, 0.9])), repetition_penalty=1.05, presence_penalty=0.5,
                        frequency_penalty=0.2) for _ in range(B)], DEV)
    perm = rng.permutation(V)
    hist = [zipf_ids(rng, int(rng.integers(hist_len // 2, hist_len + 1)), V, 1.05, perm).tolist() for _ in range(B)]
    hi, ho = pack_history(hist, DEV)
    u = torch.from_numpy(rng.random(B, dtype=np.float32)).to(DEV)
    draft = torch.from_numpy(rng.integers(0, V, B).astype(np.int32)).to(DEV)
    return x, params, u, hi, ho, draft


def call(noalloc: bool, x, params, u, hi, ho, draft):
    s = SAMPLER.resolve("hip", BackendContext(DEV, x.dtype))
    a, keep = s._args(x, params, hi, ho, u, draft)
    B = x.shape[0]
    ids = torch.full((B,), -7, dtype=torch.int32, device=DEV)
    dprob = torch.full((B,), -1.0, dtype=torch.float32, device=DEV)
    a.out_ids, a.out_draft_prob = ids.data_ptr(), dprob.data_ptr()
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    if noalloc:
        a.workspace, a.workspace_bytes = None, 0
        rc = lib.vsamp_sample_noalloc(ctypes.byref(a), stream)
    else:
        rc = lib.vsamp_sample(ctypes.byref(a), stream)
    _lib.check(rc)
    torch.cuda.synchronize()
    del keep
    return ids.cpu(), dprob.cpu()


def test_noalloc_equals_the_workspace_entry_point_twice():
    cases = [
        ("fp32 B=24 V=151936 histories <= 20000", (1, 24, 151936, torch.float32, 20000)),
        ("bf16 B=8 V=50000 histories <= 9000 (past the fast path)", (2, 8, 50000, torch.bfloat16, 9000)),
    ]
    for label, args in cases:  # the second call is smaller than the first
        print(f"noalloc vs vsamp_sample: {label}", flush=True)
        inputs = batch(*args)
        want_ids, want_dp = call(False, *inputs)
        got_ids, got_dp = call(True, *inputs)
        assert torch.equal(got_ids, want_ids), label
        assert torch.equal(got_dp.view(torch.int32), want_dp.view(torch.int32)), label
        assert (got_ids >= 0).all()


def test_noalloc_rejects_what_it_cannot_hold():
    s = SAMPLER.resolve("hip", BackendContext(DEV, torch.float32))
    x = torch.zeros(1, 1000, device=DEV)
    params = pack_params([SamplingParams(repetition_penalty=1.1)], DEV)
    hi = torch.zeros(2_000_000, dtype=torch.int32, device=DEV)  # 24 MB of workspace: past 16 MiB
    ho = torch.tensor([0, 2_000_000], dtype=torch.int32, device=DEV)
    u = torch.zeros(1, device=DEV)
    a, keep = s._args(x, params, hi, ho, u)
    out = torch.empty(1, dtype=torch.int32, device=DEV)
    a.out_ids = out.data_ptr()
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    rc = lib.vsamp_sample(ctypes.byref(a), stream)  # (a caller workspace of that size is fine)
    assert rc == 0
    rc = lib.vsamp_sample_noalloc(ctypes.byref(a), stream)
    assert rc == 1 and b"leave workspace NULL" in lib.vsamp_last_error()
    a.workspace, a.workspace_bytes = None, 0
    rc = lib.vsamp_sample_noalloc(ctypes.byref(a), stream)
    assert rc == 4 and b"more than its" in lib.vsamp_last_error()
    torch.cuda.synchronize()
    del keep
