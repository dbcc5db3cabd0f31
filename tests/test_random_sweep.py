"""Seeded random sweeps against the oracle. ``sample_batch``: shapes from 97 to 262144 tokens,
bf16 and fp32, padded row strides, plain, peaked and tied rows, every parameter (greedy to
T = 1.5, top-k past the sorted lists' 256, top-p, min-p, all three penalties) and histories up to
4096 ids, each launch run twice: every non-tie row's id and draft probability, and the two
launches bit for bit equal. Log-probabilities, raw and from tile statistics, over rows with ties,
NaNs and infinities. The speculative verify over random draft counts, vocabularies and scales.
The per-token call with its vocabulary, dtype, parameters and history form changing per call."""

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


def test_gpu_random_sweep_of_log_probabilities():
    # raw log-probabilities (vsamp_logprobs) and those from another GEMM's tile statistics
    # (vsamp_tile_stats + vsamp_logprobs_tiles) on seeded random rows: ties, one value, NaN, -inf
    # runs, +inf, padded strides, n_top up to 32; top ids exact, values within 2e-6 + 1e-6 |lp|
    # (1e-5 from the tile statistics, whose sums run in another order)
    import math

    from oracle.sampler_oracle import logprobs_row

    for seed in range(40):
        rng = np.random.default_rng(20_000 + seed)
        g = torch.Generator().manual_seed(20_000 + seed)
        V = int(rng.choice([6, 97, 1000, 4099, 32768, 151936]))
        B = int(rng.integers(1, 33))
        dtype = torch.bfloat16 if rng.random() < 0.6 else torch.float32
        n_top = int(rng.choice([0, 1, 5, 20, 32]))
        x = torch.randn(B, V, generator=g) * float(rng.choice([0.01, 1.0, 2.5, 8.0]))
        for b in range(B):
            k = rng.integers(0, 8)
            if k == 1:
                x[b] = torch.round(x[b] * 4) / 4
            elif k == 2:
                x[b] = float(rng.choice([0.0, 0.25]))
            elif k == 3:
                x[b, int(rng.integers(0, V))] = float("nan")
            elif k == 4:
                x[b, : int(rng.integers(1, V + 1))] = float("-inf")
            elif k == 5:
                x[b, int(rng.integers(0, V))] = float("inf")
        x = x.to(dtype)
        pad = int(rng.choice([0, 0, 1, 5]))
        buf = torch.zeros(B, V + pad, dtype=dtype)
        buf[:, :V] = x
        logits = buf.to(DEV)[:, :V]
        tokens = torch.from_numpy(rng.integers(-2, V + 2, B).astype(np.int32))
        print(f"logprobs sweep seed {seed} B={B} V={V} {dtype} n_top={n_top} pad={pad}", flush=True)
        s = SAMPLER.resolve("hip", BackendContext(DEV, dtype))
        outs = {"raw": s.logprobs(logits, tokens.to(DEV), n_top)}
        if dtype == torch.bfloat16:
            tm, ts = s.tile_stats(logits)
            outs["tiles"] = s.logprobs_tiles(logits, tm, ts, tokens.to(DEV), n_top)
        torch.cuda.synchronize()
        xs = x.float().numpy()
        for name, (tl, ids, lps) in outs.items():
            tl, ids, lps = tl.cpu().numpy(), ids.cpu().numpy(), lps.cpu().numpy()
            rtol, atol = (1e-6, 2e-6) if name == "raw" else (1e-5, 1e-5)
            for b in range(B):
                wt, wids, wv = logprobs_row(xs[b], int(tokens[b]), n_top)
                assert ids[b].tolist() == wids, (seed, name, b)
                fin = np.isfinite(wv)
                np.testing.assert_allclose(lps[b][fin], wv[fin], rtol=rtol, atol=atol)
                assert np.array_equal(np.isnan(lps[b]), np.isnan(wv)), (seed, name, b)
                assert np.array_equal(np.isneginf(lps[b]), np.isneginf(wv)), (seed, name, b)
                if math.isnan(wt):
                    assert math.isnan(tl[b]), (seed, name, b)
                elif math.isinf(wt):
                    assert tl[b] == wt, (seed, name, b)
                else:
                    assert abs(tl[b] - wt) <= atol + rtol * abs(wt), (seed, name, b, tl[b], wt)


def test_gpu_random_sweep_of_the_verify():
    # the speculative verify over random sequence counts, draft counts, vocabularies, dtypes and
    # logit scales (most sequences draw from a residual): every non-tie sequence's tokens
    from tests.test_verify import oracle_verify, verify_case

    residual = 0
    for seed in range(20):
        rng = np.random.default_rng(30_000 + seed)
        K = int(rng.integers(1, 4))
        V = int(rng.choice([97, 1000, 4099, 20000, 65536]))
        B = int(rng.integers(1, 40))
        dtype = torch.bfloat16 if rng.random() < 0.6 else torch.float32
        sigma, noise = float(rng.choice([0.1, 1.0, 2.0, 4.0])), float(rng.choice([0.05, 0.5, 2.0]))
        xt, xq, drafts, params, ua, ur, ub = verify_case(30_000 + seed, B, K, V, dtype, sigma=sigma, noise=noise)
        print(f"verify sweep seed {seed} B={B} K={K} V={V} {dtype}", flush=True)
        s = SAMPLER.resolve("hip", BackendContext(DEV, dtype))

        def to(a, t=None):
            return torch.from_numpy(np.ascontiguousarray(a)).to(DEV) if t is None else torch.from_numpy(a).to(t).to(DEV)

        tokens, counts = s.verify(to(xt, dtype), to(xq, dtype), to(drafts), params.to(DEV), to(ua), to(ur), to(ub))
        tokens, counts = tokens.cpu(), counts.cpu()
        for b, w in enumerate(oracle_verify(xt, xq, drafts, params, ua, ur, ub)):
            if w.ties:
                continue
            residual += len(w.tokens) <= K and w.tokens[-1] != int(drafts[b, len(w.tokens) - 1])
            assert int(counts[b]) == len(w.tokens), (seed, b)
            assert tokens[b, : len(w.tokens)].tolist() == w.tokens, (seed, b)
            assert (tokens[b, len(w.tokens) :] == -1).all(), (seed, b)
    assert residual > 0


def test_gpu_random_sweep_of_the_per_token_call():
    # the engine's per-token call sample(logits[V], params, seed, position, history) through one
    # sampler whose vocabulary, logits dtype, parameters and history form change from call to call
    # (its pinned buffers and argument block are cached per shape), rows at odd offsets of a
    # larger buffer; every non-tie token against the oracle
    from oracle.sampler_oracle import classify_ties
    from oracle.sampler_oracle import sample_batch as oracle_batch
    from vinfer_amd.sampling import uniform

    s = SAMPLER.resolve("hip", BackendContext(DEV, torch.bfloat16))
    rng = np.random.default_rng(40_000)
    g = torch.Generator().manual_seed(40_000)
    for call in range(80):
        V = int(rng.choice([97, 1000, 4099, 151936]))
        dtype = torch.bfloat16 if rng.random() < 0.5 else torch.float32
        off = int(rng.integers(0, 9))
        big = (torch.randn(V + 16, generator=g) * float(rng.choice([0.1, 2.0, 4.0]))).to(dtype)
        x = big[off : off + V]
        sp = SamplingParams(
            temperature=float(rng.choice([0.0, 0.7, 1.0])),
            top_k=int(rng.choice([0, 0, 20, 300])),
            top_p=float(rng.choice([1.0, 0.8, 0.95])),
            min_p=float(rng.choice([0.0, 0.0, 0.05])),
            repetition_penalty=float(rng.choice([1.0, 1.0, 1.2])),
            frequency_penalty=float(rng.choice([0.0, 0.3])),
        )
        hist = rng.integers(0, V, int(rng.integers(0, 3000))).tolist()
        form = call % 3
        h = [hist, torch.tensor(hist, dtype=torch.int32, device=DEV), torch.tensor(hist, dtype=torch.int64)][form]
        seed, pos = int(rng.integers(0, 1 << 40)), int(rng.integers(0, 1 << 20))
        print(f"per-token sweep call {call} V={V} {dtype} offset={off} history={len(hist)} form={form}", flush=True)
        tok = s.sample(big.to(DEV)[off : off + V], sp, seed, pos, history=h if sp.penalized else None)
        hi = np.asarray(hist if sp.penalized else [], dtype=np.int32)
        res = oracle_batch(x.float().numpy()[None], [sp.temperature], [sp.top_k], [sp.top_p], [sp.min_p],
                           [sp.repetition_penalty], [sp.presence_penalty], [sp.frequency_penalty],
                           hi, np.array([0, len(hi)], np.int32), [uniform(seed, pos)])[0]
        if not classify_ties(res):
            assert tok == res.token, (call, tok, res.token)
