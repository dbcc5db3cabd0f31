"""Log-probabilities of the raw logits (``logprobs`` / ``top_logprobs``): the oracle's
``logprobs_row``, the reference backend and the hip kernel (``vsamp_logprobs``).

The oracle is pinned by the closed form on the engine's test fixture (test_sampler.py:10: its
softmax at T = 1 in fp64, so its logs), by scipy's ``log_softmax`` on random rows, by brute-force
ordering of the top n (descending value, ties by ascending id) on rows with many ties, and by
the non-finite cases. Device results: top ids exact, logprobs within 2e-6 + 1e-6 |lp| (fp32
output of an fp64 log of a sum of fp32 exponentials)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.sampler_oracle import logprobs_row
from vinfer_amd.registry import BackendContext
from vinfer_amd.sampler import SAMPLER

LOGITS = np.array([2.0, 1.0, 0.5, 0.0, -1.0, -3.0], np.float32)
SOFTMAX_T1 = [0.560893, 0.206341, 0.125152, 0.075909, 0.027925, 0.003779]  # softmax(LOGITS), closed form


def test_closed_form_on_the_fixture():
    tok, ids, vals = logprobs_row(LOGITS, 2, 3)
    assert ids == [0, 1, 2]
    np.testing.assert_allclose(np.exp(vals), SOFTMAX_T1[:3], atol=1e-6)
    assert abs(math.exp(tok) - SOFTMAX_T1[2]) < 1e-6


def test_matches_scipy_log_softmax():
    from scipy.special import log_softmax

    rng = np.random.default_rng(0)
    for V in (7, 1000, 50000):
        x = (rng.normal(0, 3, V)).astype(np.float32)
        want = log_softmax(x.astype(np.float64))
        tok, ids, vals = logprobs_row(x, V // 2, 20)
        k = min(20, V)
        np.testing.assert_allclose(vals[:k], want[ids[:k]], rtol=1e-12, atol=1e-12)
        assert abs(tok - want[V // 2]) < 1e-12
        assert ids[:k] == np.argsort(-x, kind="stable")[:k].tolist() and ids[k:] == [-1] * (20 - k)


def test_ties_go_by_ascending_id_and_short_rows_pad():
    x = np.array([1, 3, 3, 2, 3, 1, 2], np.float32)
    _, ids, vals = logprobs_row(x, None, 5)
    assert ids == [1, 2, 4, 3, 6]
    _, ids, vals = logprobs_row(x, None, 9)
    assert ids[7:] == [-1, -1] and np.all(np.isneginf(vals[7:]))
    _, ids, _ = logprobs_row(np.array([0.0, -0.0, 0.0], np.float32), None, 3)
    assert ids == [0, 1, 2]  # -0.0 and 0.0 are one value


def test_non_finite_rows_are_nan():
    for x in ([1.0, np.inf, 0.0], [np.nan, 1.0], [-np.inf, -np.inf]):
        tok, ids, vals = logprobs_row(np.array(x, np.float32), 0, 2)
        assert math.isnan(tok) and np.all(np.isnan(vals[: min(2, len(x))]))


def test_reference_backend_matches_the_oracle():
    rng = np.random.default_rng(1)
    x = rng.normal(0, 2, (5, 300)).astype(np.float32)
    x[1, :] = np.round(x[1, :])  # ties
    x[2, 7] = np.nan
    ref = SAMPLER.resolve("reference", BackendContext(torch.device("cpu"), torch.float32))
    toks = torch.tensor([0, 5, 299, -1, 300], dtype=torch.int32)
    tl, ids, lps = ref.logprobs(torch.from_numpy(x), toks, 8)
    for b in range(5):
        t = int(toks[b])
        wt, wids, wv = logprobs_row(x[b], t, 8)
        assert ids[b].tolist() == wids
        np.testing.assert_allclose(lps[b].numpy(), wv.astype(np.float32), rtol=1e-6, atol=1e-6)
        assert (math.isnan(wt) and math.isnan(float(tl[b]))) or abs(float(tl[b]) - wt) < 1e-5


def lp_case(seed, B, V, dtype):
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, V, generator=g) * 2.5
    x[1] = torch.randn(V, generator=g) * 0.01  # few distinct bf16 values: massive ties
    x[2] = 0.0  # one value everywhere
    if V > 8:
        x[3, 5] = float("nan")
        x[4, : V // 2] = float("-inf")
    x = x.to(dtype)
    tokens = torch.from_numpy(rng.integers(-2, V + 2, B).astype(np.int32))
    return x, tokens


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("V,n_top", [(6, 20), (1000, 5), (151936, 20), (262144, 32), (4099, 0), (20000, 1)])
def test_gpu_logprobs_match_the_oracle(dtype, V, n_top):
    dev = torch.device("cuda", 0)
    B = 12
    x, tokens = lp_case(V + n_top, B, V, dtype)
    print(f"logprobs B={B} V={V} n_top={n_top} {dtype}", flush=True)
    hip = SAMPLER.resolve("hip", BackendContext(dev, dtype))
    tl, ids, lps = hip.logprobs(x.to(dev), tokens.to(dev), n_top)
    tl, ids, lps = tl.cpu().numpy(), ids.cpu().numpy(), lps.cpu().numpy()
    xs = x.float().numpy()
    for b in range(B):
        wt, wids, wv = logprobs_row(xs[b], int(tokens[b]), n_top)
        assert ids[b].tolist() == wids, (b, ids[b].tolist(), wids)
        fin = np.isfinite(wv)
        np.testing.assert_allclose(lps[b][fin], wv[fin], rtol=1e-6, atol=2e-6)
        assert np.array_equal(np.isnan(lps[b]), np.isnan(wv)) and np.array_equal(np.isneginf(lps[b]), np.isneginf(wv))
        if math.isnan(wt):
            assert math.isnan(tl[b])
        else:
            assert abs(tl[b] - wt) <= 2e-6 + 1e-6 * abs(wt), (b, tl[b], wt)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_gpu_logprobs_on_unaligned_strided_rows(dtype):
    # rows that start one element past a 16-byte boundary, with a row stride above V
    dev = torch.device("cuda", 0)
    B, V = 6, 5000
    x, tokens = lp_case(9, B, V + 3, dtype)
    view = x.to(dev)[:, 1 : V + 1]
    print(f"logprobs unaligned rows B={B} V={V} {dtype}", flush=True)
    hip = SAMPLER.resolve("hip", BackendContext(dev, dtype))
    tl, ids, lps = hip.logprobs(view, tokens.clamp(-1, V).to(dev), 7)
    xs = x[:, 1 : V + 1].float().numpy()
    for b in range(B):
        wt, wids, wv = logprobs_row(xs[b], int(tokens.clamp(-1, V)[b]), 7)
        assert ids[b].tolist() == wids
        fin = np.isfinite(wv)
        np.testing.assert_allclose(lps[b].cpu().numpy()[fin], wv[fin], rtol=1e-6, atol=2e-6)
