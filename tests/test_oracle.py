"""Pins the CPU oracle: golden values, the engine tests' known answers, library routines
(torch.topk / softmax / sort), closed forms and brute force. No check here retypes the oracle's
own formula."""

from __future__ import annotations

import json
from collections import Counter
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.sampler_oracle import MASS_QUANTUM, classify_ties, penalize, sample_row
from vinfer_amd.sampling import SamplingParams, position_seed, uniform

GOLD = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())
LOGITS = np.array(GOLD["LOGITS"], dtype=np.float32)


def probs(x, T=1.0, k=0, p=1.0, mp=0.0):
    return sample_row(np.asarray(x, np.float32), T, k, p, mp, 0.5, want_probs=True).probs


# ---- known answers (test_sampler.py, test_sampler_zero_noise.py, closed forms) ----------------
def test_greedy_is_argmax():
    g = GOLD["greedy"]
    assert sample_row(np.array(g["logits"], np.float32), 0.0, 0, 1.0, 0.0, 0.3).token == g["token"]


@pytest.mark.parametrize("key,T", [("softmax_T1", 1.0), ("softmax_T0.5", 0.5)])
def test_softmax_closed_form(key, T):
    np.testing.assert_allclose(probs(LOGITS, T), GOLD[key], rtol=1e-6)


def test_top_k_and_top_p_known_answers():
    np.testing.assert_allclose(probs(LOGITS, p=0.8), GOLD["top_p_0.8"]["probs"], rtol=1e-6, atol=0)
    np.testing.assert_allclose(probs(LOGITS, k=3), GOLD["top_k_3"]["probs"], rtol=1e-6, atol=0)
    assert int((probs(LOGITS, k=2) > 0).sum()) == GOLD["top_k_2"]["kept"]
    assert int((probs(LOGITS, p=0.8) > 0).sum()) == GOLD["top_p_0.8"]["kept"]
    assert int((probs(LOGITS, p=1e-6) > 0).sum()) == GOLD["top_p_1e-6"]["kept"]


def test_extreme_uniforms_never_pick_a_dropped_token():
    # The u-based analogue of the zero-noise regression (test_sampler_zero_noise.py:14-19).
    z = GOLD["zero_noise"]
    x = np.array(z["logits"], np.float32)
    for u in (0.0, 1.0 - 2.0**-24):
        assert sample_row(x, 1.0, 2, 1.0, 0.0, u).token in z["top_k_2_in"]
        assert sample_row(x, 1.0, 0, 0.5, 0.0, u).token == z["top_p_0.5"]


def test_position_seed_golden():
    for key, val in GOLD["position_seed"].items():
        s, p = map(int, key.split(":"))
        assert position_seed(s, p) == val


# ---- library routines: torch's topk / softmax / sort implementation of sampler.py:50-65 ------
def torch_filtered(x, T, k, p):
    # fp32 division as sampler.py:52, then fp64 so the comparison isolates the filtering rule
    z = torch.from_numpy((x / np.float32(T)).astype(np.float32)).double()
    if k and k < z.shape[0]:
        kth = torch.topk(z, k).values[-1]
        z = z.masked_fill(z < kth, float("-inf"))
    pr = torch.softmax(z, -1)
    if p < 1:
        sp, order = torch.sort(pr, descending=True, stable=True)
        before = sp.cumsum(-1) - sp
        sp = sp.masked_fill(before >= float(np.float32(p)), 0.0)
        pr = torch.zeros_like(pr).scatter(-1, order, sp)
        pr = pr / pr.sum()
    return pr.numpy()


@pytest.mark.parametrize("seed", range(8))
def test_matches_torch_library_rule(seed):
    rng = np.random.default_rng(seed)
    V = int(rng.integers(5, 3000))
    x = (rng.normal(0, 3, V)).astype(np.float32)
    T = float(rng.choice([0.3, 0.7, 1.0, 1.5]))
    k = int(rng.choice([0, 1, 5, 50, V - 1, V + 3]))
    p = float(rng.choice([1.0, 0.9, 0.5, 0.95]))
    res = sample_row(x, T, k, p, 0.0, 0.5, want_probs=True)
    if classify_ties(res):
        pytest.skip("tie row")
    np.testing.assert_allclose(res.probs, torch_filtered(x, T, k, p), rtol=1e-9, atol=1e-15)


def test_min_p_keeps_exactly_the_tokens_above_the_relative_floor():
    x = np.array([3.0, 2.0, 0.0, -1.0, 2.9], np.float32)
    pr = probs(x, mp=0.3)
    e = np.exp(x.astype(np.float64) - 3.0)  # p / max p
    assert ((pr > 0) == (e >= np.float32(0.3))).all()
    assert sample_row(x, 1.0, 0, 1.0, 1.0, 0.7).token == 0  # min_p = 1 keeps only the max


# ---- penalties: closed forms and an independent counter ---------------------------------------
def test_counts_are_exact_and_ids_outside_the_vocab_are_ignored():
    rng = np.random.default_rng(1)
    V = 300
    hist = rng.integers(-5, V + 5, 4000)
    x, counts = penalize(np.zeros(V, np.float32), hist, 1.0, 0.0, 1.0)
    ref = Counter(int(h) for h in hist if 0 <= h < V)
    assert all(counts[i] == ref.get(i, 0) for i in range(V))
    # zero logits, frequency 1: the penalised logit is exactly -count
    assert np.array_equal(x, -counts.astype(np.float32))


def test_penalty_signs_and_order():
    x = np.array([2.0, -2.0, 0.0, 4.0], np.float32)
    out, _ = penalize(x, [0, 1, 2, 0], 2.0, 0.5, 0.25)
    # id 0: 2/2 = 1, - 0.25*2, - 0.5 -> 0.0 ; id 1: -2*2 = -4, -0.25, -0.5 -> -4.75
    # id 2: 0*2 = 0, -0.25, -0.5 -> -0.75 ; id 3 not in history
    np.testing.assert_array_equal(out, np.array([0.0, -4.75, -0.75, 4.0], np.float32))


def test_penalties_off_are_the_identity():
    rng = np.random.default_rng(2)
    x = rng.normal(0, 3, 500).astype(np.float32)
    out, _ = penalize(x, rng.integers(0, 500, 100), 1.0, 0.0, 0.0)
    np.testing.assert_array_equal(out, x)


def test_penalty_steps_round_separately_in_fp32():
    # freq * c is rounded before the subtraction: with a fused multiply-add the result differs.
    x = np.array([1.0000001], np.float32)
    freq, c = np.float32(0.1), 3
    out, _ = penalize(x, [0] * c, 1.0, 0.0, float(freq))
    prod = np.float32(freq * np.float32(c))
    assert out[0] == np.float32(x[0] - prod)


# ---- the draw: inverse CDF in descending-probability order ------------------------------------------------
def test_uniform_sweep_reproduces_the_final_distribution_exactly():
    x = np.array([0.5, 2.0, -1.0, 1.5, 0.0, 1.9], np.float32)
    res = sample_row(x, 1.0, 4, 0.9, 0.0, 0.0, want_probs=True)
    n = 1 << 16
    us = (np.arange(n) + 0.5) / n
    freq = np.bincount([sample_row(x, 1.0, 4, 0.9, 0.0, u).token for u in us[::16]], minlength=6)
    np.testing.assert_allclose(freq / freq.sum(), res.probs, atol=2 * 16 / n)
    # descending-probability order: the smallest u lands on the most likely token, the largest
    # on the least likely kept one
    kept = np.flatnonzero(res.probs > 0)
    assert sample_row(x, 1.0, 4, 0.9, 0.0, 0.0).token == int(np.argmax(x))
    assert sample_row(x, 1.0, 4, 0.9, 0.0, 1 - 2.0**-24).token == kept[np.argmin(x[kept])]
    # equal probabilities: ascending id
    z = np.zeros(4, np.float32)
    assert [sample_row(z, 1.0, 0, 1.0, 0.0, u).token for u in (0.1, 0.3, 0.6, 0.9)] == [0, 1, 2, 3]


def test_draft_probability_is_the_draw_frequency_of_that_id():
    # the reported probability of a draft id is the share of uniforms whose draw lands on it
    x = np.array([0.5, 2.0, -1.0, 1.5, 0.0, 1.9, -0.2], np.float32)
    n = 1 << 14
    us = (np.arange(n) + 0.5) / n
    for T, k, p, mp in ((1.0, 0, 1.0, 0.0), (0.7, 5, 0.9, 0.0), (1.3, 0, 0.95, 0.2)):
        toks = np.array([sample_row(x, T, k, p, mp, u).token for u in us])
        for d in range(len(x)):
            dp = sample_row(x, T, k, p, mp, 0.5, draft=d).draft_prob
            assert abs(np.mean(toks == d) - dp) <= 1.0 / n, (T, k, p, mp, d)
    # greedy: probability 1 for the argmax, 0 otherwise
    assert [sample_row(x, 0.0, 0, 1.0, 0.0, 0.5, draft=d).draft_prob for d in range(7)] == [0, 1, 0, 0, 0, 0, 0]


@pytest.mark.parametrize(
    "params",
    [
        SamplingParams(temperature=1.0),
        SamplingParams(temperature=0.5),
        SamplingParams(temperature=1.0, top_k=3),
        SamplingParams(temperature=1.0, top_p=0.8),
    ],
)
def test_sampled_frequencies_match_the_filtered_distribution(params):
    # test_sampler.py:24-38 with this package's uniforms: 20,000 draws, TV < 0.015.
    counts = np.zeros(len(LOGITS))
    for pos in range(20000):
        counts[sample_row(LOGITS, params.temperature, params.top_k, params.top_p, 0.0, uniform(1, pos)).token] += 1
    expected = torch_filtered(LOGITS, params.temperature, params.top_k, params.top_p)
    assert 0.5 * np.abs(counts / 20000 - expected).sum() < 0.015


def test_greedy_nan_and_degenerate_rows():
    nan = np.float32("nan")
    assert sample_row(np.array([1.0, nan, 5.0, nan], np.float32), 0.0, 0, 1, 0, 0.5).token == 1
    assert sample_row(np.array([1.0, nan, 5.0], np.float32), 1.0, 0, 1, 0, 0.5).token == 1
    inf = np.float32("inf")
    assert sample_row(np.array([1.0, inf, 5.0, inf], np.float32), 1.0, 0, 1, 0, 0.5).token == 1
    assert sample_row(np.full(4, -inf, np.float32), 1.0, 0, 1, 0, 0.9).token == 0


def test_cutoff_ties_keep_the_lowest_ids():
    # Six equal logits, top_p 0.5: mass before the 4th is exactly 0.5 -> keep three, ids 0..2.
    res = sample_row(np.zeros(6, np.float32), 1.0, 0, 0.5, 0.0, 0.99, want_probs=True)
    assert res.kept.tolist() == [True, True, True, False, False, False]
    assert "top_p_mass" in classify_ties(res)  # exactly on the threshold: a tie by the rule
    res = sample_row(np.zeros(6, np.float32), 1.0, 0, 0.6, 0.0, 0.99, want_probs=True)
    assert res.kept.tolist() == [True, True, True, True, False, False] and not classify_ties(res)


def test_tie_classifier_flags_a_draw_on_a_boundary():
    x = np.zeros(4, np.float32)  # uniform over 4: boundaries at u = 0.25, 0.5, 0.75
    assert "draw" in classify_ties(sample_row(x, 1.0, 0, 1.0, 0.0, 0.5))
    assert not classify_ties(sample_row(x, 1.0, 0, 1.0, 0.0, 0.6))
    assert MASS_QUANTUM == 2.0**-42
