"""The oracle against the engine's own fp32 arithmetic.

The oracle decides in fp64 with ties by ascending id; the engine decides in fp32 with an
unstable sort (src/vinfer/runtime/sampler.py:52-64). ``oracle/fp32_rule.py`` redoes the engine's
fp32 steps with torch's CPU kernels and flags the rows on which the engine's rule itself is
ambiguous (equal probabilities straddling the top-p cutoff, a cutoff inside the fp32 summation
band, min-p within 4 ulp, a draw on a prefix boundary). Here, on rows of every benchmark workload shape:
wherever the engine's rule is not ambiguous, its kept set equals the oracle's, for both the
ascending-id order and torch.sort's own order of equal probabilities, and the fp32 draw picks
the oracle's token. The tie counts per shape are the ones the parity reports quote.

The temperature division is checked exhaustively: torch's ``x.float() / T`` over all 65,536
bf16 values equals numpy's IEEE ``x / float32(T)``, bit for bit, at every configured T.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.fp32_rule import fp32_rule
from oracle.sampler_oracle import classify_ties, penalize, sample_row
from vinfer_amd.workloads import make

KEPT_TIES = ("straddle", "top_p_band", "min_p")
CONFIG_TEMPERATURES = (0.3, 0.5, 0.7, 0.8, 1.0, 1.2, 1.5)
# bf16 values (of 65,536) whose z = fl32(x * fl32(1 / T)) differs from the division's
# fl32(x / T): what a reciprocal multiply would change (numpy, exhaustive).
RECIPROCAL_DIFFERS = {0.3: 9118, 0.5: 0, 0.7: 6598, 0.8: 0, 1.0: 0, 1.2: 9160, 1.5: 21338}


def all_bf16() -> np.ndarray:
    return torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float().numpy()


@pytest.mark.parametrize("T", CONFIG_TEMPERATURES)
def test_torch_division_is_ieee_division_for_every_bf16_value(T):
    x = all_bf16()
    got = (torch.from_numpy(x) / T).numpy()
    with np.errstate(all="ignore"):
        want = x / np.float32(T)
        recip = (x * (np.float32(1.0) / np.float32(T))).astype(np.float32)
    same = lambda a, b: (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))  # noqa: E731
    assert same(got, want).all()
    # A reciprocal multiply is a different function at most temperatures: the kernels and the
    # oracle divide, as torch's CPU kernel does.
    assert int((~same(recip, want)).sum()) == RECIPROCAL_DIFFERS[T]


def rows_of(name: str, batch: int):
    w = make(name, batch=batch)
    p = w.params
    for b in range(batch):
        x = w.logits[b].float().numpy()
        if w.hist_ids is not None:
            h = w.hist_ids[int(w.hist_offsets[b]) : int(w.hist_offsets[b + 1])].numpy()
            x, _ = penalize(x, h, float(p.repetition_penalty[b]), float(p.presence_penalty[b]),
                            float(p.frequency_penalty[b]))
        yield b, x, (float(p.temperature[b]), int(p.top_k[b]), float(p.top_p[b]), float(p.min_p[b]),
                     float(w.uniforms[b]))


def compare(name: str, batch: int, rule=fp32_rule):
    """Counts over the rows: fp32 tie rows, rows whose kept set differs from the oracle's under
    either order, and the differences no tie explains."""
    n = dict(rows=0, fp32_ties=0, oracle_ties=0, kept_differs=0, sort_differs=0, unexplained=[])
    for b, x, args in rows_of(name, batch):
        r = sample_row(x, *args, want_probs=True)
        f = rule(x, *args)
        n["rows"] += 1
        n["oracle_ties"] += bool(classify_ties(r))
        if f.kind != "sampled":
            assert r.kind == f.kind or f.kind == "degenerate"
            if f.kind == "greedy":
                assert f.token == r.token
            continue
        n["fp32_ties"] += bool(f.ties)
        kept_tie = any(t in f.ties for t in KEPT_TIES)
        for key, kept in (("kept_differs", f.kept), ("sort_differs", f.kept_sort)):
            if not (kept == r.kept).all():
                n[key] += 1
                if not kept_tie:
                    n["unexplained"].append((b, key))
        if f.token != r.token and not f.ties and not classify_ties(r):
            n["unexplained"].append((b, "token", f.token, r.token))
    return n


# (shape, rows, the fp32 tie rows expected among them)
SHAPES = [
    ("mixed_bf16", 64, (10, 40)),
    ("peaked_flat", 64, (32, 32)),  # every flat (odd) row, no peaked row
    ("large_fp32", 32, (0, 0)),
    ("verify_bf16", 32, (32, 32)),
]


@pytest.mark.parametrize("name,batch,expect", SHAPES, ids=[s[0] for s in SHAPES])
def test_kept_set_equals_the_engine_fp32_rule_off_its_ties(name, batch, expect):
    n = compare(name, batch)
    print(name, {k: v for k, v in n.items() if k != "unexplained"})
    assert n["unexplained"] == []
    lo, hi = expect
    assert lo <= n["fp32_ties"] <= hi
    assert n["kept_differs"] <= n["fp32_ties"] and n["sort_differs"] <= n["fp32_ties"]


def test_flat_rows_are_ties_and_peaked_rows_are_not():
    for b, x, args in rows_of("peaked_flat", 8):
        f = fp32_rule(x, *args)
        assert bool(f.ties) == (b % 2 == 1), (b, f.ties)
        if b % 2 == 1:
            assert "straddle" in f.ties  # the cutoff falls inside a run of equal probabilities


def test_a_planted_mistake_is_not_hidden_by_the_tie_classes():
    # A restatement that forgets the temperature disagrees with the oracle on rows its own
    # classifier calls clean: the comparison can fail.
    def no_temperature(x, T, k, tp, mp, u):
        return fp32_rule(x, 1.0 if T > 0 else T, k, tp, mp, u)

    n = compare("mixed_bf16", 24, rule=no_temperature)
    assert len(n["unexplained"]) > 0


@pytest.mark.parametrize("name,batch", [("mixed_bf16", 16), ("large_fp32", 8), ("peaked_flat", 8)])
def test_the_cpu_baseline_sampler_draws_the_oracle_s_tokens(name, batch):
    # bench.py's CPU baseline (torch_cpu_sample) computes the same thing as the oracle wherever
    # neither classifier flags the row
    from oracle.fp32_rule import torch_cpu_sample

    w = make(name, batch=batch)
    p = w.params
    checked = 0
    for b, x, args in rows_of(name, batch):
        h = w.hist_ids[int(w.hist_offsets[b]) : int(w.hist_offsets[b + 1])]
        tok = torch_cpu_sample(w.logits[b], h, args[0], args[1], args[2], args[3], float(p.repetition_penalty[b]),
                               float(p.presence_penalty[b]), float(p.frequency_penalty[b]), args[4])
        r = sample_row(x, *args)
        if fp32_rule(x, *args).ties or classify_ties(r):
            continue
        assert tok == r.token, (name, b)
        checked += 1
    assert checked >= batch // 2
