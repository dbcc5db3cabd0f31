"""Speculative-decoding verify: ``verify_row`` in the oracle, the reference backend and the hip
kernels (``vsamp_verify``).

The oracle is pinned by the property that defines speculative sampling: for any target p and
draft q, a draft drawn from q and put through the accept / residual rule yields a first token
distributed exactly as p (Leviathan et al. 2023, Theorem 1). The test evaluates the rule over a
fine grid of both uniforms, so a reversed acceptance ratio or a residual of max(0, q - p)
fails it. Known answers: p == q accepts every draft; a draft q puts on a token p excludes is
always rejected, and the replacement is then p's own inverse-CDF draw over ascending ids.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.sampler_oracle import sample_row, token_masses, verify_row
from vinfer_amd.registry import BackendContext
from vinfer_amd.sampler import SAMPLER
from vinfer_amd.sampling import SamplingParams, pack_params

LOGITS = np.array([2.0, 1.0, 0.5, 0.0, -1.0, -3.0], np.float32)


def rows(x, T=1.0, k=0, tp=1.0, mp=0.0, draft=None, u=0.5):
    return sample_row(np.asarray(x, np.float32), T, k, tp, mp, u, draft, want_probs=True)


def first_token_distribution(xt, xq, grid=400, **kw):
    """P(first emitted token = i) under the rule, for K = 1: the draft d ~ q, the uniforms on a
    midpoint grid. A draft is emitted only when accepted (a rejection means p(d) < q(d), where
    the residual is 0), so the acceptance rate is the rate of d coming out."""
    V = len(xt)
    q = rows(xq, **kw).probs
    us = (np.arange(grid) + 0.5) / grid
    out = np.zeros(V)
    for d in range(V):
        if q[d] == 0:
            continue
        t = [rows(xt, draft=d, **kw), rows(xt, **kw)]
        dr = [rows(xq, draft=d, **kw)]
        acc = np.mean([verify_row(t, dr, [d], [u], [0.5], V).tokens[0] == d for u in us])
        out[d] += q[d] * acc
        if acc < 1:  # the residual's tokens over the u_res grid, from a rejected draft
            toks = [verify_row(t, dr, [d], [0.999999], [u], V).tokens[0] for u in us]
            out += q[d] * (1 - acc) * np.bincount(toks, minlength=V) / grid
    return out


@pytest.mark.parametrize(
    "xt,xq,kw",
    [
        (LOGITS, LOGITS[::-1].copy(), {}),
        (LOGITS, LOGITS * 0.3, {"T": 0.8}),
        (LOGITS, np.zeros(6, np.float32), {"k": 4}),
        (LOGITS * 2, LOGITS + np.array([0, 0, 3, 0, 0, 0], np.float32), {"tp": 0.9}),
    ],
)
def test_first_emitted_token_is_distributed_as_the_target(xt, xq, kw):
    got = first_token_distribution(xt, xq, **kw)
    p = rows(xt, **kw).probs
    np.testing.assert_allclose(got, p, atol=3.0 / 400)


def test_equal_distributions_accept_every_draft():
    for d in range(6):
        t = [rows(LOGITS, draft=d), rows(LOGITS, draft=d)]
        for u in (0.0, 0.5, 0.999999):
            r = verify_row(t, [rows(LOGITS, draft=d)], [d], [u], [0.3], 6)
            assert r.tokens == [d, t[1].token]


def test_a_draft_the_target_excludes_is_replaced_by_the_target_s_draw():
    # target top-k 2 keeps ids 0 and 1; the draft proposes id 4; q is one-hot there (greedy)
    xq = np.array([0, 0, 0, 0, 9, 0], np.float32)
    for ur in (0.0, 0.3, 0.7, 0.999):
        t = [rows(LOGITS, k=2, draft=4), rows(LOGITS, k=2)]
        r = verify_row(t, [rows(xq, T=0.0, draft=4)], [4], [0.0], [ur], 6)
        # q is a point mass at 4 (mass 2^42 of 2^42), so w_i = P_i * 2^42 >> s with s = 42 +
        # floor(log2(S_t)) - 42: the target's masses, scaled by a power of two
        P, St, _ = token_masses(t[0], 6)
        sh = max(St, 2**42).bit_length() - 1
        w = [max(0, ((p << 42) >> sh) - ((2**42 * St if i == 4 else 0) >> sh)) for i, p in enumerate(P)]
        m = int(np.float32(ur) * np.float32(2**24))
        want = int(np.searchsorted(np.cumsum(w), min((m * sum(w)) >> 24, sum(w) - 1), side="right"))
        assert r.tokens == [want] and want in (0, 1)


def test_reference_backend_matches_the_oracle():
    rng = np.random.default_rng(3)
    B, K, V = 6, 2, 50
    xt = rng.normal(0, 2, (B, K + 1, V)).astype(np.float32)
    xq = (xt[:, :K] + rng.normal(0, 0.7, (B, K, V))).astype(np.float32)
    sp = [SamplingParams(temperature=[0.0, 0.7, 1.0, 1.3, 1.0, 0.9][b], top_k=[0, 0, 10, 0, 5, 0][b],
                         top_p=[1.0, 0.9, 1.0, 0.8, 1.0, 0.95][b], min_p=[0, 0, 0, 0, 0.1, 0][b]) for b in range(B)]
    params = pack_params(sp)
    drafts = rng.integers(0, V, (B, K)).astype(np.int32)
    ua, ur, ub = rng.random((B, K), np.float32), rng.random((B, K), np.float32), rng.random(B, dtype=np.float32)
    ref = SAMPLER.resolve("reference", BackendContext(torch.device("cpu"), torch.float32))
    tokens, counts = ref.verify(torch.from_numpy(xt), torch.from_numpy(xq), torch.from_numpy(drafts), params,
                                torch.from_numpy(ua), torch.from_numpy(ur), torch.from_numpy(ub))
    for b in range(B):
        r = params.row(b)
        t = [sample_row(xt[b, j], r["temperature"], r["top_k"], r["top_p"], r["min_p"], float(ub[b]),
                        int(drafts[b, j]) if j < K else None, want_probs=True) for j in range(K + 1)]
        d = [sample_row(xq[b, j], r["temperature"], r["top_k"], r["top_p"], r["min_p"], 0.0, int(drafts[b, j]),
                        want_probs=True) for j in range(K)]
        want = verify_row(t, d, drafts[b], ua[b], ur[b], V)
        if want.ties:
            continue
        assert int(counts[b]) == len(want.tokens)
        assert tokens[b, : len(want.tokens)].tolist() == want.tokens
        assert (tokens[b, len(want.tokens) :] == -1).all()


def verify_case(seed, B, K, V, dtype, sigma=2.0, noise=0.5):
    """Target and draft logits (the draft a noisy copy for 3 rows in 4, independent for the rest),
    drafts drawn from the draft distribution (a random id for every 5th row), mixed parameters."""
    rng = np.random.default_rng(seed)
    xt = rng.normal(0, sigma, (B, K + 1, V)).astype(np.float32)
    xq = (xt[:, :K] + rng.normal(0, noise, (B, K, V))).astype(np.float32)
    for b in range(3, B, 4):
        xq[b] = rng.normal(0, sigma, (K, V))
    xt = torch.from_numpy(xt).to(dtype).float().numpy()  # values the dtype can hold
    xq = torch.from_numpy(xq).to(dtype).float().numpy()
    kinds = [dict(temperature=0.0), dict(temperature=0.8, top_k=20), dict(temperature=1.0, top_p=0.9),
             dict(temperature=1.2, min_p=0.05, top_p=0.95), dict(temperature=1.0), dict(temperature=0.6, top_k=200)]
    params = pack_params([SamplingParams(**kinds[b % len(kinds)]) for b in range(B)])
    drafts = np.zeros((B, K), np.int32)
    for b in range(B):
        r = params.row(b)
        for j in range(K):
            if b % 5 == 4:
                drafts[b, j] = rng.integers(0, V)
            else:
                drafts[b, j] = sample_row(xq[b, j], r["temperature"], r["top_k"], r["top_p"], r["min_p"],
                                          float(rng.random(dtype=np.float32))).token
    ua, ur, ub = rng.random((B, K), np.float32), rng.random((B, K), np.float32), rng.random(B, dtype=np.float32)
    return xt, xq, drafts, params, ua, ur, ub


def oracle_verify(xt, xq, drafts, params, ua, ur, ub):
    B, K1, V = xt.shape
    K = K1 - 1
    out = []
    for b in range(B):
        r = params.row(b)
        t = [sample_row(xt[b, j], r["temperature"], r["top_k"], r["top_p"], r["min_p"], float(ub[b]),
                        int(drafts[b, j]) if j < K else None, want_probs=True) for j in range(K + 1)]
        d = [sample_row(xq[b, j], r["temperature"], r["top_k"], r["top_p"], r["min_p"], 0.0, int(drafts[b, j]),
                        want_probs=True) for j in range(K)]
        out.append(verify_row(t, d, drafts[b], ua[b], ur[b], V))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("K,V,B", [(1, 1000, 48), (3, 1000, 48), (1, 151936, 12), (2, 151936, 8), (2, 4099, 24)])
def test_gpu_verify_matches_the_oracle(dtype, K, V, B):
    dev = torch.device("cuda", 0)
    xt, xq, drafts, params, ua, ur, ub = verify_case(100 + K + V % 97, B, K, V, dtype)
    print(f"verify B={B} K={K} V={V} {dtype}", flush=True)
    hip = SAMPLER.resolve("hip", BackendContext(dev, dtype))
    to = lambda a, t=None: torch.from_numpy(np.ascontiguousarray(a)).to(dev) if t is None else torch.from_numpy(a).to(t).to(dev)  # noqa: E731
    tokens, counts = hip.verify(to(xt, dtype), to(xq, dtype), to(drafts), params.to(dev), to(ua), to(ur), to(ub))
    tokens, counts = tokens.cpu(), counts.cpu()
    want = oracle_verify(xt, xq, drafts, params, ua, ur, ub)
    ties = 0
    rejected = 0
    for b, w in enumerate(want):
        if w.ties:
            ties += 1
            continue
        rejected += len(w.tokens) <= K and w.tokens[-1] != int(drafts[b, len(w.tokens) - 1])
        assert int(counts[b]) == len(w.tokens), (b, counts[b], w.tokens)
        assert tokens[b, : len(w.tokens)].tolist() == w.tokens, (b, tokens[b].tolist(), w.tokens)
        assert (tokens[b, len(w.tokens) :] == -1).all()
    assert ties <= max(2, B // 8), ties
    assert rejected > 0  # the residual path ran


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_gpu_verify_on_tied_rows_with_split_cutoff_groups(dtype):
    # few distinct values (N(0, 0.1^2) rounded to bf16): top-k and top-p cut inside a group of
    # equal values, so each row's kept set ends at an id inside that group
    dev = torch.device("cuda", 0)
    B, K, V = 24, 2, 20000
    xt, xq, drafts, params, ua, ur, ub = verify_case(77, B, K, V, dtype, sigma=0.1, noise=0.05)
    xt = torch.from_numpy(xt).to(torch.bfloat16).float().numpy()
    xq = torch.from_numpy(xq).to(torch.bfloat16).float().numpy()
    kinds = [dict(temperature=1.0, top_k=1000), dict(temperature=0.7, top_p=0.5), dict(temperature=1.0, top_k=7)]
    params = pack_params([SamplingParams(**kinds[b % 3]) for b in range(B)])
    print(f"verify tied rows B={B} K={K} V={V} {dtype}", flush=True)
    hip = SAMPLER.resolve("hip", BackendContext(dev, dtype))
    to = lambda a, t=None: torch.from_numpy(np.ascontiguousarray(a)).to(dev) if t is None else torch.from_numpy(a).to(t).to(dev)  # noqa: E731
    tokens, counts = hip.verify(to(xt, dtype), to(xq, dtype), to(drafts), params.to(dev), to(ua), to(ur), to(ub))
    want = oracle_verify(xt, xq, drafts, params, ua, ur, ub)
    tokens, counts = tokens.cpu(), counts.cpu()
    bad = [b for b, w in enumerate(want) if not w.ties and
           (int(counts[b]) != len(w.tokens) or tokens[b, : len(w.tokens)].tolist() != w.tokens)]
    assert not bad, [(b, tokens[b].tolist(), want[b].tokens) for b in bad]
    assert sum(bool(w.ties) for w in want) <= B // 4


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_gpu_saved_draft_states_give_the_same_verify(dtype):
    # the drafts drawn with sample_states, then verify with those states: the same tokens as a
    # verify that samples the draft rows itself
    dev = torch.device("cuda", 0)
    B, K, V = 24, 3, 151936
    xt, xq, _, params, ua, ur, ub = verify_case(55, B, K, V, dtype)
    hip = SAMPLER.resolve("hip", BackendContext(dev, dtype))
    to = lambda a, t=None: torch.from_numpy(np.ascontiguousarray(a)).to(dev) if t is None else torch.from_numpy(a).to(t).to(dev)  # noqa: E731
    tq = to(xq, dtype)
    p = params.to(dev)
    u = torch.rand(B, K, device=dev)
    drafts, states = [], []
    for j in range(K):
        ids, st = hip.sample_states(tq[:, j].contiguous(), p, u[:, j].contiguous())
        ids2, _ = hip.sample_batch(tq[:, j].contiguous(), p, u[:, j].contiguous())
        assert torch.equal(ids, ids2)
        drafts.append(ids)
        states.append(st)
    drafts = torch.stack(drafts, dim=1)
    print(f"saved draft states B={B} K={K} V={V} {dtype}", flush=True)
    a = hip.verify(to(xt, dtype), tq, drafts, p, to(ua), to(ur), to(ub))
    b = hip.verify(to(xt, dtype), tq, drafts, p, to(ua), to(ur), to(ub), draft_states=torch.stack(states, dim=1))
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_gpu_verify_with_a_point_row_on_one_side(dtype):
    # a +inf logit makes a row a point mass at that id: even rows put it in the draft row (at the
    # drafted id) against a sampled target row, odd rows in the target row against a sampled draft
    dev = torch.device("cuda", 0)
    B, K, V = 16, 1, 151936
    xt, xq, drafts, _, ua, ur, ub = verify_case(91, B, K, V, dtype)
    kinds = [dict(temperature=1.0, top_p=0.9), dict(temperature=0.8, top_k=50), dict(temperature=1.2, min_p=0.05)]
    params = pack_params([SamplingParams(**kinds[b % 3]) for b in range(B)])
    rng = np.random.default_rng(5)
    for b in range(B):
        i = int(rng.integers(0, V))
        if b % 2 == 0:
            xq[b, 0, i] = np.inf
            drafts[b, 0] = i
        else:
            xt[b, 0, i] = np.inf
    print(f"verify point rows B={B} K={K} V={V} {dtype}", flush=True)
    hip = SAMPLER.resolve("hip", BackendContext(dev, dtype))
    to = lambda a, t=None: torch.from_numpy(np.ascontiguousarray(a)).to(dev) if t is None else torch.from_numpy(a).to(t).to(dev)  # noqa: E731
    tokens, counts = hip.verify(to(xt, dtype), to(xq, dtype), to(drafts), params.to(dev), to(ua), to(ur), to(ub))
    want = oracle_verify(xt, xq, drafts, params, ua, ur, ub)
    tokens, counts = tokens.cpu(), counts.cpu()
    rejected = 0
    for b, w in enumerate(want):
        assert not w.ties
        rejected += len(w.tokens) == 1 and w.tokens[0] != int(drafts[b, 0])
        assert int(counts[b]) == len(w.tokens), (b, counts[b], w.tokens)
        assert tokens[b, : len(w.tokens)].tolist() == w.tokens, (b, tokens[b].tolist(), w.tokens)
    assert rejected >= B // 2  # both kinds reach the residual draw


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_gpu_verify_residual_over_signed_zeros(dtype):
    # The target keeps only its max, 0, held by 32 tokens of +0.0 and 32 of -0.0 (min-p 1): one
    # value. Each draft proposes a token the target drops, so the residual is drawn over the 64
    # zeros, uniformly: -0.0 tokens must carry the same weight as +0.0 ones.
    dev = torch.device("cuda", 0)
    B, K, V = 48, 1, 4096
    rng = np.random.default_rng(31)
    xt = -rng.uniform(1.0, 5.0, (B, K + 1, V)).astype(np.float32)
    xq = rng.normal(0, 1, (B, K, V)).astype(np.float32)
    drafts = np.zeros((B, K), np.int32)
    neg = []
    for b in range(B):
        z = rng.choice(V, 65, replace=False)
        xt[b, :, z[:32]] = 0.0
        xt[b, :, z[32:64]] = -0.0
        neg.append(set(z[32:64].tolist()))
        drafts[b, 0] = z[64]  # a token the target drops
        xq[b, 0, z[64]] = 30.0  # the draft keeps only it
    xt = torch.from_numpy(xt).to(dtype).float().numpy()
    xq = torch.from_numpy(xq).to(dtype).float().numpy()
    params = pack_params([SamplingParams(temperature=1.0, min_p=1.0) for _ in range(B)])
    ua, ur, ub = rng.random((B, K), np.float32), rng.random((B, K), np.float32), rng.random(B, dtype=np.float32)
    print(f"verify signed zeros B={B} V={V} {dtype}", flush=True)
    hip = SAMPLER.resolve("hip", BackendContext(dev, dtype))
    to = lambda a, t=None: torch.from_numpy(np.ascontiguousarray(a)).to(dev) if t is None else torch.from_numpy(a).to(t).to(dev)  # noqa: E731
    tokens, counts = hip.verify(to(xt, dtype), to(xq, dtype), to(drafts), params.to(dev), to(ua), to(ur), to(ub))
    tokens, counts = tokens.cpu(), counts.cpu()
    want = oracle_verify(xt, xq, drafts, params, ua, ur, ub)
    on_neg = 0
    for b, w in enumerate(want):
        assert not w.ties
        assert int(counts[b]) == 1 and tokens[b, 0].item() == w.tokens[0], (b, tokens[b].tolist(), w.tokens)
        on_neg += w.tokens[0] in neg[b]
    assert 10 <= on_neg <= 38  # about half the draws land on a -0.0 token
