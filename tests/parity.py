"""Helpers that run the oracle on a workload and compare device results with it."""

from __future__ import annotations

import numpy as np
import torch

from oracle.sampler_oracle import classify_ties, sample_batch


def oracle(w, want_probs: bool = False):
    p = w.params
    f = lambda t: t.detach().cpu().numpy()  # noqa: E731
    hi = f(w.hist_ids) if w.hist_ids is not None else np.zeros(0, np.int32)
    ho = f(w.hist_offsets) if w.hist_offsets is not None else np.zeros(w.batch + 1, np.int32)
    return sample_batch(
        w.logits.detach().float().cpu().numpy(),
        f(p.temperature),
        f(p.top_k),
        f(p.top_p),
        f(p.min_p),
        f(p.repetition_penalty),
        f(p.presence_penalty),
        f(p.frequency_penalty),
        hi,
        ho,
        f(w.uniforms),
        None if w.draft_ids is None else f(w.draft_ids),
        want_probs=want_probs,
    )


def compare_ids(ids: torch.Tensor, res, dprob: torch.Tensor | None = None, rtol: float = 1e-5):
    """Non-tie rows must match exactly; returns (n_ties, mismatching row list)."""
    ids = ids.cpu().tolist()
    dp = None if dprob is None else dprob.cpu().tolist()
    ties, bad = 0, []
    for b, r in enumerate(res):
        if classify_ties(r):
            ties += 1
            continue
        if ids[b] != r.token:
            bad.append((b, ids[b], r.token, r.kind))
        elif dp is not None:
            want = r.draft_prob
            if abs(dp[b] - want) > rtol * abs(want) + 1e-30:
                bad.append((b, "draft_prob", dp[b], want))
    return ties, bad
