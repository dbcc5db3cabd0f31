"""The engine's fp32 kept-set rule in torch on the CPU, and the rows it leaves undefined.
TEST INFRASTRUCTURE ONLY: imported by ``tests/`` and by the CPU leg of ``bench.py`` (to count
tie rows), never by product code.

The engine decides the kept set in fp32 (src/vinfer/runtime/sampler.py:52-64): ``z = x / T``;
the top-k threshold (the k-th largest ``z``, ties kept); ``p = softmax(z)``; the probabilities
sorted in descending order by an unstable sort; ``before = cumsum(p) - p``; tokens with
``before >= top_p`` dropped. ``fp32_rule`` redoes those steps with torch's CPU fp32 kernels (the
build's extensions in the oracle's order: penalties already applied to ``x``, min-p after the
softmax, top-p then relative to the kept mass). Where several tokens share one fp32
probability the engine's order among them is whatever its sort returns; this restatement sorts
them by ascending id, and flags every row on which that choice, or fp32 rounding, could change
the result.

A row is a tie under the engine's rule when:

1. ``straddle``: tokens with equal fp32 ``p`` fall on both sides of the top-p cutoff, so which
   of them are kept depends on the sort's order (sampler.py:60);
2. ``top_p_band``: the mass before the last kept or first dropped token is within
   ``(n + 4) 2^-24 + |sum(p) - 1|`` of the threshold (``n`` tokens summed by the fp32
   ``cumsum``, sampler.py:61-62, plus the softmax's own normalisation error);
3. ``min_p``: a token's ``p`` is within 4 ulp of ``min_p * max p``;
4. ``draw`` / ``merged_draw``: the inverse-CDF target ``u * S`` is within ``(n + 4) 2^-24 S``
   of a prefix boundary, or the drawn token's fp32 probability is shared by tokens of distinct
   logits (the fixed-point order of the oracle and the kernels separates them).

Rows whose top-k threshold, softmax or draw is degenerate (NaN or infinite ``z``) and greedy
rows are not classified: the engine's softmax turns the former into NaN, and greedy is exact.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

EPS32 = 2.0**-24


@dataclass
class Fp32Row:
    kind: str  # "sampled" | "greedy" | "degenerate"
    kept: np.ndarray | None  # bool [V], equal probabilities ordered by ascending id
    kept_sort: np.ndarray | None  # bool [V], equal probabilities in torch.sort's own order
    token: int  # the inverse-CDF draw over the kept set (descending p, ascending id)
    ties: list[str] = field(default_factory=list)


def fp32_rule(x: np.ndarray, temperature: float, top_k: int, top_p: float, min_p: float, u: float) -> Fp32Row:
    """The kept set and draw of one penalised fp32 row ``x`` under the engine's fp32 arithmetic,
    with the reasons (possibly none) why the engine's rule does not fix them."""
    xt = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    V = xt.numel()
    T = float(np.float32(temperature))
    if not T > 0:
        return Fp32Row("greedy", None, None, int(torch.argmax(xt)))
    z = xt / T  # a Python float divisor: torch's CPU kernel divides by fp32(T)
    if bool(torch.isnan(z).any()) or not bool(torch.isfinite(z.max())):
        return Fp32Row("degenerate", None, None, -1)
    keep = torch.ones(V, dtype=torch.bool)
    if 0 < top_k < V:
        kth = torch.kthvalue(z, V - top_k + 1).values  # the top_k-th largest
        keep = z >= kth
    p = torch.softmax(torch.where(keep, z, torch.tensor(-float("inf"))), dim=0)
    ties: list[str] = []
    # the softmax's normalisation error, in units of the total mass
    norm_err = abs(float(p.double().sum()) - 1.0)
    mp = float(np.float32(min_p))
    if mp > 0:
        pmax = p.max()
        cut = (pmax * torch.tensor(mp, dtype=torch.float32)).item()  # fp32 product
        near = (p - cut).abs() <= 4 * float(np.spacing(np.float32(cut)))
        near &= keep & (p != pmax)
        if bool(near.any()):
            ties.append("min_p")
        keep &= p >= cut
    n0 = int(keep.sum())
    tp = float(np.float32(top_p))
    kept_sort = None
    if tp < 1:
        pk = torch.where(keep, p, torch.zeros(()))
        # descending p, ascending id among equals (stable sort of -p)
        order = torch.sort(-pk, stable=True).indices[:n0]
        sp = pk[order]
        before = torch.cumsum(sp, 0) - sp
        thr32 = torch.tensor(tp, dtype=torch.float32) * (sp.sum() if mp > 0 else torch.tensor(1.0))
        nk = int((before < thr32).sum())
        nk = max(nk, 1)  # the most likely token is always kept
        if 0 < nk < n0 and float(sp[nk - 1]) == float(sp[nk]):
            ties.append("straddle")
        # the same sums in fp64 over the same order, against the threshold in fp64
        spd = sp.double()
        before64 = torch.cumsum(spd, 0) - spd
        thr64 = tp * (float(spd.sum()) if mp > 0 else 1.0)
        eps = (n0 + 4) * EPS32 + norm_err
        for b in (nk - 1, nk):
            if 0 <= b < n0 and abs(float(before64[b]) - thr64) <= eps:
                ties.append("top_p_band")
                break
        # the same rule over torch.sort's own order of equal probabilities (descending, not
        # stable): the kept set the engine's call would produce on this build of torch
        order_u = torch.sort(pk, descending=True).indices[:n0]
        sp_u = pk[order_u]
        nk_u = max(int((torch.cumsum(sp_u, 0) - sp_u < thr32).sum()), 1)
        keep_u = keep.clone()
        keep_u[order_u[nk_u:]] = False
        kept_sort = keep_u.numpy().copy()
        keep[order[nk:]] = False
    kept = keep.numpy().copy()
    if kept_sort is None:
        kept_sort = kept
    # the draw: inverse CDF over the kept set, descending p, ascending id, in fp32
    pk = torch.where(keep, p, torch.zeros(()))
    n = int(keep.sum())
    order = torch.sort(-pk, stable=True).indices[:n]
    C = torch.cumsum(pk[order], 0)
    S = float(C[-1])
    target = float(np.float32(u)) * S
    j = int(torch.searchsorted(C, torch.tensor([target], dtype=torch.float32), right=True)[0])
    j = min(j, n - 1)
    eps = (n + 4) * EPS32 * S
    if abs(float(C[j]) - target) <= eps or (j > 0 and abs(float(C[j - 1]) - target) <= eps):
        ties.append("draw")
    tok = int(order[j])
    grp = keep & (p == p[tok])
    if int(grp.sum()) > 1 and torch.unique(z[grp]).numel() > 1:
        ties.append("merged_draw")
    return Fp32Row("sampled", kept, kept_sort, tok, ties)


def torch_cpu_sample(row: torch.Tensor, hist: torch.Tensor, temperature: float, top_k: int, top_p: float,
                     min_p: float, rep: float, pres: float, freq: float, u: float) -> int:
    """One row through the engine's fp32 rule with torch's CPU kernels, the way the engine's
    sampler would run on a CPU (sampler.py:50-77, with the extensions: penalties from the
    history, min-p, and the inverse-CDF draw on ``u`` over the kept tokens in descending
    probability). The CPU baseline's unit of work; no tie classification."""
    x = row.float()
    V = x.numel()
    if hist.numel() and (rep != 1.0 or pres != 0.0 or freq != 0.0):
        h = hist[(hist >= 0) & (hist < V)].long()
        counts = torch.bincount(h, minlength=V)
        sel = counts > 0
        xs = x[sel]
        xs = torch.where(xs > 0, xs / rep, xs * rep)
        xs = xs - freq * counts[sel].float()
        x = x.clone()
        x[sel] = xs - pres
    if not temperature > 0:
        return int(torch.argmax(x))
    z = x / temperature
    if 0 < top_k < V:
        kth = torch.topk(z, top_k).values[-1]
        z = torch.where(z >= kth, z, torch.tensor(-float("inf")))
    p = torch.softmax(z, dim=0)
    if min_p > 0:
        p = torch.where(p >= p.max() * min_p, p, torch.zeros(()))
    sp, order = torch.sort(p, descending=True)
    C = torch.cumsum(sp, 0)
    if top_p < 1:
        before = C - sp
        n = max(int((before < top_p * C[-1]).sum()), 1)
        sp, order, C = sp[:n], order[:n], C[:n]
    j = int(torch.searchsorted(C, torch.tensor([u * float(C[-1])]), right=True)[0])
    return int(order[min(j, order.numel() - 1)])
