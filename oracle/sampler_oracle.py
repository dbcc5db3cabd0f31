"""CPU oracle for the token-sampling path. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` may import
this module, and only as the checker: no product code path calls it.

What it restates, row by row, in numpy (fp32 where the engine computes in fp32, fp64 for masses):

1. ``x = fp32(logits)`` (src/vinfer/runtime/sampler.py:52; exact for bf16).
2. Penalties (not in the engine; field names and off-values from server/protocol.py:133-135),
   in vLLM's order, each step rounded to fp32, for every id with history count ``c > 0``:
   ``x = x / rep if x > 0 else x * rep``; ``x = x - freq * c``; ``x = x - pres``. History ids
   outside ``[0, V)`` are ignored.
3. Greedy (``T == 0``; for raw inputs also ``T < 0`` or NaN): first index of the max, NaN counting as the max (sampler.py:70-71; numpy's
   ``argmax`` has the same rule as ``torch.argmax``).
4. ``z = x / fp32(T)``, IEEE fp32 division (sampler.py:52).
   Degenerate rows (not specified by the engine, whose softmax turns them into NaN): a NaN in
   ``z`` -> the first NaN index; max ``z == +inf`` -> the first ``+inf`` index; every ``z`` is
   ``-inf`` -> index 0 (what the engine's argmax over an all-NaN vector returns).
5. Top-k if ``0 < k < V``: keep ``z >= kth largest z`` (threshold semantics, sampler.py:53-55).
6. ``p~ = exp(z - max z)`` in fp64 over kept tokens (sampler.py:56, in fp64 instead of fp32).
7. Min-p if ``> 0`` (extension, protocol.py:142): drop ``p~ < min_p`` (``p~`` is ``p / max p``).
8. Top-p if ``< 1``: in descending ``p~`` order, ties by ascending id (the engine's sort is
   unstable there, sampler.py:60), drop a token when the mass strictly before it is
   ``>= top_p * S`` with ``S`` the kept mass (sampler.py:57-62, renormalised after min-p).
9. Draw (replaces the exponential race of sampler.py:73-77): over kept tokens in the order
   top-p sorts them (descending ``p~``, ties by ascending id), the first ``j`` with inclusive
   prefix ``C_j > u * S``; the last kept token with positive mass if rounding leaves none.
   Draft probability ``p~_d / S`` (0 if ``d`` was dropped).

10. Speculative-decoding verify (not in the engine, which skips its checkpoint's MTP head,
   src/vinfer/models/loader.py:27): ``verify_row`` restates speculative sampling (Leviathan,
   Kalman, Matias 2023; Chen et al. 2023) over rows of steps 1-9; its own docstring states the
   fixed-point residual and the tie rules.

11. Log-probabilities (``logprobs_row``, not in the engine, whose API layer rejects the
   ``logprobs`` / ``top_logprobs`` fields, server/protocol.py:131-132): the log-softmax of the
   raw logits in fp64 and the top n by descending logit, ties by ascending id.

``classify_ties`` flags rows whose result two correct implementations may legitimately disagree
on; the device kernels' masses are fixed-point with quantum ``2**-42`` (``p~ <= 1``), so a
decision is fragile when it sits within ``(n + 4) * 2**-42`` of its threshold.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

F32 = np.float32
MASS_QUANTUM = 2.0**-42  # fixed-point quantum of the device kernels' masses


def penalize(x: np.ndarray, hist: np.ndarray, rep: float, pres: float, freq: float):
    """Apply the three penalties to fp32 row ``x`` given its history ids; returns
    ``(x_penalised, counts)`` with ``counts`` int64[V]."""
    x = np.asarray(x, dtype=F32).copy()
    V = x.shape[0]
    hist = np.asarray(hist, dtype=np.int64)
    hist = hist[(hist >= 0) & (hist < V)]
    counts = np.bincount(hist, minlength=V).astype(np.int64)
    sel = counts > 0
    xs = x[sel]
    rep32, pres32, freq32 = F32(rep), F32(pres), F32(freq)
    xs = np.where(xs > 0, xs / rep32, xs * rep32).astype(F32)
    xs = (xs - (freq32 * counts[sel].astype(F32)).astype(F32)).astype(F32)
    xs = (xs - pres32).astype(F32)
    x[sel] = xs
    return x, counts


@dataclass
class RowResult:
    """One row's outcome plus the facts ``classify_ties`` needs."""

    token: int
    draft_prob: float
    kind: str  # "greedy" | "degenerate" | "sampled"
    probs: np.ndarray | None = None  # fp64 [V] final probabilities (when requested)
    kept: np.ndarray | None = None  # bool [V] final kept set
    info: dict = field(default_factory=dict)


def _one_hot(V: int, i: int) -> np.ndarray:
    p = np.zeros(V, dtype=np.float64)
    p[i] = 1.0
    return p


def sample_row(
    x: np.ndarray,
    temperature: float,
    top_k: int,
    top_p: float,
    min_p: float,
    u: float,
    draft: int | None = None,
    want_probs: bool = False,
) -> RowResult:
    """Steps 3-9 for one penalised fp32 row ``x``."""
    x = np.asarray(x, dtype=F32)
    V = x.shape[0]
    T = F32(temperature)
    if not T > 0:  # 0 (and, for raw inputs, negative or NaN) selects greedy
        tok = int(np.argmax(x))
        return _point(V, tok, draft, "greedy", want_probs)
    z = (x / T).astype(F32)
    nan = np.isnan(z)
    if nan.any():
        return _point(V, int(np.argmax(nan)), draft, "degenerate", want_probs)
    m = z.max()
    if m == np.inf:
        return _point(V, int(np.argmax(z == np.inf)), draft, "degenerate", want_probs)
    if m == -np.inf:
        return _point(V, 0, draft, "degenerate", want_probs)

    keep = np.ones(V, dtype=bool)
    if 0 < top_k < V:
        kth = np.partition(z, V - top_k)[V - top_k]
        keep &= z >= kth
    pt = np.zeros(V, dtype=np.float64)
    pt[keep] = np.exp(z[keep].astype(np.float64) - np.float64(m))
    mp = float(F32(min_p))
    pt_topk = pt[keep]
    if mp > 0:
        keep &= pt >= mp
    pt[~keep] = 0.0
    kept0 = np.flatnonzero(keep)
    S0 = math.fsum(pt[kept0])
    info: dict = {"n_kept0": int(kept0.size), "S0": S0, "min_p": mp, "pt_topk": pt_topk}

    tp = float(F32(top_p))
    if tp < 1:
        P = tp * S0
        order = kept0[np.argsort(-pt[kept0], kind="stable")]  # p~ desc, id asc
        sp = pt[order]
        before = np.cumsum(sp) - sp
        nk = int(np.count_nonzero(before < P))  # a prefix: before is non-decreasing
        dropped = order[nk:]
        keep[dropped] = False
        pt[dropped] = 0.0
        info.update(P=P, before=before, order=order, n_top_p=nk, xs=x[order], sp=sp)
    kept = np.flatnonzero(keep)
    korder = kept[np.argsort(-pt[kept], kind="stable")]  # p~ desc, id asc
    S = math.fsum(pt[kept])
    C = np.cumsum(pt[korder])
    target = float(F32(u)) * S
    j = int(np.searchsorted(C, target, side="right"))  # first C_j > target
    if j >= korder.size:  # rounding left none: the last kept token with positive mass
        j = int(np.flatnonzero(pt[korder] > 0)[-1])
    tok = int(korder[j])
    info.update(S=S, C=C, target=target, j=j, n_kept=int(kept.size), korder=korder, x=x, pt=pt)
    dp = float(pt[draft] / S) if draft is not None and 0 <= draft < V else 0.0
    res = RowResult(tok, dp, "sampled", info=info)
    if want_probs:
        res.probs = pt / S
        res.kept = keep
    return res


def _point(V, tok, draft, kind, want_probs) -> RowResult:
    dp = 1.0 if draft is not None and draft == tok else 0.0
    res = RowResult(tok, dp, kind)
    if want_probs:
        res.probs = _one_hot(V, tok)
        res.kept = res.probs > 0
    return res


def classify_ties(res: RowResult) -> list[str]:
    """Reasons (possibly none) why ``res`` is a tie row: a decision within the device's
    arithmetic error of its threshold, so its token may legitimately differ."""
    if res.kind != "sampled":
        return []
    info = res.info
    reasons = []
    # Min-p: the device's fp64 exp may differ from numpy's by an ulp or two. The max token has
    # p~ = exp(0) = 1 exactly everywhere, so it is never fragile.
    mp = info["min_p"]
    if mp > 0:
        ptk = info["pt_topk"]
        ptk = ptk[ptk != 1.0]
        if ptk.size and np.any(np.abs(ptk - mp) <= 8 * np.spacing(mp)):
            reasons.append("min_p")
    if "P" in info:
        before, P, order, nk = info["before"], info["P"], info["order"], info["n_top_p"]
        eps = (info["n_kept0"] + 4) * MASS_QUANTUM + 1e-15 * info["S0"]
        near = [b for b in (nk - 1, nk) if 0 <= b < before.size]
        if any(abs(before[b] - P) <= eps for b in near):
            reasons.append("top_p_mass")
        # The device orders tokens by penalised logit, the oracle by p~. Both group equal
        # values the same way unless distinct z share one fp64 p~ inside the group that the
        # cutoff splits; then which members are kept depends on that choice.
        sp = info["sp"]
        if 0 < nk < sp.size and sp[nk - 1] == sp[nk]:
            grp = sp == sp[nk]
            if np.unique(info["xs"][grp]).size > 1:
                reasons.append("merged_group")
    C, target, j = info["C"], info["target"], info["j"]
    eps = (info["n_kept"] + 4) * MASS_QUANTUM + 1e-15 * info["S"]
    if abs(C[j] - target) <= eps or (j > 0 and abs(C[j - 1] - target) <= eps):
        reasons.append("draw")
    # The drawn token's position inside its p~ group depends on the grouping (see above).
    korder, pt, x = info["korder"], info["pt"], info["x"]
    grp = korder[pt[korder] == pt[korder[j]]]
    if grp.size > 1 and np.unique(x[grp]).size > 1:
        reasons.append("merged_draw")
    return reasons


def sample_batch(
    logits: np.ndarray,
    temperature,
    top_k,
    top_p,
    min_p,
    rep,
    pres,
    freq,
    hist_ids: np.ndarray,
    hist_offsets: np.ndarray,
    u,
    draft=None,
    want_probs: bool = False,
) -> list[RowResult]:
    """Rows of a ``[B, V]`` batch (fp32 or bf16-valued fp32) with CSR histories."""
    logits = np.asarray(logits, dtype=F32)
    out = []
    for b in range(logits.shape[0]):
        h = hist_ids[hist_offsets[b] : hist_offsets[b + 1]]
        x, _ = penalize(logits[b], h, rep[b], pres[b], freq[b])
        d = None if draft is None else int(draft[b])
        out.append(
            sample_row(x, temperature[b], int(top_k[b]), top_p[b], min_p[b], u[b], d, want_probs)
        )
    return out


# ---- speculative-decoding verify ----------------------------------------------------------------
POINT_MASS = 2**42  # mass of a point-mass row's token (and its kept mass)


@dataclass
class VerifyResult:
    tokens: list[int]  # the emitted tokens: accepted drafts, then the residual or bonus token
    ties: list[str] = field(default_factory=list)


def token_masses(res: RowResult, V: int) -> tuple[list[int], int, int]:
    """Fixed-point masses of a row's tokens, ``rint(p~ * 2^42)`` (0 for dropped tokens), their
    sum S and the number of kept tokens; a point-mass row has 2^42 at its token."""
    if res.kind != "sampled":
        P = [0] * V
        P[res.token] = POINT_MASS
        return P, POINT_MASS, 1
    P = np.rint(res.info["pt"] * 2.0**42).astype(np.int64).tolist()
    return P, int(sum(P)), int(res.info["n_kept"])


def verify_row(target: list[RowResult], draft: list[RowResult], drafts, u_acc, u_res, V: int) -> VerifyResult:
    """Speculative sampling for one sequence (Leviathan, Kalman, Matias 2023; Chen et al. 2023),
    in the device kernels' fixed point, exact integer arithmetic.

    ``target`` holds K + 1 rows (each drawn with the sequence's bonus uniform), ``draft`` K rows. With P,
    Q the token masses (``token_masses``) and S_t, S_d their sums, draft j is accepted when
    ``m * Q_d * S_t < P_d * S_d * 2^24`` (m = floor(u_acc[j] * 2^24)), i.e. ``u < p / q``. At
    the first rejection the token is the first id (ascending) whose inclusive prefix of
    ``w_i = max(0, (P_i * S_d >> s) - (Q_i * S_t >> s))`` (s = floor(log2(max(S_t, S_d)))) exceeds
    ``floor(m * R / 2^24)``, m from u_res[j] and R the sum; R = 0 takes the target's own draw
    there. With every draft accepted, the target's draw at K is added.

    Ties: a row whose own result is fragile, or a decision within what the masses can move
    between two exp implementations (each mass by one unit, so each S by its kept count)."""
    K = len(drafts)
    res = VerifyResult([])
    for j in range(K):
        if classify_ties(target[j]) or classify_ties(draft[j]):
            res.ties.append(f"row {j}")
        d = int(drafts[j])
        P, St, nt = token_masses(target[j], V)
        Q, Sd, nd = token_masses(draft[j], V)
        if not 0 <= d < V:
            accept = False
        else:
            m = int(F32(u_acc[j]) * F32(2.0**24))
            lhs, rhs = m * Q[d] * St, (P[d] * Sd) << 24
            eps = m * (St + Q[d] * nt) + ((Sd + P[d] * nd) << 24)
            if lhs != rhs and abs(lhs - rhs) <= eps:
                res.ties.append("accept")
            accept = lhs < rhs
        if accept:
            res.tokens.append(d)
            continue
        s = max(St, Sd).bit_length() - 1
        w = [max(0, ((p * Sd) >> s) - ((q * St) >> s)) for p, q in zip(P, Q)]
        R = sum(w)
        if R == 0:
            res.tokens.append(target[j].token)
            return res
        m = int(F32(u_res[j]) * F32(2.0**24))
        tg = min((m * R) >> 24, R - 1)
        C = np.cumsum(np.array(w, dtype=np.int64))
        tok = int(np.searchsorted(C, tg, side="right"))
        err = ((V * (Sd + St) + St * nd + Sd * nt) >> s) + V
        lo = int(C[tok - 1]) if tok > 0 else 0
        if tg - lo <= 2 * err or int(C[tok]) - 1 - tg <= 2 * err:
            res.ties.append("residual")
        res.tokens.append(tok)
        return res
    if classify_ties(target[K]):
        res.ties.append("bonus")
    res.tokens.append(target[K].token)
    return res


# ---- log-probabilities of the raw logits -----------------------------------------------------
def logprobs_row(x: np.ndarray, token: int | None, n_top: int) -> tuple[float | None, list[int], np.ndarray]:
    """The log-softmax of one raw fp32 row in fp64 (``x - M - log(sum exp(x - M))``, M the max;
    NaN throughout when M is not finite): the logprob of ``token`` (NaN outside the row) and the
    row's ``n_top`` largest logits, descending, ties by ascending id (NaN counts as largest);
    entries past the row are id -1, logprob -inf."""
    x = np.asarray(x, dtype=F32).astype(np.float64)
    V = x.size
    m = np.max(x) if not np.isnan(x).any() else np.nan
    if np.isfinite(m):
        lp = x - m - math.log(math.fsum(np.exp(x - m)))
    else:
        lp = np.full(V, np.nan)
    tok = None if token is None else (float(lp[token]) if 0 <= token < V else float("nan"))
    key = np.where(np.isnan(x), -np.inf, -x)
    order = np.lexsort((np.arange(V), key))[: min(n_top, V)]
    ids = order.tolist() + [-1] * (n_top - order.size)
    vals = np.concatenate([lp[order], np.full(n_top - order.size, -np.inf)])
    return tok, ids, vals
