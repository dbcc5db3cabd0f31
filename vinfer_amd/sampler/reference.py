"""The ``reference`` sampler backend: slow, readable torch code on any device.

It restates, row by row in torch, the batched semantics the ``hip`` backend implements:
penalties, fp32 division by the temperature, top-k, fp64 softmax, min-p, top-p with ties broken
by ascending id, and the inverse-CDF draw from the caller's uniform over the kept tokens in that
same order (descending probability, ties by ascending id). ``sample`` is the engine's per-token
call (src/vinfer/runtime/sampler.py:68) through that same draw, with the uniform of
``(seed, position)``; it does not reproduce the engine's exponential race (sampler.py:73-77),
whose tokens depend on the torch version and device. In the engine, the ``reference`` name
stays bound to the engine's own ``sample``.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

from vinfer_amd.registry import BackendContext
from vinfer_amd.sampler.base import SAMPLER, require_history
from vinfer_amd.sampling import SamplingParams, pack_params, penalized, uniform


def _penalize(x: torch.Tensor, hist: torch.Tensor, rep, pres, freq):
    V = x.shape[0]
    hist = hist.long()
    hist = hist[(hist >= 0) & (hist < V)]
    counts = torch.bincount(hist, minlength=V)
    sel = counts > 0
    xs = x[sel]
    xs = torch.where(xs > 0, xs / rep, xs * rep)
    xs = xs - freq * counts[sel].float()
    xs = xs - pres
    x = x.clone()
    x[sel] = xs
    return x, counts.int()


def _row(x: torch.Tensor, T, k: int, tp, mp):
    """Final fp64 probabilities of one penalised fp32 row (``T`` etc. are 0-dim fp32)."""
    pt = _ptilde(x, T, k, tp, mp)
    return pt / pt.sum()


def _ptilde(x: torch.Tensor, T, k: int, tp, mp):
    """``exp(z - max z)`` (fp64) over the tokens every filter keeps, 0 elsewhere; a one-hot
    1.0 for greedy and degenerate rows."""
    V = x.shape[0]
    if not bool(T > 0):
        out = torch.zeros(V, dtype=torch.float64, device=x.device)
        out[int(torch.argmax(x))] = 1.0
        return out
    z = x / T
    nan = torch.isnan(z)
    m = z.max() if not bool(nan.any()) else None
    point = None
    if m is None:
        point = int(torch.argmax(nan.int()))
    elif bool(m == float("inf")):
        point = int(torch.argmax((z == float("inf")).int()))
    elif bool(m == float("-inf")):
        point = 0
    if point is not None:
        out = torch.zeros(V, dtype=torch.float64, device=x.device)
        out[point] = 1.0
        return out
    keep = torch.ones(V, dtype=torch.bool, device=x.device)
    if 0 < k < V:
        kth = torch.topk(z, k).values[-1]
        keep &= z >= kth
    pt = torch.where(keep, torch.exp(z.double() - m.double()), torch.zeros((), dtype=torch.float64))
    if float(mp) > 0:
        keep &= pt >= float(mp)
    pt = torch.where(keep, pt, torch.zeros_like(pt))
    if float(tp) < 1:
        ids = torch.arange(V, device=x.device)
        # descending p~, ascending id: sort by id first, then a stable sort by -p~
        order = torch.sort(-pt[ids], stable=True).indices
        sp = pt[order]
        before = torch.cumsum(sp, 0) - sp
        drop = order[(before >= float(tp) * pt.sum()) & (sp > 0)]
        pt[drop] = 0.0
    return pt


@SAMPLER.register("reference")
class ReferenceSampler:
    def __init__(self, ctx: BackendContext) -> None:
        self.ctx = ctx

    def _rows(self, logits, params, hist_ids, hist_offsets):
        B, V = logits.shape
        for b in range(B):
            x = logits[b].float()
            if hist_ids is not None:
                if hist_offsets.dim() == 2:  # per-row [start, end) ranges
                    h = hist_ids[int(hist_offsets[b, 0]) : int(hist_offsets[b, 1])]
                else:
                    h = hist_ids[int(hist_offsets[b]) : int(hist_offsets[b + 1])]
            else:
                h = torch.zeros(0, dtype=torch.int32, device=logits.device)
            row = {k: getattr(params, k)[b] for k in params.__dataclass_fields__}
            x, counts = _penalize(
                x, h, row["repetition_penalty"], row["presence_penalty"], row["frequency_penalty"]
            )
            yield x, counts, row

    def penalized_logits(self, logits, params, hist_ids=None, hist_offsets=None):
        xs, cs = zip(*[(x, c) for x, c, _ in self._rows(logits, params, hist_ids, hist_offsets)])
        return torch.stack(xs), torch.stack(cs)

    def probs(self, logits, params, hist_ids=None, hist_offsets=None):
        out = [
            _row(x, r["temperature"], int(r["top_k"]), r["top_p"], r["min_p"])
            for x, _, r in self._rows(logits, params, hist_ids, hist_offsets)
        ]
        return torch.stack(out).float()

    def sample_batch(self, logits, params, uniforms, hist_ids=None, hist_offsets=None, draft_ids=None):
        ids, dps = [], []
        for b, (x, _, r) in enumerate(self._rows(logits, params, hist_ids, hist_offsets)):
            p = _row(x, r["temperature"], int(r["top_k"]), r["top_p"], r["min_p"])
            # kept tokens by descending probability, ties by ascending id
            kept = torch.sort(-p, stable=True).indices[: int((p > 0).sum())]
            c = torch.cumsum(p[kept], 0)
            j = int(torch.searchsorted(c, uniforms[b].double() * c[-1], right=True))
            ids.append(int(kept[min(j, kept.numel() - 1)]))
            if draft_ids is not None:
                d = int(draft_ids[b])
                dps.append(float(p[d]) if 0 <= d < p.numel() else 0.0)
        dev = logits.device
        out = torch.tensor(ids, dtype=torch.int32, device=dev)
        dp = torch.tensor(dps, dtype=torch.float32, device=dev) if draft_ids is not None else None
        return out, dp

    def logprobs(self, logits, tokens=None, n_top=0):
        """Log-softmax of the raw fp32 logits in fp64; top ``n_top`` by descending logit, ties by
        ascending id."""
        if not 0 <= n_top <= 32:
            raise ValueError(f"n_top must be in [0, 32], got {n_top}")
        B, V = logits.shape
        x = logits.double()
        m = x.max(dim=1, keepdim=True).values
        finite = torch.isfinite(m)
        lp = x - m - torch.log(torch.exp(x - m).sum(dim=1, keepdim=True))
        lp = torch.where(finite, lp, torch.full_like(lp, float("nan")))
        out_tok = None
        if tokens is not None:
            t = tokens.long()
            ok = (t >= 0) & (t < V)
            out_tok = torch.where(ok, lp.gather(1, t.clamp(0, V - 1).view(-1, 1)).view(-1),
                                  torch.full((B,), float("nan"), dtype=torch.float64, device=x.device)).float()
        k = min(n_top, V)
        # descending value, ascending id: a stable sort of the negated values (NaN first, as largest)
        key = torch.where(torch.isnan(x), torch.full_like(x, -float("inf")), -x)
        order = torch.sort(key, dim=1, stable=True).indices[:, :k]
        ids = torch.full((B, n_top), -1, dtype=torch.int32, device=x.device)
        lps = torch.full((B, n_top), -float("inf"), dtype=torch.float32, device=x.device)
        ids[:, :k] = order.int()
        lps[:, :k] = lp.gather(1, order).float()
        return out_tok, ids, lps

    def verify(self, target_logits, draft_logits, draft_tokens, params, u_accept, u_residual, u_bonus,
               draft_params=None, draft_states=None):
        """Speculative sampling (see the protocol) in exact integers: token masses
        ``rint(p~ * 2^42)`` and their sums S; accept when ``m * Q_d * S_t < P_d * S_d * 2^24``
        (``m = floor(u * 2^24)``); the residual ``max(0, (P_i * S_d >> s) - (Q_i * S_t >> s))`` with
        ``s = floor(log2(max(S_t, S_d)))`` over ascending ids. ``draft_states`` (the hip backend's
        saved draft states) are not needed here: the draft rows are always recomputed."""
        B, K1, V = target_logits.shape
        K = K1 - 1
        dparams = params if draft_params is None else draft_params
        dev = target_logits.device
        tokens = torch.full((B, K1), -1, dtype=torch.int32)
        counts = torch.zeros(B, dtype=torch.int32)

        def masses(x, prm, b):
            r = {k: getattr(prm, k)[b] for k in prm.__dataclass_fields__}
            pt = _ptilde(x.float(), r["temperature"], int(r["top_k"]), r["top_p"], r["min_p"])
            P = torch.round(pt.cpu() * 2.0**42).long().tolist()
            return P, sum(P)

        def m24(u):
            return int(torch.tensor(float(u), dtype=torch.float32) * 2.0**24)

        def own_draw(b, j, u):
            row = {k: getattr(params, k)[b : b + 1] for k in params.__dataclass_fields__}
            ids, _ = self.sample_batch(target_logits[b, j : j + 1], type(params)(**row),
                                       torch.full((1,), float(u), dtype=torch.float32, device=dev))
            return int(ids[0])

        for b in range(B):
            out = []
            for j in range(K):
                P, St = masses(target_logits[b, j], params, b)
                Q, Sd = masses(draft_logits[b, j], dparams, b)
                d = int(draft_tokens[b, j])
                if 0 <= d < V and m24(u_accept[b, j]) * Q[d] * St < (P[d] * Sd) << 24:
                    out.append(d)
                    continue
                sh = max(St, Sd).bit_length() - 1
                w = [max(0, ((p * Sd) >> sh) - ((q * St) >> sh)) for p, q in zip(P, Q)]
                R = sum(w)
                if R == 0:  # the target's own draw at this position (the sequence's bonus uniform)
                    out.append(own_draw(b, j, u_bonus[b]))
                else:
                    tg = min((m24(u_residual[b, j]) * R) >> 24, R - 1)
                    c = 0
                    for i, wi in enumerate(w):
                        c += wi
                        if c > tg:
                            out.append(i)
                            break
                break
            else:
                out.append(own_draw(b, K, u_bonus[b]))
            tokens[b, : len(out)] = torch.tensor(out, dtype=torch.int32)
            counts[b] = len(out)
        return tokens.to(dev), counts.to(dev)

    def sample(
        self,
        logits: torch.Tensor,
        params: SamplingParams,
        seed: int,
        position: int,
        history: Sequence[int] | torch.Tensor | None = None,
    ) -> int:
        require_history(params, history)
        dev = logits.device
        hist = off = None
        if penalized(params) and len(history) > 0:
            hist = torch.as_tensor(history, dtype=torch.int32).to(dev)
            off = torch.tensor([0, hist.numel()], dtype=torch.int32, device=dev)
        u = torch.tensor([uniform(seed, position)], dtype=torch.float32, device=dev)
        ids, _ = self.sample_batch(logits.reshape(1, -1), pack_params([params], dev), u, hist, off)
        return int(ids[0])


__all__ = ["ReferenceSampler"]
