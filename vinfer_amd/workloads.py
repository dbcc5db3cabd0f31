"""Seeded synthetic sampler workloads: logits, per-row parameters, histories, uniforms.

Five shapes of sampler step (the last one an MTP-style verify step), each generated on the host
from a fixed seed so a GPU run and a CPU run see identical inputs:

- ``single_fp32``   1 x 151936 fp32 logits ~ N(0, 2^2) with 5 random ids boosted by +8;
                     T 0.7, top-k 20, top-p 0.8, no penalties.
- ``mixed_bf16``    64 x 151936 bf16 ~ N(0, 3^2); per row 25% greedy, else T ~ U[0.3, 1.5],
                     top-k from {0, 20, 50, 1000}, top-p ~ U[0.5, 1.0]; repetition 1.05,
                     presence 0.5, frequency 0.2; Zipf(1.1) history of length 2048.
- ``peaked_flat``   256 x 151936 bf16, even rows peaked (one id +15 over N(0, 1)), odd rows flat
                     (N(0, 0.1^2), i.e. variance 0.01); T 1, top-p 0.95, min-p 0.05, top-k 0;
                     penalties as above with a Zipf(1.1) history of length 4096.
- ``large_fp32``    1024 x 151936 fp32 ~ N(0, 2^2); history lengths ~ U[1, 32768] of Zipf(1.05)
                     ids; penalties as above, T 0.8, top-k 50, top-p 0.9.
- ``verify_bf16``   192 x 262144 bf16 ~ N(0, 2.5^2); T ~ U[0.5, 1.2], top-p 0.95; one draft id
                     per row (uniformly random) whose final probability is reported.

Zipf histories: ranks 1..V drawn by inverse CDF of the truncated Zipf(s) law, then mapped to
ids through a seeded random permutation. Uniforms: fp32 U[0, 1), one per row.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from vinfer_amd.sampling import PackedParams

NAMES = ("single_fp32", "mixed_bf16", "peaked_flat", "large_fp32", "verify_bf16")
SEEDS = {name: 1000 + i for i, name in enumerate(NAMES)}
PENALTIES = (1.05, 0.5, 0.2)  # repetition, presence, frequency


@dataclass
class Workload:
    name: str
    logits: torch.Tensor  # [B, V] bf16 or fp32, host
    params: PackedParams  # host
    uniforms: torch.Tensor  # fp32 [B]
    hist_ids: torch.Tensor | None  # int32 [sum L]
    hist_offsets: torch.Tensor | None  # int32 [B + 1]
    draft_ids: torch.Tensor | None  # int32 [B]

    @property
    def batch(self) -> int:
        return int(self.logits.shape[0])

    @property
    def vocab(self) -> int:
        return int(self.logits.shape[1])

    def to(self, device) -> Workload:
        mv = lambda t: None if t is None else t.to(device)  # noqa: E731
        return Workload(
            self.name,
            self.logits.to(device),
            self.params.to(device),
            self.uniforms.to(device),
            mv(self.hist_ids),
            mv(self.hist_offsets),
            mv(self.draft_ids),
        )

    def algorithmic_bytes(self) -> int:
        """One read of the logits, the int32 history, and 24 B of parameters and outputs per
        row: the bytes a single-pass sampler must move."""
        h = 0 if self.hist_ids is None else 4 * int(self.hist_ids.numel())
        return self.logits.numel() * self.logits.element_size() + h + 24 * self.batch


def zipf_ids(rng: np.random.Generator, n: int, V: int, s: float, perm: np.ndarray) -> np.ndarray:
    ranks = np.arange(1, V + 1, dtype=np.float64)
    cdf = np.cumsum(ranks**-s)
    cdf /= cdf[-1]
    r = np.searchsorted(cdf, rng.random(n), side="right")
    return perm[np.minimum(r, V - 1)].astype(np.int32)


def _params(B, T, k, p, mp, rep, pres, freq) -> PackedParams:
    f = lambda v: torch.as_tensor(np.broadcast_to(np.asarray(v, np.float32), (B,)).copy())  # noqa: E731
    return PackedParams(
        temperature=f(T),
        top_k=torch.as_tensor(np.broadcast_to(np.asarray(k, np.int32), (B,)).copy()),
        top_p=f(p),
        min_p=f(mp),
        repetition_penalty=f(rep),
        presence_penalty=f(pres),
        frequency_penalty=f(freq),
    )


def _csr(hists: list[np.ndarray]) -> tuple[torch.Tensor, torch.Tensor]:
    off = np.zeros(len(hists) + 1, np.int64)
    off[1:] = np.cumsum([len(h) for h in hists])
    ids = np.concatenate(hists).astype(np.int32) if hists else np.zeros(0, np.int32)
    return torch.from_numpy(ids), torch.from_numpy(off.astype(np.int32))


def make(name: str, batch: int | None = None, vocab: int | None = None, seed: int | None = None,
         regime: str | None = None) -> Workload:
    """The named workload; ``batch``/``vocab`` shrink it for tests (same generator).
    ``peaked_flat`` with ``regime`` "peaked" or "flat" makes every row of that regime instead
    of alternating them (the other inputs are generated the same way)."""
    rng = np.random.default_rng(SEEDS[name] if seed is None else seed)
    g = torch.Generator().manual_seed(SEEDS[name] if seed is None else seed)
    rep, pres, freq = PENALTIES
    if name == "single_fp32":
        B, V = batch or 1, vocab or 151936
        x = torch.randn(B, V, generator=g) * 2.0
        for b in range(B):
            x[b, torch.from_numpy(rng.choice(V, 5, replace=False))] += 8.0
        params = _params(B, 0.7, 20, 0.8, 0.0, 1.0, 0.0, 0.0)
        return Workload(name, x, params, torch.from_numpy(rng.random(B, dtype=np.float32)), None, None, None)
    if name == "mixed_bf16":
        B, V = batch or 64, vocab or 151936
        x = (torch.randn(B, V, generator=g) * 3.0).to(torch.bfloat16)
        greedy = rng.random(B) < 0.25
        T = np.where(greedy, 0.0, rng.uniform(0.3, 1.5, B))
        k = rng.choice(np.array([0, 20, 50, 1000]), B)
        p = rng.uniform(0.5, 1.0, B)
        params = _params(B, T, k, p, 0.0, rep, pres, freq)
        perm = rng.permutation(V)
        hi, ho = _csr([zipf_ids(rng, 2048, V, 1.1, perm) for _ in range(B)])
        return Workload(name, x, params, torch.from_numpy(rng.random(B, dtype=np.float32)), hi, ho, None)
    if name == "peaked_flat":
        B, V = batch or 256, vocab or 151936
        x = torch.randn(B, V, generator=g)
        flat = [b % 2 == 1 for b in range(B)] if regime is None else [regime == "flat"] * B
        if regime not in (None, "flat", "peaked"):
            raise ValueError(f"regime must be 'peaked' or 'flat', got {regime!r}")
        peak = rng.integers(0, V, B)
        for b in range(B):
            if flat[b]:
                x[b] *= 0.1
            else:
                x[b, int(peak[b])] += 15.0
        x = x.to(torch.bfloat16)
        params = _params(B, 1.0, 0, 0.95, 0.05, rep, pres, freq)
        perm = rng.permutation(V)
        hi, ho = _csr([zipf_ids(rng, 4096, V, 1.1, perm) for _ in range(B)])
        return Workload(name, x, params, torch.from_numpy(rng.random(B, dtype=np.float32)), hi, ho, None)
    if name == "large_fp32":
        B, V = batch or 1024, vocab or 151936
        x = torch.randn(B, V, generator=g) * 2.0
        params = _params(B, 0.8, 50, 0.9, 0.0, rep, pres, freq)
        perm = rng.permutation(V)
        lens = rng.integers(1, 32768 + 1, B)
        hi, ho = _csr([zipf_ids(rng, int(n), V, 1.05, perm) for n in lens])
        return Workload(name, x, params, torch.from_numpy(rng.random(B, dtype=np.float32)), hi, ho, None)
    if name == "verify_bf16":
        B, V = batch or 192, vocab or 262144
        x = (torch.randn(B, V, generator=g) * 2.5).to(torch.bfloat16)
        params = _params(B, rng.uniform(0.5, 1.2, B), 0, 0.95, 0.0, 1.0, 0.0, 0.0)
        draft = torch.from_numpy(rng.integers(0, V, B).astype(np.int32))
        return Workload(name, x, params, torch.from_numpy(rng.random(B, dtype=np.float32)), None, None, draft)
    raise ValueError(f"unknown workload {name!r}; known: {list(NAMES)}")


class SyntheticLM:
    """A stand-in model for the decode loop: the logits of a position are a random rank-``dim``
    map of its token and position, ``(E[token] + P[position mod 64]) @ W``, in ``dtype`` (W scaled
    so logits are about N(0, scale^2)). Slots hold no state: the logits depend on the last token
    and its position only, so any order of steps over any set of slots gives the same rows."""

    def __init__(self, vocab: int, *, dim: int = 64, scale: float = 3.0, dtype=torch.bfloat16,
                 device="cpu", seed: int = 0) -> None:
        g = torch.Generator().manual_seed(seed)
        self.device = torch.device(device)
        self.vocab_size = vocab
        self.dtype = dtype
        self.emb = torch.randn(vocab, dim, generator=g).to(dtype).to(self.device)
        self.pos = torch.randn(64, dim, generator=g).to(dtype).to(self.device)
        self.head = (torch.randn(dim, vocab, generator=g) * (scale / (2 * dim) ** 0.5)).to(dtype).to(self.device)

    stateless = True  # (a decode loop need not feed it tokens whose logits it does not use)

    def decode(self, slots: torch.Tensor, tokens: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        h = self.emb[tokens] + self.pos[positions % 64]
        return h @ self.head

    def decode_into(self, slots: torch.Tensor, tokens: torch.Tensor, positions: torch.Tensor,
                    out: torch.Tensor) -> None:
        """``decode`` with its logits written into ``out`` ``[B, V]``."""
        torch.matmul(self.emb[tokens] + self.pos[positions % 64], self.head, out=out)

    def prefill(self, slot: int, prompt_ids: torch.Tensor) -> torch.Tensor:
        n = int(prompt_ids.shape[0])
        last = prompt_ids[n - 1 :]
        return self.decode(torch.tensor([slot], device=self.device), last,
                           torch.tensor([n - 1], device=self.device))[0]
