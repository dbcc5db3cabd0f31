"""The sampler op family: its interface and its registry.

``sample`` keeps the engine's per-token call unchanged (src/vinfer/runtime/sampler.py:68,
called from runtime/generate.py:129): one 1-D ``[V]`` logits row in the model dtype, the
request's ``SamplingParams``, its seed and the token position, returning a Python ``int``.
Batched entry points are new methods of the interface, as the engine's convention for kernel
families prescribes (kernels/gdn/base.py:7-8). Logits are caller-owned and never written.
"""

from __future__ import annotations

from collections.abc import Sequence
from typing import Protocol

import torch

from vinfer_amd.registry import BackendRegistry
from vinfer_amd.sampling import PackedParams, SamplingParams, penalized


class SamplerBackend(Protocol):
    def sample(
        self,
        logits: torch.Tensor,
        params: SamplingParams,
        seed: int,
        position: int,
        history: Sequence[int] | torch.Tensor | None = None,
    ) -> int:
        """One token id from ``logits`` (``[V]``) for the token at ``position``. ``history`` is
        the request's token ids so far (empty for the first token): it is required when a
        penalty is on (``ValueError`` if it is ``None``), since the penalties are computed from
        it, and ignored otherwise."""
        ...

    def sample_batch(
        self,
        logits: torch.Tensor,
        params: PackedParams,
        uniforms: torch.Tensor,
        hist_ids: torch.Tensor | None = None,
        hist_offsets: torch.Tensor | None = None,
        draft_ids: torch.Tensor | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor | None]:
        """One token per row of ``logits`` ``[B, V]``: ids int32 ``[B]`` and, when ``draft_ids``
        (int32 ``[B]``) is given, the final probability of each draft id (fp32 ``[B]``).
        ``uniforms`` fp32 ``[B]`` in [0, 1). Histories (int32) are in CSR form (``hist_offsets``
        ``[B + 1]``) or per-row ranges (``hist_offsets`` ``[B, 2]``: row b's ids are
        ``hist_ids[start_b:end_b]``; ranges of different rows must not overlap)."""
        ...

    def probs(
        self,
        logits: torch.Tensor,
        params: PackedParams,
        hist_ids: torch.Tensor | None = None,
        hist_offsets: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """The fp32 ``[B, V]`` distribution ``sample_batch`` draws from (``filtered_probs``,
        sampler.py:50-65, plus penalties and min-p)."""
        ...

    def verify(
        self,
        target_logits: torch.Tensor,
        draft_logits: torch.Tensor,
        draft_tokens: torch.Tensor,
        params: PackedParams,
        u_accept: torch.Tensor,
        u_residual: torch.Tensor,
        u_bonus: torch.Tensor,
        draft_params: PackedParams | None = None,
        draft_states: torch.Tensor | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Speculative-decoding verify of ``K`` drafted tokens per sequence: draft ``j`` is
        accepted when ``u_accept[b, j] * q < p`` (``p``, ``q``: the target's and the draft's
        final probabilities of it); at the first rejection the token is drawn with
        ``u_residual[b, j]`` from ``max(0, p - q)`` over ascending ids; with every draft
        accepted, the target's draw at position ``K`` (uniform ``u_bonus[b]``) is added.
        ``target_logits`` ``[B, K + 1, V]``, ``draft_logits`` ``[B, K, V]`` (same dtype),
        ``draft_tokens`` int32 ``[B, K]``, uniforms fp32; ``params`` (one row per sequence)
        apply to the target rows, ``draft_params`` (default: the same) to the draft rows;
        penalties are not applied. A backend with ``sample_states`` (an optional method: the
        draws plus each row's opaque sampling state) takes the drafts' saved states as
        ``draft_states`` ``[B, K, ...]`` instead of sampling the draft rows again. Returns
        ``tokens`` int32 ``[B, K + 1]`` (emitted tokens, then -1) and ``counts`` int32 ``[B]``
        (1 .. K + 1)."""
        ...

    def logprobs(
        self, logits: torch.Tensor, tokens: torch.Tensor | None = None, n_top: int = 0
    ) -> tuple[torch.Tensor | None, torch.Tensor, torch.Tensor]:
        """Log-probabilities of the raw logits ``[B, V]`` (log-softmax before penalties,
        temperature and filters: what ``logprobs`` / ``top_logprobs`` report): of ``tokens``
        (int32 ``[B]``, NaN outside the vocabulary) and of each row's ``n_top`` (0 .. 32)
        largest logits, descending with ties by ascending id. Returns ``(token_logprobs fp32
        [B] or None, top_ids int32 [B, n_top], top_logprobs fp32 [B, n_top])``; a row whose max
        logit is not finite reports NaN."""
        ...

    def penalized_logits(
        self,
        logits: torch.Tensor,
        params: PackedParams,
        hist_ids: torch.Tensor | None = None,
        hist_offsets: torch.Tensor | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Penalised fp32 logits ``[B, V]`` and the history count of every id (int32 ``[B, V]``)."""
        ...


def require_history(params: SamplingParams, history) -> None:
    """``ValueError`` when ``params`` turns a penalty on and no history was passed: the engine's
    per-token call (src/vinfer/runtime/generate.py:129) passes none, and silently sampling
    without the penalties would be a fallback (kernels/registry.py:5-7 rules those out)."""
    if penalized(params) and history is None:
        raise ValueError(
            "repetition/presence/frequency penalties need the request's token history: "
            "pass history= (the token ids so far, empty for the first token)"
        )


SAMPLER: BackendRegistry[SamplerBackend] = BackendRegistry("sampler")
