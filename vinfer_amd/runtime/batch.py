"""Continuous-batching decode loop: every live sequence goes through one model step and one
``sample_batch`` call per iteration.

The engine decodes one sequence at a time (src/vinfer/runtime/generate.py:105-146, one request
after another by scheduler/serial.py:1-5), so its sampler only ever sees one row. This loop keeps
the engine's per-request behaviour and batches the rest:

- requests are checked as generate.py:91-103 checks them (``check_request``), and a request
  without a seed gets one from a ``random.Random(seed)`` of the loop (serial.py:36, :48-49);
- the token at position ``n`` of a sequence is drawn with the uniform of ``(seed, n)``, the same
  one the per-token ``sample`` uses, from that sequence's own logits and history, so batching
  never changes a request's tokens;
- a request ends, as in generate.py:130-142, on a stop id (the request's ``stop_token_ids``,
  plus the end-of-sequence ids unless ``ignore_eos``; the stop token's own text is not output),
  on a stop string, or after ``max_tokens`` tokens ("length"); each token yields one ``Step``.

Detokenization and stop strings are the caller's: ``text_stream(stop_strings)`` makes one
``TextStream`` per request (the engine passes its own, generate.py:27-88), whose ``push`` and
``flush`` give each step's text and report a stop string; without it steps carry no text and
stop strings are not checked.

Requests join whenever a slot is free (prefill, then their first token is sampled in the same
iteration as everyone else's next token) and leave as soon as they finish, freeing their slot.

An iteration launches the next model step right behind the draw, on the drawn ids as they lie
on the device, and waits only for those ids: the host's per-request logic then runs while the
GPU computes the model step. A request that draws a stop token has had that step computed too;
its row is dropped (and ``release`` of its slot comes after that step was enqueued).

With ``graphs=True`` (a GPU model whose ``decode`` can be captured), a membership that stays the
same for ``graph_after`` iterations is captured into HIP graphs -- the inputs' copy, the draw,
the history append, the ids' copy back, then the model step on the drawn ids into the logits
buffer the draw reads -- and its later iterations replay them: one graph launch instead of a
dozen torch and library calls, the staged inputs moved on in place, and the host polls the
ids' pinned copy instead of waiting for an event. Two such graphs alternate so that, while no
request waits for a free slot, the next iteration is launched before the host takes this one's
ids: the host's per-request work then overlaps the GPU's whole iteration. When a row ends, the
iteration already in flight still draws it; that token is dropped.

Histories for the penalties live on the device, one row of ``max_seq_len + 1`` ids per slot,
and are handed to the sampler as per-row ranges (no per-step packing): a sampled id is written
into its row on the device right after the draw. A row's history is the request's generated
tokens, preceded by its prompt when ``penalize_prompt`` is set.
"""

from __future__ import annotations

import dataclasses
import random
from collections import deque
from collections.abc import Callable, Iterable
from dataclasses import dataclass, field
from typing import Protocol

import numpy as np
import torch

from vinfer_amd._lib import position_uniforms
from vinfer_amd.sampler.base import SamplerBackend
from vinfer_amd.sampling import PackedParams, SamplingParams, pack_params, penalized
from vinfer_amd.sampling import field as param_field


class TextStream(Protocol):
    """One request's streamed text, supplied by the caller (the engine's ``_TextStream``,
    generate.py:27-88): ``push(token)`` returns ``(text that is safe to show, stop string
    hit)``; ``flush()`` returns what was held back, once the request ends."""

    def push(self, token: int) -> tuple[str, bool]: ...

    def flush(self) -> str: ...


@dataclass(slots=True)
class Step:
    """One generated token of a request (generate.py:20-24)."""

    token_id: int
    text: str  # new text that is safe to show (empty while it could still be a stop string)
    finish_reason: str | None = None  # "stop" | "length" | None
    # with SamplingParams.logprobs: the token's log-probability under the raw logits, and the
    # top_logprobs most likely (token id, log-probability) pairs
    logprob: float | None = None
    top_logprobs: list[tuple[int, float]] | None = None


def check_request(prompt_len: int, params: SamplingParams, max_seq_len: int) -> None:
    """Raise ``ValueError`` if a request cannot run in ``max_seq_len`` positions (the rule of
    generate.py:91-103: the last sampled token is never fed back, so a request needs
    ``prompt_len + max_tokens - 1`` positions)."""
    if prompt_len == 0:
        raise ValueError("empty prompt")
    needed = prompt_len + params.max_tokens - 1
    if needed > max_seq_len:
        raise ValueError(
            f"prompt ({prompt_len}) + max_tokens ({params.max_tokens}) needs {needed} positions, "
            f"more than max_seq_len ({max_seq_len})"
        )


class DecodeModel(Protocol):
    """What the loop needs of a model: a prefill into a slot and a batched one-token step. A
    model may also define ``release(slot)``, called when a slot's request ends (where a state
    pool would free it, generate.py:146), possibly after one more ``decode`` of that slot was
    enqueued (the step launched before the request's last token was known to be a stop), and
    ``decode_into(slots, tokens, positions, out)``, ``decode`` writing its logits into ``out``
    (the captured loop then needs no copy of them; ``out`` may be a row-strided view), and
    ``stateless = True`` when its slots keep no state (a speculative loop then does not feed it
    tokens whose logits it does not use)."""

    device: torch.device

    def prefill(self, slot: int, prompt_ids: torch.Tensor) -> torch.Tensor:
        """Run ``prompt_ids`` (int64 ``[P]``) into ``slot``; the logits ``[V]`` of its last
        position."""
        ...

    def decode(self, slots: torch.Tensor, tokens: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        """Feed ``tokens[b]`` at ``positions[b]`` into ``slots[b]`` (int64 ``[B]`` each); the
        logits ``[B, V]`` of those positions, row b for ``slots[b]``."""
        ...


class _Staging:
    """Small per-step inputs (int32 words) gathered in one host buffer and sent to the device in
    one copy. On a GPU the host buffer is pinned and the copy asynchronous: the host may refill
    it only after a later synchronisation (the loop alternates two, and waits once per step)."""

    def __init__(self, device: torch.device, words: int) -> None:
        self.host = torch.empty(words, dtype=torch.int32, pin_memory=device.type == "cuda")
        self.dev = torch.empty(words, dtype=torch.int32, device=device)
        self.np = self.host.numpy()
        self.n = 0

    def reset(self) -> None:
        self.n = 0

    def reserve(self, n: int, align: int = 1) -> int:
        at = -(-self.n // align) * align
        if at + n > self.np.shape[0]:
            raise RuntimeError("staging buffer too small")
        self.n = at + n
        return at

    def put(self, words: np.ndarray) -> int:
        at = self.reserve(words.shape[0])
        self.np[at : at + words.shape[0]] = words
        return at

    def host_view(self, at: int, n: int) -> np.ndarray:
        return self.np[at : at + n]

    def send(self) -> None:
        if self.n:
            self.dev[: self.n].copy_(self.host[: self.n], non_blocking=True)

    def device(self, at: int, n: int) -> torch.Tensor:
        return self.dev[at : at + n]


@dataclass(eq=False)
class _Seq:
    rid: int
    prompt: list[int]
    params: SamplingParams  # seed always set
    stop_ids: frozenset[int]
    stream: TextStream | None
    slot: int = -1
    position: int = 0  # position of the next token to sample (= tokens in the sequence so far)
    generated: list[int] = field(default_factory=list)
    # (speculative loop) a token the draft model has not been fed yet: (token, position)
    draft_gap: tuple[int, int] | None = None


@dataclass(eq=False)
class _Group:
    """What a step needs of one membership (the sequences of a draw, in order) that does not
    change from step to step: built when the membership changes, not per step."""

    slots: np.ndarray  # int64 [n]
    seeds: np.ndarray  # int64 [n]
    pen: np.ndarray  # bool [n]: rows with penalties
    pen_slots: np.ndarray  # int64: the slots of those rows
    params: PackedParams
    n_top: int  # largest top_logprobs of a row asking for log-probabilities, or -1 if none asks
    key: tuple[int, ...]  # the request ids, in order


@dataclass(eq=False)
class _StepGraphs:
    """A membership's two captured iterations (graph slots 0 and 1, launched alternately), the
    buffers they hold, and the host views of their staged inputs. Iteration t (counted from the
    eager state) draws every row at position pos0 + t with history end ends0 + t (rows with
    penalties) -- every row moves on by one per iteration while the membership lasts."""

    key: tuple[int, ...]
    graphs: list
    keep: list  # per slot: staging, the sampler's prepared launch, the ids' pinned copy
    logits: torch.Tensor
    ids_np: list  # per slot: the drawn ids' pinned copy (numpy view)
    pen_slots: np.ndarray
    slots: np.ndarray
    pen: np.ndarray
    base: np.ndarray  # the rows' history rows' first index
    pos0: np.ndarray
    ends0: np.ndarray | None  # (None: no row has penalties)
    pos: list  # per slot: staged positions (int64 view)
    seeds: np.ndarray
    u: list  # per slot: staged uniforms
    ends: list  # per slot: staged history ends (or None)
    pen_inc: np.ndarray  # 1 for a row with penalties (its history grows by one a step), else 0
    t: int = 0  # the next iteration to launch
    next: int = 0  # the slot it goes to


@dataclass(eq=False)
class _SpecGraph:
    """A membership's captured speculative iteration, twice (the two captures differ only in the
    pinned buffers their tokens and counts go to, so that two replays can be in flight): the draft
    model fed the token before each last one (unless it keeps no state), K draft steps and draws,
    the target's step, the verify, the next iteration's inputs and uniforms advanced on the
    device from this one's tokens (``vsamp_spec_advance``), and the tokens and counts copied to
    pinned memory (the counts last: the host polls them). The inputs live on the device between
    replays; the host stages them only when a run of replays starts."""

    key: tuple[int, ...]
    graphs: list
    keep: list
    st: object  # _Staging: the inputs' host words and their device copy
    ints: np.ndarray  # int64 [4 + K + (K + 1), n] (host): slots, last, earlier token, its position, positions
    ints_d: object  # the same words on the device (what the graphs read and advance)
    seeds_d: object  # int64 [n]
    ud: object  # float32 [(3K + 1) n]: the iteration's uniforms
    tokens_np: list  # per capture: int32 [n, K + 1]
    counts_np: list  # per capture: int32 [n]
    next: int = 0  # the capture the next replay uses


class BatchDecoder:
    def __init__(
        self,
        model: DecodeModel,
        sampler: SamplerBackend,
        *,
        num_slots: int,
        max_seq_len: int,
        eos_token_ids: Iterable[int] = (),
        text_stream: Callable[[tuple[str, ...]], TextStream] | None = None,
        seed: int = 0,
        penalize_prompt: bool = False,
        graphs: bool = False,
        graph_after: int = 4,
    ) -> None:
        if num_slots < 1 or max_seq_len < 1:
            raise ValueError("num_slots and max_seq_len must be >= 1")
        if graphs and (model.device.type != "cuda" or not hasattr(sampler, "prepare_batch")):
            raise ValueError("graphs need a model on a GPU and a sampler with prepare_batch")
        self.model = model
        self.sampler = sampler
        self.num_slots = num_slots
        self.max_seq_len = max_seq_len
        self.eos_token_ids = frozenset(eos_token_ids)
        self.text_stream = text_stream
        self.penalize_prompt = penalize_prompt
        self._rng = random.Random(seed)
        self._free = list(range(num_slots - 1, -1, -1))  # pop() hands out the lowest slot
        self._waiting: deque[_Seq] = deque()
        self._running: dict[int, _Seq] = {}
        self._next_rid = 0
        # Logits of the last model step, not yet sampled: (sequences, [n, V]).
        self._pending: tuple[list[_Seq], torch.Tensor] | None = None
        self._groups: dict[tuple[int, ...], _Group] = {}
        self._lp: list = []  # this step's log-probability launches
        # One history row per slot; the extra column takes the id drawn at the last position.
        self._hist_row = max_seq_len + 1
        self.hist = torch.zeros(num_slots * self._hist_row, dtype=torch.int32, device=model.device)
        self._hist_len = np.zeros(num_slots, dtype=np.int64)  # ids in each slot's history row
        # One step's inputs, one copy: uniforms and ranges (3 words a row), then the next model
        # step's slots, positions and row indices (int64: 6 words a row), with alignment.
        self._stage = (_Staging(model.device, 9 * num_slots + 8),)
        # the drawn ids' host copy, and the event after it (the iteration's one wait)
        cuda = model.device.type == "cuda"
        self._ids_host = torch.empty(num_slots, dtype=torch.int32, pin_memory=cuda)
        self._ids_np = self._ids_host.numpy()
        self._ids_ready = torch.cuda.Event() if cuda else None
        self.graphs = graphs
        self._appends = bool(getattr(sampler, "appends_history", False))
        self.graph_after = graph_after
        self._graph: _StepGraphs | None = None
        self._graph_key: tuple[int, ...] | None = None  # the last eligible membership and its run
        self._graph_run = 0
        self.graph_steps = 0  # iterations run by replaying graphs
        self._inflight: tuple[_StepGraphs, int, list[_Seq]] | None = None  # (graphs, slot, rows)

    # ---- requests ------------------------------------------------------------------------------
    def submit(self, prompt_ids: list[int], params: SamplingParams) -> int:
        """Queue a request; returns its id. Raises ``ValueError`` if it can never run."""
        check_request(len(prompt_ids), params, self.max_seq_len)
        if params.seed is None:
            params = dataclasses.replace(params, seed=self._rng.getrandbits(63))
        stop_ids = frozenset(params.stop_token_ids) | (frozenset() if params.ignore_eos else self.eos_token_ids)
        stream = self.text_stream(params.stop) if self.text_stream else None
        rid = self._next_rid
        self._next_rid += 1
        self._waiting.append(_Seq(rid, list(prompt_ids), params, stop_ids, stream))
        return rid

    def cancel(self, rid: int) -> bool:
        """Drop a request (waiting or running); True if it was there."""
        for s in self._waiting:
            if s.rid == rid:
                self._waiting.remove(s)
                return True
        s = self._running.pop(rid, None)
        if s is None:
            return False
        if self._pending is not None and any(t is s for t in self._pending[0]):
            seqs, logits = self._pending
            keep = [i for i, t in enumerate(seqs) if t is not s]
            self._pending = (
                ([seqs[i] for i in keep], logits[torch.tensor(keep, device=logits.device)]) if keep else None
            )
        self._retire(s, running=False)
        self._free.sort(reverse=True)
        return True

    @property
    def busy(self) -> bool:
        return bool(self._waiting or self._running)

    @property
    def num_running(self) -> int:
        return len(self._running)

    # ---- one iteration -----------------------------------------------------------------------
    def step(self) -> list[tuple[int, Step]]:
        """Admit what fits, draw one token for every running request, advance the model.
        Returns ``(request id, Step)`` per request that produced a token."""
        if self._inflight is not None:
            return self._step_inflight()
        groups = []
        if self._pending is not None:
            groups.append(self._pending)
            self._pending = None
        admitted = self._admit()
        if admitted is not None:
            groups.append(admitted)
        if not groups:
            return []
        seqs = [s for g in groups for s in g[0]]
        n = len(seqs)
        # rows whose next model step is launched before their token is known: all but the rows
        # drawing their last token by max_tokens
        nxt = [i for i, s in enumerate(seqs) if len(s.generated) + 1 < s.params.max_tokens]
        m = len(nxt)
        key = None
        if self.graphs and admitted is None and m == n:
            g = self._group(seqs, self.model.device)
            key = g.key if g.n_top < 0 else None
        if key is not None and key == self._graph_key:
            self._graph_run += 1
        else:
            self._graph_key, self._graph_run = key, 0
        self._lp = []
        if key is not None and (self._graph_run >= self.graph_after or (self._graph and self._graph.key == key)):
            tokens, nxt_logits = self._graph_step(key, seqs, groups[0][1])
        else:
            tokens, nxt_logits = self._eager_step(groups, seqs, nxt)
        lp_of = self._host_logprobs() if self._lp else None
        out: list[tuple[int, Step]] = []
        going: list[_Seq] = []
        keep: list[int] = []  # the rows of nxt_logits that go on
        advance = self._advance
        j = 0  # position in nxt
        for i, (s, tok) in enumerate(zip(seqs, tokens)):
            step = advance(s, tok)
            if lp_of is not None and param_field(s.params, "logprobs"):
                step.logprob, top = lp_of[id(s)]
                n_top = param_field(s.params, "top_logprobs")
                step.top_logprobs = top[:n_top] if n_top else None
            out.append((s.rid, step))
            launched = j < m and nxt[j] == i
            if step.finish_reason is None:
                going.append(s)
                keep.append(j)
            else:
                self._retire(s)
            j += launched
        if len(going) < n:
            self._free.sort(reverse=True)
        if going and self._inflight is None:  # (with an iteration in flight, it draws them next)
            if len(keep) < m:
                nxt_logits = nxt_logits.index_select(0, torch.tensor(keep, device=nxt_logits.device))
            self._pending = (going, nxt_logits)
        return out

    def _step_inflight(self) -> list[tuple[int, Step]]:
        """An iteration whose graph was launched by the previous call: launch the one after it
        first when every row is still running and no request waits for a free slot, then take
        its ids. A row that ended meanwhile (a stop, a cancel) has its token dropped; without a
        following launch the model step's rows of the rows going on become the pending logits."""
        gs, slot, rows = self._inflight
        self._inflight = None
        alive = [s.rid in self._running for s in rows]
        if all(alive) and not (self._waiting and self._free):
            self._launch(gs, 1 - slot)
            self._inflight = (gs, 1 - slot, rows)
        tokens = self._wait_ids(gs, slot)
        out: list[tuple[int, Step]] = []
        going: list[_Seq] = []
        keep: list[int] = []
        advance = self._advance
        for i, (s, tok) in enumerate(zip(rows, tokens)):
            if not alive[i]:
                continue
            step = advance(s, tok)
            out.append((s.rid, step))
            if step.finish_reason is None:
                going.append(s)
                keep.append(i)
            else:
                self._retire(s)
        if len(going) < len(rows):
            self._free.sort(reverse=True)
        if going and self._inflight is None:
            x = gs.logits
            if len(keep) < len(rows):
                x = x.index_select(0, torch.tensor(keep, device=x.device))
            self._pending = (going, x)
        return out

    def _stage_step(self, st: _Staging, groups, seqs: list[_Seq], nxt) -> tuple[list, int]:
        """Stage a step's inputs: each group's uniforms and ranges, then the next model step's
        slots, positions and rows (int64). Returns the groups' columns and the model's offset."""
        st.reset()
        cols = [self._stage_draw(st, g) for g, _ in groups]
        m = len(nxt)
        at_m = st.reserve(6 * m, align=2)
        if m:
            v = st.host_view(at_m, 6 * m).view(np.int64).reshape(3, m)
            v[0] = np.fromiter((seqs[i].slot for i in nxt), np.int64, m)
            v[1] = np.fromiter((seqs[i].position for i in nxt), np.int64, m)  # the drawn token's
            v[2] = nxt
        return cols, at_m

    def _eager_step(self, groups, seqs: list[_Seq], nxt) -> tuple[list[int], torch.Tensor | None]:
        """Draw every group, launch the next model step on the drawn ids, wait for the ids."""
        n, m = len(seqs), len(nxt)
        st = self._stage[0]
        cols, at_m = self._stage_step(st, groups, seqs, nxt)
        st.send()
        drawn = [self._draw(g, logits, st, c) for (g, logits), c in zip(groups, cols)]
        ids = torch.cat(drawn) if len(drawn) > 1 else drawn[0]
        if self._ids_ready is not None:
            self._ids_host[:n].copy_(ids, non_blocking=True)
            self._ids_ready.record()
        else:
            self._ids_host[:n].copy_(ids)
        nxt_logits = None
        if m:
            mv = st.device(at_m, 6 * m).view(torch.int64).view(3, m)
            toks = ids if m == n else ids.index_select(0, mv[2])
            nxt_logits = self.model.decode(mv[0], toks.long(), mv[1])
        if self._ids_ready is not None:
            self._ids_ready.synchronize()  # (the draws, not the model step behind them)
        return self._ids_np[:n].tolist(), nxt_logits

    def _graph_step(self, key, seqs: list[_Seq], logits: torch.Tensor) -> tuple[list[int], torch.Tensor]:
        """An iteration of a captured membership from the eager state: launch it, launch the next
        one too when no request waits for a free slot (it is then in flight when this returns),
        and take this one's ids."""
        gs = self._graph
        if gs is None or gs.key != key:
            self._graph = None  # (the old graphs' memory goes back before the new capture)
            gs = self._graph = self._capture(key, seqs, logits)
        if logits is not gs.logits:  # (the eager model step's rows)
            gs.logits.copy_(logits)
        # (positions move on from the rows' own: the captured offsets are relative to them)
        gs.pos0[:] = np.fromiter((s.position for s in seqs), np.int64, len(seqs))
        if gs.ends0 is not None:
            gs.ends0[:] = gs.base + np.where(gs.pen, self._hist_len[gs.slots], 0)
        gs.t = 0
        slot = gs.next
        self._launch(gs, slot)
        if not (self._waiting and self._free):
            self._launch(gs, 1 - slot)
            self._inflight = (gs, 1 - slot, seqs)
        return self._wait_ids(gs, slot), gs.logits

    def _launch(self, gs: "_StepGraphs", slot: int) -> None:
        """Stage iteration gs.t's inputs in the slot's buffers and launch its graph."""
        t = gs.t
        gs.t += 1
        gs.next = 1 - slot
        pos = gs.pos[slot]
        np.add(gs.pos0, t, out=pos)
        position_uniforms(gs.seeds, pos, out=gs.u[slot])
        if gs.ends0 is not None:
            np.add(gs.ends0, t * gs.pen_inc, out=gs.ends[slot])
        gs.ids_np[slot][:] = -1  # (drawn ids are >= 0)
        gs.graphs[slot].replay()
        self.graph_steps += 1

    def _wait_ids(self, gs: "_StepGraphs", slot: int) -> list[int]:
        """The slot's drawn ids, by polling their pinned copy (the graph writes it before its
        model step, which runs on meanwhile)."""
        ids = gs.ids_np[slot]
        spins = 0
        while (ids < 0).any():
            spins += 1
            if spins == 1 << 20:  # (long past any draw: the graph's end settles it)
                torch.cuda.current_stream(gs.logits.device).synchronize()
                if (ids < 0).any():
                    raise RuntimeError("the drawn ids never reached the host")
        if gs.pen_slots.size:
            self._hist_len[gs.pen_slots] += 1
        return ids.tolist()

    def _capture(self, key, seqs: list[_Seq], logits: torch.Tensor) -> "_StepGraphs":
        """Two graphs of the membership's iteration (launched alternately, each with its own
        staged inputs, so one can be launched while the other's ids are still awaited): the
        inputs' copy, the draw from ``x``, the history append, the ids to pinned memory, the
        model step on them into ``x``."""
        n = len(seqs)
        dev = logits.device
        g = self._group(seqs, dev)
        x = torch.empty_like(logits)  # the draw's logits, which each graph's model step rewrites
        decode_into = getattr(self.model, "decode_into", None)
        graphs, keep, pos, us, ends, ids_np = [], [], [], [], [], []
        for _ in range(2):
            st = _Staging(dev, 9 * n + 8)
            cols, at_m = self._stage_step(st, [(seqs, None)], seqs, range(n))
            at_u, at_r = cols[0]
            u = st.device(at_u, n).view(torch.float32)
            ranges = None if at_r is None else st.device(at_r, 2 * n).view(n, 2)
            append = {"append_history": True} if ranges is not None and self._appends else {}
            prep = self.sampler.prepare_batch(x, g.params, u, None if ranges is None else self.hist, ranges,
                                              **append)
            ids_host = torch.empty(n, dtype=torch.int32, pin_memory=True)
            mv = st.device(at_m, 6 * n).view(torch.int64).view(3, n)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                st.dev[: st.n].copy_(st.host[: st.n], non_blocking=True)
                prep.launch()
                if ranges is not None and not append:  # the drawn id joins its row's history
                    self.hist.index_copy_(0, ranges[:, 1].long(), prep.ids)
                ids_host.copy_(prep.ids, non_blocking=True)
                if decode_into is not None:
                    decode_into(mv[0], prep.ids.long(), mv[1], x)
                else:
                    x.copy_(self.model.decode(mv[0], prep.ids.long(), mv[1]))
            graphs.append(graph)
            keep.append((st, prep, ids_host))
            # host views of the staged words that move from one iteration to the next
            pos.append(st.host_view(at_m, 6 * n).view(np.int64).reshape(3, n)[1])
            us.append(st.host_view(at_u, n).view(np.float32))
            ends.append(None if at_r is None else st.host_view(at_r, 2 * n).reshape(n, 2)[:, 1])
            ids_np.append(ids_host.numpy())
        pen = g.pen
        return _StepGraphs(key, graphs, keep, x, ids_np, g.pen_slots, g.slots, pen, g.slots * self._hist_row,
                           np.zeros(n, np.int64), None if ends[0] is None else np.zeros(n, np.int32), pos, g.seeds,
                           us, ends, pen.astype(np.int32))

    def run(self) -> dict[int, list[Step]]:
        """Step until every queued request has finished; each request's steps in order."""
        done: dict[int, list[Step]] = {}
        while self.busy:
            for rid, step in self.step():
                done.setdefault(rid, []).append(step)
        return done

    # ---- internals ---------------------------------------------------------------------------
    def _retire(self, s: _Seq, running: bool = True) -> None:
        if running:
            del self._running[s.rid]
        self._free.append(s.slot)
        release = getattr(self.model, "release", None)
        if release is not None:
            release(s.slot)

    def _admit(self) -> tuple[list[_Seq], torch.Tensor] | None:
        seqs, rows = [], []
        dev = self.model.device
        while self._waiting and self._free:
            s = self._waiting.popleft()
            s.slot = self._free.pop()
            s.position = len(s.prompt)
            prompt = torch.tensor(s.prompt, dtype=torch.int64)
            self._hist_len[s.slot] = 0
            if penalized(s.params) and self.penalize_prompt:
                base = s.slot * self._hist_row
                self.hist[base : base + len(s.prompt)] = prompt.to(torch.int32).to(dev)
                self._hist_len[s.slot] = len(s.prompt)
            rows.append(self.model.prefill(s.slot, prompt.to(dev)).reshape(-1))
            self._running[s.rid] = s
            seqs.append(s)
        return (seqs, torch.stack(rows)) if seqs else None

    def _group(self, seqs: list[_Seq], dev: torch.device) -> _Group:
        key = tuple(s.rid for s in seqs)
        g = self._groups.get(key)
        if g is None:
            if len(self._groups) > 64:  # memberships change as requests come and go
                self._groups.clear()
            ps = [s.params for s in seqs]
            slots = np.array([s.slot for s in seqs], dtype=np.int64)
            pen = np.array([penalized(p) for p in ps], dtype=bool)
            lps = [param_field(p, "top_logprobs") for p in ps if param_field(p, "logprobs")]
            g = self._groups[key] = _Group(slots, np.array([p.seed for p in ps], dtype=np.int64), pen, slots[pen],
                                           pack_params(ps, dev), max(lps) if lps else -1, key)
        return g

    def _params(self, seqs: list[_Seq], dev: torch.device) -> PackedParams:
        return self._group(seqs, dev).params

    def _stage_draw(self, st: _Staging, seqs: list[_Seq]) -> tuple[int, int | None]:
        """Stage one group's uniforms and (when a row has penalties) history ranges."""
        n = len(seqs)
        g = self._group(seqs, self.model.device)
        at_u = st.reserve(n)
        position_uniforms(g.seeds, np.fromiter((s.position for s in seqs), np.int64, n),
                          out=st.host_view(at_u, n).view(np.float32))
        if not g.pen_slots.size:
            return at_u, None
        # Rows without penalties get an empty range (their slot's history is not kept).
        at_r = st.reserve(2 * n)
        r = st.host_view(at_r, 2 * n).reshape(n, 2)
        base = g.slots * self._hist_row
        r[:, 0] = base
        r[:, 1] = base + np.where(g.pen, self._hist_len[g.slots], 0)
        return at_u, at_r

    def _draw(self, seqs: list[_Seq], logits: torch.Tensor, st: _Staging, cols) -> torch.Tensor:
        """Launch the sampler over one group; the drawn ids stay on the device. With a row that
        asks for log-probabilities, their launch follows (results kept for ``_advance``)."""
        n = len(seqs)
        at_u, at_r = cols
        u = st.device(at_u, n).view(torch.float32)
        g = self._group(seqs, logits.device)
        if at_r is None:
            ids, _ = self.sampler.sample_batch(logits, g.params, u)
        else:
            # The drawn id joins its row's history right behind the range just used (by the
            # sampler's own launch when it can).
            ranges = st.device(at_r, 2 * n).view(n, 2)
            if self._appends:
                ids, _ = self.sampler.sample_batch(logits, g.params, u, self.hist, ranges, append_history=True)
            else:
                ids, _ = self.sampler.sample_batch(logits, g.params, u, self.hist, ranges)
                self.hist.index_copy_(0, ranges[:, 1].long(), ids)
            self._hist_len[g.pen_slots] += 1
        if g.n_top >= 0:
            tok_lp, top_ids, top_lp = self.sampler.logprobs(logits, ids, g.n_top)
            self._lp.append((seqs, tok_lp, top_ids, top_lp))
        return ids

    def _host_logprobs(self) -> dict[int, tuple[float, list[tuple[int, float]]]]:
        """The step's log-probabilities on the host, by sequence (after the step's wait)."""
        out = {}
        for seqs, tok_lp, top_ids, top_lp in self._lp:
            tl, ti, tv = tok_lp.tolist(), top_ids.tolist(), top_lp.tolist()
            for i, s in enumerate(seqs):
                if param_field(s.params, "logprobs"):
                    out[id(s)] = (tl[i], list(zip(ti[i], tv[i])))
        return out

    def _advance(self, s: _Seq, tok: int) -> Step:
        """The request-side logic of one token (generate.py:130-142)."""
        s.generated.append(tok)
        s.position += 1
        if tok in s.stop_ids:  # the stop token's own text is not part of the output
            return Step(tok, s.stream.flush() if s.stream else "", "stop")
        text, hit = s.stream.push(tok) if s.stream else ("", False)
        if hit:
            return Step(tok, text, "stop")
        if len(s.generated) == s.params.max_tokens:
            return Step(tok, text + (s.stream.flush() if s.stream else ""), "length")
        return Step(tok, text)


class SpeculativeDecoder(BatchDecoder):
    """The batched loop with speculative decoding: a draft model proposes ``num_draft`` tokens
    per sequence, the target scores them in one step, and ``verify`` keeps each draft with
    probability min(1, p / q), replacing the first rejected one from the residual, or adds the
    target's bonus token when all are kept -- so a sequence advances 1 .. K + 1 tokens per
    iteration and its tokens are distributed exactly as the target's sampling (the MTP flow of
    the engine's reference deployments, vllm/configs/tuned-mtp.sh:13, whose head the engine's
    loader skips, models/loader.py:27).

    A sequence's first token is drawn from its prefill as in ``BatchDecoder``. After that, the
    token at position n is decided with uniforms of ``(seed, -(4n + c))``, c = 1 (the draft's
    draw), 2 (acceptance), 3 (residual), 4 (bonus): independent streams of the same per-request
    seed. Greedy requests therefore get exactly the tokens the plain loop gives them, whatever
    the draft proposes. Penalties and log-probabilities are not available here (``verify``
    applies no penalties).

    The target may define ``extend(slots, tokens [B, T], positions [B]) -> logits [B, T, V]``
    (T tokens per slot from ``positions[b]``); without it the loop calls ``decode`` on the
    flattened tokens, which is right for a model without per-slot state only. The draft model
    is a ``DecodeModel`` fed every token of the sequence at its position: a rejected draft leaves
    positions that the next iteration overwrites, and after a block with every draft accepted the
    last draft (which the draft model proposed but was never fed) is fed at the start of the next
    iteration, before the new drafts, so a draft with per-slot state never attends to a stale
    position.
    """

    def __init__(self, model: DecodeModel, sampler: SamplerBackend, *, draft_model: DecodeModel, num_draft: int,
                 **kw) -> None:
        if num_draft < 1:
            raise ValueError("num_draft must be >= 1")
        super().__init__(model, sampler, **kw)
        self.draft_model = draft_model
        self.num_draft = num_draft
        self._ready: list[_Seq] = []  # sequences with a first token, waiting for an iteration
        self._spec_graph: _SpecGraph | None = None
        self._spec_key: tuple[int, ...] | None = None  # the last membership and its run
        self._spec_run = 0
        # (graphs) iterations launched before the host took their tokens, oldest first: (the
        # graph, its capture, the sequences); at most two
        self._spec_q: deque[tuple[_SpecGraph, int, list[_Seq]]] = deque()

    def submit(self, prompt_ids: list[int], params: SamplingParams) -> int:
        if penalized(params):
            raise ValueError("speculative decoding applies no penalties")
        if param_field(params, "logprobs"):
            raise ValueError("speculative decoding reports no log-probabilities")
        # positions up to prompt + max_tokens - 1 + num_draft are scored (the last block's drafts)
        check_request(len(prompt_ids), dataclasses.replace(params, max_tokens=params.max_tokens + self.num_draft),
                      self.max_seq_len)
        return super().submit(prompt_ids, params)

    def step(self) -> list[tuple[int, Step]]:
        out: list[tuple[int, Step]] = []
        if self._spec_q:
            out += self._take_inflight()
        else:
            spec = [s for s in self._ready if s.rid in self._running]
            self._ready = []
            if spec:
                out += self._speculate(spec)
        admitted = self._admit()
        if admitted is not None:
            seqs, logits = admitted
            for s in seqs:
                self.draft_model.prefill(s.slot, torch.tensor(s.prompt, dtype=torch.int64, device=self.draft_model.device))
            st = self._stage[0]
            st.reset()
            cols = self._stage_draw(st, seqs)
            st.send()
            self._lp = []
            tokens = self._draw(seqs, logits, st, cols).tolist()
            for s, tok in zip(seqs, tokens):
                step = self._advance(s, tok)
                out.append((s.rid, step))
                if step.finish_reason is None:
                    self._ready.append(s)
                else:
                    self._retire(s)
        self._free.sort(reverse=True)
        return out

    def _speculate(self, seqs: list[_Seq]) -> list[tuple[int, Step]]:
        if self.graphs and hasattr(self.sampler, "spec_advance"):
            key = tuple(s.rid for s in seqs)
            if key == self._spec_key:
                self._spec_run += 1
            else:
                self._spec_key, self._spec_run = key, 0
            if self._spec_run >= self.graph_after or (self._spec_graph is not None and self._spec_graph.key == key):
                return self._speculate_graph(key, seqs)
        K = self.num_draft
        n = len(seqs)
        dev = self.model.device
        g = self._group(seqs, dev)
        params = g.params
        # the step's host inputs in two copies: slots, last tokens and their positions; then every
        # uniform of the step, of streams c = 1 (draft draws, [K, n]: one contiguous row per
        # draft), 2 (acceptance) and 3 (residual) ([n, K] each) at positions + 0 .. K - 1, and
        # 4 (bonus) at position + K
        position = np.fromiter((s.position for s in seqs), np.int64, n)
        ints = np.stack([g.slots, np.fromiter((s.generated[-1] for s in seqs), np.int64, n), position - 1])
        offs = np.arange(K, dtype=np.int64)
        at = position[:, None] + offs[None, :]  # [n, K]
        useeds = np.concatenate([np.tile(g.seeds, K), np.repeat(g.seeds, K), np.repeat(g.seeds, K), g.seeds])
        upos = np.concatenate([-(4 * at.T + 1).ravel(), -(4 * at + 2).ravel(), -(4 * at + 3).ravel(),
                               -(4 * (position + K) + 4)])
        u = torch.from_numpy(position_uniforms(useeds, upos)).to(dev)
        ints_d = torch.from_numpy(ints).to(dev)
        slots, last, pos0 = ints_d[0], ints_d[1], ints_d[2]  # (pos0: the last token's position)
        nk = n * K
        u_draft = u[:nk].view(K, n)
        u_accept, u_residual, u_bonus = u[nk:2 * nk].view(n, K), u[2 * nk:3 * nk].view(n, K), u[3 * nk:]
        # the last draft of a fully accepted block reaches the draft model first (logits unused)
        gap = [s for s in seqs if s.draft_gap is not None]
        if gap and getattr(self.draft_model, "stateless", False):
            for s in gap:  # (a draft model without state needs no feed)
                s.draft_gap = None
            gap = []
        if gap:
            gd = torch.from_numpy(np.array([[s.slot for s in gap], [s.draft_gap[0] for s in gap],
                                            [s.draft_gap[1] for s in gap]], dtype=np.int64))
            gd = gd.to(self.draft_model.device)
            self.draft_model.decode(gd[0], gd[1], gd[2])
            for s in gap:
                s.draft_gap = None
        # the draft proposes K tokens
        x = last
        draft_rows, drafts, states = [], [], []
        with_states = hasattr(self.sampler, "sample_states")  # (the draft rows' states, for verify)
        for j in range(K):
            logits = self.draft_model.decode(slots, x, pos0 + j)
            if with_states:
                ids, st = self.sampler.sample_states(logits, params, u_draft[j])
                states.append(st)
            else:
                ids, _ = self.sampler.sample_batch(logits, params, u_draft[j])
            draft_rows.append(logits)
            drafts.append(ids)
            x = ids.long()
        drafts_t = torch.stack(drafts, dim=1)  # [n, K]
        # the target scores the last token and the K drafts
        toks = torch.cat([last.view(n, 1), drafts_t.long()], dim=1)  # [n, K + 1]
        extend = getattr(self.model, "extend", None)
        if extend is not None:
            target = extend(slots, toks, pos0)
        else:
            steps = torch.arange(K + 1, device=dev)
            target = self.model.decode(slots.repeat_interleave(K + 1), toks.reshape(-1),
                                       (pos0.view(n, 1) + steps).reshape(-1)).view(n, K + 1, -1)
        tokens, counts = self.sampler.verify(
            target, torch.stack(draft_rows, dim=1), drafts_t, params, u_accept, u_residual, u_bonus,
            draft_states=torch.stack(states, dim=1) if with_states else None,
        )
        tokens, counts = tokens.tolist(), counts.tolist()  # the iteration's wait
        return self._emit(seqs, tokens, counts)

    def _emit(self, seqs: list[_Seq], tokens: list[list[int]], counts: list[int],
              ready: bool = True) -> list[tuple[int, Step]]:
        """Each sequence's emitted tokens through the per-request logic; the ones going on wait
        for the next iteration (unless it is already in flight: ``ready`` false)."""
        K = self.num_draft
        out: list[tuple[int, Step]] = []
        for s, row, c in zip(seqs, tokens, counts):
            if c == K + 1:  # every draft kept: the draft model has not seen the last one
                s.draft_gap = (row[K - 1], s.position + K - 1)
            for tok in row[:c]:
                step = self._advance(s, tok)
                out.append((s.rid, step))
                if step.finish_reason is not None:
                    self._retire(s)
                    break
            else:
                if ready:
                    self._ready.append(s)
        return out

    # ---- the iteration as a HIP graph -----------------------------------------------------------
    def _speculate_graph(self, key: tuple[int, ...], seqs: list[_Seq]) -> list[tuple[int, Step]]:
        """The iteration of a membership that held for ``graph_after`` iterations, replayed from a
        HIP graph. The host stages the inputs from the sequences once; from then on each replay
        advances them on the device for the next, so while the membership can hold (no request
        waits for a free slot) the next iteration is queued before the host waits for this one,
        and the host's per-request logic overlaps the GPU's work. Every sequence's draft model is
        fed the token before its last one, at its position (a sequence whose previous block was
        fully accepted needs it; for the others it repeats a step already taken, which a model
        whose state is indexed by position, as the loop's overwriting of rejected positions
        already assumes, takes unchanged; a draft model without state is not fed)."""
        gs = self._spec_graph
        if gs is None or gs.key != key:
            self._spec_graph = None  # (the old graph's memory goes back before the new capture)
            gs = self._spec_graph = self._capture_spec(key, seqs)
        self._stage_spec(gs, seqs)
        gs.st.send()
        self.sampler.spec_advance(gs.ints_d, self.num_draft, gs.seeds_d, gs.ud)  # (this iteration's uniforms)
        self._launch_spec(gs, seqs)
        return self._take_inflight()

    def _take_inflight(self) -> list[tuple[int, Step]]:
        """The oldest iteration in flight: first the next one is queued when the membership can
        hold (at most two in flight), then its tokens, for the sequences still running (a
        sequence that ended meanwhile has its block dropped)."""
        gs, buf, seqs = self._spec_q[0]
        if (len(self._spec_q) == 1 and gs is self._spec_graph and not (self._waiting and self._free)
                and not self._ready and all(s.rid in self._running for s in seqs)):
            self._launch_spec(gs, seqs)
        tokens, counts = self._wait_spec(gs, buf)
        self._spec_q.popleft()
        ready = not self._spec_q  # (else these sequences are in the iteration still in flight)
        alive = [s.rid in self._running for s in seqs]
        if not all(alive):
            keep = [i for i, a in enumerate(alive) if a]
            seqs, tokens, counts = [seqs[i] for i in keep], [tokens[i] for i in keep], [counts[i] for i in keep]
        for s in seqs:
            s.draft_gap = None  # (the graph feeds every sequence the token before its last)
        return self._emit(seqs, tokens, counts, ready=ready)

    def _launch_spec(self, gs: _SpecGraph, seqs: list[_Seq]) -> None:
        buf = gs.next
        gs.next = 1 - buf
        gs.counts_np[buf][:] = -1  # (counts are >= 1; this capture's last replay was read)
        gs.graphs[buf].replay()
        self._spec_q.append((gs, buf, seqs))
        self.graph_steps += 1

    def _wait_spec(self, gs: _SpecGraph, buf: int) -> tuple[list[list[int]], list[int]]:
        counts = gs.counts_np[buf]
        spins = 0
        while (counts < 0).any():
            spins += 1
            if spins == 1 << 20:  # (long past any iteration: the graph's end settles it)
                torch.cuda.current_stream(self.model.device).synchronize()
                if (counts < 0).any():
                    raise RuntimeError("the verified tokens never reached the host")
        return gs.tokens_np[buf].tolist(), counts.tolist()

    def _stage_spec(self, gs: _SpecGraph, seqs: list[_Seq]) -> None:
        """An iteration's inputs, from the sequences as they stand, into the graph's pinned
        staging words (sent to the device before a run of replays starts)."""
        n = len(seqs)
        K = self.num_draft
        ints = gs.ints
        position = np.fromiter((s.position for s in seqs), np.int64, n)
        ints[1] = np.fromiter((s.generated[-1] for s in seqs), np.int64, n)
        # the token at position - 2: the second-to-last generated one, or the prompt's last
        ints[2] = np.fromiter((s.generated[-2] if len(s.generated) >= 2 else s.prompt[-1] for s in seqs),
                              np.int64, n)
        ints[3] = position - 2
        ints[4:4 + K] = position[None, :] - 1 + np.arange(K, dtype=np.int64)[:, None]  # draft steps
        # the target's positions, sequence-major: token c of sequence b at b (K + 1) + c
        ints[4 + K:].reshape(-1)[:] = (position[:, None] - 1 + np.arange(K + 1, dtype=np.int64)[None, :]).reshape(-1)

    def _capture_spec(self, key: tuple[int, ...], seqs: list[_Seq]) -> _SpecGraph:
        n = len(seqs)
        K = self.num_draft
        dev = self.model.device
        g = self._group(seqs, dev)
        params = g.params
        rows = 4 + K + (K + 1)
        st = _Staging(dev, 2 * rows * n + 8)
        at_i = st.reserve(2 * rows * n, align=2)
        ints = st.host_view(at_i, 2 * rows * n).view(np.int64).reshape(rows, n)
        ints[0] = g.slots
        ints_d = st.device(at_i, 2 * rows * n).view(torch.int64).view(rows, n)
        seeds_d = torch.from_numpy(g.seeds).to(dev)
        ud = torch.empty((3 * K + 1) * n, dtype=torch.float32, device=dev)
        gs = _SpecGraph(key, [], [], st, ints, ints_d, seeds_d, ud, [], [])
        self._stage_spec(gs, seqs)
        slots, last, gtok, gpos = ints_d[0], ints_d[1], ints_d[2], ints_d[3]
        dpos = ints_d[4:4 + K]  # [K, n]: the draft steps' positions
        tpos = ints_d[4 + K:].reshape(-1)  # [n (K + 1)]: position of target token c of sequence b at b (K + 1) + c
        nk = n * K
        u_draft = ud[:nk].view(K, n)
        u_accept, u_residual, u_bonus = ud[nk:2 * nk].view(n, K), ud[2 * nk:3 * nk].view(n, K), ud[3 * nk:]
        with_states = hasattr(self.sampler, "sample_states")
        extend = getattr(self.model, "extend", None)
        draft_into = getattr(self.draft_model, "decode_into", None)
        target_into = getattr(self.model, "decode_into", None)
        feed = not getattr(self.draft_model, "stateless", False)
        # The logits' shape from one eager feed of the token before the last (the graph's own
        # first step, so a model with state sees nothing it would not see anyway), then the
        # buffers the graph writes the draft and target logits into.
        st.send()
        self.sampler.spec_advance(ints_d, K, seeds_d, ud)
        probe = self.draft_model.decode(slots, gtok, gpos)
        vocab, ldt = int(probe.shape[-1]), probe.dtype
        del probe
        dbuf = torch.empty(n, K, vocab, dtype=ldt, device=dev) if draft_into is not None else None
        tbuf = torch.empty(n, K + 1, vocab, dtype=ldt, device=dev) if extend is None and target_into else None
        toks = torch.empty(n, K + 1, dtype=torch.int64, device=dev)  # the last token, then the drafts
        slots_rep = slots.repeat_interleave(K + 1) if extend is None else None  # (fixed per membership)
        torch.cuda.synchronize(dev)
        pool = None
        outs = []
        for _ in range(2):
            tokens_host = torch.empty(n, K + 1, dtype=torch.int32, pin_memory=True)
            counts_host = torch.empty(n, dtype=torch.int32, pin_memory=True)
            graph = torch.cuda.CUDAGraph()
            # (the two captures share a memory pool: they are replayed one after the other on one
            # stream, never at once)
            with torch.cuda.graph(graph, pool=pool):
                if feed:
                    self.draft_model.decode(slots, gtok, gpos)
                toks[:, 0].copy_(last)
                x = last
                draft_rows, states = [], []
                for j in range(K):
                    if dbuf is not None:
                        draft_into(slots, x, dpos[j], dbuf[:, j])
                        logits = dbuf[:, j]
                    else:
                        logits = self.draft_model.decode(slots, x, dpos[j])
                        draft_rows.append(logits)
                    if with_states:
                        ids, state = self.sampler.sample_states(logits, params, u_draft[j])
                        states.append(state)
                    else:
                        ids, _ = self.sampler.sample_batch(logits, params, u_draft[j])
                    toks[:, j + 1].copy_(ids)
                    x = toks[:, j + 1]
                dl = dbuf if dbuf is not None else torch.stack(draft_rows, dim=1)
                if extend is not None:
                    target = extend(slots, toks, dpos[0])
                else:
                    tt = toks.reshape(-1)
                    if tbuf is not None:
                        target_into(slots_rep, tt, tpos, tbuf.view(n * (K + 1), vocab))
                        target = tbuf
                    else:
                        target = self.model.decode(slots_rep, tt, tpos).view(n, K + 1, -1)
                tokens, counts = self.sampler.verify(
                    target, dl, toks[:, 1:], params, u_accept, u_residual, u_bonus,
                    draft_states=torch.stack(states, dim=1) if with_states else None,
                )
                # the next iteration's inputs and uniforms, then the tokens and counts to the host
                self.sampler.spec_advance(ints_d, K, seeds_d, ud, tokens, counts)
                tokens_host.copy_(tokens, non_blocking=True)
                counts_host.copy_(counts, non_blocking=True)  # (after the tokens: the host polls these)
            torch.cuda.synchronize(dev)
            pool = graph.pool()
            gs.graphs.append(graph)
            gs.tokens_np.append(tokens_host.numpy())
            gs.counts_np.append(counts_host.numpy())
            outs += [tokens_host, counts_host]
        gs.keep = [toks, slots_rep, dbuf, tbuf, *outs]
        return gs
