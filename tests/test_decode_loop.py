"""The continuous-batching decode loop (``vinfer_amd.runtime``).

The central property: batching never changes a request's tokens. Every test that runs several
requests through ``BatchDecoder`` compares each request with a one-sequence loop that restates
the engine's generate.py:118-144 (prefill, then per token: ``sample(logits, params, seed,
position)``, stop checks, feed the token back) on the same model and sampler backend. The other
tests port the engine's loop tests (tests/unit/runtime/test_generate.py) to the batched loop:
stop ids and ``ignore_eos``, streamed text, stop strings, seeded reproducibility and the
``max_seq_len`` rule. Text and stop strings come from a caller-supplied stream; here a plain
test-local one (``WholeTextStream``) stands in for the engine's.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from vinfer_amd.registry import BackendContext
from vinfer_amd.runtime import BatchDecoder, Step, check_request
from vinfer_amd.sampler import SAMPLER
from vinfer_amd.sampling import SamplingParams, pack_params, uniform
from vinfer_amd.workloads import SyntheticLM

LETTERS = "abcdefghijklmnopqrstuvwxyz"
PROMPT = [5, 17, 3, 88, 42, 9, 61, 70, 12]


def decode(ids: list[int]) -> str:
    return "".join(LETTERS[i % 26] for i in ids)


class WholeTextStream:
    """A test-local text stream: decodes every token so far on each push, reports the first stop
    string (the text ends before it), and holds back the longest stop string's length minus one
    characters until the request ends."""

    def __init__(self, decode_fn, stops):
        self.decode_fn, self.stops, self.ids, self.sent = decode_fn, tuple(stops), [], 0
        self.hold = max((len(x) for x in self.stops), default=1) - 1

    def push(self, token):
        self.ids.append(token)
        text = self.decode_fn(self.ids)
        hits = [i for i in (text.find(x) for x in self.stops) if i >= 0]
        end = min(hits) if hits else max(self.sent, len(text) - self.hold)
        piece, self.sent = text[self.sent : end], max(self.sent, end)
        return piece, bool(hits)

    def flush(self):
        text = self.decode_fn(self.ids)
        piece, self.sent = text[self.sent :], len(text)
        return piece


def streams(decode_fn):
    return lambda stops: WholeTextStream(decode_fn, stops)


def one_at_a_time(model, sampler, prompt, params, eos=frozenset(), text=None, penalize_prompt=False):
    """The engine's one-sequence loop (generate.py:118-144) over a ``DecodeModel``, calling the
    backend's per-token ``sample`` (the engine's call, generate.py:129)."""
    stream = WholeTextStream(text, params.stop) if text else None
    stop_ids = set(params.stop_token_ids) | (set() if params.ignore_eos else set(eos))
    dev = model.device
    logits = model.prefill(0, torch.tensor(prompt, device=dev))
    position = len(prompt)
    generated: list[int] = []
    steps = []
    for n in range(1, params.max_tokens + 1):
        history = (list(prompt) if penalize_prompt else []) + generated
        token = sampler.sample(logits, params, params.seed, position, history=history)
        generated.append(token)
        if token in stop_ids:
            steps.append(Step(token, stream.flush() if stream else "", "stop"))
            return steps
        delta, hit = stream.push(token) if stream else ("", False)
        if hit:
            steps.append(Step(token, delta, "stop"))
            return steps
        if n == params.max_tokens:
            steps.append(Step(token, delta + (stream.flush() if stream else ""), "length"))
            return steps
        steps.append(Step(token, delta))
        logits = model.decode(
            torch.tensor([0], device=dev), torch.tensor([token], device=dev), torch.tensor([position], device=dev)
        )[0]
        position += 1
    return steps


def mixed_requests(n: int, vocab: int, seed: int = 0) -> list[tuple[list[int], SamplingParams]]:
    """Prompts and parameters of every kind: greedy, top-k, top-p, min-p, penalties."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        prompt = rng.integers(0, vocab, size=int(rng.integers(1, 12))).tolist()
        kind = i % 6
        kw = dict(max_tokens=int(rng.integers(1, 20)), seed=int(rng.integers(0, 2**62)))
        if kind == 0:
            kw.update(temperature=0.0)
        elif kind == 1:
            kw.update(temperature=0.8, top_k=int(rng.choice([1, 5, 20])))
        elif kind == 2:
            kw.update(temperature=1.2, top_p=0.7)
        elif kind == 3:
            kw.update(min_p=0.1, top_p=0.95)
        elif kind == 4:
            kw.update(repetition_penalty=1.3, presence_penalty=0.5, frequency_penalty=0.4, temperature=0.7)
        else:
            kw.update(repetition_penalty=1.1, frequency_penalty=1.0, top_k=50, top_p=0.9)
        out.append((prompt, SamplingParams(**kw)))
    return out


def run_batched(model, sampler, reqs, num_slots, max_seq_len=64, **kw):
    dec = BatchDecoder(model, sampler, num_slots=num_slots, max_seq_len=max_seq_len, **kw)
    rids = [dec.submit(p, sp) for p, sp in reqs]
    done = dec.run()
    assert dec._free == sorted(range(num_slots), reverse=True)  # every slot came back
    return [done[r] for r in rids]


@pytest.fixture(scope="module")
def cpu_model():
    return SyntheticLM(96, dim=16, scale=3.0, dtype=torch.float32)


@pytest.fixture(scope="module")
def ref_sampler():
    return SAMPLER.resolve("reference", BackendContext(torch.device("cpu"), torch.float32))


# ---- batching never changes a request's tokens ----------------------------------------------


@pytest.mark.parametrize("num_slots", [1, 3, 16])
@pytest.mark.parametrize("penalize_prompt", [False, True])
def test_batched_tokens_equal_one_sequence_at_a_time(cpu_model, ref_sampler, num_slots, penalize_prompt):
    reqs = mixed_requests(14, cpu_model.vocab_size)
    got = run_batched(cpu_model, ref_sampler, reqs, num_slots, penalize_prompt=penalize_prompt)
    for (prompt, sp), steps in zip(reqs, got):
        want = one_at_a_time(cpu_model, ref_sampler, prompt, sp, penalize_prompt=penalize_prompt)
        assert steps == want


def test_penalties_see_the_request_s_own_history(cpu_model, ref_sampler):
    # A strong frequency penalty on a greedy request forbids repeats while the history holds
    # the token: the loop must hand each row its own, complete history.
    sp = SamplingParams(max_tokens=20, temperature=0.0, frequency_penalty=100.0)
    got = run_batched(cpu_model, ref_sampler, [(PROMPT, sp), ([1, 2], sp), ([7], sp)], num_slots=2)
    for steps in got:
        toks = [s.token_id for s in steps]
        assert len(set(toks)) == len(toks)


def test_unseeded_requests_draw_seeds_from_the_loop_seed(cpu_model, ref_sampler):
    sp = SamplingParams(max_tokens=8, temperature=1.0)
    runs = [run_batched(cpu_model, ref_sampler, [(PROMPT, sp)] * 3, num_slots=2, seed=11) for _ in range(2)]
    assert runs[0] == runs[1]
    other = run_batched(cpu_model, ref_sampler, [(PROMPT, sp)] * 3, num_slots=2, seed=12)
    assert other != runs[0]


def test_cancel_frees_the_slot_and_keeps_the_others(cpu_model, ref_sampler):
    reqs = mixed_requests(4, cpu_model.vocab_size, seed=3)
    reqs = [(p, SamplingParams(**{**sp.__dict__, "max_tokens": 15})) for p, sp in reqs]
    dec = BatchDecoder(cpu_model, ref_sampler, num_slots=2, max_seq_len=64)
    rids = [dec.submit(p, sp) for p, sp in reqs]
    steps: dict[int, list[Step]] = {}
    for rid, st in dec.step():
        steps.setdefault(rid, []).append(st)
    assert dec.cancel(rids[0]) and dec.cancel(rids[3])  # one running, one waiting
    assert not dec.cancel(rids[3])
    for rid, st in dec.run().items():
        steps.setdefault(rid, []).extend(st)
    assert rids[3] not in steps
    for i in (1, 2):
        assert steps[rids[i]] == one_at_a_time(cpu_model, ref_sampler, *reqs[i])


# ---- the engine's loop tests, on the batched loop --------------------------------------------


def test_greedy_output_is_the_argmax_chain(cpu_model, ref_sampler):
    sp = SamplingParams(max_tokens=15, temperature=0)
    (steps,) = run_batched(cpu_model, ref_sampler, [(PROMPT, sp)], num_slots=1)
    tok, pos, want = PROMPT[-1], len(PROMPT) - 1, []
    for _ in range(15):
        row = cpu_model.decode(torch.tensor([0]), torch.tensor([tok]), torch.tensor([pos]))[0]
        tok, pos = int(torch.argmax(row)), pos + 1
        want.append(tok)
    assert [s.token_id for s in steps] == want
    assert steps[-1].finish_reason == "length" and all(s.finish_reason is None for s in steps[:-1])


def test_eos_stops_unless_ignored(cpu_model, ref_sampler):
    greedy = SamplingParams(max_tokens=10, temperature=0)
    (steps,) = run_batched(cpu_model, ref_sampler, [(PROMPT, greedy)], num_slots=1)
    tokens = [s.token_id for s in steps]
    eos = {tokens[3]}
    first = tokens.index(tokens[3])
    (stopped,) = run_batched(cpu_model, ref_sampler, [(PROMPT, greedy)], num_slots=1, eos_token_ids=eos)
    assert len(stopped) == first + 1 and stopped[-1].finish_reason == "stop"
    ignored = SamplingParams(max_tokens=10, temperature=0, ignore_eos=True)
    (kept,) = run_batched(cpu_model, ref_sampler, [(PROMPT, ignored)], num_slots=1, eos_token_ids=eos)
    assert len(kept) == 10
    stop_id = SamplingParams(max_tokens=10, temperature=0, stop_token_ids=(tokens[3],), ignore_eos=True)
    (by_id,) = run_batched(cpu_model, ref_sampler, [(PROMPT, stop_id)], num_slots=1)
    assert len(by_id) == first + 1 and by_id[-1].finish_reason == "stop"


def test_streamed_text_is_the_decoded_output(cpu_model, ref_sampler):
    reqs = [(PROMPT, SamplingParams(max_tokens=12, temperature=0)), ([3, 4], SamplingParams(max_tokens=9, seed=5))]
    for (prompt, sp), steps in zip(reqs, run_batched(cpu_model, ref_sampler, reqs, num_slots=2, text_stream=streams(decode))):
        assert "".join(s.text for s in steps) == decode([s.token_id for s in steps])
        assert steps == one_at_a_time(cpu_model, ref_sampler, prompt, sp, text=decode)


def test_stop_string_ends_the_text_before_it(cpu_model, ref_sampler):
    greedy = SamplingParams(max_tokens=12, temperature=0)
    (steps,) = run_batched(cpu_model, ref_sampler, [(PROMPT, greedy)], num_slots=1)
    full = decode([s.token_id for s in steps])
    stop = full[5:7]
    sp = SamplingParams(max_tokens=12, temperature=0, stop=(stop,))
    (cut,) = run_batched(cpu_model, ref_sampler, [(PROMPT, sp)], num_slots=1, text_stream=streams(decode))
    assert "".join(s.text for s in cut) == full[: full.index(stop)]
    assert cut[-1].finish_reason == "stop"


def test_sampling_is_reproducible_with_a_seed(cpu_model, ref_sampler):
    sp = SamplingParams(max_tokens=10, temperature=1.0, seed=3)
    runs = [run_batched(cpu_model, ref_sampler, [(PROMPT, sp)], num_slots=1) for _ in range(2)]
    assert runs[0] == runs[1]


def test_prompt_plus_max_tokens_must_fit(cpu_model, ref_sampler):
    # 9 prompt tokens + 4 generated: the last one is never fed back, so 12 positions suffice.
    sp = SamplingParams(max_tokens=4, temperature=0, ignore_eos=True)
    (steps,) = run_batched(cpu_model, ref_sampler, [(PROMPT, sp)], num_slots=1, max_seq_len=12)
    assert len(steps) == 4
    dec = BatchDecoder(cpu_model, ref_sampler, num_slots=1, max_seq_len=12)
    with pytest.raises(ValueError, match="max_seq_len"):
        dec.submit(PROMPT, SamplingParams(max_tokens=5))
    with pytest.raises(ValueError, match="empty prompt"):
        check_request(0, sp, 12)


def test_history_rows_stay_inside_their_slot(cpu_model, ref_sampler):
    # Every request runs to the last position its slot allows, with penalties (so its history
    # grows to prompt + max_tokens ids): the neighbouring slots' rows must stay untouched.
    sp = SamplingParams(max_tokens=4, temperature=0.9, repetition_penalty=1.2, ignore_eos=True, seed=1)
    reqs = [(PROMPT[:2], sp), (PROMPT[2:4], sp), (PROMPT[4:6], sp)]
    got = run_batched(cpu_model, ref_sampler, reqs, num_slots=3, max_seq_len=5, penalize_prompt=True)
    for (prompt, p), steps in zip(reqs, got):
        assert steps == one_at_a_time(cpu_model, ref_sampler, prompt, p, penalize_prompt=True)


# ---- on the GPU: the hip backend, bf16 logits at V = 151936 ---------------------------------


@pytest.mark.gpu
def test_gpu_batched_tokens_equal_one_sequence_at_a_time():
    dev = torch.device("cuda", 0)
    model = SyntheticLM(151936, dim=64, scale=3.0, dtype=torch.bfloat16, device=dev)
    hip = SAMPLER.resolve("hip", BackendContext(dev, torch.bfloat16))
    reqs = mixed_requests(24, model.vocab_size, seed=7)
    print("decode loop: 24 requests, 8 slots, V 151936 bf16", flush=True)
    got = run_batched(model, hip, reqs, num_slots=8, max_seq_len=64, penalize_prompt=True)
    for i, ((prompt, sp), steps) in enumerate(zip(reqs, got)):
        want = one_at_a_time(model, hip, prompt, sp, penalize_prompt=True)
        assert steps == want, f"request {i}"


@pytest.mark.gpu
def test_gpu_graph_replays_give_the_per_token_tokens():
    """graphs=True: a membership that holds for two iterations is captured into HIP graphs and
    replayed while it holds (the program's own eager steps, admissions and waits in between);
    every token of every request still equals the per-token loop's. One request's tenth token is
    made a stop id, so requests also end mid-run on a drawn stop (the replayed model step's row
    of a stopped request is dropped)."""
    dev = torch.device("cuda", 0)
    model = SyntheticLM(151936, dim=64, scale=3.0, dtype=torch.bfloat16, device=dev)
    hip = SAMPLER.resolve("hip", BackendContext(dev, torch.bfloat16))
    reqs = [(p, dataclasses.replace(sp, max_tokens=24 + 3 * i))
            for i, (p, sp) in enumerate(mixed_requests(10, model.vocab_size, seed=11))]
    first = one_at_a_time(model, hip, reqs[0][0], reqs[0][1], penalize_prompt=True)
    eos = frozenset({first[9].token_id})
    print("decode loop with graphs: 10 requests, 6 slots, V 151936 bf16", flush=True)
    dec = BatchDecoder(model, hip, num_slots=6, max_seq_len=160, penalize_prompt=True, eos_token_ids=eos,
                       graphs=True, graph_after=2)
    rids = [dec.submit(p, sp) for p, sp in reqs]
    done = dec.run()
    assert dec.graph_steps > 20
    for i, ((prompt, sp), rid) in enumerate(zip(reqs, rids)):
        want = one_at_a_time(model, hip, prompt, sp, eos=eos, penalize_prompt=True)
        assert done[rid] == want, f"request {i}"
    assert done[rids[0]][-1].finish_reason == "stop" and len(done[rids[0]]) <= 10


@pytest.mark.gpu
def test_gpu_decode_loop_rows_match_the_oracle():
    """Each token the loop draws is the oracle's token for the same logits row, history and
    uniform (rows the tie classifier flags excepted)."""
    from oracle.sampler_oracle import classify_ties, penalize, sample_row

    dev = torch.device("cuda", 0)
    model = SyntheticLM(151936, dim=64, scale=3.0, dtype=torch.bfloat16, device=dev)
    hip = SAMPLER.resolve("hip", BackendContext(dev, torch.bfloat16))
    reqs = mixed_requests(6, model.vocab_size, seed=9)
    got = run_batched(model, hip, reqs, num_slots=4, max_seq_len=64)
    checked = 0
    for (prompt, sp), steps in zip(reqs, got):
        tok, pos = prompt[-1], len(prompt) - 1
        history: list[int] = []
        for st in steps:
            row = model.decode(*(torch.tensor([v], device=dev) for v in (0, tok, pos)))[0]
            x = row.float().cpu().numpy()
            if sp.penalized:
                x, _ = penalize(x, np.asarray(history, np.int32), sp.repetition_penalty, sp.presence_penalty,
                                sp.frequency_penalty)
            r = sample_row(x, sp.temperature, sp.top_k, sp.top_p, sp.min_p, uniform(sp.seed, pos + 1))
            if not classify_ties(r):
                assert st.token_id == r.token
                checked += 1
            tok, pos = st.token_id, pos + 1
            history.append(tok)
    assert checked > 20


def test_graphs_need_a_gpu_model_and_a_prepared_sampler(cpu_model, ref_sampler):
    with pytest.raises(ValueError, match="graphs need"):
        BatchDecoder(cpu_model, ref_sampler, num_slots=2, max_seq_len=16, graphs=True)


def test_the_model_hears_when_a_slot_is_released(cpu_model, ref_sampler):
    class Tracking:
        def __init__(self, inner):
            self.inner, self.device, self.live = inner, inner.device, set()

        def prefill(self, slot, prompt):
            assert slot not in self.live
            self.live.add(slot)
            return self.inner.prefill(slot, prompt)

        def decode(self, slots, tokens, positions):
            assert set(slots.tolist()) <= self.live
            return self.inner.decode(slots, tokens, positions)

        def release(self, slot):
            self.live.remove(slot)

    m = Tracking(cpu_model)
    reqs = mixed_requests(9, cpu_model.vocab_size, seed=4)
    dec = BatchDecoder(m, ref_sampler, num_slots=3, max_seq_len=64)
    rids = [dec.submit(p, sp) for p, sp in reqs]
    dec.step()
    dec.cancel(rids[1])
    dec.run()
    assert m.live == set()


def logprob_steps_match_the_oracle(model, sampler, atol):
    from oracle.sampler_oracle import logprobs_row

    sp = SamplingParams(max_tokens=6, temperature=0.9, top_p=0.9, seed=5, logprobs=True, top_logprobs=3)
    plain = SamplingParams(max_tokens=6, temperature=0.9, seed=6)
    got = run_batched(model, sampler, [(PROMPT, sp), ([4, 2], plain)], num_slots=2)
    assert all(st.logprob is None and st.top_logprobs is None for st in got[1])
    tok, pos = PROMPT[-1], len(PROMPT) - 1
    dev = model.device
    for st in got[0]:
        row = model.decode(*(torch.tensor([v], device=dev) for v in (0, tok, pos)))[0]
        wt, wids, wv = logprobs_row(row.float().cpu().numpy(), st.token_id, 3)
        assert abs(st.logprob - wt) <= atol + 2.0**-22 * abs(wt)  # (fp32 outputs)
        assert [i for i, _ in st.top_logprobs] == wids
        assert all(abs(v - w) <= atol + 2.0**-22 * abs(w) for (_, v), w in zip(st.top_logprobs, wv))
        tok, pos = st.token_id, pos + 1


def test_requested_logprobs_come_with_each_step(cpu_model, ref_sampler):
    logprob_steps_match_the_oracle(cpu_model, ref_sampler, 1e-6)


def test_logprob_fields_are_validated():
    with pytest.raises(ValueError, match="top_logprobs"):
        SamplingParams(top_logprobs=21, logprobs=True)
    with pytest.raises(ValueError, match="needs logprobs"):
        SamplingParams(top_logprobs=2)


@pytest.mark.gpu
def test_gpu_requested_logprobs_come_with_each_step():
    dev = torch.device("cuda", 0)
    model = SyntheticLM(151936, dim=64, scale=3.0, dtype=torch.bfloat16, device=dev)
    hip = SAMPLER.resolve("hip", BackendContext(dev, torch.bfloat16))
    logprob_steps_match_the_oracle(model, hip, 2e-5)


# ---- speculative decoding ----------------------------------------------------------------------


def run_speculative(model, draft, sampler, reqs, num_slots, K, max_seq_len=80, **kw):
    from vinfer_amd.runtime import SpeculativeDecoder

    dec = SpeculativeDecoder(model, sampler, draft_model=draft, num_draft=K, num_slots=num_slots,
                             max_seq_len=max_seq_len, **kw)
    rids = [dec.submit(p, sp) for p, sp in reqs]
    done = dec.run()
    assert dec._free == sorted(range(num_slots), reverse=True)
    return [done[r] for r in rids]


def greedy_requests(n, vocab, seed=0, **kw):
    rng = np.random.default_rng(seed)
    return [(rng.integers(0, vocab, int(rng.integers(1, 8))).tolist(),
             SamplingParams(max_tokens=int(rng.integers(1, 25)), temperature=0.0, **kw)) for _ in range(n)]


@pytest.mark.parametrize("K", [1, 3])
def test_speculative_greedy_equals_the_plain_loop(cpu_model, ref_sampler, K):
    # whatever the draft proposes, a greedy target keeps its own argmax chain
    draft = SyntheticLM(96, dim=16, scale=3.0, dtype=torch.float32, seed=1)
    reqs = greedy_requests(7, 96)
    want = run_batched(cpu_model, ref_sampler, reqs, num_slots=3)
    got = run_speculative(cpu_model, draft, ref_sampler, reqs, num_slots=3, K=K)
    assert got == want


def test_speculative_stops_inside_a_block(cpu_model, ref_sampler):
    draft = SyntheticLM(96, dim=16, scale=3.0, dtype=torch.float32, seed=2)
    (plain,) = run_batched(cpu_model, ref_sampler, [(PROMPT, SamplingParams(max_tokens=12, temperature=0))], 1)
    stop = plain[4].token_id
    sp = SamplingParams(max_tokens=12, temperature=0, stop_token_ids=(stop,))
    (want,) = run_batched(cpu_model, ref_sampler, [(PROMPT, sp)], 1)
    (got,) = run_speculative(cpu_model, draft, ref_sampler, [(PROMPT, sp)], 1, K=3)
    assert got == want and got[-1].finish_reason == "stop"


def test_a_perfect_draft_is_always_accepted(cpu_model, ref_sampler):
    from vinfer_amd.runtime import SpeculativeDecoder

    sp = SamplingParams(max_tokens=13, temperature=1.0, top_p=0.9, seed=3)
    dec = SpeculativeDecoder(cpu_model, ref_sampler, draft_model=cpu_model, num_draft=3, num_slots=1, max_seq_len=40)
    dec.submit(PROMPT, sp)
    sizes = []
    while dec.busy:
        sizes.append(len(dec.step()))
    assert sizes == [1, 4, 4, 4]  # the first token from the prefill, then K + 1 per iteration
    with pytest.raises(ValueError, match="penalties"):
        dec.submit(PROMPT, SamplingParams(repetition_penalty=1.2))


class RecordingDraft:
    """A draft model that checks, on every decode, that each earlier position of the slot holds
    the sequence's own token: the position's token was fed since the slot's prefill, and later
    feeds replaced the rejected drafts."""

    def __init__(self, model, sequences):
        self.model, self.device, self.seqs = model, model.device, sequences
        self.fed: dict[int, dict[int, int]] = {}
        self.slot_rid: dict[int, int] = {}
        self.calls = 0

    def prefill(self, slot, prompt_ids):
        self.fed[slot] = dict(enumerate(prompt_ids.tolist()))
        return self.model.prefill(slot, prompt_ids)

    def decode(self, slots, tokens, positions):
        for sl, t, p in zip(slots.tolist(), tokens.tolist(), positions.tolist()):
            fed = self.fed[sl]
            missing = [q for q in range(p) if q not in fed]
            assert not missing, f"slot {sl}: position {p} decoded, positions {missing} never fed"
            fed[p] = t
            for q in [q for q in fed if q > p]:  # positions past p are stale now
                del fed[q]
        self.calls += 1
        return self.model.decode(slots, tokens, positions)


def test_the_draft_model_is_fed_every_position(cpu_model, ref_sampler):
    # A perfect draft keeps every block (K drafts + the bonus): its last draft must still reach
    # the draft model, at its position, before the next block's drafts.
    reqs = [(PROMPT, SamplingParams(max_tokens=14, temperature=1.0, seed=4)),
            ([3, 9], SamplingParams(max_tokens=11, temperature=0.7, top_p=0.9, seed=5))]
    draft = RecordingDraft(cpu_model, reqs)
    got = run_speculative(cpu_model, draft, ref_sampler, reqs, num_slots=2, K=3)
    assert [len(g) for g in got] == [14, 11] and draft.calls > 0
    # a draft that disagrees (rejections leave positions to overwrite)
    other = RecordingDraft(SyntheticLM(96, dim=16, scale=3.0, dtype=torch.float32, seed=2), reqs)
    run_speculative(cpu_model, other, ref_sampler, reqs, num_slots=2, K=2)


def test_speculative_sampling_is_seeded(cpu_model, ref_sampler):
    draft = SyntheticLM(96, dim=16, scale=3.0, dtype=torch.float32, seed=1)
    reqs = [(PROMPT, SamplingParams(max_tokens=15, temperature=0.9, seed=s)) for s in (1, 2, 3)]
    a = run_speculative(cpu_model, draft, ref_sampler, reqs, 2, K=2)
    b = run_speculative(cpu_model, draft, ref_sampler, reqs, 3, K=2)
    assert a == b and all(len(x) == 15 for x in a)


@pytest.mark.gpu
def test_gpu_speculative_greedy_equals_the_plain_loop():
    dev = torch.device("cuda", 0)
    model = SyntheticLM(151936, dim=64, scale=3.0, dtype=torch.bfloat16, device=dev)
    draft = SyntheticLM(151936, dim=64, scale=3.0, dtype=torch.bfloat16, device=dev, seed=1)
    hip = SAMPLER.resolve("hip", BackendContext(dev, torch.bfloat16))
    reqs = greedy_requests(10, 151936, seed=4)
    print("speculative greedy: 10 requests, K=2, V 151936 bf16", flush=True)
    want = run_batched(model, hip, reqs, num_slots=4)
    got = run_speculative(model, draft, hip, reqs, num_slots=4, K=2)
    assert got == want


def spec_requests(n: int, vocab: int, seed: int = 0) -> list[tuple[list[int], SamplingParams]]:
    """Requests speculation can serve (no penalties): greedy, top-k, top-p, min-p, stop ids."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        prompt = rng.integers(0, vocab, size=int(rng.integers(1, 12))).tolist()
        kw = dict(max_tokens=int(rng.integers(20, 45)), seed=int(rng.integers(0, 2**62)))
        kind = i % 5
        if kind == 0:
            kw.update(temperature=0.0)
        elif kind == 1:
            kw.update(temperature=0.8, top_k=int(rng.choice([5, 20, 50])))
        elif kind == 2:
            kw.update(temperature=1.1, top_p=0.8)
        elif kind == 3:
            kw.update(min_p=0.1, top_p=0.95)
        else:
            kw.update(temperature=0.7, stop_token_ids=tuple(int(t) for t in rng.integers(0, vocab, 40)))
        out.append((prompt, SamplingParams(**kw)))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("K", [2, 3])
def test_gpu_speculative_graph_replays_give_the_eager_tokens(K):
    """graphs=True: a membership that holds for two iterations is captured into a HIP graph and
    replayed while it holds; every request's steps must equal the eager loop's, and graph
    replays must have happened."""
    from vinfer_amd.runtime import SpeculativeDecoder

    dev = torch.device("cuda", 0)
    model = SyntheticLM(151936, dim=64, scale=3.0, dtype=torch.bfloat16, device=dev)
    draft = SyntheticLM(151936, dim=64, scale=3.0, dtype=torch.bfloat16, device=dev, seed=1)
    hip = SAMPLER.resolve("hip", BackendContext(dev, torch.bfloat16))
    reqs = spec_requests(9, 151936, seed=K)
    print(f"speculative graphs: 9 requests, 4 slots, K={K}, V 151936 bf16", flush=True)
    want = run_speculative(model, draft, hip, reqs, num_slots=4, K=K, max_seq_len=64)
    dec = SpeculativeDecoder(model, hip, draft_model=draft, num_draft=K, num_slots=4, max_seq_len=64,
                             graphs=True, graph_after=2)
    rids = [dec.submit(p, sp) for p, sp in reqs]
    done = dec.run()
    assert dec.graph_steps > 5, dec.graph_steps
    assert [done[r] for r in rids] == want


@pytest.mark.gpu
def test_gpu_speculative_graphs_greedy_equals_the_plain_loop():
    dev = torch.device("cuda", 0)
    model = SyntheticLM(151936, dim=64, scale=3.0, dtype=torch.bfloat16, device=dev)
    draft = SyntheticLM(151936, dim=64, scale=3.0, dtype=torch.bfloat16, device=dev, seed=1)
    hip = SAMPLER.resolve("hip", BackendContext(dev, torch.bfloat16))
    reqs = greedy_requests(10, 151936, seed=5)
    print("speculative greedy with graphs: 10 requests, K=2, V 151936 bf16", flush=True)
    want = run_batched(model, hip, reqs, num_slots=4)
    got = run_speculative(model, draft, hip, reqs, num_slots=4, K=2, graphs=True, graph_after=2)
    assert got == want
