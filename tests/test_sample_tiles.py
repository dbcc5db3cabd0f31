"""The draw over logits with their tile maxima: bf16 logits from the LM head's epilogue
(``vsamp_sample_tiles``), or bf16 and fp32 logits whose maxima a launch computes itself
(``vsamp_sample_tile_pass``, which the per-token call and small batches take).

Both must give exactly what the row passes give on the same logits and arguments (``sample_batch``
with ``tile_pass`` off):
the same ids and the same draft probabilities, bit for bit, whether a row is decided from a few
tiles (greedy rows, and top-k or min-p rows, without penalties) or takes the row passes
(penalties, top-p alone, NaN and infinite rows, too many candidates). Both are then checked
against the oracle on every non-tie row. Logits come from ``vsamp_lm_head`` (real GEMM output,
with peaked rows made by a hidden state close to one weight row) and from crafted rows whose
tile maxima the test computes (ties of the max across tiles, signed zeros, -inf, NaN and +inf
rows, massive ties at the top-k boundary)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from tests.parity import compare_ids, oracle
from vinfer_amd import _lib
from vinfer_amd.registry import BackendContext
from vinfer_amd.sampler import SAMPLER
from vinfer_amd.sampling import SamplingParams, pack_history, pack_params
from vinfer_amd.workloads import Workload

DEV = torch.device("cuda", 0)
TILE = _lib.LM_TILE


def hip():
    return SAMPLER.resolve("hip", BackendContext(DEV, torch.bfloat16))


def row_passes(s, *args):
    """``sample_batch`` through the row passes alone (no tile pass)."""
    s.tile_pass = False
    try:
        return s.sample_batch(*args)
    finally:
        s.tile_pass = True


def tile_max(logits: torch.Tensor) -> torch.Tensor:
    """The max of every TILE logits of each row (a NaN is the largest), fp32 [B, nT]."""
    B, V = logits.shape
    nT = (V + TILE - 1) // TILE
    x = torch.full((B, nT * TILE), -math.inf, dtype=torch.float32, device=logits.device)
    x[:, :V] = logits.float()
    return x.view(B, nT, TILE).amax(dim=2).contiguous()


def mixed_params(rng, B, V, penalties_every=0):
    """Every kind of row: greedy, top-k (some past the list's 256), min-p, both, top-p alone."""
    out = []
    for b in range(B):
        kind = b % 8
        kw = dict(temperature=float(rng.choice([0.3, 0.7, 1.0, 1.5])))
        if kind == 0:
            kw = dict(temperature=0.0)
        elif kind == 1:
            kw.update(top_k=int(rng.choice([1, 5, 20, 50, 256, 300])))
        elif kind == 2:
            kw.update(min_p=float(rng.choice([0.05, 0.3, 1.0])))
        elif kind == 3:
            kw.update(top_k=int(rng.choice([20, 50])), min_p=0.1, top_p=float(rng.choice([0.5, 0.9])))
        elif kind == 4:
            kw.update(top_p=0.9)  # (top-p alone: the row passes)
        elif kind == 5:
            kw.update(top_k=20, top_p=float(rng.choice([0.8, 1e-6])))
        elif kind == 6:
            kw.update(min_p=0.05, top_p=0.95)
        else:
            kw.update(top_k=int(rng.choice([1, 2, V - 1])))
        if penalties_every and b % penalties_every == penalties_every - 1:
            kw.update(repetition_penalty=1.3, frequency_penalty=0.5)
        out.append(SamplingParams(**kw))
    return out


def check(logits, params, seed, hist=None, label="", draft=None):
    B, V = logits.shape
    rng = np.random.default_rng(seed)
    s = hip()
    tm = tile_max(logits)
    pp = pack_params(params)
    u = torch.from_numpy(rng.random(B, dtype=np.float32))
    if draft is None:
        draft = torch.from_numpy(rng.integers(0, V, B).astype(np.int32))
    if hist is not None:
        hi, ho = pack_history(hist)
    else:
        hi = ho = None
    d = lambda t: None if t is None else t.to(DEV)  # noqa: E731
    print(f"sample_tiles {label} B={B} V={V}", flush=True)
    a, ap = s.sample_tiles(logits, tm, pp.to(DEV), d(u), d(hi), d(ho), d(draft))
    b, bp = row_passes(s, logits, pp.to(DEV), d(u), d(hi), d(ho), d(draft))
    c, cp = s.sample_batch(logits, pp.to(DEV), d(u), d(hi), d(ho), d(draft))  # (a small batch: the tile pass)
    torch.cuda.synchronize()
    assert torch.equal(a.cpu(), b.cpu()), (label, a.cpu(), b.cpu())
    assert torch.equal(ap.cpu().view(torch.int32), bp.cpu().view(torch.int32)), label
    assert torch.equal(c.cpu(), b.cpu()) and torch.equal(cp.cpu().view(torch.int32), bp.cpu().view(torch.int32)), label
    w = Workload(label, logits.cpu(), pp, u, hi, ho, draft)
    ties, bad = compare_ids(a.cpu(), oracle(w), ap.cpu())
    assert not bad, (label, bad[:10])
    return a


def lm_logits(seed, B, d, V, peaked=0.0):
    """bf16 logits of vsamp_lm_head; with `peaked` > 0 each hidden row is that multiple of one
    weight row plus noise, so one logit stands far above the rest."""
    g = torch.Generator().manual_seed(seed)
    weight = (torch.randn(V, d, generator=g) / math.sqrt(d) * 4).to(torch.bfloat16)
    hidden = torch.randn(B, d, generator=g) * 0.5
    if peaked:
        rows = torch.randint(0, V, (B,), generator=g)
        hidden = hidden * 0.1 + peaked * weight[rows].float()
    logits, tmax, _ = hip().lm_head(hidden.to(torch.bfloat16).to(DEV), weight.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(tmax, tile_max(logits))  # (the kernel's maxima are the rows' own)
    return logits


@pytest.mark.gpu
@pytest.mark.parametrize("B,d,V,peaked", [(16, 512, 20000, 0.0), (32, 1024, 151936, 0.0), (64, 4096, 151936, 3.0),
                                          (8, 256, 300, 0.0), (1, 4096, 151936, 3.0)])
def test_gpu_sample_tiles_on_lm_head_logits(B, d, V, peaked):
    logits = lm_logits(B * 7 + V, B, d, V, peaked)
    rng = np.random.default_rng(B + V)
    check(logits, mixed_params(rng, B, V), B + d, label=f"lm_head peaked={peaked}")


@pytest.mark.gpu
def test_gpu_sample_tiles_with_penalties_and_histories():
    # rows with penalties take the row passes; rows without them in the same launch do not
    B, d, V = 24, 1024, 151936
    logits = lm_logits(5, B, d, V)
    rng = np.random.default_rng(9)
    hist = [rng.integers(-2, V + 2, int(rng.integers(0, 300))).tolist() for _ in range(B)]
    check(logits, mixed_params(rng, B, V, penalties_every=3), 11, hist=hist, label="penalties")


@pytest.mark.gpu
def test_gpu_sample_tiles_on_crafted_rows():
    V = 4099  # 33 tiles, the last one partial
    g = torch.Generator().manual_seed(3)
    rows = []
    base = torch.randn(V, generator=g)
    # the max in three tiles: greedy takes the first of them
    x = base.clone()
    x[[700, 300, 4098]] = 9.0
    rows.append(x)
    # the max is zero, +0 in a late tile and -0 in an earlier one (equal values)
    x = -base.abs() - 1.0
    x[2000] = 0.0
    x[129] = -0.0
    rows.append(x)
    rows.append(torch.full((V,), -math.inf))  # every logit -inf
    x = base.clone()
    x[1500] = float("nan")  # a NaN: the row passes
    rows.append(x)
    x = base.clone()
    x[17] = math.inf  # an infinite logit
    rows.append(x)
    rows.append(torch.full((V,), 0.25))  # one value everywhere
    x = (base * 0.01).clone()  # a few values, massive ties at every boundary
    rows.append(x)
    x = base.clone()
    x[:300] = 5.0  # 300 equal values above the rest: a top-k 20 boundary inside the tie
    rows.append(x)
    logits = torch.stack(rows).to(torch.bfloat16).to(DEV)
    B = logits.shape[0]
    for T, kw in [(0.0, {}), (1.0, dict(top_k=20)), (0.7, dict(min_p=0.3)), (1.2, dict(top_k=5, min_p=0.05)),
                  (1.0, dict(top_k=1)), (0.5, dict(top_k=20, top_p=0.5))]:
        params = [SamplingParams(temperature=T, **kw) for _ in range(B)]
        check(logits, params, int(T * 10) + len(kw), label=f"crafted T={T} {kw}")


@pytest.mark.gpu
@pytest.mark.parametrize("V", [4099, 8192])
def test_gpu_partial_cutoff_member_then_draw(V):
    # Rows of massive ties whose top-p cutoff splits a group of equal values, each with a draft
    # id inside that group: the row finds the group's r-th member (the draft's probability needs
    # it) and then the draw's member, two member searches in one workgroup through the same LDS
    # result word. Unaligned rows (V = 4099) search their elements one by one, aligned ones from
    # the low bytes kept in registers. Every row against the row passes, the tile pass and the
    # oracle.
    g = torch.Generator().manual_seed(11)
    B = 48
    rows, drafts = [], []
    for b in range(B):
        kind = b % 3
        if kind == 0:
            x = torch.full((V,), 0.25)  # one value: the cutoff inside it
        elif kind == 1:
            x = torch.randn(V, generator=g)
            x[: 300 + b] = 5.0  # a tied group above the rest, the cutoff inside it
        else:
            x = (torch.randn(V, generator=g) * 0.01).clone()  # a few values, ties at every boundary
            x[b % 97 : b % 97 + 600] = 0.0390625
        rows.append(x)
        drafts.append(b % 150)  # (inside the kept part of the tied group)
    logits = torch.stack(rows).to(torch.bfloat16).to(DEV)
    draft = torch.tensor(drafts, dtype=torch.int32)
    for T, kw in [(0.5, dict(top_k=20, top_p=0.5)), (1.0, dict(top_p=0.3)), (0.8, dict(top_k=400, top_p=0.4))]:
        params = [SamplingParams(temperature=T, **kw) for _ in range(B)]
        check(logits, params, 7 + len(kw), label=f"partial V={V} T={T} {kw}", draft=draft)


@pytest.mark.gpu
def test_gpu_sample_tiles_rejects_bad_arguments():
    s = hip()
    logits = torch.zeros(2, 1000, dtype=torch.bfloat16, device=DEV)
    pp = pack_params([SamplingParams(), SamplingParams()], DEV)
    u = torch.zeros(2, dtype=torch.float32, device=DEV)
    with pytest.raises(ValueError, match="tile_max"):
        s.sample_tiles(logits, torch.zeros(2, 7, device=DEV), pp, u)
    with pytest.raises(ValueError, match="bf16"):
        s.sample_tiles(logits.float(), torch.zeros(2, 8, device=DEV), pp, u)


@pytest.mark.gpu
@pytest.mark.parametrize("B,V,pad,offset,dtype", [
    (1, 151936, 0, 0, torch.bfloat16), (3, 4099, 5, 0, torch.bfloat16), (8, 151936, 0, 3, torch.bfloat16),
    (16, 20000, 0, 0, torch.bfloat16), (2, 100, 0, 1, torch.bfloat16), (16, 151936, 0, 0, torch.bfloat16),
    (13, 151936, 0, 1, torch.bfloat16),
    (1, 151936, 0, 0, torch.float32), (3, 4099, 5, 0, torch.float32), (8, 151936, 0, 3, torch.float32),
    (2, 100, 0, 1, torch.float32), (14, 151936, 0, 0, torch.float32), (13, 151936, 0, 2, torch.float32)])
def test_gpu_tile_pass_equals_sample_batch(B, V, pad, offset, dtype):
    # logits from any source: the tile maxima computed by the same launch while B times the
    # workgroups per row fits one round on the CUs (B <= 13 at V = 151936), else by their own
    # launch first (rows not 16-byte aligned when offset is not a multiple of 16 bytes: the
    # maxima are read element by element); against the row passes and the oracle
    g = torch.Generator().manual_seed(B * 7 + V)
    rng = np.random.default_rng(V + B)
    x = torch.randn(B, V, generator=g) * 2.0
    x[:, :5] += 8.0
    buf = torch.zeros(B * (V + pad) + offset + 8, dtype=dtype)
    view = buf[offset : offset + B * (V + pad)].view(B, V + pad)[:, :V]
    view.copy_(x.to(dtype))
    logits = buf.to(DEV)[offset : offset + B * (V + pad)].view(B, V + pad)[:, :V]
    params = mixed_params(rng, B, V, penalties_every=4)
    hist = [rng.integers(0, V, 50).tolist() for _ in range(B)]
    hi, ho = pack_history(hist)
    pp = pack_params(params)
    u = torch.from_numpy(rng.random(B, dtype=np.float32))
    draft = torch.from_numpy(rng.integers(0, V, B).astype(np.int32))
    s = hip()
    print(f"tile pass B={B} V={V} pad={pad} offset={offset} {dtype}", flush=True)
    d = lambda t: t.to(DEV)  # noqa: E731
    a, ap = s.sample_tile_pass(logits, pp.to(DEV), d(u), d(hi), d(ho), d(draft))
    b, bp = row_passes(s, logits, pp.to(DEV), d(u), d(hi), d(ho), d(draft))
    torch.cuda.synchronize()
    # (small batches run one launch whose rows' last workgroups reset the arrival words)
    assert not s._local.tiles[DEV][1].any()
    assert torch.equal(a.cpu(), b.cpu())
    assert torch.equal(ap.cpu().view(torch.int32), bp.cpu().view(torch.int32))
    w = Workload("tile pass", logits.cpu(), pp, u, hi, ho, draft)
    ties, bad = compare_ids(a.cpu(), oracle(w), ap.cpu())
    assert not bad, bad[:10]


@pytest.mark.gpu
def test_gpu_per_token_call_through_the_tile_pass():
    # the engine's per-token call on bf16 rows with parameters the tile maxima decide (it takes
    # the tile pass) against the batched call on the same row and uniform
    from vinfer_amd.sampling import uniform

    s = hip()
    V = 151936
    g = torch.Generator().manual_seed(17)
    row = (torch.randn(V, generator=g) * 2).to(torch.bfloat16).to(DEV)
    cases = [SamplingParams(temperature=0.7, top_k=20, top_p=0.8), SamplingParams(temperature=0.0),
             SamplingParams(temperature=1.0, min_p=0.2, top_p=0.95), SamplingParams(temperature=1.3, top_k=256),
             SamplingParams(temperature=0.9, top_k=300)]
    print("per-token call through the tile pass", flush=True)
    for r in (row, (torch.randn(V, generator=g) * 2).to(DEV)):  # (bf16, then fp32)
        for ci, sp in enumerate(cases):
            for pos in range(6):
                tok = s.sample(r, sp, 3 + ci, pos)
                u = torch.tensor([uniform(3 + ci, pos)], dtype=torch.float32, device=DEV)
                want, _ = row_passes(s, r.view(1, V), pack_params([sp], DEV), u)
                assert tok == int(want[0]), (r.dtype, ci, pos)


@pytest.mark.gpu
def test_gpu_tile_pass_on_crafted_fp32_rows():
    # fp32 rows whose values bf16 cannot hold: ties of the max across tiles below bf16's
    # resolution, signed zeros, -inf, NaN and +inf rows, a top-k boundary inside a tie of 300
    V = 4099
    g = torch.Generator().manual_seed(5)
    base = torch.randn(V, generator=g, dtype=torch.float64).float()
    rows = []
    x = base.clone()
    x[[700, 300, 4098]] = 9.000001
    x[301] = 9.0  # (just below the max: one fp32 ulp apart)
    rows.append(x)
    x = -base.abs() - 1.0
    x[2000] = 0.0
    x[129] = -0.0
    rows.append(x)
    rows.append(torch.full((V,), -math.inf))
    x = base.clone()
    x[1500] = float("nan")
    rows.append(x)
    x = base.clone()
    x[17] = math.inf
    rows.append(x)
    x = base * 1e-6  # values packed into a tiny range: many tiles' maxima within a few ulps
    rows.append(x)
    x = base.clone()
    x[:300] = 5.0
    rows.append(x)
    logits = torch.stack(rows).to(DEV)
    B = logits.shape[0]
    s = hip()
    rng = np.random.default_rng(2)
    for T, kw in [(0.0, {}), (1.0, dict(top_k=20)), (0.7, dict(min_p=0.3)), (1.2, dict(top_k=5, min_p=0.05)),
                  (1.0, dict(top_k=1)), (0.5, dict(top_k=20, top_p=0.5)), (0.9, dict(top_k=256))]:
        params = [SamplingParams(temperature=T, **kw) for _ in range(B)]
        pp = pack_params(params)
        u = torch.from_numpy(rng.random(B, dtype=np.float32))
        draft = torch.from_numpy(rng.integers(0, V, B).astype(np.int32))
        print(f"crafted fp32 T={T} {kw}", flush=True)
        a, ap = s.sample_tile_pass(logits, pp.to(DEV), u.to(DEV), None, None, draft.to(DEV))
        b, bp = row_passes(s, logits, pp.to(DEV), u.to(DEV), None, None, draft.to(DEV))
        torch.cuda.synchronize()
        assert torch.equal(a.cpu(), b.cpu()), (T, kw, a.cpu(), b.cpu())
        assert torch.equal(ap.cpu().view(torch.int32), bp.cpu().view(torch.int32)), (T, kw)
        w = Workload("crafted fp32", logits.cpu(), pp, u, None, None, draft)
        ties, bad = compare_ids(a.cpu(), oracle(w), ap.cpu())
        assert not bad, (T, kw, bad[:10])


@pytest.mark.gpu
def test_gpu_tile_pass_random_shapes_and_parameters():
    # seeded random batches of either dtype, vocabularies with ragged last tiles, peaked and flat
    # rows, every kind of parameters: the tile pass against the row passes, and the oracle
    s = hip()
    rng = np.random.default_rng(2024)
    for case in range(24):
        dtype = torch.float32 if case % 2 else torch.bfloat16
        B = int(rng.integers(1, 14))
        V = int(rng.choice([int(rng.integers(100, 5000)), int(rng.integers(5000, 60000)), 151936]))
        scale = float(rng.choice([0.01, 1.0, 3.0]))
        g = torch.Generator().manual_seed(case)
        x = torch.randn(B, V, generator=g) * scale
        peaked = rng.random(B) < 0.3
        for b in np.nonzero(peaked)[0]:
            x[b, int(rng.integers(0, V))] += 12.0
        logits = x.to(dtype).to(DEV)
        params = mixed_params(rng, B, V)
        pp = pack_params(params)
        u = torch.from_numpy(rng.random(B, dtype=np.float32))
        draft = torch.from_numpy(rng.integers(0, V, B).astype(np.int32))
        print(f"random tile pass case {case}: B={B} V={V} {dtype} scale={scale}", flush=True)
        a, ap = s.sample_tile_pass(logits, pp.to(DEV), u.to(DEV), None, None, draft.to(DEV))
        b, bp = row_passes(s, logits, pp.to(DEV), u.to(DEV), None, None, draft.to(DEV))
        torch.cuda.synchronize()
        assert torch.equal(a.cpu(), b.cpu()), (case, a.cpu(), b.cpu())
        assert torch.equal(ap.cpu().view(torch.int32), bp.cpu().view(torch.int32)), case
        w = Workload("random tile pass", logits.cpu(), pp, u, None, None, draft)
        ties, bad = compare_ids(a.cpu(), oracle(w), ap.cpu())
        assert not bad, (case, bad[:10])


@pytest.mark.gpu
def test_gpu_prepared_launches_equal_the_calls():
    # prepare_tiles (sample_tiles on fixed buffers) and prepare_batch on a small batch (the
    # one-launch tile pass on its own maxima and arrival words), each launched three times with
    # the logits (and the maxima) rewritten in place between launches: the same ids and draft
    # probabilities as the one-off calls on those logits
    s = hip()
    B, V = 8, 151936
    g = torch.Generator().manual_seed(21)
    rng = np.random.default_rng(21)
    logits = torch.empty(B, V, dtype=torch.bfloat16, device=DEV)
    tm = torch.empty(B, (V + TILE - 1) // TILE, dtype=torch.float32, device=DEV)
    pp = pack_params(mixed_params(rng, B, V), DEV)
    u = torch.from_numpy(rng.random(B, dtype=np.float32)).to(DEV)
    draft = torch.from_numpy(rng.integers(0, V, B).astype(np.int32)).to(DEV)
    st_tiles = s.prepare_tiles(logits, tm, pp, u, None, None, draft)
    st_batch = s.prepare_batch(logits, pp, u, None, None, draft)
    for rep in range(3):
        x = torch.randn(B, V, generator=g) * float(rng.choice([0.5, 2.0, 4.0]))
        x[rep % B, 1234] = 30.0  # (a peaked row)
        logits.copy_(x.to(torch.bfloat16).to(DEV))
        tm.copy_(tile_max(logits))
        print(f"prepared launches rep {rep}", flush=True)
        st_tiles.launch()
        st_batch.launch()
        torch.cuda.synchronize()
        a, ap = st_tiles.ids.clone(), st_tiles.draft_prob.clone()
        b, bp = st_batch.ids.clone(), st_batch.draft_prob.clone()
        want, wantp = row_passes(s, logits, pp, u, None, None, draft)
        c, cp = s.sample_tiles(logits, tm, pp, u, None, None, draft)
        torch.cuda.synchronize()
        for ids, dp in ((a, ap), (b, bp), (c, cp)):
            assert torch.equal(ids, want), rep
            assert torch.equal(dp.view(torch.int32), wantp.view(torch.int32)), rep
