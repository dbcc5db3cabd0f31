"""Device parity: the ``hip`` backend, called through the C ABI, against the CPU oracle.

Token ids must be identical on every row the oracle does not classify as a tie; greedy ids and
penalty counts always; probabilities within 1e-5 relative (fp32 output of fp64 math)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.sampler_oracle import classify_ties, penalize
from tests.parity import compare_ids, oracle
from vinfer_amd import _lib, workloads
from vinfer_amd.registry import BackendContext
from vinfer_amd.sampler import SAMPLER
from vinfer_amd.sampling import SamplingParams, pack_history, pack_params, uniform
from vinfer_amd.workloads import Workload

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
PROB_RTOL = 1e-5


def hip(dtype=torch.bfloat16):
    return SAMPLER.resolve("hip", BackendContext(DEV, dtype))


def run(w: Workload):
    d = w.to(DEV)
    s = hip(w.logits.dtype)
    ids, dp = s.sample_batch(d.logits, d.params, d.uniforms, d.hist_ids, d.hist_offsets, d.draft_ids)
    torch.cuda.synchronize()
    return ids.cpu(), None if dp is None else dp.cpu()


def check(w: Workload, max_tie_frac: float = 0.05):
    print(f"case {w.name} B={w.batch} V={w.vocab} dtype={w.logits.dtype}", flush=True)
    ids, dp = run(w)
    res = oracle(w)
    ties, bad = compare_ids(ids, res, dp)
    assert not bad, bad[:10]
    assert ties <= max(1, max_tie_frac * w.batch), (ties, w.batch)
    return ties


def random_workload(seed, B, V, dtype, penalties=True, hist_len=64, name="random") -> Workload:
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, V, generator=g) * float(rng.choice([0.5, 2.0, 3.0]))).to(dtype)
    params = [
        SamplingParams(
            temperature=float(rng.choice([0.0, 0.3, 0.7, 1.0, 1.5])),
            top_k=int(rng.choice([0, 0, 1, 5, 50, V - 1, V, V + 7])),
            top_p=float(rng.choice([1.0, 1.0, 0.5, 0.9, 0.99, 1e-6])),
            min_p=float(rng.choice([0.0, 0.0, 0.05, 0.3, 1.0])),
            repetition_penalty=float(rng.choice([1.0, 1.05, 1.3])) if penalties else 1.0,
            presence_penalty=float(rng.choice([0.0, 0.5, -0.5])) if penalties else 0.0,
            frequency_penalty=float(rng.choice([0.0, 0.2, 1.0])) if penalties else 0.0,
        )
        for _ in range(B)
    ]
    hist = [rng.integers(-2, V + 2, int(rng.integers(0, hist_len + 1))).tolist() for _ in range(B)]
    hi, ho = pack_history(hist)
    u = torch.from_numpy(rng.random(B, dtype=np.float32))
    draft = torch.from_numpy(rng.integers(0, V, B).astype(np.int32))
    return Workload(name, x, pack_params(params), u, hi, ho, draft)


def test_device_is_supported():
    assert _lib.query(0) is None
    assert SAMPLER.unsupported("hip", BackendContext(DEV, torch.bfloat16)) is None


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("V", [1, 6, 96, 1000, 4099, 20000])
def test_random_rows_match_the_oracle(dtype, V):
    check(random_workload(V, 48, V, dtype), max_tie_frac=0.1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_probabilities_match_the_oracle(dtype):
    w = random_workload(7, 32, 3000, dtype)
    d = w.to(DEV)
    pr = hip(dtype).probs(d.logits, d.params, d.hist_ids, d.hist_offsets).cpu().double().numpy()
    for b, r in enumerate(oracle(w, want_probs=True)):
        if classify_ties(r):
            continue
        assert ((pr[b] > 0) == r.kept).all(), b
        np.testing.assert_allclose(pr[b], r.probs, rtol=PROB_RTOL, atol=1e-30)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_long_history_counts_are_exact(dtype):
    # histories past the hash table's length: counted through a presence bitmap of the
    # vocabulary, or in windows of ids when the distinct ids do not fit beside it (60000 here)
    V = 151936
    rng = np.random.default_rng(8)
    w = random_workload(4, 4, V, dtype, hist_len=10)
    perm = rng.permutation(V)
    hist = [
        workloads.zipf_ids(rng, 20000, V, 1.05, perm).tolist(),
        rng.permutation(V)[:60000].tolist(),  # 60000 distinct ids
        (workloads.zipf_ids(rng, 30000, V, 1.1, perm).tolist() + [-3, V, V + 9]),
        rng.integers(0, V, 65535).tolist(),
    ]
    w.hist_ids, w.hist_offsets = pack_history(hist)
    p = w.params
    p.presence_penalty.fill_(0.5)
    d = w.to(DEV)
    xs, counts = hip(dtype).penalized_logits(d.logits, d.params, d.hist_ids, d.hist_offsets)
    xs, counts = xs.cpu().numpy(), counts.cpu().numpy()
    for b in range(w.batch):
        x, c = penalize(w.logits[b].float().numpy(), np.array(hist[b]), float(p.repetition_penalty[b]),
                        float(p.presence_penalty[b]), float(p.frequency_penalty[b]))
        assert np.array_equal(counts[b], c), b
        assert np.array_equal(xs[b].view(np.uint32), x.view(np.uint32)), b
    check(w, max_tie_frac=0.5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_penalty_counts_and_values_are_exact(dtype):
    w = random_workload(3, 16, 5000, dtype, hist_len=3000)
    # one row with a single id repeated far past 2^16
    hist = [list(range(5)) * 3] * 15 + [[17] * 70000 + [4999, -1, 5000]]
    w.hist_ids, w.hist_offsets = pack_history(hist)
    d = w.to(DEV)
    xs, counts = hip(dtype).penalized_logits(d.logits, d.params, d.hist_ids, d.hist_offsets)
    xs, counts = xs.cpu().numpy(), counts.cpu().numpy()
    p = w.params
    for b in range(w.batch):
        h = np.array(hist[b])
        x, c = penalize(
            w.logits[b].float().numpy(),
            h,
            float(p.repetition_penalty[b]),
            float(p.presence_penalty[b]),
            float(p.frequency_penalty[b]),
        )
        assert np.array_equal(counts[b], c), b
        if p.repetition_penalty[b] != 1 or p.presence_penalty[b] != 0 or p.frequency_penalty[b] != 0:
            assert np.array_equal(xs[b].view(np.uint32), x.view(np.uint32)), b
        else:
            assert np.array_equal(xs[b], w.logits[b].float().numpy()), b


def csr_as_ranges(hist_ids: torch.Tensor, hist_offsets: torch.Tensor, seed: int = 0):
    """The same histories as per-row [start, end) ranges into a larger buffer: rows placed in a
    shuffled order with gaps of junk ids between them."""
    rng = np.random.default_rng(seed)
    off = hist_offsets.tolist()
    B = len(off) - 1
    buf, ranges = [], [None] * B
    for b in rng.permutation(B):
        buf += rng.integers(0, 50, int(rng.integers(0, 5))).tolist()  # junk between rows
        ranges[b] = (len(buf), len(buf) + off[b + 1] - off[b])
        buf += hist_ids[off[b] : off[b + 1]].tolist()
    buf += [7, 7, 7]
    return torch.tensor(buf, dtype=torch.int32), torch.tensor(ranges, dtype=torch.int32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_history_ranges_give_the_csr_results(dtype):
    # 151936 (bf16: the fast path's presence bitmap) and 200000 (its hash table; fp32 and the
    # penalty workspace throughout), with histories up to 5000 ids
    for V, seed in ((151936, 21), (200000, 22)):
        w = random_workload(seed, 24, V, dtype, hist_len=5000)
        rid, rng_ = csr_as_ranges(w.hist_ids, w.hist_offsets, seed)
        d = w.to(DEV)
        s = hip(dtype)
        print(f"ranges vs CSR V={V} {dtype}", flush=True)
        a = s.sample_batch(d.logits, d.params, d.uniforms, d.hist_ids, d.hist_offsets, d.draft_ids)
        b = s.sample_batch(d.logits, d.params, d.uniforms, rid.to(DEV), rng_.to(DEV), d.draft_ids)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
        pa = s.probs(d.logits, d.params, d.hist_ids, d.hist_offsets)
        pb = s.probs(d.logits, d.params, rid.to(DEV), rng_.to(DEV))
        assert torch.equal(pa, pb)
        xa, ca = s.penalized_logits(d.logits, d.params, d.hist_ids, d.hist_offsets)
        xb, cb = s.penalized_logits(d.logits, d.params, rid.to(DEV), rng_.to(DEV))
        assert torch.equal(ca, cb) and torch.equal(xa.view(torch.int32), xb.view(torch.int32))
        ties, bad = compare_ids(b[0].cpu(), oracle(w), b[1].cpu())
        assert not bad, bad[:10]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_history_append_writes_each_draw_behind_its_range(dtype):
    """VSAMP_HIST_APPEND: the same draws as without it, each row's id written at its range's end
    and nothing else of the buffer changed. Histories sit in per-slot regions in a shuffled
    order, as the decode loop keeps them (fast path and hash table at 151936 / 200000 for bf16;
    the generic path for fp32)."""
    for V, seed in ((151936, 31), (200000, 32)):
        w = random_workload(seed, 24, V, dtype, hist_len=3000)
        off = w.hist_offsets.tolist()
        B = w.batch
        cap = max(off[b + 1] - off[b] for b in range(B)) + 3
        buf = torch.full((B * cap,), -5, dtype=torch.int32)  # (ids outside [0, V) are ignored)
        ranges = [None] * B
        for slot, b in enumerate(np.random.default_rng(seed).permutation(B)):
            n = off[b + 1] - off[b]
            buf[slot * cap : slot * cap + n] = w.hist_ids[off[b] : off[b + 1]]
            ranges[b] = (slot * cap, slot * cap + n)
        d = w.to(DEV)
        s = hip(dtype)
        hb = buf.to(DEV)
        rg = torch.tensor(ranges, dtype=torch.int32, device=DEV)
        print(f"history append V={V} {dtype}", flush=True)
        a = s.sample_batch(d.logits, d.params, d.uniforms, hb, rg, d.draft_ids)
        hb2 = hb.clone()
        b_ = s.sample_batch(d.logits, d.params, d.uniforms, hb2, rg, d.draft_ids, append_history=True)
        assert torch.equal(a[0], b_[0]) and torch.equal(a[1], b_[1])
        want = hb.clone()
        want[rg[:, 1].long()] = a[0]
        assert torch.equal(hb2, want)


@pytest.mark.parametrize("name,B", [("mixed_bf16", 64), ("peaked_flat", 64), ("verify_bf16", 24), ("large_fp32", 12), ("single_fp32", 1)])
def test_workload_rows_match_the_oracle(name, B):
    check(workloads.make(name, batch=B), max_tie_frac=0.1)


def fp32_rule_ties(w: Workload, rows) -> int:
    """Rows of ``w`` on which the engine's own fp32 rule is ambiguous (oracle/fp32_rule.py)."""
    from oracle.fp32_rule import fp32_rule

    p, n = w.params, 0
    for b in rows:
        x = w.logits[b].float().numpy()
        if w.hist_ids is not None:
            h = w.hist_ids[int(w.hist_offsets[b]) : int(w.hist_offsets[b + 1])].numpy()
            x, _ = penalize(x, h, float(p.repetition_penalty[b]), float(p.presence_penalty[b]),
                            float(p.frequency_penalty[b]))
        n += bool(fp32_rule(x, float(p.temperature[b]), int(p.top_k[b]), float(p.top_p[b]),
                            float(p.min_p[b]), float(w.uniforms[b])).ties)
    return n


def test_headline_shape_full_batch():
    w = workloads.make("peaked_flat")
    ties = check(w, max_tie_frac=0.1)
    print(f"headline B=256: oracle ties {ties}, fp32-rule ties {fp32_rule_ties(w, range(w.batch))}", flush=True)


def check_subset(w: Workload, n: int, seed: int):
    """One launch over the whole batch; a seeded subset of ``n`` rows against the oracle."""
    print(f"case {w.name} full B={w.batch} V={w.vocab}, {n} rows checked", flush=True)
    ids, dp = run(w)
    rows = np.sort(np.random.default_rng(seed).choice(w.batch, n, replace=False))
    sub = Workload(w.name, w.logits[rows], w.params.select(torch.from_numpy(rows)), w.uniforms[rows],
                   *_sub_hist(w, rows), None if w.draft_ids is None else w.draft_ids[rows])
    res = oracle(sub)
    ties, bad = compare_ids(ids[rows], res, None if dp is None else dp[rows])
    assert not bad, bad[:10]
    assert ties <= max(1, 0.1 * n), ties
    return rows, ties


def _sub_hist(w: Workload, rows):
    if w.hist_ids is None:
        return None, None
    hs = [w.hist_ids[int(w.hist_offsets[b]) : int(w.hist_offsets[b + 1])].tolist() for b in rows]
    return pack_history(hs)


def test_large_fp32_full_launch():
    # 1024 x 151936 fp32 rows, histories up to 32768 ids, one launch: a 1024-workgroup grid and
    # the full-size history workspace; every row checked, and the exact counts of the 8 longest
    # histories
    w = workloads.make("large_fp32")
    check_subset(w, w.batch, seed=11)
    lens = (w.hist_offsets[1:] - w.hist_offsets[:-1]).numpy()
    longest = np.argsort(-lens, kind="stable")[:8]
    d = w.to(DEV)
    _, counts = hip(torch.float32).penalized_logits(d.logits, d.params, d.hist_ids, d.hist_offsets)
    got = counts[torch.from_numpy(longest).to(DEV)].cpu().numpy()
    for i, b in enumerate(longest):
        h = w.hist_ids[int(w.hist_offsets[b]) : int(w.hist_offsets[b + 1])].numpy()
        assert lens[b] > 30000
        assert (got[i] == np.bincount(h, minlength=w.vocab)).all(), int(b)


def test_verify_bf16_full_launch():
    # 192 x 262144 bf16 rows with draft probabilities, one launch; every row checked
    w = workloads.make("verify_bf16")
    check_subset(w, w.batch, seed=12)


def test_gpu_torch_division_by_a_scalar():
    # The engine runs sample() on the model's device: torch's GPU kernel computes
    # logits.float() / T (sampler.py:52) as x * fl32(1 / T), a reciprocal multiply, over every
    # bf16 value; its CPU kernel divides. The kernels divide (the CPU rule); the values where
    # the two differ are counted in tests/test_fp32_rule.py (RECIPROCAL_DIFFERS).
    x = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    xn = x.float().numpy()
    same = lambda a, b: (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))  # noqa: E731
    for T in (0.3, 0.5, 0.7, 0.8, 1.0, 1.2, 1.5):
        got = (x.to(DEV).float() / T).cpu().numpy()
        with np.errstate(all="ignore"):
            div = xn / np.float32(T)
            rec = (xn * (np.float32(1.0) / np.float32(T))).astype(np.float32)
        n_div, n_rec = int((~same(got, div)).sum()), int((~same(got, rec)).sum())
        print(f"T={T}: torch GPU differs from division on {n_div}, from the reciprocal multiply on {n_rec}",
              flush=True)
        assert n_rec == 0


def test_single_row_many_steps():
    # 200 steps of the single-row fp32 workload (new logits and uniform per step)
    for step in range(0, 200, 40):
        check(workloads.make("single_fp32", batch=40, seed=5000 + step))


def test_degenerate_rows():
    V = 37
    nan, inf = float("nan"), float("inf")
    rows = torch.randn(6, V)
    rows[0, 5] = nan
    rows[0, 9] = nan
    rows[1, 3] = inf
    rows[1, 30] = inf
    rows[2, :] = -inf
    rows[3, 11] = 3e38  # overflows to +inf at T = 1e-3
    rows[4, :] = 0.0  # all equal: top-p cutoff inside one group
    rows[5, 2] = nan
    params = pack_params(
        [
            SamplingParams(temperature=1.0, top_p=0.9),
            SamplingParams(temperature=0.7, top_k=3),
            SamplingParams(temperature=1.0, min_p=0.1),
            SamplingParams(temperature=1e-3),
            SamplingParams(temperature=1.0, top_p=0.4),
            SamplingParams(temperature=0.0),
        ]
    )
    u = torch.tensor([0.3, 0.9, 0.5, 0.5, 0.99, 0.1])
    for dtype in (torch.float32, torch.bfloat16):
        w = Workload("degenerate", rows.to(dtype), params, u, None, None, torch.arange(6, dtype=torch.int32))
        ids, _ = run(w)
        assert ids.tolist() == [r.token for r in oracle(w)]
        assert ids.tolist()[:3] == [5, 3, 0] and ids.tolist()[5] == 2


def _colliding_ids(V: int, first_bucket: int, buckets: int, per_bucket: int) -> list[int]:
    """Ids whose 4096-slot Fibonacci hash lands in `buckets` consecutive buckets, `per_bucket`
    of each: inserted together they form one long probe run in the kernel's history table."""
    h = (np.arange(V, dtype=np.uint64) * np.uint64(2654435761)) % np.uint64(1 << 32) >> np.uint64(20)
    out = []
    for b in range(first_bucket, first_bucket + buckets):
        out += np.flatnonzero(h == b)[:per_bucket].tolist()
    return out


@pytest.mark.parametrize("V", [4096, 151936])
def test_signed_zeros_are_one_value(V):
    # -0.0 and +0.0 are one value: the bf16 histogram counts them under one key (a count past
    # 65535 sends the row to the generic path), and the member search takes both bit patterns
    rng = np.random.default_rng(17)
    B = 8
    x = (torch.randn(B, V, generator=torch.Generator().manual_seed(17)) * 0.5).to(torch.bfloat16)
    zero = torch.from_numpy(rng.random((B, V)) < 0.5)
    sign = torch.from_numpy(rng.random((B, V)) < 0.5)
    z = torch.where(sign, torch.tensor(-0.0), torch.tensor(0.0)).to(torch.bfloat16)
    x = torch.where(zero, z, x)
    x[1] = torch.where(sign[1], torch.tensor(-0.0), torch.tensor(0.0)).to(torch.bfloat16)  # all zero
    x[2] = torch.full((V,), -0.0).to(torch.bfloat16)  # all -0.0 but one +0.0
    x[2, V // 3] = 0.0
    x[3] = -x[3].abs()  # max 0 (either sign): greedy takes the first zero
    params = pack_params(
        [SamplingParams(temperature=float(t), top_p=float(tp), presence_penalty=0.5)
         for t, tp in zip([1.0, 1.0, 1.0, 0.0, 0.7, 1.0, 0.0, 1.3], [0.9, 1.0, 0.5, 1.0, 0.95, 0.3, 1.0, 0.99])]
    )
    hist = [rng.integers(0, V, 50).tolist() for _ in range(B)]
    hi, ho = pack_history(hist)
    u = torch.from_numpy(rng.random(B, dtype=np.float32))
    check(Workload("signed_zero", x, params, u, hi, ho, None), max_tie_frac=0.5)


def test_few_penalised_values_inside_the_walked_chunk():
    # every logit is one of the 64 bf16 values 1 + k/128 (one chunk of 64 keys), so the cutoff
    # and draw walks both run in that chunk; three penalised ids move by 2^-9 and stay in it, at
    # keys whose lanes lie past the penalised list's length (the walk's per-key counts are then
    # written only by other lanes)
    rng = np.random.default_rng(5)
    B, V = 16, 2048
    vals = (1.0 + np.arange(64) / 128.0).astype(np.float32)
    x = torch.from_numpy(vals[rng.integers(0, 64, (B, V))]).to(torch.bfloat16)
    hist = []
    for _ in range(B):
        k = rng.integers(16, 60, 3)  # value indices: mid-chunk keys
        ids = [int(rng.choice(np.flatnonzero(np.isclose(x[len(hist)].float().numpy(), vals[i])))) for i in k]
        hist.append(ids)
    hi, ho = pack_history(hist)
    params = pack_params(
        [SamplingParams(temperature=1.0, top_p=float(rng.choice([0.3, 0.5, 0.8])), presence_penalty=2.0**-9)
         for _ in range(B)]
    )
    u = torch.from_numpy(rng.random(B, dtype=np.float32))
    check(Workload("walk_chunk", x, params, u, hi, ho, None), max_tie_frac=0.25)


@pytest.mark.parametrize("shift", ["frequency", "presence"])
def test_many_penalised_values_share_the_walked_keys(shift):
    # every logit is one of the 64 bf16 values 1 + k/128 (one chunk), and about 100 distinct
    # ids per row are penalised, so the top-k count, top-p cutoff and draw walks all land on keys
    # that hold the bf16 value together with penalised values: a frequency penalty of 2^-10 per
    # occurrence leaves up to three distinct fp32 values inside the key below (above its bf16
    # value); a presence penalty of 2^-7 moves values exactly onto the next bf16 value down
    rng = np.random.default_rng(17 if shift == "frequency" else 18)
    B, V = 32, 2048
    vals = (1.0 + np.arange(64) / 128.0).astype(np.float32)
    x = torch.from_numpy(vals[rng.integers(0, 64, (B, V))]).to(torch.bfloat16)
    hist = []
    for _ in range(B):
        ids = rng.permutation(V)[:100]
        reps = rng.integers(1, 4, ids.size)
        hist.append(np.repeat(ids, reps).tolist())
    hi, ho = pack_history(hist)
    freq, pres = (2.0**-10, 0.0) if shift == "frequency" else (0.0, 2.0**-7)
    params = pack_params(
        [SamplingParams(temperature=float(rng.choice([0.7, 1.0])), top_k=int(rng.choice([0, 0, 100, 700])),
                        top_p=float(rng.choice([0.3, 0.5, 0.8, 1.0])), presence_penalty=pres,
                        frequency_penalty=freq)
         for _ in range(B)]
    )
    u = torch.from_numpy(rng.random(B, dtype=np.float32))
    check(Workload(f"walk_keys_{shift}", x, params, u, hi, ho, None), max_tie_frac=0.5)


@pytest.mark.parametrize("n_pen", [60, 64, 65, 120, 128, 129])
def test_one_walked_key_holds_many_equal_penalised_values(n_pen):
    # four distinct bf16 values (1 + k/128, k = 0..3: one chunk); n_pen ids of value 1 + 3/128
    # are penalised by 2^-7 onto 1 + 2/128 exactly, so one key holds n_pen equal penalised values
    # (both halves of the walk's list past 64) merged with that bf16 value's own group; past 128
    # in the chunk the row goes to the generic path
    rng = np.random.default_rng(n_pen)
    B, V = 16, 4096
    vals = (1.0 + np.arange(4) / 128.0).astype(np.float32)
    xs = vals[rng.integers(0, 4, (B, V))]
    hist = []
    for b in range(B):
        top = np.flatnonzero(xs[b] == vals[3])
        hist.append(rng.choice(top, n_pen, replace=False).tolist())
    x = torch.from_numpy(xs).to(torch.bfloat16)
    hi, ho = pack_history(hist)
    params = pack_params(
        [SamplingParams(temperature=1.0, top_k=int(rng.choice([0, 0, 1500, 3000])),
                        top_p=float(rng.choice([0.2, 0.45, 0.7, 1.0])), presence_penalty=2.0**-7)
         for _ in range(B)]
    )
    u = torch.from_numpy(rng.random(B, dtype=np.float32))
    check(Workload(f"equal_penalised_{n_pen}", x, params, u, hi, ho, None), max_tie_frac=0.5)


@pytest.mark.parametrize("V", [200003, 262144, 300001])
def test_long_bf16_rows_search_their_later_blocks(V):
    # rows past the blocks whose low bytes the pass keeps (V > 155,648): the member search reads
    # a later block again only when its largest key reaches the drawn value's, and every block
    # past 270,336 ids; rows of 16 distinct values (members in every block), and N(0, s) rows
    # (the drawn value in the upper tail), greedy and sampled, with and without histories
    rng = np.random.default_rng(V)
    B = 24
    g = torch.Generator().manual_seed(V)
    x = torch.randn(B, V, generator=g) * 2.5
    x[::3] = torch.from_numpy(rng.integers(-8, 8, (len(range(0, B, 3)), V)).astype(np.float32) / 4.0)
    params = pack_params(
        [SamplingParams(temperature=float(rng.choice([0.0, 0.6, 1.0])), top_k=int(rng.choice([0, 0, 40])),
                        top_p=float(rng.choice([1.0, 0.95, 0.5])), repetition_penalty=float(rng.choice([1.0, 1.2])))
         for _ in range(B)]
    )
    hist = [rng.integers(0, V, int(rng.integers(0, 200))).tolist() for _ in range(B)]
    hi, ho = pack_history(hist)
    u = torch.from_numpy(rng.random(B, dtype=np.float32))
    check(Workload(f"long_rows_{V}", x.to(torch.bfloat16), params, u, hi, ho, None), max_tie_frac=0.25)


@pytest.mark.parametrize("V", [151936, 157248, 157249, 200000])  # presence bitmap up to 157248, then hash
def test_bf16_rows_the_histogram_path_hands_to_the_generic_path(V):
    # histories the bf16 histogram path does not count itself: longer than its table takes,
    # more distinct ids than its list holds, one probe run past its limit; beside normal rows
    # and histories of dense id ranges, the vocabulary's ends and ids outside it
    B = 10
    rng = np.random.default_rng(11)
    w = random_workload(21, B, V, torch.bfloat16, hist_len=100)
    hist = [rng.integers(0, V, 200).tolist() for _ in range(B)]
    hist[0] = list(range(2048)) + list(range(0, 2048, 3))  # dense: whole bitmap words
    hist[1] = rng.integers(0, V, 9000).tolist()  # longer than 8190 ids
    hist[2] = [0, V - 1, -5, V + 3, V - 1, 0, 2**31 - 1, 64, 63]
    hist[3] = rng.permutation(V)[:3000].tolist()  # 3000 distinct ids
    hist[4] = list(range(V - 2048, V)) * 3  # the top of the vocabulary, exactly the capacity
    hist[5] = _colliding_ids(V, 100, 72, 2) * 2  # a 144-slot probe run
    hist[6] = rng.permutation(V)[:2048].tolist() * 2  # exactly the list's capacity
    hist[8] = rng.permutation(V)[:2049].tolist()  # one past it
    w.hist_ids, w.hist_offsets = pack_history(hist)
    p = w.params
    for t in (p.repetition_penalty, p.presence_penalty, p.frequency_penalty):
        t.fill_(0.0)
    p.repetition_penalty.fill_(1.1)
    p.temperature[1::2] = 0.0  # greedy rows take the same paths
    check(w, max_tie_frac=0.25)


def test_unaligned_and_padded_rows():
    base = torch.randn(20, 1003)
    for dtype in (torch.bfloat16, torch.float32):
        x = base.to(dtype)[:, 1:1000]  # unaligned start, stride 1003
        params = pack_params([SamplingParams(temperature=0.8, top_p=0.9)] * 20)
        u = torch.rand(20)
        s = hip(dtype)
        ids, _ = s.sample_batch(x.to(DEV)[:, :], params.to(DEV), u.to(DEV))
        w = Workload("strided", x.contiguous(), params, u, None, None, None)
        ties, bad = compare_ids(ids, oracle(w))
        assert not bad


def test_temperature_division_merges_adjacent_fp32_values():
    # T = 3 maps pairs of adjacent fp32 values to one z; top-k keeps every element whose z
    # equals the kth z, which only a correctly rounded division reproduces.
    rng = np.random.default_rng(11)
    B, V = 32, 512
    base = rng.normal(0, 2, (B, V // 2)).astype(np.float32)
    x = np.concatenate([base, np.nextafter(base, np.float32(np.inf))], axis=1)
    x = np.ascontiguousarray(x[:, rng.permutation(V)])
    params = pack_params([SamplingParams(temperature=3.0, top_k=int(k)) for k in rng.integers(1, 60, B)])
    w = Workload("merge", torch.from_numpy(x), params, torch.from_numpy(rng.random(B, dtype=np.float32)), None, None, None)
    d = w.to(DEV)
    pr = hip(torch.float32).probs(d.logits, d.params).cpu().numpy()
    for b, r in enumerate(oracle(w, want_probs=True)):
        assert ((pr[b] > 0) == r.kept).all(), b


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
def test_small_top_k_lists_with_tied_values(dtype):
    # top-k candidate lists of at most 256 elements are sorted once and read by index (the K-th
    # value, the top-p cutoff group, the draw): rows of values on a 0.25 grid give groups of
    # equal values at the K-th value and at a cutoff that splits them, drafts sit inside those
    # groups, and the same rows' probabilities check the kept sets
    rng = np.random.default_rng(21)
    B, V = 96, 3000
    x = np.round(rng.normal(0, 2, (B, V)) * 4).astype(np.float32) / 4
    params = pack_params([
        SamplingParams(temperature=float(rng.choice([0.5, 1.0, 2.0])), top_k=int(rng.choice([1, 3, 10, 50, 200])),
                       top_p=float(rng.choice([1.0, 0.3, 0.6, 0.9])), min_p=float(rng.choice([0.0, 0.0, 0.05, 0.2])))
        for _ in range(B)])
    order = np.argsort(-x, axis=1, kind="stable")
    draft = torch.from_numpy(order[np.arange(B), rng.integers(0, 40, B)].astype(np.int32))
    w = Workload("sorted", torch.from_numpy(x).to(dtype), params, torch.from_numpy(rng.random(B, dtype=np.float32)),
                 None, None, draft)
    check(w, max_tie_frac=0.1)
    d = w.to(DEV)
    pr = hip(dtype).probs(d.logits, d.params).cpu().double().numpy()
    for b, r in enumerate(oracle(w, want_probs=True)):
        if classify_ties(r):
            continue
        assert ((pr[b] > 0) == r.kept).all(), b
        np.testing.assert_allclose(pr[b], r.probs, rtol=PROB_RTOL, atol=1e-30)


@pytest.mark.parametrize("order", ["ascending", "descending", "shuffled"])
def test_streamed_top_k_candidates_fall_back_on_ordered_rows(order):
    # fp32 rows with a small top-k take their candidates from a sample of the row's first
    # stripes: ascending rows (the sample holds the smallest values) overflow the staged list,
    # descending rows (it holds the largest) stage fewer than K; both fall back to counting the
    # row and a candidate pass, and must give the oracle's ids
    rng = np.random.default_rng(31)
    B, V = 12, 151936
    x = rng.normal(0, 2, (B, V)).astype(np.float32)
    if order == "ascending":
        x.sort(axis=1)
    elif order == "descending":
        x = -np.sort(-x, axis=1)
    params = pack_params([SamplingParams(temperature=float(rng.choice([0.7, 1.0])), top_k=int(k), top_p=0.9)
                          for k in rng.choice([5, 50, 300], B)])
    draft = torch.from_numpy(rng.integers(0, V, B).astype(np.int32))
    w = Workload("ordered", torch.from_numpy(np.ascontiguousarray(x)), params,
                 torch.from_numpy(rng.random(B, dtype=np.float32)), None, None, draft)
    check(w, max_tie_frac=0.1)


def test_draw_frequencies_match_the_distribution():
    # 20,000 draws of one row with the package's uniforms: TV < 0.015 (test_sampler.py:24-38)
    logits = torch.tensor([2.0, 1.0, 0.5, 0.0, -1.0, -3.0])
    for sp in (SamplingParams(), SamplingParams(temperature=0.5), SamplingParams(top_k=3), SamplingParams(top_p=0.8)):
        n = 20000
        params = pack_params([sp] * n).to(DEV)
        u = torch.tensor([uniform(1, p) for p in range(n)], dtype=torch.float32, device=DEV)
        s = hip(torch.float32)
        ids, _ = s.sample_batch(logits.expand(n, 6).contiguous().to(DEV), params, u)
        freq = torch.bincount(ids.long().cpu(), minlength=6).double() / n
        expected = s.probs(logits[None].to(DEV), pack_params([sp]).to(DEV))[0].double().cpu()
        assert 0.5 * (freq - expected).abs().sum() < 0.015


@pytest.mark.parametrize("pen", [False, True], ids=["plain", "penalties"])
def test_greedy_rows_take_the_first_of_repeated_maxima(pen):
    """Greedy bf16 rows whose max repeats: the first id holding it (the member search from the
    pass's kept low bytes, or the row pass), against the oracle; rows of signed zeros, a max
    only a penalised value reaches, and maxima in the ragged tail included."""
    from oracle.sampler_oracle import sample_batch as oracle_batch

    rng = np.random.default_rng(41 + pen)
    rows, V = [], 151939  # (a ragged tail of 3 elements)
    for b in range(24):
        x = rng.normal(0, 1, V).astype(np.float32)
        m = float(rng.choice([2.0, 3.5, 7.0]))
        k = int(rng.integers(1, 40))
        x[rng.choice(V, size=k, replace=False)] = m
        if b % 6 == 1:
            x[:] = 0.0
            x[rng.choice(V, size=V // 2, replace=False)] = -0.0
        if b % 6 == 2:
            x[V - 1] = m  # the last element (the tail) is one of the maxima
        rows.append(x)
    x = torch.from_numpy(np.stack(rows)).to(torch.bfloat16)
    B = x.shape[0]
    sp = SamplingParams(temperature=0.0, repetition_penalty=0.5 if pen else 1.0)  # (0.5: negative rows gain)
    hist = [rng.integers(0, V, 200).tolist() for _ in range(B)] if pen else [[] for _ in range(B)]
    hi, ho = pack_history(hist)
    u = torch.zeros(B)
    s = hip(torch.bfloat16)
    print(f"greedy repeated maxima pen={pen}", flush=True)
    ids, _ = s.sample_batch(x.to(DEV), pack_params([sp] * B, DEV), u.to(DEV), hi.to(DEV) if pen else None,
                            ho.to(DEV) if pen else None)
    xs = x.float().numpy()
    res = oracle_batch(xs, [0.0] * B, [0] * B, [1.0] * B, [0.0] * B, [sp.repetition_penalty] * B, [0.0] * B,
                       [0.0] * B, hi.numpy(), ho.numpy(), [0.0] * B)
    got = ids.cpu().tolist()
    assert got == [r.token for r in res]


def test_per_token_call_matches_the_batch():
    s = hip(torch.bfloat16)
    logits = (torch.randn(1000) * 2).to(torch.bfloat16).to(DEV)
    params = SamplingParams(temperature=0.9, top_p=0.9, repetition_penalty=1.2)
    hist = [1, 2, 3, 3, 999]
    for pos in range(10):
        tok = s.sample(logits, params, 7, pos, history=hist)
        u = torch.tensor([uniform(7, pos)], device=DEV)
        hi, ho = pack_history([hist], DEV)
        ids, _ = s.sample_batch(logits[None], pack_params([params], DEV), u, hi, ho)
        assert tok == int(ids[0])
    assert s.sample(torch.tensor([0.1, 3.0, -2.0], device=DEV), SamplingParams(temperature=0), 0, 0) == 1


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_per_token_call_matches_the_oracle(dtype):
    # the engine's unchanged call (generate.py:129) at the model's vocabulary, one row per call,
    # with penalties over a history passed as a list, a device int32 tensor (read in place), a
    # host int64 tensor and a device int64 tensor, against the oracle
    from oracle.sampler_oracle import sample_batch as oracle_batch

    s = hip(dtype)
    g = torch.Generator().manual_seed(5)
    V = 151936
    x = (torch.randn(V, generator=g) * 2).to(dtype)
    row = x.to(DEV)
    xs = x.float().numpy()
    cases = [
        (SamplingParams(temperature=0.7, top_k=20, top_p=0.8), []),
        (SamplingParams(temperature=1.0, top_p=0.95, min_p=0.05, repetition_penalty=1.05, presence_penalty=0.5,
                        frequency_penalty=0.2), list(range(0, 3000, 7)) + [5, 5, 5, V + 3, -1]),
        (SamplingParams(temperature=0.0, repetition_penalty=1.3), [int(np.argmax(xs))]),
    ]
    print(f"per-token call V={V} {dtype}", flush=True)
    for ci, (sp, hist) in enumerate(cases):
        for pos in range(8):
            h = [hist, torch.tensor(hist, dtype=torch.int32, device=DEV), torch.tensor(hist, dtype=torch.int64),
                 torch.tensor(hist, dtype=torch.int64, device=DEV)][pos % 4]
            tok = s.sample(row, sp, 11 + ci, pos, history=h if sp.penalized else None)
            hi = np.asarray(hist, dtype=np.int32)
            res = oracle_batch(xs[None], [sp.temperature], [sp.top_k], [sp.top_p], [sp.min_p],
                               [sp.repetition_penalty], [sp.presence_penalty], [sp.frequency_penalty],
                               hi, np.array([0, len(hi)], np.int32), [uniform(11 + ci, pos)])[0]
            if not classify_ties(res):
                assert tok == res.token, (ci, pos, tok, res.token)


def test_deterministic_and_stream_safe():
    w = workloads.make("mixed_bf16", batch=32).to(DEV)
    s = hip()
    a, _ = s.sample_batch(w.logits, w.params, w.uniforms, w.hist_ids, w.hist_offsets)
    st = torch.cuda.Stream(DEV)
    with torch.cuda.stream(st):
        b, _ = s.sample_batch(w.logits, w.params, w.uniforms, w.hist_ids, w.hist_offsets)
    st.synchronize()
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_errors_are_raised_not_swallowed():
    s = hip()
    x = torch.randn(4, 100, device=DEV).to(torch.bfloat16)
    p = pack_params([SamplingParams()] * 4, DEV)
    with pytest.raises(ValueError, match="uniforms"):
        s.sample_batch(x, p, torch.zeros(3, device=DEV))
    with pytest.raises(ValueError):
        s.sample_batch(x.half(), p, torch.zeros(4, device=DEV))
    assert math.isfinite(float(s.probs(x, p).sum()))


def _launch(a, lib):
    import ctypes

    _lib.check(lib.vsamp_sample(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)))


@pytest.mark.parametrize("pen", [False, True], ids=["plain", "penalties"])
@pytest.mark.parametrize("B,V,pad", [(1, 151936, 0), (1, 32768, 0), (3, 151939, 5), (17, 65536, 0),
                                     (64, 151936, 0), (128, 40000, 8), (8, 262144, 0)])
def test_split_rows_equal_whole_rows(B, V, pad, pen):
    # Small bf16 batches split each row over several workgroups of one launch when the workspace
    # holds the slice records (the row's last slice to arrive finishes it); with a workspace too
    # small for them the same call runs one workgroup per row. Both must draw the same ids (and
    # probabilities of the draft ids), bit for bit; and both match the oracle. Three launches in a
    # row on the same workspace: the arrival words left by one launch must not confuse the next.
    w = random_workload(B * 1000 + V + pen, B, V, torch.bfloat16, penalties=pen, hist_len=300 if pen else 0)
    w.params.top_k[::3] = 0  # (more rows through the top-p / min-p path)
    s = hip(torch.bfloat16)
    x = torch.zeros(B, V + pad, dtype=torch.bfloat16, device=DEV)
    x[:, :V] = w.logits.to(DEV)
    x = x[:, :V]  # row stride V + pad: a ragged vocabulary on 16-byte aligned rows
    d = w.to(DEV)
    print(f"split vs whole B={B} V={V} stride={V + pad} penalties={pen}", flush=True)
    hi, ho = (d.hist_ids, d.hist_offsets) if pen else (None, None)
    s.split_rows = True
    try:
        a, keep = s._args(x, d.params, hi, ho, d.uniforms, d.draft_ids)
    finally:
        s.split_rows = False
    assert a.flags & _lib.VSAMP_SPLIT_ROWS
    need = a.workspace_bytes
    assert need > 0  # (the slice records)
    lib = _lib.load()
    outs = []
    for ws in (True, True, False, True):
        ids = torch.full((B,), -1, dtype=torch.int32, device=DEV)
        dp = torch.full((B,), -1.0, dtype=torch.float32, device=DEV)
        a.out_ids, a.out_draft_prob = ids.data_ptr(), dp.data_ptr()
        # (one byte short of the records: the whole-row path, with the penalty part intact)
        a.workspace_bytes = need if ws else need - 1
        _launch(a, lib)
        torch.cuda.synchronize()
        outs.append((ids.cpu(), dp.cpu()))
    del keep
    i1, p1 = outs[0]
    for i2, p2 in outs[1:]:
        assert torch.equal(i1, i2) and torch.equal(p1.view(torch.int32), p2.view(torch.int32))
    ties, bad = compare_ids(i1, oracle(w), p1)
    assert not bad, bad[:10]


@pytest.mark.parametrize("pen", [False, True], ids=["plain", "penalties"])
def test_split_rows_replayed_from_a_graph(pen):
    # A HIP graph keeps the arguments of the launch it captured, the rows' arrival epoch among
    # them: each replay must still finish every row (the last slice sets the arrival count back
    # to 0 under that epoch). Three replays with new logits and uniforms each, eager work between
    # them, against whole-row launches of the same inputs and the oracle.
    B, V = 4, 151936
    s = hip(torch.bfloat16)
    w0 = random_workload(31 + pen, B, V, torch.bfloat16, penalties=pen, hist_len=300 if pen else 0)
    w0.params.top_k[::2] = 0
    d0 = w0.to(DEV)
    x = d0.logits.clone()
    u = d0.uniforms.clone()
    hi, ho = (d0.hist_ids, d0.hist_offsets) if pen else (None, None)
    s.split_rows = True
    try:
        st = s.prepare_batch(x, d0.params, u, hi, ho, d0.draft_ids)
    finally:
        s.split_rows = False
    assert st._args.flags & _lib.VSAMP_SPLIT_ROWS
    print(f"split rows in a graph B={B} V={V} penalties={pen}", flush=True)
    st.launch()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st.launch()
    torch.cuda.synchronize()
    for rep in range(3):
        fresh = random_workload(100 * rep + 7 + pen, B, V, torch.bfloat16, penalties=False)
        w = Workload(f"replay {rep}", fresh.logits, w0.params, fresh.uniforms, w0.hist_ids, w0.hist_offsets,
                     w0.draft_ids)
        x.copy_(w.logits.to(DEV))
        u.copy_(w.uniforms.to(DEV))
        st.ids.fill_(-1)
        graph.replay()
        torch.cuda.synchronize()
        got, gp = st.ids.cpu(), st.draft_prob.cpu()
        want, wp = s.sample_batch(x, d0.params, u, hi, ho, d0.draft_ids)  # (whole rows, eager)
        torch.cuda.synchronize()
        assert torch.equal(got, want.cpu()), (rep, got, want)
        assert torch.equal(gp.view(torch.int32), wp.cpu().view(torch.int32))
        ties, bad = compare_ids(got, oracle(w), gp)
        assert not bad, (rep, bad[:10])
