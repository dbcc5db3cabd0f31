"""Sampler step benchmark on one MI355X: B=256, V=151936 bf16 (peaked/flat rows), penalties,
top-p 0.95, min-p 0.05 -> rows/s, us/step and the fraction of the HBM roofline.

A step is one ``hip`` sampler launch over all 256 rows with inputs resident in HBM. Timed steps
rotate through four distinct input sets (4 x 77.8 MB of logits > the 256 MB MALL) so each
step's logits come from HBM. Per-launch durations come from HIP events recorded on the stream
the kernel runs on; the CPU baseline is the CPU oracle timed on a bounded sample of the same
rows on this host.

Usage: python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-cpu]
                       [--decode [--num-draft K] | --verify | --logprobs | --workloads]
Prints one JSON line (``--decode``: the batched decode loop's line instead; ``--verify``: the
speculative-decoding verify's; ``--logprobs``: the raw log-probabilities').

`roofline.traffic` (HBM bytes per launch) comes from the rocprofv3 FETCH_SIZE / WRITE_SIZE
counter runs recorded in profiles/k_sample_bf16_peaked_flat_B256.md, each scaled by what the
counter reads for a plain copy of known size (`python bench.py --copy-probe` runs that copy).
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

METRIC = "sampled rows/sec + µs/step at B=256, V=151936 bf16; % HBM roofline"
HBM_PEAK_GBS = 8000.0
# What "dtype" stands for: the sampling decisions are taken on fp32 z, as the engine's are.
ARITHMETIC = ("bf16/fp32 logits widened exactly to fp32; z = x / T in fp32 (IEEE division); "
              "exp(z - max z) in fp64; masses as u64 fixed point (units of 2^-42), summed exactly")
N_SETS = 4
PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "k_sample_bf16_peaked_flat_B256.md")
COPY_PROBE_BYTES = 1 << 30  # bytes read (and written) by one launch of the copy probe


def measured_traffic(key: str = "traffic_bytes_per_launch") -> int | None:
    """HBM bytes per launch of the sampler kernel, from the counter summary's `<key>:` line
    (traffic: FETCH_SIZE and WRITE_SIZE scaled; fetch_bytes_per_launch: the reads alone; None
    when the summary has no such line)."""
    try:
        with open(PROFILE) as fh:
            for line in fh:
                if line.startswith(key + ":"):
                    return int(line.split(":", 1)[1].strip().replace(",", ""))
    except OSError:
        return None
    return None


def copy_probe() -> int:
    """A plain device copy of COPY_PROBE_BYTES (bf16), launched 5 times: the reference the
    FETCH_SIZE / WRITE_SIZE counters are scaled by."""
    import torch

    dev = torch.device("cuda", 0)
    src = torch.empty(COPY_PROBE_BYTES // 2, dtype=torch.bfloat16, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": COPY_PROBE_BYTES, "launches": 5}), flush=True)
    return 0


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(w, budget_s: float = 5.0):
    """The CPU reference sampler on rows of the same workload, one row per call as the engine's
    ``sample`` runs (sampler.py:68-77), cycling through the batch: torch's CPU kernels on the
    engine's fp32 rule plus the extensions (oracle/fp32_rule.py:torch_cpu_sample), for
    ``budget_s`` with torch's default thread count on this host's share and again with one
    thread; beside it, the fp64 numpy oracle on one thread."""
    import torch

    from oracle.fp32_rule import torch_cpu_sample  # the checker's CPU restatement, timed as the baseline
    from oracle.sampler_oracle import sample_batch

    p = w.params
    rows_args = []
    for b in range(w.batch):
        h = w.hist_ids[int(w.hist_offsets[b]) : int(w.hist_offsets[b + 1])]
        rows_args.append((w.logits[b], h, float(p.temperature[b]), int(p.top_k[b]), float(p.top_p[b]),
                          float(p.min_p[b]), float(p.repetition_penalty[b]), float(p.presence_penalty[b]),
                          float(p.frequency_penalty[b]), float(w.uniforms[b])))

    def timed(threads):
        torch.set_num_threads(threads)
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < budget_s:
            torch_cpu_sample(*rows_args[n % w.batch])
            n += 1
        return n, time.perf_counter() - t0

    default_threads = torch.get_num_threads()
    n_all, dt_all = timed(default_threads)
    n_one, dt_one = timed(1)
    torch.set_num_threads(default_threads)

    # the numpy fp64 oracle, one thread, 8 rows per call
    f = lambda t: t.detach().float().cpu().numpy()  # noqa: E731
    logits = f(w.logits)
    cols = [f(getattr(p, k)) for k in ("temperature", "top_k", "top_p", "min_p")]
    pens = [f(getattr(p, k)) for k in ("repetition_penalty", "presence_penalty", "frequency_penalty")]
    hist, off, u = w.hist_ids.numpy(), w.hist_offsets.numpy(), f(w.uniforms)
    rows, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        r0 = rows % w.batch
        sl = slice(r0, r0 + 8)
        sample_batch(logits[sl], *[c[sl] for c in cols], *[c[sl] for c in pens], hist, off[r0 : r0 + 9], u[sl])
        rows += 8
    dt_np = time.perf_counter() - t0
    return {
        "value": n_all / dt_all,
        "unit": "rows/s",
        "cores": default_threads,
        "kind": "port",
        "sample": f"{n_all} rows of the same workload (cycling through its {w.batch} rows, half peaked, half flat), "
        f"one row per call: torch CPU fp32 sampler (penalties, softmax, min-p, sorted top-p, inverse-CDF draw) "
        f"on {default_threads} threads, {dt_all:.1f} s",
        "single_thread": {"value": n_one / dt_one, "unit": "rows/s", "rows": n_one, "seconds": round(dt_one, 2)},
        "numpy_oracle_fp64_one_thread": {"value": rows / dt_np, "unit": "rows/s", "rows": rows,
                                         "seconds": round(dt_np, 2)},
        "cpu_model": cpu_model(),
        "os_cpu_count": os.cpu_count(),
        "torch": torch.__version__,
    }


def tie_counts(w, ids) -> dict:
    """Tie rows of the batch under both classifiers, and the kernel's ids against the oracle off
    the oracle's ties (the launch's own parity check)."""
    import numpy as np

    from oracle.fp32_rule import fp32_rule
    from oracle.sampler_oracle import classify_ties, penalize, sample_row

    p = w.params
    n_or = n_fp = bad = 0
    ids = ids.tolist()
    for b in range(w.batch):
        h = w.hist_ids[int(w.hist_offsets[b]) : int(w.hist_offsets[b + 1])].numpy()
        x, _ = penalize(w.logits[b].float().numpy(), h, float(p.repetition_penalty[b]), float(p.presence_penalty[b]),
                        float(p.frequency_penalty[b]))
        args = (float(p.temperature[b]), int(p.top_k[b]), float(p.top_p[b]), float(p.min_p[b]), float(w.uniforms[b]))
        r = sample_row(x, *args)
        tie = bool(classify_ties(r))
        n_or += tie
        n_fp += bool(fp32_rule(np.asarray(x), *args).ties)
        bad += (not tie) and ids[b] != r.token
    return {"rows": w.batch, "oracle_fixed_point": n_or, "engine_fp32_rule": n_fp,
            "kernel_differs_off_oracle_ties": bad}


def decode_loop(args) -> int:
    """``--decode``: the continuous-batching decode loop at 64 live sequences, V=151936 bf16
    (SyntheticLM logits, mixed per-request parameters with penalties). Prints one JSON line:
    tokens/s of the whole loop and, beside it, the model step and the sampler call timed alone on
    the same shapes."""
    import numpy as np
    import torch

    from vinfer_amd.registry import BackendContext
    from vinfer_amd.runtime import BatchDecoder, SpeculativeDecoder
    from vinfer_amd.sampler import SAMPLER
    from vinfer_amd.sampling import SamplingParams
    from vinfer_amd.workloads import SyntheticLM

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    V, B, L = 151936, 64, 4096
    model = SyntheticLM(V, dim=64, scale=3.0, dtype=torch.bfloat16, device=dev)
    hip = SAMPLER.resolve("hip", BackendContext(dev, torch.bfloat16))
    K = args.num_draft
    if K:
        # the draft: the target's map with its head perturbed (a cheap, mostly agreeing proposer)
        draft = SyntheticLM(V, dim=64, scale=3.0, dtype=torch.bfloat16, device=dev)
        g = torch.Generator(device=dev).manual_seed(7)
        draft.head = (draft.head.float() + torch.randn(draft.head.shape, generator=g, device=dev)
                      * draft.head.float().std() * 0.5).to(torch.bfloat16)

    def run(graphs: bool):
        """The loop's timed iterations: (decoder, us per iteration, tokens)."""
        if K:
            # (graphs: a steady membership's iterations replay one captured HIP graph)
            dec = SpeculativeDecoder(model, hip, draft_model=draft, num_draft=K, num_slots=B, max_seq_len=L,
                                     graphs=graphs)
        else:
            # (graphs: the steady membership's iterations replay two captured HIP graphs)
            dec = BatchDecoder(model, hip, num_slots=B, max_seq_len=L, penalize_prompt=True, graphs=graphs)
        rng = np.random.default_rng(1001)
        ks = (0, 20, 50, 1000)
        for i in range(B):
            kw = dict(max_tokens=L - 64, ignore_eos=True, seed=int(rng.integers(0, 2**62)))
            if not K:
                kw.update(repetition_penalty=1.05, presence_penalty=0.5, frequency_penalty=0.2)
            if i % 4 == 0:
                kw.update(temperature=0.0)
            else:
                kw.update(temperature=float(rng.uniform(0.3, 1.5)), top_k=ks[i % 4],
                          top_p=float(rng.uniform(0.5, 1.0)))
            dec.submit(rng.integers(0, V, size=32).tolist(), SamplingParams(**kw))
        for _ in range(args.warmup):
            dec.step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        n_tok = 0
        for _ in range(args.steps):
            n_tok += len(dec.step())
        torch.cuda.synchronize()
        return dec, (time.perf_counter() - t0) / args.steps * 1e6, n_tok

    steps = args.steps
    _, eager_us, eager_tok = run(False)
    dec, loop_us, n_tok = run(True)

    # the two device parts alone, on the same shapes
    slots = torch.arange(B, device=dev)
    toks = torch.randint(0, V, (B,), device=dev)
    pos = torch.full((B,), 100, device=dev)

    def timed(fn, n=50):
        for _ in range(5):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / n

    model_us = timed(lambda: model.decode(slots, toks, pos))
    logits = model.decode(slots, toks, pos)
    u = torch.rand(B, device=dev)
    seqs = list(dec._running.values())
    params = dec._params(seqs, dev)
    if K:
        sampler_us = timed(lambda: hip.sample_batch(logits, params, u))
    else:
        ranges = torch.tensor([[s.slot * dec._hist_row, s.slot * dec._hist_row + int(dec._hist_len[s.slot])] for s in seqs],
                              dtype=torch.int32, device=dev)
        sampler_us = timed(lambda: hip.sample_batch(logits, params, u, dec.hist, ranges))
    out = {
        "metric": "decode-loop tokens/s at 64 live sequences, V=151936 bf16"
        + (f", speculative K={K}" if K else ""),
        "value": n_tok / (loop_us * steps * 1e-6),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": loop_us / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "arithmetic": ARITHMETIC,
        "data": "synthetic",
        "config": {
            "workload": "decode_loop",
            "live_sequences": B,
            "vocab": V,
            "logits_dtype": "bf16",
            "model": "SyntheticLM rank 64",
            "params": "25% greedy, else T U[0.3,1.5], top-k {20,50,1000}, top-p U[0.5,1]"
            + ("" if K else "; penalties 1.05/0.5/0.2"),
            "history": "prompt (32) + generated ids, per-slot ranges" if not K else "none (no penalties)",
            "num_draft": K,
            "draft": "target head + N(0, (0.5 sd)^2)" if K else None,
        },
        "tokens_per_iteration": n_tok / args.steps,
        "us_per_step_loop": loop_us,
        "graphs": True,
        "graph_iterations": getattr(dec, "graph_steps", 0),
        "us_per_step_loop_without_graphs": eager_us,
        "tokens_per_iteration_without_graphs": eager_tok / args.steps,
        "us_model_step_alone": model_us,
        "us_sampler_call_alone": sampler_us,
        "us_host_and_rest": loop_us - model_us - sampler_us,
    }
    print(json.dumps(out), flush=True)
    return 0


def verify_bench(args) -> int:
    """``--verify``: speculative-decoding verify of one draft per sequence at 192 sequences,
    V=262144 bf16 (target logits ~ N(0, 2.5^2) at two positions, the draft a noisy copy of the
    first, drafts drawn from the draft distribution; T U[0.5, 1.2], top-p 0.95). Prints one
    JSON line: sequences/s, us per verify call, and the HBM roofline fraction over one read of
    the target and draft logits."""
    import numpy as np
    import torch

    from vinfer_amd.registry import BackendContext
    from vinfer_amd.sampler import SAMPLER
    from vinfer_amd.sampling import PackedParams

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, K, V = 192, 1, 262144
    g = torch.Generator(device=dev).manual_seed(1005)
    tgt = (torch.randn(B, K + 1, V, generator=g, device=dev) * 2.5).to(torch.bfloat16)
    drf = (tgt[:, :K].float() + torch.randn(B, K, V, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    rng = np.random.default_rng(1005)
    f32 = lambda a: torch.from_numpy(np.asarray(a, np.float32)).to(dev)  # noqa: E731
    params = PackedParams(
        temperature=f32(rng.uniform(0.5, 1.2, B)), top_k=torch.zeros(B, dtype=torch.int32, device=dev),
        top_p=f32(np.full(B, 0.95)), min_p=f32(np.zeros(B)), repetition_penalty=f32(np.ones(B)),
        presence_penalty=f32(np.zeros(B)), frequency_penalty=f32(np.zeros(B)))
    hip = SAMPLER.resolve("hip", BackendContext(dev, torch.bfloat16))
    # the drafts, drawn as a drafter would, keeping their rows' states for the verify
    drafts, states = hip.sample_states(drf.reshape(B * K, V), params.repeat_rows(K), f32(rng.random(B * K)))
    drafts, states = drafts.reshape(B, K), states.reshape(B, K, -1)
    ua, ur, ub = f32(rng.random((B, K))), f32(rng.random((B, K))), f32(rng.random(B))

    def timed(call):
        for _ in range(args.warmup):
            call()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            res = call()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / args.steps, res

    us, (tokens, counts) = timed(lambda: hip.verify(tgt, drf, drafts, params, ua, ur, ub, draft_states=states))
    us_recompute, _ = timed(lambda: hip.verify(tgt, drf, drafts, params, ua, ur, ub))
    algo = (tgt.numel() + drf.numel()) * 2 + B * (K * 16 + 8)
    achieved = algo / (us * 1e-6) / 1e9
    cpu = None
    if not args.no_cpu:
        # the oracle's verify on the same sequences, cycling, for a bounded time
        from oracle.sampler_oracle import sample_row, verify_row  # the checker, timed here as the baseline

        xt, xd = tgt.float().cpu().numpy(), drf.float().cpu().numpy()
        T, d = params.temperature.cpu().numpy(), drafts.cpu().numpy()
        a_, r_, b_ = ua.cpu().numpy(), ur.cpu().numpy(), ub.cpu().numpy()
        done, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 10.0:
            b = done % B
            t = [sample_row(xt[b, j], T[b], 0, 0.95, 0.0, float(b_[b]), int(d[b, j]) if j < K else None,
                            want_probs=True) for j in range(K + 1)]
            q = [sample_row(xd[b, j], T[b], 0, 0.95, 0.0, 0.0, int(d[b, j]), want_probs=True) for j in range(K)]
            verify_row(t, q, d[b], a_[b], r_[b], V)
            done += 1
        dt = time.perf_counter() - t0
        cpu = {"value": done / dt, "unit": "sequences/s", "cores": 1, "kind": "port",
               "sample": f"{done} sequences of the same batch (cycling), numpy fp64 oracle on one thread; {dt:.1f} s"}
    out = {
        "metric": "verified sequences/s + us/call at B=192, K=1, V=262144 bf16; % HBM roofline",
        "value": B / (us * 1e-6),
        "unit": "sequences/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": us / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "arithmetic": ARITHMETIC,
        "data": "synthetic",
        "config": {"workload": "verify_k1", "batch": B, "num_draft": K, "vocab": V, "logits_dtype": "bf16",
                   "temperature": "U[0.5,1.2]", "top_p": 0.95, "draft": "target + N(0, 0.5^2)"},
        "us_per_call": us,
        "draft_states": "saved when the drafts were drawn (vsamp_sample_states)",
        "us_per_call_recomputing_draft_states": us_recompute,
        "mean_tokens_emitted": float(counts.float().mean()),
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "algorithmic_bytes_per_call": algo},
    }
    if cpu is not None:
        out["cpu_baseline"] = cpu
    print(json.dumps(out), flush=True)
    return 0


def logprobs_bench(args) -> int:
    """``--logprobs``: raw log-probabilities of the sampled token and the top 20 per row over the
    headline logits (256 x 151936 bf16, four rotated input sets). Prints one JSON line: rows/s,
    us per launch and the HBM roofline fraction over one read of the logits."""
    import torch

    from vinfer_amd.registry import BackendContext
    from vinfer_amd.sampler import SAMPLER
    from vinfer_amd.workloads import make

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    w = make("peaked_flat")
    x = w.logits.to(dev)
    sets = [x] + [torch.roll(x, shifts=7919 * i, dims=1).contiguous() for i in range(1, N_SETS)]
    hip = SAMPLER.resolve("hip", BackendContext(dev, torch.bfloat16))
    tokens = torch.randint(0, w.vocab, (w.batch,), dtype=torch.int32, device=dev)
    for i in range(args.warmup):
        hip.logprobs(sets[i % N_SETS], tokens, 20)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(args.steps):
        hip.logprobs(sets[i % N_SETS], tokens, 20)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / args.steps
    algo = x.numel() * 2 + w.batch * (4 + 4 + 20 * 8)
    achieved = algo / (us * 1e-6) / 1e9
    cpu = None
    if not args.no_cpu:
        from oracle.sampler_oracle import logprobs_row  # the checker, timed here as the baseline

        xs, tk = w.logits.float().numpy(), tokens.cpu().numpy()
        done, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 10.0:
            logprobs_row(xs[done % w.batch], int(tk[done % w.batch]), 20)
            done += 1
        dt = time.perf_counter() - t0
        cpu = {"value": done / dt, "unit": "rows/s", "cores": 1, "kind": "port",
               "sample": f"{done} rows of the same logits (cycling), numpy fp64 oracle on one thread; {dt:.1f} s"}
    out = {
        "metric": "logprob rows/s + us/launch at B=256, V=151936 bf16, top 20; % HBM roofline",
        "value": w.batch / (us * 1e-6),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": us / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "arithmetic": ARITHMETIC,
        "data": "synthetic",
        "config": {"workload": "logprobs_peaked_flat", "batch": w.batch, "vocab": w.vocab, "logits_dtype": "bf16",
                   "n_top": 20, "input_sets": N_SETS},
        "us_per_launch": us,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "algorithmic_bytes_per_launch": algo},
    }
    if cpu is not None:
        out["cpu_baseline"] = cpu
    print(json.dumps(out), flush=True)
    return 0


def lm_head_bench(args) -> int:
    """``--lm-head``: the LM head plus log-probabilities (token and top 20) at d=4096, V=151936,
    B in {256, 64, 1}: unfused (the engine's ``F.linear(hidden, W)``, i.e. hipBLASLt, then
    ``vsamp_logprobs``'s two passes over each row) against fused (the backend's ``lm_head``: up to
    64 rows ``vsamp_lm_head``, the hand-written GEMM whose epilogue writes the tile statistics;
    above, ``F.linear`` and ``vsamp_tile_stats``; then ``vsamp_logprobs_tiles``). One JSON line
    per batch, HIP events on the launch stream, synthetic bf16 operands."""
    import math

    import torch

    from vinfer_amd.registry import BackendContext
    from vinfer_amd.sampler import SAMPLER

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    s = SAMPLER.resolve("hip", BackendContext(dev, torch.bfloat16))
    d, V, n_top = 4096, 151936, 20
    g = torch.Generator(device=dev).manual_seed(0)
    W = (torch.randn(V, d, generator=g, device=dev) * (4 / math.sqrt(d))).to(torch.bfloat16)
    stream = torch.cuda.current_stream(dev)
    for B in (256, 64, 1):
        hidden = (torch.randn(B, d, generator=g, device=dev) * 0.5).to(torch.bfloat16)
        tokens = torch.randint(0, V, (B,), generator=g, device=dev, dtype=torch.int32)

        def timed(fn, n=20):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(n):
                fn()
            e1.record(stream)
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) * 1e3 / n

        linear = torch.nn.functional.linear
        logits_t = linear(hidden, W)
        logits_f, tmax, tsum = s.lm_head(hidden, W)
        us = {
            "torch_matmul": timed(lambda: linear(hidden, W)),
            "logprobs_rows": timed(lambda: s.logprobs(logits_t, tokens, n_top)),
            "lm_head_fused": timed(lambda: s.lm_head(hidden, W)),
            "logprobs_tiles": timed(lambda: s.logprobs_tiles(logits_f, tmax, tsum, tokens, n_top)),
        }
        us["unfused_total"] = us["torch_matmul"] + us["logprobs_rows"]
        us["fused_total"] = us["lm_head_fused"] + us["logprobs_tiles"]
        same = float((logits_f == logits_t).float().mean())
        nT = (V + 127) // 128
        bytes_ = V * d * 2 + B * d * 2 + B * V * 2 + B * nT * 8
        flops = 2.0 * B * d * V
        t = us["lm_head_fused"] * 1e-6
        path = ("vsamp_lm_head: k_lm_gemv" if B <= 4 else "vsamp_lm_head: k_lm_stream" if B <= 64
                else "F.linear + vsamp_tile_stats")
        print(json.dumps({"lm_head": {"batch": B, "dim": d, "vocab": V, "n_top": n_top, "path": path}, "us": us,
                          "fused_speedup": us["unfused_total"] / us["fused_total"],
                          "k_lm_head": {"tflops": flops / t / 1e12, "mfma_frac_bf16": flops / t / 2.5e15,
                                        "gbs": bytes_ / t / 1e9, "hbm_frac": bytes_ / t / 1e9 / HBM_PEAK_GBS,
                                        "bytes": bytes_},
                          "logits_equal_torch_frac": same}), flush=True)
        del hidden, logits_t, logits_f, tmax, tsum
    return 0


def lm_head_sample_bench(args) -> int:
    """``--lm-head-sample``: the LM head plus the draw at d=4096, V=151936, B in {1, 64, 256}, for three
    kinds of rows without penalties: greedy, peaked (one logit far above the rest: the hidden
    state near one weight row; T 1.0, top-p 0.95, min-p 0.05 as the headline's peaked rows) and
    top-k (T 0.7, top-k 20, top-p 0.8). Unfused: the engine's ``F.linear``, then ``sample_batch``;
    fused: the backend's ``lm_head`` (``vsamp_lm_head`` up to 64 rows, ``F.linear`` and
    ``vsamp_tile_stats`` above), then ``sample_tiles`` over its tile maxima; each draw a prepared
    launch. Both draws are also run on the fused logits, whose ids must agree. One JSON line per
    (batch, kind), HIP events on the launch stream, synthetic bf16 operands."""
    import math

    import torch

    from vinfer_amd.registry import BackendContext
    from vinfer_amd.sampler import SAMPLER
    from vinfer_amd.sampling import SamplingParams, pack_params

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    s = SAMPLER.resolve("hip", BackendContext(dev, torch.bfloat16))
    d, V = 4096, 151936
    g = torch.Generator(device=dev).manual_seed(0)
    W = (torch.randn(V, d, generator=g, device=dev) * (4 / math.sqrt(d))).to(torch.bfloat16)
    stream = torch.cuda.current_stream(dev)

    def timed(fn, n=20):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / n

    kinds = {
        "greedy": SamplingParams(temperature=0.0),
        "peaked": SamplingParams(temperature=1.0, top_p=0.95, min_p=0.05),
        "top_k": SamplingParams(temperature=0.7, top_k=20, top_p=0.8),
    }
    for B in (1, 64, 256):
        for kind, sp in kinds.items():
            hidden = torch.randn(B, d, generator=g, device=dev) * 0.5
            if kind == "peaked":
                rows = torch.randint(0, V, (B,), generator=g, device=dev)
                hidden = hidden * 0.1 + 3.0 * W[rows].float()
            hidden = hidden.to(torch.bfloat16)
            params = pack_params([sp] * B, dev)
            u = torch.rand(B, generator=g, device=dev)
            linear = torch.nn.functional.linear
            logits_t = linear(hidden, W)
            logits_f, tmax, _ = s.lm_head(hidden, W)
            a, _ = s.sample_tiles(logits_f, tmax, params, u)
            b, _ = s.sample_batch(logits_f, params, u)
            # (the draws as prepared launches: argument blocks built once, as a decode loop does)
            st_rows = s.prepare_batch(logits_t, params, u)
            st_tiles = s.prepare_tiles(logits_f, tmax, params, u)
            us = {
                "torch_matmul": timed(lambda: linear(hidden, W)),
                "sample_batch": timed(lambda: st_rows.launch(stream.cuda_stream)),
                "lm_head_fused": timed(lambda: s.lm_head(hidden, W)),
                "sample_tiles": timed(lambda: st_tiles.launch(stream.cuda_stream)),
            }
            us["unfused_total"] = us["torch_matmul"] + us["sample_batch"]
            us["fused_total"] = us["lm_head_fused"] + us["sample_tiles"]
            print(json.dumps({"lm_head_sample": {"batch": B, "dim": d, "vocab": V, "rows": kind,
                                                 "params": {"temperature": sp.temperature, "top_k": sp.top_k,
                                                            "top_p": sp.top_p, "min_p": sp.min_p}},
                              "us": us, "fused_speedup": us["unfused_total"] / us["fused_total"],
                              "draw_speedup": us["sample_batch"] / us["sample_tiles"],
                              "ids_equal": bool(torch.equal(a, b))}), flush=True)
            del hidden, logits_t, logits_f, tmax
    return 0


def regimes_bench(args) -> int:
    """``--regimes``: the headline batch (B=256, V=151936 bf16) split by regime: its flat rows
    alone, its peaked rows alone, each with and without the rows' histories, then the mixed
    batch itself. One JSON line each, timed as ``--workloads`` times a workload (the launches
    of a variant follow each other in this order, which a counter run pairs with dispatches)."""
    import dataclasses

    import torch

    from vinfer_amd.registry import BackendContext
    from vinfer_amd.sampler import SAMPLER
    from vinfer_amd.workloads import make

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    s = SAMPLER.resolve("hip", BackendContext(dev, torch.bfloat16))
    stream = torch.cuda.current_stream(dev)
    K = max(1, args.steps // 4)
    variants = []
    for regime in ("flat", "peaked"):
        w = make("peaked_flat", regime=regime)
        variants.append((regime, True, w))
        variants.append((regime, False, dataclasses.replace(w, hist_ids=None, hist_offsets=None)))
    variants.append(("mixed (the headline batch)", True, make("peaked_flat")))
    for regime, hist, w in variants:
        d = w.to(dev)
        sets = [d.logits] + [torch.roll(d.logits, shifts=7919 * i, dims=1).contiguous() for i in range(1, N_SETS)]
        steps = [s.prepare_batch(x, d.params, d.uniforms, d.hist_ids, d.hist_offsets) for x in sets]
        for i in range(args.warmup):
            steps[i % len(steps)].launch(stream.cuda_stream)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(K):
            steps[i % len(steps)].launch(stream.cuda_stream)
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / K
        algo = w.algorithmic_bytes()
        print(json.dumps({"workload": "peaked_flat", "regime": regime, "histories": hist, "batch": w.batch,
                          "vocab": w.vocab, "us_per_launch": us, "rows_per_s": w.batch / (us * 1e-6),
                          "launches": K, "warmup": args.warmup, "input_sets": len(sets), "algorithmic_bytes": algo,
                          "roofline_frac": algo / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}), flush=True)
        del steps, sets, d
    return 0


def workload_cpu_baseline(w, budget_s: float = 3.0) -> dict:
    """The CPU reference sampler on the workload, one row per call as the engine's ``sample``
    runs (sampler.py:68-77): torch's CPU kernels on the engine's fp32 rule plus the extensions
    (oracle/fp32_rule.py:torch_cpu_sample), with torch's default thread count on this host and
    with one thread; the median per-row time of each. single_fp32 (one row per step) is timed
    as 1000 steps, each on a new row and uniform of the same generator; the other workloads
    cycle through their rows for ``budget_s``. Beside it, the numpy fp64 oracle on one thread."""
    import numpy as np
    import torch

    from oracle.fp32_rule import torch_cpu_sample  # the checker's CPU restatement, timed as the baseline
    from oracle.sampler_oracle import sample_batch
    from vinfer_amd.workloads import make

    steps = 1000 if w.batch == 1 else None
    src = make(w.name if w.name != "single_bf16" else "single_fp32", batch=steps) if steps else w
    if w.logits.dtype == torch.bfloat16 and src is not w:
        src.logits = src.logits.to(torch.bfloat16)
    p = src.params
    empty = torch.zeros(0, dtype=torch.int32)

    def row(b):
        h = src.hist_ids[int(src.hist_offsets[b]) : int(src.hist_offsets[b + 1])] if src.hist_ids is not None else empty
        return (src.logits[b], h, float(p.temperature[b]), int(p.top_k[b]), float(p.top_p[b]), float(p.min_p[b]),
                float(p.repetition_penalty[b]), float(p.presence_penalty[b]), float(p.frequency_penalty[b]),
                float(src.uniforms[b]))

    def timed(threads):
        torch.set_num_threads(threads)
        per = []
        t0 = time.perf_counter()
        b = 0
        while (b < steps) if steps else (time.perf_counter() - t0 < budget_s):
            args = row(b % src.batch)
            t1 = time.perf_counter()
            torch_cpu_sample(*args)
            per.append(time.perf_counter() - t1)
            b += 1
        return {"rows_per_s": len(per) / sum(per), "median_us_per_row": float(np.median(per)) * 1e6,
                "rows": len(per), "threads": threads}

    default_threads = torch.get_num_threads()
    every = timed(default_threads)
    one = timed(1)
    torch.set_num_threads(default_threads)
    f = lambda t: t.detach().float().cpu().numpy()  # noqa: E731
    cols = [f(getattr(w.params, k)) for k in ("temperature", "top_k", "top_p", "min_p", "repetition_penalty",
                                               "presence_penalty", "frequency_penalty")]
    hist = w.hist_ids.numpy() if w.hist_ids is not None else np.zeros(0, np.int32)
    off = w.hist_offsets.numpy() if w.hist_offsets is not None else np.zeros(w.batch + 1, np.int32)
    x, u = f(w.logits), f(w.uniforms)
    dr = w.draft_ids.numpy() if w.draft_ids is not None else None
    rows, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        r = rows % w.batch
        sample_batch(x[r : r + 1], *[c[r : r + 1] for c in cols], hist, off[r : r + 2], u[r : r + 1],
                     None if dr is None else dr[r : r + 1])
        rows += 1
    dt = time.perf_counter() - t0
    what = (f"{every['rows']} steps of one new row each" if steps else
            f"{every['rows']} rows of the workload (cycling through its {w.batch} rows)")
    return {"value": every["rows_per_s"], "unit": "rows/s", "cores": default_threads, "kind": "port",
            "sample": f"{what}, one row per call: torch CPU fp32 sampler on {default_threads} threads",
            "median_us_per_row": every["median_us_per_row"], "single_thread": one,
            "numpy_oracle_fp64_one_thread": {"value": rows / dt, "unit": "rows/s", "rows": rows,
                                             "seconds": round(dt, 2)},
            "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(), "torch": torch.__version__}


def workloads_bench(args) -> int:
    """``--workloads``: every named sampler workload (``vinfer_amd.workloads.NAMES``), one JSON line
    each: the launch time (back-to-back launches between HIP events on the launch stream, after
    warmup; inputs rotated over four copies when they fit in 8 GB), the HBM roofline fraction of
    its algorithmic bytes, and the CPU reference sampler beside it (``workload_cpu_baseline``)."""
    import numpy as np
    import torch

    from vinfer_amd.registry import BackendContext
    from vinfer_amd.sampler import SAMPLER
    from vinfer_amd.workloads import NAMES, make

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    names = NAMES + ("single_bf16",)
    if args.only:
        names = tuple(n for n in names if n in args.only.split(","))
    for name in names:
        if name == "single_bf16":  # the per-token row in the model's dtype
            w = make("single_fp32")
            w.logits = w.logits.to(torch.bfloat16)
            w.name = name
        else:
            w = make(name)
        d = w.to(dev)
        s = SAMPLER.resolve("hip", BackendContext(dev, w.logits.dtype))
        nbytes = d.logits.numel() * d.logits.element_size()
        sets = [d.logits] + ([torch.roll(d.logits, shifts=7919 * i, dims=1).contiguous() for i in range(1, N_SETS)]
                             if nbytes * N_SETS <= 8 << 30 else [])
        stream = torch.cuda.current_stream(dev)
        K = max(1, args.steps // 4)

        def timed(split_rows: bool) -> float:
            s.split_rows = split_rows
            steps = [s.prepare_batch(x, d.params, d.uniforms, d.hist_ids, d.hist_offsets, d.draft_ids) for x in sets]
            s.split_rows = False
            for i in range(args.warmup):
                steps[i % len(steps)].launch(stream.cuda_stream)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for i in range(K):
                steps[i % len(steps)].launch(stream.cuda_stream)
            e1.record(stream)
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) * 1e3 / K

        us = timed(False)
        algo = w.algorithmic_bytes()
        out = {"workload": name, "batch": w.batch, "vocab": w.vocab, "logits_dtype": str(w.logits.dtype).split(".")[-1],
               "us_per_launch": us, "rows_per_s": w.batch / (us * 1e-6), "launches": K,
               "input_sets": len(sets), "algorithmic_bytes": algo,
               "roofline_frac": algo / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}
        if args.split_rows and w.logits.dtype == torch.bfloat16 and w.batch <= 128:
            out["us_per_launch_split_rows"] = timed(True)  # (VSAMP_SPLIT_ROWS: identical ids)
        if not args.no_cpu:
            out["cpu_baseline"] = workload_cpu_baseline(w)
        print(json.dumps(out), flush=True)
        del sets, d
        torch.cuda.empty_cache()
    # the engine's per-token call, unchanged (generate.py:129): sample(logits[V], params, seed,
    # position) -> int, host work and the id's copy back included
    if args.only and "per_token" not in args.only.split(","):
        return 0
    from vinfer_amd.sampling import SamplingParams

    for dtype in (torch.bfloat16, torch.float32):
        s = SAMPLER.resolve("hip", BackendContext(dev, dtype))
        w = make("single_fp32")
        row = w.logits[0].to(dtype).to(dev)
        sp = SamplingParams(temperature=0.7, top_k=20, top_p=0.8)
        for i in range(20):
            s.sample(row, sp, 7, i)
        torch.cuda.synchronize()
        n, t0 = 200, time.perf_counter()
        for i in range(n):
            s.sample(row, sp, 7, i)
        us = (time.perf_counter() - t0) / n * 1e6
        print(json.dumps({"call": "sample(logits[V], params, seed, position)", "vocab": w.vocab,
                          "logits_dtype": str(dtype).split(".")[-1], "us_per_call_host_inclusive": us}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--copy-probe", action="store_true", help="run the counter-calibration copy and exit")
    ap.add_argument("--decode", action="store_true", help="time the batched decode loop instead")
    ap.add_argument("--num-draft", type=int, default=0, help="with --decode: speculative decoding, K drafts")
    ap.add_argument("--verify", action="store_true", help="time the speculative-decoding verify instead")
    ap.add_argument("--logprobs", action="store_true", help="time the raw log-probabilities instead")
    ap.add_argument("--workloads", action="store_true", help="time every named workload (one line each)")
    ap.add_argument("--regimes", action="store_true",
                    help="time the headline batch's flat and peaked rows apart, with and without histories")
    ap.add_argument("--lm-head", action="store_true",
                    help="time the LM head + log-probabilities, fused against torch's matmul + vsamp_logprobs")
    ap.add_argument("--only", default="",
                    help="with --workloads: a comma-separated subset of the workloads (per_token: the per-token call)")
    ap.add_argument("--lm-head-sample", action="store_true",
                    help="time the LM head plus the draw, fused (tile maxima) against unfused")
    ap.add_argument("--split-rows", action="store_true",
                    help="with --workloads: also time small bf16 batches with split rows (VSAMP_SPLIT_ROWS)")
    args = ap.parse_args()
    if args.copy_probe:
        return copy_probe()
    if args.gpus != 1:
        print(
            "bench.py measures one GPU: the sampler shards rows across GPUs with no communication, "
            "so run it with --gpus 1",
            file=sys.stderr,
        )
        return 2
    if args.decode:
        return decode_loop(args)
    if args.verify:
        return verify_bench(args)
    if args.logprobs:
        return logprobs_bench(args)
    if args.regimes:
        return regimes_bench(args)
    if args.workloads:
        return workloads_bench(args)
    if args.lm_head_sample:
        return lm_head_sample_bench(args)
    if args.lm_head:
        return lm_head_bench(args)

    import numpy as np
    import torch

    from vinfer_amd.registry import BackendContext
    from vinfer_amd.sampler import SAMPLER
    from vinfer_amd.workloads import make

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    w = make("peaked_flat")
    s = SAMPLER.resolve("hip", BackendContext(dev, torch.bfloat16))
    d = w.to(dev)
    # four distinct logits buffers with the same statistics (rolled along the vocabulary)
    sets = [d.logits] + [torch.roll(d.logits, shifts=7919 * i, dims=1).contiguous() for i in range(1, N_SETS)]
    steps = [s.prepare_batch(x, d.params, d.uniforms, d.hist_ids, d.hist_offsets) for x in sets]
    stream = torch.cuda.current_stream(dev)

    for i in range(args.warmup):
        steps[i % N_SETS].launch(stream.cuda_stream)
    torch.cuda.synchronize()

    # the timed region: K back-to-back launches between two events on the launch stream
    K = args.steps
    e_start, e_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e_start.record(stream)
    for i in range(K):
        steps[i % N_SETS].launch(stream.cuda_stream)
    e_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    total_us = e_start.elapsed_time(e_end) * 1e3

    # spread of single launches (an event pair around each; the events add their own gap)
    n_spread = min(K, 50)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n_spread + 1)]
    ev[0].record(stream)
    for i in range(n_spread):
        steps[i % N_SETS].launch(stream.cuda_stream)
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    per = np.array([ev[i].elapsed_time(ev[i + 1]) * 1e3 for i in range(n_spread)])  # us per launch

    # cache-resident variant: the same input set every step
    for _ in range(10):
        steps[0].launch(stream.cuda_stream)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(50):
        steps[0].launch(stream.cuda_stream)
    e1.record(stream)
    torch.cuda.synchronize()
    cached_us = e0.elapsed_time(e1) * 1e3 / 50

    # the two regimes of the headline alone (every row peaked, every row flat), same method
    regimes = {}
    for regime in ("peaked", "flat"):
        wr = make("peaked_flat", regime=regime)
        dr = wr.to(dev)
        rs = [dr.logits] + [torch.roll(dr.logits, shifts=7919 * i, dims=1).contiguous() for i in range(1, N_SETS)]
        rsteps = [s.prepare_batch(x, dr.params, dr.uniforms, dr.hist_ids, dr.hist_offsets) for x in rs]
        for i in range(10):
            rsteps[i % N_SETS].launch(stream.cuda_stream)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(50):
            rsteps[i % N_SETS].launch(stream.cuda_stream)
        e1.record(stream)
        torch.cuda.synchronize()
        regimes[regime] = e0.elapsed_time(e1) * 1e3 / 50
        del rsteps, rs, dr
    # the ids of the headline inputs (input set 0), for the parity check beside the CPU leg
    steps[0].launch(stream.cuda_stream)
    torch.cuda.synchronize()
    ids0 = steps[0].ids.cpu()

    B = w.batch
    us_step = total_us / K
    algo = w.algorithmic_bytes()
    logits_bytes = w.logits.numel() * w.logits.element_size()
    achieved = algo / (us_step * 1e-6) / 1e9  # average launch: the timed region over K
    fetched = measured_traffic("fetch_bytes_per_launch")
    out = {
        "metric": METRIC,
        "value": B / (us_step * 1e-6),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": us_step / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "arithmetic": ARITHMETIC,
        "data": "synthetic",
        "config": {
            "workload": "peaked_flat",
            "batch": B,
            "vocab": w.vocab,
            "logits_dtype": "bf16",
            "rows": "even peaked (one id +15 over N(0,1)), odd flat (N(0,0.1^2))",
            "temperature": 1.0,
            "top_k": 0,
            "top_p": 0.95,
            "min_p": 0.05,
            "penalties": {"repetition": 1.05, "presence": 0.5, "frequency": 0.2},
            "history_len": 4096,
            "input_sets": N_SETS,
        },
        "us_per_step": us_step,
        "us_per_launch_event_bracketed_p10_p50_p90": [float(np.percentile(per, q)) for q in (10, 50, 90)],
        "us_per_step_cache_resident": cached_us,
        "us_per_step_peaked_rows_only": regimes["peaked"],
        "us_per_step_flat_rows_only": regimes["flat"],
        "wall_s": wall,
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": measured_traffic(),
            # HBM reads per launch over one read of the logits (the counters' read bytes, the
            # histories' included)
            "logits_passes": None if fetched is None else fetched / logits_bytes,
            "algorithmic_bytes_per_launch": algo,
            "logits_only_frac": logits_bytes / (us_step * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "kernel": "vs::k_sample<bf16, penalties>",
        },
        "gpu": torch.cuda.get_device_name(dev),
        "host": platform.processor() or platform.machine(),
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(w)
        out["ties"] = tie_counts(w, ids0)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
