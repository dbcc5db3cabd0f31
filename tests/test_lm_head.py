"""The LM head fused with the log-softmax's statistics (``vsamp_lm_head``) and the log-softmax that
takes them (``vsamp_logprobs_tiles``).

The GEMM is floating point: its bf16 logits are checked against a plain torch fp32 product of
the same bf16 operands (``hidden.float() @ weight.float().T``): every logit within one bf16 ulp
plus 2^-16 of sum |h_i w_i| of the fp32 value (the kernel's fp32 sums differ from torch's in
order, which shows where terms cancel, and a value next to a rounding boundary may round the
other way), and at least 99 % of them rounding identically. The
tile statistics are recomputed in fp64 from the kernel's own bf16 logits: the maxima exactly,
the sums of exponentials within 1e-5 relative (fp32 exponentials summed in fp32).

The tile-mode log-softmax must give what ``vsamp_logprobs`` gives on the same logits (top ids
exact, logprobs within 2e-6 + 1e-6 |lp|, the bound the oracle test uses), which the oracle's
``logprobs_row`` then pins on a subset of rows; rows with massive ties (more candidate tiles
than the tile path reads) take its fallback passes and must agree too."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.sampler_oracle import logprobs_row
from vinfer_amd import _lib
from vinfer_amd.registry import BackendContext
from vinfer_amd.sampler import SAMPLER

DEV = torch.device("cuda", 0)
TILE = _lib.LM_TILE


def hip():
    return SAMPLER.resolve("hip", BackendContext(DEV, torch.bfloat16))


def operands(seed, B, d, V):
    g = torch.Generator().manual_seed(seed)
    hidden = (torch.randn(B, d, generator=g) * 0.5).to(torch.bfloat16)
    weight = (torch.randn(V, d, generator=g) / math.sqrt(d) * 4).to(torch.bfloat16)
    return hidden.to(DEV), weight.to(DEV)


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    # spacing of bf16 values at |x| (8 significant bits); the smallest normal's spacing below it
    a = x.abs().clamp_min(2.0**-126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


def tile_stats(logits: torch.Tensor):
    B, V = logits.shape
    nT = (V + TILE - 1) // TILE
    x = torch.full((B, nT * TILE), -math.inf, dtype=torch.float64, device=logits.device)
    x[:, :V] = logits.double()
    x = x.view(B, nT, TILE)
    m = x.max(dim=2).values
    s = torch.exp(x - m.unsqueeze(2)).sum(dim=2)
    return m, s


@pytest.mark.gpu
@pytest.mark.parametrize("B,d,V", [(1, 64, 1000), (1, 512, 3001), (1, 2048, 20000), (1, 4096, 151936),
                                   (2, 1024, 7001), (3, 2048, 20000), (4, 4096, 151936), (3, 128, 4099),
                                   (17, 512, 20000), (100, 192, 9000), (300, 256, 5000), (600, 64, 2100),
                                   (256, 4096, 151936)])
def test_gpu_lm_head_matches_torch_fp32(B, d, V):
    print(f"lm_head B={B} d={d} V={V}", flush=True)
    hidden, weight = operands(B + d + V, B, d, V)
    logits, tmax, tsum = hip().lm_head(hidden, weight)
    torch.cuda.synchronize()
    ref = hidden.float() @ weight.float().T
    # the two fp32 sums differ by their order: up to a few eps32 of sum |h_i w_i| (2^-16 of it
    # here), which shows where terms cancel; then one bf16 ulp for the rounding
    mag = hidden.float().abs() @ weight.float().abs().T
    err = (logits.float() - ref).abs()
    tol = bf16_ulp(ref) + mag * 2.0**-16
    assert bool((err <= tol).all()), float((err / tol).max())
    same = float((logits == ref.to(torch.bfloat16)).float().mean())
    assert same >= 0.99, same
    m, s = tile_stats(logits)
    assert torch.equal(tmax.double(), m)
    torch.testing.assert_close(tsum.double(), s, rtol=1e-5, atol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("B,d,V", [(65, 128, 5000), (100, 192, 9000), (300, 256, 5000), (600, 64, 2100),
                                   (256, 4096, 151936)])
def test_gpu_c_abi_lm_head_above_64_rows(B, d, V):
    # above 64 rows the backend's lm_head takes the library GEMM, while vsamp_lm_head itself (a C
    # caller's route) runs the 256 x 128 MFMA tiles: called here through the C ABI directly
    import ctypes

    print(f"vsamp_lm_head B={B} d={d} V={V}", flush=True)
    hidden, weight = operands(B + d + V, B, d, V)
    nT = (V + TILE - 1) // TILE
    logits = torch.empty(B, V, dtype=torch.bfloat16, device=DEV)
    tmax = torch.empty(B, nT, dtype=torch.float32, device=DEV)
    tsum = torch.empty(B, nT, dtype=torch.float32, device=DEV)
    a = _lib.VsampLmHeadArgs()
    a.hidden, a.hidden_stride = hidden.data_ptr(), d
    a.weight, a.weight_stride = weight.data_ptr(), d
    a.logits, a.logits_stride = logits.data_ptr(), V
    a.tile_max, a.tile_sum = tmax.data_ptr(), tsum.data_ptr()
    a.batch, a.dim, a.vocab = B, d, V
    stream = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    _lib.check(_lib.load().vsamp_lm_head(ctypes.byref(a), stream))
    torch.cuda.synchronize()
    ref = hidden.float() @ weight.float().T
    mag = hidden.float().abs() @ weight.float().abs().T
    err = (logits.float() - ref).abs()
    tol = bf16_ulp(ref) + mag * 2.0**-16
    assert bool((err <= tol).all()), float((err / tol).max())
    assert float((logits == ref.to(torch.bfloat16)).float().mean()) >= 0.99
    m, s = tile_stats(logits)
    assert torch.equal(tmax.double(), m)
    torch.testing.assert_close(tsum.double(), s, rtol=1e-5, atol=0)


def check_logprobs_tiles(logits, tmax, tsum, tokens, n_top, oracle_rows=()):
    s = hip()
    t1, i1, l1 = s.logprobs_tiles(logits, tmax, tsum, tokens, n_top)
    t0, i0, l0 = s.logprobs(logits, tokens, n_top)
    assert torch.equal(i1, i0)
    fin = torch.isfinite(l0)
    assert torch.equal(torch.isnan(l1), torch.isnan(l0)) and torch.equal(torch.isneginf(l1), torch.isneginf(l0))
    assert bool(((l1 - l0).abs()[fin] <= 2e-6 + 1e-6 * l0.abs()[fin]).all())
    if tokens is not None:
        ok = torch.isfinite(t0)
        assert torch.equal(torch.isnan(t1), torch.isnan(t0))
        assert bool(((t1 - t0).abs()[ok] <= 2e-6 + 1e-6 * t0.abs()[ok]).all())
    xs = logits.float().cpu().numpy()
    for b in oracle_rows:
        wt, wids, wv = logprobs_row(xs[b], int(tokens[b]) if tokens is not None else None, n_top)
        assert i1[b].tolist() == wids
        f = np.isfinite(wv)
        np.testing.assert_allclose(l1[b].cpu().numpy()[f], wv[f], rtol=1e-6, atol=2e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("B,d,V,n_top", [(4, 256, 1000, 5), (9, 512, 20000, 20), (256, 4096, 151936, 20),
                                         (2, 128, 151936, 32), (5, 64, 300, 0), (1, 4096, 151936, 20),
                                         (3, 4096, 151936, 20), (2, 64, 300, 20), (3, 64, 12, 20)])
def test_gpu_logprobs_tiles_equal_logprobs(B, d, V, n_top):
    print(f"logprobs_tiles B={B} d={d} V={V} n_top={n_top}", flush=True)
    hidden, weight = operands(7 * B + V, B, d, V)
    logits, tmax, tsum = hip().lm_head(hidden, weight)
    g = torch.Generator().manual_seed(B + V)
    tokens = torch.randint(-2, V + 2, (B,), generator=g, dtype=torch.int32).to(DEV)
    check_logprobs_tiles(logits, tmax, tsum, tokens, n_top, oracle_rows=range(min(B, 4)))


@pytest.mark.gpu
def test_gpu_logprobs_tiles_on_tied_and_non_finite_rows():
    # statistics computed here from crafted bf16 rows: massive ties (every tile a candidate, so
    # the fallback passes), one value everywhere, a NaN, half the row -inf
    B, V = 6, 40000
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, V, generator=g) * 2
    x[1] = torch.randn(V, generator=g) * 0.01
    x[2] = 0.0
    x[3, 5] = float("nan")
    x[4, : V // 2] = float("-inf")
    x[5, :] = torch.round(x[5, :])
    logits = x.to(torch.bfloat16).to(DEV)
    m, s = tile_stats(logits.float())
    tmax, tsum = m.float().contiguous(), s.float().contiguous()
    tokens = torch.tensor([0, 7, V - 1, 5, 3, -1], dtype=torch.int32, device=DEV)
    print("logprobs_tiles crafted rows", flush=True)
    for n_top in (1, 20, 32):
        check_logprobs_tiles(logits, tmax, tsum, tokens, n_top, oracle_rows=range(B))


@pytest.mark.gpu
def test_gpu_lm_head_rejects_bad_shapes():
    s = hip()
    h = torch.zeros(2, 100, dtype=torch.bfloat16, device=DEV)  # d not a multiple of 64
    w = torch.zeros(10, 100, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        s.lm_head(h, w)
    with pytest.raises(ValueError):
        s.lm_head(h.float(), w)


@pytest.mark.gpu
@pytest.mark.parametrize("B,V,pad", [(3, 1000, 0), (5, 4099, 7), (2, 151936, 0), (70, 20000, 3)])
def test_gpu_tile_stats_of_logits_from_any_gemm(B, V, pad):
    # vsamp_tile_stats on bf16 rows it did not write (padded strides, a ragged last tile), with
    # NaN, +inf and all -inf rows and ties of the max: the max exactly, the sums to 1e-5
    g = torch.Generator().manual_seed(B + V)
    x = torch.randn(B, V, generator=g) * 3
    x[0, V // 2] = 40.0
    x[0, V // 3] = 40.0  # (a tie of the max in two tiles)
    if B > 1:
        x[1] = -math.inf
    if B > 2:
        x[2, 7] = float("nan")
        x[2, V - 1] = math.inf
    buf = torch.zeros(B, V + pad, dtype=torch.bfloat16)
    buf[:, :V] = x.to(torch.bfloat16)
    logits = buf.to(DEV)[:, :V]
    print(f"tile_stats B={B} V={V} pad={pad}", flush=True)
    tmax, tsum = hip().tile_stats(logits)
    torch.cuda.synchronize()
    m, s = tile_stats(logits)
    same = (tmax.double() == m) | (torch.isnan(tmax.double()) & torch.isnan(m))
    assert bool(same.all())
    fin = torch.isfinite(m)
    torch.testing.assert_close(tsum.double()[fin], s[fin], rtol=1e-5, atol=0)
    assert bool((tsum[~fin.cpu()] == 0).all())


def test_tile_stats_rejects_bad_arguments_before_any_launch():
    lib = _lib.load()
    assert lib.vsamp_tile_stats(None, 10, -1, 10, None, None, None) == 1
    assert "batch" in lib.vsamp_last_error().decode()
    assert lib.vsamp_tile_stats(None, 5, 2, 10, None, None, None) == 1
    assert "row_stride" in lib.vsamp_last_error().decode()
    assert lib.vsamp_tile_stats(None, 10, 2, 0, None, None, None) == 1
    assert lib.vsamp_tile_stats(None, 10, 0, 10, None, None, None) == 0
    assert lib.vsamp_tile_stats(None, 10, 2, 10, None, None, None) == 1
    assert "must be set" in lib.vsamp_last_error().decode()
