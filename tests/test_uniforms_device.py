"""vsamp_uniforms_device: the draw's uniforms computed on the device, as the speculative loop's
captured graph computes them from staged positions. They must equal the host derivation
(vsamp_uniforms, itself checked against the Python derivation over hashlib) bit for bit."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from vinfer_amd import _lib


def test_device_uniforms_reject_bad_arguments_before_any_launch():
    lib = _lib.load()
    assert lib.vsamp_uniforms_device(None, None, -1, None, None) == 1
    assert "n must be >= 0" in lib.vsamp_last_error().decode()
    assert lib.vsamp_uniforms_device(None, None, 0, None, None) == 0


@pytest.mark.gpu
def test_gpu_device_uniforms_equal_the_host_ones():
    from vinfer_amd.registry import BackendContext
    from vinfer_amd.sampler import SAMPLER
    from vinfer_amd.sampling import uniform

    dev = torch.device("cuda", 0)
    s = SAMPLER.resolve("hip", BackendContext(dev, torch.bfloat16))
    rng = np.random.default_rng(11)
    seeds = np.concatenate([np.array([0, 7, -1, -(1 << 63), (1 << 63) - 1, 1 << 62], np.int64),
                            rng.integers(-(1 << 63), (1 << 63) - 1, 5000, dtype=np.int64)])
    # (the loop's positions: -(4 q + c) for the streams c = 1 .. 4, and plain ones)
    q = rng.integers(0, 1 << 20, seeds.shape[0])
    positions = np.where(rng.random(seeds.shape[0]) < 0.5, -(4 * q + rng.integers(1, 5, q.shape[0])), q).astype(np.int64)
    positions[:6] = [0, 1, -5, (1 << 63) - 1, -(1 << 63), 10**12]
    want = _lib.position_uniforms(seeds, positions)
    print("device uniforms", seeds.shape[0], flush=True)
    got = s.uniforms_device(torch.from_numpy(seeds).to(dev), torch.from_numpy(positions).to(dev)).cpu().numpy()
    assert np.array_equal(got.view(np.int32), want.view(np.int32))
    assert [float(x) for x in got[:6]] == [uniform(int(a), int(b)) for a, b in zip(seeds[:6], positions[:6])]
    # into a caller's buffer, longer than n
    out = torch.full((seeds.shape[0] + 3,), -1.0, device=dev)
    s.uniforms_device(torch.from_numpy(seeds).to(dev), torch.from_numpy(positions).to(dev), out=out)
    assert np.array_equal(out[: seeds.shape[0]].cpu().numpy(), want) and (out[seeds.shape[0]:] == -1).all()
    with pytest.raises(ValueError, match="int64"):
        s.uniforms_device(torch.zeros(4, dtype=torch.int32, device=dev), torch.zeros(4, dtype=torch.int64, device=dev))


def spec_inputs(rng, n, K):
    """A speculative loop's inputs for sequences at random positions (the loop's layout)."""
    position = rng.integers(2, 1 << 30, n).astype(np.int64)
    ints = np.zeros((4 + 2 * K + 1, n), np.int64)
    ints[0] = rng.permutation(n)
    ints[1] = rng.integers(0, 151936, n)
    ints[2] = rng.integers(0, 151936, n)
    ints[3] = position - 2
    ints[4:4 + K] = position[None, :] - 1 + np.arange(K)[:, None]
    ints[4 + K:].reshape(-1)[:] = (position[:, None] - 1 + np.arange(K + 1)[None, :]).reshape(-1)
    return ints, position


def spec_uniforms(seeds, position, K):
    n = position.shape[0]
    at = position[:, None] + np.arange(K)[None, :]
    upos = np.concatenate([-(4 * at.T + 1).ravel(), -(4 * at + 2).ravel(), -(4 * at + 3).ravel(),
                           -(4 * (position + K) + 4)])
    useeds = np.concatenate([np.tile(seeds, K), np.repeat(seeds, K), np.repeat(seeds, K), seeds])
    return _lib.position_uniforms(useeds, upos)


@pytest.mark.gpu
@pytest.mark.parametrize("n,K", [(64, 2), (5, 1), (33, 3), (7, 5)])
def test_gpu_spec_advance_equals_the_host_derivation(n, K):
    # the next iteration's inputs from an iteration's tokens and counts, and its uniforms, against
    # the same derivation on the host; then the uniforms alone (no counts), inputs untouched
    from vinfer_amd.registry import BackendContext
    from vinfer_amd.sampler import SAMPLER

    dev = torch.device("cuda", 0)
    s = SAMPLER.resolve("hip", BackendContext(dev, torch.bfloat16))
    rng = np.random.default_rng(n * 10 + K)
    ints, position = spec_inputs(rng, n, K)
    seeds = rng.integers(-(1 << 63), (1 << 63) - 1, n, dtype=np.int64)
    tokens = rng.integers(0, 151936, (n, K + 1)).astype(np.int32)
    counts = rng.integers(1, K + 2, n).astype(np.int32)
    print(f"spec_advance n={n} K={K}", flush=True)
    d_ints = torch.from_numpy(ints).to(dev)
    d_u = torch.full(((3 * K + 1) * n,), -1.0, device=dev)
    d_seeds = torch.from_numpy(seeds).to(dev)
    s.spec_advance(d_ints, K, d_seeds, d_u)
    assert torch.equal(d_ints.cpu(), torch.from_numpy(ints))
    assert np.array_equal(d_u.cpu().numpy(), spec_uniforms(seeds, position, K))
    s.spec_advance(d_ints, K, d_seeds, d_u, torch.from_numpy(tokens).to(dev), torch.from_numpy(counts).to(dev))
    c = counts.astype(np.int64)
    rows = np.arange(n)
    want, pos2 = spec_inputs(np.random.default_rng(0), n, K)
    new_pos = position + c
    want[0] = ints[0]
    want[1] = tokens[rows, c - 1]
    want[2] = np.where(c >= 2, tokens[rows, np.maximum(c - 2, 0)], ints[1])
    want[3] = new_pos - 2
    want[4:4 + K] = new_pos[None, :] - 1 + np.arange(K)[:, None]
    want[4 + K:].reshape(-1)[:] = (new_pos[:, None] - 1 + np.arange(K + 1)[None, :]).reshape(-1)
    assert np.array_equal(d_ints.cpu().numpy(), want)
    assert np.array_equal(d_u.cpu().numpy(), spec_uniforms(seeds, new_pos, K))


def test_spec_advance_rejects_bad_arguments_before_any_launch():
    lib = _lib.load()
    assert lib.vsamp_spec_advance(None, 4, 0, None, None, None, None, None) == 1
    assert "num_draft" in lib.vsamp_last_error().decode()
    assert lib.vsamp_spec_advance(None, 4, 22, None, None, None, None, None) == 1
    assert lib.vsamp_spec_advance(None, -1, 2, None, None, None, None, None) == 1
    assert lib.vsamp_spec_advance(None, 0, 2, None, None, None, None, None) == 0
