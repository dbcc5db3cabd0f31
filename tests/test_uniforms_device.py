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
