"""Writes known_answers.json: closed-form answers and the engine tests' own fixtures.

Nothing here runs the engine or the oracle. Sources:
- ``LOGITS`` and the expected outcomes of tests/unit/runtime/test_sampler.py:10, :20-21, :41-48
  and tests/regression/test_sampler_zero_noise.py:14-19 (copied values).
- Softmax of ``LOGITS`` at T=1 and T=0.5 and the top-p=0.8 renormalisation, computed here in
  fp64 from the closed form ``exp(x/T) / sum exp(x/T)``.
- ``position_seed`` values computed with hashlib's BLAKE2b (the function's definition,
  sampler.py:44-47), independently of the package's implementation.
"""

import hashlib
import json
from pathlib import Path

import numpy as np

LOGITS = [2.0, 1.0, 0.5, 0.0, -1.0, -3.0]


def softmax(x, T):
    e = np.exp(np.asarray(x, dtype=np.float64) / T)
    return e / e.sum()


def pseed(seed, pos):
    d = hashlib.blake2b(f"{seed}:{pos}".encode(), digest_size=8).digest()
    return int.from_bytes(d, "little") & ((1 << 63) - 1)


def main():
    p1 = softmax(LOGITS, 1.0)
    top3 = np.zeros(6)
    top3[:3] = p1[:3] / p1[:3].sum()
    out = {
        "LOGITS": LOGITS,
        "greedy": {"logits": [0.1, 3.0, -2.0], "token": 1},
        "softmax_T1": p1.tolist(),
        "softmax_T0.5": softmax(LOGITS, 0.5).tolist(),
        "top_p_0.8": {"kept": 3, "probs": top3.tolist()},
        "top_k_3": {"probs": top3.tolist()},
        "top_k_2": {"kept": 2},
        "top_p_1e-6": {"kept": 1},
        "zero_noise": {"logits": [5.0, 4.0, 3.0, 2.0, 1.0], "top_k_2_in": [0, 1], "top_p_0.5": 0},
        "position_seed": {f"{s}:{p}": pseed(s, p) for s, p in [(7, 0), (7, 1), (7, 2), (8, 0), (0, 0)]},
    }
    path = Path(__file__).with_name("known_answers.json")
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(path)


if __name__ == "__main__":
    main()
