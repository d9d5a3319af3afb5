"""Writes the golden fixtures of tests/golden/ with the CPU oracle (no reference code runs: the reference's search
exists only as CUDA and cannot run here).  The fixtures pin the oracle's outputs against drift and are replayed
against the HIP kernels on the GPU box.

    python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402


def e8():
    g = np.random.default_rng(11)
    b = 4
    y = g.uniform(-7, 7, (2048, 8 * b)).astype(np.float32)
    y[:256] = np.round(y[:256] * 2) * 0.5  # half-integer ties
    y[256:384] = np.round(y[256:384])
    inv_f = np.float32(1.0 / 2.5)
    p, h = O.e8_batch(y, b, float(inv_f))
    np.savez_compressed(os.path.join(HERE, "e8.npz"), y=y, b=b, inv_f=inv_f, p=p, h=h)


def scores():
    g = np.random.default_rng(12)
    S, D, n = 64, 96, 64
    code = g.integers(-127, 128, (n, S)).astype(np.int8)
    scale = np.tile(g.uniform(0.01, 0.1, S).astype(np.float32), (n, 1))
    qs = g.standard_normal((n, S)).astype(np.float32)
    sketch = np.array([O.sketch_dist(c, s, q) for c, s, q in zip(code, scale, qs)], np.float32)
    x = g.standard_normal((n, D)).astype(np.float16).view(np.uint16)
    q = g.standard_normal((n, D)).astype(np.float32)
    exact = np.array([O.exact_dist(a, b) for a, b in zip(x, q)], np.float32)
    np.savez_compressed(os.path.join(HERE, "scores.npz"), code=code, scale=scale, qs=qs, sketch=sketch, x=x, q=q,
                        exact=exact)


if __name__ == "__main__":
    e8()
    scores()
    print("golden fixtures written to", HERE)
