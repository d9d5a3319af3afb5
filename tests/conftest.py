"""Shared fixtures: seeded data generators, small test indexes written by the CPU oracle's builder, and the gpu
marker.  Tests marked `gpu` need an MI355X and the built liboctex_amd.so; the others run on the CPU."""

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running")


def recall(I, gt, k=10):
    I, gt = np.asarray(I)[:, :k], np.asarray(gt)[:, :k]
    return float(np.mean([len(set(a) & set(b)) / k for a, b in zip(I, gt)]))


def clustered(n=20_000, m=200, d=64, clusters=50, seed=0):
    """A Gaussian mixture dataset and queries (tests/conftest.py:55-63 of the reference)."""
    g = np.random.default_rng(seed)
    centers = g.standard_normal((clusters, d), dtype=np.float32) * 4
    X = (centers[g.integers(clusters, size=n)] + g.standard_normal((n, d), dtype=np.float32)).astype(np.float32)
    Q = (centers[g.integers(clusters, size=m)] + g.standard_normal((m, d), dtype=np.float32)).astype(np.float32)
    return X, Q


def exact_knn(X, Q, k=10):
    """Exact k nearest neighbors by fp64 squared L2 (ties by id)."""
    X64, Q64 = X.astype(np.float64), Q.astype(np.float64)
    d2 = (Q64**2).sum(1)[:, None] - 2 * Q64 @ X64.T + (X64**2).sum(1)[None, :]
    idx = np.argsort(d2, axis=1, kind="stable")[:, :k]
    return idx, np.take_along_axis(d2, idx, 1)


@pytest.fixture(scope="session")
def small_index(tmp_path_factory):
    """A 4000 x 64 clustered index (16 copies, member lists, exact table with reverse edges) built by the
    oracle, its queries and the exact neighbors of the fp16-rounded vectors."""
    from oracle import oracle as O

    X, Q = clustered(n=4000, m=100, d=64, clusters=20, seed=3)
    path = str(tmp_path_factory.mktemp("octex") / "small")
    O.build(X, path, copies=16, list_len=32, table_len=32, log_buckets=12, member_lists=True, seed=1)
    Xh = X.astype(np.float16).astype(np.float32)
    gt, _ = exact_knn(Xh, Q)
    return dict(path=path, X=X, Q=Q, gt=gt)


@pytest.fixture(scope="session")
def wide_index(tmp_path_factory):
    """A 2000 x 96 index with sketch width 96 (Lr = 8 lanes), 3 blocks, exact lists, no reverse edges."""
    from oracle import oracle as O

    X, Q = clustered(n=2000, m=64, d=96, clusters=12, seed=5)
    path = str(tmp_path_factory.mktemp("octex") / "wide")
    O.build(X, path, copies=8, blocks=3, pca_dims=48, list_len=16, table_len=24, log_buckets=10, sketch_width=96,
            exact_lists=True, reverse_edges=False, seed=2)
    return dict(path=path, X=X, Q=Q)
