"""The GPU index builder (octex::build / cuvsOctexBuild / octexBuildInMemory): the format-1 directory it writes
(design.md:27-54), the invariants of its cells and lists, recall of the built index (test_build.py:48-66 of the
reference: >= 0.95 on clustered data with 64 copies), save / load round trips, and search parity with the CPU
oracle on the built index."""

import json
import os

import numpy as np
import pytest
from conftest import clustered, exact_knn, recall

from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def octex():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import octex_amd

    return octex_amd


@pytest.fixture(scope="module")
def data():
    X, Q = clustered()  # 20k x 64, 50 clusters (tests/conftest.py of the reference)
    gt, _ = exact_knn(X.astype(np.float16).astype(np.float32), Q)
    return X, Q, gt


@pytest.fixture(scope="module")
def built(octex, data, tmp_path_factory):
    X, Q, gt = data
    path = str(tmp_path_factory.mktemp("octex") / "index")
    index = octex.build(X, path, copies=64, seed=1, log_buckets=16, min_cell=4)
    return index, path


def test_build_writes_directory(built, data):
    index, path = built
    X = data[0]
    meta = json.load(open(os.path.join(path, "meta.json")))
    assert meta["format"] == 1 and meta["n"] == len(X) and meta["dim"] == X.shape[1]
    assert meta["copies"] == 64 and meta["metric"] == "sqeuclidean" and meta["spacings"] == [2.0, 2.5, 3.2, 4.0, 5.0]
    assert index.size == len(X) and index.dim == X.shape[1] and index.copies == 64
    C, L, n, d, S = 64, 5, len(X), X.shape[1], meta["sketch_width"]
    assert S == 64 and meta["table_len"] == 64
    for name, shape in dict(mean=(d,), proj=(C, d, 32), shift=(C, 32), base=(C, L), cells=(C, L), sketch=(n, S),
                            sketch_basis=(d, S), sketch_scale=(S,), vectors=(n, d), table=(n, 64)).items():
        assert np.load(os.path.join(path, name + ".npy"), mmap_mode="r").shape == shape, name
    assert np.array_equal(np.load(os.path.join(path, "vectors.npy")), X.astype(np.float16))


def test_cells_and_lists(built, data):
    """Keys in (bucket, id) order with CSR offsets; every list entry a member of its cell (its projection hashes
    to the cell's id), nearest to the cell center first; the table holds no self or out-of-range ids."""
    _, path = built
    ix = O.Index(path)
    X = data[0]
    T = 2 ** ix.log_buckets
    cells = np.load(os.path.join(path, "cells.npy"))
    Xh = X.astype(np.float16).astype(np.float32)
    hits = total = 0
    for c in (0, 17, 63):
        proj = np.load(os.path.join(path, "proj.npy"))[c]
        shift = np.load(os.path.join(path, "shift.npy"))[c]
        y = ((Xh - ix.mean) @ proj + shift).astype(np.float32)
        for j, f in enumerate(ix.spacings):
            M = cells[c, j]
            keys = ix.keys[c, j, :M]
            b = keys & (T - 1)
            assert (np.diff(b) >= 0).all()
            assert np.array_equal(np.searchsorted(b, np.arange(T + 1)), ix.offsets[c, j])
            _, h = O.e8_batch(y / np.float32(f), ix.blocks, 1.0)
            r0 = ix.base[c, j]
            rows = ix.lists[c, r0 * ix.list_len : (r0 + M) * ix.list_len].reshape(M, ix.list_len)
            hits += (h[rows] == keys[:, None]).sum()
            total += rows.size
            if j < len(ix.spacings) - 1:
                counts = np.bincount(np.searchsorted(np.sort(keys), h[np.isin(h, keys)]), minlength=M)
                assert counts.min() >= 4  # min_cell
    assert hits / total > 0.99
    tab = ix.table
    assert (tab < len(X)).all() and (tab != np.arange(len(X))[:, None]).all()


def test_build_recall(built, data):
    index, _ = built
    X, Q, gt = data
    D, I = index.search(Q, k=10)
    assert recall(I, gt) >= 0.95
    exact = ((X.astype(np.float16).astype(np.float64)[I] - Q[:, None, :]) ** 2).sum(-1)
    assert np.allclose(D, exact, rtol=1e-3, atol=1e-2)


def test_built_index_matches_oracle(built, data):
    index, path = built
    X, Q, _ = data
    oix = O.Index(path)
    from test_gpu_search import assert_same_results, oracle_given_gpu_projections

    D, I = index.search(Q, k=10, read=16, starts=64, waves=2)
    Do, Io, _, _, _ = oracle_given_gpu_projections(index, oix, Q, 10, read=16, starts=64, waves=2)
    assert_same_results(D, I, Do, Io)


def test_save_load_round_trip(octex, built, data, tmp_path):
    index, _ = built
    X, Q, _ = data
    D, I = index.search(Q, k=10)
    index.save(tmp_path / "copy")
    with pytest.raises(FileExistsError):
        index.save(tmp_path / "copy")
    again = octex.load(tmp_path / "copy", placement="replicate")
    D2, I2 = again.search(Q, k=10)
    assert np.array_equal(I, I2) and np.array_equal(D, D2)


def test_build_in_memory_equals_loaded(octex, built, data, tmp_path):
    """The in-memory build gives the same index, and the same results, as building then loading."""
    X, Q, _ = data
    mem, secs = octex.build_in_memory(X[:5000], tmp_path / "mem", copies=16, seed=3, log_buckets=14, table_len=32)
    assert secs > 0
    loaded = octex.load(tmp_path / "mem")
    D1, I1 = mem.search(Q, k=10, read=16, starts=64)
    D2, I2 = loaded.search(Q, k=10, read=16, starts=64)
    assert np.array_equal(I1, I2) and np.array_equal(D1, D2)


def test_build_inputs(octex, data, tmp_path):
    """float16 and device (torch) datasets build the same index as float32 host data."""
    X = data[0][:3000]
    a, _ = octex.build_in_memory(X, copies=8, seed=2, log_buckets=12, table_len=16)
    xf = torch.from_numpy(X).cuda()
    b, _ = octex.build_in_memory(xf, copies=8, seed=2, log_buckets=12, table_len=16)
    c, _ = octex.build_in_memory(X.astype(np.float16), copies=8, seed=2, log_buckets=12, table_len=16)
    xh = xf.half()
    e, _ = octex.build_in_memory(xh, copies=8, seed=2, log_buckets=12, table_len=16)
    Q = data[1]
    r = [ix.search(Q, k=10, read=16, starts=32) for ix in (a, b, c, e)]
    for D, I in r[1:]:
        assert np.array_equal(I, r[0][1]) and np.array_equal(D, r[0][0])


def test_build_errors(octex, data, tmp_path):
    from octex_amd._lib import OctexError

    X = data[0][:100]
    with pytest.raises(OctexError, match="fewer vectors than the list length"):
        octex.build(X[:10], tmp_path / "a", copies=2)
    with pytest.raises(OctexError, match="pca_dims must be at least 8 \\* blocks"):
        octex.build(X, tmp_path / "b", copies=2, pca_dims=16, list_len=8, table_len=8)
    with pytest.raises(OctexError, match="exact_lists is not supported"):
        octex.build(X, tmp_path / "c", copies=2, exact_lists=True, list_len=8, table_len=8)
