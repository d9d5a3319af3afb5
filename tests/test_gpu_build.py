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


def check_cells_and_lists(path, X, copies, members):
    """Keys in (bucket, id) order with CSR offsets, cells of at least min_cell (4) rows; list entries valid distinct
    rows, and with `members` every entry a member of its cell (its projection hashes to the cell's id); the table
    holds no self or out-of-range ids."""
    ix = O.Index(path)
    T = 2 ** ix.log_buckets
    cells = np.load(os.path.join(path, "cells.npy"))
    Xh = X.astype(np.float16).astype(np.float32)
    hits = total = 0
    for c in copies:
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
            assert (rows >= 0).all() and (rows < len(X)).all()
            if not members:
                assert all(len(set(r)) == ix.list_len for r in rows[:: max(1, M // 50)].tolist())
            hits += (h[rows] == keys[:, None]).sum()
            total += rows.size
            if j < len(ix.spacings) - 1:
                counts = np.bincount(np.searchsorted(np.sort(keys), h[np.isin(h, keys)]), minlength=M)
                assert counts.min() >= 4  # min_cell
    if members:
        assert hits / total > 0.99
    tab = ix.table
    assert (tab < len(X)).all() and (tab != np.arange(len(X))[:, None]).all()


def test_cells_and_lists(built, data):
    """The default build (IVF lists): cells, CSR and lists of valid distinct rows."""
    check_cells_and_lists(built[1], data[0], (0, 17, 63), members=False)


def test_member_lists_hold_members(octex, data, tmp_path):
    """member_lists: every list entry a member of its cell, nearest to the cell center first."""
    X = data[0]
    path = str(tmp_path / "members")
    octex.build(X, path, copies=8, seed=1, log_buckets=16, min_cell=4, member_lists=True)
    check_cells_and_lists(path, X, (0, 3, 7), members=True)


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
    X = data[0][:300]
    with pytest.raises(OctexError, match="exact lists take list_len <= 128"):
        octex.build(X, tmp_path / "c", copies=2, exact_lists=True, list_len=129, table_len=8)
    with pytest.raises(OctexError, match="table_len <= 127"):
        octex.build(X, tmp_path / "d", copies=2, list_len=8, table_len=128)


def _table(path):
    return np.load(os.path.join(path, "table.npy"))


@pytest.mark.parametrize("n,d,reverse", [(3000, 32, True), (3000, 32, False), (2500, 30, True), (100, 32, True)])
def test_exact_table_matches_oracle(octex, tmp_path, n, d, reverse):
    """The exact neighbor table (build_table.cuh:57-142, 529-554) of integer-valued rows, whose squared
    distances are exact in fp32 and fp64 alike, equals the oracle's row for row: brute force with ties
    by id, the row itself dropped, reverse edges merged by the half rule and ordered nearest first.
    d = 30 takes the kernel's unaligned loads, n = 100 a single partial step."""
    g = np.random.default_rng(n + d)
    X = g.integers(0, 8, size=(n, d)).astype(np.float32)
    b = 4 if d >= 32 else 3
    kw = dict(copies=2, blocks=b, pca_dims=d, list_len=8, table_len=16, log_buckets=10, member_lists=True,
              reverse_edges=reverse, seed=1)
    octex.build(X, tmp_path / "gpu", **kw)
    O.build(X, str(tmp_path / "cpu"), **kw)
    tg, tc = _table(tmp_path / "gpu"), _table(tmp_path / "cpu")
    assert tg.shape == (n, 16)
    assert np.array_equal(tg, tc)


def test_exact_table_real_valued(octex, data, tmp_path):
    """On real-valued rows the forward table holds the exact k nearest (fp64) up to near ties of the
    fp32 expanded distance |x|^2 + |y|^2 - 2 x.y, nearest first; no self, no duplicates."""
    X = data[0][:4000]
    k = 24
    octex.build(X, tmp_path / "gpu", copies=2, list_len=8, table_len=k, log_buckets=10, reverse_edges=False, seed=1)
    tg = _table(tmp_path / "gpu")
    Xh = X.astype(np.float16).astype(np.float64)
    d2 = (Xh**2).sum(1)[:, None] - 2 * Xh @ Xh.T + (Xh**2).sum(1)[None, :]
    np.fill_diagonal(d2, np.inf)
    kth = np.sort(d2, axis=1)[:, k - 1]
    got = np.take_along_axis(d2, tg.astype(np.int64), 1)
    assert (tg >= 0).all() and (tg != np.arange(len(X))[:, None]).all()
    assert all(len(set(r)) == k for r in tg)
    assert (got <= kth[:, None] * (1 + 1e-5) + 1e-3).all()
    assert (np.diff(got, axis=1) >= -1e-3 * got[:, 1:]).all()


def test_searched_table_when_over_exact_max(octex, data):
    """Above exact_table_max the table comes from the library's own search (build_table.cuh:557-843): rows
    without self or duplicates, and an index that still reaches the reference's recall bar."""
    X, Q, _ = data
    X = X[:6000]
    idx, _ = octex.build_in_memory(X, copies=32, seed=4, log_buckets=14, table_len=32, min_cell=4, exact_table_max=0)
    tab = idx.array("table", np.int32).reshape(len(X), 32)
    assert (tab < len(X)).all() and (tab != np.arange(len(X))[:, None]).all()
    gt, _ = exact_knn(X.astype(np.float16).astype(np.float32), Q)
    D, I = idx.search(Q, k=10)
    assert recall(I, gt) >= 0.95


def test_exact_lists(octex, tmp_path):
    """exact_lists (build_cells.cuh:506-510, 567-599): the list of every cell holds the l projected rows
    nearest to the cell's center (f times the E8 point of a member's projection / f), among all rows,
    up to near ties of fp32 distances; member_lists takes precedence."""
    from test_oracle import check_exact_lists

    X, _ = clustered(n=2000, m=10, d=32, clusters=10, seed=9)
    path = str(tmp_path / "ex")
    octex.build(X, path, copies=2, list_len=16, table_len=8, log_buckets=10, exact_lists=True, seed=5)
    assert check_exact_lists(path, X) > 50


def test_ivf_lists_probing_every_list_are_exact(octex, tmp_path):
    """The default lists (IVF, build_cells.cuh:511-516, 584-596) with every k-means list probed: each cell's list is
    the l rows nearest to its center among all rows (1,000 rows: max(64, 4 sqrt(n)) = 126 lists, list_probes 200)."""
    from test_oracle import check_exact_lists

    X, _ = clustered(n=1000, m=10, d=32, clusters=10, seed=9)
    path = str(tmp_path / "ivf_all")
    octex.build(X, path, copies=2, list_len=16, table_len=8, log_buckets=10, list_probes=200, seed=5)
    assert check_exact_lists(path, X) > 50


def test_ivf_lists_default_probes(octex, tmp_path):
    """The default lists with the default 16 probes of 565 lists (20,000 rows): l distinct rows per cell, most of
    them among the l nearest to the cell's center, and the same index on every build (the k-means sums and the list
    merges run in a fixed order)."""
    from test_oracle import check_exact_lists

    X, Q = clustered(n=20_000, m=100, d=32, clusters=40, seed=10)
    path = str(tmp_path / "ivf16")
    octex.build(X, path, copies=2, list_len=16, table_len=16, log_buckets=12, seed=5)
    assert check_exact_lists(path, X, stride=20, fraction=True) > 0.9
    again = str(tmp_path / "ivf16b")
    octex.build(X, again, copies=2, list_len=16, table_len=16, log_buckets=12, seed=5)
    assert np.array_equal(np.load(os.path.join(path, "lists.npy")), np.load(os.path.join(again, "lists.npy")))


def test_exact_table_reference_rule(octex, tmp_path):
    """The GPU builder's exact table with reverse edges meets the reference's own test of it
    (test_build.cu:266-377, mode 0)."""
    from test_oracle import check_exact_table, table_mode_data

    x, k = table_mode_data(), 12
    octex.build(x, tmp_path / "t", copies=2, blocks=2, pca_dims=16, list_len=8, log_buckets=10, sketch_width=16,
                table_len=k, reverse_edges=True, seed=0)
    check_exact_table(_table(tmp_path / "t"), x, k)


def test_place_on_host_keeps_results(octex, data):
    """Vectors, table and sketch moved to pinned host memory after an in-memory build (the load placements
    vectors_on_host, table_on_host, sketch = host) give the same results, in both search modes, with the
    device bytes reduced by their size."""
    X, Q, _ = data
    X = X[:5000]
    idx, _ = octex.build_in_memory(X, copies=16, seed=6, log_buckets=12, table_len=32)
    p = dict(read=16, starts=64, waves=2)
    ps = dict(p, sketch_rank=True, final_rerank=32)
    before = [idx.search(Q, k=10, **p), idx.search(Q, k=10, **ps)]
    dev0 = idx.device_bytes[0]
    idx.place_on_host(vectors=True, table=True, sketch=True)
    moved = len(X) * (64 * 2 + 32 * 4) + idx.array_size("sketch")
    assert idx.device_bytes[0] == dev0 - moved
    after = [idx.search(Q, k=10, **p), idx.search(Q, k=10, **ps)]
    for (D0, I0), (D1, I1) in zip(before, after):
        assert np.array_equal(I0, I1) and np.array_equal(D0, D1)
    idx.place_on_host(vectors=True)  # a second call moves nothing
    assert idx.device_bytes[0] == dev0 - moved


def same_cells(a, b, copies, lists=True):
    """The two indexes hold the same cells: keys, offsets and bases, and with `lists` the same list of every cell."""
    for name, dt in (("keys", np.int64), ("offsets", np.int32), ("base", np.int32)):
        assert np.array_equal(a.array(name, dt), b.array(name, dt)), name
    for c in range(copies if lists else 0):
        assert np.array_equal(a.array("lists", np.int32, copy=c), b.array("lists", np.int32, copy=c)), c


def test_streamed_build_equals_in_memory(octex, data, monkeypatch):
    """The streamed build (build_cells.cuh:756-1393, forced by OCTEX_BUILD_STREAM=1 as in the reference): vectors in
    pinned host memory, each copy's projection made in chunks, every level's member lists from each row's cell id
    and distance to its cell center.  It gives the same arrays and search results as the whole-projection build, with
    the vectors off the device.  OCTEX_BUILD_STREAM=0 forces the whole-projection build."""
    X, Q, _ = data
    X = X[:6000]
    args = dict(copies=12, seed=7, log_buckets=12, table_len=32, min_cell=3, member_lists=True)
    mem, _ = octex.build_in_memory(X, **args)
    monkeypatch.setenv("OCTEX_BUILD_STREAM", "1")
    st, _ = octex.build_in_memory(X, **args)
    for name, dt in (("keys", np.int64), ("offsets", np.int32), ("base", np.int32), ("sketch", np.int8),
                     ("table", np.int32)):
        assert np.array_equal(mem.array(name, dt), st.array(name, dt)), name
    for c in range(12):
        assert np.array_equal(mem.array("lists", np.int32, copy=c), st.array("lists", np.int32, copy=c)), c
    assert st.device_bytes[0] == mem.device_bytes[0] - len(X) * X.shape[1] * 2
    p = dict(read=16, starts=64, waves=2)
    (D0, I0), (D1, I1) = mem.search(Q, k=10, **p), st.search(Q, k=10, **p)
    assert np.array_equal(I0, I1) and np.array_equal(D0, D1)
    monkeypatch.setenv("OCTEX_BUILD_STREAM", "0")
    whole, _ = octex.build_in_memory(X, **args)
    assert whole.device_bytes[0] == mem.device_bytes[0]


def test_streamed_exact_lists_over_ranges(octex, data, monkeypatch):
    """Streamed exact lists (build_cells.cuh:1233-1335): each cell's center from its first row re-projected, the rows
    in three ranges (OCTEX_BUILD_RANGES=3), each range's brute-force lists merged.  The lists are those of one search
    over all rows: every array equals the whole-projection build's, and so do the search results (the reference's
    streaming test allows differences at distance ties; here the two share one distance computation)."""
    X, Q, _ = data
    X = X[:6000]
    args = dict(copies=6, seed=11, log_buckets=12, table_len=24, min_cell=3, exact_lists=True, list_len=32)
    mem, _ = octex.build_in_memory(X, **args)
    monkeypatch.setenv("OCTEX_BUILD_STREAM", "1")
    monkeypatch.setenv("OCTEX_BUILD_RANGES", "3")
    st, _ = octex.build_in_memory(X, **args)
    same_cells(mem, st, 6)
    assert st.device_bytes[0] == mem.device_bytes[0] - len(X) * X.shape[1] * 2
    p = dict(read=16, starts=32, waves=2)
    (D0, I0), (D1, I1) = mem.search(Q, k=10, **p), st.search(Q, k=10, **p)
    assert np.array_equal(I0, I1) and np.array_equal(D0, D1)


def test_streamed_ivf_lists(octex, data, tmp_path, monkeypatch):
    """Streamed IVF lists (the reference's default, build_cells.cuh:1269-1300): each row range gets its own k-means
    index, searched for every cell center with list_probes probes, the lists merged over the ranges.  One range gives
    the whole-projection build's index exactly.  Over three ranges the cells are the same, with every k-means list
    probed each list holds the l rows nearest to its center, and at the default 16 probes the search recall stays
    within 0.005 of the whole-projection build's (the reference's streaming bar, test_build_stream.cu:9-11)."""
    from test_oracle import check_exact_lists

    X, Q, _ = data
    X = X[:8000]
    gt, _ = exact_knn(X.astype(np.float16).astype(np.float32), Q)
    args = dict(copies=8, seed=13, log_buckets=12, table_len=24, min_cell=3, list_len=24)
    mem, _ = octex.build_in_memory(X, **args)
    monkeypatch.setenv("OCTEX_BUILD_STREAM", "1")
    one, _ = octex.build_in_memory(X, **args)
    same_cells(mem, one, 8)
    monkeypatch.setenv("OCTEX_BUILD_RANGES", "3")
    three, _ = octex.build_in_memory(X, **args)
    same_cells(mem, three, 8, lists=False)
    p = dict(read=8, starts=32, waves=2)
    r_mem, r_three = recall(mem.search(Q, k=10, **p)[1], gt), recall(three.search(Q, k=10, **p)[1], gt)
    assert r_three >= r_mem - 0.005, (r_mem, r_three)
    path = str(tmp_path / "ivf3")  # 3 ranges of 1,000 rows: 126 k-means lists each, all probed
    octex.build(X[:3000], path, **dict(args, copies=2, list_len=16, list_probes=200))
    assert check_exact_lists(path, X[:3000]) > 50


def test_write_behind_and_table_only_resume(octex, data, tmp_path, monkeypatch):
    """write_behind (build.cu:146-178): the arrays final before the neighbor table are written while the table is
    built: the same files as a build without it.  OCTEX_TABLE_ONLY=1 (build.cu:153-169) on a directory that stopped
    in its table phase (every array but table.npy and meta.json): only the table is built and written, the same
    table, and the directory loads with the same results."""
    X, Q, _ = data
    X = X[:5000]
    args = dict(copies=8, seed=3, log_buckets=12, table_len=24, min_cell=3, member_lists=True)
    plain, behind = str(tmp_path / "plain"), str(tmp_path / "behind")
    octex.build(X, plain, **args)
    octex.build(X, behind, write_behind=True, **args)
    names = sorted(f for f in os.listdir(plain) if f.endswith(".npy"))
    assert names == sorted(f for f in os.listdir(behind) if f.endswith(".npy")) and "table.npy" in names
    for f in names:
        assert open(os.path.join(plain, f), "rb").read() == open(os.path.join(behind, f), "rb").read(), f
    table = np.load(os.path.join(plain, "table.npy"))
    os.remove(os.path.join(behind, "table.npy"))
    os.remove(os.path.join(behind, "meta.json"))
    monkeypatch.setenv("OCTEX_TABLE_ONLY", "1")
    octex.build(X, behind, **args)
    monkeypatch.delenv("OCTEX_TABLE_ONLY")
    assert np.array_equal(np.load(os.path.join(behind, "table.npy")), table)
    meta = json.load(open(os.path.join(behind, "meta.json")))
    assert meta["table_len"] == 24 and meta["n"] == len(X) and list(meta["build_seconds"]) == ["table"]
    p = dict(read=16, starts=32, waves=2)
    (D0, I0), (D1, I1) = octex.load(plain).search(Q, k=10, **p), octex.load(behind).search(Q, k=10, **p)
    assert np.array_equal(I0, I1) and np.array_equal(D0, D1)


def test_write_behind_survives_a_table_phase_error(octex, data, tmp_path):
    """A table phase that throws (here the exact table's table_len limit, checked only in that phase) while the
    write-behind thread is still copying the index's arrays: the error reaches the caller, the writer finishes with
    its own reference to the index (no use of freed buffers), the arrays final before the table are on disk, and the
    next build and search work."""
    from octex_amd._lib import OctexError

    X, Q, _ = data
    X = X[:3000]
    bad = str(tmp_path / "bad")
    with pytest.raises(OctexError, match="table_len <= 127"):
        octex.build(X, bad, write_behind=True, copies=8, seed=3, log_buckets=12, list_len=8, table_len=128,
                    member_lists=True)
    assert not os.path.exists(os.path.join(bad, "meta.json"))  # incomplete: meta.json is written last
    for f in ("lists.npy", "keys.npy", "offsets.npy", "sketch.npy", "vectors.npy"):
        assert os.path.getsize(os.path.join(bad, f)) > 0, f
    assert np.load(os.path.join(bad, "vectors.npy")).shape == X.shape
    good = str(tmp_path / "good")
    index = octex.build(X, good, write_behind=True, copies=8, seed=3, log_buckets=12, list_len=8, table_len=16,
                        member_lists=True)
    D, I = index.search(Q, k=10, read=8, starts=32, waves=1)
    assert (I >= 0).all() and (np.diff(D, axis=1) >= 0).all()
