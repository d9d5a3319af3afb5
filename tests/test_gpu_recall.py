"""The reference's end-to-end recall contracts at its own search settings, on BASELINE.json configs[1]'s workload at
full size: 1M SIFT-like integer-valued rows x 128 (bench.py's generator, exact in fp16) and an index of bench.py's
sift1m shape built with member lists, the fast build (200 copies, lists of 32 of cells of >= 2 rows, exact neighbor
table of 64, no reverse edges), with the first 2,000 of its queries (the reference's end-to-end test takes at most
2,000).

- tests/test_recall.py:31-45: recall@10 >= 0.99 at read 8, starts 32, waves 1, and at the default search
  parameters, where the returned distances are the squared distances of the returned rows.
- test_search.cu:601-648: recall@10 > 0.94 with a quarter of the copies (copies_limit 50), read 8, starts 32,
  waves 1 and batches of 777 queries (several batches, the last one partial), every row's distances ascending.
"""

import time

import numpy as np
import pytest
from conftest import recall

import bench

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

NQ = 2000
INDEX = dict(copies=200, list_len=32, table_len=64, min_cell=2, reverse_edges=False, member_lists=True, seed=0)


@pytest.fixture(scope="module")
def octex():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import octex_amd

    return octex_amd


@pytest.fixture(scope="module")
def sift():
    t0 = time.time()
    X, Q = bench.make_data(bench.CONFIGS["sift1m"])
    Q = np.ascontiguousarray(Q[:NQ])
    top = bench.TopK(torch.from_numpy(Q).cuda(), 10, torch)
    Xd = torch.from_numpy(X).cuda()
    for r0 in range(0, len(X), 1 << 16):
        top.add(Xd[r0 : r0 + (1 << 16)], r0)
    del Xd
    print(f"data and exact neighbors: {time.time() - t0:.1f} s", flush=True)
    return X, Q, top.i.cpu().numpy()


@pytest.fixture(scope="module")
def index(octex, sift):
    X, _, _ = sift
    t0 = time.time()
    idx, secs = octex.build_in_memory(X, **INDEX)
    print(f"200-copy index: built in {secs:.1f} s ({time.time() - t0:.1f} s with the upload)", flush=True)
    return idx


def test_recall_light_settings(index, sift):
    _, Q, gt = sift
    D, I = index.search(Q, k=10, read=8, starts=32, waves=1)
    r = recall(I, gt)
    print(f"recall@10 (read 8, starts 32, waves 1): {r:.4f}", flush=True)
    assert r >= 0.99


def test_recall_defaults(index, sift):
    X, Q, gt = sift
    D, I = index.search(Q, k=10)
    r = recall(I, gt)
    print(f"recall@10 (defaults): {r:.4f}", flush=True)
    assert r >= 0.99
    # the distances are the squared Euclidean distances of the returned rows (integer rows: exact in fp16)
    rows = X[I[:20].ravel()].reshape(20, 10, -1)
    want = ((rows - Q[:20, None, :]) ** 2).sum(-1)
    np.testing.assert_allclose(D[:20], want, rtol=1e-3)


def test_end_to_end_quarter_of_the_copies(octex, index, sift):
    X, Q, gt = sift
    quarter, _ = octex.build_in_memory(X, **dict(INDEX, copies=50))
    # a copy's projection is drawn from (seed, copy) alone, so these are the first 50 copies of the 200-copy index:
    # what copies_limit = 50 loads of it
    for c in (0, 49):
        assert np.array_equal(quarter.array("lists", np.int32, copy=c), index.array("lists", np.int32, copy=c)), c
    D, I = quarter.search(Q, k=10, read=8, starts=32, waves=1, batch=777)
    r = recall(I, gt)
    print(f"recall@10 (50 copies, read 8, starts 32, waves 1, batch 777): {r:.4f}", flush=True)
    assert r > 0.94
    assert (np.diff(D, axis=1) >= 0).all()
