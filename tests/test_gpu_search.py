"""The whole search on the GPU through the cuvsOctex* C ABI, against the CPU oracle on the same index and queries.

Parity: given the GPU's own projections Y and sketch queries qs (read back from the search plan), the oracle's
search returns the same ids and bit-identical distances; against exact search, recall thresholds of the
reference's tests (test_build.py:48-54, octex_c.cu:196).  Batch splitting / padding, graph replay, device tensors,
sketch-rank mode and the parameter limits are covered too."""

import numpy as np
import pytest
from conftest import exact_knn, recall

from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def octex():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import octex_amd

    return octex_amd


PARAMS = dict(read=32, starts=64, waves=2, rerank=64, wave_rerank=64)


def oracle_given_gpu_projections(index, oix, Q, k, **params):
    """The oracle's search fed with the GPU plan's Y and qs of the last (single) batch."""
    info = index.plan_info()
    assert info["m"] == len(Q)
    C, w, S = oix.copies, oix.width, oix.sketch_width
    Y = index.plan_buffer("Y", np.uint16)[: len(Q) * C * w].reshape(len(Q), C * w)
    qs = index.plan_buffer("qs", np.float32)[: len(Q) * S].reshape(len(Q), S)
    D, I, tr = O.search(oix, Q, k=k, Y=Y, qs=qs, trace=True, **params)
    return D, I, tr, Y, qs


def assert_same_results(D, I, D2, I2):
    """Identical ids and distances, except where distances tie (then the ids at the tie may swap)."""
    assert np.array_equal(D, D2), "distances differ"
    diff = I != I2
    if diff.any():
        for q, j in zip(*np.nonzero(diff)):
            assert (D[q] == D[q, j]).sum() > 1, f"query {q} rank {j}: ids differ without a distance tie"


def test_search_matches_oracle(octex, small_index):
    index = octex.load(small_index["path"])
    oix = O.Index(small_index["path"])
    Q = small_index["Q"]
    D, I = index.search(Q, k=10, **PARAMS)
    Do, Io, tr, Y, qs = oracle_given_gpu_projections(index, oix, Q, 10, **PARAMS)
    assert_same_results(D, I, Do, Io)
    # stage by stage: probe segments, first-round candidate counts, the final kept list
    seg = index.plan_buffer("seg", np.int32)[: len(Q) * oix.copies * 2].reshape(len(Q), oix.copies, 2)
    assert np.array_equal(seg, tr["seg"])
    nin = index.plan_buffer("nin", np.int32)[: len(Q)]
    assert np.array_equal(nin, tr["n1"])
    KO = max(PARAMS["starts"], 10)
    sd = index.plan_buffer("sd", np.float32)[: len(Q) * KO].reshape(len(Q), KO)
    assert np.array_equal(sd, tr["sd"])
    # the projections themselves against the fp64 oracle: within one fp16 ulp
    qc, qh = O.center(Q, oix.mean)
    from test_gpu_stages import check_projection

    check_projection(Y, qh, oix.ucat, oix.shift)
    assert np.allclose(qs, O.sketch_query(qc, oix.basis), rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("sketch_rank", [False, True])
def test_large_wave_gather_matches_oracle(octex, small_index, sketch_rank):
    """starts 512 over table rows of 32 (configs[4]'s setting): the wave gather's hash set of 2^15 slots leaves
    no LDS for the candidates' slot list, which then lives in the query's row of cand; results as the oracle's."""
    index = octex.load(small_index["path"])
    oix = O.Index(small_index["path"])
    Q = small_index["Q"]
    assert oix.table_len == 32
    p = dict(read=16, starts=512, waves=2, rerank=128, wave_rerank=128, sketch_rank=sketch_rank, final_rerank=32)
    D, I = index.search(Q, k=10, **p)
    assert index.plan_info()["W2"] == 1 << 15
    Do, Io, tr, _, _ = oracle_given_gpu_projections(index, oix, Q, 10, **p)
    assert_same_results(D, I, Do, Io)


def test_search_recall_and_distances(octex, small_index):
    index = octex.load(small_index["path"])
    Q = small_index["Q"]
    D, I = index.search(Q, k=10, **PARAMS)
    assert recall(I, small_index["gt"]) >= 0.95
    Xh = small_index["X"].astype(np.float16).astype(np.float64)
    exact = ((Xh[I] - Q[:, None, :].astype(np.float64)) ** 2).sum(-1)
    assert np.allclose(D, exact, rtol=1e-3)
    assert (np.diff(D, axis=1) >= 0).all()


def test_batch_split_and_padding(octex, small_index):
    """Results do not depend on the batch size: batches of 37 (last one padded) equal one batch."""
    index = octex.load(small_index["path"])
    Q = small_index["Q"]
    D1, I1 = index.search(Q, k=10, batch=1000, **PARAMS)
    D2, I2 = index.search(Q, k=10, batch=37, **PARAMS)
    assert np.array_equal(I1, I2) and np.array_equal(D1, D2)


def test_graph_equals_direct_launches(octex, small_index):
    index = octex.load(small_index["path"])
    Q = small_index["Q"]
    D1, I1 = index.search(Q, k=10, **PARAMS)
    assert index.plan_info()["graph"] == 1
    D2, I2 = index.search(Q, k=10, use_graph=False, **PARAMS)
    assert index.plan_info()["graph"] == 0
    assert np.array_equal(I1, I2) and np.array_equal(D1, D2)
    for _ in range(3):  # replays of one graph, with eager work in between
        D3, I3 = index.search(Q, k=10, **PARAMS)
        assert np.array_equal(I1, I3) and np.array_equal(D1, D3)


def test_concurrent_searches(octex, small_index):
    """Threads searching one index with different parameter sets (each call evicts the other's cached plan,
    search.cu:804-813, while that plan's batch may still run) get the results of serial searches."""
    import threading

    index = octex.load(small_index["path"])
    Q = small_index["Q"]
    sets = [dict(k=10, **PARAMS), dict(k=5, read=8, starts=32, waves=1), dict(k=10, batch=37, **PARAMS)]
    want = [index.search(Q, **p) for p in sets]
    errors = []

    def worker(t):
        try:
            for r in range(6):
                j = (t + r) % len(sets)
                D, I = index.search(Q, **sets[j])
                if not (np.array_equal(I, want[j][1]) and np.array_equal(D, want[j][0])):
                    errors.append((t, r, j))
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append((t, repr(e)))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(3)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors


class _Foreign:
    """An array of a framework octex_amd does not know, exporting DLPack only (as CuPy's arrays do)."""

    __module__ = "fakearrays"

    def __init__(self, t):
        self.t = t

    def __dlpack__(self, **kw):
        return self.t.__dlpack__(**kw)

    def __dlpack_device__(self):
        return self.t.__dlpack_device__()


def test_foreign_arrays(octex, small_index, monkeypatch):
    """Queries of another framework are searched without a copy and answered in that framework (through its
    module's from_dlpack, octex/_arrays.py); given output arrays of it are written (int32 ids too)."""
    import sys
    import types

    mod = types.ModuleType("fakearrays")
    mod.from_dlpack = lambda x: _Foreign(torch.from_dlpack(x))
    monkeypatch.setitem(sys.modules, "fakearrays", mod)
    index = octex.load(small_index["path"])
    Q = small_index["Q"]
    D1, I1 = index.search(Q, k=10, **PARAMS)
    q = _Foreign(torch.from_numpy(Q).cuda())
    D2, I2 = index.search(q, k=10, **PARAMS)
    assert isinstance(D2, _Foreign) and isinstance(I2, _Foreign) and I2.t.is_cuda
    assert np.array_equal(I1, I2.t.cpu().numpy()) and np.array_equal(D1, D2.t.cpu().numpy())
    nb = _Foreign(torch.empty((len(Q), 10), dtype=torch.int32, device="cuda"))
    ds = _Foreign(torch.empty((len(Q), 10), dtype=torch.float32, device="cuda"))
    D3, I3 = index.search(q, k=10, neighbors=nb, distances=ds, **PARAMS)
    assert I3 is nb and D3 is ds
    assert np.array_equal(nb.t.cpu().numpy(), I1) and np.array_equal(ds.t.cpu().numpy(), D1)
    host_ids = np.empty((len(Q), 10), np.uint32)  # numpy outputs of device queries
    index.search(torch.from_numpy(Q).cuda(), k=10, neighbors=host_ids, **PARAMS)
    assert np.array_equal(host_ids, I1)


def test_device_tensors(octex, small_index):
    index = octex.load(small_index["path"])
    Q = small_index["Q"]
    D1, I1 = index.search(Q, k=10, **PARAMS)
    D2, I2 = index.search(torch.from_numpy(Q).cuda(), k=10, **PARAMS)
    assert D2.is_cuda and I2.dtype == torch.int64
    assert np.array_equal(I1, I2.cpu().numpy()) and np.array_equal(D1, D2.cpu().numpy())


def test_search_on_a_side_stream(octex, small_index):
    """Device queries written on a torch side stream (after long work on it) are searched on that stream: the
    search waits for them, and its results are ready on that stream, as a serial host search's."""
    index = octex.load(small_index["path"])
    Q = small_index["Q"]
    D1, I1 = index.search(Q, k=10, **PARAMS)
    side = torch.cuda.Stream()  # default priority
    with torch.cuda.stream(side):
        q = torch.zeros(Q.shape, dtype=torch.float32, device="cuda")
        src = torch.from_numpy(Q).cuda()
        a = torch.randn((4096, 4096), device="cuda")
        for _ in range(12):  # keeps the side stream busy before the queries are written
            a = torch.mm(a, a) * 1e-3
        q.copy_(src + a[:1, :1] * 0)
        D2, I2 = index.search(q, k=10, **PARAMS)
        D2, I2 = D2.cpu().numpy(), I2.cpu().numpy()
    assert np.array_equal(I1, I2) and np.array_equal(D1, D2)
    torch.cuda.synchronize()


def test_sketch_rank_matches_oracle(octex, small_index):
    index = octex.load(small_index["path"])
    oix = O.Index(small_index["path"])
    Q = small_index["Q"]
    p = dict(read=16, starts=96, waves=2, sketch_rank=True, final_rerank=48)
    D, I = index.search(Q, k=10, **p)
    Do, Io, _, _, _ = oracle_given_gpu_projections(index, oix, Q, 10, **p)
    assert_same_results(D, I, Do, Io)
    p0 = dict(p, final_rerank=0)  # sketch order, sketch distances out
    D, I = index.search(Q, k=10, **p0)
    Do, Io, _, _, _ = oracle_given_gpu_projections(index, oix, Q, 10, **p0)
    assert_same_results(D, I, Do, Io)


def test_waves_zero_and_k_above_starts(octex, small_index):
    index = octex.load(small_index["path"])
    oix = O.Index(small_index["path"])
    Q = small_index["Q"][:50]
    for p, k in ((dict(read=8, starts=32, waves=0), 10), (dict(read=32, starts=8, waves=1), 20)):
        D, I = index.search(Q, k=k, **p)
        Do, Io, _, _, _ = oracle_given_gpu_projections(index, oix, Q, k, **p)
        assert_same_results(D, I, Do, Io)


def test_wide_index_matches_oracle(octex, wide_index):
    """Sketch width 96 (8 lanes per candidate, two of them idle), 3 blocks, dimension 96."""
    index = octex.load(wide_index["path"])
    oix = O.Index(wide_index["path"])
    Q = wide_index["Q"]
    D, I = index.search(Q, k=10, **PARAMS)
    Do, Io, _, _, _ = oracle_given_gpu_projections(index, oix, Q, 10, **PARAMS)
    assert_same_results(D, I, Do, Io)
    gt, _ = exact_knn(wide_index["X"].astype(np.float16).astype(np.float32), Q)
    assert recall(I, gt) >= 0.9


def test_load_limits_match_oracle(octex, small_index):
    index = octex.load(small_index["path"], copies_limit=5, list_limit=8)
    assert index.copies == 5
    oix = O.Index(small_index["path"], copies_limit=5, list_limit=8)
    Q = small_index["Q"][:40]
    D, I = index.search(Q, k=10, **PARAMS)
    Do, Io, _, _, _ = oracle_given_gpu_projections(index, oix, Q, 10, **PARAMS)
    assert_same_results(D, I, Do, Io)


def test_probe_without_bucket_lines(octex, small_index, monkeypatch):
    """The search's probe reads each bucket's line (first key and key range) when the index has its bucket lines,
    the offsets and keys otherwise (OCTEX_PROBE_LINES=0 at load): the same segments and results, and the lines are
    C L 2^log_buckets 16-byte entries of device memory."""
    oix = O.Index(small_index["path"])
    Q = small_index["Q"][:60]
    a = octex.load(small_index["path"])
    Da, Ia = a.search(Q, k=10, **PARAMS)
    seg_a = a.plan_buffer("seg", np.int32)[: len(Q) * oix.copies * 2].copy()
    monkeypatch.setenv("OCTEX_PROBE_LINES", "0")
    b = octex.load(small_index["path"])
    Db, Ib = b.search(Q, k=10, **PARAMS)
    seg_b = b.plan_buffer("seg", np.int32)[: len(Q) * oix.copies * 2]
    assert np.array_equal(seg_a, seg_b) and np.array_equal(Ia, Ib) and np.array_equal(Da, Db)
    lines = oix.copies * len(oix.spacings) * 2**oix.log_buckets * 16
    assert a.device_bytes[0] - b.device_bytes[0] == lines


@pytest.mark.parametrize("mode", ["1", "prev", "all"])
def test_wave_gathers_with_and_without_earlier_scores(octex, small_index, monkeypatch, mode):
    """The first wave's gather takes the scores of candidates found in the first round's row; with prev every wave from
    the previous round's row, with all the later waves also from the first round's.  With OCTEX_GATHER_REUSE=0 (read
    when a plan is made) they score every candidate: the same results, and the profile counts the candidates found
    (three waves)."""
    Q = small_index["Q"][:60]
    params = dict(PARAMS, waves=3)
    monkeypatch.setenv("OCTEX_GATHER_REUSE", mode)
    a = octex.load(small_index["path"])
    Da, Ia = a.search(Q, k=10, **params)
    _, cnt = a.profile_batch(Q, k=10, reps=1, **params)
    monkeypatch.setenv("OCTEX_GATHER_REUSE", "0")
    b = octex.load(small_index["path"])
    Db, Ib = b.search(Q, k=10, **params)
    _, cnt0 = b.profile_batch(Q, k=10, reps=1, **params)
    assert np.array_equal(Ia, Ib) and np.array_equal(Da, Db)
    used = 3 if mode != "1" else 1  # the waves that read earlier rows
    assert all(k > 0 for k in cnt["known2"][:used]) and all(o > 0 for o in cnt["oldread2"][:used])
    assert sum(cnt["known2"][used:]) == 0 and sum(cnt["oldread2"][used:]) == 0
    assert sum(cnt0["known2"]) == 0 and sum(cnt0["oldread2"]) == 0
    assert cnt["distinct2"][:3] == cnt0["distinct2"][:3]


def test_placements_on_host(octex, small_index):
    """Vectors, table and sketch in pinned host memory give the same results."""
    Q = small_index["Q"][:40]
    D1, I1 = octex.load(small_index["path"]).search(Q, k=10, **PARAMS)
    index = octex.load(small_index["path"], vectors_on_host=True, table_on_host=True, sketch="host")
    D2, I2 = index.search(Q, k=10, **PARAMS)
    assert np.array_equal(I1, I2) and np.array_equal(D1, D2)


def test_errors(octex, small_index):
    from octex_amd._lib import OctexError

    index = octex.load(small_index["path"])
    Q = small_index["Q"][:4]
    with pytest.raises(ValueError, match="dimension"):
        index.search(Q[:, :10], k=10)
    with pytest.raises(OctexError, match="max\\(starts, k\\) must be <= 512"):
        index.search(Q, k=10, starts=600)
    with pytest.raises(OctexError, match="read, starts >= 1"):
        index.search(Q, k=10, read=0)
    with pytest.raises(FileNotFoundError):
        octex.load(small_index["path"] + "_missing")
    assert index.size == 4000 and index.dim == 64 and index.copies == 16 and len(index.devices) == 1
    assert index.device_bytes[0] > 0


def test_oracle_index_with_probed_rows_only(octex, small_index):
    """The host copy that keeps only the list rows a sample's probes reach (the CPU baseline of an index
    too large for host memory) searches that sample exactly like the full copy; array ranges read the
    same bytes as whole arrays and reject ranges outside them."""
    from octex_amd._lib import OctexError

    index = octex.load(small_index["path"])
    Q = small_index["Q"][:50]
    full = O.Index(index)
    part = O.Index(index, queries=Q, read=PARAMS["read"])
    assert (part.lists != 0).sum() < (full.lists != 0).sum()
    D1, I1 = O.search(full, Q, k=10, **PARAMS)
    D2, I2 = O.search(part, Q, k=10, **PARAMS)
    assert np.array_equal(I1, I2) and np.array_equal(D1, D2)
    lists3 = index.array("lists", np.int32, copy=3)
    assert np.array_equal(index.array_range("lists", np.int32, 100, 37, copy=3), lists3[100:137])
    assert index.array_size("lists", copy=3) == lists3.nbytes
    starts = np.array([0, 64, 7, len(lists3) - 16])
    got = index.array_ranges("lists", np.int32, starts, 16, copy=3)
    assert np.array_equal(got, np.stack([lists3[s : s + 16] for s in starts]))
    with pytest.raises(OctexError, match="outside the array"):
        index.array_ranges("lists", np.int32, [len(lists3) - 8], 16, copy=3)
    with pytest.raises(OctexError, match="outside the array"):
        index.array_range("lists", np.int32, len(lists3) - 2, 3, copy=3)
