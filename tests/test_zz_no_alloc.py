"""octexSearchNoAlloc: the search of device queries with every per-batch buffer in the library's file-scope
scratch array (no device allocation, direct launches on the caller's stream), against cuvsOctexSearch on the
same index and queries: identical ids and distances on two calls in a row (the second smaller, so the scratch
holds the first call's contents), with several batches and a partial last one, in both rank modes; a batch that
does not fit the scratch is refused before any launch."""

import ctypes as ct

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

PARAMS = dict(read=32, starts=64, waves=2, rerank=64, wave_rerank=64)


@pytest.fixture(scope="module")
def octex():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import octex_amd

    return octex_amd


def call_no_alloc(index, q, I, D, **params):
    """octexSearchNoAlloc through the C ABI on torch's current stream, into the device outputs I, D; no sync."""
    from octex_amd import _lib
    from octex_amd import index as octex_index

    p = octex_index.search_params(**params)
    n, d = q.shape
    stream = ct.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.call("octexSearchNoAlloc", ct.byref(p), index.handle, ct.c_void_p(q.data_ptr()), ct.c_int64(n),
              ct.c_int64(d), ct.c_int64(I.shape[1]), ct.c_void_p(I.data_ptr()), ct.c_void_p(D.data_ptr()), stream)


def no_alloc(index, q, k, **params):
    """octexSearchNoAlloc on torch's current stream; results on the host."""
    n = q.shape[0]
    I = torch.full((n, k), -7, dtype=torch.int64, device="cuda")
    D = torch.full((n, k), float("nan"), dtype=torch.float32, device="cuda")
    call_no_alloc(index, q, I, D, **params)
    torch.cuda.synchronize()
    return D.cpu().numpy(), I.cpu().numpy()


@pytest.mark.parametrize("extra", [dict(), dict(sketch_rank=True, final_rerank=32), dict(batch=37),
                                   dict(fused_merge=False, balanced_gather=False)])
def test_no_alloc_equals_search(octex, small_index, extra):
    index = octex.load(small_index["path"])
    Q = small_index["Q"]
    params = dict(PARAMS, **extra)
    for n in (len(Q), 29):  # two calls in a row, the second smaller
        q = torch.from_numpy(np.ascontiguousarray(Q[:n])).cuda()
        Dr, Ir = index.search(Q[:n], k=10, **params)
        D, I = no_alloc(index, q, 10, **params)
        print(f"no-alloc search: {n} queries, {params}", flush=True)
        assert np.array_equal(I, Ir) and np.array_equal(D, Dr)


def test_no_alloc_refuses_a_batch_beyond_the_scratch(octex, small_index):
    from octex_amd._lib import OctexError

    index = octex.load(small_index["path"])
    g = np.random.default_rng(3)
    q = torch.from_numpy(g.standard_normal((8000, index.dim)).astype(np.float32)).cuda()
    with pytest.raises(OctexError, match="needs \\d+ bytes of scratch for a batch of 8000 queries"):
        no_alloc(index, q, 10, batch=8000, **PARAMS)
    # the same queries in batches that fit
    D, I = no_alloc(index, q[:300], 10, batch=100, **PARAMS)
    Dr, Ir = index.search(q[:300].cpu().numpy(), k=10, batch=100, **PARAMS)
    assert np.array_equal(I, Ir) and np.array_equal(D, Dr)


def test_no_alloc_allocates_nothing_and_runs_under_capture(octex, small_index):
    """The defining property: after a warm-up call, a call leaves the device's free memory unchanged; and the call
    can be captured into a graph (torch's stream capture), whose replays, with new queries copied into the captured
    input and eager work and synchronizations between them, each give the eager search's results."""
    index = octex.load(small_index["path"])
    Q = np.ascontiguousarray(small_index["Q"][:60])
    q = torch.from_numpy(Q).cuda()
    I = torch.full((len(Q), 10), -7, dtype=torch.int64, device="cuda")
    D = torch.full((len(Q), 10), float("nan"), dtype=torch.float32, device="cuda")
    call_no_alloc(index, q, I, D, **PARAMS)  # warm-up: code objects loaded, the scratch's address looked up
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    call_no_alloc(index, q, I, D, **PARAMS)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    print(f"no-alloc: free device memory {free0} before, {free1} after a call", flush=True)
    assert free1 == free0
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            call_no_alloc(index, q, I, D, **PARAMS)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = np.random.default_rng(5)
    for rep in range(3):
        Qr = np.ascontiguousarray(Q[g.permutation(len(Q))]) if rep else Q
        q.copy_(torch.from_numpy(Qr).cuda())
        Dr, Ir = index.search(Qr, k=10, **PARAMS)  # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"no-alloc graph replay {rep}", flush=True)
        assert np.array_equal(I.cpu().numpy(), Ir) and np.array_equal(D.cpu().numpy(), Dr)
