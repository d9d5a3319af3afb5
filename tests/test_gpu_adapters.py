"""The adapters as drop-ins on the GPU (tests/test_dropin.py of the reference): the calls of
cuvs.neighbors.cagra and of a Faiss GPU index give the native octex_amd results."""

import numpy as np
import pytest
from conftest import clustered, exact_knn, recall

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
K = 10
SMALL = dict(copies=32, log_buckets=14, table_len=32, min_cell=2, seed=1)


@pytest.fixture(scope="module")
def data():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    X, Q = clustered(n=12_000, m=200, d=64, seed=2)
    gt, _ = exact_knn(X.astype(np.float16).astype(np.float32), Q)
    return X, Q, gt


def test_cuvs_calls(data, tmp_path):
    import octex_amd
    from octex_amd import cuvs as cagra

    X, Q, gt = data
    index = cagra.build(cagra.IndexParams(metric="sqeuclidean", graph_degree=32, **SMALL), torch.from_numpy(X).cuda())
    assert index.trained and index.dim == 64 and index.size == len(X)
    sp = cagra.SearchParams(read=16, starts=64, itopk_size=64)
    D, I = cagra.search(sp, index, Q, K)
    assert recall(I, gt) >= 0.9
    Dn, In = index.octex.search(Q, k=K, read=16, starts=64)
    assert np.array_equal(I, In) and np.array_equal(D, Dn)
    Qd = torch.from_numpy(Q).cuda()
    nb = torch.empty((len(Q), K), dtype=torch.int64, device="cuda")
    ds = torch.empty((len(Q), K), dtype=torch.float32, device="cuda")
    D2, I2 = cagra.search(sp, index, Qd, K, neighbors=nb, distances=ds)
    assert I2 is nb and D2 is ds and np.array_equal(nb.cpu().numpy(), In)
    cagra.save(tmp_path / "saved", index)
    a = cagra.load(tmp_path / "saved")
    b = cagra.load(cagra.Index(), tmp_path / "saved", placement="replicate")
    for other in (a, b):
        Do, Io = cagra.search(sp, other, Q, K)
        assert np.array_equal(Io, In)
    del octex_amd


def test_faiss_calls(data, tmp_path):
    from octex_amd import faiss

    X, Q, gt = data
    index = faiss.IndexOctex(X.shape[1], **SMALL)
    index.train(X)
    index.add(X[:7000])
    index.add(torch.from_numpy(X[7000:]).cuda())  # ids continue in the order of the adds
    assert index.ntotal == len(X)
    D, I = index.search(Q, K)
    assert D.dtype == np.float32 and I.dtype == np.int64 and I.shape == (len(Q), K)
    assert recall(I, gt) >= 0.9
    faiss.write_index(index, tmp_path / "f")
    again = faiss.read_index(tmp_path / "f")
    assert again.ntotal == len(X) and again.d == X.shape[1]
    D2, I2 = again.search(Q, K)
    assert np.array_equal(I, I2)
    like = faiss.GpuIndexCagra(faiss.StandardGpuResources(), X.shape[1], faiss.METRIC_L2, **SMALL)
    like.train(X)
    D3, I3 = like.search(Q, K, params=faiss.SearchParametersCagra(read=16, starts=64))
    assert recall(I3, gt) >= 0.9
