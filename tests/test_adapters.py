"""The cuVS-style and Faiss-style adapters without a GPU: metric checks, parameter splitting (CAGRA fields
accepted and ignored, unknown names rejected), Faiss add bookkeeping (tests/test_cpu.py:28-60 of the
reference)."""

import numpy as np
import pytest

import octex_amd
from octex_amd import cuvs as cagra
from octex_amd import faiss
from octex_amd import index as octex_index


def test_version():
    assert octex_amd.__version__ == "0.1.0"


def test_metrics():
    for metric in ("sqeuclidean", "l2", "L2"):
        octex_index.check_metric(metric)
        cagra.IndexParams(metric=metric)
    for metric in ("inner_product", "cosine", "euclidean"):
        with pytest.raises(ValueError):
            cagra.IndexParams(metric=metric)
    with pytest.raises(ValueError):
        faiss.IndexOctex(16, faiss.METRIC_INNER_PRODUCT)
    with pytest.raises(ValueError):
        faiss.GpuIndexCagra(faiss.StandardGpuResources(), 16, faiss.METRIC_INNER_PRODUCT)


def test_adapter_parameters():
    p = cagra.IndexParams(copies=32, graph_degree=64, placement="replicate")
    assert p.params == {"copies": 32} and p.load_args == {"placement": "replicate"}
    s = cagra.SearchParams(max_queries=500, itopk_size=64, read=8)
    assert s.params == {"read": 8, "batch": 500}
    assert cagra.SearchParams(max_queries=500, batch=64).params == {"batch": 64}
    with pytest.raises(TypeError):
        cagra.IndexParams(not_a_parameter=1)
    with pytest.raises(TypeError):
        cagra.SearchParams(not_a_parameter=1)
    with pytest.raises(TypeError):
        faiss.IndexOctex(16, not_a_parameter=1)
    index = faiss.IndexOctex(16, copies=8, read=4, placement="replicate")
    assert index.index_params == {"copies": 8} and index.search_params == {"read": 4}
    assert index.load_args == {"placement": "replicate"}
    index.add(np.zeros((5, 16), np.float64))
    index.add(np.zeros((3, 16), np.float32))
    assert index.ntotal == 8 and index.d == 16 and index.is_trained
    with pytest.raises(ValueError):
        index.add(np.zeros((3, 8), np.float32))
    index.reset()
    assert index.ntotal == 0
    with pytest.raises(RuntimeError, match="empty"):
        index.build()


def test_empty_handles():
    idx = cagra.Index()
    assert not idx.trained and idx.dim == 0 and idx.size == 0 and len(idx) == 0
    with pytest.raises(ValueError, match="empty"):
        cagra.search(cagra.SearchParams(), idx, np.zeros((1, 4), np.float32), 1)
    with pytest.raises(ValueError, match="filtered"):
        cagra.search(None, idx, np.zeros((1, 4), np.float32), 1, filter=object())
    with pytest.raises(TypeError):
        cagra.load()


def test_cagra_constructor_forms():
    a = faiss.GpuIndexCagra(24)
    assert a.d == 24 and not a.is_trained
    cfg = faiss.GpuIndexCagraConfig()
    cfg.device = 0
    b = faiss.GpuIndexCagra(faiss.StandardGpuResources(), 24, faiss.METRIC_L2, cfg)
    assert b.index_params == {"devices": [0]}
    b.add(np.ones((2, 24), np.float16))
    assert b.is_trained and b.ntotal == 2 and b._pending[0].dtype == np.float16
    sp = faiss.SearchParametersCagra(read=8, itopk_size=32)
    assert sp.params == {"read": 8}


def test_host_rows_conversions():
    torch = pytest.importorskip("torch")
    x = faiss._host_rows(torch.arange(12, dtype=torch.float64).reshape(3, 4))
    assert x.dtype == np.float32 and x.shape == (3, 4) and x.flags.c_contiguous
    f = np.asfortranarray(np.ones((4, 5), np.float32))
    assert faiss._host_rows(f).flags.c_contiguous
    with pytest.raises(ValueError, match="matrix"):
        faiss._host_rows(np.ones(3, np.float32))
