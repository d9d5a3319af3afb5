"""The cuVS-style and Faiss-style adapters without a GPU: metric checks, parameter splitting (CAGRA fields
accepted and ignored, unknown names rejected), Faiss add bookkeeping (tests/test_cpu.py:28-60 of the
reference)."""

import os

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
    assert b.is_trained and b.ntotal == 2 and b._rows.blocks[0].dtype == np.float16
    sp = faiss.SearchParametersCagra(read=8, itopk_size=32)
    assert sp.params == {"read": 8}


def test_host_rows_conversions():
    from octex_amd import _arrays

    torch = pytest.importorskip("torch")
    x = _arrays.host_rows(torch.arange(12, dtype=torch.float64).reshape(3, 4))
    assert x.dtype == np.float32 and x.shape == (3, 4) and x.flags.c_contiguous
    f = np.asfortranarray(np.ones((4, 5), np.float32))
    assert _arrays.host_rows(f).flags.c_contiguous
    assert _arrays.host_rows(np.ones(3, np.float32)).shape == (1, 3)  # a vector is one row
    with pytest.raises(ValueError, match="matrix"):
        _arrays.host_rows(np.ones((2, 3, 4), np.float32))


def test_operands_and_streams():
    """Host operands carry no stream; a __cuda_array_interface__ array's 'stream' entry maps to HIP's null
    stream (1, the legacy default), the per-thread stream (2) or the stream handle itself."""
    from octex_amd import _arrays

    op = _arrays.operand(np.arange(12, dtype=np.float64).reshape(3, 4))
    assert op.value.dtype == np.float32 and op.stream is None and not op.on_device
    assert op.respond(np.zeros(2)) is not None and isinstance(op.respond(np.zeros(2)), np.ndarray)
    half = _arrays.operand(np.ones((2, 2), np.float16), (np.float32, np.float16))
    assert half.value.dtype == np.float16
    assert _arrays._hip_stream_of_cai(None) is None
    assert _arrays._hip_stream_of_cai(1) == 0 and _arrays._hip_stream_of_cai(2) == 2
    assert _arrays._hip_stream_of_cai(0x7F00DEAD) == 0x7F00DEAD

    class Foreign:  # a device array of some other framework, produced on stream 0x1234
        __cuda_array_interface__ = dict(shape=(2, 2), typestr="<f4", data=(0, False), version=3, stream=0x1234)

    assert _arrays._foreign_stream(Foreign()) == 0x1234
    assert _arrays.is_foreign_device(Foreign()) and not _arrays.is_foreign_device(np.zeros(1))
    torch = pytest.importorskip("torch")
    top = _arrays.operand(torch.ones((3, 4), dtype=torch.float64))
    assert top.stream is None and top.value.dtype == np.float32
    assert isinstance(top.respond(np.zeros((3, 2))), torch.Tensor)  # torch in, torch out


def test_parameter_structs():
    """Keyword arguments into the C ABI's structs: library defaults, arrays with their counts, unknown names."""
    p = octex_index.index_params(copies=12, spacings=[1.0, 2.0, 3.5], devices=0)
    assert p.copies == 12 and p.n_spacings == 3 and [p.spacings[i] for i in range(3)] == [1.0, 2.0, 3.5]
    assert p.n_devices == 1 and p.devices[0] == 0 and p.list_len == 64  # the library's default
    s = octex_index.search_params(read=7, use_graph=False)
    assert s.read == 7 and not s.use_graph and s.starts == 128
    lp = octex_index.load_params(placement="replicate", sketch="host", copies_limit=3)
    assert lp.placement == 0 and lp.sketch == 2 and lp.copies_limit == 3
    with pytest.raises(TypeError, match="unknown index parameter 'copiez'; valid: copies, blocks"):
        octex_index.index_params(copiez=1)
    with pytest.raises(ValueError, match="sketch must be one of"):
        octex_index.load_params(sketch="disk")


def test_save_copies_the_directory(tmp_path):
    """Index.save copies every file (subdirectories included) and refuses a non-empty target."""
    import shutil

    src = tmp_path / "src"
    shutil.copytree(os.path.join(os.path.dirname(__file__), "golden", "refdir"), src)
    idx = object.__new__(octex_index.Index)
    idx._path, idx._handle = str(src), None
    out = idx.save(str(tmp_path / "dst"))
    for root, _, files in os.walk(src):
        for f in files:
            rel = os.path.relpath(os.path.join(root, f), src)
            assert open(os.path.join(out, rel), "rb").read() == open(os.path.join(src, rel), "rb").read()
    with pytest.raises(FileExistsError, match="exists and is not an empty directory"):
        idx.save(out)
    assert octex_index.stored_vectors(out).shape == (400, 16)
