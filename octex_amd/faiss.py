"""Faiss-style GPU index answered by octex on MI355X: the interface of faiss.Index (octex/faiss.py:10-166 of the
reference), without importing faiss.

    from octex_amd import faiss
    index = faiss.IndexOctex(d, copies=64)      # or faiss.GpuIndexCagra(faiss.StandardGpuResources(), d)
    index.add(xb)                               # the index is built by the first search after an add
    D, I = index.search(xq, 10)                 # float32 squared distances, int64 ids, nearest first
    faiss.write_index(index, "index_dir"); index = faiss.read_index("index_dir")

Vectors are added in batches (numpy or torch, host or GPU); ids are positions in the order of the adds.  Results
come back in the framework of the queries.  Only METRIC_L2 is supported.
"""

import os

import numpy as np

from . import index as _index

METRIC_INNER_PRODUCT, METRIC_L2 = 0, 1  # faiss.METRIC_INNER_PRODUCT, faiss.METRIC_L2
LOAD_ARGS = ("placement", "vectors_on_host", "shard_vectors", "table_on_host", "sketch")


def _check_metric(metric):
    if metric != METRIC_L2:
        raise ValueError("octex.faiss: only METRIC_L2 is supported (octex searches by squared Euclidean distance)")


def _host_rows(x):
    """A host numpy matrix (float32, or float16 kept as is) of a numpy, torch or DLPack array."""
    if type(x).__module__.startswith("torch"):
        x = x.detach().cpu().numpy()
    elif not isinstance(x, np.ndarray) and hasattr(x, "__dlpack__"):
        try:
            x = np.from_dlpack(x)
        except (RuntimeError, BufferError, TypeError):  # device memory: through torch
            import torch

            x = torch.from_dlpack(x).cpu().numpy()
    x = np.asarray(x)
    if x.dtype not in (np.float32, np.float16):
        x = x.astype(np.float32)
    if x.ndim != 2:
        raise ValueError("octex.faiss: vectors must be a matrix [n, d]")
    return np.ascontiguousarray(x)


class SearchParametersOctex:
    """Per-call search parameters (fields of cuvs::neighbors::octex::search_params); other names are ignored."""

    def __init__(self, **kwargs):
        self.params = {k: v for k, v in kwargs.items() if k in _index.SEARCH_PARAMS}


SearchParametersCagra = SearchParametersOctex


class IndexOctex:
    """An octex index with the faiss.Index interface: d, ntotal, is_trained, metric_type, train, add, search, reset.

    Keyword arguments: octex index parameters (copies, list_len, table_len, seed, devices, ...), load arguments
    (placement, vectors_on_host, ...) and default search parameters (read, starts, waves, ...).
    """

    def __init__(self, d, metric=METRIC_L2, **kwargs):
        _check_metric(metric)
        self.d, self.metric_type, self.is_trained = int(d), metric, True
        self.index_params = {k: v for k, v in kwargs.items() if k in _index.INDEX_PARAMS}
        self.load_args = {k: v for k, v in kwargs.items() if k in LOAD_ARGS}
        self.search_params = {k: v for k, v in kwargs.items() if k in _index.SEARCH_PARAMS}
        unknown = set(kwargs) - set(self.index_params) - set(self.load_args) - set(self.search_params)
        if unknown:
            raise TypeError(f"octex.faiss: unknown parameters {sorted(unknown)}")
        self.reset()

    @property
    def ntotal(self):
        return (0 if self._built is None else self._built.size) + sum(len(x) for x in self._pending)

    def reset(self):
        self._parts = []  # host batches of the built index, in order
        self._pending = []  # batches added since
        self._built = None

    def train(self, x):
        pass

    def add(self, x):
        x = _host_rows(x)
        if x.shape[1] != self.d:
            raise ValueError(f"octex.faiss: vectors have dimension {x.shape[1]}, the index {self.d}")
        self._pending.append(x)

    def build(self):
        """Build the index of every vector added so far (otherwise the next search does)."""
        if self._built is not None and not self._pending:
            return self
        if self._built is not None and not self._parts:  # read from a directory: start from its vectors
            self._parts = [np.asarray(_index.stored_vectors(self._built.path))]
        parts = self._parts + self._pending
        if not parts:
            raise RuntimeError("octex.faiss: the index is empty")
        data = parts[0] if len(parts) == 1 else np.concatenate([p.astype(np.float32, copy=False) for p in parts])
        self._built = _index.build(data, **self.load_args, **self.index_params)
        self._parts, self._pending = parts, []
        return self

    def search(self, x, k, *, params=None, D=None, I=None):
        if self._built is None or self._pending:
            self.build()
        sp = dict(self.search_params)
        if params is not None:
            sp.update(getattr(params, "params", {}))
        return self._built.search(x, k, distances=D, neighbors=I, **sp)

    @property
    def octex(self):
        """The octex_amd.Index underneath (built on access)."""
        return self.build()._built


class StandardGpuResources:
    """Accepted for faiss.StandardGpuResources compatibility; octex keeps its own streams."""

    def noTempMemory(self):
        pass

    def setTempMemory(self, size):
        pass


class GpuIndexCagraConfig:
    """Accepted for faiss.GpuIndexCagraConfig compatibility: `device` picks the GPU, the rest is ignored."""

    def __init__(self):
        self.device = None
        self.graph_degree = 64
        self.intermediate_graph_degree = 128


class GpuIndexCagra(IndexOctex):
    """faiss.GpuIndexCagra(res, d, metric, config): train(x) builds the index of x, as in Faiss."""

    def __init__(self, res=None, d=None, metric=METRIC_L2, config=None, **kwargs):
        if d is None and isinstance(res, int):  # GpuIndexCagra(d)
            res, d = None, res
        if config is not None and getattr(config, "device", None) is not None:
            kwargs.setdefault("devices", [int(config.device)])
        super().__init__(d, metric, **kwargs)
        self.is_trained = False

    def train(self, x):
        self.reset()
        self.add(x)
        self.build()
        self.is_trained = True

    def add(self, x):
        super().add(x)
        self.is_trained = True


def write_index(index, path):
    """Write the index directory of an IndexOctex (built first when needed) to `path`."""
    index.octex.save(os.fspath(path))


def read_index(path, **kwargs):
    """An IndexOctex over an index directory; keyword arguments: load placement and default search parameters."""
    loaded = _index.load(os.fspath(path), **{k: v for k, v in kwargs.items() if k not in _index.SEARCH_PARAMS})
    out = IndexOctex(loaded.dim, **{k: v for k, v in kwargs.items() if k in _index.SEARCH_PARAMS})
    out._built = loaded
    return out
