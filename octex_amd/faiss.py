"""Faiss-style adapter: GPU index classes with the faiss.Index calls (d, ntotal, is_trained, metric_type, train,
add, search, reset) answered by an octex index, so that

    from octex_amd import faiss                  # instead of: import faiss
    index = faiss.IndexOctex(d)                  # or faiss.GpuIndexCagra(faiss.StandardGpuResources(), d)
    index.add(xb)
    D, I = index.search(xq, k)

runs unchanged.  The reference ships the same adapter (octex/faiss.py); class names, constructor forms and
error texts follow it.  Added vectors are kept on the host in the order of the adds (ids are their positions)
and the octex index is built when a search first needs it, or by build().  Only METRIC_L2 is served.
faiss itself is never imported.
"""

import os

import numpy as np

from . import _arrays
from . import index as _octex

METRIC_INNER_PRODUCT, METRIC_L2 = 0, 1  # faiss.METRIC_INNER_PRODUCT / faiss.METRIC_L2
PLACEMENT_FIELDS = ("placement", "vectors_on_host", "shard_vectors", "table_on_host", "sketch")


def _l2_only(metric):
    if metric != METRIC_L2:
        raise ValueError("octex.faiss: only METRIC_L2 is supported (octex searches by squared Euclidean distance)")


class SearchParametersOctex:
    """Per-call search parameters: octex's search_params fields (`params`); other names (CAGRA's) are dropped."""

    def __init__(self, **kwargs):
        self.params = {k: kwargs[k] for k in kwargs if k in _octex.SEARCH_PARAMS}


SearchParametersCagra = SearchParametersOctex


class _Rows:
    """The vectors added so far, on the host, in order; fp16 blocks stay fp16 while every block is fp16."""

    def __init__(self, d):
        self.d = d
        self.blocks = []
        self.count = 0

    def add(self, x):
        x = _arrays.host_rows(x, (np.float32, np.float16), "vectors")
        if x.shape[1] != self.d:
            raise ValueError(f"octex.faiss: vectors have dimension {x.shape[1]}, the index {self.d}")
        self.blocks.append(x)
        self.count += x.shape[0]

    def matrix(self):
        if len(self.blocks) == 1:
            return self.blocks[0]
        dtype = np.float16 if all(b.dtype == np.float16 for b in self.blocks) else np.float32
        return np.concatenate([b.astype(dtype, copy=False) for b in self.blocks])


class IndexOctex:
    """An octex index with the faiss.Index interface.

    Keyword arguments are octex's index parameters (copies, list_len, table_len, seed, devices, ...: kept in
    `index_params`), the load placement (placement, vectors_on_host, ...: `load_args`) and default search
    parameters (read, starts, waves, ...: `search_params`).
    """

    def __init__(self, d, metric=METRIC_L2, **kwargs):
        _l2_only(metric)
        self.d, self.metric_type, self.is_trained = int(d), metric, True
        self.index_params, self.load_args, self.search_params = {}, {}, {}
        for name, value in kwargs.items():
            if name in _octex.INDEX_PARAMS:
                self.index_params[name] = value
            elif name in PLACEMENT_FIELDS:
                self.load_args[name] = value
            elif name in _octex.SEARCH_PARAMS:
                self.search_params[name] = value
            else:
                raise TypeError(f"octex.faiss: unknown parameters {sorted(set(kwargs) - set(self._accepted()))}")
        self.reset()

    @staticmethod
    def _accepted():
        return set(_octex.INDEX_PARAMS) | set(PLACEMENT_FIELDS) | set(_octex.SEARCH_PARAMS)

    def reset(self):
        self._rows = _Rows(self.d)  # None after read_index: the rows are in the index directory
        self._index = None          # the octex index of the rows, once built
        self._stale = False         # rows added since the build

    @property
    def ntotal(self):
        if self._rows is None:
            return self._index.size
        return self._rows.count

    def train(self, x):
        """Nothing to train (as for Faiss's flat indexes)."""

    def add(self, x):
        if self._rows is None:  # read from a directory: its stored vectors come first
            self._rows = _Rows(self.d)
            self._rows.add(np.asarray(_octex.stored_vectors(self._index.path)))
        self._rows.add(x)
        self._stale = True

    def build(self):
        """Build the octex index of every vector added so far (a search does it when needed)."""
        if self._index is not None and not self._stale:
            return self
        if self._rows is None or self._rows.count == 0:
            raise RuntimeError("octex.faiss: the index is empty")
        self._index = _octex.build(self._rows.matrix(), **self.load_args, **self.index_params)
        self._stale = False
        return self

    def search(self, x, k, *, params=None, D=None, I=None):
        self.build()
        p = dict(self.search_params, **(getattr(params, "params", None) or {}))
        return self._index.search(x, k, distances=D, neighbors=I, **p)

    @property
    def octex(self):
        """The octex_amd.Index of the added vectors (built on access)."""
        return self.build()._index


class StandardGpuResources:
    """faiss.StandardGpuResources stand-in: octex manages its own HIP resources."""

    def noTempMemory(self):
        pass

    def setTempMemory(self, size):
        pass


class GpuIndexCagraConfig:
    """faiss.GpuIndexCagraConfig stand-in: `device` chooses the GPU; the graph fields are not used."""

    def __init__(self):
        self.device = None
        self.graph_degree = 64
        self.intermediate_graph_degree = 128


class GpuIndexCagra(IndexOctex):
    """faiss.GpuIndexCagra(res, d, metric, config), or GpuIndexCagra(d): train(x) builds the index of x."""

    def __init__(self, res=None, d=None, metric=METRIC_L2, config=None, **kwargs):
        if d is None and isinstance(res, int):
            d = res
        device = getattr(config, "device", None)
        if device is not None and "devices" not in kwargs:
            kwargs["devices"] = [int(device)]
        super().__init__(d, metric, **kwargs)
        self.is_trained = False

    def train(self, x):
        self.reset()
        self.add(x)
        self.build()

    def add(self, x):
        super().add(x)
        self.is_trained = True


def write_index(index, path):
    """Write the index directory of an IndexOctex (built first when needed) to `path`."""
    index.octex.save(os.fspath(path))


def read_index(path, **kwargs):
    """An IndexOctex over an index directory; keyword arguments are load arguments and search defaults."""
    search = {k: v for k, v in kwargs.items() if k in _octex.SEARCH_PARAMS}
    loaded = _octex.load(os.fspath(path), **{k: v for k, v in kwargs.items() if k not in search})
    index = IndexOctex(loaded.dim, **search)
    index._rows, index._index = None, loaded
    return index
