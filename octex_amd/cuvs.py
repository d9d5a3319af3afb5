"""cuVS-style calls answered by octex on MI355X: the names of `cuvs.neighbors.cagra` (octex/cuvs.py:10-167 of the
reference).

    from octex_amd import cuvs as cagra
    index = cagra.build(cagra.IndexParams(copies=64), dataset)
    distances, neighbors = cagra.search(cagra.SearchParams(), index, queries, 10)
    cagra.save("index_dir", index); index = cagra.load("index_dir")

IndexParams takes the octex build parameters and the load placement; SearchParams the octex search parameters
(`max_queries` is the batch size).  CAGRA's own parameters are accepted and have no effect; any other name is a
TypeError.  Only metric "sqeuclidean" is supported (ValueError otherwise).  An index is a directory: save copies
it, load reads it.
"""

import os

from . import index as _index

# CAGRA parameters that are accepted and ignored (octex/cuvs.py:27-56)
CAGRA_INDEX_PARAMS = frozenset((
    "intermediate_graph_degree", "graph_degree", "build_algo", "nn_descent_niter", "ivf_pq_build_params",
    "ivf_pq_search_params", "ace_params", "refinement_rate", "compression", "guarantee_connectivity",
    "add_data_on_build",
))
CAGRA_SEARCH_PARAMS = frozenset((
    "itopk_size", "max_iterations", "algo", "team_size", "search_width", "min_iterations", "thread_block_size",
    "hashmap_mode", "hashmap_min_bitlen", "hashmap_max_fill_rate", "num_random_samplings", "rand_xor_mask",
    "persistent", "persistent_lifetime", "persistent_device_usage",
))
LOAD_ARGS = ("placement", "vectors_on_host", "shard_vectors", "table_on_host", "sketch")


def _take(kwargs, names, ignored, what):
    """The keyword arguments named in `names`; names in `ignored` are dropped, any other is a TypeError."""
    out = {}
    for key, value in kwargs.items():
        if key in names:
            out[key] = value
        elif key not in ignored:
            raise TypeError(f"octex.cuvs: unknown {what} parameter {key!r}")
    return out


class IndexParams:
    """metric plus the fields of cuvs::neighbors::octex::index_params and the load placement."""

    def __init__(self, metric="sqeuclidean", **kwargs):
        _index.check_metric(metric)
        self.metric = metric
        taken = _take(kwargs, _index.INDEX_PARAMS + LOAD_ARGS, CAGRA_INDEX_PARAMS, "index")
        self.load_args = {k: taken.pop(k) for k in LOAD_ARGS if k in taken}
        self.params = taken

    def __repr__(self):
        return f"octex.cuvs.IndexParams(metric={self.metric!r}, {self.params}, {self.load_args})"


class SearchParams:
    """The fields of cuvs::neighbors::octex::search_params; max_queries sets `batch` unless it is given."""

    def __init__(self, max_queries=0, **kwargs):
        self.params = _take(kwargs, _index.SEARCH_PARAMS, CAGRA_SEARCH_PARAMS, "search")
        if max_queries:
            self.params.setdefault("batch", int(max_queries))

    def __repr__(self):
        return f"octex.cuvs.SearchParams({self.params})"


class Index:
    """A cuVS-style handle of an octex index; empty until build or load fills it."""

    def __init__(self, octex_index=None):
        self._index = octex_index

    @property
    def trained(self):
        return self._index is not None

    @property
    def dim(self):
        return 0 if self._index is None else self._index.dim

    @property
    def size(self):
        return 0 if self._index is None else self._index.size

    def __len__(self):
        return self.size

    @property
    def octex(self):
        """The octex_amd.Index underneath."""
        return self._need()

    def _need(self):
        if self._index is None:
            raise ValueError("octex.cuvs: the index is empty (build or load it first)")
        return self._index

    def __repr__(self):
        return f"octex.cuvs.Index({self._index!r})"


def build(index_params, dataset, resources=None):
    """An index of dataset [n, dim] (float32 or float16, host or GPU) built with IndexParams."""
    ip = IndexParams() if index_params is None else index_params
    return Index(_index.build(dataset, metric=ip.metric, **ip.load_args, **ip.params))


def search(search_params, index, queries, k, neighbors=None, distances=None, resources=None, filter=None):
    """(distances, neighbors) of the k nearest, written into `neighbors` / `distances` when given."""
    if filter is not None:
        raise ValueError("octex.cuvs: filtered search is not supported")
    sp = SearchParams() if search_params is None else search_params
    return index._need().search(queries, k, neighbors=neighbors, distances=distances, **sp.params)


def save(filename, index, include_dataset=True, resources=None):
    """Copy the index directory to `filename` (a new directory); the vectors are always part of it."""
    index._need().save(filename)


def load(*args, resources=None, **load_args):
    """load(path), load(index, path) (cuVS 26.10, filling an empty Index) or load(path, index); returns the index.
    Keyword arguments are those of octex_amd.load."""
    if len(args) == 1:
        target, path = Index(), args[0]
    elif len(args) == 2 and isinstance(args[0], Index):
        target, path = args
    elif len(args) == 2:
        path, target = args[0], Index()
    else:
        raise TypeError("octex.cuvs.load(path) or load(index, path)")
    target._index = _index.load(os.fspath(path), **load_args)
    return target
