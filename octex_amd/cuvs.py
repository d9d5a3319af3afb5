"""cuVS-style adapter: the module-level calls of cuvs.neighbors.cagra (IndexParams, SearchParams, Index, build,
search, save, load), answered by an octex index, so that

    from octex_amd import cuvs as cagra          # instead of: from cuvs.neighbors import cagra
    index = cagra.build(cagra.IndexParams(), dataset)
    distances, neighbors = cagra.search(cagra.SearchParams(), index, queries, k)

runs unchanged.  The reference ships the same adapter (octex/cuvs.py); names, accepted parameters and error
texts follow it.  Parameter objects take octex's own fields and accept CAGRA's, which do nothing here;
`max_queries` is the batch size unless `batch` is given.  Only the squared Euclidean metric is served.
"""

import os

from . import index as _octex

# cuvs.neighbors.cagra's IndexParams / SearchParams fields: accepted, without effect on an octex index
CAGRA_INDEX_FIELDS = frozenset((
    "intermediate_graph_degree", "graph_degree", "build_algo", "nn_descent_niter", "ivf_pq_build_params",
    "ivf_pq_search_params", "ace_params", "refinement_rate", "compression", "guarantee_connectivity",
    "add_data_on_build"))
CAGRA_SEARCH_FIELDS = frozenset((
    "itopk_size", "max_iterations", "algo", "team_size", "search_width", "min_iterations", "thread_block_size",
    "hashmap_mode", "hashmap_min_bitlen", "hashmap_max_fill_rate", "num_random_samplings", "rand_xor_mask",
    "persistent", "persistent_lifetime", "persistent_device_usage"))
PLACEMENT_FIELDS = ("placement", "vectors_on_host", "shard_vectors", "table_on_host", "sketch")


def _routes(**groups):
    """name -> destination for every accepted keyword (None: accepted and dropped)."""
    table = {}
    for dest, names in groups.items():
        for n in names:
            table[n] = None if dest == "ignored" else dest
    return table


_INDEX_ROUTES = _routes(params=_octex.INDEX_PARAMS, load_args=PLACEMENT_FIELDS, ignored=CAGRA_INDEX_FIELDS)
_SEARCH_ROUTES = _routes(params=_octex.SEARCH_PARAMS, ignored=CAGRA_SEARCH_FIELDS)


def _sort(kwargs, routes, what, into):
    for name, value in kwargs.items():
        if name not in routes:
            raise TypeError(f"octex.cuvs: unknown {what} parameter {name!r}")
        dest = routes[name]
        if dest is not None:
            into[dest][name] = value


class IndexParams:
    """Build parameters: the metric, octex's index_params fields (`params`) and the load placement
    (`load_args`)."""

    def __init__(self, metric="sqeuclidean", **kwargs):
        _octex.check_metric(metric)
        self.metric = metric
        groups = {"params": {}, "load_args": {}}
        _sort(kwargs, _INDEX_ROUTES, "index", groups)
        self.params, self.load_args = groups["params"], groups["load_args"]

    def __repr__(self):
        return f"octex.cuvs.IndexParams(metric={self.metric!r}, {self.params}, {self.load_args})"


class SearchParams:
    """Search parameters: octex's search_params fields (`params`); max_queries is the batch size."""

    def __init__(self, max_queries=0, **kwargs):
        groups = {"params": {}}
        _sort(kwargs, _SEARCH_ROUTES, "search", groups)
        self.params = groups["params"]
        if max_queries and "batch" not in self.params:
            self.params["batch"] = int(max_queries)

    def __repr__(self):
        return f"octex.cuvs.SearchParams({self.params})"


class Index:
    """A cuVS-style handle of an octex index; empty until build or load fills it."""

    def __init__(self, octex_index=None):
        self._index = octex_index

    def _loaded(self):
        if self._index is None:
            raise ValueError("octex.cuvs: the index is empty (build or load it first)")
        return self._index

    trained = property(lambda self: self._index is not None)
    dim = property(lambda self: 0 if self._index is None else self._index.dim)
    size = property(lambda self: 0 if self._index is None else self._index.size)
    octex = property(lambda self: self._loaded(), doc="the octex_amd.Index underneath")

    def __len__(self):
        return self.size

    def __repr__(self):
        return f"octex.cuvs.Index({self._index!r})"


def build(index_params, dataset, resources=None):
    """An index of `dataset` [n, dim] (float32 or float16, host or GPU) built with `index_params`."""
    p = index_params if index_params is not None else IndexParams()
    return Index(_octex.build(dataset, metric=p.metric, **p.params, **p.load_args))


def search(search_params, index, queries, k, neighbors=None, distances=None, resources=None, filter=None):
    """(distances, neighbors) of the k nearest indexed vectors of every query, written into the given arrays
    when there are any."""
    if filter is not None:
        raise ValueError("octex.cuvs: filtered search is not supported")
    p = search_params if search_params is not None else SearchParams()
    return index._loaded().search(queries, k, neighbors=neighbors, distances=distances, **p.params)


def save(filename, index, include_dataset=True, resources=None):
    """Copy the index directory to `filename` (a new directory); the vectors are always part of it."""
    index._loaded().save(filename)


def load(*args, resources=None, **load_args):
    """load(path), or load(index, path) as in cuVS 26.10, which fills the given empty Index; keyword arguments are
    octex_amd.load's (devices, placement, copies_limit, ...).  Returns the index."""
    if len(args) not in (1, 2):
        raise TypeError("octex.cuvs.load(path) or load(index, path)")
    fill = len(args) == 2 and isinstance(args[0], Index)
    target, path = (args[0], args[1]) if fill else (Index(), args[0])
    target._index = _octex.load(os.fspath(path), **load_args)
    return target
