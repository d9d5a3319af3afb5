"""The octex index for MI355X: build() writes an index directory and loads it, load() places a directory on the GPU,
and Index.search() answers batches of queries.  The Python surface of the reference package (octex/index.py:
names, keyword arguments, defaults and error texts), bound to the cuvsOctex* C ABI through ctypes and DLPack.

    import octex_amd as octex
    index = octex.load("sift.octex")
    D, I = index.search(xq, k=10)      # (squared distances, int64 ids), nearest first

Results come back in the framework of the queries: numpy for host arrays, tensors on the same GPU for torch
tensors, and the origin framework's arrays for other DLPack / __cuda_array_interface__ arrays.  A search of
GPU queries is ordered on the stream they were produced on (torch's current stream, CuPy's current stream, or
the interface's "stream" entry) and returns without waiting: its results are ready on that stream.
"""

import ctypes as ct
import json
import os
import shutil
import tempfile

import numpy as np

from . import _arrays, _lib

PLACEMENTS = ("shard", "replicate")
SKETCH_PLACEMENTS = ("replicate", "shard", "host")
SEARCH_PARAMS = ("read", "starts", "waves", "rerank", "wave_rerank", "batch", "sketch_rank", "final_rerank")
ABLATION_PARAMS = ("balanced_gather", "fused_merge", "use_graph")
INDEX_PARAMS = tuple(f for f, _ in _lib.IndexParams._fields_ if f not in ("n_spacings", "n_devices"))
LOAD_PARAMS = tuple(["devices", "placement"] + [f for f, _ in _lib.LoadParams._fields_
                                                if f not in ("devices", "n_devices", "placement")])
METRICS = ("sqeuclidean", "l2")
_METRIC_OF = {name: "sqeuclidean" for name in METRICS}


def check_metric(metric):
    """octex ranks by squared Euclidean distance; "l2" is accepted as its name in cuVS and Faiss."""
    if _METRIC_OF.get(str(metric).lower()) is None:
        raise ValueError(
            f"octex: metric {metric!r} is not supported; octex searches by squared Euclidean distance "
            "(metric='sqeuclidean')"
        )


class _Spec:
    """How keyword arguments become one of the C ABI's parameter structs: the struct type, its Create / Destroy
    entry points (the defaults come from the library itself), the accepted names, and the fields that are
    (pointer, count) arrays."""

    def __init__(self, what, struct, create, destroy, names, arrays=()):
        self.what, self.struct, self.create, self.destroy = what, struct, create, destroy
        self.names, self.arrays = tuple(names), dict(arrays)

    def defaults(self):
        p = ct.POINTER(self.struct)()
        _lib.call(self.create, ct.byref(p))
        try:
            return self.struct.from_buffer_copy(p.contents)
        finally:
            _lib.call(self.destroy, p)

    def check(self, values):
        bad = [n for n in values if n not in self.names]
        if bad:
            raise TypeError(f"octex: unknown {self.what} parameter {bad[0]!r}; valid: {', '.join(self.names)}")

    def make(self, values):
        self.check(values)
        out = self.defaults()
        out._keep = []  # arrays the struct points into live as long as it does
        for name, value in values.items():
            if value is None:
                continue
            if name in self.arrays:
                ctype, count_field = self.arrays[name]
                items = [value] if np.isscalar(value) else list(value)
                arr = (ctype * len(items))(*items)
                out._keep.append(arr)
                setattr(out, name, ct.cast(arr, ct.POINTER(ctype)))
                setattr(out, count_field, len(items))
            else:
                setattr(out, name, value)
        return out


_INDEX = _Spec("index", _lib.IndexParams, "cuvsOctexIndexParamsCreate", "cuvsOctexIndexParamsDestroy", INDEX_PARAMS,
               arrays={"spacings": (ct.c_float, "n_spacings"), "devices": (ct.c_int32, "n_devices")})
_SEARCH = _Spec("search", _lib.SearchParams, "cuvsOctexSearchParamsCreate", "cuvsOctexSearchParamsDestroy",
                SEARCH_PARAMS + ABLATION_PARAMS)
_LOAD = _Spec("load", _lib.LoadParams, "cuvsOctexLoadParamsCreate", "cuvsOctexLoadParamsDestroy", LOAD_PARAMS,
              arrays={"devices": (ct.c_int32, "n_devices")})


def index_params(**kw):
    """cuvsOctexIndexParams from keyword arguments (names of cuvs::neighbors::octex::index_params)."""
    return _INDEX.make(kw)


def search_params(**kw):
    """cuvsOctexSearchParams from keyword arguments (names of cuvs::neighbors::octex::search_params)."""
    return _SEARCH.make(kw)


def load_params(placement="shard", sketch="replicate", **kw):
    """cuvsOctexLoadParams from keyword arguments; placement and sketch by name."""
    for value, allowed, what in ((placement, PLACEMENTS, "placement"), (sketch, SKETCH_PLACEMENTS, "sketch")):
        if value not in allowed:
            raise ValueError(f"octex: {what} must be one of {allowed}, not {value!r}")
    kw = dict(kw, placement=1 if placement == "shard" else 0, sketch=SKETCH_PLACEMENTS.index(sketch))
    return _LOAD.make(kw)


def _read_meta(path):
    """meta.json of an index directory; a directory without one is not an index."""
    meta = os.path.join(path, "meta.json")
    if not os.path.isfile(meta):
        raise FileNotFoundError(f"octex: {path} is not an index directory (no meta.json)")
    with open(meta) as f:
        return json.load(f)


def _array_file(path, meta, name):
    """Where an array of the directory lies: its "files" entry (absolute, or relative to the directory) or
    <path>/<name>.npy (load.cu:229-234)."""
    where = meta.get("files", {}).get(name, name + ".npy")
    return where if os.path.isabs(where) else os.path.join(path, where)


def stored_vectors(path):
    """The fp16 vectors [N, D] of an index directory, memory mapped."""
    return np.load(_array_file(path, _read_meta(path), "vectors"), mmap_mode="r")


def _copy_tree(src, dst):
    """Every file below src at the same relative place below dst (arrays named by absolute "files" entries lie
    outside src and stay where they are)."""
    for root, _, files in os.walk(src):
        rel = os.path.relpath(root, src)
        target = os.path.normpath(os.path.join(dst, rel))
        os.makedirs(target, exist_ok=True)
        for f in files:
            shutil.copy2(os.path.join(root, f), os.path.join(target, f))


class Index:
    """An octex index placed on a GPU.  Create it with build(), build_in_memory() or load()."""

    def __init__(self, handle, path, tmpdir=None, load_args=None):
        self._handle = handle
        self._path = os.fspath(path)
        self._tmpdir = tmpdir  # a temporary build directory lives as long as the index
        self._load_args = dict(load_args or {})

    def __del__(self):
        handle, self._handle = getattr(self, "_handle", None), None
        if handle is not None and _lib._lib is not None:
            _lib._lib.cuvsOctexIndexDestroy(handle)

    def _scalar(self, entry, ctype):
        v = ctype()
        _lib.call(entry, self._handle, ct.byref(v))
        return v.value

    def _per_device(self, entry, ctype):
        n = self._scalar("cuvsOctexIndexGetNumDevices", ct.c_int32)
        arr = (ctype * n)()
        _lib.call(entry, self._handle, arr)
        return list(arr)

    handle = property(lambda self: self._handle)
    size = property(lambda self: int(self._scalar("cuvsOctexIndexGetSize", ct.c_int64)), doc="indexed vectors")
    dim = property(lambda self: int(self._scalar("cuvsOctexIndexGetDim", ct.c_int64)))
    copies = property(lambda self: int(self._scalar("cuvsOctexIndexGetCopies", ct.c_int32)), doc="loaded copies")
    devices = property(lambda self: self._per_device("cuvsOctexIndexGetDevices", ct.c_int32))
    device_bytes = property(lambda self: self._per_device("cuvsOctexIndexGetDeviceBytes", ct.c_int64))
    path = property(lambda self: self._path, doc="the index directory")
    metric = property(lambda self: "sqeuclidean")

    def __len__(self):
        return self.size

    def __repr__(self):
        fields = dict(size=self.size, dim=self.dim, copies=self.copies, devices=self.devices)
        return "octex.Index(" + ", ".join(f"{k}={v}" for k, v in fields.items()) + ")"

    def search(self, queries, k=10, *, read=32, starts=128, waves=2, rerank=128, wave_rerank=128, batch=10000,
               sketch_rank=False, final_rerank=32, neighbors=None, distances=None, **ablation):
        """Approximate k nearest neighbors of a batch of queries [m, dim] (float32; other types are converted).

        Returns (distances, neighbors): float32 squared Euclidean distances and int64 ids [m, k], nearest first,
        in the framework (and on the GPU) of the queries.  `read` list entries per copy, `starts` kept entries
        expanded per wave and `waves` rounds over the neighbor table trade speed for recall.  Given `neighbors` /
        `distances` arrays receive the results (cast if needed) and are returned.  balanced_gather, fused_merge
        and use_graph select the reference's ablation paths and the graph replay.
        """
        k = int(k)
        if k <= 0:
            raise ValueError("octex: k must be positive")
        params = search_params(read=read, starts=starts, waves=waves, rerank=rerank, wave_rerank=wave_rerank,
                               batch=batch, sketch_rank=sketch_rank, final_rerank=final_rerank, **ablation)
        q = _arrays.operand(queries, (np.float32,), "queries")
        m, d = q.shape
        if d != self.dim:
            raise ValueError(f"octex: queries have dimension {d}, the index {self.dim}")
        I, D = q.new(m, k, np.int64), q.new(m, k, np.float32)
        res = _lib.Resources(stream=q.stream)  # device queries: ordered on their producer's stream
        tensors = [_lib.Dl(t) for t in (q.value, I, D)]
        _lib.call("cuvsOctexSearch", res.h, ct.byref(params), self._handle, *(t.ptr for t in tensors))
        out = []
        for given, got in ((distances, D), (neighbors, I)):
            if given is None:
                out.append(q.respond(got))
            else:
                if _arrays.shape_of(given) != (m, k):
                    raise ValueError(f"octex: output arrays must have shape {(m, k)}, not {_arrays.shape_of(given)}")
                out.append(_arrays.write_into(given, got))
        return tuple(out)

    # ---------------------------------------------------------------- introspection (octex_amd.h)

    def _sized_copy(self, entry, name, dtype, *lead):
        size = ct.c_int64(0)
        _lib.call(entry, self._handle, name.encode(), *lead, None, ct.c_int64(0), ct.byref(size))
        out = np.empty(size.value // np.dtype(dtype).itemsize, dtype)
        _lib.call(entry, self._handle, name.encode(), *lead, ct.c_void_p(out.ctypes.data), ct.c_int64(out.nbytes),
                  None)
        return out

    def plan_buffer(self, name, dtype):
        """A host copy of a buffer of the cached search plan (see octexIndexCopyPlanBuffer)."""
        return self._sized_copy("octexIndexCopyPlanBuffer", name, dtype)

    def array(self, name, dtype, copy=0):
        """A host copy of an index array (see octexIndexCopyArray)."""
        return self._sized_copy("octexIndexCopyArray", name, dtype, ct.c_int32(copy))

    def array_size(self, name, copy=0):
        """Bytes of an index array."""
        size = ct.c_int64(0)
        _lib.call("octexIndexCopyArray", self._handle, name.encode(), ct.c_int32(copy), None, ct.c_int64(0),
                  ct.byref(size))
        return size.value

    def array_range(self, name, dtype, start, count, copy=0):
        """Elements [start, start + count) of an index array (see octexIndexCopyArrayRange)."""
        out = np.empty(count, dtype)
        isz = np.dtype(dtype).itemsize
        _lib.call("octexIndexCopyArrayRange", self._handle, name.encode(), ct.c_int32(copy), ct.c_int64(start * isz),
                  ct.c_void_p(out.ctypes.data), ct.c_int64(out.nbytes))
        return out

    def array_ranges(self, name, dtype, starts, count, copy=0):
        """Rows [starts[r], starts[r] + count) of an index array, gathered on the GPU: [len(starts), count]."""
        isz = np.dtype(dtype).itemsize
        offs = np.ascontiguousarray(np.asarray(starts, np.int64) * isz)
        out = np.empty((len(offs), count), dtype)
        _lib.call("octexIndexCopyArrayRanges", self._handle, name.encode(), ct.c_int32(copy),
                  ct.c_void_p(offs.ctypes.data), ct.c_int64(len(offs)), ct.c_int64(count * isz),
                  ct.c_void_p(out.ctypes.data))
        return out

    def profile_batch(self, queries, k=10, reps=3, **params):
        """Per-kernel milliseconds of one batch (HIP events around every launch) and its work counters."""
        p = search_params(**params)
        dq = _lib.Dl(queries)
        names = ct.create_string_buffer(64 * 32)
        ms = (ct.c_double * 64)()
        ns = ct.c_int32(0)
        cnt = (ct.c_int64 * 108)()
        _lib.call("octexIndexProfileBatch", self._handle, ct.byref(p), dq.ptr, ct.c_int64(k), ct.c_int32(reps), names,
                  ms, ct.byref(ns), cnt)
        stages = [(names.raw[32 * i : 32 * (i + 1)].split(b"\0")[0].decode(), ms[i]) for i in range(ns.value)]
        c = list(cnt)
        counters = dict(seg_hits=c[0], entries1=c[1], distinct1=c[2], reranked1=c[3], starts2=c[4:20],
                        distinct2=c[20:36], reranked2=c[36:52], hit_level=c[52:60], skipped2=c[60:76],
                        known2=c[76:92], oldread2=c[92:108])
        return stages, counters

    def place_on_host(self, vectors=True, table=False, sketch=False):
        """Move the vectors / neighbor table / sketch to pinned host memory (the load placements vectors_on_host,
        table_on_host and sketch="host" for an index built in memory)."""
        flags = [ct.c_int32(int(bool(v))) for v in (vectors, table, sketch)]
        _lib.call("octexIndexPlaceOnHost", self._handle, *flags)
        return self

    def plan_info(self):
        arr = (ct.c_int32 * 10)()
        _lib.call("octexIndexPlanInfo", self._handle, arr)
        keys = ("m", "k", "KO", "lr", "W", "W2", "rerank", "wave_rerank", "final_rerank", "graph")
        return dict(zip(keys, list(arr)))

    def save(self, path):
        """Copy the index directory to `path` (a new or empty directory); load(path) restores the index.  Arrays
        that meta.json names by absolute path stay where they are."""
        path = os.fspath(path)
        if os.path.exists(path) and (not os.path.isdir(path) or os.listdir(path)):
            raise FileExistsError(f"octex: {path} exists and is not an empty directory")
        if os.path.abspath(path) != os.path.abspath(self._path):
            _copy_tree(self._path, path)
        return path


def _dataset(dataset):
    """A build's dataset as the C ABI takes it: float32 or float16, dense, host or device."""
    return _arrays.operand(dataset, (np.float32, np.float16), "dataset").value


def _new_handle():
    handle = ct.POINTER(_lib.IndexHandle)()
    _lib.call("cuvsOctexIndexCreate", ct.byref(handle))
    return handle


def _fill(handle, entry, *args):
    """Run entry(..., handle) on a fresh handle; the handle is released if it fails."""
    try:
        _lib.call(entry, *args)
    except Exception:
        _lib.lib().cuvsOctexIndexDestroy(handle)
        raise
    return handle


def load(path, devices=None, placement="shard", vectors_on_host=False, *, shard_vectors=False,
         table_on_host=False, sketch="replicate", parts=0, copies_per_part=0, copies_limit=0, list_limit=0):
    """Load an index directory onto the GPU (the first of `devices`, default the current one)."""
    path = os.fspath(path)
    check_metric(_read_meta(path).get("metric", "sqeuclidean"))
    args = dict(devices=devices, placement=placement, vectors_on_host=vectors_on_host, shard_vectors=shard_vectors,
                table_on_host=table_on_host, sketch=sketch, parts=parts, copies_per_part=copies_per_part,
                copies_limit=copies_limit, list_limit=list_limit)
    lp = load_params(**args)
    handle = _new_handle()
    _fill(handle, "cuvsOctexLoad", _lib.Resources().h, os.fsencode(path), ct.byref(lp), handle)
    return Index(handle, path, load_args=args)


def build(dataset, path=None, *, metric="sqeuclidean", placement="shard", vectors_on_host=False,
          table_on_host=False, shard_vectors=False, sketch="replicate", **index_params_):
    """Build an index of `dataset` [n, dim] (float32 or float16; host or GPU) into `path` (a temporary directory
    that lives as long as the index when None) and load it."""
    check_metric(metric)
    params = index_params(**index_params_)
    x = _lib.Dl(_dataset(dataset))
    tmp = tempfile.TemporaryDirectory(prefix="octex-") if path is None else None
    path = os.fspath(tmp.name if tmp is not None else path)
    os.makedirs(path, exist_ok=True)
    _lib.call("cuvsOctexBuild", _lib.Resources().h, ct.byref(params), x.ptr, os.fsencode(path))
    idx = load(path, devices=index_params_.get("devices"), placement=placement, vectors_on_host=vectors_on_host,
               table_on_host=table_on_host, shard_vectors=shard_vectors, sketch=sketch)
    idx._tmpdir = tmp
    return idx


def build_in_memory(dataset, path=None, **index_params_):
    """Build an index of `dataset` [n, dim] in the GPU's memory and return it ready to search (no round trip
    through files); with `path` the index directory is written as well.  Returns (index, build seconds)."""
    params = index_params(**index_params_)
    x = _lib.Dl(_dataset(dataset))
    secs = ct.c_double(0)
    handle = _new_handle()
    _fill(handle, "octexBuildInMemory", _lib.Resources().h, ct.byref(params), x.ptr,
          os.fsencode(path) if path is not None else None, handle, ct.byref(secs))
    return Index(handle, path if path is not None else "", load_args={}), secs.value
