"""The octex index for MI355X: build() writes an index directory and loads it, load() places a directory on the
GPU, and Index.search() answers batches of queries.  Same names, arguments and error behaviour as the reference's
Python API (octex/index.py:83-375), bound to the cuvsOctex* C ABI through ctypes and DLPack.

    import octex_amd as octex
    index = octex.load("sift.octex")
    D, I = index.search(xq, k=10)      # (squared distances, int64 ids), nearest first

Results come back in the framework of the queries: numpy for host arrays, torch tensors on the same GPU for
torch GPU tensors.
"""

import ctypes as ct
import json
import os
import shutil
import sys
import tempfile

import numpy as np

from . import _lib

METRICS = ("sqeuclidean", "l2")
INDEX_PARAMS = tuple(f for f, _ in _lib.IndexParams._fields_ if f not in ("n_spacings", "n_devices"))
SEARCH_PARAMS = ("read", "starts", "waves", "rerank", "wave_rerank", "batch", "sketch_rank", "final_rerank")
LOAD_PARAMS = ("devices", "placement", "vectors_on_host", "shard_vectors", "table_on_host", "sketch", "parts",
               "copies_per_part", "copies_limit", "list_limit")
PLACEMENTS = ("shard", "replicate")
SKETCH_PLACEMENTS = ("replicate", "shard", "host")


def check_metric(metric):
    if str(metric).lower() not in METRICS:
        raise ValueError(
            f"octex: metric {metric!r} is not supported; octex searches by squared Euclidean distance "
            "(metric='sqeuclidean')"
        )


def _unknown(names, kw, what):
    for name in kw:
        if name not in names:
            raise TypeError(f"octex: unknown {what} parameter {name!r}; valid: {', '.join(names)}")


def index_params(**kw):
    """cuvsOctexIndexParams from keyword arguments (names of cuvs::neighbors::octex::index_params)."""
    _unknown(INDEX_PARAMS, kw, "index")
    p = ct.POINTER(_lib.IndexParams)()
    _lib.call("cuvsOctexIndexParamsCreate", ct.byref(p))
    out = _lib.IndexParams.from_buffer_copy(p.contents)
    _lib.call("cuvsOctexIndexParamsDestroy", p)
    keep = []
    for name, value in kw.items():
        if value is None:
            continue
        if name == "spacings":
            arr = (ct.c_float * len(value))(*[float(v) for v in value])
            keep.append(arr)
            out.spacings, out.n_spacings = ct.cast(arr, ct.POINTER(ct.c_float)), len(value)
        elif name == "devices":
            value = [value] if isinstance(value, int) else list(value)
            arr = (ct.c_int32 * len(value))(*[int(v) for v in value])
            keep.append(arr)
            out.devices, out.n_devices = ct.cast(arr, ct.POINTER(ct.c_int32)), len(value)
        else:
            setattr(out, name, value)
    out._keep = keep
    return out


def search_params(**kw):
    """cuvsOctexSearchParams from keyword arguments (names of cuvs::neighbors::octex::search_params)."""
    _unknown(SEARCH_PARAMS + ("balanced_gather", "fused_merge", "use_graph"), kw, "search")
    p = ct.POINTER(_lib.SearchParams)()
    _lib.call("cuvsOctexSearchParamsCreate", ct.byref(p))
    out = _lib.SearchParams.from_buffer_copy(p.contents)
    _lib.call("cuvsOctexSearchParamsDestroy", p)
    for name, value in kw.items():
        if value is not None:
            setattr(out, name, value)
    return out


def load_params(placement="shard", sketch="replicate", **kw):
    if placement not in PLACEMENTS:
        raise ValueError(f"octex: placement must be one of {PLACEMENTS}, not {placement!r}")
    if sketch not in SKETCH_PLACEMENTS:
        raise ValueError(f"octex: sketch must be one of {SKETCH_PLACEMENTS}, not {sketch!r}")
    _unknown(LOAD_PARAMS, kw, "load")
    p = ct.POINTER(_lib.LoadParams)()
    _lib.call("cuvsOctexLoadParamsCreate", ct.byref(p))
    out = _lib.LoadParams.from_buffer_copy(p.contents)
    _lib.call("cuvsOctexLoadParamsDestroy", p)
    out.placement = 1 if placement == "shard" else 0
    out.sketch = SKETCH_PLACEMENTS.index(sketch)
    keep = []
    for name, value in kw.items():
        if value is None:
            continue
        if name == "devices":
            value = [value] if isinstance(value, int) else list(value)
            arr = (ct.c_int32 * len(value))(*[int(v) for v in value])
            keep.append(arr)
            out.devices, out.n_devices = ct.cast(arr, ct.POINTER(ct.c_int32)), len(value)
        else:
            setattr(out, name, value)
    out._keep = keep
    return out


def _meta(path):
    with open(os.path.join(path, "meta.json")) as f:
        return json.load(f)


def stored_vectors(path):
    """The fp16 vectors [N, D] of an index directory, memory mapped."""
    f = _meta(path).get("files", {}).get("vectors", os.path.join(path, "vectors.npy"))
    return np.load(f if os.path.isabs(f) else os.path.join(path, f), mmap_mode="r")


def _is_torch(a):
    return type(a).__module__.startswith("torch")


def _is_foreign(a):
    """An array of another framework (CuPy, JAX, ...) that exports DLPack or __cuda_array_interface__."""
    return (not isinstance(a, np.ndarray) and not _is_torch(a)
            and (hasattr(a, "__dlpack__") or hasattr(a, "__cuda_array_interface__")))


def _as_torch(a):
    """A torch view of a foreign array (no copy): through DLPack, or __cuda_array_interface__."""
    import torch

    return torch.from_dlpack(a) if hasattr(a, "__dlpack__") else torch.as_tensor(a, device="cuda")


def _in_framework_of(a, t):
    """The torch result t as an array of a's framework, through its module's from_dlpack when it has one
    (octex/_arrays.py answers in the framework of the input); torch otherwise."""
    mod = sys.modules.get(type(a).__module__.partition(".")[0])
    conv = getattr(mod, "from_dlpack", None)
    return conv(t) if conv is not None else t


def _copy_into(dst, src):
    """Write the result src (numpy or torch) into the caller's array dst (numpy, torch, or foreign)."""
    if isinstance(dst, np.ndarray):
        dst[...] = src.cpu().numpy() if _is_torch(src) else src
        return
    import torch

    d = dst if _is_torch(dst) else _as_torch(dst)
    d.copy_(src if _is_torch(src) else torch.from_numpy(np.ascontiguousarray(src)))


class Index:
    """An octex index placed on a GPU. Create it with build() or load()."""

    def __init__(self, handle, path, tmpdir=None, load_args=None):
        self._handle = handle
        self._path = os.fspath(path)
        self._tmpdir = tmpdir
        self._load_args = dict(load_args or {})
        self._res = _lib.Resources()

    def __del__(self):
        h = getattr(self, "_handle", None)
        if h is not None and _lib._lib is not None:
            _lib._lib.cuvsOctexIndexDestroy(h)
            self._handle = None

    def _get(self, name, ctype):
        v = ctype()
        _lib.call(name, self._handle, ct.byref(v))
        return v.value

    @property
    def handle(self):
        return self._handle

    @property
    def size(self):
        return int(self._get("cuvsOctexIndexGetSize", ct.c_int64))

    @property
    def dim(self):
        return int(self._get("cuvsOctexIndexGetDim", ct.c_int64))

    @property
    def copies(self):
        return int(self._get("cuvsOctexIndexGetCopies", ct.c_int32))

    @property
    def devices(self):
        n = self._get("cuvsOctexIndexGetNumDevices", ct.c_int32)
        arr = (ct.c_int32 * n)()
        _lib.call("cuvsOctexIndexGetDevices", self._handle, arr)
        return list(arr)

    @property
    def device_bytes(self):
        n = self._get("cuvsOctexIndexGetNumDevices", ct.c_int32)
        arr = (ct.c_int64 * n)()
        _lib.call("cuvsOctexIndexGetDeviceBytes", self._handle, arr)
        return list(arr)

    @property
    def path(self):
        return self._path

    @property
    def metric(self):
        return "sqeuclidean"

    def __len__(self):
        return self.size

    def __repr__(self):
        return f"octex.Index(size={self.size}, dim={self.dim}, copies={self.copies}, devices={self.devices})"

    def search(self, queries, k=10, *, read=32, starts=128, waves=2, rerank=128, wave_rerank=128, batch=10000,
               sketch_rank=False, final_rerank=32, neighbors=None, distances=None, **ablation):
        """Approximate k nearest neighbors of a batch of queries [m, dim] (float32): numpy, torch (host or GPU), or
        any array with DLPack or __cuda_array_interface__.

        Returns (distances, neighbors): float32 squared Euclidean distances and int64 ids [m, k], nearest first,
        in the framework (and on the GPU) of the queries; given `neighbors` / `distances` arrays are written.
        """
        k = int(k)
        if k <= 0:
            raise ValueError("octex: k must be positive")
        params = search_params(read=read, starts=starts, waves=waves, rerank=rerank, wave_rerank=wave_rerank,
                               batch=batch, sketch_rank=sketch_rank, final_rerank=final_rerank, **ablation)
        if _is_foreign(queries):  # searched as a torch view, answered in the queries' framework
            D, I = self.search(_as_torch(queries), k, read=read, starts=starts, waves=waves, rerank=rerank,
                               wave_rerank=wave_rerank, batch=batch, sketch_rank=sketch_rank,
                               final_rerank=final_rerank, **ablation)
            if neighbors is not None:
                _copy_into(neighbors, I)
            if distances is not None:
                _copy_into(distances, D)
            return (distances if distances is not None else _in_framework_of(queries, D),
                    neighbors if neighbors is not None else _in_framework_of(queries, I))
        if _is_torch(queries):
            import torch

            q = queries.detach()
            if q.dtype != torch.float32:
                q = q.float()
            q = q.contiguous()
            if q.ndim != 2:
                raise ValueError("octex: queries must be a matrix [m, dim]")
            m, d = q.shape
            I = torch.empty((m, k), dtype=torch.int64, device=q.device)
            D = torch.empty((m, k), dtype=torch.float32, device=q.device)
        else:
            q = np.ascontiguousarray(np.asarray(queries, dtype=np.float32))
            if q.ndim != 2:
                raise ValueError("octex: queries must be a matrix [m, dim]")
            m, d = q.shape
            I = np.empty((m, k), np.int64)
            D = np.empty((m, k), np.float32)
        if d != self.dim:
            raise ValueError(f"octex: queries have dimension {d}, the index {self.dim}")
        dq, di, dd = _lib.Dl(q), _lib.Dl(I), _lib.Dl(D)
        _lib.call("cuvsOctexSearch", self._res.h, ct.byref(params), self._handle, dq.ptr, di.ptr, dd.ptr)
        if _is_torch(queries) and q.is_cuda:
            self._res.sync()
        if neighbors is not None:
            _copy_into(neighbors, I)
            I = neighbors
        if distances is not None:
            _copy_into(distances, D)
            D = distances
        return D, I

    def plan_buffer(self, name, dtype):
        """A copy (numpy) of a buffer of the cached search plan (introspection for tests and the bench)."""
        size = ct.c_int64(0)
        _lib.call("octexIndexCopyPlanBuffer", self._handle, name.encode(), None, ct.c_int64(0), ct.byref(size))
        out = np.empty(size.value // np.dtype(dtype).itemsize, dtype)
        _lib.call("octexIndexCopyPlanBuffer", self._handle, name.encode(), ct.c_void_p(out.ctypes.data),
                  ct.c_int64(out.nbytes), None)
        return out

    def array(self, name, dtype, copy=0):
        """A host copy (numpy) of an array of the index (introspection; see octexIndexCopyArray)."""
        size = ct.c_int64(0)
        _lib.call("octexIndexCopyArray", self._handle, name.encode(), ct.c_int32(copy), None, ct.c_int64(0),
                  ct.byref(size))
        out = np.empty(size.value // np.dtype(dtype).itemsize, dtype)
        _lib.call("octexIndexCopyArray", self._handle, name.encode(), ct.c_int32(copy), ct.c_void_p(out.ctypes.data),
                  ct.c_int64(out.nbytes), None)
        return out

    def array_size(self, name, copy=0):
        """Bytes of an index array (see octexIndexCopyArray)."""
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
        cnt = (ct.c_int64 * 60)()
        _lib.call("octexIndexProfileBatch", self._handle, ct.byref(p), dq.ptr, ct.c_int64(k), ct.c_int32(reps), names,
                  ms, ct.byref(ns), cnt)
        raw = names.raw
        stages = [(raw[32 * i : 32 * i + 32].split(b"\0")[0].decode(), ms[i]) for i in range(ns.value)]
        c = list(cnt)
        counters = dict(seg_hits=c[0], entries1=c[1], distinct1=c[2], reranked1=c[3], starts2=c[4:20],
                        distinct2=c[20:36], reranked2=c[36:52], hit_level=c[52:60])
        return stages, counters

    def place_on_host(self, vectors=True, table=False, sketch=False):
        """Move the vectors / neighbor table / sketch to pinned host memory (the load placements
        vectors_on_host, table_on_host and sketch="host" for an index built in memory)."""
        _lib.call("octexIndexPlaceOnHost", self._handle, ct.c_int32(int(bool(vectors))),
                  ct.c_int32(int(bool(table))), ct.c_int32(int(bool(sketch))))
        return self

    def plan_info(self):
        arr = (ct.c_int32 * 10)()
        _lib.call("octexIndexPlanInfo", self._handle, arr)
        keys = ("m", "k", "KO", "lr", "W", "W2", "rerank", "wave_rerank", "final_rerank", "graph")
        return dict(zip(keys, list(arr)))

    def save(self, path):
        """Copy the index directory to `path` (a new directory); load(path) restores the index."""
        path = os.fspath(path)
        if os.path.exists(path) and (not os.path.isdir(path) or os.listdir(path)):
            raise FileExistsError(f"octex: {path} exists and is not an empty directory")
        if os.path.abspath(path) == os.path.abspath(self._path):
            return path
        shutil.copytree(self._path, path, dirs_exist_ok=True)
        return path


def load(path, devices=None, placement="shard", vectors_on_host=False, *, shard_vectors=False,
         table_on_host=False, sketch="replicate", parts=0, copies_per_part=0, copies_limit=0, list_limit=0):
    """Load an index directory onto the GPU (the first of `devices`, default the current one)."""
    path = os.fspath(path)
    if not os.path.isfile(os.path.join(path, "meta.json")):
        raise FileNotFoundError(f"octex: {path} is not an index directory (no meta.json)")
    check_metric(_meta(path).get("metric", "sqeuclidean"))
    args = dict(devices=devices, placement=placement, vectors_on_host=vectors_on_host, shard_vectors=shard_vectors,
                table_on_host=table_on_host, sketch=sketch, parts=parts, copies_per_part=copies_per_part,
                copies_limit=copies_limit, list_limit=list_limit)
    lp = load_params(**args)
    res = _lib.Resources()
    handle = ct.POINTER(_lib.IndexHandle)()
    _lib.call("cuvsOctexIndexCreate", ct.byref(handle))
    try:
        _lib.call("cuvsOctexLoad", res.h, os.fsencode(path), ct.byref(lp), handle)
    except Exception:
        _lib.lib().cuvsOctexIndexDestroy(handle)
        raise
    return Index(handle, path, load_args=args)


def build(dataset, path=None, *, metric="sqeuclidean", placement="shard", vectors_on_host=False,
          table_on_host=False, shard_vectors=False, sketch="replicate", **index_params_):
    """Build an index of `dataset` [n, dim] (float32 or float16; host or GPU) into `path` and load it."""
    check_metric(metric)
    params = index_params(**index_params_)
    if _is_torch(dataset):
        x = dataset.detach().contiguous()
    else:
        x = np.asarray(dataset)
        if x.dtype not in (np.float32, np.float16):
            x = x.astype(np.float32)
        x = np.ascontiguousarray(x)
    tmp = None
    if path is None:
        tmp = tempfile.TemporaryDirectory(prefix="octex-")
        path = tmp.name
    path = os.fspath(path)
    os.makedirs(path, exist_ok=True)
    res = _lib.Resources()
    dx = _lib.Dl(x)
    _lib.call("cuvsOctexBuild", res.h, ct.byref(params), dx.ptr, os.fsencode(path))
    idx = load(path, devices=index_params_.get("devices"), placement=placement, vectors_on_host=vectors_on_host,
               table_on_host=table_on_host, shard_vectors=shard_vectors, sketch=sketch)
    idx._tmpdir = tmp
    return idx


def build_in_memory(dataset, path=None, **index_params_):
    """Build an index of `dataset` [n, dim] in the GPU's memory and return it ready to search (no round trip
    through files); with `path` the index directory is written as well.  Returns (index, build seconds)."""
    params = index_params(**index_params_)
    if _is_torch(dataset):
        x = dataset.detach().contiguous()
    else:
        x = np.asarray(dataset)
        if x.dtype not in (np.float32, np.float16):
            x = x.astype(np.float32)
        x = np.ascontiguousarray(x)
    res = _lib.Resources()
    dx = _lib.Dl(x)
    handle = ct.POINTER(_lib.IndexHandle)()
    _lib.call("cuvsOctexIndexCreate", ct.byref(handle))
    secs = ct.c_double(0)
    try:
        _lib.call("octexBuildInMemory", res.h, ct.byref(params), dx.ptr,
                  os.fsencode(path) if path is not None else None, handle, ct.byref(secs))
    except Exception:
        _lib.lib().cuvsOctexIndexDestroy(handle)
        raise
    return Index(handle, path if path is not None else "", load_args={}), secs.value
