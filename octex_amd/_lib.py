"""ctypes binding of liboctex_amd.so: the cuvsOctex* C ABI (include/cuvs/neighbors/octex.h), the cuVS core
calls it needs (include/cuvs/core/c_api.h), and the introspection / stage entry points
(include/octex_amd/octex_amd.h).  Tensors cross the boundary as DLPack structs built here from numpy arrays
(kDLCPU) or PyTorch tensors (kDLROCM on the GPU, kDLCPU on the host)."""

import ctypes as ct
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "liboctex_amd.so")

kDLCPU, kDLROCM, kDLROCMHost = 1, 10, 11
kDLInt, kDLUInt, kDLFloat = 0, 1, 2
CUVS_ERROR, CUVS_SUCCESS = 0, 1


class DLDevice(ct.Structure):
    _fields_ = [("device_type", ct.c_int), ("device_id", ct.c_int32)]


class DLDataType(ct.Structure):
    _fields_ = [("code", ct.c_uint8), ("bits", ct.c_uint8), ("lanes", ct.c_uint16)]


class DLTensor(ct.Structure):
    _fields_ = [
        ("data", ct.c_void_p),
        ("device", DLDevice),
        ("ndim", ct.c_int32),
        ("dtype", DLDataType),
        ("shape", ct.POINTER(ct.c_int64)),
        ("strides", ct.POINTER(ct.c_int64)),
        ("byte_offset", ct.c_uint64),
    ]


class DLManagedTensor(ct.Structure):
    _fields_ = [("dl_tensor", DLTensor), ("manager_ctx", ct.c_void_p), ("deleter", ct.c_void_p)]


class IndexParams(ct.Structure):
    """struct cuvsOctexIndexParams (octex.h; the reference's octex.h:31-76, same field order)."""

    _fields_ = [
        ("copies", ct.c_int32),
        ("blocks", ct.c_int32),
        ("pca_dims", ct.c_int32),
        ("spacings", ct.POINTER(ct.c_float)),
        ("n_spacings", ct.c_int32),
        ("list_len", ct.c_int32),
        ("min_cell", ct.c_int32),
        ("log_buckets", ct.c_int32),
        ("sketch_width", ct.c_int32),
        ("table_len", ct.c_int32),
        ("reverse_edges", ct.c_bool),
        ("exact_lists", ct.c_bool),
        ("list_probes", ct.c_int32),
        ("member_lists", ct.c_bool),
        ("exact_table_max", ct.c_int64),
        ("table_passes", ct.c_int32),
        ("table_sketch_order", ct.c_bool),
        ("write_behind", ct.c_bool),
        ("seed", ct.c_uint64),
        ("devices", ct.POINTER(ct.c_int32)),
        ("n_devices", ct.c_int32),
    ]


class LoadParams(ct.Structure):
    """struct cuvsOctexLoadParams (the reference's octex.h:117-140)."""

    _fields_ = [
        ("devices", ct.POINTER(ct.c_int32)),
        ("n_devices", ct.c_int32),
        ("placement", ct.c_int),
        ("vectors_on_host", ct.c_bool),
        ("shard_vectors", ct.c_bool),
        ("table_on_host", ct.c_bool),
        ("sketch", ct.c_int),
        ("parts", ct.c_int32),
        ("copies_per_part", ct.c_int32),
        ("copies_limit", ct.c_int32),
        ("list_limit", ct.c_int32),
    ]


class SearchParams(ct.Structure):
    """struct cuvsOctexSearchParams (the reference's octex.h:161-184)."""

    _fields_ = [
        ("read", ct.c_int32),
        ("starts", ct.c_int32),
        ("waves", ct.c_int32),
        ("rerank", ct.c_int32),
        ("wave_rerank", ct.c_int32),
        ("batch", ct.c_int32),
        ("sketch_rank", ct.c_bool),
        ("final_rerank", ct.c_int32),
        ("balanced_gather", ct.c_bool),
        ("fused_merge", ct.c_bool),
        ("use_graph", ct.c_bool),
    ]


class IndexHandle(ct.Structure):
    _fields_ = [("addr", ct.c_size_t)]


EXPORTS = (
    "cuvsResourcesCreate", "cuvsResourcesDestroy", "cuvsStreamSet", "cuvsStreamGet", "cuvsStreamSync",
    "cuvsGetLastErrorText", "cuvsSetLastErrorText",
    "cuvsOctexIndexParamsCreate", "cuvsOctexIndexParamsDestroy", "cuvsOctexLoadParamsCreate",
    "cuvsOctexLoadParamsDestroy", "cuvsOctexSearchParamsCreate", "cuvsOctexSearchParamsDestroy",
    "cuvsOctexIndexCreate", "cuvsOctexIndexDestroy", "cuvsOctexIndexGetSize", "cuvsOctexIndexGetDim",
    "cuvsOctexIndexGetCopies", "cuvsOctexIndexGetNumDevices", "cuvsOctexIndexGetDevices",
    "cuvsOctexIndexGetDeviceBytes", "cuvsOctexBuild", "cuvsOctexLoad", "cuvsOctexSearch",
    "octexIndexCopyPlanBuffer", "octexIndexPlanInfo", "octexBuildInMemory", "octexIndexProfileBatch", "octexIndexCopyArray",
    "octexIndexCopyArrayRange", "octexIndexCopyArrayRanges", "octexIndexCheckDirectory", "octexSearchNoAlloc",
    "octexStageCenter", "octexStageProject", "octexStageSketchQuery", "octexStageE8", "octexStageProbe",
    "octexStageGather", "octexStageRerankKeep", "octexStageSketchKeep", "octexStagePickStarts",
    "octexStageFinalRerank", "octexStageTakeK", "octexMeasureRowReads",
)

_lib = None


class OctexError(RuntimeError):
    pass


def lib():
    """The loaded library; a missing or unloadable library is an error (there is no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"octex_amd: {LIB_PATH} is missing; build it with __graft_entry__.build()")
        L = ct.CDLL(LIB_PATH)
        for name in EXPORTS:
            getattr(L, name).restype = ct.c_int
        L.cuvsGetLastErrorText.restype = ct.c_char_p
        L.cuvsSetLastErrorText.restype = None
        _lib = L
    return _lib


def check(rc):
    if rc != CUVS_SUCCESS:
        raise OctexError(lib().cuvsGetLastErrorText().decode())


def call(name, *args):
    check(getattr(lib(), name)(*args))


# ---------------------------------------------------------------- DLPack


_DTYPES = {
    np.dtype(np.float32): (kDLFloat, 32),
    np.dtype(np.float16): (kDLFloat, 16),
    np.dtype(np.int64): (kDLInt, 64),
    np.dtype(np.int32): (kDLInt, 32),
    np.dtype(np.int8): (kDLInt, 8),
    np.dtype(np.uint8): (kDLUInt, 8),
}


class Dl:
    """A DLManagedTensor over a numpy array or torch tensor (the owner is kept alive with it)."""

    def __init__(self, a):
        self.owner = a
        if isinstance(a, np.ndarray):
            data, shape, strides_b, itemsize = a.ctypes.data, a.shape, a.strides, a.itemsize
            dt = a.dtype
            dev = DLDevice(kDLCPU, 0)
        else:  # torch
            import torch

            t = a
            data, shape, itemsize = t.data_ptr(), tuple(t.shape), t.element_size()
            strides_b = tuple(s * itemsize for s in t.stride())
            dt = np.dtype(str(t.dtype).replace("torch.", ""))
            dev = DLDevice(kDLROCM, t.device.index or 0) if t.is_cuda else DLDevice(kDLCPU, 0)
        code, bits = _DTYPES[np.dtype(dt)]
        nd = len(shape)
        self.shape = (ct.c_int64 * max(nd, 1))(*shape)
        self.strides = (ct.c_int64 * max(nd, 1))(*[s // itemsize for s in strides_b])
        self.m = DLManagedTensor()
        self.m.dl_tensor = DLTensor(
            ct.c_void_p(data), dev, nd, DLDataType(code, bits, 1), self.shape, self.strides, 0
        )
        self.m.manager_ctx = None
        self.m.deleter = None

    @property
    def ptr(self):
        return ct.byref(self.m)


class Resources:
    """A cuvsResources_t (current device, null stream unless set)."""

    def __init__(self, stream=None):
        self.h = ct.c_size_t(0)
        call("cuvsResourcesCreate", ct.byref(self.h))
        if stream is not None:
            call("cuvsStreamSet", self.h, ct.c_void_p(stream))

    def sync(self):
        call("cuvsStreamSync", self.h)

    def __del__(self):
        if getattr(self, "h", None) is not None and self.h.value and _lib is not None:
            _lib.cuvsResourcesDestroy(self.h)
            self.h = None
