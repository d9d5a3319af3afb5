"""The drop-in boundary without a GPU: liboctex_amd.so loads and exports every function that include/*.h
declares; parameter defaults are the reference's (octex.hpp:32-176; c/tests/neighbors/octex_c.cu:203-215); the
C ABI's error texts (octex_c.cu:221-242) and struct layouts."""

import ctypes as ct
import os
import re
import subprocess

import numpy as np
import pytest

from octex_amd import _lib
from octex_amd import index as octex_index

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = ["include/cuvs/core/c_api.h", "include/cuvs/neighbors/octex.h", "include/octex_amd/octex_amd.h"]


def declared_functions():
    names = set()
    for h in HEADERS:
        text = open(os.path.join(ROOT, h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(\w+)\s*\(", text, flags=re.M))
    return names - {"if", "while", "for"}


def test_library_exports_every_declared_function():
    names = declared_functions()
    assert len(names) >= 37
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = names - exported
    assert not missing, f"declared but not exported: {sorted(missing)}"
    L = _lib.lib()
    for n in names:
        getattr(L, n)


def test_struct_layouts_match_the_header(tmp_path):
    src = tmp_path / "sz.c"
    src.write_text(
        "#include <stdio.h>\n#include <stddef.h>\n#include <cuvs/neighbors/octex.h>\n"
        "int main(void){printf(\"%zu %zu %zu %zu %zu %zu\\n\", sizeof(struct cuvsOctexIndexParams),"
        " sizeof(struct cuvsOctexSearchParams), sizeof(struct cuvsOctexLoadParams),"
        " offsetof(struct cuvsOctexIndexParams, seed), offsetof(struct cuvsOctexSearchParams, use_graph),"
        " offsetof(struct cuvsOctexLoadParams, list_limit)); return 0;}\n"
    )
    exe = tmp_path / "sz"
    subprocess.run(["gcc", "-std=c99", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    exp = [ct.sizeof(_lib.IndexParams), ct.sizeof(_lib.SearchParams), ct.sizeof(_lib.LoadParams),
           _lib.IndexParams.seed.offset, _lib.SearchParams.use_graph.offset, _lib.LoadParams.list_limit.offset]
    assert [int(v) for v in got] == exp


def test_parameter_defaults():
    p = octex_index.search_params()
    assert (p.read, p.starts, p.waves, p.rerank, p.wave_rerank, p.batch) == (32, 128, 2, 128, 128, 10000)
    assert (p.sketch_rank, p.final_rerank, p.balanced_gather, p.fused_merge, p.use_graph) == (False, 32, True, True, True)
    ip = octex_index.index_params()
    assert (ip.copies, ip.blocks, ip.pca_dims, ip.list_len, ip.min_cell, ip.log_buckets) == (200, 4, 64, 64, 1, 20)
    assert (ip.sketch_width, ip.table_len, ip.reverse_edges, ip.exact_lists, ip.list_probes) == (0, 64, True, False, 16)
    assert (ip.member_lists, ip.exact_table_max, ip.table_passes, ip.seed, ip.n_spacings) == (False, 20000000, 3, 0, 0)
    lp = octex_index.load_params()
    assert (lp.placement, lp.sketch, lp.vectors_on_host, lp.parts, lp.copies_limit, lp.list_limit) == (1, 0, False, 0, 0, 0)


def test_error_texts_without_gpu():
    h = ct.POINTER(_lib.IndexHandle)()
    _lib.call("cuvsOctexIndexCreate", ct.byref(h))
    v = ct.c_int64()
    assert _lib.lib().cuvsOctexIndexGetSize(h, ct.byref(v)) == _lib.CUVS_ERROR
    assert "empty" in _lib.lib().cuvsGetLastErrorText().decode()
    res = _lib.Resources()
    # a float64 dataset is refused before any work
    x = np.zeros((10, 4), np.float64)
    t = _lib.Dl.__new__(_lib.Dl)
    t.owner = x
    t.shape = (ct.c_int64 * 2)(10, 4)
    t.strides = (ct.c_int64 * 2)(4, 1)
    t.m = _lib.DLManagedTensor()
    t.m.dl_tensor = _lib.DLTensor(ct.c_void_p(x.ctypes.data), _lib.DLDevice(_lib.kDLCPU, 0), 2,
                                  _lib.DLDataType(_lib.kDLFloat, 64, 1), t.shape, t.strides, 0)
    ip = octex_index.index_params()
    assert _lib.lib().cuvsOctexBuild(res.h, ct.byref(ip), t.ptr, b"/tmp/never") == _lib.CUVS_ERROR
    assert "float32 or float16" in _lib.lib().cuvsGetLastErrorText().decode()
    # an unknown placement is refused before the directory is read
    lp = octex_index.load_params()
    lp.placement = 7
    assert _lib.lib().cuvsOctexLoad(res.h, b"/tmp/never", ct.byref(lp), h) == _lib.CUVS_ERROR
    assert "placement" in _lib.lib().cuvsGetLastErrorText().decode()
    assert _lib.lib().cuvsOctexSearch(res.h, None, h, None, None, None) == _lib.CUVS_ERROR
    _lib.call("cuvsOctexIndexDestroy", h)
    # a success clears the text
    _lib.call("cuvsOctexIndexCreate", ct.byref(h))
    assert _lib.lib().cuvsGetLastErrorText().decode() == ""
    _lib.call("cuvsOctexIndexDestroy", h)


def test_python_parameter_errors():
    with pytest.raises(TypeError, match="unknown search parameter"):
        octex_index.search_params(reads=3)
    with pytest.raises(ValueError, match="placement must be one of"):
        octex_index.load_params(placement="everywhere")
    with pytest.raises(ValueError, match="squared Euclidean"):
        octex_index.check_metric("cosine")
