"""The index directory format (format 1) on the CPU: the committed directory in the reference's on-disk form
(tests/golden/refdir, written by numpy with 1.0 and 2.0 headers, a relative "files" entry and a build_seconds
object; tests/golden/make_refdir.py) opens through the library's own checker (octexIndexCheckDirectory: the
host half of cuvsOctexLoad, no GPU call) and through the oracle's loader, with absolute "files" entries and the
parts / copies_per_part selection of load.cu:215-263; directories whose arrays disagree with meta.json are
refused with an error naming the file, before any array is read past its end."""

import ctypes as ct
import json
import os
import shutil

import numpy as np
import pytest
from conftest import exact_knn, recall

from oracle import oracle as O

REFDIR = os.path.join(os.path.dirname(__file__), "golden", "refdir")
QUERIES = os.path.join(os.path.dirname(__file__), "golden", "refdir_queries.npy")


@pytest.fixture(scope="module")
def L():
    from octex_amd import _lib

    return _lib


def check_directory(L, path, **load):
    from octex_amd import index as octex_index

    lp = octex_index.load_params(**load)
    info = (ct.c_int64 * 10)()
    L.call("octexIndexCheckDirectory", os.fsencode(path), ct.byref(lp), info)
    keys = ("n", "dim", "copies", "all_copies", "blocks", "levels", "list_len", "log_buckets", "sketch_width",
            "table_len")
    return dict(zip(keys, list(info)))


def refdir_copy(tmp_path, absolute=("table",)):
    """A copy of the reference-format directory with the arrays in `absolute` moved elsewhere and named in
    meta.json's "files" by absolute path (the remapping of load.cu:229-234)."""
    d = tmp_path / "refdir"
    shutil.copytree(REFDIR, d)
    text = (d / "meta.json").read_text()
    meta = json.loads(text)
    files = dict(meta["files"])
    far = tmp_path / "elsewhere"
    far.mkdir()
    for name in absolute:
        shutil.move(str(d / (name + ".npy")), str(far / (name + ".npy")))
        files[name] = str(far / (name + ".npy"))
    entries = ", ".join(f'"{k}": "{v}"' for k, v in files.items())
    text = text.replace(' "files": {"vectors": "data/vectors.npy"},', f' "files": {{{entries}}},')
    assert json.loads(text)["files"] == files
    (d / "meta.json").write_text(text)
    return str(d)


def test_refdir_is_in_the_reference_form():
    """What the fixture claims: numpy-written 1.0 and 2.0 headers, relative files entry, build_seconds."""
    meta = json.load(open(os.path.join(REFDIR, "meta.json")))
    assert meta["files"] == {"vectors": "data/vectors.npy"} and "total" in meta["build_seconds"]
    assert not os.path.exists(os.path.join(REFDIR, "vectors.npy"))
    versions = {}
    for name in ("lists", "keys", "table", "mean", "offsets"):
        with open(os.path.join(REFDIR, name + ".npy"), "rb") as f:
            versions[name] = np.lib.format.read_magic(f)
    assert versions["lists"] == versions["keys"] == versions["table"] == (2, 0)
    assert versions["mean"] == versions["offsets"] == (1, 0)


def test_check_directory_reads_the_reference_form(L, tmp_path):
    meta = json.load(open(os.path.join(REFDIR, "meta.json")))
    info = check_directory(L, REFDIR)
    assert info == dict(n=meta["n"], dim=meta["dim"], copies=meta["copies"], all_copies=meta["copies"],
                        blocks=meta["blocks"], levels=len(meta["spacings"]), list_len=meta["list_len"],
                        log_buckets=meta["log_buckets"], sketch_width=meta["sketch_width"],
                        table_len=meta["table_len"])
    moved = refdir_copy(tmp_path, absolute=("table", "sketch"))
    assert check_directory(L, moved) == info


@pytest.mark.parametrize("load,copies", [
    (dict(parts=2, copies_per_part=2), [0, 1, 3, 4]),
    (dict(parts=3), [0, 1, 2, 3, 4, 5]),
    (dict(copies_limit=4), [0, 1, 2, 3]),
    (dict(parts=2, copies_per_part=5), [0, 1, 2, 3, 4, 5]),
])
def test_copy_selection(L, load, copies):
    assert check_directory(L, REFDIR, **load)["copies"] == len(copies)
    assert list(O.copy_selection(6, **load)) == copies


def test_oracle_loads_and_searches_the_reference_form(tmp_path):
    moved = refdir_copy(tmp_path)
    ix = O.Index(moved)
    Q = np.load(QUERIES)
    X = O.h2f(ix.vectors).reshape(ix.n, ix.dim)
    gt, _ = exact_knn(X, Q)
    D, I = O.search(ix, Q, k=10, read=8, starts=32, waves=2, rerank=32, wave_rerank=32)
    assert recall(I, gt) >= 0.9
    # two parts of two copies: the arrays of copies 0, 1, 3, 4 of the whole directory
    part = O.Index(moved, parts=2, copies_per_part=2)
    full = O.Index(moved)
    sel = [0, 1, 3, 4]
    assert part.copies == 4
    assert np.array_equal(part.lists, full.lists[sel]) and np.array_equal(part.keys, full.keys[sel])
    w = full.width
    assert np.array_equal(part.ucat.reshape(ix.dim, 4, w), full.ucat.reshape(ix.dim, 6, w)[:, sel])


def rewrite(path, name, array):
    np.save(os.path.join(path, name + ".npy"), array)


@pytest.mark.parametrize("name,bad,match", [
    ("shift", lambda a: a[:, :-1], r"shift.npy has shape \(6, 15\), meta.json needs \(6, 16\)"),
    ("mean", lambda a: a.astype(np.float64), r"mean.npy has dtype <f8, expected <f4"),
    ("keys", lambda a: a[:5], r"keys.npy has shape \(5, 3, \d+\), meta.json needs \(6, 3, \*\)"),
    ("offsets", lambda a: a[:, :, :-1], r"offsets.npy has shape"),
    ("sketch_basis", lambda a: a[:, :-1], r"sketch_basis.npy has shape \(16, 15\), meta.json needs \(16, 16\)"),
    ("table", lambda a: a[:-1], r"table.npy has shape \(399, 8\)"),
    ("lists", lambda a: a[:, :-3], r"lists rows hold \d+ entries, not a multiple of list_len 8"),
    ("offsets", lambda a: np.where(np.arange(a.shape[2]) == a.shape[2] - 1, a + 10**6, a),
     r"its cells run past keys"),
    # a middle entry past the end of keys (first and last entries intact): the probe would read keys out of bounds
    ("offsets", lambda a: np.where((np.arange(a.shape[2]) == 3)[None, None, :] & (np.arange(a.shape[0]) == 2)[:, None, None],
                                   a[:, :, -1:] + 10**6, a).astype(np.int32),
     r"copy 2 level 0: .*bucket offsets decrease"),
    # a middle entry below its predecessor
    ("offsets", lambda a: np.where((np.arange(a.shape[2]) == a.shape[2] // 2)[None, None, :]
                                   & (np.arange(a.shape[1]) == 1)[None, :, None], -5, a).astype(np.int32),
     r"copy 0 level 1: .*bucket offsets decrease"),
])
def test_mismatched_directory_is_refused(L, tmp_path, name, bad, match):
    from octex_amd._lib import OctexError

    d = refdir_copy(tmp_path, absolute=())
    rewrite(d, name, bad(np.load(os.path.join(d, name + ".npy"))))
    with pytest.raises(OctexError, match=match):
        check_directory(L, d)


def test_truncated_and_foreign_files_are_refused(L, tmp_path):
    from octex_amd._lib import OctexError

    d = refdir_copy(tmp_path, absolute=())
    p = os.path.join(d, "sketch.npy")
    data = open(p, "rb").read()
    open(p, "wb").write(data[:-100])
    with pytest.raises(OctexError, match="sketch.npy holds \\d+ data bytes, its shape needs 6400"):
        check_directory(L, d)
    open(p, "wb").write(b"not an array at all")
    with pytest.raises(OctexError, match="sketch.npy is not an .npy file"):
        check_directory(L, d)
    np.save(p, np.asfortranarray(np.zeros((400, 16), np.int8)))
    with pytest.raises(OctexError, match="Fortran-order"):
        check_directory(L, d)
    os.remove(p)
    with pytest.raises(OctexError, match="cannot open .*sketch.npy"):
        check_directory(L, d)


def test_meta_json_errors(L, tmp_path):
    from octex_amd._lib import OctexError

    d = refdir_copy(tmp_path, absolute=())
    meta = os.path.join(d, "meta.json")
    text = open(meta).read()
    open(meta, "w").write(text.replace('"format": 1', '"format": 2'))
    with pytest.raises(OctexError, match="unknown index format"):
        check_directory(L, d)
    open(meta, "w").write(text.replace('"dim": 16', '"dim": 15'))
    with pytest.raises(OctexError, match="the dimension must be even"):
        check_directory(L, d)
    open(meta, "w").write(text.replace('"n": 400', '"n": -4'))
    with pytest.raises(OctexError, match="n must be a non-negative integer"):
        check_directory(L, d)
    open(meta, "w").write(text.replace('"copies": 6', '"copies": 0'))
    with pytest.raises(OctexError, match="a device holds no copies"):
        check_directory(L, d)


def npy_bytes(header, data=b"\0" * 64):
    """A version-1.0 .npy file with the given header dictionary text (padded as numpy pads it)."""
    h = header.encode() + b" "
    h += b" " * ((-(10 + len(h) + 1)) % 64) + b"\n"
    return b"\x93NUMPY\x01\x00" + len(h).to_bytes(2, "little") + h + data


@pytest.mark.parametrize("shape,match", [
    ("(4611686018427387904, 16)", r"malformed .npy header \(a dimension of 2\^62 or more\)"),
    ("(99999999999999999999999, 16)", r"malformed .npy header \(a dimension of 2\^62 or more\)"),
    ("(9999999999999999999, 16)", r"malformed .npy header \(a dimension of 2\^62 or more\)"),  # 19 digits
    ("(4611686018427387903, 1)", r"sketch.npy holds \d+ data bytes, its shape needs 4611686018427387903"),  # 2^62 - 1
    ("(4294967296, 4294967296, 16)", r"the shape's byte count overflows"),  # 2^68 elements: the count wraps
    ("(2305843009213693952, 4)", r"the shape's byte count overflows"),  # 2^63 elements x 1 byte
    ("(1152921504606846976, 16)", r"the shape's byte count overflows"),  # 2^64 bytes: wraps to zero
    ("(4000000000, 16)", r"sketch.npy holds \d+ data bytes, its shape needs 64000000000"),
])
def test_crafted_npy_shapes_are_refused(L, tmp_path, shape, match):
    """A header whose shape overflows int64 (elements or bytes) cannot pass the data-size check by wrapping."""
    from octex_amd._lib import OctexError

    d = refdir_copy(tmp_path, absolute=())
    with open(os.path.join(d, "sketch.npy"), "wb") as f:
        f.write(npy_bytes("{'descr': '|i1', 'fortran_order': False, 'shape': %s, }" % shape))
    with pytest.raises(OctexError, match=match):
        check_directory(L, d)
