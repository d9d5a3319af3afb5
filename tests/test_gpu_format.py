"""The committed directory in the reference's on-disk form (tests/golden/refdir: numpy-written 1.0 / 2.0 headers,
relative and absolute "files" entries, a build_seconds object) loaded by cuvsOctexLoad and searched on the GPU
against the CPU oracle over the same files, whole and as two parts of two copies (load.cu:215-263); and the
directory this library's builder writes, byte for byte what numpy.save writes for the same arrays."""

import json
import os

import numpy as np
import pytest
from test_format import QUERIES, refdir_copy
from test_gpu_search import assert_same_results, oracle_given_gpu_projections

from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def octex():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import octex_amd

    return octex_amd


P = dict(read=8, starts=32, waves=2, rerank=32, wave_rerank=32)


@pytest.mark.parametrize("load", [dict(), dict(parts=2, copies_per_part=2), dict(copies_limit=3, list_limit=5)])
def test_reference_form_directory_search_matches_oracle(octex, tmp_path, load):
    d = refdir_copy(tmp_path, absolute=("table", "sketch"))
    Q = np.load(QUERIES)
    index = octex.load(d, **load)
    oix = O.Index(d, **load)
    assert index.copies == oix.copies and index.size == 400 and index.dim == 16
    D, I = index.search(Q, k=10, **P)
    Do, Io, _, _, _ = oracle_given_gpu_projections(index, oix, Q, 10, **P)
    assert_same_results(D, I, Do, Io)


def test_builder_writes_numpy_files(octex, tmp_path):
    """Every .npy the builder writes equals numpy.save of the array it holds (header and data), and meta.json
    carries the reference writer's keys, build_seconds ending in total."""
    import io

    from conftest import clustered

    X, _ = clustered(n=3000, m=4, d=32, clusters=10, seed=8)
    path = str(tmp_path / "built")
    octex.build(X, path, copies=4, list_len=16, table_len=8, log_buckets=10, sketch_width=32, member_lists=True)
    names = [f for f in sorted(os.listdir(path)) if f.endswith(".npy")]
    assert {"mean.npy", "proj.npy", "shift.npy", "lists.npy", "keys.npy", "offsets.npy", "base.npy", "cells.npy",
            "sketch_basis.npy", "sketch_scale.npy", "sketch.npy", "vectors.npy", "table.npy"} <= set(names)
    for name in names:
        raw = open(os.path.join(path, name), "rb").read()
        buf = io.BytesIO()
        np.save(buf, np.load(os.path.join(path, name)))
        assert raw == buf.getvalue(), name
    meta = json.load(open(os.path.join(path, "meta.json")))
    assert list(meta)[:12] == ["format", "n", "dim", "copies", "blocks", "spacings", "list_len", "log_buckets",
                               "sketch_width", "table_len", "metric", "files"]
    assert list(meta["build_seconds"])[-1] == "total"
