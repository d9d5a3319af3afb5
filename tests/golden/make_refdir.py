"""Writes tests/golden/refdir/: a small index directory in the reference's on-disk form (docs/design.md:27-54 of
the reference; meta.json as its writer lays it out, build.cu:67-98), so that the loader is tested on files that
did not come from this repository's own writers:

- every array saved by numpy itself: np.save (format 1.0 headers) for most, np.lib.format.write_array with
  version (2, 0) for lists, keys and table;
- meta.json with the reference writer's key order and spacing, a "files" map sending `vectors` to a
  subdirectory by a relative path, and a "build_seconds" object ending in "total";
- 6 copies, so that a load with parts = 2 and copies_per_part selects copies {0, 1, 3, 4}.

The index content comes from the CPU oracle's builder (a restatement of the reference's build, seeded); only
the file encoding is redone here.  Tests copy the directory and add an absolute "files" entry at run time.

    python tests/golden/make_refdir.py
"""

import json
import os
import shutil
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402

OUT = os.path.join(HERE, "refdir")
V2 = ("lists", "keys", "table")


def data(n=400, m=32, d=16, clusters=6, seed=17):
    g = np.random.default_rng(seed)
    centers = g.standard_normal((clusters, d)).astype(np.float32) * 3
    X = (centers[g.integers(clusters, size=n)] + g.standard_normal((n, d))).astype(np.float32)
    Q = (centers[g.integers(clusters, size=m)] + g.standard_normal((m, d))).astype(np.float32)
    return X, Q


def main():
    X, Q = data()
    with tempfile.TemporaryDirectory() as tmp:
        O.build(X, tmp, copies=6, blocks=2, pca_dims=16, spacings=[1.5, 2.5, 4.0], list_len=8, min_cell=1,
                log_buckets=6, sketch_width=16, table_len=8, reverse_edges=True, member_lists=True, seed=9)
        meta = json.load(open(os.path.join(tmp, "meta.json")))
        if os.path.isdir(OUT):
            shutil.rmtree(OUT)
        os.makedirs(os.path.join(OUT, "data"))
        for name in ("mean", "proj", "shift", "lists", "keys", "offsets", "base", "cells", "sketch_basis",
                     "sketch_scale", "sketch", "table", "vectors"):
            a = np.load(os.path.join(tmp, name + ".npy"))
            where = os.path.join(OUT, "data" if name == "vectors" else "", name + ".npy")
            if name in V2:
                with open(where, "wb") as f:
                    np.lib.format.write_array(f, a, version=(2, 0))
            else:
                np.save(where, a)
    # the reference writer's layout (build.cu:67-98): one key per line, spacings as shortest floats
    spacings = ", ".join(repr(float(v)) for v in meta["spacings"])
    text = (
        "{\n"
        f' "format": 1,\n "n": {meta["n"]},\n "dim": {meta["dim"]},\n "copies": {meta["copies"]},\n'
        f' "blocks": {meta["blocks"]},\n "spacings": [{spacings}],\n "list_len": {meta["list_len"]},\n'
        f' "log_buckets": {meta["log_buckets"]},\n "sketch_width": {meta["sketch_width"]},\n'
        f' "table_len": {meta["table_len"]},\n "metric": "sqeuclidean",\n'
        ' "files": {"vectors": "data/vectors.npy"},\n'
        ' "build_seconds": {"setup": 0.012, "cells": 0.034, "table": 0.056, "total": 0.102}\n'
        "}\n"
    )
    with open(os.path.join(OUT, "meta.json"), "w") as f:
        f.write(text)
    np.save(os.path.join(HERE, "refdir_queries.npy"), Q)
    print("reference-format index directory written to", OUT)


if __name__ == "__main__":
    main()
