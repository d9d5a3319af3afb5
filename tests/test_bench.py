"""bench.py's helpers on the CPU: the workloads of BASELINE.json, the algorithmic byte counts of every stage
(both search modes), the committed rocprof traffic lookup, the distance check, and the one-GPU refusal."""

import os
import subprocess
import sys

import numpy as np
from conftest import ROOT

sys.path.insert(0, ROOT)
import bench  # noqa: E402

COUNTERS = dict(seg_hits=1_400_000, entries1=10_000 * 1800, distinct1=10_000 * 1700, reranked1=10_000 * 128,
                starts2=[10_000 * 64] * 16, distinct2=[10_000 * 3000] * 16, reranked2=[10_000 * 128] * 16,
                hit_level=[600_000, 500_000, 200_000, 80_000, 20_000, 0, 0, 0])


def test_workloads():
    assert {"deep100m", "sift1m", "gist1m", "cpu100k", "deep100m-host"} <= set(bench.CONFIGS)
    assert bench.CONFIGS["deep100m"]["n"] == 100_000_000 and bench.CONFIGS["deep100m"]["d"] == 96
    assert bench.CONFIGS["deep100m-host"]["host"] == ("vectors",)


def test_stage_bytes_cover_every_stage():
    args = dict(m=10_000, C=150, S=96, D=96, KO=64, table_len=64, starts=64, w=32, L=5, FR=32)
    for name in ("gather_lists", "gather_rows", "rerank_keep", "rerank_keep_wave", "probe", "project", "sketch_keep",
                 "sketch_keep_wave", "final_rerank"):
        b = bench.stage_bytes(name, 0, COUNTERS, **args)
        assert isinstance(b, int) and b > 0, name
    assert bench.stage_bytes("center", 0, COUNTERS, **args) is None
    # gather_rows: starts + table rows + every distinct sketch row at S + 8 bytes + the query's sketch
    want = 10_000 * 64 * 8 + 10_000 * 64 * 64 * 4 + 10_000 * 3000 * (96 + 8) + 10_000 * (96 * 4 + 4)
    assert bench.stage_bytes("gather_rows", 0, COUNTERS, **args) == want
    # candidates whose scores came from earlier rows: no sketch row, 8 bytes per earlier-row entry read
    reuse = dict(COUNTERS, known2=[1000] + [0] * 15, oldread2=[2500] + [0] * 15)
    assert bench.stage_bytes("gather_rows", 0, reuse, **args) == want - 1000 * 96 + 2500 * 8
    # the wave rerank does not read the rows of the selected candidates an earlier round reranked
    skip = dict(COUNTERS, skipped2=[300] + [0] * 15)
    assert (bench.stage_bytes("rerank_keep_wave", 0, COUNTERS, **args)
            - bench.stage_bytes("rerank_keep_wave", 0, skip, **args)) == 300 * 2 * 96


def test_measured_traffic_from_the_committed_profile():
    """The committed counters are of the workload's fixed point: its line reads them as measured."""
    import json

    prof = json.load(open(os.path.join(ROOT, "profiles", "traffic_deep100m.json")))
    p = bench.CONFIGS["deep100m"]["point"]
    assert all(prof["params"][x] == p[x] for x in ("read", "starts", "waves", "rerank", "wave_rerank"))
    t, src = bench.measured_traffic("deep100m", p, "gather_rows", 100_000_000, 2.5e9)
    assert t == prof["kernels"]["gather_rows"]["hbm_bytes_per_launch"] and "same parameters" in src
    t2, src2 = bench.measured_traffic("deep100m", dict(p, read=16), "gather_rows", 100_000_000, 2.5e9)
    assert t2 is not None and "per algorithmic byte" in src2
    assert bench.measured_traffic("sift1m", p, "gather_rows", 1_000_000, 1e9) == (None, None)


def test_distance_error():
    g = np.random.default_rng(0)
    X = g.standard_normal((500, 16)).astype(np.float32)
    Q = g.standard_normal((20, 16)).astype(np.float32)
    I = g.integers(0, 500, (20, 10))
    Xh = X.astype(np.float16).astype(np.float64)
    D = ((Xh[I] - Q.astype(np.float64)[:, None, :]) ** 2).sum(-1).astype(np.float32)
    assert bench.distance_error(X, Q, D, I) < 1e-6
    assert bench.distance_error(X, Q, D * 1.01, I) > 5e-3


def test_one_gpu_only():
    out = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert out.returncode != 0 and "one GPU" in (out.stdout + out.stderr)


def test_host_path_refuses_large_workloads():
    out = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--host-path"], capture_output=True, text=True)
    assert out.returncode == 2 and "at most 2,000,000 rows" in out.stderr and "100,000,000" in out.stderr


def test_every_workload_has_a_fixed_point():
    for name, cfg in bench.CONFIGS.items():
        if name == "small":
            continue
        p = cfg["point"]
        assert {"read", "starts", "waves", "rerank", "wave_rerank"} <= set(p), name


def test_host_cpu_record():
    h = bench.host_cpu()
    assert 1 <= h["threads"] <= 16 and h["threads"] <= h["affinity"] <= h["nproc"]
    assert isinstance(h["model"], str) and "16" in h["rule"]


def test_cpu_passes():
    """The CPU baseline repeats a whole batch that takes under half the target time, to about the target."""
    assert bench.cpu_passes(500, 1000, 1.0, 15.0) == 1  # a partial sample: one pass
    assert bench.cpu_passes(1000, 1000, 9.0, 15.0) == 1  # the whole batch, long enough
    assert bench.cpu_passes(1000, 1000, 2.4, 15.0) == 6
    assert bench.cpu_passes(1000, 1000, 7.4, 15.0) == 2
    assert bench.cpu_passes(1000, 1000, 0.0, 15.0) > 1000


def test_host_path():
    """configs[0]'s CPU path on a small mixture: the oracle builds with the workload's index parameters (member
    lists), searches every query on the host, and the result is checked against fp64 brute force."""
    cfg = dict(bench.CONFIGS["cpu100k"], n=4000, nq=64)
    assert cfg["host_path"]
    X, Q = bench.make_gauss(cfg)
    index = dict(cfg["index"], copies=16, list_len=32, table_len=32, log_buckets=12)
    point = dict(cfg["point"], batch=64)
    r = bench.host_path(X, Q, 10, index, point, threads=4)
    assert r["index"]["member_lists"] and not r["index"]["exact_lists"] and r["index"]["copies"] == 16
    assert r["index"]["log_buckets"] == 12 and r["search"] == point and r["threads"] == 4
    assert r["build_seconds"] >= 0 and r["value"] > 0 and r["unit"] == "queries/s"
    assert r["recall"] >= 0.95 and r["distance_max_rel_err"] < 1e-3
