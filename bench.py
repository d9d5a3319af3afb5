#!/usr/bin/env python3
"""Benchmark of octex's batched search on one MI355X: queries/sec at recall@10 >= 0.99 (k = 10), with the achieved
HBM bandwidth of the dominant kernel against the roofline and the CPU oracle's rate on the same index.

Workload (default --config deep100m, BASELINE.json configs[3], the north star's target): 100M L2-normalized rows,
d = 96, of a 10,000-component Gaussian mixture (centroids N(0, 1), sigma 0.4) stored fp16 in HBM; 10,000 queries
from the same mixture; k = 10, batch 10,000.  --config sift1m is configs[1] (1M x 128 SIFT-like mixture).  Seeded
synthetic data (no datasets are downloaded).  The index is built on the GPU by this library's builder at the start
of the run (about 6 minutes at 100M).

Protocol (the reference's octex_bench.cu:223-242): queries resident in HBM, one capture run, warm-up, then `steps`
timed searches of the whole batch bracketed by device synchronizations.  A short sweep over search parameters picks
the fastest setting whose recall@10 against exact search is >= 0.99.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, vendor figure
HOST_PATH_MAX_ROWS = 2_000_000  # the CPU oracle's build holds every copy's projection and an n^2 exact table pass

# Cell lists, per workload (every BENCH line records its index parameters in config.index):
# - sift1m: exact lists, as the reference's paper builds (bench/paper_build.sh:29, --exact-lists): 818 s to build here;
# - gist1m: member lists.  The paper's exact lists (bench/paper_build.sh:30) took 850 s for 80 of the 150 copies here,
#   about 27 minutes in all, more than one GPU session allows; member lists hold members of the query's cell;
# - deep100m and deep100m-host: member lists, the reference's fast build mode (--member-lists).  The paper's Deep100M
#   build uses the default IVF lists (bench/paper_build.sh:36), whose k-means and probed list search over 100M rows for
#   every copy do not fit a GPU session here; member lists hold members of the query's cell instead of the rows
#   nearest to its center, so this index is not the paper's;
# - cpu100k: the reference's default index, IVF lists included.
CONFIGS = {
    # configs[1] of BASELINE.json; the index as the reference's paper SIFT1M build (copies 200, lists of 32, exact
    # lists, table 64, no reverse edges) with the reference's default sketch width for d = 128 (128; the paper's 64)
    "sift1m": dict(n=1_000_000, d=128, nq=10_000, clusters=1000, kind="sift", batch=10_000,
                   desc="seeded Gaussian mixture as BASELINE.json configs[1]",
                   index=dict(copies=200, list_len=32, table_len=64, reverse_edges=False, exact_lists=True, seed=0),
                   point=dict(read=4, starts=16, waves=1, rerank=16, wave_rerank=16)),
    # configs[3] of BASELINE.json: 100M L2-normalized rows, d = 96, of a 10,000-component mixture (centroids N(0, 1),
    # sigma 0.4) stored fp16; the index shaped as the reference's paper Deep100M build (lists of 64, cells of >= 10
    # rows, table 64) but with member lists (see above), the reference's default sketch width for d = 96 (96: this
    # mixture's variance is spread over all 96 PCA axes, so a 64-wide sketch ranks poorly), and as many copies as fit
    # one MI355X's 288 GB next to the vectors, sketch, table and search buffers (1.3 GB of lists per copy here)
    "deep100m": dict(n=100_000_000, d=96, nq=10_000, clusters=10_000, kind="deep", batch=10_000,
                     desc="seeded normalized Gaussian mixture as BASELINE.json configs[3], fp16 rows",
                     index=dict(copies=150, list_len=64, min_cell=10, table_len=64, member_lists=True, seed=0),
                     point=dict(read=12, starts=64, waves=2, rerank=64, wave_rerank=64)),
    # configs[4] of BASELINE.json (1B rows, fp16 vectors in pinned host memory, sketch-rank search) at a tenth of its
    # size: a 1B index does not build within one GPU session here.  The rows of deep100m; the index as configs[4]
    # (lists of 16, searched table of 32, sketch 96 in HBM) with the vectors moved to pinned host memory after the
    # build; sketch-rank search with a final exact rerank of 32 over the host link (frontier_deep1B.jsonl:41 of
    # the reference: read 16, starts 512, waves 5)
    "deep100m-host": dict(n=100_000_000, d=96, nq=10_000, clusters=10_000, kind="deep", batch=10_000,
                          desc="seeded normalized Gaussian mixture as BASELINE.json configs[3]/[4], fp16 rows, "
                               "vectors in pinned host memory",
                          index=dict(copies=150, list_len=16, min_cell=10, table_len=32, member_lists=True, seed=0),
                          host=("vectors",),
                          point=dict(read=16, starts=128, waves=3, rerank=128, wave_rerank=128, sketch_rank=True,
                                     final_rerank=32)),
    # configs[2] of BASELINE.json: 1M x 960 non-negative half-normal features (scale 0.05) plus per-cluster offsets
    # U[0, 0.1] of a 1,000-component mixture, 1,000 queries, batch 1,000; the index shaped as the reference's paper
    # GIST build (lists of 64, sketch 128, exact table of 64, no reverse edges) with member lists of cells of >= 16
    # rows (see above) and 150 copies (the paper's 400 do not fit next to this index's arrays: 0.70 GB a copy)
    "gist1m": dict(n=1_000_000, d=960, nq=1_000, clusters=1000, kind="gist", batch=1_000,
                   desc="seeded half-normal mixture as BASELINE.json configs[2]",
                   index=dict(copies=150, list_len=64, min_cell=16, table_len=64, sketch_width=128,
                              reverse_edges=False, member_lists=True, seed=0),
                   point=dict(read=32, starts=64, waves=3, rerank=512, wave_rerank=512)),
    # configs[0] of BASELINE.json, the reference's CPU-runnable case: 100k rows, d = 128, of a 100-component
    # Gaussian mixture (centroids N(0, 1), sigma 0.3), 1,000 queries, the reference's default index (200 copies,
    # lists of 64, exact table of 64 with reverse edges) but for log_buckets 16; the search sweep ends at the
    # default read 32 / starts 128 / waves 2.  Its CPU baseline also times the host path the configuration names
    # (host_path): the CPU oracle builds the index and searches it on the host
    "cpu100k": dict(n=100_000, d=128, nq=1_000, clusters=100, kind="gauss", batch=1_000,
                    desc="seeded Gaussian mixture as BASELINE.json configs[0]",
                    index=dict(log_buckets=16, seed=0), host_path=True,
                    point=dict(read=32, starts=128, waves=2, rerank=128, wave_rerank=128)),
    # a small stand-in for quick checks
    "small": dict(n=100_000, d=128, nq=10_000, clusters=100, kind="sift", batch=10_000, desc="small SIFT-like mixture",
                  index=dict(copies=64, list_len=32, table_len=64, min_cell=2, reverse_edges=False, member_lists=True,
                             seed=0, log_buckets=18)),
}

SWEEP_DEEP = [
    dict(read=8, starts=32, waves=1, rerank=64, wave_rerank=64),
    dict(read=16, starts=32, waves=1, rerank=64, wave_rerank=64),
    dict(read=16, starts=32, waves=2, rerank=64, wave_rerank=64),
    dict(read=16, starts=64, waves=1, rerank=128, wave_rerank=128),
    dict(read=16, starts=48, waves=2, rerank=96, wave_rerank=96),
    dict(read=12, starts=64, waves=2, rerank=128, wave_rerank=128),
    dict(read=12, starts=64, waves=2, rerank=64, wave_rerank=128),
    dict(read=12, starts=64, waves=2, rerank=96, wave_rerank=96),
    dict(read=12, starts=64, waves=2, rerank=64, wave_rerank=64),
    dict(read=10, starts=64, waves=2, rerank=64, wave_rerank=64),
    dict(read=12, starts=64, waves=2, rerank=128, wave_rerank=96),
    dict(read=10, starts=64, waves=2, rerank=128, wave_rerank=128),
    dict(read=12, starts=56, waves=2, rerank=112, wave_rerank=112),
    dict(read=16, starts=64, waves=2, rerank=96, wave_rerank=96),
    dict(read=16, starts=64, waves=2, rerank=64, wave_rerank=128),
    dict(read=16, starts=64, waves=2, rerank=128, wave_rerank=128),
    dict(read=32, starts=64, waves=2, rerank=128, wave_rerank=128),
    dict(read=16, starts=128, waves=2, rerank=128, wave_rerank=128),
    dict(read=32, starts=128, waves=2, rerank=128, wave_rerank=256),
]

SWEEP_GIST = [
    dict(read=16, starts=32, waves=1, rerank=64, wave_rerank=64),
    dict(read=32, starts=64, waves=2, rerank=128, wave_rerank=128),
    dict(read=64, starts=128, waves=3, rerank=256, wave_rerank=256),
    dict(read=32, starts=64, waves=3, rerank=512, wave_rerank=512),
    dict(read=64, starts=64, waves=4, rerank=512, wave_rerank=512),
    dict(read=64, starts=128, waves=3, rerank=512, wave_rerank=512),
    dict(read=64, starts=128, waves=4, rerank=256, wave_rerank=512),
    dict(read=32, starts=128, waves=4, rerank=512, wave_rerank=512),
    dict(read=64, starts=128, waves=4, rerank=512, wave_rerank=512),
]

SWEEP_HOST = [  # sketch-rank mode: the exact distances only in the final rerank, over the host link
    dict(read=16, starts=128, waves=3, rerank=128, wave_rerank=128, sketch_rank=True, final_rerank=32),
    dict(read=16, starts=128, waves=4, rerank=128, wave_rerank=128, sketch_rank=True, final_rerank=32),
    dict(read=16, starts=192, waves=3, rerank=128, wave_rerank=128, sketch_rank=True, final_rerank=32),
    dict(read=16, starts=192, waves=4, rerank=128, wave_rerank=128, sketch_rank=True, final_rerank=32),
    dict(read=16, starts=256, waves=4, rerank=128, wave_rerank=128, sketch_rank=True, final_rerank=32),
    dict(read=16, starts=512, waves=5, rerank=128, wave_rerank=128, sketch_rank=True, final_rerank=32),
    dict(read=32, starts=512, waves=5, rerank=128, wave_rerank=128, sketch_rank=True, final_rerank=64),
]

SWEEP = [  # ordered from cheaper to dearer; the fastest one at recall >= 0.99 is timed
    dict(read=4, starts=16, waves=1, rerank=16, wave_rerank=16),
    dict(read=4, starts=32, waves=1, rerank=16, wave_rerank=16),
    dict(read=8, starts=16, waves=1, rerank=16, wave_rerank=16),
    dict(read=8, starts=32, waves=1, rerank=32, wave_rerank=32),
    dict(read=16, starts=32, waves=1, rerank=32, wave_rerank=32),
    dict(read=32, starts=64, waves=2, rerank=64, wave_rerank=64),
    dict(read=32, starts=128, waves=2, rerank=128, wave_rerank=128),
]


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def make_data(cfg):
    """SIFT-like mixture: centroids U[0, 128]^d, sigma 12, clipped to [0, 255], rounded (data seed 0, queries 1)."""
    d, C = cfg["d"], cfg["clusters"]
    g = np.random.default_rng(0)
    centers = g.uniform(0, 128, (C, d)).astype(np.float32)
    X = np.empty((cfg["n"], d), np.float32)
    step = 1 << 18
    for r0 in range(0, cfg["n"], step):
        m = min(step, cfg["n"] - r0)
        a = g.integers(0, C, m)
        X[r0 : r0 + m] = np.rint(np.clip(centers[a] + 12 * g.standard_normal((m, d), dtype=np.float32), 0, 255))
    gq = np.random.default_rng(1)
    a = gq.integers(0, C, cfg["nq"])
    Q = np.rint(np.clip(centers[a] + 12 * gq.standard_normal((cfg["nq"], d), dtype=np.float32), 0, 255))
    return X, Q.astype(np.float32)


class TopK:
    """Running exact k nearest neighbors of the queries Qd (fp32 on the GPU) over row blocks of the base."""

    def __init__(self, Qd, k, torch):
        self.torch, self.Q, self.k = torch, Qd, k
        self.d = torch.full((len(Qd), k), float("inf"), device=Qd.device)
        self.i = torch.zeros((len(Qd), k), dtype=torch.int64, device=Qd.device)

    def add(self, Xb, r0):
        torch = self.torch
        dd = (Xb * Xb).sum(1)[None, :] - 2 * (self.Q @ Xb.T)
        v, i = torch.topk(dd, self.k, dim=1, largest=False)
        cd = torch.cat([self.d, v], 1)
        ci = torch.cat([self.i, i + r0], 1)
        o = torch.argsort(cd, dim=1)[:, : self.k]
        self.d, self.i = torch.gather(cd, 1, o), torch.gather(ci, 1, o)


def make_deep(cfg, k, torch):
    """Deep-like rows on the GPU: centroids N(0, 1)^d, rows = centroid + 0.4 N(0, 1), L2-normalized, stored fp16
    (torch's CUDA generator, seed 0 for the base and 1 for the queries).  The exact neighbors are computed block
    by block as the rows are made, over the fp16 values; the base goes to host memory."""
    d, C, n, nq = cfg["d"], cfg["clusters"], cfg["n"], cfg["nq"]
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    centers = torch.randn((C, d), generator=g, device="cuda")
    gq = torch.Generator(device="cuda")
    gq.manual_seed(1)
    Q = centers[torch.randint(0, C, (nq,), generator=gq, device="cuda")]
    Q = Q + 0.4 * torch.randn((nq, d), generator=gq, device="cuda")
    Q = (Q / Q.norm(dim=1, keepdim=True)).contiguous()
    X = np.empty((n, d), np.float16)
    top = TopK(Q, k, torch)
    step = 1 << 18
    for r0 in range(0, n, step):
        m = min(step, n - r0)
        x = centers[torch.randint(0, C, (m,), generator=g, device="cuda")]
        x = x + 0.4 * torch.randn((m, d), generator=g, device="cuda")
        xh = (x / x.norm(dim=1, keepdim=True)).half()
        top.add(xh.float(), r0)
        X[r0 : r0 + m] = xh.cpu().numpy()
        if r0 % (1 << 24) == 0:
            log(f"data: {r0 + m:,} of {n:,} rows")
    return X, Q.cpu().numpy(), top.i.cpu().numpy()


def make_gauss(cfg):
    """Gaussian mixture: centroids N(0, 1)^d, rows = centroid + 0.3 N(0, 1) (data seed 0, queries 1)."""
    d, C = cfg["d"], cfg["clusters"]
    g = np.random.default_rng(0)
    centers = g.standard_normal((C, d), dtype=np.float32)
    X = (centers[g.integers(0, C, cfg["n"])] + 0.3 * g.standard_normal((cfg["n"], d), dtype=np.float32))
    gq = np.random.default_rng(1)
    Q = centers[gq.integers(0, C, cfg["nq"])] + 0.3 * gq.standard_normal((cfg["nq"], d), dtype=np.float32)
    return X.astype(np.float32), Q.astype(np.float32)


def distance_error(X, Q, D, I, rows=1000):
    """Largest relative error of the returned distances against fp64 distances over the fp16 rows (first rows
    queries)."""
    Qs, Ds, Is = Q[:rows].astype(np.float64), np.asarray(D[:rows], np.float64), np.asarray(I[:rows])
    V = np.asarray(X[np.clip(Is, 0, None).ravel()], dtype=np.float16).astype(np.float64).reshape(*Is.shape, -1)
    exact = ((V - Qs[:, None, :]) ** 2).sum(-1)
    ok = Is >= 0
    return float(np.max(np.abs(Ds[ok] - exact[ok]) / np.maximum(exact[ok], 1e-12)))


def make_gist(cfg, torch):
    """GIST-like rows on the GPU: |N(0, 0.05^2)| features plus a per-cluster offset U[0, 0.1] of one of `clusters`
    components (torch's CUDA generator, seed 0 for the base and 1 for the queries), fp32 on the host."""
    d, C, n, nq = cfg["d"], cfg["clusters"], cfg["n"], cfg["nq"]
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    offs = 0.1 * torch.rand((C, d), generator=g, device="cuda")
    X = np.empty((n, d), np.float32)
    step = 1 << 17
    for r0 in range(0, n, step):
        m = min(step, n - r0)
        x = offs[torch.randint(0, C, (m,), generator=g, device="cuda")]
        X[r0 : r0 + m] = (x + (0.05 * torch.randn((m, d), generator=g, device="cuda")).abs()).cpu().numpy()
    gq = torch.Generator(device="cuda")
    gq.manual_seed(1)
    q = offs[torch.randint(0, C, (nq,), generator=gq, device="cuda")]
    Q = (q + (0.05 * torch.randn((nq, d), generator=gq, device="cuda")).abs()).cpu().numpy()
    return X, Q


def ground_truth(X, Q, k, torch):
    """Exact k nearest neighbors on the GPU (fp32; integer-valued data makes every distance exact)."""
    top = TopK(torch.from_numpy(Q).cuda(), k, torch)
    step = 1 << 17
    for r0 in range(0, len(X), step):
        top.add(torch.from_numpy(X[r0 : r0 + step]).cuda(), r0)
    return top.i.cpu().numpy()


class ProfilerRegion:
    """roctxProfilerResume/Pause around the measured search, so that `rocprofv3 --selected-regions` traces
    the search kernels only (not the index build); does nothing when the roctx library is absent."""

    def __init__(self):
        import ctypes

        self.lib = None
        rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
        for name in (os.path.join(rocm, "lib", "librocprofiler-sdk-roctx.so.1"), "librocprofiler-sdk-roctx.so.1"):
            try:
                self.lib = ctypes.CDLL(name)
                break
            except OSError:
                continue
        log(f"profiler region markers: {'roctx' if self.lib is not None else 'none (roctx library not found)'}")
        if self.lib is not None:  # roctxProfilerResume / Pause(roctx_thread_id_t tid), tid 0 = every thread
            for fn in (self.lib.roctxProfilerResume, self.lib.roctxProfilerPause):
                fn.argtypes = [ctypes.c_uint64]
                fn.restype = ctypes.c_int

    def __enter__(self):
        if self.lib is not None:
            self.lib.roctxProfilerResume(0)

    def __exit__(self, *exc):
        if self.lib is not None:
            self.lib.roctxProfilerPause(0)


def recall(I, gt, k=10):
    I, gt = np.asarray(I)[:, :k], np.asarray(gt)[:, :k]
    hits = sum(len(set(a) & set(b)) for a, b in zip(I.tolist(), gt.tolist()))
    return hits / (k * len(I))


def time_search(index, Qd, k, params, steps, warmup, torch):
    for _ in range(warmup):
        index.search(Qd, k=k, **params)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        index.search(Qd, k=k, **params)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def stage_bytes(name, wave, cnt, m, C, S, D, KO, table_len, starts, w, L, FR=0, k=10):
    """Algorithmic bytes of one launch: every distinct row read once at its natural size (no cache-line inflation)."""
    if name == "sketch_keep":
        return cnt["distinct1"] * 8 + m * 24 * KO
    if name == "sketch_keep_wave":
        return cnt["distinct2"][wave] * 8 + m * 24 * KO
    if name == "final_rerank":  # FR rows per query (from host memory when the vectors are there)
        return m * (FR * 2 * D + 12 * KO + 4 * D + 12 * k)
    if name == "gather_lists":
        return m * C * 8 + cnt["entries1"] * 4 + cnt["distinct1"] * (S + 8) + m * (S * 4 + 4)
    if name == "gather_rows":  # the sketch rows of candidates no earlier row scored; 8 bytes an earlier-row entry read
        known = cnt.get("known2", [0] * 16)[wave]
        old = cnt.get("oldread2", [0] * 16)[wave]
        return (m * starts * 8 + cnt["starts2"][wave] * table_len * 4 + (cnt["distinct2"][wave] - known) * S
                + cnt["distinct2"][wave] * 8 + old * 8 + m * (S * 4 + 4))
    if name == "rerank_keep":
        return cnt["distinct1"] * 8 + cnt["reranked1"] * 2 * D + m * (12 * KO + 4 * D + 4)
    if name == "rerank_keep_wave":  # the selected candidates' rows, less those an earlier round reranked
        skipped = cnt.get("skipped2", [0] * 16)[wave]
        return (cnt["distinct2"][wave] * 8 + (cnt["reranked2"][wave] - skipped) * 2 * D
                + m * (24 * KO + 4 * D + 4))
    if name == "probe":  # Y rows and segments out; an offsets pair and a key per level tried (finest first)
        tried = sum((j + 1) * h for j, h in enumerate(cnt["hit_level"])) + L * (m * C - cnt["seg_hits"])
        return m * C * (2 * w + 8) + tried * (8 + 8)
    if name == "project":
        return m * D * 2 + C * w * D * 2 + m * C * w * 2
    return None


def measured_traffic(config, params, stage, n, algorithmic):
    """HBM bytes per launch of a stage from the committed rocprof counter summary of this workload
    (profiles/traffic_<config>.json: FETCH_SIZE and WRITE_SIZE per dispatch, scaled by what the same counters
    read for a 1 GiB device copy).  Measured with the same search parameters: that figure; with others: the
    measured bytes per algorithmic byte of the stage times this run's algorithmic bytes (labelled so)."""
    path = os.path.join(ROOT, "profiles", f"traffic_{config}.json")
    if not os.path.isfile(path):
        return None, None
    with open(path) as f:
        t = json.load(f)
    k = t.get("kernels", {}).get(stage)
    if t.get("n") != n or k is None:
        return None, None
    keys = ("read", "starts", "waves", "rerank", "wave_rerank")
    if all(t.get("params", {}).get(x) == params.get(x) for x in keys):
        return int(k["hbm_bytes_per_launch"]), "rocprof FETCH_SIZE + WRITE_SIZE, same parameters"
    if k.get("algorithmic_bytes_per_launch"):
        ratio = k["hbm_bytes_per_launch"] / k["algorithmic_bytes_per_launch"]
        return int(ratio * algorithmic), f"rocprof bytes per algorithmic byte ({ratio:.3f}) measured at {t['params']}"
    return None, None


def cpu_passes(n, pool, seconds, target):
    """Searches of the CPU baseline's sample: one, or when the sample is the whole batch (n == pool) and one pass
    took less than half the target time, as many as fill about `target` seconds (at least two)."""
    if n < pool or seconds >= 0.5 * target:
        return 1
    return max(2, int(round(target / max(seconds, 1e-3))))


def host_path(X, Q, k, index, params, threads, log=lambda *a: None):
    """configs[0]'s CPU path, build and search both on the host: the oracle's builder writes an index of X (member
    lists: the CPU builder has no k-means lists; every other parameter as `index`, the workload's), the oracle
    searches all of Q with `params`, and I and D are checked against fp64 brute force over the fp16 rows."""
    import shutil
    import tempfile

    from oracle import oracle as O

    kw = dict(copies=200, list_len=64, table_len=64, log_buckets=20, reverse_edges=True, seed=0)
    kw.update({key: v for key, v in index.items() if key in kw or key in ("min_cell", "sketch_width", "blocks")})
    kw.update(member_lists=True, exact_lists=False)
    tmp = tempfile.mkdtemp(prefix="octex_host_")
    try:
        t0 = time.time()
        O.build(X, tmp, threads=threads, **kw)
        build_s = time.time() - t0
        log(f"host build: {build_s:.1f} s on {threads} threads")
        oix = O.Index(tmp)
        t0 = time.time()
        D, I = O.search(oix, Q, k=k, threads=threads, **params)
        search_s = time.time() - t0
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    x16 = np.asarray(X, np.float16).astype(np.float32)
    _, gt = O.bruteforce(x16, Q, k, threads=threads)
    return dict(build_seconds=round(build_s, 1), search_seconds=round(search_s, 3),
                value=round(len(Q) / search_s, 1), unit="queries/s", threads=threads, index=kw, search=params,
                recall=round(recall(I, gt, k), 4), distance_max_rel_err=distance_error(X, Q, D, I),
                truth="fp64 brute force over the fp16 rows")


def host_cpu():
    """The host's CPU model, its logical CPU count, the CPUs this process may run on, and the threads the CPU
    baseline uses: every CPU it may run on, at most 16 (the host share of one GPU on the GPU boxes here, whatever
    the machine's count)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    nproc = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = nproc
    threads = max(1, min(16, affinity))
    return dict(model=model, nproc=nproc, affinity=affinity, threads=threads,
                rule="min(16, CPUs of the process's affinity mask): 16 host CPUs per GPU on these boxes")


# (row bytes, pitch) of the gathers' rows at deep100m: 64- and 96-byte sketch rows (a 128-byte pitch for 96), a
# 128-byte line, 192-byte fp16 vectors of d = 96, 256-byte neighbor-table rows of 64 entries
CEILING_ROWS = [(64, 64), (96, 128), (128, 128), (192, 192), (256, 256)]


def row_ceiling(args):
    """Random-row read rate of the GPU (octexMeasureRowReads): 100M rows of each (row bytes, pitch) of
    CEILING_ROWS (the footprint of the deep100m array of that row: 6.4-25.6 GB), 1, 2, 4 or 8 rows in flight per
    lane group, timed with HIP events on the launch stream.  Prints one JSON line."""
    import ctypes as ct

    import torch

    from octex_amd import _lib

    torch.cuda.init()
    rows, n, blocks, reps = 100_000_000, 1 << 26, 8192, 5
    s = torch.cuda.current_stream()
    out = torch.empty(blocks * 256, dtype=torch.int32, device="cuda")
    results = []
    for row_bytes, pitch in CEILING_ROWS:
        buf = torch.empty(rows * pitch, dtype=torch.uint8, device="cuda")
        buf.fill_(1)
        for R in (1, 2, 4, 8):
            def launch(seed):
                _lib.call("octexMeasureRowReads", ct.c_void_p(buf.data_ptr()), ct.c_int64(rows), ct.c_int32(pitch),
                          ct.c_int32(row_bytes), ct.c_int64(n), ct.c_int32(R), ct.c_int32(blocks),
                          ct.c_uint64(seed), ct.c_void_p(out.data_ptr()), ct.c_void_p(s.cuda_stream))
            launch(0)  # warm-up
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for r in range(reps):
                launch(r + 1)
            e1.record(s)
            e1.synchronize()
            ms = e0.elapsed_time(e1) / reps
            results.append(dict(row_bytes=row_bytes, pitch=pitch, in_flight=R, footprint_gb=rows * pitch / 1e9,
                                ms=round(ms, 4), g_rows_s=round(n / ms / 1e6, 2),
                                gbs_rows=round(n * row_bytes / ms / 1e6, 1)))
            log(f"rows of {row_bytes} B at pitch {pitch}, {R} in flight per group: {ms:.3f} ms for {n:,} rows, "
                f"{n / ms / 1e6:.2f} G rows/s, {n * row_bytes / ms / 1e6:,.0f} GB/s of row bytes")
        del buf
        torch.cuda.empty_cache()
    best = {}
    for r in results:
        key = (r["row_bytes"], r["pitch"])
        if key not in best or r["g_rows_s"] > best[key]["g_rows_s"]:
            best[key] = r
    print(json.dumps(dict(mode="row_ceiling", unit="G rows/s", rows=rows, reads_per_launch=n, blocks=blocks,
                          threads=256, best=list(best.values()), results=results)))


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="deep100m", choices=sorted(CONFIGS))
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="target CPU time of the CPU-baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--host-path", action="store_true",
                    help="also build the index with the CPU oracle and search it on the host (cpu_baseline.host_path; "
                         "the default of --config cpu100k, configs[0]'s CPU path)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also copy 1 GiB device to device inside the profiled region (the known-size kernel that "
                         "scales rocprof's FETCH_SIZE / WRITE_SIZE counters to bytes)")
    ap.add_argument("--params", default=None, help="JSON search parameters (skips the sweep)")
    ap.add_argument("--sweep", action="store_true",
                    help="time the fastest sweep point at recall >= 0.99 instead of the workload's fixed point")
    ap.add_argument("--stream-build", action="store_true",
                    help="build streamed (OCTEX_BUILD_STREAM=1): vectors in pinned host memory from the start, each "
                         "copy's projection in chunks (the build a dataset beyond the GPU's memory takes)")
    ap.add_argument("--row-ceiling", action="store_true",
                    help="measure the random-row read ceiling of the GPU instead of a search (no index is built)")
    ap.add_argument("--save-index", default=None, help="also write the built index directory here")
    ap.add_argument("--load-index", default=None, help="load this index directory instead of building one")
    ap.add_argument("--n", type=int, default=None, help="override the number of base vectors (a scaled-down run)")
    ap.add_argument("--index-params", default=None,
                    help="JSON index parameters merged over the workload's (e.g. exact_lists)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build searches on one GPU; runs on several GPUs are not part of it", file=sys.stderr)
        sys.exit(2)
    n_rows = args.n or CONFIGS[args.config]["n"]
    if args.host_path and n_rows > HOST_PATH_MAX_ROWS:
        print(f"bench.py: --host-path builds with the CPU oracle's builder, for at most {HOST_PATH_MAX_ROWS:,} rows "
              f"(configs[0] has 100,000); this workload has {n_rows:,}", file=sys.stderr)
        sys.exit(2)

    if args.row_ceiling:
        row_ceiling(args)
        return

    # the builder reports its phases on stderr (a 100M build runs for minutes)
    os.environ.setdefault("OCTEX_VERBOSE", "1")
    if args.stream_build:
        os.environ["OCTEX_BUILD_STREAM"] = "1"
    import torch

    import octex_amd

    torch.backends.cuda.matmul.allow_tf32 = False  # exact fp32 ground truth

    cfg = CONFIGS[args.config]
    k = 10
    if args.n:
        cfg = dict(cfg, n=args.n)
    if args.index_params:
        cfg = dict(cfg, index=dict(cfg["index"], **json.loads(args.index_params)))
    t0 = time.time()
    if cfg["kind"] == "deep":
        X, Q, gt = make_deep(cfg, k, torch)
        torch.cuda.empty_cache()  # the index needs the memory the ground-truth blocks were cached in
        log(f"data {X.shape} queries {Q.shape} and ground truth in {time.time() - t0:.1f} s")
    else:
        X, Q = {"gist": lambda: make_gist(cfg, torch), "gauss": lambda: make_gauss(cfg)}.get(
            cfg["kind"], lambda: make_data(cfg))()
        log(f"data {X.shape} queries {Q.shape} in {time.time() - t0:.1f} s")
        t0 = time.time()
        gt = ground_truth(X, Q, k, torch)
        log(f"ground truth in {time.time() - t0:.1f} s")
    if args.load_index:
        t0 = time.time()
        index = octex_amd.load(args.load_index)
        build_s = None
        log(f"index loaded in {time.time() - t0:.1f} s: {index}")
    else:
        index, build_s = octex_amd.build_in_memory(X, path=args.save_index, **cfg["index"])
        log(f"index built in {build_s:.1f} s: {index}, {index.device_bytes[0] / 2**30:.1f} GiB")
    if cfg.get("host"):  # the load placements of the workload: arrays moved to pinned host memory
        index.place_on_host(**{a: True for a in cfg["host"]})
        log(f"{', '.join(cfg['host'])} moved to pinned host memory: {index.device_bytes[0] / 2**30:.1f} GiB in HBM")
    Qd = torch.from_numpy(Q).cuda()

    # the timed point: --params, else the workload's fixed point (the same in every run, so that the committed
    # profiles of the workload describe it) while its recall@10 is >= 0.99, else (or with --sweep) the fastest
    # point of the sweep at recall >= 0.99, by 3-batch timings
    sweeps = {"deep": SWEEP_DEEP, "gist": SWEEP_GIST}
    full = SWEEP_HOST if cfg.get("host") else sweeps.get(cfg["kind"], SWEEP)
    fixed = json.loads(args.params) if args.params else (None if args.sweep else cfg.get("point"))
    points = []

    def measure(p):
        p = dict(p, batch=cfg["batch"])
        D_, I_ = index.search(Qd, k=k, **p)
        r = recall(I_.cpu().numpy(), gt)
        s = time_search(index, Qd, k, p, steps=3, warmup=1, torch=torch)
        points.append(dict(params=p, recall=round(r, 5), qps=round(len(Q) / s)))
        log(f"{'point' if fixed else 'sweep'} {p}: recall {r:.4f}, {len(Q) / s:,.0f} QPS")
        return points[-1]

    chosen = measure(fixed) if fixed else None
    if chosen is not None and chosen["recall"] < 0.99 and not args.params:
        log("the fixed point misses recall 0.99: sweeping")
        chosen, fixed = None, None
    if chosen is None:
        for p in full:
            pt = measure(p)
            if pt["recall"] >= 0.99 and (chosen is None or pt["qps"] > chosen["qps"]):
                chosen = pt
        if chosen is None:
            chosen = max(points, key=lambda x: x["recall"])
    params = chosen["params"]
    point_source = "--params" if args.params else ("fixed point of the workload" if fixed else "sweep")

    # the timed region, then the roofline of the dominant kernel: HIP events around every launch of one batch
    # on the index's stream (both inside the profiler region)
    with ProfilerRegion():
        sec = time_search(index, Qd, k, params, steps=args.steps, warmup=args.warmup, torch=torch)
        stages, cnt = index.profile_batch(Qd, k=k, reps=5, **params)
        if args.copy_calibration:  # 1 GiB read + 1 GiB written by one elementwise copy kernel
            src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
            dst = torch.empty_like(src)
            torch.cuda.synchronize()
            dst.copy_(src)
            torch.cuda.synchronize()
            log("calibration copy: 1073741824 bytes read, 1073741824 bytes written")
            del src, dst
    qps = len(Q) / sec
    D_, I_ = index.search(Qd, k=k, **params)
    rec = recall(I_.cpu().numpy(), gt)
    derr = distance_error(X, Q, D_.cpu().numpy(), I_.cpu().numpy())
    log(f"timed: {sec * 1e3:.3f} ms per batch of {len(Q)}, {qps:,.0f} QPS, recall {rec:.4f}")
    info = index.plan_info()
    meta = index.array("meta", np.int64)
    C, D, w, S = index.copies, X.shape[1], 8 * int(meta[3]), int(meta[7])
    totals, per_launch, waves_seen = {}, [], {}
    for name, ms in stages:
        wv = waves_seen.get(name, 0)
        waves_seen[name] = wv + 1
        b = stage_bytes(name, wv, cnt, len(Q), C, S, D, info["KO"], int(meta[8]), params["starts"], w, int(meta[4]),
                        FR=info["final_rerank"], k=k)
        per_launch.append(dict(stage=name, wave=wv, ms=round(ms, 4), bytes=b,
                               gbs=round(b / (ms * 1e-3) / 1e9, 1) if b else None))
        totals[name] = totals.get(name, 0.0) + ms
    dominant = max(totals, key=totals.get)
    dl = [x for x in per_launch if x["stage"] == dominant]
    avg_ms = sum(x["ms"] for x in dl) / len(dl)
    avg_bytes = sum(x["bytes"] for x in dl) / len(dl)
    achieved = avg_bytes / (avg_ms * 1e-3) / 1e9
    traffic, traffic_source = measured_traffic(args.config, params, dominant, X.shape[0], avg_bytes)
    log(f"probe hits by level {cnt['hit_level'][:int(meta[4])]}, misses {len(Q) * C - cnt['seg_hits']}")
    nw = params.get("waves", 0)
    if nw:
        log("waves: distinct " + str(cnt["distinct2"][:nw]) + ", scored in earlier rows " + str(cnt["known2"][:nw])
            + ", earlier-row entries read " + str(cnt["oldread2"][:nw]) + ", selected " + str(cnt["reranked2"][:nw])
            + ", of them reranked by an earlier round " + str(cnt["skipped2"][:nw]))
    log("stages: " + ", ".join(f"{x['stage']}[{x['wave']}] {x['ms']:.3f} ms {x['gbs']} GB/s" for x in per_launch))

    # CPU baseline: the oracle (C++ restatement of the search) on the same index, a bounded query sample
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle as O

        host = host_cpu()
        threads = host["threads"]
        t0 = time.time()
        big = index.device_bytes[0] > (48 << 30)
        # a large index keeps its lists on the GPU: the host copy holds the list rows the sample's probes
        # reach (all the first round reads) and every other array in full
        pool = len(Q)
        oix = O.Index(index, queries=Q[:pool], read=params["read"]) if big else O.Index(index)
        log(f"oracle index copied to the host in {time.time() - t0:.1f} s")
        n_s = 32
        t0 = time.time()
        O.search(oix, Q[:n_s], k=k, threads=threads, **params)
        first = time.time() - t0
        n_s = int(min(pool, max(n_s, n_s * args.cpu_seconds / max(first, 1e-3))))
        t0 = time.time()
        Dc, Ic = O.search(oix, Q[:n_s], k=k, threads=threads, **params)
        cs = time.time() - t0
        passes = cpu_passes(n_s, pool, cs, args.cpu_seconds)
        if passes > 1:
            t0 = time.time()
            for _ in range(passes):
                O.search(oix, Q[:n_s], k=k, threads=threads, **params)
            cs = time.time() - t0
        cpu = dict(value=round(passes * n_s / cs, 1), unit="queries/s", cores=threads, kind="port",
                   sample=(f"first {n_s} of the {len(Q)} queries" if passes == 1 else
                           f"the {len(Q)} queries searched {passes} times")
                          + f", same index and parameters, {cs:.1f} s"
                          + (" (list rows copied for these queries only)" if big else ""),
                   recall=round(recall(Ic, gt[:n_s]), 4), nproc=host["nproc"], affinity=host["affinity"],
                   cpu_model=host["model"], threads_rule=host["rule"])
        if cfg.get("host_path") or args.host_path:  # configs[0]: build and search both on the host
            cpu["host_path"] = host_path(X, Q, k, cfg["index"], params, threads, log=log)
        log(f"cpu baseline: {cpu}")

    out = {
        "metric": "queries/sec at recall@10>=0.99, k=10, 1 MI355X; achieved HBM GB/s",
        "value": round(qps, 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 rerank, int8 sketch, fp32 accumulate",
        "data": f"synthetic ({cfg['desc']})",
        "config": {
            "workload": f"{args.config}: {X.shape[0]} x {X.shape[1]} {cfg['kind']}-like mixture, {len(Q)} queries, "
                        f"k=10, batch {cfg['batch']}",
            "index": cfg["index"],
            "host_arrays": list(cfg.get("host", ())),
            "search": params,
            "search_point": point_source,
            "recall@10": round(rec, 5),
            "distance_max_rel_err": derr,
            "recall_target_met": rec >= 0.99,
            "build_seconds": round(build_s, 1) if build_s is not None else None,
            "build_streamed": bool(args.stream_build),
            "index_gib": round(index.device_bytes[0] / 2**30, 2),
            "sweep": points,
            "stages": per_launch,
            # per wave: distinct candidates, those whose scores came from earlier rows (no sketch row read), the
            # earlier rows' entries read, the candidates selected for the exact rerank, and of those the ones an earlier
            # round reranked (their rows not read again)
            "wave_reuse": {key: cnt[key][: params.get("waves", 0)]
                           for key in ("distinct2", "known2", "oldread2", "reranked2", "skipped2")},
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dominant,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            # the measured HBM bytes as a rate over the same launches, against the same peak
            "traffic_gbs": round(traffic / (avg_ms * 1e-3) / 1e9, 1) if traffic else None,
            "traffic_frac": round(traffic / (avg_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4) if traffic else None,
            "avg_launch_ms": round(avg_ms, 4),
            "algorithmic_bytes_per_launch": int(avg_bytes),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
