"""Every BASELINE.json workload on the GPU against the CPU oracle, with each workload's own data generator (bench.py)
and index shape, at sizes the oracle searches in seconds: configs[0] at full size (100k x 128, 1,000 queries, the
reference's default index and search parameters but log_buckets 16), configs[1] scaled to 50k integer-valued
SIFT-like rows (exact table, sketch 128), configs[2] scaled to 20k x 960 (D = 960 exact distances, sketch 128),
configs[3] scaled to 200k normalized rows (sketch 96 at a 128-byte pitch, searched table), and configs[4]'s mode
(vectors in pinned host memory, sketch-rank search, starts 512 over a table of 32, final rerank 32).

Parity: given the GPU's own projections Y and sketch queries qs, the oracle returns the same ids (up to distance
ties) and bit-identical distances; recall@10 against exact search is then within 0.002 of the oracle's (it is the
same), and meets the workload's floor."""

import numpy as np
import pytest
from conftest import recall
from test_gpu_search import assert_same_results, oracle_given_gpu_projections

import bench
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def octex():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import octex_amd

    return octex_amd


def exact_ids(X, Q, k=10):
    """Exact neighbors over the stored fp16 rows (fp32 on the GPU; ties by id as torch.topk returns them)."""
    Xh = torch.from_numpy(np.asarray(X, np.float16).astype(np.float32)).cuda()
    top = bench.TopK(torch.from_numpy(Q).cuda(), k, torch)
    for r0 in range(0, len(Xh), 1 << 16):
        top.add(Xh[r0 : r0 + (1 << 16)], r0)
    return top.i.cpu().numpy()


def run_config(octex, X, Q, index_params, search, floor, host=(), oracle_rows=None, k=10):
    print(f"config: {X.shape[0]} x {X.shape[1]}, {len(Q)} queries, index {index_params}, search {search}",
          flush=True)
    index, _ = octex.build_in_memory(X, **index_params)
    if host:
        index.place_on_host(**{a: True for a in host})
    gt = exact_ids(X, Q, k)
    D, I = index.search(torch.from_numpy(Q).cuda(), k=k, batch=len(Q), **search)
    D, I = D.cpu().numpy(), I.cpu().numpy()
    oix = O.Index(index, queries=Q if oracle_rows else None, read=search["read"])
    Do, Io, _, _, _ = oracle_given_gpu_projections(index, oix, Q, k, batch=len(Q), **search)
    assert_same_results(D, I, Do, Io)
    r, ro = recall(I, gt), recall(Io, gt)
    print(f"recall@10 GPU {r:.4f}, oracle {ro:.4f}", flush=True)
    assert abs(r - ro) <= 0.002 and r >= floor
    return index


def test_config0_cpu100k_reference_defaults(octex):
    cfg = bench.CONFIGS["cpu100k"]
    X, Q = bench.make_gauss(cfg)
    index = run_config(octex, X, Q, cfg["index"], dict(read=32, starts=128, waves=2, rerank=128, wave_rerank=128),
                       floor=0.99, oracle_rows=True)
    assert index.copies == 200 and index.size == 100_000


def test_config1_sift_like_exact_table(octex):
    cfg = dict(bench.CONFIGS["sift1m"], n=50_000, nq=1_000)
    X, Q = bench.make_data(cfg)
    ip = dict(cfg["index"], copies=64, sketch_width=128)
    for search in (dict(read=4, starts=16, waves=1, rerank=16, wave_rerank=16),
                   dict(read=16, starts=64, waves=2, rerank=64, wave_rerank=64)):
        run_config(octex, X, Q, ip, search, floor=0.95, oracle_rows=True)


def test_config2_gist_like_d960(octex):
    cfg = dict(bench.CONFIGS["gist1m"], n=20_000, nq=200, clusters=200)
    X, Q = bench.make_gist(cfg, torch)
    ip = dict(cfg["index"], copies=32)
    run_config(octex, X, Q, ip, dict(read=32, starts=64, waves=2, rerank=256, wave_rerank=256), floor=0.9)


def test_config3_deep_like_searched_table(octex):
    cfg = dict(bench.CONFIGS["deep100m"], n=200_000, nq=1_000, clusters=2_000)
    X, Q, _ = bench.make_deep(cfg, 10, torch)
    ip = dict(cfg["index"], copies=48, sketch_width=96, exact_table_max=0)
    index = run_config(octex, X, Q, ip, dict(read=16, starts=64, waves=2, rerank=128, wave_rerank=128), floor=0.97,
                       oracle_rows=True)
    meta = index.array("meta", np.int64)
    assert int(meta[7]) == 96 and int(meta[11]) == 128  # sketch width 96 at a 128-byte pitch


def test_config4_host_vectors_sketch_rank(octex):
    cfg = dict(bench.CONFIGS["deep100m-host"], n=200_000, nq=500, clusters=2_000)
    X, Q, _ = bench.make_deep(cfg, 10, torch)
    ip = dict(cfg["index"], copies=48, sketch_width=96, exact_table_max=0)
    search = dict(read=16, starts=512, waves=3, rerank=128, wave_rerank=128, sketch_rank=True, final_rerank=32)
    index = run_config(octex, X, Q, ip, search, floor=0.9, host=("vectors",), oracle_rows=True)
    assert index.plan_info()["W2"] == 1 << 15  # starts 512 x table 32: the largest hash set
