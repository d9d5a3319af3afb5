"""The reference's ablation switches (search_params::balanced_gather, fused_merge, use_graph) on the GPU: every
combination returns the neighbors and distances of the optimized search (the reference's test_search.cu:509-597,
whose bar is at most 0.1 % differing ids; here the selections break ties by (distance, id) in every path, so the
results are identical), in both rank modes, over several batches with a partial last one; and the switches do
change the kernels a batch launches."""

import itertools

import numpy as np
import pytest
from test_gpu_search import assert_same_results, oracle_given_gpu_projections

from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ablation_index(tmp_path_factory):
    """The reference test's data and index: 20,000 x 48 rows, N(0, 1) plus i % 37 on the first 4 coordinates,
    600 queries near data points; copies 8, blocks 2, pca_dims 32, lists of 16, log_buckets 12, sketch 32,
    table 16."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import octex_amd

    g = np.random.default_rng(11)
    n, d, nq = 20_000, 48, 600
    x = g.standard_normal((n, d)).astype(np.float32)
    x[:, :4] += (np.arange(n) % 37)[:, None].astype(np.float32)
    q = x[(np.arange(nq) * 31) % n] + 0.3 * g.standard_normal((nq, d)).astype(np.float32)
    path = str(tmp_path_factory.mktemp("octex") / "ablation")
    index = octex_amd.build(x, path, copies=8, blocks=2, pca_dims=32, list_len=16, log_buckets=12, sketch_width=32,
                            table_len=16)
    return index, path, q.astype(np.float32)


BASE = dict(read=8, starts=32, waves=2, rerank=64, wave_rerank=64, batch=256)


@pytest.mark.parametrize("sketch_rank", [False, True])
def test_every_switch_combination_gives_the_same_results(ablation_index, sketch_rank):
    index, _, q = ablation_index
    base = dict(BASE, sketch_rank=sketch_rank)
    D0, I0 = index.search(q, k=10, **base)
    for balanced, fused, graph in itertools.product((True, False), repeat=3):
        D, I = index.search(q, k=10, balanced_gather=balanced, fused_merge=fused, use_graph=graph, **base)
        print(f"sketch_rank={sketch_rank} balanced_gather={balanced} fused_merge={fused} use_graph={graph}",
              flush=True)
        assert np.array_equal(I, I0) and np.array_equal(D, D0), (balanced, fused, graph)


@pytest.mark.parametrize("fused,balanced", [(False, False), (False, True), (True, False)])
def test_ablations_match_oracle(ablation_index, fused, balanced):
    """The unfused and unbalanced paths against the CPU oracle given the GPU's projections (one batch)."""
    index, path, q = ablation_index
    oix = O.Index(path)
    p = dict(BASE, batch=600, waves=3, fused_merge=fused, balanced_gather=balanced)
    D, I = index.search(q, k=10, **p)
    Do, Io, _, _, _ = oracle_given_gpu_projections(index, oix, q, 10, **{k: v for k, v in p.items()
                                                                        if k not in ("fused_merge", "balanced_gather")})
    assert_same_results(D, I, Do, Io)


def test_switches_change_the_kernels(ablation_index):
    """The profiled stages name the kernels that ran: the whole-segment gathers and the unfused merges and picks."""
    index, _, q = ablation_index
    qd = torch.from_numpy(q[:256]).cuda()
    fused, _ = index.profile_batch(qd, k=10, reps=1, **BASE)
    unfused, _ = index.profile_batch(qd, k=10, reps=1, fused_merge=False, balanced_gather=False, **BASE)
    names_f, names_u = [n for n, _ in fused], [n for n, _ in unfused]
    assert names_f.count("gather_rows") == 2 and names_f.count("rerank_keep_wave") == 2
    assert names_u == [n + ("_whole" if n.startswith("gather") else "_unfused" if ("keep" in n or "pick" in n) else "")
                       for n in names_f]
