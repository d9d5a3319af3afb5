"""Every HIP kernel of the search path against the CPU oracle on the same inputs, through the stage entry points
of liboctex_amd.so (include/octex_amd/octex_amd.h).  Bit-exact: E8 points and hashes, probe segments, candidate
sets, sketch scores, selections, kept lists, start points.  The fp16 projection: within 1 fp16 ulp of the fp64
value (its MFMA accumulation order is not the oracle's); the fp32 sketch query: 1e-5 relative."""

import ctypes as ct

import numpy as np
import pytest
from conftest import clustered
from test_oracle import check_e8, check_probe, e8_inputs, probe_construction

from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def L():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from octex_amd import _lib

    return _lib


def dev(a):
    return torch.from_numpy(np.array(a, copy=True)).cuda()


def P(t):
    """The device address of a tensor; the caller keeps the tensor alive (a temporary would be freed, and its
    block reused by the next allocation, before the kernel reads it)."""
    return ct.c_void_p(t.data_ptr())


def host(t):
    return t.cpu().numpy()


def i32(v):
    return ct.c_int32(int(v))


def i64(v):
    return ct.c_int64(int(v))


# ---------------------------------------------------------------- E8 and projections


@pytest.mark.parametrize("b", [4, 1, 3, 8])
def test_e8_kernel_matches_oracle(L, b):
    x = e8_inputs(n=20000 if b == 4 else 4000, b=b, seed=b)
    inv_f = np.float32(1.0 / 2.5)
    dx = dev(x)
    dp = torch.empty_like(dx)
    dh = torch.empty(x.shape[0], dtype=torch.int64, device="cuda")
    L.call("octexStageE8", P(dx), i64(x.shape[0]), i32(b), ct.c_float(inv_f), P(dp), P(dh), None)
    p, h = O.e8_batch(x, b, float(inv_f))
    assert np.array_equal(host(dp), p)
    assert np.array_equal(host(dh), h)
    check_e8(x, host(dp), host(dh), b, inv_f)


def test_e8_golden(L):
    import os

    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "e8.npz"))
    dx = dev(g["y"])
    dp = torch.empty_like(dx)
    dh = torch.empty(g["y"].shape[0], dtype=torch.int64, device="cuda")
    L.call("octexStageE8", P(dx), i64(g["y"].shape[0]), i32(g["b"]), ct.c_float(g["inv_f"]), P(dp), P(dh), None)
    assert np.array_equal(host(dp), g["p"]) and np.array_equal(host(dh), g["h"])


def test_center_kernel(L):
    g = np.random.default_rng(0)
    q = g.standard_normal((77, 96)).astype(np.float32)
    mu = g.standard_normal(96).astype(np.float32)
    dq, dmu = dev(q), dev(mu)
    qc = torch.empty_like(dq)
    qh = torch.empty(q.shape, dtype=torch.int16, device="cuda")
    L.call("octexStageCenter", P(dq), P(dmu), i64(77), i32(96), P(qc), P(qh), None)
    rc, rh = O.center(q, mu)
    assert np.array_equal(host(qc), rc) and np.array_equal(host(qh).view(np.uint16), rh)


def ulp_diff(a_bits, b_bits):
    """Distance in fp16 units in the last place between two arrays of fp16 bit patterns."""
    def ordered(h):
        h = h.astype(np.int32)
        return np.where(h & 0x8000, -(h & 0x7FFF), h & 0x7FFF)

    return np.abs(ordered(a_bits) - ordered(b_bits))


@pytest.mark.parametrize("m,K,N", [(300, 96, 6400 // 8), (1000, 128, 256), (65, 100, 72), (17, 34, 40), (130, 960, 96)])
def test_projection_within_one_ulp(L, m, K, N):
    g = np.random.default_rng(m + K + N)
    qh = (g.standard_normal((m, K)) * 0.5).astype(np.float16)
    ucat = (g.standard_normal((K, N)) / np.sqrt(K)).astype(np.float16)
    shift = g.uniform(0, 2, N).astype(np.float16)
    dY = torch.empty((m, N), dtype=torch.int16, device="cuda")
    ucatT = np.ascontiguousarray(ucat.T)
    dqh, du, ds = dev(qh.view(np.int16)), dev(ucatT.view(np.int16)), dev(shift.view(np.int16))
    L.call("octexStageProject", P(dqh), P(du), P(ds), i32(m), i32(K), i32(N), P(dY), None)
    got = host(dY).view(np.uint16)
    check_projection(got, qh.view(np.uint16), ucat.view(np.uint16), shift.view(np.uint16))


def check_projection(got, qh, ucat, shift):
    """The fp16 projection against its fp64 value: off by at most one fp16 ulp plus the fp32 accumulation bound
    K 2^-23 sum |qh ucat| (which matters only under cancellation), and by no ulp at all for >= 98% of entries."""
    Y, Yd = O.project(qh, ucat, shift)
    u = ulp_diff(got, Y)
    g = O.h2f(got).astype(np.float64)
    K = qh.shape[1]
    mag = np.abs(O.h2f(qh).astype(np.float64)) @ np.abs(O.h2f(ucat).astype(np.float64))
    ulp16 = np.maximum(np.spacing(np.abs(Yd).astype(np.float16)).astype(np.float64), 2.0**-24)
    bound = ulp16 + K * 2.0**-23 * mag
    assert (np.abs(g - Yd) <= bound).all(), f"max error / bound {(np.abs(g - Yd) / bound).max()}"
    assert (u > 0).mean() < 0.02, f"ulp mismatch rate {(u > 0).mean()}"
    return u


def test_sketch_query_kernel(L):
    g = np.random.default_rng(1)
    qc = g.standard_normal((500, 96)).astype(np.float32)
    basis = g.standard_normal((96, 64)).astype(np.float32)
    qs = torch.empty((500, 64), dtype=torch.float32, device="cuda")
    dqc, db = dev(qc), dev(basis)
    L.call("octexStageSketchQuery", P(dqc), P(db), i32(500), i32(96), i32(64), P(qs), None)
    ref = qc.astype(np.float64) @ basis.astype(np.float64)
    assert np.allclose(host(qs), ref, rtol=1e-5, atol=1e-4)


# ---------------------------------------------------------------- probe, gather


@pytest.fixture(scope="module")
def ix(small_index):
    return O.Index(small_index["path"])


@pytest.fixture(scope="module")
def dix(L, ix):
    """The oracle's index arrays on the device (the loader's layout)."""
    return dict(
        inv_f=dev(ix.inv_f), offsets=dev(ix.offsets), keys=dev(ix.keys), base=dev(ix.base), lists=dev(ix.lists),
        sketch=dev(ix.sketch), scale=dev(ix.scale), vectors=dev(ix.vectors.view(np.int16)), table=dev(ix.table),
    )


def queries_Y(ix, X, extra_random=64, seed=0):
    """Projections of database rows (cells exist) and of random points (mostly misses)."""
    qc, qh = O.center(X, ix.mean)
    Y, _ = O.project(qh, ix.ucat, ix.shift)
    g = np.random.default_rng(seed)
    R = O.f2h(g.standard_normal((extra_random, Y.shape[1])).astype(np.float32) * 3)
    return np.concatenate([Y, R])


PROBES = ["octexStageProbe", "octexStageProbeLines"]  # buckets read from the offsets, or from bucket lines


def run_probe(L, ix, dix, Y, lr, stage="octexStageProbe"):
    m, C = Y.shape[0], ix.copies
    seg = torch.empty((m, C, 2), dtype=torch.int32, device="cuda")
    dY = dev(Y.view(np.int16))
    L.call(stage, P(dY), i32(m), i32(C), i32(len(ix.spacings)), i32(ix.blocks),
           P(dix["inv_f"]), P(dix["offsets"]), i64(ix.offsets.shape[2]), P(dix["keys"]), i64(ix.keys.shape[2]),
           P(dix["base"]), i32(ix.list_len), i32(lr), i32(ix.log_buckets), P(seg), None)
    return seg


@pytest.mark.parametrize("case", [
    dict(),  # the reference's probe test shape (test_search.cu:86-170)
    dict(m=60, C=5, spacing=(0.5, 1.0, 2.0, 4.0, 8.0), logT=3, l=16, lr=9, seed=3, absent=(5, 6, 17)),
    dict(m=300, C=7, spacing=(1.0, 2.0, 4.0), b=2, logT=5, l=8, lr=8, seed=4, absent=tuple(range(0, 300, 13))),
])
@pytest.mark.parametrize("stage", PROBES)
def test_probe_construction_matches_reference(L, case, stage):
    """The probe over hand-built cell tables: exactly (row * l, lr) at the finest level holding each query's
    cell, (0, 0) when none does; the oracle gives the same segments."""
    arrays, Y, want = probe_construction(**case)
    pix = O.Index.from_arrays(**arrays)
    pdix = dict(inv_f=dev(pix.inv_f), offsets=dev(pix.offsets), keys=dev(pix.keys), base=dev(pix.base))
    lr = int(want[:, :, 1].max())
    seg = host(run_probe(L, pix, pdix, Y, lr, stage))
    check_probe(seg, want)
    check_probe(O.probe(pix, Y, read=lr), want)


@pytest.mark.parametrize("stage", PROBES)
def test_probe_matches_oracle(L, ix, dix, small_index, stage):
    Y = queries_Y(ix, small_index["X"][:200])
    for lr in (ix.list_len, 5):
        seg = run_probe(L, ix, dix, Y, lr, stage)
        ref = O.probe(ix, Y, read=lr)
        assert np.array_equal(host(seg), ref)
    assert (ref[:200, :, 1] > 0).mean() > 0.9 and (ref[200:, :, 1] == 0).mean() > 0.5


@pytest.mark.parametrize("blocks,spacings,log_buckets,min_cell", [
    (2, [1.5, 2.0, 2.5, 3.2, 4.0, 5.0, 6.5], 4, 3),  # 7 levels, 16 buckets: many keys per bucket
    (3, [2.5], 6, 1),                                # one level
    (1, [1.0, 1.4, 2.0, 2.8, 4.0, 5.6, 8.0, 11.0, 16.0, 22.0, 32.0], 8, 4),  # 11 levels: 5 groups per wavefront
])
@pytest.mark.parametrize("stage", PROBES)
def test_probe_level_and_bucket_shapes(L, tmp_path, blocks, spacings, log_buckets, min_cell, stage):
    X, _ = clustered(n=1500, m=10, d=32, clusters=8, seed=11)
    path = str(tmp_path / "probe")
    O.build(X, path, copies=6, blocks=blocks, pca_dims=32, spacings=spacings, list_len=8, table_len=0,
            log_buckets=log_buckets, min_cell=min_cell, member_lists=True, seed=4)
    pix = O.Index(path)
    pdix = dict(inv_f=dev(pix.inv_f), offsets=dev(pix.offsets), keys=dev(pix.keys), base=dev(pix.base))
    Y = queries_Y(pix, X[:300], extra_random=100)
    seg = run_probe(L, pix, pdix, Y, pix.list_len, stage)
    ref = O.probe(pix, Y, read=pix.list_len)
    assert np.array_equal(host(seg), ref)
    rows = ref[:, :, 0] // pix.list_len
    levels = (rows[..., None] >= pix.base.reshape(1, pix.copies, -1)).sum(-1) - 1
    hit = ref[:, :, 1] > 0
    assert hit.mean() > 0.3 and (len(spacings) == 1 or len(np.unique(levels[hit])) > 1)  # hits at several levels


def gather_gpu(L, ix, dix, seg, qs, rows, W=4096):
    m, nseg = seg.shape[0], seg.shape[1]
    cand = torch.full((m, W), -5, dtype=torch.int32, device="cuda")
    dist = torch.zeros((m, W), dtype=torch.float32, device="cuda")
    nout = torch.zeros(m, dtype=torch.int32, device="cuda")
    dqs = dev(qs)
    L.call("octexStageGather", i32(rows), P(seg), i32(nseg), i32(m), P(dix["lists"]), i64(ix.lists.shape[1]),
           P(dix["table"]), i32(ix.table_len), i64(ix.n), P(dix["sketch"]), P(dix["scale"]), P(dqs),
           i32(ix.sketch_width), i32(W), P(cand), P(dist), P(nout), None)
    return host(cand), host(dist), host(nout)


def check_gather(ix, seg, qs, cand, dist, nout, rows):
    for q in range(seg.shape[0]):
        rc, rd = O.gather(ix, seg[q], qs[q], rows=rows)
        n = nout[q]
        assert n == len(rc)
        order = np.argsort(cand[q, :n])
        assert np.array_equal(cand[q, :n][order], rc), f"query {q}: candidate sets differ"
        assert np.array_equal(dist[q, :n][order], rd), f"query {q}: sketch scores differ"


def test_gather_lists_matches_oracle(L, ix, dix, small_index):
    Y = queries_Y(ix, small_index["X"][:64], extra_random=8)
    seg = run_probe(L, ix, dix, Y, ix.list_len)
    qs = np.random.default_rng(2).standard_normal((Y.shape[0], ix.sketch_width)).astype(np.float32)
    cand, dist, nout = gather_gpu(L, ix, dix, seg, qs, rows=0)
    check_gather(ix, host(seg), qs, cand, dist, nout, rows=False)


def test_gather_rows_matches_oracle(L, ix, dix):
    g = np.random.default_rng(3)
    m, S = 48, 64
    seg2 = np.stack([g.integers(0, ix.n, (m, S)), np.full((m, S), ix.table_len)], -1).astype(np.int32)
    seg2[:, -7:] = 0  # unused start points
    seg2[0] = 0  # a query without starts
    qs = g.standard_normal((m, ix.sketch_width)).astype(np.float32)
    dseg2 = dev(seg2)
    cand, dist, nout = gather_gpu(L, ix, dix, dseg2, qs, rows=1)
    check_gather(ix, seg2, qs, cand, dist, nout, rows=True)
    assert nout[0] == 0


def gather_reuse_gpu(L, ix, dix, seg, qs, old, W=4096):
    """octexStageGatherReuse over table rows with the earlier rows `old` [(cand, dist, n, W)] (device tensors)."""
    m, nseg = seg.shape[0], seg.shape[1]
    cand = torch.full((m, W), -5, dtype=torch.int32, device="cuda")
    dist = torch.zeros((m, W), dtype=torch.float32, device="cuda")
    nout = torch.zeros(m, dtype=torch.int32, device="cuda")
    nk = torch.full((m,), -1, dtype=torch.int32, device="cuda")
    dqs, dseg = dev(qs), dev(seg)
    k = len(old)
    oc = (ct.c_void_p * max(k, 1))(*[o[0].data_ptr() for o in old])
    od = (ct.c_void_p * max(k, 1))(*[o[1].data_ptr() for o in old])
    on = (ct.c_void_p * max(k, 1))(*[o[2].data_ptr() for o in old])
    ow = (ct.c_int32 * max(k, 1))(*[o[3] for o in old])
    L.call("octexStageGatherReuse", P(dseg), i32(nseg), i32(m), P(dix["table"]), i32(ix.table_len), i64(ix.n),
           P(dix["sketch"]), P(dix["scale"]), P(dqs), i32(ix.sketch_width), i32(W), P(cand), P(dist), P(nout), i32(k),
           oc, od, on, ow, P(nk), None)
    return host(cand), host(dist), host(nout), host(nk)


def test_gather_takes_scores_from_earlier_rows(L, ix, dix):
    """A wave gather given two earlier rows (of another width, with repeated ids between them, one query's rows
    empty): the oracle's candidate set with bit-identical scores; the candidates found in an earlier row come last
    and number nknown; a query without starts has none."""
    g = np.random.default_rng(21)
    m, S = 40, 64

    def rows_of(starts, dead=0):
        seg = np.stack([starts, np.full(starts.shape, ix.table_len)], -1).astype(np.int32)
        if dead:
            seg[:, -dead:] = 0
        return seg

    qs = g.standard_normal((m, ix.sketch_width)).astype(np.float32)
    starts_a = g.integers(0, ix.n, (m, S))
    seg_a = rows_of(starts_a, dead=5)
    seg_a[2] = 0  # an earlier row without candidates
    ca, da, na = gather_gpu(L, ix, dix, dev(seg_a), qs, rows=1, W=2048)
    starts_b = np.where(g.random((m, S)) < 0.5, starts_a, g.integers(0, ix.n, (m, S)))
    cb, db, nb = gather_gpu(L, ix, dix, dev(rows_of(starts_b)), qs, rows=1, W=4096)
    starts_c = np.where(g.random((m, S)) < 0.5, starts_b, g.integers(0, ix.n, (m, S)))
    seg_c = rows_of(starts_c, dead=3)
    seg_c[1] = 0  # a query without starts
    old = [(dev(ca), dev(da), dev(na), 2048), (dev(cb), dev(db), dev(nb), 4096)]
    cand, dist, nout, nk = gather_reuse_gpu(L, ix, dix, seg_c, qs, old)
    check_gather(ix, seg_c, qs, cand, dist, nout, rows=True)
    for q in range(m):
        n = nout[q]
        seen = {int(v) for v in ca[q, : na[q]]} | {int(v) for v in cb[q, : nb[q]]}
        known = np.array([int(v) in seen for v in cand[q, :n]], bool)
        assert nk[q] == known.sum(), f"query {q}"
        assert not known[: n - nk[q]].any() and known[n - nk[q] :].all(), f"query {q}: the found candidates come last"
    assert nout[1] == 0 and nk[1] == 0
    assert nk.sum() > 0.3 * nout.sum()  # half the starts repeat: many candidates come from the earlier rows
    # no earlier rows: the plain gather's result
    cand0, dist0, nout0, nk0 = gather_reuse_gpu(L, ix, dix, seg_c, qs, [])
    check_gather(ix, seg_c, qs, cand0, dist0, nout0, rows=True)
    assert (nk0 == 0).all()


# ---------------------------------------------------------------- keep, pick, final


CACHED = 1024  # the selection's register-held keys on 128 threads (8 a thread): the first 1024 of a row


def key_bits(bits):
    return np.asarray(bits, np.uint32).view(np.float32)


def random_candidates(g, m, W, n_max, N, ties=True, kind=None):
    """Candidate rows of m queries: integer distances in [0, 40) (ties), uniform ones, or all equal; or rows whose keys
    past the first CACHED lie outside the range of the first CACHED (the selection's bins come from those): spread on
    both sides (tails), all equal below it (low_ties), or a last bin of thousands of keys at and above its top
    (last_bin: keys of bits K and K + 2^24 - 1 in the cache, K + 2^25 past it)."""
    kind = kind or ("ties" if ties else "uniform")
    cand = np.full((m, W), -9, np.int32)
    dist = np.zeros((m, W), np.float32)
    nin = g.integers(1, n_max, m).astype(np.int32)
    nin[0] = n_max
    nin[1] = 3
    for q in range(m):
        n = nin[q]
        cand[q, :n] = g.choice(N, n, replace=False)
        if kind == "ties":
            dist[q, :n] = g.integers(0, 40, n)
        elif kind == "uniform":
            dist[q, :n] = g.uniform(0, 100, n)
        elif kind == "tails":
            dist[q, :n] = np.where(np.arange(n) < CACHED, g.uniform(40, 60, n), g.uniform(0, 100, n))
        elif kind == "low_ties":
            dist[q, :n] = np.where(np.arange(n) < CACHED, g.uniform(40, 60, n), 5.0)
        elif kind == "last_bin":
            K = 0x41000000
            bits = np.where(np.arange(n) < 24, K, np.where(np.arange(n) < CACHED, K + 0xFFFFFF, K + 0x2000000))
            dist[q, :n] = key_bits(bits)
        else:
            dist[q, :n] = 7.25
    return cand, dist, nin


# (KO, R): the kept list and the reranked rows sort together on 128 threads a query, C keys a thread for the smallest C
# that holds KO + R (C = 1, 2, 4 and 8 below)
@pytest.mark.parametrize("KO,R", [(64, 16), (64, 48), (10, 20), (256, 256), (512, 512)])
@pytest.mark.parametrize("fresh", [True, False])
@pytest.mark.parametrize("W", [2048, 8192])
def test_rerank_keep_matches_oracle(L, ix, dix, small_index, fresh, KO, R, W):
    g = np.random.default_rng(4 + fresh)
    m = 40
    # more candidates than a workgroup holds in registers (8 keys a thread), so the selection also streams keys
    cand, dist, nin = random_candidates(g, m, W, 1500 if W == 2048 else 3000, ix.n)
    Q = small_index["Q"][:m]
    si = np.full((m, KO), -1, np.int64)
    sd = np.full((m, KO), np.inf, np.float32)
    if not fresh:
        for q in range(m):
            ids = g.choice(ix.n, min(50, KO), replace=False)
            ex = np.array([O.exact_dist(ix.vectors[i], Q[q]) for i in ids], np.float32)
            si[q], sd[q] = O.merge_keep(si[q], sd[q], ids.astype(np.int32), ex, True)
    dsi, dsd = dev(si), dev(sd)
    dc, dd, dn, dQ = dev(cand), dev(dist), dev(nin), dev(Q)
    L.call("octexStageRerankKeep", P(dc), P(dd), P(dn), i32(m), i32(W), P(dix["vectors"]), i32(ix.dim), P(dQ),
           i32(R), i32(KO), P(dsi), P(dsd), i32(fresh), None)
    for q in range(m):
        ri, rd = O.rerank_keep(ix, cand[q, : nin[q]], dist[q, : nin[q]], Q[q], R, si[q], sd[q], fresh)
        assert np.array_equal(host(dsi)[q], ri), f"query {q}"
        assert np.array_equal(host(dsd)[q], rd), f"query {q}"


# the selection's paths: a threshold bin of a few keys (uniform), of many equal keys ranked by id (ties), of more keys
# than the ranked buffer holds (equal: every key in one bin, narrowed by histogram passes over (key, id)), and keys past
# the register cache outside its range, in the first bin (tails, low_ties) or the last (last_bin)
@pytest.mark.parametrize("kind", ["uniform", "ties", "equal", "tails", "low_ties", "last_bin"])
def test_rerank_keep_selection_paths(L, ix, dix, small_index, kind):
    g = np.random.default_rng(9)
    m, W, KO, R = 24, 4096, 64, 128
    cand, dist, nin = random_candidates(g, m, W, 3000, ix.n, kind=kind)
    Q = small_index["Q"][:m]
    si = np.full((m, KO), -1, np.int64)
    sd = np.full((m, KO), np.inf, np.float32)
    dsi, dsd = dev(si), dev(sd)
    dc, dd, dn, dQ = dev(cand), dev(dist), dev(nin), dev(Q)
    L.call("octexStageRerankKeep", P(dc), P(dd), P(dn), i32(m), i32(W), P(dix["vectors"]), i32(ix.dim), P(dQ),
           i32(R), i32(KO), P(dsi), P(dsd), i32(1), None)
    for q in range(m):
        ri, rd = O.rerank_keep(ix, cand[q, : nin[q]], dist[q, : nin[q]], Q[q], R, si[q], sd[q], True)
        assert np.array_equal(host(dsi)[q], ri), f"query {q}"
        assert np.array_equal(host(dsd)[q], rd), f"query {q}"


@pytest.mark.parametrize("fresh", [True, False])
def test_sketch_keep_matches_oracle(L, fresh):
    g = np.random.default_rng(6 + fresh)
    m, W, KO = 32, 4096, 200
    cand, dist, nin = random_candidates(g, m, W, 3000, 100_000)
    si = np.full((m, KO), -1, np.int64)
    sd = np.full((m, KO), np.inf, np.float32)
    if not fresh:
        for q in range(m):
            ids = g.choice(100_000, 150, replace=False).astype(np.int32)
            si[q], sd[q] = O.merge_keep(si[q], sd[q], ids, g.integers(0, 40, 150).astype(np.float32), True)
    dsi, dsd = dev(si), dev(sd)
    dc, dd, dn = dev(cand), dev(dist), dev(nin)
    L.call("octexStageSketchKeep", P(dc), P(dd), P(dn), i32(m), i32(W), i32(KO), P(dsi), P(dsd), i32(fresh), None)
    for q in range(m):
        ri, rd = O.sketch_keep(cand[q, : nin[q]], dist[q, : nin[q]], si[q], sd[q], fresh)
        assert np.array_equal(host(dsi)[q], ri) and np.array_equal(host(dsd)[q], rd), f"query {q}"


def test_pick_starts_matches_oracle(L):
    g = np.random.default_rng(8)
    m, KO, S, waves = 30, 256, 64, 4
    E = S * waves
    si = np.stack([g.choice(50_000, KO, replace=False) for _ in range(m)]).astype(np.int64)
    si[:, 200:] = -1
    done = np.full((m, E), -3, np.int64)
    for off in (0, S, 2 * S):
        dd, dsi = dev(done), dev(si)
        seg2 = torch.zeros((m, S, 2), dtype=torch.int32, device="cuda")
        L.call("octexStagePickStarts", P(dsi), i32(m), i32(KO), P(dd), i32(E), i32(off), i32(S), i32(40),
               P(seg2), None)
        for q in range(m):
            rdone, rseg = O.pick_starts(si[q], done[q], off, S, 40)
            assert np.array_equal(host(dd)[q, : off + S], rdone[: off + S]), f"query {q} off {off}"
            assert np.array_equal(host(seg2)[q], rseg)
        done = host(dd)
        si = np.stack([np.concatenate([g.permutation(r[:200]), r[200:]]) for r in si])  # a new kept order


@pytest.mark.parametrize("R", [20, 64])
def test_final_rerank_and_take_k(L, ix, dix, small_index, R):
    g = np.random.default_rng(9)
    m, KO, k = 25, 128, 10
    si = np.stack([g.choice(ix.n, KO, replace=False) for _ in range(m)]).astype(np.int64)
    si[:, 40:50] = -1
    Q = small_index["Q"][:m]
    bi = torch.empty((m, k), dtype=torch.int64, device="cuda")
    bd = torch.empty((m, k), dtype=torch.float32, device="cuda")
    dsi, dQ = dev(si), dev(Q)
    L.call("octexStageFinalRerank", P(dsi), i32(m), i32(KO), i32(R), P(dix["vectors"]), i32(ix.dim), P(dQ),
           i32(k), P(bi), P(bd), None)
    for q in range(m):
        ri, rd = O.final_rerank(ix, si[q], R, Q[q], k)
        assert np.array_equal(host(bi)[q], ri) and np.array_equal(host(bd)[q], rd)
    sd = g.uniform(0, 1, (m, KO)).astype(np.float32)
    dsd = dev(sd)
    L.call("octexStageTakeK", P(dsi), P(dsd), i32(m), i32(KO), i32(k), P(bi), P(bd), None)
    assert np.array_equal(host(bi), si[:, :k]) and np.array_equal(host(bd), sd[:, :k])


def test_stage_errors(L):
    from octex_amd._lib import OctexError

    with pytest.raises(OctexError, match="blocks must be 1-6 or 8"):
        x = torch.zeros((4, 56), device="cuda")
        L.call("octexStageE8", P(x), i64(4), i32(7), ct.c_float(1.0), P(x), P(x), None)
    with pytest.raises(OctexError, match="multiple of 8"):
        L.call("octexStageProject", P(x), P(x), P(x), i32(4), i32(8), i32(36), P(x), None)
    with pytest.raises(OctexError, match="rerank in \\[1, 512\\]"):
        L.call("octexStageRerankKeep", P(x), P(x), P(x), i32(1), i32(2048), P(x), i32(64), P(x), i32(600), i32(10),
               P(x), P(x), i32(1), None)


# ---------------------------------------------------------------- lane layouts of the row kernels

# (D, S): the sketch scores put a row's S / 16 chunks on that many adjacent lanes (16 and 32 lanes per row at
# S = 256 / 512, 6 at 96, 3 at 48, 1 at 16) and the exact distances a row's D / 8 chunks on D / 8 lanes up to 32
# (12 lanes at D = 96, 25 at 200, 6 at 48); D = 960 takes several chunks per lane, D = 100 the unaligned path
@pytest.mark.parametrize("D,S", [(960, 512), (960, 256), (100, 48), (200, 96), (96, 96), (48, 16)])
def test_row_layouts_match_oracle(L, D, S):
    import octex_amd

    X, Q = clustered(n=1200, m=24, d=D, clusters=6, seed=D + S)
    index, _ = octex_amd.build_in_memory(X, copies=3, blocks=2, pca_dims=min(D, 32), list_len=8, table_len=16,
                                         log_buckets=8, sketch_width=S, member_lists=True, reverse_edges=False,
                                         seed=3)
    rix = O.Index(index)  # the GPU-built arrays, copied to the host
    assert rix.sketch_width == S and rix.dim == D
    rdix = dict(lists=dev(rix.lists), table=dev(rix.table), sketch=dev(rix.sketch), scale=dev(rix.scale),
                vectors=dev(rix.vectors.view(np.int16)))
    g = np.random.default_rng(D * 7 + S)
    m, nst = len(Q), 24
    seg2 = np.stack([g.integers(0, rix.n, (m, nst)), np.full((m, nst), rix.table_len)], -1).astype(np.int32)
    seg2[:, -3:] = 0
    qs = g.standard_normal((m, S)).astype(np.float32)
    cand, dist, nout = gather_gpu(L, rix, rdix, dev(seg2), qs, rows=1, W=2048)
    check_gather(rix, seg2, qs, cand, dist, nout, rows=True)
    # exact rerank of these candidates into a fresh kept list, then into a kept list that holds entries
    KO, R, W = 32, 48, 2048
    si = np.full((m, KO), -1, np.int64)
    sd = np.full((m, KO), np.inf, np.float32)
    dsi, dsd = dev(si), dev(sd)
    dc, dd, dn, dQ = dev(cand), dev(dist), dev(nout), dev(Q)
    for fresh in (True, False):
        L.call("octexStageRerankKeep", P(dc), P(dd), P(dn), i32(m), i32(W), P(rdix["vectors"]), i32(D), P(dQ),
               i32(R), i32(KO), P(dsi), P(dsd), i32(fresh), None)
        for q in range(m):
            n = nout[q]
            ri, rd = O.rerank_keep(rix, cand[q, :n], dist[q, :n], Q[q], R, si[q], sd[q], fresh)
            assert np.array_equal(host(dsi)[q], ri), f"query {q} fresh {fresh}"
            assert np.array_equal(host(dsd)[q], rd), f"query {q} fresh {fresh}"
            si[q], sd[q] = ri, rd
        dist = dist + g.uniform(0, 4, dist.shape).astype(np.float32)  # the second round: another sketch order
        dd = dev(dist)


# ---------------------------------------------------------------- the rerank's history of selected ids


def rerank_history(L, dix, ix, cand, dist, nin, W, Q, R, KO, si, sd, fresh, hist, H, hoff, hstore):
    """One octexStageRerankKeepHistory call on host arrays (si, sd, hist device tensors, updated in place); the
    per-query count of selected ids not reranked again."""
    m = cand.shape[0]
    nskip = torch.full((m,), -7, dtype=torch.int32, device="cuda")
    dc, dd, dn, dQ = dev(cand), dev(dist), dev(nin), dev(Q)  # alive until the kernel has run
    L.call("octexStageRerankKeepHistory", P(dc), P(dd), P(dn), i32(m), i32(W), P(dix["vectors"]), i32(ix.dim), P(dQ),
           i32(R), i32(KO), P(si), P(sd), i32(fresh), P(hist) if hist is not None else None, i32(H), i32(hoff),
           i32(hstore), P(nskip), None)
    return host(nskip)


def test_rerank_history_rounds_match_oracle(L, ix, dix, small_index):
    """The rounds of the fused rerank as a search runs them (a first round of R1, three waves of R2): each round but
    the last stores its selected ids in the history, and each later round skips the selected ids found there.  The
    kept lists equal the oracle's rerank_keep (which reranks every selected id) after every round; the history holds
    each round's selection (-1 padded); the skip counts are the selected ids an earlier round selected."""
    g = np.random.default_rng(22)
    m, W, KO, R1, R2, waves = 32, 4096, 64, 96, 64, 3
    H = R1 + R2 * (waves - 1)
    Q = small_index["Q"][:m]
    score = g.uniform(0, 100, ix.n).astype(np.float32)  # one sketch score per id, as within one query's search
    si = torch.full((m, KO), -3, dtype=torch.int64, device="cuda")  # stale contents: the first round is fresh
    sd = torch.full((m, KO), -1.0, dtype=torch.float32, device="cuda")
    hist = torch.full((m, H), -5, dtype=torch.int32, device="cuda")
    si_h = np.full((m, KO), -1, np.int64)
    sd_h = np.full((m, KO), np.inf, np.float32)
    earlier = [set() for _ in range(m)]  # ids selected by earlier rounds, per query
    skipped, before = 0, None
    for rnd in range(waves + 1):
        R = R1 if rnd == 0 else R2
        hoff = 0 if rnd == 0 else R1 + (rnd - 1) * R2
        store = rnd < waves
        nin = g.integers(200, 2000, m).astype(np.int32)
        nin[0] = 40 + rnd  # fewer candidates than R: all selected
        nin[1] = 0 if rnd == 2 else nin[1]  # a round without candidates
        cand = np.full((m, W), -9, np.int32)
        dist = np.zeros((m, W), np.float32)
        for q in range(m):
            old = np.array(sorted(earlier[q]), np.int64)
            k_old = min(len(old), nin[q] // 3)
            pick = g.choice(old, k_old, replace=False) if k_old else np.zeros(0, np.int64)
            others = g.permutation(np.setdiff1d(np.arange(ix.n), old))[: nin[q] - k_old]
            row = np.concatenate([pick, others])[g.permutation(nin[q])].astype(np.int32)
            cand[q, : nin[q]] = row
            dist[q, : nin[q]] = score[row]
        sk = rerank_history(L, dix, ix, cand, dist, nin, W, Q, R, KO, si, sd, rnd == 0, hist, H, hoff, store)
        gsi, gsd, gh = host(si), host(sd), host(hist)
        for q in range(m):
            n = nin[q]
            ri, rd = O.rerank_keep(ix, cand[q, :n], dist[q, :n], Q[q], R, si_h[q], sd_h[q], rnd == 0)
            assert np.array_equal(gsi[q], ri) and np.array_equal(gsd[q], rd), f"round {rnd} query {q}"
            si_h[q], sd_h[q] = ri, rd
            sel, _ = O.select(cand[q, :n], dist[q, :n], R)
            sel = {int(v) for v in sel}
            want_skip = 0 if rnd == 0 else len(sel & earlier[q])
            assert sk[q] == want_skip, f"round {rnd} query {q}: skipped reranks"
            skipped += want_skip
            if store:
                row = gh[q, hoff : hoff + R]
                assert {int(v) for v in row[row >= 0]} == sel and (row < 0).sum() == R - len(sel), f"round {rnd} {q}"
                assert np.all(row[: len(sel)] >= 0), f"round {rnd} query {q}: selected ids first"
            earlier[q] |= sel
        if not store:  # the last round leaves the history as it was
            assert np.array_equal(gh, before)
        before = gh
    assert skipped > 0


def test_rerank_history_uses_its_last_256_entries(L, ix, dix, small_index):
    """Only the ids of the history's last 256 entries are skipped: ids stored before them are reranked again.  Here the
    history's early entries name ids never merged (skipping them would lose them from the kept list, which then
    differs from the oracle's) and its last 256 entries ids that were merged."""
    g = np.random.default_rng(25)
    m, W, KO, R, H, hoff = 16, 4096, 64, 512, 1024, 1000
    Q = small_index["Q"][:m]
    score = g.uniform(0, 100, ix.n).astype(np.float32)
    si = torch.full((m, KO), -1, dtype=torch.int64, device="cuda")
    sd = torch.full((m, KO), float("inf"), dtype=torch.float32, device="cuda")
    si_h = np.full((m, KO), -1, np.int64)
    sd_h = np.full((m, KO), np.inf, np.float32)
    A = [g.choice(ix.n, 200, replace=False).astype(np.int32) for _ in range(m)]
    cand = np.full((m, W), -9, np.int32)
    dist = np.zeros((m, W), np.float32)
    nin = np.full(m, 200, np.int32)
    for q in range(m):
        cand[q, :200], dist[q, :200] = A[q], score[A[q]]
    assert rerank_history(L, dix, ix, cand, dist, nin, W, Q, R, KO, si, sd, True, None, 0, 0, False).sum() == 0
    hist = np.full((m, H), -1, np.int32)
    B = []
    for q in range(m):
        ri, rd = O.rerank_keep(ix, cand[q, :200], dist[q, :200], Q[q], R, si_h[q], sd_h[q], True)
        si_h[q], sd_h[q] = ri, rd
        b = np.setdiff1d(g.choice(ix.n, 900, replace=False), A[q])[:400].astype(np.int32)
        B.append(b)
        hist[q, : len(b)] = b  # outside the window: never merged
        hist[q, hoff - 256 : hoff - 256 + 200] = A[q]  # inside the window: merged above
        hist[q, hoff - 257] = b[0]  # just outside the window
    dh = dev(hist)
    nin = np.full(m, 600, np.int32)
    for q in range(m):
        row = np.concatenate([A[q], B[q]])[g.permutation(600)]
        cand[q, :600], dist[q, :600] = row, score[row]
    sk = rerank_history(L, dix, ix, cand, dist, nin, W, Q, R, KO, si, sd, False, dh, H, hoff, False)
    for q in range(m):
        ri, rd = O.rerank_keep(ix, cand[q, :600], dist[q, :600], Q[q], R, si_h[q], sd_h[q], False)
        assert np.array_equal(host(si)[q], ri) and np.array_equal(host(sd)[q], rd), f"query {q}"
        sel, _ = O.select(cand[q, :600], dist[q, :600], R)
        assert sk[q] == len({int(v) for v in sel} & {int(v) for v in A[q]}), f"query {q}"
    assert np.array_equal(host(dh), hist)  # not stored: the history is unchanged


@pytest.mark.parametrize("kind", ["equal", "few", "tails"])
def test_selection_of_many_equal_keys_at_the_largest_width(L, ix, dix, small_index, kind):
    """Candidate rows of 2^15 slots whose threshold bin holds thousands of keys (all equal, or three values): the
    selection narrows them by further histogram passes over (key, id) and takes the smallest ids, as the oracle;
    through the sketch merge (up to 30,000 candidates, KO 1000) and the exact rerank (every id of the index)."""
    g = np.random.default_rng(23)
    m, W = 12, 1 << 15

    def rows(n_max, N):
        cand = np.full((m, W), -9, np.int32)
        dist = np.zeros((m, W), np.float32)
        nin = g.integers(n_max // 2, n_max, m).astype(np.int32)
        nin[0] = n_max
        for q in range(m):
            n = nin[q]
            cand[q, :n] = g.choice(N, n, replace=False)
            if kind == "tails":  # keys past the first 4096 (the sketch merge's register cache) on both sides
                dist[q, :n] = np.where(np.arange(n) < 4096, g.uniform(40, 60, n), g.integers(0, 100, n))
            else:
                dist[q, :n] = 7.25 if kind == "equal" else g.integers(0, 3, n).astype(np.float32)
        return cand, dist, nin

    cand, dist, nin = rows(30_000, 1_000_000)
    KO = 1000
    si = torch.full((m, KO), -1, dtype=torch.int64, device="cuda")
    sd = torch.full((m, KO), float("inf"), dtype=torch.float32, device="cuda")
    dc, dd, dn = dev(cand), dev(dist), dev(nin)
    L.call("octexStageSketchKeep", P(dc), P(dd), P(dn), i32(m), i32(W), i32(KO), P(si), P(sd), i32(1), None)
    for q in range(m):
        ri, rd = O.sketch_keep(cand[q, : nin[q]], dist[q, : nin[q]], np.full(KO, -1, np.int64),
                               np.full(KO, np.inf, np.float32), True)
        assert np.array_equal(host(si)[q], ri) and np.array_equal(host(sd)[q], rd), f"sketch_keep query {q}"
    cand, dist, nin = rows(ix.n, ix.n)
    KO, R = 64, 512
    Q = small_index["Q"][:m]
    si = np.full((m, KO), -1, np.int64)
    sd = np.full((m, KO), np.inf, np.float32)
    dsi, dsd, dc, dd, dn, dQ = dev(si), dev(sd), dev(cand), dev(dist), dev(nin), dev(Q)
    L.call("octexStageRerankKeep", P(dc), P(dd), P(dn), i32(m), i32(W), P(dix["vectors"]), i32(ix.dim), P(dQ),
           i32(R), i32(KO), P(dsi), P(dsd), i32(1), None)
    for q in range(m):
        ri, rd = O.rerank_keep(ix, cand[q, : nin[q]], dist[q, : nin[q]], Q[q], R, si[q], sd[q], True)
        assert np.array_equal(host(dsi)[q], ri) and np.array_equal(host(dsd)[q], rd), f"rerank_keep query {q}"
