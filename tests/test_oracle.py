"""The CPU oracle pinned against the reference's known-answer rules and against independent mathematics:
IEEE fp16 (numpy), E8 lattice membership / optimality and the reference test's hash_ref (test_build.cu:79-176),
fp64 scores, brute-force sets and selections, the keep / pick-starts rules (test_search.cu:347-504), recall
against exact search, and the committed golden fixtures.  CPU only."""

import json
import os

import numpy as np
import pytest
from conftest import clustered, exact_knn, recall

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------- fp16


def test_fp16_matches_numpy_all_halves():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = O.h2f(h)
    ref = h.view(np.float16).astype(np.float32)
    same = (f == ref) | (np.isnan(f) & np.isnan(ref))
    assert same.all()


def test_fp16_rounding_matches_numpy():
    g = np.random.default_rng(0)
    x = np.concatenate([
        g.standard_normal(200_000).astype(np.float32) * 10,
        g.standard_normal(50_000).astype(np.float32) * 1e-5,  # subnormal range
        (g.integers(-4096, 4096, 50_000) + 0.5).astype(np.float32) / 2,  # exact ties
        np.array([65504, 65520, 65519.99, 1e9, -1e9, 0.0, -0.0, 2**-25, 2**-24, 3 * 2**-26], np.float32),
    ])
    with np.errstate(over="ignore"):  # 65520 and beyond round to infinity, as they should
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f2h(x), ref)


# ---------------------------------------------------------------- E8 (test_build.cu:94-176)

PRIMES = np.array([1000003, 998244353, 1000000007, 2147483647, 1099511627791, 4398042316799, 70368744177643,
                   1125899906842597], dtype=np.uint64)
MIX = np.uint64(0x9E3779B97F4A7C15)


def hash_ref(p, b):
    """The reference test's hash of decoded points (test_build.cu:79-92): lround(2 p) times the primes."""
    with np.errstate(over="ignore"):
        h = np.zeros(p.shape[0], np.uint64)
        for j in range(b):
            two_p = np.rint(2.0 * p[:, 8 * j : 8 * j + 8].astype(np.float64)).astype(np.int64).astype(np.uint64)
            hb = (two_p * PRIMES[None, :]).sum(axis=1, dtype=np.uint64)
            h = hb if j == 0 else h * MIX + hb
        s = h.view(np.int64)
        s = ((s ^ (s >> 31)).view(np.uint64) * MIX).view(np.int64)
        return s ^ (s >> 29)


def e8_roots():
    roots = []
    for i in range(8):
        for j in range(i + 1, 8):
            for si in (-1, 1):
                for sj in (-1, 1):
                    r = np.zeros(8)
                    r[i], r[j] = si, sj
                    roots.append(r)
    for m in range(256):
        if bin(m).count("1") % 2 == 0:
            roots.append(np.array([-0.5 if (m >> k) & 1 else 0.5 for k in range(8)]))
    return np.array(roots)


def e8_inputs(n=20000, b=4, seed=7):
    g = np.random.default_rng(seed)
    x = g.uniform(-6, 6, (n, 8 * b)).astype(np.float32)
    x[:500] = np.round(x[:500] * 2) * 0.5  # half-integer ties
    x[500:800] = np.round(x[500:800])  # integer points
    return x


def check_e8(x, p, h, b, inv_f):
    roots = e8_roots()
    assert len(roots) == 240
    xs = (x * np.float32(inv_f)).astype(np.float64)
    pp = p.astype(np.float64)
    for j in range(b):
        blk = pp[:, 8 * j : 8 * j + 8]
        fr = blk - np.floor(blk)
        all_int = (fr == 0).all(1)
        all_half = (fr == 0.5).all(1)
        assert (all_int | all_half).all(), "not in D8 u (D8 + 1/2)"
        assert (np.fmod(np.abs(blk.sum(1)), 2.0) == 0).all(), "odd coordinate sum"
        r = xs[:, 8 * j : 8 * j + 8] - blk
        d0 = (r**2).sum(1)
        d1 = ((r[:, None, :] - roots[None, :, :]) ** 2).sum(2)
        assert (d1 >= d0[:, None] - 1e-6).all(), "a root improves the decoded point"
    assert np.array_equal(h, hash_ref(p, b)), "hash differs from hash_ref"


def test_e8_invariants_and_hash_ref():
    x = e8_inputs()
    p, h = O.e8_batch(x, 4, 1.0 / 2.5)
    check_e8(x, p, h, 4, 1.0 / 2.5)


@pytest.mark.parametrize("b", [1, 2, 3, 8])
def test_e8_blocks(b):
    x = e8_inputs(n=3000, b=b, seed=b)
    p, h = O.e8_batch(x, b, 0.5)
    check_e8(x, p, h, b, 0.5)


def test_e8_plausible_mistakes_fail():
    """The checks above catch a wrong coset choice or a dropped parity fix (a planted mistake on the CPU)."""
    x = e8_inputs(n=2000)
    p, h = O.e8_batch(x, 4, 1.0)
    bad = p.copy()
    bad[:, :8] = np.round(x[:, :8])  # plain rounding: parity not fixed, coset never half
    with pytest.raises(AssertionError):
        check_e8(x, bad, hash_ref(bad, 4), 4, 1.0)
    with pytest.raises(AssertionError):
        check_e8(x, p, h ^ 1, 4, 1.0)


def test_golden_e8():
    g = np.load(os.path.join(GOLDEN, "e8.npz"))
    p, h = O.e8_batch(g["y"], int(g["b"]), float(g["inv_f"]))
    assert np.array_equal(p, g["p"]) and np.array_equal(h, g["h"])


# ---------------------------------------------------------------- scores


@pytest.mark.parametrize("S", [16, 48, 64, 96, 128, 512])
def test_sketch_dist_formula(S):
    g = np.random.default_rng(S)
    code = g.integers(-127, 128, S).astype(np.int8)
    scale = g.uniform(0.01, 0.1, S).astype(np.float32)
    qs = g.standard_normal(S).astype(np.float32)
    d = O.sketch_dist(code, scale, qs)
    ref = ((code.astype(np.float64) * scale.astype(np.float64) - qs.astype(np.float64)) ** 2).sum()
    assert abs(d - ref) <= 1e-5 * ref


@pytest.mark.parametrize("D", [2, 64, 96, 128, 130, 960])
def test_exact_dist_formula(D):
    g = np.random.default_rng(D)
    x = g.standard_normal(D).astype(np.float16)
    q = g.standard_normal(D).astype(np.float32)
    d = O.exact_dist(x.view(np.uint16), q)
    ref = ((x.astype(np.float64) - q.astype(np.float64)) ** 2).sum()
    assert abs(d - ref) <= 1e-5 * ref


def test_golden_scores():
    g = np.load(os.path.join(GOLDEN, "scores.npz"))
    for code, scale, qs, d in zip(g["code"], g["scale"], g["qs"], g["sketch"]):
        assert np.float32(O.sketch_dist(code, scale, qs)) == d
    for x, q, d in zip(g["x"], g["q"], g["exact"]):
        assert np.float32(O.exact_dist(x, q)) == d


# ---------------------------------------------------------------- selection and merges


def test_select_is_lexicographic():
    g = np.random.default_rng(1)
    cand = g.permutation(5000).astype(np.int32)
    dist = g.integers(0, 50, 5000).astype(np.float32)  # many ties
    for R in (1, 7, 128, 5000, 6000):
        sid, sd = O.select(cand, dist, R)
        order = np.lexsort((cand, dist))[: min(R, 5000)]
        assert np.array_equal(sid, cand[order]) and np.array_equal(sd, dist[order])


def keep_rule(si, sd, new_ids, new_d, KO, fresh):
    """test_search.cu:347-375: sort (distance, id), take the first KO distinct, pad (-1, +inf)."""
    pairs = [] if fresh else [(float(d), int(i)) for i, d in zip(si, sd) if i >= 0]
    pairs += [(float(d), int(i)) for i, d in zip(new_ids, new_d)]
    pairs = sorted(set(pairs))[:KO]
    out_i = [i for _, i in pairs] + [-1] * (KO - len(pairs))
    out_d = [d for d, _ in pairs] + [np.inf] * (KO - len(pairs))
    return np.array(out_i), np.array(out_d, np.float32)


def test_merge_keep_rule():
    g = np.random.default_rng(2)
    for fresh in (True, False):
        KO = 64
        si = g.choice(1000, KO, replace=False).astype(np.int64)
        sd = g.uniform(0, 10, KO).astype(np.float32)
        si[-5:] = -1
        ids = g.integers(0, 1000, 100).astype(np.int32)
        d = g.uniform(0, 10, 100).astype(np.float32)
        d[:10] = 3.0  # distance ties
        ids[10:20] = si[:10]  # the same ids again, with their own distances
        d[10:20] = sd[:10]
        oi, od = O.merge_keep(si, sd, ids, d, fresh)
        ri, rd = keep_rule(si, sd, ids, d, KO, fresh)
        assert np.array_equal(oi, ri) and np.array_equal(od, rd)


def test_pick_starts_rule():
    """test_search.cu:476-504: the first S kept entries not expanded before, -1 padded."""
    g = np.random.default_rng(3)
    KO, S, E = 200, 32, 96
    si = g.choice(10_000, KO, replace=False).astype(np.int64)
    si[150:] = -1
    done = np.full(E, -7, np.int64)
    done[:64] = g.choice(si[:150], 64, replace=False)
    done_out, seg2 = O.pick_starts(si, done, 64, S, 48)
    fresh = [v for v in si if v >= 0 and v not in set(done[:64].tolist())][:S]
    fresh += [-1] * (S - len(fresh))
    assert np.array_equal(done_out[64 : 64 + S], fresh)
    assert np.array_equal(done_out[:64], done[:64])
    exp = np.array([(v, 48) if v >= 0 else (0, 0) for v in fresh])
    assert np.array_equal(seg2, exp)


def rerank_rule_case(m=16, N=5000, D=32, KO=40, seed=11):
    """The inputs of the reference's rule test (test_search.cu:293-343): fp16 rows, fp32 queries; query q holds
    300 + 400 (q % 4) candidates of distinct sketch distances (a random rank times 0.01f, so the sketch order is
    unrelated to the exact one) and a kept list of KO / 2 other ids with their exact distances, sorted, padded
    with (-1, +inf).  The reference runs 4 queries; 16 here, so each planted mistake below changes some query."""
    g = np.random.default_rng(seed)
    X = g.standard_normal((N, D)).astype(np.float16)
    Q = g.standard_normal((m, D)).astype(np.float32)
    X64 = X.astype(np.float64)
    exact = lambda q, ids: ((X64[np.asarray(ids)] - Q[q].astype(np.float64)) ** 2).sum(-1)  # noqa: E731
    cands, dists, si, sd = [], [], np.full((m, KO), -1, np.int64), np.full((m, KO), np.inf, np.float32)
    for q in range(m):
        n = 300 + 400 * (q % 4)
        ids = g.permutation(N).astype(np.int32)
        rank = g.permutation(np.arange(1, n + 1))
        cands.append(ids[:n])
        dists.append(rank.astype(np.float32) * np.float32(0.01))
        kept = ids[n : n + KO // 2]
        order = np.argsort(exact(q, kept), kind="stable")
        si[q, : KO // 2] = kept[order]
        sd[q, : KO // 2] = exact(q, kept[order]).astype(np.float32)
    return O.Index.from_vectors(X.view(np.uint16)), Q, exact, cands, dists, si, sd


def same_up_to_near_ties(got_ids, got_d, want_ids, want_d64, exact_of):
    """Ids equal position by position, except where the fp64 distances of the two ids agree within 1e-5 relative
    (a near tie that fp32 and fp64 may order differently); distances within 1e-3 relative (the north star's bar)."""
    for j, (a, b) in enumerate(zip(got_ids, want_ids)):
        if a == b:
            continue
        assert a >= 0 and b >= 0, f"position {j}: {a} vs {b}"
        da, db = exact_of(a), exact_of(b)
        assert abs(da - db) <= 1e-5 * (1 + db), f"position {j}: {a} ({da}) vs {b} ({db})"
    valid = np.asarray(want_ids) >= 0
    assert np.all(np.abs(np.asarray(got_d)[valid] - np.asarray(want_d64)[valid]) <= 1e-3 * (1 + np.asarray(want_d64)[valid]))


def check_rerank_rule(cand, dist, si, sd, out_i, out_d, R, KO, exact_q):
    """test_search.cu:350-375: the pool of the R sketch-nearest candidates and the kept ids, exact (fp64) distances,
    the best KO distinct, padded with -1."""
    sk = sorted(zip(dist.tolist(), cand.tolist()))[: min(R, len(cand))]
    pool = {int(i) for _, i in sk} | {int(i) for i in si if i >= 0}
    ids = np.array(sorted(pool), np.int64)
    d64 = exact_q(ids)
    order = np.lexsort((ids, d64))[:KO]
    want_i = np.full(KO, -1, np.int64)
    want_d = np.full(KO, np.inf)
    want_i[: len(order)], want_d[: len(order)] = ids[order], d64[order]
    same_up_to_near_ties(out_i, out_d, want_i, want_d, lambda i: float(exact_q([i])[0]))


def check_sketch_keep_rule(cand, dist, out_i, out_d, KO):
    """test_search.cu:381-396: the KO sketch-nearest, by sketch distance, into an empty list (distinct distances
    here, so the ids are fixed too)."""
    sk = sorted(zip(dist.tolist(), cand.tolist()))[:KO]
    assert np.array_equal(out_d[: len(sk)], np.array([d for d, _ in sk], np.float32))
    assert np.array_equal(out_i[: len(sk)], np.array([i for _, i in sk], np.int64))


def check_final_rule(si, out_i, out_d, FR, k, exact_q):
    """test_search.cu:398-410: the first FR kept entries reranked exactly (fp64) into the best k."""
    ids = np.asarray(si[:FR], np.int64)
    ids = ids[ids >= 0]
    d64 = exact_q(ids)
    order = np.lexsort((ids, d64))[:k]
    same_up_to_near_ties(out_i, out_d, ids[order], d64[order], lambda i: float(exact_q([i])[0]))


def test_rerank_sketch_keep_final_rerank_rules():
    """The reference's rule test of rerank_keep, sketch_keep and final_rerank (test_search.cu:293-412) against the
    oracle's functions: exact rerank of the R sketch-nearest merged into the kept KO, the sketch merge into an
    empty list, then the final exact rerank of the first 24 kept entries into the best 10."""
    ix, Q, exact, cands, dists, si, sd = rerank_rule_case()
    R, KO, k, FR = 64, 40, 10, 24
    for q in range(len(Q)):
        ex = lambda ids, q=q: exact(q, ids)  # noqa: E731
        oi, od = O.rerank_keep(ix, cands[q], dists[q], Q[q], R, si[q], sd[q], fresh=False)
        check_rerank_rule(cands[q], dists[q], si[q], sd[q], oi, od, R, KO, ex)
        ki, kd = O.sketch_keep(cands[q], dists[q], si[q], sd[q], fresh=True)
        check_sketch_keep_rule(cands[q], dists[q], ki, kd, KO)
        bi, bd = O.final_rerank(ix, ki, FR, Q[q], k)
        check_final_rule(ki, bi, bd, FR, k, ex)


def test_rerank_rules_catch_plausible_mistakes():
    """Each plausible mistake in the composition fails the rules above on some query (planted on the CPU by
    feeding the oracle's own functions the wrong arguments)."""
    ix, Q, exact, cands, dists, si, sd = rerank_rule_case()
    R, KO, k, FR = 64, 40, 10, 24

    def fails(run):
        for q in range(len(Q)):
            try:
                run(q, lambda ids, q=q: exact(q, ids))
            except AssertionError:
                return True
        return False

    def rerank(R_used, fresh):
        def run(q, ex):
            oi, od = O.rerank_keep(ix, cands[q], dists[q], Q[q], R_used, si[q], sd[q], fresh=fresh)
            check_rerank_rule(cands[q], dists[q], si[q], sd[q], oi, od, R, KO, ex)
        return run

    assert not fails(rerank(R, False))
    assert fails(rerank(R + 1, False))  # one candidate too many reranked
    assert fails(rerank(R - 1, False))  # one too few
    assert fails(rerank(R, True))  # the kept list ignored when not fresh

    def sketch_keep_not_fresh(q, ex):  # the previous kept list merged into what should start empty
        ki, kd = O.sketch_keep(cands[q], dists[q], si[q], np.zeros_like(sd[q]), fresh=False)
        check_sketch_keep_rule(cands[q], dists[q], ki, kd, KO)

    assert fails(sketch_keep_not_fresh)

    def final(kind):
        def run(q, ex):
            ki, _ = O.sketch_keep(cands[q], dists[q], si[q], sd[q], fresh=True)
            if kind == "sketch":  # the first k kept entries with their sketch distances, not reranked
                bi, bd = ki[:k], O.sketch_keep(cands[q], dists[q], si[q], sd[q], fresh=True)[1][:k]
            else:  # reranked over every kept entry instead of the first FR
                bi, bd = O.final_rerank(ix, ki, KO, Q[q], k)
            check_final_rule(ki, bi, bd, FR, k, ex)
        return run

    assert fails(final("sketch"))
    assert fails(final("all"))


def test_rerank_history_skip_keeps_the_same_lists():
    """The rule the HIP rerank's history skip rests on, checked with the oracle's functions over four rounds: merging
    only the selected ids no earlier round selected gives the kept list that reranking every selected id gives (the
    kept list is the KO smallest distinct keys of every key merged so far, so an id merged before is either in it
    already or above all KO of it).  Rows repeat earlier rounds' ids with the same sketch scores, as a query's do.
    Skipping ids selected for the first time (a planted mistake: ids never merged) changes some query's list."""
    ix, Q, exact, cands, dists, si0, sd0 = rerank_rule_case(m=24, seed=13)
    g = np.random.default_rng(14)
    KO, R = 40, 48
    N = ix.n
    score = g.permutation(N).astype(np.float32) * np.float32(0.01)  # one sketch score per id and query
    planted_differs = False
    for q in range(len(Q)):
        full_i, full_d = si0[q].copy(), sd0[q].copy()
        skip_i, skip_d = si0[q].copy(), sd0[q].copy()
        bad_i, bad_d = si0[q].copy(), sd0[q].copy()
        seen, never_merged = set(), set()
        for rnd in range(4):
            old = np.array(sorted(seen), np.int32)
            k_old = min(len(old), 150)
            row = np.concatenate([g.choice(old, k_old, replace=False) if k_old else np.zeros(0, np.int32),
                                  g.choice(N, 400, replace=False).astype(np.int32)])
            row = np.unique(row)[g.permutation(len(np.unique(row)))]
            d = score[row]
            full_i, full_d = O.rerank_keep(ix, row, d, Q[q], R, full_i, full_d, fresh=False)
            sel, seld = O.select(row, d, R)
            keep = np.array([int(v) not in seen for v in sel], bool)
            skip_i, skip_d = O.rerank_keep(ix, sel[keep], seld[keep], Q[q], max(1, int(keep.sum())), skip_i, skip_d,
                                           fresh=False)
            assert np.array_equal(skip_i, full_i) and np.array_equal(skip_d, full_d), f"query {q} round {rnd}"
            # planted: four of the ids selected for the first time are treated as seen too
            new_ids = [int(v) for v in sel if int(v) not in seen][:4]
            never_merged |= set(new_ids)
            bkeep = np.array([int(v) not in seen and int(v) not in never_merged for v in sel], bool)
            bad_i, bad_d = O.rerank_keep(ix, sel[bkeep], seld[bkeep], Q[q], max(1, int(bkeep.sum())), bad_i, bad_d,
                                         fresh=False)
            planted_differs |= not np.array_equal(bad_i, full_i)
            seen |= {int(v) for v in sel}
    assert planted_differs


# ---------------------------------------------------------------- index-level stages


def test_gather_is_the_union(small_index):
    ix = O.Index(small_index["path"])
    g = np.random.default_rng(4)
    qs = g.standard_normal(ix.sketch_width).astype(np.float32)
    # list segments of random cell rows of every copy
    C = ix.copies
    seg = np.zeros((C, 2), np.int32)
    for c in range(C):
        rows = ix.lists.shape[1] // ix.list_len
        seg[c] = (g.integers(0, rows) * ix.list_len, g.integers(0, ix.list_len + 1))
    seg[3] = (0, 0)
    cand, dist = O.gather(ix, seg, qs)
    union = set()
    for c in range(C):
        union |= set(ix.lists[c, seg[c, 0] : seg[c, 0] + seg[c, 1]].tolist())
    assert set(cand.tolist()) == union and len(cand) == len(union)
    ref = ((ix.sketch[cand].astype(np.float64) * ix.scale - qs) ** 2).sum(1)
    assert np.allclose(dist, ref, rtol=1e-5)
    # table rows, with -1 padding skipped
    seg2 = np.stack([g.integers(0, ix.n, 40), np.full(40, ix.table_len)], 1).astype(np.int32)
    seg2[5] = (0, 0)
    cand2, _ = O.gather(ix, seg2, qs, rows=True)
    rows = set(ix.table[seg2[seg2[:, 1] > 0, 0]].ravel().tolist()) - {-1}
    assert set(cand2.tolist()) == rows


def probe_construction(m=7, C=3, spacing=(1.0, 4.0), b=4, logT=4, l=5, lr=3, seed=7, absent=()):
    """The reference's probe test (test_search.cu:86-170): projections y [m, C, 8b] ~ N(0, 2) rounded to fp16;
    per copy and level a cell table holding the cell of every second query at the finest level (query q even)
    and of all queries at every coarser level, keys in (bucket, hash) order with their CSR offsets and the
    levels' first rows.  Queries listed in `absent` get no cell at any level.  Returns the probe's arrays, the
    fp16 projections and the segments it must produce: (row * l, lr) at the finest level holding the query's
    cell, (0, 0) when no level does (the absent queries' projections lie far from every other query's, so no
    shared coarse cell lists them)."""
    g = np.random.default_rng(seed)
    L, w, T = len(spacing), 8 * b, 1 << logT
    y = g.normal(0.0, 2.0, (m, C, w))
    y[list(absent)] = y[list(absent)] * 40 + 300  # far from every other query's cell at every level
    y = O.h2f(O.f2h(y.reshape(m * C, w).astype(np.float32)))
    inv = np.array([np.float32(1.0) / np.float32(f) for f in spacing], np.float32)  # 1.f / spacing[j]
    h = np.stack([O.e8_batch(y, b, float(inv[j]))[1] for j in range(L)], 1).reshape(m, C, L)
    keys = np.zeros((C, L, m), np.int64)
    off = np.zeros((C, L, T + 1), np.int32)
    base = np.zeros((C, L), np.int32)
    row = {}
    rows = 0
    for c in range(C):
        for j in range(L):
            base[c, j] = rows
            cells = sorted({(int(h[q, c, j]) & (T - 1), int(h[q, c, j])) for q in range(m)
                            if q not in absent and (j > 0 or q % 2 == 0)})
            for p, (_, hh) in enumerate(cells):
                keys[c, j, p] = hh
                row[c, j, hh] = rows + p
            cnt = np.bincount([bk for bk, _ in cells], minlength=T)
            off[c, j, 1:] = np.cumsum(cnt)
            rows += len(cells)
    want = np.zeros((m, C, 2), np.int32)
    for q in range(m):
        for c in range(C):
            if q in absent:
                continue
            j = 0 if q % 2 == 0 else 1
            want[q, c] = (row[c, j, int(h[q, c, j])] * l, lr)
    arrays = dict(inv_f=inv, offsets=off, keys=keys, base=base, list_len=l, blocks=b)
    return arrays, O.f2h(y).reshape(m, C * w), want


def check_probe(seg, want):
    assert np.array_equal(seg, want), f"{(seg != want).any(-1).sum()} of {want.shape[0] * want.shape[1]} segments differ"


def test_probe_construction_reference():
    """The reference test's exact shape: m 7, C 3, L 2 (spacings 1 and 4), b 4, 16 buckets, l 5, lr 3."""
    arrays, Y, want = probe_construction()
    seg = O.probe(O.Index.from_arrays(**arrays), Y, read=3)
    check_probe(seg, want)


def test_probe_construction_levels_and_misses():
    """More queries and copies, five levels, eight buckets (several keys per bucket), queries with no cell."""
    arrays, Y, want = probe_construction(m=60, C=5, spacing=(0.5, 1.0, 2.0, 4.0, 8.0), logT=3, l=16, lr=9,
                                         seed=3, absent=(5, 6, 17))
    assert (want[[5, 6, 17], :, 1] == 0).all() and (want[:, :, 1] > 0).sum() == 57 * 5
    check_probe(O.probe(O.Index.from_arrays(**arrays), Y, read=9), want)


def test_probe_construction_catches_plausible_mistakes():
    """Planted mistakes on the CPU: a probe walking the levels coarse to fine (the oracle over the same tables
    with the level order reversed), a first row off by one, and segments of the wrong length all fail."""
    arrays, Y, want = probe_construction(m=40, C=4, spacing=(1.0, 2.0, 4.0), seed=11)
    rev = dict(arrays, inv_f=arrays["inv_f"][::-1], offsets=arrays["offsets"][:, ::-1], keys=arrays["keys"][:, ::-1],
               base=arrays["base"][:, ::-1])
    with pytest.raises(AssertionError):
        check_probe(O.probe(O.Index.from_arrays(**rev), Y, read=3), want)
    with pytest.raises(AssertionError):
        check_probe(O.probe(O.Index.from_arrays(**dict(arrays, base=arrays["base"] + 1)), Y, read=3), want)
    with pytest.raises(AssertionError):
        check_probe(O.probe(O.Index.from_arrays(**arrays), Y, read=4), want)


# ---------------------------------------------------------------- query preparation against fp64 numpy


def check_center(q, mu, qc, qh):
    """qc = q - mu in fp32 (one IEEE rounding), qh = fp16(qc) rounded to nearest even (search_kernels.cuh:57-69)."""
    assert np.array_equal(qc, q - mu[None, :])
    assert np.array_equal(qh, qc.astype(np.float16).view(np.uint16))


def test_center_matches_numpy():
    g = np.random.default_rng(21)
    q = (g.standard_normal((50, 96)) * 3).astype(np.float32)
    mu = g.standard_normal(96).astype(np.float32)
    q[0, :8] = mu[:8] + np.float32(2.0**-20)  # cancellation: tiny centred values, fp16 subnormals
    check_center(q, mu, *O.center(q, mu))
    qc, qh = O.center(q, mu)
    with pytest.raises(AssertionError):  # not centred before the fp16 rounding
        check_center(q, mu, qc, q.astype(np.float16).view(np.uint16))
    with pytest.raises(AssertionError):  # rounded toward zero instead of to nearest
        check_center(q, mu, qc, (qc.view(np.uint32) >> 13 << 13).view(np.float32).astype(np.float16).view(np.uint16))


def project_fp64(qh, ucat, shift):
    """qh @ ucat + shift of fp16 operands in fp64: every product is exact, the sum of at most a few thousand
    terms is within 1e-13 relative of the exact one."""
    return O.h2f(qh).astype(np.float64) @ O.h2f(ucat).astype(np.float64) + O.h2f(shift).astype(np.float64)[None, :]


def check_project(qh, ucat, shift, Y, Yd):
    """Yd equals the fp64 product plus shift (search.cu:305-320: Y = qh ucat + shift, fp16 operands), and Y is
    Yd rounded once to fp16 (numpy's float64 -> float16 rounds directly)."""
    ref = project_fp64(qh, ucat, shift)
    mag = np.abs(O.h2f(qh).astype(np.float64)) @ np.abs(O.h2f(ucat).astype(np.float64)) + np.abs(O.h2f(shift))
    assert (np.abs(Yd - ref) <= 1e-13 * mag + 1e-300).all()
    assert np.array_equal(Y, Yd.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("m,D,wdt", [(40, 96, 256), (16, 128, 64), (9, 960, 32), (20, 32, 32)])
def test_project_matches_numpy(m, D, wdt):
    g = np.random.default_rng(m * D)
    qh = O.f2h(g.standard_normal((m, D)).astype(np.float32))
    ucat = O.f2h((g.standard_normal((D, wdt)) / np.sqrt(D)).astype(np.float32))
    shift = O.f2h(g.uniform(0, 2, wdt).astype(np.float32))
    Y, Yd = O.project(qh, ucat, shift)
    check_project(qh, ucat, shift, Y, Yd)


def test_project_rounds_once_at_fp16_ties():
    """Sums on and just beside an fp16 tie (1 + 2^-11 is halfway between 1 and 1 + 2^-10): 1 + 2^-11 + 2^-30
    must round up, which a detour through fp32 (where 2^-30 vanishes, leaving the tie) would round to 1."""
    qh = O.f2h(np.array([[1.0, 2.0**-11, 2.0**-15, 0.0], [1.0, 2.0**-11, 0.0, 0.0], [1.0, 2.0**-11, -(2.0**-15), 0.0]],
                        np.float32))
    ucat = O.f2h(np.array([[1.0, 0.0], [1.0, 0.0], [2.0**-15, 0.0], [0.0, 1.0]], np.float32))
    shift = O.f2h(np.zeros(2, np.float32))
    Y, Yd = O.project(qh, ucat, shift)
    assert Yd[0, 0] == 1 + 2.0**-11 + 2.0**-30
    check_project(qh, ucat, shift, Y, Yd)
    assert list(Y[:, 0]) == list(O.f2h(np.array([1 + 2.0**-10, 1.0, 1.0], np.float32)))


def test_project_catches_plausible_mistakes():
    g = np.random.default_rng(5)
    D = wdt = 64
    qh = O.f2h(g.standard_normal((12, D)).astype(np.float32))
    ucat = O.f2h((g.standard_normal((D, wdt)) / 8).astype(np.float32))
    shift = O.f2h(g.uniform(0, 2, wdt).astype(np.float32))
    Y, Yd = O.project(qh, ucat, shift)
    with pytest.raises(AssertionError):  # transposed projection
        Yt, Ydt = O.project(qh, np.ascontiguousarray(ucat.T), shift)
        check_project(qh, ucat, shift, Yt, Ydt)
    with pytest.raises(AssertionError):  # shift dropped
        Y0, Yd0 = O.project(qh, ucat, np.zeros_like(shift))
        check_project(qh, ucat, shift, Y0, Yd0)
    with pytest.raises(AssertionError):  # fp32 accumulation rounded twice
        Yf = (O.h2f(qh) @ O.h2f(ucat) + O.h2f(shift)).astype(np.float16).view(np.uint16)
        check_project(qh, ucat, shift, Yf, (O.h2f(qh) @ O.h2f(ucat) + O.h2f(shift)).astype(np.float64))


def check_sketch_query(qc, basis, qs):
    """qs = qc @ basis as the fp32 rounding of the fp64 sum: within half an fp32 ulp plus the fp64 sum's own error
    (search.cu:323-341 computes it in TF32, which no MI355X arithmetic reproduces; full fp32 is the pin)."""
    ref = qc.astype(np.float64) @ basis.astype(np.float64)
    mag = np.abs(qc.astype(np.float64)) @ np.abs(basis.astype(np.float64))
    half_ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64) / 2
    assert (np.abs(qs.astype(np.float64) - ref) <= half_ulp + 1e-13 * mag).all()


@pytest.mark.parametrize("m,D,S", [(30, 96, 64), (8, 960, 128), (5, 128, 512)])
def test_sketch_query_matches_numpy(m, D, S):
    g = np.random.default_rng(D + S)
    qc = g.standard_normal((m, D)).astype(np.float32)
    basis = (g.standard_normal((D, S)) / np.sqrt(D)).astype(np.float32)
    check_sketch_query(qc, basis, O.sketch_query(qc, basis))


def test_sketch_query_catches_plausible_mistakes():
    g = np.random.default_rng(6)
    D = S = 64
    qc = g.standard_normal((20, D)).astype(np.float32)
    basis = g.standard_normal((D, S)).astype(np.float32)
    with pytest.raises(AssertionError):  # transposed basis
        check_sketch_query(qc, basis, O.sketch_query(qc, np.ascontiguousarray(basis.T)))
    with pytest.raises(AssertionError):  # the last coordinate dropped
        check_sketch_query(qc, basis, O.sketch_query(qc[:, :-1], basis[:-1]))
    with pytest.raises(AssertionError):  # a sequential fp32 sum (error grows with D)
        acc = np.zeros((20, S), np.float32)
        for d in range(D):
            acc = (acc + qc[:, d : d + 1] * basis[d][None, :]).astype(np.float32)
        check_sketch_query(qc, basis, acc)


def test_search_recall(small_index):
    ix = O.Index(small_index["path"])
    D, I = O.search(ix, small_index["Q"], k=10, read=32, starts=64, waves=2)
    assert recall(I, small_index["gt"]) >= 0.95
    assert (np.diff(D, axis=1) >= 0).all()
    Xh = small_index["X"].astype(np.float16).astype(np.float64)
    exact = ((Xh[I] - small_index["Q"][:, None, :].astype(np.float64)) ** 2).sum(-1)
    assert np.allclose(D, exact, rtol=1e-4)


def test_search_sketch_rank(small_index):
    """Sketch-rank mode (search_kernels.cuh:471-508, 634-669): the returned distances are the exact ones of the
    returned ids (fp64 over the fp16 rows, within fp32 accumulation error), sorted; with final_rerank 0 they are
    the sketch distances, which that check rejects."""
    ix = O.Index(small_index["path"])
    Q = small_index["Q"]
    Xh = small_index["X"].astype(np.float16).astype(np.float64)
    D, I = O.search(ix, Q, k=10, read=32, starts=64, waves=2, sketch_rank=True, final_rerank=64)
    assert recall(I, small_index["gt"]) >= 0.8
    assert (np.diff(D, axis=1) >= 0).all()
    exact = ((Xh[I] - Q[:, None, :].astype(np.float64)) ** 2).sum(-1)
    assert np.allclose(D, exact, rtol=1e-4)
    Ds, Is = O.search(ix, Q, k=10, read=32, starts=64, waves=2, sketch_rank=True, final_rerank=0)
    exact_s = ((Xh[Is] - Q[:, None, :].astype(np.float64)) ** 2).sum(-1)
    assert not np.allclose(Ds, exact_s, rtol=1e-4)


def test_search_limits(small_index):
    ix = O.Index(small_index["path"])
    q = small_index["Q"][:2]
    with pytest.raises(ValueError, match="max\\(starts, k\\) must be <= 512"):
        O.search(ix, q, k=10, starts=600)
    with pytest.raises(ValueError, match="rerank in \\[1, 512\\]"):
        O.search(ix, q, k=10, rerank=0)
    with pytest.raises(ValueError, match="starts \\* \\(waves - 1\\) <= 6144"):
        O.search(ix, q, k=10, starts=512, waves=14, rerank=1, wave_rerank=1)


def test_list_limit_and_copies_limit(small_index):
    ix = O.Index(small_index["path"], list_limit=8, copies_limit=4)
    full = O.Index(small_index["path"])
    assert ix.copies == 4 and ix.list_len == 8
    rows = full.lists.shape[1] // full.list_len
    assert np.array_equal(ix.lists.reshape(4, rows, 8), full.lists[:4].reshape(4, rows, full.list_len)[:, :, :8])
    D, I = O.search(ix, small_index["Q"][:10], k=10, read=32, starts=32, waves=1)
    assert (I >= 0).all()


def test_index_directory_format(small_index):
    """The builder writes the files and shapes of the format-1 directory (design.md:27-54)."""
    path = small_index["path"]
    meta = json.load(open(os.path.join(path, "meta.json")))
    assert meta["format"] == 1 and meta["metric"] == "sqeuclidean" and meta["files"] == {}
    C, L, n, d = meta["copies"], len(meta["spacings"]), meta["n"], meta["dim"]
    w = 8 * meta["blocks"]
    shapes = dict(mean=(d,), proj=(C, d, w), shift=(C, w), base=(C, L), cells=(C, L), sketch_scale=(meta["sketch_width"],),
                  sketch_basis=(d, meta["sketch_width"]), sketch=(n, meta["sketch_width"]), vectors=(n, d),
                  table=(n, meta["table_len"]))
    for name, shape in shapes.items():
        assert np.load(os.path.join(path, name + ".npy"), mmap_mode="r").shape == shape, name
    offs = np.load(os.path.join(path, "offsets.npy"))
    keys = np.load(os.path.join(path, "keys.npy"))
    cells = np.load(os.path.join(path, "cells.npy"))
    assert offs.shape == (C, L, 2 ** meta["log_buckets"] + 1)
    assert (offs[:, :, -1] == cells).all() and (np.diff(offs, axis=2) >= 0).all()
    T = 2 ** meta["log_buckets"]
    for c in range(C):
        for j in range(L):
            k = keys[c, j, : cells[c, j]]
            b = k & (T - 1)
            assert (np.diff(b) >= 0).all()  # (bucket, hash) order
            assert np.array_equal(np.searchsorted(b, np.arange(T + 1)), offs[c, j])


def table_mode_data(n=1500, d=32, seed=5):
    """The rows of the reference's table test (test_build.cu:268-277): N(0, 1) plus i % 23 on the first 3
    coordinates."""
    g = np.random.default_rng(seed)
    x = g.standard_normal((n, d)).astype(np.float32)
    x[:, :3] += (np.arange(n) % 23).astype(np.float32)[:, None]
    return x


def check_exact_table(table, x, k):
    """The reference's check of an exact table with reverse edges (test_build.cu:278-377): the exact top k of
    every row (fp64 over the fp16 rows, self excluded); the expected row by the prototype rule (first k/2
    forward, up to k/2 reverse entries of rank < k/2 by (rank, id), then the rest forward, duplicates dropped,
    cut to k); every table row complete, without self or duplicates, sorted by distance, and its entries in
    the expected row (at most 1 in 1000 outside, for near ties)."""
    n = len(x)
    xh = x.astype(np.float16).astype(np.float64)
    d2 = (xh**2).sum(1)[:, None] - 2 * xh @ xh.T + (xh**2).sum(1)[None, :]
    np.fill_diagonal(d2, np.inf)
    exact = np.argsort(d2, axis=1, kind="stable")[:, :k]
    h = k // 2
    rv = [[] for _ in range(n)]
    for v in range(n):
        for r in range(h):
            rv[exact[v, r]].append((r, v))
    outside = 0
    for u in range(n):
        cand = list(exact[u, :h]) + [v for _, v in sorted(rv[u])[:h]] + list(exact[u, h:])
        expect = []
        for v in cand:
            if len(expect) < k and v not in expect:
                expect.append(v)
        row = table[u]
        assert (row >= 0).all() and (row != u).all() and len(set(row.tolist())) == k
        dv = d2[u, row]
        assert (np.diff(dv) >= -1e-3 * (1 + dv[:-1])).all()
        outside += int(np.sum(~np.isin(row, expect)))
    assert outside <= n * k // 1000


def test_exact_table_rule(tmp_path):
    """The oracle's exact neighbor table with reverse edges meets the reference's own test of it."""
    x, k = table_mode_data(), 12
    O.build(x, str(tmp_path / "t"), copies=2, blocks=2, pca_dims=16, list_len=8, log_buckets=10, sketch_width=16,
            table_len=k, reverse_edges=True, member_lists=True, seed=0)
    check_exact_table(np.load(tmp_path / "t" / "table.npy"), x, k)


def test_exact_table_rule_catches_a_wrong_merge(tmp_path):
    """The check fails on the forward-only table (reverse edges dropped): it is not vacuous."""
    x, k = table_mode_data(), 12
    O.build(x, str(tmp_path / "f"), copies=2, blocks=2, pca_dims=16, list_len=8, log_buckets=10, sketch_width=16,
            table_len=k, reverse_edges=False, member_lists=True, seed=0)
    with pytest.raises(AssertionError):
        check_exact_table(np.load(tmp_path / "f" / "table.npy"), x, k)


def check_exact_lists(path, X, stride=40, fraction=False):
    """Every sampled cell's list holds the l rows nearest to the cell's center among all rows: the projections
    y = (x16 - mean) @ proj + shift recomputed in fp64 from the directory, the center f times the E8 point of a
    member's y / f; up to near ties of fp32 distances (a few ulp of the squared norms).  Returns the number of
    cells checked; with `fraction` (approximate lists), only that every list holds l distinct rows, and the fraction
    of the checked entries that are among the l nearest."""
    ix = O.Index(path)
    hits = total = 0
    l = ix.list_len
    Xh = X.astype(np.float16).astype(np.float64)
    cells = np.load(os.path.join(path, "cells.npy"))
    checked = 0
    for c in range(ix.copies):
        proj = np.load(os.path.join(path, "proj.npy"))[c].astype(np.float64)
        shift = np.load(os.path.join(path, "shift.npy"))[c].astype(np.float64)
        y = (Xh - ix.mean.astype(np.float64)) @ proj + shift
        for j, f in enumerate(ix.spacings):
            M = cells[c, j]
            keys = ix.keys[c, j, :M]
            p, h = O.e8_batch((y / f).astype(np.float32), ix.blocks, 1.0)
            first = {}
            for r, hv in enumerate(h):
                first.setdefault(int(hv), r)
            r0 = ix.base[c, j]
            rows = ix.lists[c, r0 * l : (r0 + M) * l].reshape(M, l)
            for ci in range(0, M, max(1, M // stride)):
                if int(keys[ci]) not in first:
                    continue  # the member's fp64 projection rounds to another cell
                z = p[first[int(keys[ci])]].astype(np.float64) * f
                dz = ((y - z) ** 2).sum(1)
                lth = np.sort(dz)[l - 1]
                tol = 1e-5 * ((z**2).sum() + (y**2).sum(1).max()) + 1e-4 * lth
                assert len(set(rows[ci].tolist())) == l and (rows[ci] >= 0).all()
                within = dz[rows[ci]] <= lth + tol
                if not fraction:
                    assert within.all()
                hits += int(within.sum())
                total += l
                checked += 1
    return hits / max(total, 1) if fraction else checked


def test_oracle_exact_lists(tmp_path):
    """The oracle's exact lists (build_cells.cuh:506-510, 567-599) hold each cell center's l nearest rows."""
    X, _ = clustered(n=1500, m=10, d=32, clusters=10, seed=9)
    O.build(X, str(tmp_path / "e"), copies=2, list_len=16, table_len=8, log_buckets=10, exact_lists=True, seed=5)
    assert check_exact_lists(str(tmp_path / "e"), X) > 50


def test_exact_list_check_catches_member_lists(tmp_path):
    """The same check fails on member lists (the l nearest members of the cell only): it is not vacuous."""
    X, _ = clustered(n=1500, m=10, d=32, clusters=10, seed=9)
    O.build(X, str(tmp_path / "m"), copies=2, list_len=16, table_len=8, log_buckets=10, member_lists=True, seed=5)
    with pytest.raises(AssertionError):
        check_exact_lists(str(tmp_path / "m"), X)


@pytest.mark.parametrize("lists", ["member_lists", "exact_lists"])
def test_oracle_build_files_do_not_depend_on_threads(tmp_path, lists):
    """The CPU builder splits its copies and table rows over threads: one thread and three threads over seven
    copies (uneven ranges) write byte-identical files."""
    X, _ = clustered(n=1200, m=10, d=32, clusters=10, seed=4)
    kw = dict(copies=7, list_len=16, table_len=12, log_buckets=10, min_cell=2, seed=3, **{lists: True})
    O.build(X, str(tmp_path / "one"), threads=1, **kw)
    O.build(X, str(tmp_path / "three"), threads=3, **kw)
    names = sorted(os.listdir(tmp_path / "one"))
    assert names == sorted(os.listdir(tmp_path / "three")) and "lists.npy" in names and "table.npy" in names
    for name in names:
        assert (tmp_path / "one" / name).read_bytes() == (tmp_path / "three" / name).read_bytes(), name


@pytest.mark.parametrize("n,m,k,d", [(50, 37, 70, 8), (1000, 33, 17, 5), (2000, 100, 64, 128), (16, 1, 16, 1)])
def test_bruteforce_matches_a_sort_of_all_distances(n, m, k, d):
    """The brute force (16 queries a pass, heaps of the k smallest) equals a lexicographic sort of all (distance,
    id) pairs: integer rows (exact fp64 sums, many ties broken by id), fewer rows than k (padded with -1 and inf),
    query counts that are not multiples of 16."""
    g = np.random.default_rng(n + m)
    X = g.integers(-2, 3, (n, d)).astype(np.float32)
    Q = g.integers(-2, 3, (m, d)).astype(np.float32)
    D, I = O.bruteforce(X, Q, k, threads=3)
    d2 = ((Q[:, None, :].astype(np.float64) - X[None, :, :]) ** 2).sum(-1)
    kk = min(k, n)
    for r in range(m):
        order = np.lexsort((np.arange(n), d2[r]))[:kk]
        assert (I[r, :kk] == order).all() and (D[r, :kk] == d2[r, order].astype(np.float32)).all()
        assert (I[r, kk:] == -1).all() and np.isinf(D[r, kk:]).all()
