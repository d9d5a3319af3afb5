"""ctypes wrapper of the CPU oracle (oracle/_build/liboctex_oracle.so): TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module; the product
package octex_amd never does.  `load_index` restates the reference loader's host-side conversions
(cpp/src/neighbors/octex/load.cu:215-237 meta parsing, :361-402 list_limit, fp16 ucat/shift, inv_f).
"""

import ctypes as ct
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboctex_oracle.so")

_lib = None


class OrcIndex(ct.Structure):
    _fields_ = [
        ("n", ct.c_int64),
        ("dim", ct.c_int64),
        ("copies", ct.c_int32),
        ("blocks", ct.c_int32),
        ("levels", ct.c_int32),
        ("list_len", ct.c_int32),
        ("log_buckets", ct.c_int32),
        ("sketch_width", ct.c_int32),
        ("table_len", ct.c_int32),
        ("inv_f", ct.c_void_p),
        ("lists", ct.c_void_p),
        ("stride", ct.c_int64),
        ("keys", ct.c_void_p),
        ("mmax", ct.c_int64),
        ("offsets", ct.c_void_p),
        ("T1", ct.c_int64),
        ("base", ct.c_void_p),
        ("ucat", ct.c_void_p),
        ("shift", ct.c_void_p),
        ("mean", ct.c_void_p),
        ("basis", ct.c_void_p),
        ("scale", ct.c_void_p),
        ("sketch", ct.c_void_p),
        ("vectors", ct.c_void_p),
        ("table", ct.c_void_p),
    ]


class OrcSearchParams(ct.Structure):
    _fields_ = [
        (n, ct.c_int32)
        for n in ("read", "starts", "waves", "rerank", "wave_rerank", "batch", "sketch_rank", "final_rerank")
    ]


class OrcTrace(ct.Structure):
    _fields_ = [
        ("seg", ct.c_void_p),
        ("n1", ct.c_void_p),
        ("si1", ct.c_void_p),
        ("sd1", ct.c_void_p),
        ("n2", ct.c_void_p),
        ("si", ct.c_void_p),
        ("sd", ct.c_void_p),
    ]


class OrcBuildParams(ct.Structure):
    _fields_ = [
        ("copies", ct.c_int32),
        ("blocks", ct.c_int32),
        ("pca_dims", ct.c_int32),
        ("spacings", ct.c_void_p),
        ("n_spacings", ct.c_int32),
        ("list_len", ct.c_int32),
        ("min_cell", ct.c_int32),
        ("log_buckets", ct.c_int32),
        ("sketch_width", ct.c_int32),
        ("table_len", ct.c_int32),
        ("reverse_edges", ct.c_int32),
        ("exact_lists", ct.c_int32),
        ("member_lists", ct.c_int32),
        ("seed", ct.c_uint64),
        ("threads", ct.c_int32),
    ]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run __graft_entry__.build())")
        L = ct.CDLL(LIB_PATH)
        L.orc_e8b_hash64.restype = ct.c_int64
        L.orc_e8b_hash64.argtypes = [ct.c_void_p, ct.c_int, ct.c_float]
        L.orc_f2h.restype = ct.c_uint16
        L.orc_f2h.argtypes = [ct.c_float]
        L.orc_h2f.restype = ct.c_float
        L.orc_h2f.argtypes = [ct.c_uint16]
        L.orc_sketch_dist.restype = ct.c_float
        L.orc_exact_dist.restype = ct.c_float
        L.orc_last_error.restype = ct.c_char_p
        for name in ("orc_gather", "orc_select", "orc_pick_starts", "orc_search", "orc_build"):
            getattr(L, name).restype = ct.c_int
        _lib = L
    return _lib


def _p(a):
    return ct.c_void_p(a.ctypes.data) if a is not None else ct.c_void_p(0)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- fp16 / E8 / projections


def f2h(x):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f2h_n(_p(x), ct.c_int64(x.size), _p(out))
    return out


def h2f(h):
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_h2f_n(_p(h), ct.c_int64(h.size), _p(out))
    return out


def e8_batch(y, b, inv_f):
    """E8^b points of y * inv_f and their 64-bit hashes (y [n, 8b] float32)."""
    y = _c(y, np.float32)
    n = y.shape[0]
    p = np.empty_like(y)
    h = np.empty(n, np.int64)
    lib().orc_e8_batch(_p(y), ct.c_int64(n), ct.c_int(b), ct.c_float(inv_f), _p(p), _p(h))
    return p, h


def center(q, mu):
    q, mu = _c(q, np.float32), _c(mu, np.float32)
    m, D = q.shape
    qc = np.empty_like(q)
    qh = np.empty(q.shape, np.uint16)
    lib().orc_center(_p(q), _p(mu), ct.c_int64(m), ct.c_int(D), _p(qc), _p(qh))
    return qc, qh


def project(qh, ucat, shift):
    """Y = fp16(qh @ ucat + shift) from an fp64 sum; also the fp64 values."""
    qh, ucat, shift = _c(qh, np.uint16), _c(ucat, np.uint16), _c(shift, np.uint16)
    m, D = qh.shape
    wdt = ucat.shape[1]
    Y = np.empty((m, wdt), np.uint16)
    Yd = np.empty((m, wdt), np.float64)
    lib().orc_project(_p(qh), ct.c_int64(m), ct.c_int(D), _p(ucat), ct.c_int(wdt), _p(shift), _p(Y), _p(Yd))
    return Y, Yd


def sketch_query(qc, basis):
    qc, basis = _c(qc, np.float32), _c(basis, np.float32)
    m, D = qc.shape
    S = basis.shape[1]
    qs = np.empty((m, S), np.float32)
    lib().orc_sketch_query(_p(qc), ct.c_int64(m), ct.c_int(D), _p(basis), ct.c_int(S), _p(qs))
    return qs


def sketch_dist(code, scale, qs):
    code, scale, qs = _c(code, np.int8), _c(scale, np.float32), _c(qs, np.float32)
    lib().orc_sketch_dist.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_void_p, ct.c_int]
    return float(lib().orc_sketch_dist(_p(code), _p(scale), _p(qs), code.shape[-1]))


def exact_dist(x_h, q):
    x_h, q = _c(x_h, np.uint16), _c(q, np.float32)
    lib().orc_exact_dist.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_int]
    return float(lib().orc_exact_dist(_p(x_h), _p(q), q.shape[-1]))


# ---------------------------------------------------------------- index


def copy_selection(all_copies, parts=0, copies_per_part=0, copies_limit=0):
    """The copies a load places (load.cu:252-263): `parts` equal consecutive ranges, each cut to copies_per_part,
    or the first copies_limit copies of a single part."""
    nparts = max(1, parts)
    sel = []
    for q in range(nparts):
        lo, hi = all_copies * q // nparts, all_copies * (q + 1) // nparts
        if copies_per_part > 0:
            hi = min(hi, lo + copies_per_part)
        if nparts == 1 and copies_limit > 0:
            hi = min(hi, lo + copies_limit)
        sel.extend(range(lo, hi))
    if not sel:
        raise ValueError("octex: a device holds no copies (fewer copies or parts than devices)")
    return np.array(sel, np.int64)


class Index:
    """The arrays of an index directory as the loader places them (one device, replicate)."""

    def __init__(self, path, list_limit=0, copies_limit=0, queries=None, read=32, parts=0, copies_per_part=0):
        """path: an index directory, or a live octex_amd.Index whose arrays are copied to the host.  For a
        live index, `queries` (with the search's `read`) limits the lists copied to the rows these
        queries' probes reach; the other rows read as zeros (an index too large for host memory).
        parts / copies_per_part / copies_limit select copies as the reference's loader does
        (load.cu:252-263)."""
        if not isinstance(path, (str, bytes, os.PathLike)):
            self._from_live(path, queries, read)
            return
        with open(os.path.join(path, "meta.json")) as f:
            meta = json.load(f)
        if int(meta.get("format", 1)) != 1:
            raise ValueError("octex: unknown index format")
        files = meta.get("files", {})

        def load(name):
            p = files.get(name, os.path.join(path, name + ".npy"))
            if not os.path.isabs(p):
                p = os.path.join(path, p)
            return np.load(p, mmap_mode="r")

        self.meta = meta
        self.n, self.dim = int(meta["n"]), int(meta["dim"])
        all_copies = int(meta["copies"])
        self.blocks = int(meta.get("blocks", 4))
        list_len = int(meta["list_len"])
        self.log_buckets = int(meta.get("log_buckets", 20))
        self.sketch_width = int(meta.get("sketch_width", 0))
        self.table_len = int(meta.get("table_len", 0))
        self.spacings = [float(v) for v in meta["spacings"]]
        L = len(self.spacings)
        sel = copy_selection(all_copies, parts, copies_per_part, copies_limit)
        C = len(sel)
        self.copies = C
        w = 8 * self.blocks
        ll = min(list_limit, list_len) if list_limit > 0 else list_len
        lists = np.asarray(load("lists")[sel])
        if ll != list_len:  # load.cu:361-379
            rows = lists.shape[1] // list_len
            lists = np.ascontiguousarray(lists[:, : rows * list_len].reshape(C, rows, list_len)[:, :, :ll].reshape(C, -1))
        self.list_len = ll
        self.lists = _c(lists, np.int32)
        self.keys = _c(load("keys")[sel], np.int64)
        self.offsets = _c(load("offsets")[sel], np.int32)
        self.base = _c(load("base")[sel], np.int32)
        proj = np.asarray(load("proj")[sel], np.float32)  # [C, D, w]
        self.ucat = f2h(np.ascontiguousarray(proj.transpose(1, 0, 2)).reshape(self.dim, C * w))  # load.cu:385-393
        self.shift = f2h(np.asarray(load("shift")[sel], np.float32).reshape(-1))
        self.inv_f = np.array([np.float32(1.0 / f) for f in self.spacings], np.float32)  # load.cu:397-399: the JSON double
        self.mean = _c(load("mean"), np.float32)
        self.basis = _c(load("sketch_basis"), np.float32)
        self.scale = _c(load("sketch_scale"), np.float32)
        self.sketch = _c(load("sketch"), np.int8)
        self.vectors = _c(load("vectors"), np.float16).view(np.uint16)
        self.table = _c(load("table"), np.int32) if self.table_len > 0 else None
        assert self.keys.shape[1] == L and proj.shape[2] == w, "octex: bad shapes"
        self._struct(L)

    @classmethod
    def from_arrays(cls, *, inv_f, offsets, keys, base, list_len, blocks, lists=None, n=0, dim=8):
        """An index of the probe's arrays only (keys [C, L, mmax], offsets [C, L, 2^logT + 1], base [C, L],
        inv_f [L]), for hand-built cell tables such as the reference's probe test (test_search.cu:86-170);
        the other arrays are empty placeholders."""
        self = cls.__new__(cls)
        self.keys = _c(keys, np.int64)
        self.offsets = _c(offsets, np.int32)
        self.base = _c(base, np.int32)
        self.inv_f = _c(inv_f, np.float32)
        C, L = self.keys.shape[:2]
        T1 = self.offsets.shape[2]
        assert self.offsets.shape[:2] == (C, L) and self.base.shape == (C, L) and self.inv_f.shape == (L,)
        assert T1 >= 2 and (T1 - 1) & (T1 - 2) == 0, "offsets rows hold 2^logT + 1 entries"
        self.n, self.dim, self.copies, self.blocks, self.list_len = n, dim, C, blocks, list_len
        self.log_buckets = (T1 - 1).bit_length() - 1
        self.sketch_width, self.table_len = 0, 0
        self.spacings = [float(1.0 / v) for v in self.inv_f]
        self.lists = _c(lists if lists is not None else np.zeros((C, 1)), np.int32)
        w = 8 * blocks
        self.ucat = np.zeros((dim, C * w), np.uint16)
        self.shift = np.zeros(C * w, np.uint16)
        self.mean = np.zeros(dim, np.float32)
        self.basis = np.zeros((dim, 1), np.float32)
        self.scale = np.zeros(1, np.float32)
        self.sketch = np.zeros((1, 1), np.int8)
        self.vectors = np.zeros((1, dim), np.uint16)
        self.table = None
        self.meta = {}
        self._struct(L)
        return self

    @classmethod
    def from_vectors(cls, vectors):
        """An index holding only fp16 vectors [N, D] (uint16 bits): the input of the exact reranks
        (rerank_keep, final_rerank), for rule tests such as test_search.cu:293-412; no cell tables."""
        vectors = _c(vectors, np.uint16)
        n, dim = vectors.shape
        self = cls.from_arrays(inv_f=np.ones(1, np.float32), offsets=np.zeros((1, 1, 3), np.int32),
                               keys=np.zeros((1, 1, 1), np.int64), base=np.zeros((1, 1), np.int32), list_len=1,
                               blocks=1, n=n, dim=dim)
        self.vectors = vectors
        self._struct(1)
        return self

    def _from_live(self, live, queries=None, read=32):
        """The arrays of a loaded or built octex_amd index, copied to the host (the same index the GPU searches)."""
        meta = live.array("meta", np.int64)
        n, dim, C, blocks, L, list_len, log_buckets, S, table_len, mmax, T1, pitch = (int(v) for v in meta)
        self.n, self.dim, self.copies, self.blocks, self.list_len = n, dim, C, blocks, list_len
        self.log_buckets, self.sketch_width, self.table_len = log_buckets, S, table_len
        self.spacings = [float(v) for v in live.array("spacings", np.float32)]
        w = 8 * blocks
        if queries is None:
            per = [live.array("lists", np.int32, copy=c) for c in range(C)]
            stride = max(len(p) for p in per)
            self.lists = np.zeros((C, stride), np.int32)
            for c, p in enumerate(per):
                self.lists[c, : len(p)] = p
            del per
        else:  # zero-filled and lazily committed: only the rows copied below take host memory
            stride = max(live.array_size("lists", copy=c) for c in range(C)) // 4
            self.lists = np.zeros((C, stride), np.int32)
        self.keys = live.array("keys", np.int64).reshape(C, L, mmax)
        self.offsets = live.array("offsets", np.int32).reshape(C, L, T1)
        self.base = live.array("base", np.int32).reshape(C, L)
        ucatT = live.array("ucatT", np.uint16).reshape(C * w, dim)
        self.ucat = np.ascontiguousarray(ucatT.T)
        self.shift = live.array("shift", np.uint16)
        self.inv_f = live.array("inv_f", np.float32)
        self.mean = live.array("mean", np.float32)
        self.basis = live.array("basis", np.float32).reshape(dim, S)
        self.scale = live.array("scale", np.float32)
        self.sketch = np.ascontiguousarray(live.array("sketch", np.int8).reshape(n, pitch)[:, :S])
        self.vectors = live.array("vectors", np.uint16).reshape(n, dim)
        self.table = live.array("table", np.int32).reshape(n, table_len) if table_len > 0 else None
        self.meta = {}
        self._struct(L)
        if queries is not None:  # the list rows of these queries' probes (the segments the search reads)
            _, qh = center(queries, self.mean)
            Y, _ = project(qh, self.ucat, self.shift)
            seg = probe(self, Y, read)
            for c in range(C):
                sc = seg[:, c, :]
                sc = sc[sc[:, 1] > 0]
                if len(sc) == 0:
                    continue
                ln = int(sc[:, 1].max())  # every segment reads min(read, list_len) entries
                starts = np.unique(sc[:, 0]).astype(np.int64)
                rows = live.array_ranges("lists", np.int32, starts, ln, copy=c)
                self.lists[c, starts[:, None] + np.arange(ln)[None, :]] = rows

    def _struct(self, L):
        s = OrcIndex()
        s.n, s.dim = self.n, self.dim
        s.copies, s.blocks, s.levels, s.list_len = self.copies, self.blocks, L, self.list_len
        s.log_buckets, s.sketch_width, s.table_len = self.log_buckets, self.sketch_width, self.table_len
        s.inv_f = self.inv_f.ctypes.data
        s.lists, s.stride = self.lists.ctypes.data, self.lists.shape[1]
        s.keys, s.mmax = self.keys.ctypes.data, self.keys.shape[2]
        s.offsets, s.T1 = self.offsets.ctypes.data, self.offsets.shape[2]
        s.base = self.base.ctypes.data
        s.ucat, s.shift = self.ucat.ctypes.data, self.shift.ctypes.data
        s.mean, s.basis, s.scale = self.mean.ctypes.data, self.basis.ctypes.data, self.scale.ctypes.data
        s.sketch, s.vectors = self.sketch.ctypes.data, self.vectors.ctypes.data
        s.table = self.table.ctypes.data if self.table is not None else None
        self.c = s

    @property
    def width(self):
        return 8 * self.blocks


def _sp(read=32, starts=128, waves=2, rerank=128, wave_rerank=128, batch=10000, sketch_rank=False, final_rerank=32):
    p = OrcSearchParams()
    p.read, p.starts, p.waves, p.rerank, p.wave_rerank = read, starts, waves, rerank, wave_rerank
    p.batch, p.sketch_rank, p.final_rerank = batch, int(bool(sketch_rank)), final_rerank
    return p


def search(ix, q, k=10, Y=None, qs=None, threads=8, trace=False, **params):
    """The oracle search; returns (D, I) and, with trace=True, a dict of per-query intermediates."""
    q = _c(q, np.float32)
    nq = q.shape[0]
    sp = _sp(**params)
    KO = max(sp.starts, k)
    I = np.empty((nq, k), np.int64)
    D = np.empty((nq, k), np.float32)
    if Y is not None:
        Y = _c(Y, np.uint16)
    if qs is not None:
        qs = _c(qs, np.float32)
    tr = None
    out = None
    if trace:
        out = dict(
            seg=np.zeros((nq, ix.copies, 2), np.int32),
            n1=np.zeros(nq, np.int32),
            si1=np.zeros((nq, KO), np.int64),
            sd1=np.zeros((nq, KO), np.float32),
            n2=np.zeros((nq, max(1, sp.waves)), np.int32),
            si=np.zeros((nq, KO), np.int64),
            sd=np.zeros((nq, KO), np.float32),
        )
        tr = OrcTrace(*[out[f].ctypes.data for f, _ in OrcTrace._fields_])
    rc = lib().orc_search(
        ct.byref(ix.c), ct.byref(sp), _p(q), ct.c_int64(nq), ct.c_int(k), _p(Y), _p(qs), _p(I), _p(D),
        ct.c_int(threads), ct.byref(tr) if tr is not None else None,
    )
    if rc != 0:
        raise ValueError(lib().orc_last_error().decode())
    return (D, I, out) if trace else (D, I)


def probe(ix, Y, read):
    Y = _c(Y, np.uint16)
    m = Y.shape[0]
    seg = np.empty((m, ix.copies, 2), np.int32)
    lib().orc_probe(ct.byref(ix.c), _p(Y), ct.c_int64(m), ct.c_int(min(read, ix.list_len)), _p(seg))
    return seg


def gather(ix, seg, qs, rows=False, cap=1 << 15):
    """Distinct candidates of one query's segments [nseg, 2], ascending, with sketch scores."""
    seg, qs = _c(seg, np.int32), _c(qs, np.float32)
    cand = np.empty(cap, np.int32)
    dist = np.empty(cap, np.float32)
    n = lib().orc_gather(ct.byref(ix.c), _p(seg), ct.c_int(seg.shape[0]), ct.c_int(int(rows)), _p(qs), _p(cand), _p(dist), ct.c_int(cap))
    return cand[:n].copy(), dist[:n].copy()


def select(cand, dist, R):
    cand, dist = _c(cand, np.int32), _c(dist, np.float32)
    sid = np.empty(max(1, R), np.int32)
    sd = np.empty(max(1, R), np.float32)
    n = lib().orc_select(_p(cand), _p(dist), ct.c_int(len(cand)), ct.c_int(R), _p(sid), _p(sd))
    return sid[:n].copy(), sd[:n].copy()


def merge_keep(si, sd, new_ids, new_d, fresh):
    si, sd = _c(si, np.int64).copy(), _c(sd, np.float32).copy()
    new_ids, new_d = _c(new_ids, np.int32), _c(new_d, np.float32)
    lib().orc_merge_keep(_p(si), _p(sd), ct.c_int(len(si)), ct.c_int(int(fresh)), _p(new_ids), _p(new_d), ct.c_int(len(new_ids)))
    return si, sd


def rerank_keep(ix, cand, dist, q, R, si, sd, fresh):
    cand, dist, q = _c(cand, np.int32), _c(dist, np.float32), _c(q, np.float32)
    si, sd = _c(si, np.int64).copy(), _c(sd, np.float32).copy()
    lib().orc_rerank_keep(ct.byref(ix.c), _p(cand), _p(dist), ct.c_int(len(cand)), _p(q), ct.c_int(R), ct.c_int(len(si)), ct.c_int(int(fresh)), _p(si), _p(sd))
    return si, sd


def sketch_keep(cand, dist, si, sd, fresh):
    cand, dist = _c(cand, np.int32), _c(dist, np.float32)
    si, sd = _c(si, np.int64).copy(), _c(sd, np.float32).copy()
    lib().orc_sketch_keep(_p(cand), _p(dist), ct.c_int(len(cand)), ct.c_int(len(si)), ct.c_int(int(fresh)), _p(si), _p(sd))
    return si, sd


def pick_starts(si, done, off, S, rowlen):
    si = _c(si, np.int64)
    done = _c(done, np.int64).copy()
    seg2 = np.empty((S, 2), np.int32)
    lib().orc_pick_starts(_p(si), ct.c_int(len(si)), _p(done), ct.c_int(off), ct.c_int(S), ct.c_int(rowlen), _p(seg2))
    return done, seg2


def final_rerank(ix, si, R, q, k):
    si, q = _c(si, np.int64), _c(q, np.float32)
    bi = np.empty(k, np.int64)
    bd = np.empty(k, np.float32)
    lib().orc_final_rerank(ct.byref(ix.c), _p(si), ct.c_int(R), _p(q), ct.c_int(k), _p(bi), _p(bd))
    return bi, bd


def bruteforce(x, q, k, threads=8):
    x, q = _c(x, np.float32), _c(q, np.float32)
    I = np.empty((q.shape[0], k), np.int64)
    D = np.empty((q.shape[0], k), np.float32)
    lib().orc_bruteforce(_p(x), ct.c_int64(x.shape[0]), _p(q), ct.c_int64(q.shape[0]), ct.c_int64(x.shape[1]), ct.c_int(k), _p(I), _p(D), ct.c_int(threads))
    return D, I


def build(x, path, copies=8, blocks=4, pca_dims=64, spacings=None, list_len=64, min_cell=1, log_buckets=20,
          sketch_width=0, table_len=64, reverse_edges=True, exact_lists=False, member_lists=False, seed=0, threads=8):
    """The oracle's small CPU builder: writes a format-1 index directory at `path` (copies and table rows over
    `threads` host threads; the files do not depend on the count)."""
    x = _c(x, np.float32)
    sp = np.array(spacings if spacings is not None else [2.0, 2.5, 3.2, 4.0, 5.0], np.float32)
    p = OrcBuildParams()
    p.copies, p.blocks, p.pca_dims = copies, blocks, pca_dims
    p.spacings, p.n_spacings = sp.ctypes.data, len(sp)
    p.list_len, p.min_cell, p.log_buckets, p.sketch_width, p.table_len = list_len, min_cell, log_buckets, sketch_width, table_len
    p.reverse_edges, p.exact_lists, p.member_lists, p.seed = int(reverse_edges), int(exact_lists), int(member_lists), seed
    p.threads = threads
    os.makedirs(path, exist_ok=True)
    rc = lib().orc_build(_p(x), ct.c_int64(x.shape[0]), ct.c_int64(x.shape[1]), ct.byref(p), os.fsencode(path))
    if rc != 0:
        raise ValueError(lib().orc_last_error().decode())
    return path
