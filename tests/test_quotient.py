"""The float-reciprocal quotient of the probe and gather kernels, checked exactly on the CPU in IEEE fp32 (numpy):
probe_kernel takes a work item's copy as item / m and collect_candidates an entry's segment as i / len by

    q = (int) (((float) i + 0.5f) * (1.f / (float) d))          for 0 <= i < 2^22, d >= 1

(the kernels divide in integers for larger i).  Both sides of the check are the same IEEE operations: the
int-to-float conversion is exact below 2^24, 1.f / d and the product are correctly rounded (HIP's default fp32
division; the kernels are built with -ffp-contract=off, and (a + b) * c has no fused form), and (int) truncates.

The check is exhaustive.  For a fixed d the computed value is non-decreasing in i (a correctly rounded sum and
product with positive operands are monotone), so q is wrong for some i in [k d, (k + 1) d) only if it is wrong at
i = k d or at i = (k + 1) d - 1.  Those two boundaries are tested for every d in [1, 2^22) and every k with
k d < 2^22: about 130 million cases."""

import numpy as np

LIM = 1 << 22


def quotient(i, d, half=np.float32(0.5)):
    """The kernels' quotient in fp32: trunc((float(i) + half) * fl(1 / d)); i, d int64 arrays."""
    inv = np.float32(1.0) / d.astype(np.float32)
    return ((i.astype(np.float32) + half) * inv).astype(np.int64)


def boundary_mismatches(half=np.float32(0.5), dmax=LIM):
    """Divisors d < dmax for which the quotient differs from i // d at a boundary i = k d - 1 or k d below 2^22."""
    bad = set()
    small = min(dmax, 2048)
    for d in range(1, small):  # many quotients per divisor: vectorized over k
        k = np.arange(1, (LIM - 1) // d + 1, dtype=np.int64)
        dd = np.full(1, d, np.int64)
        for i in (k * d - 1, k * d):
            if (quotient(i, dd, half) != i // d).any():
                bad.add(d)
    d = np.arange(small, dmax, dtype=np.int64)  # few quotients per divisor: vectorized over d, ascending
    for k in range(1, (LIM - 1) // small + 1):
        dk = d[: np.searchsorted(d, (LIM - 1) // k, side="right")]  # k d < 2^22
        if len(dk) == 0:
            break
        for i in (k * dk - 1, k * dk):
            w = quotient(i, dk, half) != i // dk
            if w.any():
                bad.update(dk[w].tolist())
    return bad


def test_reciprocal_quotient_is_exact_for_every_divisor():
    assert boundary_mismatches() == set()


def test_quotient_check_catches_the_form_without_the_half():
    """Planted mistake: trunc(i * fl(1 / d)) is one low at i = d for divisors whose reciprocal rounds down (41,
    47, 55, ...), the kind of error that would index one segment or one query past the right one."""
    bad = boundary_mismatches(half=np.float32(0.0), dmax=4096)
    assert {41, 47, 55, 61} <= bad
    assert (quotient(np.array([41]), np.array([41]), np.float32(0.0)) == 0).all()
