"""cx_qcsr_head_order (qcsr_exec.hip) on host arrays, checked from outside by brute force
with exact rational arithmetic: each decoded value fma(code, scale, offset) is computed as a
rational and rounded once to float32 (the reference codec's one rounding,
include/Cellerator/quantized/access.cuh:81-91), then

* every head gene decodes exactly in the matrix-core head under the exponent the layout
  gives the head (k = 14 - floor(log2 B), B the head's largest decoded magnitude, plus the
  largest |row offset| under that policy): each 2^k x is an integer multiple of 2^-14 below
  2^15 and the scaled metadata stays a normal float -- the condition under which the three
  fp16 parts carry the value exactly;
* no gene left out of the head that is stored more often than some head gene could join it:
  the head plus that gene is not exact under its own exponent (counts are distinct here);
* the order is the head genes by popularity, then every other gene by popularity;
* wide-range, near-zero, NaN, infinite and subnormal-metadata genes stay out; off-grid row
  offsets leave no head; 8-bit codes with zero offsets and arbitrary scales leave none either.

No GPU is needed: the entry point is host code."""
from __future__ import annotations

import ctypes as C
import math
from fractions import Fraction

import numpy as np
import pytest

PER_GENE, ROW_OFFSET, PAIRS = 1, 2, 3


def _lib():
    from cellerator_amd import _native as N
    try:
        return N.engine()
    except ImportError as e:  # pragma: no cover - the build step makes it
        pytest.skip(str(e))


def head_order(counts, bits, policy, scales, offsets=None, row_offsets=None, head=1024):
    lib = _lib()
    cols = len(counts)
    counts = np.ascontiguousarray(counts, np.uint32)
    perm = np.empty(cols, np.uint32)
    inv = np.empty(cols, np.uint32)
    h = C.c_uint32()

    def ptr(a):
        return None if a is None else np.ascontiguousarray(a, np.float32).ctypes.data

    keep = [np.ascontiguousarray(a, np.float32) if a is not None else None for a in (scales, offsets, row_offsets)]
    st = lib.cx_qcsr_head_order(counts.ctypes.data, cols, bits, policy, ptr(keep[0]), ptr(keep[1]), ptr(keep[2]),
                                0 if row_offsets is None else len(row_offsets), head, perm.ctypes.data,
                                inv.ctypes.data, C.byref(h))
    assert st == 0, lib.cx_last_error().decode()
    assert np.array_equal(inv[perm], np.arange(cols))
    return perm, int(h.value)


def _parts(x) -> tuple[int, int]:
    """A finite float32 as an exact m * 2^e (m an integer)."""
    m, e = math.frexp(float(np.float32(x)))
    return int(m * (1 << 24)), e - 24


def fma32(c: int, s, o) -> tuple[int, int]:
    """fma(c, s, o) rounded once to float32 (ties to even), exactly: (m, e) with value m 2^e.
    The exact sum is an integer times 2^min(es, eo); it is rounded to 24 significant bits
    (fewer below 2^-126)."""
    ms, es = _parts(s)
    mo, eo = _parts(o)
    base = min(es, eo)
    n = ((c * ms) << (es - base)) + (mo << (eo - base))
    if n == 0:
        return 0, 0
    sign, a = (-1 if n < 0 else 1), abs(n)
    top = base + a.bit_length() - 1
    q = max(top - 23, -149)
    shift = q - base
    if shift > 0:
        fl, rem = a >> shift, a & ((1 << shift) - 1)
        half = 1 << (shift - 1)
        if rem > half or (rem == half and fl & 1):
            fl += 1
        a, base = fl, q
    return sign * a, base


def v2(m: int, e: int) -> int:
    """2-adic valuation of the nonzero m 2^e."""
    return (m & -m).bit_length() - 1 + e


def as_fraction(m: int, e: int) -> Fraction:
    return Fraction(m) * Fraction(2) ** e


def layout_exp(total: float) -> int:
    if total == 0.0:
        return 0
    return int(max(-100, min(100, 14 - int(np.floor(np.log2(np.float64(total)))))))


def floor_log2(q: Fraction) -> int:
    e = q.numerator.bit_length() - q.denominator.bit_length()
    return e - 1 if Fraction(2) ** e > q else e


class Gene:
    """A per-gene-policy gene's decoded values (exact), its bound as the layout computes it
    (float32), and from them the smallest exponent k with every 2^k x on the 2^-14 grid and
    the scaled metadata normal (need) and its largest |x| (under 2^(15-k) for the split)."""

    def __init__(self, s, o, qmax):
        self.s, self.o = np.float32(s), np.float32(o)
        self.finite = bool(np.isfinite(self.s) and np.isfinite(self.o))
        if not self.finite:
            return
        values = [fma32(c, self.s, self.o) for c in range(qmax + 1)]
        self.finite = all(m == 0 or abs(m).bit_length() + e <= 128 for m, e in values)
        if not self.finite:
            return
        self.bound = float(max(abs(self.o), np.float32(abs(float(as_fraction(*values[qmax]))))))
        self.maxabs = max(abs(as_fraction(m, e)) for m, e in values)
        need = [-14 - v2(m, e) for m, e in values if m != 0]
        need += [-126 - floor_log2(abs(Fraction(float(x)))) for x in (self.s, self.o) if x != 0]
        self.need = max(need, default=-(10 ** 9))

    def exact(self, k: int) -> bool:
        return self.finite and k >= self.need and self.maxabs * Fraction(2) ** k < 2 ** 15


def set_exact(genes, ids) -> bool:
    if not all(genes[g].finite for g in ids):
        return False
    bound = max((genes[g].bound for g in ids), default=0.0)
    if not np.isfinite(bound) or bound >= 2.0 ** 115:
        return False
    k = layout_exp(bound)
    return all(genes[g].exact(k) for g in ids)


class _Lazy(dict):
    def __init__(self, make):
        super().__init__()
        self.make = make

    def __missing__(self, g):
        self[g] = v = self.make(g)
        return v


def _check_per_gene(counts, bits, s, o, head, expect_head=None):
    perm, h = head_order(counts, bits, PER_GENE, s, o, head=head)
    qmax = (1 << bits) - 1
    genes = _Lazy(lambda g: Gene(s[g], o[g], qmax))
    if expect_head is not None:
        assert h == expect_head
    popular = np.argsort(-counts.astype(np.int64), kind="stable")
    in_head = np.zeros(len(counts), bool)
    in_head[perm[:h]] = True
    # the order: head genes by popularity, then the rest by popularity
    assert np.array_equal(perm[:h], popular[in_head[popular]])
    assert np.array_equal(perm[h:], popular[~in_head[popular]])
    # the head is exact under the layout's exponent
    assert set_exact(genes, perm[:h].tolist())
    # no left-out gene stored more often than the head's least stored gene could join
    if h:
        floor = counts[perm[h - 1]]
        for g in np.nonzero(~in_head & (counts > floor))[0]:
            assert not set_exact(genes, perm[:h].tolist() + [int(g)]), int(g)
    return perm, h, genes


def _friendly(rng, cols, bits):
    """Decoded values 0.5 .. 8.5 whatever the width: the head carries all of them."""
    qmax = (1 << bits) - 1
    return (rng.uniform(0.05, 0.5, cols) * 15.0 / qmax).astype(np.float32), rng.uniform(0.5, 1.0, cols).astype(np.float32)


def test_hostile_genes_leave_the_head():
    rng = np.random.default_rng(1)
    cols = 2300
    counts = rng.permutation(np.arange(10, 10 + cols)).astype(np.uint32)  # distinct
    s, o = _friendly(rng, cols, 4)
    popular = np.argsort(-counts.astype(np.int64), kind="stable")
    hostile = {
        int(popular[0]): (1000.0, 0.5),       # wide range: would drop every other gene off the grid
        int(popular[1]): (0.01, 0.01),        # values near zero: deep low bits
        int(popular[2]): (np.nan, 0.5),
        int(popular[5]): (0.1, np.inf),
        int(popular[7]): (1e-40, 0.7),        # subnormal scale (a fine gene otherwise)
        int(popular[9]): (0.03, -0.2),        # values crossing zero
    }
    for g, (sg, og) in hostile.items():
        s[g], o[g] = np.float32(sg), np.float32(og)
    perm, h, genes = _check_per_gene(counts, 4, s, o, 2048, expect_head=2048)
    head = set(perm[:h].tolist())
    for g in hostile:
        if g == int(popular[7]):
            continue  # fma(c, 1e-40, 0.7) rounds to 0.7: exact whatever the scale; kept or not, brute force decides
        assert g not in head
    # the wide gene alone would fit its own head, but not beside the others
    assert genes[int(popular[0])].exact(layout_exp(genes[int(popular[0])].bound))


@pytest.mark.parametrize("bits", [1, 2, 8])
def test_other_widths_and_a_mixed_population(bits):
    rng = np.random.default_rng(10 + bits)
    cols = 1200
    counts = rng.permutation(np.arange(1, cols + 1)).astype(np.uint32)
    s, o = _friendly(rng, cols, bits)
    bad = rng.random(cols) < 0.1
    s[bad] = rng.uniform(0.05, 0.5, int(bad.sum())).astype(np.float32)
    o[bad] = rng.uniform(-0.5, 1.0, int(bad.sum())).astype(np.float32)
    _check_per_gene(counts, bits, s, o, 1024, expect_head=1024)


def test_pairs_equal_separate_arrays():
    rng = np.random.default_rng(3)
    cols = 1300
    counts = rng.integers(0, 50, cols).astype(np.uint32)
    s, o = _friendly(rng, cols, 4)
    s[::7] = np.float32(0.02)
    o[::7] = np.float32(-0.1)
    a = head_order(counts, 4, PER_GENE, s, o, head=1024)
    b = head_order(counts, 4, PAIRS, np.stack([s, o], 1).ravel(), head=1024)
    assert a[1] == b[1] == 1024 and np.array_equal(a[0], b[0])


def test_eight_bit_zero_offsets_leave_no_head_and_log_like_ones_a_full_one():
    """8-bit codes with zero offsets and arbitrary scales: 2^k s has about 2^6 magnitude and
    24 significant bits, off the 2^-14 grid unless its last 3 bits are zero, so no 1,024 genes
    fit (a head of 0 keeps the popularity order). Offsets of at least 1/64 of the gene's
    largest value (log-normalised counts quantized from their smallest stored value) fit."""
    rng = np.random.default_rng(4)
    cols = 1200
    counts = rng.permutation(np.arange(cols)).astype(np.uint32)
    s = rng.uniform(0.001, 0.05, cols).astype(np.float32)
    perm, h = head_order(counts, 8, PER_GENE, s, np.zeros(cols, np.float32), head=1024)
    assert h == 0 and np.array_equal(perm, np.argsort(-counts.astype(np.int64), kind="stable"))
    lo = np.log1p(rng.integers(1, 3, cols)).astype(np.float32)
    hi = np.log1p(rng.integers(50, 900, cols)).astype(np.float32)
    _check_per_gene(counts, 8, ((hi - lo) / 255).astype(np.float32), lo, 1024, expect_head=1024)


def test_row_offsets():
    """Under the row-offset policy a head needs 2^k s and every 2^k r on the 2^-14 grid: row
    offsets on a 2^-12 grid give a full head (checked value by value over every row), one
    off-grid offset gives none."""
    rng = np.random.default_rng(5)
    cols, rows, bits = 1100, 24, 2
    counts = rng.permutation(np.arange(cols)).astype(np.uint32)
    s = (np.round(rng.uniform(0.25, 2.5, cols) * 4096) / 4096).astype(np.float32)
    s[counts.argmax()] = np.float32(0.0031)  # off the grid under the head's exponent
    r = (np.round(rng.uniform(-1, 1, rows) * 4096) / 4096).astype(np.float32)
    perm, h = head_order(counts, bits, ROW_OFFSET, s, row_offsets=r, head=1024)
    assert h == 1024 and counts.argmax() not in set(perm[:h].tolist())
    qmax = (1 << bits) - 1
    total = np.float32(np.float32(np.max(np.abs(s[perm[:h]])) * np.float32(qmax)) + np.float32(np.max(np.abs(r))))
    k = layout_exp(float(total))
    for g in perm[:h]:
        for c in range(qmax + 1):
            for rr in r:
                m, e = fma32(c, s[g], rr)
                assert m == 0 or (abs(m).bit_length() + e + k <= 15 and v2(m, e) + k >= -14)
    r2 = r.copy()
    r2[3] = np.float32(0.01)
    perm, h = head_order(counts, bits, ROW_OFFSET, s, row_offsets=r2, head=1024)
    assert h == 0


def test_head_width_rules():
    rng = np.random.default_rng(6)
    cols = 2500
    counts = rng.integers(0, 100, cols).astype(np.uint32)
    s, o = _friendly(rng, cols, 4)
    assert head_order(counts, 4, PER_GENE, s, o, head=4096)[1] == 2048  # capped at cols rounded down
    assert head_order(counts, 4, PER_GENE, s, o, head=0)[1] == 0
    lib = _lib()
    perm = np.empty(cols, np.uint32)
    h = C.c_uint32()
    assert lib.cx_qcsr_head_order(counts.ctypes.data, cols, 4, PER_GENE, s.ctypes.data, o.ctypes.data, None, 0,
                                  1000, perm.ctypes.data, perm.ctypes.data, C.byref(h)) == 2  # INVALID_SHAPE
    assert lib.cx_qcsr_head_order(counts.ctypes.data, cols, 3, PER_GENE, s.ctypes.data, o.ctypes.data, None, 0,
                                  1024, perm.ctypes.data, perm.ctypes.data, C.byref(h)) == 3  # UNSUPPORTED


def test_exact_rounding_helper_matches_libm_fmaf():
    """The brute force's exact fma32 equals the C library's fmaf (one correctly rounded
    operation) over random operands with wide exponent spreads, ties, cancellations and
    subnormal results."""
    libm = C.CDLL("libm.so.6")
    libm.fmaf.argtypes = [C.c_float, C.c_float, C.c_float]
    libm.fmaf.restype = C.c_float
    rng = np.random.default_rng(7)
    n = 4000
    s = (rng.standard_normal(n) * 2.0 ** rng.integers(-140, 60, n)).astype(np.float32)
    o = (rng.standard_normal(n) * 2.0 ** rng.integers(-140, 60, n)).astype(np.float32)
    c = rng.integers(0, 256, n)
    o[::5] = -(c[::5] * s[::5].astype(np.float64)).astype(np.float32)  # near cancellation
    cases = list(zip(c.tolist(), s.tolist(), o.tolist()))
    cases += [(1, 1.0, 2.0 ** -24), (1, 1.0, 3 * 2.0 ** -24), (3, 2.0 ** -130, 0.0), (1, 2.0 ** -149, -2.0 ** -149)]
    for ci, si, oi in cases:
        want = np.float32(libm.fmaf(float(ci), si, oi))
        if not np.isfinite(want):
            continue
        m, e = fma32(ci, si, oi)
        assert np.float32(float(as_fraction(m, e))) == want, (ci, si, oi)
