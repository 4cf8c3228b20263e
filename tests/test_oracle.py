"""CPU tests that pin the oracle: the reference's known-answer fixtures, closed forms,
brute force and planted errors. No GPU."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from tests.helpers import random_csr

GOLDEN = Path(__file__).resolve().parent / "golden"


# ------------------------------------------------------------------ codec
# Fixture of tests/quantized_matrix_test.cu:15-28 (4 x 8 CSR, per-gene scales/offsets,
# row offsets) with codes (index + row + gene) % (max + 1) (:78-96).
KAT_ROW_PTR = np.array([0, 4, 7, 10, 12], np.int32)
KAT_COLS = np.array([0, 2, 5, 7, 1, 4, 6, 0, 3, 7, 2, 5], np.int32)
KAT_SCALES = np.array([0.25, 0.50, 0.75, 1.00, 1.25, 1.50, 1.75, 2.00], np.float32)
KAT_OFFSETS = np.array([0.0, 0.5, -0.5, 1.0, -1.0, 0.25, -0.25, 2.0], np.float32)
KAT_ROW_OFFSETS = np.array([0.0, 1.5, -0.75, 0.25], np.float32)


def kat_codes(bits: int) -> np.ndarray:
    qmax = (1 << bits) - 1
    rows = np.repeat(np.arange(4), np.diff(KAT_ROW_PTR))
    return (np.arange(len(KAT_COLS)) + rows + KAT_COLS) % (qmax + 1)


def numpy_pack(bits: int, row_ptr: np.ndarray, codes: np.ndarray) -> np.ndarray:
    """Independent vectorised statement of the packed layout: code i of a row sits in
    byte i // (8/bits) of that row at bit offset (i % (8/bits)) * bits; rows start on
    byte boundaries with no padding (format.cuh:39-48, layout.cuh:106-129)."""
    cpb = 8 // bits
    counts = np.diff(row_ptr)
    row_bytes = (counts + cpb - 1) // cpb
    starts = np.concatenate([[0], np.cumsum(row_bytes)])
    out = np.zeros(int(starts[-1]), np.uint8)
    rows = np.repeat(np.arange(len(counts)), counts)
    local = np.arange(len(codes)) - row_ptr[rows]
    np.bitwise_or.at(out, starts[rows] + local // cpb,
                     (codes.astype(np.uint8) << ((local % cpb) * bits)).astype(np.uint8))
    return out


def exact_fma_f32(code, scale, offset):
    """Correctly rounded fma in float32, via an exact 64-bit-mantissa sum."""
    s = np.longdouble(code) * np.longdouble(scale) + np.longdouble(offset)
    return np.float32(s)


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("policy", [1, 2])
def test_codec_reference_kat(oracle, bits, policy):
    codes = kat_codes(bits)
    rows = np.repeat(np.arange(4), np.diff(KAT_ROW_PTR))
    off = KAT_OFFSETS[KAT_COLS] if policy == 1 else KAT_ROW_OFFSETS[rows]
    values = (off + KAT_SCALES[KAT_COLS] * codes.astype(np.float32)).astype(np.float32)
    prp = oracle.build_packed_row_ptr(bits, KAT_ROW_PTR)
    cpb = 8 // bits
    assert np.array_equal(np.diff(prp), (np.diff(KAT_ROW_PTR) + cpb - 1) // cpb)
    packed = oracle.pack_csr(bits, policy, KAT_ROW_PTR, prp, KAT_COLS, values, KAT_SCALES,
                             KAT_OFFSETS if policy == 1 else None,
                             KAT_ROW_OFFSETS if policy == 2 else None)
    assert np.array_equal(packed, numpy_pack(bits, KAT_ROW_PTR, codes))
    for r in range(4):
        for i in range(KAT_ROW_PTR[r], KAT_ROW_PTR[r + 1]):
            got = oracle.unpack_code(bits, packed[prp[r]:], i - KAT_ROW_PTR[r])
            assert got == codes[i]
    decoded = oracle.decode_csr(bits, policy, KAT_ROW_PTR, prp, KAT_COLS, packed, KAT_SCALES,
                                KAT_OFFSETS if policy == 1 else None,
                                KAT_ROW_OFFSETS if policy == 2 else None)
    # the reference's own check (quantized_matrix_test.cu:359-371): round trip to 1e-6
    assert np.max(np.abs(decoded - values)) <= 1e-6
    # and the bit-exact contract: one rounding of code*scale+offset
    exact = np.array([exact_fma_f32(c, KAT_SCALES[g], o) for c, g, o in zip(codes, KAT_COLS, off)])
    assert np.array_equal(decoded.view(np.uint32), exact.view(np.uint32))


def test_codec_golden_file_matches(oracle):
    """tests/golden/codec_kat.json holds the packed bytes of the reference fixture."""
    data = json.loads((GOLDEN / "codec_kat.json").read_text())
    for case in data["cases"]:
        bits, policy = case["bits"], case["policy"]
        codes = kat_codes(bits)
        rows = np.repeat(np.arange(4), np.diff(KAT_ROW_PTR))
        off = KAT_OFFSETS[KAT_COLS] if policy == 1 else KAT_ROW_OFFSETS[rows]
        values = (off + KAT_SCALES[KAT_COLS] * codes.astype(np.float32)).astype(np.float32)
        prp = oracle.build_packed_row_ptr(bits, KAT_ROW_PTR)
        packed = oracle.pack_csr(bits, policy, KAT_ROW_PTR, prp, KAT_COLS, values, KAT_SCALES,
                                 KAT_OFFSETS if policy == 1 else None,
                                 KAT_ROW_OFFSETS if policy == 2 else None)
        assert packed.tolist() == case["packed"]
        assert prp.tolist() == case["packed_row_ptr"]


def test_decode_exhaustive_closed_form(oracle):
    rng = np.random.default_rng(7)
    scales = rng.uniform(1e-6, 4.0, 64).astype(np.float32)
    offsets = rng.uniform(-8.0, 8.0, 64).astype(np.float32)
    for s, o in zip(scales, offsets):
        for code in range(256):
            got = np.float32(oracle.dequantize(code, float(s), float(o)))
            assert got.view(np.uint32) == exact_fma_f32(code, s, o).view(np.uint32)


def test_quantize_rounding_rule(oracle):
    # round half away from zero, clamp to [0, 2^bits-1], scale 0 -> 0 (access.cuh:104-131)
    assert oracle.quantize(8, 2.5, 1.0, 0.0) == 3
    assert oracle.quantize(8, 1.5, 1.0, 0.0) == 2
    assert oracle.quantize(8, 1.49999, 1.0, 0.0) == 1
    assert oracle.quantize(8, -0.5, 1.0, 0.0) == 0
    assert oracle.quantize(4, 100.0, 1.0, 0.0) == 15
    assert oracle.quantize(1, 0.6, 1.0, 0.0) == 1
    assert oracle.quantize(8, 7.0, 0.0, 1.0) == 0
    assert oracle.quantize(8, 1.0, 0.25, 0.5) == 2


def test_packed_row_ptr_odd_rows(oracle):
    row_ptr = np.array([0, 1, 4, 4, 9], np.int32)
    assert oracle.build_packed_row_ptr(4, row_ptr).tolist() == [0, 1, 3, 3, 6]
    assert oracle.build_packed_row_ptr(2, row_ptr).tolist() == [0, 1, 2, 2, 4]
    assert oracle.build_packed_row_ptr(8, row_ptr).tolist() == row_ptr.tolist()


# ------------------------------------------------------------------ referee
def test_referee_kat_bias_relu_and_transpose(oracle):
    """tests/math_referee_foundation_test.cc:61-106: alpha=2, beta=0.5, bias+ReLU."""
    offsets = np.array([0, 2, 4], np.uint64)
    cols = np.array([0, 2, 1, 2], np.uint32)
    vals = np.array([1, 2, 3, 4], np.float32)
    rhs = np.array([1, 2, 3, 4, 5, 6], np.float32).reshape(3, 2)
    prior = np.full((2, 2), 2.0, np.float32)
    bias = np.array([-30.0, 1.0], np.float32)
    out = oracle.spmm_referee(2, 3, 2, offsets, cols, vals, rhs, alpha=2.0, beta=0.5, c0=prior,
                              epilogue=oracle.EPI_BIAS_RELU, bias=bias)
    assert np.allclose(out.ravel(), [0.0, 30.0, 29.0, 74.0], atol=1e-12)
    t_offsets = np.array([0, 1, 2, 4], np.uint64)
    t_cols = np.array([0, 1, 0, 1], np.uint32)
    t_vals = np.array([1, 3, 2, 4], np.float32)
    t_rhs = np.array([1, 3, 5, 2, 4, 6], np.float32).reshape(2, 3)
    out_t = oracle.spmm_referee(2, 3, 2, t_offsets, t_cols, t_vals, t_rhs, transpose_sparse=True,
                                transpose_dense=True, ldb=3, alpha=2.0, beta=0.5, c0=prior,
                                epilogue=oracle.EPI_BIAS_RELU, bias=bias)
    assert np.allclose(out_t.ravel(), [0.0, 30.0, 29.0, 74.0], atol=1e-12)


def test_referee_kat_sparse_ops_fixture(oracle):
    """tests/sparse_ops_runtime_test.cu:140-161,279-297 -> {201,402,430,860,5,10}."""
    offsets = np.array([0, 2, 4, 5], np.uint64)
    cols = np.array([0, 2, 1, 2, 0], np.uint32)
    vals = np.array([1, 2, 3, 4, 5], np.float16)
    rhs = np.array([1, 2, 10, 20, 100, 200], np.float32).reshape(3, 2)
    out = oracle.spmm_referee(3, 3, 2, offsets, cols, vals, rhs)
    assert out.ravel().tolist() == [201.0, 402.0, 430.0, 860.0, 5.0, 10.0]


@pytest.mark.parametrize("epilogue", [0, 1, 2, 3, 4, 5, 6, 7])
def test_referee_brute_force(oracle, epilogue):
    rng = np.random.default_rng(11 + epilogue)
    m, k, n = 37, 53, 19
    row_ptr, cols = random_csr(rng, m, k, 9.0, empty_every=7)
    vals = rng.standard_normal(len(cols)).astype(np.float32)
    rhs = rng.standard_normal((k, n)).astype(np.float32)
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    dense = np.zeros((m, k))
    for r in range(m):
        dense[r, cols[row_ptr[r]:row_ptr[r + 1]]] = vals[row_ptr[r]:row_ptr[r + 1]]
    z = 1.5 * dense @ rhs.astype(np.float64) + 0.25 * c0
    if epilogue in (1, 5, 6, 7):
        z = z + bias
    if epilogue in (2, 5):
        z = np.maximum(z, 0.0)
    if epilogue in (3, 6):
        from scipy.special import erf
        z = 0.5 * z * (1.0 + erf(z / np.sqrt(2.0)))
    if epilogue in (4, 7):
        z = 0.5 * z * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (z + 0.044715 * z ** 3)))
    out = oracle.spmm_referee(m, k, n, row_ptr.astype(np.uint64), cols, vals, rhs, alpha=1.5,
                              beta=0.25, c0=c0, epilogue=epilogue,
                              bias=bias if epilogue in (1, 5, 6, 7) else None)
    assert np.allclose(out, z, rtol=1e-12, atol=1e-12)


def test_qcsr_referee_matches_dense_gemm(oracle):
    from tests.helpers import quantized_fixture
    rng = np.random.default_rng(5)
    for bits in (1, 2, 4, 8):
        for policy in (1, 2):
            fx = quantized_fixture(oracle, rng, 41, 67, 12.0, bits, policy, empty_every=5)
            rhs = (rng.standard_normal((67, 24)) * 0.02).astype(np.float16)
            ref, mag = oracle.qcsr_spmm_referee(bits, policy, 41, 67, fx["row_ptr"],
                                                fx["packed_row_ptr"], fx["col_idx"], fx["packed"],
                                                fx["scales"], fx["offsets"], fx["row_offsets"], rhs)
            values = oracle.decode_csr(bits, policy, fx["row_ptr"], fx["packed_row_ptr"],
                                       fx["col_idx"], fx["packed"], fx["scales"], fx["offsets"],
                                       fx["row_offsets"])
            dense = np.zeros((41, 67))
            for r in range(41):
                s, e = fx["row_ptr"][r], fx["row_ptr"][r + 1]
                dense[r, fx["col_idx"][s:e]] = values[s:e]
            expect = dense @ rhs.astype(np.float64)
            assert np.allclose(ref, expect, rtol=1e-12, atol=1e-14)
            assert np.allclose(mag, np.abs(dense) @ np.abs(rhs.astype(np.float64)), rtol=1e-12)
            mt = oracle.qcsr_spmm_f32_mt(bits, policy, 41, 67, fx["row_ptr"], fx["packed_row_ptr"],
                                         fx["col_idx"], fx["packed"], fx["scales"], fx["offsets"],
                                         fx["row_offsets"], rhs, threads=3)
            cmp = oracle.compare(ref, mt, 1e-4, 1e-4, mag)
            assert cmp["within_tolerance"], cmp


def test_compare_detects_planted_error(oracle):
    rng = np.random.default_rng(3)
    ref = rng.standard_normal(1000)
    mag = np.abs(ref) + 1.0
    cand = ref.astype(np.float32)
    assert oracle.compare(ref, cand, 1e-4, 1e-4, mag)["within_tolerance"]
    bad = cand.copy()
    bad[417] += np.float32(3e-4 * mag[417] + 1e-3)
    res = oracle.compare(ref, bad, 1e-4, 1e-4, mag)
    assert not res["within_tolerance"] and res["mismatch_count"] == 1 and res["worst_index"] == 417
    nan = cand.copy()
    nan[3] = np.nan
    assert oracle.compare(ref, nan, 1e-4, 1e-4, mag)["non_finite_candidate_count"] == 1


# ------------------------------------------------------------------ Blocked-ELL
def test_bell_referee_kat(oracle):
    """Blocked-ELL (block 1, ell_cols 2) of the 3x3 fixture reproduces {201,...,10}
    (tests/sparse_ops_runtime_test.cu:299-358)."""
    idx = np.array([0, 2, 1, 2, 0, 0xFFFFFFFF], np.uint32)
    vals = np.array([1, 2, 3, 4, 5, 0], np.float16)
    rhs = np.array([1, 2, 10, 20, 100, 200], np.float32).reshape(3, 2)
    out, _ = oracle.bell_spmm_referee(3, 3, 1, 2, idx, vals, rhs, value_type=oracle.F16)
    assert out.ravel().tolist() == [201.0, 402.0, 430.0, 860.0, 5.0, 10.0]
    # 8-bit per-gene quantized BELL with unit scales (:366-402)
    codes = np.array([1, 2, 3, 4, 5, 0], np.uint8)
    out8, _ = oracle.bell_spmm_referee(3, 3, 1, 2, idx, None, rhs, bits=8, policy=1,
                                       row_stride_bytes=2, packed=codes,
                                       scales=np.ones(3, np.float32))
    assert out8.ravel().tolist() == [201.0, 402.0, 430.0, 860.0, 5.0, 10.0]
    # 4-bit column-scale/row-offset quantized BELL (:404-470): offsets {0,3,5}
    row_off = np.array([0.0, 3.0, 5.0], np.float32)
    codes4 = np.array([(1 - 0) | ((2 - 0) << 4), (3 - 3) | ((4 - 3) << 4), (5 - 5) | 0], np.uint8)
    out4, _ = oracle.bell_spmm_referee(3, 3, 1, 2, idx, None, rhs, bits=4, policy=2,
                                       row_stride_bytes=1, packed=codes4,
                                       scales=np.ones(3, np.float32), row_offsets=row_off)
    assert out4.ravel().tolist() == [201.0, 402.0, 430.0, 860.0, 5.0, 10.0]


def test_bell_referee_brute_force(oracle):
    rng = np.random.default_rng(21)
    bs, rows, cols, width = 4, 16, 30, 3
    rb = rows // bs
    idx = np.full((rb, width), 0xFFFFFFFF, np.uint32)
    for b in range(rb):
        c = rng.integers(1, width + 1)
        idx[b, :c] = np.sort(rng.choice((cols + bs - 1) // bs, size=c, replace=False))
    vals = (rng.standard_normal((rows, width * bs)) * (rng.random((rows, width * bs)) < 0.4)).astype(np.float32)
    rhs = rng.standard_normal((cols, 7)).astype(np.float32)
    dense = np.zeros((rows, cols))
    for r in range(rows):
        for s in range(width * bs):
            bc = idx[r // bs, s // bs]
            if bc == 0xFFFFFFFF:
                continue
            c = int(bc) * bs + s % bs
            if c < cols:
                dense[r, c] += vals[r, s]
    out, _ = oracle.bell_spmm_referee(rows, cols, bs, width * bs, idx, vals, rhs,
                                      value_type=oracle.F32)
    assert np.allclose(out, dense @ rhs.astype(np.float64), rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- backward

_BWD_ROW_PTR = np.array([0, 2, 4, 5], np.int32)
_BWD_COLS = np.array([0, 2, 1, 2, 0], np.int32)
_BWD_VALUES = np.array([1, 2, 3, 4, 5], np.float16)
_BWD_RHS = np.array([[1, 2], [10, 20], [100, 200]], np.float32)
_BWD_GRAD = np.array([[1, 2], [3, 4], [5, 6]], np.float32)


def test_bwd_values_reference_kat(oracle):
    """tests/sparse_ops_runtime_test.cu:566-582: {5, 500, 110, 1100, 17}."""
    gv = oracle.spmm_bwd_values(_BWD_ROW_PTR, _BWD_COLS, _BWD_GRAD, _BWD_RHS)
    assert gv.tolist() == [5.0, 500.0, 110.0, 1100.0, 17.0]


def test_bwd_rhs_reference_kat(oracle):
    """tests/sparse_ops_runtime_test.cu:584-604: X^T . grad = {26,32, 9,12, 14,20}."""
    g = oracle.spmm_referee(3, 3, 2, _BWD_ROW_PTR, _BWD_COLS, _BWD_VALUES, _BWD_GRAD,
                            transpose_sparse=True)
    assert g.ravel().tolist() == [26.0, 32.0, 9.0, 12.0, 14.0, 20.0]


@pytest.mark.parametrize("rhs_dtype", [np.float32, np.float16])
def test_bwd_values_adjoint_identity(oracle, rhs_dtype):
    """sum_i grad_values[i] x_i = <G, X . W>: the gradient is the adjoint of the forward."""
    from tests.helpers import random_csr
    rng = np.random.default_rng(31)
    rows, cols, n = 70, 90, 13
    row_ptr, col_idx = random_csr(rng, rows, cols, 9.0, empty_every=6)
    x = rng.standard_normal(len(col_idx)).astype(np.float32)
    w = rng.standard_normal((cols, n)).astype(rhs_dtype)
    g = rng.standard_normal((rows, n)).astype(np.float32)
    gv = oracle.spmm_bwd_values(row_ptr, col_idx, g, w)
    y = oracle.spmm_referee(rows, cols, n, row_ptr, col_idx, x, w)
    lhs = float(np.dot(gv, x.astype(np.float64)))
    rhs = float(np.sum(g.astype(np.float64) * y))
    assert abs(lhs - rhs) <= 1e-9 * max(1.0, abs(rhs))
    # and per entry against the dense product G . W^T sampled at the pattern
    dense = g.astype(np.float64) @ w.astype(np.float64).T
    rows_of = np.repeat(np.arange(rows), np.diff(row_ptr))
    assert np.allclose(gv, dense[rows_of, col_idx], rtol=1e-12, atol=1e-12)


def test_digest_logical_dense_properties(oracle):
    """digest_logical_dense (include/Cellerator/compute/math/referee.hh:219-244): the
    reference test's property on its 2x2 fixture (one element changed by 0.25 changes the
    digest, tests/math_referee_foundation_test.cc:108-127), equal digests for the row- and
    column-major views of one logical matrix and for a strided view, the value type code in
    the digest, empty views, and the invalid-argument and unsupported-type statuses. The
    exact digest values are unpinned (no recorded value in the reference)."""
    import numpy as np
    view = np.array([[0.0, 30.0], [29.0, 74.0]], np.float32)
    st, first = oracle.digest_logical_dense(view)
    assert st == 0
    changed = view.copy()
    changed[1, 0] += 0.25
    assert oracle.digest_logical_dense(changed)[1] != first
    assert oracle.digest_logical_dense(view.copy())[1] == first
    rng = np.random.default_rng(3)
    a = rng.standard_normal((5, 7)).astype(np.float32)
    st_r, d_r = oracle.digest_logical_dense(a)
    st_c, d_c = oracle.digest_logical_dense(np.ascontiguousarray(a.T), column_major=True, ld=5, shape=(5, 7))
    assert st_r == st_c == 0 and d_r == d_c
    wide = np.zeros((5, 9), np.float32)
    wide[:, :7] = a
    assert oracle.digest_logical_dense(wide, ld=9, shape=(5, 7))[1] == d_r
    # f16 and f32 views of the same values differ only through the type code
    h = a.astype(np.float16)
    assert oracle.digest_logical_dense(h)[1] != oracle.digest_logical_dense(h.astype(np.float32))[1]
    assert oracle.digest_logical_dense(h.astype(np.float64))[1] != oracle.digest_logical_dense(h.astype(np.float32))[1]
    # element order matters (a transposed operand is caught)
    sq = rng.standard_normal((4, 4)).astype(np.float32)
    assert oracle.digest_logical_dense(sq)[1] != oracle.digest_logical_dense(np.ascontiguousarray(sq.T))[1]
    # empty views digest their shape only; invalid views and types are rejected
    assert oracle.digest_logical_dense(np.zeros((0, 3), np.float32), shape=(0, 3))[0] == 0
    assert oracle.digest_logical_dense(a, ld=6, shape=(5, 7))[0] == 1
    assert oracle.digest_logical_dense(a.astype(np.int32))[0] == 3
