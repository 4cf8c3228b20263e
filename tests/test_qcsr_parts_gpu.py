"""GPU parity of the gene-part quantized CSR kernels (qcsr_parts.hip).

cx_qcsr_spmm_fwd takes the row-group kernel for quantized codes with fp16 weights and
N = 64 (N = 128..256 in 64-column launches): the weight panel is streamed through LDS in
parts of 1,024 genes, each 8-lane group owns a row with a 64-entry register window and a
cursor, and rows the part walk cannot finish (columns out of order across parts, or
outside [0, cols)) are recomputed on a plain per-row path. These cases pin each of those
paths against the float64 referee on the same inputs: many parts, runs that fill whole
windows inside one part, skewed row lengths within and across workgroups of 512 rows (the
balanced row assignment), windows at the ends of the column and code arrays, unsorted and
duplicated columns, and out-of-range columns (which contribute nothing on this path).
"""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import check_against_referee, quantized_fixture, to_device_qcsr

pytestmark = pytest.mark.gpu


def _run(m, rhs_np):
    import torch

    from cellerator_amd import qcsr_spmm
    out = qcsr_spmm(m, torch.from_numpy(rhs_np).cuda())
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _referee(oracle, fx, rhs):
    return oracle.qcsr_spmm_referee(fx["bits"], fx["policy"], fx["rows"], fx["cols"], fx["row_ptr"],
                                    fx["packed_row_ptr"], fx["col_idx"], fx["packed"], fx["scales"],
                                    fx["offsets"], fx["row_offsets"], rhs)


def _skewed_fixture(oracle, rng, rows, cols, bits, policy):
    """Row lengths from 0 to several thousand (a few rows span every part, several rows
    are empty), sorted unique columns."""
    fx = quantized_fixture(oracle, rng, rows, cols, 10.0, bits, policy)
    lengths = np.minimum(rng.lognormal(np.log(400.0), 1.1, rows).astype(np.int64), cols)
    lengths[rng.choice(rows, rows // 15, replace=False)] = 0
    lengths[rng.choice(rows, 3, replace=False)] = cols  # dense rows: every gene
    row_ptr = np.zeros(rows + 1, np.int64)
    row_ptr[1:] = np.cumsum(lengths)
    col_idx = np.empty(int(row_ptr[-1]), np.int32)
    for r in range(rows):
        if lengths[r]:
            col_idx[row_ptr[r]:row_ptr[r + 1]] = np.sort(rng.choice(cols, lengths[r], replace=False))
    return _rebuild(oracle, rng, fx, row_ptr.astype(np.int32), col_idx)


def _rebuild(oracle, rng, fx, row_ptr, col_idx):
    """Same metadata, new structure: fresh codes packed by the oracle."""
    bits, policy, rows = fx["bits"], fx["policy"], fx["rows"]
    codes = rng.integers(0, (1 << bits), len(col_idx))
    if policy == oracle.PER_GENE_AFFINE:
        values = (fx["offsets"][col_idx] + fx["scales"][col_idx] * codes).astype(np.float32)
    else:
        row_of = np.repeat(np.arange(rows), np.diff(row_ptr))
        values = (fx["row_offsets"][row_of] + fx["scales"][col_idx] * codes).astype(np.float32)
    packed_row_ptr = oracle.build_packed_row_ptr(bits, row_ptr)
    packed = oracle.pack_csr(bits, policy, row_ptr, packed_row_ptr, col_idx, values, fx["scales"],
                             fx["offsets"], fx["row_offsets"])
    return dict(fx, row_ptr=row_ptr, col_idx=col_idx, packed_row_ptr=packed_row_ptr, packed=packed)


@pytest.mark.parametrize("bits,policy", [(4, 1), (8, 1), (2, 2), (1, 1)])
def test_many_parts_skewed_rows(oracle, bits, policy):
    """5 parts (the last one partial), one ragged workgroup, rows from empty to all 4,700
    genes (windows reloaded inside a part)."""
    rng = np.random.default_rng(900 + bits * 10 + policy)
    fx = _skewed_fixture(oracle, rng, 400, 4700, bits, policy)
    rhs = (rng.standard_normal((4700, 64)) * 0.02).astype(np.float16)
    ref, mag = _referee(oracle, fx, rhs)
    check_against_referee(oracle, ref, mag, _run(to_device_qcsr(fx), rhs))


def _long_tail_fixture(oracle, rng, bits, rows=1300, cols=2600):
    """Workgroups of 512, 512 and 276 rows; long rows across the first block boundary and at
    the end of the matrix (whole-window runs inside a part, windows reaching the ends of the
    column and code arrays, code tails ending inside a byte)."""
    fx = quantized_fixture(oracle, rng, rows, cols, 10.0, bits, 1)
    lengths = np.minimum(rng.lognormal(np.log(300.0), 0.9, rows).astype(np.int64), cols)
    lengths[rng.choice(rows - 5, 40, replace=False)] = 0
    lengths[510:514] = [cols, 0, 2049, 1]
    lengths[-5:] = [cols, 1777, 3, cols - 1, 1501]
    row_ptr = np.zeros(rows + 1, np.int64)
    row_ptr[1:] = np.cumsum(lengths)
    col_idx = np.empty(int(row_ptr[-1]), np.int32)
    for r in range(rows):
        if lengths[r]:
            col_idx[row_ptr[r]:row_ptr[r + 1]] = np.sort(rng.choice(cols, lengths[r], replace=False))
    return _rebuild(oracle, rng, fx, row_ptr.astype(np.int32), col_idx)


def _per_round(monkeypatch, units):
    """Workgroups per round of the row-group walk: the device's compute units (None) or an
    override (1: the fewest full workgroups of 512 rows)."""
    if units is None:
        monkeypatch.delenv("CX_BLOCKS_PER_ROUND", raising=False)
    else:
        monkeypatch.setenv("CX_BLOCKS_PER_ROUND", str(units))


@pytest.mark.parametrize("units", [1, None])
@pytest.mark.parametrize("bits", [4, 8])
def test_many_workgroups_long_last_rows(oracle, monkeypatch, bits, units):
    """Three workgroups (one per round), long rows at a block boundary and at the array ends:
    block-end and array-end window loads are both exercised; and the same rows spread over a
    round of the device's compute units (workgroups of ~8 rows)."""
    rng = np.random.default_rng(971 + bits)
    fx = _long_tail_fixture(oracle, rng, bits)
    rhs = (rng.standard_normal((fx["cols"], 64)) * 0.02).astype(np.float16)
    ref, mag = _referee(oracle, fx, rhs)
    _per_round(monkeypatch, units)
    check_against_referee(oracle, ref, mag, _run(to_device_qcsr(fx), rhs))


def test_workgroup_geometries_agree(oracle, monkeypatch):
    """The launch splits the rows into whole rounds of workgroups (at most 512 rows each, an
    even share per workgroup). Every geometry gives each row the same summation order, so the
    sums agree (as values: a pad may turn an all-zero sum's -0.0 into +0.0) and match the
    referee: the fewest full workgroups, 3 and 7 per round, and the device's compute units."""
    import torch
    rng = np.random.default_rng(4242)
    fx = _long_tail_fixture(oracle, rng, 4)
    rhs = (rng.standard_normal((fx["cols"], 64)) * 0.02).astype(np.float16)
    ref, mag = _referee(oracle, fx, rhs)
    m = to_device_qcsr(fx)
    outs = []
    for units in (1, 3, 7, None):
        _per_round(monkeypatch, units)
        outs.append(_run(m, rhs))
        check_against_referee(oracle, ref, mag, outs[-1])
    for o in outs[1:]:
        assert torch.equal(torch.from_numpy(o), torch.from_numpy(outs[0]))


def test_interleaved_pairs_through_parts(oracle):
    """The pairs policy copies (scale, offset) into LDS by direct loads: equal bitwise to
    the separate arrays across several parts."""
    import torch

    from cellerator_amd import qcsr_pack_gene_affine, qcsr_spmm
    rng = np.random.default_rng(931)
    fx = _skewed_fixture(oracle, rng, 300, 3100, 4, oracle.PER_GENE_AFFINE)
    m = to_device_qcsr(fx)
    rhs = torch.from_numpy((rng.standard_normal((3100, 64)) * 0.02).astype(np.float16)).cuda()
    a = qcsr_spmm(m, rhs)
    b = qcsr_spmm(qcsr_pack_gene_affine(m), rhs)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    ref, mag = _referee(oracle, fx, rhs.cpu().numpy())
    check_against_referee(oracle, ref, mag, a.cpu().numpy())


def test_unsorted_and_duplicate_columns(oracle):
    """Rows whose columns go back across a part boundary take the per-row path; columns out
    of order inside one part and repeated columns stay on the part walk. Every row must
    match the referee, which sums entries in storage order."""
    rng = np.random.default_rng(947)
    fx = _skewed_fixture(oracle, rng, 260, 3000, 4, 1)
    row_ptr, col_idx = fx["row_ptr"], fx["col_idx"].copy()
    for r in range(0, 260, 3):  # reverse every third row: out of order across parts
        s, e = row_ptr[r], row_ptr[r + 1]
        col_idx[s:e] = col_idx[s:e][::-1]
    for r in range(1, 260, 7):  # swap neighbours inside a part, duplicate a column
        s, e = row_ptr[r], row_ptr[r + 1]
        seg = col_idx[s:e]
        inside = [i for i in range(len(seg) - 1) if seg[i] // 1024 == seg[i + 1] // 1024]
        if inside:
            i = inside[len(inside) // 2]
            seg[i], seg[i + 1] = seg[i + 1], seg[i]
        if len(seg) > 2:
            seg[-1] = seg[-2]
    fx = _rebuild(oracle, rng, fx, row_ptr, col_idx)
    rhs = (rng.standard_normal((3000, 64)) * 0.02).astype(np.float16)
    ref, mag = _referee(oracle, fx, rhs)
    check_against_referee(oracle, ref, mag, _run(to_device_qcsr(fx), rhs))


def test_out_of_range_columns_contribute_nothing(oracle):
    """Columns >= cols or negative are skipped on this path. The expected output is the
    referee's on one extra gene whose weight row is zero, with those entries pointed at it."""
    rng = np.random.default_rng(953)
    cols = 2100
    fx = _skewed_fixture(oracle, rng, 200, cols, 4, 1)
    col_idx = fx["col_idx"].copy()
    bad = rng.choice(len(col_idx), 40, replace=False)
    col_idx[bad[:20]] = cols + 5
    col_idx[bad[20:]] = -3
    rhs = (rng.standard_normal((cols, 64)) * 0.02).astype(np.float16)
    # device matrix: the out-of-range columns as they are
    dev = dict(fx, col_idx=col_idx)
    got = _run(to_device_qcsr(dev), rhs)
    # referee: cols + 1 genes, the bad entries on gene `cols` whose weight row is zero
    ref_cols = col_idx.copy()
    ref_cols[bad] = cols
    ext = dict(fx, cols=cols + 1, col_idx=ref_cols,
               scales=np.append(fx["scales"], np.float32(0.25)),
               offsets=np.append(fx["offsets"], np.float32(0.0)))
    rhs_ext = np.vstack([rhs, np.zeros((1, 64), np.float16)])
    ref, mag = _referee(oracle, ext, rhs_ext)
    check_against_referee(oracle, ref, mag, got)


def test_generated_c3_rows_with_epilogue(oracle):
    """GPU-generated C3-distributed rows (33,538 genes: 33 parts) through the part walk with
    a fused bias + ReLU epilogue, against the referee followed by the same epilogue."""
    import torch

    from cellerator_amd import Epilogue, qcsr_pack_gene_affine, qcsr_spmm
    from cellerator_amd._native import EPILOGUE_BIAS_RELU
    from cellerator_amd.synth import C3, dense_normal, generate_qcsr
    from tests.helpers import qcsr_to_host
    m = generate_qcsr(C3.scaled(700))
    w = dense_normal((m.cols, 64), 0.02, torch.float16, seed=C3.seed + 1)
    bias = torch.linspace(-0.05, 0.05, 64, device="cuda", dtype=torch.float32)
    out = qcsr_spmm(qcsr_pack_gene_affine(m), w, epilogue=Epilogue(kind=EPILOGUE_BIAS_RELU, bias=bias))
    torch.cuda.synchronize()
    h = qcsr_to_host(m)
    ref, mag = oracle.qcsr_spmm_referee(4, 1, m.rows, m.cols, h["row_ptr"], h["packed_row_ptr"],
                                        h["col_idx"], h["packed"], h["scales"], h["offsets"], None,
                                        w.cpu().numpy())
    expect = np.maximum(ref.reshape(m.rows, 64) + bias.cpu().numpy().astype(np.float64), 0.0)
    got = out.cpu().numpy().astype(np.float64)
    tol = 1e-4 * np.abs(expect) + 1e-4 * mag.reshape(m.rows, 64)  # the suite's bound
    assert np.all(np.abs(got - expect) <= tol)


@pytest.mark.parametrize("n", [128, 192])
def test_wide_outputs_in_64_column_blocks_with_epilogue(oracle, n):
    """N = 128 and 192 run one launch per 64 output columns; the bias and the beta * C
    operand are shifted with each block (in-place affine update plus bias + GELU)."""
    import torch

    from cellerator_amd import Epilogue, qcsr_spmm
    from cellerator_amd._native import EPILOGUE_BIAS_GELU_ERF
    from math import erf, sqrt
    rng = np.random.default_rng(961 + n)
    fx = _skewed_fixture(oracle, rng, 330, 2500, 4, 1)
    rhs = (rng.standard_normal((2500, n)) * 0.02).astype(np.float16)
    c0 = (rng.standard_normal((330, n)) * 0.1).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.05).astype(np.float32)
    out = torch.from_numpy(c0.copy()).cuda()
    ep = Epilogue(kind=EPILOGUE_BIAS_GELU_ERF, alpha=0.5, beta=2.0,
                  bias=torch.from_numpy(bias).cuda(), initial=out)
    qcsr_spmm(to_device_qcsr(fx), torch.from_numpy(rhs).cuda(), out=out, epilogue=ep)
    torch.cuda.synchronize()
    ref, mag = _referee(oracle, fx, rhs)
    pre = 0.5 * ref.reshape(330, n) + 2.0 * c0.astype(np.float64) + bias.astype(np.float64)
    expect = np.vectorize(lambda v: 0.5 * v * (1.0 + erf(v / sqrt(2.0))))(pre)
    got = out.cpu().numpy().astype(np.float64)
    tol = 1e-4 * np.abs(expect) + 1e-4 * (0.5 * mag.reshape(330, n) + 2.0 * np.abs(c0)) + 1e-6
    assert np.all(np.abs(got - expect) <= tol)


def _bwd_values_check(oracle, fx, g, w, got):
    ref = oracle.spmm_bwd_values(fx["row_ptr"], fx["col_idx"], g, w)
    rows_of = np.repeat(np.arange(fx["rows"]), np.diff(fx["row_ptr"]))
    mag = np.einsum("ij,ij->i", np.abs(g.astype(np.float64))[rows_of],
                    np.abs(w.astype(np.float64))[fx["col_idx"]])
    check_against_referee(oracle, ref, mag, got)


def test_bwd_values_parts_skewed_rows(oracle):
    """grad_values by the row-group walk (fp16 W, N = 64): 5 parts, rows from empty to every
    gene; against the float64 restatement of csr_spmm_bwd_values."""
    import torch

    from cellerator_amd import qcsr_spmm_bwd_values
    rng = np.random.default_rng(971)
    fx = _skewed_fixture(oracle, rng, 420, 4700, 8, 1)
    g = rng.standard_normal((420, 64)).astype(np.float32)
    w = (rng.standard_normal((4700, 64)) * 0.1).astype(np.float16)
    gv = qcsr_spmm_bwd_values(to_device_qcsr(fx), torch.from_numpy(g).cuda(), torch.from_numpy(w).cuda())
    torch.cuda.synchronize()
    _bwd_values_check(oracle, fx, g, w, gv.cpu().numpy())


def test_bwd_values_parts_unsorted_and_out_of_range(oracle):
    """Rows out of order across parts, and rows stopped by a column outside [0, cols), are
    recomputed whole on the per-row path; entries with such columns get 0."""
    import torch

    from cellerator_amd import qcsr_spmm_bwd_values
    rng = np.random.default_rng(977)
    cols = 3000
    fx = _skewed_fixture(oracle, rng, 260, cols, 4, 1)
    row_ptr, col_idx = fx["row_ptr"], fx["col_idx"].copy()
    for r in range(0, 260, 3):
        s, e = row_ptr[r], row_ptr[r + 1]
        col_idx[s:e] = col_idx[s:e][::-1]
    bad = rng.choice(len(col_idx), 30, replace=False)
    col_idx[bad[:15]] = cols + 7
    col_idx[bad[15:]] = -1
    dev = dict(fx, col_idx=col_idx)
    g = rng.standard_normal((260, 64)).astype(np.float32)
    w = (rng.standard_normal((cols, 64)) * 0.1).astype(np.float16)
    gv = qcsr_spmm_bwd_values(to_device_qcsr(dev), torch.from_numpy(g).cuda(), torch.from_numpy(w).cuda())
    torch.cuda.synchronize()
    got = gv.cpu().numpy()
    assert np.all(got[bad] == 0.0)
    good = np.ones(len(col_idx), bool)
    good[bad] = False
    ref_cols = col_idx.copy()
    ref_cols[bad] = 0
    ref = oracle.spmm_bwd_values(row_ptr, ref_cols, g, w)
    rows_of = np.repeat(np.arange(260), np.diff(row_ptr))
    mag = np.einsum("ij,ij->i", np.abs(g.astype(np.float64))[rows_of],
                    np.abs(w.astype(np.float64))[ref_cols])
    check_against_referee(oracle, ref[good], mag[good], got[good])


def test_bwd_values_many_workgroups_long_last_rows(oracle):
    """grad_values over three workgroups with long rows at a block boundary and at the end
    of the column array (whole-window runs, array-end windows, partial last stores)."""
    import torch

    from cellerator_amd import qcsr_spmm_bwd_values
    rng = np.random.default_rng(983)
    fx = _long_tail_fixture(oracle, rng, 4)
    g = rng.standard_normal((fx["rows"], 64)).astype(np.float32)
    w = (rng.standard_normal((fx["cols"], 64)) * 0.1).astype(np.float16)
    gv = qcsr_spmm_bwd_values(to_device_qcsr(fx), torch.from_numpy(g).cuda(), torch.from_numpy(w).cuda())
    torch.cuda.synchronize()
    _bwd_values_check(oracle, fx, g, w, gv.cpu().numpy())


def test_check_columns_and_sorted_flag(oracle):
    """qcsr_check_columns sets QCSR_COLUMNS_SORTED exactly for non-decreasing in-range rows
    (repeats allowed); with the flag the row-group kernels skip their out-of-order check and
    give bit-identical forward outputs and gradients on sorted input."""
    import torch

    from cellerator_amd import _native as N
    from cellerator_amd import qcsr_check_columns, qcsr_spmm, qcsr_spmm_bwd_values
    rng = np.random.default_rng(991)
    fx = _long_tail_fixture(oracle, rng, 4, rows=700, cols=2300)
    m = to_device_qcsr(fx)
    ms = qcsr_check_columns(m)
    assert ms.flags == N.QCSR_COLUMNS_SORTED
    rhs = torch.from_numpy((rng.standard_normal((2300, 64)) * 0.02).astype(np.float16)).cuda()
    a, b = qcsr_spmm(m, rhs), qcsr_spmm(ms, rhs)
    g = torch.from_numpy(rng.standard_normal((700, 64)).astype(np.float32)).cuda()
    ga, gb = qcsr_spmm_bwd_values(m, g, rhs), qcsr_spmm_bwd_values(ms, g, rhs)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    assert torch.equal(ga.view(torch.int32), gb.view(torch.int32))
    ref, mag = _referee(oracle, fx, rhs.cpu().numpy())
    check_against_referee(oracle, ref, mag, b.cpu().numpy())
    # a repeated column keeps the flag; a descent, a column >= cols or < 0 clears it
    row_ptr = fx["row_ptr"]
    r = int(np.argmax(np.diff(row_ptr) > 10))
    s = int(row_ptr[r])
    for change, expect in ((lambda c: c.__setitem__(s + 1, c[s]), N.QCSR_COLUMNS_SORTED),
                           (lambda c: c.__setitem__(s, c[s + 1] + 1), 0),
                           (lambda c: c.__setitem__(int(row_ptr[-1]) - 1, 2300), 0),
                           (lambda c: c.__setitem__(0 if row_ptr[1] > 0 else s, -1), 0)):
        col_idx = fx["col_idx"].copy()
        change(col_idx)
        assert qcsr_check_columns(to_device_qcsr(dict(fx, col_idx=col_idx))).flags == expect


@pytest.mark.parametrize("n", [64, 128])
@pytest.mark.parametrize("policy", [1, 2, 3])
@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_sorted_flag_forms_bitwise_and_referee(oracle, bits, policy, n):
    """Every instantiation the column-order flag selects (bits x metadata policy, where 3 is
    the interleaved pairs, N = 64 and two 64-column blocks at N = 128) gives bitwise the
    same output as the checked kernel, and is within tolerance of the referee, over three
    workgroups of rows with a ragged last one."""
    import torch

    from cellerator_amd import qcsr_check_columns, qcsr_pack_gene_affine, qcsr_spmm
    rng = np.random.default_rng(1200 + 10 * bits + policy + n)
    fx = _long_tail_fixture(oracle, rng, bits, rows=1300, cols=2300)
    if policy == 2:
        fx = _rebuild(oracle, rng, dict(fx, policy=2, offsets=None,
                                        row_offsets=rng.uniform(-1, 1, fx["rows"]).astype(np.float32)),
                      fx["row_ptr"], fx["col_idx"])
    m = to_device_qcsr(fx)
    if policy == 3:
        m = qcsr_pack_gene_affine(m)
    ms = qcsr_check_columns(m)
    assert ms.flags == 1
    rhs = torch.from_numpy((rng.standard_normal((fx["cols"], n)) * 0.02).astype(np.float16)).cuda()
    a, b = qcsr_spmm(m, rhs), qcsr_spmm(ms, rhs)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    ref, mag = _referee(oracle, fx, rhs.cpu().numpy())
    check_against_referee(oracle, ref, mag, b.cpu().numpy())


def test_sorted_flag_with_epilogue(oracle):
    """Sorted + pairs with a fused bias-GELU epilogue and beta * C: bitwise the checked
    kernel's output."""
    import torch

    from cellerator_amd import Epilogue, qcsr_check_columns, qcsr_pack_gene_affine, qcsr_spmm
    rng = np.random.default_rng(1333)
    fx = _long_tail_fixture(oracle, rng, 4, rows=1100, cols=2100)
    m = qcsr_pack_gene_affine(to_device_qcsr(fx))
    ms = qcsr_check_columns(m)
    rhs = torch.from_numpy((rng.standard_normal((fx["cols"], 64)) * 0.02).astype(np.float16)).cuda()
    bias = torch.randn(64, device="cuda")
    c0 = torch.randn(fx["rows"], 64, device="cuda")
    a = c0.clone()
    b = c0.clone()
    qcsr_spmm(m, rhs, out=a, epilogue=Epilogue(6, 0.75, -0.5, bias, a))
    qcsr_spmm(ms, rhs, out=b, epilogue=Epilogue(6, 0.75, -0.5, bias, b))
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_benched_instantiation_on_c3_rows(oracle):
    """The exact form bench.py times at C3 -- 4-bit codes, interleaved pairs, the checked
    column-order flag, N = 64 -- on C3-generated rows spanning three full workgroups of 512
    rows and a ragged fourth (the tail block whose windows reach the array ends), against the
    float64 referee on every row."""
    import torch

    from cellerator_amd import qcsr_check_columns, qcsr_pack_gene_affine, qcsr_spmm
    from cellerator_amd.synth import C3, dense_normal, generate_qcsr
    from tests.helpers import qcsr_to_host
    m = generate_qcsr(C3.scaled(3 * 512 + 77))
    fast = qcsr_check_columns(qcsr_pack_gene_affine(m))
    assert fast.flags == 1 and fast.decode_policy == 3
    w = dense_normal((m.cols, 64), 0.02, torch.float16, seed=77)
    y = qcsr_spmm(fast, w)
    torch.cuda.synchronize()
    h = qcsr_to_host(m)
    ref, mag = oracle.qcsr_spmm_referee(4, 1, m.rows, m.cols, h["row_ptr"], h["packed_row_ptr"],
                                        h["col_idx"], h["packed"], h["scales"], h["offsets"], None,
                                        w.cpu().numpy())
    check_against_referee(oracle, ref, mag, y.cpu().numpy())
