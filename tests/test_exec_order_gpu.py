"""Execution feature order on the GPU: the device packer equals the host packer (the
reference's {5, 6, 1, 2, 7, 8, 3, 4} known answer, tests/math_execution_csr_test.cu:96-144),
per-gene counts equal numpy's bincount, the quantized CSR relabelled into execution order
decodes to exactly the same (row, gene, value) triples, and the projection on
(X_exec, W_exec) equals the canonical referee's X . W."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from tests.helpers import check_against_referee, qcsr_to_host, quantized_fixture, to_device_qcsr

pytestmark = pytest.mark.gpu


def test_device_pack_matches_host_kat():
    import torch

    from cellerator_amd import _native as N
    from tests.test_exec_order import GEOMETRY, _canonical_w, _plan
    lib = N.engine()
    plan, src = _plan(), _canonical_w()
    host = np.zeros(8, np.float32)
    hv = N.CxDenseOperand()
    assert lib.cx_pack_dense_operand_host(C.byref(plan), GEOMETRY, C.byref(src), host.ctypes.data, 32,
                                          C.byref(hv)) == 0
    perm_d = torch.tensor([2, 0, 3, 1], dtype=torch.int32).cuda()
    w_d = torch.from_numpy(src._keep.copy()).cuda()
    out_d = torch.zeros(8, dtype=torch.float32, device="cuda")
    dplan = N.CxCpbpPlan(4, 2, perm_d.data_ptr(), plan._keep[0].ctypes.data)
    dsrc = _canonical_w()
    dsrc.values = w_d.data_ptr()
    dv = N.CxDenseOperand()
    assert lib.cx_pack_dense_operand_device(C.byref(dplan), GEOMETRY, C.byref(dsrc), out_d.data_ptr(), 32,
                                            torch.cuda.current_stream().cuda_stream, C.byref(dv)) == 0, \
        lib.cx_exec_last_error()
    torch.cuda.synchronize()
    assert out_d.cpu().tolist() == [5, 6, 1, 2, 7, 8, 3, 4] == host.tolist()
    assert dv.operand_identity == hv.operand_identity


def test_column_counts_match_bincount(oracle):
    import torch

    from cellerator_amd.exec_order import column_counts
    for cols, rows in ((500, 3000), (40000, 700)):  # LDS bins and the global-atomic path
        rng = np.random.default_rng(cols)
        fx = quantized_fixture(oracle, rng, rows, cols, 60.0, 4, 1)
        got = column_counts(to_device_qcsr(fx)).cpu().numpy()
        torch.cuda.synchronize()
        assert np.array_equal(got, np.bincount(fx["col_idx"], minlength=cols))


def _triples(oracle, h, order_perm=None):
    decoded = oracle.decode_csr(h["bits"], h["policy"], h["row_ptr"], h["packed_row_ptr"], h["col_idx"],
                                h["packed"], h["scales"], h["offsets"], h["row_offsets"]) if h["bits"] else h["values"]
    rows = np.repeat(np.arange(h["rows"]), np.diff(h["row_ptr"]))
    cols = h["col_idx"] if order_perm is None else order_perm[h["col_idx"]]
    key = rows.astype(np.int64) * h["cols"] + cols
    idx = np.argsort(key, kind="stable")
    return key[idx], np.asarray(decoded)[idx]


@pytest.mark.parametrize("bits,policy", [(4, 1), (8, 1), (2, 2), (1, 1), (4, 3)])
def test_to_execution_order_is_a_relabelling(oracle, bits, policy):
    import torch

    from cellerator_amd import qcsr_pack_gene_affine
    from cellerator_amd.exec_order import popularity_order, to_execution_order
    rng = np.random.default_rng(300 + bits + policy)
    fx = quantized_fixture(oracle, rng, 900, 2600, 70.0, bits, 1 if policy == 3 else policy, empty_every=13)
    m = to_device_qcsr(fx)
    if policy == 3:
        m = qcsr_pack_gene_affine(m)
    order = popularity_order(m)
    mx = to_execution_order(m, order)
    torch.cuda.synchronize()
    perm = order.feature_permutation.cpu().numpy()
    counts = np.bincount(fx["col_idx"], minlength=2600)
    assert np.all(np.diff(counts[perm]) <= 0)  # most frequent first
    hx = qcsr_to_host(mx)
    assert np.array_equal(hx["row_ptr"], fx["row_ptr"])
    # every row strictly increasing in execution order
    for r in range(0, 900, 37):
        seg = hx["col_idx"][fx["row_ptr"][r]:fx["row_ptr"][r + 1]]
        assert np.all(np.diff(seg) > 0)
    if policy == 3:  # compare through the separate-array decode
        pairs = hx["scales"].reshape(-1, 2)
        hx = dict(hx, policy=1, scales=np.ascontiguousarray(pairs[:, 0]), offsets=np.ascontiguousarray(pairs[:, 1]))
    inv = order.inverse_permutation.cpu().numpy()
    k0, v0 = _triples(oracle, dict(fx, values=None), inv)
    k1, v1 = _triples(oracle, hx)
    assert np.array_equal(k0, k1)
    assert np.array_equal(v0.view(np.uint32), v1.view(np.uint32))  # decoded bitwise equal


def test_projection_is_order_invariant(oracle):
    import torch

    from cellerator_amd import qcsr_spmm
    from cellerator_amd.exec_order import pack_rows, popularity_order, to_execution_order
    rng = np.random.default_rng(77)
    fx = quantized_fixture(oracle, rng, 1500, 3000, 90.0, 4, 1)
    m = to_device_qcsr(fx)
    w = torch.from_numpy((rng.standard_normal((3000, 64)) * 0.02).astype(np.float16)).cuda()
    order = popularity_order(m)
    y = qcsr_spmm(to_execution_order(m, order), pack_rows(order, w))
    torch.cuda.synchronize()
    ref, mag = oracle.qcsr_spmm_referee(4, 1, 1500, 3000, fx["row_ptr"], fx["packed_row_ptr"], fx["col_idx"],
                                        fx["packed"], fx["scales"], fx["offsets"], None, w.cpu().numpy())
    check_against_referee(oracle, ref, mag, y.cpu().numpy())


def test_plain_values_and_repeated_gene():
    import torch

    from cellerator_amd import QcsrMatrix
    from cellerator_amd.exec_order import ExecutionOrder, to_execution_order
    row_ptr = torch.tensor([0, 3, 5], dtype=torch.int32).cuda()
    col_idx = torch.tensor([0, 2, 3, 1, 3], dtype=torch.int32).cuda()
    vals = torch.tensor([1, 2, 3, 4, 5], dtype=torch.float16).cuda()
    m = QcsrMatrix(2, 4, 0, row_ptr, col_idx, values=vals)
    perm = torch.tensor([3, 1, 0, 2], dtype=torch.int32).cuda()   # execution -> canonical
    inv = torch.tensor([2, 1, 3, 0], dtype=torch.int32).cuda()    # canonical -> execution
    mx = to_execution_order(m, ExecutionOrder(perm, inv))
    torch.cuda.synchronize()
    assert mx.col_idx.cpu().tolist() == [0, 2, 3, 0, 1]
    assert mx.values.cpu().tolist() == [3.0, 1.0, 2.0, 5.0, 4.0]
    dup = QcsrMatrix(2, 4, 0, row_ptr, torch.tensor([0, 2, 2, 1, 3], dtype=torch.int32).cuda(), values=vals)
    with pytest.raises(ValueError, match="repeats"):
        to_execution_order(dup, ExecutionOrder(perm, inv))
