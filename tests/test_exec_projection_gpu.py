"""GPU parity of the prepared execution-order projection (cx_qcsr_exec_*, qcsr_exec.hip) --
the path bench.py times and the CP-Math execution-order candidate runs -- and of that
candidate through the reference's own operation core.

* The projection's product equals, bitwise, the step-by-step path (popularity order,
  relabelled matrix, dense head, tail stream: exec_order.py) with the same head width, and
  matches the float64 referee of the canonical matrix (canonical W in, canonical rows out).
* At the benchmark configurations' shapes: C3-generated rows (4-bit codes, 33,538 genes)
  with the 2,048-gene head and the tail stream in three block geometries (one block per
  compute unit; three full 1,024-row blocks and a ragged one; seven partly filled blocks),
  N = 64 and 128; C2-generated rows (8-bit codes) with the 3,072-gene head (and 6,144).
* Through register -> prepare -> run_prepared_operation: bitwise equal to the direct call,
  with and without a fused epilogue; without its persistent state the candidate runs the
  row-group kernel (bitwise equal to it); its launch costs no more than the direct call.
* A row that repeats a gene is rejected when the projection is prepared."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from tests.cpmath import harness as H
from tests.helpers import check_against_referee, qcsr_to_host, to_device_qcsr
from tests.test_cpmath_gpu import _time_ms, qcsr_case
from tests.test_hybrid_gpu import _exec, _referee, _skewed

pytestmark = pytest.mark.gpu


def _stepwise(m, w, head):
    """The same product by the step-by-step path of exec_order.py."""
    from cellerator_amd.exec_order import hybrid_prepare, hybrid_spmm, pack_rows
    mx, order = _exec(m, head)
    return hybrid_spmm(hybrid_prepare(mx, head, stream_tail=True), pack_rows(order, w))


def _referee_of(oracle, m, w):
    h = qcsr_to_host(m)
    return oracle.qcsr_spmm_referee(m.bits, 1 if m.decode_policy == 3 else m.decode_policy, m.rows, m.cols,
                                    h["row_ptr"], h["packed_row_ptr"], h["col_idx"], h["packed"],
                                    h["scales"] if m.decode_policy != 3 else h["scales"].reshape(-1, 2)[:, 0].copy(),
                                    h["offsets"] if m.decode_policy != 3 else h["scales"].reshape(-1, 2)[:, 1].copy(),
                                    h["row_offsets"], w.cpu().numpy())


@pytest.mark.parametrize("bits,policy,head", [(4, 1, 2048), (8, 1, 1024), (2, 2, 2048), (4, 3, 1024), (1, 1, 0)])
def test_projection_equals_stepwise_path_and_referee(oracle, bits, policy, head):
    import torch

    from cellerator_amd import qcsr_pack_gene_affine
    from cellerator_amd.exec_order import ExecProjection
    rng = np.random.default_rng(5000 + 10 * bits + policy + head)
    fx = _skewed(oracle, rng, 2300, 3100, bits, policy)
    m = to_device_qcsr(fx)
    if policy == 3:
        m = qcsr_pack_gene_affine(m)
    w = torch.from_numpy((rng.standard_normal((3100, 64)) * 0.02).astype(np.float16)).cuda()
    p = ExecProjection(m, head)
    info = p.info()
    assert info.head_cols == head and info.rows == 2300 and info.persistent_bytes > 0
    y = p.spmm(w)
    y2 = p.spmm(w)
    step = _stepwise(m, w, head)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32))
    assert torch.equal(y.view(torch.int32), step.view(torch.int32))
    ref, mag = _referee(oracle, dict(fx, policy=1 if policy == 3 else policy), w.cpu().numpy())
    check_against_referee(oracle, ref, mag, y.cpu().numpy())
    p.close()


@pytest.mark.parametrize("units", [None, 1, 7])
@pytest.mark.parametrize("n", [64, 128])
def test_c3_rows_at_the_benchmark_form(oracle, monkeypatch, n, units):
    """C3-generated rows as bench.py runs them: 2,048 head genes on the matrix cores, the rest
    through the tail stream, in each block geometry of the stream: one block per compute unit
    of the device (blocks of ~14 rows), three full 1,024-row blocks and a ragged one (C3's own
    geometry: the fewest full blocks), and seven partly filled blocks of ~510 rows."""
    import torch

    from cellerator_amd import qcsr_pack_gene_affine
    from cellerator_amd.exec_order import ExecProjection
    from cellerator_amd.synth import C3, dense_normal, generate_qcsr
    if units is None:
        monkeypatch.delenv("CX_BLOCKS_PER_ROUND", raising=False)
    else:
        monkeypatch.setenv("CX_BLOCKS_PER_ROUND", str(units))
    rows = 3 * 1024 + 500
    m = qcsr_pack_gene_affine(generate_qcsr(C3.scaled(rows)))
    w = dense_normal((m.cols, n), 0.02, torch.float16, seed=11 + n)
    p = ExecProjection(m, 2048)
    info = p.info()
    assert info.head_cols == 2048 and info.head_form == 2 and info.tail_fills > 0
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert int(info.tail_blocks) == {None: min(cus, -(-rows // 8)), 1: 4, 7: 7}[units]
    y = p.spmm(w)
    step = _stepwise(m, w, 2048)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), step.view(torch.int32))
    ref, mag = _referee_of(oracle, m, w)
    check_against_referee(oracle, ref, mag, y.cpu().numpy())
    p.close()


@pytest.mark.parametrize("head", [3072, 6144])
def test_c2_rows_at_the_benchmark_form(oracle, head):
    """C2-generated rows (8-bit codes, the words form of the head) with the 3,072-gene head
    bench.py runs at C2 (and 6,144) and the tail stream."""
    import torch

    from cellerator_amd import qcsr_pack_gene_affine
    from cellerator_amd.exec_order import ExecProjection
    from cellerator_amd.synth import C2, dense_normal, generate_qcsr
    m = qcsr_pack_gene_affine(generate_qcsr(C2.scaled(2 * 1024 + 300)))
    w = dense_normal((m.cols, 64), 0.02, torch.float16, seed=23)
    p = ExecProjection(m, head)
    assert p.info().head_form == 1
    y = p.spmm(w)
    step = _stepwise(m, w, head)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), step.view(torch.int32))
    ref, mag = _referee_of(oracle, m, w)
    check_against_referee(oracle, ref, mag, y.cpu().numpy())
    p.close()


def test_wide_range_genes_leave_the_head(oracle):
    """The three most stored genes get values the head cannot carry beside the others (a scale
    of 1,000; values near zero; values crossing zero): the projection orders them after a
    full 2,048-gene head. An identity W over those genes and 61 head genes returns every
    decoded value bitwise (the head's split, the tail's fp32 sum), and a random W matches the
    referee."""
    import torch

    from cellerator_amd.exec_order import ExecProjection, head_order
    from tests.test_qcsr_parts_gpu import _rebuild
    rng = np.random.default_rng(61)
    fx = _skewed(oracle, rng, 900, 2600, 4, 1, hostile=0.0)
    top = np.argsort(-np.bincount(fx["col_idx"], minlength=2600), kind="stable")[:3]
    s_, o_ = fx["scales"].copy(), fx["offsets"].copy()
    for g, (sg, og) in zip(top, ((1000.0, 0.5), (0.01, 0.01), (0.03, -0.2))):
        s_[g], o_[g] = sg, og
    fx = _rebuild(oracle, rng, dict(fx, scales=s_, offsets=o_), fx["row_ptr"], fx["col_idx"])
    m = to_device_qcsr(fx)
    order, h = head_order(m, 2048)
    assert h == 2048
    assert np.all(order.inverse_permutation.cpu().numpy()[top] >= 2048)
    p = ExecProjection(m, 2048)
    assert p.info().head_cols == 2048
    genes = np.concatenate([top, order.feature_permutation.cpu().numpy()[:61]])
    w = torch.zeros((2600, 64), dtype=torch.float16, device="cuda")
    w[torch.from_numpy(genes.astype(np.int64)).cuda(), torch.arange(64, device="cuda")] = 1.0
    y = p.spmm(w)
    wr = torch.from_numpy((rng.standard_normal((2600, 64)) * 0.02).astype(np.float16)).cuda()
    yr = p.spmm(wr)
    torch.cuda.synchronize()
    decoded = oracle.decode_csr(4, 1, fx["row_ptr"], fx["packed_row_ptr"], fx["col_idx"], fx["packed"],
                                fx["scales"], fx["offsets"], None)
    column = np.full(2600, -1)
    column[genes] = np.arange(64)
    rows = np.repeat(np.arange(900), np.diff(fx["row_ptr"]))
    sel = column[fx["col_idx"]] >= 0
    want = np.zeros((900, 64), np.float32)
    want[rows[sel], column[fx["col_idx"][sel]]] = decoded[sel]
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))
    ref, mag = _referee(oracle, fx, wr.cpu().numpy())
    check_against_referee(oracle, ref, mag, yr.cpu().numpy())
    p.close()


def test_projection_rejects_repeated_genes(oracle):
    from cellerator_amd import _native as N
    from cellerator_amd.exec_order import ExecProjection
    rng = np.random.default_rng(17)
    fx = _skewed(oracle, rng, 300, 2100, 4, 1)
    col = fx["col_idx"].copy()
    b = int(fx["row_ptr"][7])
    assert fx["row_ptr"][8] - b >= 2
    col[b + 1] = col[b]
    with pytest.raises(N.EngineError, match="repeats a gene"):
        ExecProjection(to_device_qcsr(dict(fx, col_idx=col)), 1024)


def _exec_case(m, w, y, head):
    import torch
    c = qcsr_case(m, w, y)
    c.exec_order, c.head_genes = 1, head
    nbytes = C.c_uint64()
    from cellerator_amd import _native as N
    assert N.engine().cx_qcsr_exec_workspace_for(m.rows, m.cols, head, w.shape[1], C.byref(nbytes)) == 0
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device="cuda")
    c.workspace, c.workspace_bytes = ws.data_ptr(), nbytes.value
    c._keep = c._keep + (ws,)
    return c


@pytest.mark.parametrize("bits", [4, 8])
def test_execution_order_candidate_through_reference_core(oracle, bits):
    import torch

    from cellerator_amd import qcsr_spmm
    from cellerator_amd.exec_order import ExecProjection
    rng = np.random.default_rng(300 + bits)
    fx = _skewed(oracle, rng, 2200, 3100, bits, 1)
    m = to_device_qcsr(fx)
    w = torch.from_numpy((rng.standard_normal((3100, 128)) * 0.02).astype(np.float16)).cuda()
    y = torch.full((2200, 128), float("nan"), device="cuda")
    r = H.run(_exec_case(m, w, y, 1024))
    assert (r.prepare_status, r.state_status, r.status) == (H.OK, H.OK, H.OK), (r.message, r.engine)
    assert r.dispatch == b"qcsr:execution-order"
    assert r.persistent_bytes > 0
    torch.cuda.synchronize()
    direct = ExecProjection(m, 1024).spmm(w)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), direct.view(torch.int32))
    ref, mag = _referee(oracle, fx, w.cpu().numpy())
    check_against_referee(oracle, ref, mag, y.cpu().numpy())
    # without the persistent state the candidate runs the row-group kernel on the bound CSR
    y2 = torch.full_like(y, float("nan"))
    c = _exec_case(m, w, y2, 1024)
    c.exec_order = 2
    r = H.run(c)
    assert (r.prepare_status, r.status) == (H.OK, H.OK), (r.message, r.engine)
    assert r.dispatch == b"qcsr:execution-order->row-group"
    torch.cuda.synchronize()
    assert torch.equal(y2.view(torch.int32), qcsr_spmm(m, w).view(torch.int32))


def test_execution_order_candidate_epilogue(oracle):
    """A fused epilogue (bias + ReLU, affine accumulate) through the candidate equals the
    direct call with the same epilogue, bitwise."""
    import torch

    from cellerator_amd import Epilogue
    from cellerator_amd.exec_order import ExecProjection
    rng = np.random.default_rng(44)
    fx = _skewed(oracle, rng, 1500, 2600, 4, 1)
    m = to_device_qcsr(fx)
    w = torch.from_numpy((rng.standard_normal((2600, 64)) * 0.02).astype(np.float16)).cuda()
    c0 = torch.from_numpy(rng.standard_normal((1500, 64)).astype(np.float32)).cuda()
    bias = torch.from_numpy(rng.standard_normal(64).astype(np.float32)).cuda()
    y = c0.clone()
    c = _exec_case(m, w, y, 1024)
    c.fused, c.epilogue_kind, c.affine, c.alpha, c.beta = 1, 5, 1, 0.5, 2.0
    c.bias = bias.data_ptr()
    r = H.run(c)
    assert (r.prepare_status, r.status) == (H.OK, H.OK), (r.message, r.engine)
    assert r.dispatch == b"qcsr:execution-order"
    direct = c0.clone()
    ExecProjection(m, 1024).spmm(w, out=direct, epilogue=Epilogue(kind=5, alpha=0.5, beta=2.0, bias=bias,
                                                                   initial=direct))
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), direct.view(torch.int32))


def test_execution_order_candidate_launch_costs_no_more_than_direct():
    """On C3-generated rows (131,072 cells, 2,048-gene head) the core's prepared launch takes
    no more than the direct call: within 5% (plus 20 us of host dispatch) over 20 launches."""
    import torch

    from cellerator_amd import qcsr_pack_gene_affine
    from cellerator_amd.exec_order import ExecProjection
    from cellerator_amd.synth import C3, dense_normal, generate_qcsr
    m = generate_qcsr(C3.scaled(131072))
    w = dense_normal((m.cols, 64), 0.02, torch.float16, seed=5)
    y = torch.empty((m.rows, 64), device="cuda")
    c = _exec_case(m, w, y, 2048)
    c.repeats = 20
    r = H.run(c)  # builds the state once, then 20 timed launches
    assert (r.state_status, r.status) == (H.OK, H.OK), (r.message, r.engine)
    assert r.dispatch == b"qcsr:execution-order"
    p = ExecProjection(qcsr_pack_gene_affine(m), 2048)
    out = torch.empty_like(y)
    direct_ms = _time_ms(lambda: p.spmm(w, out=out), 20)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), out.view(torch.int32))
    print(f"direct {direct_ms:.4f} ms, through the core {r.launch_ms:.4f} ms per launch")
    assert r.launch_ms <= direct_ms * 1.05 + 0.02
    p.close()
