"""GPU: the engine's CP-Math candidates prepared and run through the reference's own
operation core (register -> find -> prepare -> run_prepared_operation), checked bitwise
against the same kernels called directly through the C-ABI and against the oracle.
Also: rebinding a prepared operation to new W / Y without re-preparing, and capture of
the run in a HIP graph replayed with fresh inputs."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from tests.cpmath import harness as H
from tests.helpers import check_against_referee, quantized_fixture, to_device_qcsr

pytestmark = pytest.mark.gpu


def _ptr(t):
    return None if t is None else t.data_ptr()


def qcsr_case(m, w, y, bits_view=None):
    """HCase for a device QcsrMatrix `m`: the view keeps the structure arrays only."""
    import torch

    d = m.descriptor()
    view = type(d).from_buffer_copy(d)
    view.packed_values = view.values = view.column_scales = view.column_offsets = None
    view.row_offsets = None
    view.decode_policy = 0
    quantized = m.bits != 0
    vals = m.packed_values if quantized else m.values
    dense = H.NT_F16 if w.dtype == torch.float16 else H.NT_F32
    sparse = H.NT_U8 if quantized else (H.NT_F16 if vals.dtype == torch.float16 else H.NT_F32)
    c = H.HCase(kind=H.KIND_QCSR, view=C.addressof(view), view_bytes=C.sizeof(view),
                variant=m.bits, rows=m.rows, cols=m.cols, out_cols=w.shape[1], block_size=0,
                sparse_type=sparse, dense_type=dense, nnz=m.nnz, values=vals.data_ptr(),
                value_count=m.nnz, value_bytes=vals.numel() * vals.element_size(),
                scales=_ptr(m.column_scales), offsets=_ptr(m.column_offsets), w=w.data_ptr(),
                w_ld=w.stride(0), y=y.data_ptr(), y_ld=y.stride(0),
                stream=torch.cuda.current_stream().cuda_stream, device=torch.cuda.current_device())
    c._keep = (view, m, w, y)
    return c


@pytest.mark.parametrize("bits", [4, 8])
def test_quantized_csr_through_reference_core(oracle, bits):
    import torch

    from cellerator_amd import qcsr_spmm
    rng = np.random.default_rng(40 + bits)
    fx = quantized_fixture(oracle, rng, 900, 1700, 60.0, bits, oracle.PER_GENE_AFFINE,
                           empty_every=13)
    m = to_device_qcsr(fx)
    w_host = (rng.standard_normal((fx["cols"], 64)) * 0.02).astype(np.float16)
    w = torch.from_numpy(w_host).cuda()
    y = torch.full((fx["rows"], 64), float("nan"), device="cuda")
    r = H.run(qcsr_case(m, w, y))
    assert (r.prepare_status, r.status) == (H.OK, H.OK), (r.message, r.engine)
    torch.cuda.synchronize()
    direct = qcsr_spmm(m, w)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), direct.view(torch.int32))
    ref, mag = oracle.qcsr_spmm_referee(bits, fx["policy"], fx["rows"], fx["cols"], fx["row_ptr"],
                                        fx["packed_row_ptr"], fx["col_idx"], fx["packed"],
                                        fx["scales"], fx["offsets"], None, w_host)
    check_against_referee(oracle, ref, mag, y.cpu().numpy())


def test_rebinding_without_reprepare(oracle):
    import torch

    from cellerator_amd import qcsr_spmm
    rng = np.random.default_rng(7)
    fx = quantized_fixture(oracle, rng, 500, 800, 40.0, 4, oracle.PER_GENE_AFFINE)
    m = to_device_qcsr(fx)
    w1 = (torch.randn(fx["cols"], 128, device="cuda") * 0.02).half()
    w2 = (torch.randn(fx["cols"], 128, device="cuda") * 0.02).half()
    y1 = torch.empty(fx["rows"], 128, device="cuda")
    y2 = torch.empty(fx["rows"], 128, device="cuda")
    c = qcsr_case(m, w1, y1)
    c.w2, c.y2 = w2.data_ptr(), y2.data_ptr()
    r = H.run(c)
    assert (r.status, r.second_status) == (H.OK, H.OK), r.message
    torch.cuda.synchronize()
    assert torch.equal(y1, qcsr_spmm(m, w1))
    assert torch.equal(y2, qcsr_spmm(m, w2))


def test_plain_f32_csr_through_reference_core():
    import torch

    from cellerator_amd import QcsrMatrix, qcsr_spmm
    # tests/sparse_ops_runtime_test.cu:140-161: 3x3 x 3x2 -> {201, 402, 430, 860, 5, 10}
    row_ptr = torch.tensor([0, 2, 4, 5], dtype=torch.int32).cuda()
    col_idx = torch.tensor([0, 2, 1, 2, 0], dtype=torch.int32).cuda()
    vals = torch.tensor([1, 2, 3, 4, 5], dtype=torch.float32).cuda()
    m = QcsrMatrix(3, 3, 0, row_ptr, col_idx, values=vals)
    w = torch.tensor([[1, 2], [10, 20], [100, 200]], dtype=torch.float32).cuda()
    y = torch.zeros(3, 2, device="cuda")
    r = H.run(qcsr_case(m, w, y))
    assert r.status == H.OK, r.message
    torch.cuda.synchronize()
    assert y.cpu().numpy().ravel().tolist() == [201.0, 402.0, 430.0, 860.0, 5.0, 10.0]
    assert torch.equal(y, qcsr_spmm(m, w))


def bell_case(m, w, y, workspace=None):
    import torch

    d = m.descriptor()
    view = type(d).from_buffer_copy(d)
    view.values = None
    dense = {torch.bfloat16: H.NT_BF16, torch.float16: H.NT_F16, torch.float32: H.NT_F32}
    vals = m.values
    c = H.HCase(kind=H.KIND_BELL, view=C.addressof(view), view_bytes=C.sizeof(view), variant=0,
                rows=m.rows, cols=m.cols, out_cols=w.shape[1], block_size=m.block_size,
                sparse_type=dense[vals.dtype], dense_type=dense[w.dtype],
                nnz=m.rows * m.ell_cols, values=vals.data_ptr(), value_count=vals.numel(),
                value_bytes=vals.numel() * vals.element_size(), w=w.data_ptr(),
                w_ld=w.stride(0), y=y.data_ptr(), y_ld=y.stride(0),
                workspace=_ptr(workspace),
                workspace_bytes=0 if workspace is None else workspace.numel(),
                stream=torch.cuda.current_stream().cuda_stream, device=torch.cuda.current_device())
    c._keep = (view, m, w, y, workspace)
    return c


def _bell(n_rows_blocks=40, cols=1000, width=9, seed=3):
    import torch

    from cellerator_amd import BellMatrix
    from tests.test_bell_gpu import _bf16_round, random_bell
    rng = np.random.default_rng(seed)
    idx, vals = random_bell(rng, 32 * n_rows_blocks, cols, 32, width)
    vbits = _bf16_round(vals)
    m = BellMatrix(32 * n_rows_blocks, cols, 32, width * 32,
                   torch.from_numpy(idx.view(np.int32)).cuda(),
                   values=torch.from_numpy(vbits.view(np.int16)).view(torch.bfloat16).cuda())
    return m, rng


@pytest.mark.parametrize("n", [64, 256])
def test_blocked_ell_mfma_through_reference_core(n):
    import torch

    from cellerator_amd import bell_pack_rhs, bell_spmm_packed
    m, rng = _bell()
    w = (torch.randn(m.cols, n, device="cuda") * 0.02).bfloat16()
    y = torch.empty(m.rows, n, device="cuda")
    ws = torch.empty(((m.cols + 31) // 32) * 32 * n * 2, dtype=torch.uint8, device="cuda")
    r = H.run(bell_case(m, w, y, ws))
    assert (r.prepare_status, r.status) == (H.OK, H.OK), (r.message, r.engine)
    assert r.kernel_high == 2 and r.workspace_bytes == ws.numel()
    torch.cuda.synchronize()
    direct = bell_spmm_packed(m, bell_pack_rhs(w), n)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), direct.view(torch.int32))


def test_blocked_ell_generic_through_reference_core():
    import torch

    from cellerator_amd import bell_spmm
    m, rng = _bell(seed=5)
    w = torch.randn(m.cols, 96, device="cuda") * 0.02
    y = torch.empty(m.rows, 96, device="cuda")
    r = H.run(bell_case(m, w, y))
    assert (r.prepare_status, r.status) == (H.OK, H.OK), (r.message, r.engine)
    assert r.kernel_high == 3
    torch.cuda.synchronize()
    assert torch.equal(y, bell_spmm(m, w))


def test_cpbp_through_reference_core(oracle):
    import torch

    from cellerator_amd import cpbp, cpbp_reduce
    from tests.test_cpbp_build import random_csr, random_plan
    rng = np.random.default_rng(17)
    plan = random_plan(rng, 700)
    offs, feats, vals = random_csr(rng, 1500, 700, 30.0, np.float32)
    t = cpbp.build_tiles(plan, offs, feats, vals, group_width=64, window_size=256)
    dev = cpbp.to_device(plan, t)
    w = torch.from_numpy(rng.standard_normal(700).astype(np.float32)).cuda()
    y = torch.empty(1500, device="cuda")
    d = dev.descriptor()
    view = type(d).from_buffer_copy(d)
    view.values = None
    c = H.HCase(kind=H.KIND_CPBP, view=C.addressof(view), view_bytes=C.sizeof(view), variant=0,
                rows=1500, cols=700, out_cols=0, block_size=0, sparse_type=H.NT_F32,
                dense_type=H.NT_F32, nnz=int(t.req["nnz_count"]), values=dev.values.data_ptr(),
                value_count=dev.values.numel(), value_bytes=dev.values.numel() * 4,
                w=w.data_ptr(), w_ld=1, y=y.data_ptr(), y_ld=1,
                stream=torch.cuda.current_stream().cuda_stream, device=torch.cuda.current_device())
    r = H.run(c)
    assert (r.prepare_status, r.status) == (H.OK, H.OK), (r.message, r.engine)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), cpbp_reduce(dev, w).view(torch.int32))
    ref, mag = oracle.cpbp_canonical_f64(offs, feats, vals, w.cpu().numpy())
    assert np.all(np.abs(y.cpu().numpy() - ref) <= 1e-5 + 1e-5 * np.abs(ref) + 2.0 ** -22 * mag)


def test_graph_capture_replays_match_eager(oracle):
    """The prepared run captured in a HIP graph (candidate_graph_capture), replayed with
    new W contents, eager work and synchronizations between replays."""
    import torch

    from cellerator_amd import qcsr_spmm
    rng = np.random.default_rng(23)
    fx = quantized_fixture(oracle, rng, 700, 1200, 50.0, 4, oracle.PER_GENE_AFFINE)
    m = to_device_qcsr(fx)
    w = (torch.randn(fx["cols"], 64, device="cuda") * 0.02).half()
    y = torch.empty(fx["rows"], 64, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up launch outside capture
        assert H.run(qcsr_case(m, w, y)).status == H.OK
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        r = H.run(qcsr_case(m, w, y))
    assert r.status == H.OK, r.message
    for step in range(4):
        w.copy_((torch.randn(fx["cols"], 64, device="cuda") * 0.02).half())
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        eager = qcsr_spmm(m, w)
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {step} differs"


@pytest.mark.parametrize("kind,affine", [(7, False), (6, True), (2, True), (0, True)])
def test_quantized_csr_epilogue_through_reference_core(oracle, kind, affine):
    """problem.operation = spmm_operation(kind, affine): bias through inputs[2], alpha / beta
    through scalar bindings with Y updated in place; bitwise equal to the C-ABI call with the
    same epilogue, and within tolerance of the referee."""
    import torch

    from cellerator_amd import Epilogue, qcsr_spmm
    rng = np.random.default_rng(80 + kind)
    fx = quantized_fixture(oracle, rng, 400, 900, 50.0, 4, oracle.PER_GENE_AFFINE)
    m = to_device_qcsr(fx)
    w_host = (rng.standard_normal((fx["cols"], 64)) * 0.05).astype(np.float16)
    w = torch.from_numpy(w_host).cuda()
    c0 = rng.standard_normal((fx["rows"], 64)).astype(np.float32)
    bias = (rng.standard_normal(64) * 0.5).astype(np.float32) if kind in (1, 5, 6, 7) else None
    bias_dev = None if bias is None else torch.from_numpy(bias).cuda()
    alpha, beta = (0.5, -1.5) if affine else (1.0, 0.0)
    y = torch.from_numpy(c0.copy()).cuda()
    c = qcsr_case(m, w, y)
    c.fused, c.epilogue_kind, c.affine = 1, kind, int(affine)
    c.alpha, c.beta = alpha, beta
    c.bias = _ptr(bias_dev)
    r = H.run(c, "f64_scalars" if kind == 2 else "none")
    assert (r.prepare_status, r.status) == (H.OK, H.OK), (r.message, r.engine)
    torch.cuda.synchronize()
    direct = torch.from_numpy(c0.copy()).cuda()
    qcsr_spmm(m, w, out=direct, epilogue=Epilogue(kind, alpha, beta, bias_dev,
                                                  direct if affine else None))
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), direct.view(torch.int32))
    decoded = oracle.decode_csr(4, fx["policy"], fx["row_ptr"], fx["packed_row_ptr"],
                                fx["col_idx"], fx["packed"], fx["scales"], fx["offsets"], None)
    ref = oracle.spmm_referee(fx["rows"], fx["cols"], 64, fx["row_ptr"], fx["col_idx"], decoded,
                              w_host, alpha=alpha, beta=beta, c0=c0 if beta else None,
                              epilogue=kind, bias=bias)
    cmp = oracle.compare(ref, y.cpu().numpy(), 1e-4, 1e-4)
    assert cmp["status"] == 0 and cmp["within_tolerance"], cmp


def test_blocked_ell_epilogue_through_reference_core():
    import torch

    from cellerator_amd import Epilogue, bell_pack_rhs, bell_spmm_packed
    m, rng = _bell(seed=9)
    n = 128
    w = (torch.randn(m.cols, n, device="cuda") * 0.02).bfloat16()
    bias = torch.randn(n, device="cuda")
    c0 = torch.randn(m.rows, n, device="cuda")
    y = c0.clone()
    ws = torch.empty(((m.cols + 31) // 32) * 32 * n * 2, dtype=torch.uint8, device="cuda")
    c = bell_case(m, w, y, ws)
    c.fused, c.epilogue_kind, c.affine, c.alpha, c.beta = 1, 6, 1, 2.0, 0.25
    c.bias = bias.data_ptr()
    r = H.run(c)
    assert (r.prepare_status, r.status) == (H.OK, H.OK), (r.message, r.engine)
    torch.cuda.synchronize()
    direct = c0.clone()
    bell_spmm_packed(m, bell_pack_rhs(w), n, out=direct,
                     epilogue=Epilogue(6, 2.0, 0.25, bias, direct))
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), direct.view(torch.int32))


# ---------------------------------------------------------------- prepared physical state

def _time_ms(fn, reps: int) -> float:
    import torch
    fn()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / reps


@pytest.mark.parametrize("bits", [4, 8])
def test_quantized_csr_prepared_state_runs_the_fast_form(oracle, bits):
    """prepare_quantized_csr_state: the column-order check and interleaved pairs make the
    core's launch run the sorted + pairs kernel, bitwise equal to the direct C-ABI call on the
    same prepared matrix; a new value generation falls back to the plane's own arrays."""
    import torch

    from cellerator_amd import qcsr_check_columns, qcsr_pack_gene_affine, qcsr_spmm
    rng = np.random.default_rng(90 + bits)
    fx = quantized_fixture(oracle, rng, 3000, 2500, 80.0, bits, oracle.PER_GENE_AFFINE, empty_every=11)
    m = to_device_qcsr(fx)
    w = torch.from_numpy((rng.standard_normal((fx["cols"], 64)) * 0.02).astype(np.float16)).cuda()
    y = torch.full((fx["rows"], 64), float("nan"), device="cuda")
    pairs = torch.empty(2 * fx["cols"], dtype=torch.float32, device="cuda")
    c = qcsr_case(m, w, y)
    c.pairs, c.check_columns = pairs.data_ptr(), 1
    r = H.run(c)
    assert (r.prepare_status, r.state_status, r.status) == (H.OK, H.OK, H.OK), (r.message, r.engine)
    assert r.dispatch == b"qcsr:pairs+sorted"
    torch.cuda.synchronize()
    fast = qcsr_check_columns(qcsr_pack_gene_affine(m))
    assert fast.flags == 1
    direct = qcsr_spmm(fast, w)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), direct.view(torch.int32))
    ref, mag = oracle.qcsr_spmm_referee(bits, 1, fx["rows"], fx["cols"], fx["row_ptr"],
                                        fx["packed_row_ptr"], fx["col_idx"], fx["packed"],
                                        fx["scales"], fx["offsets"], None, w.cpu().numpy())
    check_against_referee(oracle, ref, mag, y.cpu().numpy())


def test_quantized_csr_view_flags_are_not_the_callers():
    """A view that arrives with flags set is rejected: only the backend's own check sets
    CX_QCSR_COLUMNS_SORTED."""
    import torch

    from cellerator_amd import QcsrMatrix
    row_ptr = torch.tensor([0, 2, 4, 5], dtype=torch.int32).cuda()
    col_idx = torch.tensor([2, 0, 1, 2, 0], dtype=torch.int32).cuda()  # row 0 out of order
    vals = torch.tensor([1, 2, 3, 4, 5], dtype=torch.float32).cuda()
    m = QcsrMatrix(3, 3, 0, row_ptr, col_idx, values=vals, flags=1)
    w = torch.ones(3, 64, dtype=torch.float32, device="cuda")
    y = torch.zeros(3, 64, device="cuda")
    r = H.run(qcsr_case(m, w, y))
    assert r.status == H.INVALID_LAUNCH and b"flags" in r.message
    # the backend's own check finds the disorder and keeps the checked path
    m.flags = 0
    c = qcsr_case(m, w, y)
    c.check_columns = 1
    r = H.run(c)
    assert (r.state_status, r.status) == (H.OK, H.OK), r.message
    assert r.dispatch == b"qcsr:plain"
    torch.cuda.synchronize()
    assert y[:, 0].cpu().tolist() == [3.0, 7.0, 5.0]


def test_prepared_quantized_csr_launch_costs_no_more_than_direct(oracle):
    """The core's prepared launch runs the same kernel as the direct call: over 20 launches
    of a C2-sized slice the time per launch stays within 5% (plus 20 us of host dispatch)."""
    import torch

    from cellerator_amd import qcsr_check_columns, qcsr_pack_gene_affine, qcsr_spmm
    from cellerator_amd.synth import C3, dense_normal, generate_qcsr
    m = generate_qcsr(C3.scaled(30000))
    w = dense_normal((m.cols, 64), 0.02, torch.float16, seed=5)
    y = torch.empty((m.rows, 64), device="cuda")
    pairs = torch.empty(2 * m.cols, dtype=torch.float32, device="cuda")
    c = qcsr_case(m, w, y)
    c.pairs, c.check_columns, c.repeats = pairs.data_ptr(), 1, 20
    r = H.run(c)  # prepares the state once; also the warm-up
    assert r.status == H.OK and r.dispatch == b"qcsr:pairs+sorted", (r.message, r.engine)
    fast = qcsr_check_columns(qcsr_pack_gene_affine(m))
    out = torch.empty_like(y)
    direct_ms = _time_ms(lambda: qcsr_spmm(fast, w, out=out), 20)
    core_ms = _time_ms(lambda: H.run(c), 1) / 20.0
    print(f"direct {direct_ms:.4f} ms, through the core {core_ms:.4f} ms per launch")
    assert core_ms <= direct_ms * 1.05 + 0.02


def test_blocked_ell_prepared_panel_and_groups(monkeypatch):
    """prepare_blocked_ell_state: a prepacked panel and the grouping plan make the core's
    launch run the grouped kernel without repacking, bitwise equal to the direct grouped call;
    a launch with another W pointer repacks into the workspace."""
    import torch

    from cellerator_amd import bell_pack_rhs, bell_plan_groups, bell_spmm_grouped
    from cellerator_amd import _native as N
    m, rng = _bell(n_rows_blocks=64, seed=13)
    n = 128
    w = (torch.randn(m.cols, n, device="cuda") * 0.02).bfloat16()
    y = torch.empty(m.rows, n, device="cuda")
    ws = torch.empty(((m.cols + 31) // 32) * 32 * n * 2, dtype=torch.uint8, device="cuda")
    panel = torch.empty(((m.cols + 31) // 32) * 32 * n, dtype=torch.bfloat16, device="cuda")
    groups = bell_plan_groups(m)
    gd = groups.descriptor()
    c = bell_case(m, w, y, ws)
    c.panel, c.groups = panel.data_ptr(), C.addressof(gd)
    c._keep2 = (panel, groups, gd)
    r = H.run(c)
    assert (r.state_status, r.status) == (H.OK, H.OK), (r.message, r.engine)
    assert r.dispatch == b"bell:grouped+panel"
    torch.cuda.synchronize()
    direct = bell_spmm_grouped(m, bell_pack_rhs(w), groups, n)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), direct.view(torch.int32))
    assert torch.equal(panel, bell_pack_rhs(w))
    # second launch with a different W (not the packed one): repacked into the workspace
    w2 = (torch.randn(m.cols, n, device="cuda") * 0.02).bfloat16()
    y2 = torch.empty_like(y)
    c.w2, c.y2 = w2.data_ptr(), y2.data_ptr()
    r = H.run(c)
    assert (r.status, r.second_status) == (H.OK, H.OK), r.message
    assert r.dispatch == b"bell:grouped+repack"
    torch.cuda.synchronize()
    assert torch.equal(y2.view(torch.int32), bell_spmm_grouped(m, bell_pack_rhs(w2), groups, n).view(torch.int32))
    del N


def test_cpbp_native_tile_view_through_reference_core(oracle):
    """The reference's native tile view (cx_native_tile_view, its layout) as the CP-BP
    operand: built on a validated host CPK1 image with its sidecars, moved to the uploaded
    copy (cx_native_tile_view_rebind), bound with the image's values as the value plane. The
    core runs it (dispatch "cpbp:native-tile"), bitwise equal to the reduction on the image's
    tiles; a view whose values are not the bound plane is rejected."""
    import torch

    from cellerator_amd import _native as N
    from cellerator_amd import cpbp, cpbp_reduce, cpk1
    from tests.test_cpbp_build import random_csr, random_plan
    rng = np.random.default_rng(29)
    plan = random_plan(rng, 600)
    offs, feats, vals = random_csr(rng, 2100, 600, 20.0, np.float16)
    tiles = cpbp.build_tiles(plan, offs, feats, vals, group_width=32, window_size=1024)
    meta = cpk1.Metadata(0xA11, 0xB22, 5_000, global_row_begin=700, group_width=32, window_size=1024)
    image, host = cpk1.write_image(plan, tiles, meta)  # host: the validated view of `image`
    lib = N.engine()
    req = N.CxNativeTileRequirements()
    assert lib.cx_query_native_tile_requirements_from_cpk1_host(C.byref(host), C.byref(req)) == 0, lib.cx_last_error()
    unions = np.zeros(req.union_mask_count, np.uint32)
    offsets = np.zeros(req.packed_offset_count, np.uint32)
    metrics = (N.CxNativeTileBlockMetrics * req.block_metric_count)()
    bufs = N.CxNativeTileBuffers(unions.size, unions.ctypes.data, offsets.size, offsets.ctypes.data,
                                 len(metrics), C.addressof(metrics))
    view_host = N.CxNativeTileView()
    assert lib.cx_build_native_tile_view_from_cpk1_host(C.byref(host), C.byref(bufs), C.byref(view_host)) == 0
    dev = cpk1.upload(host, image)
    view = N.CxNativeTileView()
    assert lib.cx_native_tile_view_rebind(C.byref(view_host), image.ctypes.data, image.nbytes,
                                          dev.image.data_ptr(), C.byref(view)) == 0
    assert view.tiles.values == dev.view.tiles.values and view.union_gene_masks == unions.ctypes.data
    nnz = int(view.tiles.nnz_count)
    w = torch.from_numpy(rng.standard_normal(600).astype(np.float32)).cuda()
    y = torch.full((2100,), float("nan"), device="cuda")

    def case(values_ptr):
        return H.HCase(kind=H.KIND_CPBP, view=C.addressof(view), view_bytes=C.sizeof(view), variant=0,
                       rows=2100, cols=600, out_cols=0, block_size=0, sparse_type=H.NT_F16,
                       dense_type=H.NT_F32, nnz=nnz, values=values_ptr, value_count=nnz, value_bytes=nnz * 2,
                       w=w.data_ptr(), w_ld=1, y=y.data_ptr(), y_ld=1,
                       stream=torch.cuda.current_stream().cuda_stream, device=torch.cuda.current_device())

    r = H.run(case(view.tiles.values))
    assert (r.prepare_status, r.status) == (H.OK, H.OK), (r.message, r.engine)
    assert r.dispatch == b"cpbp:native-tile"
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), cpbp_reduce(dev, w).view(torch.int32))
    other = torch.empty(nnz, dtype=torch.float16, device="cuda")
    r = H.run(case(other.data_ptr()))
    assert r.status == H.INVALID_LAUNCH


def test_cpbp_checked_entry_rows_through_reference_core():
    """prepare_cpbp_state with a validated reduction view and an entry-rows array: the core's
    launch reads each entry's row and block start from it (dispatch
    "cpbp:checked+entry-rows"), bitwise equal to the reduction from the descriptors; without
    the array it keeps the descriptor walk ("cpbp:checked")."""
    import torch

    from cellerator_amd import cpbp_reduce, cpk1
    from tests.test_cpk1 import _reduction_view, build_reference_image
    _, _, image, view = build_reference_image()
    dev = cpk1.upload(cpk1.validate(image, cpk1.expected_of(view)), image)
    rv = _reduction_view(dev.view)
    d = dev.descriptor()
    tview = type(d).from_buffer_copy(d)
    tview.values = None
    half = int(d.value_dtype) == 1  # CELLERATOR_DTYPE_F16: the image's values are fp16
    values_ptr = int(d.values)  # the values section inside the uploaded image
    w = torch.from_numpy((0.5 + 0.125 * np.arange(int(d.feature_count))).astype(np.float32)).cuda()
    expect = cpbp_reduce(dev, w)
    n_entries = int(d.row_block_entry_count)
    for with_rows in (True, False):
        rows = torch.full((max(n_entries, 1),), -1, dtype=torch.int32, device="cuda")
        y = torch.full((int(d.row_count),), -3.0, device="cuda")
        c = H.HCase(kind=H.KIND_CPBP, view=C.addressof(tview), view_bytes=C.sizeof(tview), variant=0,
                    rows=int(d.row_count), cols=int(d.feature_count), out_cols=0, block_size=0,
                    sparse_type=H.NT_F16 if half else H.NT_F32,
                    dense_type=H.NT_F32, nnz=int(d.nnz_count), values=values_ptr,
                    value_count=int(d.nnz_count), value_bytes=int(d.nnz_count) * (2 if half else 4),
                    w=w.data_ptr(), w_ld=1, y=y.data_ptr(), y_ld=1,
                    stream=torch.cuda.current_stream().cuda_stream, device=torch.cuda.current_device(),
                    reduction_view=C.addressof(rv),
                    entry_rows=rows.data_ptr() if with_rows else None,
                    entry_rows_capacity=rows.numel() if with_rows else 0)
        r = H.run(c)
        assert (r.prepare_status, r.state_status, r.status) == (H.OK, H.OK, H.OK), (r.message, r.engine)
        assert r.dispatch == (b"cpbp:checked+entry-rows" if with_rows else b"cpbp:checked")
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), expect.view(torch.int32))
        if with_rows:
            assert bool((rows[:n_entries] >= 0).all())
