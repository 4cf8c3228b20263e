"""The request-driven quantized CSR SpMM (cx_qcsr_spmm_fwd_request): a validated math
request runs the same kernels as cx_qcsr_spmm_fwd_epilogue (bitwise equal outputs, with
alpha, beta in place and a bias epilogue), epilogue-only requests (alpha 0) write
act(beta C + bias) without reading the operands (NaN weights do not leak; no sparse or
dense binding is needed), and rejected requests and unsupported forms fail before any
launch."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import quantized_fixture, to_device_qcsr

pytestmark = pytest.mark.gpu


def _setup(oracle, n=64):
    import torch
    rng = np.random.default_rng(77)
    fx = quantized_fixture(oracle, rng, 900, 1500, 20.0, 4, 1)
    m = to_device_qcsr(fx)
    w = torch.from_numpy((rng.standard_normal((1500, n)) * 0.05).astype(np.float16)).cuda()
    c0 = torch.from_numpy(rng.standard_normal((900, n)).astype(np.float32)).cuda()
    bias = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).cuda()
    return m, w, c0, bias


def test_request_matches_direct_epilogue(oracle):
    import torch

    from cellerator_amd import Epilogue, qcsr_spmm
    from cellerator_amd import spmm_request as R
    m, w, c0, bias = _setup(oracle)
    r = R.qcsr_request(m, 64, alpha=1.25, beta=0.5, epilogue=6)
    assert R.validate(r)[0] == "ok"
    y = c0.clone()
    R.qcsr_spmm_request(r, m, w, y, bias)
    want = c0.clone()
    qcsr_spmm(m, w, out=want, epilogue=Epilogue(6, 1.25, 0.5, bias, want))
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), want.view(torch.int32))
    # plain product
    r = R.qcsr_request(m, 64)
    y = torch.empty_like(c0)
    R.qcsr_spmm_request(r, m, w, y)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), qcsr_spmm(m, w).view(torch.int32))


def test_epilogue_only_reads_no_operand(oracle):
    import torch

    from cellerator_amd import spmm_request as R
    m, w, c0, bias = _setup(oracle)
    w_nan = torch.full_like(w, float("nan"))
    r = R.qcsr_request(m, 64, alpha=0.0, beta=2.0, epilogue=5)
    y = c0.clone()
    R.qcsr_spmm_request(r, m, w_nan, y, bias)
    torch.cuda.synchronize()
    want = torch.relu(2.0 * c0 + bias)
    assert torch.equal(y, want)
    y = c0.clone()
    R.qcsr_spmm_request(r, None, None, y, bias)  # no sparse or dense binding at all
    torch.cuda.synchronize()
    assert torch.equal(y, want)


def test_rejected_and_unsupported_requests(oracle):
    import torch

    from cellerator_amd import _native as N
    from cellerator_amd import spmm_request as R
    m, w, c0, bias = _setup(oracle)
    y = torch.zeros_like(c0)
    r = R.qcsr_request(m, 64)
    r.dense_feature_order.kind, r.dense_feature_order.packing_geometry_identity = R.PACKED, 9
    with pytest.raises(N.EngineError, match="different feature orders"):
        R.qcsr_spmm_request(r, m, w, y)
    r = R.qcsr_request(m, 64)
    r.transpose_dense = 1
    r.dense_rhs_leading_dimension = 1500
    with pytest.raises(N.EngineError, match="untransposed row-major"):
        R.qcsr_spmm_request(r, m, w, y)
    r = R.qcsr_request(m, 64)
    r.k += 1
    for o in (r.sparse_feature_order, r.dense_feature_order):
        o.feature_count += 1
    with pytest.raises(N.EngineError, match="does not describe the bound matrix"):
        R.qcsr_spmm_request(r, m, w, y)
    torch.cuda.synchronize()
    assert not y.any()
