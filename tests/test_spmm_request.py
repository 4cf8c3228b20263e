"""The backend-neutral SpMM request (spmm_request.cpp) against the reference's own contract
test (tests/math_operation_contract_test.cc): the request fixture (:29-50) validates, its
operation signature is the reference's recorded value (:69-72), layout, structure and GELU
mode change the signature, every rejection rule returns the reference's code (:75-208), and
the trivial-work classes are the reference's (:210-240). The struct layout is the byte
layout of the reference's spmm_request (include/Cellerator/compute/math/operation.hh:136-164)."""
from __future__ import annotations

import ctypes as C

import pytest

from cellerator_amd import spmm_request as R


def fixture() -> R.CxSpmmRequest:
    """math_operation_contract_test.cc:29-50."""
    r = R.new_request()
    r.m, r.k, r.n, r.sparse_nnz = 8, 16, 32, 24
    r.sparse_structure.identity_version, r.sparse_structure.value = 1, 0xC511E7A70
    r.dense_rhs_leading_dimension = r.output_leading_dimension = 32
    r.sparse_storage_type_code = r.dense_storage_type_code = R.F16
    r.output_storage_type_code = r.compute_type_code = r.accumulation_type_code = R.F32
    r.alpha, r.beta = R.scalar_f32(1.0), R.scalar_f32(0.0)
    for o in (r.sparse_feature_order, r.dense_feature_order):
        o.feature_count, o.feature_axis_identity_version, o.feature_axis_identity = 16, 1, 0x12345678
    return r


def bound(r=None):
    """bound_request_fixture (:52-62): three distinct non-null addresses."""
    keep = (C.c_int(), C.c_int(), C.c_int())
    b = R.CxSpmmBindings(C.addressof(keep[0]), C.addressof(keep[1]), C.addressof(keep[2]), None, 0, 0, 0)
    b._keep = keep
    return (r if r is not None else fixture()), b


def test_struct_layout_is_the_references():
    S = R.CxSpmmRequest
    assert C.sizeof(S) == 264
    expected = {"m": 8, "sparse_nnz": 32, "sparse_structure": 40, "transpose_sparse": 56, "output_layout": 68,
                "dense_rhs_leading_dimension": 72, "sparse_storage_type_code": 88, "accumulation_type_code": 104,
                "alpha": 112, "beta": 128, "determinism": 144, "workspace": 152, "reuse": 168, "epilogue": 184,
                "sparse_feature_order": 200, "dense_feature_order": 232}
    for name, off in expected.items():
        assert getattr(S, name).offset == off, name
    assert C.sizeof(R.CxFeatureOrderIdentity) == 32 and C.sizeof(R.CxSpmmBindings) == 56


def test_signature_and_order_identity():
    r = fixture()
    assert R.validate(r)[0] == "ok"
    first = R.signature(r)
    assert first == R.signature(r)
    assert first == (0xA7E9D18214BE8880, 0xC02E69BB5DAE6EFB)  # :69-72
    r.dense_rhs_layout = R.COLUMN_MAJOR
    assert R.signature(r) != first
    r = fixture()
    r.sparse_structure.value += 1
    assert R.signature(r) != first
    r = fixture()
    r.dense_feature_order.kind, r.dense_feature_order.packing_geometry_identity = R.PACKED, 0xABCD
    assert R.validate(r)[0] == "feature_order_mismatch"


def test_packed_plan_identity_mismatch():
    r = fixture()
    r.sparse_feature_order.kind = r.dense_feature_order.kind = R.PACKED
    r.sparse_feature_order.packing_geometry_identity = 0x100
    r.dense_feature_order.packing_geometry_identity = 0x200
    assert R.validate(r)[0] == "feature_order_mismatch"
    r.dense_feature_order.packing_geometry_identity = 0x100
    assert R.validate(r)[0] == "ok"


def test_binding_and_policy_validation():
    r, b = bound()
    assert R.validate(r, b)[0] == "ok"
    b.dense_rhs = None
    assert R.validate(r, b)[0] == "missing_binding"
    r, b = bound()
    r.workspace.kind = R.CALLER_LIMIT
    assert R.validate(r, b)[0] == "invalid_workspace_policy"
    r, b = bound()
    r.reuse.kind = R.PERSISTENT
    assert R.validate(r, b)[0] == "invalid_reuse"
    r.reuse.expected_run_count = 0
    assert R.validate(r, b)[0] == "ok"


@pytest.mark.parametrize("change,code", [
    (lambda r: setattr(r, "sparse_nnz", r.m * r.k + 1), "invalid_shape"),
    (lambda r: (setattr(r, "m", (1 << 64) - 1), setattr(r, "n", 2)), "invalid_shape"),
    (lambda r: (setattr(r, "k", (1 << 64) - 1), setattr(r, "n", 2)), "invalid_shape"),
    (lambda r: setattr(r, "dense_rhs_layout", 99), "invalid_layout"),
    (lambda r: setattr(r, "dense_rhs_leading_dimension", r.n - 1), "invalid_layout"),
    (lambda r: setattr(r, "determinism", 99), "invalid_determinism"),
    # the remaining rules of operation.cc:119-249, each in isolation
    (lambda r: setattr(r, "schema_version", 2), "unsupported_version"),
    (lambda r: (setattr(r, "m", 0), setattr(r, "sparse_nnz", 1)), "invalid_shape"),
    (lambda r: setattr(r, "transpose_dense", 7), "invalid_layout"),
    (lambda r: setattr(r, "output_leading_dimension", 31), "invalid_layout"),
    (lambda r: setattr(r, "compute_type_code", 9), "invalid_type"),
    (lambda r: setattr(r, "beta", R.scalar_f64(0.0)), "invalid_scalar"),
    (lambda r: setattr(r.alpha, "bits", 1 << 40), "invalid_scalar"),
    (lambda r: setattr(r.workspace, "byte_limit", 4096), "invalid_workspace_policy"),
    (lambda r: (setattr(r.reuse, "kind", R.BOUNDED), setattr(r.reuse, "expected_run_count", 0)), "invalid_reuse"),
    (lambda r: setattr(r.sparse_structure, "value", 0), "invalid_identity"),
    (lambda r: setattr(r.sparse_feature_order, "feature_count", 15), "invalid_feature_order"),
    (lambda r: setattr(r.dense_feature_order, "packing_geometry_identity", 5), "invalid_feature_order"),
    (lambda r: setattr(r.epilogue, "kind", 8), "invalid_epilogue"),
    (lambda r: setattr(r.epilogue, "kind", 1), "missing_bias"),
    (lambda r: setattr(r.epilogue, "bias_element_count", 32), "unexpected_bias"),
])
def test_rejections(change, code):
    r = fixture()
    change(r)
    assert R.validate(r)[0] == code


def test_bias_contract():
    r, b = bound()
    r.epilogue.kind, r.epilogue.bias_type_code, r.epilogue.bias_element_count = 5, R.F32, r.n
    assert R.validate(r, b)[0] == "missing_bias"
    bias = (C.c_float * 32)()
    b.bias = C.addressof(bias)
    assert R.validate(r, b)[0] == "ok"
    r.epilogue.kind, r.epilogue.bias_type_code, r.epilogue.bias_element_count = 2, 0, 0
    assert R.validate(r, b)[0] == "unexpected_bias"


def test_explicit_gelu_semantics():
    exact, approx = fixture(), fixture()
    exact.epilogue.kind, approx.epilogue.kind = 3, 4
    assert R.validate(exact)[0] == "ok" and R.validate(approx)[0] == "ok"
    assert R.signature(exact) != R.signature(approx)
    r, b = bound()
    r.epilogue.kind, r.epilogue.bias_type_code, r.epilogue.bias_element_count = 6, R.F32, r.n
    bias = (C.c_float * 32)()
    b.bias = C.addressof(bias)
    assert R.validate(r, b)[0] == "ok"


def test_trivial_semantics():
    r = fixture()
    r.m, r.sparse_nnz = 0, 0
    assert R.classify(r) == R.NO_OUTPUT
    r = fixture()
    r.alpha = R.scalar_f32(0.0)
    assert R.classify(r) == R.EPILOGUE_ONLY
    keep = C.c_int()
    b = R.CxSpmmBindings(None, None, C.addressof(keep), None, 0, 0, 0)
    assert R.validate(r, b)[0] == "ok"  # alpha = 0 needs no sparse or dense binding
    r = fixture()
    r.k, r.sparse_nnz = 0, 0
    for o in (r.sparse_feature_order, r.dense_feature_order):
        o.feature_count = 0
    assert R.classify(r) == R.EPILOGUE_ONLY
