"""The backend-neutral SpMM request (spmm_request.cpp): ctypes mirrors of cx_spmm_request
and friends (the byte layout of the reference's spmm_request,
include/Cellerator/compute/math/operation.hh:89-186), its validation, operation signature
and trivial-work classification, and the request-driven quantized CSR SpMM."""
from __future__ import annotations

import ctypes as C
import struct
from typing import Optional

import torch

from . import _native as N
from .engine import Epilogue, QcsrMatrix, _require_cuda, _stream  # noqa: F401

u32, u64, p_void = C.c_uint32, C.c_uint64, C.c_void_p
F16, F32, F64, BF16, FP8_E4M3, FP8_E5M2 = 3, 4, 5, 6, 7, 8
CANONICAL, PACKED = 1, 2
ROW_MAJOR, COLUMN_MAJOR = 1, 2
REUSABLE_POOL, CALLER_LIMIT, NO_WORKSPACE = 1, 2, 3
SINGLE_RUN, BOUNDED, PERSISTENT = 1, 2, 3
TRIVIAL_NONE, NO_OUTPUT, EPILOGUE_ONLY = 0, 1, 2
CODES = ["ok", "unsupported_version", "invalid_shape", "invalid_type", "invalid_scalar",
         "invalid_workspace_policy", "invalid_reuse", "invalid_feature_order", "feature_order_mismatch",
         "missing_bias", "unexpected_bias", "invalid_layout", "invalid_identity", "missing_binding",
         "invalid_determinism", "invalid_epilogue"]


class CxFeatureOrderIdentity(C.Structure):
    _fields_ = [("schema_version", u32), ("kind", u32), ("feature_count", u32),
                ("feature_axis_identity_version", u32), ("feature_axis_identity", u64),
                ("packing_geometry_identity", u64)]


class CxSparseStructureIdentity(C.Structure):
    _fields_ = [("schema_version", u32), ("identity_version", u32), ("value", u64)]


class CxScalarValue(C.Structure):
    _fields_ = [("type_code", u32), ("reserved", u32), ("bits", u64)]


class CxWorkspacePolicy(C.Structure):
    _fields_ = [("kind", u32), ("reserved", u32), ("byte_limit", u64)]


class CxExpectedReuse(C.Structure):
    _fields_ = [("kind", u32), ("reserved", u32), ("expected_run_count", u64)]


class CxEpilogueDescriptor(C.Structure):
    _fields_ = [("kind", u32), ("bias_type_code", u32), ("bias_element_count", u64)]


class CxSpmmRequest(C.Structure):
    _fields_ = [("schema_version", u32), ("operation", u32), ("m", u64), ("k", u64), ("n", u64),
                ("sparse_nnz", u64), ("sparse_structure", CxSparseStructureIdentity), ("transpose_sparse", u32),
                ("transpose_dense", u32), ("dense_rhs_layout", u32), ("output_layout", u32),
                ("dense_rhs_leading_dimension", u64), ("output_leading_dimension", u64),
                ("sparse_storage_type_code", u32), ("dense_storage_type_code", u32),
                ("output_storage_type_code", u32), ("compute_type_code", u32), ("accumulation_type_code", u32),
                ("alpha", CxScalarValue), ("beta", CxScalarValue), ("determinism", u32),
                ("workspace", CxWorkspacePolicy), ("reuse", CxExpectedReuse), ("epilogue", CxEpilogueDescriptor),
                ("sparse_feature_order", CxFeatureOrderIdentity), ("dense_feature_order", CxFeatureOrderIdentity)]


class CxSpmmBindings(C.Structure):
    _fields_ = [("sparse_matrix", p_void), ("dense_rhs", p_void), ("output", p_void), ("bias", p_void),
                ("sparse_matrix_identity", u64), ("dense_rhs_identity", u64), ("output_identity", u64)]


class CxOperationSignature(C.Structure):
    _fields_ = [("schema_version", u32), ("operation", u32), ("low", u64), ("high", u64)]


_SIGS = {
    "cx_spmm_request_init": (None, [C.POINTER(CxSpmmRequest)]),
    "cx_scalar_f32": (CxScalarValue, [C.c_float]),
    "cx_scalar_f64": (CxScalarValue, [C.c_double]),
    "cx_validate_spmm_request": (u32, [C.POINTER(CxSpmmRequest), C.POINTER(C.c_char_p)]),
    "cx_validate_math_request": (u32, [C.POINTER(CxSpmmRequest), C.POINTER(CxSpmmBindings), C.POINTER(C.c_char_p)]),
    "cx_make_operation_signature": (CxOperationSignature, [C.POINTER(CxSpmmRequest)]),
    "cx_classify_trivial_operation": (u32, [C.POINTER(CxSpmmRequest)]),
    "cx_qcsr_spmm_fwd_request": (C.c_int, [C.POINTER(CxSpmmRequest), C.POINTER(CxSpmmBindings), p_void]),
}


def _lib():
    lib = N.engine()
    if not getattr(lib, "_request_sigs", False):
        for name, (res, args) in _SIGS.items():
            f = getattr(lib, name)
            f.restype, f.argtypes = res, args
        lib._request_sigs = True
    return lib


def new_request() -> CxSpmmRequest:
    r = CxSpmmRequest()
    _lib().cx_spmm_request_init(C.byref(r))
    return r


def scalar_f32(v: float) -> CxScalarValue:
    return _lib().cx_scalar_f32(v)


def scalar_f64(v: float) -> CxScalarValue:
    return _lib().cx_scalar_f64(v)


def validate(r: CxSpmmRequest, bindings: Optional[CxSpmmBindings] = None) -> tuple[str, str]:
    """(code name, message) of validate_spmm_request, or validate_math_request with bindings."""
    msg = C.c_char_p()
    if bindings is None:
        code = _lib().cx_validate_spmm_request(C.byref(r), C.byref(msg))
    else:
        code = _lib().cx_validate_math_request(C.byref(r), C.byref(bindings), C.byref(msg))
    return CODES[code], msg.value.decode()


def signature(r: CxSpmmRequest) -> tuple[int, int]:
    s = _lib().cx_make_operation_signature(C.byref(r))
    return s.low, s.high


def classify(r: CxSpmmRequest) -> int:
    return int(_lib().cx_classify_trivial_operation(C.byref(r)))


def qcsr_request(m: QcsrMatrix, n: int, rhs_dtype: torch.dtype = torch.float16, *, alpha: float = 1.0,
                 beta: float = 0.0, epilogue: int = 0, structure_identity: int = 0xC511E7A70,
                 feature_axis_identity: int = 0x12345678, ldb: Optional[int] = None,
                 ldc: Optional[int] = None) -> CxSpmmRequest:
    """A request describing Y = act(alpha X W + beta Y + bias) for the matrix m (canonical
    feature order, row-major F16/F32 W [cols, n], F32 Y [rows, n])."""
    r = new_request()
    r.m, r.k, r.n, r.sparse_nnz = m.rows, m.cols, n, m.nnz
    r.sparse_structure.identity_version, r.sparse_structure.value = 1, structure_identity
    r.dense_rhs_leading_dimension = n if ldb is None else ldb
    r.output_leading_dimension = n if ldc is None else ldc
    r.sparse_storage_type_code = F32 if m.bits else (F16 if m.values.dtype == torch.float16 else F32)
    r.dense_storage_type_code = F16 if rhs_dtype == torch.float16 else F32
    r.output_storage_type_code = r.compute_type_code = r.accumulation_type_code = F32
    r.alpha, r.beta = scalar_f32(alpha), scalar_f32(beta)
    r.epilogue.kind = epilogue
    if epilogue in (1, 5, 6, 7):
        r.epilogue.bias_type_code, r.epilogue.bias_element_count = F32, n
    for o in (r.sparse_feature_order, r.dense_feature_order):
        o.kind, o.feature_count = CANONICAL, m.cols
        o.feature_axis_identity_version, o.feature_axis_identity = 1, feature_axis_identity
    return r


def qcsr_spmm_request(r: CxSpmmRequest, m: Optional[QcsrMatrix], rhs: Optional[torch.Tensor], out: torch.Tensor,
                      bias: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Runs the request through cx_qcsr_spmm_fwd_request (bindings from the tensors)."""
    d = m.descriptor() if m is not None else None
    b = CxSpmmBindings(C.addressof(d) if d is not None else None, rhs.data_ptr() if rhs is not None else None,
                       out.data_ptr(), bias.data_ptr() if bias is not None else None, 0, 0, 0)
    N.check("cx_qcsr_spmm_fwd_request", _lib().cx_qcsr_spmm_fwd_request(C.byref(r), C.byref(b), _stream(stream)))
    return out


def f32_bits(v: float) -> int:
    return struct.unpack("<I", struct.pack("<f", v))[0]
