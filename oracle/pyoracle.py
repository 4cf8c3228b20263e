"""ctypes front-end of the CPU oracle (oracle/liboracle.so). TEST INFRASTRUCTURE ONLY:
imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
checker; the engine never imports it. Every function forwards to the C restatement
in oracle.c, whose comments cite the reference file:line each one follows."""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

F16, F32, F64, BF16 = 3, 4, 5, 6
PER_GENE_AFFINE, COLUMN_SCALE_ROW_OFFSET = 1, 2
EPI_NONE, EPI_BIAS, EPI_RELU, EPI_GELU_ERF, EPI_GELU_TANH = 0, 1, 2, 3, 4
EPI_BIAS_RELU, EPI_BIAS_GELU_ERF, EPI_BIAS_GELU_TANH = 5, 6, 7

_lib = None


class Comparison(C.Structure):
    _fields_ = [("element_count", C.c_uint64), ("mismatch_count", C.c_uint64),
                ("non_finite_reference_count", C.c_uint64),
                ("non_finite_candidate_count", C.c_uint64), ("worst_index", C.c_uint64),
                ("max_absolute_error", C.c_double), ("max_relative_error", C.c_double),
                ("mean_absolute_error", C.c_double), ("root_mean_square_error", C.c_double),
                ("within_tolerance", C.c_int)]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


def build() -> Path:
    """Compiles liboracle.so from oracle.c / oracle_mt.c (gcc, no GPU)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


REFERENCE_ROOT = Path("/root/reference")
REF_DIR = HERE / "_ref"


def build_reference() -> bool:
    """Where the reference tree is present, compiles its host-only operation core from
    source into oracle/_ref/ together with the CP-Math test harness (`make ref`).
    Elsewhere (the GPU box) the prebuilt files are used as they are."""
    if not (REFERENCE_ROOT / "src/compute/math/operation_core/operation_core.cc").exists():
        return False
    subprocess.run(["make", "-s", "-C", str(HERE), "ref", f"REF={REFERENCE_ROOT}"], check=True)
    return True


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = C.CDLL(str(LIB_PATH))
        _lib.or_half_to_float.restype = C.c_float
        _lib.or_half_to_float.argtypes = [C.c_uint16]
        _lib.or_float_to_half.restype = C.c_uint16
        _lib.or_float_to_half.argtypes = [C.c_float]
        _lib.or_bf16_to_float.restype = C.c_float
        _lib.or_bf16_to_float.argtypes = [C.c_uint16]
        _lib.or_float_to_bf16.restype = C.c_uint16
        _lib.or_float_to_bf16.argtypes = [C.c_float]
        _lib.or_unpack_code.restype = C.c_uint32
        _lib.or_unpack_code.argtypes = [C.c_uint32, C.c_void_p, C.c_int64]
        _lib.or_dequantize_code.restype = C.c_float
        _lib.or_dequantize_code.argtypes = [C.c_uint32, C.c_float, C.c_float]
        _lib.or_quantize_code.restype = C.c_uint32
        _lib.or_quantize_code.argtypes = [C.c_uint32, C.c_float, C.c_float, C.c_float]
        _lib.or_build_packed_row_ptr.restype = C.c_int64
        _lib.or_compare.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.c_double, C.c_double,
                                    C.c_double, C.c_void_p, C.POINTER(Comparison)]
        _lib.or_digest_logical_dense.argtypes = [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_int,
                                                 C.c_uint32, C.POINTER(C.c_uint64 * 2)]
        _lib.or_spmm_referee.argtypes = [
            C.c_uint64, C.c_uint64, C.c_uint64, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
            C.c_void_p, C.c_int, C.c_uint64, C.c_void_p, C.c_int, C.c_int, C.c_uint64,
            C.c_double, C.c_double, C.c_void_p, C.c_int, C.c_int, C.c_uint64, C.c_int,
            C.c_void_p, C.c_int, C.c_void_p]
        _lib.or_qcsr_spmm_referee.argtypes = [
            C.c_uint32, C.c_uint32, C.c_int32, C.c_int32] + [C.c_void_p] * 8 + [
            C.c_int, C.c_uint32, C.c_uint64, C.c_int32, C.c_int32, C.c_void_p, C.c_void_p]
        _lib.or_qcsr_spmm_f32_mt.argtypes = [
            C.c_uint32, C.c_uint32, C.c_int32, C.c_int32] + [C.c_void_p] * 8 + [
            C.c_int, C.c_uint32, C.c_uint64, C.c_int32, C.c_int32, C.c_void_p, C.c_int]
        _lib.or_qcsr_spmm_f32_mt_magnitude.argtypes = _lib.or_qcsr_spmm_f32_mt.argtypes
        _lib.or_cpbp_canonical_mt.argtypes = [C.c_uint32] + [C.c_void_p] * 3 + [C.c_int] + [
            C.c_void_p] * 2 + [C.c_int]
        _lib.or_bell_spmm_bf16_mt.argtypes = [C.c_int32] * 4 + [C.c_void_p] * 3 + [
            C.c_uint32, C.c_void_p, C.c_int]
        _lib.or_bell_spmm_referee.argtypes = [
            C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_void_p, C.c_void_p, C.c_int,
            C.c_uint32, C.c_uint32, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
            C.c_void_p, C.c_int, C.c_uint32, C.c_uint64, C.c_void_p, C.c_void_p]
        _lib.or_cpbp_canonical.argtypes = [C.c_uint32] + [C.c_void_p] * 3 + [C.c_int] + [C.c_void_p] * 2
        _lib.or_cpbp_canonical_f64.argtypes = [C.c_uint32] + [C.c_void_p] * 3 + [C.c_int] + [C.c_void_p] * 3
        _lib.or_cpbp_tiles.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32] + [
            C.c_void_p] * 9 + [C.c_int] + [C.c_void_p] * 3
        _lib.or_cpbp_within_tolerance.argtypes = [C.c_float, C.c_float, C.c_double, C.c_double]
        _lib.or_spmm_bwd_values.argtypes = [C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p,
                                            C.c_uint64, C.c_void_p, C.c_int, C.c_uint64,
                                            C.c_uint64, C.c_void_p]
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- codec
def unpack_code(bits: int, row: np.ndarray, i: int) -> int:
    row = _c(row, np.uint8)
    return lib().or_unpack_code(bits, _p(row), i)


def dequantize(code: int, scale: float, offset: float) -> float:
    return lib().or_dequantize_code(code, scale, offset)


def quantize(bits: int, value: float, scale: float, offset: float) -> int:
    return lib().or_quantize_code(bits, value, scale, offset)


def build_packed_row_ptr(bits: int, row_ptr: np.ndarray) -> np.ndarray:
    row_ptr = _c(row_ptr, np.int32)
    out = np.zeros_like(row_ptr)
    rc = lib().or_build_packed_row_ptr(bits, _p(row_ptr), len(row_ptr) - 1, _p(out))
    if rc < 0:
        raise ValueError("build_packed_row_ptr failed")
    return out


def pack_csr(bits, policy, row_ptr, packed_row_ptr, col_idx, values, col_scales=None,
             col_offsets=None, row_offsets=None) -> np.ndarray:
    row_ptr, packed_row_ptr = _c(row_ptr, np.int32), _c(packed_row_ptr, np.int32)
    col_idx, values = _c(col_idx, np.int32), _c(values, np.float32)
    col_scales, col_offsets = _c(col_scales, np.float32), _c(col_offsets, np.float32)
    row_offsets = _c(row_offsets, np.float32)
    out = np.zeros(int(packed_row_ptr[-1]), dtype=np.uint8)
    rc = lib().or_pack_csr(bits, policy, len(row_ptr) - 1, _p(row_ptr), _p(packed_row_ptr),
                           _p(col_idx), _p(values), _p(col_scales), _p(col_offsets),
                           _p(row_offsets), _p(out))
    if rc != 0:
        raise ValueError("pack_csr failed")
    return out


def decode_csr(bits, policy, row_ptr, packed_row_ptr, col_idx, packed, col_scales=None,
               col_offsets=None, row_offsets=None) -> np.ndarray:
    row_ptr, packed_row_ptr = _c(row_ptr, np.int32), _c(packed_row_ptr, np.int32)
    col_idx, packed = _c(col_idx, np.int32), _c(packed, np.uint8)
    col_scales, col_offsets = _c(col_scales, np.float32), _c(col_offsets, np.float32)
    row_offsets = _c(row_offsets, np.float32)
    out = np.zeros(len(col_idx), dtype=np.float32)
    rc = lib().or_decode_csr(bits, policy, len(row_ptr) - 1, _p(row_ptr), _p(packed_row_ptr),
                             _p(col_idx), _p(packed), _p(col_scales), _p(col_offsets),
                             _p(row_offsets), _p(out))
    if rc != 0:
        raise ValueError("decode_csr failed")
    return out


# ---------------------------------------------------------------- referee
_TYPE_OF = {np.dtype(np.float16): F16, np.dtype(np.float32): F32, np.dtype(np.float64): F64}


def spmm_referee(m, k, n, row_offsets, cols, values, rhs, *, transpose_sparse=False,
                 transpose_dense=False, rhs_col_major=False, ldb=None, alpha=1.0, beta=0.0,
                 c0=None, c0_col_major=False, ldc0=None, epilogue=EPI_NONE, bias=None,
                 value_type=None, rhs_type=None) -> np.ndarray:
    row_offsets = _c(row_offsets, np.uint64)
    cols = _c(cols, np.uint32)
    values = np.ascontiguousarray(values)
    rhs = np.ascontiguousarray(rhs)
    vt = value_type or _TYPE_OF[values.dtype]
    rt = rhs_type or _TYPE_OF[rhs.dtype]
    if ldb is None:
        ldb = rhs.shape[1] if rhs.ndim == 2 and not rhs_col_major else rhs.shape[0]
    c0a = None if c0 is None else np.ascontiguousarray(c0)
    if ldc0 is None and c0a is not None:
        ldc0 = c0a.shape[1] if not c0_col_major else c0a.shape[0]
    biasa = None if bias is None else np.ascontiguousarray(bias)
    out = np.zeros(m * n, dtype=np.float64)
    rc = lib().or_spmm_referee(
        m, k, n, int(transpose_sparse), int(transpose_dense), _p(row_offsets), _p(cols),
        _p(values), vt, len(cols), _p(rhs), rt, int(rhs_col_major), ldb, alpha, beta, _p(c0a),
        _TYPE_OF[c0a.dtype] if c0a is not None else 0, int(c0_col_major), ldc0 or 0, epilogue,
        _p(biasa), _TYPE_OF[biasa.dtype] if biasa is not None else 0, _p(out))
    if rc != 0:
        raise ValueError(f"spmm_referee failed ({rc})")
    return out.reshape(m, n)


def compare(reference: np.ndarray, candidate: np.ndarray, abs_tol: float, rel_tol: float,
            magnitude: np.ndarray | None = None, relative_floor: float = 1e-30) -> dict:
    ref = _c(reference.ravel(), np.float64)
    cand = _c(candidate.ravel(), np.float32)
    mag = None if magnitude is None else _c(magnitude.ravel(), np.float64)
    out = Comparison()
    rc = lib().or_compare(_p(ref), _p(cand), ref.size, abs_tol, rel_tol, relative_floor,
                          _p(mag), C.byref(out))
    d = out.as_dict()
    d["status"] = rc
    return d


def digest_logical_dense(values: np.ndarray, column_major: bool = False, ld: int | None = None,
                         shape: tuple[int, int] | None = None) -> tuple[int, tuple[int, int]]:
    """(status, (low, high)) of digest_logical_dense over a 2-D f16/f32/f64 array (row-major
    as given, or the array read column-major when column_major: its transpose's memory)."""
    types = {np.dtype(np.float16): F16, np.dtype(np.float32): F32, np.dtype(np.float64): F64}
    a = np.ascontiguousarray(values)
    rows, cols = shape if shape is not None else (a.shape if not column_major else a.shape[::-1])
    ld = ld if ld is not None else a.shape[1] if a.ndim == 2 else 0
    out = (C.c_uint64 * 2)()
    st = lib().or_digest_logical_dense(_p(a), rows, cols, ld, int(column_major),
                                       types.get(a.dtype, 0), C.byref(out))
    return st, (int(out[0]), int(out[1]))


def _rhs_type(rhs: np.ndarray) -> int:
    return F16 if rhs.dtype == np.float16 else F32


def qcsr_spmm_referee(bits, policy, rows, cols, row_ptr, packed_row_ptr, col_idx, packed,
                      scales, offsets, row_offsets, rhs, row_begin=0, row_end=None,
                      want_magnitude=True):
    """float64 referee output (and sum |x||w|) for rows [row_begin, row_end)."""
    row_end = rows if row_end is None else row_end
    row_ptr, packed_row_ptr = _c(row_ptr, np.int32), _c(packed_row_ptr, np.int32)
    col_idx, packed = _c(col_idx, np.int32), _c(packed, np.uint8)
    scales, offsets, row_offsets = _c(scales, np.float32), _c(offsets, np.float32), _c(row_offsets, np.float32)
    rhs = np.ascontiguousarray(rhs)
    n = rhs.shape[1]
    out = np.zeros((row_end - row_begin) * n, dtype=np.float64)
    mag = np.zeros_like(out) if want_magnitude else None
    rc = lib().or_qcsr_spmm_referee(bits, policy, rows, cols, _p(row_ptr), _p(packed_row_ptr),
                                    _p(col_idx), _p(packed), _p(scales), _p(offsets),
                                    _p(row_offsets), _p(rhs), _rhs_type(rhs), n, rhs.shape[1],
                                    row_begin, row_end, _p(out), _p(mag))
    if rc != 0:
        raise ValueError(f"qcsr_spmm_referee failed ({rc})")
    shape = (row_end - row_begin, n)
    return out.reshape(shape), (None if mag is None else mag.reshape(shape))


def qcsr_spmm_f32_mt(bits, policy, rows, cols, row_ptr, packed_row_ptr, col_idx, packed,
                     scales, offsets, row_offsets, rhs, row_begin=0, row_end=None, threads=1,
                     magnitude=False):
    """Row-parallel fp32 product (or, with magnitude=True, Sigma |x||w| per element)."""
    row_end = rows if row_end is None else row_end
    row_ptr, packed_row_ptr = _c(row_ptr, np.int32), _c(packed_row_ptr, np.int32)
    col_idx, packed = _c(col_idx, np.int32), _c(packed, np.uint8)
    scales, offsets, row_offsets = _c(scales, np.float32), _c(offsets, np.float32), _c(row_offsets, np.float32)
    rhs = np.ascontiguousarray(rhs)
    n = rhs.shape[1]
    out = np.zeros((row_end - row_begin, n), dtype=np.float32)
    fn = lib().or_qcsr_spmm_f32_mt_magnitude if magnitude else lib().or_qcsr_spmm_f32_mt
    rc = fn(bits, policy, rows, cols, _p(row_ptr), _p(packed_row_ptr), _p(col_idx), _p(packed),
            _p(scales), _p(offsets), _p(row_offsets), _p(rhs), _rhs_type(rhs), n, rhs.shape[1],
            row_begin, row_end, _p(out), threads)
    if rc != 0:
        raise ValueError(f"qcsr_spmm_f32_mt failed ({rc})")
    return out


def bell_spmm_referee(rows, cols, block_size, ell_cols, block_col_idx, values, rhs, *,
                      value_type=None, bits=0, policy=PER_GENE_AFFINE, row_stride_bytes=0,
                      packed=None, scales=None, offsets=None, row_offsets=None,
                      rhs_type=None, want_magnitude=True):
    block_col_idx = _c(block_col_idx, np.uint32)
    values = None if values is None else np.ascontiguousarray(values)
    rhs = np.ascontiguousarray(rhs)
    n = rhs.shape[1]
    out = np.zeros(rows * n, dtype=np.float64)
    mag = np.zeros_like(out) if want_magnitude else None
    rc = lib().or_bell_spmm_referee(
        rows, cols, block_size, ell_cols, _p(block_col_idx), _p(values), value_type or 0,
        bits, policy, row_stride_bytes, _p(_c(packed, np.uint8)), _p(_c(scales, np.float32)),
        _p(_c(offsets, np.float32)), _p(_c(row_offsets, np.float32)), _p(rhs),
        rhs_type or _TYPE_OF[rhs.dtype], n, n, _p(out), _p(mag))
    if rc != 0:
        raise ValueError(f"bell_spmm_referee failed ({rc})")
    return out.reshape(rows, n), (None if mag is None else mag.reshape(rows, n))


# ---------------------------------------------------------------- backward
def spmm_bwd_values(row_ptr, col_idx, grad_out, rhs) -> np.ndarray:
    """float64 grad_values of Y = X . rhs (csr_spmm_bwd_values_kernel_); grad_out f32
    [rows, n], rhs f16/f32 [cols, n], both row-major."""
    row_ptr, col_idx = _c(row_ptr, np.int32), _c(col_idx, np.int32)
    grad_out = _c(grad_out, np.float32)
    rhs = np.ascontiguousarray(rhs)
    n = grad_out.shape[1]
    out = np.zeros(len(col_idx), dtype=np.float64)
    rc = lib().or_spmm_bwd_values(len(row_ptr) - 1, _p(row_ptr), _p(col_idx), _p(grad_out),
                                  grad_out.shape[1], _p(rhs), _TYPE_OF[rhs.dtype], rhs.shape[1],
                                  n, _p(out))
    if rc != 0:
        raise ValueError(f"spmm_bwd_values failed ({rc})")
    return out


# ---------------------------------------------------------------- CP-BP
def cpbp_canonical(row_offsets, features, values, weights, value_type=F32) -> np.ndarray:
    row_offsets, features = _c(row_offsets, np.uint32), _c(features, np.uint32)
    values = np.ascontiguousarray(values)
    weights = _c(weights, np.float32)
    out = np.zeros(len(row_offsets) - 1, dtype=np.float32)
    rc = lib().or_cpbp_canonical(len(out), _p(row_offsets), _p(features), _p(values),
                                 value_type, _p(weights), _p(out))
    if rc != 0:
        raise ValueError("cpbp_canonical failed")
    return out


def cpbp_canonical_mt(row_offsets, features, values, weights, value_type=F32, threads=1):
    """Row-parallel cpbp_canonical (bitwise equal to it)."""
    row_offsets, features = _c(row_offsets, np.uint32), _c(features, np.uint32)
    values = np.ascontiguousarray(values)
    weights = _c(weights, np.float32)
    out = np.zeros(len(row_offsets) - 1, dtype=np.float32)
    rc = lib().or_cpbp_canonical_mt(len(out), _p(row_offsets), _p(features), _p(values),
                                    value_type, _p(weights), _p(out), threads)
    if rc != 0:
        raise ValueError("cpbp_canonical_mt failed")
    return out


def bell_spmm_bf16_mt(rows, cols, block_size, ell_cols, block_col_idx, values_bf16, rhs_bf16,
                      threads=1):
    """Row-block-parallel bf16 Blocked-ELL SpMM (fp32 [rows, n]); values and rhs as uint16
    bf16 bit patterns."""
    block_col_idx = _c(block_col_idx, np.uint32)
    values_bf16, rhs_bf16 = _c(values_bf16, np.uint16), _c(rhs_bf16, np.uint16)
    n = rhs_bf16.shape[1]
    out = np.zeros((rows, n), dtype=np.float32)
    rc = lib().or_bell_spmm_bf16_mt(rows, cols, block_size, ell_cols, _p(block_col_idx),
                                    _p(values_bf16), _p(rhs_bf16), n, _p(out), threads)
    if rc != 0:
        raise ValueError("bell_spmm_bf16_mt failed")
    return out


def cpbp_canonical_f64(row_offsets, features, values, weights, value_type=F32):
    row_offsets, features = _c(row_offsets, np.uint32), _c(features, np.uint32)
    values = np.ascontiguousarray(values)
    weights = _c(weights, np.float32)
    out = np.zeros(len(row_offsets) - 1, dtype=np.float64)
    mag = np.zeros_like(out)
    rc = lib().or_cpbp_canonical_f64(len(out), _p(row_offsets), _p(features), _p(values),
                                     value_type, _p(weights), _p(out), _p(mag))
    if rc != 0:
        raise ValueError("cpbp_canonical_f64 failed")
    return out, mag


def cpbp_tiles(row_count, tile_row_width, mask_bits, feature_block_offsets,
               feature_permutation, tile_block_offsets, tile_block_ids, cell_masks,
               block_row_entry_offsets, gene_masks, value_offsets, values, row_permutation,
               weights, value_type=F32) -> np.ndarray:
    arrs = [_c(a, np.uint32) for a in (feature_block_offsets, feature_permutation,
                                        tile_block_offsets, tile_block_ids)]
    masks = _c(cell_masks, np.uint32 if mask_bits == 32 else np.uint64)
    rest = [_c(a, np.uint32) for a in (block_row_entry_offsets, gene_masks, value_offsets)]
    values = np.ascontiguousarray(values)
    rp = _c(row_permutation, np.uint32)
    weights = _c(weights, np.float32)
    out = np.zeros(row_count, dtype=np.float32)
    tile_count = len(arrs[2]) - 1
    rc = lib().or_cpbp_tiles(row_count, tile_count, tile_row_width, mask_bits, _p(arrs[0]),
                             _p(arrs[1]), _p(arrs[2]), _p(arrs[3]), _p(masks), _p(rest[0]),
                             _p(rest[1]), _p(rest[2]), _p(values), value_type, _p(rp),
                             _p(weights), _p(out))
    if rc != 0:
        raise ValueError("cpbp_tiles failed")
    return out
