"""The quantized codec as device passes over a row block (qcsr_codec.hip): ctypes mirror of
cx_qcsr_block and front-ends for cx_qcsr_get_block / cx_qcsr_quantize_block /
cx_qcsr_dequantize_block (the reference's get_block, launch_quantize_block and
launch_dequantize_block, include/Cellerator/quantized/access.cuh:7-45, dispatch.cuh:35-61)."""
from __future__ import annotations

import ctypes as C
from typing import Optional

import numpy as np
import torch

from . import _native as N
from .engine import QcsrMatrix, _require_cuda, _stream

i32, p_void = C.c_int32, C.c_void_p


class CxQcsrBlock(C.Structure):
    _fields_ = [("block_index", i32), ("row_begin", i32), ("row_end", i32), ("nnz_begin", i32), ("nnz_end", i32),
                ("packed_begin", i32), ("packed_end", i32), ("reserved", i32)]


_SIGS = {
    "cx_qcsr_get_block": (C.c_int, [p_void, i32, p_void, p_void, i32, i32, C.POINTER(CxQcsrBlock)]),
    "cx_qcsr_quantize_block": (C.c_int, [C.POINTER(N.CxQcsrMatrix), C.POINTER(CxQcsrBlock), p_void, p_void, p_void]),
    "cx_qcsr_dequantize_block": (C.c_int, [C.POINTER(N.CxQcsrMatrix), C.POINTER(CxQcsrBlock), p_void, p_void]),
}


def _lib():
    lib = N.engine()
    if not getattr(lib, "_codec_sigs", False):
        for name, (res, args) in _SIGS.items():
            f = getattr(lib, name)
            f.restype, f.argtypes = res, args
        lib._codec_sigs = True
    return lib


def get_block(block_row_ptr: Optional[np.ndarray], row_ptr: np.ndarray, packed_row_ptr: np.ndarray,
              index: int) -> CxQcsrBlock:
    """Block `index` of host block_row_ptr (None: the whole matrix), from host row arrays."""
    rp = np.ascontiguousarray(row_ptr, np.int32)
    prp = np.ascontiguousarray(packed_row_ptr, np.int32)
    brp = None if block_row_ptr is None else np.ascontiguousarray(block_row_ptr, np.int32)
    out = CxQcsrBlock()
    N.check("cx_qcsr_get_block", _lib().cx_qcsr_get_block(
        brp.ctypes.data if brp is not None else None, len(brp) - 1 if brp is not None else 0, rp.ctypes.data,
        prp.ctypes.data, len(rp) - 1, index, C.byref(out)))
    return out


def quantize(m: QcsrMatrix, values: torch.Tensor, packed_out: Optional[torch.Tensor] = None,
             block: Optional[CxQcsrBlock] = None, stream=None) -> torch.Tensor:
    """Encodes F32 values (the block's entries, from its first entry) into packed codes with
    m's structure and metadata; packed_out defaults to m.packed_values."""
    _require_cuda(m.row_ptr, values)
    if values.dtype != torch.float32 or not values.is_contiguous():
        raise ValueError("values must be a contiguous float32 tensor")
    out = m.packed_values if packed_out is None else packed_out
    d = m.descriptor()
    N.check("cx_qcsr_quantize_block", _lib().cx_qcsr_quantize_block(
        C.byref(d), C.byref(block) if block is not None else None, values.data_ptr(), out.data_ptr(),
        _stream(stream)))
    return out


def dequantize(m: QcsrMatrix, values_out: Optional[torch.Tensor] = None, block: Optional[CxQcsrBlock] = None,
               stream=None) -> torch.Tensor:
    """Decodes the block's (or every) entry to F32, indexed from the block's first entry."""
    _require_cuda(m.row_ptr)
    n = m.nnz if block is None else block.nnz_end - block.nnz_begin
    if values_out is None:
        values_out = torch.empty(max(n, 1), dtype=torch.float32, device=m.row_ptr.device)
    d = m.descriptor()
    N.check("cx_qcsr_dequantize_block", _lib().cx_qcsr_dequantize_block(
        C.byref(d), C.byref(block) if block is not None else None, values_out.data_ptr(), _stream(stream)))
    return values_out[:n]
