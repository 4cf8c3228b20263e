"""cx_qcsr_get_block on the host: the reference's get_block rules
(include/Cellerator/quantized/access.cuh:7-45): block ranges from block_row_ptr and the row
arrays, the whole matrix without block metadata, an empty block out of range; and
build_uniform_block_row_ptr's partition (layout.cuh:138-156) as the tests' block source."""
from __future__ import annotations

import numpy as np
import pytest

from cellerator_amd import _native as N
from cellerator_amd.codec import get_block


def uniform_blocks(rows: int, per_block: int) -> np.ndarray:
    """build_uniform_block_row_ptr (layout.cuh:138-156)."""
    count = (rows + per_block - 1) // per_block if rows > 0 else 0
    return np.array([min(b * per_block, rows) for b in range(count)] + [rows], np.int32)


def test_get_block_ranges(oracle):
    row_ptr = np.array([0, 3, 3, 10, 11, 20], np.int32)
    prp = oracle.build_packed_row_ptr(4, row_ptr)
    assert prp.tolist() == [0, 2, 2, 6, 7, 12]
    brp = uniform_blocks(5, 2)
    assert brp.tolist() == [0, 2, 4, 5]
    b = get_block(brp, row_ptr, prp, 1)
    assert (b.block_index, b.row_begin, b.row_end, b.nnz_begin, b.nnz_end, b.packed_begin, b.packed_end) == \
        (1, 2, 4, 3, 11, 2, 7)
    whole = get_block(None, row_ptr, prp, 7)
    assert (whole.block_index, whole.row_begin, whole.row_end, whole.nnz_end, whole.packed_end) == (0, 0, 5, 20, 12)
    with pytest.raises(N.EngineError, match="out of range"):
        get_block(brp, row_ptr, prp, 3)
