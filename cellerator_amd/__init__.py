"""MI355X-native engine for Cellerator's sparse expression-matrix projection hot path.

Hand-written gfx950 HIP kernels behind a C-ABI (include/cellerator_amd.h):
quantized CSR SpMM, Blocked-ELL SpMM on bf16 MFMA, and the CP-BP warp-tile
feature-weighted row reduction. This package is the Python host mirror of that ABI;
PyTorch supplies device memory and streams only.
"""
from .engine import (BellGroups, BellMatrix, CpbpTiles, Epilogue, QcsrMatrix,  # noqa: F401
                     bell_block_major, bell_pack_rhs, bell_plan_groups, bell_spmm, bell_spmm_grouped,
                     bell_spmm_packed, cpbp_entry_rows, cpbp_reduce, cpbp_reduce_rows, csr_spmv,
                     exclusive_scan_u32,
                     qcsr_check_columns, qcsr_pack_gene_affine, qcsr_spmm, qcsr_spmm_balanced, qcsr_spmm_bwd_rhs, qcsr_spmm_bwd_values,
                     qcsr_transpose, qcsr_transpose_panelled, sort_pairs)

__all__ = ["QcsrMatrix", "BellMatrix", "BellGroups", "CpbpTiles", "Epilogue", "bell_plan_groups",
           "bell_spmm_grouped", "qcsr_spmm", "bell_spmm", "bell_pack_rhs", "bell_block_major",
           "bell_spmm_packed", "cpbp_reduce", "cpbp_entry_rows", "cpbp_reduce_rows", "csr_spmv", "qcsr_check_columns", "qcsr_pack_gene_affine",
           "qcsr_spmm_balanced", "qcsr_transpose", "qcsr_transpose_panelled", "qcsr_spmm_bwd_values", "qcsr_spmm_bwd_rhs", "sort_pairs",
           "exclusive_scan_u32"]
