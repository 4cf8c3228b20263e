"""ctypes bindings of the engine's C-ABI (include/cellerator_amd.h) and of the synthetic
input library (include/cellerator_amd_synth.h).

The libraries are built in-tree by ``cellerator_amd.build`` (``__graft_entry__.build()``).
Loading fails loudly when a library is missing: there is no CPU fallback for any
operation of the engine.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

PKG = Path(__file__).resolve().parent
ENGINE_PATH = PKG / "libcellerator_amd.so"
SYNTH_PATH = PKG / "libcx_synth.so"

# cellerator_dtype (include/cellerator_amd.h)
DTYPE_F16, DTYPE_F32, DTYPE_U8, DTYPE_U32, DTYPE_BF16 = 1, 2, 3, 4, 5
DECODE_PER_GENE_AFFINE, DECODE_COLUMN_SCALE_ROW_OFFSET, DECODE_PER_GENE_AFFINE_PAIRS = 1, 2, 3
QCSR_COLUMNS_SORTED = 1  # cx_qcsr_matrix.flags
# CX_EPILOGUE_* = the reference's epilogue_kind values
(EPILOGUE_NONE, EPILOGUE_BIAS, EPILOGUE_RELU, EPILOGUE_GELU_ERF, EPILOGUE_GELU_TANH,
 EPILOGUE_BIAS_RELU, EPILOGUE_BIAS_GELU_ERF, EPILOGUE_BIAS_GELU_TANH) = range(8)
STATUS_NAMES = {0: "SUCCESS", 1: "INVALID_ARGUMENT", 2: "INVALID_SHAPE", 3: "UNSUPPORTED",
                4: "HIP_ERROR", 5: "INTERNAL_ERROR"}

p_void = C.c_void_p
u32, u64, i32, i64 = C.c_uint32, C.c_uint64, C.c_int32, C.c_int64


class CxQcsrMatrix(C.Structure):
    _fields_ = [
        ("rows", u32), ("cols", u32), ("nnz", u64), ("bits", u32), ("decode_policy", u32),
        ("row_ptr", p_void), ("packed_row_ptr", p_void), ("col_idx", p_void),
        ("packed_values", p_void), ("column_scales", p_void), ("column_offsets", p_void),
        ("row_offsets", p_void), ("values", p_void), ("value_dtype", u32), ("flags", u32),
    ]


class CxBellMatrix(C.Structure):
    _fields_ = [
        ("rows", u32), ("cols", u32), ("block_size", u32), ("ell_cols", u32),
        ("block_col_idx", p_void), ("values", p_void), ("value_dtype", u32), ("bits", u32),
        ("decode_policy", u32), ("row_stride_bytes", u32), ("packed_values", p_void),
        ("column_scales", p_void), ("column_offsets", p_void), ("row_offsets", p_void),
        ("value_layout_flags", u32), ("reserved", u32),
    ]


BELL_BLOCK_MAJOR_VALUES = 1


class CxSpmmEpilogue(C.Structure):
    _fields_ = [("kind", u32), ("reserved", u32), ("alpha", C.c_float), ("beta", C.c_float),
                ("bias", p_void), ("initial", p_void), ("initial_ld", i64)]


class CxBellGroups(C.Structure):
    _fields_ = [("group_count", u32), ("grouped_row_blocks", u32), ("single_count", u32),
                ("reserved", u32), ("order", p_void), ("group_offsets", p_void)]


class CxCpbpTiles(C.Structure):
    _fields_ = [
        ("row_count", u32), ("feature_count", u32), ("feature_block_count", u32),
        ("tile_row_width", u32), ("tile_count", u32), ("tile_block_count", u32),
        ("row_block_entry_count", u32), ("nnz_count", u32), ("value_dtype", u32),
        ("reserved", u32),
        ("feature_block_offsets", p_void), ("feature_permutation", p_void),
        ("tile_block_offsets", p_void), ("tile_block_ids", p_void),
        ("tile_block_cell_masks", p_void), ("block_row_entry_offsets", p_void),
        ("row_block_gene_masks", p_void), ("row_block_value_offsets", p_void),
        ("values", p_void), ("row_permutation", p_void),
    ]


class CxCpbpPlan(C.Structure):
    _fields_ = [("feature_count", u32), ("feature_block_count", u32),
                ("feature_permutation", p_void), ("feature_block_offsets", p_void)]


class CxCpbpCsr(C.Structure):
    _fields_ = [("rows", u32), ("value_size_bytes", u32), ("row_offsets", p_void),
                ("canonical_features", p_void), ("values", p_void)]


class CxCpbpOrderConfig(C.Structure):
    _fields_ = [("kind", u32), ("window_size", u32), ("group_width", u32), ("reserved", u32),
                ("seed", u64), ("global_row_begin", u64)]


class CxCpbpTileRequirements(C.Structure):
    _fields_ = [("row_count", u32), ("feature_count", u32), ("feature_block_count", u32),
                ("tile_row_width", u32), ("tile_count", u32), ("tile_block_count", u32),
                ("row_block_entry_count", u32), ("nnz_count", u32), ("value_size_bytes", u32),
                ("cell_mask_bytes", u32)]


class CxCpbpTileBuffers(C.Structure):
    _fields_ = [("tile_block_offsets", p_void), ("tile_block_ids", p_void),
                ("tile_block_cell_masks", p_void), ("block_row_entry_offsets", p_void),
                ("row_block_gene_masks", p_void), ("row_block_value_offsets", p_void),
                ("values", p_void), ("row_permutation", p_void), ("primary_keys", p_void)]


class CxCpk1Expected(C.Structure):
    _fields_ = [("global_row_begin", u64), ("row_count", u32), ("feature_count", u32),
                ("reserved0", u32), ("feature_axis_fingerprint", u64),
                ("feature_axis_fingerprint_version", u32), ("reserved1", u32),
                ("row_domain_identity", u64), ("payload_identity", u64)]


class CxCpk1View(C.Structure):
    _fields_ = [("payload_identity", u64), ("image_base", p_void), ("image_bytes", u64),
                ("global_row_begin", u64), ("full_row_count", u32), ("row_group_count", u32),
                ("row_group_width", u32), ("maximum_feature_block_width", u32),
                ("feature_axis_fingerprint", u64), ("feature_axis_fingerprint_version", u32),
                ("row_domain_kind", u32), ("row_domain_identity", u64),
                ("feature_block_geometry_identity", u64), ("ordering_identity", u64),
                ("tile_identity", u64), ("order", CxCpbpOrderConfig),
                ("inverse_feature_permutation", p_void), ("feature_to_block", p_void),
                ("feature_to_local", p_void), ("row_group_offsets", p_void),
                ("inverse_row_permutation", p_void), ("tiles", CxCpbpTiles)]


class CxCpbpReductionView(C.Structure):
    _fields_ = [("schema_version", u32), ("storage_type_code", u32), ("weight_type_code", u32),
                ("accumulation_type_code", u32), ("feature_weight_identity", u64), ("reduction_identity", u64),
                ("plan_schema_version", u32), ("plan_geometry_identity_version", u32), ("plan_feature_count", u32),
                ("plan_feature_block_count", u32), ("plan_geometry_identity", u64), ("tile_schema_version", u32),
                ("tiles_plan_schema_version", u32), ("tiles_geometry_identity_version", u32),
                ("feature_axis_fingerprint_version", u32), ("tile_identity", u64), ("tiles_geometry_identity", u64),
                ("tiles_ordering_identity", u64), ("tiles_global_row_begin", u64), ("feature_axis_fingerprint", u64),
                ("tiles_row_domain_identity", u64), ("tiles_full_row_count", u32), ("order_schema_version", u32),
                ("order_signature_version", u32), ("order_full_row_count", u32), ("order_row_count", u32),
                ("order_feature_block_count", u32), ("order_group_width", u32), ("reserved", u32),
                ("order_ordering_identity", u64), ("order_global_row_begin", u64), ("order_geometry_identity", u64),
                ("order_row_domain_identity", u64), ("tiles", CxCpbpTiles)]


class CxFwrPlanView(C.Structure):
    """cellpack::feature_weighted_row_reduction_plan_view (40 bytes)."""
    _fields_ = [("semantic_plan_schema_version", u32), ("geometry_identity_version", u32),
                ("feature_count", u32), ("feature_block_count", u32),
                ("feature_block_geometry_identity", u64), ("feature_block_offsets", p_void),
                ("feature_permutation", p_void)]


class CxLocalCellOrderView(C.Structure):
    """cellpack::local_cell_order_view (128 bytes)."""
    _fields_ = [("order_schema_version", u32), ("signature_algorithm_version", u32), ("kind", u32),
                ("window_size", u32), ("group_width", u32), ("reserved0", u32), ("seed", u64),
                ("ordering_identity", u64), ("global_row_begin", u64), ("full_row_count", u32),
                ("row_count", u32), ("feature_block_count", u32), ("reserved1", u32),
                ("feature_block_geometry_identity", u64), ("row_domain_identity", u64),
                ("primary_keys", p_void), ("secondary_keys", p_void), ("active_block_counts", p_void),
                ("row_nnz_counts", p_void), ("row_permutation", p_void), ("inverse_row_permutation", p_void)]


class CxWarpTileView(C.Structure):
    """cellpack::warp_tile_view (176 bytes)."""
    _fields_ = [("tile_schema_version", u32), ("record_schema_version", u32),
                ("semantic_plan_schema_version", u32), ("geometry_identity_version", u32),
                ("order_schema_version", u32), ("reserved0", u32), ("tile_identity", u64),
                ("feature_block_geometry_identity", u64), ("ordering_identity", u64),
                ("global_row_begin", u64), ("full_row_count", u32), ("row_count", u32),
                ("feature_count", u32), ("feature_block_count", u32), ("tile_row_width", u32),
                ("tile_count", u32), ("nnz_count", u32), ("tile_block_count", u32),
                ("row_block_entry_count", u32), ("value_size_bytes", u32), ("feature_axis_fingerprint", u64),
                ("feature_axis_fingerprint_version", u32), ("reserved1", u32), ("row_domain_identity", u64),
                ("tile_block_offsets", p_void), ("tile_block_ids", p_void), ("tile_block_cell_masks", p_void),
                ("block_row_entry_offsets", p_void), ("row_block_gene_masks", p_void),
                ("row_block_value_offsets", p_void), ("values", p_void)]


class CxNativeTileBlockMetrics(C.Structure):
    _fields_ = [("active_rows", u32), ("active_features", u32), ("nnz", u32), ("dense_workload", u32),
                ("density", C.c_double), ("feature_reuse", C.c_double)]


class CxNativeTileRequirements(C.Structure):
    _fields_ = [("union_mask_count", u64), ("packed_offset_count", u64), ("block_metric_count", u64),
                ("sidecar_bytes", u64)]


class CxNativeTileBuffers(C.Structure):
    _fields_ = [("union_mask_capacity", u64), ("union_gene_masks", p_void), ("packed_offset_capacity", u64),
                ("packed_value_offsets", p_void), ("block_metric_capacity", u64), ("block_metrics", p_void)]


class CxNativeTileView(C.Structure):
    """math::native_tile_view (384 bytes)."""
    _fields_ = [("schema_version", u32), ("reserved", u32), ("plan", CxFwrPlanView),
                ("order", CxLocalCellOrderView), ("tiles", CxWarpTileView), ("union_gene_masks", p_void),
                ("packed_value_offsets", p_void), ("block_metrics", p_void), ("dense_workload", u64)]


class CxNativeTileDecodedValue(C.Structure):
    _fields_ = [("value_index", u32), ("execution_row", u32), ("canonical_row", u32), ("reserved0", u32),
                ("global_row", u64), ("execution_feature", u32), ("canonical_feature", u32), ("value", p_void)]


class CxCpk1Metadata(C.Structure):
    _fields_ = [("feature_axis_fingerprint", u64), ("feature_axis_fingerprint_version", u32),
                ("row_domain_kind", u32), ("row_domain_identity", u64),
                ("evaluation_source_identity", u64), ("sampling_provenance_identity", u64),
                ("cost_policy_identity", u64), ("objective_kind", u32), ("full_row_count", u32),
                ("maximum_feature_block_width", u32), ("row_group_width", u32),
                ("row_group_count", u32), ("reserved", u32), ("row_group_offsets", p_void),
                ("global_row_begin", u64), ("order", CxCpbpOrderConfig)]


class CxsQcsrParams(C.Structure):
    _fields_ = [
        ("seed", u64), ("rows", u32), ("cols", u32), ("row_dist", u32), ("bits", u32),
        ("nnz_mean", C.c_double), ("nnz_sigma", C.c_double), ("nnz_min", u32),
        ("nnz_max", u32), ("zipf_s", C.c_double), ("nb_mean", C.c_double),
        ("nb_size", C.c_double),
    ]


class CxsCpbpParams(C.Structure):
    _fields_ = [
        ("seed", u64), ("rows", u32), ("genes", u32), ("modules", u32), ("module_size", u32),
        ("min_active", u32), ("max_active", u32), ("active_genes", u32), ("background", u32),
        ("nb_mean", C.c_double), ("nb_size", C.c_double),
    ]


class CxFeatureOrder(C.Structure):
    _fields_ = [("schema_version", u32), ("kind", u32), ("feature_count", u32),
                ("feature_axis_identity_version", u32), ("feature_axis_identity", u64),
                ("packing_geometry_identity", u64)]


class CxDenseOperand(C.Structure):
    _fields_ = [("values", p_void), ("feature_count", u32), ("value_size_bytes", u32),
                ("column_count", u64), ("leading_dimension", u64), ("column_major", u32),
                ("reserved", u32), ("feature_order", CxFeatureOrder), ("operand_identity", u64)]


class CxOrderedPartition(C.Structure):
    _fields_ = [("global_row_begin", u64), ("full_row_count", u32), ("row_count", u32),
                ("feature_count", u32), ("nnz_count", u32), ("value_size_bytes", u32),
                ("feature_axis_fingerprint_version", u32), ("feature_axis_fingerprint", u64),
                ("row_domain_identity", u64), ("row_offsets", p_void), ("block_ids", p_void),
                ("local_feature_ids", p_void), ("canonical_feature_ids", p_void), ("values", p_void)]


class CxExecutionCsr(C.Structure):
    _fields_ = [("global_row_begin", u64), ("full_row_count", u32), ("row_count", u32),
                ("feature_count", u32), ("nnz_count", u32), ("value_size_bytes", u32),
                ("reserved", u32), ("row_domain_identity", u64), ("structure_identity", u64),
                ("feature_order", CxFeatureOrder), ("row_offsets", p_void),
                ("execution_feature_ids", p_void), ("values", p_void)]


class CxLazyCsrRequirements(C.Structure):
    _fields_ = [("row_offset_count", u64), ("execution_feature_count", u64), ("value_bytes", u64),
                ("row_cursor_count", u64), ("total_bytes", u64)]


class CxLazyCsrBuffers(C.Structure):
    _fields_ = [("row_offset_capacity", u64), ("execution_feature_capacity", u64),
                ("value_capacity_bytes", u64), ("row_cursor_capacity", u64), ("row_offsets", p_void),
                ("execution_feature_ids", p_void), ("values", p_void), ("row_cursors", p_void)]


FEATURE_ORDER_CANONICAL, FEATURE_ORDER_PACKED = 1, 2


class CxQcsrHybridLayout(C.Structure):
    _fields_ = [("head_cols", u32), ("rows", u32), ("rows_ld", u32), ("bits", u32), ("decode_policy", u32),
                ("scale_exp", i32), ("nnz", u64), ("codes", p_void), ("masks", p_void), ("head_end", p_void),
                ("meta", p_void), ("row_offsets", p_void), ("tail", p_void), ("head_form", u32),
                ("reserved", u32), ("code_bytes", p_void), ("lut", p_void)]


HEAD_FORM_WORDS, HEAD_FORM_TABLE = 1, 2


class CxQcsrTailStream(C.Structure):
    _fields_ = [("rows", u32), ("first_part", u32), ("parts", u32), ("blocks", u32), ("block_rows", u32),
                ("layers", u32), ("bits", u32), ("entry_bytes", u32), ("fills", u64), ("nnz", u64),
                ("slot_rows", p_void), ("fill_index", p_void), ("entries", p_void)]


class CxQcsrExecInfo(C.Structure):
    _fields_ = [("rows", u32), ("cols", u32), ("bits", u32), ("head_cols", u32), ("nnz", u64),
                ("tail_fills", u64), ("persistent_bytes", u64), ("head_form", u32), ("tail_blocks", u32)]


# ---- public context ABI structs (include/Cellerator/abi.h layout) ----
class CelleratorExecutionConfig(C.Structure):
    _fields_ = [("version", u32), ("size", C.c_size_t), ("device", i32), ("stream", p_void),
                ("scratch", p_void), ("scratch_bytes", C.c_size_t)]


class CelleratorTensorDesc(C.Structure):
    _fields_ = [("version", u32), ("size", C.c_size_t), ("data", p_void), ("dtype", C.c_int),
                ("rank", u32), ("shape", u64 * 4), ("stride", i64 * 4)]


class CelleratorSparseLayoutDesc(C.Structure):
    _fields_ = [
        ("version", u32), ("size", C.c_size_t), ("layout", C.c_int), ("rows", u32),
        ("cols", u32), ("nnz", u32), ("block_size", u32), ("ell_cols", u32),
        ("row_stride_bytes", u32), ("bits", u32), ("decode_policy", u32),
        ("value_dtype", C.c_int), ("major_ptr", p_void), ("minor_idx", p_void),
        ("block_col_idx", p_void), ("values", p_void), ("packed_values", p_void),
        ("column_scales", p_void), ("column_offsets", p_void), ("row_offsets", p_void),
    ]


# Every symbol include/cellerator_amd.h declares, with its ctypes signature.
ENGINE_SIGNATURES = {
    "cx_qcsr_spmm_fwd": (C.c_int, [C.POINTER(CxQcsrMatrix), p_void, u32, i64, i64, p_void, i64, p_void]),
    "cx_qcsr_spmm_fwd_epilogue": (C.c_int, [C.POINTER(CxQcsrMatrix), p_void, u32, i64, i64, p_void,
                                            i64, C.POINTER(CxSpmmEpilogue), p_void]),
    "cx_qcsr_pack_gene_affine": (C.c_int, [p_void, p_void, u32, p_void, p_void]),
    "cx_qcsr_check_columns": (C.c_int, [p_void, p_void, p_void]),
    "cx_qcsr_check_columns_sync": (C.c_int, [p_void, C.POINTER(u32), p_void]),
    "cx_stream_synchronize": (C.c_int, [p_void]),
    "cx_qcsr_transpose_workspace": (C.c_int, [C.POINTER(CxQcsrMatrix), C.POINTER(u64)]),
    "cx_qcsr_transpose": (C.c_int, [C.POINTER(CxQcsrMatrix), p_void, p_void, p_void, p_void, u64,
                                    p_void]),
    "cx_qcsr_transpose_panelled_workspace": (C.c_int, [C.POINTER(CxQcsrMatrix), u32, C.POINTER(u64)]),
    "cx_qcsr_transpose_panelled": (C.c_int, [C.POINTER(CxQcsrMatrix), u32, p_void, p_void, p_void,
                                             p_void, u64, p_void]),
    "cx_qcsr_spmm_bwd_rhs_panelled_workspace": (C.c_int, [C.POINTER(CxQcsrMatrix), u32, i64,
                                                          C.POINTER(u64)]),
    "cx_qcsr_spmm_bwd_rhs_panelled": (C.c_int, [C.POINTER(CxQcsrMatrix), u32, p_void, i64, i64,
                                                p_void, i64, p_void, u64, p_void]),
    "cx_qcsr_spmm_bwd_values": (C.c_int, [C.POINTER(CxQcsrMatrix), p_void, i64, p_void, u32, i64,
                                          i64, p_void, p_void]),
    "cx_qcsr_spmm_bwd_rhs": (C.c_int, [C.POINTER(CxQcsrMatrix), p_void, i64, i64, p_void, i64,
                                       p_void, u64, p_void]),
    "cx_qcsr_spmm_balanced_workspace": (C.c_int, [C.POINTER(CxQcsrMatrix), i64, C.POINTER(u64)]),
    "cx_qcsr_spmm_fwd_balanced": (C.c_int, [C.POINTER(CxQcsrMatrix), p_void, u32, i64, i64, p_void,
                                            i64, C.POINTER(CxSpmmEpilogue), p_void, u64, p_void]),
    "cx_qcsr_spmm_fwd_balanced_noalloc": (C.c_int, [C.POINTER(CxQcsrMatrix), p_void, u32, i64, i64,
                                                    p_void, i64, C.POINTER(CxSpmmEpilogue), p_void]),
    "cx_sort_pairs_workspace": (C.c_int, [u64, u32, C.POINTER(u64)]),
    "cx_sort_pairs": (C.c_int, [p_void, p_void, p_void, p_void, u64, u32, p_void, u64, p_void]),
    "cx_exclusive_scan_u32_workspace": (C.c_int, [u64, C.POINTER(u64)]),
    "cx_exclusive_scan_u32": (C.c_int, [p_void, p_void, u64, p_void, u64, p_void]),
    "cx_bell_spmm_fwd": (C.c_int, [C.POINTER(CxBellMatrix), p_void, u32, i64, i64, p_void, i64, p_void]),
    "cx_bell_spmm_fwd_ordered": (C.c_int, [C.POINTER(CxBellMatrix), p_void, u32, i64, i64, p_void, i64, p_void,
                                           p_void]),
    "cx_bell_spmm_fwd_epilogue": (C.c_int, [C.POINTER(CxBellMatrix), p_void, u32, i64, i64, p_void,
                                            i64, C.POINTER(CxSpmmEpilogue), p_void]),
    "cx_bell_pack_rhs": (C.c_int, [p_void, i64, u32, u32, p_void, p_void]),
    "cx_bell_block_major_values": (C.c_int, [C.POINTER(CxBellMatrix), p_void, u64, p_void]),
    "cx_bell_spmm_fwd_packed": (C.c_int, [C.POINTER(CxBellMatrix), p_void, i64, p_void, i64, p_void]),
    "cx_bell_spmm_fwd_packed_epilogue": (C.c_int, [C.POINTER(CxBellMatrix), p_void, i64, p_void, i64,
                                                   C.POINTER(CxSpmmEpilogue), p_void]),
    "cx_bell_plan_groups": (C.c_int, [p_void, u32, u32, u32, p_void, p_void, C.POINTER(u32),
                                      C.POINTER(u32)]),
    "cx_bell_schedule_groups": (C.c_int, [p_void, u32, u32, p_void, p_void, u32, u32, p_void, p_void,
                                          C.POINTER(u32)]),
    "cx_bell_plan_last_error": (C.c_char_p, []),
    "cx_bell_spmm_fwd_grouped": (C.c_int, [C.POINTER(CxBellMatrix), p_void, C.POINTER(CxBellGroups),
                                           i64, p_void, i64, p_void]),
    "cx_bell_spmm_fwd_grouped_epilogue": (C.c_int, [C.POINTER(CxBellMatrix), p_void,
                                                    C.POINTER(CxBellGroups), i64, p_void, i64,
                                                    C.POINTER(CxSpmmEpilogue), p_void]),
    "cx_cpbp_reduce": (C.c_int, [C.POINTER(CxCpbpTiles), p_void, u64, p_void, u64, p_void]),
    "cx_cpbp_entry_rows": (C.c_int, [C.POINTER(CxCpbpTiles), p_void, u64, p_void]),
    "cx_cpbp_reduce_rows": (C.c_int, [C.POINTER(CxCpbpTiles), p_void, p_void, u64, p_void, u64, p_void]),
    "cx_cpbp_reduction_identity": (u64, [C.POINTER(CxCpbpReductionView)]),
    "cx_cpbp_reduction_view_from_cpk1": (C.c_int, [C.POINTER(CxCpk1View), u64, C.POINTER(CxCpbpReductionView)]),
    "cx_cpbp_reduce_checked": (C.c_int, [C.POINTER(CxCpbpReductionView), p_void, u64, p_void, u64, p_void]),
    "cx_cpk1_image_bytes": (C.c_int, [C.POINTER(CxCpbpTileRequirements), u32, C.POINTER(u64)]),
    "cx_cpk1_write": (C.c_int, [C.POINTER(CxCpbpPlan), C.POINTER(CxCpk1Metadata),
                                C.POINTER(CxCpbpTileRequirements), C.POINTER(CxCpbpTileBuffers),
                                p_void, u64, C.POINTER(CxCpk1View)]),
    "cx_cpk1_validate": (C.c_int, [p_void, u64, C.POINTER(CxCpk1Expected), C.POINTER(CxCpk1View)]),
    "cx_cpk1_rebind": (C.c_int, [C.POINTER(CxCpk1View), p_void, u64, C.POINTER(CxCpk1View)]),
    "cx_cpk1_last_error": (C.c_char_p, []),
    "cx_csr_spmv_fwd": (C.c_int, [u32, p_void, p_void, p_void, u32, p_void, p_void, p_void]),
    "cx_packed_dense_operand_describe": (C.c_int, [C.POINTER(CxCpbpPlan), u64, C.POINTER(CxDenseOperand),
                                                   C.POINTER(CxDenseOperand), C.POINTER(u64)]),
    "cx_pack_dense_operand_host": (C.c_int, [C.POINTER(CxCpbpPlan), u64, C.POINTER(CxDenseOperand), p_void,
                                             u64, C.POINTER(CxDenseOperand)]),
    "cx_pack_dense_operand_device": (C.c_int, [C.POINTER(CxCpbpPlan), u64, C.POINTER(CxDenseOperand),
                                               p_void, u64, p_void, C.POINTER(CxDenseOperand)]),
    "cx_pack_dense_operand": (C.c_int, [p_void, u32, p_void, u64, u64, u32, u32, p_void, u64, p_void]),
    "cx_build_execution_csr_host": (C.c_int, [C.POINTER(CxCpbpPlan), u64, C.POINTER(CxOrderedPartition),
                                              p_void, u64, C.POINTER(CxExecutionCsr)]),
    "cx_lazy_execution_csr_requirements": (C.c_int, [C.POINTER(CxCpk1View), C.POINTER(CxLazyCsrRequirements)]),
    "cx_materialize_execution_csr_from_cpk1_host": (C.c_int, [C.POINTER(CxCpk1View), C.POINTER(CxLazyCsrBuffers),
                                                              C.POINTER(CxExecutionCsr)]),
    "cx_qcsr_column_counts": (C.c_int, [C.POINTER(CxQcsrMatrix), p_void, p_void]),
    "cx_popularity_order": (C.c_int, [p_void, u32, p_void, p_void]),
    "cx_qcsr_to_execution_order": (C.c_int, [C.POINTER(CxQcsrMatrix), p_void, p_void, p_void, p_void, p_void,
                                             p_void]),
    "cx_qcsr_execution_order_lds_bytes": (C.c_int, [C.POINTER(CxQcsrMatrix), C.POINTER(u64)]),
    "cx_exec_last_error": (C.c_char_p, []),
    "cx_qcsr_hybrid_layout_bytes": (C.c_int, [C.POINTER(CxQcsrMatrix), u32, C.POINTER(u64)]),
    "cx_qcsr_hybrid_prepare": (C.c_int, [C.POINTER(CxQcsrMatrix), u32, p_void, u64,
                                         C.POINTER(CxQcsrHybridLayout), p_void]),
    "cx_qcsr_hybrid_workspace": (C.c_int, [C.POINTER(CxQcsrMatrix), u32, i64, C.POINTER(u64)]),
    "cx_qcsr_tail_plan_bytes": (C.c_int, [C.POINTER(CxQcsrMatrix), C.POINTER(CxQcsrHybridLayout), C.POINTER(u64)]),
    "cx_qcsr_tail_plan": (C.c_int, [C.POINTER(CxQcsrMatrix), C.POINTER(CxQcsrHybridLayout), p_void, u64,
                                    C.POINTER(CxQcsrTailStream), C.POINTER(u64), p_void]),
    "cx_qcsr_tail_fill": (C.c_int, [C.POINTER(CxQcsrMatrix), C.POINTER(CxQcsrHybridLayout),
                                    C.POINTER(CxQcsrTailStream), p_void, u64, p_void]),
    "cx_qcsr_spmm_fwd_hybrid": (C.c_int, [C.POINTER(CxQcsrMatrix), C.POINTER(CxQcsrHybridLayout), p_void, i64,
                                          i64, p_void, i64, C.POINTER(CxSpmmEpilogue), p_void, u64, p_void]),
    "cx_query_native_tile_requirements_host": (C.c_int, [C.POINTER(CxFwrPlanView), C.POINTER(CxLocalCellOrderView),
                                                         C.POINTER(CxWarpTileView),
                                                         C.POINTER(CxNativeTileRequirements)]),
    "cx_build_native_tile_view_host": (C.c_int, [C.POINTER(CxFwrPlanView), C.POINTER(CxLocalCellOrderView),
                                                 C.POINTER(CxWarpTileView), C.POINTER(CxNativeTileBuffers),
                                                 C.POINTER(CxNativeTileView)]),
    "cx_query_native_tile_requirements_from_cpk1_host": (C.c_int, [C.POINTER(CxCpk1View),
                                                                   C.POINTER(CxNativeTileRequirements)]),
    "cx_build_native_tile_view_from_cpk1_host": (C.c_int, [C.POINTER(CxCpk1View), C.POINTER(CxNativeTileBuffers),
                                                           C.POINTER(CxNativeTileView)]),
    "cx_decode_native_tile_value_host": (C.c_int, [C.POINTER(CxNativeTileView), u32,
                                                   C.POINTER(CxNativeTileDecodedValue)]),
    "cx_cpbp_tiles_from_native_view": (C.c_int, [C.POINTER(CxNativeTileView), C.POINTER(CxCpbpTiles)]),
    "cx_native_tile_view_rebind": (C.c_int, [C.POINTER(CxNativeTileView), p_void, u64, p_void,
                                             C.POINTER(CxNativeTileView)]),
    "cx_qcsr_head_order": (C.c_int, [p_void, u32, u32, u32, p_void, p_void, p_void, u32, u32, p_void, p_void,
                                     C.POINTER(u32)]),
    "cx_qcsr_exec_prepare": (C.c_int, [C.POINTER(CxQcsrMatrix), u32, C.POINTER(p_void), p_void]),
    "cx_qcsr_exec_query": (C.c_int, [p_void, C.POINTER(CxQcsrExecInfo)]),
    "cx_qcsr_exec_workspace_bytes": (C.c_int, [p_void, i64, C.POINTER(u64)]),
    "cx_qcsr_exec_spmm": (C.c_int, [p_void, p_void, i64, i64, p_void, i64, C.POINTER(CxSpmmEpilogue), p_void, u64,
                                    p_void]),
    "cx_qcsr_exec_destroy": (C.c_int, [p_void]),
    "cx_qcsr_exec_workspace_for": (C.c_int, [u32, u32, u32, i64, C.POINTER(u64)]),
    "cx_cpbp_reduction_validate": (C.c_int, [C.POINTER(CxCpbpReductionView)]),
    "cx_cpbp_builder_create": (C.c_int, [C.POINTER(CxCpbpPlan), C.POINTER(CxCpbpCsr),
                                         C.POINTER(CxCpbpOrderConfig), u32, C.POINTER(p_void)]),
    "cx_cpbp_builder_requirements": (C.c_int, [p_void, C.POINTER(CxCpbpTileRequirements)]),
    "cx_cpbp_builder_export": (C.c_int, [p_void, C.POINTER(CxCpbpTileBuffers)]),
    "cx_cpbp_builder_destroy": (None, [p_void]),
    "cx_cpbp_build_last_error": (C.c_char_p, []),
    "cx_cpbp_device_builder_create": (C.c_int, [C.POINTER(CxCpbpPlan), C.POINTER(CxCpbpCsr),
                                                C.POINTER(CxCpbpOrderConfig), p_void,
                                                C.POINTER(p_void)]),
    "cx_cpbp_device_builder_requirements": (C.c_int, [p_void, C.POINTER(CxCpbpTileRequirements)]),
    "cx_cpbp_device_builder_export": (C.c_int, [p_void, C.POINTER(CxCpbpTileBuffers), p_void]),
    "cx_cpbp_device_builder_destroy": (None, [p_void]),
    "cx_cpbp_device_build_last_error": (C.c_char_p, []),
    "cx_last_error": (C.c_char_p, []),
    "cx_build_info": (C.c_char_p, []),
    "cellerator_status_string": (C.c_char_p, [C.c_int]),
    "cellerator_last_error": (C.c_char_p, []),
    "cellerator_context_create": (C.c_int, [C.POINTER(CelleratorExecutionConfig), C.POINTER(p_void)]),
    "cellerator_context_synchronize": (C.c_int, [p_void]),
    "cellerator_context_destroy": (None, [p_void]),
    "cellerator_saved_state_destroy": (None, [p_void]),
    "cellerator_sparse_projection_forward": (
        C.c_int, [p_void, C.POINTER(CelleratorSparseLayoutDesc), C.POINTER(CelleratorTensorDesc),
                  C.POINTER(CelleratorTensorDesc), C.POINTER(p_void)]),
    "cellerator_sparse_projection_backward": (
        C.c_int, [p_void, C.POINTER(CelleratorSparseLayoutDesc), C.POINTER(CelleratorTensorDesc),
                  C.POINTER(CelleratorTensorDesc), C.POINTER(CelleratorTensorDesc),
                  C.POINTER(CelleratorTensorDesc)]),
}

SYNTH_SIGNATURES = {
    "cxs_qcsr_create": (C.c_int, [C.POINTER(CxsQcsrParams), C.POINTER(p_void)]),
    "cxs_destroy": (None, [p_void]),
    "cxs_qcsr_count": (C.c_int, [p_void, p_void, p_void]),
    "cxs_qcsr_fill": (C.c_int, [p_void, p_void, p_void, p_void, p_void, p_void]),
    "cxs_qcsr_calibrate": (C.c_int, [p_void, p_void, p_void, p_void, p_void, p_void]),
    "cxs_qcsr_encode": (C.c_int, [p_void, p_void, p_void, p_void, p_void, p_void, p_void, p_void,
                                  p_void]),
    "cxs_dense_normal": (C.c_int, [u64, u64, C.c_float, u32, p_void, p_void]),
    "cxs_bell_generate": (C.c_int, [u64, u32, u32, u32, u32, u32, u32, u32, C.c_float, C.c_double,
                                    C.c_double, p_void, p_void, p_void]),
    "cxs_cpbp_count": (C.c_int, [C.POINTER(CxsCpbpParams), p_void, u32]),
    "cxs_cpbp_fill": (C.c_int, [C.POINTER(CxsCpbpParams), p_void, p_void, p_void, u32]),
    "cxs_last_error": (C.c_char_p, []),
}

_engine = None
_synth = None


class EngineError(RuntimeError):
    """A C-ABI entry point returned a non-success status."""

    def __init__(self, name: str, status: int, message: str):
        super().__init__(f"{name} -> {STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


def _bind(path: Path, signatures: dict) -> C.CDLL:
    if not path.exists():
        raise ImportError(
            f"{path.name} is not built; run __graft_entry__.build() (python -m cellerator_amd.build)")
    lib = C.CDLL(str(path))
    for name, (res, args) in signatures.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def engine() -> C.CDLL:
    global _engine
    if _engine is None:
        _engine = _bind(ENGINE_PATH, ENGINE_SIGNATURES)
    return _engine


def synth() -> C.CDLL:
    global _synth
    if _synth is None:
        _synth = _bind(SYNTH_PATH, SYNTH_SIGNATURES)
    return _synth


def check(name: str, status: int) -> None:
    if status != 0:
        msg = engine().cx_last_error().decode()
        raise EngineError(name, status, msg)


def check_synth(name: str, status: int) -> None:
    if status != 0:
        raise RuntimeError(f"{name}: {synth().cxs_last_error().decode()}")
