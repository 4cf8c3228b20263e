/*
 * cellerator_amd.h -- C-ABI of the MI355X projection engine (libcellerator_amd.so).
 *
 * Two layers, both plain C (pointers, sizes, POD descriptors; no C++ or torch types):
 *
 *  1. The thin launch layer (cx_*). One entry point per hot-path operation; each
 *     validates its descriptor on the host, then enqueues hand-written gfx950
 *     kernels on the caller's hipStream_t (passed as void*). Nothing synchronises,
 *     nothing allocates on the launch path. These replace the reference's launchers:
 *       cx_qcsr_spmm_fwd  <- sparse_project::csr_spmm_fwd_f16_f32
 *                            (src/compute/sparse/project/project.hh:12-23, project.cu:31-48)
 *                            generalised to the quantized csr_matrix container
 *                            (include/Cellerator/quantized/layout.cuh:12-39) decoded by
 *                            dequantize_code (include/Cellerator/quantized/access.cuh:81-91)
 *       cx_bell_spmm_fwd  <- sparse_project::blocked_ell_spmm_fwd_f16_f32 and
 *                            quantized_blocked_ell_spmm_fwd_f32
 *                            (src/compute/sparse/project/project.hh:25-62, project.cu:50-168)
 *       cx_cpbp_reduce    <- cellpack::evaluate_feature_weighted_row_reduction_tiles_cuda
 *                            (components/CellPack/include/CellPack/feature_weighted_row_reduction_cuda.hh:17-22,
 *                             components/CellPack/src/feature_weighted_row_reduction_cuda.cu:238-262)
 *
 *  2. The public context ABI (cellerator_*), layout-compatible with the reference's
 *     include/Cellerator/abi.h:11-152 for the structs and functions of the projection
 *     forward path, with two additive enum values: CELLERATOR_DTYPE_BF16 and
 *     CELLERATOR_LAYOUT_QUANTIZED_CSR.
 *
 * Status codes are shared by both layers and equal the reference's cellerator_status
 * values (include/Cellerator/abi.h:14-21). The thread-local message of the last failure
 * is returned by cx_last_error() / cellerator_last_error().
 */
#ifndef CELLERATOR_AMD_H
#define CELLERATOR_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------------- */
/* Shared enums                                                                    */
/* ------------------------------------------------------------------------------- */

#define CELLERATOR_ABI_VERSION 1u
#define CELLERATOR_TENSOR_MAX_RANK 4u

/* include/Cellerator/abi.h:14-21 */
typedef enum cellerator_status {
    CELLERATOR_STATUS_SUCCESS = 0,
    CELLERATOR_STATUS_INVALID_ARGUMENT = 1,
    CELLERATOR_STATUS_INVALID_SHAPE = 2,
    CELLERATOR_STATUS_UNSUPPORTED = 3,
    CELLERATOR_STATUS_CUDA_ERROR = 4, /* a HIP runtime error on this engine */
    CELLERATOR_STATUS_INTERNAL_ERROR = 5
} cellerator_status;

#define CX_STATUS_SUCCESS CELLERATOR_STATUS_SUCCESS
#define CX_STATUS_INVALID_ARGUMENT CELLERATOR_STATUS_INVALID_ARGUMENT
#define CX_STATUS_INVALID_SHAPE CELLERATOR_STATUS_INVALID_SHAPE
#define CX_STATUS_UNSUPPORTED CELLERATOR_STATUS_UNSUPPORTED
#define CX_STATUS_HIP_ERROR CELLERATOR_STATUS_CUDA_ERROR
#define CX_STATUS_INTERNAL_ERROR CELLERATOR_STATUS_INTERNAL_ERROR

/* include/Cellerator/abi.h:23-29, plus BF16 (additive). */
typedef enum cellerator_dtype {
    CELLERATOR_DTYPE_INVALID = 0,
    CELLERATOR_DTYPE_F16 = 1,
    CELLERATOR_DTYPE_F32 = 2,
    CELLERATOR_DTYPE_U8 = 3,
    CELLERATOR_DTYPE_U32 = 4,
    CELLERATOR_DTYPE_BF16 = 5
} cellerator_dtype;

/* include/Cellerator/quantized/blocked_ell.cuh:10-14 */
#define CX_DECODE_PER_GENE_AFFINE 1u
#define CX_DECODE_COLUMN_SCALE_ROW_OFFSET 2u
/* Engine addition (no counterpart in the reference): per-gene affine decode with the
 * metadata interleaved, column_scales -> cols (scale, offset) float pairs (8-byte
 * aligned), column_offsets = NULL. Decodes bit-identically to CX_DECODE_PER_GENE_AFFINE;
 * one 8-byte gather per stored code instead of two 4-byte ones. Built once per metadata
 * generation by cx_qcsr_pack_gene_affine. */
#define CX_DECODE_PER_GENE_AFFINE_PAIRS 3u

/* Fused SpMM epilogue kinds: the values of the reference's epilogue_kind
 * (include/Cellerator/compute/math/operation.hh:49-58). */
#define CX_EPILOGUE_NONE 0u
#define CX_EPILOGUE_BIAS 1u
#define CX_EPILOGUE_RELU 2u
#define CX_EPILOGUE_GELU_ERF 3u
#define CX_EPILOGUE_GELU_TANH 4u
#define CX_EPILOGUE_BIAS_RELU 5u
#define CX_EPILOGUE_BIAS_GELU_ERF 6u
#define CX_EPILOGUE_BIAS_GELU_TANH 7u

/* ------------------------------------------------------------------------------- */
/* 1. Thin launch layer                                                            */
/* ------------------------------------------------------------------------------- */

/* Fused epilogue of an SpMM: every output element is
 *     Y[r,c] = act(alpha * (A . W)[r,c] + beta * C[r,c] + bias[c])
 * applied to the fp32 accumulator before its single store. This is the alpha / beta /
 * epilogue part of spmm_request (include/Cellerator/compute/math/operation.hh:136-164)
 * as the CPU referee applies it (src/compute/math/referee.cc:75-97,170-250): beta * C,
 * plus alpha * the product, then the bias (bias kinds only), then the activation --
 * ReLU max(v, 0); exact GELU 0.5 v (1 + erf(v / sqrt 2)); tanh GELU
 * 0.5 v (1 + tanh(0.7978845608 (v + 0.044715 v^3))). Computed in fp32 (the referee
 * uses double). alpha == 0 skips the product: the contract's epilogue-only case
 * (src/compute/math/operation.cc:282-292). A NULL epilogue, or kind NONE with alpha 1
 * and beta 0, is the plain product (bit-identical to the entry without an epilogue). */
typedef struct cx_spmm_epilogue {
    uint32_t kind;          /* CX_EPILOGUE_* */
    uint32_t reserved;      /* must be 0 */
    float alpha;
    float beta;
    const float *bias;      /* out_cols f32 values for the bias kinds; NULL otherwise */
    const float *initial;   /* C: rows x out_cols f32, row-major, leading dimension
                               initial_ld; read only when beta != 0. May be the output
                               itself with initial_ld == out_ld (in-place update); must
                               not otherwise overlap the output. */
    int64_t initial_ld;
} cx_spmm_epilogue;

/* Quantized (or plain) CSR cells x genes matrix. Field meaning follows
 * cellerator::quantized::csr_matrix (include/Cellerator/quantized/layout.cuh:24-37):
 * row_ptr are nnz offsets, packed_row_ptr are byte offsets of each row's unpadded
 * packed codes (layout.cuh:106-129), codes are little-endian within a byte
 * (format.cuh:39-48). bits == 0 selects unquantized values: `values` of
 * `value_dtype` (F16 or F32), one per nnz, as csr_spmm_fwd_f16_f32 consumes. */
typedef struct cx_qcsr_matrix {
    uint32_t rows;
    uint32_t cols;
    uint64_t nnz;
    uint32_t bits;          /* 1, 2, 4, 8; 0 = unquantized `values` */
    uint32_t decode_policy; /* CX_DECODE_* (ignored when bits == 0) */
    const int32_t *row_ptr;        /* rows + 1 */
    const int32_t *packed_row_ptr; /* rows + 1 (ignored when bits == 0) */
    const int32_t *col_idx;        /* nnz */
    const uint8_t *packed_values;  /* packed_row_ptr[rows] bytes */
    const float *column_scales;    /* cols or NULL (-> 1) */
    const float *column_offsets;   /* cols or NULL (-> 0); per_gene_affine */
    const float *row_offsets;      /* rows or NULL (-> 0); column_scale_row_offset */
    const void *values;            /* nnz of value_dtype when bits == 0 */
    uint32_t value_dtype;          /* cellerator_dtype, bits == 0 only */
    uint32_t flags;                /* CX_QCSR_* properties the caller vouches for; 0 = none */
} cx_qcsr_matrix;

/* cx_qcsr_matrix.flags: every row's columns are non-decreasing and lie in [0, cols), as the
 * reference's containers store them (cx_qcsr_check_columns establishes it). The gene-part
 * kernels then skip the per-entry check that sends rows out of order to a per-row path; a
 * row that breaks the promise gets wrong sums, never an out-of-bounds read. Engine addition,
 * no counterpart in the reference. */
#define CX_QCSR_COLUMNS_SORTED 1u

/* Y[rows x out_cols] (fp32, row stride out_ld) = decode(A) . RHS[cols x out_cols]
 * (row stride rhs_ld, dtype F16 or F32; F16 widens exactly). fp32 multiply and
 * fp32 accumulation, deterministic (fixed per-row summation order). Quantized codes with
 * F16 RHS at out_cols = 64, 128, 192 or 256 stream RHS through LDS by gene part, 64 output
 * columns per launch: fastest with each row's columns ascending; rows out of order across parts are
 * recomputed per row, and columns outside [0, cols) contribute nothing on that path.
 * Replaces csr_spmm_fwd_f16_f32 (src/compute/sparse/project/project.hh:12-23). */
int cx_qcsr_spmm_fwd(const cx_qcsr_matrix *a, const void *rhs, uint32_t rhs_dtype,
                     int64_t rhs_ld, int64_t out_cols, float *out, int64_t out_ld,
                     void *stream);

/* cx_qcsr_spmm_fwd with a fused epilogue (cx_spmm_epilogue; NULL = none): the
 * spmm_request alpha / beta / epilogue (operation.hh:136-164) on the quantized CSR path.
 * Same kernels and summation order; the epilogue runs on each output element once. */
int cx_qcsr_spmm_fwd_epilogue(const cx_qcsr_matrix *a, const void *rhs, uint32_t rhs_dtype,
                              int64_t rhs_ld, int64_t out_cols, float *out, int64_t out_ld,
                              const cx_spmm_epilogue *epilogue, void *stream);

/* Load-balanced form of cx_qcsr_spmm_fwd_epilogue for skewed row lengths (the transpose of an
 * expression matrix has genes stored in nearly every cell): the nnz range is cut into equal
 * chunks (about 65,536 of at least 1,024 entries), one wave per chunk. Rows inside a chunk
 * are stored directly; the pieces of rows crossing a chunk edge are written to `workspace`
 * and summed by a second kernel in chunk order, so results are deterministic (per element
 * the summation order differs from the row-wave form's). Applies to N = 64 or 128 with
 * aligned operands; other shapes run the row-wave form. workspace (16-byte aligned) holds
 * cx_qcsr_spmm_balanced_workspace bytes; no counterpart in the reference. */
int cx_qcsr_spmm_balanced_workspace(const cx_qcsr_matrix *a, int64_t out_cols, uint64_t *bytes);
int cx_qcsr_spmm_fwd_balanced(const cx_qcsr_matrix *a, const void *rhs, uint32_t rhs_dtype,
                              int64_t rhs_ld, int64_t out_cols, float *out, int64_t out_ld,
                              const cx_spmm_epilogue *epilogue, void *workspace,
                              uint64_t workspace_bytes, void *stream);

/* cx_qcsr_spmm_fwd_balanced without a workspace argument: the partial rows of rows that
 * cross a chunk edge live in a 32 MiB device array of the library (one per GPU, held until
 * the process ends; resolved on the first call on a device), so the call allocates nothing.
 * Same kernels, chunking and results (bitwise) as cx_qcsr_spmm_fwd_balanced. Returns
 * INVALID_SHAPE when the partial rows need more than 32 MiB (N = 128 with more than 32,768
 * chunks, i.e. above about 33.5M entries). The array keeps the last call's contents and is
 * shared by every call on its GPU: calls that overlap on one GPU race. The stream's device
 * must be the current device. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (HIP graph capture, tight serving loops, allocation-free harnesses). */
int cx_qcsr_spmm_fwd_balanced_noalloc(const cx_qcsr_matrix *a, const void *rhs, uint32_t rhs_dtype,
                                      int64_t rhs_ld, int64_t out_cols, float *out, int64_t out_ld,
                                      const cx_spmm_epilogue *epilogue, void *stream);

/* Interleaves per-gene metadata for CX_DECODE_PER_GENE_AFFINE_PAIRS:
 * pairs[2c] = scales[c] (1 if scales is NULL), pairs[2c+1] = offsets[c] (0 if NULL),
 * for c < cols; pairs (device, 8-byte aligned) holds 2 * cols floats. No counterpart in
 * the reference: it prepares the layout the decode reads in one gather. */
int cx_qcsr_pack_gene_affine(const float *scales, const float *offsets, uint32_t cols,
                             float *pairs, void *stream);

/* Writes CX_QCSR_COLUMNS_SORTED to *device_flag (one uint32 in device memory) when every row
 * of a has non-decreasing columns in [0, cols), else 0; stream-ordered, reads row_ptr and
 * col_idx once. The prepare step behind cx_qcsr_matrix.flags; engine addition, no
 * counterpart in the reference. */
int cx_qcsr_check_columns(const cx_qcsr_matrix *a, uint32_t *device_flag, void *stream);

/* Synchronous form for preparation steps: runs cx_qcsr_check_columns on `stream`, waits for
 * it and stores CX_QCSR_COLUMNS_SORTED or 0 in *host_flag. Allocates (and frees) one word of
 * device memory, so it is not for launch paths. Engine addition, no reference counterpart. */
int cx_qcsr_check_columns_sync(const cx_qcsr_matrix *a, uint32_t *host_flag, void *stream);

/* Waits for the work enqueued on `stream` (a hipStream_t; NULL = the null stream). For host
 * code that reaches the engine only through this C-ABI. Engine addition. */
int cx_stream_synchronize(void *stream);

/* ---- the quantized codec as device passes over a row block -----------------------------
 * csr_block (include/Cellerator/quantized/layout.cuh:41-49): a row range of the matrix and
 * its entry and packed-byte ranges. */
typedef struct cx_qcsr_block {
    int32_t block_index;
    int32_t row_begin;
    int32_t row_end;
    int32_t nnz_begin;
    int32_t nnz_end;
    int32_t packed_begin;
    int32_t packed_end;
    int32_t reserved;  /* the reference's alignas(32) */
} cx_qcsr_block;

/* get_block (include/Cellerator/quantized/access.cuh:7-45) over host arrays: block
 * block_index of block_row_ptr (block_count + 1 row starts), or the whole matrix when
 * block_row_ptr is NULL or block_count <= 0. */
int cx_qcsr_get_block(const int32_t *block_row_ptr, int32_t block_count, const int32_t *row_ptr,
                      const int32_t *packed_row_ptr, int32_t rows, int32_t block_index, cx_qcsr_block *out);
/* launch_quantize_block (include/Cellerator/quantized/dispatch.cuh:35-47) with
 * pack_row_values (packing.cuh:13-146): the F32 values of the block's entries
 * (values_by_nnz_block[i - block->nnz_begin]) encoded by the portable rule
 * (access.cuh:104-131) with a's metadata and packed into packed_out (a's packed layout; the
 * high bits of a row's last byte are zero). block NULL = every row (values from entry 0).
 * Writes only the block's packed bytes. */
int cx_qcsr_quantize_block(const cx_qcsr_matrix *a, const cx_qcsr_block *block,
                           const float *values_by_nnz_block, uint8_t *packed_out, void *stream);
/* launch_dequantize_block (dispatch.cuh:49-61) with unpack_row_values (packing.cuh:148-260):
 * values_by_nnz_block[i - block->nnz_begin] = fma(code, scale, offset) for the block's
 * entries. */
int cx_qcsr_dequantize_block(const cx_qcsr_matrix *a, const cx_qcsr_block *block, float *values_by_nnz_block,
                             void *stream);

/* ---- backend-neutral SpMM request (include/Cellerator/compute/math/operation.hh) -------
 * The reference's math contract as plain C structs with the same member order, sizes and
 * values (so the bytes of a reference spmm_request are a valid cx_spmm_request), its
 * validation, its 128-bit operation signature, the trivial-work classification, and a
 * request-driven entry onto the quantized CSR kernels. Type codes are the reference's
 * real::value_* codes (f16 3, f32 4, f64 5, bf16 6, fp8 e4m3 7, fp8 e5m2 8). */
#define CX_OPERATION_CONTRACT_SCHEMA_VERSION 1u
#define CX_OPERATION_SPMM 1u
#define CX_TRANSPOSE_NONE 0u
#define CX_TRANSPOSE 1u
#define CX_LAYOUT_ROW_MAJOR 1u
#define CX_LAYOUT_COLUMN_MAJOR 2u
#define CX_ALLOW_NONDETERMINISTIC 0u
#define CX_DETERMINISTIC 1u
#define CX_WORKSPACE_REUSABLE_POOL 1u
#define CX_WORKSPACE_CALLER_LIMIT 2u
#define CX_WORKSPACE_NONE 3u
#define CX_REUSE_SINGLE_RUN 1u
#define CX_REUSE_BOUNDED 2u
#define CX_REUSE_PERSISTENT 3u
#define CX_FEATURE_ORDER_KIND_CANONICAL 1u
#define CX_FEATURE_ORDER_KIND_PACKED 2u
#define CX_REAL_F16 3u
#define CX_REAL_F32 4u
#define CX_REAL_F64 5u
#define CX_REAL_BF16 6u
#define CX_REAL_FP8_E4M3 7u
#define CX_REAL_FP8_E5M2 8u
/* request_validation_code (operation.hh:68-85) */
#define CX_REQUEST_OK 0u
#define CX_REQUEST_UNSUPPORTED_VERSION 1u
#define CX_REQUEST_INVALID_SHAPE 2u
#define CX_REQUEST_INVALID_TYPE 3u
#define CX_REQUEST_INVALID_SCALAR 4u
#define CX_REQUEST_INVALID_WORKSPACE_POLICY 5u
#define CX_REQUEST_INVALID_REUSE 6u
#define CX_REQUEST_INVALID_FEATURE_ORDER 7u
#define CX_REQUEST_FEATURE_ORDER_MISMATCH 8u
#define CX_REQUEST_MISSING_BIAS 9u
#define CX_REQUEST_UNEXPECTED_BIAS 10u
#define CX_REQUEST_INVALID_LAYOUT 11u
#define CX_REQUEST_INVALID_IDENTITY 12u
#define CX_REQUEST_MISSING_BINDING 13u
#define CX_REQUEST_INVALID_DETERMINISM 14u
#define CX_REQUEST_INVALID_EPILOGUE 15u
/* trivial_operation_kind (operation.hh:197-201) */
#define CX_TRIVIAL_NONE 0u
#define CX_TRIVIAL_NO_OUTPUT 1u
#define CX_TRIVIAL_EPILOGUE_ONLY 2u

typedef struct cx_feature_order_identity {  /* operation.hh:89-96 */
    uint32_t schema_version;                /* 1 */
    uint32_t kind;                          /* CX_FEATURE_ORDER_KIND_* */
    uint32_t feature_count;
    uint32_t feature_axis_identity_version;
    uint64_t feature_axis_identity;
    uint64_t packing_geometry_identity;     /* nonzero exactly for packed orders */
} cx_feature_order_identity;

typedef struct cx_sparse_structure_identity {  /* operation.hh:100-104 */
    uint32_t schema_version;                   /* 1 */
    uint32_t identity_version;
    uint64_t value;
} cx_sparse_structure_identity;

typedef struct cx_scalar_value {  /* operation.hh:106-110: f32 bits in the low word, or f64 */
    uint32_t type_code;
    uint32_t reserved;
    uint64_t bits;
} cx_scalar_value;

typedef struct cx_workspace_policy {  /* operation.hh:112-117 */
    uint32_t kind;
    uint32_t reserved;
    uint64_t byte_limit;
} cx_workspace_policy;

typedef struct cx_expected_reuse {  /* operation.hh:119-124 */
    uint32_t kind;
    uint32_t reserved;
    uint64_t expected_run_count;
} cx_expected_reuse;

typedef struct cx_epilogue_descriptor {  /* operation.hh:126-130 */
    uint32_t kind;                       /* CX_EPILOGUE_* */
    uint32_t bias_type_code;
    uint64_t bias_element_count;
} cx_epilogue_descriptor;

typedef struct cx_spmm_request {  /* spmm_request, operation.hh:136-164 */
    uint32_t schema_version;
    uint32_t operation;
    uint64_t m, k, n;
    uint64_t sparse_nnz;
    cx_sparse_structure_identity sparse_structure;
    uint32_t transpose_sparse;
    uint32_t transpose_dense;
    uint32_t dense_rhs_layout;
    uint32_t output_layout;
    uint64_t dense_rhs_leading_dimension;
    uint64_t output_leading_dimension;
    uint32_t sparse_storage_type_code;
    uint32_t dense_storage_type_code;
    uint32_t output_storage_type_code;
    uint32_t compute_type_code;
    uint32_t accumulation_type_code;
    cx_scalar_value alpha;
    cx_scalar_value beta;
    uint32_t determinism;
    cx_workspace_policy workspace;
    cx_expected_reuse reuse;
    cx_epilogue_descriptor epilogue;
    cx_feature_order_identity sparse_feature_order;
    cx_feature_order_identity dense_feature_order;
} cx_spmm_request;

typedef struct cx_spmm_bindings {  /* operation.hh:166-174 */
    const void *sparse_matrix;
    const void *dense_rhs;
    void *output;
    const void *bias;
    uint64_t sparse_matrix_identity;
    uint64_t dense_rhs_identity;
    uint64_t output_identity;
} cx_spmm_bindings;

typedef struct cx_operation_signature {  /* operation.hh:181-186 */
    uint32_t schema_version;
    uint32_t operation;
    uint64_t low;
    uint64_t high;
} cx_operation_signature;

/* A cx_spmm_request with the reference's defaults (request_fixture-neutral: schema 1,
 * SpMM, row-major layouts, reusable pool, single run, canonical feature orders). */
void cx_spmm_request_init(cx_spmm_request *request);
cx_scalar_value cx_scalar_f32(float value);
cx_scalar_value cx_scalar_f64(double value);
/* validate_spmm_request (src/compute/math/operation.cc:119-249): CX_REQUEST_* code;
 * *message (may be NULL) gets the reference's text. */
uint32_t cx_validate_spmm_request(const cx_spmm_request *request, const char **message);
/* validate_math_request (operation.cc:251-280): the request, then the bindings. */
uint32_t cx_validate_math_request(const cx_spmm_request *request, const cx_spmm_bindings *bindings,
                                  const char **message);
/* make_operation_signature (src/compute/math/operation_signature.cc:30-68). */
cx_operation_signature cx_make_operation_signature(const cx_spmm_request *request);
/* classify_trivial_operation (operation.cc:282-293). */
uint32_t cx_classify_trivial_operation(const cx_spmm_request *request);
/* Runs a validated math request on a quantized CSR: bindings.sparse_matrix is a
 * cx_qcsr_matrix, dense_rhs the weights, output the fp32 output, bias the fp32 bias. The
 * request must describe this matrix (m = rows, k = cols, sparse_nnz = nnz), untransposed
 * row-major operands, F16 or F32 dense storage, F32 output / compute / accumulation,
 * feature orders that agree (checked by validation; a packed order means the matrix and W
 * are both in that execution order). alpha and beta f32, or f64 exactly representable in
 * f32. No-output requests return at once; epilogue-only requests (alpha 0, K 0 or no
 * stored entries) write act(beta C + bias) without reading the matrix's values.
 * INVALID_ARGUMENT with the validation text for a rejected request, UNSUPPORTED for a valid
 * form this entry does not run. */
int cx_qcsr_spmm_fwd_request(const cx_spmm_request *request, const cx_spmm_bindings *bindings, void *stream);

/* ---- transpose and backward of the CSR SpMM ------------------------------------ */

/* Device bytes of workspace cx_qcsr_transpose needs for `a`. */
int cx_qcsr_transpose_workspace(const cx_qcsr_matrix *a, uint64_t *bytes);

/* Builds A^T (cols x rows) as a plain f32 CSR on the device: t_row_ptr[cols + 1],
 * t_col_idx[nnz] (cell rows, ascending within each gene row), t_values[nnz] (each entry
 * decoded exactly as the forward decodes it). Viewed as a cx_qcsr_matrix {rows = a.cols,
 * cols = a.rows, bits = 0, value_dtype = F32}, it computes A^T . B with cx_qcsr_spmm_fwd --
 * the referee's transpose_sparse product (src/compute/math/referee.cc:170-232) -- and the
 * backward grad_W (cx_qcsr_spmm_bwd_rhs). Deterministic: a stable device radix sort of the
 * column indices (no atomics). Built once per structure and value generation; no
 * counterpart in the reference, whose backward scatters with atomics instead. */
int cx_qcsr_transpose(const cx_qcsr_matrix *a, int32_t *t_row_ptr, int32_t *t_col_idx,
                      float *t_values, void *workspace, uint64_t workspace_bytes, void *stream);

/* Panelled transpose for grad_rhs at large row counts: rows ordered by (cell panel, gene), a
 * panel being panel_rows consecutive cells, i.e. row p * cols + g holds the cells of gene g
 * inside panel p, ascending (a.cols * ceil(a.rows / panel_rows) rows, t_row_ptr one more).
 * While the balanced SpMM walks it, the grad_out rows of one panel (panel_rows x N x 4 bytes)
 * stay in L2 instead of being gathered from all of grad_out for every gene. */
int cx_qcsr_transpose_panelled_workspace(const cx_qcsr_matrix *a, uint32_t panel_rows,
                                         uint64_t *bytes);
int cx_qcsr_transpose_panelled(const cx_qcsr_matrix *a, uint32_t panel_rows, int32_t *t_row_ptr,
                               int32_t *t_col_idx, float *t_values, void *workspace,
                               uint64_t workspace_bytes, void *stream);

/* grad_rhs = A^T . grad_out on a panelled transpose of `panels` panels: the balanced SpMM
 * writes one partial row per (panel, gene) into the workspace, then a reduction sums each
 * gene's partials in panel order (deterministic). workspace: 16-byte aligned, the query's
 * bytes (partials + balanced-SpMM scratch). */
int cx_qcsr_spmm_bwd_rhs_panelled_workspace(const cx_qcsr_matrix *panelled, uint32_t panels,
                                            int64_t out_cols, uint64_t *bytes);
int cx_qcsr_spmm_bwd_rhs_panelled(const cx_qcsr_matrix *panelled, uint32_t panels,
                                  const float *grad_out, int64_t grad_out_ld, int64_t out_cols,
                                  float *grad_rhs, int64_t grad_rhs_ld, void *workspace,
                                  uint64_t workspace_bytes, void *stream);

/* grad_values[i] = sum_{c < out_cols} grad_out[row_i, c] * rhs[col_i, c] for every stored
 * entry i: the gradient of Y = A . RHS with respect to A's (decoded) values. Replaces
 * csr_spmm_bwd_values_f16_f32 (src/compute/sparse/ops/ops.hh:111-120,
 * kernels/base_sparse/csr_spmm_bwd_values_kernel_.cuh), whose kernel reads grad_out with the
 * rhs leading dimension; here each operand has its own. Reads only A's structure. fp32
 * products and sums in a fixed order; rhs F16 or F32, grad_out F32. With F16 rhs at
 * out_cols = 64 the rhs streams through LDS by gene part (fastest with each row's columns
 * ascending); there an entry whose column lies outside [0, cols) gets 0. */
int cx_qcsr_spmm_bwd_values(const cx_qcsr_matrix *a, const float *grad_out,
                            int64_t grad_out_ld, const void *rhs, uint32_t rhs_dtype,
                            int64_t rhs_ld, int64_t out_cols, float *grad_values, void *stream);

/* grad_rhs[cols x out_cols] = A^T . grad_out, with `transposed` the f32 transpose built by
 * cx_qcsr_transpose: cx_qcsr_spmm_fwd_balanced on A^T (workspace sized by
 * cx_qcsr_spmm_balanced_workspace(transposed, out_cols)), every element in a fixed order. Replaces csr_spmm_bwd_rhs_f16_f32 (src/compute/sparse/ops/ops.hh:122-133,
 * kernels/base_sparse/csr_spmm_bwd_rhs_kernel_.cuh), which zero-fills grad_rhs and adds
 * with float atomics. */
int cx_qcsr_spmm_bwd_rhs(const cx_qcsr_matrix *transposed, const float *grad_out,
                         int64_t grad_out_ld, int64_t out_cols, float *grad_rhs,
                         int64_t grad_rhs_ld, void *workspace, uint64_t workspace_bytes,
                         void *stream);

/* Stable LSD radix sort of (key, value) u32 pairs on the device, on the keys' low key_bits
 * bits (8 bits per pass); vals_in == NULL sorts the identity permutation (value = input
 * position). Outputs must not alias inputs. Deterministic. Engine utility behind the
 * transpose (no counterpart in the reference, which uses CUB). */
int cx_sort_pairs_workspace(uint64_t count, uint32_t key_bits, uint64_t *bytes);
int cx_sort_pairs(const uint32_t *keys_in, const uint32_t *vals_in, uint32_t *keys_out,
                  uint32_t *vals_out, uint64_t count, uint32_t key_bits, void *workspace,
                  uint64_t workspace_bytes, void *stream);

/* Exclusive prefix sum of u32 values on the device (wraps modulo 2^32). */
int cx_exclusive_scan_u32_workspace(uint64_t count, uint64_t *bytes);
int cx_exclusive_scan_u32(const uint32_t *in, uint32_t *out, uint64_t count, void *workspace,
                          uint64_t workspace_bytes, void *stream);

/* Blocked-ELL matrix (include/Cellerator/quantized/blocked_ell.cuh:18-35 and the
 * cs::sparse::blocked_ell layout consumed by blocked_ell_spmm_fwd_kernel_):
 * block_col_idx is (rows/block_size) x (ell_cols/block_size), 0xffffffff marks an
 * empty slot; values are row-major rows x ell_cols. bits != 0 selects the quantized
 * form (packed codes, row stride row_stride_bytes). */
typedef struct cx_bell_matrix {
    uint32_t rows;
    uint32_t cols;
    uint32_t block_size;
    uint32_t ell_cols;
    const uint32_t *block_col_idx;
    const void *values;  /* rows x ell_cols of value_dtype (BF16, F16 or F32) */
    uint32_t value_dtype;
    uint32_t bits;       /* 0 = plain values; 1, 2, 4, 8 = packed codes */
    uint32_t decode_policy;
    uint32_t row_stride_bytes;
    const uint8_t *packed_values;
    const float *column_scales;
    const float *column_offsets;
    const float *row_offsets;
    uint32_t value_layout_flags; /* 0 or CX_BELL_BLOCK_MAJOR_VALUES */
    uint32_t reserved;           /* 0 */
} cx_bell_matrix;

/* cx_bell_matrix.value_layout_flags: the unquantized values are block-major,
 * [ceil(rows / block_size)][slot][row in block][column in block] with every block whole
 * (rows past the matrix are padding) -- the layout the CSR -> Blocked-ELL lowering emits as
 * CX_BELL_VALUES_BLOCK_MAJOR (physical_bell.hh) -- instead of row-major [rows][ell_cols].
 * Every Blocked-ELL entry point takes either layout with the same results; quantized
 * (packed) values are row-major only. Engine addition (the reference's projection kernels
 * read row-major values). */
#define CX_BELL_BLOCK_MAJOR_VALUES 1u

/* Copies the row-major unquantized values of `a` into block-major order
 * (CX_BELL_BLOCK_MAJOR_VALUES), zero rows for the padding of the last row block:
 * ceil(rows / block_size) * ell_cols * block_size elements of a->value_dtype; `capacity`
 * is the size of `out` in bytes. Engine addition, done once per matrix. */
int cx_bell_block_major_values(const cx_bell_matrix *a, void *out, uint64_t capacity,
                               void *stream);

/* Y = X_bell . RHS with a row-major RHS (F32, F16 or BF16), any block size and N, plain
 * (BF16/F16/F32) or quantized values: fp32 accumulation in slot order per output
 * element, the semantics of blocked_ell_spmm_fwd_kernel_ / quantized_blocked_ell_spmm_fwd_kernel_
 * (src/compute/sparse/project/kernels/blocked_ell_spmm_fwd_kernel_.cuh:1-33,
 *  quantized_blocked_ell_spmm_fwd_kernel_.cuh:1-39). Replaces
 * blocked_ell_spmm_fwd_f16_f32 / quantized_blocked_ell_spmm_fwd_f32
 * (src/compute/sparse/project/project.cu:50-168). */
int cx_bell_spmm_fwd(const cx_bell_matrix *a, const void *rhs, uint32_t rhs_dtype,
                     int64_t rhs_ld, int64_t out_cols, float *out, int64_t out_ld,
                     void *stream);

/* cx_bell_spmm_fwd with the row blocks taken in `row_block_order` (device, one u32 per row
 * block, a permutation of them; entries past the row-block count are skipped): the
 * quantized matrix-core forms give workgroup slot i (XCD-major) row block
 * row_block_order[i]; other forms ignore it. Same results. An order from
 * cx_bell_schedule_groups (every XCD's range about the same number of value blocks, a
 * module's row blocks together) took C4's quantized projection 3.89 -> 3.80 ms. No
 * counterpart in the reference; no epilogue. */
int cx_bell_spmm_fwd_ordered(const cx_bell_matrix *a, const void *rhs, uint32_t rhs_dtype,
                             int64_t rhs_ld, int64_t out_cols, float *out, int64_t out_ld,
                             const uint32_t *row_block_order, void *stream);

/* cx_bell_spmm_fwd with a fused epilogue (cx_spmm_epilogue; NULL = none), the
 * spmm_request alpha / beta / epilogue (operation.hh:136-164). */
int cx_bell_spmm_fwd_epilogue(const cx_bell_matrix *a, const void *rhs, uint32_t rhs_dtype,
                              int64_t rhs_ld, int64_t out_cols, float *out, int64_t out_ld,
                              const cx_spmm_epilogue *epilogue, void *stream);

/* Packs a row-major bf16 RHS [k x n] (n a multiple of 32) into the matrix-core operand
 * panel, in fragment order: for every 32-gene block column kb, output-column tile t
 * (32 columns) and K half h (16 genes), 64 groups of 8 bf16, group l holding column
 * 32 t + l % 32, genes 32 kb + 16 h + 8 (l / 32) .. + 7 -- exactly the 16 bytes lane l of a
 * v_mfma_f32_32x32x16_bf16 B operand takes, so one wave reads each 1 KB piece contiguously
 * (genes past k are zero). The Blocked-ELL counterpart of pack_dense_operand_cuda
 * (include/Cellerator/compute/math/packed_dense_operand.hh:16-70). `packed` holds
 * ceil(k/32) * n * 32 bf16. Done once per weight generation. */
int cx_bell_pack_rhs(const uint16_t *rhs_bf16, int64_t rhs_ld, uint32_t k, uint32_t n,
                     uint16_t *packed, void *stream);

/* MFMA Blocked-ELL: bf16 32x32 value blocks x packed bf16 panel -> fp32 Y, N in
 * {64, 128, 256}, v_mfma_f32_32x32x16_bf16 with fp32 accumulation. Same result
 * contract as cx_bell_spmm_fwd within fp32 reordered-sum tolerance. */
int cx_bell_spmm_fwd_packed(const cx_bell_matrix *a, const uint16_t *packed_rhs,
                            int64_t out_cols, float *out, int64_t out_ld, void *stream);

/* cx_bell_spmm_fwd_packed with a fused epilogue (cx_spmm_epilogue; NULL = none). */
int cx_bell_spmm_fwd_packed_epilogue(const cx_bell_matrix *a, const uint16_t *packed_rhs,
                                     int64_t out_cols, float *out, int64_t out_ld,
                                     const cx_spmm_epilogue *epilogue, void *stream);

/* Row-block groups for the grouped MFMA path (engine addition, no counterpart in the
 * reference; a persistent preprocessing of the Blocked-ELL projection, like the packed
 * panel). order[0 .. grouped_row_blocks) holds group_count groups of 1..4 row blocks
 * (group g = order[group_offsets[g] .. group_offsets[g+1]), longest member last) whose valid
 * block-column lists are prefixes of the longest member's; order[grouped_row_blocks ..)
 * holds single_count row blocks run one per workgroup. cx_bell_plan_groups forms groups of
 * 2..4 and leaves the rest single; cx_bell_schedule_groups folds the singles in as
 * one-member groups. order and group_offsets are device arrays. */
typedef struct cx_bell_groups {
    uint32_t group_count;
    uint32_t grouped_row_blocks;
    uint32_t single_count;
    uint32_t reserved;
    const uint32_t *order;         /* ceil(rows/32) row block ids */
    const uint32_t *group_offsets; /* group_count + 1 */
} cx_bell_groups;

/* Host planner for cx_bell_groups: block_col_idx (HOST copy, row_blocks x slots, 0xffffffff
 * = empty) -> order (row_blocks), group_offsets (row_blocks + 1 capacity), counts. Groups hold
 * up to max_group (1..4) row blocks. Deterministic. */
int cx_bell_plan_groups(const uint32_t *block_col_idx, uint32_t row_blocks, uint32_t slots,
                        uint32_t max_group, uint32_t *order, uint32_t *group_offsets,
                        uint32_t *group_count, uint32_t *single_count);

/* Launch schedule of a cx_bell_plan_groups plan (host arrays in, host arrays out): every
 * group and every single row block becomes one unit (a group of 1..4 row blocks), and the
 * units are ordered so that the eight contiguous ranges the grouped kernels give the eight
 * XCDs (workgroup i runs unit (i % 8) * (units / 8) + i / 8; the last units % 8 keep their
 * index) carry about the same number of value blocks, units of one module (same first block
 * column) kept in one range where they fit. sched_order holds row_blocks ids, sched_offsets
 * units + 1 entries (capacity row_blocks + 1); pass them as a cx_bell_groups with
 * group_count = units, grouped_row_blocks = row_blocks and single_count = 0. Deterministic.
 * No counterpart in the reference: its Blocked-ELL kernel runs one block row per thread
 * block in matrix order. */
int cx_bell_schedule_groups(const uint32_t *block_col_idx, uint32_t row_blocks, uint32_t slots,
                            const uint32_t *order, const uint32_t *group_offsets,
                            uint32_t group_count, uint32_t single_count, uint32_t *sched_order,
                            uint32_t *sched_offsets, uint32_t *unit_count);
const char *cx_bell_plan_last_error(void);

/* Same result contract as cx_bell_spmm_fwd_packed: per group, each N x 32 panel slice is
 * loaded once for all members (staged in LDS at N = 64; at N = 128 and 256 each wave loads
 * its column slab and the members' value blocks are shared through LDS); per output element
 * the MFMA accumulation runs in the same slot order as the ungrouped kernel, so the results
 * are bitwise equal. One launch: single row blocks run as one-member groups. At most 64
 * slots per row block. */
int cx_bell_spmm_fwd_grouped(const cx_bell_matrix *a, const uint16_t *packed_rhs,
                             const cx_bell_groups *groups, int64_t out_cols, float *out,
                             int64_t out_ld, void *stream);

/* cx_bell_spmm_fwd_grouped with a fused epilogue (cx_spmm_epilogue; NULL = none). */
int cx_bell_spmm_fwd_grouped_epilogue(const cx_bell_matrix *a, const uint16_t *packed_rhs,
                                      const cx_bell_groups *groups, int64_t out_cols,
                                      float *out, int64_t out_ld,
                                      const cx_spmm_epilogue *epilogue, void *stream);

/* ---- CSR -> Blocked-ELL lowering (include/Cellerator/compute/math/physical_bell.hh) -----
 * A canonical partition-local CSR, a frozen plan's feature blocks and permutation, and a
 * local row order lower to a Blocked-ELL candidate of block size 8, 16 or 32: rows in
 * execution order padded to a block multiple, features in execution order with every
 * semantic feature block padded on its own to a block multiple (membership and order are
 * never changed), one ELL slot list per block row as wide as the fullest block row. The
 * query reports all three candidates with their metrics and the safety rule's verdict
 * (value-slot expansion, storage expansion, persistent bytes); materialization re-checks
 * the candidate against the inputs and fills caller buffers. Status values are the
 * reference's bell_lowering_status_code; cx_bell_lowering_last_error() has the message. */
#define CX_BELL_LOWERING_SCHEMA_VERSION 1u
#define CX_BELL_CANDIDATE_COUNT 3u
/* bell_candidate_state */
#define CX_BELL_CANDIDATE_LEGAL 0u
#define CX_BELL_CANDIDATE_EMPTY_SOURCE 1u
#define CX_BELL_CANDIDATE_VALUE_EXPANSION_EXCEEDED 2u
#define CX_BELL_CANDIDATE_STORAGE_EXPANSION_EXCEEDED 3u
#define CX_BELL_CANDIDATE_PERSISTENT_BYTES_EXCEEDED 4u
#define CX_BELL_CANDIDATE_OVERFLOW 5u
/* bell_lowering_status_code */
#define CX_BELL_LOWERING_OK 0
#define CX_BELL_LOWERING_INVALID_ARGUMENT 1
#define CX_BELL_LOWERING_INVALID_SOURCE 2
#define CX_BELL_LOWERING_INCOMPATIBLE_PLAN 3
#define CX_BELL_LOWERING_INCOMPATIBLE_ORDER 4
#define CX_BELL_LOWERING_INSUFFICIENT_CAPACITY 5
#define CX_BELL_LOWERING_CANDIDATE_REJECTED 6
#define CX_BELL_LOWERING_CANDIDATE_MISMATCH 7
#define CX_BELL_LOWERING_OVERFLOW 8
/* value layouts of a materialized candidate */
#define CX_BELL_VALUES_BLOCK_MAJOR 0u /* the reference's: [block row][slot][row in block][column in block] */
#define CX_BELL_VALUES_ROW_MAJOR 1u   /* the engine's cx_bell_matrix: [padded row][ell column] */

/* bell_csr_source_view (physical_bell.hh:47-57): feature ids canonical and strictly
 * increasing per row; values copied byte for byte (1..16 bytes each). */
typedef struct cx_bell_csr_source {
    uint32_t row_count;
    uint32_t feature_count;
    uint32_t nnz_count;
    uint32_t value_size_bytes;
    const uint32_t *row_offsets;
    const uint32_t *feature_ids;
    const void *values;
} cx_bell_csr_source;

/* bell_semantic_plan_view (physical_bell.hh:62-72). */
typedef struct cx_bell_semantic_plan {
    uint32_t semantic_schema_version; /* 1 */
    uint32_t full_row_count;
    uint32_t feature_count;
    uint32_t feature_block_count;
    uint64_t feature_block_geometry_identity;
    uint64_t row_domain_identity;
    const uint32_t *feature_block_offsets;       /* execution order, feature_block_count + 1 */
    const uint32_t *feature_permutation;         /* execution -> canonical */
    const uint32_t *inverse_feature_permutation; /* canonical -> execution */
} cx_bell_semantic_plan;

/* The fields of local_cell_order_view (components/CellPack/include/CellPack/
 * local_cell_ordering.hh:47-67) the lowering reads. */
typedef struct cx_bell_row_order {
    uint32_t order_schema_version;        /* 1 */
    uint32_t signature_algorithm_version; /* 1 */
    uint32_t kind;
    uint32_t window_size;
    uint32_t group_width;
    uint32_t full_row_count;
    uint32_t row_count;
    uint32_t feature_block_count;
    uint64_t ordering_identity;
    uint64_t global_row_begin;
    uint64_t feature_block_geometry_identity;
    uint64_t row_domain_identity;
    const uint32_t *row_permutation;         /* execution row -> canonical row */
    const uint32_t *inverse_row_permutation; /* canonical row -> execution row */
} cx_bell_row_order;

/* bell_lowering_policy (physical_bell.hh:91-95); the reference's defaults are 64, 64 and
 * the largest size_t. */
typedef struct cx_bell_lowering_policy {
    double maximum_value_slot_expansion;
    double maximum_storage_expansion;
    uint64_t maximum_persistent_bytes;
} cx_bell_lowering_policy;

typedef struct cx_bell_candidate_metrics {
    uint64_t occupied_blocks;
    uint64_t stored_blocks;
    uint64_t dense_value_slots;
    uint64_t persistent_bytes;
    uint64_t source_bytes;
    double scalar_occupancy;
    double ell_slot_utilization;
    double value_slot_expansion;
    double storage_expansion;
} cx_bell_candidate_metrics;

/* bell_candidate_requirements (physical_bell.hh:109-124). */
typedef struct cx_bell_candidate {
    uint32_t state;
    uint32_t block_size;
    uint32_t row_count;
    uint32_t feature_count;
    uint32_t padded_row_count;
    uint32_t padded_feature_count;
    uint32_t block_row_count;
    uint32_t ell_blocks_per_row;
    uint32_t ell_columns;
    uint32_t reserved;
    uint64_t feature_block_offset_count;
    uint64_t column_index_count;
    uint64_t value_bytes;
    uint64_t candidate_identity;
    cx_bell_candidate_metrics metrics;
} cx_bell_candidate;

typedef struct cx_bell_lowering_workspace {
    uint64_t marker_capacity;
    uint32_t *markers;
    uint64_t feature_block_offset_capacity;
    uint32_t *feature_block_block_offsets;
} cx_bell_lowering_workspace;

typedef struct cx_bell_candidate_buffers {
    uint64_t feature_block_offset_capacity;
    uint32_t *padded_feature_block_offsets;
    uint64_t column_index_capacity;
    int32_t *column_indices; /* -1 = empty slot (the engine reads it as 0xffffffff) */
    uint64_t value_capacity_bytes;
    void *values;
    uint32_t value_layout;   /* CX_BELL_VALUES_* */
} cx_bell_candidate_buffers;

/* physical_bell_view (physical_bell.hh:150-168) plus the value layout. */
typedef struct cx_physical_bell_view {
    uint32_t schema_version;
    uint32_t block_size;
    uint32_t row_count;
    uint32_t feature_count;
    uint32_t padded_row_count;
    uint32_t padded_feature_count;
    uint32_t ell_columns;
    uint32_t value_size_bytes;
    uint64_t feature_block_geometry_identity;
    uint64_t ordering_identity;
    uint64_t row_domain_identity;
    uint64_t candidate_identity;
    const uint32_t *padded_feature_block_offsets;
    const int32_t *column_indices;
    const void *values;
    cx_bell_candidate_metrics metrics;
    uint32_t value_layout;
} cx_physical_bell_view;

/* query_bell_lowering_workspace_requirements (physical_bell.cc:84-96): marker_count =
 * max(rows, features), feature_block_offset_count = feature blocks + 1. Host. */
int cx_bell_lowering_workspace_requirements(const cx_bell_csr_source *source, const cx_bell_semantic_plan *plan,
                                            const cx_bell_row_order *order, uint64_t *marker_count,
                                            uint64_t *feature_block_offset_count);
/* query_bell_candidates_host (physical_bell_candidates.cc:216-238): validates every input
 * (permutations are inverses, CSR sorted and unique) and evaluates block sizes 8, 16, 32
 * into out[0..2]. NULL policy = the reference's defaults. Host. */
int cx_bell_query_candidates_host(const cx_bell_csr_source *source, const cx_bell_semantic_plan *plan,
                                  const cx_bell_row_order *order, const cx_bell_lowering_policy *policy,
                                  const cx_bell_lowering_workspace *workspace, cx_bell_candidate *out);
/* materialize_bell_candidate_host (physical_bell.cc:98-200): re-queries, rejects a
 * non-legal or stale candidate (CANDIDATE_REJECTED / CANDIDATE_MISMATCH), then writes the
 * padded block offsets, slot columns (-1 = empty) and values (zeros where not stored) in
 * buffers->value_layout. Host. */
int cx_bell_materialize_candidate_host(const cx_bell_csr_source *source, const cx_bell_semantic_plan *plan,
                                       const cx_bell_row_order *order, const cx_bell_lowering_policy *policy,
                                       const cx_bell_candidate *candidate,
                                       const cx_bell_lowering_workspace *workspace,
                                       const cx_bell_candidate_buffers *buffers, cx_physical_bell_view *out);
/* Canonical feature of every physical (padded) feature column of `view`, -1 for padding:
 * the gather map that lays a canonical weight matrix out for the engine's Blocked-ELL
 * SpMM (W_phys[p] = W[map[p]] or 0). map holds view->padded_feature_count entries. Host. */
int cx_bell_physical_feature_map(const cx_physical_bell_view *view, const cx_bell_semantic_plan *plan,
                                 int32_t *map, uint64_t capacity);
const char *cx_bell_lowering_last_error(void);

/* CP-BP warp-tile projection (components/CellPack/include/CellPack/warp_tiles.hh:41-79)
 * plus the plan subset of feature_weighted_row_reduction_plan_view
 * (components/CellPack/include/CellPack/feature_weighted_row_reduction.hh:16-26).
 * tile_row_width <= 32 uses u32 cell masks (the reference's v1 contract);
 * 32 < tile_row_width <= 64 uses u64 cell masks (the wave64 projection).
 * values are F16 (reference storage_t) or F32. */
typedef struct cx_cpbp_tiles {
    uint32_t row_count;
    uint32_t feature_count;
    uint32_t feature_block_count;
    uint32_t tile_row_width;
    uint32_t tile_count;
    uint32_t tile_block_count;
    uint32_t row_block_entry_count;
    uint32_t nnz_count;
    uint32_t value_dtype;
    uint32_t reserved;
    const uint32_t *feature_block_offsets; /* feature_block_count + 1 */
    const uint32_t *feature_permutation;   /* feature_count: execution -> canonical */
    const uint32_t *tile_block_offsets;    /* tile_count + 1 */
    const uint32_t *tile_block_ids;        /* tile_block_count */
    const void *tile_block_cell_masks;     /* tile_block_count of u32 or u64 */
    const uint32_t *block_row_entry_offsets; /* tile_block_count + 1 */
    const uint32_t *row_block_gene_masks;    /* row_block_entry_count */
    const uint32_t *row_block_value_offsets; /* row_block_entry_count + 1 */
    const void *values;                      /* nnz_count */
    const uint32_t *row_permutation;         /* row_count: execution -> canonical row */
} cx_cpbp_tiles;

/* row_values[row_permutation[exec_row]] = sum over the row's stored values of
 * fp32(value) * feature_weights[canonical feature], fp32 accumulation. Output in
 * canonical partition-local row order, as the reference kernel writes it
 * (feature_weighted_row_reduction_cuda.cu:180-218). Validates the metadata and output
 * aliasing on the host first (:57-178). */
int cx_cpbp_reduce(const cx_cpbp_tiles *tiles, const float *feature_weights,
                   uint64_t feature_weight_capacity, float *row_values,
                   uint64_t row_capacity, void *stream);

/* Per-entry rows for repeated reductions over one tile structure (engine addition, no
 * counterpart in the reference; a persistent preprocessing of the tiles, like the
 * Blocked-ELL panel). cx_cpbp_entry_rows writes, for every row-block entry, its block's
 * first permuted feature (clamped to feature_count) << 6 | its row in the tile: the entry's
 * descriptor looked up once, on the device (entry_rows: row_block_entry_count u32, device;
 * feature_count below 2^26). cx_cpbp_reduce_rows is cx_cpbp_reduce with those read per
 * entry instead of looked up per launch: same result contract, same checks; entry_rows
 * must be the array cx_cpbp_entry_rows made for these tiles (any change to the tile
 * structure, not to the values or weights, needs a new one). */
int cx_cpbp_entry_rows(const cx_cpbp_tiles *tiles, uint32_t *entry_rows, uint64_t entry_rows_capacity,
                       void *stream);
int cx_cpbp_reduce_rows(const cx_cpbp_tiles *tiles, const uint32_t *entry_rows,
                        const float *feature_weights, uint64_t feature_weight_capacity,
                        float *row_values, uint64_t row_capacity, void *stream);

/* ---- CP-BP construction (host): canonical CSR -> records -> local order -> tiles ----
 * Replaces the host producers apply_frozen_plan_host + build_cell_block_records_host +
 * build_local_cell_order_host + build_warp_tiles_host
 * (components/CellPack/include/CellPack/apply_plan.hh, cell_block_records.hh,
 *  local_cell_ordering.hh:13-67, warp_tiles.hh:131-150) for one row partition, and
 * extends the tile width to 64 rows (u64 cell masks). Runs on host threads; nothing here
 * touches the GPU. */

/* frozen_packing_plan subset (components/CellPack/include/CellPack/packing_plan.hh:39-128):
 * feature_permutation[execution] = canonical feature; blocks hold 1..32 execution
 * features. */
typedef struct cx_cpbp_plan {
    uint32_t feature_count;
    uint32_t feature_block_count;
    const uint32_t *feature_permutation;   /* feature_count */
    const uint32_t *feature_block_offsets; /* feature_block_count + 1 */
} cx_cpbp_plan;

/* plan_application_source_view subset (apply_plan.hh): canonical rows, canonical feature
 * ids strictly increasing per row, values of value_size_bytes (2 = f16, 4 = f32). */
typedef struct cx_cpbp_csr {
    uint32_t rows;
    uint32_t value_size_bytes;
    const uint32_t *row_offsets;        /* rows + 1 */
    const uint32_t *canonical_features; /* row_offsets[rows] */
    const void *values;                 /* row_offsets[rows] */
} cx_cpbp_csr;

/* local_cell_order_kind (local_cell_ordering.hh:15-20) */
#define CX_CPBP_ORDER_INFERRED_MINHASH 1u
#define CX_CPBP_ORDER_ORIGINAL 2u
#define CX_CPBP_ORDER_DETERMINISTIC_RANDOM 3u
#define CX_CPBP_ORDER_ROW_NNZ_DESCENDING 4u

/* local_cell_order_config (local_cell_ordering.hh:22-27) plus the partition's global
 * row begin used by the deterministic_random keys. group_width is the tile width. */
typedef struct cx_cpbp_order_config {
    uint32_t kind;
    uint32_t window_size; /* reference default 1024 */
    uint32_t group_width; /* 1..64; window_size % group_width == 0 */
    uint32_t reserved;
    uint64_t seed;        /* reference default 0x6a09e667f3bcc909 */
    uint64_t global_row_begin;
} cx_cpbp_order_config;

/* Exact output sizes (warp_tile_requirements, warp_tiles.hh:15-22, in elements). */
typedef struct cx_cpbp_tile_requirements {
    uint32_t row_count;
    uint32_t feature_count;
    uint32_t feature_block_count;
    uint32_t tile_row_width;
    uint32_t tile_count;            /* tile_block_offsets holds tile_count + 1 */
    uint32_t tile_block_count;      /* block_row_entry_offsets holds this + 1 */
    uint32_t row_block_entry_count; /* row_block_value_offsets holds this + 1 */
    uint32_t nnz_count;
    uint32_t value_size_bytes;
    uint32_t cell_mask_bytes;       /* 4 (width <= 32) or 8 */
} cx_cpbp_tile_requirements;

/* Caller-owned host outputs (warp_tile_buffers, warp_tiles.hh:24-38, plus the order). */
typedef struct cx_cpbp_tile_buffers {
    uint32_t *tile_block_offsets;
    uint32_t *tile_block_ids;
    void *tile_block_cell_masks; /* u32 or u64 per cell_mask_bytes */
    uint32_t *block_row_entry_offsets;
    uint32_t *row_block_gene_masks;
    uint32_t *row_block_value_offsets;
    void *values;
    uint32_t *row_permutation;   /* execution row -> canonical partition-local row */
    uint64_t *primary_keys;      /* optional: local-order primary key per canonical row */
} cx_cpbp_tile_buffers;

typedef struct cx_cpbp_builder cx_cpbp_builder;

/* Validates and builds everything on `threads` host threads (0 -> 1); the result is
 * identical for every thread count. Errors: CX_STATUS_*, message in
 * cx_cpbp_build_last_error(). */
int cx_cpbp_builder_create(const cx_cpbp_plan *plan, const cx_cpbp_csr *csr,
                           const cx_cpbp_order_config *config, uint32_t threads,
                           cx_cpbp_builder **out);
int cx_cpbp_builder_requirements(const cx_cpbp_builder *builder, cx_cpbp_tile_requirements *out);
int cx_cpbp_builder_export(const cx_cpbp_builder *builder, const cx_cpbp_tile_buffers *buffers);
void cx_cpbp_builder_destroy(cx_cpbp_builder *builder);
const char *cx_cpbp_build_last_error(void);

/* Device construction of the same projection: plan and CSR arrays (cx_cpbp_plan,
 * cx_cpbp_csr) are DEVICE pointers; the result is bit-identical to cx_cpbp_builder_create's
 * for the same inputs and config. Replaces the reference's CUDA producers
 * (components/CellPack/include/CellPack/{apply_plan,cell_block_records_cuda,
 * local_cell_ordering_cuda,warp_tiles_cuda}.hh: apply_frozen_plan_cuda,
 * build_cell_block_records_cuda, build_local_cell_order_cuda, build_warp_tiles_cuda) with the
 * engine's radix sort and scans. create validates on the device, enqueues the construction on
 * `stream` and synchronizes it (twice, to size the intermediates, which it allocates);
 * export fills caller-allocated DEVICE buffers (sizes from requirements) on `stream`
 * without synchronizing. A one-time preprocessing step, not a launch-path call. */
typedef struct cx_cpbp_device_builder cx_cpbp_device_builder;
int cx_cpbp_device_builder_create(const cx_cpbp_plan *device_plan, const cx_cpbp_csr *device_csr,
                                  const cx_cpbp_order_config *config, void *stream,
                                  cx_cpbp_device_builder **out);
int cx_cpbp_device_builder_requirements(const cx_cpbp_device_builder *builder,
                                        cx_cpbp_tile_requirements *out);
int cx_cpbp_device_builder_export(const cx_cpbp_device_builder *builder,
                                  const cx_cpbp_tile_buffers *device_buffers, void *stream);
void cx_cpbp_device_builder_destroy(cx_cpbp_device_builder *builder);
const char *cx_cpbp_device_build_last_error(void);

/* ---- CPK1 persistent packing payload --------------------------------------------
 * The reference's pointer-free image of one packed partition
 * (components/CellPack/include/CellPack/persistent_packing_payload.hh:9-96,
 * components/CellPack/src/persistent_packing_payload.cc): a 352-byte header and fifteen
 * 64-byte-aligned sections. CPK1 v1 holds u32 cell masks (tile widths 1..32) and f16
 * values. Load = validate on the host, upload the bytes in one copy, rebind the view to
 * the device copy, and pass view.tiles to cx_cpbp_reduce. */

/* persistent_packing_payload_compatibility (persistent_packing_payload.hh:23-31) */
typedef struct cx_cpk1_expected {
    uint64_t global_row_begin;
    uint32_t row_count;
    uint32_t feature_count;
    uint32_t reserved0;
    uint64_t feature_axis_fingerprint;
    uint32_t feature_axis_fingerprint_version;
    uint32_t reserved1;
    uint64_t row_domain_identity;
    uint64_t payload_identity;
} cx_cpk1_expected;

/* persistent_packing_payload_view (persistent_packing_payload.hh:35-56), with the tile
 * arrays as a cx_cpbp_tiles (value_dtype F16, u32 cell masks). Pointers point into the
 * image: host after validate, device after rebind. */
typedef struct cx_cpk1_view {
    uint64_t payload_identity;
    const void *image_base;
    uint64_t image_bytes;
    uint64_t global_row_begin;
    uint32_t full_row_count;
    uint32_t row_group_count;
    uint32_t row_group_width;
    uint32_t maximum_feature_block_width;
    uint64_t feature_axis_fingerprint;
    uint32_t feature_axis_fingerprint_version;
    uint32_t row_domain_kind;
    uint64_t row_domain_identity;
    uint64_t feature_block_geometry_identity;
    uint64_t ordering_identity;
    uint64_t tile_identity;
    cx_cpbp_order_config order;
    const uint32_t *inverse_feature_permutation;
    const uint32_t *feature_to_block;
    const uint32_t *feature_to_local;
    const uint32_t *row_group_offsets;
    const uint32_t *inverse_row_permutation;
    cx_cpbp_tiles tiles;
} cx_cpk1_view;

/* What the image records about the plan, its row domain and the local order, beyond the
 * tiles themselves (the frozen packing plan identity and local_cell_order_config the
 * reference's writer reads, build_persistent_packing_payload_host,
 * persistent_packing_payload.cc:483-571). row_group_offsets NULL = uniform groups of
 * row_group_width over full_row_count; maximum_feature_block_width 0 = the widest block. */
typedef struct cx_cpk1_metadata {
    uint64_t feature_axis_fingerprint;
    uint32_t feature_axis_fingerprint_version;
    uint32_t row_domain_kind;          /* 1 full dataset, 2 sampled rows */
    uint64_t row_domain_identity;
    uint64_t evaluation_source_identity;
    uint64_t sampling_provenance_identity;
    uint64_t cost_policy_identity;
    uint32_t objective_kind;           /* 1 total bytes, 2 row-active block references, 3 weighted */
    uint32_t full_row_count;
    uint32_t maximum_feature_block_width;
    uint32_t row_group_width;
    uint32_t row_group_count;
    uint32_t reserved;
    const uint32_t *row_group_offsets; /* row_group_count + 1, or NULL */
    uint64_t global_row_begin;
    cx_cpbp_order_config order;        /* kind, window_size, group_width (= tile width), seed */
} cx_cpk1_metadata;

/* Image bytes for tiles of `req` with row_group_count row groups. */
int cx_cpk1_image_bytes(const cx_cpbp_tile_requirements *req, uint32_t row_group_count,
                        uint64_t *bytes);
/* Writes the image of HOST plan and tile arrays (cx_cpbp_builder_export's layout) into
 * `image` (host, capacity bytes), computes the geometry, ordering, tile and payload
 * identities, then validates it into `out` (build_persistent_packing_payload_host). */
int cx_cpk1_write(const cx_cpbp_plan *plan, const cx_cpk1_metadata *meta,
                  const cx_cpbp_tile_requirements *req, const cx_cpbp_tile_buffers *tiles,
                  void *image, uint64_t capacity, cx_cpk1_view *out);
/* validate_persistent_packing_payload_host: header, identity (FNV-1a over the image),
 * layout, the caller's expected identity, plan and tile arrays. HOST image. */
int cx_cpk1_validate(const void *image, uint64_t image_bytes, const cx_cpk1_expected *expected,
                     cx_cpk1_view *out);
/* rebind_persistent_packing_payload: the view of an equal-sized copy at new_base (e.g. a
 * device upload); no copy, allocation or dereference of new_base. */
int cx_cpk1_rebind(const cx_cpk1_view *validated, const void *new_base, uint64_t new_bytes,
                   cx_cpk1_view *out);
const char *cx_cpk1_last_error(void);

/* ---- CPE2 execution image (components/CellPack/include/CellPack/persistence/
 * execution_image_v2.hh, EXECUTION_IMAGE_V2.md) ---------------------------------------------
 * Pointer-free container of one relation / semantic geometry and a directory of projections
 * of it; the byte format, checks and messages are the reference's. Host build and validate;
 * rebind and prebind only form addresses (a device destination is never touched). */
#define CX_CPE2_SCHEMA_VERSION 2u
#define CX_CPE2_PAYLOAD_KIND 0x43504532u /* "CPE2" */
#define CX_CPE2_ALIGNMENT 64u
#define CX_CPE2_ENDIAN_MARKER 0x01020304u
#define CX_CPE2_INVALID_INDEX 0xffffffffu
/* execution_section_kind */
#define CX_CPE2_SECTION_DOMAIN_TABLE 1u
#define CX_CPE2_SECTION_ORDER_PARTITION_TABLE 2u
#define CX_CPE2_SECTION_RELATION_STRUCTURE 3u
#define CX_CPE2_SECTION_SEMANTIC_GEOMETRY 4u
#define CX_CPE2_SECTION_INITIAL_VALUES 5u
#define CX_CPE2_SECTION_PROJECTION_PAYLOAD 6u
#define CX_CPE2_SECTION_FORWARD_VALUE_MAP 7u
#define CX_CPE2_SECTION_TRANSPOSE_VALUE_MAP 8u
#define CX_CPE2_SECTION_HIERARCHY_PARTITION_INDEX 9u
#define CX_CPE2_SECTION_SCHEDULING_SUMMARY 10u
#define CX_CPE2_SECTION_CPK1_V1_COMPATIBILITY 11u
/* execution_projection_kind */
#define CX_CPE2_PROJECTION_NATIVE_ROW_MASKED 1u
#define CX_CPE2_PROJECTION_CSR 5u
#define CX_CPE2_PROJECTION_BLOCKED_ELL 8u
#define CX_CPE2_PROJECTION_ARCHITECTURE_SPECIFIC 11u
/* execution_directory_flags */
#define CX_CPE2_DIRECTORY_OPTIONAL 1u
#define CX_CPE2_DIRECTORY_DEVICE_READABLE 2u
#define CX_CPE2_PROJECTION_LAZY_CONSTRUCTIBLE 4u
#define CX_CPE2_PROJECTION_FORWARD_CAPABLE 8u
#define CX_CPE2_PROJECTION_TRANSPOSE_CAPABLE 16u

typedef struct cx_cpe2_id {
    uint64_t low, high;
} cx_cpe2_id;

typedef struct cx_cpe2_axis_record {  /* execution_axis_record_v1 */
    uint64_t domain_low, domain_high, order_low, order_high;
    uint64_t geometry_low, geometry_high, partition_low, partition_high;
} cx_cpe2_axis_record;

typedef struct cx_cpe2_axis_identity {  /* persistent_axis_identity (execution/identity.hh:94-100) */
    uint16_t schema_version;            /* 1 */
    uint16_t record_kind;               /* 1 */
    uint32_t byte_count;                /* 72 */
    cx_cpe2_id domain, order, geometry, partition;
} cx_cpe2_axis_identity;

typedef struct cx_cpe2_header {  /* execution_image_v2_header, 256 bytes */
    unsigned char magic[8];      /* "CELLEX02" */
    uint32_t schema_version;
    uint32_t header_bytes;
    uint32_t endian;
    uint32_t alignment;
    uint64_t image_bytes;
    uint64_t image_identity;
    uint64_t structure_identity_low, structure_identity_high;
    uint64_t structure_epoch;
    uint64_t semantic_geometry_identity_low, semantic_geometry_identity_high;
    uint64_t projection_catalog_identity_low, projection_catalog_identity_high;
    uint64_t initial_value_generation;
    cx_cpe2_axis_record source_axis;
    cx_cpe2_axis_record destination_axis;
    uint32_t section_count;
    uint32_t projection_count;
    uint64_t section_directory_offset;
    uint64_t projection_directory_offset;
} cx_cpe2_header;

typedef struct cx_cpe2_section_entry {  /* execution_section_entry_v1, 64 bytes */
    uint32_t kind, schema_version, flags, alignment;
    uint64_t identity_low, identity_high;
    uint64_t offset, bytes, checksum;
    uint32_t element_count, element_bytes;
} cx_cpe2_section_entry;

typedef struct cx_cpe2_projection_entry {  /* execution_projection_entry_v1, 64 bytes */
    uint64_t identity_low, identity_high;
    uint32_t kind, schema_version, flags, operation_family;
    uint16_t storage_type, compute_type, accumulation_type, orientation;
    uint32_t architecture_class;
    uint32_t payload_section, forward_map_section, transpose_map_section;
    uint32_t scheduling_summary_section, capability_section;
} cx_cpe2_projection_entry;

typedef struct cx_cpe2_section_source {
    uint32_t kind, schema_version, flags, alignment;
    uint64_t identity_low, identity_high;
    const void *data;
    uint64_t bytes;
    uint32_t element_count, element_bytes;
} cx_cpe2_section_source;

typedef struct cx_cpe2_build_request {
    cx_cpe2_id structure_identity;
    uint64_t structure_epoch;
    cx_cpe2_id semantic_geometry_identity;
    cx_cpe2_id projection_catalog_identity;
    uint64_t initial_value_generation;
    cx_cpe2_axis_identity source_axis;
    cx_cpe2_axis_identity destination_axis;
    const cx_cpe2_section_source *sections;
    uint32_t section_count, reserved;
    const cx_cpe2_projection_entry *projections;
    uint32_t projection_count, reserved2;
} cx_cpe2_build_request;

typedef struct cx_cpe2_requirements {
    uint64_t image_bytes, directory_bytes, section_bytes, alignment_padding_bytes;
} cx_cpe2_requirements;

typedef struct cx_cpe2_expected {
    cx_cpe2_id structure_identity;
    uint64_t structure_epoch;
    cx_cpe2_id semantic_geometry_identity;
    cx_cpe2_id projection_catalog_identity;
    uint64_t image_identity;  /* 0 = any */
} cx_cpe2_expected;

typedef struct cx_cpe2_view {
    cx_cpe2_header header;
    const void *image_base;
    uint64_t image_bytes;
    const cx_cpe2_section_entry *sections;
    const cx_cpe2_projection_entry *projections;
} cx_cpe2_view;

typedef struct cx_cpe2_prebound_projection {  /* prebound_projection_view_v1 */
    cx_cpe2_projection_entry descriptor;
    const void *payload;
    uint64_t payload_bytes;
    const void *forward_map;
    uint64_t forward_map_bytes;
    const void *transpose_map;
    uint64_t transpose_map_bytes;
    const void *scheduling_summary;
    uint64_t scheduling_summary_bytes;
} cx_cpe2_prebound_projection;

/* query_execution_image_v2_requirements_host (execution_image_v2.cc:288-300) */
int cx_cpe2_query_requirements(const cx_cpe2_build_request *request, cx_cpe2_requirements *out);
/* build_execution_image_v2_host (:302-377): writes and then validates the image. */
int cx_cpe2_build(const cx_cpe2_build_request *request, void *image, uint64_t capacity, cx_cpe2_view *out);
/* validate_execution_image_v2_host (:379-518). */
int cx_cpe2_validate(const void *image, uint64_t image_bytes, const cx_cpe2_expected *expected, cx_cpe2_view *out);
/* rebind_execution_image_v2 (:520-541): directory pointers of an equal-sized copy. */
int cx_cpe2_rebind(const cx_cpe2_view *validated, const void *new_base, uint64_t new_bytes, cx_cpe2_view *out);
/* prebind_execution_projection_host / _for_base_host (:543-591): hot pointers = base +
 * validated section offset; no dereference of destination_base. */
int cx_cpe2_prebind(const cx_cpe2_view *validated_host, uint32_t projection_index, cx_cpe2_prebound_projection *out);
int cx_cpe2_prebind_for_base(const cx_cpe2_view *validated_host, uint32_t projection_index,
                             const void *destination_base, uint64_t destination_bytes,
                             cx_cpe2_prebound_projection *out);
/* load_cpk1_v1_compatibility_host (execution_image_v2_cpk1.cc:5-31): the CPK1 section of a
 * native row-masked projection through the CPK1 validator, unconverted. */
int cx_cpe2_load_cpk1(const cx_cpe2_view *validated_host, uint32_t projection_index,
                      const cx_cpk1_expected *expected, cx_cpk1_view *out);
const char *cx_cpe2_last_error(void);

/* ---- CP-BP reduction under the reference's full direct-consumer contract ----------------
 * feature_weighted_row_reduction_view (components/CellPack/include/CellPack/
 * feature_weighted_row_reduction.hh:20-44) with the warp_tile_view identity fields
 * (warp_tiles.hh:49-79) and the local_cell_order_view fields the reduction checks
 * (local_cell_ordering.hh:47-67), around the engine's cx_cpbp_tiles. */
typedef struct cx_cpbp_reduction_view {
    uint32_t schema_version;               /* 1 */
    uint32_t storage_type_code;            /* cellerator real code of the values: f16 3, f32 4 */
    uint32_t weight_type_code;             /* f32 4 */
    uint32_t accumulation_type_code;       /* f32 4 */
    uint64_t feature_weight_identity;      /* the caller's weight generation, nonzero */
    uint64_t reduction_identity;           /* cx_cpbp_reduction_identity of this view */
    /* plan (feature_weighted_row_reduction_plan_view) */
    uint32_t plan_schema_version;          /* 1 */
    uint32_t plan_geometry_identity_version; /* 1 */
    uint32_t plan_feature_count;
    uint32_t plan_feature_block_count;
    uint64_t plan_geometry_identity;
    /* tiles (warp_tile_view identities) */
    uint32_t tile_schema_version;          /* 1 */
    uint32_t tiles_plan_schema_version;    /* 1 */
    uint32_t tiles_geometry_identity_version; /* 1 */
    uint32_t feature_axis_fingerprint_version;
    uint64_t tile_identity;
    uint64_t tiles_geometry_identity;
    uint64_t tiles_ordering_identity;
    uint64_t tiles_global_row_begin;
    uint64_t feature_axis_fingerprint;
    uint64_t tiles_row_domain_identity;
    uint32_t tiles_full_row_count;
    /* local order */
    uint32_t order_schema_version;         /* 1 */
    uint32_t order_signature_version;      /* 1 */
    uint32_t order_full_row_count;
    uint32_t order_row_count;
    uint32_t order_feature_block_count;
    uint32_t order_group_width;
    uint32_t reserved;
    uint64_t order_ordering_identity;
    uint64_t order_global_row_begin;
    uint64_t order_geometry_identity;
    uint64_t order_row_domain_identity;
    cx_cpbp_tiles tiles;
} cx_cpbp_reduction_view;

/* reduction_identity (components/CellPack/src/feature_weighted_row_reduction_cuda.cu:44-55). */
uint64_t cx_cpbp_reduction_identity(const cx_cpbp_reduction_view *view);
/* The view of a validated (or rebound) CPK1 image and a weight generation: every identity
 * and domain field from the image, reduction_identity computed. */
int cx_cpbp_reduction_view_from_cpk1(const cx_cpk1_view *image, uint64_t feature_weight_identity,
                                     cx_cpbp_reduction_view *out);
/* validate_metadata (feature_weighted_row_reduction_cuda.cu:57-136) then cx_cpbp_reduce:
 * UNSUPPORTED for a version, INVALID_ARGUMENT for the numeric contract or an identity
 * (including a reduction identity that is not the recomputed one), INVALID_SHAPE when plan,
 * order and tiles disagree on their domain. */
int cx_cpbp_reduce_checked(const cx_cpbp_reduction_view *view, const float *feature_weights,
                           uint64_t feature_weight_capacity, float *row_values, uint64_t row_capacity,
                           void *stream);
/* The checks of cx_cpbp_reduce_checked alone (host only, same statuses), for callers that
 * validate a view once and launch cx_cpbp_reduce on its tiles many times. */
int cx_cpbp_reduction_validate(const cx_cpbp_reduction_view *view);

/* ---- native tile view: the reference's math projection of a CP-BP partition ----------------
 * Layout-identical mirrors of cellpack::feature_weighted_row_reduction_plan_view
 * (components/CellPack/include/CellPack/feature_weighted_row_reduction.hh:19-27, 40 bytes),
 * cellpack::local_cell_order_view (local_cell_ordering.hh:47-67, 128 bytes),
 * cellpack::warp_tile_view (warp_tiles.hh:49-79, 176 bytes) and
 * cellerator::compute::math::native_tile_view with its sidecars
 * (include/Cellerator/compute/math/native_tile_view.hh:17-64; view 384 bytes, block metrics
 * 32 bytes), so a view the reference's own adapter built can be passed by pointer. The
 * reserved fields name the padding the C++ layout has there. v1 tiles: u32 cell masks,
 * tile_row_width <= 32. */
typedef struct cx_fwr_plan_view {
    uint32_t semantic_plan_schema_version;
    uint32_t geometry_identity_version;
    uint32_t feature_count;
    uint32_t feature_block_count;
    uint64_t feature_block_geometry_identity;
    const uint32_t *feature_block_offsets;
    const uint32_t *feature_permutation;
} cx_fwr_plan_view;
typedef struct cx_local_cell_order_view {
    uint32_t order_schema_version;
    uint32_t signature_algorithm_version;
    uint32_t kind;
    uint32_t window_size;
    uint32_t group_width;
    uint32_t reserved0;
    uint64_t seed;
    uint64_t ordering_identity;
    uint64_t global_row_begin;
    uint32_t full_row_count;
    uint32_t row_count;
    uint32_t feature_block_count;
    uint32_t reserved1;
    uint64_t feature_block_geometry_identity;
    uint64_t row_domain_identity;
    const uint64_t *primary_keys;
    const uint32_t *secondary_keys;
    const uint32_t *active_block_counts;
    const uint32_t *row_nnz_counts;
    const uint32_t *row_permutation;
    const uint32_t *inverse_row_permutation;
} cx_local_cell_order_view;
typedef struct cx_warp_tile_view {
    uint32_t tile_schema_version;
    uint32_t record_schema_version;
    uint32_t semantic_plan_schema_version;
    uint32_t geometry_identity_version;
    uint32_t order_schema_version;
    uint32_t reserved0;
    uint64_t tile_identity;
    uint64_t feature_block_geometry_identity;
    uint64_t ordering_identity;
    uint64_t global_row_begin;
    uint32_t full_row_count;
    uint32_t row_count;
    uint32_t feature_count;
    uint32_t feature_block_count;
    uint32_t tile_row_width;
    uint32_t tile_count;
    uint32_t nnz_count;
    uint32_t tile_block_count;
    uint32_t row_block_entry_count;
    uint32_t value_size_bytes;
    uint64_t feature_axis_fingerprint;
    uint32_t feature_axis_fingerprint_version;
    uint32_t reserved1;
    uint64_t row_domain_identity;
    const uint32_t *tile_block_offsets;
    const uint32_t *tile_block_ids;
    const uint32_t *tile_block_cell_masks;
    const uint32_t *block_row_entry_offsets;
    const uint32_t *row_block_gene_masks;
    const uint32_t *row_block_value_offsets;
    const void *values;
} cx_warp_tile_view;
/* native_tile_block_metrics / _requirements / _buffers (native_tile_view.hh:17-41). */
typedef struct cx_native_tile_block_metrics {
    uint32_t active_rows;
    uint32_t active_features;
    uint32_t nnz;
    uint32_t dense_workload;
    double density;
    double feature_reuse;
} cx_native_tile_block_metrics;
typedef struct cx_native_tile_requirements {
    uint64_t union_mask_count;
    uint64_t packed_offset_count;
    uint64_t block_metric_count;
    uint64_t sidecar_bytes;
} cx_native_tile_requirements;
typedef struct cx_native_tile_buffers {
    uint64_t union_mask_capacity;
    uint32_t *union_gene_masks;
    uint64_t packed_offset_capacity;
    uint32_t *packed_value_offsets;
    uint64_t block_metric_capacity;
    cx_native_tile_block_metrics *block_metrics;
} cx_native_tile_buffers;
#define CX_NATIVE_TILE_VIEW_SCHEMA 1u
typedef struct cx_native_tile_view {
    uint32_t schema_version;  /* CX_NATIVE_TILE_VIEW_SCHEMA */
    uint32_t reserved;
    cx_fwr_plan_view plan;
    cx_local_cell_order_view order;
    cx_warp_tile_view tiles;
    const uint32_t *union_gene_masks;
    const uint32_t *packed_value_offsets;
    const cx_native_tile_block_metrics *block_metrics;
    uint64_t dense_workload;
} cx_native_tile_view;
/* native_tile_decoded_value (native_tile_view.hh:66-76). */
typedef struct cx_native_tile_decoded_value {
    uint32_t value_index;
    uint32_t execution_row;
    uint32_t canonical_row;
    uint32_t reserved0;
    uint64_t global_row;
    uint32_t execution_feature;
    uint32_t canonical_feature;
    const void *value;
} cx_native_tile_decoded_value;
/* query_native_tile_requirements_host / build_native_tile_view_host /
 * decode_native_tile_value_host and their CPK1 forms (native_tile_view.hh:78-136,
 * src/compute/math/native_tile_view.cc): host only; the view aliases plan, order, tiles and
 * values, only the sidecars are new. Statuses: INVALID_ARGUMENT (invalid argument,
 * incompatible identity, small sidecars), INVALID_SHAPE (invalid geometry, overflow); the
 * message is the reference's. The CPK1 forms take the engine's view of a validated (or
 * rebound) image and fill plan, order and tiles from it. */
int cx_query_native_tile_requirements_host(const cx_fwr_plan_view *plan, const cx_local_cell_order_view *order,
                                           const cx_warp_tile_view *tiles, cx_native_tile_requirements *out);
int cx_build_native_tile_view_host(const cx_fwr_plan_view *plan, const cx_local_cell_order_view *order,
                                   const cx_warp_tile_view *tiles, const cx_native_tile_buffers *buffers,
                                   cx_native_tile_view *out);
int cx_query_native_tile_requirements_from_cpk1_host(const cx_cpk1_view *payload, cx_native_tile_requirements *out);
int cx_build_native_tile_view_from_cpk1_host(const cx_cpk1_view *payload, const cx_native_tile_buffers *buffers,
                                             cx_native_tile_view *out);
int cx_decode_native_tile_value_host(const cx_native_tile_view *view, uint32_t value_index,
                                     cx_native_tile_decoded_value *out);
/* The engine's tile operand of a native view (for cx_cpbp_reduce): plan arrays, tiles,
 * row permutation; value_dtype from value_size_bytes (2: F16, 4: F32). Host, no checks
 * beyond the schema and the value size. */
int cx_cpbp_tiles_from_native_view(const cx_native_tile_view *view, cx_cpbp_tiles *out);
/* A view built on a validated host CPK1 image moved to an equal copy of the image (its
 * device upload): plan, order and tile pointers inside [old_base, old_base + bytes) move by
 * new_base - old_base (rebind_persistent_packing_payload's rule, persistent_packing_payload.hh:
 * 81-86); sidecars and pointers outside the image stay. */
int cx_native_tile_view_rebind(const cx_native_tile_view *view, const void *old_base, uint64_t bytes,
                               const void *new_base, cx_native_tile_view *out);

/* ---- execution feature order: packed dense operand and execution-order CSR ---------------
 * feature_permutation[e] = the canonical gene at execution position e (cx_cpbp_plan's
 * convention). X . W does not change when the genes of X and the rows of W are relabelled
 * together, so a projection can run on (X_exec, W_exec). Identities follow the reference's
 * FNV-1a rules, including its offset basis. */

/* feature_order_identity (include/Cellerator/compute/math/operation.hh:63-96) */
#define CX_FEATURE_ORDER_CANONICAL 1u
#define CX_FEATURE_ORDER_PACKED 2u
typedef struct cx_feature_order {
    uint32_t schema_version; /* 1 */
    uint32_t kind;           /* CX_FEATURE_ORDER_* */
    uint32_t feature_count;
    uint32_t feature_axis_identity_version;
    uint64_t feature_axis_identity;
    uint64_t packing_geometry_identity; /* 0 for the canonical order */
} cx_feature_order;

/* canonical_dense_operand_view / packed_dense_operand_view
 * (include/Cellerator/compute/math/packed_dense_operand.hh:16-38): a feature-major dense
 * operand; column_major 0 = row-major [features x columns] with leading_dimension >= columns,
 * 1 = column-major with leading_dimension >= features. */
typedef struct cx_dense_operand {
    const void *values;
    uint32_t feature_count;
    uint32_t value_size_bytes; /* 2, 4 or 8 */
    uint64_t column_count;
    uint64_t leading_dimension;
    uint32_t column_major;
    uint32_t reserved;
    cx_feature_order feature_order;
    uint64_t operand_identity;
} cx_dense_operand;

/* query_packed_dense_operand_requirements (packed_dense_operand.cu:163-175): validates the
 * canonical operand against the plan (whose geometry identity is geometry_identity) and
 * describes the packed result (row-major [features x columns], packed feature order, its
 * identity) without values; *value_bytes = the packed size. */
int cx_packed_dense_operand_describe(const cx_cpbp_plan *plan, uint64_t geometry_identity,
                                     const cx_dense_operand *canonical, cx_dense_operand *packed,
                                     uint64_t *value_bytes);
/* pack_dense_operand_host (packed_dense_operand.cu:177-215): packed row e = canonical feature
 * plan->feature_permutation[e]. Host plan and buffers. */
int cx_pack_dense_operand_host(const cx_cpbp_plan *plan, uint64_t geometry_identity,
                               const cx_dense_operand *canonical, void *packed, uint64_t capacity_bytes,
                               cx_dense_operand *out);
/* pack_dense_operand_cuda (packed_dense_operand.cu:217-260): the same on the device (device
 * permutation and values; the block offsets are not read). Enqueues on `stream`, one pass. */
int cx_pack_dense_operand_device(const cx_cpbp_plan *device_plan, uint64_t geometry_identity,
                                 const cx_dense_operand *canonical, void *packed, uint64_t capacity_bytes,
                                 void *stream, cx_dense_operand *out);
/* The raw device gather behind it: packed[e][c] = canonical[perm[e]][c] (row-major source) or
 * canonical[c][perm[e]] (column-major), value_size_bytes 1, 2, 4 or 8. Also permutes per-gene
 * metadata (columns = 1; 8-byte values for interleaved scale/offset pairs). */
int cx_pack_dense_operand(const uint32_t *feature_permutation, uint32_t feature_count,
                          const void *canonical, uint64_t column_count, uint64_t leading_dimension,
                          uint32_t column_major, uint32_t value_size_bytes, void *packed,
                          uint64_t packed_capacity_bytes, void *stream);

/* ordered_plan_partition_view subset (components/CellPack/include/CellPack/apply_plan.hh):
 * rows in canonical order, entries per row in execution order as (block, local) plus the
 * canonical feature id they stand for. */
typedef struct cx_ordered_partition {
    uint64_t global_row_begin;
    uint32_t full_row_count;
    uint32_t row_count;
    uint32_t feature_count;
    uint32_t nnz_count;
    uint32_t value_size_bytes;
    uint32_t feature_axis_fingerprint_version;
    uint64_t feature_axis_fingerprint;
    uint64_t row_domain_identity;
    const uint32_t *row_offsets;        /* row_count + 1 */
    const uint32_t *block_ids;          /* nnz_count */
    const uint32_t *local_feature_ids;  /* nnz_count */
    const uint32_t *canonical_feature_ids; /* nnz_count */
    const void *values;                 /* nnz_count x value_size_bytes */
} cx_ordered_partition;

/* execution_csr_view (include/Cellerator/compute/math/physical_csr.hh:40-56): a row-compressed
 * view in frozen execution-feature order with its FNV structure identity (:92-110). */
typedef struct cx_execution_csr {
    uint64_t global_row_begin;
    uint32_t full_row_count;
    uint32_t row_count;
    uint32_t feature_count;
    uint32_t nnz_count;
    uint32_t value_size_bytes;
    uint32_t reserved;
    uint64_t row_domain_identity;
    uint64_t structure_identity; /* sparse_structure_identity.value, identity version 1 */
    cx_feature_order feature_order;
    const uint32_t *row_offsets;
    const uint32_t *execution_feature_ids;
    const void *values;
} cx_execution_csr;

/* build_execution_csr_view_host (src/compute/math/physical_csr.cc:16-97): maps every entry to
 * its execution feature (block offset + local id), checks it stands for the recorded canonical
 * feature and that each row is strictly increasing in execution order; aliases the partition's
 * row offsets and values, writes execution_feature_ids (capacity >= nnz). */
int cx_build_execution_csr_host(const cx_cpbp_plan *plan, uint64_t geometry_identity,
                                const cx_ordered_partition *ordered, uint32_t *execution_feature_ids,
                                uint64_t capacity, cx_execution_csr *out);

/* lazy_execution_csr_requirements / _buffers (physical_csr.hh:58-77, :180-207), in elements
 * and bytes. */
typedef struct cx_lazy_csr_requirements {
    uint64_t row_offset_count;
    uint64_t execution_feature_count;
    uint64_t value_bytes;
    uint64_t row_cursor_count;
    uint64_t total_bytes;
} cx_lazy_csr_requirements;
typedef struct cx_lazy_csr_buffers {
    uint64_t row_offset_capacity;
    uint64_t execution_feature_capacity;
    uint64_t value_capacity_bytes;
    uint64_t row_cursor_capacity;
    uint32_t *row_offsets;
    uint32_t *execution_feature_ids;
    void *values;
    uint32_t *row_cursors;
} cx_lazy_csr_buffers;
int cx_lazy_execution_csr_requirements(const cx_cpk1_view *payload, cx_lazy_csr_requirements *out);
/* materialize_execution_csr_from_cpk1_host (physical_csr.cc:99-240): rebuilds the CSR of a
 * validated HOST CPK1 view (tiles of any width up to 64) into caller-owned buffers, rows in
 * tile order, entries in execution order; the image is not modified. */
int cx_materialize_execution_csr_from_cpk1_host(const cx_cpk1_view *payload, const cx_lazy_csr_buffers *buffers,
                                                cx_execution_csr *out);

/* Per-gene stored-entry counts of `a` (device, cols u32; columns outside [0, cols) are not
 * counted), and the popularity order of such counts (host): genes by descending count, ties by
 * gene index -- an execution order that puts the most frequently stored genes first. Engine
 * additions: the reference takes its orders from a frozen packing plan. */
int cx_qcsr_column_counts(const cx_qcsr_matrix *a, uint32_t *counts, void *stream);
int cx_popularity_order(const uint32_t *counts, uint32_t genes, uint32_t *feature_permutation,
                        uint32_t *inverse_permutation);

/* The quantized (or plain) CSR `a` relabelled into execution order on the device: entry
 * (row, g) becomes (row, inverse_permutation[g]) and every row is re-sorted by the new label
 * with its code (or value) carried along. row_ptr and packed_row_ptr are unchanged (the
 * outputs reuse them); col_idx_out [nnz] and packed_out [packed bytes] (or values_out [nnz]
 * for bits == 0) must not alias the inputs. Rows need not be sorted on input, but a gene may
 * occur once per row: a repeated gene or a column outside [0, cols) sets *device_error to
 * nonzero (outputs undefined). Per-gene metadata is permuted with cx_pack_dense_operand.
 * The execution-order CSR of build_execution_csr_view_host, produced on the device for a
 * quantized matrix. */
int cx_qcsr_to_execution_order(const cx_qcsr_matrix *a, const uint32_t *inverse_permutation,
                               int32_t *col_idx_out, uint8_t *packed_out, void *values_out,
                               uint32_t *device_error, void *stream);
int cx_qcsr_execution_order_lds_bytes(const cx_qcsr_matrix *a, uint64_t *bytes);
const char *cx_exec_last_error(void);

/* ---- execution-order quantized CSR SpMM with a dense head on the matrix cores -----------
 * For a matrix in an execution order whose first head_cols genes are the most frequently
 * stored ones (cx_popularity_order + cx_qcsr_to_execution_order), the product splits into
 * Y = X[:, 0:H) . W[0:H, :] + X[:, H:) . W[H:, :]. The head runs on the matrix cores (fp16 MFMA)
 * over a dense copy of X[:, 0:H) (codes and presence bits, built once per matrix): every
 * code is decoded exactly as the reference codec does (fma(code, scale, offset),
 * include/Cellerator/quantized/access.cuh:81-91), scaled by a power of two 2^k and split
 * into three fp16 parts whose sum is the scaled value, so each product is exact in fp32 and
 * only the fp32 summation order differs from the plain kernel. The split is exact for a
 * scaled value on the 2^-14 grid (every |x| >= 2^(9-k) is): cx_qcsr_hybrid_prepare checks
 * every value the head can decode on the device and returns CX_STATUS_UNSUPPORTED naming a
 * gene (or row offset) that is not -- order such genes after the head
 * (cx_qcsr_head_order does). The tail runs on the row-group VALU
 * kernel from each row's first entry >= H, adds the head's sums and applies the epilogue.
 * W is F16 (the execution-order packed dense operand). Engine addition; the reference's
 * projection has no matrix-core path for CSR. */
typedef struct cx_qcsr_hybrid_layout {
    uint32_t head_cols;     /* H, a multiple of 1,024 (0: no head) */
    uint32_t rows;
    uint32_t rows_ld;       /* rows rounded up to 512: the row stride of the head planes */
    uint32_t bits;
    uint32_t decode_policy;
    int32_t scale_exp;      /* k: meta and row_offsets hold values times 2^k */
    uint64_t nnz;           /* of the matrix it was built from */
    uint32_t *codes;        /* words form: [H * bits / 32][rows_ld]: word w of a row = codes of genes
                               [w * 32 / bits, (w + 1) * 32 / bits), 0 where not stored; else NULL */
    uint32_t *masks;        /* words form: [H / 32][rows_ld]: presence bit of gene g at bit g % 32; else NULL */
    int32_t *head_end;      /* [rows]: first entry of each row with gene >= H */
    float *meta;            /* [H] (scale, offset) pairs times 2^k */
    float *row_offsets;     /* [rows] times 2^k (column-scale / row-offset policy), else NULL */
    const struct cx_qcsr_tail_stream *tail;  /* prepared tail stream (cx_qcsr_tail_fill), or NULL:
                                                the tail then runs on the row-group kernel */
    uint32_t head_form;     /* CX_HEAD_FORM_WORDS (codes, masks) or CX_HEAD_FORM_TABLE (code_bytes, lut) */
    uint32_t reserved;
    uint8_t *code_bytes;    /* table form: [H/32][rows_ld][32]: code * 8 of each (row, gene), 128 where not stored */
    uint16_t *lut;          /* table form: [H/32][32][17][4] fp16: (hi, mid, lo, 0) of each code's value times
                               2^k (the three-part split above), entry 16 zero */
} cx_qcsr_hybrid_layout;

/* Head forms: code words and presence bits, decoded per value (8-bit codes or the
 * column-scale / row-offset policy); or code bytes and a per-gene table of the pre-split
 * values (codes of up to 4 bits under a per-gene policy). Same values and sums either way. */
#define CX_HEAD_FORM_WORDS 1u
#define CX_HEAD_FORM_TABLE 2u

/* Device bytes of the head layout of `a` (a.flags must include CX_QCSR_COLUMNS_SORTED). */
int cx_qcsr_hybrid_layout_bytes(const cx_qcsr_matrix *a, uint32_t head_cols, uint64_t *bytes);
/* Builds the head layout into `storage` (256-byte aligned, cx_qcsr_hybrid_layout_bytes) and
 * fills *layout with its pointers and k. Once per matrix; synchronizes `stream`. Rejects
 * rows whose genes are not strictly increasing (INVALID_ARGUMENT) and non-finite metadata
 * (UNSUPPORTED). */
int cx_qcsr_hybrid_prepare(const cx_qcsr_matrix *a, uint32_t head_cols, void *storage, uint64_t storage_bytes,
                           cx_qcsr_hybrid_layout *layout, void *stream);
/* Workspace bytes of cx_qcsr_spmm_fwd_hybrid: the head's sums (rows x 64 fp32, 256-byte
 * aligned, once per gene part of the head: a words-form head over fewer rows than four
 * 64-row waves per SIMD of the current device splits its genes into up to three parts) and
 * the head genes' weight panel ([H/32][out_cols][32] F16, 256-byte aligned). Query it on
 * the device that runs the product. */
int cx_qcsr_hybrid_workspace(const cx_qcsr_matrix *a, uint32_t head_cols, int64_t out_cols, uint64_t *bytes);
/* Y = act(alpha * (A . W) + beta * C + bias) for A in execution order with a.flags including
 * CX_QCSR_COLUMNS_SORTED, codes of 1/2/4/8 bits (any decode policy), F16 W [cols x out_cols]
 * (row stride rhs_ld), out_cols 64..256 in steps of 64 (one head and one tail launch per 64
 * columns), 16-byte aligned operands, `layout` from cx_qcsr_hybrid_prepare on this matrix.
 * head_cols == 0 runs the plain row-group kernel (or the tail stream over the whole matrix
 * when layout.tail is set). workspace: 256-byte aligned, cx_qcsr_hybrid_workspace bytes.
 * Deterministic. */
int cx_qcsr_spmm_fwd_hybrid(const cx_qcsr_matrix *a, const cx_qcsr_hybrid_layout *layout, const void *rhs,
                            int64_t rhs_ld, int64_t out_cols, float *out, int64_t out_ld,
                            const cx_spmm_epilogue *epilogue, void *workspace, uint64_t workspace_bytes,
                            void *stream);

/* ---- prepared tail stream ----------------------------------------------------------------
 * The entries of every row from its first tail entry (layout.head_end) on, rearranged once
 * per structure into the order the row-group walk consumes them: the rows sorted by tail
 * length over the whole matrix (descending, ties by row), sets of 8 adjacent rows dealt
 * round-robin to blocks of 1,024 rows, each block's sets given heaviest first to the
 * least-loaded of 16 waves (8 layers of 8 rows each); per gene part of
 * 1,024 and layer, the 8 rows' runs as fills of 16 steps x 8 rows (group-major), padded with
 * the zero row, each row's run even genes first in even groups and odd genes first in odd
 * groups; fills in (block, wave, part, layer) order, so a wave's fills are contiguous. With the
 * stream the tail kernel loads its entries instead of finding them (no per-pass run count,
 * window or reload). Built in two steps because the stream's size depends on the data:
 * cx_qcsr_tail_plan (slot rows and fill index; returns the entry bytes) and
 * cx_qcsr_tail_fill. Then set layout.tail to the stream. head_cols may be 0: the whole
 * matrix is then the tail. Engine addition; no counterpart in the reference. */
typedef struct cx_qcsr_tail_stream {
    uint32_t rows;
    uint32_t first_part;    /* head_cols / 1024 */
    uint32_t parts;         /* gene parts of 1,024 in the stream: ceil(cols / 1024) - first_part */
    uint32_t blocks;        /* ceil(rows / block_rows), or, when that is below the device's compute units
                               (the environment's CX_BLOCKS_PER_ROUND, a positive integer, replaces their
                               count), min(compute units, ceil(rows / 8)) blocks of fewer rows; the walk
                               launches one workgroup per block */
    uint32_t block_rows;    /* row slots per block: 16 waves x layers x 8 (1,024) */
    uint32_t layers;        /* layers of 8 rows per wave (8) */
    uint32_t bits;
    uint32_t entry_bytes;   /* 2 (codes of up to 4 bits: gene in part | code << 11) or 4 (8-bit: gene | code << 16) */
    uint64_t fills;         /* fills of 128 entries */
    uint64_t nnz;           /* of the matrix it was built from */
    uint32_t *slot_rows;    /* [blocks][block_rows]: row of slot (wave * layers + layer) * 8 + group, 0xffffffff none */
    uint32_t *fill_index;   /* [blocks * parts * (block_rows / 8) + 1], (block, wave, part, layer) order: first
                               fill of the layer's part in the low 28 bits, steps of its last fill - 1 in the
                               high 4; last entry: the total */
    void *entries;          /* [fills + 3][128] entries (set by cx_qcsr_tail_fill) */
} cx_qcsr_tail_stream;

/* Device bytes of the plan storage (slot rows, fill index, counts, scan workspace). */
int cx_qcsr_tail_plan_bytes(const cx_qcsr_matrix *a, const cx_qcsr_hybrid_layout *layout, uint64_t *bytes);
/* Plans the stream of `a` (rows sorted: CX_QCSR_COLUMNS_SORTED) after `layout`'s head into
 * `storage` (256-byte aligned, cx_qcsr_tail_plan_bytes); *entry_bytes receives the bytes the
 * entries need. Synchronizes `stream`. Rejects rows not sorted within [head_cols, cols)
 * (INVALID_ARGUMENT) and streams of 2^28 fills or more (INVALID_SHAPE). */
int cx_qcsr_tail_plan(const cx_qcsr_matrix *a, const cx_qcsr_hybrid_layout *layout, void *storage,
                      uint64_t storage_bytes, cx_qcsr_tail_stream *out, uint64_t *entry_bytes, void *stream);
/* Writes the entries into `entries` (256-byte aligned, the bytes cx_qcsr_tail_plan returned)
 * and sets out->entries. Stream-ordered, no synchronization. */
int cx_qcsr_tail_fill(const cx_qcsr_matrix *a, const cx_qcsr_hybrid_layout *layout, cx_qcsr_tail_stream *stream_out,
                      void *entries, uint64_t entry_bytes, void *stream);

/* The execution order of a prepared projection (host arrays; counts from
 * cx_qcsr_column_counts, metadata as the matrix holds it: scales [cols] or interleaved
 * (scale, offset) pairs [2 * cols] for CX_DECODE_PER_GENE_AFFINE_PAIRS, offsets [cols] or
 * NULL (0), row_offsets [rows] or NULL (0) under CX_DECODE_COLUMN_SCALE_ROW_OFFSET, scales
 * NULL = 1). It is the popularity order (cx_popularity_order) except that genes the
 * matrix-core head cannot carry exactly are moved after the head. A gene fits a layout
 * exponent K when every decoded value times 2^K lies on the 2^-14 grid with its scaled
 * metadata a normal float (under the row-offset policy: 2^K s on the grid, and 2^K r for every
 * row offset) and its largest decoded magnitude (plus the largest |row offset| under that
 * policy) is below 2^(15-K). The head is the most popular genes that fit the K under which
 * they cover the most stored entries (whole 1,024-gene parts, at most head_cols); the
 * layout's own exponent (14 - floor(log2) of the head's largest magnitude) is then at least K,
 * so cx_qcsr_hybrid_prepare's check passes. Head genes keep their popularity order, then
 * every other gene in popularity order. *head_out = the head width: head_cols capped at cols
 * rounded down to 1,024, or fewer when fewer genes fit (0 when a row offset never does).
 * Engine addition. */
int cx_qcsr_head_order(const uint32_t *counts, uint32_t cols, uint32_t bits, uint32_t decode_policy,
                       const float *scales, const float *offsets, const float *row_offsets, uint32_t rows,
                       uint32_t head_cols, uint32_t *feature_permutation, uint32_t *inverse_permutation,
                       uint32_t *head_out);

/* ---- prepared execution-order projection ------------------------------------------------
 * One object that owns everything the prepared path reads: the execution order of the genes
 * (cx_qcsr_head_order), the per-gene metadata in that order, the dense head layout
 * (cx_qcsr_hybrid_prepare) and the tail stream (cx_qcsr_tail_plan / cx_qcsr_tail_fill) of the
 * matrix relabelled into that order. Built once per structure and code generation from the
 * canonical matrix `a` (quantized codes of 1/2/4/8 bits, any decode policy, each gene at most
 * once per row; rows need not be sorted); the relabelled column indices and codes exist only
 * during the build. Launches take the CANONICAL operands: W [cols x out_cols] F16 in canonical
 * gene order (row stride rhs_ld) is gathered into execution order in the workspace, then the
 * head (matrix cores) and the tail stream run; Y rows are the matrix's rows. Same values and
 * sums as cx_qcsr_spmm_fwd_hybrid on the relabelled matrix with the same head width.
 * head_cols: a multiple of 1,024 (capped at cols rounded down to 1,024; 0: no head); the
 * head used may be narrower when fewer genes decode exactly in it (cx_qcsr_exec_query).
 * cx_qcsr_exec_prepare allocates device memory and synchronizes `stream`; cx_qcsr_exec_spmm
 * allocates nothing and does not synchronize (workspace: 256-byte aligned,
 * cx_qcsr_exec_workspace_bytes). A projection may be launched from several streams at once
 * with separate workspaces. Engine addition: the reference's quantized CSR projection has no
 * prepared execution-order form; this is the persistent state behind the CP-Math
 * execution-order candidate (cellerator_amd/cpmath/cpmath_backend.hh). */
typedef struct cx_qcsr_exec_projection cx_qcsr_exec_projection;
typedef struct cx_qcsr_exec_info {
    uint32_t rows;
    uint32_t cols;
    uint32_t bits;
    uint32_t head_cols;         /* the head width used */
    uint64_t nnz;
    uint64_t tail_fills;        /* fills of 128 entries in the tail stream */
    uint64_t persistent_bytes;  /* device bytes the projection holds */
    uint32_t head_form;         /* CX_HEAD_FORM_* */
    uint32_t tail_blocks;       /* workgroups of the tail walk (cx_qcsr_tail_stream.blocks) */
} cx_qcsr_exec_info;
int cx_qcsr_exec_prepare(const cx_qcsr_matrix *a, uint32_t head_cols, cx_qcsr_exec_projection **out, void *stream);
int cx_qcsr_exec_query(const cx_qcsr_exec_projection *p, cx_qcsr_exec_info *info);
int cx_qcsr_exec_workspace_bytes(const cx_qcsr_exec_projection *p, int64_t out_cols, uint64_t *bytes);
/* The same from the shape alone, before a projection exists (head_cols as passed to prepare);
 * sized for the larger of the head forms, since the code width is not given. */
int cx_qcsr_exec_workspace_for(uint32_t rows, uint32_t cols, uint32_t head_cols, int64_t out_cols, uint64_t *bytes);
/* Y = act(alpha * (A . W) + beta * C + bias) with canonical W; out_cols 64..256 by 64, Y 16-byte
 * aligned with a 16-byte multiple row stride; deterministic. */
int cx_qcsr_exec_spmm(const cx_qcsr_exec_projection *p, const void *rhs, int64_t rhs_ld, int64_t out_cols,
                      float *out, int64_t out_ld, const cx_spmm_epilogue *epilogue, void *workspace,
                      uint64_t workspace_bytes, void *stream);
/* Frees the projection's device memory (NULL is accepted). No launch on it may be in flight. */
int cx_qcsr_exec_destroy(cx_qcsr_exec_projection *p);

/* N = 1 CSR comparator: csr_spmv_fwd_f16_f32 (src/compute/sparse/ops/ops.hh:83-90);
 * y[r] = sum fp32(values) * x[col]. values F16 or F32. */
int cx_csr_spmv_fwd(uint32_t rows, const uint32_t *row_ptr, const uint32_t *col_idx,
                    const void *values, uint32_t value_dtype, const float *x, float *y,
                    void *stream);

/* Message of the last failing call on this thread ("" if none). */
const char *cx_last_error(void);
/* Engine build identity, e.g. "cellerator_amd gfx950". */
const char *cx_build_info(void);

/* ------------------------------------------------------------------------------- */
/* 2. Public context ABI (include/Cellerator/abi.h:31-152)                          */
/* ------------------------------------------------------------------------------- */

typedef enum cellerator_sparse_layout {
    CELLERATOR_LAYOUT_CSR = 1,
    CELLERATOR_LAYOUT_BLOCKED_ELL = 2,
    CELLERATOR_LAYOUT_SLICED_ELL = 3,
    CELLERATOR_LAYOUT_QUANTIZED_BLOCKED_ELL = 4,
    CELLERATOR_LAYOUT_QUANTIZED_CSR = 5 /* additive: packed codes + major_ptr/minor_idx */
} cellerator_sparse_layout;

typedef enum cellerator_saved_state_kind {
    CELLERATOR_SAVED_STATE_NONE = 0,
    CELLERATOR_SAVED_STATE_SPARSE_PROJECTION = 1,
    CELLERATOR_SAVED_STATE_ROW_SCALE = 2,
    CELLERATOR_SAVED_STATE_RECONSTRUCTION_LOSS = 3
} cellerator_saved_state_kind;

typedef struct cellerator_context cellerator_context;
typedef struct cellerator_saved_state cellerator_saved_state;

typedef struct cellerator_execution_config {
    uint32_t version;
    size_t size;
    int32_t device;
    void *stream;
    void *scratch;
    size_t scratch_bytes;
} cellerator_execution_config;

typedef struct cellerator_tensor_desc {
    uint32_t version;
    size_t size;
    void *data;
    cellerator_dtype dtype;
    uint32_t rank;
    uint64_t shape[CELLERATOR_TENSOR_MAX_RANK];
    int64_t stride[CELLERATOR_TENSOR_MAX_RANK];
} cellerator_tensor_desc;

/* For CELLERATOR_LAYOUT_QUANTIZED_CSR, major_ptr holds the rows + 1 nnz offsets,
 * minor_idx the gene of each nnz, packed_values the codes, and block_col_idx (unused by
 * CSR layouts) carries the rows + 1 packed row byte offsets that build_packed_row_ptr
 * produces (include/Cellerator/quantized/layout.cuh:106-129). */
typedef struct cellerator_sparse_layout_desc {
    uint32_t version;
    size_t size;
    cellerator_sparse_layout layout;
    uint32_t rows;
    uint32_t cols;
    uint32_t nnz;
    uint32_t block_size;
    uint32_t ell_cols;
    uint32_t row_stride_bytes;
    uint32_t bits;
    uint32_t decode_policy;
    cellerator_dtype value_dtype;
    const uint32_t *major_ptr;
    const uint32_t *minor_idx;
    const uint32_t *block_col_idx;
    const void *values;
    const uint8_t *packed_values;
    const float *column_scales;
    const float *column_offsets;
    const float *row_offsets;
} cellerator_sparse_layout_desc;

const char *cellerator_status_string(cellerator_status status);
const char *cellerator_last_error(void);

cellerator_status cellerator_context_create(const cellerator_execution_config *config,
                                            cellerator_context **out_context);
cellerator_status cellerator_context_synchronize(cellerator_context *context);
void cellerator_context_destroy(cellerator_context *context);
void cellerator_saved_state_destroy(cellerator_saved_state *saved_state);

/* rhs: F32 (reference contract) or F16/BF16 rank-2 [cols x N] row-major;
 * out: F32 rank-2 [rows x N] row-major. Layouts: CSR (F16/F32 values), BLOCKED_ELL
 * (F16/BF16/F32 values), QUANTIZED_BLOCKED_ELL, QUANTIZED_CSR. SLICED_ELL returns
 * UNSUPPORTED, as the reference does (src/abi/abi.cu:326-328). */
cellerator_status cellerator_sparse_projection_forward(cellerator_context *context,
                                                       const cellerator_sparse_layout_desc *layout,
                                                       const cellerator_tensor_desc *rhs,
                                                       cellerator_tensor_desc *out,
                                                       cellerator_saved_state **saved_state);

/* include/Cellerator/abi.h:120-126, src/abi/abi.cu:337-400: gradients of
 * out = A . rhs. grad_values (F32 rank-1 [nnz], optional) = <grad_out[row_i,:], rhs[col_i,:]>;
 * grad_rhs (F32 rank-2 [cols x N], optional) = A^T . grad_out; at least one is required.
 * Layouts: CSR (F16, or additively F32, values) and QUANTIZED_CSR (additive); others return
 * UNSUPPORTED as the reference does. rhs F32 (reference contract) or F16; grad_out F32.
 * Deterministic: grad_rhs builds A^T (stable device sort) in the context scratch and sums
 * each gene row in a fixed order, where the reference adds with float atomics. The scratch
 * is the config's (too small -> INVALID_ARGUMENT) or, without one, the context's own block,
 * grown on demand and released by cellerator_context_destroy. */
cellerator_status cellerator_sparse_projection_backward(cellerator_context *context,
                                                        const cellerator_sparse_layout_desc *layout,
                                                        const cellerator_tensor_desc *rhs,
                                                        const cellerator_tensor_desc *grad_out,
                                                        cellerator_tensor_desc *grad_values,
                                                        cellerator_tensor_desc *grad_rhs);

#ifdef __cplusplus
}
#endif

#endif /* CELLERATOR_AMD_H */
