/*
 * oracle.h -- CPU restatement of Cellerator's sparse expression-matrix projection
 * arithmetic. TEST INFRASTRUCTURE ONLY: the pytest suite, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg load this library as the checker. Nothing in the
 * product (cellerator_amd/, include/) links, loads or calls it.
 *
 * Every function cites the reference file:line it restates (paths are relative to
 * the tumlinso/Cellerator source tree).
 *
 * Pinning (what checks each function against something other than itself):
 *   codec (unpack/dequantize/quantize/packed_row_ptr/pack/decode)
 *       - reference KAT tests/quantized_matrix_test.cu:15-28,78-96 (4x8 fixture,
 *         bits 1/2/4/8 x both metadata policies) -> tests/golden/codec_kat.json
 *       - exhaustive closed form: every code x sampled scale/offset equals
 *         fma(code, scale, offset) computed in float64 and rounded once.
 *   or_spmm_referee
 *       - reference KATs {0,30,29,74} (tests/math_referee_foundation_test.cc:61-106,
 *         both plain and transposed) and {201,402,430,860,5,10}
 *         (tests/sparse_ops_runtime_test.cu:140-161,279-297)
 *       - brute force: dense float64 GEMM of the densified matrix on random inputs.
 *   or_qcsr_spmm_referee / or_qcsr_spmm_f32_mt
 *       - composition of the pinned codec and the pinned referee; also checked
 *         against a numpy dense GEMM of the decoded matrix.
 *   or_bell_spmm_referee
 *       - reference KAT: Blocked-ELL of the 3x3 fixture reproduces {201,...,10}
 *         (tests/sparse_ops_runtime_test.cu:299-358); per-gene 8-bit and row-offset
 *         4-bit quantized BELL KATs (:366-470); brute force against densified GEMM.
 *   or_cpbp_canonical / or_cpbp_tiles
 *       - the two referees agree within 1e-5/1e-5 (the reference's own invariant,
 *         components/CellPack/include/CellPack/feature_weighted_row_reduction.hh:13-14);
 *         36-feature plan fixture shape of
 *         components/CellPack/tests/feature_weighted_row_reduction_cuda_test.cu:69-151;
 *         brute force: dense mat-vec in float64.
 *   or_spmm_bwd_values
 *       - reference KAT {5,500,110,1100,17} (tests/sparse_ops_runtime_test.cu:140-161,566-582);
 *       - adjoint identity: sum_i grad_values[i] * x_i == <grad_out, X . W> (Frobenius),
 *         with X . W from the pinned referee, on random inputs (a transposed operand or a
 *         wrong row/column index breaks it).
 *   grad_rhs = X^T . grad_out is or_spmm_referee with transpose_sparse = 1, pinned by the
 *       reference KAT {26,32,9,12,14,20} (tests/sparse_ops_runtime_test.cu:584-604).
 *   or_compare
 *       - restates compare_spmm_reference (include/Cellerator/compute/math/referee.hh:143-211);
 *         pinned by planted-error tests in tests/test_oracle.py.
 *   or_digest_logical_dense
 *       - the reference test's property (tests/math_referee_foundation_test.cc:108-127: one
 *         element changed by 0.25 changes the digest), layout invariance (row- and
 *         column-major views of one logical matrix digest equally), f16/f32 views of equal
 *         values differing only through the mixed type code. Parity of the exact digest
 *         values is UNPINNED: no recorded digest exists in the reference, and referee.hh
 *         needs cuda_fp16.h, so it cannot be built here.
 */
#ifndef CELLERATOR_ORACLE_H
#define CELLERATOR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Value type codes follow cellerator::real (include/Cellerator/types.cuh:150-157). */
enum { OR_F16 = 3, OR_F32 = 4, OR_F64 = 5, OR_BF16 = 6 };
/* Decode policies follow quantized/blocked_ell.cuh:10-14. */
enum { OR_POLICY_PER_GENE_AFFINE = 1, OR_POLICY_COLUMN_SCALE_ROW_OFFSET = 2 };
/* Epilogue kinds follow include/Cellerator/compute/math/operation.hh:49-58. */
enum {
    OR_EPI_NONE = 0, OR_EPI_BIAS = 1, OR_EPI_RELU = 2, OR_EPI_GELU_ERF = 3,
    OR_EPI_GELU_TANH = 4, OR_EPI_BIAS_RELU = 5, OR_EPI_BIAS_GELU_ERF = 6,
    OR_EPI_BIAS_GELU_TANH = 7
};

/* ---- scalar conversions (exact widening; RNE narrowing) ---- */
float or_half_to_float(uint16_t h);
uint16_t or_float_to_half(float f);
float or_bf16_to_float(uint16_t b);
uint16_t or_float_to_bf16(float f);

/* ---- codec: include/Cellerator/quantized/{format,access,layout,packing}.cuh ---- */
uint32_t or_unpack_code(uint32_t bits, const uint8_t *row_base, int64_t local_index);
float or_dequantize_code(uint32_t code, float scale, float offset);
uint32_t or_quantize_code(uint32_t bits, float value, float scale, float offset);
int64_t or_build_packed_row_ptr(uint32_t bits, const int32_t *row_ptr, int32_t rows,
                                int32_t *packed_row_ptr);
int or_pack_csr(uint32_t bits, uint32_t policy, int32_t rows, const int32_t *row_ptr,
                const int32_t *packed_row_ptr, const int32_t *col_idx, const float *values,
                const float *col_scales, const float *col_offsets, const float *row_offsets,
                uint8_t *packed);
int or_decode_csr(uint32_t bits, uint32_t policy, int32_t rows, const int32_t *row_ptr,
                  const int32_t *packed_row_ptr, const int32_t *col_idx, const uint8_t *packed,
                  const float *col_scales, const float *col_offsets, const float *row_offsets,
                  float *values);

/* ---- CP-Math CPU referee: src/compute/math/referee.cc:101-253 ---- */
int or_spmm_referee(uint64_t m, uint64_t k, uint64_t n, int transpose_sparse,
                    int transpose_dense, const uint64_t *row_offsets, const uint32_t *cols,
                    const void *values, int value_type, uint64_t nnz, const void *rhs,
                    int rhs_type, int rhs_col_major, uint64_t ldb, double alpha, double beta,
                    const void *c0, int c0_type, int c0_col_major, uint64_t ldc0, int epilogue,
                    const void *bias, int bias_type, double *out);

typedef struct or_comparison {
    uint64_t element_count;
    uint64_t mismatch_count;
    uint64_t non_finite_reference_count;
    uint64_t non_finite_candidate_count;
    uint64_t worst_index;
    double max_absolute_error;
    double max_relative_error;
    double mean_absolute_error;
    double root_mean_square_error;
    int within_tolerance;
} or_comparison;

/* compare_spmm_reference (include/Cellerator/compute/math/referee.hh:143-211);
 * when `magnitude` is non-null the absolute term becomes abs_tol * magnitude[i]
 * (the reordered-summation bound scaled by sum |x||w| of element i). */
int or_compare(const double *reference, const float *candidate, uint64_t count,
               double abs_tol, double rel_tol, double relative_floor,
               const double *magnitude, or_comparison *out);

/* ---- quantized CSR SpMM = codec dequantize_code (access.cuh:81-91) composed with
 * the referee (referee.cc:101-253), alpha=1, beta=0, no epilogue. Rows
 * [row_begin, row_end) only; out is (row_end-row_begin) x n row-major float64.
 * `magnitude` (optional) receives sum |x||w| per element. ---- */
int or_qcsr_spmm_referee(uint32_t bits, uint32_t policy, int32_t rows, int32_t cols,
                         const int32_t *row_ptr, const int32_t *packed_row_ptr,
                         const int32_t *col_idx, const uint8_t *packed,
                         const float *col_scales, const float *col_offsets,
                         const float *row_offsets, const void *rhs, int rhs_type,
                         uint32_t n, uint64_t ldb, int32_t row_begin, int32_t row_end,
                         double *out, double *magnitude);

/* Row-parallel fp32 restatement used as the CPU baseline: decode, fp32 multiply,
 * fp32 accumulate in nnz order (the semantics of csr_spmm_fwd_kernel_,
 * src/compute/sparse/project/kernels/csr_spmm_fwd_kernel_.cuh:1-22). */
int or_qcsr_spmm_f32_mt(uint32_t bits, uint32_t policy, int32_t rows, int32_t cols,
                        const int32_t *row_ptr, const int32_t *packed_row_ptr,
                        const int32_t *col_idx, const uint8_t *packed,
                        const float *col_scales, const float *col_offsets,
                        const float *row_offsets, const void *rhs, int rhs_type, uint32_t n,
                        uint64_t ldb, int32_t row_begin, int32_t row_end, float *out,
                        int threads);
/* The same walk with |decoded x| and |w|: out = Sigma |x||w| per element (fp32), the
 * magnitude term of the reordered-summation tolerance for a full-output comparison. */
int or_qcsr_spmm_f32_mt_magnitude(uint32_t bits, uint32_t policy, int32_t rows, int32_t cols,
                                  const int32_t *row_ptr, const int32_t *packed_row_ptr,
                                  const int32_t *col_idx, const uint8_t *packed,
                                  const float *col_scales, const float *col_offsets,
                                  const float *row_offsets, const void *rhs, int rhs_type,
                                  uint32_t n, uint64_t ldb, int32_t row_begin, int32_t row_end,
                                  float *out, int threads);
/* Row-parallel or_cpbp_canonical (bitwise equal to it: rows are independent). */
int or_cpbp_canonical_mt(uint32_t rows, const uint32_t *row_offsets,
                         const uint32_t *canonical_features, const void *values, int value_type,
                         const float *weights, float *out, int threads);
/* Row-block-parallel bf16 Blocked-ELL SpMM, fp32 accumulation in slot order per output
 * element (blocked_ell_spmm_fwd_kernel_.cuh:1-33); rhs bf16 [cols x n] row-major, out fp32
 * [rows x n]. Zero values are skipped (their products add nothing). CPU baseline. */
int or_bell_spmm_bf16_mt(int32_t rows, int32_t cols, int32_t block_size, int32_t ell_cols,
                         const uint32_t *block_col_idx, const uint16_t *values,
                         const uint16_t *rhs, uint32_t n, float *out, int threads);

/* ---- Blocked-ELL: quantized/blocked_ell.cuh:120-150 (column_for_slot, get_value);
 * kernels/blocked_ell_spmm_fwd_kernel_.cuh:1-33. value_type OR_BF16/OR_F16/OR_F32 for
 * plain BELL, or bits in {1,2,4,8} (value_type ignored) for quantized BELL when
 * `packed` is non-null. Output float64 rows x n. ---- */
int or_bell_spmm_referee(int32_t rows, int32_t cols, int32_t block_size, int32_t ell_cols,
                         const uint32_t *block_col_idx, const void *values, int value_type,
                         uint32_t bits, uint32_t policy, int32_t row_stride_bytes,
                         const uint8_t *packed, const float *col_scales,
                         const float *col_offsets, const float *row_offsets, const void *rhs,
                         int rhs_type, uint32_t n, uint64_t ldb, double *out,
                         double *magnitude);

/* ---- CP-BP feature-weighted row reduction:
 * components/CellPack/src/feature_weighted_row_reduction.cc:213-221 (accumulate),
 * :293-319 (canonical), :358-402 (tiles). value_type OR_F16 or OR_F32.
 * Accumulation is float32, as the reference's accum_t. ---- */
int or_cpbp_canonical(uint32_t rows, const uint32_t *row_offsets,
                      const uint32_t *canonical_features, const void *values, int value_type,
                      const float *weights, float *out);
int or_cpbp_tiles(uint32_t row_count, uint32_t tile_count, uint32_t tile_row_width,
                  uint32_t mask_bits, const uint32_t *feature_block_offsets,
                  const uint32_t *feature_permutation, const uint32_t *tile_block_offsets,
                  const uint32_t *tile_block_ids, const void *tile_block_cell_masks,
                  const uint32_t *block_row_entry_offsets, const uint32_t *row_block_gene_masks,
                  const uint32_t *row_block_value_offsets, const void *values, int value_type,
                  const uint32_t *row_permutation, const float *weights, float *out);
/* ---- backward of the CSR SpMM ----
 * csr_spmm_bwd_values_kernel_ (src/compute/sparse/ops/kernels/base_sparse/
 * csr_spmm_bwd_values_kernel_.cuh:1-19): grad_values[i] = sum_c grad_out[row_i, c] *
 * rhs[col_i, c], accumulated in float64 over c in order. Each operand has its own leading
 * dimension (the reference kernel reads both with rhs_ld). */
int or_spmm_bwd_values(uint32_t rows, const int32_t *row_ptr, const int32_t *col_idx,
                       const float *grad_out, uint64_t grad_out_ld, const void *rhs,
                       int rhs_type, uint64_t rhs_ld, uint64_t n, double *grad_values);
/* float64 canonical sum, for tolerance checks that do not depend on order. */
int or_cpbp_canonical_f64(uint32_t rows, const uint32_t *row_offsets,
                          const uint32_t *canonical_features, const void *values,
                          int value_type, const float *weights, double *out,
                          double *magnitude);
/* within_tolerance rule of feature_weighted_row_reduction.cc:225-241 */
int or_cpbp_within_tolerance(float reference, float candidate, double abs_tol,
                             double rel_tol);

/* ---- determinism digest ----
 * digest_logical_dense (include/Cellerator/compute/math/referee.hh:219-244, with
 * referee_detail::dense_offset / valid_dense / read_dense / digest_mix at :85-130): two
 * 64-bit lanes seeded (1469598103934665603, 0x6a09e667f3bcc909); rows, columns and the
 * value type code are mixed in, then every element in logical row-major order as the bits
 * of its float64 widening. Views are row-major (column_major = 0) or column-major with
 * leading dimension ld. Returns 0 (ok), 1 (invalid_argument: NULL digest or an invalid
 * view) or 3 (unsupported_type: a value type other than f16, f32, f64, met on the first
 * element). */
int or_digest_logical_dense(const void *values, uint64_t rows, uint64_t columns, uint64_t ld,
                            int column_major, uint32_t value_type, uint64_t digest[2]);

#ifdef __cplusplus
}
#endif

#endif
