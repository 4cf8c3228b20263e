/*
 * oracle.c -- CPU restatement of the reference arithmetic for the projection hot path.
 * TEST INFRASTRUCTURE ONLY (see oracle.h): loaded by tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg as the checker; never by the product.
 *
 * Built with -ffp-contract=off so that every float expression rounds exactly where
 * the reference's host code rounds (explicit fmaf where the reference's device code
 * contracts to an FMA).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* scalar conversions                                                          */
/* ------------------------------------------------------------------------- */

float or_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exponent = (h >> 10) & 0x1fu;
    uint32_t mantissa = h & 0x3ffu;
    uint32_t bits;
    if (exponent == 0x1fu) {
        bits = sign | 0x7f800000u | (mantissa << 13);
    } else if (exponent == 0u) {
        if (mantissa == 0u) {
            bits = sign;
        } else {
            /* subnormal half: renormalise into a float */
            int e = -1;
            do {
                ++e;
                mantissa <<= 1;
            } while ((mantissa & 0x400u) == 0u);
            mantissa &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (mantissa << 13);
        }
    } else {
        bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    float out;
    memcpy(&out, &bits, sizeof(out));
    return out;
}

uint16_t or_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof(x));
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t abs = x & 0x7fffffffu;
    if (abs >= 0x7f800000u) { /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (abs > 0x7f800000u ? 0x200u : 0u));
    }
    if (abs >= 0x477ff000u) { /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (abs < 0x38800000u) { /* below the smallest normal half: subnormal or zero */
        if (abs < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to 0 */
        const uint32_t exponent = abs >> 23;
        const uint32_t mantissa = (abs & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - exponent; /* 14..24 */
        uint32_t half = mantissa >> shift;
        const uint32_t rem = mantissa & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (half & 1u))) ++half;
        return (uint16_t)(sign | half);
    }
    uint32_t half = ((abs >> 13) - (112u << 10));
    const uint32_t rem = abs & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) ++half;
    return (uint16_t)(sign | half);
}

float or_bf16_to_float(uint16_t b) {
    const uint32_t bits = (uint32_t)b << 16;
    float out;
    memcpy(&out, &bits, sizeof(out));
    return out;
}

uint16_t or_float_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof(x));
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    const uint32_t lsb = (x >> 16) & 1u;
    x += 0x7fffu + lsb;
    return (uint16_t)(x >> 16);
}

static double read_typed(const void *values, int type, uint64_t index) {
    switch (type) {
    case OR_F16: return (double)or_half_to_float(((const uint16_t *)values)[index]);
    case OR_BF16: return (double)or_bf16_to_float(((const uint16_t *)values)[index]);
    case OR_F32: return (double)((const float *)values)[index];
    case OR_F64: return ((const double *)values)[index];
    default: return NAN;
    }
}

static float read_typed_f(const void *values, int type, uint64_t index) {
    switch (type) {
    case OR_F16: return or_half_to_float(((const uint16_t *)values)[index]);
    case OR_BF16: return or_bf16_to_float(((const uint16_t *)values)[index]);
    case OR_F32: return ((const float *)values)[index];
    default: return NAN;
    }
}

/* ------------------------------------------------------------------------- */
/* codec                                                                       */
/* ------------------------------------------------------------------------- */

static int valid_bits(uint32_t bits) {
    return bits == 1u || bits == 2u || bits == 4u || bits == 8u;
}

/* format_traits<Bits>::unpack (include/Cellerator/quantized/format.cuh:39-48):
 * code i lives in byte i / codes_per_byte, low bits first. */
uint32_t or_unpack_code(uint32_t bits, const uint8_t *row_base, int64_t local_index) {
    const int64_t codes_per_byte = 8 / (int64_t)bits;
    const uint32_t mask = (1u << bits) - 1u;
    const uint32_t shift = (uint32_t)(local_index % codes_per_byte) * bits;
    return ((uint32_t)row_base[local_index / codes_per_byte] >> shift) & mask;
}

/* dequantize_code (include/Cellerator/quantized/access.cuh:81-91) with
 * fast_fma = a*b+c contracted to one FMA on the device (numeric.cuh:34-36). */
float or_dequantize_code(uint32_t code, float scale, float offset) {
    return fmaf((float)code, scale, offset);
}

/* quantize_code, portable rule (include/Cellerator/quantized/access.cuh:104-131):
 * IEEE divide, round half away from zero, clamp to [0, 2^bits - 1], scale 0 -> 0. */
uint32_t or_quantize_code(uint32_t bits, float value, float scale, float offset) {
    const float centered = value - offset;
    if (scale == 0.0f) return 0u;
    const float q = centered / scale;
    const int rounded = q >= 0.0f ? (int)(q + 0.5f) : (int)(q - 0.5f);
    const int max_code = (int)((1u << bits) - 1u);
    if (rounded < 0) return 0u;
    if (rounded > max_code) return (uint32_t)max_code;
    return (uint32_t)rounded;
}

/* build_packed_row_ptr (include/Cellerator/quantized/layout.cuh:106-129):
 * unpadded, byte-granular row starts. Returns the total packed byte count. */
int64_t or_build_packed_row_ptr(uint32_t bits, const int32_t *row_ptr, int32_t rows,
                                int32_t *packed_row_ptr) {
    if (!valid_bits(bits) || row_ptr == NULL || packed_row_ptr == NULL || rows < 0) return -1;
    const int64_t cpb = 8 / (int64_t)bits;
    int64_t total = 0;
    packed_row_ptr[0] = 0;
    for (int32_t r = 0; r < rows; ++r) {
        const int64_t nnz = (int64_t)row_ptr[r + 1] - row_ptr[r];
        total += nnz <= 0 ? 0 : (nnz + cpb - 1) / cpb;
        if (total > INT32_MAX) return -1;
        packed_row_ptr[r + 1] = (int32_t)total;
    }
    return total;
}

/* per_gene_affine / column_scale_row_offset (include/Cellerator/quantized/metadata.cuh:7-56):
 * null scale -> 1, null offset -> 0. */
static void metadata_for(uint32_t policy, int32_t row, int32_t col, const float *col_scales,
                         const float *col_offsets, const float *row_offsets, float *scale,
                         float *offset) {
    *scale = col_scales != NULL ? col_scales[col] : 1.0f;
    if (policy == OR_POLICY_COLUMN_SCALE_ROW_OFFSET) {
        *offset = row_offsets != NULL ? row_offsets[row] : 0.0f;
    } else {
        *offset = col_offsets != NULL ? col_offsets[col] : 0.0f;
    }
}

/* pack_row_values (include/Cellerator/quantized/packing.cuh:13-170), host form:
 * codes assembled low bits first, unused high bits of a row's last byte are zero. */
int or_pack_csr(uint32_t bits, uint32_t policy, int32_t rows, const int32_t *row_ptr,
                const int32_t *packed_row_ptr, const int32_t *col_idx, const float *values,
                const float *col_scales, const float *col_offsets, const float *row_offsets,
                uint8_t *packed) {
    if (!valid_bits(bits) || rows < 0) return -1;
    const int64_t cpb = 8 / (int64_t)bits;
    for (int32_t r = 0; r < rows; ++r) {
        uint8_t *out = packed + packed_row_ptr[r];
        const int64_t begin = row_ptr[r], end = row_ptr[r + 1];
        const int64_t bytes = packed_row_ptr[r + 1] - (int64_t)packed_row_ptr[r];
        memset(out, 0, (size_t)bytes);
        for (int64_t i = begin; i < end; ++i) {
            float scale, offset;
            metadata_for(policy, r, col_idx[i], col_scales, col_offsets, row_offsets, &scale,
                         &offset);
            const uint32_t code = or_quantize_code(bits, values[i], scale, offset);
            const int64_t local = i - begin;
            out[local / cpb] |= (uint8_t)((code & ((1u << bits) - 1u))
                                          << ((uint32_t)(local % cpb) * bits));
        }
    }
    return 0;
}

/* unpack_row_values (include/Cellerator/quantized/packing.cuh:172-260) */
int or_decode_csr(uint32_t bits, uint32_t policy, int32_t rows, const int32_t *row_ptr,
                  const int32_t *packed_row_ptr, const int32_t *col_idx, const uint8_t *packed,
                  const float *col_scales, const float *col_offsets, const float *row_offsets,
                  float *values) {
    if (!valid_bits(bits) || rows < 0) return -1;
    for (int32_t r = 0; r < rows; ++r) {
        const uint8_t *base = packed + packed_row_ptr[r];
        for (int64_t i = row_ptr[r]; i < row_ptr[r + 1]; ++i) {
            float scale, offset;
            metadata_for(policy, r, col_idx[i], col_scales, col_offsets, row_offsets, &scale,
                         &offset);
            values[i] = or_dequantize_code(or_unpack_code(bits, base, i - row_ptr[r]), scale,
                                           offset);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* CP-Math referee: src/compute/math/referee.cc:101-253                        */
/* ------------------------------------------------------------------------- */

static int bias_epilogue(int kind) {
    return kind == OR_EPI_BIAS || kind == OR_EPI_BIAS_RELU || kind == OR_EPI_BIAS_GELU_ERF
        || kind == OR_EPI_BIAS_GELU_TANH;
}

/* apply_epilogue (referee.cc:81-97) */
static double apply_epilogue(double value, double bias, int kind) {
    if (bias_epilogue(kind)) value += bias;
    if (kind == OR_EPI_RELU || kind == OR_EPI_BIAS_RELU) return fmax(value, 0.0);
    if (kind == OR_EPI_GELU_ERF || kind == OR_EPI_BIAS_GELU_ERF)
        return 0.5 * value * (1.0 + erf(value * 0.7071067811865475244));
    if (kind == OR_EPI_GELU_TANH || kind == OR_EPI_BIAS_GELU_TANH)
        return 0.5 * value
            * (1.0 + tanh(0.7978845608028653559 * (value + 0.044715 * value * value * value)));
    return value;
}

static uint64_t dense_at(int col_major, uint64_t ld, uint64_t row, uint64_t col) {
    return col_major ? col * ld + row : row * ld + col;
}

int or_spmm_referee(uint64_t m, uint64_t k, uint64_t n, int transpose_sparse,
                    int transpose_dense, const uint64_t *row_offsets, const uint32_t *cols,
                    const void *values, int value_type, uint64_t nnz, const void *rhs,
                    int rhs_type, int rhs_col_major, uint64_t ldb, double alpha, double beta,
                    const void *c0, int c0_type, int c0_col_major, uint64_t ldc0, int epilogue,
                    const void *bias, int bias_type, double *out) {
    const uint64_t sparse_rows = transpose_sparse ? k : m;
    const uint64_t sparse_cols = transpose_sparse ? m : k;
    if (sparse_rows != 0u && (row_offsets[0] != 0u || row_offsets[sparse_rows] != nnz))
        return -2;
    if (beta != 0.0 && c0 == NULL) return -2;
    if (bias_epilogue(epilogue) && bias == NULL) return -1;
    for (uint64_t r = 0; r < m; ++r) {
        for (uint64_t c = 0; c < n; ++c) {
            const double initial = beta != 0.0
                ? read_typed(c0, c0_type, dense_at(c0_col_major, ldc0, r, c)) : 0.0;
            out[r * n + c] = beta * initial;
        }
    }
    for (uint64_t prow = 0; prow < sparse_rows; ++prow) {
        const uint64_t begin = row_offsets[prow], end = row_offsets[prow + 1];
        if (begin > end || end > nnz) return -2;
        for (uint64_t e = begin; e < end; ++e) {
            const uint64_t pcol = cols[e];
            if (pcol >= sparse_cols) return -2;
            const uint64_t out_row = transpose_sparse ? pcol : prow;
            const uint64_t reduction = transpose_sparse ? prow : pcol;
            const double sv = read_typed(values, value_type, e);
            for (uint64_t oc = 0; oc < n; ++oc) {
                const uint64_t rr = transpose_dense ? oc : reduction;
                const uint64_t rc = transpose_dense ? reduction : oc;
                const double dv = read_typed(rhs, rhs_type, dense_at(rhs_col_major, ldb, rr, rc));
                out[out_row * n + oc] += alpha * sv * dv;
            }
        }
    }
    for (uint64_t r = 0; r < m; ++r) {
        for (uint64_t c = 0; c < n; ++c) {
            const double b = bias_epilogue(epilogue) ? read_typed(bias, bias_type, c) : 0.0;
            double *v = &out[r * n + c];
            *v = apply_epilogue(*v, b, epilogue);
            if (!isfinite(*v)) return -5;
        }
    }
    return 0;
}

/* compare_spmm_reference (include/Cellerator/compute/math/referee.hh:143-211) */
int or_compare(const double *reference, const float *candidate, uint64_t count,
               double abs_tol, double rel_tol, double relative_floor,
               const double *magnitude, or_comparison *out) {
    if (out == NULL || abs_tol < 0.0 || rel_tol < 0.0 || relative_floor <= 0.0) return -1;
    or_comparison c;
    memset(&c, 0, sizeof(c));
    c.element_count = count;
    c.within_tolerance = 1;
    long double abs_sum = 0.0L, sq_sum = 0.0L;
    for (uint64_t i = 0; i < count; ++i) {
        const double actual = (double)candidate[i];
        const double expected = reference[i];
        if (!isfinite(expected)) {
            ++c.non_finite_reference_count;
            c.within_tolerance = 0;
            continue;
        }
        if (!isfinite(actual)) {
            ++c.non_finite_candidate_count;
            c.within_tolerance = 0;
            continue;
        }
        const double absolute = fabs(actual - expected);
        const double relative = absolute / fmax(fabs(expected), relative_floor);
        abs_sum += absolute;
        sq_sum += (long double)absolute * absolute;
        if (absolute > c.max_absolute_error) {
            c.max_absolute_error = absolute;
            c.worst_index = i;
        }
        c.max_relative_error = fmax(c.max_relative_error, relative);
        const double abs_term = magnitude != NULL ? abs_tol * magnitude[i] : abs_tol;
        if (absolute > abs_term + rel_tol * fabs(expected)) {
            ++c.mismatch_count;
            c.within_tolerance = 0;
        }
    }
    if (count != 0u) {
        c.mean_absolute_error = (double)(abs_sum / count);
        c.root_mean_square_error = sqrt((double)(sq_sum / count));
    }
    *out = c;
    if (c.non_finite_reference_count != 0u) return -5;
    if (c.non_finite_candidate_count != 0u) return -6;
    return 0;
}

/* ------------------------------------------------------------------------- */
/* quantized CSR SpMM                                                          */
/* ------------------------------------------------------------------------- */

int or_qcsr_spmm_referee(uint32_t bits, uint32_t policy, int32_t rows, int32_t cols,
                         const int32_t *row_ptr, const int32_t *packed_row_ptr,
                         const int32_t *col_idx, const uint8_t *packed,
                         const float *col_scales, const float *col_offsets,
                         const float *row_offsets, const void *rhs, int rhs_type,
                         uint32_t n, uint64_t ldb, int32_t row_begin, int32_t row_end,
                         double *out, double *magnitude) {
    if (!valid_bits(bits) || row_begin < 0 || row_end > rows || row_begin > row_end) return -1;
    const uint64_t count = (uint64_t)(row_end - row_begin) * n;
    memset(out, 0, count * sizeof(double));
    if (magnitude != NULL) memset(magnitude, 0, count * sizeof(double));
    for (int32_t r = row_begin; r < row_end; ++r) {
        const uint8_t *base = packed + packed_row_ptr[r];
        double *orow = out + (uint64_t)(r - row_begin) * n;
        double *mrow = magnitude != NULL ? magnitude + (uint64_t)(r - row_begin) * n : NULL;
        for (int64_t i = row_ptr[r]; i < row_ptr[r + 1]; ++i) {
            const int32_t col = col_idx[i];
            if (col < 0 || col >= cols) return -2;
            float scale, offset;
            metadata_for(policy, r, col, col_scales, col_offsets, row_offsets, &scale, &offset);
            const double x = (double)or_dequantize_code(
                or_unpack_code(bits, base, i - row_ptr[r]), scale, offset);
            for (uint32_t c = 0; c < n; ++c) {
                const double w = read_typed(rhs, rhs_type, (uint64_t)col * ldb + c);
                orow[c] += x * w;
                if (mrow != NULL) mrow[c] += fabs(x * w);
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* Blocked-ELL                                                                 */
/* ------------------------------------------------------------------------- */

int or_bell_spmm_referee(int32_t rows, int32_t cols, int32_t block_size, int32_t ell_cols,
                         const uint32_t *block_col_idx, const void *values, int value_type,
                         uint32_t bits, uint32_t policy, int32_t row_stride_bytes,
                         const uint8_t *packed, const float *col_scales,
                         const float *col_offsets, const float *row_offsets, const void *rhs,
                         int rhs_type, uint32_t n, uint64_t ldb, double *out,
                         double *magnitude) {
    if (rows < 0 || cols < 0 || block_size <= 0 || ell_cols < 0 || ell_cols % block_size != 0)
        return -1;
    if (packed != NULL && !valid_bits(bits)) return -1;
    const int32_t width = ell_cols / block_size;
    memset(out, 0, sizeof(double) * (uint64_t)rows * n);
    if (magnitude != NULL) memset(magnitude, 0, sizeof(double) * (uint64_t)rows * n);
    for (int32_t r = 0; r < rows; ++r) {
        const int32_t rb = r / block_size;
        for (int32_t slot = 0; slot < ell_cols; ++slot) {
            /* column_for_slot (quantized/blocked_ell.cuh:120-138) */
            const uint32_t bc = block_col_idx[(uint64_t)rb * width + slot / block_size];
            if (bc == 0xffffffffu) continue;
            const int64_t col = (int64_t)bc * block_size + slot % block_size;
            if (col >= cols) continue; /* padded tail of the last block column */
            double x;
            if (packed != NULL) {
                float scale, offset;
                metadata_for(policy, r, (int32_t)col, col_scales, col_offsets, row_offsets,
                             &scale, &offset);
                x = (double)or_dequantize_code(
                    or_unpack_code(bits, packed + (uint64_t)r * row_stride_bytes, slot), scale,
                    offset);
            } else {
                x = read_typed(values, value_type, (uint64_t)r * ell_cols + slot);
            }
            if (x == 0.0) continue;
            for (uint32_t c = 0; c < n; ++c) {
                const double w = read_typed(rhs, rhs_type, (uint64_t)col * ldb + c);
                out[(uint64_t)r * n + c] += x * w;
                if (magnitude != NULL) magnitude[(uint64_t)r * n + c] += fabs(x * w);
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* CP-BP feature-weighted row reduction                                        */
/* ------------------------------------------------------------------------- */

/* accumulate (components/CellPack/src/feature_weighted_row_reduction.cc:213-221):
 * product rounded to float, then added to a float accumulator. */
static void cpbp_accumulate(float *out, uint32_t row, uint32_t feature, float value,
                            const float *weights) {
    const float product = value * weights[feature];
    out[row] += product;
}

int or_cpbp_canonical(uint32_t rows, const uint32_t *row_offsets,
                      const uint32_t *canonical_features, const void *values, int value_type,
                      const float *weights, float *out) {
    if (value_type != OR_F16 && value_type != OR_F32) return -3;
    for (uint32_t r = 0; r < rows; ++r) out[r] = 0.0f;
    for (uint32_t r = 0; r < rows; ++r)
        for (uint32_t e = row_offsets[r]; e < row_offsets[r + 1]; ++e)
            cpbp_accumulate(out, r, canonical_features[e], read_typed_f(values, value_type, e),
                            weights);
    return 0;
}

int or_cpbp_canonical_f64(uint32_t rows, const uint32_t *row_offsets,
                          const uint32_t *canonical_features, const void *values,
                          int value_type, const float *weights, double *out,
                          double *magnitude) {
    if (value_type != OR_F16 && value_type != OR_F32) return -3;
    for (uint32_t r = 0; r < rows; ++r) {
        double s = 0.0, m = 0.0;
        for (uint32_t e = row_offsets[r]; e < row_offsets[r + 1]; ++e) {
            const double p = (double)read_typed_f(values, value_type, e)
                * (double)weights[canonical_features[e]];
            s += p;
            m += fabs(p);
        }
        out[r] = s;
        if (magnitude != NULL) magnitude[r] = m;
    }
    return 0;
}

/* evaluate_feature_weighted_row_reduction_tiles_host
 * (components/CellPack/src/feature_weighted_row_reduction.cc:358-402), generalised to
 * 64-lane tiles: mask_bits selects u32 or u64 cell masks. */
int or_cpbp_tiles(uint32_t row_count, uint32_t tile_count, uint32_t tile_row_width,
                  uint32_t mask_bits, const uint32_t *feature_block_offsets,
                  const uint32_t *feature_permutation, const uint32_t *tile_block_offsets,
                  const uint32_t *tile_block_ids, const void *tile_block_cell_masks,
                  const uint32_t *block_row_entry_offsets, const uint32_t *row_block_gene_masks,
                  const uint32_t *row_block_value_offsets, const void *values, int value_type,
                  const uint32_t *row_permutation, const float *weights, float *out) {
    if (value_type != OR_F16 && value_type != OR_F32) return -3;
    if ((mask_bits != 32u && mask_bits != 64u) || tile_row_width == 0u
        || tile_row_width > mask_bits)
        return -1;
    for (uint32_t r = 0; r < row_count; ++r) out[r] = 0.0f;
    for (uint32_t tile = 0; tile < tile_count; ++tile) {
        const uint32_t tile_begin = tile * tile_row_width;
        for (uint32_t d = tile_block_offsets[tile]; d < tile_block_offsets[tile + 1]; ++d) {
            const uint32_t block = tile_block_ids[d];
            const uint32_t block_begin = feature_block_offsets[block];
            const uint32_t block_width = feature_block_offsets[block + 1] - block_begin;
            const uint64_t cell_mask = mask_bits == 32u
                ? (uint64_t)((const uint32_t *)tile_block_cell_masks)[d]
                : ((const uint64_t *)tile_block_cell_masks)[d];
            uint32_t entry = block_row_entry_offsets[d];
            for (uint32_t lane = 0; lane < tile_row_width; ++lane) {
                if ((cell_mask & (1ull << lane)) == 0u) continue;
                const uint32_t row = row_permutation[tile_begin + lane];
                const uint32_t gene_mask = row_block_gene_masks[entry];
                uint32_t value = row_block_value_offsets[entry];
                for (uint32_t local = 0; local < block_width; ++local) {
                    if ((gene_mask & (1u << local)) == 0u) continue;
                    cpbp_accumulate(out, row, feature_permutation[block_begin + local],
                                    read_typed_f(values, value_type, value), weights);
                    ++value;
                }
                ++entry;
            }
        }
    }
    return 0;
}

/* feature_weighted_row_reduction_within_tolerance
 * (components/CellPack/src/feature_weighted_row_reduction.cc:225-241) */
int or_cpbp_within_tolerance(float reference, float candidate, double abs_tol,
                             double rel_tol) {
    if (abs_tol < 0.0 || rel_tol < 0.0 || isnan(reference) || isnan(candidate)) return 0;
    if (reference == candidate) return 1;
    const double rv = (double)reference, cv = (double)candidate;
    if (!isfinite(rv) || !isfinite(cv)) return 0;
    return fabs(cv - rv) <= abs_tol + rel_tol * fabs(rv);
}

/* csr_spmm_bwd_values_kernel_
 * (src/compute/sparse/ops/kernels/base_sparse/csr_spmm_bwd_values_kernel_.cuh:1-19) */
int or_spmm_bwd_values(uint32_t rows, const int32_t *row_ptr, const int32_t *col_idx,
                       const float *grad_out, uint64_t grad_out_ld, const void *rhs,
                       int rhs_type, uint64_t rhs_ld, uint64_t n, double *grad_values) {
    if (rows != 0u && (row_ptr == NULL || grad_out == NULL || rhs == NULL)) return -1;
    if (grad_out_ld < n || rhs_ld < n) return -2;
    for (uint32_t r = 0; r < rows; ++r) {
        const float *g = grad_out + (uint64_t)r * grad_out_ld;
        for (int32_t i = row_ptr[r]; i < row_ptr[r + 1]; ++i) {
            const uint64_t base = (uint64_t)col_idx[i] * rhs_ld;
            double acc = 0.0;
            for (uint64_t c = 0; c < n; ++c)
                acc += (double)g[c] * read_typed_f(rhs, rhs_type, base + c);
            grad_values[i] = acc;
        }
    }
    return 0;
}

/* ---- digest_logical_dense (include/Cellerator/compute/math/referee.hh:219-244) ---- */
static void or_digest_mix(uint64_t value, uint64_t d[2]) {
    /* referee_detail::digest_mix (referee.hh:125-130) */
    d[0] ^= value;
    d[0] *= 1099511628211ull;
    d[1] ^= value + 0x9e3779b97f4a7c15ull + (d[1] << 6u) + (d[1] >> 2u);
}

int or_digest_logical_dense(const void *values, uint64_t rows, uint64_t columns, uint64_t ld,
                            int column_major, uint32_t value_type, uint64_t digest[2]) {
    if (digest == NULL) return 1;
    if (rows != 0u && columns != 0u) {  /* referee_detail::valid_dense (referee.hh:94-101) */
        const uint64_t minimum = column_major ? rows : columns;
        if (values == NULL || ld < minimum) return 1;
    }
    uint64_t d[2] = {1469598103934665603ull, 0x6a09e667f3bcc909ull};
    or_digest_mix(rows, d);
    or_digest_mix(columns, d);
    or_digest_mix(value_type, d);
    for (uint64_t r = 0; r < rows; ++r) {
        for (uint64_t c = 0; c < columns; ++c) {
            const uint64_t at = column_major ? c * ld + r : r * ld + c;  /* dense_offset */
            double v;
            if (value_type == OR_F16) v = (double)or_half_to_float(((const uint16_t *)values)[at]);
            else if (value_type == OR_F32) v = (double)((const float *)values)[at];
            else if (value_type == OR_F64) v = ((const double *)values)[at];
            else return 3;
            uint64_t bits;
            memcpy(&bits, &v, sizeof bits);
            or_digest_mix(bits, d);
        }
    }
    digest[0] = d[0];
    digest[1] = d[1];
    return 0;
}
