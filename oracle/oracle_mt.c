/*
 * oracle_mt.c -- row-parallel fp32 quantized CSR SpMM on the host: the CPU baseline
 * that bench.py times beside the GPU kernel (TEST INFRASTRUCTURE, see oracle.h).
 *
 * Semantics: decode each code with dequantize_code
 * (include/Cellerator/quantized/access.cuh:81-91, one fmaf), widen the fp16 weight
 * exactly, multiply and accumulate in fp32 in nnz order per output column (the
 * per-(row, col) sum of csr_spmm_fwd_kernel_,
 * src/compute/sparse/project/kernels/csr_spmm_fwd_kernel_.cuh:13-19, which nvcc
 * contracts to FMAs). Built with AVX2/FMA/F16C so the baseline is a fair vectorised
 * host implementation rather than a scalar strawman.
 */
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>

typedef struct qcsr_mt_job {
    uint32_t bits, policy;
    int32_t cols;
    const int32_t *row_ptr, *packed_row_ptr, *col_idx;
    const uint8_t *packed;
    const float *col_scales, *col_offsets, *row_offsets;
    const void *rhs;
    int rhs_type;
    uint32_t n;
    uint64_t ldb;
    int32_t row_begin, row_end;
    float *out;
    int magnitude;  /* accumulate |x| * |w| instead: the Sigma |x||w| term of the tolerance */
    _Atomic int32_t next;
    _Atomic int failed;
} qcsr_mt_job;

static void *qcsr_mt_worker(void *arg) {
    qcsr_mt_job *job = (qcsr_mt_job *)arg;
    const int32_t chunk = 16;
    const uint32_t cpb = 8u / job->bits;
    const uint32_t mask = (1u << job->bits) - 1u;
    const uint32_t n = job->n;
    for (;;) {
        const int32_t start = atomic_fetch_add(&job->next, chunk);
        if (start >= job->row_end) break;
        const int32_t stop = start + chunk < job->row_end ? start + chunk : job->row_end;
        for (int32_t r = start; r < stop; ++r) {
            float *orow = job->out + (uint64_t)(r - job->row_begin) * n;
            for (uint32_t c = 0; c < n; ++c) orow[c] = 0.0f;
            const uint8_t *base = job->packed + job->packed_row_ptr[r];
            const int64_t begin = job->row_ptr[r];
            const float row_offset = job->policy == OR_POLICY_COLUMN_SCALE_ROW_OFFSET
                ? (job->row_offsets != NULL ? job->row_offsets[r] : 0.0f) : 0.0f;
            for (int64_t i = begin; i < job->row_ptr[r + 1]; ++i) {
                const int32_t col = job->col_idx[i];
                if (col < 0 || col >= job->cols) {
                    atomic_store(&job->failed, 1);
                    continue;
                }
                const int64_t local = i - begin;
                const uint32_t code = ((uint32_t)base[local / cpb] >> ((local % cpb) * job->bits))
                    & mask;
                const float scale = job->col_scales != NULL ? job->col_scales[col] : 1.0f;
                const float offset = job->policy == OR_POLICY_COLUMN_SCALE_ROW_OFFSET
                    ? row_offset
                    : (job->col_offsets != NULL ? job->col_offsets[col] : 0.0f);
                const float xd = fmaf((float)code, scale, offset);
                const float x = job->magnitude ? fabsf(xd) : xd;
                const __m256 xv = _mm256_set1_ps(x);
                const __m256 sign = _mm256_set1_ps(job->magnitude ? -0.0f : 0.0f);
                uint32_t c = 0;
                if (job->rhs_type == OR_F16) {
                    const uint16_t *w = (const uint16_t *)job->rhs + (uint64_t)col * job->ldb;
                    for (; c + 8 <= n; c += 8) {
                        const __m256 wv = _mm256_andnot_ps(sign, _mm256_cvtph_ps(
                            _mm_loadu_si128((const __m128i *)(w + c))));
                        _mm256_storeu_ps(orow + c,
                                         _mm256_fmadd_ps(xv, wv, _mm256_loadu_ps(orow + c)));
                    }
                    for (; c < n; ++c) {
                        const float wc = or_half_to_float(w[c]);
                        orow[c] = fmaf(x, job->magnitude ? fabsf(wc) : wc, orow[c]);
                    }
                } else {
                    const float *w = (const float *)job->rhs + (uint64_t)col * job->ldb;
                    for (; c + 8 <= n; c += 8)
                        _mm256_storeu_ps(orow + c,
                                         _mm256_fmadd_ps(xv, _mm256_andnot_ps(sign, _mm256_loadu_ps(w + c)),
                                                         _mm256_loadu_ps(orow + c)));
                    for (; c < n; ++c) orow[c] = fmaf(x, job->magnitude ? fabsf(w[c]) : w[c], orow[c]);
                }
            }
        }
    }
    return NULL;
}

static int qcsr_mt_run(uint32_t bits, uint32_t policy, int32_t rows, int32_t cols,
                       const int32_t *row_ptr, const int32_t *packed_row_ptr,
                       const int32_t *col_idx, const uint8_t *packed,
                       const float *col_scales, const float *col_offsets,
                       const float *row_offsets, const void *rhs, int rhs_type, uint32_t n,
                       uint64_t ldb, int32_t row_begin, int32_t row_end, float *out,
                       int threads, int magnitude);

int or_qcsr_spmm_f32_mt(uint32_t bits, uint32_t policy, int32_t rows, int32_t cols,
                        const int32_t *row_ptr, const int32_t *packed_row_ptr,
                        const int32_t *col_idx, const uint8_t *packed,
                        const float *col_scales, const float *col_offsets,
                        const float *row_offsets, const void *rhs, int rhs_type, uint32_t n,
                        uint64_t ldb, int32_t row_begin, int32_t row_end, float *out,
                        int threads) {
    return qcsr_mt_run(bits, policy, rows, cols, row_ptr, packed_row_ptr, col_idx, packed,
                       col_scales, col_offsets, row_offsets, rhs, rhs_type, n, ldb, row_begin,
                       row_end, out, threads, 0);
}

int or_qcsr_spmm_f32_mt_magnitude(uint32_t bits, uint32_t policy, int32_t rows, int32_t cols,
                                  const int32_t *row_ptr, const int32_t *packed_row_ptr,
                                  const int32_t *col_idx, const uint8_t *packed,
                                  const float *col_scales, const float *col_offsets,
                                  const float *row_offsets, const void *rhs, int rhs_type,
                                  uint32_t n, uint64_t ldb, int32_t row_begin, int32_t row_end,
                                  float *out, int threads) {
    return qcsr_mt_run(bits, policy, rows, cols, row_ptr, packed_row_ptr, col_idx, packed,
                       col_scales, col_offsets, row_offsets, rhs, rhs_type, n, ldb, row_begin,
                       row_end, out, threads, 1);
}

static int qcsr_mt_run(uint32_t bits, uint32_t policy, int32_t rows, int32_t cols,
                       const int32_t *row_ptr, const int32_t *packed_row_ptr,
                       const int32_t *col_idx, const uint8_t *packed,
                       const float *col_scales, const float *col_offsets,
                       const float *row_offsets, const void *rhs, int rhs_type, uint32_t n,
                       uint64_t ldb, int32_t row_begin, int32_t row_end, float *out,
                       int threads, int magnitude) {
    if (!(bits == 1u || bits == 2u || bits == 4u || bits == 8u) || row_begin < 0
        || row_end > rows || row_begin > row_end)
        return -1;
    if (rhs_type != OR_F32 && rhs_type != OR_F16) return -3;
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    qcsr_mt_job job;
    job.bits = bits;
    job.policy = policy;
    job.cols = cols;
    job.row_ptr = row_ptr;
    job.packed_row_ptr = packed_row_ptr;
    job.col_idx = col_idx;
    job.packed = packed;
    job.col_scales = col_scales;
    job.col_offsets = col_offsets;
    job.row_offsets = row_offsets;
    job.rhs = rhs;
    job.rhs_type = rhs_type;
    job.n = n;
    job.ldb = ldb;
    job.row_begin = row_begin;
    job.row_end = row_end;
    job.out = out;
    job.magnitude = magnitude;
    atomic_init(&job.next, row_begin);
    atomic_init(&job.failed, 0);
    pthread_t tids[256];
    int started = 0;
    for (int t = 0; t < threads; ++t) {
        if (pthread_create(&tids[t], NULL, qcsr_mt_worker, &job) != 0) break;
        ++started;
    }
    if (started == 0) qcsr_mt_worker(&job);
    for (int t = 0; t < started; ++t) pthread_join(tids[t], NULL);
    return atomic_load(&job.failed) ? -2 : 0;
}

/* ---- CP-BP canonical referee, row-parallel ---------------------------------------------
 * Each row exactly as or_cpbp_canonical (components/CellPack/src/feature_weighted_row_reduction.cc:213-221,
 * 293-319): product rounded to float, added to the row's float accumulator in CSR order.
 * Rows are independent, so the result is bitwise equal to the single-thread referee. */
typedef struct cpbp_mt_job {
    const uint32_t *row_offsets, *features;
    const void *values;
    int value_type;
    const float *weights;
    float *out;
    uint32_t rows;
    _Atomic uint32_t next;
} cpbp_mt_job;

static void *cpbp_mt_worker(void *arg) {
    cpbp_mt_job *job = (cpbp_mt_job *)arg;
    const uint32_t chunk = 256;
    for (;;) {
        const uint32_t start = atomic_fetch_add(&job->next, chunk);
        if (start >= job->rows) break;
        const uint32_t stop = start + chunk < job->rows ? start + chunk : job->rows;
        for (uint32_t r = start; r < stop; ++r) {
            float acc = 0.0f;
            for (uint32_t e = job->row_offsets[r]; e < job->row_offsets[r + 1]; ++e) {
                const float v = job->value_type == OR_F16
                    ? or_half_to_float(((const uint16_t *)job->values)[e])
                    : ((const float *)job->values)[e];
                const float product = v * job->weights[job->features[e]];
                acc += product;
            }
            job->out[r] = acc;
        }
    }
    return NULL;
}

int or_cpbp_canonical_mt(uint32_t rows, const uint32_t *row_offsets,
                         const uint32_t *canonical_features, const void *values, int value_type,
                         const float *weights, float *out, int threads) {
    if (value_type != OR_F16 && value_type != OR_F32) return -3;
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    cpbp_mt_job job;
    job.row_offsets = row_offsets;
    job.features = canonical_features;
    job.values = values;
    job.value_type = value_type;
    job.weights = weights;
    job.out = out;
    job.rows = rows;
    atomic_init(&job.next, 0u);
    pthread_t tids[256];
    int started = 0;
    for (int t = 0; t < threads; ++t) {
        if (pthread_create(&tids[t], NULL, cpbp_mt_worker, &job) != 0) break;
        ++started;
    }
    if (started == 0) cpbp_mt_worker(&job);
    for (int t = 0; t < started; ++t) pthread_join(tids[t], NULL);
    return 0;
}

/* ---- Blocked-ELL SpMM, row-block-parallel ----------------------------------------------
 * bf16 values x bf16 weights -> fp32, the semantics of blocked_ell_spmm_fwd_kernel_
 * (src/compute/sparse/project/kernels/blocked_ell_spmm_fwd_kernel_.cuh:1-33): per output
 * element, fp32 accumulation over the row's ELL slots in slot order (0xffffffff = empty),
 * each product exact (bf16 x bf16 fits in fp32) and added with one fmaf. Vectorised over
 * the output columns (AVX2/FMA). */
typedef struct bell_mt_job {
    int32_t rows, cols, block_size, ell_cols;
    const uint32_t *block_col_idx;
    const uint16_t *values, *rhs;
    uint32_t n;
    float *out;
    _Atomic int32_t next;
} bell_mt_job;

static inline __m256 bf16x8_to_ps(const uint16_t *p) {
    const __m128i h = _mm_loadu_si128((const __m128i *)p);
    return _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(h), 16));
}

static void *bell_mt_worker(void *arg) {
    bell_mt_job *job = (bell_mt_job *)arg;
    const int32_t bs = job->block_size;
    const int32_t slots = job->ell_cols / bs;
    const int32_t row_blocks = (job->rows + bs - 1) / bs;
    const uint32_t n = job->n;
    for (;;) {
        const int32_t rb = atomic_fetch_add(&job->next, 1);
        if (rb >= row_blocks) break;
        for (int32_t r = rb * bs; r < job->rows && r < (rb + 1) * bs; ++r) {
            float *orow = job->out + (uint64_t)r * n;
            for (uint32_t c = 0; c < n; ++c) orow[c] = 0.0f;
            for (int32_t s = 0; s < slots; ++s) {
                const uint32_t bc = job->block_col_idx[(uint64_t)rb * slots + s];
                if (bc == 0xffffffffu) continue;
                for (int32_t k = 0; k < bs; ++k) {
                    const int64_t col = (int64_t)bc * bs + k;
                    if (col >= job->cols) continue;
                    const uint16_t vb = job->values[(uint64_t)r * job->ell_cols + (uint64_t)s * bs + k];
                    union { uint32_t u; float f; } cv;
                    cv.u = (uint32_t)vb << 16;
                    if (cv.f == 0.0f) continue;
                    const __m256 xv = _mm256_set1_ps(cv.f);
                    const uint16_t *w = job->rhs + (uint64_t)col * n;
                    uint32_t c = 0;
                    for (; c + 8 <= n; c += 8)
                        _mm256_storeu_ps(orow + c, _mm256_fmadd_ps(xv, bf16x8_to_ps(w + c),
                                                                   _mm256_loadu_ps(orow + c)));
                    for (; c < n; ++c) {
                        union { uint32_t u; float f; } wv;
                        wv.u = (uint32_t)w[c] << 16;
                        orow[c] = fmaf(cv.f, wv.f, orow[c]);
                    }
                }
            }
        }
    }
    return NULL;
}

int or_bell_spmm_bf16_mt(int32_t rows, int32_t cols, int32_t block_size, int32_t ell_cols,
                         const uint32_t *block_col_idx, const uint16_t *values,
                         const uint16_t *rhs, uint32_t n, float *out, int threads) {
    if (rows < 0 || cols <= 0 || block_size <= 0 || ell_cols % block_size != 0) return -1;
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    bell_mt_job job;
    job.rows = rows;
    job.cols = cols;
    job.block_size = block_size;
    job.ell_cols = ell_cols;
    job.block_col_idx = block_col_idx;
    job.values = values;
    job.rhs = rhs;
    job.n = n;
    job.out = out;
    atomic_init(&job.next, 0);
    pthread_t tids[256];
    int started = 0;
    for (int t = 0; t < threads; ++t) {
        if (pthread_create(&tids[t], NULL, bell_mt_worker, &job) != 0) break;
        ++started;
    }
    if (started == 0) bell_mt_worker(&job);
    for (int t = 0; t < started; ++t) pthread_join(tids[t], NULL);
    return 0;
}
