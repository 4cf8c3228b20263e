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
                const float x = fmaf((float)code, scale, offset);
                const __m256 xv = _mm256_set1_ps(x);
                uint32_t c = 0;
                if (job->rhs_type == OR_F16) {
                    const uint16_t *w = (const uint16_t *)job->rhs + (uint64_t)col * job->ldb;
                    for (; c + 8 <= n; c += 8) {
                        const __m256 wv = _mm256_cvtph_ps(
                            _mm_loadu_si128((const __m128i *)(w + c)));
                        _mm256_storeu_ps(orow + c,
                                         _mm256_fmadd_ps(xv, wv, _mm256_loadu_ps(orow + c)));
                    }
                    for (; c < n; ++c) orow[c] = fmaf(x, or_half_to_float(w[c]), orow[c]);
                } else {
                    const float *w = (const float *)job->rhs + (uint64_t)col * job->ldb;
                    for (; c + 8 <= n; c += 8)
                        _mm256_storeu_ps(orow + c, _mm256_fmadd_ps(xv, _mm256_loadu_ps(w + c),
                                                                   _mm256_loadu_ps(orow + c)));
                    for (; c < n; ++c) orow[c] = fmaf(x, w[c], orow[c]);
                }
            }
        }
    }
    return NULL;
}

int or_qcsr_spmm_f32_mt(uint32_t bits, uint32_t policy, int32_t rows, int32_t cols,
                        const int32_t *row_ptr, const int32_t *packed_row_ptr,
                        const int32_t *col_idx, const uint8_t *packed,
                        const float *col_scales, const float *col_offsets,
                        const float *row_offsets, const void *rhs, int rhs_type, uint32_t n,
                        uint64_t ldb, int32_t row_begin, int32_t row_end, float *out,
                        int threads) {
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
