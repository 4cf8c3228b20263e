/*
 * cellerator_amd_synth.h -- seeded synthetic single-cell inputs generated on the GPU
 * (libcx_synth.so). Bench and test support only: the engine (libcellerator_amd.so)
 * does not depend on it. Every draw is a counter-based hash of (seed, row, gene), so a
 * matrix is a pure function of its parameters and independent of launch shape.
 *
 * Quantized CSR recipe:
 *   row size  : LogNormal(arithmetic mean, sigma) or Poisson(mean), clipped, rounded;
 *   genes     : Poisson sampling without replacement, gene g kept with probability
 *               min(1, c_r * rank(g)^-s) (Zipf exponent s over a seeded permutation of
 *               the genes; s = 0 is uniform), c_r solved per row so the expected row
 *               size equals the drawn target; columns come out sorted ascending;
 *   values    : count = 1 + NB(mean, size r) (stored entries are never zero),
 *               value = fp32(log1p(count));
 *   codec     : per-gene min/max calibration, offset = min, scale = max((max-min) /
 *               (2^bits-1), 1e-6), codes by the portable encode rule, packed low bits
 *               first with unpadded byte-granular rows.
 */
#ifndef CELLERATOR_AMD_SYNTH_H
#define CELLERATOR_AMD_SYNTH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct cxs_qcsr_params {
    uint64_t seed;
    uint32_t rows;
    uint32_t cols;
    uint32_t row_dist; /* 0 = lognormal(nnz_mean, nnz_sigma), 1 = poisson(nnz_mean) */
    uint32_t bits;     /* 1, 2, 4, 8: packed codes; 0: fp32 values */
    double nnz_mean;
    double nnz_sigma;
    uint32_t nnz_min;
    uint32_t nnz_max;
    double zipf_s;
    double nb_mean;
    double nb_size;
} cxs_qcsr_params;

typedef struct cxs_generator cxs_generator;

/* Builds the host tables (gene popularity, row targets' solver prefix sums, NB CDF,
 * log1p table) and uploads them; allocates only the generator's own tables. */
int cxs_qcsr_create(const cxs_qcsr_params *params, cxs_generator **out);
void cxs_destroy(cxs_generator *gen);

/* Pass 1: row_nnz[rows] (int32) = realised size of every row. */
int cxs_qcsr_count(cxs_generator *gen, int32_t *row_nnz, void *stream);
/* Pass 2: col_idx for every row (row_ptr = exclusive scan of row_nnz), and the per-gene
 * minimum / maximum count (gene_min initialised to 0xffffffff, gene_max to 0). */
int cxs_qcsr_fill(cxs_generator *gen, const int32_t *row_ptr, int32_t *col_idx,
                  uint32_t *gene_min, uint32_t *gene_max, void *stream);
/* Pass 3: per-gene scale / offset from the calibration counts. */
int cxs_qcsr_calibrate(cxs_generator *gen, const uint32_t *gene_min, const uint32_t *gene_max,
                       float *scales, float *offsets, void *stream);
/* Pass 4: packed codes (bits != 0; packed_row_ptr as build_packed_row_ptr) or fp32
 * values (bits == 0; scales/offsets/packed_row_ptr ignored). */
int cxs_qcsr_encode(cxs_generator *gen, const int32_t *row_ptr, const int32_t *packed_row_ptr,
                    const int32_t *col_idx, const float *scales, const float *offsets,
                    uint8_t *packed, float *values, void *stream);

/* count i.i.d. N(0, stddev) values (dtype 1 = f16, 2 = f32, 5 = bf16, RNE narrowing). */
int cxs_dense_normal(uint64_t seed, uint64_t count, float stddev, uint32_t dtype, void *out,
                     void *stream);

/* Blocked-ELL recipe: row block b takes module pattern
 * p ~ U{0..patterns-1} and c ~ U{min_blocks..max_blocks}; the pattern is a seeded list
 * of max_blocks distinct block columns; the row block uses its first c, sorted
 * ascending, padded to ell_width with 0xffffffff. Each element of a valid block is
 * non-zero with probability `density`, value log1p(1 + NB(mean, size)). Values bf16,
 * row-major rows x (ell_width * block_size); padded slots are zero. */
int cxs_bell_generate(uint64_t seed, uint32_t rows, uint32_t cols, uint32_t block_size,
                      uint32_t ell_width, uint32_t patterns, uint32_t min_blocks,
                      uint32_t max_blocks, float density, double nb_mean, double nb_size,
                      uint32_t *block_col_idx, uint16_t *values_bf16, void *stream);

/* CP-BP structured-support matrix, generated on `threads` host threads
 * (identical output for any count). Row r activates k ~ U{min_active..max_active} distinct
 * modules (module m = genes [m*module_size, (m+1)*module_size)), takes active_genes of each
 * without replacement, adds `background` genes uniform over the axis excluding genes already
 * present, sorts; value = log1p(1 + NB(nb_mean, nb_size)) fp32. Pass 1 gives row sizes,
 * pass 2 fills canonical features and values at the caller's exclusive-scan offsets. */
typedef struct cxs_cpbp_params {
    uint64_t seed;
    uint32_t rows;
    uint32_t genes;
    uint32_t modules;
    uint32_t module_size;
    uint32_t min_active;
    uint32_t max_active;
    uint32_t active_genes;
    uint32_t background;
    double nb_mean;
    double nb_size;
} cxs_cpbp_params;

int cxs_cpbp_count(const cxs_cpbp_params *params, uint32_t *row_nnz, uint32_t threads);
int cxs_cpbp_fill(const cxs_cpbp_params *params, const uint32_t *row_offsets, uint32_t *features,
                  float *values, uint32_t threads);

const char *cxs_last_error(void);

#ifdef __cplusplus
}
#endif

#endif
