// synth.hip -- seeded synthetic single-cell matrices generated directly in HBM
// (bench/test support; see include/cellerator_amd_synth.h for the recipe).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <vector>
#include <thread>
#include <atomic>

#include "cellerator_amd_synth.h"

namespace {

thread_local char g_error[512];

int fail(const char *fmt, ...) {
    va_list args;
    va_start(args, fmt);
    std::vsnprintf(g_error, sizeof(g_error), fmt, args);
    va_end(args);
    return 1;
}

int hip_check(hipError_t status, const char *what) {
    if (status == hipSuccess) return 0;
    return fail("%s: %s", what, hipGetErrorString(status));
}

constexpr int kWave = 64;
constexpr int kCountMax = 4095; // NB tail beyond this is clamped (mass < 1e-12 here)

__host__ __device__ inline std::uint64_t splitmix64(std::uint64_t x) {
    x += 0x9e3779b97f4a7c15ull;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
    return x ^ (x >> 31);
}

__host__ __device__ inline std::uint32_t lowbias32(std::uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// Independent streams of one seed.
enum Stream : std::uint64_t {
    kTarget = 1, kInclude = 2, kCount = 3, kPerm = 4, kDense = 5, kBellRow = 6,
    kBellValue = 7, kBellPattern = 8, kCpbpRow = 9, kCpbpValue = 10
};

__host__ __device__ inline std::uint64_t stream_base(std::uint64_t seed, std::uint64_t stream) {
    return splitmix64(seed ^ (stream * 0xd1b54a32d192ed03ull));
}

__device__ inline std::uint32_t pair_hash(std::uint64_t row_key, std::uint32_t gene) {
    return lowbias32(static_cast<std::uint32_t>(row_key)
                     ^ lowbias32(gene + static_cast<std::uint32_t>(row_key >> 32)));
}

__device__ inline double unit_open(std::uint64_t h) {
    return (static_cast<double>(h >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

// Smallest k with u < cdf[k] (cdf scaled to 2^32), i.e. an NB(mean, size) draw.
__device__ inline int nb_draw(const std::uint32_t *cdf, std::uint32_t u) {
    int lo = 0, hi = kCountMax;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (u < cdf[mid]) hi = mid;
        else lo = mid + 1;
    }
    return lo;
}

// Portable encode rule (include/Cellerator/quantized/access.cuh:104-131): IEEE divide,
// round half away from zero, clamp.
__device__ inline unsigned quantize(float value, float scale, float offset, int bits) {
    const float centered = value - offset;
    if (scale == 0.0f) return 0u;
    const float q = centered / scale;
    const int rounded = q >= 0.0f ? static_cast<int>(q + 0.5f) : static_cast<int>(q - 0.5f);
    const int max_code = (1 << bits) - 1;
    if (rounded < 0) return 0u;
    return static_cast<unsigned>(rounded > max_code ? max_code : rounded);
}

struct Device {
    float *gene_weight = nullptr;   // cols: rank(g)^-s
    double *rank_prefix = nullptr;  // cols + 1: sum_{k<=m} k^-s
    std::uint32_t *nb_cdf = nullptr;
    float *log1p_lut = nullptr;     // kCountMax + 2
    float *row_c = nullptr;         // rows
};

} // namespace

struct cxs_generator {
    cxs_qcsr_params p{};
    Device d{};
    bool targets_ready = false;
};

namespace {

__global__ void k_row_targets(cxs_qcsr_params p, const double *prefix, float *row_c) {
    const std::uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= p.rows) return;
    const std::uint64_t h1 = splitmix64(stream_base(p.seed, kTarget) + r);
    const std::uint64_t h2 = splitmix64(h1);
    double target;
    if (p.row_dist == 0u) {
        const double z = sqrt(-2.0 * log(unit_open(h1))) * cos(6.283185307179586 * unit_open(h2));
        const double mu = log(p.nnz_mean) - 0.5 * p.nnz_sigma * p.nnz_sigma;
        target = exp(mu + p.nnz_sigma * z);
    } else {
        // exact Poisson inversion (mean up to a few thousand)
        const double u = unit_open(h1);
        double prob = exp(-p.nnz_mean), cdf = prob;
        int k = 0;
        while (u > cdf && k < 100000) {
            ++k;
            prob *= p.nnz_mean / k;
            cdf += prob;
        }
        target = k;
    }
    const double hi = fmin(static_cast<double>(p.nnz_max), static_cast<double>(p.cols));
    target = fmin(fmax(rint(target), static_cast<double>(p.nnz_min)), hi);
    double c;
    if (p.zipf_s == 0.0) {
        c = target / p.cols;
    } else {
        // F(c) = m + c (H_K - H_m), m = #genes with c k^-s >= 1; monotone in c.
        double lo = 0.0, up = pow(static_cast<double>(p.cols), p.zipf_s);
        for (int it = 0; it < 64; ++it) {
            const double mid = 0.5 * (lo + up);
            double mf = floor(pow(mid, 1.0 / p.zipf_s));
            const std::uint32_t m = mf >= p.cols ? p.cols : static_cast<std::uint32_t>(mf);
            const double f = m + mid * (prefix[p.cols] - prefix[m]);
            if (f < target) lo = mid;
            else up = mid;
        }
        c = 0.5 * (lo + up);
    }
    row_c[r] = static_cast<float>(c);
}

__device__ inline bool included(float c, float weight, std::uint32_t h) {
    const float p = c * weight;
    if (p >= 1.0f) return true;
    const float t = fminf(p * 4294967296.0f, 4294967040.0f);
    return h < static_cast<std::uint32_t>(t);
}

__global__ __launch_bounds__(256) void k_count(cxs_qcsr_params p, const float *gene_weight,
                                               const float *row_c, std::int32_t *row_nnz) {
    const int lane = threadIdx.x % kWave;
    const std::uint32_t r = (blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    if (r >= p.rows) return;
    const float c = row_c[r];
    const std::uint64_t key = splitmix64(stream_base(p.seed, kInclude) + r);
    int count = 0;
    for (std::uint32_t g0 = 0; g0 < p.cols; g0 += kWave) {
        const std::uint32_t g = g0 + lane;
        const bool inc = g < p.cols && included(c, gene_weight[g], pair_hash(key, g));
        count += __popcll(__ballot(inc));
    }
    if (lane == 0) row_nnz[r] = count;
}

__global__ __launch_bounds__(256) void k_fill(cxs_qcsr_params p, const float *gene_weight,
                                              const float *row_c, const std::uint32_t *nb_cdf,
                                              const std::int32_t *row_ptr, std::int32_t *col_idx,
                                              std::uint32_t *gene_min, std::uint32_t *gene_max) {
    const int lane = threadIdx.x % kWave;
    const std::uint32_t r = (blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    if (r >= p.rows) return;
    const float c = row_c[r];
    const std::uint64_t key = splitmix64(stream_base(p.seed, kInclude) + r);
    const std::uint64_t ckey = splitmix64(stream_base(p.seed, kCount) + r);
    std::int64_t out = row_ptr[r];
    const std::int64_t end = row_ptr[r + 1];
    for (std::uint32_t g0 = 0; g0 < p.cols; g0 += kWave) {
        const std::uint32_t g = g0 + lane;
        const bool inc = g < p.cols && included(c, gene_weight[g], pair_hash(key, g));
        const std::uint64_t mask = __ballot(inc);
        if (inc) {
            const std::uint64_t below = lane == 0 ? 0ull : (mask & ((1ull << lane) - 1ull));
            const std::int64_t slot = out + __popcll(below);
            if (slot < end) col_idx[slot] = static_cast<std::int32_t>(g);
            const std::uint32_t count = 1u + nb_draw(nb_cdf, pair_hash(ckey, g));
            if (count < gene_min[g]) atomicMin(&gene_min[g], count);
            if (count > gene_max[g]) atomicMax(&gene_max[g], count);
        }
        out += __popcll(mask);
    }
}

__global__ void k_calibrate(std::uint32_t cols, int bits, const float *lut,
                            const std::uint32_t *gene_min, const std::uint32_t *gene_max,
                            float *scales, float *offsets) {
    const std::uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= cols) return;
    if (gene_min[g] > gene_max[g]) { // gene never sampled
        scales[g] = 1.0f;
        offsets[g] = 0.0f;
        return;
    }
    const float lo = lut[gene_min[g]], hi = lut[gene_max[g]];
    const float qmax = static_cast<float>((1 << bits) - 1);
    offsets[g] = lo;
    scales[g] = fmaxf((hi - lo) / qmax, 1.0e-6f);
}

__global__ __launch_bounds__(256) void k_encode(cxs_qcsr_params p, const std::uint32_t *nb_cdf,
                                                const float *lut, const std::int32_t *row_ptr,
                                                const std::int32_t *packed_row_ptr,
                                                const std::int32_t *col_idx, const float *scales,
                                                const float *offsets, std::uint8_t *packed,
                                                float *values) {
    const int lane = threadIdx.x % kWave;
    const std::uint32_t r = (blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    if (r >= p.rows) return;
    const std::uint64_t ckey = splitmix64(stream_base(p.seed, kCount) + r);
    const std::int64_t begin = row_ptr[r], end = row_ptr[r + 1];
    const int bits = static_cast<int>(p.bits);
    const int cpb = bits > 0 ? 8 / bits : 1;
    for (std::int64_t c0 = begin; c0 < end; c0 += kWave) {
        const std::int64_t i = c0 + lane;
        unsigned code = 0u;
        if (i < end) {
            const std::uint32_t g = static_cast<std::uint32_t>(col_idx[i]);
            const float v = lut[1 + nb_draw(nb_cdf, pair_hash(ckey, g))];
            if (bits == 0) values[i] = v;
            else code = quantize(v, scales[g], offsets[g], bits);
        }
        if (bits == 0) continue;
        unsigned byte = 0u;
        for (int t = 0; t < cpb; ++t) {
            const unsigned other = __shfl_down(code, t, kWave);
            byte |= (other & ((1u << bits) - 1u)) << (t * bits);
        }
        const std::int64_t local = i - begin;
        if (i < end && local % cpb == 0) packed[packed_row_ptr[r] + local / cpb] =
            static_cast<std::uint8_t>(byte);
    }
}

__global__ void k_dense_normal(std::uint64_t base, std::uint64_t count, float stddev,
                               std::uint32_t dtype, void *out) {
    const std::uint64_t pair = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x;
    const std::uint64_t i0 = pair * 2;
    if (i0 >= count) return;
    const std::uint64_t h1 = splitmix64(base + pair);
    const std::uint64_t h2 = splitmix64(h1 ^ 0x5851f42d4c957f2dull);
    const double rad = sqrt(-2.0 * log(unit_open(h1)));
    const double ang = 6.283185307179586 * unit_open(h2);
    const float v[2] = {static_cast<float>(rad * cos(ang) * stddev),
                        static_cast<float>(rad * sin(ang) * stddev)};
    for (int k = 0; k < 2 && i0 + k < count; ++k) {
        const std::uint64_t i = i0 + k;
        if (dtype == 2u) {
            static_cast<float *>(out)[i] = v[k];
        } else if (dtype == 1u) {
            const _Float16 h = static_cast<_Float16>(v[k]);
            std::uint16_t b;
            __builtin_memcpy(&b, &h, 2);
            static_cast<std::uint16_t *>(out)[i] = b;
        } else {
            std::uint32_t x = __float_as_uint(v[k]);
            x += 0x7fffu + ((x >> 16) & 1u);
            static_cast<std::uint16_t *>(out)[i] = static_cast<std::uint16_t>(x >> 16);
        }
    }
}

__global__ __launch_bounds__(256) void k_bell(std::uint64_t seed, std::uint32_t rows,
                                              std::uint32_t cols, std::uint32_t bs,
                                              std::uint32_t ell_width, std::uint32_t patterns,
                                              std::uint32_t min_blocks, std::uint32_t max_blocks,
                                              float density, const std::uint32_t *pattern_cols,
                                              const std::uint32_t *nb_cdf, const float *lut,
                                              std::uint32_t *block_col_idx,
                                              std::uint16_t *values) {
    __shared__ std::uint32_t slot_col[256];
    const std::uint32_t b = blockIdx.x;
    const std::uint64_t h = splitmix64(stream_base(seed, kBellRow) + b);
    const std::uint32_t p = static_cast<std::uint32_t>(h % patterns);
    const std::uint32_t c = min_blocks
        + static_cast<std::uint32_t>((h >> 32) % (max_blocks - min_blocks + 1));
    const std::uint32_t *list = pattern_cols + static_cast<std::uint64_t>(p) * max_blocks;
    for (std::uint32_t t = threadIdx.x; t < c; t += blockDim.x) {
        // rank of list[t] among the first c entries -> ascending slot order
        const std::uint32_t mine = list[t];
        std::uint32_t rank = 0;
        for (std::uint32_t u = 0; u < c; ++u) rank += list[u] < mine ? 1u : 0u;
        slot_col[rank] = mine;
    }
    __syncthreads();
    for (std::uint32_t t = threadIdx.x; t < ell_width; t += blockDim.x)
        block_col_idx[static_cast<std::uint64_t>(b) * ell_width + t] =
            t < c ? slot_col[t] : 0xffffffffu;
    const std::uint64_t ell_cols = static_cast<std::uint64_t>(ell_width) * bs;
    const std::uint64_t vbase = stream_base(seed, kBellValue);
    const std::uint32_t threshold = static_cast<std::uint32_t>(fminf(density, 1.0f) * 4294967040.0f);
    const std::uint64_t elems = static_cast<std::uint64_t>(bs) * ell_cols;
    for (std::uint64_t e = threadIdx.x; e < elems; e += blockDim.x) {
        const std::uint32_t rr = static_cast<std::uint32_t>(e / ell_cols);
        const std::uint32_t slot = static_cast<std::uint32_t>(e % ell_cols);
        const std::uint32_t sb = slot / bs;
        const std::uint64_t row = static_cast<std::uint64_t>(b) * bs + rr;
        if (row >= rows) break;
        std::uint16_t out = 0;
        if (sb < c) {
            const std::uint64_t col = static_cast<std::uint64_t>(slot_col[sb]) * bs + slot % bs;
            if (col < cols) {
                const std::uint64_t key = splitmix64(vbase + row);
                const std::uint32_t hv = pair_hash(key, static_cast<std::uint32_t>(col));
                if (hv < threshold) {
                    const std::uint32_t hc = lowbias32(hv ^ 0x68e31da4u);
                    const float v = lut[1 + nb_draw(nb_cdf, hc)];
                    std::uint32_t x = __float_as_uint(v);
                    x += 0x7fffu + ((x >> 16) & 1u);
                    out = static_cast<std::uint16_t>(x >> 16);
                }
            }
        }
        values[row * ell_cols + slot] = out;
    }
}

// NB(mean, size) CDF for k = 0..kCountMax scaled to 2^32 (host, float64).
std::vector<std::uint32_t> nb_cdf_table(double mean, double size) {
    std::vector<std::uint32_t> out(kCountMax + 1);
    const double q = mean / (size + mean);
    double logp = size * std::log(size / (size + mean)); // P(0)
    double cdf = 0.0;
    for (int k = 0; k <= kCountMax; ++k) {
        cdf += std::exp(logp);
        const double scaled = std::min(cdf, 1.0) * 4294967296.0;
        out[k] = scaled >= 4294967295.0 ? 0xffffffffu : static_cast<std::uint32_t>(scaled);
        logp += std::log((k + size) / (k + 1.0)) + std::log(q);
    }
    out[kCountMax] = 0xffffffffu;
    return out;
}

std::vector<float> log1p_table() {
    std::vector<float> lut(kCountMax + 2);
    for (int k = 0; k < kCountMax + 2; ++k) lut[k] = static_cast<float>(std::log1p(double(k)));
    return lut;
}

// Seeded permutation (Fisher-Yates driven by splitmix64).
std::vector<std::uint32_t> permutation(std::uint32_t n, std::uint64_t seed) {
    std::vector<std::uint32_t> perm(n);
    for (std::uint32_t i = 0; i < n; ++i) perm[i] = i;
    std::uint64_t state = seed;
    for (std::uint32_t i = n; i > 1; --i) {
        state = splitmix64(state);
        const std::uint32_t j = static_cast<std::uint32_t>(state % i);
        std::swap(perm[i - 1], perm[j]);
    }
    return perm;
}

template<typename T>
int upload(T **dst, const std::vector<T> &src) {
    if (hip_check(hipMalloc(reinterpret_cast<void **>(dst), src.size() * sizeof(T)), "hipMalloc"))
        return 1;
    return hip_check(hipMemcpy(*dst, src.data(), src.size() * sizeof(T), hipMemcpyHostToDevice),
                     "hipMemcpy");
}


// ---- CP-BP structured-support matrix, generated on host threads ----
// Row r: k ~ U{min_active..max_active} distinct modules (module m = genes
// [m*module_size, (m+1)*module_size)), active_genes of each chosen module without
// replacement, then `background` genes uniform over the axis excluding genes already
// present; genes sorted ascending; value = log1p(1 + NB(nb_mean, nb_size)) (a stored entry
// is never zero). Every draw is a splitmix64 of (seed stream, row, draw index), so the
// matrix does not depend on the thread count.
inline std::uint64_t cpbp_draw(std::uint64_t row_key, std::uint64_t i) {
    return splitmix64(row_key ^ (i * 0xd1b54a32d192ed03ull));
}

int host_nb_draw(const std::vector<std::uint32_t> &cdf, std::uint32_t u) {
    int lo = 0, hi = kCountMax;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (u < cdf[mid]) hi = mid;
        else lo = mid + 1;
    }
    return lo;
}

int cpbp_check(const cxs_cpbp_params *p) {
    if (p == nullptr) return fail("null CP-BP parameters");
    if (p->modules == 0u || p->module_size == 0u || p->module_size > 1024u
        || static_cast<std::uint64_t>(p->modules) * p->module_size > p->genes)
        return fail("modules must fit the gene axis (module_size <= 1024)");
    if (p->min_active == 0u || p->min_active > p->max_active || p->max_active > p->modules)
        return fail("active module range must be within [1, modules]");
    if (p->active_genes > p->module_size) return fail("active genes exceed the module size");
    if (static_cast<std::uint64_t>(p->max_active) * p->active_genes + p->background > p->genes / 2)
        return fail("a row may hold at most half of the gene axis");
    if (p->nb_mean <= 0.0 || p->nb_size <= 0.0) return fail("bad NB moments");
    return 0;
}

std::uint32_t cpbp_active(const cxs_cpbp_params *p, std::uint64_t key) {
    return p->min_active
        + static_cast<std::uint32_t>(cpbp_draw(key, 0) % (p->max_active - p->min_active + 1u));
}

template<typename Fn>
void host_parallel(std::uint32_t count, std::uint32_t threads, Fn fn) {
    threads = std::max(1u, std::min(threads, count));
    std::vector<std::thread> pool;
    const std::uint32_t per = count / threads, extra = count % threads;
    std::uint32_t begin = 0;
    for (std::uint32_t t = 0; t < threads; ++t) {
        const std::uint32_t end = begin + per + (t < extra ? 1u : 0u);
        pool.emplace_back([=] { fn(begin, end); });
        begin = end;
    }
    for (auto &th : pool) th.join();
}

} // namespace

extern "C" {

const char *cxs_last_error(void) { return g_error; }

int cxs_cpbp_count(const cxs_cpbp_params *p, std::uint32_t *row_nnz, std::uint32_t threads) {
    if (int rc = cpbp_check(p)) return rc;
    if (row_nnz == nullptr && p->rows != 0u) return fail("null row_nnz");
    const std::uint64_t base = stream_base(p->seed, kCpbpRow);
    host_parallel(p->rows, threads, [&](std::uint32_t lo, std::uint32_t hi) {
        for (std::uint32_t r = lo; r < hi; ++r)
            row_nnz[r] = cpbp_active(p, splitmix64(base ^ r)) * p->active_genes + p->background;
    });
    return 0;
}

int cxs_cpbp_fill(const cxs_cpbp_params *p, const std::uint32_t *row_offsets,
                  std::uint32_t *features, float *values, std::uint32_t threads) {
    if (int rc = cpbp_check(p)) return rc;
    if (p->rows != 0u && (row_offsets == nullptr || features == nullptr || values == nullptr))
        return fail("null CP-BP output");
    const std::uint64_t base = stream_base(p->seed, kCpbpRow);
    const std::uint64_t vbase = stream_base(p->seed, kCpbpValue);
    const std::vector<std::uint32_t> cdf = nb_cdf_table(p->nb_mean, p->nb_size);
    const std::vector<float> lut = log1p_table();
    std::atomic<int> bad{0};
    host_parallel(p->rows, threads, [&](std::uint32_t lo, std::uint32_t hi) {
        std::vector<std::uint8_t> present(p->genes, 0u);
        std::vector<std::uint32_t> genes, mods, local(p->module_size);
        for (std::uint32_t r = lo; r < hi; ++r) {
            const std::uint64_t key = splitmix64(base ^ r);
            const std::uint32_t k = cpbp_active(p, key);
            std::uint64_t draw = 1;
            mods.clear();
            genes.clear();
            while (mods.size() < k) {
                const std::uint32_t m = static_cast<std::uint32_t>(cpbp_draw(key, draw++) % p->modules);
                if (std::find(mods.begin(), mods.end(), m) == mods.end()) mods.push_back(m);
            }
            for (std::uint32_t m : mods) {
                for (std::uint32_t t = 0; t < p->module_size; ++t) local[t] = t;
                for (std::uint32_t t = 0; t < p->active_genes; ++t) {
                    const std::uint32_t j = t + static_cast<std::uint32_t>(
                        cpbp_draw(key, draw++) % (p->module_size - t));
                    std::swap(local[t], local[j]);
                    const std::uint32_t g = m * p->module_size + local[t];
                    genes.push_back(g);
                    present[g] = 1u;
                }
            }
            for (std::uint32_t t = 0; t < p->background;) {
                const std::uint32_t g = static_cast<std::uint32_t>(cpbp_draw(key, draw++) % p->genes);
                if (present[g]) continue;
                present[g] = 1u;
                genes.push_back(g);
                ++t;
            }
            std::sort(genes.begin(), genes.end());
            const std::uint32_t off = row_offsets[r];
            if (row_offsets[r + 1] - off != genes.size()) { bad = 1; continue; }
            const std::uint64_t vkey = splitmix64(vbase ^ r);
            for (std::size_t i = 0; i < genes.size(); ++i) {
                const std::uint32_t u = static_cast<std::uint32_t>(splitmix64(vkey ^ genes[i]) >> 32);
                features[off + i] = genes[i];
                values[off + i] = lut[1 + host_nb_draw(cdf, u)];
                present[genes[i]] = 0u;
            }
        }
    });
    return bad ? fail("row_offsets disagree with cxs_cpbp_count") : 0;
}


int cxs_qcsr_create(const cxs_qcsr_params *params, cxs_generator **out) {
    if (params == nullptr || out == nullptr) return fail("null argument");
    const cxs_qcsr_params &p = *params;
    if (p.rows == 0 || p.cols == 0) return fail("rows and cols must be positive");
    if (!(p.bits == 0 || p.bits == 1 || p.bits == 2 || p.bits == 4 || p.bits == 8))
        return fail("bits must be 0, 1, 2, 4 or 8");
    if (p.nnz_mean <= 0.0 || p.nb_mean <= 0.0 || p.nb_size <= 0.0) return fail("bad moments");
    auto *gen = new cxs_generator();
    gen->p = p;
    std::vector<float> weight(p.cols);
    std::vector<double> prefix(p.cols + 1, 0.0);
    for (std::uint32_t k = 1; k <= p.cols; ++k)
        prefix[k] = prefix[k - 1] + (p.zipf_s == 0.0 ? 1.0 : std::pow(double(k), -p.zipf_s));
    const std::vector<std::uint32_t> rank = permutation(p.cols, stream_base(p.seed, kPerm));
    for (std::uint32_t g = 0; g < p.cols; ++g)
        weight[g] = p.zipf_s == 0.0 ? 1.0f
                                    : static_cast<float>(std::pow(double(rank[g] + 1), -p.zipf_s));
    int rc = upload(&gen->d.gene_weight, weight);
    rc = rc ? rc : upload(&gen->d.rank_prefix, prefix);
    rc = rc ? rc : upload(&gen->d.nb_cdf, nb_cdf_table(p.nb_mean, p.nb_size));
    rc = rc ? rc : upload(&gen->d.log1p_lut, log1p_table());
    rc = rc ? rc : hip_check(hipMalloc(reinterpret_cast<void **>(&gen->d.row_c),
                                       sizeof(float) * p.rows), "hipMalloc");
    if (rc) {
        cxs_destroy(gen);
        return rc;
    }
    *out = gen;
    return 0;
}

void cxs_destroy(cxs_generator *gen) {
    if (gen == nullptr) return;
    (void)hipFree(gen->d.gene_weight);
    (void)hipFree(gen->d.rank_prefix);
    (void)hipFree(gen->d.nb_cdf);
    (void)hipFree(gen->d.log1p_lut);
    (void)hipFree(gen->d.row_c);
    delete gen;
}

int cxs_qcsr_count(cxs_generator *gen, std::int32_t *row_nnz, void *stream) {
    if (gen == nullptr || row_nnz == nullptr) return fail("null argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const cxs_qcsr_params &p = gen->p;
    hipLaunchKernelGGL(k_row_targets, dim3((p.rows + 255) / 256), dim3(256), 0, s, p,
                       gen->d.rank_prefix, gen->d.row_c);
    const std::uint64_t threads = static_cast<std::uint64_t>(p.rows) * kWave;
    hipLaunchKernelGGL(k_count, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0,
                       s, p, gen->d.gene_weight, gen->d.row_c, row_nnz);
    gen->targets_ready = true;
    return hip_check(hipGetLastError(), "k_count");
}

int cxs_qcsr_fill(cxs_generator *gen, const std::int32_t *row_ptr, std::int32_t *col_idx,
                  std::uint32_t *gene_min, std::uint32_t *gene_max, void *stream) {
    if (gen == nullptr || row_ptr == nullptr || col_idx == nullptr || gene_min == nullptr
        || gene_max == nullptr)
        return fail("null argument");
    if (!gen->targets_ready) return fail("cxs_qcsr_count must run first");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const cxs_qcsr_params &p = gen->p;
    const std::uint64_t threads = static_cast<std::uint64_t>(p.rows) * kWave;
    hipLaunchKernelGGL(k_fill, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0,
                       s, p, gen->d.gene_weight, gen->d.row_c, gen->d.nb_cdf, row_ptr, col_idx,
                       gene_min, gene_max);
    return hip_check(hipGetLastError(), "k_fill");
}

int cxs_qcsr_calibrate(cxs_generator *gen, const std::uint32_t *gene_min,
                       const std::uint32_t *gene_max, float *scales, float *offsets,
                       void *stream) {
    if (gen == nullptr || gene_min == nullptr || gene_max == nullptr || scales == nullptr
        || offsets == nullptr)
        return fail("null argument");
    if (gen->p.bits == 0) return fail("calibration applies to quantized matrices only");
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(k_calibrate, dim3((gen->p.cols + 255) / 256), dim3(256), 0, s,
                       gen->p.cols, static_cast<int>(gen->p.bits), gen->d.log1p_lut, gene_min,
                       gene_max, scales, offsets);
    return hip_check(hipGetLastError(), "k_calibrate");
}

int cxs_qcsr_encode(cxs_generator *gen, const std::int32_t *row_ptr,
                    const std::int32_t *packed_row_ptr, const std::int32_t *col_idx,
                    const float *scales, const float *offsets, std::uint8_t *packed,
                    float *values, void *stream) {
    if (gen == nullptr || row_ptr == nullptr || col_idx == nullptr) return fail("null argument");
    if (gen->p.bits != 0 && (packed_row_ptr == nullptr || scales == nullptr || offsets == nullptr
                             || packed == nullptr))
        return fail("quantized encode needs packed_row_ptr, scales, offsets and packed");
    if (gen->p.bits == 0 && values == nullptr) return fail("fp32 encode needs values");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const cxs_qcsr_params &p = gen->p;
    const std::uint64_t threads = static_cast<std::uint64_t>(p.rows) * kWave;
    hipLaunchKernelGGL(k_encode, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0,
                       s, p, gen->d.nb_cdf, gen->d.log1p_lut, row_ptr, packed_row_ptr, col_idx,
                       scales, offsets, packed, values);
    return hip_check(hipGetLastError(), "k_encode");
}

int cxs_dense_normal(std::uint64_t seed, std::uint64_t count, float stddev, std::uint32_t dtype,
                     void *out, void *stream) {
    if (out == nullptr && count != 0) return fail("null output");
    if (dtype != 1u && dtype != 2u && dtype != 5u) return fail("dtype must be 1, 2 or 5");
    if (count == 0) return 0;
    const std::uint64_t pairs = (count + 1) / 2;
    hipLaunchKernelGGL(k_dense_normal, dim3(static_cast<unsigned>((pairs + 255) / 256)), dim3(256),
                       0, static_cast<hipStream_t>(stream), stream_base(seed, kDense), count,
                       stddev, dtype, out);
    return hip_check(hipGetLastError(), "k_dense_normal");
}

int cxs_bell_generate(std::uint64_t seed, std::uint32_t rows, std::uint32_t cols,
                      std::uint32_t block_size, std::uint32_t ell_width, std::uint32_t patterns,
                      std::uint32_t min_blocks, std::uint32_t max_blocks, float density,
                      double nb_mean, double nb_size, std::uint32_t *block_col_idx,
                      std::uint16_t *values_bf16, void *stream) {
    if (block_col_idx == nullptr || values_bf16 == nullptr) return fail("null output");
    if (block_size == 0 || rows % block_size != 0) return fail("rows must be a multiple of block_size");
    const std::uint32_t block_cols = (cols + block_size - 1) / block_size;
    if (patterns == 0 || min_blocks == 0 || min_blocks > max_blocks || max_blocks > ell_width
        || max_blocks > block_cols || ell_width > 256)
        return fail("invalid Blocked-ELL pattern parameters");
    // Each pattern: the first max_blocks entries of a seeded permutation of block columns.
    std::vector<std::uint32_t> pattern_cols(static_cast<std::size_t>(patterns) * max_blocks);
    for (std::uint32_t p = 0; p < patterns; ++p) {
        const auto perm = permutation(block_cols, splitmix64(stream_base(seed, kBellPattern) + p));
        std::copy(perm.begin(), perm.begin() + max_blocks,
                  pattern_cols.begin() + static_cast<std::size_t>(p) * max_blocks);
    }
    std::uint32_t *d_patterns = nullptr, *d_cdf = nullptr;
    float *d_lut = nullptr;
    int rc = upload(&d_patterns, pattern_cols);
    rc = rc ? rc : upload(&d_cdf, nb_cdf_table(nb_mean, nb_size));
    rc = rc ? rc : upload(&d_lut, log1p_table());
    if (rc == 0) {
        hipStream_t s = static_cast<hipStream_t>(stream);
        hipLaunchKernelGGL(k_bell, dim3(rows / block_size), dim3(256), 0, s, seed, rows, cols,
                           block_size, ell_width, patterns, min_blocks, max_blocks, density,
                           d_patterns, d_cdf, d_lut, block_col_idx, values_bf16);
        rc = hip_check(hipGetLastError(), "k_bell");
        rc = rc ? rc : hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    }
    (void)hipFree(d_patterns);
    (void)hipFree(d_cdf);
    (void)hipFree(d_lut);
    return rc;
}

} // extern "C"
