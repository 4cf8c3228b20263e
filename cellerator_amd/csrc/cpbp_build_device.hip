// cpbp_build_device.hip -- device construction of the CP-BP warp-tile projection: the same
// output, bit for bit, as the host builder (cpbp_build.cpp), which restates the reference's
// host producers (apply_plan.cc, cell_block_records.cc, local_cell_ordering.cc,
// warp_tiles.cc). The reference builds the same structures on the device with CUB sorts and
// scans (components/CellPack/src/{apply_plan_cuda,cell_block_records_cuda,
// local_cell_ordering_cuda,warp_tiles_cuda}.cu); here every step is a kernel of this file or
// the radix sort / scan of sort.hip.
//
//   1. plan tables   canonical feature -> (block, local bit); plan and CSR validated on the
//                    device (error bits in one word read back once).
//   2. records       entries ordered by (row, execution feature) with two stable radix sorts
//                    (execution key, then row); a record starts where the row or the block
//                    changes; heads are scanned into record ids; each head ORs its record's
//                    gene bits (at most 32 entries); values gathered into record order.
//   3. local order   per-row (primary, secondary) keys (inferred MinHash over the row's block
//                    ids, deterministic random, nnz descending, or original order); rows are
//                    stably sorted by (window, primary, secondary) -- four LSD sorts of the
//                    row index -- which is the reference's per-window sort with ties broken
//                    by row index.
//   4. tiles         one wave per tile of `group_width` execution rows, one lane per row:
//                    the lanes' record lists are merged in increasing block order (wave min
//                    of the current block ids, ballot of the lanes holding it); a first pass
//                    counts descriptors / entries / values per tile, a scan places them, a
//                    second pass writes descriptors, entries and values.
// Every step is deterministic. Construction synchronizes the stream twice (to size the
// record and tile arrays) and allocates its intermediates with hipMalloc: it is a one-time
// preprocessing, not a launch-path call.
#include "cx_common.hpp"

#include <cstdio>
#include <new>

namespace {

using cx::kWave;

constexpr std::uint32_t kInvalid = 0xffffffffu;
constexpr int kThreads = 256;

// validation error bits
constexpr std::uint32_t kErrPlanSpan = 1u, kErrPlanBlock = 2u, kErrPlanPerm = 4u;
constexpr std::uint32_t kErrCsrOffsets = 8u, kErrCsrFeature = 16u, kErrCsrOrder = 32u;

__device__ __forceinline__ std::uint64_t splitmix64(std::uint64_t value) {
    value += 0x9e3779b97f4a7c15ull;
    value = (value ^ (value >> 30u)) * 0xbf58476d1ce4e5b9ull;
    value = (value ^ (value >> 27u)) * 0x94d049bb133111ebull;
    return value ^ (value >> 31u);
}

__device__ __forceinline__ void flag(std::uint32_t *err, std::uint32_t bit) { atomicOr(err, bit); }

__global__ void fill_u32(std::uint32_t *p, std::uint64_t n, std::uint32_t v) {
    const std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x;
    if (i < n) p[i] = v;
}

// ---- 1. plan tables and validation ------------------------------------------------------

__global__ void plan_tables_kernel(const std::uint32_t *perm, const std::uint32_t *offsets,
                                   std::uint32_t features, std::uint32_t blocks,
                                   std::uint32_t *to_block, std::uint32_t *to_local,
                                   std::uint32_t *seen, std::uint32_t *err) {
    const std::uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b == 0u && (offsets[0] != 0u || offsets[blocks] != features)) flag(err, kErrPlanSpan);
    if (b >= blocks) return;
    const std::uint32_t lo = offsets[b], hi = offsets[b + 1u];
    if (hi <= lo || hi - lo > 32u || hi > features) {
        flag(err, kErrPlanBlock);
        return;
    }
    for (std::uint32_t e = lo; e < hi; ++e) {
        const std::uint32_t c = perm[e];
        if (c >= features) {
            flag(err, kErrPlanPerm);
            continue;
        }
        atomicAdd(&seen[c], 1u);
        to_block[c] = b;
        to_local[c] = e - lo;
    }
}

__global__ void plan_seen_kernel(const std::uint32_t *seen, std::uint32_t features, std::uint32_t *err) {
    const std::uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c < features && seen[c] != 1u) flag(err, kErrPlanPerm);
}

__global__ void csr_check_kernel(const std::uint32_t *row_offsets, const std::uint32_t *features_of,
                                 std::uint32_t rows, std::uint32_t nnz, std::uint32_t features,
                                 std::uint32_t *err) {
    const std::uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r == 0u && row_offsets[0] != 0u) flag(err, kErrCsrOffsets);
    if (r >= rows) return;
    const std::uint32_t b = row_offsets[r], e = row_offsets[r + 1u];
    if (e < b || e > nnz) {
        flag(err, kErrCsrOffsets);
        return;
    }
    for (std::uint32_t i = b; i < e; ++i) {
        const std::uint32_t f = features_of[i];
        if (f >= features) flag(err, kErrCsrFeature);
        if (i > b && f <= features_of[i - 1u]) flag(err, kErrCsrOrder);
    }
}

// ---- 2. records -------------------------------------------------------------------------

__global__ void exec_key_kernel(const std::uint32_t *features_of, std::uint32_t nnz,
                                const std::uint32_t *to_block, const std::uint32_t *to_local,
                                std::uint32_t *key) {
    const std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nnz) return;
    const std::uint32_t f = features_of[i];
    key[i] = (to_block[f] << 5u) | to_local[f];
}

// Row holding entry e: last r with row_offsets[r] <= e.
__device__ __forceinline__ std::uint32_t row_of_entry(const std::uint32_t *row_offsets,
                                                      std::uint32_t rows, std::uint32_t e) {
    std::uint32_t lo = 0u, hi = rows;
    while (hi - lo > 1u) {
        const std::uint32_t mid = lo + (hi - lo) / 2u;
        if (row_offsets[mid] <= e) lo = mid;
        else hi = mid;
    }
    return lo;
}

__global__ void row_key_kernel(const std::uint32_t *perm, std::uint32_t nnz,
                               const std::uint32_t *row_offsets, std::uint32_t rows,
                               std::uint32_t *row_key) {
    const std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nnz) return;
    row_key[i] = row_of_entry(row_offsets, rows, perm[i]);
}

// head[i] = 1 where the (row, block) of sorted position i differs from i - 1's.
__global__ void head_kernel(const std::uint32_t *order, const std::uint32_t *features_of,
                            const std::uint32_t *to_block, std::uint32_t nnz, std::uint32_t *head) {
    const std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i > nnz) return;
    if (i == nnz) {
        head[i] = 0u;
        return;
    }
    const std::uint32_t blk = to_block[features_of[order[i]]];
    head[i] = (i == 0u || blk != to_block[features_of[order[i - 1u]]]) ? 1u : 0u;
}

__global__ void row_start_kernel(const std::uint32_t *row_offsets, std::uint32_t rows,
                                 std::uint32_t *head) {
    const std::uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r < rows && row_offsets[r] < row_offsets[r + 1u]) head[row_offsets[r]] = 1u;
}

__global__ void records_kernel(const std::uint32_t *order, const std::uint32_t *features_of,
                               const std::uint32_t *to_block, const std::uint32_t *to_local,
                               const std::uint32_t *head, const std::uint32_t *rec_id,
                               std::uint32_t nnz, std::uint32_t nrec, std::uint32_t *block_ids,
                               std::uint32_t *gene_masks, std::uint32_t *value_offsets) {
    const std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i == 0u) value_offsets[nrec] = nnz;
    if (i >= nnz || head[i] == 0u) return;
    const std::uint32_t rec = rec_id[i];
    std::uint32_t mask = 0u;
    std::uint32_t j = i;
    do {
        mask |= 1u << to_local[features_of[order[j]]];
        ++j;
    } while (j < nnz && head[j] == 0u);
    block_ids[rec] = to_block[features_of[order[i]]];
    gene_masks[rec] = mask;
    value_offsets[rec] = i;
}

__global__ void rec_row_offsets_kernel(const std::uint32_t *row_offsets, const std::uint32_t *rec_id,
                                       std::uint32_t rows, std::uint32_t *rec_row_offsets) {
    const std::uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r <= rows) rec_row_offsets[r] = rec_id[row_offsets[r]];
}

template<typename V>
__global__ void gather_values_kernel(const V *src, const std::uint32_t *order, std::uint32_t nnz, V *dst) {
    const std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < nnz) dst[i] = src[order[i]];
}

// ---- 3. local order ---------------------------------------------------------------------

struct OrderKeys {
    std::uint32_t kind;
    std::uint32_t rows;
    std::uint64_t seed;
    std::uint64_t global_row_begin;
};

// Restates the host builder's row_keys (local_cell_ordering.cc:96-160).
__global__ void order_keys_kernel(OrderKeys k, const std::uint32_t *rec_row_offsets,
                                  const std::uint32_t *rec_block_ids,
                                  const std::uint32_t *rec_value_offsets, std::uint64_t *primary,
                                  std::uint32_t *secondary) {
    const std::uint32_t row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= k.rows) return;
    const std::uint32_t b = rec_row_offsets[row], e = rec_row_offsets[row + 1u];
    const std::uint32_t nnz = rec_value_offsets[e] - rec_value_offsets[b];
    std::uint64_t p;
    std::uint32_t s = e - b;
    switch (k.kind) {
    case CX_CPBP_ORDER_INFERRED_MINHASH: {
        if (b == e) {
            p = ~0ull;
            break;
        }
        std::uint64_t packed = 0u;
        for (std::uint32_t lane = 0u; lane < 4u; ++lane) {
            std::uint64_t minimum = ~0ull;
            const std::uint64_t lane_seed = splitmix64(k.seed ^ (static_cast<std::uint64_t>(lane) << 32u));
            for (std::uint32_t r = b; r < e; ++r) {
                const std::uint64_t h = splitmix64(lane_seed ^ static_cast<std::uint64_t>(rec_block_ids[r]));
                minimum = h < minimum ? h : minimum;
            }
            packed = (packed << 16u) | ((minimum >> 48u) & 0xffffu);
        }
        p = packed;
        break;
    }
    case CX_CPBP_ORDER_ORIGINAL:
        p = row;
        s = 0u;
        break;
    case CX_CPBP_ORDER_DETERMINISTIC_RANDOM:
        p = splitmix64(k.seed ^ (k.global_row_begin + row));
        s = 0u;
        break;
    default:
        p = ~0ull - nnz;
        break;
    }
    primary[row] = p;
    secondary[row] = s;
}

// key[i] of the next LSD pass for the row at sorted position i
__global__ void order_pass_key_kernel(const std::uint32_t *perm, std::uint32_t rows, int which,
                                      const std::uint64_t *primary, const std::uint32_t *secondary,
                                      std::uint32_t window, std::uint32_t *key) {
    const std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows) return;
    const std::uint32_t r = perm != nullptr ? perm[i] : i;
    switch (which) {
    case 0: key[i] = secondary[r]; break;
    case 1: key[i] = static_cast<std::uint32_t>(primary[r]); break;
    case 2: key[i] = static_cast<std::uint32_t>(primary[r] >> 32u); break;
    default: key[i] = r / window; break;
    }
}

// ---- 4. tiles ---------------------------------------------------------------------------

__device__ __forceinline__ std::uint32_t wave_min_u32(std::uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const std::uint32_t u = __shfl_xor(v, o, kWave);
        v = u < v ? u : v;
    }
    return v;
}

__device__ __forceinline__ std::uint32_t wave_sum_u32(std::uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

__device__ __forceinline__ std::uint32_t wave_exclusive_u32(std::uint32_t v, int lane) {
    std::uint32_t inc = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const std::uint32_t up = __shfl_up(inc, o, kWave);
        if (lane >= o) inc += up;
    }
    return inc - v;
}

__device__ __forceinline__ std::uint64_t lanes_below(int lane) {
    return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

struct TileArgs {
    const std::uint32_t *row_permutation;
    const std::uint32_t *rec_row_offsets;
    const std::uint32_t *rec_block_ids;
    const std::uint32_t *rec_gene_masks;
    const std::uint32_t *rec_value_offsets;
    const void *rec_values;
    std::uint32_t rows;
    std::uint32_t width;
    std::uint32_t tiles;
    std::uint32_t nnz;
    // counts (pass 1) or scanned offsets (pass 2): tiles + 1 each
    std::uint32_t *desc;
    std::uint32_t *entries;
    std::uint32_t *values;
    // outputs (pass 2)
    std::uint32_t *tile_block_ids;
    void *cell_masks;
    std::uint32_t *block_row_entry_offsets;
    std::uint32_t *gene_masks;
    std::uint32_t *value_offsets;
    void *out_values;
};

// One wave per tile; lane l holds execution row t * width + l. kFill = false counts, true
// writes at the scanned offsets.
template<bool kFill, typename MaskT, typename V>
__global__ __launch_bounds__(kThreads) void tile_kernel(TileArgs a) {
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const std::uint32_t t = (blockIdx.x * kThreads + threadIdx.x) / kWave;
    if (t >= a.tiles) return;
    const std::uint32_t first = t * a.width;
    const bool active = static_cast<std::uint32_t>(lane) < a.width && first + lane < a.rows;
    std::uint32_t cur = 0u, end = 0u;
    if (active) {
        const std::uint32_t canon = a.row_permutation[first + lane];
        cur = a.rec_row_offsets[canon];
        end = a.rec_row_offsets[canon + 1u];
    }
    if constexpr (!kFill) {
        const std::uint32_t recs = wave_sum_u32(end - cur);
        const std::uint32_t vals = wave_sum_u32(active ? a.rec_value_offsets[end] - a.rec_value_offsets[cur] : 0u);
        std::uint32_t descriptors = 0u;
        for (;;) {
            const std::uint32_t mine = cur < end ? a.rec_block_ids[cur] : kInvalid;
            const std::uint32_t block = wave_min_u32(mine);
            if (block == kInvalid) break;
            ++descriptors;
            if (mine == block) ++cur;
        }
        if (lane == 0) {
            a.desc[t] = descriptors;
            a.entries[t] = recs;
            a.values[t] = vals;
        }
    } else {
        std::uint32_t d = a.desc[t], e = a.entries[t], v = a.values[t];
        const V *src = static_cast<const V *>(a.rec_values);
        V *dst = static_cast<V *>(a.out_values);
        for (;;) {
            const std::uint32_t mine = cur < end ? a.rec_block_ids[cur] : kInvalid;
            const std::uint32_t block = wave_min_u32(mine);
            if (block == kInvalid) break;
            const bool has = mine == block;
            const std::uint64_t mask = __ballot(has);
            const std::uint32_t vb = has ? a.rec_value_offsets[cur] : 0u;
            const std::uint32_t vc = has ? a.rec_value_offsets[cur + 1u] - vb : 0u;
            const std::uint32_t vpre = wave_exclusive_u32(vc, lane);
            if (lane == 0) {
                a.tile_block_ids[d] = block;
                static_cast<MaskT *>(a.cell_masks)[d] = static_cast<MaskT>(mask);
                a.block_row_entry_offsets[d] = e;
            }
            if (has) {
                const std::uint32_t my_e = e + static_cast<std::uint32_t>(__popcll(mask & lanes_below(lane)));
                a.gene_masks[my_e] = a.rec_gene_masks[cur];
                a.value_offsets[my_e] = v + vpre;
                for (std::uint32_t k = 0; k < vc; ++k) dst[v + vpre + k] = src[vb + k];
                ++cur;
            }
            ++d;
            e += static_cast<std::uint32_t>(__popcll(mask));
            v += wave_sum_u32(vc);
        }
    }
}

__global__ void tile_sentinels_kernel(std::uint32_t *block_row_entry_offsets, std::uint32_t nblocks,
                                      std::uint32_t nentries, std::uint32_t *value_offsets,
                                      std::uint32_t nnz) {
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        block_row_entry_offsets[nblocks] = nentries;
        value_offsets[nentries] = nnz;
    }
}

// ---- host helpers -------------------------------------------------------------------------

unsigned grid_for(std::uint64_t n) { return static_cast<unsigned>((n + kThreads - 1) / kThreads); }

std::uint32_t bit_width(std::uint32_t max_value) {
    std::uint32_t b = 1u;
    while (b < 32u && (max_value >> b) != 0u) ++b;
    return b;
}

// Owned device allocation, freed on scope exit.
struct DevBuf {
    void *p = nullptr;
    DevBuf() = default;
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    ~DevBuf() { if (p != nullptr) (void)hipFree(p); }
    int alloc(std::uint64_t bytes) {
        if (bytes == 0u) bytes = 4u;
        const hipError_t s = hipMalloc(&p, bytes);
        if (s != hipSuccess) {
            p = nullptr;
            return cx::hip_fail(s, "CP-BP device build: hipMalloc");
        }
        return CX_STATUS_SUCCESS;
    }
    template<typename T> T *as() const { return static_cast<T *>(p); }
    void *release() { void *q = p; p = nullptr; return q; }
};

thread_local char g_device_build_error[256] = "";

int build_fail(int status, const char *message) {
    cx::set_error("%s", message);
    std::snprintf(g_device_build_error, sizeof(g_device_build_error), "%s", message);
    return status;
}

#define CX_TRY(expr)                                    \
    do {                                                \
        const int rc_ = (expr);                         \
        if (rc_ != CX_STATUS_SUCCESS) return rc_;       \
    } while (0)

int launched(const char *what) { return cx::check_launch(what); }

int sync(hipStream_t s) {
    const hipError_t st = hipStreamSynchronize(s);
    return st == hipSuccess ? CX_STATUS_SUCCESS : cx::hip_fail(st, "CP-BP device build");
}

int read_u32(const std::uint32_t *dev, std::uint32_t *host, hipStream_t s) {
    hipError_t st = hipMemcpyAsync(host, dev, 4u, hipMemcpyDeviceToHost, s);
    if (st == hipSuccess) st = hipStreamSynchronize(s);
    return st == hipSuccess ? CX_STATUS_SUCCESS : cx::hip_fail(st, "CP-BP device build: readback");
}

} // namespace

struct cx_cpbp_device_builder {
    cx_cpbp_tile_requirements req{};
    std::uint32_t value_size = 0u;
    std::uint32_t nrec = 0u;
    DevBuf rec_row_offsets, rec_block_ids, rec_gene_masks, rec_value_offsets, rec_values;
    DevBuf row_permutation, primary_keys;
    DevBuf tile_desc, tile_entries, tile_values;  // scanned offsets, tiles + 1 each
};

namespace {

int sort_into(const std::uint32_t *keys, const std::uint32_t *vals, std::uint32_t *keys_out,
              std::uint32_t *vals_out, std::uint32_t n, std::uint32_t key_bits, hipStream_t s) {
    const std::uint64_t ws_bytes = cx::sort_pairs_workspace_bytes(n, key_bits);
    DevBuf ws;
    CX_TRY(ws.alloc(ws_bytes));
    CX_TRY(cx::sort_pairs(keys, vals, keys_out, vals_out, n, key_bits, ws.p, ws_bytes, s));
    return sync(s);  // before the workspace is freed
}

int scan_into(const std::uint32_t *in, std::uint32_t *out, std::uint64_t n, hipStream_t s) {
    DevBuf ws;
    CX_TRY(ws.alloc(cx::scan_workspace_bytes(n)));
    CX_TRY(cx::exclusive_scan_u32(in, out, n, ws.p, s));
    return sync(s);
}

int build(cx_cpbp_device_builder *b, const cx_cpbp_plan *plan, const cx_cpbp_csr *csr,
          const cx_cpbp_order_config &cfg, hipStream_t s) {
    const std::uint32_t rows = csr->rows, features = plan->feature_count, nb = plan->feature_block_count;
    const std::uint32_t vs = csr->value_size_bytes, w = cfg.group_width;
    std::uint32_t nnz = 0u;
    if (rows != 0u) CX_TRY(read_u32(csr->row_offsets + rows, &nnz, s));
    if (nnz != 0u && (csr->canonical_features == nullptr || csr->values == nullptr))
        return build_fail(CX_STATUS_INVALID_ARGUMENT, "CP-BP source features or values are null");

    // 1. plan tables + validation
    DevBuf to_block, to_local, seen, err;
    CX_TRY(to_block.alloc(features * 4ull));
    CX_TRY(to_local.alloc(features * 4ull));
    CX_TRY(seen.alloc(features * 4ull));
    CX_TRY(err.alloc(4u));
    hipLaunchKernelGGL(fill_u32, dim3(grid_for(features)), dim3(kThreads), 0, s, seen.as<std::uint32_t>(), features, 0u);
    hipLaunchKernelGGL(fill_u32, dim3(1), dim3(kThreads), 0, s, err.as<std::uint32_t>(), 1ull, 0u);
    hipLaunchKernelGGL(plan_tables_kernel, dim3(grid_for(nb + 1ull)), dim3(kThreads), 0, s,
                       plan->feature_permutation, plan->feature_block_offsets, features, nb,
                       to_block.as<std::uint32_t>(), to_local.as<std::uint32_t>(), seen.as<std::uint32_t>(),
                       err.as<std::uint32_t>());
    hipLaunchKernelGGL(plan_seen_kernel, dim3(grid_for(features)), dim3(kThreads), 0, s,
                       seen.as<std::uint32_t>(), features, err.as<std::uint32_t>());
    if (rows != 0u)
        hipLaunchKernelGGL(csr_check_kernel, dim3(grid_for(rows)), dim3(kThreads), 0, s, csr->row_offsets,
                           csr->canonical_features, rows, nnz, features, err.as<std::uint32_t>());
    CX_TRY(launched("CP-BP device build: validation"));
    std::uint32_t bits = 0u;
    CX_TRY(read_u32(err.as<std::uint32_t>(), &bits, s));
    if (bits & kErrPlanSpan) return build_fail(CX_STATUS_INVALID_SHAPE, "CP-BP plan block offsets must span [0, feature_count]");
    if (bits & kErrPlanBlock) return build_fail(CX_STATUS_INVALID_SHAPE, "CP-BP plan feature blocks must hold 1..32 features");
    if (bits & kErrPlanPerm) return build_fail(CX_STATUS_INVALID_ARGUMENT, "CP-BP plan feature permutation is not a permutation");
    if (bits & kErrCsrOffsets) return build_fail(CX_STATUS_INVALID_SHAPE, "CP-BP source row offsets are not monotonic from zero");
    if (bits & kErrCsrFeature) return build_fail(CX_STATUS_INVALID_SHAPE, "CP-BP source feature id is outside the feature axis");
    if (bits & kErrCsrOrder) return build_fail(CX_STATUS_INVALID_ARGUMENT, "CP-BP source feature ids must be strictly increasing per row");

    // 2. records
    DevBuf order, head, rec_id;
    CX_TRY(head.alloc((nnz + 1ull) * 4u));
    CX_TRY(rec_id.alloc((nnz + 1ull) * 4u));
    CX_TRY(order.alloc(nnz * 4ull));
    if (nnz != 0u) {
        DevBuf key, key_sorted, perm1;
        CX_TRY(key.alloc(nnz * 4ull));
        CX_TRY(key_sorted.alloc(nnz * 4ull));
        CX_TRY(perm1.alloc(nnz * 4ull));
        hipLaunchKernelGGL(exec_key_kernel, dim3(grid_for(nnz)), dim3(kThreads), 0, s, csr->canonical_features,
                           nnz, to_block.as<std::uint32_t>(), to_local.as<std::uint32_t>(), key.as<std::uint32_t>());
        CX_TRY(launched("CP-BP device build: execution keys"));
        CX_TRY(sort_into(key.as<std::uint32_t>(), nullptr, key_sorted.as<std::uint32_t>(), perm1.as<std::uint32_t>(),
                         nnz, bit_width(((nb - 1u) << 5u) | 31u), s));
        hipLaunchKernelGGL(row_key_kernel, dim3(grid_for(nnz)), dim3(kThreads), 0, s, perm1.as<std::uint32_t>(), nnz,
                           csr->row_offsets, rows, key.as<std::uint32_t>());
        CX_TRY(launched("CP-BP device build: row keys"));
        CX_TRY(sort_into(key.as<std::uint32_t>(), perm1.as<std::uint32_t>(), key_sorted.as<std::uint32_t>(),
                         order.as<std::uint32_t>(), nnz, bit_width(rows - 1u), s));
    }
    hipLaunchKernelGGL(head_kernel, dim3(grid_for(nnz + 1ull)), dim3(kThreads), 0, s, order.as<std::uint32_t>(),
                       csr->canonical_features, to_block.as<std::uint32_t>(), nnz, head.as<std::uint32_t>());
    if (rows != 0u)
        hipLaunchKernelGGL(row_start_kernel, dim3(grid_for(rows)), dim3(kThreads), 0, s, csr->row_offsets, rows,
                           head.as<std::uint32_t>());
    CX_TRY(launched("CP-BP device build: record heads"));
    CX_TRY(scan_into(head.as<std::uint32_t>(), rec_id.as<std::uint32_t>(), nnz + 1ull, s));
    std::uint32_t nrec = 0u;
    CX_TRY(read_u32(rec_id.as<std::uint32_t>() + nnz, &nrec, s));
    b->nrec = nrec;
    CX_TRY(b->rec_row_offsets.alloc((rows + 1ull) * 4u));
    CX_TRY(b->rec_block_ids.alloc(nrec * 4ull));
    CX_TRY(b->rec_gene_masks.alloc(nrec * 4ull));
    CX_TRY(b->rec_value_offsets.alloc((nrec + 1ull) * 4u));
    CX_TRY(b->rec_values.alloc(static_cast<std::uint64_t>(nnz) * vs));
    hipLaunchKernelGGL(records_kernel, dim3(grid_for(nnz + 1ull)), dim3(kThreads), 0, s, order.as<std::uint32_t>(),
                       csr->canonical_features, to_block.as<std::uint32_t>(), to_local.as<std::uint32_t>(),
                       head.as<std::uint32_t>(), rec_id.as<std::uint32_t>(), nnz, nrec,
                       b->rec_block_ids.as<std::uint32_t>(), b->rec_gene_masks.as<std::uint32_t>(),
                       b->rec_value_offsets.as<std::uint32_t>());
    if (rows != 0u)
        hipLaunchKernelGGL(rec_row_offsets_kernel, dim3(grid_for(rows + 1ull)), dim3(kThreads), 0, s,
                           csr->row_offsets, rec_id.as<std::uint32_t>(), rows, b->rec_row_offsets.as<std::uint32_t>());
    if (nnz != 0u) {
        if (vs == 2u)
            hipLaunchKernelGGL(gather_values_kernel<std::uint16_t>, dim3(grid_for(nnz)), dim3(kThreads), 0, s,
                               static_cast<const std::uint16_t *>(csr->values), order.as<std::uint32_t>(), nnz,
                               b->rec_values.as<std::uint16_t>());
        else
            hipLaunchKernelGGL(gather_values_kernel<std::uint32_t>, dim3(grid_for(nnz)), dim3(kThreads), 0, s,
                               static_cast<const std::uint32_t *>(csr->values), order.as<std::uint32_t>(), nnz,
                               b->rec_values.as<std::uint32_t>());
    }
    CX_TRY(launched("CP-BP device build: records"));

    // 3. local order
    CX_TRY(b->row_permutation.alloc(rows * 4ull));
    CX_TRY(b->primary_keys.alloc(rows * 8ull));
    if (rows != 0u) {
        DevBuf secondary, key, key_sorted, perm_a;
        CX_TRY(secondary.alloc(rows * 4ull));
        CX_TRY(key.alloc(rows * 4ull));
        CX_TRY(key_sorted.alloc(rows * 4ull));
        CX_TRY(perm_a.alloc(rows * 4ull));
        const OrderKeys ok{cfg.kind, rows, cfg.seed, cfg.global_row_begin};
        hipLaunchKernelGGL(order_keys_kernel, dim3(grid_for(rows)), dim3(kThreads), 0, s, ok,
                           b->rec_row_offsets.as<std::uint32_t>(), b->rec_block_ids.as<std::uint32_t>(),
                           b->rec_value_offsets.as<std::uint32_t>(), b->primary_keys.as<std::uint64_t>(),
                           secondary.as<std::uint32_t>());
        CX_TRY(launched("CP-BP device build: order keys"));
        // LSD: secondary, primary low, primary high, window
        // pass p sorts (key, permutation so far) into perm_a (even p) or row_permutation
        // (odd p): identity -> A -> R -> A -> R
        std::uint32_t *perm_in = nullptr;
        const std::uint32_t windows = (rows + cfg.window_size - 1u) / cfg.window_size;
        const std::uint32_t pass_bits[4] = {32u, 32u, 32u, bit_width(windows - 1u)};
        for (int pass = 0; pass < 4; ++pass) {
            std::uint32_t *perm_out = pass % 2 == 0 ? perm_a.as<std::uint32_t>()
                                                    : b->row_permutation.as<std::uint32_t>();
            hipLaunchKernelGGL(order_pass_key_kernel, dim3(grid_for(rows)), dim3(kThreads), 0, s, perm_in, rows,
                               pass, b->primary_keys.as<std::uint64_t>(), secondary.as<std::uint32_t>(),
                               cfg.window_size, key.as<std::uint32_t>());
            CX_TRY(launched("CP-BP device build: order pass keys"));
            CX_TRY(sort_into(key.as<std::uint32_t>(), perm_in, key_sorted.as<std::uint32_t>(), perm_out, rows,
                             pass_bits[pass], s));
            perm_in = perm_out;
        }
    }

    // 4. tile counts and offsets
    const std::uint32_t tiles = (rows + w - 1u) / w;
    CX_TRY(b->tile_desc.alloc((tiles + 1ull) * 4u));
    CX_TRY(b->tile_entries.alloc((tiles + 1ull) * 4u));
    CX_TRY(b->tile_values.alloc((tiles + 1ull) * 4u));
    std::uint32_t nblocks = 0u, nentries = 0u;
    if (tiles != 0u) {
        DevBuf cd, ce, cv;
        CX_TRY(cd.alloc((tiles + 1ull) * 4u));
        CX_TRY(ce.alloc((tiles + 1ull) * 4u));
        CX_TRY(cv.alloc((tiles + 1ull) * 4u));
        for (DevBuf *c : {&cd, &ce, &cv})
            hipLaunchKernelGGL(fill_u32, dim3(grid_for(tiles + 1ull)), dim3(kThreads), 0, s, c->as<std::uint32_t>(),
                               tiles + 1ull, 0u);
        TileArgs ta{};
        ta.row_permutation = b->row_permutation.as<std::uint32_t>();
        ta.rec_row_offsets = b->rec_row_offsets.as<std::uint32_t>();
        ta.rec_block_ids = b->rec_block_ids.as<std::uint32_t>();
        ta.rec_gene_masks = b->rec_gene_masks.as<std::uint32_t>();
        ta.rec_value_offsets = b->rec_value_offsets.as<std::uint32_t>();
        ta.rows = rows;
        ta.width = w;
        ta.tiles = tiles;
        ta.nnz = nnz;
        ta.desc = cd.as<std::uint32_t>();
        ta.entries = ce.as<std::uint32_t>();
        ta.values = cv.as<std::uint32_t>();
        const unsigned tgrid = static_cast<unsigned>((static_cast<std::uint64_t>(tiles) * kWave + kThreads - 1) / kThreads);
        hipLaunchKernelGGL((tile_kernel<false, std::uint32_t, std::uint32_t>), dim3(tgrid), dim3(kThreads), 0, s, ta);
        CX_TRY(launched("CP-BP device build: tile counts"));
        CX_TRY(scan_into(cd.as<std::uint32_t>(), b->tile_desc.as<std::uint32_t>(), tiles + 1ull, s));
        CX_TRY(scan_into(ce.as<std::uint32_t>(), b->tile_entries.as<std::uint32_t>(), tiles + 1ull, s));
        CX_TRY(scan_into(cv.as<std::uint32_t>(), b->tile_values.as<std::uint32_t>(), tiles + 1ull, s));
        CX_TRY(read_u32(b->tile_desc.as<std::uint32_t>() + tiles, &nblocks, s));
        CX_TRY(read_u32(b->tile_entries.as<std::uint32_t>() + tiles, &nentries, s));
    } else {
        hipLaunchKernelGGL(fill_u32, dim3(1), dim3(kThreads), 0, s, b->tile_desc.as<std::uint32_t>(), 1ull, 0u);
        CX_TRY(launched("CP-BP device build: empty tiles"));
    }
    const hipError_t st = hipStreamSynchronize(s);
    if (st != hipSuccess) return cx::hip_fail(st, "CP-BP device build");

    b->value_size = vs;
    b->req.row_count = rows;
    b->req.feature_count = features;
    b->req.feature_block_count = nb;
    b->req.tile_row_width = w;
    b->req.tile_count = tiles;
    b->req.tile_block_count = nblocks;
    b->req.row_block_entry_count = nentries;
    b->req.nnz_count = nnz;
    b->req.value_size_bytes = vs;
    b->req.cell_mask_bytes = w > 32u ? 8u : 4u;
    return CX_STATUS_SUCCESS;
}

} // namespace

extern "C" const char *cx_cpbp_device_build_last_error(void) { return g_device_build_error; }

extern "C" int cx_cpbp_device_builder_create(const cx_cpbp_plan *plan, const cx_cpbp_csr *csr,
                                             const cx_cpbp_order_config *config, void *stream,
                                             cx_cpbp_device_builder **out) {
    cx::clear_error();
    g_device_build_error[0] = '\0';
    if (out == nullptr || config == nullptr || plan == nullptr || csr == nullptr)
        return build_fail(CX_STATUS_INVALID_ARGUMENT, "CP-BP device builder: null argument");
    *out = nullptr;
    if (plan->feature_permutation == nullptr || plan->feature_block_offsets == nullptr)
        return build_fail(CX_STATUS_INVALID_ARGUMENT, "CP-BP plan has a null array");
    if (plan->feature_block_count == 0u && plan->feature_count != 0u)
        return build_fail(CX_STATUS_INVALID_SHAPE, "CP-BP plan has features but no blocks");
    if (plan->feature_count == 0u) return build_fail(CX_STATUS_INVALID_SHAPE, "CP-BP plan has no features");
    if (csr->value_size_bytes != 2u && csr->value_size_bytes != 4u)
        return build_fail(CX_STATUS_UNSUPPORTED, "CP-BP values must be 2-byte (f16) or 4-byte (f32)");
    if (csr->rows != 0u && csr->row_offsets == nullptr)
        return build_fail(CX_STATUS_INVALID_ARGUMENT, "CP-BP source row offsets are null");
    const cx_cpbp_order_config cfg = *config;
    if (!(cfg.kind == CX_CPBP_ORDER_INFERRED_MINHASH || cfg.kind == CX_CPBP_ORDER_ORIGINAL
          || cfg.kind == CX_CPBP_ORDER_DETERMINISTIC_RANDOM || cfg.kind == CX_CPBP_ORDER_ROW_NNZ_DESCENDING))
        return build_fail(CX_STATUS_UNSUPPORTED, "local-cell order kind is unsupported");
    if (cfg.window_size == 0u || cfg.group_width == 0u || cfg.group_width > cfg.window_size
        || cfg.window_size % cfg.group_width != 0u)
        return build_fail(CX_STATUS_INVALID_SHAPE, "local-cell windows must contain an integral nonzero number of groups");
    if (cfg.group_width > 64u) return build_fail(CX_STATUS_INVALID_SHAPE, "tile width must be at most 64 rows");
    cx_cpbp_device_builder *b = new (std::nothrow) cx_cpbp_device_builder();
    if (b == nullptr) return build_fail(CX_STATUS_INTERNAL_ERROR, "CP-BP device builder allocation failed");
    const int rc = build(b, plan, csr, cfg, static_cast<hipStream_t>(stream));
    if (rc != CX_STATUS_SUCCESS) {
        if (g_device_build_error[0] == '\0') {
            const char *m = cx_last_error();
            std::snprintf(g_device_build_error, sizeof(g_device_build_error), "%s", m != nullptr ? m : "");
        }
        delete b;
        return rc;
    }
    *out = b;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_cpbp_device_builder_requirements(const cx_cpbp_device_builder *b,
                                                   cx_cpbp_tile_requirements *out) {
    if (b == nullptr || out == nullptr)
        return build_fail(CX_STATUS_INVALID_ARGUMENT, "CP-BP device builder: null builder or output");
    *out = b->req;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_cpbp_device_builder_export(const cx_cpbp_device_builder *b,
                                             const cx_cpbp_tile_buffers *buf, void *stream) {
    cx::clear_error();
    if (b == nullptr || buf == nullptr)
        return build_fail(CX_STATUS_INVALID_ARGUMENT, "CP-BP device builder: null builder or buffers");
    const cx_cpbp_tile_requirements &r = b->req;
    if (buf->tile_block_offsets == nullptr || buf->block_row_entry_offsets == nullptr
        || buf->row_block_value_offsets == nullptr
        || (r.row_count != 0u && buf->row_permutation == nullptr)
        || (r.tile_block_count != 0u && (buf->tile_block_ids == nullptr || buf->tile_block_cell_masks == nullptr))
        || (r.row_block_entry_count != 0u && buf->row_block_gene_masks == nullptr)
        || (r.nnz_count != 0u && buf->values == nullptr))
        return build_fail(CX_STATUS_INVALID_ARGUMENT, "CP-BP export buffer is null");
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t st = hipMemcpyAsync(buf->tile_block_offsets, b->tile_desc.p, (r.tile_count + 1ull) * 4u,
                                   hipMemcpyDeviceToDevice, s);
    if (st == hipSuccess && r.row_count != 0u)
        st = hipMemcpyAsync(buf->row_permutation, b->row_permutation.p, r.row_count * 4ull, hipMemcpyDeviceToDevice, s);
    if (st == hipSuccess && r.row_count != 0u && buf->primary_keys != nullptr)
        st = hipMemcpyAsync(buf->primary_keys, b->primary_keys.p, r.row_count * 8ull, hipMemcpyDeviceToDevice, s);
    if (st != hipSuccess) return cx::hip_fail(st, "CP-BP device export: copy");
    if (r.tile_count != 0u) {
        TileArgs ta{};
        ta.row_permutation = b->row_permutation.as<std::uint32_t>();
        ta.rec_row_offsets = b->rec_row_offsets.as<std::uint32_t>();
        ta.rec_block_ids = b->rec_block_ids.as<std::uint32_t>();
        ta.rec_gene_masks = b->rec_gene_masks.as<std::uint32_t>();
        ta.rec_value_offsets = b->rec_value_offsets.as<std::uint32_t>();
        ta.rec_values = b->rec_values.p;
        ta.rows = r.row_count;
        ta.width = r.tile_row_width;
        ta.tiles = r.tile_count;
        ta.nnz = r.nnz_count;
        ta.desc = b->tile_desc.as<std::uint32_t>();
        ta.entries = b->tile_entries.as<std::uint32_t>();
        ta.values = b->tile_values.as<std::uint32_t>();
        ta.tile_block_ids = buf->tile_block_ids;
        ta.cell_masks = buf->tile_block_cell_masks;
        ta.block_row_entry_offsets = buf->block_row_entry_offsets;
        ta.gene_masks = buf->row_block_gene_masks;
        ta.value_offsets = buf->row_block_value_offsets;
        ta.out_values = buf->values;
        const unsigned tgrid = static_cast<unsigned>((static_cast<std::uint64_t>(r.tile_count) * kWave + kThreads - 1) / kThreads);
        const bool wide = r.cell_mask_bytes == 8u;
        if (wide && b->value_size == 2u)
            hipLaunchKernelGGL((tile_kernel<true, std::uint64_t, std::uint16_t>), dim3(tgrid), dim3(kThreads), 0, s, ta);
        else if (wide)
            hipLaunchKernelGGL((tile_kernel<true, std::uint64_t, std::uint32_t>), dim3(tgrid), dim3(kThreads), 0, s, ta);
        else if (b->value_size == 2u)
            hipLaunchKernelGGL((tile_kernel<true, std::uint32_t, std::uint16_t>), dim3(tgrid), dim3(kThreads), 0, s, ta);
        else
            hipLaunchKernelGGL((tile_kernel<true, std::uint32_t, std::uint32_t>), dim3(tgrid), dim3(kThreads), 0, s, ta);
    }
    hipLaunchKernelGGL(tile_sentinels_kernel, dim3(1), dim3(64), 0, s, buf->block_row_entry_offsets,
                       r.tile_block_count, r.row_block_entry_count, buf->row_block_value_offsets, r.nnz_count);
    return launched("CP-BP device export: tiles");
}

extern "C" void cx_cpbp_device_builder_destroy(cx_cpbp_device_builder *b) { delete b; }
