// cpbp_reduce.hip -- CP-BP warp-tile feature-weighted row reduction on gfx950.
//
// Contract (components/CellPack/src/feature_weighted_row_reduction_cuda.cu:180-218): for
// every execution row of every tile, the sum over its stored values of
// fp32(value) * w[feature_permutation[block_begin + local]], written to
// row_values[row_permutation[execution_row]] (canonical order).
//
// Why not the reference's mapping (one lane per tile row, looping over the tile's
// descriptors): with module-sparse cells a 64-row tile carries ~790 descriptors of ~6 rows
// each, so a lane-per-row wave is ~9% busy.
//
// Entry-batch mapping. One wave owns one tile at a time (each workgroup's tiles taken from
// an LDS queue); 16 waves share a workgroup and the plan staged once in LDS (permuted
// weights wp[f] = w[perm[f]], block starts). A tile's row-block entries are contiguous, and
// so are their values. The wave takes the entries in batches of up to 64 (at most 512
// values):
//   1. lane j holds entry j (value offset, gene mask) and lane k descriptor k (first entry,
//      cell mask, block id), loaded coalesced;
//   2. each entry finds its descriptor (descriptor starts scattered into LDS slots, then a
//      wave max-scan) and its row (the rank-th set bit of the descriptor's cell mask) -- or,
//      with entry rows prepared once per tile structure (cx_cpbp_entry_rows), reads its row
//      and block start from one word per entry instead;
//   3. the batch's values, loaded coalesced, are staged in LDS; each entry lane sums
//      value * wp[block start + bit] over its own values in a register (fp32 FMA) and adds
//      the sum to its row's accumulator in LDS: an integer atomic numbers the batch's
//      entries of each row, and the j-th entries of all rows are added in round j with a
//      plain read and write (no float atomics: they are an order of magnitude slower).
// Loads are raw buffer loads over the tile's slices (0 past the end, no branches) and run
// one batch ahead on ping-pong registers, so a batch's waits cover only its own loads.
// The summation order (per entry, then entries per row) differs from the reference's
// (descriptor, then bit) order; results agree within the reference's tolerance
// (feature_weighted_row_reduction.hh:13-14) widened for fp32 reordering.
#include <cstdio>

#include "cx_common.hpp"

namespace cx {
namespace {

struct CpbpArgs {
    const std::uint32_t *feature_block_offsets;
    const std::uint32_t *feature_permutation;
    const std::uint32_t *tile_block_offsets;
    const std::uint32_t *tile_block_ids;
    const void *cell_masks;
    const std::uint32_t *block_row_entry_offsets;
    const std::uint32_t *gene_masks;
    const std::uint32_t *value_offsets;
    const void *values;
    const std::uint32_t *row_permutation;
    const float *weights;
    float *row_values;
    std::uint32_t *entry_rows;  // per entry: block start << 6 | tile row (written by the rows walk)
    std::uint32_t row_count;
    std::uint32_t tile_count;
    std::uint32_t tile_row_width;
    std::uint32_t feature_count;
    std::uint32_t feature_block_count;
};

constexpr int kCpbpWaves = 16;         // waves (tiles in flight) per workgroup
constexpr int kCpbpGrid = 256;         // one workgroup per CU (LDS-limited)
constexpr std::uint32_t kBatchValues = 512;  // values of one entry batch (staged in LDS)
constexpr std::uint32_t kWeightsLds = 20480;  // features whose weights fit the LDS stage
constexpr std::uint32_t kBlocksLds = 2048;    // feature block offsets staged in LDS

struct WaveLds {
    float acc[64];            // the tile's row sums
    std::uint32_t occ[64];    // per batch: entries counted per row
    float stage[kBatchValues + 4];  // + one step of the 4-wide read past an entry's end
    std::int32_t slot[64];
};

__device__ __forceinline__ void lds_order() { __asm__ volatile("" ::: "memory"); }

__device__ __forceinline__ std::uint32_t uniform(std::uint32_t v) {
    return static_cast<std::uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
}

// Inclusive max-scan over the wave of non-negative values, in DPP (no LDS crossbar traffic):
// row shifts by 1, 2, 4, 8 scan each 16-lane row, then the row broadcasts of lanes 15 and
// 31 carry the running maximum into the later rows. Lanes without a source see 0.
template<int kCtrl, int kRowMask>
__device__ __forceinline__ int dpp_max_step(int v) {
    const int o = __builtin_amdgcn_update_dpp(0, v, kCtrl, kRowMask, 0xf, false);
    return v > o ? v : o;
}

__device__ __forceinline__ int wave_inclusive_max(int v, int /*lane*/) {
    v = dpp_max_step<0x111, 0xf>(v);  // row_shr:1
    v = dpp_max_step<0x112, 0xf>(v);  // row_shr:2
    v = dpp_max_step<0x114, 0xf>(v);  // row_shr:4
    v = dpp_max_step<0x118, 0xf>(v);  // row_shr:8
    v = dpp_max_step<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v = dpp_max_step<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}

// Position of the rank-th (0-based) set bit of a 32-bit mask (rank < popcount).
__device__ __forceinline__ std::uint32_t select_bit32(std::uint32_t m, std::uint32_t r) {
    std::uint32_t base = 0u, c;
    c = __builtin_popcount(m & 0xFFFFu); if (r >= c) { r -= c; m >>= 16; base += 16u; }
    c = __builtin_popcount(m & 0xFFu);   if (r >= c) { r -= c; m >>= 8;  base += 8u; }
    c = __builtin_popcount(m & 0xFu);    if (r >= c) { r -= c; m >>= 4;  base += 4u; }
    c = __builtin_popcount(m & 0x3u);    if (r >= c) { r -= c; m >>= 2;  base += 2u; }
    c = m & 1u;                          if (r >= c) { base += 1u; }
    return base;
}

// One 32-bit select on the half that holds the bit, chosen by selects: a branch here would
// be divergent across the wave and run both halves.
__device__ __forceinline__ std::uint32_t select_bit(std::uint64_t m, std::uint32_t r) {
    const std::uint32_t lo = static_cast<std::uint32_t>(m);
    const std::uint32_t c = static_cast<std::uint32_t>(__builtin_popcount(lo));
    const bool up = r >= c;
    return (up ? 32u : 0u)
        + select_bit32(up ? static_cast<std::uint32_t>(m >> 32) : lo, up ? r - c : r);
}

__device__ __forceinline__ std::uint32_t select_bit(std::uint32_t m, std::uint32_t r) {
    return select_bit32(m, r);
}

template<typename ValT>
__device__ __forceinline__ float load_value(const ValT *values, std::uint32_t i) {
    if constexpr (sizeof(ValT) == 2) return h2f(values[i]);
    else return values[i];
}

// Buffer resources over one tile's slices of the tile arrays. Raw buffer loads return 0
// past the end of the slice, so the batch loads need no branches: every iteration issues
// the same straight-line loads, which lets the wait counts of the prefetch pipeline cover
// only the loads actually needed next.
using rsrc_t = __amdgpu_buffer_rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void *base, std::uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
}

__device__ __forceinline__ std::uint32_t bload32(rsrc_t r, std::uint32_t byte_offset) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(byte_offset), 0, 0);
}

template<typename MaskT>
__device__ __forceinline__ MaskT bload_mask(rsrc_t r, std::uint32_t index) {
    if constexpr (sizeof(MaskT) == 8) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(index * 8u), 0, 0);
        return static_cast<MaskT>(v[0]) | (static_cast<MaskT>(v[1]) << 32);
    } else {
        return bload32(r, index * 4u);
    }
}

template<typename ValT>
__device__ __forceinline__ float bload_value(rsrc_t r, std::uint32_t index) {
    if constexpr (sizeof(ValT) == 2) {
        const std::uint16_t h = __builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(index * 2u), 0, 0);
        return h2f(h);
    } else {
        return __uint_as_float(bload32(r, index * 4u));
    }
}

// What one walk over the tiles does: reduce from the descriptors (the reference layout
// alone), reduce with each entry's row and block start read from a prepared per-entry array,
// or compute that array.
enum class Walk { reduce, with_rows, make_rows };

struct TileRsrc {
    rsrc_t value_offsets, gene_masks, entry_offsets, masks, block_ids, values, rows;
    std::uint32_t e0, d0, v0;
};

// Per-lane inputs of one entry batch: entry `lane` of the batch (value offset, next value
// offset, gene mask) and descriptor `lane` from the batch's first descriptor (first entry,
// cell mask, block id).
template<typename MaskT>
struct BatchInput {
    std::uint32_t s_j, s_next, gm, eo_k, blk_k, rb;
    MaskT mask_k;
    bool has_entry, has_desc;
};

template<typename MaskT, Walk kWalk>
__device__ __forceinline__ BatchInput<MaskT> load_batch(const TileRsrc &r, std::uint32_t e,
                                                        std::uint32_t e_end, std::uint32_t d,
                                                        std::uint32_t d_end, int lane) {
    BatchInput<MaskT> b;
    const std::uint32_t ul = static_cast<std::uint32_t>(lane);
    b.has_entry = e < e_end && ul < min(64u, e_end - e);
    b.has_desc = e < e_end && ul < min(64u, d_end - d);
    const std::uint32_t ei = e - r.e0 + ul, di = d - r.d0 + ul;
    // loads first, selects after: no branch around a load
    const std::uint32_t s_j = bload32(r.value_offsets, ei * 4u);
    const std::uint32_t s_next = bload32(r.value_offsets, ei * 4u + 4u);
    const std::uint32_t gm = bload32(r.gene_masks, ei * 4u);
    b.s_j = b.has_entry ? s_j : 0u;
    b.s_next = b.has_entry ? s_next : 0u;
    b.gm = b.has_entry ? gm : 0u;
    if constexpr (kWalk == Walk::with_rows) {
        const std::uint32_t rb = bload32(r.rows, ei * 4u);
        b.rb = b.has_entry ? rb : 0u;
        b.eo_k = 0u;
        b.mask_k = 0u;
        b.blk_k = 0u;
    } else {
        b.eo_k = bload32(r.entry_offsets, di * 4u);
        b.mask_k = bload_mask<MaskT>(r.masks, di);
        b.blk_k = bload32(r.block_ids, di * 4u);
        b.rb = 0u;
    }
    return b;
}

// Extent of a batch: its first value offset, entry count n (values <= kBatchValues) and
// value count.
struct BatchExtent {
    std::uint32_t s0, n, nv;
};

template<typename MaskT>
__device__ __forceinline__ BatchExtent batch_extent(const BatchInput<MaskT> &b) {
    BatchExtent x;
    x.s0 = uniform(b.s_j);
    const std::uint64_t fit = __builtin_amdgcn_ballot_w64(b.has_entry && b.s_next - x.s0 <= kBatchValues);
    x.n = max(1u, static_cast<std::uint32_t>(__popcll(fit)));
    const std::uint32_t v_end = static_cast<std::uint32_t>(
        __builtin_amdgcn_readlane(static_cast<int>(b.s_next), static_cast<int>(x.n) - 1));
    x.nv = min(v_end - x.s0, kBatchValues);
    return x;
}

// First descriptor of the batch that starts at entry e_next: the last loaded descriptor
// whose first entry is <= e_next.
template<typename MaskT>
__device__ __forceinline__ std::uint32_t next_descriptor(const BatchInput<MaskT> &b, std::uint32_t d,
                                                         std::uint32_t e_next) {
    const std::uint64_t passed = __builtin_amdgcn_ballot_w64(b.has_desc && b.eo_k <= e_next);
    return d + max(1u, static_cast<std::uint32_t>(__popcll(passed))) - 1u;
}

// The batch's values (lanes past the batch read the next values of the tile, or 0 past
// the tile; neither is used).
template<typename ValT>
__device__ __forceinline__ void load_values(float (&x)[kBatchValues / kWave], const TileRsrc &r,
                                            std::uint32_t s0, int lane) {
#pragma unroll
    for (std::uint32_t c = 0; c < kBatchValues / kWave; ++c)
        x[c] = bload_value<ValT>(r.values, s0 - r.v0 + c * kWave + static_cast<std::uint32_t>(lane));
}

template<typename MaskT, typename ValT, bool kLdsPlan, Walk kWalk>
__global__ __launch_bounds__(kWave *kCpbpWaves) void cpbp_reduce_kernel(CpbpArgs a) {
    // Plan staged in LDS: permuted weights (zero-padded by one block) and block starts.
    constexpr bool kStageWeights = kLdsPlan && kWalk != Walk::make_rows;
    constexpr bool kStageBlocks = kLdsPlan && kWalk == Walk::reduce;
    __shared__ float wp[kStageWeights ? kWeightsLds + 32 : 1];
    __shared__ std::uint32_t block_begin[kStageBlocks ? kBlocksLds : 1];
    __shared__ WaveLds wave_lds[kCpbpWaves];
    __shared__ std::uint32_t next_tile;  // the workgroup's tile queue (below)
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const std::uint32_t wave = uniform(threadIdx.x / kWave);
    if (threadIdx.x == 0) next_tile = kCpbpWaves;
    if constexpr (kStageWeights)
        for (std::uint32_t f = threadIdx.x; f < a.feature_count + 32u; f += blockDim.x)
            wp[f] = f < a.feature_count ? a.weights[a.feature_permutation[f]] : 0.0f;
    if constexpr (kStageBlocks)
        for (std::uint32_t k = threadIdx.x; k <= a.feature_block_count; k += blockDim.x)
            block_begin[k] = a.feature_block_offsets[k];
    __syncthreads();
    WaveLds &L = wave_lds[wave];
    const MaskT *masks = static_cast<const MaskT *>(a.cell_masks);
    const ValT *values = static_cast<const ValT *>(a.values);

    // Workgroup b (one per CU) owns tiles b, b + gridDim.x, b + 2 gridDim.x, ...: every CU
    // gets the same number of tiles to within one. Its waves take them first come, first
    // served from an LDS counter (wave w starts with the w-th), so a wave that drew light
    // tiles takes more and the CU's SIMDs end together. Each tile is still reduced by one
    // wave in a fixed order, so results do not depend on which wave takes it. (Dealt
    // statically wave-major, tile t to wave t % (gridDim.x * 16), the first CUs' waves all
    // held one tile more than the last CUs', and the heaviest CU carried 5% above the mean.)
    for (std::uint32_t k = wave;;) {
        const std::uint64_t t64 = blockIdx.x + static_cast<std::uint64_t>(gridDim.x) * k;
        if (t64 >= a.tile_count) break;
        const std::uint32_t t = static_cast<std::uint32_t>(t64);
        L.acc[lane] = 0.0f;
        // tile bounds are wave-uniform: keep them (and the buffer resources) in SGPRs
        const std::uint32_t d_end = uniform(a.tile_block_offsets[t + 1]);
        std::uint32_t d = uniform(a.tile_block_offsets[t]);
        std::uint32_t e = uniform(a.block_row_entry_offsets[d]);
        const std::uint32_t e_end = uniform(a.block_row_entry_offsets[d_end]);
        TileRsrc r;
        r.e0 = e;
        r.d0 = d;
        r.v0 = uniform(a.value_offsets[e]);
        const std::uint32_t v_tile_end = uniform(a.value_offsets[e_end]);
        r.value_offsets = make_rsrc(a.value_offsets + e, (e_end - e + 1u) * 4u);
        r.gene_masks = make_rsrc(a.gene_masks + e, (e_end - e) * 4u);
        r.entry_offsets = make_rsrc(a.block_row_entry_offsets + d, (d_end - d + 1u) * 4u);
        r.masks = make_rsrc(masks + d, (d_end - d) * static_cast<std::uint32_t>(sizeof(MaskT)));
        r.block_ids = make_rsrc(a.tile_block_ids + d, (d_end - d) * 4u);
        r.values = make_rsrc(values + r.v0, (v_tile_end - r.v0) * static_cast<std::uint32_t>(sizeof(ValT)));
        if constexpr (kWalk == Walk::with_rows) r.rows = make_rsrc(a.entry_rows + e, (e_end - e) * 4u);

        // Two-stage pipeline over ping-pong register sets (no copies, so no forced waits):
        // while batch i is reduced, the entries/descriptors of batch i+1 and the 512-value
        // window that starts where batch i ends (it contains batch i+1) are in flight.
        auto step = [&](BatchInput<MaskT> &cur, float (&x_cur)[kBatchValues / kWave],
                        BatchInput<MaskT> &nxt, float (&x_nxt)[kBatchValues / kWave]) {
            const BatchExtent cur_x = batch_extent(cur);
            const std::uint32_t e_next = e + cur_x.n;
            const std::uint32_t d_next = kWalk == Walk::with_rows ? d : next_descriptor(cur, d, e_next);
            nxt = load_batch<MaskT, kWalk>(r, e_next, e_end, d_next, d_end, lane);
            if constexpr (kWalk != Walk::make_rows) load_values<ValT>(x_nxt, r, cur_x.s0 + cur_x.nv, lane);

            std::uint32_t row, bb;
            if constexpr (kWalk == Walk::with_rows) {
                row = cur.rb & 63u;
                bb = cur.rb >> 6;
            } else {
                // entry -> descriptor (slots + max-scan) -> row and block start
                L.slot[lane] = 0;
                lds_order();
                const std::uint32_t q = cur.eo_k - e;
                if (cur.has_desc && q < 64u)
                    __hip_atomic_fetch_max(&L.slot[q], lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
                lds_order();
                const int kd = wave_inclusive_max(L.slot[lane], lane);
                const std::uint32_t my_eo = __shfl(cur.eo_k, kd, kWave);
                const MaskT my_mask = __shfl(cur.mask_k, kd, kWave);
                const std::uint32_t my_blk = __shfl(cur.blk_k, kd, kWave);
                row = select_bit(my_mask, e + lane - my_eo) & 63u;
                if constexpr (kStageBlocks) bb = min(block_begin[min(my_blk, a.feature_block_count)], a.feature_count);
                else bb = min(a.feature_block_offsets[min(my_blk, a.feature_block_count)], a.feature_count);
            }
            if constexpr (kWalk == Walk::make_rows) {
                if (static_cast<std::uint32_t>(lane) < cur_x.n) a.entry_rows[e + static_cast<std::uint32_t>(lane)] = bb << 6 | row;
            } else {

                // stage the batch's values; each entry sums its own values in a register
#pragma unroll
                for (std::uint32_t c = 0; c < kBatchValues / kWave; ++c)
                    L.stage[c * kWave + static_cast<std::uint32_t>(lane)] = x_cur[c];
                lds_order();
                const bool has = static_cast<std::uint32_t>(lane) < cur_x.n;
                float sum = 0.0f;
                if (has) {
                    std::uint32_t m = cur.gm;
                    const float *v = &L.stage[min(cur.s_j - cur_x.s0, kBatchValues)];
                    if constexpr (kLdsPlan) {
                        const float *w = &wp[bb];
                        // An absent bit reads weight 31 of the block (m | bit 31 is never 0, and
                        // the weight stage is padded by one block) and at most the stage's
                        // 4-value tail, so every read is in bounds and needs no exec mask. Its
                        // product is dropped by one select on the sum (zeroing only one operand
                        // would let a non-finite value or weight from outside the entry in).
                        constexpr std::uint32_t kStop = 0x80000000u;
                        while (m != 0u) {  // four stored values per step
                            const std::uint32_t b0 = static_cast<std::uint32_t>(__builtin_ctz(m));
                            m &= m - 1u;
                            const bool h1 = m != 0u;
                            const std::uint32_t b1 = static_cast<std::uint32_t>(__builtin_ctz(m | kStop));
                            m &= m - 1u;
                            const bool h2 = m != 0u;
                            const std::uint32_t b2 = static_cast<std::uint32_t>(__builtin_ctz(m | kStop));
                            m &= m - 1u;
                            const bool h3 = m != 0u;
                            const std::uint32_t b3 = static_cast<std::uint32_t>(__builtin_ctz(m | kStop));
                            m &= m - 1u;
                            const float v0 = v[0], v1 = v[1], v2 = v[2], v3 = v[3];
                            const float w0 = w[b0], w1 = w[b1], w2 = w[b2], w3 = w[b3];
                            // keeps the reads unconditional (the compiler would otherwise sink
                            // them under a divergent branch per select)
                            __asm__ volatile("" ::"v"(v1), "v"(v2), "v"(v3), "v"(w1), "v"(w2), "v"(w3));
                            sum = __builtin_fmaf(v0, w0, sum);
                            sum = h1 ? __builtin_fmaf(v1, w1, sum) : sum;
                            sum = h2 ? __builtin_fmaf(v2, w2, sum) : sum;
                            sum = h3 ? __builtin_fmaf(v3, w3, sum) : sum;
                            v += 4;
                        }
                    } else {
                        while (m != 0u) {
                            const std::uint32_t b = static_cast<std::uint32_t>(__builtin_ctz(m));
                            m &= m - 1u;
                            const std::uint32_t f = min(bb + b, a.feature_count - 1u);
                            sum = __builtin_fmaf(*v, a.weights[a.feature_permutation[f]], sum);
                            ++v;
                        }
                    }
                }
                // Each entry's sum goes to its row. Rows repeat within a batch (one entry per
                // descriptor that holds the row), and LDS float atomics cost ~190 CU cycles per
                // wave instruction here, against ~16 for an integer atomic with return and ~10 for
                // a plain read and write: so each entry takes its occurrence number among the
                // batch's entries of its row from an integer atomic, and round j adds the sums of
                // the j-th occurrences with a plain read, add and write (the rows of one round are
                // distinct). Two or three rounds cover a batch.
                if (has) L.occ[row] = 0u;
                lds_order();
                std::uint32_t occ = 0u;
                if (has) occ = __hip_atomic_fetch_add(&L.occ[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
                for (std::uint32_t j = 0u;; ++j) {
                    if (has && occ == j) L.acc[row] += sum;
                    lds_order();
                    if (__builtin_amdgcn_ballot_w64(has && occ > j) == 0ull) break;
                }
            }
            e = e_next;
            d = d_next;
        };

        BatchInput<MaskT> in_a = load_batch<MaskT, kWalk>(r, e, e_end, d, d_end, lane), in_b;
        float x_a[kBatchValues / kWave], x_b[kBatchValues / kWave];
        if constexpr (kWalk != Walk::make_rows) load_values<ValT>(x_a, r, r.v0, lane);
        while (e < e_end) {
            step(in_a, x_a, in_b, x_b);
            if (e >= e_end) break;
            step(in_b, x_b, in_a, x_a);
        }
        lds_order();
        const std::uint32_t exec_row = t * a.tile_row_width + static_cast<std::uint32_t>(lane);
        if (kWalk != Walk::make_rows && static_cast<std::uint32_t>(lane) < a.tile_row_width && exec_row < a.row_count) {
            a.row_values[a.row_permutation[exec_row]] = L.acc[lane];
        }
        lds_order();
        std::uint32_t nk = 0u;
        if (lane == 0)
            nk = __hip_atomic_fetch_add(&next_tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        k = uniform(static_cast<std::uint32_t>(__shfl(static_cast<int>(nk), 0, kWave)));
    }
}

} // namespace
} // namespace cx

namespace cx {
namespace {

// Metadata, dimension, pointer and aliasing checks of cx_cpbp_reduce (validate_metadata and
// validate_output, feature_weighted_row_reduction_cuda.cu:57-178) for the walks over tiles
// `t`. `weights`/`out` are checked when `reduce`; `entry_rows`/`rows_capacity` when given.
int check_walk(const cx_cpbp_tiles *t, bool reduce, const float *feature_weights,
               uint64_t feature_weight_capacity, const float *row_values, uint64_t row_capacity,
               const std::uint32_t *entry_rows, uint64_t rows_capacity, const char *who) {
    char msg[160];
    auto bad = [&](int status, const char *what) {
        std::snprintf(msg, sizeof(msg), "%s: %s", who, what);
        return fail(status, msg);
    };
    if (t == nullptr) return bad(CX_STATUS_INVALID_ARGUMENT, "null tiles");
    if (t->value_dtype != CELLERATOR_DTYPE_F16 && t->value_dtype != CELLERATOR_DTYPE_F32)
        return bad(CX_STATUS_UNSUPPORTED, "values must be F16 or F32");
    if (t->tile_row_width == 0u || t->tile_row_width > 64u)
        return bad(CX_STATUS_INVALID_SHAPE, "tile_row_width must be 1..64");
    const std::uint64_t expected_tiles = (static_cast<std::uint64_t>(t->row_count) + t->tile_row_width - 1u)
        / t->tile_row_width;
    if (t->tile_count != expected_tiles || t->tile_block_count > t->row_block_entry_count
        || t->row_block_entry_count > t->nnz_count)
        return bad(CX_STATUS_INVALID_SHAPE, "tile, descriptor or entry counts are inconsistent");
    if (reduce && feature_weight_capacity < t->feature_count)
        return bad(CX_STATUS_INVALID_SHAPE, "feature weight capacity is too small");
    if (reduce && row_capacity < t->row_count)
        return bad(CX_STATUS_INVALID_SHAPE, "output capacity is insufficient");
    if (t->feature_block_offsets == nullptr
        || (reduce && t->feature_count != 0u && (t->feature_permutation == nullptr || feature_weights == nullptr))
        || t->tile_block_offsets == nullptr || t->block_row_entry_offsets == nullptr
        || (reduce && t->row_count != 0u && (t->row_permutation == nullptr || row_values == nullptr))
        || (t->tile_block_count != 0u && (t->tile_block_ids == nullptr || t->tile_block_cell_masks == nullptr))
        || (t->row_block_entry_count != 0u
            && (t->row_block_gene_masks == nullptr || t->row_block_value_offsets == nullptr))
        || (reduce && t->nnz_count != 0u && t->values == nullptr))
        return bad(CX_STATUS_INVALID_ARGUMENT, "device input pointer is null");
    if (rows_capacity != 0u || entry_rows != nullptr) {
        if (entry_rows == nullptr && t->row_block_entry_count != 0u)
            return bad(CX_STATUS_INVALID_ARGUMENT, "null entry rows");
        if (rows_capacity < t->row_block_entry_count)
            return bad(CX_STATUS_INVALID_SHAPE, "entry rows capacity is below the entry count");
        // block start << 6 | row in 32 bits
        if (t->feature_count >= (1u << 26))
            return bad(CX_STATUS_UNSUPPORTED, "entry rows need fewer than 2^26 features");
    }
    if (reduce) {
        const void *inputs[] = {feature_weights, t->feature_block_offsets, t->feature_permutation,
                                t->tile_block_offsets, t->tile_block_ids, t->tile_block_cell_masks,
                                t->block_row_entry_offsets, t->row_block_gene_masks,
                                t->row_block_value_offsets, t->values, t->row_permutation, entry_rows};
        for (const void *q : inputs)
            if (q != nullptr && q == static_cast<const void *>(row_values))
                return bad(CX_STATUS_INVALID_ARGUMENT, "output aliases an input");
    } else {
        const void *inputs[] = {t->feature_block_offsets, t->tile_block_offsets, t->tile_block_ids,
                                t->tile_block_cell_masks, t->block_row_entry_offsets,
                                t->row_block_gene_masks, t->row_block_value_offsets};
        for (const void *q : inputs)
            if (q != nullptr && q == static_cast<const void *>(entry_rows))
                return bad(CX_STATUS_INVALID_ARGUMENT, "entry rows alias an input");
    }
    return CX_STATUS_SUCCESS;
}

template<Walk kWalk>
int launch_walk(const cx_cpbp_tiles *t, const float *feature_weights, float *row_values,
                std::uint32_t *entry_rows, void *stream, const char *who) {
    CpbpArgs a{};
    a.feature_block_offsets = t->feature_block_offsets;
    a.feature_permutation = t->feature_permutation;
    a.tile_block_offsets = t->tile_block_offsets;
    a.tile_block_ids = t->tile_block_ids;
    a.cell_masks = t->tile_block_cell_masks;
    a.block_row_entry_offsets = t->block_row_entry_offsets;
    a.gene_masks = t->row_block_gene_masks;
    a.value_offsets = t->row_block_value_offsets;
    a.values = t->values;
    a.row_permutation = t->row_permutation;
    a.weights = feature_weights;
    a.row_values = row_values;
    a.entry_rows = entry_rows;
    a.row_count = t->row_count;
    a.tile_count = t->tile_count;
    a.tile_row_width = t->tile_row_width;
    a.feature_count = t->feature_count;  // 0 features: no descriptors, every row sums to 0
    a.feature_block_count = t->feature_block_count;
    const std::uint32_t wgs = (t->tile_count + kCpbpWaves - 1u) / kCpbpWaves;
    const dim3 grid(wgs < static_cast<std::uint32_t>(kCpbpGrid) ? wgs : kCpbpGrid), block(kWave * kCpbpWaves);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool wide = t->tile_row_width > 32u;
    const bool half = t->value_dtype == CELLERATOR_DTYPE_F16;
    const bool lds = t->feature_count <= kWeightsLds && t->feature_block_count < kBlocksLds;
#define CX_CPBP_LAUNCH(M, V, W) hipLaunchKernelGGL((cpbp_reduce_kernel<M, V, W, kWalk>), grid, block, 0, s, a)
    if constexpr (kWalk == Walk::make_rows) {
        // no weights or values read: one form per mask width
        if (wide) CX_CPBP_LAUNCH(std::uint64_t, float, false);
        else CX_CPBP_LAUNCH(std::uint32_t, float, false);
    } else if (lds) {
        if (wide && half) CX_CPBP_LAUNCH(std::uint64_t, std::uint16_t, true);
        else if (wide) CX_CPBP_LAUNCH(std::uint64_t, float, true);
        else if (half) CX_CPBP_LAUNCH(std::uint32_t, std::uint16_t, true);
        else CX_CPBP_LAUNCH(std::uint32_t, float, true);
    } else {
        if (wide && half) CX_CPBP_LAUNCH(std::uint64_t, std::uint16_t, false);
        else if (wide) CX_CPBP_LAUNCH(std::uint64_t, float, false);
        else if (half) CX_CPBP_LAUNCH(std::uint32_t, std::uint16_t, false);
        else CX_CPBP_LAUNCH(std::uint32_t, float, false);
    }
#undef CX_CPBP_LAUNCH
    return check_launch(who);
}

} // namespace
} // namespace cx

extern "C" int cx_cpbp_reduce(const cx_cpbp_tiles *t, const float *feature_weights,
                              uint64_t feature_weight_capacity, float *row_values,
                              uint64_t row_capacity, void *stream) {
    using namespace cx;
    clear_error();
    const int rc = check_walk(t, true, feature_weights, feature_weight_capacity, row_values, row_capacity,
                              nullptr, 0u, "cx_cpbp_reduce");
    if (rc != CX_STATUS_SUCCESS || t->row_count == 0u) return rc;
    return launch_walk<Walk::reduce>(t, feature_weights, row_values, nullptr, stream, "cpbp_reduce");
}

extern "C" int cx_cpbp_entry_rows(const cx_cpbp_tiles *t, uint32_t *entry_rows, uint64_t entry_rows_capacity,
                                  void *stream) {
    using namespace cx;
    clear_error();
    if (entry_rows == nullptr && t != nullptr && t->row_block_entry_count != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_cpbp_entry_rows: null entry rows");
    const int rc = check_walk(t, false, nullptr, 0u, nullptr, 0u, entry_rows, entry_rows_capacity,
                              "cx_cpbp_entry_rows");
    if (rc != CX_STATUS_SUCCESS || t->row_count == 0u || t->row_block_entry_count == 0u) return rc;
    return launch_walk<Walk::make_rows>(t, nullptr, nullptr, entry_rows, stream, "cpbp_entry_rows");
}

extern "C" int cx_cpbp_reduce_rows(const cx_cpbp_tiles *t, const uint32_t *entry_rows,
                                   const float *feature_weights, uint64_t feature_weight_capacity,
                                   float *row_values, uint64_t row_capacity, void *stream) {
    using namespace cx;
    clear_error();
    if (entry_rows == nullptr && t != nullptr && t->row_block_entry_count != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_cpbp_reduce_rows: null entry rows");
    const int rc = check_walk(t, true, feature_weights, feature_weight_capacity, row_values, row_capacity,
                              entry_rows, t != nullptr ? t->row_block_entry_count : 0u, "cx_cpbp_reduce_rows");
    if (rc != CX_STATUS_SUCCESS || t->row_count == 0u) return rc;
    return launch_walk<Walk::with_rows>(t, feature_weights, row_values, const_cast<std::uint32_t *>(entry_rows),
                                        stream, "cpbp_reduce_rows");
}

// ---- the reference's full direct-consumer contract --------------------------------------
// validate_metadata (components/CellPack/src/feature_weighted_row_reduction_cuda.cu:57-136):
// schema versions, the numeric contract, every identity (the reduction identity recomputed),
// then agreement of the plan, the local order and the tiles on their shared domain, before
// the dimension, pointer and aliasing checks of cx_cpbp_reduce.

namespace cx {
namespace {

constexpr std::uint32_t kReductionSchema = 1u, kTileSchema = 1u, kPlanSchema = 1u, kGeometryVersion = 1u;
constexpr std::uint32_t kOrderSchema = 1u, kSignatureVersion = 1u;
constexpr std::uint32_t kRealF16 = 3u, kRealF32 = 4u;  // cellerator::real codes

std::uint64_t splitmix64(std::uint64_t x) {
    x += 0x9e3779b97f4a7c15ull;
    x = (x ^ (x >> 30u)) * 0xbf58476d1ce4e5b9ull;
    x = (x ^ (x >> 27u)) * 0x94d049bb133111ebull;
    return x ^ (x >> 31u);
}

std::uint32_t storage_code(const cx_cpbp_tiles &t) {
    return t.value_dtype == CELLERATOR_DTYPE_F16 ? kRealF16 : t.value_dtype == CELLERATOR_DTYPE_F32 ? kRealF32 : 0u;
}

} // namespace
} // namespace cx

// reduction_identity (feature_weighted_row_reduction_cuda.cu:44-55): a splitmix64 chain over
// the tile identity, the plan geometry, the weight identity, the schema version and the
// storage / weight / accumulation type codes.
extern "C" uint64_t cx_cpbp_reduction_identity(const cx_cpbp_reduction_view *v) {
    using namespace cx;
    if (v == nullptr) return 0u;
    std::uint64_t h = splitmix64(v->tile_identity);
    h = splitmix64(h ^ v->plan_geometry_identity);
    h = splitmix64(h ^ v->feature_weight_identity);
    h = splitmix64(h ^ (static_cast<std::uint64_t>(v->schema_version) << 32u) ^ v->storage_type_code);
    h = splitmix64(h ^ (static_cast<std::uint64_t>(v->weight_type_code) << 32u) ^ v->accumulation_type_code);
    return h == 0u ? 1u : h;
}

extern "C" int cx_cpbp_reduction_view_from_cpk1(const cx_cpk1_view *image, uint64_t feature_weight_identity,
                                                cx_cpbp_reduction_view *out) {
    using namespace cx;
    clear_error();
    if (image == nullptr || out == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_cpbp_reduction_view_from_cpk1: null argument");
    cx_cpbp_reduction_view v{};
    v.schema_version = kReductionSchema;
    v.storage_type_code = storage_code(image->tiles);
    v.weight_type_code = v.accumulation_type_code = kRealF32;
    v.feature_weight_identity = feature_weight_identity;
    v.plan_schema_version = v.tiles_plan_schema_version = kPlanSchema;
    v.plan_geometry_identity_version = v.tiles_geometry_identity_version = kGeometryVersion;
    v.plan_feature_count = image->tiles.feature_count;
    v.plan_feature_block_count = image->tiles.feature_block_count;
    v.plan_geometry_identity = image->feature_block_geometry_identity;
    v.tile_schema_version = kTileSchema;
    v.tile_identity = image->tile_identity;
    v.tiles_geometry_identity = image->feature_block_geometry_identity;
    v.tiles_ordering_identity = image->ordering_identity;
    v.tiles_global_row_begin = image->global_row_begin;
    v.tiles_full_row_count = image->full_row_count;
    v.feature_axis_fingerprint = image->feature_axis_fingerprint;
    v.feature_axis_fingerprint_version = image->feature_axis_fingerprint_version;
    v.tiles_row_domain_identity = image->row_domain_identity;
    v.order_schema_version = kOrderSchema;
    v.order_signature_version = kSignatureVersion;
    v.order_ordering_identity = image->ordering_identity;
    v.order_global_row_begin = image->global_row_begin;
    v.order_full_row_count = image->full_row_count;
    v.order_row_count = image->tiles.row_count;
    v.order_feature_block_count = image->tiles.feature_block_count;
    v.order_group_width = image->order.group_width;
    v.order_geometry_identity = image->feature_block_geometry_identity;
    v.order_row_domain_identity = image->row_domain_identity;
    v.tiles = image->tiles;
    v.reduction_identity = cx_cpbp_reduction_identity(&v);
    *out = v;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_cpbp_reduction_validate(const cx_cpbp_reduction_view *v) {
    using namespace cx;
    clear_error();
    if (v == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "cx_cpbp_reduction_validate: null view");
    const cx_cpbp_tiles &t = v->tiles;
    if (v->schema_version != kReductionSchema || v->tile_schema_version != kTileSchema
        || v->plan_schema_version != kPlanSchema || v->tiles_plan_schema_version != kPlanSchema
        || v->plan_geometry_identity_version != kGeometryVersion
        || v->tiles_geometry_identity_version != kGeometryVersion || v->order_schema_version != kOrderSchema
        || v->order_signature_version != kSignatureVersion)
        return fail(CX_STATUS_UNSUPPORTED, "weighted-row-reduction version is unsupported");
    if (v->storage_type_code == 0u || v->storage_type_code != storage_code(t) || v->weight_type_code != kRealF32
        || v->accumulation_type_code != kRealF32)
        return fail(CX_STATUS_INVALID_ARGUMENT, "weighted-row-reduction numeric contract is incompatible");
    if (v->feature_weight_identity == 0u || v->reduction_identity == 0u || v->tile_identity == 0u
        || v->tiles_ordering_identity == 0u || v->feature_axis_fingerprint == 0u
        || v->feature_axis_fingerprint_version == 0u || v->tiles_row_domain_identity == 0u
        || v->reduction_identity != cx_cpbp_reduction_identity(v))
        return fail(CX_STATUS_INVALID_ARGUMENT, "weighted-row-reduction identity is invalid");
    if (v->plan_feature_count != t.feature_count || v->plan_feature_block_count != t.feature_block_count
        || v->plan_geometry_identity != v->tiles_geometry_identity
        || v->order_geometry_identity != v->tiles_geometry_identity
        || v->order_ordering_identity != v->tiles_ordering_identity
        || v->order_global_row_begin != v->tiles_global_row_begin
        || v->order_full_row_count != v->tiles_full_row_count || v->order_row_count != t.row_count
        || v->order_feature_block_count != t.feature_block_count
        || v->order_row_domain_identity != v->tiles_row_domain_identity || v->order_group_width != t.tile_row_width)
        return fail(CX_STATUS_INVALID_SHAPE, "weighted-row-reduction plan, order, and tile domains disagree");
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_cpbp_reduce_checked(const cx_cpbp_reduction_view *v, const float *feature_weights,
                                      uint64_t feature_weight_capacity, float *row_values, uint64_t row_capacity,
                                      void *stream) {
    const int rc = cx_cpbp_reduction_validate(v);
    if (rc != CX_STATUS_SUCCESS) return rc;
    return cx_cpbp_reduce(&v->tiles, feature_weights, feature_weight_capacity, row_values, row_capacity, stream);
}
